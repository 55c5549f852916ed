// Tied f16 LM head with fused final RMSNorm and greedy argmax, token
// embedding gather, and the load-time I2_S repack, for gfx950.
//
// Reference: sh/f32_matmul.wgsl:27-74 (logits[v] = sum_d h[d] E[v,d]),
// sh/rmsnorm.wgsl:27-63 (final norm, rs/nn/model.rs:354-391),
// sh/embedding.wgsl:23-46, rs/sampling.rs:4-80 with top_k = 1 (argmax).
// The reference reads the 513 KB of logits back to the host every token; here
// the argmax is reduced on the device (last-block pattern) and written to the
// decode state, so a decode step never needs the host.
#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

constexpr int kLmBlocks = 1024;  // persistent-style grid: 4 workgroups per CU
constexpr int kLmRowsInFlight = 4;
constexpr int kLmMaxLoads = 8;   // 16-byte loads per row per lane: D <= 8*64*8 = 4096

struct LmParams {
    const float *x;        // residual stream row [D] (pre final-norm)
    const float *gamma;    // final norm weight [D]
    float eps;
    const uint4 *E;        // [V][D] f16
    int V, D;
    float *logits;         // [V]
    float2 *part;          // [gridDim.x] (max value, index bits)
    int *state;            // decode state (see oxb_kernels.h)
    int *tok_hist;         // [max_gen] generated tokens, may be null
    int advance;           // positions to add to state.pos (tokens in this forward)
};

__device__ inline bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

template <int NL>  // 16-byte loads per row per lane: D = 512 * NL
__global__ __launch_bounds__(256) void lm_head_kernel(LmParams p) {
    __shared__ float red[256];
    __shared__ __align__(16) float h_lds[kLmMaxLoads * 64 * 8];
    __shared__ float bval[4];
    __shared__ int bidx[4];
    __shared__ int ticket_s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = p.D;

    // rows of this block
    const int per = (p.V + gridDim.x - 1) / gridDim.x;
    const int r0 = blockIdx.x * per, r1 = min(p.V, r0 + per);

    // final RMSNorm in the shader's order (strided partials + tree)
    float ss = 0.0f;
    for (int c = tid; c < D; c += 256) {
        float v = p.x[c];
        float sq = v * v;
        ss = ss + sq;
    }
    const float sum = block256_tree_sum(ss, red);
    const float rms = 1.0f / sqrtf(sum / (float)D + p.eps);
    for (int c = tid; c < D; c += 256) {
        float a = p.x[c] * rms;
        h_lds[c] = a * p.gamma[c];
    }
    __syncthreads();
    float hv[NL][8];
#pragma unroll
    for (int j = 0; j < NL; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) hv[j][i] = h_lds[(j * 64 + lane) * 8 + i];

    // One wave per row, reproducing sh/f32_matmul.wgsl:51-68 exactly: shader
    // thread t accumulates pairs dh = t, t+256, ... as acc += h*e0; acc += h*e1,
    // then the halving tree.  Lane l plays threads 4l .. 4l+3, so its 16-byte
    // load j holds the pairs dh = 256j + 4l + i of those four threads.
    float best = -INFINITY;
    int besti = 0x7fffffff;
    const int rowstride = D >> 3;   // uint4 per row
    for (int rb = r0 + w * kLmRowsInFlight; rb < r1; rb += 4 * kLmRowsInFlight) {
        uint4 e[kLmRowsInFlight][NL];
#pragma unroll
        for (int q = 0; q < kLmRowsInFlight; ++q) {
            const int row = min(rb + q, r1 - 1);
#pragma unroll
            for (int j = 0; j < NL; ++j)
                e[q][j] = load_nt(p.E + (size_t)row * rowstride + j * 64 + lane);
        }
#pragma unroll
        for (int q = 0; q < kLmRowsInFlight; ++q) {
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                const __half2 *hh = (const __half2 *)&e[q][j];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float2 f = __half22float2(hh[i]);
                    float m0 = hv[j][2 * i] * f.x;
                    a[i] = a[i] + m0;
                    float m1 = hv[j][2 * i + 1] * f.y;
                    a[i] = a[i] + m1;
                }
            }
            // tree: strides 128..4 pair lane l with lane l + stride/4
#pragma unroll
            for (int sl = 32; sl >= 1; sl >>= 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float o = __shfl_down(a[i], sl, 64);
                    a[i] = a[i] + o;
                }
            }
            a[0] = a[0] + a[2];   // stride 2
            a[1] = a[1] + a[3];
            const float acc = __shfl(a[0] + a[1], 0, 64);  // stride 1, broadcast
            const int row = rb + q;
            if (row < r1) {
                if (lane == 0) p.logits[row] = acc;
                if (better(acc, row, best, besti)) { best = acc; besti = row; }
            }
        }
    }
    if (lane == 0) { bval[w] = best; bidx[w] = besti; }
    __syncthreads();
    if (tid == 0) {
        float bv = bval[0];
        int bi = bidx[0];
        for (int k = 1; k < 4; ++k)
            if (better(bval[k], bidx[k], bv, bi)) { bv = bval[k]; bi = bidx[k]; }
        p.part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
    }
    __threadfence();
    __syncthreads();
    if (tid == 0)
        ticket_s = __hip_atomic_fetch_add(&p.state[OXB_ST_LM_COUNTER], 1, __ATOMIC_ACQ_REL,
                                          __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket_s != (int)gridDim.x - 1) return;
    __threadfence();
    // last block: reduce the per-block winners (lowest index on ties)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int b = tid; b < (int)gridDim.x; b += 256) {
        const float v = __hip_atomic_load(&p.part[b].x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int i = __float_as_int(
            __hip_atomic_load(&p.part[b].y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        const float ov = __shfl_xor(bv, s, 64);
        const int oi = __shfl_xor(bi, s, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { bval[w] = bv; bidx[w] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int k = 1; k < 4; ++k)
            if (better(bval[k], bidx[k], bval[0], bidx[0])) { bval[0] = bval[k]; bidx[0] = bidx[k]; }
        const int tok = bidx[0];
        int *st = p.state;
        st[OXB_ST_TOKEN] = tok;
        if (p.tok_hist && st[OXB_ST_NGEN] < st[OXB_ST_HIST_CAP]) p.tok_hist[st[OXB_ST_NGEN]] = tok;
        st[OXB_ST_NGEN] = st[OXB_ST_NGEN] + 1;
        st[OXB_ST_POS] = st[OXB_ST_POS] + p.advance;
        st[OXB_ST_LM_COUNTER] = 0;
    }
}

// x[t][d] = E[id_t][d] (f16 -> f32); ids out of range give zeros.
// ids == nullptr: the single id is the decode state's current token.
__global__ __launch_bounds__(256) void embedding_kernel(const uint16_t *__restrict__ E, int V,
                                                        int D, const int *__restrict__ ids,
                                                        const int *__restrict__ state,
                                                        float *__restrict__ x) {
    const int t = blockIdx.x;
    const int id = ids ? ids[t] : state[OXB_ST_TOKEN];
    for (int d = threadIdx.x; d < D; d += 256)
        x[(size_t)t * D + d] =
            (id >= 0 && id < V) ? __half2float(__ushort_as_half(E[(size_t)id * D + d])) : 0.0f;
}

// Natural I2_S rows [N][K/4] -> tile-chunk layout (see oxb_common.h).
__global__ void repack_tiled_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                    int N, int KC) {
    const size_t total = (size_t)N * KC;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int row = (int)(i / KC), kc = (int)(i % KC);
        dst[tiled_offset16(row, kc, KC)] = src[i];
    }
}

}  // namespace oxb

using namespace oxb;

extern "C" int oxb_lm_head_argmax(const float *x, const float *gamma, float eps,
                                  const uint16_t *E, int V, int D, float *logits, float *part,
                                  int *state, int *tok_hist, int advance, void *stream) {
    OXB_REQUIRE(D % 512 == 0 && D <= kLmMaxLoads * 512,
                "lm_head: hidden %d must be a multiple of 512 and <= %d", D, kLmMaxLoads * 512);
    OXB_REQUIRE(V > 0, "lm_head: vocab %d", V);
    LmParams p{x, gamma, eps, (const uint4 *)E, V, D, logits, (float2 *)part, state, tok_hist,
               advance};
    hipStream_t s = (hipStream_t)stream;
    switch (D / 512) {
#define OXB_NL(n)                                                                       \
    case n:                                                                             \
        hipLaunchKernelGGL(lm_head_kernel<n>, dim3(kLmBlocks), dim3(256), 0, s, p);     \
        break;
        OXB_NL(1) OXB_NL(2) OXB_NL(3) OXB_NL(4) OXB_NL(5) OXB_NL(6) OXB_NL(7) OXB_NL(8)
#undef OXB_NL
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_lm_head_partials(void) { return kLmBlocks; }

extern "C" int oxb_embedding(const uint16_t *E, int V, int D, const int *ids, int n_tok,
                             const int *state, float *x, void *stream) {
    OXB_REQUIRE(n_tok > 0 && D > 0, "embedding: bad shape");
    hipLaunchKernelGGL(embedding_kernel, dim3(n_tok), dim3(256), 0, (hipStream_t)stream, E, V, D,
                       ids, state, x);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_repack_i2s_tiled(const void *natural, void *tiled, int N, int K,
                                    void *stream) {
    OXB_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 128 == 0,
                "repack: N %d must be a multiple of 16 and K %d a multiple of 128", N, K);
    OXB_REQUIRE(natural != tiled, "repack: in-place repack is not supported");
    const int KC = K / 64;
    hipLaunchKernelGGL(repack_tiled_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)natural, (uint4 *)tiled, N, KC);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}
