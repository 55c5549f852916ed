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

// Row-per-lane layout of the tied embedding for the LM head ("lm-tiled"):
// 64-row tiles; each lane (row) streams the pairs (E[2dh], E[2dh+1]) of its
// row in the order the shader's reduction consumes them: shader thread
// t = bitrev8(i) for i = 0..255, and for each t its pairs dh = t + 256 j,
// j = 0..NJ-1 (NJ = D/512).  Dword u = i*NJ + j of row r of tile T sits at
// uint4 ((T*NQ + u/4)*64 + r), component u%4 (NQ = 64*NJ uint4 per lane).
// The halving tree of sh/f32_matmul.wgsl:59-68 is the balanced pairwise
// tree over the 256 thread sums taken in bit-reversed order, so a lane can
// fold it left to right: 16-leaf subtrees in registers, then the 16 subtree
// sums.  Result: the shader's exact f32 value, no cross-lane traffic.
__host__ __device__ inline int bitrev4(int x) {
    return ((x & 1) << 3) | ((x & 2) << 1) | ((x & 4) >> 1) | ((x & 8) >> 3);
}

template <int NJ>  // D = 512 * NJ
__global__ __launch_bounds__(256) void lm_head_kernel(LmParams p) {
    __shared__ float red[324];
    __shared__ __align__(16) float h_lds[kLmMaxLoads * 512];
    __shared__ __align__(16) float2 hp[256 * NJ];   // h pairs in consumption order
    __shared__ float bval[4];
    __shared__ int bidx[4];
    __shared__ int ticket_s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = p.D;
    constexpr int NQ = 64 * NJ;   // uint4 per lane per tile

    // final RMSNorm (sh/rmsnorm.wgsl order), h to LDS
    float ss = 0.0f;
    for (int c = tid; c < D; c += 256) {
        float v = p.x[c];
        float sq = v * v;
        ss = ss + sq;
    }
    const float sum = block256_tree_sum_fast(ss, red);
    const float rms = 1.0f / sqrtf(sum / (float)D + p.eps);
    for (int c = tid; c < D; c += 256) {
        float a = p.x[c] * rms;
        h_lds[c] = a * p.gamma[c];
    }
    __syncthreads();
    for (int u = tid; u < 256 * NJ; u += 256) {
        const int i = u / NJ, j = u % NJ;
        const int t = (bitrev4(i & 15) << 4) | bitrev4(i >> 4);
        const int dh = t + 256 * j;
        hp[u] = make_float2(h_lds[2 * dh], h_lds[2 * dh + 1]);
    }
    __syncthreads();

    const int ntiles = (p.V + 63) >> 6;
    float best = -INFINITY;
    int besti = 0x7fffffff;
    __shared__ float Tl[4][16][64];   // per-lane 16-leaf subtree sums
    for (int tile = blockIdx.x * 4 + w; tile < ntiles; tile += gridDim.x * 4) {
        const uint4 *src = p.E + (size_t)tile * NQ * 64 + lane;
#pragma unroll 1
        for (int k = 0; k < 16; ++k) {
            // 16 leaves i = 16k + m, m = 0..15: 16*NJ dwords = 4*NJ uint4
            uint4 e[4 * NJ];
#pragma unroll
            for (int qq = 0; qq < 4 * NJ; ++qq) e[qq] = load_nt(src + (size_t)(k * 4 * NJ + qq) * 64);
            const float2 *hk = hp + k * 16 * NJ;
            float L[16];
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int u = m * NJ + j;
                    const uint32_t word = (&e[u >> 2].x)[u & 3];
                    const float2 hh = hk[u];
                    const float e0 = __half2float(__ushort_as_half((uint16_t)(word & 0xffffu)));
                    const float e1 = __half2float(__ushort_as_half((uint16_t)(word >> 16)));
                    float m0 = hh.x * e0;
                    acc = acc + m0;
                    float m1 = hh.y * e1;
                    acc = acc + m1;
                }
                L[m] = acc;
            }
#pragma unroll
            for (int st = 1; st < 16; st <<= 1)
#pragma unroll
                for (int m = 0; m < 16; m += 2 * st) L[m] = L[m] + L[m + st];
            Tl[w][k][lane] = L[0];
        }
        float T[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) T[k] = Tl[w][k][lane];
#pragma unroll
        for (int st = 1; st < 16; st <<= 1)
#pragma unroll
            for (int m = 0; m < 16; m += 2 * st) T[m] = T[m] + T[m + st];
        const int row = tile * 64 + lane;
        if (row < p.V) {
            p.logits[row] = T[0];
            if (better(T[0], row, best, besti)) { best = T[0]; besti = row; }
        }
    }
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        const float ov = __shfl_xor(best, s, 64);
        const int oi = __shfl_xor(besti, s, 64);
        if (better(ov, oi, best, besti)) { best = ov; besti = oi; }
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

// Natural f16 embedding [V][D] -> the LM head's lm-tiled layout (above).
__global__ void repack_lm_kernel(const uint32_t *__restrict__ E, uint4 *__restrict__ dst, int V,
                                 int D) {
    const int NJ = D / 512, NQ = 64 * NJ;
    const int ntiles = (V + 63) / 64;
    const size_t total = (size_t)ntiles * NQ * 64;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(idx % 64);
        const size_t rest = idx / 64;
        const int qq = (int)(rest % NQ);
        const int tile = (int)(rest / NQ);
        const int row = tile * 64 + r;
        uint32_t wv[4];
        for (int c = 0; c < 4; ++c) {
            const int u = qq * 4 + c;
            const int i = u / NJ, j = u % NJ;
            const int t = (bitrev4(i & 15) << 4) | bitrev4(i >> 4);
            const int dh = t + 256 * j;
            wv[c] = row < V ? E[(size_t)row * (D / 2) + dh] : 0u;
        }
        dst[idx] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
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
                                  const void *E, int V, int D, float *logits, float *part,
                                  int *state, int *tok_hist, int advance, void *stream) {
    OXB_REQUIRE(D % 512 == 0 && D <= 5 * 512,
                "lm_head: hidden %d must be a multiple of 512 and <= 2560", D);
    OXB_REQUIRE(V > 0, "lm_head: vocab %d", V);
    LmParams p{x, gamma, eps, (const uint4 *)E, V, D, logits, (float2 *)part, state, tok_hist,
               advance};
    hipStream_t s = (hipStream_t)stream;
    switch (D / 512) {
#define OXB_NL(n)                                                                       \
    case n:                                                                             \
        hipLaunchKernelGGL(lm_head_kernel<n>, dim3(kLmBlocks), dim3(256), 0, s, p);     \
        break;
        OXB_NL(1) OXB_NL(2) OXB_NL(3) OXB_NL(4) OXB_NL(5)
#undef OXB_NL
        default:
            oxb::set_error("lm_head: hidden %d unsupported (512 .. 2560)", D);
            return -1;
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_lm_head_partials(void) { return kLmBlocks; }

extern "C" int oxb_repack_lm(const uint16_t *E, void *E_lm, int V, int D, void *stream) {
    OXB_REQUIRE(D % 512 == 0 && D <= 5 * 512 && V > 0, "repack_lm: bad shape V %d D %d", V, D);
    hipLaunchKernelGGL(repack_lm_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream,
                       (const uint32_t *)E, (uint4 *)E_lm, V, D);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" size_t oxb_lm_bytes(int V, int D) { return (size_t)((V + 63) / 64) * 64 * D * 2; }

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
