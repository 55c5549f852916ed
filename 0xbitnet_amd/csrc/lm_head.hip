// Tied f16 LM head with fused final RMSNorm and greedy argmax, token
// embedding gather, and the load-time I2_S repack, for gfx950.
//
// Reference: sh/f32_matmul.wgsl:27-74 (logits[v] = sum_d h[d] E[v,d]),
// sh/rmsnorm.wgsl:27-63 (final norm, rs/nn/model.rs:354-391),
// sh/embedding.wgsl:23-46, rs/sampling.rs:4-80 with top_k = 1 (argmax).
// The reference reads the 513 KB of logits back to the host every token; here
// the argmax is reduced on the device (one atomic max per block, then a
// one-block finish kernel) and written to the decode state, so a decode step
// never needs the host.
#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

struct LmParams {
    const float *x;        // residual stream row [D] (pre final-norm)
    const float *gamma;    // final norm weight [D]
    float eps;
    const uint4 *E;        // lm-tiled embedding (below)
    int V, D;
    float *logits;         // [NV][V]
    int *state;            // decode state (see oxb_kernels.h), one block per row
    int *tok_hist;         // [max_gen] generated tokens per row, may be null
    int advance;           // positions to add to state.pos (tokens in this forward)
    size_t x_stride;       // floats between rows of x
    int state_stride;      // ints between the rows' state blocks
    int hist_stride;       // ints between the rows' token histories
};

// Row-per-lane layout of the tied embedding for the LM head ("lm-tiled"):
// 64-row tiles; each lane (row) streams the pairs (E[2dh], E[2dh+1]) of its
// row in the order the shader's reduction consumes them: shader thread
// t = bitrev8(i) for i = 0..255, and for each t its pairs dh = t + 256 j,
// j = 0..NJ-1 (NJ = D/512).  Dword u = i*NJ + j of row r of tile T sits at
// uint4 ((T*NQ + u/4)*64 + r), component u%4 (NQ = 64*NJ uint4 per lane).
// The halving tree of sh/f32_matmul.wgsl:59-68 is the balanced pairwise
// tree over the 256 thread sums taken in bit-reversed order, so a lane can
// fold it left to right: 8-leaf subtrees in registers, pairs of them into
// the 16 sums of 16 leaves, then the tree over those 16.  Result: the
// shader's exact f32 value.

// (value, index) -> u64 whose unsigned maximum is the largest value with the
// lowest index on ties (rs/sampling.rs argmax semantics); -0 counts as +0,
// as the comparison v > best does.
__device__ inline unsigned long long argmax_key(float v, int i) {
    if (v == 0.0f) v = 0.0f;
    const uint32_t b = __float_as_uint(v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (0xffffffffu - (uint32_t)i);
}

__device__ inline bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}


// 8 leaves (half of a 16-leaf group) of one row: 8*NJ pairs = 2*NJ uint4.
// Each step of a leaf's sum is one fused multiply-add acc = fma(h, e, acc)
// (the restatement's rounding for sh/f32_matmul.wgsl's `sum += a * b`) that
// takes the f16 operand directly (v_fma_mix_f32).
template <int NJ>
__device__ inline float lm_half_group(const uint4 (&e)[2 * NJ], const float2 *hk) {
    float L[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int u = m * NJ + j;
            const uint32_t word = (&e[u >> 2].x)[u & 3];
            const float2 hh = hk[u];
            const float e0 = __half2float(__ushort_as_half((uint16_t)(word & 0xffffu)));
            const float e1 = __half2float(__ushort_as_half((uint16_t)(word >> 16)));
            acc = __builtin_fmaf(hh.x, e0, acc);
            acc = __builtin_fmaf(hh.y, e1, acc);
        }
        L[m] = acc;
    }
#pragma unroll
    for (int st = 1; st < 8; st <<= 1)
#pragma unroll
        for (int m = 0; m < 8; m += 2 * st) L[m] = L[m] + L[m + st];
    return L[0];
}

// The same 8 leaves for NV rows at once, h read from the global pair table
// hk [8*NJ][NV] (pair u of every row contiguous): the address is
// workgroup-uniform, so the pairs arrive through scalar loads and enter each
// v_fma_mix as SGPR operands (no LDS traffic); one E word feeds NV rows.
template <int NJ, int NV>
__device__ inline void lm_half_group_rows(const uint4 (&e)[2 * NJ], const float2 *__restrict__ hk,
                                          float (&g)[NV]) {
    float L[NV][8];
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int m = 0; m < 8; ++m) L[v][m] = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int u = m * NJ + j;
            const uint32_t word = (&e[u >> 2].x)[u & 3];
            const float e0 = __half2float(__ushort_as_half((uint16_t)(word & 0xffffu)));
            const float e1 = __half2float(__ushort_as_half((uint16_t)(word >> 16)));
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const float2 hh = hk[u * NV + v];
                L[v][m] = __builtin_fmaf(hh.x, e0, L[v][m]);
                L[v][m] = __builtin_fmaf(hh.y, e1, L[v][m]);
            }
        }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
        for (int st = 1; st < 8; st <<= 1)
#pragma unroll
            for (int m = 0; m < 8; m += 2 * st) L[v][m] = L[v][m] + L[v][m + st];
        g[v] = L[v][0];
    }
}

// Final RMSNorm of row blockIdx.x (sh/rmsnorm.wgsl order, as the LM head's
// own prologue) into the pair table hn [256*NJ][nv]: pair u of every row of
// the pass contiguous, in the order the LM head consumes them.
template <int NJ>
__global__ __launch_bounds__(256) void lm_norm_pairs_kernel(const float *__restrict__ x,
                                                             size_t x_stride,
                                                             const float *__restrict__ gamma,
                                                             float eps, int D, int nv,
                                                             float2 *__restrict__ hn) {
    __shared__ float red[324];
    const int v = blockIdx.x, tid = threadIdx.x;
    x += (size_t)v * x_stride;
    float ss = 0.0f;
    for (int c = tid; c < D; c += 256) {
        const float xv = x[c];
        const float sq = xv * xv;
        ss = ss + sq;
    }
    const float sum = block256_tree_sum_fast(ss, red);
    const float rms = 1.0f / sqrtf(sum / (float)D + eps);
    for (int u = tid; u < 256 * NJ; u += 256) {
        const int i = u / NJ, j = u % NJ;
        const int t = (bitrev4(i & 15) << 4) | bitrev4(i >> 4);
        const int d0 = 2 * (t + 256 * j);
        const float a0 = x[d0] * rms, a1 = x[d0 + 1] * rms;
        hn[(size_t)u * nv + v] = make_float2(a0 * gamma[d0], a1 * gamma[d0 + 1]);
    }
}

// One workgroup per lm tile at a time (tiles blockIdx.x + i*gridDim.x); its
// 4 waves split the tile's 32 half-groups (8 leaves each) 8 apiece and
// stream them double-buffered, so 20 KiB per wave stay in flight.  The 16
// group sums meet in LDS; one wave per tile folds them, writes the logits and
// keeps a running argmax.  Block winners meet in one 64-bit atomic max
// (argmax_key) in the decode state; lm_finish_kernel, launched right after,
// publishes the token.  (A last-block ticket would need a release per block
// to order the maxima before it: an agent-scope release writes back the L2,
// and with ~63 blocks per XCD those write-backs cost ~9 us per pass, against
// ~1.6 us for the second launch.)
// HG: the normalised rows come from the pair table p_hn (lm_norm_pairs_kernel)
// instead of the workgroup's own prologue.
template <int NJ, int NV, bool HG = false>  // D = 512 * NJ; NV rows of x (one pass over E)
__global__ __launch_bounds__(256) void lm_head_kernel(LmParams p, const float2 *__restrict__ p_hn) {
    __shared__ float red[324];
    __shared__ __align__(16) float2 hp[HG ? 1 : NV][HG ? 2 : 256 * NJ];   // h pairs in consumption order
    __shared__ float Tl[NV][2][16][64];                  // group sums, double-buffered per tile
    __shared__ float bval[NV][4];
    __shared__ int bidx[NV][4];
    constexpr int NQ = 64 * NJ, HQ = 2 * NJ;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = p.D;
    const int ntiles = (p.V + 63) >> 6;
    const int my_tiles =
        (int)blockIdx.x < ntiles ? (ntiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int nseq = my_tiles * 8;  // half-groups of this wave
    auto src_of = [&](int s) {
        const int tile = blockIdx.x + (s >> 3) * gridDim.x;
        const int hg = 8 * w + (s & 7);
        return p.E + ((size_t)tile * NQ + (size_t)hg * HQ) * 64 + lane;
    };
    auto load_hg = [&](uint4 (&dst)[HQ], int s) {
        const uint4 *sp = src_of(s);
        // keep each batch together so the wait for one batch never covers the next
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < HQ; ++q) dst[q] = load_nt(sp + q * 64);
        __builtin_amdgcn_sched_barrier(0);
    };
    uint4 A[HQ], B[HQ];
    // One row: its values, pairs and gamma pairs are loaded first, then the
    // first two weight batches, so the norm waits for the row only (not for
    // the weights queued behind it) and both batches stay in flight across
    // the barrier.  D = 512 NJ: 2 NJ strided values and NJ pairs per thread.
    // (One pass of the 2B head 98.5 -> 98.1 us, decode 1298 -> 1300 tok/s.)
    constexpr bool EARLY = NV == 1 && !HG;
    [[maybe_unused]] float xr[EARLY ? 2 * NJ : 1];
    [[maybe_unused]] float2 xp[EARLY ? NJ : 1], gp[EARLY ? NJ : 1];
    if constexpr (EARLY) {
#pragma unroll
        for (int k = 0; k < 2 * NJ; ++k) xr[k] = p.x[tid + 256 * k];
#pragma unroll
        for (int k = 0; k < NJ; ++k) {
            const int u = tid + 256 * k, i = u / NJ, j = u % NJ;
            const int t = (bitrev4(i & 15) << 4) | bitrev4(i >> 4);
            const int d0 = 2 * (t + 256 * j);
            xp[k] = make_float2(p.x[d0], p.x[d0 + 1]);
            gp[k] = make_float2(p.gamma[d0], p.gamma[d0 + 1]);
        }
    }
    if (nseq > 0) load_hg(A, 0);   // weights do not depend on the norm: start early
    if constexpr (EARLY) {
        if (nseq > 0) load_hg(B, 1);
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < 2 * NJ; ++k) {
            const float sq = xr[k] * xr[k];
            ss = ss + sq;
        }
        const float sum = block256_tree_sum_fast(ss, red);
        const float rms = 1.0f / sqrtf(sum / (float)D + p.eps);
#pragma unroll
        for (int k = 0; k < NJ; ++k) {
            const float a0 = xp[k].x * rms, a1 = xp[k].y * rms;
            hp[0][tid + 256 * k] = make_float2(a0 * gp[k].x, a1 * gp[k].y);
        }
    }

    // final RMSNorm (sh/rmsnorm.wgsl order) of each row straight into its pair table
#pragma unroll 1
    for (int v = 0; v < (HG || EARLY ? 0 : NV); ++v) {
        const float *x = p.x + (size_t)v * p.x_stride;
        float ss = 0.0f;
        for (int c = tid; c < D; c += 256) {
            const float xv = x[c];
            const float sq = xv * xv;
            ss = ss + sq;
        }
        const float sum = block256_tree_sum_fast(ss, red);
        const float rms = 1.0f / sqrtf(sum / (float)D + p.eps);
        for (int u = tid; u < 256 * NJ; u += 256) {
            const int i = u / NJ, j = u % NJ;
            const int t = (bitrev4(i & 15) << 4) | bitrev4(i >> 4);
            const int d0 = 2 * (t + 256 * j);
            const float a0 = x[d0] * rms, a1 = x[d0 + 1] * rms;
            if constexpr (!HG) hp[v][u] = make_float2(a0 * p.gamma[d0], a1 * p.gamma[d0 + 1]);
        }
    }
    if constexpr (!HG) __syncthreads();

    float best[NV];
    int besti[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) { best[v] = -INFINITY; besti[v] = 0x7fffffff; }
    auto finish_pair = [&](const float (&g0)[NV], const float (&g1)[NV], int s) {
        const int k = (8 * w + (s & 7)) >> 1;   // 16-leaf group
        const int i = s >> 3;                   // tile ordinal within this block
#pragma unroll
        for (int v = 0; v < NV; ++v) Tl[v][i & 1][k][lane] = g0[v] + g1[v];
        if ((s & 7) == 6) {                     // this tile's groups are all done
            lds_barrier();
            if (w == (i & 3)) {
                const int row = (blockIdx.x + i * gridDim.x) * 64 + lane;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    float T[16];
#pragma unroll
                    for (int kk = 0; kk < 16; ++kk) T[kk] = Tl[v][i & 1][kk][lane];
#pragma unroll
                    for (int st = 1; st < 16; st <<= 1)
#pragma unroll
                        for (int m = 0; m < 16; m += 2 * st) T[m] = T[m] + T[m + st];
                    if (row < p.V) {
                        p.logits[(size_t)v * p.V + row] = T[0];
                        if (better(T[0], row, best[v], besti[v])) { best[v] = T[0]; besti[v] = row; }
                    }
                }
            }
        }
    };
    auto half_groups = [&](const uint4 (&e)[HQ], int hg, float (&g)[NV]) {
        if constexpr (HG) {
            const int hgu = __builtin_amdgcn_readfirstlane(hg);   // wave-uniform
            lm_half_group_rows<NJ, NV>(e, p_hn + (size_t)hgu * 8 * NJ * NV, g);
        } else {
#pragma unroll
            for (int v = 0; v < NV; ++v) g[v] = lm_half_group<NJ>(e, hp[v] + hg * 8 * NJ);
        }
    };
    int s = 0;
    float g0[NV], g1[NV];
    if constexpr (EARLY) {   // B already holds half-group 1 (nseq is a multiple of 8)
        for (; s < nseq - 2; s += 2) {
            half_groups(A, 8 * w + (s & 7), g0);
            load_hg(A, s + 2);
            half_groups(B, 8 * w + (s & 7) + 1, g1);
            load_hg(B, s + 3);
            finish_pair(g0, g1, s);
        }
    } else {
        for (; s < nseq - 2; s += 2) {
            load_hg(B, s + 1);
            half_groups(A, 8 * w + (s & 7), g0);
            load_hg(A, s + 2);
            half_groups(B, 8 * w + (s & 7) + 1, g1);
            finish_pair(g0, g1, s);
        }
    }
    if (nseq > 0) {   // last pair: nothing left to prefetch
        if constexpr (!EARLY) load_hg(B, s + 1);
        half_groups(A, 8 * w + (s & 7), g0);
        half_groups(B, 8 * w + (s & 7) + 1, g1);
        finish_pair(g0, g1, s);
    }

#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best[v], o, 64);
            const int oi = __shfl_xor(besti[v], o, 64);
            if (better(ov, oi, best[v], besti[v])) { best[v] = ov; besti[v] = oi; }
        }
        if (lane == 0) { bval[v][w] = best[v]; bidx[v][w] = besti[v]; }
    }
    __syncthreads();
    if (tid != 0) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        float bv = bval[v][0];
        int bi = bidx[v][0];
        for (int k = 1; k < 4; ++k)
            if (better(bval[v][k], bidx[v][k], bv, bi)) { bv = bval[v][k]; bi = bidx[v][k]; }
        unsigned long long *key =
            (unsigned long long *)(p.state + (size_t)v * p.state_stride + OXB_ST_LM_KEY);
        __hip_atomic_fetch_max(key, argmax_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// After the LM head (the kernel boundary orders every block's max before
// this): publish each row's token from its argmax key, append it to the
// row's history, advance the position and clear the key for the next pass.
__global__ __launch_bounds__(64) void lm_finish_kernel(LmParams p, int nv) {
    const int v = threadIdx.x;
    if (v >= nv) return;
    int *st = p.state + (size_t)v * p.state_stride;
    unsigned long long *key = (unsigned long long *)(st + OXB_ST_LM_KEY);
    const unsigned long long k = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int tok = (int)(0xffffffffu - (uint32_t)k);
    int *hist = p.tok_hist ? p.tok_hist + (size_t)v * p.hist_stride : nullptr;
    st[OXB_ST_TOKEN] = tok;
    if (hist && st[OXB_ST_NGEN] < st[OXB_ST_HIST_CAP]) hist[st[OXB_ST_NGEN]] = tok;
    st[OXB_ST_NGEN] = st[OXB_ST_NGEN] + 1;
    st[OXB_ST_POS] = st[OXB_ST_POS] + p.advance;
    __hip_atomic_store(key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// x[t][d] = E[id_t][d] (f16 -> f32); ids out of range give zeros.
// ids == nullptr: the single id is the decode state's current token.
__global__ __launch_bounds__(256) void embedding_kernel(const uint16_t *__restrict__ E, int V,
                                                        int D, const int *__restrict__ ids,
                                                        int ids_stride,
                                                        const int *__restrict__ state,
                                                        float *__restrict__ x) {
    const int t = blockIdx.x;
    const int id = ids ? ids[(size_t)t * ids_stride] : state[OXB_ST_TOKEN];
    for (int d = threadIdx.x; d < D; d += 256)
        x[(size_t)t * D + d] =
            (id >= 0 && id < V) ? __half2float(__ushort_as_half(E[(size_t)id * D + d])) : 0.0f;
}

// The same rows read from the LM head's lm-tiled copy of the table (the
// model keeps no other): element d of row `id` is half d % 2 of dword
// lm_dword(id, d / 2).
__global__ __launch_bounds__(256) void embedding_lm_kernel(const uint32_t *__restrict__ E_lm,
                                                           int V, int D, const int *__restrict__ ids,
                                                           int ids_stride,
                                                           const int *__restrict__ state,
                                                           float *__restrict__ x) {
    const int t_row = blockIdx.x;
    const int id = ids ? ids[(size_t)t_row * ids_stride] : state[OXB_ST_TOKEN];
    const int NJ = D / 512;
    const bool in = id >= 0 && id < V;
    for (int d = threadIdx.x; d < D; d += 256) {
        const uint32_t w = in ? E_lm[lm_dword(id, d >> 1, NJ)] : 0u;
        x[(size_t)t_row * D + d] =
            in ? __half2float(__ushort_as_half((uint16_t)((d & 1) ? w >> 16 : w & 0xffffu))) : 0.0f;
    }
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

template <int NV, bool HG = false>
static int lm_launch(const LmParams &p, hipStream_t s, const float2 *hn = nullptr) {
    // One row streams the table fastest with at most one workgroup per CU
    // and long runs of tiles each (about 0.8 x CUs workgroups: 10 tiles
    // apiece at V = 128256 on 256 CUs, 98.5 us against 107.8 us with 4
    // tiles and two workgroups per CU); passes over several rows do more
    // arithmetic per byte and keep 4 tiles per workgroup.
    const int ntiles = (p.V + 63) / 64;
    const int tpw = NV == 1 ? std::max(1, (ntiles + device_cus() * 4 / 5 - 1) / (device_cus() * 4 / 5)) : 4;
    const int grid = (ntiles + tpw - 1) / tpw;
    switch (p.D / 512) {
#define OXB_NL(n)                                                                              \
    case n:                                                                                    \
        if constexpr (HG)                                                                      \
            hipLaunchKernelGGL((lm_norm_pairs_kernel<n>), dim3(NV), dim3(256), 0, s, p.x,      \
                               p.x_stride, p.gamma, p.eps, p.D, NV, (float2 *)hn);            \
        hipLaunchKernelGGL((lm_head_kernel<n, NV, HG>), dim3(grid), dim3(256), 0, s, p, hn);   \
        hipLaunchKernelGGL(lm_finish_kernel, dim3(1), dim3(64), 0, s, p, NV);                  \
        break;
        OXB_NL(1) OXB_NL(2) OXB_NL(3) OXB_NL(4) OXB_NL(5)
#undef OXB_NL
        default:
            oxb::set_error("lm_head: hidden %d unsupported (512 .. 2560)", p.D);
            return -1;
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_lm_head_argmax(const float *x, const float *gamma, float eps,
                                  const void *E, int V, int D, float *logits, int *state,
                                  int *tok_hist, int advance, void *stream) {
    return oxb_lm_head_argmax_batch(x, (size_t)D, gamma, eps, E, V, D, logits, state,
                                    OXB_STATE_INTS, tok_hist, 0, 1, advance, stream);
}

extern "C" int oxb_lm_head_argmax_batch(const float *x, size_t x_stride, const float *gamma,
                                        float eps, const void *E, int V, int D, float *logits,
                                        int *state, int state_stride, int *tok_hist,
                                        int hist_stride, int n_rows, int advance, void *stream) {
    OXB_REQUIRE(D % 512 == 0 && D <= 5 * 512,
                "lm_head: hidden %d must be a multiple of 512 and <= 2560", D);
    OXB_REQUIRE(V > 0, "lm_head: vocab %d", V);
    OXB_REQUIRE(n_rows > 0, "lm_head: %d rows", n_rows);
    OXB_REQUIRE(((uintptr_t)state & 7) == 0 && state_stride % 2 == 0 &&
                    (n_rows == 1 || state_stride >= OXB_STATE_INTS),
                "lm_head: state blocks must be 8-byte aligned and not overlap");
    hipStream_t s = (hipStream_t)stream;
    // rows in groups of 4 (one pass over the table each), then 2, then 1
    for (int r0 = 0; r0 < n_rows;) {
        const int left = n_rows - r0;
        const int nv = left >= 4 ? 4 : left >= 2 ? 2 : 1;
        LmParams p{x + (size_t)r0 * x_stride, gamma, eps, (const uint4 *)E, V, D,
                   logits + (size_t)r0 * V, state + (size_t)r0 * state_stride,
                   tok_hist ? tok_hist + (size_t)r0 * hist_stride : nullptr, advance,
                   x_stride, state_stride, hist_stride};
        const int rc = nv == 4 ? lm_launch<4>(p, s) : nv == 2 ? lm_launch<2>(p, s) : lm_launch<1>(p, s);
        if (rc) return rc;
        r0 += nv;
    }
    return 0;
}

namespace oxb {
// The batched LM head with a workspace hn of n_rows * D floats: rows in passes
// of 8 (then 4, 2, 1), each pass's normalised rows written once as a pair
// table that the LM head reads through scalar loads.  Same logits and tokens
// as oxb_lm_head_argmax_batch.
int lm_head_argmax_rows(const float *x, size_t x_stride, const float *gamma, float eps,
                        const void *E, int V, int D, float *logits, int *state, int state_stride,
                        int *tok_hist, int hist_stride, int n_rows, int advance, float *hn,
                        void *stream) {
    OXB_REQUIRE(D % 512 == 0 && D <= 5 * 512,
                "lm_head: hidden %d must be a multiple of 512 and <= 2560", D);
    OXB_REQUIRE(V > 0 && n_rows > 0 && hn, "lm_head: vocab %d, %d rows", V, n_rows);
    OXB_REQUIRE(((uintptr_t)state & 7) == 0 && state_stride % 2 == 0 &&
                    (n_rows == 1 || state_stride >= OXB_STATE_INTS),
                "lm_head: state blocks must be 8-byte aligned and not overlap");
    hipStream_t s = (hipStream_t)stream;
    for (int r0 = 0; r0 < n_rows;) {
        const int left = n_rows - r0;
        const int nv = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        LmParams p{x + (size_t)r0 * x_stride, gamma, eps, (const uint4 *)E, V, D,
                   logits + (size_t)r0 * V, state + (size_t)r0 * state_stride,
                   tok_hist ? tok_hist + (size_t)r0 * hist_stride : nullptr, advance,
                   x_stride, state_stride, hist_stride};
        const float2 *h = (const float2 *)(hn + (size_t)r0 * D);
        const int rc = nv == 8   ? lm_launch<8, true>(p, s, h)
                       : nv == 4 ? lm_launch<4, true>(p, s, h)
                       : nv == 2 ? lm_launch<2, true>(p, s, h)
                                 : lm_launch<1, true>(p, s, h);
        if (rc) return rc;
        r0 += nv;
    }
    return 0;
}
}  // namespace oxb

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
                       ids, 1, state, x);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

namespace oxb {
// Rows from the lm-tiled table: ids[t * ids_stride] for t < n_tok, or the
// decode state's token when ids is null (n_tok 1).
int embedding_lm(const void *E_lm, int V, int D, const int *ids, int ids_stride, const int *state,
                 int n_tok, float *x, void *stream) {
    OXB_REQUIRE(n_tok > 0 && D % 512 == 0 && D <= 5 * 512 && (ids || (state && n_tok == 1)),
                "embedding: bad shape");
    hipLaunchKernelGGL(embedding_lm_kernel, dim3(n_tok), dim3(256), 0, (hipStream_t)stream,
                       (const uint32_t *)E_lm, V, D, ids, ids_stride, state, x);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace oxb

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
