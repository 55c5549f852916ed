// Decode ternary GEMV family for gfx950 (one token, int8 activations,
// 2-bit weights streamed from HBM in the tile-chunk layout).
//
// Reference: sh/ternary_gemv.wgsl:39-97 (GEMV), sh/quantize.wgsl:28-74,
// sh/rmsnorm.wgsl:27-63 (fused prologue), sh/rope.wgsl:25-56 +
// rs/nn/attention.rs:171-184 (QKV epilogue), sh/activation.wgsl +
// sh/elementwise.wgsl (gate/up epilogue, residual epilogue).
//
// One workgroup (4 or 8 waves) owns one 16-row tile.  Lane l of wave w
// streams chunks (row l%16, 4 NW j + 4w + l/16): every wave load is one
// contiguous KiB, and at each step j the workgroup's waves read one
// contiguous 4 NW KiB stretch of the tile.
// All loads are branch-free (clamped addresses, masked values; none at all
// when K is a multiple of 256) so the compiler's memory counters stay exact:
// the weights are in flight while the prologue runs.  The prologue keeps
// every activation in registers in the shaders' thread mapping: one barrier
// for the RMS sum, one for the absmax, one after the int8 values land in LDS.
#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

constexpr int kMaxNormReg = 28; // f32 values per thread in a norm prologue (D <= 7168)

enum Pro { PRO_INT8 = 0, PRO_QUANT = 1 };           // PRO_QUANT: optional RMSNorm + quantize
// EPI_QKV stores K/V as f16 bits, EPI_QKV32 as f32 (the reference's cache type)
enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_GATEUP = 3, EPI_QKV32 = 4 };
__host__ __device__ constexpr bool is_qkv(int epi) { return epi == EPI_QKV || epi == EPI_QKV32; }

struct GemvParams {
    const uint4 *W;        // tile-chunk layout
    const float *wscale;   // [N]
    int N, K;
    // PRO_INT8
    const int8_t *xq;
    const float *xscale;   // [1]
    const int *xsum;       // [1]
    // PRO_QUANT
    const float *x;        // [K]
    const float *gamma;    // [K] or nullptr (no norm)
    float eps;
    // epilogues
    float *y;              // STORE: [N]; RESID: residual stream [N] (in place)
    int32_t *acc_out;      // optional raw int32 accumulators [N]
    int8_t *xq_out;        // optional: the prologue's int8 vector [K] (block 0 writes)
    float *xscale_out;     // optional
    // QKV
    float *q_out;          // [Dq]
    void *kcache, *vcache;  // [Hkv][max_seq][hd] f16 bits (EPI_QKV) or f32 (EPI_QKV32)
    uint16_t *vcache8;      // optional (EPI_QKV): V also in position octets (v8_index)
    const float2 *rope;    // [max_seq][hd/2] (cos, sin)
    const int *pos;        // device position
    int Dq, Dkv, hd, max_seq;
};

// ---------------------------------------------------------------------------
// Row prologue for the several-token kernels: RMSNorm (optional) + per-token
// absmax int8 quantize of one row of D f32 values by all 256 threads with
// the shaders' thread mapping (thread t owns columns t, t+256, ...:
// sh/rmsnorm.wgsl:41-45, sh/quantize.wgsl:42-45).  Writes int8 into LDS,
// returns the scale and this wave's share of sum(q) in wq[w] (summed after
// the caller's next barrier).  LDS: red >= 324 floats, wq >= 4 ints.
// ---------------------------------------------------------------------------
// Issues the loads only (clamped addresses, no use of the values), so a
// caller can put more loads behind them; mask_row then zeroes columns >= D.
template <int NREG>
__device__ inline void load_row(const float *__restrict__ x, const float *__restrict__ gamma,
                                int D, float (&v)[NREG], float (&g)[NREG]) {
    const int t = threadIdx.x & 255;   // a 256-thread row group
    const float *gp = gamma ? gamma : x;   // loads stay unconditional
#pragma unroll
    for (int j = 0; j < NREG; ++j) {
        const int c = min(t + j * 256, D - 1);
        v[j] = x[c];
        g[j] = gp[c];
    }
}

template <int NREG>
__device__ inline void mask_row(int D, float (&v)[NREG], float (&g)[NREG]) {
    const int t = threadIdx.x & 255;
#pragma unroll
    for (int j = 0; j < NREG; ++j) {
        const bool in = t + j * 256 < D;
        v[j] = in ? v[j] : 0.0f;
        g[j] = in ? g[j] : 0.0f;
    }
}

template <int NREG>
__device__ inline float norm_quant_regs(float (&v)[NREG], const float (&g)[NREG], bool norm,
                                        float eps, int D, int8_t *xq_lds, float *red, int *wq) {
    const int t = threadIdx.x & 255;
    mask_row<NREG>(D, v, const_cast<float (&)[NREG]>(g));
    if (norm) {
        float ss = 0.0f;   // columns past D hold +0 and add exactly nothing
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            float sq = v[j] * v[j];
            ss = ss + sq;
        }
        const float sum = block256_tree_sum_1b(ss, red);
        const float rms = 1.0f / sqrtf(sum / (float)D + eps);  // inverseSqrt
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            float a = v[j] * rms;
            v[j] = a * g[j];
        }
    }
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < NREG; ++j) am = fmaxf(am, fabsf(v[j]));
    am = wave_nonneg_max_dpp(am);
    if ((t & 63) == 0) red[320 + (t >> 6)] = am;
    lds_barrier();
    am = fmaxf(fmaxf(red[320], red[321]), fmaxf(red[322], red[323]));
    const float scale = am == 0.0f ? 1.0f : am / 127.0f;   // sh/quantize.wgsl:59
    const float inv = am == 0.0f ? 0.0f : 127.0f / am;     // :68
    int s = 0;
#pragma unroll
    for (int j = 0; j < NREG; ++j) {
        const int c = t + j * 256;
        if (c < D) {
            const int q = quant_one(v[j], inv);
            xq_lds[c] = (int8_t)q;
            s += q;
        }
    }
    s = wave_isum_dpp(s);
    if ((t & 63) == 0) wq[t >> 6] = s;
    return scale;
}

__device__ inline uint16_t f32_to_f16_bits(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// LDS of the GEMV: xq [K] int8 | red [256] f32 | wmax [4] | wq [4] | wpart [TT][64 NW].
__host__ __device__ inline size_t gemv_smem(int K, int TT, int NW = 4) {
    return (size_t)K + (256 + 4 + 4 + 64 * NW * TT) * 4;
}

// x[t + 256 j], gamma[t + 256 j] for K == 256 * NREG (no clamps needed).
template <int NREG>
__device__ inline void load_row_exact(const float *__restrict__ x, const float *__restrict__ gp,
                                      float (&v)[NREG], float (&g)[NREG]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NREG; ++j) {
        v[j] = x[t + j * 256];
        g[j] = gp[t + j * 256];
    }
}

// NREG: strided f32 values per thread in the prologue (ceil(K/256)); for int8
// rows, the activation row's 16-byte groups per thread;
// PF: 16-byte weight chunks per lane per batch.
// Waves per SIMD the register budget must allow: 4 (<= 128 VGPRs) for the
// one-batch shapes, so that e.g. 864 workgroups of a 13824-row GEMV are all
// resident at once; the 4-chunk double-buffered batches need more registers.
// EXACT: K == 256 * NREG.  TT: 16-row tiles per workgroup (> 1 amortises the
// prologue over more rows when the grid would otherwise oversubscribe the
// CUs, e.g. the 13824-row gate|up GEMV); each chunk's activations are read
// from LDS once for all TT tiles.  NW: waves per workgroup, each taking 1/NW
// of K.  STREAM: double-buffered batches of PF chunks (else one batch covers
// a lane's chunks).  Long int8 rows (e.g. K = 28672) stream best with 8 waves
// and 1-chunk batches: 16 waves per CU keep more loads in flight than 4-chunk
// batches of 4 waves, at under half the registers.
template <int PRO, int EPI, int NREG, int PF, bool EXACT, int TT, int NW = 4, bool STREAM = PF == 4>
__global__ __launch_bounds__(64 * NW, NW == 8 ? 2 : PF * TT <= 3 ? 4 : 2) void gemv_kernel(GemvParams p) {
    static_assert(TT == 1 || !STREAM, "multi-batch streaming is single-tile");
    static_assert(NW == 4 || (PRO == PRO_INT8 && NW == 8), "the norm prologue runs on 256 threads");
    extern __shared__ __align__(16) int8_t smem[];
    const int K = p.K;
    int8_t *xq_lds = smem;
    float *red = (float *)(smem + K);
    float *wmax = red + 256;
    int *wq = (int *)(wmax + 4);
    int *wpart = wq + 4;

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, c = lane >> 4;
    const int KC = K >> 6;
    // chunk j of lane (c, wave w): kc = 4 NW j + 4w + c, so at each step the
    // workgroup's waves read 4 NW consecutive chunks (one contiguous 4 NW KiB
    // stretch of the tile) rather than NW separate ones
    const int cpl = (KC + 4 * NW - 1) / (4 * NW);   // chunks per lane
    const int nb = (cpl + PF - 1) / PF;           // batches (uniform; 1 unless STREAM)
    const int tile0 = blockIdx.x * TT;

    // ---- loads: every input of the epilogue first (the position, this
    // thread's row scale, the residual), then the prologue's row, then the
    // weights, so that the epilogue after the reduction waits on nothing.
    // All kernel arguments are pinned in SGPRs here: read where they are used,
    // the late ones are further kernarg round trips at the end of the kernel.
    asm volatile("" ::"s"(p.x), "s"(p.gamma), "s"(p.eps), "s"(p.y), "s"(p.wscale),
                 "s"(p.acc_out), "s"(p.xq_out), "s"(p.q_out), "s"(p.kcache), "s"(p.vcache),
                 "s"(p.rope));
    const int n_ep = tile0 * 16 + (tid & (16 * TT - 1));   // the row this thread may finish
    [[maybe_unused]] int pos = 0;
    // read per lane (an index the compiler cannot see is zero): a uniform
    // value would be moved to an SGPR, and that copy waits for the load
    // before the weights are even issued
    if constexpr (is_qkv(EPI)) pos = p.pos[opaque_zero()];
    const float ws_ep = p.wscale[n_ep];
    float resid = 0.0f;
    if constexpr (EPI == EPI_RESID) resid = p.y[n_ep];
    __builtin_amdgcn_sched_barrier(0);
    float v[NREG], g[NREG];
    if constexpr (PRO == PRO_QUANT) {
        if constexpr (EXACT) load_row_exact<NREG>(p.x, p.gamma ? p.gamma : p.x, v, g);
        else load_row<NREG>(p.x, p.gamma, K, v, g);
    }
    auto load_batch = [&](uint4 (&dst)[TT][PF], int b) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const uint4 *tw = p.W + (size_t)(tile0 + t) * KC * 16;
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const int kc = 4 * NW * (b * PF + u) + 4 * w + c;
                dst[t][u] = load_nt(tw + (size_t)min(kc, KC - 1) * 16 + r);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    uint4 A[TT][PF];
    [[maybe_unused]] uint4 B[TT][PF];
    // int8 rows: the activation row's loads go out first, all at once,
    // then the weights (two batches when streamed); its LDS writes then wait
    // for those loads only, not for the weights behind them, and the barrier
    // passes while the weights are in flight (a copy loop after the first
    // batch waited for that batch from HBM, then for each further group in
    // turn, before a second batch went out: 8192 x 28672 / 28672 x 8192 /
    // 2560 x 6912 took 11.8 / 12.1 / 3.95 us, now 11.4 / 11.4 / 3.53; one
    // batch, K = 2560: 6912 / 3840 / 13824 rows 3.15 / 2.71 / 4.00 -> 2.96 /
    // 2.55 / 3.81 us)
    constexpr int XU = PRO == PRO_INT8 ? NREG : 1;
    [[maybe_unused]] u32x4_t xr[XU];
    if constexpr (PRO == PRO_INT8) {
#pragma unroll
        for (int u = 0; u < XU; ++u)   // clamped: the ragged group re-reads the row's last 16 B
            xr[u] = ((const u32x4_t *)p.xq)[min(tid + u * 64 * NW, (K >> 4) - 1)];
    }
    load_batch(A, 0);
    if constexpr (STREAM && PRO == PRO_INT8) {
        if (nb > 1) load_batch(B, 1);
    }
    // RoPE pair of this thread's row at the position (q and k rows), issued
    // as soon as the position is back; clamped so the load stays in the table
    [[maybe_unused]] float2 cs = make_float2(1.0f, 0.0f);
    if constexpr (is_qkv(EPI)) {
        const int d = (n_ep < p.Dq ? n_ep : n_ep - p.Dq) % p.hd;
        const int pc = min(max(pos, 0), p.max_seq - 1);
        if (n_ep < p.Dq + p.Dkv) cs = p.rope[(size_t)pc * (p.hd >> 1) + (d >> 1)];
    }

    // ---- prologue ---------------------------------------------------------
    float in_scale;
    int xsum = 0;
    if constexpr (PRO == PRO_INT8) {
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int i = tid + u * 64 * NW;
            if (i < (K >> 4)) ((u32x4_t *)xq_lds)[i] = xr[u];
        }
        in_scale = p.xscale[0];
        xsum = p.xsum[0];
        lds_barrier();
    } else {
        if constexpr (!EXACT) mask_row<NREG>(K, v, g);
        if (p.gamma) {
            float ss = 0.0f;   // columns past K hold +0 and add exactly nothing
#pragma unroll
            for (int j = 0; j < NREG; ++j) {
                float sq = v[j] * v[j];
                ss = ss + sq;
            }
            const float sum = block256_tree_sum_1b(ss, red);
            const float rms = 1.0f / sqrtf(sum / (float)K + p.eps);  // inverseSqrt
#pragma unroll
            for (int j = 0; j < NREG; ++j) {
                float a = v[j] * rms;
                v[j] = a * g[j];
            }
        }
        float am = 0.0f;
#pragma unroll
        for (int j = 0; j < NREG; ++j) am = fmaxf(am, fabsf(v[j]));
        am = wave_nonneg_max_dpp(am);
        if (lane == 0) wmax[w] = am;
        lds_barrier();
        am = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        in_scale = am == 0.0f ? 1.0f : am / 127.0f;   // sh/quantize.wgsl:59
        const float inv = am == 0.0f ? 0.0f : 127.0f / am;  // :68
        int sq = 0;
        int qv[NREG];
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            const int col = tid + 256 * j;
            qv[j] = quant_one(v[j], inv);
            if (EXACT || col < K) {
                xq_lds[col] = (int8_t)qv[j];
                sq += qv[j];
            }
        }
        sq = wave_isum_dpp(sq);
        if (lane == 0) wq[w] = sq;
        if (tile0 == 0 && p.xq_out) {   // parity checks only
#pragma unroll
            for (int j = 0; j < NREG; ++j)
                if (EXACT || tid + 256 * j < K) p.xq_out[tid + 256 * j] = (int8_t)qv[j];
            if (tid == 0 && p.xscale_out) p.xscale_out[0] = in_scale;
        }
        lds_barrier();   // the int8 vector is complete
    }

    // ---- main loop: chunks past K multiply zero codes -----------------------
    CodeAcc acc[TT];
    auto mac_batch = [&](const uint4 (&src)[TT][PF], int b) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int kc = 4 * NW * (b * PF + u) + 4 * w + c;
            const int kcl = min(kc, KC - 1);
            const int xo = (kcl >> 1) * 128 + (kcl & 1) * 16;
            const int4 x0 = *(const int4 *)(xq_lds + xo);
            const int4 x1 = *(const int4 *)(xq_lds + xo + 32);
            const int4 x2 = *(const int4 *)(xq_lds + xo + 64);
            const int4 x3 = *(const int4 *)(xq_lds + xo + 96);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const uint4 wv = kc < KC ? src[t][u] : make_uint4(0, 0, 0, 0);
                acc[t].add(wv.x, x0.x, x1.x, x2.x, x3.x);
                acc[t].add(wv.y, x0.y, x1.y, x2.y, x3.y);
                acc[t].add(wv.z, x0.z, x1.z, x2.z, x3.z);
                acc[t].add(wv.w, x0.w, x1.w, x2.w, x3.w);
            }
        }
    };
    if constexpr (!STREAM) {   // the launcher picks one batch only when it covers the range
        mac_batch(A, 0);
    } else if constexpr (PRO == PRO_INT8) {   // B already holds batch 1
        int b = 0;
        for (; b + 2 < nb; b += 2) {
            mac_batch(A, b);
            load_batch(A, b + 2);
            mac_batch(B, b + 1);
            if (b + 3 < nb) load_batch(B, b + 3);
        }
        if (b + 1 < nb) {
            mac_batch(A, b);
            mac_batch(B, b + 1);
        } else {
            mac_batch(A, b);
        }
    } else {
        int b = 0;
        for (; b + 2 < nb; b += 2) {
            load_batch(B, b + 1);
            mac_batch(A, b);
            load_batch(A, b + 2);
            mac_batch(B, b + 1);
        }
        if (b + 1 < nb) {
            load_batch(B, b + 1);
            mac_batch(A, b);
            mac_batch(B, b + 1);
        } else {
            mac_batch(A, b);
        }
    }

    // ---- reduction: 4 NW partials per row (4 lanes x NW waves) through LDS --
#pragma unroll
    for (int t = 0; t < TT; ++t) wpart[t * 64 * NW + tid] = acc[t].codes();
    lds_barrier();
    if (tid >= 16 * TT) return;
    int a = 0;
#pragma unroll
    for (int k = 0; k < 4 * NW; ++k) a += wpart[(tid >> 4) * 64 * NW + k * 16 + r];
    if constexpr (PRO == PRO_QUANT) xsum = wq[0] + wq[1] + wq[2] + wq[3];
    a -= xsum;
    const int n = n_ep;   // == tile0 * 16 + tid here
    if (p.acc_out) p.acc_out[n] = a;
    // sh/ternary_gemv.wgsl:94-95: (f32(acc) * scales[row]) * input_scale
    float yv = (float)a * ws_ep;
    yv = yv * in_scale;

    if constexpr (EPI == EPI_STORE) {
        p.y[n] = yv;
    } else if constexpr (EPI == EPI_RESID) {
        p.y[n] = resid + yv;   // rs/nn/transformer.rs:157 add(input, out)
    } else if constexpr (EPI == EPI_GATEUP) {
        // fused rows interleave gate (even) and up (odd): rs/nn/ffn.rs:60-80
        const float other = __shfl_xor(yv, 1, 64);
        if ((n & 1) == 0) {
            float gt = fmaxf(0.0f, yv);   // sh/activation.wgsl:32-33
            gt = gt * gt;
            p.y[n >> 1] = gt * other;     // sh/elementwise.wgsl:32
        }
    } else {  // EPI_QKV, EPI_QKV32
        if (pos < 0 || pos >= p.max_seq) return;  // host checks too; never write out of range
        const float other = __shfl_xor(yv, 1, 64);
        const int Dk = p.Dq + p.Dkv;
        float outv = yv;
        if (n < Dk) {  // q or k: RoPE on the interleaved pair (2i, 2i+1)
            if ((n & 1) == 0) {
                float a0 = yv * cs.x, a1 = other * cs.y;
                outv = a0 - a1;
            } else {
                float a0 = other * cs.y, a1 = yv * cs.x;
                outv = a0 + a1;
            }
        }
        if (n < p.Dq) {
            p.q_out[n] = outv;
        } else {
            const int j = n < Dk ? n - p.Dq : n - Dk;
            const int head = j / p.hd, d = j % p.hd;
            const size_t at = ((size_t)head * p.max_seq + pos) * p.hd + d;
            void *cache = n < Dk ? p.kcache : p.vcache;
            if constexpr (EPI == EPI_QKV32) {
                ((float *)cache)[at] = outv;
            } else {
                const uint16_t bits = f32_to_f16_bits(outv);
                ((uint16_t *)cache)[at] = bits;
                if (n >= Dk && p.vcache8)
                    p.vcache8[(size_t)head * v8_head_elems(p.max_seq, p.hd) +
                              v8_index(pos, d, p.hd)] = bits;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row-wise (optional RMSNorm) + quantize for several tokens (prefill):
// one workgroup per token row, writes int8 X, per-row scale and sum(q).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void norm_quant_rows_kernel(
    const float *__restrict__ x, const float *__restrict__ gamma, float eps, int D,
    int8_t *__restrict__ xq, float *__restrict__ scales, int *__restrict__ sums) {
    extern __shared__ __align__(16) int8_t smem[];
    int8_t *q_lds = smem;
    float *red = (float *)(smem + ((D + 15) & ~15));
    int *wq = (int *)(red + 324);
    const int row = blockIdx.x;
    float v[kMaxNormReg], g[kMaxNormReg];
    load_row<kMaxNormReg>(x + (size_t)row * D, gamma, D, v, g);
    const float scale = norm_quant_regs<kMaxNormReg>(v, g, gamma != nullptr, eps, D, q_lds, red, wq);
    lds_barrier();
    for (int i = threadIdx.x; i < (D >> 4); i += 256)
        ((int4 *)(xq + (size_t)row * D))[i] = ((const int4 *)q_lds)[i];
    if (threadIdx.x == 0) {
        scales[row] = scale;
        if (sums) sums[row] = wq[0] + wq[1] + wq[2] + wq[3];
    }
}

// ---------------------------------------------------------------------------
// Same row transform, writing the token-tiled int8 layout the MFMA GEMM reads:
// [ceil16(n_tok)/16][K/256 stages][4 planes g][4 chunks c][16 tokens][16 B],
// the 16 B of (g, chunk kc = 4*stage + c) holding k = (kc/2)*128 + g*32 +
// (kc%2)*16 + 0..15.  Rows past n_tok (padding to 16) are zeros with scale 1
// and sum 0.  A workgroup takes kTiledRows consecutive rows, one per
// 256-thread group (each in the shaders' 256-thread order).  One row per
// workgroup: a row of 6912 holds 127 VGPRs per thread, so four one-row
// workgroups fit on a CU where one two-row workgroup did (two rows made the
// stores 32-byte runs of 2 tokens, but 2048 x 6912 took 22.0 against 17.1
// us, 2048 x 2560 7.2 against 6.9).  The 16 / kTiledRows workgroups of a
// 16-token tile are blockIdx values congruent mod 8, which the dispatcher
// places on one XCD, so each 128-byte line of the tile is completed in one
// L2: workgroup b runs row group (b / 8) % WPT of tile (b / (8 WPT)) * 8 +
// b % 8, WPT = 16 / kTiledRows (grid: 8 WPT per 8 tiles; those past the
// last tile exit).
// ---------------------------------------------------------------------------
constexpr int kTiledRows = 1;
constexpr int kTiledWpt = 16 / kTiledRows;   // workgroups per 16-token tile

template <int NREG>   // >= D / 256 values per thread (the row's loads)
__global__ __launch_bounds__(256 * kTiledRows) void quantize_rows_tiled_kernel(
    const float *__restrict__ x, const float *__restrict__ gamma, float eps, int D, int n_tok,
    uint4 *__restrict__ Xt, float *__restrict__ scales, int *__restrict__ sums) {
    extern __shared__ __align__(16) int8_t smem[];
    const int grp = threadIdx.x >> 8, tl = threadIdx.x & 255;
    const int dpad = (D + 15) & ~15;
    int8_t *q_lds = smem + grp * dpad;
    float *red = (float *)(smem + kTiledRows * dpad) + grp * 328;
    int *wq = (int *)(red + 324);
    const int b = blockIdx.x, tile = b / (8 * kTiledWpt) * 8 + (b & 7);
    const int r0 = (b >> 3) % kTiledWpt * kTiledRows;
    if (tile * 16 >= n_tok) return;   // whole workgroup: past the last 16-token tile
    const int row = tile * 16 + r0 + grp;
    float scale = 1.0f;
    if (row < n_tok) {
        float v[NREG], g[NREG];
        load_row<NREG>(x + (size_t)row * D, gamma, D, v, g);
        scale = norm_quant_regs<NREG>(v, g, gamma != nullptr, eps, D, q_lds, red, wq);
    } else {
        // padding rows: the group still meets the row path's barriers (one in
        // the norm's tree sum, one for the absmax)
        for (int i = tl; i < (D >> 4); i += 256) ((int4 *)q_lds)[i] = make_int4(0, 0, 0, 0);
        if (gamma != nullptr) (void)block256_tree_sum_1b(0.0f, red);
        lds_barrier();
        if (tl < 4) wq[tl] = 0;
    }
    lds_barrier();
    const int KC = D >> 6;
    // unit i: row group i % kTiledRows, plane (i / kTiledRows) % 4, chunk
    // i / (4 kTiledRows)
    for (int i = threadIdx.x; i < KC * 4 * kTiledRows; i += 256 * kTiledRows) {
        const int rr = i % kTiledRows, gp = (i / kTiledRows) & 3, kc = i / (4 * kTiledRows);
        const int src = (kc >> 1) * 128 + gp * 32 + (kc & 1) * 16;
        Xt[(size_t)tile * KC * 64 + ((kc >> 2) * 4 + gp) * 64 + (kc & 3) * 16 + r0 + rr] =
            *(const uint4 *)(smem + rr * dpad + src);
    }
    if (tl == 0) {
        scales[row] = scale;
        sums[row] = wq[0] + wq[1] + wq[2] + wq[3];
    }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
template <int PRO, int EPI, int NREG, int PF, bool EXACT, int TT = 1, int NW = 4, bool STREAM = PF == 4>
static int launch_n(const GemvParams &p, hipStream_t s) {
    const size_t sm = gemv_smem(p.K, TT, NW);
    if (sm > 64 * 1024 &&
        allow_dynamic_lds((const void *)gemv_kernel<PRO, EPI, NREG, PF, EXACT, TT, NW, STREAM>))
        return -1;
    hipLaunchKernelGGL((gemv_kernel<PRO, EPI, NREG, PF, EXACT, TT, NW, STREAM>),
                       dim3(p.N / (16 * TT)), dim3(64 * NW), sm, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

// NREG = ceil(K/256) bucket for PRO_QUANT (EXACT when K == 256 * NREG), all of
// a lane's weight chunks in one batch.  PRO_INT8: PF from the chunks per
// lane; past 3 chunks per lane, 8 waves stream 1-chunk batches double-buffered.
// Grids over ~3 workgroups per CU take 4 tiles per workgroup.
template <int PRO, int EPI>
static int launch(const GemvParams &p, hipStream_t s) {
    const int KC = p.K >> 6;
    const int cpl = (((((KC + 3) >> 2) + 1) & ~1) + 3) >> 2;
    if constexpr (PRO == PRO_INT8) {
        // one batch of 1 or 3 chunks per lane: K <= 3072, one activation group
        // per thread (256 threads)
        if (cpl <= 1) return launch_n<PRO, EPI, 1, 1, false>(p, s);
        if (cpl <= 3) return launch_n<PRO, EPI, 1, 3, false>(p, s);
        // NREG: the activation row's 16-byte groups per thread (512 threads)
        const int xu = ((p.K >> 4) + 511) / 512;
        if (xu <= 1) return launch_n<PRO, EPI, 1, 1, false, 1, 8, true>(p, s);
        if (xu <= 2) return launch_n<PRO, EPI, 2, 1, false, 1, 8, true>(p, s);
        if (xu <= 4) return launch_n<PRO, EPI, 4, 1, false, 1, 8, true>(p, s);
        return launch_n<PRO, EPI, 8, 1, false, 1, 8, true>(p, s);
    } else {
        if (p.K <= 1024) return launch_n<PRO, EPI, 4, 1, false>(p, s);
        if (p.K == 2560) {
            if (p.N >= 8192 && p.N % 64 == 0) return launch_n<PRO, EPI, 10, 3, true, 4>(p, s);
            return launch_n<PRO, EPI, 10, 3, true>(p, s);
        }
        if (p.K <= 2560) return launch_n<PRO, EPI, 10, 3, false>(p, s);
        if (p.K == 6912) return launch_n<PRO, EPI, 27, 7, true>(p, s);
        return launch_n<PRO, EPI, kMaxNormReg, 7, false>(p, s);
    }
}

static int check_shape(int N, int K, bool norm) {
    OXB_REQUIRE(N > 0 && N % 16 == 0, "ternary GEMV: out_dim %d must be a positive multiple of 16", N);
    OXB_REQUIRE(K > 0 && K % 128 == 0, "ternary GEMV: in_dim %d must be a positive multiple of 128", K);
    OXB_REQUIRE(K <= 65536, "ternary GEMV: in_dim %d exceeds 65536", K);
    OXB_REQUIRE(!norm || K <= 256 * kMaxNormReg,
                "ternary GEMV: fused norm/quantize supports in_dim <= %d (got %d)",
                256 * kMaxNormReg, K);
    return 0;
}

}  // namespace oxb

using namespace oxb;

#define OXB_STREAM hipStream_t stream = (hipStream_t)stream_

extern "C" int oxb_gemv_i8(const void *W_tiled, const int8_t *xq, const float *xscale,
                           const int *xsum, const float *wscale, int N, int K, float *y,
                           int32_t *acc_out, void *stream_) {
    OXB_STREAM;
    if (check_shape(N, K, false)) return -1;
    GemvParams p{};
    p.W = (const uint4 *)W_tiled;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.xq = xq;
    p.xscale = xscale;
    p.xsum = xsum;
    p.y = y;
    p.acc_out = acc_out;
    return launch<PRO_INT8, EPI_STORE>(p, stream);
}

extern "C" int oxb_bitlinear_gemv(const void *W_tiled, const float *x, const float *gamma,
                                  float eps, const float *wscale, int N, int K, float *y,
                                  int residual, int32_t *acc_out, int8_t *xq_out,
                                  float *xscale_out, void *stream_) {
    OXB_STREAM;
    if (check_shape(N, K, true)) return -1;
    GemvParams p{};
    p.W = (const uint4 *)W_tiled;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.x = x;
    p.gamma = gamma;
    p.eps = eps;
    p.y = y;
    p.acc_out = acc_out;
    p.xq_out = xq_out;
    p.xscale_out = xscale_out;
    return residual ? launch<PRO_QUANT, EPI_RESID>(p, stream)
                    : launch<PRO_QUANT, EPI_STORE>(p, stream);
}

extern "C" int oxb_bitlinear_gateup(const void *W_tiled, const float *x, const float *gamma,
                                    float eps, const float *wscale, int N2, int K, float *h,
                                    void *stream_) {
    OXB_STREAM;
    if (check_shape(N2, K, true)) return -1;
    GemvParams p{};
    p.W = (const uint4 *)W_tiled;
    p.wscale = wscale;
    p.N = N2;
    p.K = K;
    p.x = x;
    p.gamma = gamma;
    p.eps = eps;
    p.y = h;
    return launch<PRO_QUANT, EPI_GATEUP>(p, stream);
}

namespace oxb {
int bitlinear_qkv(const void *W_tiled, const float *x, const float *gamma, float eps,
                  const float *wscale, int Dq, int Dkv, int hd, int K, float *q_out, void *kcache,
                  void *vcache, bool kv_f32, int max_seq, const float *rope_cs, const int *pos,
                  void *stream_, uint16_t *vcache8) {
    OXB_STREAM;
    const int N = Dq + 2 * Dkv;
    if (check_shape(N, K, true)) return -1;
    OXB_REQUIRE(Dq % hd == 0 && Dkv % hd == 0 && hd % 16 == 0 && Dq % 16 == 0,
                "qkv: head_dim %d must divide Dq %d and Dkv %d", hd, Dq, Dkv);
    GemvParams p{};
    p.W = (const uint4 *)W_tiled;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.x = x;
    p.gamma = gamma;
    p.eps = eps;
    p.q_out = q_out;
    p.kcache = kcache;
    p.vcache = vcache;
    p.vcache8 = kv_f32 ? nullptr : vcache8;
    p.rope = (const float2 *)rope_cs;
    p.pos = pos;
    p.Dq = Dq;
    p.Dkv = Dkv;
    p.hd = hd;
    p.max_seq = max_seq;
    return kv_f32 ? launch<PRO_QUANT, EPI_QKV32>(p, stream) : launch<PRO_QUANT, EPI_QKV>(p, stream);
}
}  // namespace oxb

extern "C" int oxb_bitlinear_qkv(const void *W_tiled, const float *x, const float *gamma,
                                 float eps, const float *wscale, int Dq, int Dkv, int hd, int K,
                                 float *q_out, uint16_t *kcache, uint16_t *vcache, int max_seq,
                                 const float *rope_cs, const int *pos, void *stream_) {
    return oxb::bitlinear_qkv(W_tiled, x, gamma, eps, wscale, Dq, Dkv, hd, K, q_out, kcache,
                              vcache, false, max_seq, rope_cs, pos, stream_);
}

extern "C" int oxb_norm_quant_rows(const float *x, const float *gamma, float eps, int n_rows,
                                   int D, int8_t *xq, float *scales, int *sums,
                                   void *stream_) {
    OXB_STREAM;
    OXB_REQUIRE(D > 0 && D % 16 == 0 && D <= 256 * kMaxNormReg,
                "norm_quant_rows: D %d must be a multiple of 16 and <= %d", D, 256 * kMaxNormReg);
    OXB_REQUIRE(n_rows > 0, "norm_quant_rows: n_rows %d", n_rows);
    const size_t sm = (size_t)((D + 15) & ~15) + 324 * 4 + 16 + 16;
    hipLaunchKernelGGL(norm_quant_rows_kernel, dim3(n_rows), dim3(256), sm, stream, x, gamma,
                       eps, D, xq, scales, sums);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_quantize_rows_tiled(const float *x, const float *gamma, float eps, int n_tok,
                                       int D, void *Xt, float *scales, int *sums, void *stream_) {
    OXB_STREAM;
    OXB_REQUIRE(D > 0 && D % 256 == 0 && D <= 256 * kMaxNormReg,
                "quantize_rows_tiled: D %d must be a multiple of 256 and <= %d", D, 256 * kMaxNormReg);
    OXB_REQUIRE(n_tok > 0, "quantize_rows_tiled: n_tok %d", n_tok);
    const int grid = (n_tok + 127) / 128 * 8 * kTiledWpt;   // 8 tiles of 16 tokens per 8 WPT
    const size_t sm = (size_t)kTiledRows * (((D + 15) & ~15) + 328 * 4);
    // loads per thread: the row length's bucket (the model's 2560 and 6912 exactly)
    const int nr = D / 256;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(grid), dim3(256 * kTiledRows), sm, stream, x,
                           gamma, eps, D, n_tok, (uint4 *)Xt, scales, sums);
    };
    if (nr <= 4) go(quantize_rows_tiled_kernel<4>);
    else if (nr <= 10) go(quantize_rows_tiled_kernel<10>);
    else if (nr <= 16) go(quantize_rows_tiled_kernel<16>);
    else if (nr <= 27) go(quantize_rows_tiled_kernel<27>);
    else go(quantize_rows_tiled_kernel<kMaxNormReg>);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}
