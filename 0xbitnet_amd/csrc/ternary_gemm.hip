// Prefill ternary GEMM on int8 MFMA for gfx950.
//
// Reference: shaders/ternary_gemm.wgsl:40-136 (64x64 tile, scalar i32 MACs,
// Y[n*M+m] = f32(acc) * (scales[m] * input_scales[n])), dispatched by
// nn/bitlinear.rs:207-247; epilogues fuse nn/ffn.rs:60-80 (ReLU^2 gate),
// nn/transformer.rs:157 (residual), nn/attention.rs:97-107,127-184 (RoPE +
// cache append).
//
// MFMA mapping (v_mfma_i32_16x16x64_i8, A = 16x64, B = 64x16, C = 16x16):
//   A = weight codes of a 16-row tile: lane l supplies row l%16; its 16
//       bytes are one bit plane g of the chunk (row, kc = 4s + l/16), i.e.
//       weights k = (kc/2)*128 + g*32 + (kc%2)*16 + 0..15 as codes 0..2.
//   B = int8 activations: lane l supplies token l%16, the same 16 k values,
//       read from the token-tiled activation layout (below).
//   C: lane l holds rows 4*(l/16) .. +3 (features) of column l%16 (token).
// Integer accumulation is exact, so any consistent k order gives the
// reference's int32 accumulator: acc = C(codes) - sum_k x[t][k].
//
// Token-tiled activation layout (written by oxb_quantize_rows_tiled):
//   [n_tok/16 tiles][KC][16 tokens][64 B], 64 B = planes g = 0..3 x 16 B of
//   x[t][(kc/2)*128 + g*32 + (kc%2)*16 + 0..15].
#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

typedef int v4i __attribute__((ext_vector_type(4)));

enum GemmEpi { GE_STORE = 0, GE_RESID = 1, GE_GATEUP = 2, GE_QKV = 3 };

struct GemmParams {
    const uint4 *W;        // tiled weights
    const uint4 *X;        // token-tiled int8 activations
    const float *xscale;   // [n_tok]
    const int *xsum;       // [n_tok]
    const float *wscale;   // [N]
    int N, K, n_tok;
    float *Y;              // [n_tok][N] (GATEUP: [n_tok][N/2])
    int32_t *acc_out;      // optional [n_tok][N]
    // QKV
    float *q_out;          // [n_tok][Dq]
    uint16_t *kcache, *vcache;
    const float2 *rope;
    int Dq, Dkv, hd, max_seq, pos0;
    // optional: token t is at position tok_pos[t] of its own cache, which
    // starts kv_tok_stride elements after token t-1's (batched decode)
    const int *tok_pos;
    int tok_pos_stride;    // ints between consecutive tokens' positions
    size_t kv_tok_stride;
    // 1: one-token GEMV rounding (f32(acc) * ws) * is (sh/ternary_gemv.wgsl:94-95),
    // for rows that are independent single-token steps (batched decode)
    int gemv_order;
};

__device__ inline v4i plane(uint4 w, int g) {
    const int sh = 6 - 2 * g;
    v4i a;
    a.x = (int)((w.x >> sh) & 0x03030303u);
    a.y = (int)((w.y >> sh) & 0x03030303u);
    a.z = (int)((w.z >> sh) & 0x03030303u);
    a.w = (int)((w.w >> sh) & 0x03030303u);
    return a;
}

__device__ inline v4i as_v4i(uint4 u) {
    v4i a;
    a.x = (int)u.x; a.y = (int)u.y; a.z = (int)u.z; a.w = (int)u.w;
    return a;
}

// Epilogue for one lane's 4 accumulators: features n0 .. n0+3 of token t.
template <int EPI>
__device__ inline void gemm_store(const GemmParams &p, const v4i &c, int t, int n0) {
    const int xs = p.xsum[t];
    const float is = p.xscale[t];
    float y[4];
    int32_t a[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        a[v] = c[v] - xs;
        if (p.gemv_order) {
            y[v] = (float)a[v] * p.wscale[n0 + v];
            y[v] = y[v] * is;
        } else {
            // shaders/ternary_gemm.wgsl:132-133: f32(acc) * (w_scale * in_scale)
            const float sc = p.wscale[n0 + v] * is;
            y[v] = (float)a[v] * sc;
        }
    }
    if (p.acc_out) *(int4 *)(p.acc_out + (size_t)t * p.N + n0) = make_int4(a[0], a[1], a[2], a[3]);
    if constexpr (EPI == GE_STORE) {
        *(float4 *)(p.Y + (size_t)t * p.N + n0) = make_float4(y[0], y[1], y[2], y[3]);
    } else if constexpr (EPI == GE_RESID) {
        float4 *dst = (float4 *)(p.Y + (size_t)t * p.N + n0);
        float4 o = *dst;
        o.x = o.x + y[0]; o.y = o.y + y[1]; o.z = o.z + y[2]; o.w = o.w + y[3];
        *dst = o;
    } else if constexpr (EPI == GE_GATEUP) {
        float g0 = fmaxf(0.0f, y[0]), g1 = fmaxf(0.0f, y[2]);
        g0 = g0 * g0;
        g1 = g1 * g1;
        *(float2 *)(p.Y + (size_t)t * (p.N >> 1) + (n0 >> 1)) = make_float2(g0 * y[1], g1 * y[3]);
    } else {  // GE_QKV
        const int pos = p.tok_pos ? p.tok_pos[(size_t)t * p.tok_pos_stride] : p.pos0 + t;
        if (pos < 0 || pos >= p.max_seq) return;   // host checks too; never write out of range
        const int Dk = p.Dq + p.Dkv;
        float o[4] = {y[0], y[1], y[2], y[3]};
        if (n0 < Dk) {
            const int d0 = (n0 < p.Dq ? n0 : n0 - p.Dq) % p.hd;
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const float2 cs = p.rope[(size_t)pos * (p.hd >> 1) + (d0 >> 1) + pr];
                const float x0 = y[2 * pr], x1 = y[2 * pr + 1];
                float a0 = x0 * cs.x, a1 = x1 * cs.y;
                float b0 = x0 * cs.y, b1 = x1 * cs.x;
                o[2 * pr] = a0 - a1;
                o[2 * pr + 1] = b0 + b1;
            }
        }
        if (n0 < p.Dq) {
            *(float4 *)(p.q_out + (size_t)t * p.Dq + n0) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
            const int j = n0 < Dk ? n0 - p.Dq : n0 - Dk;
            const int head = j / p.hd, d = j % p.hd;
            uint16_t *cache = (n0 < Dk ? p.kcache : p.vcache) + (p.tok_pos ? t * p.kv_tok_stride : 0);
            uint16_t *dst = cache + ((size_t)head * p.max_seq + pos) * p.hd + d;
#pragma unroll
            for (int v = 0; v < 4; ++v) dst[v] = __half_as_ushort(__float2half_rn(o[v]));
        }
    }
}

// Workgroup tile: 64 features x 64 tokens; 4 waves in a 2x2 grid, each wave
// 2 feature tiles x 2 token tiles of 16x16.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int KC = p.K >> 6;
    const int f0 = blockIdx.x * 64 + (w & 1) * 32;
    const int tt0 = blockIdx.y * 4 + (w >> 1) * 2;   // first token tile of this wave
    const int ntt = (p.n_tok + 15) >> 4;
    if (f0 >= p.N || tt0 >= ntt) return;
    const bool t1ok = tt0 + 1 < ntt;
    const bool f1ok = f0 + 16 < p.N;

    v4i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const uint4 *Wt0 = p.W + (size_t)(f0 >> 4) * KC * 16;
    const uint4 *Wt1 = p.W + (size_t)((f1ok ? f0 + 16 : f0) >> 4) * KC * 16;
    const uint4 *Xt0 = p.X + ((size_t)tt0 * KC * 16) * 4;
    const uint4 *Xt1 = p.X + ((size_t)(t1ok ? tt0 + 1 : tt0) * KC * 16) * 4;

    const int steps = KC >> 2;
    uint4 wa[2], xa[2][4];
    auto load = [&](int s, uint4 (&wv)[2], uint4 (&xv)[2][4]) {
        const int kc = 4 * s + q;
        wv[0] = load_nt(Wt0 + (size_t)kc * 16 + r);
        wv[1] = load_nt(Wt1 + (size_t)kc * 16 + r);
        const uint4 *x0 = Xt0 + ((size_t)kc * 16 + r) * 4;
        const uint4 *x1 = Xt1 + ((size_t)kc * 16 + r) * 4;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            xv[0][g] = x0[g];
            xv[1][g] = x1[g];
        }
    };
    load(0, wa, xa);
    for (int s = 0; s < steps; ++s) {
        uint4 wb[2], xb[2][4];
        if (s + 1 < steps) load(s + 1, wb, xb);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const v4i a0 = plane(wa[0], g), a1 = plane(wa[1], g);
            const v4i b0 = as_v4i(xa[0][g]), b1 = as_v4i(xa[1][g]);
            acc[0][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (s + 1 < steps) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                wa[i] = wb[i];
#pragma unroll
                for (int g = 0; g < 4; ++g) xa[i][g] = xb[i][g];
            }
        }
    }

    // epilogue: lane holds features n = f0 + ft*16 + 4q + v of token t
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) {
        if (ft == 1 && !f1ok) continue;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            if (tt == 1 && !t1ok) continue;
            const int t = (tt0 + tt) * 16 + r;
            if (t >= p.n_tok) continue;
            gemm_store<EPI>(p, acc[ft][tt], t, f0 + ft * 16 + 4 * q);
        }
    }
}


// ---------------------------------------------------------------------------
// LDS-staged GEMM for n_tok > 64.  Workgroup tile: 32*FW features x 32*TW
// tokens; 4 waves in a 2x2 grid, each FW x TW MFMA tiles of 16x16, so every
// A operand (a weight plane) feeds TW MFMAs and every B operand FW.  K runs
// in stages of 4 chunks (256 k), double-buffered in LDS; the weights stay
// 2-bit in LDS and are unpacked into A operands in registers.
//   W stage: [32FW rows][4 chunks] x 16 B; chunk c of row f at slot
//            4f + (c ^ (f/4 % 4)): 16 lanes reading (row r, chunk q) and 16
//            lanes writing (chunk c, row r) both hit 16 distinct bank groups.
//   X stage: [32TW tokens][16 units] x 16 B, unit u = 4c + g (chunk c, plane
//            g); unit u of token t at slot 16t + (u ^ (5t % 16)): readers
//            (tokens r = 0..15, one unit) and writers (tokens r = 0..3 x 4
//            planes) both hit 16 distinct bank groups.
// Token tiles past the activation buffer are clamped to its last tile; their
// accumulators are never stored.
// ---------------------------------------------------------------------------
// Staging of one stage: this thread's WPT weight and XPT activation units
// (global offsets of stage 0 in uint4; stage st is 64 uint4 of W and 256 of
// X further) into registers, and from registers into its LDS slots.
template <int WPT, int XPT>
__device__ __forceinline__ void gemm_stage_load(u32x4_t (&rw)[WPT], u32x4_t (&rx)[XPT],
                                                const uint4 *W, const uint4 *X,
                                                const size_t (&wsrc)[WPT],
                                                const size_t (&xsrc)[XPT], int st) {
#pragma unroll
    for (int k = 0; k < WPT; ++k)
        rw[k] = __builtin_nontemporal_load((const u32x4_t *)(W + wsrc[k] + (size_t)st * 64));
#pragma unroll
    for (int k = 0; k < XPT; ++k) rx[k] = *(const u32x4_t *)(X + xsrc[k] + (size_t)st * 256);
}

template <int WPT, int XPT>
__device__ __forceinline__ void gemm_stage_store(const u32x4_t (&rw)[WPT],
                                                 const u32x4_t (&rx)[XPT], uint4 *swb,
                                                 uint4 *sxb, const int (&wdst)[WPT],
                                                 const int (&xdst)[XPT]) {
#pragma unroll
    for (int k = 0; k < WPT; ++k) *(u32x4_t *)(swb + wdst[k]) = rw[k];
#pragma unroll
    for (int k = 0; k < XPT; ++k) *(u32x4_t *)(sxb + xdst[k]) = rx[k];
}

// One LDS stage (4 chunks) of a wave's FW x TW tiles: per plane g, FW A
// operands unpacked from the 2-bit weights and TW B operands, FW*TW MFMAs.
// Slots follow the swizzles of gemm_lds_kernel's stage layouts.
template <int FW, int TW>
__device__ __forceinline__ void gemm_mma_stage(v4i (&acc)[FW][TW], const uint4 *swb,
                                               const uint4 *sxb, int wf, int wt, int r, int q) {
    uint4 wu[FW];
#pragma unroll
    for (int i = 0; i < FW; ++i) {
        const int f = (wf + i) * 16 + r;
        wu[i] = swb[4 * f + (q ^ ((f >> 2) & 3))];
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        v4i a[FW];
#pragma unroll
        for (int i = 0; i < FW; ++i) a[i] = plane(wu[i], g);
#pragma unroll
        for (int j = 0; j < TW; ++j) {
            const int t = (wt + j) * 16 + r;
            const v4i bv = as_v4i(sxb[16 * t + (((q << 2) | g) ^ ((5 * t) & 15))]);
#pragma unroll
            for (int i = 0; i < FW; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], bv, acc[i][j], 0, 0, 0);
        }
    }
}

template <int EPI, int FW, int TW>
__global__ __launch_bounds__(256, 2) void gemm_lds_kernel(GemmParams p) {
    constexpr int FT = 32 * FW, TK = 32 * TW;      // features, tokens per workgroup
    constexpr int WU = FT * 4, XU = TK * 16;       // 16-byte units per stage
    constexpr int WPT = WU / 256, XPT = XU / 256;  // per thread
    __shared__ uint4 sw[2][WU];
    __shared__ uint4 sx[2][XU];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int KC = p.K >> 6, steps = KC >> 2;
    const int ftile0 = blockIdx.x * (FT / 16), ttile0 = blockIdx.y * (TK / 16);
    const int ntt = (p.n_tok + 15) >> 4;
    const int wf = (w & 1) * FW, wt = (w >> 1) * TW;   // this wave's local tiles

    // this thread's staging units: W unit tid + 256k is (local tile fi, chunk
    // c, row rr); X unit tid + 256k is (local tile ti, chunk c, token rr, plane g)
    size_t wsrc[WPT], xsrc[XPT];   // global offsets of stage 0, in uint4
    int wdst[WPT], xdst[XPT];      // LDS slots
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int i = tid + 256 * k, fi = i >> 6, c = (i >> 4) & 3, rr = i & 15;
        const int f = (fi << 4) | rr;
        wsrc[k] = ((size_t)(ftile0 + fi) * KC + c) * 16 + rr;
        wdst[k] = 4 * f + (c ^ ((f >> 2) & 3));
    }
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        const int i = tid + 256 * k, ti = i >> 8, c = (i >> 6) & 3, rr = (i >> 2) & 15, g = i & 3;
        const int tt = min(ttile0 + ti, ntt - 1), t = (ti << 4) | rr, u = (c << 2) | g;
        xsrc[k] = (((size_t)tt * KC + c) * 16 + rr) * 4 + g;
        xdst[k] = 16 * t + (u ^ ((5 * t) & 15));
    }
    v4i acc[FW][TW];
#pragma unroll
    for (int i = 0; i < FW; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // Two register sets hold stages s+1 and s+2 while stage s is multiplied,
    // so each stage's loads have two stages of MFMA work to arrive.  Loads
    // past the last stage reload the last one (branch-free; never stored).
    u32x4_t aw[WPT], ax[XPT], bw[WPT], bx_[XPT];
    const int last = steps - 1;
    gemm_stage_load(aw, ax, p.W, p.X, wsrc, xsrc, 0);
    gemm_stage_store(aw, ax, sw[0], sx[0], wdst, xdst);
    gemm_stage_load(aw, ax, p.W, p.X, wsrc, xsrc, min(1, last));
    lds_barrier();
    // iteration s: load stage s+2, multiply stage s (buffer s&1), store stage
    // s+1 into the idle buffer (its last reads ended before the previous barrier)
    int s = 0;
    for (; s + 2 <= steps; s += 2) {
        gemm_stage_load(bw, bx_, p.W, p.X, wsrc, xsrc, min(s + 2, last));
        gemm_mma_stage<FW, TW>(acc, sw[0], sx[0], wf, wt, r, q);
        gemm_stage_store(aw, ax, sw[1], sx[1], wdst, xdst);
        lds_barrier();
        gemm_stage_load(aw, ax, p.W, p.X, wsrc, xsrc, min(s + 3, last));
        gemm_mma_stage<FW, TW>(acc, sw[1], sx[1], wf, wt, r, q);
        gemm_stage_store(bw, bx_, sw[0], sx[0], wdst, xdst);
        lds_barrier();
    }
    if (s < steps) gemm_mma_stage<FW, TW>(acc, sw[0], sx[0], wf, wt, r, q);   // odd count: buffer 0

    // epilogue: lane holds features 16 ftile + 4q + v of token 16 ttile + r
#pragma unroll
    for (int i = 0; i < FW; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j) {
            const int t = (ttile0 + wt + j) * 16 + r;
            if (t < p.n_tok) gemm_store<EPI>(p, acc[i][j], t, (ftile0 + wf + i) * 16 + 4 * q);
        }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for n_tok <= 64 (batched decode, small-M sweeps): the GEMV's
// decomposition with MFMA inside.  A workgroup owns TF 16-row feature tiles
// and all TT = ceil(n_tok/16) token tiles; its 4 waves split K (in 4-chunk
// MFMA steps) and meet in LDS, where each wave sums a quarter of the tiles
// (int32, exact) and runs the epilogue.  N/16/TF workgroups keep the chip
// busy where the 64x64 tiling launches too few.
// ---------------------------------------------------------------------------
template <int EPI, int TT, int TF>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmParams p) {
    constexpr int NT = TF * TT;   // 16x16 tiles per wave
    __shared__ v4i red[4][NT][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int KC = p.K >> 6, steps = KC >> 2;
    const int per = (steps + 3) >> 2;
    const int s0 = min(w * per, steps), s1 = min(steps, s0 + per);
    const int ftile0 = blockIdx.x * TF;

    v4i acc[TF][TT];
#pragma unroll
    for (int i = 0; i < TF; ++i)
#pragma unroll
        for (int j = 0; j < TT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    auto load = [&](int s, uint4 (&wv)[TF], uint4 (&xv)[TT][4]) {
        const int kc = 4 * s + q;
#pragma unroll
        for (int f = 0; f < TF; ++f)
            wv[f] = load_nt(p.W + ((size_t)(ftile0 + f) * KC + kc) * 16 + r);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const uint4 *x = p.X + (((size_t)t * KC + kc) * 16 + r) * 4;
#pragma unroll
            for (int g = 0; g < 4; ++g) xv[t][g] = x[g];
        }
    };
    auto mac = [&](const uint4 (&wv)[TF], const uint4 (&xv)[TT][4]) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int f = 0; f < TF; ++f) {
                const v4i a = plane(wv[f], g);
#pragma unroll
                for (int t = 0; t < TT; ++t)
                    acc[f][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, as_v4i(xv[t][g]), acc[f][t],
                                                                      0, 0, 0);
            }
        }
    };
    if (s0 < s1) {
        uint4 wa[TF], xa[TT][4], wb[TF], xb[TT][4];
        load(s0, wa, xa);
        int s = s0;
        for (; s + 2 < s1; s += 2) {
            load(s + 1, wb, xb);
            mac(wa, xa);
            load(s + 2, wa, xa);
            mac(wb, xb);
        }
        if (s + 1 < s1) {
            load(s + 1, wb, xb);
            mac(wa, xa);
            mac(wb, xb);
        } else {
            mac(wa, xa);
        }
    }
#pragma unroll
    for (int f = 0; f < TF; ++f)
#pragma unroll
        for (int t = 0; t < TT; ++t) red[w][f * TT + t][lane] = acc[f][t];
    lds_barrier();
    const int ntok = p.n_tok;
    for (int i = w; i < NT; i += 4) {
        v4i c = red[0][i][lane];
#pragma unroll
        for (int k = 1; k < 4; ++k) c += red[k][i][lane];
        const int f = i / TT, t = (i % TT) * 16 + r;
        if (t < ntok) gemm_store<EPI>(p, c, t, (ftile0 + f) * 16 + 4 * q);
    }
}

}  // namespace oxb

using namespace oxb;

static int gemm_check(int N, int K, int n_tok) {
    OXB_REQUIRE(N > 0 && N % 32 == 0, "ternary GEMM: out_dim %d must be a multiple of 32", N);
    OXB_REQUIRE(K > 0 && K % 256 == 0, "ternary GEMM: in_dim %d must be a multiple of 256", K);
    OXB_REQUIRE(n_tok > 0, "ternary GEMM: n_tok %d", n_tok);
    return 0;
}

template <int EPI, int TT, int TF>
static int skinny_launch(const GemmParams &p, hipStream_t s) {
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, TT, TF>), dim3(p.N / (16 * TF)), dim3(256), 0, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

template <int EPI, int FW, int TW>
static int lds_launch(const GemmParams &p, hipStream_t s) {
    dim3 grid(p.N / (32 * FW), (p.n_tok + 32 * TW - 1) / (32 * TW));
    hipLaunchKernelGGL((gemm_lds_kernel<EPI, FW, TW>), grid, dim3(256), 0, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

// n_tok <= 64: skinny kernel (2 feature tiles per workgroup once there are
// 3+ token tiles and enough rows, to halve the activation re-reads); else
// the LDS-staged kernel (the 64x64 register-tiled kernel for N % 64 != 0).
template <int EPI>
static int gemm_launch(const GemmParams &p, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    if (p.n_tok <= 64) {
        const int tt = (p.n_tok + 15) >> 4;
        const bool two = tt >= 3 && p.N % 32 == 0 && p.N / 32 >= 256;
        switch (tt) {
            case 1: return skinny_launch<EPI, 1, 1>(p, s);
            case 2: return skinny_launch<EPI, 2, 1>(p, s);
            case 3: return two ? skinny_launch<EPI, 3, 2>(p, s) : skinny_launch<EPI, 3, 1>(p, s);
            default: return two ? skinny_launch<EPI, 4, 2>(p, s) : skinny_launch<EPI, 4, 1>(p, s);
        }
    }
    // LDS-staged tiles: the largest of 128x128, 128x64, 64x128, 64x64 whose
    // grid still gives every CU a workgroup (N a multiple of the tile).
    const int cus = 256;
    auto blocks = [&](int ft, int tk) { return (long)(p.N / ft) * ((p.n_tok + tk - 1) / tk); };
    if (p.N % 128 == 0 && blocks(128, 128) >= cus) return lds_launch<EPI, 4, 4>(p, s);
    if (p.N % 128 == 0 && blocks(128, 64) >= cus) return lds_launch<EPI, 4, 2>(p, s);
    if (p.N % 64 == 0 && blocks(64, 128) >= cus) return lds_launch<EPI, 2, 4>(p, s);
    if (p.N % 64 == 0) return lds_launch<EPI, 2, 2>(p, s);
    dim3 grid((p.N + 63) / 64, (p.n_tok + 63) / 64);
    hipLaunchKernelGGL((gemm_kernel<EPI>), grid, dim3(256), 0, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_gemm_i8(const void *W_tiled, const int8_t *X, const float *xscale,
                           const int *xsum, const float *wscale, int N, int K, int n_tok,
                           float *Y, int32_t *acc_out, int epilogue, void *stream) {
    if (gemm_check(N, K, n_tok)) return -1;
    GemmParams p{};
    p.W = (const uint4 *)W_tiled;
    p.X = (const uint4 *)X;
    p.xscale = xscale;
    p.xsum = xsum;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.n_tok = n_tok;
    p.Y = Y;
    p.acc_out = acc_out;
    switch (epilogue) {
        case GE_STORE: return gemm_launch<GE_STORE>(p, stream);
        case GE_RESID: return gemm_launch<GE_RESID>(p, stream);
        case GE_GATEUP: return gemm_launch<GE_GATEUP>(p, stream);
        default: oxb::set_error("ternary GEMM: epilogue %d unsupported here", epilogue); return -1;
    }
}

extern "C" int oxb_gemm_qkv(const void *W_tiled, const int8_t *X, const float *xscale,
                            const int *xsum, const float *wscale, int Dq, int Dkv, int hd, int K,
                            int n_tok, int pos0, float *q_out, uint16_t *kcache,
                            uint16_t *vcache, int max_seq, const float *rope_cs, void *stream) {
    const int N = Dq + 2 * Dkv;
    if (gemm_check(N, K, n_tok)) return -1;
    OXB_REQUIRE(Dq % 32 == 0 && Dkv % 32 == 0 && hd % 16 == 0, "gemm qkv: bad head split");
    OXB_REQUIRE(pos0 >= 0 && pos0 + n_tok <= max_seq, "gemm qkv: positions exceed max_seq");
    GemmParams p{};
    p.W = (const uint4 *)W_tiled;
    p.X = (const uint4 *)X;
    p.xscale = xscale;
    p.xsum = xsum;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.n_tok = n_tok;
    p.q_out = q_out;
    p.kcache = kcache;
    p.vcache = vcache;
    p.rope = (const float2 *)rope_cs;
    p.Dq = Dq;
    p.Dkv = Dkv;
    p.hd = hd;
    p.max_seq = max_seq;
    p.pos0 = pos0;
    return gemm_launch<GE_QKV>(p, stream);
}

namespace oxb {

int gemm_rows(const void *W, const int8_t *X, const float *xscale, const int *xsum,
              const float *wscale, int N, int K, int n_tok, float *Y, int epilogue,
              bool gemv_order, void *stream) {
    if (gemm_check(N, K, n_tok)) return -1;
    GemmParams p{};
    p.W = (const uint4 *)W;
    p.X = (const uint4 *)X;
    p.xscale = xscale;
    p.xsum = xsum;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.n_tok = n_tok;
    p.Y = Y;
    p.gemv_order = gemv_order ? 1 : 0;
    switch (epilogue) {
        case GE_STORE: return gemm_launch<GE_STORE>(p, stream);
        case GE_RESID: return gemm_launch<GE_RESID>(p, stream);
        case GE_GATEUP: return gemm_launch<GE_GATEUP>(p, stream);
        default: set_error("ternary GEMM: epilogue %d unsupported here", epilogue); return -1;
    }
}

int gemm_qkv_rows(const void *W, const int8_t *X, const float *xscale, const int *xsum,
                  const float *wscale, int Dq, int Dkv, int hd, int K, int n_tok,
                  const int *tok_pos, int tok_pos_stride, size_t kv_tok_stride, float *q_out,
                  uint16_t *kcache, uint16_t *vcache, int max_seq, const float *rope_cs,
                  bool gemv_order, void *stream) {
    const int N = Dq + 2 * Dkv;
    if (gemm_check(N, K, n_tok)) return -1;
    OXB_REQUIRE(Dq % 32 == 0 && Dkv % 32 == 0 && hd % 16 == 0, "gemm qkv: bad head split");
    GemmParams p{};
    p.W = (const uint4 *)W;
    p.X = (const uint4 *)X;
    p.xscale = xscale;
    p.xsum = xsum;
    p.wscale = wscale;
    p.N = N;
    p.K = K;
    p.n_tok = n_tok;
    p.q_out = q_out;
    p.kcache = kcache;
    p.vcache = vcache;
    p.rope = (const float2 *)rope_cs;
    p.Dq = Dq;
    p.Dkv = Dkv;
    p.hd = hd;
    p.max_seq = max_seq;
    p.tok_pos = tok_pos;
    p.tok_pos_stride = tok_pos_stride;
    p.kv_tok_stride = kv_tok_stride;
    p.gemv_order = gemv_order ? 1 : 0;
    return gemm_launch<GE_QKV>(p, stream);
}

}  // namespace oxb
