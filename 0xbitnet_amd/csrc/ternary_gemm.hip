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
//   [n_tok/16 tiles][K/256 stages][4 planes g][4 chunks c][16 tokens][16 B],
//   the 16 B of (g, chunk kc = 4*stage + c, token t) being
//   x[t][(kc/2)*128 + g*32 + (kc%2)*16 + 0..15].  For one plane, the B
//   operands of a stage's four chunks are 1 KB in lane order, so global
//   loads, LDS stores and LDS operand reads are all contiguous per wave.
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
    void *kcache, *vcache;     // f16 bits, or f32 when kv_f32
    uint16_t *vcache8;         // optional (f16): V also in position octets (v8_index)
    size_t kv8_tok_stride;     // tok_pos: elements between consecutive tokens' octet caches
    int kv_f32;
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

// Epilogue inputs, loaded in two groups before any result is stored so that a
// lane's loads are in flight together: per token (xsum, xscale, position) and
// per tile (RESID: the old residual; QKV: the RoPE (cos, sin) of the tile's
// two pairs).  Tokens past n_tok read token n_tok-1's values; their results
// are never stored.
struct EpiTok {
    int xs;
    float is;
    int pos;
};

template <int EPI>
__device__ inline EpiTok epi_tok(const GemmParams &p, int t) {
    const int tc = min(t, p.n_tok - 1);
    EpiTok e;
    e.xs = p.xsum[tc];
    e.is = p.xscale[tc];
    e.pos = 0;
    if constexpr (EPI == GE_QKV)
        e.pos = p.tok_pos ? p.tok_pos[(size_t)tc * p.tok_pos_stride] : p.pos0 + tc;
    return e;
}

template <int EPI>
__device__ inline float4 epi_old(const GemmParams &p, int t, int n0, const EpiTok &e) {
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (EPI == GE_RESID) {
        o = *(const float4 *)(p.Y + (size_t)min(t, p.n_tok - 1) * p.N + n0);
    } else if constexpr (EPI == GE_QKV) {
        if (n0 < p.Dq + p.Dkv && e.pos >= 0 && e.pos < p.max_seq) {
            const int d0 = (n0 < p.Dq ? n0 : n0 - p.Dq) % p.hd;   // multiple of 4
            o = *(const float4 *)(p.rope + (size_t)e.pos * (p.hd >> 1) + (d0 >> 1));
        }
    }
    return o;
}

// Epilogue for one lane's 4 accumulators: features n0 .. n0+3 of token t, with
// ws = wscale[n0 .. n0+3] and the inputs above.
template <int EPI>
__device__ inline void gemm_store(const GemmParams &p, const v4i &c, int t, int n0,
                                  const EpiTok &e, const float4 &ws4, const float4 &old) {
    const float ws[4] = {ws4.x, ws4.y, ws4.z, ws4.w};
    float y[4];
    int32_t a[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        a[v] = c[v] - e.xs;
        if (p.gemv_order) {
            y[v] = (float)a[v] * ws[v];
            y[v] = y[v] * e.is;
        } else {
            // shaders/ternary_gemm.wgsl:132-133: f32(acc) * (w_scale * in_scale)
            const float sc = ws[v] * e.is;
            y[v] = (float)a[v] * sc;
        }
    }
    if (p.acc_out) *(int4 *)(p.acc_out + (size_t)t * p.N + n0) = make_int4(a[0], a[1], a[2], a[3]);
    if constexpr (EPI == GE_STORE) {
        *(float4 *)(p.Y + (size_t)t * p.N + n0) = make_float4(y[0], y[1], y[2], y[3]);
    } else if constexpr (EPI == GE_RESID) {
        *(float4 *)(p.Y + (size_t)t * p.N + n0) =
            make_float4(old.x + y[0], old.y + y[1], old.z + y[2], old.w + y[3]);
    } else if constexpr (EPI == GE_GATEUP) {
        float g0 = fmaxf(0.0f, y[0]), g1 = fmaxf(0.0f, y[2]);
        g0 = g0 * g0;
        g1 = g1 * g1;
        *(float2 *)(p.Y + (size_t)t * (p.N >> 1) + (n0 >> 1)) = make_float2(g0 * y[1], g1 * y[3]);
    } else {  // GE_QKV
        const int pos = e.pos;
        if (pos < 0 || pos >= p.max_seq) return;   // host checks too; never write out of range
        const int Dk = p.Dq + p.Dkv;
        float o[4] = {y[0], y[1], y[2], y[3]};
        if (n0 < Dk) {
            const float2 cs[2] = {make_float2(old.x, old.y), make_float2(old.z, old.w)};
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const float x0 = y[2 * pr], x1 = y[2 * pr + 1];
                float a0 = x0 * cs[pr].x, a1 = x1 * cs[pr].y;
                float b0 = x0 * cs[pr].y, b1 = x1 * cs[pr].x;
                o[2 * pr] = a0 - a1;
                o[2 * pr + 1] = b0 + b1;
            }
        }
        if (n0 < p.Dq) {
            *(float4 *)(p.q_out + (size_t)t * p.Dq + n0) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
            const int j = n0 < Dk ? n0 - p.Dq : n0 - Dk;
            const int head = j / p.hd, d = j % p.hd;
            const size_t at = (p.tok_pos ? t * p.kv_tok_stride : 0) +
                              ((size_t)head * p.max_seq + pos) * p.hd + d;
            void *cache = n0 < Dk ? p.kcache : p.vcache;
            if (p.kv_f32) {
                *(float4 *)((float *)cache + at) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
                uint16_t *dst = (uint16_t *)cache + at;
                uint16_t bits[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) dst[v] = bits[v] = __half_as_ushort(__float2half_rn(o[v]));
                if (n0 >= Dk && p.vcache8) {
                    uint16_t *d8 = p.vcache8 + (p.tok_pos ? t * p.kv8_tok_stride : 0) +
                                   (size_t)head * v8_head_elems(p.max_seq, p.hd);
#pragma unroll
                    for (int v = 0; v < 4; ++v) d8[v8_index(pos, d + v, p.hd)] = bits[v];
                }
            }
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
    const uint4 *Xt0 = p.X + (size_t)tt0 * KC * 64 + q * 16 + r;
    const uint4 *Xt1 = p.X + (size_t)(t1ok ? tt0 + 1 : tt0) * KC * 64 + q * 16 + r;

    const int steps = KC >> 2;
    uint4 wa[2], xa[2][4];
    auto load = [&](int s, uint4 (&wv)[2], uint4 (&xv)[2][4]) {
        const int kc = 4 * s + q;
        wv[0] = load_nt(Wt0 + (size_t)kc * 16 + r);
        wv[1] = load_nt(Wt1 + (size_t)kc * 16 + r);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            xv[0][g] = Xt0[(size_t)(4 * s + g) * 64];
            xv[1][g] = Xt1[(size_t)(4 * s + g) * 64];
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
    const int fn[2] = {f0 + 4 * q, (f1ok ? f0 + 16 : f0) + 4 * q};
    EpiTok e[2];
    float4 ws[2], old[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) e[tt] = epi_tok<EPI>(p, (tt0 + tt) * 16 + r);
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) {
        ws[ft] = *(const float4 *)(p.wscale + fn[ft]);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) old[ft][tt] = epi_old<EPI>(p, (tt0 + tt) * 16 + r, fn[ft], e[tt]);
    }
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) {
        if (ft == 1 && !f1ok) continue;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            if (tt == 1 && !t1ok) continue;
            const int t = (tt0 + tt) * 16 + r;
            if (t >= p.n_tok) continue;
            gemm_store<EPI>(p, acc[ft][tt], t, fn[ft], e[tt], ws[ft], old[ft][tt]);
        }
    }
}


// ---------------------------------------------------------------------------
// LDS-staged GEMM for n_tok > 64, on v_mfma_i32_32x32x32_i8 (A = 32x32,
// B = 32x32, C = 32x32 in 16 registers).  On gfx950 one wave issues this
// MFMA at ~85% of the chip's int8 rate, against ~50% for 16x16x64, so the
// product keeps its rate while the other wave of a SIMD waits on a barrier.
//   A: lane l supplies feature row l%32 of a 32-row tile and 16 codes of
//      chunk 2cp + l/32 of the stage's chunk pair cp, one bit plane g at a
//      time (4 planes per packed 16 B).
//   B: lane l supplies token l%32 of a 32-token tile and the same 16 k.
//   C: lane l holds features 8(v/4) + 4(l/32) + v%4 (v = 0..15) of token l%32.
// Workgroup tile: 32*MF*NWF features x 64*MT tokens; NWF x 2 waves (NWF
// along features), each MF x MT MFMA tiles.  The 256 x 128 tile (NWF = 4,
// 512 threads, one workgroup per CU) stages 40% fewer bytes per output than
// two 128 x 128 workgroups; staging is the largest cost after the MFMAs.  K runs in stages of 4 chunks (256 k), double-buffered
// in LDS; the weights stay 2-bit in LDS and are unpacked in registers.  The
// stage buffers are ordered so that each operand read is one contiguous 1 KB
// in lane order (the ds_read_b128 pattern that runs at full LDS rate on
// gfx950; bank-permuting swizzles measured at half rate):
//   W stage: [2 chunk pairs cp][2MF row pairs][2 chunks h][2 tiles][16 rows]
//   X stage: [4 planes g][2 chunk pairs cp][2MT token pairs][2 chunks h]
//            [2 tiles][16 tokens]   (16 B units)
// Each thread stages the units whose LDS slots are tid + 256k, so the LDS
// writes are contiguous too; their global sources are 256 B runs.  Token
// tiles past the activation buffer are clamped to its last tile; their
// accumulators are never stored.
// ---------------------------------------------------------------------------
typedef int v16i __attribute__((ext_vector_type(16)));

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

template <int WPT, int XPT, int NTH>
__device__ __forceinline__ void gemm_stage_store(const u32x4_t (&rw)[WPT],
                                                 const u32x4_t (&rx)[XPT], uint4 *swb,
                                                 uint4 *sxb, int tid) {
#pragma unroll
    for (int k = 0; k < WPT; ++k) *(u32x4_t *)(swb + tid + NTH * k) = rw[k];
#pragma unroll
    for (int k = 0; k < XPT; ++k) *(u32x4_t *)(sxb + tid + NTH * k) = rx[k];
}

// One LDS stage of a wave's MF x MT tiles (wf, wt: its first row pair and
// token pair in the workgroup; NF, NT: the workgroup's row and token pairs).
template <int MF, int MT, int NF, int NT>
__device__ __forceinline__ void gemm_mma_stage(v16i (&acc)[MF][MT], const uint4 *swb,
                                               const uint4 *sxb, int wf, int wt, int l) {
#pragma unroll
    for (int cp = 0; cp < 2; ++cp) {
        uint4 wu[MF];
#pragma unroll
        for (int i = 0; i < MF; ++i) wu[i] = swb[(cp * NF + wf + i) * 64 + l];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            v4i a[MF];
#pragma unroll
            for (int i = 0; i < MF; ++i) a[i] = plane(wu[i], g);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const v4i bv = as_v4i(sxb[((g * 2 + cp) * NT + wt + j) * 64 + l]);
#pragma unroll
                for (int i = 0; i < MF; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], bv, acc[i][j], 0, 0, 0);
            }
        }
    }
}

// Epilogue of the LDS-staged kernels: register v of tile (i, j) holds feature
// 32(fp) + 8(v/4) + 4(l/32) + v%4 of token 32(tp) + l%32; stored as 4 groups
// of 4 consecutive features, with every input loaded before the first store.
template <int EPI, int MF, int MT>
__device__ __forceinline__ void gemm_lds_epilogue(const GemmParams &p, const v16i (&acc)[MF][MT],
                                                  int ftile0, int ttile0, int wf, int wt, int l) {
    EpiTok e[MT];
    float4 ws[MF][4], old[MF][MT][4];
#pragma unroll
    for (int j = 0; j < MT; ++j) e[j] = epi_tok<EPI>(p, (ttile0 + 2 * (wt + j)) * 16 + (l & 31));
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
            const int n0 = (ftile0 + 2 * (wf + i)) * 16 + 8 * v4 + 4 * (l >> 5);
            ws[i][v4] = *(const float4 *)(p.wscale + n0);
#pragma unroll
            for (int j = 0; j < MT; ++j)
                old[i][j][v4] = epi_old<EPI>(p, (ttile0 + 2 * (wt + j)) * 16 + (l & 31), n0, e[j]);
        }
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            const int t = (ttile0 + 2 * (wt + j)) * 16 + (l & 31);
            if (t >= p.n_tok) continue;
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4) {
                const v4i c = {acc[i][j][4 * v4], acc[i][j][4 * v4 + 1], acc[i][j][4 * v4 + 2],
                               acc[i][j][4 * v4 + 3]};
                gemm_store<EPI>(p, c, t, (ftile0 + 2 * (wf + i)) * 16 + 8 * v4 + 4 * (l >> 5), e[j],
                                ws[i][v4], old[i][j][v4]);
            }
        }
}

template <int EPI, int MF, int MT, int NWF>
__global__ __launch_bounds__(128 * NWF, 4 / NWF) void gemm_lds_kernel(GemmParams p) {
    constexpr int NTH = 128 * NWF;                 // threads
    constexpr int NF = NWF * MF, NT = 2 * MT;      // 32-row / 32-token pairs per workgroup
    constexpr int FT = 32 * NF, TK = 32 * NT;      // features, tokens per workgroup
    constexpr int WU = FT * 4, XU = TK * 16;       // 16-byte units per stage
    constexpr int WPT = WU / NTH, XPT = XU / NTH;  // per thread
    static_assert(WPT * NTH == WU && XPT * NTH == XU, "stage units must split evenly");
    __shared__ uint4 sw[2][WU];
    __shared__ uint4 sx[2][XU];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
    const int KC = p.K >> 6, steps = KC >> 2;
    const int ftile0 = blockIdx.x * (FT / 16), ttile0 = blockIdx.y * (TK / 16);
    const int ntt = (p.n_tok + 15) >> 4;
    const int wf = (w % NWF) * MF, wt = (w / NWF) * MT;   // this wave's row / token pairs

    // global sources of this thread's LDS slots i = tid + NTH*k (stage 0);
    // within a slot's 64-unit block, unit u = 32h + 16*tile + row/token
    size_t wsrc[WPT], xsrc[XPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int i = tid + NTH * k, u = i & 63, blk = i >> 6;
        const int cp = blk / NF, fp = blk % NF, h = u >> 5, ft = 2 * fp + ((u >> 4) & 1);
        wsrc[k] = ((size_t)(ftile0 + ft) * KC + 2 * cp + h) * 16 + (u & 15);
    }
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        const int i = tid + NTH * k, u = i & 63, blk = i >> 6;
        const int tp = blk % NT, gc = blk / NT, cp = gc & 1, g = gc >> 1, h = u >> 5;
        const int tt = min(ttile0 + 2 * tp + ((u >> 4) & 1), ntt - 1);
        xsrc[k] = (size_t)tt * KC * 64 + g * 64 + (2 * cp + h) * 16 + (u & 15);
    }
    v16i acc[MF][MT];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    // Two register sets hold stages s+1 and s+2 while stage s is multiplied,
    // so each stage's loads have two stages of MFMA work to arrive.  Loads
    // past the last stage reload the last one (branch-free; never stored).
    // The scheduling barriers keep each stage's loads at the top of its half
    // (left alone, the compiler sinks them below the MFMAs) and its stores
    // after the MFMAs.
    u32x4_t aw[WPT], ax[XPT], bw[WPT], bx_[XPT];
    const int last = steps - 1;
    gemm_stage_load(aw, ax, p.W, p.X, wsrc, xsrc, 0);
    gemm_stage_store<WPT, XPT, NTH>(aw, ax, sw[0], sx[0], tid);
    gemm_stage_load(aw, ax, p.W, p.X, wsrc, xsrc, min(1, last));
    lds_barrier();
    int s = 0;
    for (; s + 2 <= steps; s += 2) {
        gemm_stage_load(bw, bx_, p.W, p.X, wsrc, xsrc, min(s + 2, last));
        __builtin_amdgcn_sched_barrier(0);
        gemm_mma_stage<MF, MT, NF, NT>(acc, sw[0], sx[0], wf, wt, l);
        gemm_stage_store<WPT, XPT, NTH>(aw, ax, sw[1], sx[1], tid);
        lds_barrier();
        gemm_stage_load(aw, ax, p.W, p.X, wsrc, xsrc, min(s + 3, last));
        __builtin_amdgcn_sched_barrier(0);
        gemm_mma_stage<MF, MT, NF, NT>(acc, sw[1], sx[1], wf, wt, l);
        gemm_stage_store<WPT, XPT, NTH>(bw, bx_, sw[0], sx[0], tid);
        lds_barrier();
    }
    if (s < steps) gemm_mma_stage<MF, MT, NF, NT>(acc, sw[0], sx[0], wf, wt, l);   // odd count: buffer 0

    gemm_lds_epilogue<EPI, MF, MT>(p, acc, ftile0, ttile0, wf, wt, l);
}

// The same tiles with direct global -> LDS staging (global_load_lds_dwordx4:
// each lane's 16 B land at the wave's LDS base + 16 * lane, which is exactly
// the slot order above), so staging takes no VGPRs and no LDS store
// instructions.  NBUF stage buffers let each stage's loads be issued NBUF-1
// stages ahead (256 x 128: 3 buffers, 144 KB; small tiles, whose stages are
// short, 4 or more), with one barrier per stage:
//   iteration s: wait for this thread's stage-s loads (later stages may still
//   be in flight), barrier (every thread's stage s has landed, and every wave
//   is done reading the buffer that stage s+NBUF-1 reuses), issue stage
//   s+NBUF-1, multiply stage s.
// (lds_dma16 and wait_vmcnt: oxb_common.h)

// workgroups per CU that the LDS of a DMA-staged tile allows (160 KB)
__host__ __device__ constexpr int dma_occupancy(int MF, int MT, int NWF, int NBUF) {
    return 160 * 1024 / (NBUF * (32 * NWF * MF * 4 + 64 * MT * 16) * 16) >= 2 ? 2 : 1;
}

template <int EPI, int MF, int MT, int NWF, int NBUF>
__global__ __launch_bounds__(128 * NWF, dma_occupancy(MF, MT, NWF, NBUF)) void gemm_dma_kernel(
    GemmParams p) {
    constexpr int NTH = 128 * NWF;
    constexpr int NF = NWF * MF, NT = 2 * MT;
    constexpr int FT = 32 * NF, TK = 32 * NT;
    constexpr int WU = FT * 4, XU = TK * 16;
    constexpr int WPT = WU / NTH, XPT = XU / NTH, LPT = WPT + XPT;
    static_assert(WPT * NTH == WU && XPT * NTH == XU, "stage units must split evenly");
    static_assert(NBUF >= 3 && (NBUF - 2) * LPT < 64, "vmcnt holds the loads in flight");
    __shared__ uint4 sw[NBUF][WU];
    __shared__ uint4 sx[NBUF][XU];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
    const int KC = p.K >> 6, steps = KC >> 2;
    const int ftile0 = blockIdx.x * (FT / 16), ttile0 = blockIdx.y * (TK / 16);
    const int ntt = (p.n_tok + 15) >> 4;
    const int wf = (w % NWF) * MF, wt = (w / NWF) * MT;

    // global sources of this thread's LDS slots i = tid + NTH*k (stage 0),
    // as in gemm_lds_kernel
    const uint4 *wsrc[WPT], *xsrc[XPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int i = tid + NTH * k, u = i & 63, blk = i >> 6;
        const int cp = blk / NF, fp = blk % NF, h = u >> 5, ft = 2 * fp + ((u >> 4) & 1);
        wsrc[k] = p.W + ((size_t)(ftile0 + ft) * KC + 2 * cp + h) * 16 + (u & 15);
    }
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        const int i = tid + NTH * k, u = i & 63, blk = i >> 6;
        const int tp = blk % NT, gc = blk / NT, cp = gc & 1, g = gc >> 1, h = u >> 5;
        const int tt = min(ttile0 + 2 * tp + ((u >> 4) & 1), ntt - 1);
        xsrc[k] = p.X + (size_t)tt * KC * 64 + g * 64 + (2 * cp + h) * 16 + (u & 15);
    }
    auto issue = [&](int st, int b) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) lds_dma16(wsrc[k] + (size_t)st * 64, sw[b] + NTH * k + 64 * w);
#pragma unroll
        for (int k = 0; k < XPT; ++k) lds_dma16(xsrc[k] + (size_t)st * 256, sx[b] + NTH * k + 64 * w);
    };
    v16i acc[MF][MT];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    for (int st = 0; st < NBUF - 1; ++st)
        if (st < steps) issue(st, st);
    int b = 0;   // buffer of stage s
    for (int s = 0; s < steps; ++s) {
        // stages s+1 .. min(s+NBUF-2, steps-1) may stay in flight
        const int later = min(NBUF - 2, steps - 1 - s);
        if constexpr (NBUF == 3) {
            if (later == 1) wait_vmcnt<LPT>();
            else wait_vmcnt<0>();
        } else {
            if (later >= NBUF - 2) wait_vmcnt<(NBUF - 2) * LPT>();
            else if (later == 2) wait_vmcnt<2 * LPT>();
            else if (later == 1) wait_vmcnt<LPT>();
            else wait_vmcnt<0>();
        }
        lds_barrier();
        if (s + NBUF - 1 < steps) issue(s + NBUF - 1, b == 0 ? NBUF - 1 : b - 1);
        gemm_mma_stage<MF, MT, NF, NT>(acc, sw[b], sx[b], wf, wt, l);
        b = b == NBUF - 1 ? 0 : b + 1;
    }
    gemm_lds_epilogue<EPI, MF, MT>(p, acc, ftile0, ttile0, wf, wt, l);
}

// ---------------------------------------------------------------------------
// Split-K of the DMA-staged tiles, for deep K and too few output tiles to
// fill the CUs (8192 x 28672 at 512 tokens: 128 tiles of 256 x 128 for 256
// CUs).  Each tile's K stages are cut into P equal pieces, one workgroup per
// piece (grid tiles * P, tile-major).  Every workgroup stores its int32
// accumulators into its slot of the workspace (agent-scope stores, visible
// to every XCD once complete), waits for them, and counts in on the tile's
// counter; the last of the P to arrive adds the others' accumulators to its
// own and runs the epilogue.  Integer sums do not depend on their order, so
// the result is the unsplit kernel's bit for bit.  No workgroup waits for
// another (no co-residency is assumed), and the last arrival puts the
// counter back to zero, so a workspace stays ready for the next call.
// ---------------------------------------------------------------------------
struct SplitParams {
    int P;           // pieces per tile
    int tiles_f;     // feature tiles per row of token tiles
    int *cnt;        // [tiles] arrival counters, zero between launches
    int32_t *part;   // [tiles * P][FT * TK], slot g = workgroup g's piece
};

// Every split form keeps its arrival counters in one fixed area at the start
// of the workspace and its slots after it, so one workspace can serve calls of
// any shapes in turn: a call leaves every counter it used at zero, and no
// form's slots overlap another form's counters.
constexpr int kSplitCounters = 4096;
constexpr size_t kSplitCounterBytes = kSplitCounters * sizeof(int);

template <int EPI, int MF, int MT, int NWF, int NBUF>
__global__ __launch_bounds__(128 * NWF, dma_occupancy(MF, MT, NWF, NBUF)) void gemm_split_kernel(
    GemmParams p, SplitParams sp) {
    constexpr int NTH = 128 * NWF;
    constexpr int NF = NWF * MF, NT = 2 * MT;
    constexpr int FT = 32 * NF, TK = 32 * NT;
    constexpr int WU = FT * 4, XU = TK * 16;
    constexpr int WPT = WU / NTH, XPT = XU / NTH, LPT = WPT + XPT;
    constexpr int NPAIR = MF * MT * 8;   // 8-byte accumulator pairs per thread
    static_assert(WPT * NTH == WU && XPT * NTH == XU, "stage units must split evenly");
    static_assert(NBUF >= 3 && (NBUF - 2) * LPT < 64, "vmcnt holds the loads in flight");
    __shared__ uint4 sw[NBUF][WU];
    __shared__ uint4 sx[NBUF][XU];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, g = blockIdx.x;
    const int KC = p.K >> 6, S = p.K >> 8;
    const int t = g / sp.P, piece = g - t * sp.P;
    const int s0 = piece * S / sp.P, steps = (piece + 1) * S / sp.P - s0;
    const int ftile0 = (t % sp.tiles_f) * (FT / 16), ttile0 = (t / sp.tiles_f) * (TK / 16);
    const int ntt = (p.n_tok + 15) >> 4;
    const int wf = (w % NWF) * MF, wt = (w / NWF) * MT;

    // global sources of this thread's LDS slots i = tid + NTH*k at stage s0,
    // as in gemm_lds_kernel
    const uint4 *wsrc[WPT], *xsrc[XPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int i = tid + NTH * k, u = i & 63, blk = i >> 6;
        const int cp = blk / NF, fp = blk % NF, h = u >> 5, ft = 2 * fp + ((u >> 4) & 1);
        wsrc[k] = p.W + ((size_t)(ftile0 + ft) * KC + 2 * cp + h) * 16 + (u & 15) + (size_t)s0 * 64;
    }
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        const int i = tid + NTH * k, u = i & 63, blk = i >> 6;
        const int tp = blk % NT, gc = blk / NT, cp = gc & 1, gg = gc >> 1, h = u >> 5;
        const int tt = min(ttile0 + 2 * tp + ((u >> 4) & 1), ntt - 1);
        xsrc[k] = p.X + (size_t)tt * KC * 64 + gg * 64 + (2 * cp + h) * 16 + (u & 15) +
                  (size_t)s0 * 256;
    }
    auto issue = [&](int st, int b) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) lds_dma16(wsrc[k] + (size_t)st * 64, sw[b] + NTH * k + 64 * w);
#pragma unroll
        for (int k = 0; k < XPT; ++k) lds_dma16(xsrc[k] + (size_t)st * 256, sx[b] + NTH * k + 64 * w);
    };
    v16i acc[MF][MT];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    // the DMA kernel's pipeline over this piece's stages
    for (int st = 0; st < NBUF - 1; ++st)
        if (st < steps) issue(st, st);
    int b = 0;
    for (int s = 0; s < steps; ++s) {
        const int later = min(NBUF - 2, steps - 1 - s);
        if constexpr (NBUF == 3) {
            if (later == 1) wait_vmcnt<LPT>();
            else wait_vmcnt<0>();
        } else {
            if (later >= NBUF - 2) wait_vmcnt<(NBUF - 2) * LPT>();
            else if (later == 2) wait_vmcnt<2 * LPT>();
            else if (later == 1) wait_vmcnt<LPT>();
            else wait_vmcnt<0>();
        }
        lds_barrier();
        if (s + NBUF - 1 < steps) issue(s + NBUF - 1, b == 0 ? NBUF - 1 : b - 1);
        gemm_mma_stage<MF, MT, NF, NT>(acc, sw[b], sx[b], wf, wt, l);
        b = b == NBUF - 1 ? 0 : b + 1;
    }

    // hand-off: element (pair e, thread tid) of a slot holds this thread's
    // registers 2(e%8), 2(e%8)+1 of tile (e/8/MT, e/8%MT); every piece of a
    // tile has the same register layout
    uint64_t *const mine = (uint64_t *)(sp.part + (size_t)g * FT * TK);
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                const uint64_t pr = (uint64_t)(uint32_t)acc[i][j][2 * v] |
                                    ((uint64_t)(uint32_t)acc[i][j][2 * v + 1] << 32);
                __hip_atomic_store(mine + ((i * MT + j) * 8 + v) * NTH + tid, pr, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();   // every thread's stores are complete; every LDS read is done
    // the last-arrival flag, in a stage buffer word that no wave reads any
    // more (every stage load has landed and every wave is past its MFMAs)
    int *const s_last = (int *)&sw[0][0];
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(sp.cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool fin = old == sp.P - 1;
        if (fin) __hip_atomic_store(sp.cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_last = fin;
    }
    __syncthreads();
    if (!*s_last) return;
    for (int o = t * sp.P; o < (t + 1) * sp.P; ++o) {
        if (o == g) continue;
        const uint64_t *src = (const uint64_t *)(sp.part + (size_t)o * FT * TK);
        uint64_t v8[NPAIR];
#pragma unroll
        for (int e = 0; e < NPAIR; ++e)
            v8[e] = __hip_atomic_load(src + (size_t)e * NTH + tid, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
            for (int j = 0; j < MT; ++j)
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const uint64_t pr = v8[(i * MT + j) * 8 + v];
                    acc[i][j][2 * v] += (int)(uint32_t)pr;
                    acc[i][j][2 * v + 1] += (int)(uint32_t)(pr >> 32);
                }
    }
    gemm_lds_epilogue<EPI, MF, MT>(p, acc, ftile0, ttile0, wf, wt, l);
}

// ---------------------------------------------------------------------------
// Skinny GEMM for n_tok <= 64 (batched decode, small-M sweeps): the GEMV's
// decomposition with MFMA inside.  A workgroup owns TF 16-row feature tiles
// and all TT = ceil(n_tok/16) token tiles; its 4 waves split K (in 4-chunk
// MFMA steps) and meet in LDS, where each wave sums a quarter of the tiles
// (int32, exact) and runs the epilogue.  N/16/TF workgroups keep the chip
// busy where the 64x64 tiling launches too few.
// ---------------------------------------------------------------------------
// SPLIT: the K stages are cut into sp.P equal pieces over blockIdx.y (long
// rows: fewer, wider feature groups, so each group re-reads less of X); each
// workgroup stores its summed tiles to its workspace slot and counts in on
// its feature group's counter, and the last of the P to arrive adds the
// other slots (int32, exact) and runs the epilogue, as gemm_split_kernel.
template <int EPI, int TT, int TF, bool SPLIT = false>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmParams p, SplitParams sp) {
    constexpr int NT = TF * TT;   // 16x16 tiles per wave
    __shared__ v4i red[4][NT][64];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int KC = p.K >> 6, steps_all = KC >> 2;
    const int P = SPLIT ? sp.P : 1, piece = SPLIT ? (int)blockIdx.y : 0;
    const int k0 = piece * steps_all / P, steps = (piece + 1) * steps_all / P - k0;
    const int per = (steps + 3) >> 2;
    const int s0 = k0 + min(w * per, steps), s1 = k0 + min(steps, w * per + per);
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
            const uint4 *x = p.X + (size_t)t * KC * 64 + (size_t)s * 256 + q * 16 + r;
#pragma unroll
            for (int g = 0; g < 4; ++g) xv[t][g] = x[g * 64];
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
    if constexpr (SPLIT) {   // hand the summed tiles over; the last piece finishes
        uint64_t *mine = (uint64_t *)(sp.part + ((size_t)blockIdx.x * P + piece) * NT * 64 * 4);
        for (int i = w; i < NT; i += 4) {
            v4i c = red[0][i][lane];
#pragma unroll
            for (int k = 1; k < 4; ++k) c += red[k][i][lane];
            const size_t at = ((size_t)i * 64 + lane) * 2;
            __hip_atomic_store(mine + at, (uint64_t)(uint32_t)c[0] | ((uint64_t)(uint32_t)c[1] << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(mine + at + 1, (uint64_t)(uint32_t)c[2] | ((uint64_t)(uint32_t)c[3] << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(sp.cnt + blockIdx.x, 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            const bool fin = old == P - 1;
            if (fin) __hip_atomic_store(sp.cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = fin;
        }
        __syncthreads();
        if (!s_last) return;
    }
    for (int i = w; i < NT; i += 4) {
        v4i c = red[0][i][lane];
#pragma unroll
        for (int k = 1; k < 4; ++k) c += red[k][i][lane];
        if constexpr (SPLIT) {
            for (int o = 0; o < P; ++o) {
                if (o == piece) continue;
                const uint64_t *src =
                    (const uint64_t *)(sp.part + ((size_t)blockIdx.x * P + o) * NT * 64 * 4) +
                    ((size_t)i * 64 + lane) * 2;
                const uint64_t lo = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t hi = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                c[0] += (int)(uint32_t)lo;
                c[1] += (int)(uint32_t)(lo >> 32);
                c[2] += (int)(uint32_t)hi;
                c[3] += (int)(uint32_t)(hi >> 32);
            }
        }
        const int f = i / TT, t = (i % TT) * 16 + r, n0 = (ftile0 + f) * 16 + 4 * q;
        const EpiTok e = epi_tok<EPI>(p, t);
        const float4 ws = *(const float4 *)(p.wscale + n0);
        const float4 old = epi_old<EPI>(p, t, n0, e);
        if (t < ntok) gemm_store<EPI>(p, c, t, n0, e, ws, old);
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
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, TT, TF>), dim3(p.N / (16 * TF)), dim3(256), 0, s, p,
                       SplitParams{});
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

// The skinny kernel split over K (<= 64 tokens, long rows): 4 feature tiles
// per workgroup, each group's K in P pieces.  Workspace: the counter area,
// then one slot of TT * 4 tiles of 16x16 int32 per (group, piece).
static int skinny_split_pieces(int N, int K, int n_tok) {
    if (n_tok > 64 || N % 64 || K < 8192 || N / 64 > kSplitCounters) return 0;
    const int groups = N / 64;
    const int pieces = std::min(device_cus() / groups, K / 1024);
    return pieces >= 2 ? pieces : 0;
}

static size_t skinny_split_ws_bytes(int N, int n_tok, int pieces) {
    if (!pieces) return 0;
    const size_t groups = (size_t)N / 64, tt = (n_tok + 15) / 16;
    return kSplitCounterBytes + groups * pieces * tt * 4 * 64 * 16;
}

template <int EPI, int TT>
static int skinny_split_launch(const GemmParams &p, int pieces, void *ws, hipStream_t s) {
    SplitParams sp{};
    sp.P = pieces;
    const size_t groups = (size_t)p.N / 64;
    sp.cnt = (int *)ws;
    sp.part = (int32_t *)((char *)ws + kSplitCounterBytes);
    hipLaunchKernelGGL((gemm_skinny_kernel<EPI, TT, 4, true>), dim3((unsigned)groups, pieces),
                       dim3(256), 0, s, p, sp);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

template <int EPI, int MF, int MT, int NWF, int NBUF>
static int dma_launch(const GemmParams &p, hipStream_t s) {
    constexpr int FT = 32 * MF * NWF, TK = 64 * MT;
    dim3 grid(p.N / FT, (p.n_tok + TK - 1) / TK);
    hipLaunchKernelGGL((gemm_dma_kernel<EPI, MF, MT, NWF, NBUF>), grid, dim3(128 * NWF), 0, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

template <int EPI, int MF, int MT, int NWF = 2>
static int lds_launch(const GemmParams &p, hipStream_t s) {
    constexpr int FT = 32 * MF * NWF, TK = 64 * MT;
    dim3 grid(p.N / FT, (p.n_tok + TK - 1) / TK);
    hipLaunchKernelGGL((gemm_lds_kernel<EPI, MF, MT, NWF>), grid, dim3(128 * NWF), 0, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

// Split-K plans: pieces per tile, 0 for none.  Each tile's K stages in P
// equal pieces, one workgroup each; a piece's hand-off costs about what 2-3
// stages do.  Measured on 256 CUs (graphs of 30 calls, alternated with the
// unsplit kernel in one process):
// - 64x64 tiles (> 64 tokens; tiles * P up to two workgroups per CU, pieces
//   of >= 9 stages), tried first: 2560 x 6912 at 65 / 128 / 256 / 384
//   tokens 16.4 / 16.6 / 17.0 / 17.0 -> 11.3 / 11.5 / 12.5 / 15.3 us;
//   5120 x 8192 at 65 / 128 19.3 / 19.4 -> 13.4 / 13.8; 8192 x 28672 at
//   65 / 128 60.5 / 60.9 -> 41.2 / 43.8.
// - 256x128 DMA-staged tiles where they leave CUs idle, the pieces still
//   fill 5/8 of them and keep >= 14 stages: 8192 x 28672 at 256 / 512
//   tokens 77.8 / 126.6 -> 72.2 / 107.8 us.  Shallower pieces lost or broke
//   even: 2560 x 6912 at 768 / 1536 tokens 21.6 / 37.0 unsplit against
//   31.3 / 38.7 in pieces of 9 / 13.5 stages, 5120 x 8192 at 256 tokens
//   22.8 against 33.4 in pieces of 8.
static int split64_pieces(int N, int K, int n_tok) {
    if (n_tok <= 64 || N % 64) return 0;
    const int cus = device_cus();
    const long tiles = (long)(N / 64) * ((n_tok + 63) / 64);
    if (tiles > kSplitCounters) return 0;
    const long pieces = std::min<long>(2L * cus / tiles, (K / 256) / 9);
    return pieces >= 2 ? (int)pieces : 0;
}

static int split_pieces(int N, int K, int n_tok) {
    if (n_tok <= 64 || N % 256) return 0;
    const int cus = device_cus();
    const long tiles = (long)(N / 256) * ((n_tok + 127) / 128);
    if (tiles > kSplitCounters) return 0;
    const long pieces = std::min<long>(cus / tiles, (K / 256) / 14);
    if (pieces < 2 || tiles * pieces < (long)cus * 5 / 8) return 0;
    return (int)pieces;
}

// workspace: the counter area, then one slot of int32 accumulators (FT x TK)
// per workgroup
template <int FT, int TK>
static size_t tile_split_ws_bytes(int N, int n_tok, int pieces) {
    if (!pieces) return 0;
    const size_t tiles = (size_t)(N / FT) * ((n_tok + TK - 1) / TK);
    return kSplitCounterBytes + tiles * pieces * FT * TK * 4;
}

template <int EPI, int MF, int MT, int NWF, int NBUF>
static int tile_split_launch(const GemmParams &p, int pieces, void *ws, hipStream_t s) {
    constexpr int FT = 32 * MF * NWF, TK = 64 * MT;
    SplitParams sp{};
    sp.P = pieces;
    sp.tiles_f = p.N / FT;
    const size_t tiles = (size_t)sp.tiles_f * ((p.n_tok + TK - 1) / TK);
    sp.cnt = (int *)ws;
    sp.part = (int32_t *)((char *)ws + kSplitCounterBytes);
    hipLaunchKernelGGL((gemm_split_kernel<EPI, MF, MT, NWF, NBUF>), dim3((unsigned)(tiles * pieces)),
                       dim3(128 * NWF), 0, s, p, sp);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

// With a workspace that holds it, a split over K where it pays (the 64x64
// or 256x128 tiles above 64 tokens, the skinny kernel's 64-row groups at up
// to 64).  Otherwise n_tok <= 64: skinny kernel (2 feature tiles per
// workgroup once there are 3+ token tiles and enough rows, to halve the
// activation re-reads); else the LDS-staged kernel (the 64x64
// register-tiled kernel for N % 64 != 0).
template <int EPI>
static int gemm_launch(const GemmParams &p, void *stream, void *ws = nullptr,
                       size_t ws_bytes = 0) {
    hipStream_t s = (hipStream_t)stream;
    if (ws) {
        const int p64 = split64_pieces(p.N, p.K, p.n_tok);
        if (p64 && ws_bytes >= tile_split_ws_bytes<64, 64>(p.N, p.n_tok, p64))
            return tile_split_launch<EPI, 1, 1, 2, 4>(p, p64, ws, s);
        const int pieces = split_pieces(p.N, p.K, p.n_tok);
        if (pieces && ws_bytes >= tile_split_ws_bytes<256, 128>(p.N, p.n_tok, pieces))
            return tile_split_launch<EPI, 2, 2, 4, 3>(p, pieces, ws, s);
        const int sk = skinny_split_pieces(p.N, p.K, p.n_tok);
        if (sk && ws_bytes >= skinny_split_ws_bytes(p.N, p.n_tok, sk)) {
            switch ((p.n_tok + 15) >> 4) {
                case 1: return skinny_split_launch<EPI, 1>(p, sk, ws, s);
                case 2: return skinny_split_launch<EPI, 2>(p, sk, ws, s);
                case 3: return skinny_split_launch<EPI, 3>(p, sk, ws, s);
                default: return skinny_split_launch<EPI, 4>(p, sk, ws, s);
            }
        }
    }
    if (p.n_tok <= 64) {
        const int tt = (p.n_tok + 15) >> 4;
        const bool two = tt >= 3 && p.N % 32 == 0 && p.N / 32 >= 256;
        // up to 4 feature tiles per workgroup while the grid still gives every
        // CU a workgroup (each workgroup reads all of X, so fewer workgroups
        // re-read it less)
        const int cus = device_cus();
        const bool four = p.N % 64 == 0 && p.N / 64 >= cus;
        const bool pair = p.N % 32 == 0 && p.N / 32 >= cus;
        switch (tt) {
            case 1: return four ? skinny_launch<EPI, 1, 4>(p, s)
                                : pair ? skinny_launch<EPI, 1, 2>(p, s) : skinny_launch<EPI, 1, 1>(p, s);
            case 2: return four ? skinny_launch<EPI, 2, 4>(p, s)
                                : pair ? skinny_launch<EPI, 2, 2>(p, s) : skinny_launch<EPI, 2, 1>(p, s);
            case 3: return four ? skinny_launch<EPI, 3, 4>(p, s)
                                : two ? skinny_launch<EPI, 3, 2>(p, s) : skinny_launch<EPI, 3, 1>(p, s);
            default: return four ? skinny_launch<EPI, 4, 4>(p, s)
                                 : two ? skinny_launch<EPI, 4, 2>(p, s) : skinny_launch<EPI, 4, 1>(p, s);
        }
    }
    // LDS-staged tiles: the largest of 128x128, 128x64, 64x128, 64x64 whose
    // grid still gives every CU a workgroup (N a multiple of the tile); the
    // 256x128 DMA-staged tile already from 5/8 of the CUs (N = 2560 at 2048
    // tokens, 160 workgroups: K = 6912 / 2560 take 56.3 / 29.2 us against
    // 64.4 / 33.6 us for 320 workgroups of 128x128).
    const int cus = device_cus();
    auto blocks = [&](int ft, int tk) { return (long)(p.N / ft) * ((p.n_tok + tk - 1) / tk); };
    if (p.N % 256 == 0 && blocks(256, 128) >= cus * 5 / 8) return dma_launch<EPI, 2, 2, 4, 3>(p, s);
    if (p.N % 128 == 0 && blocks(128, 128) >= cus) return lds_launch<EPI, 2, 2>(p, s);
    if (p.N % 128 == 0 && blocks(128, 64) >= cus) return lds_launch<EPI, 2, 1>(p, s);
    if (p.N % 64 == 0 && blocks(64, 128) >= cus) return lds_launch<EPI, 1, 2>(p, s);
    if (p.N % 64 == 0) return dma_launch<EPI, 1, 1, 2, 4>(p, s);
    dim3 grid((p.N + 63) / 64, (p.n_tok + 63) / 64);
    hipLaunchKernelGGL((gemm_kernel<EPI>), grid, dim3(256), 0, s, p);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" size_t oxb_gemm_ws_bytes(int N, int K, int n_tok) {
    if (N <= 0 || N % 32 || K <= 0 || K % 256 || n_tok <= 0) return 0;   // shapes the GEMM rejects
    const int p64 = split64_pieces(N, K, n_tok);
    if (p64) return tile_split_ws_bytes<64, 64>(N, n_tok, p64);
    const int pieces = split_pieces(N, K, n_tok);
    if (pieces) return tile_split_ws_bytes<256, 128>(N, n_tok, pieces);
    return skinny_split_ws_bytes(N, n_tok, skinny_split_pieces(N, K, n_tok));
}

extern "C" int oxb_gemm_i8(const void *W_tiled, const int8_t *X, const float *xscale,
                           const int *xsum, const float *wscale, int N, int K, int n_tok,
                           float *Y, int32_t *acc_out, int epilogue, void *stream) {
    return oxb_gemm_i8_ws(W_tiled, X, xscale, xsum, wscale, N, K, n_tok, Y, acc_out, epilogue,
                          nullptr, 0, stream);
}

extern "C" int oxb_gemm_i8_ws(const void *W_tiled, const int8_t *X, const float *xscale,
                              const int *xsum, const float *wscale, int N, int K, int n_tok,
                              float *Y, int32_t *acc_out, int epilogue, void *ws, size_t ws_bytes,
                              void *stream) {
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
        case GE_STORE: return gemm_launch<GE_STORE>(p, stream, ws, ws_bytes);
        case GE_RESID: return gemm_launch<GE_RESID>(p, stream, ws, ws_bytes);
        case GE_GATEUP: return gemm_launch<GE_GATEUP>(p, stream, ws, ws_bytes);
        default: oxb::set_error("ternary GEMM: epilogue %d unsupported here", epilogue); return -1;
    }
}

extern "C" int oxb_gemm_qkv(const void *W_tiled, const int8_t *X, const float *xscale,
                            const int *xsum, const float *wscale, int Dq, int Dkv, int hd, int K,
                            int n_tok, int pos0, float *q_out, uint16_t *kcache,
                            uint16_t *vcache, int max_seq, const float *rope_cs, void *stream) {
    return oxb::gemm_qkv(W_tiled, X, xscale, xsum, wscale, Dq, Dkv, hd, K, n_tok, pos0, q_out,
                         kcache, vcache, false, max_seq, rope_cs, stream);
}

namespace oxb {

int gemm_qkv(const void *W_tiled, const int8_t *X, const float *xscale, const int *xsum,
             const float *wscale, int Dq, int Dkv, int hd, int K, int n_tok, int pos0,
             float *q_out, void *kcache, void *vcache, bool kv_f32, int max_seq,
             const float *rope_cs, void *stream, uint16_t *vcache8) {
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
    p.kv_f32 = kv_f32 ? 1 : 0;
    p.vcache8 = kv_f32 ? nullptr : vcache8;
    return gemm_launch<GE_QKV>(p, stream);
}

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
                  bool gemv_order, void *stream, uint16_t *vcache8, size_t kv8_tok_stride) {
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
    p.vcache8 = vcache8;
    p.kv8_tok_stride = kv8_tok_stride;
    p.gemv_order = gemv_order ? 1 : 0;
    return gemm_launch<GE_QKV>(p, stream);
}

}  // namespace oxb
