// GQA attention over the f16 KV cache for gfx950, in the reference's
// arithmetic order, so that its f32 result is bit-identical to the
// restatement of the three reference shaders:
//   scores   sh/attention.wgsl:29-59   dot = sum_d q[d]*k[d] in order of d,
//            times 1/sqrt(hd); GQA kv head = h / (H/Hkv)
//   softmax  sh/softmax.wgsl:25-80     max; 256 strided partial sums of
//            exp(x - max) + halving tree; p = exp(x - max) * (1 / sum)
//   P.V      sh/attention.wgsl:79-105  out[d] = sum_s p[s]*v[s][d] in order of s
// Each `sum += a * b` step of the dot products and P.V sums is one fused
// multiply-add (one rounding; WGSL lets the driver contract these, and the
// restatement fixes the fused form on host and device alike).
// orchestrated by nn/attention.rs:85-124.  Causally masked positions of the
// reference (score -3.4e38) contribute exact zeros to every sum, so a query
// at absolute position `pos` is computed over S = pos + 1 positions.
//
// Each workgroup handles the whole GQA group of G q heads of a KV head, so
// each cached K/V row is read once per group (prefill: once per group and
// pair of queries).  Cache layout: [Hkv][max_seq][128] f16 bits.
#include <mutex>

#include <cstring>

#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

constexpr int kHd = 128;

// ---------------------------------------------------------------------------
// Decode (one query at position *pos, S = pos + 1), two kernels:
//  A  scores: grid (64-position blocks, Hkv); the block's K rows are loaded
//     once, coalesced, into LDS and shared by the G heads (wave w = heads w,
//     w + 4); one lane per position runs the 128-term chain; scores[h][s]
//     to global.
//  B  softmax + P.V: grid (Hkv, slices); each workgroup takes the G heads of
//     one KV head and a slice of the 128 dims: min(4, 2G) waves of 64
//     sequential sums (lane = one (head, dim) output).  The softmax runs one
//     wave per head, the V slice is staged (as f32, transposed) in LDS, so a
//     summing wave reads 4 steps per LDS load.
// ---------------------------------------------------------------------------
constexpr int kScoreP = 64;   // positions per scores workgroup (one per lane)

template <int G>
__global__ __launch_bounds__(256) void attn_scores_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const int *__restrict__ pos_ptr,
    int max_seq, float scale, float *__restrict__ scores, size_t kv_stride, int pos_stride) {
    // K rows of this position block, 16 uint4 each, padded to 17 so that the
    // 64 lanes reading one column hit different banks; the G q rows.
    __shared__ uint4 ks[kScoreP][17];
    __shared__ __align__(16) float qs[G * kHd];
    // all kernel arguments in SGPRs up front (a late one is a further kernarg
    // round trip before the chain)
    asm volatile("" ::"s"(q), "s"(kc), "s"(pos_ptr), "s"(max_seq), "s"(scale), "s"(scores),
                 "s"(kv_stride), "s"(pos_stride));
    {   // sequence blockIdx.z of a batch: its own q, cache, position, scores
        const int z = blockIdx.z, H = gridDim.y * G;
        q += (size_t)z * H * kHd;
        kc += (size_t)z * kv_stride;
        pos_ptr += (size_t)z * pos_stride;
        scores += (size_t)z * H * max_seq;
    }
    const int pos = *pos_ptr;
    if (pos < 0 || pos >= max_seq) return;
    const int S = pos + 1;
    const int b = blockIdx.x, hk = blockIdx.y;
    const int s0 = b * kScoreP;
    if (s0 >= S) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // the G q rows (float4 tid mod 32G: every thread loads and stores, so no
    // load sits under a branch), then the coalesced tile load: thread i takes
    // uint4 i, i + 256, ... of the rows
    const float4 q4 = ((const float4 *)(q + (size_t)hk * G * kHd))[tid & (G * 32 - 1)];
    const uint4 *K4 = (const uint4 *)(kc + (size_t)hk * max_seq * kHd);
    uint4 kt[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = tid + 256 * k, row = i >> 4;
        kt[k] = K4[(size_t)min(s0 + row, S - 1) * 16 + (i & 15)];
    }
    *(float4 *)(qs + 4 * (tid & (G * 32 - 1))) = q4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = tid + 256 * k;
        ks[i >> 4][i & 15] = kt[k];
    }
    lds_barrier();
    const int s = s0 + lane;
    if (w >= G || s >= S) return;
    constexpr int HPW = G > 4 ? G / 4 : 1;   // heads per wave
    // this lane's K row and the head's q row (LDS broadcasts) are read three
    // 8-term groups ahead of the chain (scalar loads of q would return out of
    // order and force full waits inside it); a ring instead of the whole K row
    // in registers keeps the kernel near 50 VGPRs, so twice the workgroups fit
    // on a CU; each step of the chain is one v_fma_mix (k converted from f16
    // inside the instruction)
    const int wu = __builtin_amdgcn_readfirstlane(w);
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        const float *qg = qs + (wu + 4 * h) * kHd;
        constexpr int kAhead = 3;
        float4 qa[16], qb[16];
        uint4 kr16[16];
        auto ld = [&](int i) {
            qa[i] = *(const float4 *)(qg + 8 * i);
            qb[i] = *(const float4 *)(qg + 8 * i + 4);
            kr16[i] = ks[lane][i];
        };
#pragma unroll
        for (int i = 0; i < kAhead; ++i) ld(i);
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            if (i + kAhead < 16) ld(i + kAhead);
            __builtin_amdgcn_sched_barrier(0);
            const float qv[8] = {qa[i].x, qa[i].y, qa[i].z, qa[i].w,
                                 qb[i].x, qb[i].y, qb[i].z, qb[i].w};
            const uint4 kr = kr16[i];
            const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const float k0 = __half2float(__ushort_as_half((uint16_t)(kw[k2] & 0xffffu)));
                const float k1 = __half2float(__ushort_as_half((uint16_t)(kw[k2] >> 16)));
                dot = __builtin_fmaf(qv[2 * k2], k0, dot);
                dot = __builtin_fmaf(qv[2 * k2 + 1], k1, dot);
            }
        }
        scores[(size_t)(hk * G + wu + 4 * h) * max_seq + s] = dot * scale;
    }
}

// The shaders' 256-thread halving tree s[t] += s[t + stride], stride
// 128 .. 1, with s[4l + i] in component i of lane l: strides 128 .. 4 pair
// lanes 32 .. 1 apart (shuffles, then DPP row_shl), strides 2 and 1 pair
// components in lane 0.  Returns s[0] to every lane.
__device__ inline float tree256_sum4(const float (&c)[4]) {
    float a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v = c[i];
        v = v + __shfl_down(v, 32, 64);
        v = v + __shfl_down(v, 16, 64);
        v = v + __int_as_float(dpp0<0x108, 0xf>(__float_as_int(v)));
        v = v + __int_as_float(dpp0<0x104, 0xf>(__float_as_int(v)));
        v = v + __int_as_float(dpp0<0x102, 0xf>(__float_as_int(v)));
        v = v + __int_as_float(dpp0<0x101, 0xf>(__float_as_int(v)));
        a[i] = v;
    }
    const float r = (a[0] + a[2]) + (a[1] + a[3]);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
}

// Softmax of one score row held in registers: NJ groups of 256 positions,
// lane l component i holding thread t = 4l + i's positions 256j + 4l + i.
// Branch-free (loads clamped to the row, selects instead of guards) so all
// NJ*4 loads are in flight at once and the waits stay exact.
// VEC: src is 16-byte aligned, one float4 load per group (clamped to the last
// whole float4 below Spad, which the row holds); else four clamped loads.
template <int NJ, bool VEC>
__device__ __forceinline__ void softmax_row_regs(float *row, const float *__restrict__ src, int S,
                                                 int Spad, int lane) {
    float x[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        if constexpr (VEC) {
            const float4 v = *(const float4 *)(src + min(256 * j + 4 * lane, Spad - 4));
            x[j][0] = v.x; x[j][1] = v.y; x[j][2] = v.z; x[j][3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[j][i] = src[min(256 * j + 4 * lane + i, S - 1)];
        }
    }
    float m = -3.402823e+38f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (VEC ? 256 * j + 4 * lane + i < S : true) m = fmaxf(m, x[j][i]);   // clamped copies repeat s = S-1
    m = wave_max_dpp(m);
    float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e = oxb_expf_nonpos(x[j][i] - m);   // <= 0 for the positions kept
            x[j][i] = 256 * j + 4 * lane + i < S ? e : 0.0f;
            c[i] = c[i] + x[j][i];
        }
    const float inv = 1.0f / tree256_sum4(c);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int s0 = 256 * j + 4 * lane;   // Spad is a multiple of 4
        if (s0 < Spad)
            *(float4 *)(row + s0) =
                make_float4(x[j][0] * inv, x[j][1] * inv, x[j][2] * inv, x[j][3] * inv);
    }
}

// Softmax of one score row (global src, S values) by one wave into the LDS
// row, in the order of sh/softmax.wgsl:25-80 for a 256-thread workgroup:
// thread t sums exp(x - max) over positions t, t + 256, ... in order (out-of-
// range positions add an exact +0), then the halving tree.  Up to 4096
// positions the row is held in registers (softmax_row_regs; vec: src is
// 16-byte aligned and holds Spad values); longer rows are staged through LDS.  exp(x - max) is evaluated once: the shader's
// normalisation pass evaluates it again with the same operands.  The max is
// exact in any order.
__device__ __forceinline__ void wave_softmax_row(float *row, const float *__restrict__ src, int S,
                                                 int Spad, int lane, bool vec) {
    if (S <= 4096) {
        const int nj = (S + 255) >> 8;
        if (vec) {
            if (nj <= 1) softmax_row_regs<1, true>(row, src, S, Spad, lane);
            else if (nj <= 2) softmax_row_regs<2, true>(row, src, S, Spad, lane);
            else if (nj <= 4) softmax_row_regs<4, true>(row, src, S, Spad, lane);
            else if (nj <= 8) softmax_row_regs<8, true>(row, src, S, Spad, lane);
            else if (nj <= 10) softmax_row_regs<10, true>(row, src, S, Spad, lane);
            else if (nj <= 12) softmax_row_regs<12, true>(row, src, S, Spad, lane);
            else softmax_row_regs<16, true>(row, src, S, Spad, lane);
        } else {
            if (nj <= 1) softmax_row_regs<1, false>(row, src, S, Spad, lane);
            else if (nj <= 2) softmax_row_regs<2, false>(row, src, S, Spad, lane);
            else if (nj <= 4) softmax_row_regs<4, false>(row, src, S, Spad, lane);
            else if (nj <= 8) softmax_row_regs<8, false>(row, src, S, Spad, lane);
            else if (nj <= 12) softmax_row_regs<12, false>(row, src, S, Spad, lane);
            else softmax_row_regs<16, false>(row, src, S, Spad, lane);
        }
        return;
    }
    for (int base = 0; base < S; base += 512) {   // stage the row, 8 loads in flight
        float t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = src[min(base + lane + 64 * k, S - 1)];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (base + lane + 64 * k < S) row[base + lane + 64 * k] = t[k];
    }
    float m = -3.402823e+38f;
    for (int s = lane; s < S; s += 64) m = fmaxf(m, row[s]);
    m = wave_max_dpp(m);
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 256) {
        const int s = s0 + lane;
        if (s < S) { const float e = oxb_expf(row[s] - m); row[s] = e; p0 = p0 + e; }
        if (s + 64 < S) { const float e = oxb_expf(row[s + 64] - m); row[s + 64] = e; p1 = p1 + e; }
        if (s + 128 < S) { const float e = oxb_expf(row[s + 128] - m); row[s + 128] = e; p2 = p2 + e; }
        if (s + 192 < S) { const float e = oxb_expf(row[s + 192] - m); row[s + 192] = e; p3 = p3 + e; }
    }
    const float inv = 1.0f / wave_tree_sum((p0 + p2) + (p1 + p3));
    for (int s = lane; s < S; s += 64) row[s] = row[s] * inv;
    for (int s = S + lane; s < Spad; s += 64) row[s] = 0.0f;
}

// acc + sum_{s < n} p[s] * v[s ^ sw], one fused multiply-add at a time in
// order of s.  The LDS operands of the next 16 positions are read while the
// current 16 are summed (p and v 16-byte aligned).  sw is a multiple of 4
// (an XOR swizzle of the staged row that keeps groups of 4 positions whole).
__device__ inline float pv_chain(const float *p, const float *v, int n, float acc, int sw = 0) {
    auto ld = [&](float4 (&P)[4], float4 (&V)[4], int at) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            P[j] = *(const float4 *)(p + at + 4 * j);
            V[j] = *(const float4 *)(v + ((at + 4 * j) ^ sw));
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto mac = [&](const float4 (&P)[4], const float4 (&V)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = __builtin_fmaf(P[j].x, V[j].x, acc);
            acc = __builtin_fmaf(P[j].y, V[j].y, acc);
            acc = __builtin_fmaf(P[j].z, V[j].z, acc);
            acc = __builtin_fmaf(P[j].w, V[j].w, acc);
        }
    };
    int s = 0;
    if (n >= 16) {
        float4 PA[4], VA[4], PB[4], VB[4];
        ld(PA, VA, 0);
        for (; s + 48 <= n; s += 32) {
            ld(PB, VB, s + 16);
            mac(PA, VA);
            ld(PA, VA, s + 32);
            mac(PB, VB);
        }
        if (s + 32 <= n) {
            ld(PB, VB, s + 16);
            mac(PA, VA);
            mac(PB, VB);
            s += 32;
        } else {
            mac(PA, VA);
            s += 16;
        }
    }
    for (; s + 4 <= n; s += 4) {
        const float4 p4 = *(const float4 *)(p + s);
        const float4 v4 = *(const float4 *)(v + (s ^ sw));
        acc = __builtin_fmaf(p4.x, v4.x, acc);
        acc = __builtin_fmaf(p4.y, v4.y, acc);
        acc = __builtin_fmaf(p4.z, v4.z, acc);
        acc = __builtin_fmaf(p4.w, v4.w, acc);
    }
    for (; s < n; ++s) acc = __builtin_fmaf(p[s], v[s ^ sw], acc);
    return acc;
}

// ---------------------------------------------------------------------------
// Decode P.V in the reference's association: out[d] = sum of p[s] * v[s][d]
// in one loop over every position s (sh/attention.wgsl:96-104), one fused
// multiply-add per position.  A sequential sum is a chain of dependent
// steps, so what bounds it is the step latency: a dependent v_fma_mix_f32
// (f16 V operand converted inside the instruction) issues every ~4.4 cycles
// from one wave per SIMD, against ~12.4 for a dependent 4x4x1 f32 MFMA.
// One 16-wave workgroup per (KV head, group of four heads, half of the dims,
// sequence):
//  - softmax of row r on waves 4r .. 4r+3 (wave 4r + j, lane l playing
//    thread 64j + l of the shader's 256-thread workgroup) into LDS rows;
//  - the V rows' half (128 bytes per position) stream into an LDS ring of NS
//    slots of kPcRows rows, staged with global_load_lds_dwordx4 by every wave
//    (8 rows per wave and slot) NS - 1 slots ahead.  Iteration c: each wave
//    waits for its own loads of slot c + 1, a barrier publishes slots c and
//    c + 1 and frees slot c - 1, whose ring entry the next loads refill;
//  - waves 0 .. 3 (one per SIMD) run the chains: wave w takes heads 2(w/2)
//    and 2(w/2) + 1 (lanes 0-31 and 32-63) and the low (w even) or high half
//    of dword lane % 32 of the half row, so lane l chains dim 64 h + 2 (l %
//    32) + w % 2 of its head.  Their barriers carry no LDS fence: reads of
//    the published slots stay in flight across them.
// Rows past the cache length are clamped to its last row (staged, never
// summed), so the loads are unconditional and the waits exact; the chains
// stop at S.
// LDS (dynamic): ring [NS][kPcRows][32 dwords] | p [4][Sp] | red [4][256] | wmax [16]
// ---------------------------------------------------------------------------
constexpr int kPcWaves = 16;
constexpr int kPcThreads = 64 * kPcWaves;
constexpr int kPcRows = 8 * kPcWaves;        // V rows per ring slot (one DMA per wave)
constexpr int kPcRowDw = kHd / 4;            // dwords of half a V row
constexpr int kPcSlotBytes = kPcRows * kPcRowDw * 4;
constexpr int kPcMaxSeq = 6144;              // score rows of up to 24 x 256 positions
constexpr int kPcMaxNI = (kPcMaxSeq + 255) / 256;

__host__ __device__ inline int pc_row_stride(int max_seq) { return ((max_seq + 15) & ~15) + 4; }
__host__ __device__ inline size_t pc_smem(int slots, int max_seq) {
    return (size_t)slots * kPcSlotBytes + ((size_t)4 * pc_row_stride(max_seq) + 4 * 256 + 16) * 4;
}

// Softmax of one score row by four waves (sh/softmax.wgsl:25-80): thread t =
// 64 j + lane of the shader's workgroup sums exp(x - max) over positions
// t + 256 i in order of i, then the halving tree; the max over the row is
// exact in any order.  Loads are clamped to the row (branch-free).  The four
// waves of the row exchange through wm (their maxima) and red (the 256
// partials); every wave of the workgroup must call (two barriers).
struct NoLoads {
    __device__ void operator()() const {}
};

// after_loads() runs once the row's loads are issued, before their first
// wait (a caller's own loads there do not delay the softmax's).
template <int NI, typename F = NoLoads>
__device__ __forceinline__ void softmax_row_4w(float *prow, const float *__restrict__ src, int S,
                                               bool has_row, float *wm, float *red, int j,
                                               int lane, const F &after_loads = F()) {
    const int t = 64 * j + lane;
    float x[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) x[i] = has_row ? src[min(t + 256 * i, S - 1)] : 0.0f;
    after_loads();
    float m = -3.402823e+38f;
#pragma unroll
    for (int i = 0; i < NI; ++i) m = t + 256 * i < S ? fmaxf(m, x[i]) : m;
    m = wave_max_dpp(m);
    if (lane == 0) wm[j] = m;
    lds_barrier();
    m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        x[i] = t + 256 * i < S ? oxb_expf_nonpos(x[i] - m) : 0.0f;
        part = part + x[i];
    }
    red[t] = part;
    lds_barrier();
    const float a = red[lane] + red[lane + 128];        // stride 128 (t = lane)
    const float c = red[lane + 64] + red[lane + 192];   // stride 128 (t = lane + 64)
    const float inv = 1.0f / wave_tree_sum(a + c);      // stride 64, then 32 .. 1
#pragma unroll
    for (int i = 0; i < NI; ++i)
        if (t + 256 * i < S) prow[t + 256 * i] = x[i] * inv;
}

template <typename F = NoLoads>
__device__ __forceinline__ void softmax_row_4w_any(float *prow, const float *src, int S,
                                                   bool has_row, float *wm, float *red, int j,
                                                   int lane, const F &after_loads = F()) {
    const int ni = (S + 255) >> 8;   // workgroup-uniform
    if (ni <= 1) softmax_row_4w<1>(prow, src, S, has_row, wm, red, j, lane, after_loads);
    else if (ni <= 2) softmax_row_4w<2>(prow, src, S, has_row, wm, red, j, lane, after_loads);
    else if (ni <= 4) softmax_row_4w<4>(prow, src, S, has_row, wm, red, j, lane, after_loads);
    else if (ni <= 8) softmax_row_4w<8>(prow, src, S, has_row, wm, red, j, lane, after_loads);
    else if (ni <= 12) softmax_row_4w<12>(prow, src, S, has_row, wm, red, j, lane, after_loads);
    else if (ni <= 16) softmax_row_4w<16>(prow, src, S, has_row, wm, red, j, lane, after_loads);
    else softmax_row_4w<kPcMaxNI>(prow, src, S, has_row, wm, red, j, lane, after_loads);
}

// acc + sum of p[s] * v_s over the n (all 4 when FULL) positions of a group,
// in order of s; v_s the low (HI false) or high half of dword V[s]
template <bool HI, bool FULL>
__device__ __forceinline__ float pv4(float acc, const uint32_t (&V)[4], const float4 &P, int n = 4) {
    const float pp[4] = {P.x, P.y, P.z, P.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t u = V[k];
        const float v = __half2float(__ushort_as_half((uint16_t)(HI ? u >> 16 : u & 0xffffu)));
        const float t = __builtin_fmaf(pp[k], v, acc);
        acc = FULL || k < n ? t : acc;
    }
    return acc;
}

// n positions (1 .. kPcRows) of one ring slot into a lane's chain: vs = the
// lane's dword in the slot's row 0 (rows kPcRowDw dwords apart), pp = the
// lane's p row at the slot's first position.  Groups of four positions,
// operands read three groups ahead; 16 positions per unrolled iteration (a
// loop's back edge would wait for every LDS read in flight), the last n % 16
// from ring entries 0..3.
template <bool HI>
__device__ __forceinline__ float pc_chain_slot(float acc, const uint32_t *vs, const float *pp,
                                               int n) {
    uint32_t V[4][4];
    float4 P[4];
    auto ld = [&](int b, int g) {   // group g (clamped into the slot) into entry b
        g = min(g, kPcRows / 4 - 1);
#pragma unroll
        for (int k = 0; k < 4; ++k) V[b][k] = vs[(4 * g + k) * kPcRowDw];
        P[b] = *(const float4 *)(pp + 4 * g);
    };
    ld(0, 0);
    ld(1, 1);
    ld(2, 2);
    int s0 = 0;
#pragma unroll
    for (int it = 0; it < kPcRows / 16; ++it) {
        if (s0 + 16 > n) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            ld((j + 3) & 3, s0 / 4 + j + 3);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv4<HI, true>(acc, V[j], P[j]);
        }
        s0 += 16;
    }
    if (s0 < n) {
        ld(3, s0 / 4 + 3);   // entries 0..2 hold groups s0/4 .. s0/4 + 2
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = n - s0 - 4 * j;
            if (m >= 4) acc = pv4<HI, true>(acc, V[j], P[j]);
            else if (m > 0) acc = pv4<HI, false>(acc, V[j], P[j], m);
        }
    }
    return acc;
}

template <int NS>
__global__ __launch_bounds__(kPcThreads) void attn_pv_chain_kernel(
    const float *__restrict__ scores, const uint16_t *__restrict__ vc,
    const int *__restrict__ pos_ptr, int G, int max_seq, float *__restrict__ out,
    size_t kv_stride, int pos_stride) {
    static_assert(NS >= 3 && NS - 3 < 64, "ring depth within vmcnt");
    const int RG = (G + 3) >> 2;                  // groups of four heads per KV head
    const int dh = blockIdx.x & 1, hg = blockIdx.x >> 1;
    const int hk = hg / RG, rg = hg % RG, z = blockIdx.y;
    const int Hkv = (gridDim.x >> 1) / RG, H = Hkv * G;
    scores += (size_t)z * H * max_seq;
    vc += (size_t)z * kv_stride + (size_t)hk * max_seq * kHd + 64 * dh;
    out += (size_t)z * H * kHd + 64 * dh;
    extern __shared__ __align__(16) int8_t smem_pc[];
    uint4 *ring = (uint4 *)smem_pc;
    const int Sp = pc_row_stride(max_seq);
    float *pr = (float *)(smem_pc + (size_t)NS * kPcSlotBytes);
    float *red = pr + 4 * Sp, *wmax = red + 4 * 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = pos_ptr[(size_t)z * pos_stride];
    if (pos < 0 || pos >= max_seq) return;   // uniform: before any barrier
    const int S = pos + 1;
    const int nslots = (S + kPcRows - 1) / kPcRows;

    // this wave's share of a slot: rows 8w .. 8w+7 (lane: row 8w + lane/8,
    // 16 bytes lane % 8 of the half row), clamped to the cache length
    auto issue = [&](int c) {
        const int row = min(c * kPcRows + 8 * w + (lane >> 3), S - 1);
        lds_dma16(vc + (size_t)row * kHd + 8 * (lane & 7),
                  ring + ((size_t)(c % NS) * kPcRows + 8 * w) * (kPcRowDw / 4));
    };
#pragma unroll
    for (int c = 0; c < NS - 1; ++c) issue(c);

    // ---- softmax: row r = w / 4 (head 4rg + r of the KV head) -------------
    {
        const int r = w >> 2, j = w & 3, head = 4 * rg + r;
        softmax_row_4w_any(pr + r * Sp, scores + (size_t)(hk * G + min(head, G - 1)) * max_seq, S,
                           head < G, wmax + 4 * r, red + 256 * r, j, lane);
    }

    // ---- P.V chains over the ring --------------------------------------------
    const int r = 2 * (w >> 1) + (lane >> 5);   // the lane's row (chain waves)
    const float *prow = pr + r * Sp;
    float acc = 0.0f;
    for (int c = 0; c < nslots; ++c) {
        wait_vmcnt<NS - 3>();   // this wave's loads of slots c and c + 1 have landed
        if (w < 4 && c > 0) {
            // no LDS fence: published slots may still be read in flight, and
            // slot c - 1, which the next loads refill, was consumed (its
            // values feed the sums computed before this point); these waves
            // write no LDS after the softmax, whose rows the first (fenced)
            // barrier publishes
            asm volatile("s_barrier" ::: "memory");
        } else {
            lds_barrier();
        }
        issue(c + NS - 1);      // into slot c - 1's ring entry (clamped past the cache)
        if (w < 4) {
            const uint32_t *vs =
                (const uint32_t *)(ring + (size_t)(c % NS) * kPcRows * (kPcRowDw / 4)) + (lane & 31);
            const int n = min(kPcRows, S - c * kPcRows);
            acc = (w & 1) ? pc_chain_slot<true>(acc, vs, prow + c * kPcRows, n)
                          : pc_chain_slot<false>(acc, vs, prow + c * kPcRows, n);
        }
    }
    wait_vmcnt<0>();   // no LDS load in flight when the workgroup ends
    if (w < 4 && 4 * rg + r < G)
        out[(size_t)(hk * G + 4 * rg + r) * kHd + 2 * (lane & 31) + (w & 1)] = acc;
}

// ---------------------------------------------------------------------------
// The same P.V with one chain wave per CU, for few sequences: a workgroup of
// 4 waves per (query head, parity of the dims, sequence).  What bounds the
// chain above is the LDS's return path: every chain wave reads 256 bytes per
// position of V (its dword of the row) and 256 of p (a broadcast read of
// four positions returns 16 bytes to each lane), ~4 cycles of the CU's LDS
// per wave and position against ~4.4 for the fused step; with four chain
// waves on a CU the LDS takes ~16.  Here wave 0 runs the CU's one chain
// wave: lane l chains dim 2l + parity (the low or high half of dword l of
// the full f16 row, read two positions at a time); all four waves run the
// row's softmax (the 256-thread order) and stage the V rows through the
// ring.  The 2G workgroups of a KV head take block indices congruent mod 8,
// so they run on one XCD and its L2 serves their shared V rows: block b ->
// KV head 8 (b / (16 G)) + b % 8, item (b / 8) % (2G); blocks whose KV head
// is past the last are idle.
// LDS (dynamic): ring [NS][kPhRows][64 dwords] | p [Sp] | red [256] | wmax [4]
// ---------------------------------------------------------------------------
constexpr int kPhWaves = 4;
constexpr int kPhThreads = 64 * kPhWaves;
constexpr int kPhRows = 64;                      // V rows per ring slot (4 DMA per wave)
constexpr int kPhSlotBytes = kPhRows * kHd * 2;
constexpr int kPhMaxBatch = 8;                  // sequences that take this kernel

__host__ __device__ inline size_t ph_smem(int slots, int max_seq) {
    return (size_t)slots * kPhSlotBytes + ((size_t)pc_row_stride(max_seq) + 256 + 8) * 4;
}

template <bool HI>
__device__ __forceinline__ float ph_chain_slot(float acc, const uint32_t *vs, const float *pp, int n) {
    uint32_t V[4][4];
    float4 P[4];
    auto ld = [&](int b, int g) {   // group g (clamped into the slot) into entry b
        g = min(g, kPhRows / 4 - 1);
#pragma unroll
        for (int k = 0; k < 4; ++k) V[b][k] = vs[(4 * g + k) * (kHd / 2)];
        P[b] = *(const float4 *)(pp + 4 * g);
    };
    ld(0, 0);
    ld(1, 1);
    ld(2, 2);
    int s0 = 0;
#pragma unroll
    for (int it = 0; it < kPhRows / 16; ++it) {
        if (s0 + 16 > n) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            ld((j + 3) & 3, s0 / 4 + j + 3);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv4<HI, true>(acc, V[j], P[j]);
        }
        s0 += 16;
    }
    if (s0 < n) {
        ld(3, s0 / 4 + 3);   // entries 0..2 hold groups s0/4 .. s0/4 + 2
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = n - s0 - 4 * j;
            if (m >= 4) acc = pv4<HI, true>(acc, V[j], P[j]);
            else if (m > 0) acc = pv4<HI, false>(acc, V[j], P[j], m);
        }
    }
    return acc;
}

template <int NS>
__global__ __launch_bounds__(kPhThreads) void attn_pv_head_kernel(
    const float *__restrict__ scores, const uint16_t *__restrict__ vc,
    const int *__restrict__ pos_ptr, int G, int Hkv, int max_seq, float *__restrict__ out,
    size_t kv_stride, int pos_stride) {
    static_assert(NS >= 3 && 4 * (NS - 3) < 64, "ring depth within vmcnt");
    const int b = blockIdx.x, z = blockIdx.y;
    const int hk = 8 * (b / (16 * G)) + (b & 7), item = (b >> 3) % (2 * G);
    if (hk >= Hkv) return;
    const int h = hk * G + (item >> 1), parity = item & 1, H = Hkv * G;
    scores += (size_t)z * H * max_seq + (size_t)h * max_seq;
    vc += (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    out += (size_t)z * H * kHd + (size_t)h * kHd;
    extern __shared__ __align__(16) int8_t smem_ph[];
    uint4 *ring = (uint4 *)smem_ph;
    float *pr = (float *)(smem_ph + (size_t)NS * kPhSlotBytes);
    float *red = pr + pc_row_stride(max_seq), *wmax = red + 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = pos_ptr[(size_t)z * pos_stride];
    if (pos < 0 || pos >= max_seq) return;   // uniform: before any barrier
    const int S = pos + 1;
    const int nslots = (S + kPhRows - 1) / kPhRows;

    // this wave's share of a slot: rows 16w .. 16w+15 as four 4-row loads
    // (lane: row + lane/16, 16 bytes lane % 16 of the row), clamped
    const uint4 *V4 = (const uint4 *)vc;
    auto issue = [&](int c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r0 = 16 * w + 4 * k;
            const int row = min(c * kPhRows + r0 + (lane >> 4), S - 1);
            lds_dma16(V4 + (size_t)row * (kHd / 8) + (lane & 15),
                      ring + ((size_t)(c % NS) * kPhRows + r0) * (kHd / 8));
        }
    };
#pragma unroll
    for (int c = 0; c < NS - 1; ++c) issue(c);

    softmax_row_4w_any(pr, scores, S, true, wmax, red, w, lane);

    float acc = 0.0f;
    for (int c = 0; c < nslots; ++c) {
        wait_vmcnt<4 * (NS - 3)>();   // this wave's loads of slots c and c + 1 have landed
        if (w == 0 && c > 0)
            asm volatile("s_barrier" ::: "memory");   // reads in flight stay (see the 4-head kernel)
        else
            lds_barrier();
        issue(c + NS - 1);
        if (w == 0) {
            const uint32_t *vs = (const uint32_t *)(ring + (size_t)(c % NS) * kPhRows * (kHd / 8)) + lane;
            const int n = min(kPhRows, S - c * kPhRows);
            acc = parity ? ph_chain_slot<true>(acc, vs, pr + c * kPhRows, n)
                         : ph_chain_slot<false>(acc, vs, pr + c * kPhRows, n);
        }
    }
    wait_vmcnt<0>();   // no LDS load in flight when the workgroup ends
    if (w == 0) out[2 * lane + parity] = acc;
}

// ---------------------------------------------------------------------------
// The same P.V over the cache's V copy in position octets (v8_index: per KV
// head, one dim's 8 consecutive positions in 16 bytes).  In the row-major
// cache a lane's dim sits 256 bytes apart from one position to the next, so
// the chain wave above reads four dwords (using half of each) and a
// probability broadcast per 4 positions; here one 16-byte read gives the
// lane its dim's next 8 positions, plus two broadcasts of their
// probabilities.  Workgroup per (query head, half of the dims, sequence):
// lane l chains dim 64 half + l, and the ring stages only that half, in
// slots of kPoRows positions (16 octets x 64 lanes x 16 bytes); each wave
// issues four of a slot's 1 KB DMA loads.  Octets past the cache length are
// clamped to its last octet (staged, never summed).  Same block -> (KV head,
// item) mapping and the same ring protocol as attn_pv_head_kernel.
// LDS (dynamic): ring [NS][16][64][16 B] | p [Sp] | red [256] | wmax [4]
// ---------------------------------------------------------------------------
constexpr int kPoRows = 128;                              // positions per ring slot
constexpr int kPoOcts = kPoRows / 8;                      // octets per slot
constexpr int kPoSlotBytes = kPoOcts * 64 * 16;

__host__ __device__ inline size_t po_smem(int slots, int max_seq) {
    return (size_t)slots * kPoSlotBytes + ((size_t)pc_row_stride(max_seq) + 256 + 8) * 4;
}

// acc + sum of p[s] * v_s over the n (all 8 when FULL) positions of one
// octet, in order of s (v_s: half s % 2 of dword s / 2 of V)
template <bool FULL>
__device__ __forceinline__ float pv8(float acc, const uint4 &V, const float4 &Pa, const float4 &Pb,
                                     int n = 8) {
    const uint32_t u[4] = {V.x, V.y, V.z, V.w};
    const float pp[8] = {Pa.x, Pa.y, Pa.z, Pa.w, Pb.x, Pb.y, Pb.z, Pb.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t w = u[k >> 1];
        const float v = __half2float(__ushort_as_half((uint16_t)((k & 1) ? w >> 16 : w & 0xffffu)));
        const float t = __builtin_fmaf(pp[k], v, acc);
        acc = FULL || k < n ? t : acc;
    }
    return acc;
}

// n positions (1 .. 8 NOCT) of one ring slot into a lane's chain: vs = the
// lane's 16 bytes of the slot's octet 0 (octets STRIDE uint4 apart), pp = the
// p row at the slot's first position.  Octet o in entry o % 4, read three
// octets ahead; four octets per iteration, whose entries are constants (a
// rotating index would put the entries in scratch), the rest from entries
// 0..3 after the loop.
template <int NOCT = kPoOcts, int STRIDE = 64>
__device__ __forceinline__ float po_chain_slot(float acc, const uint4 *vs, const float *pp, int n) {
    static_assert(NOCT % 4 == 0, "whole groups of four octets");
    uint4 V[4];
    float4 Pa[4], Pb[4];
    auto ld = [&](int b, int o) {   // octet o (clamped into the slot) into entry b
        o = min(o, NOCT - 1);
        V[b] = vs[o * STRIDE];
        Pa[b] = *(const float4 *)(pp + 8 * o);
        Pb[b] = *(const float4 *)(pp + 8 * o + 4);
    };
    ld(0, 0);
    ld(1, 1);
    ld(2, 2);
    int o0 = 0;
#pragma unroll
    for (int it = 0; it < NOCT / 4; ++it) {
        if (8 * (o0 + 4) > n) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            ld((j + 3) & 3, o0 + j + 3);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv8<true>(acc, V[j], Pa[j], Pb[j]);
        }
        o0 += 4;
    }
    if (8 * o0 < n) {
        ld(3, o0 + 3);   // entries 0..2 hold octets o0 .. o0 + 2
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = n - 8 * (o0 + j);
            if (m >= 8) acc = pv8<true>(acc, V[j], Pa[j], Pb[j]);
            else if (m > 0) acc = pv8<false>(acc, V[j], Pa[j], Pb[j], m);
        }
    }
    return acc;
}

template <int NS>
__global__ __launch_bounds__(kPhThreads) void attn_pv_oct_kernel(
    const float *__restrict__ scores, const uint16_t *__restrict__ vc8,
    const int *__restrict__ pos_ptr, int G, int Hkv, int max_seq, float *__restrict__ out,
    size_t kv8_stride, int pos_stride) {
    static_assert(NS >= 3 && 4 * (NS - 3) < 64, "ring depth within vmcnt");
    const int b = blockIdx.x, z = blockIdx.y;
    const int hk = 8 * (b / (16 * G)) + (b & 7), item = (b >> 3) % (2 * G);
    if (hk >= Hkv) return;
    const int h = hk * G + (item >> 1), half = item & 1, H = Hkv * G;
    scores += (size_t)z * H * max_seq + (size_t)h * max_seq;
    vc8 += (size_t)z * kv8_stride + (size_t)hk * v8_head_elems(max_seq, kHd);
    out += (size_t)z * H * kHd + (size_t)h * kHd;
    extern __shared__ __align__(16) int8_t smem_po[];
    uint4 *ring = (uint4 *)smem_po;
    float *pr = (float *)(smem_po + (size_t)NS * kPoSlotBytes);
    float *red = pr + pc_row_stride(max_seq), *wmax = red + 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = pos_ptr[(size_t)z * pos_stride];
    if (pos < 0 || pos >= max_seq) return;   // uniform: before any barrier
    const int S = pos + 1;
    const int nslots = (S + kPoRows - 1) / kPoRows;
    const int last_oct = (S - 1) >> 3;

    // this wave's share of a slot: octets 4w .. 4w+3, each one 1 KB load
    // (lane l: the 16 bytes of dim 64 half + l), clamped to the last octet
    const uint4 *V8 = (const uint4 *)vc8 + 64 * half + lane;
    auto issue = [&](int c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int o = c * kPoOcts + 4 * w + k;
            lds_dma16(V8 + (size_t)min(o, last_oct) * kHd,
                      ring + ((size_t)(c % NS) * kPoOcts + 4 * w + k) * 64);
        }
    };
#pragma unroll
    for (int c = 0; c < NS - 1; ++c) issue(c);

    softmax_row_4w_any(pr, scores, S, true, wmax, red, w, lane);

    float acc = 0.0f;
    for (int c = 0; c < nslots; ++c) {
        wait_vmcnt<4 * (NS - 3)>();   // this wave's loads of slots c and c + 1 have landed
        if (w == 0 && c > 0)
            asm volatile("s_barrier" ::: "memory");   // reads in flight stay (see the 4-head kernel)
        else
            lds_barrier();
        issue(c + NS - 1);
        if (w == 0) {
            const uint4 *vs = ring + (size_t)(c % NS) * kPoOcts * 64 + lane;
            acc = po_chain_slot(acc, vs, pr + c * kPoRows, min(kPoRows, S - c * kPoRows));
        }
    }
    wait_vmcnt<0>();   // no LDS load in flight when the workgroup ends
    if (w == 0) out[64 * half + lane] = acc;
}

// The same P.V with V streamed from the octet copy into registers: the
// chain wave's lanes load their dim's octets straight from global memory
// (one 1 KB wave load per 8 positions) kPoReg - 1 octets ahead in a ring of
// registers, so the LDS carries only the probability broadcasts and no
// barrier paces the chain; the other three waves only help with the
// softmax.  The first loads go out right after the softmax's score loads.
// Same grid, block -> (KV head, item) mapping and result bits as
// attn_pv_oct_kernel.  LDS (dynamic): p [Sp] | red [256] | wmax [4]
constexpr int kPoReg = 16;   // octets in the chain wave's register ring

__host__ __device__ inline size_t pr_smem(int max_seq) {
    return ((size_t)pc_row_stride(max_seq) + 256 + 8) * 4;
}

// acc over positions 0 .. S-1 of a lane's dim: octet o's V at V8[o * kHd]
// (clamped to the last octet), its p at pr[8o .. 8o+7] (read three octets
// ahead).  Passes of kPoReg octets keep the ring indices constants; then the
// whole octets left, then the last S % 8 positions.
__device__ __forceinline__ float po_chain_reg(const uint4 *__restrict__ V8, const float *pr, int S,
                                              uint4 (&vr)[kPoReg]) {
    constexpr int NB = kPoReg;
    const int last = (S - 1) >> 3, nfull = S >> 3;
    float4 pa[4], pb[4];
    auto ldv = [&](int b, int o) { vr[b] = V8[(size_t)min(o, last) * kHd]; };
    auto ldp = [&](int b, int o) {
        o = min(o, last);
        pa[b] = *(const float4 *)(pr + 8 * o);
        pb[b] = *(const float4 *)(pr + 8 * o + 4);
    };
    float acc = 0.0f;
    ldp(0, 0);
    ldp(1, 1);
    ldp(2, 2);
    int o0 = 0;
    for (; o0 + NB <= nfull; o0 += NB) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            ldv((i + NB - 1) % NB, o0 + i + NB - 1);
            ldp((i + 3) & 3, o0 + i + 3);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv8<true>(acc, vr[i], pa[i & 3], pb[i & 3]);
        }
    }
    const int r = nfull - o0;   // whole octets left (< NB), then the partial one
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (i < r) {
            __builtin_amdgcn_sched_barrier(0);
            ldv((i + NB - 1) % NB, o0 + i + NB - 1);
            ldp((i + 3) & 3, o0 + i + 3);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv8<true>(acc, vr[i], pa[i & 3], pb[i & 3]);
        } else if (i == r && (S & 7)) {
            acc = pv8<false>(acc, vr[i], pa[i & 3], pb[i & 3], S & 7);
        }
    }
    return acc;
}

__global__ __launch_bounds__(kPhThreads) void attn_pv_oreg_kernel(
    const float *__restrict__ scores, const uint16_t *__restrict__ vc8,
    const int *__restrict__ pos_ptr, int G, int Hkv, int max_seq, float *__restrict__ out,
    size_t kv8_stride, int pos_stride) {
    const int b = blockIdx.x, z = blockIdx.y;
    const int hk = 8 * (b / (16 * G)) + (b & 7), item = (b >> 3) % (2 * G);
    if (hk >= Hkv) return;
    const int h = hk * G + (item >> 1), half = item & 1, H = Hkv * G;
    scores += (size_t)z * H * max_seq + (size_t)h * max_seq;
    vc8 += (size_t)z * kv8_stride + (size_t)hk * v8_head_elems(max_seq, kHd);
    out += (size_t)z * H * kHd + (size_t)h * kHd;
    extern __shared__ __align__(16) int8_t smem_pr[];
    float *pr = (float *)smem_pr;
    float *red = pr + pc_row_stride(max_seq), *wmax = red + 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = pos_ptr[(size_t)z * pos_stride];
    if (pos < 0 || pos >= max_seq) return;   // uniform: before any barrier
    const int S = pos + 1, last = (S - 1) >> 3;
    const uint4 *V8 = (const uint4 *)vc8 + 64 * half + lane;
    uint4 vr[kPoReg];
    // wave 0's ring: octets 0 .. kPoReg - 2, issued behind its score loads
    auto first_v = [&]() {
        if (w == 0) {
#pragma unroll
            for (int i = 0; i < kPoReg - 1; ++i) vr[i] = V8[(size_t)min(i, last) * kHd];
        }
    };
    softmax_row_4w_any(pr, scores, S, true, wmax, red, w, lane, first_v);
    lds_barrier();   // every wave's probabilities are in pr
    if (w == 0) out[64 * half + lane] = po_chain_reg(V8, pr, S, vr);
}

// The 16-wave P.V above over the octet copy of V (larger batches): wave w
// stages octet w of each 128-position slot of this workgroup's half of the
// dims, and chain wave w < 4 sums row w (head 4 rg + w), lane l chaining dim
// 64 dh + l with one 16-byte read per 8 positions (po_chain_slot).  Same
// grid, ring protocol and LDS sizes (pc_smem) as attn_pv_chain_kernel.
template <int NS>
__global__ __launch_bounds__(kPcThreads) void attn_pv_chain_oct_kernel(
    const float *__restrict__ scores, const uint16_t *__restrict__ vc8,
    const int *__restrict__ pos_ptr, int G, int max_seq, float *__restrict__ out,
    size_t kv8_stride, int pos_stride) {
    static_assert(NS >= 3 && NS - 3 < 64, "ring depth within vmcnt");
    static_assert(kPcRows == kPoRows && kPcSlotBytes == kPoSlotBytes && kPcWaves == kPoOcts,
                  "one octet load per wave and slot");
    const int RG = (G + 3) >> 2;                  // groups of four heads per KV head
    const int dh = blockIdx.x & 1, hg = blockIdx.x >> 1;
    const int hk = hg / RG, rg = hg % RG, z = blockIdx.y;
    const int Hkv = (gridDim.x >> 1) / RG, H = Hkv * G;
    scores += (size_t)z * H * max_seq;
    vc8 += (size_t)z * kv8_stride + (size_t)hk * v8_head_elems(max_seq, kHd);
    out += (size_t)z * H * kHd + 64 * dh;
    extern __shared__ __align__(16) int8_t smem_pco[];
    uint4 *ring = (uint4 *)smem_pco;
    const int Sp = pc_row_stride(max_seq);
    float *pr = (float *)(smem_pco + (size_t)NS * kPcSlotBytes);
    float *red = pr + 4 * Sp, *wmax = red + 4 * 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = pos_ptr[(size_t)z * pos_stride];
    if (pos < 0 || pos >= max_seq) return;   // uniform: before any barrier
    const int S = pos + 1;
    const int nslots = (S + kPoRows - 1) / kPoRows;
    const int last_oct = (S - 1) >> 3;

    // this wave's share of a slot: octet w, one 1 KB load (lane l: dim
    // 64 dh + l), clamped to the last octet
    const uint4 *V8 = (const uint4 *)vc8 + 64 * dh + lane;
    auto issue = [&](int c) {
        const int o = c * kPoOcts + w;
        lds_dma16(V8 + (size_t)min(o, last_oct) * kHd,
                  ring + ((size_t)(c % NS) * kPoOcts + w) * 64);
    };
#pragma unroll
    for (int c = 0; c < NS - 1; ++c) issue(c);

    // ---- softmax: row r = w / 4 (head 4rg + r of the KV head) -------------
    {
        const int r = w >> 2, j = w & 3, head = 4 * rg + r;
        softmax_row_4w_any(pr + r * Sp, scores + (size_t)(hk * G + min(head, G - 1)) * max_seq, S,
                           head < G, wmax + 4 * r, red + 256 * r, j, lane);
    }

    // ---- P.V chains over the ring: wave w < 4 sums row w -------------------
    const float *prow = pr + (w & 3) * Sp;
    float acc = 0.0f;
    for (int c = 0; c < nslots; ++c) {
        wait_vmcnt<NS - 3>();   // this wave's loads of slots c and c + 1 have landed
        if (w < 4 && c > 0)
            asm volatile("s_barrier" ::: "memory");   // reads in flight stay (see above)
        else
            lds_barrier();
        issue(c + NS - 1);      // into slot c - 1's ring entry (clamped past the cache)
        if (w < 4) {
            const uint4 *vs = ring + (size_t)(c % NS) * kPoOcts * 64 + lane;
            acc = po_chain_slot(acc, vs, prow + c * kPoRows, min(kPoRows, S - c * kPoRows));
        }
    }
    wait_vmcnt<0>();   // no LDS load in flight when the workgroup ends
    if (w < 4 && 4 * rg + w < G) out[(size_t)(hk * G + 4 * rg + w) * kHd + lane] = acc;
}

// The same P.V with both halves of the dims in one workgroup per (KV head,
// group of four heads, sequence): half as many workgroups (160 for 32
// sequences of the 2B shape, one round over the CUs where the per-half
// grid needs two), each staging whole V octets (both halves) in ring slots
// of kPmRows positions: wave w loads octet w % 8 of a slot, half w / 8 (one
// 1 KB load).  Chain wave w < 8 sums head 4 rg + w % 4, lane l dim
// 64 (w / 4) + l.  Softmax and result bits as attn_pv_chain_oct_kernel.
// LDS (dynamic): ring [NS][8 octets][2 halves][64 lanes] uint4 | p [4][Sp] |
// red [4][256] | wmax [16]
constexpr int kPmRows = 64;                    // positions per ring slot
constexpr int kPmOcts = kPmRows / 8;
constexpr int kPmSlotBytes = kPmOcts * 2 * 64 * 16;

__host__ __device__ inline size_t pm_smem(int slots, int max_seq) {
    return (size_t)slots * kPmSlotBytes + ((size_t)4 * pc_row_stride(max_seq) + 4 * 256 + 16) * 4;
}

template <int NS>
__global__ __launch_bounds__(kPcThreads) void attn_pv_chain_oct2_kernel(
    const float *__restrict__ scores, const uint16_t *__restrict__ vc8,
    const int *__restrict__ pos_ptr, int G, int max_seq, float *__restrict__ out,
    size_t kv8_stride, int pos_stride) {
    static_assert(NS >= 3 && NS - 3 < 64, "ring depth within vmcnt");
    static_assert(kPcWaves == 2 * kPmOcts, "one octet half per wave and slot");
    const int RG = (G + 3) >> 2;                  // groups of four heads per KV head
    const int hg = blockIdx.x, hk = hg / RG, rg = hg % RG, z = blockIdx.y;
    const int Hkv = gridDim.x / RG, H = Hkv * G;
    scores += (size_t)z * H * max_seq;
    vc8 += (size_t)z * kv8_stride + (size_t)hk * v8_head_elems(max_seq, kHd);
    out += (size_t)z * H * kHd;
    extern __shared__ __align__(16) int8_t smem_pm[];
    uint4 *ring = (uint4 *)smem_pm;
    const int Sp = pc_row_stride(max_seq);
    float *pr = (float *)(smem_pm + (size_t)NS * kPmSlotBytes);
    float *red = pr + 4 * Sp, *wmax = red + 4 * 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = pos_ptr[(size_t)z * pos_stride];
    if (pos < 0 || pos >= max_seq) return;   // uniform: before any barrier
    const int S = pos + 1;
    const int nslots = (S + kPmRows - 1) / kPmRows;
    const int last_oct = (S - 1) >> 3;

    // this wave's share of a slot: octet w % 8, half w / 8 (lane l: dim
    // 64 (w / 8) + l), clamped to the last octet
    const uint4 *V8 = (const uint4 *)vc8 + 64 * (w >> 3) + lane;
    auto issue = [&](int c) {
        const int o = c * kPmOcts + (w & 7);
        lds_dma16(V8 + (size_t)min(o, last_oct) * kHd,
                  ring + (((size_t)(c % NS) * kPmOcts + (w & 7)) * 2 + (w >> 3)) * 64);
    };
#pragma unroll
    for (int c = 0; c < NS - 1; ++c) issue(c);

    // ---- softmax: row r = w / 4 (head 4rg + r of the KV head) -------------
    {
        const int r = w >> 2, j = w & 3, head = 4 * rg + r;
        softmax_row_4w_any(pr + r * Sp, scores + (size_t)(hk * G + min(head, G - 1)) * max_seq, S,
                           head < G, wmax + 4 * r, red + 256 * r, j, lane);
    }

    // ---- P.V chains over the ring: wave w < 8 sums row w % 4, half w / 4 ---
    const float *prow = pr + (w & 3) * Sp;
    float acc = 0.0f;
    for (int c = 0; c < nslots; ++c) {
        wait_vmcnt<NS - 3>();   // this wave's loads of slots c and c + 1 have landed
        if (w < 8 && c > 0)
            asm volatile("s_barrier" ::: "memory");   // reads in flight stay (see above)
        else
            lds_barrier();
        issue(c + NS - 1);      // into slot c - 1's ring entry (clamped past the cache)
        if (w < 8) {
            const uint4 *vs = ring + (size_t)(c % NS) * kPmOcts * 128 + 64 * (w >> 2) + lane;
            acc = po_chain_slot<kPmOcts, 128>(acc, vs, prow + c * kPmRows,
                                              min(kPmRows, S - c * kPmRows));
        }
    }
    wait_vmcnt<0>();   // no LDS load in flight when the workgroup ends
    if (w < 8 && 4 * rg + (w & 3) < G)
        out[(size_t)(hk * G + 4 * rg + (w & 3)) * kHd + 64 * (w >> 2) + lane] = acc;
}

// ---------------------------------------------------------------------------
// Prefill: one workgroup per (Q consecutive queries, KV head); query i of
// the block sits at position pos0 + q0 + i and attends over S_i = its
// position + 1 cached positions (causal).  Each K row is read once for the
// Q x G score rows (one position per thread, Q*G chains of 128 terms in
// order of d), each score row's softmax runs on one wave in the 256-thread
// order (wave_softmax_row), and each thread runs Q*G*128/256 P.V sums that
// share its dim d, one V element per step for all of them, each summed in
// order of s over its own query's S_i.  Queries past n_q repeat the last one
// and are not stored.  LDS: q [Q*G][128] f32 | scores [Q*G][Sw] f32, Sw =
// the longest row rounded up to 4 (positions a row does not attend to are
// never written or read).
// ---------------------------------------------------------------------------
constexpr int kPrefillThreads = 256;

template <int G, int Q>
__global__ __launch_bounds__(kPrefillThreads) void attn_prefill_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    int pos0, int n_q, int H, int max_seq, float scale, float *__restrict__ out) {
    constexpr int R = Q * G;   // score rows: query r / G, head r % G
    extern __shared__ __align__(16) float smem[];
    float *qs = smem;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int q0 = blockIdx.x * Q, hk = blockIdx.y;
    int Sq[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) Sq[i] = pos0 + min(q0 + i, n_q - 1) + 1;
    const int Smax = Sq[Q - 1];
    if (Smax > max_seq) return;   // host checks too; never read out of range
    const int Sw = (Smax + 3) & ~3;
    float *sc = qs + R * kHd;
    for (int i = tid; i < R * kHd; i += kPrefillThreads) {
        const int r = i / kHd, qi = min(q0 + r / G, n_q - 1);
        qs[i] = q[(size_t)qi * H * kHd + (size_t)(hk * G + r % G) * kHd + i % kHd];
    }
    lds_barrier();

    // ---- scores: one position per thread, R chains of 128 terms -----------
    const uint4 *K4 = (const uint4 *)(kc + (size_t)hk * max_seq * kHd);
    for (int s = tid; s < Smax; s += kPrefillThreads) {
        // q stays in LDS (read per use, broadcast): hoisting R x 128 values
        // out of this loop would not fit in registers
        asm volatile("" ::: "memory");
        uint4 kr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) kr[i] = K4[(size_t)s * 16 + i];
        // rows in passes of up to 4 chains over the K row held in registers
        constexpr int RG = R < 4 ? R : 4;
#pragma unroll 1
        for (int r0 = 0; r0 < R; r0 += RG) {
            float dot[RG];
#pragma unroll
            for (int r = 0; r < RG; ++r) dot[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {   // dims 8i .. 8i+7
                const __half2 *hh = (const __half2 *)&kr[i];
                float kf[8];
#pragma unroll
                for (int k2 = 0; k2 < 4; ++k2) {
                    const float2 f = __half22float2(hh[k2]);
                    kf[2 * k2] = f.x;
                    kf[2 * k2 + 1] = f.y;
                }
#pragma unroll
                for (int r = 0; r < RG; ++r) {   // q as two broadcast float4 reads
                    const float4 qa = *(const float4 *)(qs + (r0 + r) * kHd + 8 * i);
                    const float4 qb = *(const float4 *)(qs + (r0 + r) * kHd + 8 * i + 4);
                    const float qq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        dot[r] = __builtin_fmaf(qq[e], kf[e], dot[r]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RG; ++r)
                if (s < Sq[(r0 + r) / G]) sc[(r0 + r) * Sw + s] = dot[r] * scale;
        }
    }
    lds_barrier();

    // ---- softmax: one wave per row --------------------------------------------
    for (int r = w; r < R; r += kPrefillThreads / 64) wave_softmax_row(sc + r * Sw, sc + r * Sw, Sq[r / G], Sw, lane, true);
    lds_barrier();

    // ---- P.V: thread t, dim t % 128, rows t / 128 + (threads / 128) c ---------------
    constexpr int NC = R * kHd / kPrefillThreads > 0 ? R * kHd / kPrefillThreads : 1;
    if (tid >= R * kHd) return;
    const int d = tid % kHd;
    const uint16_t *Vd = vc + (size_t)hk * max_seq * kHd + d;
    int rr[NC], Sc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        rr[c] = tid / kHd + (kPrefillThreads / kHd) * c;
        Sc[c] = Sq[rr[c] / G];
    }
    // one chain per output over its row's positions, in order of s
    // (sh/attention.wgsl:96-104): the positions every row reaches in
    // unrolled steps, then the longer rows' last positions
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    const int S0 = Sq[0];   // every row attends at least this far
    constexpr int U = 16;
    int s = 0;
    for (; s + U <= S0; s += U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __half2float(__ushort_as_half(Vd[(size_t)(s + u) * kHd]));
#pragma unroll
        for (int u4 = 0; u4 < U; u4 += 4) {
            float4 pc[NC];   // probabilities of 4 positions per chain (broadcast reads)
#pragma unroll
            for (int c = 0; c < NC; ++c) pc[c] = *(const float4 *)(sc + rr[c] * Sw + s + u4);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                acc[c] = __builtin_fmaf(pc[c].x, v[u4], acc[c]);
                acc[c] = __builtin_fmaf(pc[c].y, v[u4 + 1], acc[c]);
                acc[c] = __builtin_fmaf(pc[c].z, v[u4 + 2], acc[c]);
                acc[c] = __builtin_fmaf(pc[c].w, v[u4 + 3], acc[c]);
            }
        }
    }
    for (; s < Smax; ++s) {   // the last < U common positions, then the longer rows' tails
        const float v = __half2float(__ushort_as_half(Vd[(size_t)s * kHd]));
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (s < Sc[c]) acc[c] = __builtin_fmaf(sc[rr[c] * Sw + s], v, acc[c]);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int qi = q0 + rr[c] / G;
        if (qi < n_q) out[(size_t)qi * H * kHd + (size_t)(hk * G + rr[c] % G) * kHd + d] = acc[c];
    }
}

// ---------------------------------------------------------------------------
// Prefill on f32 MFMA.  v_mfma_f32_16x16x1_4b (K = 1) adds one product to
// each output element per instruction, D = A*B + C rounded once, which is
// the fused multiply-add: a chain of them over d (or over positions) is the
// same sequential fma chain as the shaders' loops, bit for bit, at twice the
// VALU's fma rate.  Lane l supplies A[block l/16][row l%16] and B[block
// l/16][col l%16]; element (block b, row i, col j) of D is in lane
// j + 16(i/4), register 4b + i%4.
//
// The B operands come from copies of the cache laid out for them
// (attn_kv_tiles_kernel, one pass per call): per KV head
//   Kt [tile of 64 positions][d/4][64 positions][4 d]           f32
//   Vt [position/4][128 dims][4 positions]         f16
// zero past the last position, so a lane's 16-byte load is 4 steps of its
// operand (K with no conversion), and a wave's load is 1 KB contiguous.
//
// One workgroup of 16 waves (four per SIMD: a dependent MFMA chain issues at
// ~64% of the MFMA rate from one wave per SIMD, ~100% from four) per (16/G
// consecutive queries, KV head): 16 score rows, row r = query r/G, head r%G;
// query i attends over its position + 1 positions (causal).  The workgroups
// of one XCD share the K / V copies of at most two KV heads (mapping below).
//   scores: wave w takes the 64-position tiles w, w+16, ...: per d one
//     instruction covers the 16 rows (A = q[r][d], the same in the 4 blocks)
//     x 64 positions (B = K[tile + l][d]), 128 of them in order of d.
//     dot * scale goes to the row in LDS.
//   softmax: wave_softmax_row on row w, in place; positions past the row's
//     length become exact zeros.
//   P.V (sh/attention.wgsl:96-104): one chain per output over all of its
//     row's positions, in order of s, on v_mfma_f32_4x4x1_16b (one fused
//     step per output per instruction; lane l supplies A[block l/4][row
//     l%4], B[block l/4][col l%4] and holds D[block l/4][row i][col l%4] in
//     register i).  Wave w < 4 takes rows 8(w%2) .. +7 as two groups of
//     four (A = p[row][s], two chains per lane) and dims 64(w/2) .. +63 (B =
//     V[s][64(w/2) + l], one f16 operand for both groups), so the four
//     waves load each V element twice, 8 bytes per lane per 4 positions, and
//     hold kPvAhead 16-position batches of it in flight.  Positions that
//     every row of a wave covers run in whole batches; the last ones keep
//     each row's sum past its own length (a select per row).
// LDS (dynamic): q [16][132] | rows [16][Sw], Sw = the longest row rounded
// up to 64, plus 4, so that the 16 rows one read touches start in different
// banks.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kPfmWaves = 16;
constexpr int kPfmThreads = 64 * kPfmWaves;
constexpr int kPfmQs = kHd + 4;   // q row stride (floats)
constexpr int kPfmMaxS = 2368;    // longest row whose 16 rows fit the LDS (160 KB)
constexpr int kTileF4 = 64 * kHd / 4;    // float4 of one 64-position tile of Kt
constexpr int kVTileU4 = 64 * kHd / 8;   // uint4 of one 64-position tile of Vt
constexpr int kPvAhead = 3;              // P.V: V batches in flight per wave

__host__ __device__ inline int pfm_row_stride(int s_max) { return ((s_max + 63) & ~63) + 4; }
__host__ __device__ inline size_t pfm_smem(int s_max) {
    return (size_t)16 * (kPfmQs + pfm_row_stride(s_max)) * sizeof(float);
}

__device__ __forceinline__ v16f mfma_f32_k1(float a, float b, const v16f &c) {
    return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
}

// Kt and Vt tiles (layouts above) of positions [64t, 64t + 64) of KV head hk
// from the f16 caches; positions >= S are zeros.  Grid (tiles, Hkv).
__global__ __launch_bounds__(256) void attn_kv_tiles_kernel(const uint16_t *__restrict__ kc,
                                                            const uint16_t *__restrict__ vc,
                                                            int max_seq, int S, int ntile_ws,
                                                            float4 *__restrict__ Kt,
                                                            uint4 *__restrict__ Vt) {
    __shared__ uint4 ks[64][17], vs[64][17];   // 64 rows of 16 uint4, padded
    const int t = blockIdx.x, hk = blockIdx.y, tid = threadIdx.x;
    const uint4 *K4 = (const uint4 *)(kc + (size_t)hk * max_seq * kHd);
    const uint4 *V4 = (const uint4 *)(vc + (size_t)hk * max_seq * kHd);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = tid + 256 * k, row = i >> 4, c = i & 15, pos = 64 * t + row;
        uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
        if (pos < S) {
            kv = K4[(size_t)pos * 16 + c];
            vv = V4[(size_t)pos * 16 + c];
        }
        ks[row][c] = kv;
        vs[row][c] = vv;
    }
    __syncthreads();
    auto h2f = [](uint32_t h) { return __half2float(__ushort_as_half((uint16_t)h)); };
    float4 *kt = Kt + ((size_t)hk * ntile_ws + t) * kTileF4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {   // kt[c][p]: dims 4c .. 4c+3 of position p
        const int i = tid + 256 * k, c = i >> 6, pos = i & 63;
        const uint4 u = ks[pos][c >> 1];
        const uint32_t lo = (c & 1) ? u.z : u.x, hi = (c & 1) ? u.w : u.y;
        kt[i] = make_float4(h2f(lo & 0xffff), h2f(lo >> 16), h2f(hi & 0xffff), h2f(hi >> 16));
    }
    uint2 *vt = (uint2 *)(Vt + ((size_t)hk * ntile_ws + t) * kVTileU4);
#pragma unroll
    for (int k = 0; k < 8; ++k) {   // vt[g][d]: dim d of positions 4g .. 4g+3
        const int i = tid + 256 * k, g = i >> 7, d = i & (kHd - 1);
        uint32_t v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = ((const uint16_t *)&vs[4 * g + r][0])[d];
        vt[i] = make_uint2(v[0] | (v[1] << 16), v[2] | (v[3] << 16));
    }
}

template <int G>
__global__ __launch_bounds__(kPfmThreads) void attn_prefill_mfma_kernel(
    const float *__restrict__ q, const float4 *__restrict__ Kt, const uint4 *__restrict__ Vt,
    int ntile_ws, int pos0, int n_q, int H, float scale, float *__restrict__ out) {
    constexpr int QB = 16 / G;   // queries per workgroup
    extern __shared__ __align__(16) float smem[];
    float *qs = smem, *rows = smem + 16 * kPfmQs;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform loop control
    const int nblk = (n_q + QB - 1) / QB, Hkv = H / G;
    // Block b runs on XCD b % 8.  A KV head's query blocks j (longest rows
    // first) form 8 stripes j % 8 of equal work; XCD x takes stripes Hkv x ..
    // Hkv x + Hkv - 1 (in KV-head-major order: two KV heads at most, so its L2
    // holds their K / V copies), and its k-th block is stripe k % Hkv's block
    // k / Hkv, so each XCD still starts the longest rows first.
    const int x = (int)blockIdx.x & 7, k = (int)blockIdx.x >> 3;
    const int st = Hkv * x + k % Hkv, hk = st >> 3;
    const int j = (k / Hkv) * 8 + (st & 7);
    if (j >= nblk) return;   // the whole workgroup, before any barrier
    const int q0 = (nblk - 1 - j) * QB;
    const int Smax = pos0 + min(q0 + QB - 1, n_q - 1) + 1;
    const int ntile = (Smax + 63) >> 6;
    if (ntile > ntile_ws || Smax > kPfmMaxS) return;   // host checks too; never read out of range
    const int Sw = pfm_row_stride(Smax);
    auto row_len = [&](int r) { return pos0 + min(q0 + r / G, n_q - 1) + 1; };

    for (int i = tid; i < 16 * (kHd / 4); i += kPfmThreads) {
        const int r = i / (kHd / 4), c = i % (kHd / 4);
        const int qi = min(q0 + r / G, n_q - 1);
        *(float4 *)(qs + r * kPfmQs + 4 * c) =
            *(const float4 *)(q + ((size_t)qi * H + hk * G + r % G) * kHd + 4 * c);
    }
    lds_barrier();

    // ---- scores (sh/attention.wgsl:48-58) ----------------------------------
    {
        const float *qrow = qs + (lane & 15) * kPfmQs;
        for (int t = w; t < ntile; t += kPfmWaves) {
            const float4 *kt = Kt + ((size_t)hk * ntile_ws + t) * kTileF4 + lane;
            v16f acc = {};
            float4 kg[2][8];   // dims 32g .. 32g+31 of this lane's position, two groups
#pragma unroll
            for (int j = 0; j < 8; ++j) kg[0][j] = kt[64 * j];
#pragma unroll
            for (int g = 0; g < kHd / 32; ++g) {
                if (g + 1 < kHd / 32) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) kg[(g + 1) & 1][j] = kt[64 * (8 * (g + 1) + j)];
                }
                __builtin_amdgcn_sched_barrier(0);   // next group's loads ahead of these MFMAs
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int c = 8 * g + j;   // dims 4c .. 4c+3
                    const float4 qv = *(const float4 *)(qrow + 4 * c);
                    const float4 kv = kg[g & 1][j];
                    acc = mfma_f32_k1(qv.x, kv.x, acc);
                    acc = mfma_f32_k1(qv.y, kv.y, acc);
                    acc = mfma_f32_k1(qv.z, kv.z, acc);
                    acc = mfma_f32_k1(qv.w, kv.w, acc);
                }
            }
            const int r0 = 4 * (lane >> 4), p = 64 * t + (lane & 15);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int pos = p + 16 * (r >> 2);
                if (pos < Smax) rows[(r0 + (r & 3)) * Sw + pos] = acc[r] * scale;
            }
        }
    }
    lds_barrier();

    // ---- softmax (sh/softmax.wgsl:25-80) ------------------------------------
    for (int r = w; r < 16; r += kPfmWaves) {
        const int S = row_len(r);
        // wave_softmax_row for rows of up to kPfmMaxS positions (register-held row)
        float *row = rows + r * Sw;
        const int nj = (S + 255) >> 8;
        if (nj <= 1) softmax_row_regs<1, true>(row, row, S, Sw, lane);
        else if (nj <= 2) softmax_row_regs<2, true>(row, row, S, Sw, lane);
        else if (nj <= 4) softmax_row_regs<4, true>(row, row, S, Sw, lane);
        else if (nj <= 6) softmax_row_regs<6, true>(row, row, S, Sw, lane);
        else if (nj <= 8) softmax_row_regs<8, true>(row, row, S, Sw, lane);
        else softmax_row_regs<(kPfmMaxS + 255) / 256, true>(row, row, S, Sw, lane);
        for (int s = S + lane; s < Sw; s += 64) row[s] = 0.0f;   // same wave: in order
    }
    lds_barrier();

    // ---- P.V (sh/attention.wgsl:96-104): one chain per output ---------------
    if (w < 4) {
        // wave w: rows 8(w&1) .. +7 as two groups of four (chains a and b,
        // one V operand for both) x dims 64(w>>1) .. +63; lane l: dim d
        const int r0 = 8 * (w & 1), d = 64 * (w >> 1) + lane;
        int len[8];   // lengths non-decreasing in the row
#pragma unroll
        for (int i = 0; i < 8; ++i) len[i] = row_len(r0 + i);
        const int e = len[0] & ~15;   // whole batches every row of the wave covers
        const int s_end = len[7];
        const int s_last = 64 * ntile - 16;   // last batch start inside Vt and the rows
        const uint2 *vt = (const uint2 *)(Vt + (size_t)hk * ntile_ws * kVTileU4) + d;
        const float *pa = rows + (r0 + (lane & 3)) * Sw, *pb = pa + 4 * Sw;
        // 16 positions per batch: V (global) kPvAhead batches ahead in a ring
        // of registers, p (LDS) at its batch (batch starts past the rows are
        // clamped)
        constexpr int NV = kPvAhead + 1;
        uint2 vr[NV][4];
        float4 qa[4], qb[4];
        auto loadv = [&](uint2 (&vv)[4], int s) {
            const int sb = min(s, s_last);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) vv[j] = vt[(size_t)(sb / 4 + j) * kHd];
            __builtin_amdgcn_sched_barrier(0);
        };
        auto loadp = [&](int s) {
            const int sb = min(s, s_last);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qa[j] = *(const float4 *)(pa + sb + 4 * j);
                qb[j] = *(const float4 *)(pb + sb + 4 * j);
            }
        };
        auto vk = [](const uint2 &u, int k) {   // position k of the lane's quad
            const uint32_t wd = k < 2 ? u.x : u.y;
            return __half2float(__ushort_as_half((uint16_t)((k & 1) ? wd >> 16 : wd & 0xffffu)));
        };
        v4f a = {0.0f, 0.0f, 0.0f, 0.0f}, b = {0.0f, 0.0f, 0.0f, 0.0f};
        // the batch's 16 V values converted first (while its p reads land),
        // then its 32 steps back to back
        auto run = [&](const uint2 (&vv)[4]) {
            float vf[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) vf[i] = vk(vv[i >> 2], i & 3);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float pa4[4] = {qa[j].x, qa[j].y, qa[j].z, qa[j].w};
                const float pb4[4] = {qb[j].x, qb[j].y, qb[j].z, qb[j].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    a = __builtin_amdgcn_mfma_f32_4x4x1f32(pa4[k], vf[4 * j + k], a, 0, 0, 0);
                    b = __builtin_amdgcn_mfma_f32_4x4x1f32(pb4[k], vf[4 * j + k], b, 0, 0, 0);
                }
            }
        };
        // the batch at st, each row's sum kept past its own length
        auto tail = [&](const uint2 (&vv)[4], int st) {
            if (st >= s_end) return;
            loadp(st);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float pa4[4] = {qa[j].x, qa[j].y, qa[j].z, qa[j].w};
                const float pb4[4] = {qb[j].x, qb[j].y, qb[j].z, qb[j].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int s = st + 4 * j + k;
                    const float v = vk(vv[j], k);
                    const v4f ra = __builtin_amdgcn_mfma_f32_4x4x1f32(pa4[k], v, a, 0, 0, 0);
                    const v4f rb = __builtin_amdgcn_mfma_f32_4x4x1f32(pb4[k], v, b, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        a[i] = s < len[i] ? ra[i] : a[i];
                        b[i] = s < len[4 + i] ? rb[i] : b[i];
                    }
                }
            }
        };
        // batch n sits in vr[n % NV].  Passes of NV batches with no branch
        // inside (ring indices are constants, and the loads stay in flight
        // across batches), then the r < NV whole batches left, then the
        // tails: batches r and r + 1 (the positions past e, fewer than 32)
#pragma unroll
        for (int i = 0; i < NV - 1; ++i) loadv(vr[i], 16 * i);
        int s0 = 0;
        for (; s0 + 16 * NV <= e; s0 += 16 * NV) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                loadv(vr[(i + NV - 1) % NV], s0 + 16 * (i + NV - 1));
                loadp(s0 + 16 * i);
                run(vr[i]);
            }
        }
        const int r = (e - s0) >> 4;
#pragma unroll
        for (int i = 0; i < NV - 1; ++i) {
            if (i < r) {
                loadv(vr[(i + NV - 1) % NV], s0 + 16 * (i + NV - 1));
                loadp(s0 + 16 * i);
                run(vr[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (i == r) {
                tail(vr[i], s0 + 16 * i);
                tail(vr[(i + 1) % NV], s0 + 16 * (i + 1));
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = r0 + i, qi = q0 + r / G;
            if (qi < n_q) out[((size_t)qi * H + hk * G + r % G) * kHd + d] = i < 4 ? a[i] : b[i - 4];
        }
    }
}

// ---------------------------------------------------------------------------
// Decode, one kernel: two 1024-thread workgroups per KV head (one per half of
// the 128 dims) each compute the scores and softmax of its G <= 4 query
// heads, then the P.V sums of their half of the dims, so a layer's attention
// is one launch and the scores never leave LDS.  Same arithmetic as the
// two-kernel path (and the shaders).  Positions are taken in chunks: 256 K
// rows (wave w: head w%4, positions (w/4)*64 + lane of the chunk), then 256 V
// rows staged as f32 [64 dims][256 + 4 pad]; wave g < G sums head g (lane =
// one dim), so the summing waves sit on four SIMDs.
// Rows past the cache length are neither loaded nor used.
// The scores are computed twice (once per half), which costs little next to
// the P.V chains it halves.  The host picks this kernel or the two-kernel path
// by position.
// LDS (dynamic): buf 69632 B (K chunk [256][17 uint4] | V chunk [64][260] f32)
// | scores [G][Spad_max] f32.
// ---------------------------------------------------------------------------
constexpr int kFusedKC = 256;               // K rows per chunk
constexpr int kFusedVC = 256;               // V rows per chunk
constexpr int kFusedVS = kFusedVC + 4;      // padded V row (floats)
constexpr size_t kFusedBuf = (size_t)kFusedKC * 17 * 16;   // 69632 B >= 64*260*4
static_assert((size_t)(kHd / 2) * kFusedVS * 4 <= kFusedBuf, "V chunk must fit the K chunk buffer");

__host__ __device__ inline size_t attn_fused_smem(int G, int max_seq) {
    return kFusedBuf + (size_t)G * ((max_seq + 3) & ~3) * 4;
}

// K rows c0 .. c0+255 of the chunk (thread i: row i/16, uint4 column i%16),
// clamped to the cache length (rows past it are staged but never used).
// A wave whose 4 rows all lie past S loads nothing (a wave-uniform branch).
__device__ __forceinline__ void fused_load_k(u32x4_t (&kt)[4], const uint4 *__restrict__ K4, int c0,
                                             int S, int tid) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = tid + 1024 * k;
        const int wave_row = c0 + ((i & ~63) >> 4);   // the wave's first row
        kt[k] = wave_row < S
                    ? *(const u32x4_t *)(K4 + (size_t)min(c0 + (i >> 4), S - 1) * 16 + (i & 15))
                    : u32x4_t{0, 0, 0, 0};
    }
}

// V rows of a 256-position chunk for one half of the dims: thread (wave w,
// lane l) takes rows c0 + 8q .. +7, q = 2w + l/32, and the f16 pair l % 32
// of the half (row-coalesced 128-byte loads); clamped to the cache length,
// and a wave whose 16 rows all lie past S loads nothing (wave-uniform).
__device__ __forceinline__ void fused_load_v(uint32_t (&vr)[8], const uint32_t *__restrict__ V2,
                                             int c0, int S, int w, int lane) {
    const int q = 2 * w + (lane >> 5), p = lane & 31;
    const bool any = c0 + 16 * w < S;   // wave-uniform
#pragma unroll
    for (int j = 0; j < 8; ++j)
        vr[j] = any ? V2[(size_t)min(c0 + 8 * q + j, S - 1) * (kHd / 2) + p] : 0u;
}

// The staged rows as f32 V^T [dim][position]: dims 2p, 2p+1 of the half,
// positions 8q .. 8q+7 of the chunk (two float4 per dim).
__device__ __forceinline__ void fused_stage_v(float *vt, const uint32_t (&vr)[8], int w, int lane) {
    const int q = 2 * w + (lane >> 5), p = lane & 31;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float2 f0 = __half22float2(*(const __half2 *)&vr[4 * h]);
        const float2 f1 = __half22float2(*(const __half2 *)&vr[4 * h + 1]);
        const float2 f2 = __half22float2(*(const __half2 *)&vr[4 * h + 2]);
        const float2 f3 = __half22float2(*(const __half2 *)&vr[4 * h + 3]);
        *(float4 *)(vt + (2 * p) * kFusedVS + 8 * q + 4 * h) = make_float4(f0.x, f1.x, f2.x, f3.x);
        *(float4 *)(vt + (2 * p + 1) * kFusedVS + 8 * q + 4 * h) = make_float4(f0.y, f1.y, f2.y, f3.y);
    }
}

template <int G>
__global__ __launch_bounds__(1024) void attn_fused_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    const int *__restrict__ pos_ptr, int max_seq, float scale, float *__restrict__ out) {
    static_assert(G == 1 || G == 2 || G == 4, "fused decode attention: G <= 4");
    extern __shared__ __align__(16) int8_t smem_f[];
    uint4 (*ks)[17] = (uint4 (*)[17])smem_f;
    float *vt = (float *)smem_f;
    const int spad_max = (max_seq + 3) & ~3;
    float *sc = (float *)(smem_f + kFusedBuf);           // [G][spad_max]
    const int pos = *pos_ptr;
    if (pos < 0 || pos >= max_seq) return;
    const int S = pos + 1;
    const int Spad = (S + 3) & ~3;
    const int hk = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint4 *K4 = (const uint4 *)(kc + (size_t)hk * max_seq * kHd);
    const int half = blockIdx.y;   // this workgroup's half of the dims
    const uint32_t *V2 = (const uint32_t *)(vc + (size_t)hk * max_seq * kHd) + half * 32;

    // Up to 512 positions every K and V load is issued here, so the kernel
    // waits for memory once; longer caches refill each register set as soon
    // as it is consumed.
    u32x4_t ka[4], kb[4];   // native vectors: HIP's uint4 struct copies land in scratch
    uint32_t va[8], vb[8];
    fused_load_k(ka, K4, 0, S, tid);
    fused_load_k(kb, K4, kFusedKC, S, tid);
    fused_load_v(va, V2, 0, S, w, lane);
    fused_load_v(vb, V2, kFusedVC, S, w, lane);

    // ---- scores ------------------------------------------------------------
    // this wave's head and position group: consecutive waves (which sit on
    // different SIMDs) take different heads, so a partly filled chunk still
    // spreads its chains over the four SIMDs
    const int g = w & 3, pg = w >> 2;
    // 128-term chain of position c0 + pg*64 + lane: the K row from LDS in
    // quarters (the next quarter read while one is summed), the head's q row
    // (wave-uniform) through scalar loads, so each step is one v_fma_mix with
    // an SGPR operand
    auto chain = [&](int c0) {
        const int s = c0 + pg * 64 + lane;
        if (g < G && s < S) {
            const float *__restrict__ qg =
                q + (size_t)(hk * G + __builtin_amdgcn_readfirstlane(g)) * kHd;
            const uint4 *row = ks[pg * 64 + lane];
            float dot = 0.0f;
            uint4 kq[2][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) kq[0][i] = row[i];
#pragma unroll
            for (int quarter = 0; quarter < 4; ++quarter) {
                if (quarter < 3) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) kq[(quarter + 1) & 1][i] = row[4 * (quarter + 1) + i];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 kr = kq[quarter & 1][i];
                    const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
                    const int d0 = 32 * quarter + 8 * i;
#pragma unroll
                    for (int k2 = 0; k2 < 4; ++k2) {
                        const float k0 = __half2float(__ushort_as_half((uint16_t)(kw[k2] & 0xffffu)));
                        const float k1 = __half2float(__ushort_as_half((uint16_t)(kw[k2] >> 16)));
                        dot = __builtin_fmaf(qg[d0 + 2 * k2], k0, dot);
                        dot = __builtin_fmaf(qg[d0 + 2 * k2 + 1], k1, dot);
                    }
                }
            }
            sc[g * spad_max + s] = dot * scale;
        }
    };
    auto store_k = [&](const u32x4_t (&kt)[4]) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = tid + 1024 * k;
            *(u32x4_t *)&ks[i >> 4][i & 15] = kt[k];
        }
    };
    for (int c0 = 0; c0 < S; c0 += 2 * kFusedKC) {
        if (c0) lds_barrier();   // the previous chunk's rows are consumed
        store_k(ka);
        lds_barrier();
        fused_load_k(ka, K4, c0 + 2 * kFusedKC, S, tid);   // nothing past S
        chain(c0);
        const int c1 = c0 + kFusedKC;
        if (c1 < S) {
            lds_barrier();
            store_k(kb);
            lds_barrier();
            fused_load_k(kb, K4, c1 + 2 * kFusedKC, S, tid);
            chain(c1);
        }
    }
    lds_barrier();

    // ---- softmax: wave g < G owns head g's row ------------------------------
    if (w < G) wave_softmax_row(sc + w * spad_max, sc + w * spad_max, S, Spad, lane, true);

    // ---- P.V: wave g < G sums head g, lane = dim 64*half + lane --------------
    // One chain over every position (sh/attention.wgsl:96-104), continued
    // from chunk to chunk.  Chunks alternate between the two register sets,
    // each refilled (two chunks ahead) once staged.
    float acc = 0.0f;
    for (int c0 = 0; c0 < S; c0 += 2 * kFusedVC) {
        lds_barrier();   // softmax done / K rows or the previous V chunk consumed
        fused_stage_v(vt, va, w, lane);
        lds_barrier();
        fused_load_v(va, V2, c0 + 2 * kFusedVC, S, w, lane);
        if (w < G)
            acc = pv_chain(sc + w * spad_max + c0, vt + lane * kFusedVS, min(kFusedVC, S - c0), acc);
        const int c1 = c0 + kFusedVC;
        if (c1 < S) {
            lds_barrier();
            fused_stage_v(vt, vb, w, lane);
            lds_barrier();
            fused_load_v(vb, V2, c1 + 2 * kFusedVC, S, w, lane);
            if (w < G)
                acc = pv_chain(sc + w * spad_max + c1, vt + lane * kFusedVS, min(kFusedVC, S - c1), acc);
        }
    }
    if (w < G) out[(size_t)(hk * G + w) * kHd + 64 * half + lane] = acc;
}

// Grids of the per-head decode kernels: workgroups go to the 8 XCDs in turn,
// so the G workgroups of a KV head take block indices congruent mod 8 and
// run on one XCD, whose L2 then serves the K/V rows they share.  Block x ->
// KV head 8 (x / 8G) + x % 8, head G * (KV head) + (x / 8) % G; blocks past
// the last KV head have no head (-1) and return at once.
__host__ __device__ inline int head_grid_blocks(int G, int Hkv) { return 8 * G * ((Hkv + 7) / 8); }
__device__ inline int head_of_block(int x, int G, int Hkv) {
    const int hk = 8 * (x / (8 * G)) + x % 8;
    return hk < Hkv ? hk * G + (x / 8) % G : -1;
}

// ---------------------------------------------------------------------------
// Decode, one workgroup per query head (grid: heads x sequences), 256
// threads, up to 256 cached positions, for caches of fewer than 256 rows
// (the head256 kernel below stages whole 256-row blocks).  Built for latency:
//  - thread t computes the score of position t from its own K row,
//    loaded straight into registers at kernel start and clamped to the cache
//    extent (rows at or past S are stale but in bounds and never used), so
//    no load waits for the position; the head's q row is an SGPR operand of
//    each v_fma_mix step (scalar loads), and its eight cache lines are
//    fetched while the K rows are in flight;
//  - the softmax runs on all four waves in the shader's order: thread t's
//    partial exp(x_t - max), then the halving tree (strides 128 and 64
//    through LDS, 32 .. 1 in one wave);
//  - P.V: waves 0 and 1 sum dim 64 w + lane over every position in order,
//    the V elements loaded into registers with 16-bit loads one 64-position
//    chunk ahead (no LDS staging).
// Same arithmetic as the other decode kernels, so the same bits.
// ---------------------------------------------------------------------------
constexpr int kHeadChunk = 64;   // V positions per register chunk

__global__ __launch_bounds__(256) void attn_head_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    const int *__restrict__ pos_ptr, int G, int Hkv, int max_seq, float scale,
    float *__restrict__ out, size_t kv_stride, int pos_stride) {
    constexpr int NJ = 1;   // positions per thread
    __shared__ __align__(16) float pr[256 * NJ];   // probabilities
    __shared__ float red[256];
    __shared__ float wmax[4];
    __shared__ float inv_s;
    const int h = head_of_block(blockIdx.x, G, Hkv), z = blockIdx.y, H = G * Hkv;
    if (h < 0) return;
    const int hk = h / G;
    const float *__restrict__ qh = q + ((size_t)z * H + h) * kHd;
    kc += (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    vc += (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    u32x4_t kr[NJ][16];   // K rows tid + 256 j, 128 f16 each
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const u32x4_t *row = (const u32x4_t *)(kc + (size_t)min(tid + 256 * j, max_seq - 1) * kHd);
#pragma unroll
        for (int i = 0; i < 16; ++i) kr[j][i] = row[i];
    }
    __builtin_amdgcn_sched_barrier(0);
    float qw[kHd / 16];   // one dword per 64-byte line of the q row
#pragma unroll
    for (int i = 0; i < kHd / 16; ++i) qw[i] = qh[16 * i];
    const int pos = pos_ptr[(size_t)z * pos_stride];
    asm volatile("" ::"s"(pos), "s"(qw[0]), "s"(qw[1]), "s"(qw[2]), "s"(qw[3]), "s"(qw[4]),
                 "s"(qw[5]), "s"(qw[6]), "s"(qw[7]));
    // a position out of range (the host checks it too) computes one position
    // and stores nothing
    const bool valid = pos >= 0 && pos < max_seq && pos < 256 * NJ;
    const int S = valid ? pos + 1 : 1;

    // this wave's P.V block and dim; its first V chunk goes out now.  V
    // chunks are read unclamped (64 rows from a chunk start below S, so at
    // most 63 rows past the cache extent: the caller pads the cache
    // allocation by kHeadChunk rows), which keeps each load one instruction
    // with an immediate offset.
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int d = 64 * (w & 1) + lane, blk = wu >> 1;
    const int b0 = 256 * blk;
    const int nb = min(max(S - b0, 0), 256);   // positions of the block (wave-uniform)
    const uint16_t *__restrict__ vcol = vc + d;
    auto load_v = [&](uint16_t (&dst)[kHeadChunk], int s0) {
        const uint16_t *__restrict__ vrow = vcol + (size_t)s0 * kHd;
#pragma unroll
        for (int i = 0; i < kHeadChunk; ++i) dst[i] = vrow[i * kHd];
    };
    const bool pv_wave = blk == 0;   // waves 0 and 1
    uint16_t va[kHeadChunk], vb[kHeadChunk];
    load_v(va, min(b0, S - 1));   // (every wave: a conditional load would wait at the join)

    // ---- scores: 128-term chains in order of d (sh/attention.wgsl:48-58) ----
    float x[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const u32x4_t kv = kr[j][i];
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const uint32_t kw = kv[k2];
                const float k0 = __half2float(__ushort_as_half((uint16_t)(kw & 0xffffu)));
                const float k1 = __half2float(__ushort_as_half((uint16_t)(kw >> 16)));
                dot = __builtin_fmaf(qh[8 * i + 2 * k2], k0, dot);
                dot = __builtin_fmaf(qh[8 * i + 2 * k2 + 1], k1, dot);
            }
        }
        x[j] = dot * scale;
    }

    // ---- softmax (sh/softmax.wgsl:25-80) ------------------------------------
    float m = -3.402823e+38f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        if (tid + 256 * j < S) m = fmaxf(m, x[j]);
    m = wave_max_dpp(m);
    if (lane == 0) wmax[w] = m;
    lds_barrier();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    float e[NJ], part = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        e[j] = tid + 256 * j < S ? oxb_expf(x[j] - m) : 0.0f;
        part = part + e[j];   // thread t's strided partial, in order of j
    }
    red[tid] = part;
    lds_barrier();
    if (w == 0) {
        const float a = red[lane] + red[lane + 128];        // stride 128, t = lane
        const float c = red[lane + 64] + red[lane + 192];   // stride 128, t = lane + 64
        const float sum = wave_tree_sum(a + c);             // stride 64, then 32 .. 1
        if (lane == 0) inv_s = 1.0f / sum;
    }
    lds_barrier();
    const float inv = inv_s;
#pragma unroll
    for (int j = 0; j < NJ; ++j) pr[tid + 256 * j] = e[j] * inv;   // 0 past S
    lds_barrier();

    // ---- P.V (sh/attention.wgsl:96-104), this wave's block ------------------
    float acc = 0.0f;
    auto sum_chunk = [&](const uint16_t (&v)[kHeadChunk], int s0, int n) {
        const float *p = pr + s0;
        if (n == kHeadChunk) {
#pragma unroll
            for (int i = 0; i < kHeadChunk; i += 4) {
                const float4 p4 = *(const float4 *)(p + i);
                acc = __builtin_fmaf(p4.x, __half2float(__ushort_as_half(v[i])), acc);
                acc = __builtin_fmaf(p4.y, __half2float(__ushort_as_half(v[i + 1])), acc);
                acc = __builtin_fmaf(p4.z, __half2float(__ushort_as_half(v[i + 2])), acc);
                acc = __builtin_fmaf(p4.w, __half2float(__ushort_as_half(v[i + 3])), acc);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kHeadChunk; i += 4) {
                const float4 p4 = *(const float4 *)(p + i);
                const float pp[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float t = __builtin_fmaf(pp[k], __half2float(__ushort_as_half(v[i + k])), acc);
                    acc = i + k < n ? t : acc;
                }
            }
        }
    };
    // The block's (up to) four chunks as straight-line code, each chunk
    // loaded one ahead and unconditionally (its start clamped below S): a
    // load under a branch or carried around a loop makes the compiler copy
    // its registers where the paths join, which waits for the load on the
    // spot.  Only the sums are conditional.
    if (pv_wave) {
        load_v(vb, min(b0 + kHeadChunk, S - 1));
        if (nb > 0) sum_chunk(va, b0, min(kHeadChunk, nb));
        load_v(va, min(b0 + 2 * kHeadChunk, S - 1));
        if (nb > kHeadChunk) sum_chunk(vb, b0 + kHeadChunk, min(kHeadChunk, nb - kHeadChunk));
        load_v(vb, min(b0 + 3 * kHeadChunk, S - 1));
        if (nb > 2 * kHeadChunk)
            sum_chunk(va, b0 + 2 * kHeadChunk, min(kHeadChunk, nb - 2 * kHeadChunk));
        if (nb > 3 * kHeadChunk)
            sum_chunk(vb, b0 + 3 * kHeadChunk, nb - 3 * kHeadChunk);
    }
    if (blk == 0 && valid) out[((size_t)z * H + h) * kHd + d] = acc;
}

// ---------------------------------------------------------------------------
// Decode, one workgroup per query head, caches of up to 256 positions:
//  - the q row and the position, then every K and V load before the first
//    is waited for: the 256 rows (thread i: uint4 i + 256 k of each,
//    coalesced, clamped to the cache, so the loads are branch-free and do not
//    wait for the position; rows at or past S are never used);
//  - K staged in LDS as [256][17] uint4 (padded rows), q as [128] f32; the
//    V loads are still landing while thread t runs the 128-step score chain
//    of position t, q read as LDS broadcasts three 8-term groups ahead (no
//    scalar loads: their out-of-order returns force full waits in the chain);
//  - V staged row-major [256][64] dwords after the chain;
//  - softmax in the shader's order with two exchanges: every wave forms the
//    row sum from the 256 partials itself;
//  - P.V on waves 0 (even dims) and 1 (odd dims), lane j summing dim 2j + w:
//    each LDS read gives it two positions of its dword (ds_read2st64), the
//    probabilities four at a time; 4-position blocks read three ahead (12
//    LDS reads in flight, within the 15 the counter tracks), each step one
//    v_fma_mix on the dword's low or high half.
// Same arithmetic as the other forms, so the same bits.
// ---------------------------------------------------------------------------
constexpr int kH256Rows = 256;
constexpr size_t kH256KBytes = (size_t)kH256Rows * 17 * 16;   // K rows, padded
constexpr size_t kH256VBytes = (size_t)kH256Rows * kHd * 2;   // V rows
constexpr size_t kH256Lds = kH256KBytes + kH256VBytes + (kHd + 256 + 256 + 8) * 4;

// P.V of one wave: lane j's chain over the S positions (S <= ROWS) of dim
// 2j + HI, in order of s; vcol = the V rows' dword j (row stride 64 dwords)
template <bool HI, int ROWS>
__device__ __forceinline__ float pv_head(const uint32_t *vcol, const float *pr, int S) {
    float acc = 0.0f;
    uint32_t V[4][4];
    float4 P[4];
    auto ld = [&](int b, int s) {   // the block at s (clamped into the rows) into ring slot b
        s = min(s, ROWS - 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) V[b][k] = vcol[(s + k) * (kHd / 2)];
        P[b] = *(const float4 *)(pr + s);
    };
    ld(0, 0);
    ld(1, 4);
    ld(2, 8);
    // fully unrolled (exits are wave-uniform branches): across a loop's back
    // edge the compiler waits for every outstanding LDS read (lgkmcnt(0)),
    // which would drain the ring once per 16 positions
    int s0 = 0;
#pragma unroll
    for (int it = 0; it < ROWS / 16; ++it) {
        if (s0 + 16 > S) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            ld((j + 3) & 3, s0 + 4 * j + 12);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv4<HI, true>(acc, V[j], P[j]);
        }
        s0 += 16;
    }
    // the last S - s0 < 16 positions: slots 0..2 hold blocks s0, s0 + 4, s0 + 8
    ld(3, s0 + 12);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = S - s0 - 4 * j;
        if (n >= 4) acc = pv4<HI, true>(acc, V[j], P[j]);
        else if (n > 0) acc = pv4<HI, false>(acc, V[j], P[j], n);
    }
    return acc;
}

// P.V of one wave over the octet copy staged in LDS (vo: the lane's uint4 of
// octet 0; octets kHd uint4 apart): one chain over S <= ROWS positions in
// order of s, 8 positions per 16-byte read, octets read three ahead, fully
// unrolled with wave-uniform exits (as pv_head).
template <int ROWS>
__device__ __forceinline__ float pv_head_oct(const uint4 *vo, const float *pr, int S) {
    constexpr int NO = ROWS / 8;
    float acc = 0.0f;
    uint4 V[4];
    float4 Pa[4], Pb[4];
    auto ld = [&](int b, int o) {   // octet o (clamped into the rows) into entry b
        o = min(o, NO - 1);
        V[b] = vo[o * kHd];
        Pa[b] = *(const float4 *)(pr + 8 * o);
        Pb[b] = *(const float4 *)(pr + 8 * o + 4);
    };
    ld(0, 0);
    ld(1, 1);
    ld(2, 2);
    int o0 = 0;
#pragma unroll
    for (int it = 0; it < NO / 4; ++it) {
        if (8 * (o0 + 4) > S) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            ld((j + 3) & 3, o0 + j + 3);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv8<true>(acc, V[j], Pa[j], Pb[j]);
        }
        o0 += 4;
    }
    // the last S - 8 o0 < 32 positions: entries 0..2 hold octets o0 .. o0 + 2
    ld(3, o0 + 3);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = S - 8 * (o0 + j);
        if (n >= 8) acc = pv8<true>(acc, V[j], Pa[j], Pb[j]);
        else if (n > 0) acc = pv8<false>(acc, V[j], Pa[j], Pb[j], n);
    }
    return acc;
}

// OCT: vc is the octet copy of V (v8_index; sequence z at vc + z * kv8_stride),
// staged as it is and summed 8 positions per read (pv_head_oct), wave w taking
// dims 64 w .. 64 w + 63.
template <bool OCT>
__global__ __launch_bounds__(256) void attn_head256_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    const int *__restrict__ pos_ptr, int G, int Hkv, int max_seq, float scale,
    float *__restrict__ out, size_t kv_stride, int pos_stride, size_t kv8_stride) {
    // all kernel arguments in SGPRs up front: read where they are used, the
    // late ones are further kernarg round trips before the position's load
    asm volatile("" ::"s"(q), "s"(kc), "s"(vc), "s"(pos_ptr), "s"(G), "s"(Hkv), "s"(max_seq),
                 "s"(scale), "s"(out), "s"(kv_stride), "s"(pos_stride));
    extern __shared__ __align__(16) int8_t smem_h[];
    u32x4_t (*ks)[17] = (u32x4_t (*)[17])smem_h;
    u32x4_t *vs4 = (u32x4_t *)(smem_h + kH256KBytes);              // V [256][64] dwords
    const uint32_t *vs = (const uint32_t *)vs4;
    float *qs = (float *)(smem_h + kH256KBytes + kH256VBytes);      // q [128]
    float *pr = qs + kHd;                                           // probabilities [256]
    float *red = pr + 256;                                          // partial sums [256]
    float *wmax = red + 256;                                        // [4]
    const int h = head_of_block(blockIdx.x, G, Hkv), z = blockIdx.y, H = G * Hkv;
    if (h < 0) return;
    const int hk = h / G;
    const float *__restrict__ qh = q + ((size_t)z * H + h) * kHd;
    kc += (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    vc += OCT ? (size_t)z * kv8_stride + (size_t)hk * v8_head_elems(max_seq, kHd)
              : (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    const int pos = pos_ptr[(size_t)z * pos_stride];
    // the q row first (the oldest load: its wait leaves the K and V loads in
    // flight); every thread loads, so no load sits under a branch
    const float4 q4 = ((const float4 *)qh)[tid & 31];
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t kt[16], vt[16];
    const u32x4_t *__restrict__ K4 = (const u32x4_t *)kc;
    const u32x4_t *__restrict__ V4 = (const u32x4_t *)vc;
    // rows clamped to the cache, not to S, so these loads do not wait for the
    // position: rows at or past S are never used (their scores are masked,
    // and the P.V chains stop at S)
#pragma unroll
    for (int k = 0; k < 16; ++k) kt[k] = K4[min(16 * k + (tid >> 4), max_seq - 1) * 16 + (tid & 15)];
    if constexpr (OCT) {   // the first 32 octets (max_seq >= 256: all in the copy)
#pragma unroll
        for (int k = 0; k < 16; ++k) vt[k] = V4[256 * k + tid];
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k)
            vt[k] = V4[min(16 * k + (tid >> 4), max_seq - 1) * 16 + (tid & 15)];
    }
    __builtin_amdgcn_sched_barrier(0);
    const bool valid = pos >= 0 && pos < kH256Rows && pos < max_seq;
    const int S = valid ? pos + 1 : 1;
#pragma unroll
    for (int k = 0; k < 16; ++k) ks[16 * k + (tid >> 4)][tid & 15] = kt[k];
    // every thread stores (8 store the same float4 to each slot): a store
    // under a branch would take its load along
    *(float4 *)(qs + 4 * (tid & 31)) = q4;
    lds_barrier();

    // ---- score of position tid: 128 terms in order of d -----------------
    float x;
    {
        // group i: 8 terms, one K uint4 and two q float4 from LDS, read
        // three groups ahead (9 LDS reads in flight, in order)
        constexpr int kAhead = 3;
        u32x4_t kr[16];
        float4 qa[16], qb[16];
        auto ld = [&](int i) {
            kr[i] = ks[tid][i];
            qa[i] = *(const float4 *)(qs + 8 * i);
            qb[i] = *(const float4 *)(qs + 8 * i + 4);
        };
#pragma unroll
        for (int i = 0; i < kAhead; ++i) ld(i);
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            if (i + kAhead < 16) ld(i + kAhead);
            __builtin_amdgcn_sched_barrier(0);
            const float qv[8] = {qa[i].x, qa[i].y, qa[i].z, qa[i].w,
                                 qb[i].x, qb[i].y, qb[i].z, qb[i].w};
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const uint32_t kw = kr[i][k2];
                const float k0 = __half2float(__ushort_as_half((uint16_t)(kw & 0xffffu)));
                const float k1 = __half2float(__ushort_as_half((uint16_t)(kw >> 16)));
                dot = __builtin_fmaf(qv[2 * k2], k0, dot);
                dot = __builtin_fmaf(qv[2 * k2 + 1], k1, dot);
            }
        }
        x = dot * scale;
    }
    // ---- V rows (published by the next barrier) ----------------------------
#pragma unroll
    for (int k = 0; k < 16; ++k) vs4[tid + 256 * k] = vt[k];

    // ---- softmax (sh/softmax.wgsl:25-80) --------------------------------------
    float m = tid < S ? x : -3.402823e+38f;
    m = wave_max_dpp(m);
    if (lane == 0) wmax[w] = m;
    lds_barrier();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float e = tid < S ? oxb_expf(x - m) : 0.0f;
    red[tid] = e;   // thread t's strided partial: one position (0 + e = e)
    lds_barrier();
    float inv;
    {   // the halving tree, in every wave (identical values)
        const float a = red[lane] + red[lane + 128];
        const float c = red[lane + 64] + red[lane + 192];
        inv = 1.0f / wave_tree_sum(a + c);
    }
    pr[tid] = e * inv;   // 0 past S
    lds_barrier();

    // ---- P.V (sh/attention.wgsl:96-104) on waves 0 and 1 ----------------------
    if (w < 2) {
        if constexpr (OCT) {
            const float acc =
                pv_head_oct<kH256Rows>((const uint4 *)vs4 + 64 * w + lane, pr, S);
            if (valid) out[((size_t)z * H + h) * kHd + 64 * w + lane] = acc;
        } else {
            const float acc = w == 0 ? pv_head<false, kH256Rows>(vs + lane, pr, S)
                                     : pv_head<true, kH256Rows>(vs + lane, pr, S);
            if (valid) out[((size_t)z * H + h) * kHd + 2 * lane + w] = acc;
        }
    }
}

// ---------------------------------------------------------------------------
// A decode step's q|k|v BitLinear and the attention in one launch, for caches
// of 256+ rows with the query below position 256.  The grid is the q|k|v
// GEMV's: one 16-row tile of the fused weights per workgroup (512 threads):
//  - waves 0-3: the tile's GEMV as the GEMV kernel computes it (attn_norm
//    RMSNorm, int8 quantize, ternary dot, RoPE on q and k, f16 K / V append
//    with the V octet copy), the rows stored to q_out and the caches;
//  - arrival: each tile counts itself, on an agent-scope counter per query
//    head, for the heads its rows feed (a q tile: its head; a k or v tile:
//    the G query heads of its KV head), 24 tiles per head; the workgroup that
//    brings a head's count to 24 resets it to 0 and computes that head's
//    attention (nobody waits: the last one to finish does the work);
//  - the candidate: the workgroup of each head's last q tile is launched
//    last (the k and v tiles first) and its waves 4-7 load the head's K rows
//    and V octets of positions 0..255 into LDS while waves 0-3 run the GEMV,
//    so that when it completes the head, as it mostly does, only q and row
//    pos are still to read; any other workgroup that completes a head loads
//    K and V itself first.  The candidates of one KV head share block
//    indices mod 8 (one XCD, one L2).
//  - the attention: as attn_head256_kernel<true> (thread t scores position
//    t; softmax; P.V over the octets on waves 0 and 1), with row pos of K and
//    V read back from the caches.  K row t's chunk i sits in LDS slot
//    (i + t) % 16 of the row, so the score chains do not meet in one bank.
// Same bits as bitlinear_qkv followed by attn_head256_kernel<true>.
// LDS (dynamic): K [256][16] uint4 | V octets [32][128] uint4 | xq [K] |
// red [256] | wpart [256] | q [128] | p [256] | wmax [8] | wq [4] | win [8]
// ---------------------------------------------------------------------------
constexpr int kQaThreads = 512;
constexpr int kQaArrivals = 3 * (kHd / 16);   // the q, k and v tiles of a head

struct QkvAttnParams {
    const uint4 *W;          // the layer's q|k|v weights, tiled I2_S [Dq + 2 Dkv][K]
    const float *wscale;     // [Dq + 2 Dkv]
    const float *x;          // residual stream [K]
    const float *gamma;      // attn_norm weight [K]
    float eps;
    const float2 *rope;      // [max_seq][64] (cos, sin)
    const int *pos;          // decode state position
    float *q;                // q rows [H * 128]
    uint16_t *kcache, *vcache, *vcache8;   // this layer's caches (f16)
    int *cnt;                // [H] arrival counters, 0 between launches
    float *out;              // [H * 128]
    float scale;
    int G, Hkv, max_seq;
};

__host__ __device__ inline size_t qa_smem(int K) {
    return (size_t)2 * 256 * 16 * 16 + K + (256 + 256 + kHd + 256 + 8 + 4 + 8) * 4;
}

// blocks: the k and v tiles (16 Hkv), the q tiles 0-6 of each head (7 H),
// then the candidates (head_grid_blocks(G, Hkv), some idle)
__host__ __device__ inline int qa_grid_blocks(int G, int Hkv) {
    return 16 * Hkv + 7 * G * Hkv + head_grid_blocks(G, Hkv);
}

// K rows 0..255 (clamped to the cache) and V octets 0..31 of one KV head
// into LDS: 128 loads of 1 KB, nw waves from wave w0 issuing 128 / nw each.
// Lane l of load m fills K slot l % 16 of row 4m + l / 16 with chunk
// (slot - row) % 16.
__device__ inline void qa_stage_kv(const uint4 *K4, const uint4 *V8, int max_seq, uint4 *ks,
                                   uint4 *vs4, int w, int nw, int lane) {
    for (int m = w; m < 64; m += nw) {
        const int row = 4 * m + (lane >> 4);
        const int chunk = ((lane & 15) - row) & 15;
        lds_dma16(K4 + (size_t)min(row, max_seq - 1) * 16 + chunk, ks + (size_t)m * 64);
        lds_dma16(V8 + (size_t)m * 64 + lane, vs4 + (size_t)m * 64);
    }
}

template <int NREG>
__global__ __launch_bounds__(kQaThreads) void qkv_attn_kernel(QkvAttnParams p) {
    constexpr int K = 256 * NREG, KC = K / 64, CPL = (KC + 15) / 16;
    extern __shared__ __align__(16) int8_t smem_qa[];
    uint4 *ks = (uint4 *)smem_qa;                              // [256 rows][16 slots]
    uint4 *vs4 = ks + 256 * 16;                                // octets [32][128 dims]
    int8_t *xq = (int8_t *)(vs4 + 256 * 16);                   // [K]
    float *red = (float *)(xq + K);                            // [256]
    int *wpart = (int *)(red + 256);                           // [256]
    float *qs = (float *)(wpart + 256);                        // [128]
    float *pr = qs + kHd;                                      // [256]
    float *wmax = pr + 256;                                    // [8]
    int *wq = (int *)(wmax + 8);                               // [4]
    int *win = wq + 4;                                         // [8]

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int G = p.G, Hkv = p.Hkv, H = G * Hkv, max_seq = p.max_seq;
    // this workgroup's tile (rows 16 tile ..): q tiles 0 .. 8H-1, then k, then v
    int b = blockIdx.x, tile, qhead = -1;
    bool cand = false;
    if (b < 16 * Hkv) {
        tile = 8 * H + b;
    } else if ((b -= 16 * Hkv) < 7 * H) {
        qhead = b / 7;
        tile = 8 * qhead + b % 7;
    } else {
        qhead = head_of_block(b - 7 * H, G, Hkv);
        if (qhead < 0) return;   // an idle slot of the candidates' grid
        tile = 8 * qhead + 7;
        cand = true;
    }
    const int Dq = H * kHd, Dkv = Hkv * kHd;
    const int pos = p.pos[opaque_zero()];
    const bool store = pos >= 0 && pos < max_seq;
    const bool valid = store && pos < kH256Rows;
    const int S = valid ? pos + 1 : 1;
    const int n_ep = tile * 16 + (tid & 15);   // the row this thread may finish

    // ---- loads (waves 0-3): the epilogue's scale, the row, the weights, the
    // RoPE pair; waves 4-7 of a candidate: its head's K and V into LDS
    float ws_ep = 0.0f;
    float2 cs = make_float2(1.0f, 0.0f);
    float v[NREG], g[NREG];
    uint4 A[CPL];
    if (w < 4) {
        ws_ep = p.wscale[n_ep];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            v[j] = p.x[tid + 256 * j];
            g[j] = p.gamma[tid + 256 * j];
        }
        const uint4 *tw = p.W + (size_t)tile * KC * 16;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const int kc = 16 * u + 4 * w + (lane >> 4);
            A[u] = load_nt(tw + (size_t)min(kc, KC - 1) * 16 + (lane & 15));
        }
        __builtin_amdgcn_sched_barrier(0);
        if (n_ep < Dq + Dkv) {
            const int d = (n_ep < Dq ? n_ep : n_ep - Dq) & (kHd - 1);
            const int pc = min(max(pos, 0), max_seq - 1);
            cs = p.rope[(size_t)pc * (kHd / 2) + (d >> 1)];
        }
    } else if (cand) {
        const int hk = qhead / G;
        qa_stage_kv((const uint4 *)(p.kcache + (size_t)hk * max_seq * kHd),
                    (const uint4 *)(p.vcache8 + (size_t)hk * v8_head_elems(max_seq, kHd)),
                    max_seq, ks, vs4, w - 4, 4, lane);
    }

    // ---- prologue: RMSNorm + absmax quantize (waves 0-3, the GEMV's order) ---
    if (w < 4) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            float sq = v[j] * v[j];
            ss = ss + sq;
        }
        red[tid] = ss;
    }
    lds_barrier();
    if (w < 4) {
        const float sum = block256_tree_fold(red);
        const float rms = 1.0f / sqrtf(sum / (float)K + p.eps);  // inverseSqrt
        float am = 0.0f;
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            float a = v[j] * rms;
            v[j] = a * g[j];
            am = fmaxf(am, fabsf(v[j]));
        }
        am = wave_nonneg_max_dpp(am);
        if (lane == 0) wmax[w] = am;
    }
    lds_barrier();
    const float am = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float in_scale = am == 0.0f ? 1.0f : am / 127.0f;   // sh/quantize.wgsl:59
    if (w < 4) {
        const float inv = am == 0.0f ? 0.0f : 127.0f / am;    // :68
        int sq = 0;
#pragma unroll
        for (int j = 0; j < NREG; ++j) {
            const int qv = quant_one(v[j], inv);
            xq[tid + 256 * j] = (int8_t)qv;
            sq += qv;
        }
        sq = wave_isum_dpp(sq);
        if (lane == 0) wq[w] = sq;
    }
    lds_barrier();   // the int8 vector is complete

    // ---- dot products (waves 0-3): chunks past K multiply zero codes ---------
    if (w < 4) {
        CodeAcc acc;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const int kc = 16 * u + 4 * w + (lane >> 4);
            const int kcl = min(kc, KC - 1);
            const int xo = (kcl >> 1) * 128 + (kcl & 1) * 16;
            const int4 x0 = *(const int4 *)(xq + xo);
            const int4 x1 = *(const int4 *)(xq + xo + 32);
            const int4 x2 = *(const int4 *)(xq + xo + 64);
            const int4 x3 = *(const int4 *)(xq + xo + 96);
            const uint4 wv = kc < KC ? A[u] : make_uint4(0, 0, 0, 0);
            acc.add(wv.x, x0.x, x1.x, x2.x, x3.x);
            acc.add(wv.y, x0.y, x1.y, x2.y, x3.y);
            acc.add(wv.z, x0.z, x1.z, x2.z, x3.z);
            acc.add(wv.w, x0.w, x1.w, x2.w, x3.w);
        }
        wpart[tid] = acc.codes();   // lane (row r, column c) of wave w: 16 (4w + c) + r
    }
    lds_barrier();

    // ---- epilogue (lanes 0-15 of wave 0): sh/ternary_gemv.wgsl:94-95, RoPE,
    // the rows to q_out and the caches
    if (w == 0) {
        const int r = lane & 15;
        int a = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) a += wpart[k * 16 + r];
        a -= (wq[0] + wq[1]) + (wq[2] + wq[3]);
        float yv = (float)a * ws_ep;
        yv = yv * in_scale;
        const float other = __shfl_xor(yv, 1, 64);
        const int n = n_ep;
        float outv = yv;
        if (n < Dq + Dkv) {   // q or k: RoPE on the interleaved pair (2i, 2i + 1)
            if ((n & 1) == 0) {
                float a0 = yv * cs.x, a1 = other * cs.y;
                outv = a0 - a1;
            } else {
                float a0 = other * cs.y, a1 = yv * cs.x;
                outv = a0 + a1;
            }
        }
        // the rows other workgroups read in this launch: agent-scope stores
        if (lane < 16 && store) {
            if (n < Dq) {
                __hip_atomic_store(p.q + n, outv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                const int j = n < Dq + Dkv ? n - Dq : n - Dq - Dkv;
                const int hk = j >> 7, d = j & (kHd - 1);
                const size_t at = ((size_t)hk * max_seq + pos) * kHd + d;
                const uint16_t bits = __half_as_ushort(__float2half_rn(outv));
                if (n < Dq + Dkv) {
                    __hip_atomic_store(p.kcache + at, bits, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    __hip_atomic_store(p.vcache + at, bits, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    p.vcache8[(size_t)hk * v8_head_elems(max_seq, kHd) + v8_index(pos, d, kHd)] =
                        bits;
                }
            }
        }
    }

    // ---- arrival (wave 0) --------------------------------------------------
    // Agent-scope stores are visible to every XCD once complete, so waiting
    // for them orders them before the count; a release fence would also
    // write back the whole L2, in every workgroup.
    const bool qt = tile < 8 * H;
    const int n_arr = qt ? 1 : G;
    if (w == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane < n_arr) {
            const int h = qt ? tile >> 3 : ((tile - 8 * H) % (8 * Hkv) >> 3) * G + lane;
            const int old = __hip_atomic_fetch_add(p.cnt + h, 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            const bool last = old == kQaArrivals - 1;
            if (last) __hip_atomic_store(p.cnt + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            win[lane] = last ? h : -1;
        }
    }
    if (w >= 4) wait_vmcnt<0>();   // a candidate's K / V have landed in LDS
    lds_barrier();

    for (int i = 0; i < n_arr; ++i) {
        const int h = win[i];
        if (h < 0) continue;
        const int hk = h / G;
        if (!cand) {
            qa_stage_kv((const uint4 *)(p.kcache + (size_t)hk * max_seq * kHd),
                        (const uint4 *)(p.vcache8 + (size_t)hk * v8_head_elems(max_seq, kHd)),
                        max_seq, ks, vs4, w, 8, lane);
            wait_vmcnt<0>();
            lds_barrier();
        }
        // q, and row pos of K and V over what the stage read before it was
        // written (agent-scope loads: the values the other tiles stored)
        if (tid < kHd) {
            qs[tid] = __hip_atomic_load(p.q + (size_t)h * kHd + tid, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
        } else if (tid < 2 * kHd && valid) {
            const int d = tid - kHd;
            const uint16_t kb = __hip_atomic_load(p.kcache + ((size_t)hk * max_seq + pos) * kHd + d,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ((uint16_t *)(ks + (size_t)pos * 16 + (((d >> 3) + pos) & 15)))[d & 7] = kb;
        } else if (tid < 3 * kHd && valid) {
            const int d = tid - 2 * kHd;
            ((uint16_t *)vs4)[v8_index(pos, d, kHd)] =
                __hip_atomic_load(p.vcache + ((size_t)hk * max_seq + pos) * kHd + d,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        lds_barrier();

        // scores (waves 0-3: thread t, position t), 128 terms in order of d
        float x = 0.0f;
        if (w < 4) {
            const u32x4_t *kv4 = (const u32x4_t *)ks + (size_t)tid * 16;
            constexpr int kAhead = 3;
            u32x4_t kr[16];
            float4 qa[16], qb[16];
            auto ld = [&](int i2) {
                kr[i2] = kv4[(i2 + tid) & 15];
                qa[i2] = *(const float4 *)(qs + 8 * i2);
                qb[i2] = *(const float4 *)(qs + 8 * i2 + 4);
            };
#pragma unroll
            for (int i2 = 0; i2 < kAhead; ++i2) ld(i2);
            float dot = 0.0f;
#pragma unroll
            for (int i2 = 0; i2 < 16; ++i2) {
                __builtin_amdgcn_sched_barrier(0);
                if (i2 + kAhead < 16) ld(i2 + kAhead);
                __builtin_amdgcn_sched_barrier(0);
                const float qv[8] = {qa[i2].x, qa[i2].y, qa[i2].z, qa[i2].w,
                                     qb[i2].x, qb[i2].y, qb[i2].z, qb[i2].w};
#pragma unroll
                for (int k2 = 0; k2 < 4; ++k2) {
                    const uint32_t kw = kr[i2][k2];
                    const float k0 = __half2float(__ushort_as_half((uint16_t)(kw & 0xffffu)));
                    const float k1 = __half2float(__ushort_as_half((uint16_t)(kw >> 16)));
                    dot = __builtin_fmaf(qv[2 * k2], k0, dot);
                    dot = __builtin_fmaf(qv[2 * k2 + 1], k1, dot);
                }
            }
            x = dot * p.scale;
        }
        // softmax (sh/softmax.wgsl:25-80) on waves 0-3
        float m = tid < S ? x : -3.402823e+38f;
        if (w < 4) {
            m = wave_max_dpp(m);
            if (lane == 0) wmax[w] = m;
        }
        lds_barrier();
        m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        const float e = tid < S ? oxb_expf(x - m) : 0.0f;
        if (w < 4) red[tid] = e;   // thread t's strided partial: one position (0 + e = e)
        lds_barrier();
        if (w < 4) {
            const float a = red[lane] + red[lane + 128];
            const float c = red[lane + 64] + red[lane + 192];
            const float inv = 1.0f / wave_tree_sum(a + c);
            pr[tid] = e * inv;   // 0 past S
        }
        lds_barrier();
        // P.V (sh/attention.wgsl:96-104) on waves 0 and 1 over the octets
        if (w < 2) {
            const float acc = pv_head_oct<kH256Rows>(vs4 + 64 * w + lane, pr, S);
            if (valid) p.out[(size_t)h * kHd + 64 * w + lane] = acc;
        }
        lds_barrier();   // LDS is staged again for the next head
    }
}

// ---------------------------------------------------------------------------
// The same design for caches of up to 512 positions: 512 threads (thread t
// scores position t), K staged as [512][17] uint4; the V rows are loaded with
// K and written over the K rows once every score chain is done (one more
// barrier).  Softmax in the shader's 256-thread order: thread t < 256 forms
// its strided partial (0 + e_t) + e_(t+256), then the same halving tree in
// every wave.  P.V: waves 0 / 1 (even / odd dims) run the head256 chains
// over all S positions in order.  Same arithmetic as the other forms.
// ---------------------------------------------------------------------------
constexpr int kH512Rows = 512;
constexpr size_t kH512KBytes = (size_t)kH512Rows * 17 * 16;   // K rows, padded; then V rows
constexpr size_t kH512Lds = kH512KBytes + (kHd + 512 + 512 + 256 + 8) * 4;
static_assert((size_t)kH512Rows * kHd * 2 <= kH512KBytes, "V rows fit the K region");

// OCT: vc is the octet copy of V, as in attn_head256_kernel.
template <bool OCT>
__global__ __launch_bounds__(512) void attn_head512_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    const int *__restrict__ pos_ptr, int G, int Hkv, int max_seq, float scale,
    float *__restrict__ out, size_t kv_stride, int pos_stride, size_t kv8_stride) {
    asm volatile("" ::"s"(q), "s"(kc), "s"(vc), "s"(pos_ptr), "s"(G), "s"(Hkv), "s"(max_seq),
                 "s"(scale), "s"(out), "s"(kv_stride), "s"(pos_stride));
    extern __shared__ __align__(16) int8_t smem_h[];
    u32x4_t (*ks)[17] = (u32x4_t (*)[17])smem_h;
    u32x4_t *vs4 = (u32x4_t *)smem_h;                                // V [512][64] dwords (after K)
    const uint32_t *vs = (const uint32_t *)vs4;
    float *qs = (float *)(smem_h + kH512KBytes);                     // q [128]
    float *pr = qs + kHd;                                            // probabilities [512]
    float *ev = pr + 512;                                            // e [512]
    float *red = ev + 512;                                           // partial sums [256]
    float *wmax = red + 256;                                         // [8]
    const int h = head_of_block(blockIdx.x, G, Hkv), z = blockIdx.y, H = G * Hkv;
    if (h < 0) return;
    const int hk = h / G;
    const float *__restrict__ qh = q + ((size_t)z * H + h) * kHd;
    kc += (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    vc += OCT ? (size_t)z * kv8_stride + (size_t)hk * v8_head_elems(max_seq, kHd)
              : (size_t)z * kv_stride + (size_t)hk * max_seq * kHd;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    const int pos = pos_ptr[(size_t)z * pos_stride];
    const float4 q4 = ((const float4 *)qh)[tid & 31];
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t kt[16], vt[16];
    const u32x4_t *__restrict__ K4 = (const u32x4_t *)kc;
    const u32x4_t *__restrict__ V4 = (const u32x4_t *)vc;
    // rows clamped to the cache, not to S: no wait for the position (rows at
    // or past S are never used)
#pragma unroll
    for (int k = 0; k < 16; ++k) kt[k] = K4[min(32 * k + (tid >> 4), max_seq - 1) * 16 + (tid & 15)];
    if constexpr (OCT) {   // the first 64 octets, clamped to the copy (never summed past S)
        const int last = (int)(v8_head_elems(max_seq, kHd) / 8) - 1;
#pragma unroll
        for (int k = 0; k < 16; ++k) vt[k] = V4[min(512 * k + tid, last)];
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k)
            vt[k] = V4[min(32 * k + (tid >> 4), max_seq - 1) * 16 + (tid & 15)];
    }
    __builtin_amdgcn_sched_barrier(0);
    const bool valid = pos >= 0 && pos < kH512Rows && pos < max_seq;
    const int S = valid ? pos + 1 : 1;
#pragma unroll
    for (int k = 0; k < 16; ++k) ks[32 * k + (tid >> 4)][tid & 15] = kt[k];
    *(float4 *)(qs + 4 * (tid & 31)) = q4;
    lds_barrier();

    // ---- score of position tid: 128 terms in order of d -----------------
    float x;
    {
        constexpr int kAhead = 3;
        u32x4_t kr[16];
        float4 qa[16], qb[16];
        auto ld = [&](int i) {
            kr[i] = ks[tid][i];
            qa[i] = *(const float4 *)(qs + 8 * i);
            qb[i] = *(const float4 *)(qs + 8 * i + 4);
        };
#pragma unroll
        for (int i = 0; i < kAhead; ++i) ld(i);
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            if (i + kAhead < 16) ld(i + kAhead);
            __builtin_amdgcn_sched_barrier(0);
            const float qv[8] = {qa[i].x, qa[i].y, qa[i].z, qa[i].w,
                                 qb[i].x, qb[i].y, qb[i].z, qb[i].w};
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const uint32_t kw = kr[i][k2];
                const float k0 = __half2float(__ushort_as_half((uint16_t)(kw & 0xffffu)));
                const float k1 = __half2float(__ushort_as_half((uint16_t)(kw >> 16)));
                dot = __builtin_fmaf(qv[2 * k2], k0, dot);
                dot = __builtin_fmaf(qv[2 * k2 + 1], k1, dot);
            }
        }
        x = dot * scale;
    }

    // ---- softmax (sh/softmax.wgsl:25-80) --------------------------------------
    float m = tid < S ? x : -3.402823e+38f;
    m = wave_max_dpp(m);
    if (lane == 0) wmax[w] = m;
    lds_barrier();   // every score chain is done: the K rows are free
#pragma unroll
    for (int k = 0; k < 16; ++k) vs4[tid + 512 * k] = vt[k];
    m = fmaxf(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])),
              fmaxf(fmaxf(wmax[4], wmax[5]), fmaxf(wmax[6], wmax[7])));
    const float e = tid < S ? oxb_expf(x - m) : 0.0f;
    ev[tid] = e;
    lds_barrier();
    if (tid < 256) red[tid] = (0.0f + ev[tid]) + ev[tid + 256];   // thread t's strided partial
    lds_barrier();
    float inv;
    {   // the halving tree, in every wave (identical values)
        const float a = red[lane & 63] + red[(lane & 63) + 128];
        const float c = red[(lane & 63) + 64] + red[(lane & 63) + 192];
        inv = 1.0f / wave_tree_sum(a + c);
    }
    pr[tid] = e * inv;   // 0 past S
    lds_barrier();

    // ---- P.V (sh/attention.wgsl:96-104) on waves 0 and 1 ----------------------
    if (w < 2) {
        if constexpr (OCT) {
            const float acc =
                pv_head_oct<kH512Rows>((const uint4 *)vs4 + 64 * w + lane, pr, S);
            if (valid) out[((size_t)z * H + h) * kHd + 64 * w + lane] = acc;
        } else {
            const float acc = w == 0 ? pv_head<false, kH512Rows>(vs + lane, pr, S)
                                     : pv_head<true, kH512Rows>(vs + lane, pr, S);
            if (valid) out[((size_t)z * H + h) * kHd + 2 * lane + w] = acc;
        }
    }
}

// LDS of the prefill kernel for R score rows of up to s_max positions
__host__ __device__ inline size_t prefill_smem(int R, int s_max) {
    return (size_t)R * (kHd + ((s_max + 3) & ~3)) * sizeof(float);
}
constexpr size_t kPrefillLds = 150 * 1024;

template <int G, int Q>
static int launch_prefill(const float *q, const uint16_t *kc, const uint16_t *vc, int pos0,
                          int n_q, int H, int Hkv, int max_seq, int s_max, float *out,
                          hipStream_t s) {
    const size_t smem = prefill_smem(G * Q, s_max);
    if (smem > 64 * 1024 && allow_dynamic_lds((const void *)attn_prefill_kernel<G, Q>)) return -1;
    const float scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    hipLaunchKernelGGL((attn_prefill_kernel<G, Q>), dim3((n_q + Q - 1) / Q, Hkv), dim3(kPrefillThreads), smem,
                       s, q, kc, vc, pos0, n_q, H, max_seq, scale, out);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

// pairs of queries for G >= 4 when both fit the LDS budget (smaller groups
// keep one query per workgroup: their pair variants do not fit registers)
template <int G>
static int launch_prefill_g(const float *q, const uint16_t *kc, const uint16_t *vc, int pos0,
                            int n_q, int H, int Hkv, int max_seq, int s_max, float *out,
                            hipStream_t s) {
    if constexpr (G >= 4) {
        if (prefill_smem(2 * G, s_max) <= kPrefillLds)
            return launch_prefill<G, 2>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, out, s);
    }
    return launch_prefill<G, 1>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, out, s);
}

template <int G>
static int launch_prefill_mfma(const float *q, const uint16_t *kc, const uint16_t *vc, int pos0,
                               int n_q, int H, int Hkv, int max_seq, int s_max, void *ws,
                               float *out, hipStream_t s) {
    constexpr int QB = 16 / G;
    if (allow_dynamic_lds((const void *)attn_prefill_mfma_kernel<G>)) return -1;
    const int ntile = (s_max + 63) / 64;
    float4 *Kt = (float4 *)ws;
    uint4 *Vt = (uint4 *)(Kt + (size_t)Hkv * ntile * kTileF4);
    hipLaunchKernelGGL(attn_kv_tiles_kernel, dim3(ntile, Hkv), dim3(256), 0, s, kc, vc, max_seq,
                       s_max, ntile, Kt, Vt);
    OXB_CHECK_HIP(hipGetLastError());
    const float scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    hipLaunchKernelGGL((attn_prefill_mfma_kernel<G>), dim3(8 * Hkv * ((n_q + QB * 8 - 1) / (QB * 8))),
                       dim3(kPfmThreads), pfm_smem(s_max), s, q, Kt, Vt, ntile, pos0, n_q, H,
                       scale, out);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

size_t attn_prefill_ws_bytes(int Hkv, int s_max) {
    if (Hkv <= 0 || s_max <= 0 || s_max > kPfmMaxS) return 0;
    return (size_t)Hkv * ((s_max + 63) / 64) * (kTileF4 * sizeof(float4) + kVTileU4 * sizeof(uint4));
}

size_t attn_prefill_ws_max_bytes(int Hkv) { return attn_prefill_ws_bytes(Hkv, kPfmMaxS); }

// f32 MFMA kernel (with its Kt / Vt workspace) while its 16 rows fit the LDS
// (up to kPfmMaxS positions), else the VALU kernel: the same sums in the same
// order either way
int attn_prefill(const float *q, const uint16_t *kc, const uint16_t *vc, int n_q, int pos0, int H,
                 int Hkv, int hd, int max_seq, void *ws, size_t ws_bytes, float *out,
                 void *stream) {
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    OXB_REQUIRE(n_q > 0 && pos0 >= 0 && pos0 + n_q <= max_seq, "prefill attention: bad range");
    const int G = H / Hkv, s_max = pos0 + n_q;
    hipStream_t s = (hipStream_t)stream;
    const size_t need = attn_prefill_ws_bytes(Hkv, s_max);
    if (need && ws && ws_bytes >= need) {
        switch (G) {
            case 1: return launch_prefill_mfma<1>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, ws, out, s);
            case 2: return launch_prefill_mfma<2>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, ws, out, s);
            case 4: return launch_prefill_mfma<4>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, ws, out, s);
            case 8: return launch_prefill_mfma<8>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, ws, out, s);
            default: break;
        }
    }
    OXB_REQUIRE(prefill_smem(G, s_max) <= kPrefillLds,
                "attention: %d heads per KV head x %d positions exceed the LDS budget", G, s_max);
    switch (G) {
        case 1: return launch_prefill_g<1>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, out, s);
        case 2: return launch_prefill_g<2>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, out, s);
        case 4: return launch_prefill_g<4>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, out, s);
        case 8: return launch_prefill_g<8>(q, kc, vc, pos0, n_q, H, Hkv, max_seq, s_max, out, s);
        default:
            oxb::set_error("attention: GQA group %d unsupported (1, 2, 4, 8)", G);
            return -1;
    }
}

}  // namespace oxb

using namespace oxb;

// Decode attention over the f16 cache in two launches: the scores kernel
// (64-position blocks), then the softmax and the one-chain P.V of
// attn_pv_chain_kernel per (KV head, group of four heads, sequence), with a
// five-slot V ring while its LDS fits beside the score rows, else three.
template <int G>
static int launch_decode(const float *q, const uint16_t *kc, const uint16_t *vc, const int *pos,
                         int Hkv, int max_seq, float *scores, float *out, hipStream_t s,
                         int batch = 1, size_t kv_stride = 0, int pos_stride = 0,
                         const uint16_t *vc8 = nullptr, size_t kv8_stride = 0) {
    const float scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    hipLaunchKernelGGL(attn_scores_kernel<G>,
                       dim3((max_seq + kScoreP - 1) / kScoreP, Hkv, batch), dim3(256), 0, s, q,
                       kc, pos, max_seq, scale, scores, kv_stride, pos_stride);
    OXB_CHECK_HIP(hipGetLastError());
    if (vc8 && batch <= kPhMaxBatch) {   // one chain wave per CU, V in position octets
        const dim3 hgrid(16 * G * ((Hkv + 7) / 8), batch);
        // 1-2 sequences: V staged through the LDS ring (19.7 against 20.9 us
        // per layer at 2304 positions); more: V streamed into registers (27.0
        // against 40.2 us for 8 sequences)
        if (batch >= 3) {
            if (allow_dynamic_lds((const void *)attn_pv_oreg_kernel)) return -1;
            hipLaunchKernelGGL(attn_pv_oreg_kernel, hgrid, dim3(kPhThreads), pr_smem(max_seq), s,
                               scores, vc8, pos, G, Hkv, max_seq, out, kv8_stride, pos_stride);
        } else if (po_smem(6, max_seq) <= 160 * 1024) {
            if (allow_dynamic_lds((const void *)attn_pv_oct_kernel<6>)) return -1;
            hipLaunchKernelGGL(attn_pv_oct_kernel<6>, hgrid, dim3(kPhThreads), po_smem(6, max_seq),
                               s, scores, vc8, pos, G, Hkv, max_seq, out, kv8_stride, pos_stride);
        } else {
            if (allow_dynamic_lds((const void *)attn_pv_oct_kernel<4>)) return -1;
            hipLaunchKernelGGL(attn_pv_oct_kernel<4>, hgrid, dim3(kPhThreads), po_smem(4, max_seq),
                               s, scores, vc8, pos, G, Hkv, max_seq, out, kv8_stride, pos_stride);
        }
        OXB_CHECK_HIP(hipGetLastError());
        return 0;
    }
    if (batch <= kPhMaxBatch) {   // one chain wave per CU
        const dim3 hgrid(16 * G * ((Hkv + 7) / 8), batch);
        if (ph_smem(6, max_seq) <= 160 * 1024) {
            if (allow_dynamic_lds((const void *)attn_pv_head_kernel<6>)) return -1;
            hipLaunchKernelGGL(attn_pv_head_kernel<6>, hgrid, dim3(kPhThreads), ph_smem(6, max_seq),
                               s, scores, vc, pos, G, Hkv, max_seq, out, kv_stride, pos_stride);
        } else {
            if (allow_dynamic_lds((const void *)attn_pv_head_kernel<4>)) return -1;
            hipLaunchKernelGGL(attn_pv_head_kernel<4>, hgrid, dim3(kPhThreads), ph_smem(4, max_seq),
                               s, scores, vc, pos, G, Hkv, max_seq, out, kv_stride, pos_stride);
        }
        OXB_CHECK_HIP(hipGetLastError());
        return 0;
    }
    const dim3 grid(Hkv * ((G + 3) / 4) * 2, batch);
    // both halves per workgroup once the per-half grid needs more than one
    // round over the CUs (32 sequences: 53.0 against 57.2 us per layer at 2304
    // positions; 16 sequences stay per half: 31.2 against 42.7)
    if (vc8 && (int)(grid.x * grid.y) > device_cus() && pm_smem(6, max_seq) <= 160 * 1024) {
        const dim3 grid2(Hkv * ((G + 3) / 4), batch);
        if (allow_dynamic_lds((const void *)attn_pv_chain_oct2_kernel<6>)) return -1;
        hipLaunchKernelGGL(attn_pv_chain_oct2_kernel<6>, grid2, dim3(kPcThreads),
                           pm_smem(6, max_seq), s, scores, vc8, pos, G, max_seq, out, kv8_stride,
                           pos_stride);
        OXB_CHECK_HIP(hipGetLastError());
        return 0;
    }
    if (vc8) {
        if (pc_smem(5, max_seq) <= 160 * 1024) {
            if (allow_dynamic_lds((const void *)attn_pv_chain_oct_kernel<5>)) return -1;
            hipLaunchKernelGGL(attn_pv_chain_oct_kernel<5>, grid, dim3(kPcThreads),
                               pc_smem(5, max_seq), s, scores, vc8, pos, G, max_seq, out,
                               kv8_stride, pos_stride);
        } else {
            if (allow_dynamic_lds((const void *)attn_pv_chain_oct_kernel<3>)) return -1;
            hipLaunchKernelGGL(attn_pv_chain_oct_kernel<3>, grid, dim3(kPcThreads),
                               pc_smem(3, max_seq), s, scores, vc8, pos, G, max_seq, out,
                               kv8_stride, pos_stride);
        }
        OXB_CHECK_HIP(hipGetLastError());
        return 0;
    }
    if (pc_smem(5, max_seq) <= 160 * 1024) {
        if (allow_dynamic_lds((const void *)attn_pv_chain_kernel<5>)) return -1;
        hipLaunchKernelGGL(attn_pv_chain_kernel<5>, grid, dim3(kPcThreads), pc_smem(5, max_seq), s,
                           scores, vc, pos, G, max_seq, out, kv_stride, pos_stride);
    } else {
        if (allow_dynamic_lds((const void *)attn_pv_chain_kernel<3>)) return -1;
        hipLaunchKernelGGL(attn_pv_chain_kernel<3>, grid, dim3(kPcThreads), pc_smem(3, max_seq), s,
                           scores, vc, pos, G, max_seq, out, kv_stride, pos_stride);
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_attn_decode(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                               const int *pos, int H, int Hkv, int hd, int max_seq, float *scores,
                               float *out, void *stream) {
    OXB_REQUIRE(pos && scores, "attention: pos or scores is NULL");
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    OXB_REQUIRE(max_seq >= 1 && max_seq <= kPcMaxSeq,
                "attention: max_seq %d out of range (1..%d)", max_seq, kPcMaxSeq);
    hipStream_t s = (hipStream_t)stream;
    switch (H / Hkv) {
        case 1: return launch_decode<1>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s);
        case 2: return launch_decode<2>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s);
        case 4: return launch_decode<4>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s);
        case 8: return launch_decode<8>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s);
        default:
            oxb::set_error("attention: GQA group %d unsupported (1, 2, 4, 8)", H / Hkv);
            return -1;
    }
}

static int decode_batch(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                        const uint16_t *vcache8, const int *pos, int pos_stride, size_t kv_stride,
                        size_t kv8_stride, int batch, int H, int Hkv, int hd, int max_seq,
                        float *scores, float *out, void *stream) {
    OXB_REQUIRE(pos && scores, "attention: pos or scores is NULL");
    OXB_REQUIRE(batch >= 1 && batch <= 65535, "attention: batch %d", batch);
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    OXB_REQUIRE(batch == 1 || kv_stride >= (size_t)Hkv * max_seq * hd,
                "attention: caches of a batch overlap (stride %zu)", kv_stride);
    OXB_REQUIRE(!vcache8 || batch == 1 || kv8_stride >= (size_t)Hkv * v8_head_elems(max_seq, hd),
                "attention: octet caches of a batch overlap (stride %zu)", kv8_stride);
    OXB_REQUIRE(max_seq >= 1 && max_seq <= kPcMaxSeq,
                "attention: max_seq %d out of range (1..%d)", max_seq, kPcMaxSeq);
    hipStream_t s = (hipStream_t)stream;
    switch (H / Hkv) {
        case 1: return launch_decode<1>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s, batch, kv_stride, pos_stride, vcache8, kv8_stride);
        case 2: return launch_decode<2>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s, batch, kv_stride, pos_stride, vcache8, kv8_stride);
        case 4: return launch_decode<4>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s, batch, kv_stride, pos_stride, vcache8, kv8_stride);
        case 8: return launch_decode<8>(q, kcache, vcache, pos, Hkv, max_seq, scores, out, s, batch, kv_stride, pos_stride, vcache8, kv8_stride);
        default:
            oxb::set_error("attention: GQA group %d unsupported (1, 2, 4, 8)", H / Hkv);
            return -1;
    }
}

extern "C" int oxb_attn_decode_batch(const float *q, const uint16_t *kcache,
                                     const uint16_t *vcache, const int *pos, int pos_stride,
                                     size_t kv_stride, int batch, int H, int Hkv, int hd,
                                     int max_seq, float *scores, float *out, void *stream) {
    return decode_batch(q, kcache, vcache, nullptr, pos, pos_stride, kv_stride, 0, batch, H, Hkv,
                        hd, max_seq, scores, out, stream);
}

extern "C" int oxb_attn_decode_batch_v8(const float *q, const uint16_t *kcache,
                                        const uint16_t *vcache, const uint16_t *vcache8,
                                        const int *pos, int pos_stride, size_t kv_stride,
                                        size_t kv8_stride, int batch, int H, int Hkv, int hd,
                                        int max_seq, float *scores, float *out, void *stream) {
    OXB_REQUIRE(vcache8, "attention: vcache8 is NULL");
    return decode_batch(q, kcache, vcache, vcache8, pos, pos_stride, kv_stride, kv8_stride, batch,
                        H, Hkv, hd, max_seq, scores, out, stream);
}

template <int G>
static int launch_fused(const float *q, const uint16_t *kc, const uint16_t *vc, const int *pos,
                        int Hkv, int max_seq, float *out, hipStream_t s) {
    const size_t smem = attn_fused_smem(G, max_seq);
    if (allow_dynamic_lds((const void *)attn_fused_kernel<G>)) return -1;
    const float scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    hipLaunchKernelGGL(attn_fused_kernel<G>, dim3(Hkv, 2), dim3(1024), smem, s, q, kc, vc, pos,
                       max_seq, scale, out);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_attn_decode_fused_supported(int H, int Hkv, int hd, int max_seq) {
    if (hd != kHd || Hkv <= 0 || H % Hkv != 0) return 0;
    const int G = H / Hkv;
    return (G == 1 || G == 2 || G == 4) && attn_fused_smem(G, max_seq) <= 160 * 1024;
}

extern "C" int oxb_attn_decode_fused(const float *q, const uint16_t *kcache,
                                     const uint16_t *vcache, const int *pos, int H, int Hkv,
                                     int hd, int max_seq, float *out, void *stream) {
    OXB_REQUIRE(pos, "attention: pos is NULL");
    OXB_REQUIRE(oxb_attn_decode_fused_supported(H, Hkv, hd, max_seq),
                "fused decode attention: unsupported shape (H %d, Hkv %d, hd %d, max_seq %d)", H,
                Hkv, hd, max_seq);
    hipStream_t s = (hipStream_t)stream;
    switch (H / Hkv) {
        case 1: return launch_fused<1>(q, kcache, vcache, pos, Hkv, max_seq, out, s);
        case 2: return launch_fused<2>(q, kcache, vcache, pos, Hkv, max_seq, out, s);
        default: return launch_fused<4>(q, kcache, vcache, pos, Hkv, max_seq, out, s);
    }
}

// The Kt / Vt workspace is stream-ordered memory of this call (allocated and
// released on the caller's stream).
extern "C" int oxb_attn_prefill(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                int n_tok, int pos0, int H, int Hkv, int hd, int max_seq,
                                float *out, void *stream) {
    OXB_REQUIRE(n_tok > 0 && pos0 >= 0 && pos0 + n_tok <= max_seq, "prefill attention: bad range");
    // the arguments are checked before the workspace is allocated
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    OXB_REQUIRE(H / Hkv == 1 || H / Hkv == 2 || H / Hkv == 4 || H / Hkv == 8,
                "attention: GQA group %d unsupported (1, 2, 4, 8)", H / Hkv);
    hipStream_t s = (hipStream_t)stream;
    const size_t need = attn_prefill_ws_bytes(Hkv, pos0 + n_tok);
    void *ws = nullptr;
    if (need) OXB_CHECK_HIP(hipMallocAsync(&ws, need, s));
    const int rc = attn_prefill(q, kcache, vcache, n_tok, pos0, H, Hkv, hd, max_seq, ws, need, out,
                                stream);
    if (ws) {
        const hipError_t e = hipFreeAsync(ws, s);
        if (rc == 0) OXB_CHECK_HIP(e);
    }
    return rc;
}

namespace oxb {
bool qkv_attn_supported(int D, int H, int Hkv, int hd, int max_seq) {
    return hd == kHd && (D == 512 || D == 2560) && Hkv > 0 && H % Hkv == 0 &&
           max_seq >= kH256Rows && max_seq <= 65536;
}

int qkv_attn_decode(const void *W, const float *wscale, const float *x, const float *gamma,
                    float eps, const float *rope, const int *pos, float *q_out, uint16_t *kcache,
                    uint16_t *vcache, uint16_t *vcache8, int *counters, int H, int Hkv, int D,
                    int max_seq, float *out, void *stream) {
    OXB_REQUIRE(W && wscale && x && gamma && rope && pos && q_out && kcache && vcache && vcache8 &&
                    counters && out,
                "qkv attention: null argument");
    OXB_REQUIRE(qkv_attn_supported(D, H, Hkv, kHd, max_seq),
                "qkv attention: unsupported shape (hidden %d, heads %d/%d, max_seq %d)", D, H, Hkv,
                max_seq);
    QkvAttnParams p{};
    p.W = (const uint4 *)W;
    p.wscale = wscale;
    p.x = x;
    p.gamma = gamma;
    p.eps = eps;
    p.rope = (const float2 *)rope;
    p.pos = pos;
    p.q = q_out;
    p.kcache = kcache;
    p.vcache = vcache;
    p.vcache8 = vcache8;
    p.cnt = counters;
    p.out = out;
    p.scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    p.G = H / Hkv;
    p.Hkv = Hkv;
    p.max_seq = max_seq;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(qa_grid_blocks(p.G, Hkv));
    if (D == 2560) {
        if (allow_dynamic_lds((const void *)qkv_attn_kernel<10>)) return -1;
        hipLaunchKernelGGL(qkv_attn_kernel<10>, grid, dim3(kQaThreads), qa_smem(D), s, p);
    } else {
        if (allow_dynamic_lds((const void *)qkv_attn_kernel<2>)) return -1;
        hipLaunchKernelGGL(qkv_attn_kernel<2>, grid, dim3(kQaThreads), qa_smem(D), s, p);
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}
}  // namespace oxb

extern "C" int oxb_qkv_attn_decode(const void *W_tiled, const float *wscale, const float *x,
                                   const float *gamma, float eps, const float *rope_cs,
                                   const int *pos, float *q_out, uint16_t *kcache,
                                   uint16_t *vcache, uint16_t *vcache8, int *counters, int H,
                                   int Hkv, int hd, int D, int max_seq, float *out, void *stream) {
    oxb::clear_error();
    OXB_REQUIRE(hd == kHd, "qkv attention: head_dim %d unsupported (128 only)", hd);
    return oxb::qkv_attn_decode(W_tiled, wscale, x, gamma, eps, rope_cs, pos, q_out, kcache,
                                vcache, vcache8, counters, H, Hkv, D, max_seq, out, stream);
}

static int decode_head(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                       const uint16_t *vcache8, const int *pos, int pos_stride, size_t kv_stride,
                       size_t kv8_stride, int batch, int H, int Hkv, int hd, int max_seq,
                       int s_max, float *out, void *stream) {
    OXB_REQUIRE(pos, "attention: pos is NULL");
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    OXB_REQUIRE(batch >= 1 && batch <= 65535, "attention: batch %d", batch);
    OXB_REQUIRE(batch == 1 || kv_stride >= (size_t)Hkv * max_seq * hd,
                "attention: caches of a batch overlap (stride %zu)", kv_stride);
    OXB_REQUIRE(!vcache8 || batch == 1 || kv8_stride >= (size_t)Hkv * v8_head_elems(max_seq, hd),
                "attention: octet caches of a batch overlap (stride %zu)", kv8_stride);
    OXB_REQUIRE(s_max >= 1 && s_max <= 512,
                "per-head decode attention: s_max %d out of range (1..512)", s_max);
    const float scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    hipStream_t s = (hipStream_t)stream;
    const int G = H / Hkv;
    const dim3 grid(head_grid_blocks(G, Hkv), batch);
    if (s_max <= 256 && max_seq >= kH256Rows && vcache8) {
        if (allow_dynamic_lds((const void *)attn_head256_kernel<true>)) return -1;
        hipLaunchKernelGGL(attn_head256_kernel<true>, grid, dim3(256), kH256Lds, s, q, kcache,
                           vcache8, pos, G, Hkv, max_seq, scale, out, kv_stride, pos_stride,
                           kv8_stride);
    } else if (s_max <= 256 && max_seq >= kH256Rows) {
        if (allow_dynamic_lds((const void *)attn_head256_kernel<false>)) return -1;
        hipLaunchKernelGGL(attn_head256_kernel<false>, grid, dim3(256), kH256Lds, s, q, kcache,
                           vcache, pos, G, Hkv, max_seq, scale, out, kv_stride, pos_stride,
                           (size_t)0);
    } else if (s_max <= 256)
        hipLaunchKernelGGL(attn_head_kernel, grid, dim3(256), 0, s, q, kcache, vcache, pos, G, Hkv,
                           max_seq, scale, out, kv_stride, pos_stride);
    else if (vcache8) {
        if (allow_dynamic_lds((const void *)attn_head512_kernel<true>)) return -1;
        hipLaunchKernelGGL(attn_head512_kernel<true>, grid, dim3(512), kH512Lds, s, q, kcache,
                           vcache8, pos, G, Hkv, max_seq, scale, out, kv_stride, pos_stride,
                           kv8_stride);
    } else {
        if (allow_dynamic_lds((const void *)attn_head512_kernel<false>)) return -1;
        hipLaunchKernelGGL(attn_head512_kernel<false>, grid, dim3(512), kH512Lds, s, q, kcache,
                           vcache, pos, G, Hkv, max_seq, scale, out, kv_stride, pos_stride,
                           (size_t)0);
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_attn_decode_head(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                    const int *pos, int pos_stride, size_t kv_stride, int batch,
                                    int H, int Hkv, int hd, int max_seq, int s_max, float *out,
                                    void *stream) {
    return decode_head(q, kcache, vcache, nullptr, pos, pos_stride, kv_stride, 0, batch, H, Hkv,
                       hd, max_seq, s_max, out, stream);
}

extern "C" int oxb_attn_decode_head_v8(const float *q, const uint16_t *kcache,
                                       const uint16_t *vcache, const uint16_t *vcache8,
                                       const int *pos, int pos_stride, size_t kv_stride,
                                       size_t kv8_stride, int batch, int H, int Hkv, int hd,
                                       int max_seq, int s_max, float *out, void *stream) {
    OXB_REQUIRE(vcache8, "attention: vcache8 is NULL");
    return decode_head(q, kcache, vcache, vcache8, pos, pos_stride, kv_stride, kv8_stride, batch,
                       H, Hkv, hd, max_seq, s_max, out, stream);
}

// ---------------------------------------------------------------------------
// Attention over an f32 KV cache, the reference's cache type
// (nn/attention.rs:23-48 allocates f32 K/V buffers; sh/attention.wgsl reads
// them as array<f32>), in the same arithmetic order as the f16 kernels.  A
// parity mode, not the throughput path: one workgroup per (query head,
// query), 2 waves.
//   scores   thread t takes positions t, t + 128, ...: 128 fused steps in
//            order of d (q from LDS, the K row from HBM), times the scale
//   softmax  wave 0, the 256-thread order (wave_softmax_row)
//   P.V      thread d < 128: out[d] = one chain over the S positions in order
//            of s (sh/attention.wgsl:96-104)
// Query qi sits at position pos0 + qi (pos0 = *pos_ptr for a decode step
// from device state) and attends over S = its position + 1 positions.
// LDS: q [128] | scores [Sp] | probabilities [Sp], Sp = s_max rounded to 4.
// ---------------------------------------------------------------------------
constexpr int kF32Threads = 128;
constexpr int kF32MaxSeq = OXB_KV_F32_MAX_SEQ;   // LDS rows: 2 x 64 KiB

__global__ __launch_bounds__(kF32Threads) void attn_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    const int *__restrict__ pos_ptr, int pos0, int G, int max_seq, int s_max, float scale,
    float *__restrict__ out) {
    extern __shared__ __align__(16) float lds[];
    const int h = blockIdx.x, qi = blockIdx.y, H = gridDim.x;
    const int pos = (pos_ptr ? *pos_ptr : pos0) + qi;
    if (pos < 0 || pos >= max_seq || pos >= s_max) return;   // launch checks too
    const int S = pos + 1, Spad = (S + 3) & ~3;
    const int Sp = (s_max + 3) & ~3;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int hk = h / G;
    float *qs = lds, *sc = lds + kHd, *pr = sc + Sp;
    const float *K = kc + (size_t)hk * max_seq * kHd;
    const float *V = vc + (size_t)hk * max_seq * kHd;
    qs[tid] = q[((size_t)qi * H + h) * kHd + tid];
    lds_barrier();
    for (int s = tid; s < S; s += kF32Threads) {
        const float4 *kr = (const float4 *)(K + (size_t)s * kHd);
        float dot = 0.0f;
#pragma unroll 4
        for (int i = 0; i < kHd / 4; ++i) {
            const float4 k4 = kr[i];
            const float4 q4 = *(const float4 *)(qs + 4 * i);
            dot = __builtin_fmaf(q4.x, k4.x, dot);
            dot = __builtin_fmaf(q4.y, k4.y, dot);
            dot = __builtin_fmaf(q4.z, k4.z, dot);
            dot = __builtin_fmaf(q4.w, k4.w, dot);
        }
        sc[s] = dot * scale;
    }
    lds_barrier();
    if (w == 0) wave_softmax_row(pr, sc, S, Spad, lane, false);
    lds_barrier();
    const int d = tid;
    float acc = 0.0f;
    int s = 0;
    for (; s + 8 <= S; s += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = V[(size_t)(s + k) * kHd + d];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc = __builtin_fmaf(pr[s + k], v[k], acc);
    }
    for (; s < S; ++s) acc = __builtin_fmaf(pr[s], V[(size_t)s * kHd + d], acc);
    out[((size_t)qi * H + h) * kHd + d] = acc;
}

namespace oxb {
int attn_f32(const float *q, const float *kcache, const float *vcache, const int *pos_ptr,
             int pos0, int n_q, int H, int Hkv, int hd, int max_seq, float *out, void *stream) {
    OXB_REQUIRE(hd == kHd, "attention (f32 cache): head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    OXB_REQUIRE(n_q >= 1 && n_q <= 65535, "attention (f32 cache): %d queries", n_q);
    OXB_REQUIRE(max_seq >= 1 && max_seq <= kF32MaxSeq,
                "attention (f32 cache): max_seq %d beyond %d", max_seq, kF32MaxSeq);
    // decode (position from device state): any position of the cache;
    // prefill: the block's last position bounds the rows
    const int s_max = pos_ptr ? max_seq : pos0 + n_q;
    OXB_REQUIRE(pos_ptr || (pos0 >= 0 && s_max <= max_seq), "attention (f32 cache): bad range");
    const size_t lds = (size_t)(kHd + 2 * ((s_max + 3) & ~3)) * 4;
    if (lds > 64 * 1024 && allow_dynamic_lds((const void *)attn_f32_kernel)) return -1;
    const float scale = 1.0f / sqrtf((float)kHd);  // nn/attention.rs:206
    hipLaunchKernelGGL(attn_f32_kernel, dim3(H, n_q), dim3(kF32Threads), lds, (hipStream_t)stream,
                       q, kcache, vcache, pos_ptr, pos0, H / Hkv, max_seq, s_max, scale, out);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}
}  // namespace oxb

// ---------------------------------------------------------------------------
// Decode attention that allocates nothing: oxb_attn_decode with its scores
// scratch in a static device array instead of a caller buffer.  The array is
// per device (each GPU the library runs on holds its own copy until the
// process ends); its device address is looked up once per device, on the
// first call with that device current, and only that address is handed to
// the kernels.  Calls on one device share the array, so calls that overlap
// on one GPU race.  Nothing in it needs clearing: the kernels write every
// score they read (positions < S) before reading it.
// ---------------------------------------------------------------------------
namespace oxb {
constexpr size_t kNoAllocScoreFloats = (size_t)1 << 18;   // 1 MiB: H * max_seq <= 262144
static __device__ __align__(256) float scratch[kNoAllocScoreFloats];
constexpr int kMaxDevices = 64;

static float *noalloc_scratch() {
    static std::mutex mu;
    static float *ptrs[kMaxDevices] = {};
    int dev = 0;
    const hipError_t ed = hipGetDevice(&dev);
    if (ed != hipSuccess) {
        set_error("attention (no-alloc): hipGetDevice: %s", hipGetErrorString(ed));
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("attention (no-alloc): device %d beyond the %d supported", dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("attention (no-alloc): hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return nullptr;
        }
        ptrs[dev] = (float *)p;
    }
    return ptrs[dev];
}
}  // namespace oxb

extern "C" int oxb_attn_decode_noalloc(const float *q, const uint16_t *kcache,
                                       const uint16_t *vcache, const int *pos, int H, int Hkv,
                                       int hd, int max_seq, float *out, void *stream) {
    OXB_REQUIRE(H > 0 && max_seq > 0 && (size_t)H * max_seq <= kNoAllocScoreFloats,
                "attention (no-alloc): heads %d x max_seq %d exceed the %zu-score scratch", H,
                max_seq, kNoAllocScoreFloats);
    float *scores = noalloc_scratch();
    if (!scores) return -1;
    return oxb_attn_decode(q, kcache, vcache, pos, H, Hkv, hd, max_seq, scores, out, stream);
}
