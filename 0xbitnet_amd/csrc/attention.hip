// GQA attention over the f16 KV cache for gfx950.
//
// Reference: sh/attention.wgsl:29-59 (scores, causal mask, GQA kv = h/group),
// sh/softmax.wgsl:25-80, sh/attention.wgsl:79-105 (P.V), orchestrated by
// rs/nn/attention.rs:85-124.  The reference materialises [H, N, S] scores in
// f32 over an f32 cache; here each workgroup streams one block of positions
// of one KV head for the whole GQA group and keeps an online softmax, so the
// scores never leave the CU.  Results agree within float tolerance (the
// reduction order differs and K/V are stored as f16).
//
// Cache layout: [Hkv][max_seq][hd] f16 bits, hd = 128.
#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

constexpr int kHd = 128;
constexpr int kSplit = 64;     // positions per decode workgroup
constexpr int kGroupMax = 8;   // max q heads per KV head handled per workgroup

__device__ inline void f16x8_to_f32(uint4 u, float *f) {
    const __half2 *h = (const __half2 *)&u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float2 v = __half22float2(h[i]);
        f[2 * i] = v.x;
        f[2 * i + 1] = v.y;
    }
}

// ---------------------------------------------------------------------------
// Decode: one token, L = pos + 1 cached positions (the QKV epilogue has
// already appended position pos).  Grid (max_split, Hkv), 256 threads.
// Lanes: 16 lanes cover one 128-dim row (8 dims each); a wave covers 4
// positions per step; the 4 waves cover 16 positions per step.
// ---------------------------------------------------------------------------
template <int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, const int *__restrict__ pos_ptr, int max_seq,
    float scale, int max_split, float *__restrict__ part_o, float *__restrict__ part_ml,
    int *__restrict__ counters, float *__restrict__ out) {
    __shared__ float sc[G][kSplit];
    __shared__ float red_o[4][G][kHd];
    __shared__ int ticket_s;

    const int L = *pos_ptr + 1;
    if (L < 1 || L > max_seq) return;  // host checks too; never read out of range
    const int nsplit = (L + kSplit - 1) / kSplit;
    const int s = blockIdx.x, hk = blockIdx.y;
    if (s >= nsplit) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int sub = lane >> 4, dl = lane & 15;   // position-in-step, dim group
    const int p0 = s * kSplit;
    const int np = min(kSplit, L - p0);
    const uint4 *K4 = (const uint4 *)(kc + ((size_t)hk * max_seq + p0) * kHd);
    const uint4 *V4 = (const uint4 *)(vc + ((size_t)hk * max_seq + p0) * kHd);

    // q for the G heads of this group, 8 dims per lane.
    float qv[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const float4 *qp = (const float4 *)(q + (size_t)(hk * G + j) * kHd + dl * 8);
        float4 a = qp[0], b = qp[1];
        qv[j][0] = a.x; qv[j][1] = a.y; qv[j][2] = a.z; qv[j][3] = a.w;
        qv[j][4] = b.x; qv[j][5] = b.y; qv[j][6] = b.z; qv[j][7] = b.w;
    }

    // scores
    for (int pb = w * 4; pb < kSplit; pb += 16) {
        const int p = pb + sub;
        float d[G];
#pragma unroll
        for (int j = 0; j < G; ++j) d[j] = 0.0f;
        if (p < np) {
            float kf[8];
            f16x8_to_f32(K4[(size_t)p * 16 + dl], kf);
#pragma unroll
            for (int j = 0; j < G; ++j)
#pragma unroll
                for (int i = 0; i < 8; ++i) d[j] = fmaf(qv[j][i], kf[i], d[j]);
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) d[j] += __shfl_xor(d[j], m, 64);
            if (dl == 0) sc[j][p] = p < np ? d[j] * scale : -3.402823e+38f;
        }
    }
    __syncthreads();

    // softmax statistics per head (wave j handles head j; G <= 4 per pass)
    for (int j = w; j < G; j += 4) {
        const float v = sc[j][lane];
        const float m = wave_max(v);
        const float e = lane < np ? expf(v - m) : 0.0f;
        const float l = wave_sum(e);
        sc[j][lane] = e;
        if (lane == 0) {
            float *ml = part_ml + ((size_t)(hk * G + j) * max_split + s) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();

    // P.V: lane accumulates 8 dims for G heads over its positions
    float o[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[j][i] = 0.0f;
    for (int pb = w * 4; pb < np; pb += 16) {
        const int p = pb + sub;
        if (p < np) {
            float vf[8];
            f16x8_to_f32(V4[(size_t)p * 16 + dl], vf);
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float pj = sc[j][p];
#pragma unroll
                for (int i = 0; i < 8; ++i) o[j][i] = fmaf(pj, vf[i], o[j][i]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = o[j][i];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            o[j][i] = v;
        }
    if (sub == 0) {
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) red_o[w][j][dl * 8 + i] = o[j][i];
    }
    __syncthreads();
    for (int idx = tid; idx < G * kHd; idx += 256) {
        const int j = idx / kHd, dd = idx % kHd;
        const float v = red_o[0][j][dd] + red_o[1][j][dd] + red_o[2][j][dd] + red_o[3][j][dd];
        part_o[((size_t)(hk * G + j) * max_split + s) * kHd + dd] = v;
    }

    // last workgroup of this KV head combines the splits.  Every thread
    // fences its own partial stores at agent scope (L2 write-back across
    // XCDs) before thread 0 takes a ticket.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        ticket_s = __hip_atomic_fetch_add(&counters[hk], 1, __ATOMIC_ACQ_REL,
                                          __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (ticket_s != nsplit - 1) return;
    __threadfence();  // acquire side: drop stale cache lines before reading partials
    for (int idx = tid; idx < G * kHd; idx += 256) {
        const int j = idx / kHd, dd = idx % kHd;
        const int h = hk * G + j;
        const float *ml = part_ml + (size_t)h * max_split * 2;
        float M = -3.402823e+38f;
        for (int t = 0; t < nsplit; ++t)
            M = fmaxf(M, __hip_atomic_load(&ml[2 * t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        float num = 0.0f, den = 0.0f;
        for (int t = 0; t < nsplit; ++t) {
            const float mt = __hip_atomic_load(&ml[2 * t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float lt = __hip_atomic_load(&ml[2 * t + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float ot = __hip_atomic_load(&part_o[((size_t)h * max_split + t) * kHd + dd],
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float e = expf(mt - M);
            num = fmaf(e, ot, num);
            den = fmaf(e, lt, den);
        }
        out[(size_t)h * kHd + dd] = num / den;
    }
    if (tid == 0) counters[hk] = 0;  // ready for the next launch (graph replay)
}

// ---------------------------------------------------------------------------
// Prefill: n_tok new tokens at absolute positions pos0 .. pos0+n_tok-1, keys
// 0 .. pos0+n_tok-1 already in the cache.  Grid (ceil(n_tok/16), Hkv);
// 256 threads = G waves of one GQA group (G = 4); wave j = head j; lane l
// owns query qi = l/4 of the block and dims (l%4)*32 .. +31.
// q: [n_tok][H*hd] f32 (roped); out: [n_tok][H*hd] f32.
// ---------------------------------------------------------------------------
constexpr int kQB = 16;   // queries per workgroup
constexpr int kKT = 64;   // keys per tile

__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, int n_tok, int pos0, int H, int max_seq, float scale,
    float *__restrict__ out) {
    __shared__ __align__(16) uint16_t Ks[kKT * kHd];
    __shared__ __align__(16) uint16_t Vs[kKT * kHd];
    const int G = 4;
    const int tid = threadIdx.x, lane = tid & 63, j = tid >> 6;
    const int hk = blockIdx.y, h = hk * G + j;
    const int qb = blockIdx.x * kQB;
    const int qi = lane >> 2, part = lane & 3;
    const int qrow = qb + qi;
    const bool qvalid = qrow < n_tok;
    const int qpos = pos0 + (qvalid ? qrow : n_tok - 1);
    const int last_key = pos0 + min(n_tok, qb + kQB) - 1;  // inclusive

    float qv[32], o[32];
    {
        const float4 *qp = (const float4 *)(q + (size_t)(qvalid ? qrow : 0) * H * kHd +
                                            (size_t)h * kHd + part * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float4 a = qp[i];
            qv[4 * i] = a.x; qv[4 * i + 1] = a.y; qv[4 * i + 2] = a.z; qv[4 * i + 3] = a.w;
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) o[i] = 0.0f;
    float m = -3.402823e+38f, l = 0.0f;

    const uint4 *Kg = (const uint4 *)(kc + (size_t)hk * max_seq * kHd);
    const uint4 *Vg = (const uint4 *)(vc + (size_t)hk * max_seq * kHd);
    for (int k0 = 0; k0 <= last_key; k0 += kKT) {
        __syncthreads();
        for (int i = tid; i < kKT * 16; i += 256) {
            const int key = k0 + i / 16;
            uint4 kz = make_uint4(0, 0, 0, 0), vz = kz;
            if (key <= last_key) {
                kz = Kg[(size_t)key * 16 + (i & 15)];
                vz = Vg[(size_t)key * 16 + (i & 15)];
            }
            ((uint4 *)Ks)[i] = kz;
            ((uint4 *)Vs)[i] = vz;
        }
        __syncthreads();
        float sc[kKT];
        float tmax = -3.402823e+38f;
#pragma unroll
        for (int kk = 0; kk < kKT; ++kk) {
            const uint4 *kr = (const uint4 *)(Ks + kk * kHd + part * 32);
            float d = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float kf[8];
                f16x8_to_f32(kr[u], kf);
#pragma unroll
                for (int i = 0; i < 8; ++i) d = fmaf(qv[8 * u + i], kf[i], d);
            }
            d += __shfl_xor(d, 1, 64);
            d += __shfl_xor(d, 2, 64);
            // causal: key > query's absolute position is masked (sh/attention.wgsl:54)
            const float sv = (k0 + kk > qpos) ? -3.402823e+38f : d * scale;
            sc[kk] = sv;
            tmax = fmaxf(tmax, sv);
        }
        const float mn = fmaxf(m, tmax);
        const float corr = expf(m - mn);
        l *= corr;
#pragma unroll
        for (int i = 0; i < 32; ++i) o[i] *= corr;
#pragma unroll
        for (int kk = 0; kk < kKT; ++kk) {
            const float pv = (k0 + kk > qpos) ? 0.0f : expf(sc[kk] - mn);
            l += pv;
            const uint4 *vr = (const uint4 *)(Vs + kk * kHd + part * 32);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float vf[8];
                f16x8_to_f32(vr[u], vf);
#pragma unroll
                for (int i = 0; i < 8; ++i) o[8 * u + i] = fmaf(pv, vf[i], o[8 * u + i]);
            }
        }
        m = mn;
    }
    if (qvalid) {
        const float inv = 1.0f / l;
        float4 *op = (float4 *)(out + (size_t)qrow * H * kHd + (size_t)h * kHd + part * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            op[i] = make_float4(o[4 * i] * inv, o[4 * i + 1] * inv, o[4 * i + 2] * inv,
                                o[4 * i + 3] * inv);
    }
}

}  // namespace oxb

using namespace oxb;

extern "C" int oxb_attn_decode(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                               const int *pos, int H, int Hkv, int hd, int max_seq,
                               float *part_o, float *part_ml, int *counters, float *out,
                               void *stream) {
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H % Hkv == 0, "attention: heads %d not a multiple of kv heads %d", H, Hkv);
    const int G = H / Hkv;
    const int max_split = (max_seq + kSplit - 1) / kSplit;
    const float scale = 1.0f / sqrtf((float)hd);  // rs/nn/attention.rs:206
    hipStream_t s = (hipStream_t)stream;
    switch (G) {
#define OXB_G(g)                                                                        \
    case g:                                                                             \
        hipLaunchKernelGGL(attn_decode_kernel<g>, dim3(max_split, Hkv), dim3(256), 0, s, \
                           q, kcache, vcache, pos, max_seq, scale, max_split, part_o,   \
                           part_ml, counters, out);                                     \
        break;
        OXB_G(1) OXB_G(2) OXB_G(4) OXB_G(8)
#undef OXB_G
        default:
            oxb::set_error("attention: GQA group %d unsupported (1, 2, 4, 8)", G);
            return -1;
    }
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

extern "C" int oxb_attn_prefill(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                                int n_tok, int pos0, int H, int Hkv, int hd, int max_seq,
                                float *out, void *stream) {
    OXB_REQUIRE(hd == kHd, "attention: head_dim %d unsupported (128 only)", hd);
    OXB_REQUIRE(Hkv > 0 && H == 4 * Hkv, "prefill attention: needs GQA group 4 (H %d, Hkv %d)", H, Hkv);
    OXB_REQUIRE(n_tok > 0 && pos0 >= 0 && pos0 + n_tok <= max_seq, "prefill attention: bad range");
    const float scale = 1.0f / sqrtf((float)hd);
    hipLaunchKernelGGL(attn_prefill_kernel, dim3((n_tok + kQB - 1) / kQB, Hkv), dim3(256), 0,
                       (hipStream_t)stream, q, kcache, vcache, n_tok, pos0, H, max_seq, scale, out);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}
