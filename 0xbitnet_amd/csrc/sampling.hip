// Token sampling on the device for gfx950: repetition penalty, temperature,
// top-k threshold, softmax and the inverse-CDF draw of rs/sampling.rs:4-80,
// for a uniform draw u that the caller supplies (the reference takes it from
// rand's thread generator, sampling.rs:69-70).  Same token as the host
// restatement oxb_sample_logits (capi.cpp) for the same logits and u.
//
// Two kernels:
//  1. sample_local_kernel, one 256-thread block per 2048 logits: the
//     penalty for this block's ids of the window (each distinct id once, as
//     many times as it occurs, sampling.rs:14-24), the temperature
//     (x * (1/T) when T != 1, :27-33), the values y written out, and the
//     block's k largest (value, index) keys, found by a radix select (four
//     8-bit digits of an order-preserving u32 of the value, LDS histograms).
//  2. sample_final_kernel, one 256-thread block: the k-th largest over the
//     blocks' lists is the top-k threshold (:36-59) -- each value of the
//     global top k is in its own block's top k --, the largest is the
//     softmax maximum.  After the threshold every other value is -inf, whose
//     exp(-inf - max) is exactly 0 and leaves a float running sum unchanged,
//     so the values >= threshold taken in index order give the reference's
//     sum and running sum over all V (:62-78) bit for bit.
// Dense path (no top-k, k > 256, or values equal to the threshold past some
// block's list): the same sums over all V values in index order, one thread
// adding, with the running sums kept for the search.
// Values NaN or +inf anywhere make the reference's sum NaN, which no running
// sum reaches: the token is V - 1 (:80), as on the host.
#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

constexpr int kSmpLocal = 256;         // threads of the first kernel
constexpr int kSmpChunk = 2048;        // logits per block of the first kernel
constexpr int kSmpThreads = 256;       // threads of the final kernel
constexpr int kSmpKMax = 256;          // largest k of the candidate-list path
constexpr int kSmpFinalKeys = 16384;   // candidate keys the final kernel holds (128 KB)
constexpr int kSmpSurv = 2048;         // values >= threshold it orders by index
constexpr int kSmpDense = 8192;        // values per chunk of the dense running sum

struct SmpArgs {
    const float *logits;
    int V;
    SampleCtl ctl;              // used when ctl_dev is null
    const SampleCtl *ctl_dev;   // read at run time (a captured graph's parameters)
    const int *win;             // window ids, or the token history when state is set
    int nwin;                   // window length when state is null
    int *state;                 // decode state: window, draw index and token from NGEN
    int *hist;                  // token history (state path): the token is stored at NGEN-1
    const float *u;             // draws: u[NGEN-1] (state path) or u[0]
    int *out;                   // the token (may be null on the state path)
    float *y, *pre;             // workspace: values after penalty/temperature, running sums
    unsigned long long *cand;   // [G][kSmpKMax] each block's k largest keys (any order)
    int *bflag;                 // [G] bit 0: values equal to the block's k-th past its
                                //     list, bit 1: a NaN or +inf value
    uint32_t *bthr;             // [G] the block's k-th value (as smp_ord)
    int G;
};

// Order-preserving map of a float to u32 (-0 taken as +0, as the float
// comparisons of the reference see them); 0 is below every value and marks
// an empty list slot.  Keys: value, then the lower index first.
__device__ inline uint32_t smp_ord(float v) {
    if (v == 0.0f) v = 0.0f;
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float smp_unord(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ inline unsigned long long smp_key(uint32_t ord, int i) {
    return ((unsigned long long)ord << 32) | (0xffffffffu - (uint32_t)i);
}
__device__ inline int smp_index(unsigned long long k) { return (int)(0xffffffffu - (uint32_t)k); }

__device__ inline SampleCtl smp_ctl(const SmpArgs &a) { return a.ctl_dev ? *a.ctl_dev : a.ctl; }

// top-k in effect: 0 (keep all) unless 0 < k < V (sampling.rs:36)
__device__ inline int smp_kk(const SampleCtl &c, int V) {
    return (c.top_k > 0 && c.top_k < V) ? c.top_k : 0;
}

// The window of lib.rs:156-161: the last last_n tokens before the
// current one (all of them when last_n is 0).
__device__ inline int smp_window(const SmpArgs &a, const SampleCtl &c, const int **w) {
    if (!a.state) {
        *w = a.win;
        return a.nwin;
    }
    int done = a.state[OXB_ST_NGEN] - 1;   // tokens before the current one
    done = min(max(done, 0), a.state[OXB_ST_HIST_CAP]);
    const int start = (c.last_n > 0 && done > c.last_n) ? done - c.last_n : 0;
    *w = a.win + start;
    return done - start;
}

__device__ inline int smp_draw_index(const SmpArgs &a) {
    return a.state ? min(max(a.state[OXB_ST_NGEN] - 1, 0), a.state[OXB_ST_HIST_CAP] - 1) : 0;
}

// One digit of a radix select, by wave 0 over hist[256] (the counts of the
// current 8-bit digit among the keys that match the digits chosen so far):
// the digit d, largest first, with (count above d) < rem <= (count above d)
// + hist[d]; writes the extended prefix and what remains of rem.
__device__ inline void smp_pick_digit(const uint32_t *hist, int rem, uint32_t prefix, int shift,
                                      uint32_t *s_prefix, int *s_rem) {
    const int lane = threadIdx.x;
    int h[4], local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h[j] = (int)hist[255 - 4 * lane - j];
        local += h[j];
    }
    int incl = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    int acc = incl - local;
    if (acc < rem && rem <= incl) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (acc + h[j] >= rem) {
                *s_prefix = prefix | ((uint32_t)(255 - 4 * lane - j) << shift);
                *s_rem = rem - acc;
                break;
            }
            acc += h[j];
        }
    }
}

// The k-th largest of the block's keys key_at(i), i < n (k <= n), by the
// whole block.  hist: 256 words of LDS.  Its barriers order LDS only: the
// keys come from LDS or from memory no thread of the block writes.
template <int NT, typename KeyAt>
__device__ uint32_t smp_select(int n, int k, KeyAt key_at, uint32_t *hist, uint32_t *s_prefix,
                               int *s_rem) {
    uint32_t prefix = 0, mask = 0;
    int rem = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += NT) hist[i] = 0;
        lds_barrier();
        for (int i = threadIdx.x; i < n; i += NT) {
            const uint32_t o = key_at(i);
            if ((o & mask) == prefix) atomicAdd(&hist[(o >> shift) & 255u], 1u);
        }
        lds_barrier();
        if (threadIdx.x < 64) smp_pick_digit(hist, rem, prefix, shift, s_prefix, s_rem);
        lds_barrier();
        prefix = *s_prefix;
        rem = *s_rem;
        mask |= 255u << shift;
    }
    return prefix;
}

__global__ __launch_bounds__(kSmpLocal) void sample_local_kernel(SmpArgs a) {
    __shared__ float vals[kSmpChunk];
    __shared__ uint32_t ords[kSmpChunk];
    __shared__ int cnt[kSmpChunk];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_prefix;
    __shared__ int s_rem, s_bad, s_gt, s_eq;
    const SampleCtl c = smp_ctl(a);
    const int tid = threadIdx.x, b = blockIdx.x, base = b * kSmpChunk;
    const int n = min(kSmpChunk, a.V - base);
    const int *w;
    const int nw = smp_window(a, c, &w);
    const bool pen = c.penalty != 1.0f && nw > 0;
    {   // the block's logits: every load out before the first store
        constexpr int kPer = kSmpChunk / kSmpLocal;
        float lv[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) lv[q] = a.logits[base + min(tid + q * kSmpLocal, n - 1)];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = tid + q * kSmpLocal;
            if (i < n) {
                vals[i] = lv[q];
                cnt[i] = 0;
            }
        }
    }
    if (tid == 0) {
        s_bad = 0;
        s_gt = 0;
        s_eq = 0;
    }
    lds_barrier();
    // occurrences of this block's ids in the window: the penalty is applied
    // once per occurrence, each time to the value left by the previous one
    // (sampling.rs:14-24)
    if (pen)
        for (int j = tid; j < nw; j += kSmpLocal) {
            const int id = w[j];
            if ((unsigned)id < (unsigned)a.V && id >= base && id < base + n)
                atomicAdd(&cnt[id - base], 1);
        }
    lds_barrier();
    const bool temp = c.temperature != 1.0f;
    const float inv = 1.0f / c.temperature;
    int bad = 0;
    for (int i = tid; i < n; i += kSmpLocal) {
        float y = vals[i];
        for (int r = cnt[i]; r > 0; --r) y = y > 0.0f ? y / c.penalty : y * c.penalty;
        if (temp) y = y * inv;
        a.y[base + i] = y;
        bad |= (y != y) | (y == __builtin_inff());
        ords[i] = smp_ord(y);
    }
    if (bad) atomicOr(&s_bad, 1);
    const int kk = smp_kk(c, a.V);
    const int kl = (kk >= 1 && kk <= kSmpKMax) ? kk : 1;   // list length
    unsigned long long *list = a.cand + (size_t)b * kSmpKMax;
    lds_barrier();
    if (n <= kl) {   // the whole block is its list
        for (int j = tid; j < kl; j += kSmpLocal)
            list[j] = j < n ? smp_key(ords[j], base + j) : 0ull;
        if (tid == 0) {
            a.bflag[b] = s_bad ? 2 : 0;
            a.bthr[b] = 0;
        }
        return;
    }
    const uint32_t t = smp_select<kSmpLocal>(
        n, kl, [&](int i) { return ords[i]; }, hist, &s_prefix, &s_rem);
    // fewer than kl keys are above t; values equal to t fill the rest
    for (int i = tid; i < n; i += kSmpLocal)
        if (ords[i] > t) list[atomicAdd(&s_gt, 1)] = smp_key(ords[i], base + i);
    lds_barrier();
    const int gt = s_gt;
    for (int i = tid; i < n; i += kSmpLocal)
        if (ords[i] == t) {
            const int slot = gt + atomicAdd(&s_eq, 1);
            if (slot < kl) list[slot] = smp_key(t, base + i);
        }
    lds_barrier();
    if (tid == 0) {
        a.bflag[b] = (s_bad ? 2 : 0) | (gt + s_eq > kl ? 1 : 0);
        a.bthr[b] = t;
    }
}

__global__ __launch_bounds__(kSmpThreads) void sample_final_kernel(SmpArgs a) {
    extern __shared__ unsigned long long sk[];   // kSmpFinalKeys keys, then kSmpSurv
    unsigned long long *sv = sk + kSmpFinalKeys;
    __shared__ int s_flag, s_nc, s_nl, s_tok, s_rem;
    __shared__ uint32_t s_mx, s_lo, s_prefix, s_hist[256];
    __shared__ float s_r;
    const SampleCtl c = smp_ctl(a);
    const int tid = threadIdx.x, G = a.G, V = a.V;
    const int kk = smp_kk(c, V);
    const float u = a.u[smp_draw_index(a)];
    if (tid == 0) {
        s_flag = 0;
        s_nc = 0;
        s_nl = 0;
        s_mx = 0;
        s_lo = 0;
        s_tok = V - 1;
    }
    lds_barrier();
    const int kl = (kk >= 1 && kk <= kSmpKMax) ? kk : 1;
    const bool sparse = kk >= 1 && kk <= kSmpKMax && G * kk <= kSmpFinalKeys;
    const int nk = G * kl;
    // the k-th largest overall is at least every block's k-th largest (that
    // block alone has k values at or above it): only list keys at or above
    // the largest block threshold lo can be the threshold or reach it
    uint32_t lo = 0;
    for (int b = tid; b < G; b += kSmpThreads) {
        if (a.bflag[b] & 2) atomicOr(&s_flag, 2);
        lo = max(lo, a.bthr[b]);
    }
    atomicMax(&s_lo, lo);
    lds_barrier();
    lo = s_lo;
    // the largest key is in its block's list whatever k is.  The keys are
    // read 8 per thread at a time, all 8 loads out before the first use (one
    // at a time, the LDS atomics between them kept each a round trip of its
    // own: 13 for k = 50 over 63 blocks)
    uint32_t mx = 0;
    constexpr int kB = 8;
    for (int i0 = tid; i0 < nk; i0 += kB * kSmpThreads) {
        unsigned long long kv[kB];
#pragma unroll
        for (int q = 0; q < kB; ++q) {
            const int i = min(i0 + q * kSmpThreads, nk - 1);   // clamped; used only below nk
            kv[q] = a.cand[(size_t)(i / kl) * kSmpKMax + (i % kl)];
        }
#pragma unroll
        for (int q = 0; q < kB; ++q) {
            if (i0 + q * kSmpThreads >= nk) break;
            const unsigned long long k = kv[q];
            mx = max(mx, (uint32_t)(k >> 32));
            if (sparse && (uint32_t)(k >> 32) >= lo) sk[atomicAdd(&s_nl, 1)] = k;
        }
    }
    atomicMax(&s_mx, mx);
    lds_barrier();
    const int nl = s_nl;
    const float mxv = smp_unord(s_mx);
    // NaN / +inf (sum NaN) or every value -inf (exp(-inf - -inf) is NaN): V - 1
    const bool degenerate = (s_flag & 2) || mxv == -__builtin_inff();
    uint32_t thr = 0;   // threshold as smp_ord (0: below everything)
    bool dense = !degenerate && !sparse;
    if (!degenerate && sparse) {
        thr = smp_select<kSmpThreads>(
            nl, kk, [&](int i) { return (uint32_t)(sk[i] >> 32); }, s_hist, &s_prefix, &s_rem);
        for (int b = tid; b < G; b += kSmpThreads)
            if ((a.bflag[b] & 1) && a.bthr[b] == thr) atomicOr(&s_flag, 1);
        // the values >= threshold, (index, value) keys in any order
        for (int i = tid; i < nl; i += kSmpThreads) {
            const uint32_t o = (uint32_t)(sk[i] >> 32);
            if (o >= thr) {
                const int slot = atomicAdd(&s_nc, 1);
                if (slot < kSmpSurv)
                    sv[slot] = ((unsigned long long)(uint32_t)smp_index(sk[i]) << 32) | o;
            }
        }
        lds_barrier();
        if ((s_flag & 1) || s_nc > kSmpSurv) {
            dense = true;   // more values reach the threshold than the lists hold
        } else {
            const int nc = s_nc;
            // order by index (distinct): each key's rank is its place; e = exp(v - max)
            for (int j = tid; j < nc; j += kSmpThreads) {
                const unsigned long long kj = sv[j];
                int rank = 0;
                for (int i = 0; i < nc; ++i) rank += sv[i] < kj;
                const float e = oxb_expf(smp_unord((uint32_t)kj) - mxv);
                sk[rank] = (kj & 0xffffffff00000000ull) | __float_as_uint(e);
            }
            lds_barrier();
            if (tid == 0) {
                float s = 0.0f;
                for (int i = 0; i < nc; ++i) s = s + __uint_as_float((uint32_t)sk[i]);
                const float r = u * s;
                int tok = V - 1;
                if (r <= 0.0f) {
                    tok = 0;   // the running sum at index 0 (>= 0) already reaches r
                } else {
                    float cum = 0.0f;
                    for (int i = 0; i < nc; ++i) {
                        cum = cum + __uint_as_float((uint32_t)sk[i]);
                        if (cum >= r) {
                            tok = (int)(sk[i] >> 32);
                            break;
                        }
                    }
                }
                s_tok = tok;
            }
        }
    }
    if (dense) {
        lds_barrier();
        const bool filter = kk > 0;
        if (filter && !sparse)
            thr = smp_select<kSmpThreads>(
                V, kk, [&](int i) { return smp_ord(a.y[i]); }, s_hist, &s_prefix, &s_rem);
        const float tv = smp_unord(thr);
        float4 *buf = (float4 *)sk;
        float s = 0.0f;   // thread 0's running sum
        for (int c0 = 0; c0 < V; c0 += kSmpDense) {
            const int n = min(kSmpDense, V - c0);
            for (int i = tid; i < kSmpDense; i += kSmpThreads) {
                float e = 0.0f;   // past the end: adds nothing
                if (i < n) {
                    float y = a.y[c0 + i];
                    if (filter && y < tv) y = -__builtin_inff();
                    e = oxb_expf(y - mxv);
                }
                ((float *)buf)[i] = e;
            }
            lds_barrier();
            if (tid == 0) {
                const int n4 = (n + 3) >> 2;
#pragma unroll 4
                for (int i = 0; i < n4; ++i) {
                    float4 q = buf[i];
                    s = s + q.x;
                    q.x = s;
                    s = s + q.y;
                    q.y = s;
                    s = s + q.z;
                    q.z = s;
                    s = s + q.w;
                    q.w = s;
                    buf[i] = q;
                }
            }
            lds_barrier();
            for (int i = tid; i < n; i += kSmpThreads) a.pre[c0 + i] = ((const float *)buf)[i];
            __syncthreads();   // the running sums in memory, for the search below
        }
        if (tid == 0) {
            s_r = u * s;
            s_tok = 0x7fffffff;
        }
        lds_barrier();
        const float r = s_r;
        if (r <= 0.0f) {
            if (tid == 0) s_tok = 0;
        } else if (r == r) {
            for (int i = tid; i < V; i += kSmpThreads)
                if (a.pre[i] >= r) {
                    atomicMin(&s_tok, i);
                    break;
                }
        }
        lds_barrier();
        if (tid == 0 && (s_tok == 0x7fffffff || r != r)) s_tok = V - 1;
    }
    lds_barrier();
    if (tid == 0) {
        const int tok = s_tok;
        if (a.out) *a.out = tok;
        if (a.state) {
            const int ng = a.state[OXB_ST_NGEN];
            a.state[OXB_ST_TOKEN] = tok;
            if (a.hist && ng >= 1 && ng - 1 < a.state[OXB_ST_HIST_CAP]) a.hist[ng - 1] = tok;
        }
    }
}

static size_t smp_align(size_t b) { return (b + 255) & ~(size_t)255; }

static int smp_blocks(int V) { return (V + kSmpChunk - 1) / kSmpChunk; }

size_t sample_ws_bytes(int V) {
    if (V <= 0) return 0;
    const size_t G = (size_t)smp_blocks(V);
    return 2 * smp_align((size_t)V * 4) + smp_align(G * kSmpKMax * 8) + 2 * smp_align(G * 4);
}

int sample_enqueue(const float *logits, int V, const SampleCtl *ctl_dev, SampleCtl ctl,
                   const int *win, int nwin, int *state, int *hist, const float *u, int *out,
                   void *ws, size_t ws_bytes, void *stream) {
    OXB_REQUIRE(logits && V > 0 && u && ws, "sample: null logits, draws or workspace");
    OXB_REQUIRE(state || out, "sample: no output");
    OXB_REQUIRE(state || nwin == 0 || win, "sample: null window");
    OXB_REQUIRE(nwin >= 0, "sample: window length %d", nwin);
    OXB_REQUIRE(ws_bytes >= sample_ws_bytes(V), "sample: workspace %zu bytes < %zu", ws_bytes,
                sample_ws_bytes(V));
    const int G = smp_blocks(V);
    char *p = (char *)ws;
    SmpArgs a{};
    a.logits = logits;
    a.V = V;
    a.ctl = ctl;
    a.ctl_dev = ctl_dev;
    a.win = win;
    a.nwin = nwin;
    a.state = state;
    a.hist = hist;
    a.u = u;
    a.out = out;
    a.y = (float *)p;
    p += smp_align((size_t)V * 4);
    a.pre = (float *)p;
    p += smp_align((size_t)V * 4);
    a.cand = (unsigned long long *)p;
    p += smp_align((size_t)G * kSmpKMax * 8);
    a.bflag = (int *)p;
    p += smp_align((size_t)G * 4);
    a.bthr = (uint32_t *)p;
    a.G = G;
    hipStream_t s = (hipStream_t)stream;
    if (allow_dynamic_lds((const void *)sample_final_kernel)) return -1;
    hipLaunchKernelGGL(sample_local_kernel, dim3(G), dim3(kSmpLocal), 0, s, a);
    OXB_CHECK_HIP(hipGetLastError());
    hipLaunchKernelGGL(sample_final_kernel, dim3(1), dim3(kSmpThreads),
                       (kSmpFinalKeys + kSmpSurv) * sizeof(unsigned long long), s, a);
    OXB_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace oxb

extern "C" size_t oxb_sample_ws_bytes(int V) { return oxb::sample_ws_bytes(V); }

extern "C" int oxb_sample_device(const float *logits, int V, float temperature, size_t top_k,
                                 float repeat_penalty, const int32_t *recent, int n_recent,
                                 const float *u, int32_t *token, void *ws, size_t ws_bytes,
                                 void *stream) {
    oxb::clear_error();
    OXB_REQUIRE(token, "sample: null token output");
    oxb::SampleCtl c{temperature, (top_k > 0 && top_k < (size_t)V) ? (int)top_k : 0,
                     repeat_penalty, 0};
    return oxb::sample_enqueue(logits, V, nullptr, c, recent, n_recent, nullptr, nullptr, u,
                               token, ws, ws_bytes, stream);
}
