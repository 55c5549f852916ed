// Shared definitions for the MI355X (gfx950) ternary inference kernels.
//
// Device-side conventions:
//  - wave64; every workgroup reduction that must be bit-identical to the
//    reference shaders uses their order: 256 strided partials, then the
//    halving tree s[t] += s[t + stride] (stride 128 .. 1).
//  - all f32 arithmetic is compiled with -ffp-contract=off; explicit fmaf()
//    is used only where the result is compared within a tolerance.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>

namespace oxb {

// Thread-local last-error plumbing shared by every extern "C" entry point.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
const char *last_error();

// Raises a kernel's dynamic-LDS ceiling on the current device to what a CU
// leaves beside the kernel's static LDS, once per (device, kernel) and safe to
// call from several host threads (the attribute is a ceiling: a launch's own
// dynamic size still sets its occupancy).  0, or -1 with the error set.
int allow_dynamic_lds(const void *kernel);
// Compute units of the current device (queried once; 256 if the query fails).
int device_cus();

}  // namespace oxb

#define OXB_CHECK_HIP(call)                                                   \
    do {                                                                      \
        hipError_t oxb_e_ = (call);                                           \
        if (oxb_e_ != hipSuccess) {                                           \
            oxb::set_error("%s: %s (%s:%d)", #call, hipGetErrorString(oxb_e_), \
                           __FILE__, __LINE__);                               \
            return -1;                                                        \
        }                                                                     \
    } while (0)

#define OXB_REQUIRE(cond, ...)            \
    do {                                  \
        if (!(cond)) {                    \
            oxb::set_error(__VA_ARGS__);  \
            return -1;                    \
        }                                 \
    } while (0)

namespace oxb {

constexpr int kWave = 64;
constexpr int kTileRows = 16;   // rows per tile of the repacked ternary layout
constexpr int kChunkBytes = 16; // one lane load: 64 ternary weights

// Repacked ternary matrix ("tile-chunk" order, built once at load time):
//   tile t = rows [16t, 16t+16); inside a tile the 16-byte chunks are stored
//   chunk-major: offset(t, kc, r) = (t*KC + kc)*16 + r  [in 16-byte units],
//   KC = K/64.  Chunk (r, kc) is bytes [16kc, 16kc+16) of the row's natural
//   I2_S encoding, i.e. 4 bit-planes x 16 consecutive weights
//   k = (kc/2)*128 + g*32 + (kc%2)*16 + j, g = 0..3, j = 0..15.
// A wave load of lane l -> (r = l%16, kc = kc0 + l/16) reads 1 KiB contiguous.
__host__ __device__ inline size_t tiled_offset16(int row, int kc, int KC) {
    return ((size_t)(row >> 4) * KC + kc) * 16 + (row & 15);
}

// The decode V copy in position octets (per KV head of a layer): element
// (position s, dim d) of a head of hd dims at ((s / 8) * hd + d) * 8 + s % 8,
// so one 16-byte load gives one dim's 8 consecutive positions and a wave's
// 64 lanes (64 consecutive dims) read 1 KB contiguous.  A head holds
// max_seq rounded up to 8 positions.
__host__ __device__ inline size_t v8_head_elems(int max_seq, int hd) {
    return (size_t)((max_seq + 7) & ~7) * hd;
}
__host__ __device__ inline size_t v8_index(int s, int d, int hd) {
    return ((size_t)(s >> 3) * hd + d) * 8 + (s & 7);
}

// exp(x) for the softmaxes and the sampler, fixed so that host and device give
// the same bits:
// Cody-Waite reduction x = k*ln2 + r (15-bit head of ln2 plus the tail),
// degree-7 Taylor polynomial of e^r by Horner, ldexp by k.  Every step after
// the first product is an explicit fused multiply-add (one IEEE rounding,
// the same on the host's fmaf); ~1 ulp.
// Branch-free: the polynomial path runs for every x and the special cases
// are selected afterwards (NaN last), which gives the same value as testing
// them first and lets many independent exps interleave.
__host__ __device__ inline float oxb_expf(float x) {
    const float kf = rintf(x * 1.44269502f);
    float r = __builtin_fmaf(-kf, 0.693145751953125f, x);
    r = __builtin_fmaf(-kf, 1.42860677e-06f, r);
    float p = __builtin_fmaf(1.98412701e-04f, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    // |k| <= 150 in range; the clamp keeps the conversion defined elsewhere
    float y = ldexpf(p, (int)fminf(fmaxf(kf, -200.0f), 200.0f));
    y = x > 88.7228394f ? __builtin_inff() : y;
    y = x < -103.972084f ? 0.0f : y;
    return x != x ? x : y;
}

}  // namespace oxb

namespace oxb {
// The LM head's lm-tiled layout of the tied f16 table [V][D] (oxb_repack_lm,
// NJ = D / 512): 64-row tiles; within a tile, row r's dwords in uint4 u / 4
// (component u % 4) of lane slot r, where dword dh = t + 256 j of the row has
// u = i NJ + j and t is the bit-reversal image of i (its own inverse).
__host__ __device__ inline int bitrev4(int x) {
    return ((x & 1) << 3) | ((x & 2) << 1) | ((x & 4) >> 1) | ((x & 8) >> 3);
}
// the dword holding elements 2 dh and 2 dh + 1 of row `row`
__host__ __device__ inline size_t lm_dword(int row, int dh, int NJ) {
    const int t = dh & 255, j = dh >> 8;
    const int i = (bitrev4(t & 15) << 4) | bitrev4(t >> 4);
    const int u = i * NJ + j;
    return (((size_t)(row >> 6) * 64 * NJ + (u >> 2)) * 64 + (row & 63)) * 4 + (u & 3);
}
}  // namespace oxb

#ifdef __HIPCC__
namespace oxb {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: weights are read once per step).
__device__ inline uint4 load_nt(const uint4 *p) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 0 in a VGPR the compiler cannot see through.  A load indexed by it stays a
// per-lane value: a load of a uniform address would be copied to an SGPR
// where it is first used, and that copy waits for the load on the spot.
__device__ inline int opaque_zero() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// Workgroup barrier that orders LDS only.  __syncthreads() also fences
// global memory, which makes every wave wait for all of its loads in flight
// (weight or V prefetch for later stages) at each barrier; the kernels'
// barriers only hand LDS data between waves.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// f32 workgroup sum in the shaders' tree order for a 256-thread block.
// Every thread passes its strided partial; the result is returned to all.
// red must hold >= 256 floats of LDS.
__device__ inline float block256_tree_sum(float part, float *red) {
    const int t = threadIdx.x;
    red[t] = part;
    lds_barrier();
    if (t < 128) red[t] = red[t] + red[t + 128];
    lds_barrier();
    if (t < 64) red[t] = red[t] + red[t + 64];
    lds_barrier();
    if (t < 64) {
        float v = red[t];
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) v = v + __shfl_down(v, s, 64);
        if (t == 0) red[0] = v;
    }
    lds_barrier();
    float r = red[0];
    lds_barrier();
    return r;
}

__device__ inline float block256_max(float v, float *red) {
    const int t = threadIdx.x;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    if ((t & 63) == 0) red[t >> 6] = v;
    lds_barrier();
    float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    lds_barrier();
    return r;
}

__device__ inline int block256_isum(int v, int *red) {
    const int t = threadIdx.x;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
    if ((t & 63) == 0) red[t >> 6] = v;
    lds_barrier();
    int r = red[0] + red[1] + red[2] + red[3];
    lds_barrier();
    return r;
}

// Order-free wave reductions over DPP (row_shr 1/2/4/8, row_bcast 15/31);
// the identity of the inactive sources is 0, so these are for integer sums
// and maxima of non-negative floats.  The result is lane 63's, returned
// to every lane.
template <int CTRL, int ROWMASK>
__device__ inline int dpp0(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWMASK, 0xf, false);
}

__device__ inline int wave_isum_dpp(int v) {
    v += dpp0<0x111, 0xf>(v);
    v += dpp0<0x112, 0xf>(v);
    v += dpp0<0x114, 0xf>(v);
    v += dpp0<0x118, 0xf>(v);
    v += dpp0<0x142, 0xa>(v);
    v += dpp0<0x143, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ inline float wave_nonneg_max_dpp(float f) {
    int v = __float_as_int(f);
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp0<0x111, 0xf>(v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp0<0x112, 0xf>(v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp0<0x114, 0xf>(v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp0<0x118, 0xf>(v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp0<0x142, 0xa>(v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp0<0x143, 0xc>(v))));
    return __int_as_float(__builtin_amdgcn_readlane(v, 63));
}

// The shaders' 256-thread halving tree (s[t] += s[t+stride], stride 128..1)
// with one LDS pass: wave 0 folds strides 128 and 64 in registers, then
// every thread evaluates strides 32..1 of the 64 survivors locally.  red
// holds >= 320 floats; all 256 threads must call; result to all threads.
__device__ inline float block256_tree_sum_fast(float part, float *red) {
    const int t = threadIdx.x;
    red[t] = part;
    lds_barrier();
    if (t < 64) red[256 + t] = (red[t] + red[t + 128]) + (red[t + 64] + red[t + 192]);
    lds_barrier();
    float a[64];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 f = *(const float4 *)(red + 256 + 4 * i);
        a[4 * i] = f.x; a[4 * i + 1] = f.y; a[4 * i + 2] = f.z; a[4 * i + 3] = f.w;
    }
#pragma unroll
    for (int st = 32; st > 0; st >>= 1)
#pragma unroll
        for (int i = 0; i < st; ++i) a[i] = a[i] + a[i + st];
    return a[0];
}

// The same 256-thread halving tree with a single barrier.  After the
// strides 128..32 and 16 the survivor i < 16 is
//   w[i] = (u[i] + u[i+32]) + (u[i+16] + u[i+48]),
//   u[j] = (s[j] + s[j+128]) + (s[j+64] + s[j+192]),
// so lane i of every 16-lane row reads its 16 leaves from LDS and folds them
// in that order; DPP row_shl:8,4,2,1 (lane l takes lane l+k of its row) does
// strides 8..1 and lane 0 holds the shader's sum.  red >= 256 floats.
// block256_tree_fold: the fold once the 256 partials are in red (a barrier
// published them), by one whole wave, result to every lane;
// block256_tree_sum_1b: store, barrier and fold, all 256 threads must call.
__device__ inline float block256_tree_fold(const float *red) {
    const int i = threadIdx.x & 15;
    float u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = i + 16 * k;
        u[k] = (red[j] + red[j + 128]) + (red[j + 64] + red[j + 192]);
    }
    float s = (u[0] + u[2]) + (u[1] + u[3]);
    s = s + __int_as_float(dpp0<0x108, 0xf>(__float_as_int(s)));
    s = s + __int_as_float(dpp0<0x104, 0xf>(__float_as_int(s)));
    s = s + __int_as_float(dpp0<0x102, 0xf>(__float_as_int(s)));
    s = s + __int_as_float(dpp0<0x101, 0xf>(__float_as_int(s)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
}

__device__ inline float block256_tree_sum_1b(float part, float *red) {
    const int t = threadIdx.x & 255;   // a 256-thread group, red its own 256 slots
    red[t] = part;
    lds_barrier();
    return block256_tree_fold(red);
}

// Max over the wave of finite floats (lanes without a DPP source keep their
// own value), returned to every lane.
template <int CTRL, int ROWMASK>
__device__ inline float dpp_keep(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
__device__ inline float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_keep<0x111, 0xf>(v));
    v = fmaxf(v, dpp_keep<0x112, 0xf>(v));
    v = fmaxf(v, dpp_keep<0x114, 0xf>(v));
    v = fmaxf(v, dpp_keep<0x118, 0xf>(v));
    v = fmaxf(v, dpp_keep<0x142, 0xa>(v));
    v = fmaxf(v, dpp_keep<0x143, 0xc>(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Halving tree s[l] += s[l + stride], stride 32..1, over the 64 lanes (the
// last six levels of the shaders' 256-thread tree); lane 0's value returned
// to every lane.  Strides 32 and 16 by lane shuffles, 8..1 by DPP row_shl.
__device__ inline float wave_tree_sum(float c) {
    c = c + __shfl_down(c, 32, 64);
    c = c + __shfl_down(c, 16, 64);
    c = c + __int_as_float(dpp0<0x108, 0xf>(__float_as_int(c)));
    c = c + __int_as_float(dpp0<0x104, 0xf>(__float_as_int(c)));
    c = c + __int_as_float(dpp0<0x102, 0xf>(__float_as_int(c)));
    c = c + __int_as_float(dpp0<0x101, 0xf>(__float_as_int(c)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), 0));
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
    return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    return v;
}

// oxb_expf for the softmax's arguments x - max <= 0 (or NaN): the same bits
// there, in fewer instructions (no overflow test, and NaN propagates through
// the arithmetic).  For x > 0 the result is not oxb_expf's; the softmax only
// evaluates x > 0 for positions it discards.
__device__ inline float oxb_expf_nonpos(float x) {
    const float kf = rintf(x * 1.44269502f);
    float r = __builtin_fmaf(-kf, 0.693145751953125f, x);
    r = __builtin_fmaf(-kf, 1.42860677e-06f, r);
    float p = __builtin_fmaf(1.98412701e-04f, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float y = ldexpf(p, (int)fmaxf(kf, -200.0f));   // kf <= 0 for x <= 0
    return x < -103.972084f ? 0.0f : y;
}

// Direct global -> LDS loads (global_load_lds_dwordx4): each lane's 16 B
// land at the wave's LDS base + 16 * lane, taking no VGPRs and no LDS
// store instructions.
// The loads are issued from inline assembly with explicit vmcnt waits: the
// compiler's builtin for them makes every later LDS read wait for all
// outstanding loads, which would serialise the prefetch.  The compiler does
// not count these loads, so its own vmcnt waits can only come out stricter.
// The LDS base goes through m0, which the asm saves and restores itself (m0 is
// a reserved register: declaring it clobbered is not allowed).
__device__ __forceinline__ void lds_dma16(const void *g, const uint4 *lds_wave_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)lds_wave_base);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(g)
        : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // s_waitcnt immediate: vmcnt[3:0] | expcnt 7 << 4 | lgkmcnt 15 << 8 | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// sh/quantize.wgsl:59,68,71 for one value given the row absmax.
__device__ inline int quant_one(float v, float inv) {
    int q = (int)rintf(v * inv);
    return q < -127 ? -127 : (q > 127 ? 127 : q);
}

// Dot of four 2-bit planes of one packed dword against four int8 activation
// dwords (one per plane).  Codes c in {0,1,2} are used unshifted where the
// masked field still fits a signed byte: plane 3 (bits 1:0) x1, plane 2
// (bits 3:2) x4, planes 1 (bits 5:4) and 0 (bits 7:6, moved down by 2) x16.
// The true dot is acc1 + acc4/4 + acc16/16 - sum(x) (w = c - 1).
struct CodeAcc {
    int a1 = 0, a4 = 0, a16 = 0;
    __device__ inline void add(uint32_t w, int x0, int x1, int x2, int x3) {
        a1 = __builtin_amdgcn_sdot4((int)(w & 0x03030303u), x3, a1, false);
        a4 = __builtin_amdgcn_sdot4((int)(w & 0x0c0c0c0cu), x2, a4, false);
        a16 = __builtin_amdgcn_sdot4((int)(w & 0x30303030u), x1, a16, false);
        a16 = __builtin_amdgcn_sdot4((int)((w >> 2) & 0x30303030u), x0, a16, false);
    }
    __device__ inline int codes() const { return a1 + (a4 >> 2) + (a16 >> 4); }
};

}  // namespace oxb
#endif
