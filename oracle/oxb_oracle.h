/*
 * oxb_oracle.h — CPU restatement of 0xBitNet's ternary inference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP product
 * is compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and never as the thing measured or shipped.
 *
 * Every function restates one WGSL entry point (or one Rust orchestration
 * routine) of the reference and cites the file:line it follows.  Paths are
 * relative to the reference root:
 *   sh/  = packages/rust/crates/oxbitnet/src/shaders/
 *   rs/  = packages/rust/crates/oxbitnet/src/
 *   ts/  = packages/core/src/shaders/__tests__/helpers/
 *
 * Float conventions (chosen once, used by both this oracle and the product):
 *   - every f32 op is a separately rounded IEEE op: no implicit FMA
 *     contraction (built with -ffp-contract=off).  Explicit fused
 *     multiply-adds (fmaf, one rounding, the same bits on host and device)
 *     are used in three places: the attention dot products and P.V sums
 *     (sh/attention.wgsl:48-58,96-104) and the LM-head dot products
 *     (sh/f32_matmul.wgsl:51-57), all `sum += a * b`, which WGSL lets the
 *     driver contract into an fma, so the reference's own rounding there is
 *     driver-defined; and oxo_expf below;
 *   - WGSL inverseSqrt(v) is restated as 1.0f / sqrtf(v);
 *   - WGSL exp() (implementation-defined) is restated as oxo_expf: Cody-Waite
 *     reduction x = k*ln2 + r (ln2 split into a 15-bit head and a tail),
 *     degree-7 Taylor polynomial of e^r by Horner, then ldexp(p, k), every
 *     step an explicit fmaf (the one place fused ops are used: fmaf is
 *     correctly rounded on host and device alike); max error ~1 ulp,
 *     pinned against double-precision exp in the tests;
 *   - WGSL round() is round-half-to-even (rintf), NOT the TS spec's
 *     Math.round (ts/reference.ts:70), which differs on .5 ties;
 *   - workgroup reductions follow the shaders' order exactly: 256 strided
 *     partial sums (col = t, t+256, ...) followed by the halving tree
 *     s[t] += s[t + stride], stride = 128 .. 1.
 */
#ifndef OXB_ORACLE_H
#define OXB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 <-> f32 (IEEE binary16, round-to-nearest-even) ---------------- */
float    oxo_f16_to_f32(uint16_t h);
uint16_t oxo_f32_to_f16(float f);

/* ---- exp used wherever the shaders call exp() (softmax, SiLU) ---------- */
float oxo_expf(float x);

/* ---- I2_S packing ------------------------------------------------------ */
/* Pack K ternary values {-1,0,+1} of one row into I2_S bytes (K padded to a
 * multiple of 128 with zeros).  Output has ceil(K/128)*32 bytes.
 * Follows ts/i2s-pack.ts:110-138. */
void oxo_i2s_pack_row(const int8_t *w, int K, uint8_t *out);
/* Decode element k of an I2_S row: w = ((byte >> shift) & 3) - 1 with
 * byte = row[(k/128)*32 + k%32], shift = 6 - 2*((k%128)/32).
 * Follows sh/ternary_gemv.wgsl:58-71. */
int  oxo_i2s_get(const uint8_t *row, int k);
void oxo_i2s_unpack_row(const uint8_t *row, int K, int8_t *w);

/* ---- per-token absmax int8 quantize: sh/quantize.wgsl:28-74 ------------ */
void oxo_quantize(const float *x, int n_tok, int D, int8_t *q, float *scales);

/* ---- RMSNorm: sh/rmsnorm.wgsl:27-63 ------------------------------------ */
void oxo_rmsnorm(const float *x, const float *w, int n_tok, int D, float eps,
                 float *y);

/* ---- ternary GEMV (n_tok == 1): sh/ternary_gemv.wgsl:39-97 -------------- */
/* W: [out_dim][K/4] I2_S bytes.  acc (optional) gets the exact int32 dot.
 * y[r] = ((float)acc * wscale[r]) * in_scale. */
void oxo_gemv(const uint8_t *W, const int8_t *x, const float *wscale,
              float in_scale, int out_dim, int K, int32_t *acc, float *y);

/* ---- ternary GEMM (n_tok > 1): sh/ternary_gemm.wgsl:40-136 -------------- */
/* X: [n_tok][K] int8.  Y: [n_tok][out_dim] f32.
 * Y[t][r] = (float)acc * (wscale[r] * in_scales[t]). */
void oxo_gemm(const uint8_t *W, const int8_t *X, const float *wscale,
              const float *in_scales, int out_dim, int n_tok, int K,
              int32_t *acc, float *Y);

/* ---- activation / elementwise: sh/activation.wgsl:19-38,
 *      sh/elementwise.wgsl:20-34 ------------------------------------------ */
void oxo_relu2(const float *x, size_t n, float *y);
void oxo_silu(const float *x, size_t n, float *y);
void oxo_add(const float *a, const float *b, size_t n, float *y);
void oxo_mul(const float *a, const float *b, size_t n, float *y);

/* ---- RoPE: sh/rope.wgsl:25-56 ------------------------------------------ */
void oxo_rope(const float *x, int n_tok, int heads, int hd, int pos_offset,
              float theta_base, float *y);

/* ---- attention: sh/attention.wgsl:29-59 (scores), sh/softmax.wgsl:25-80,
 *      sh/attention.wgsl:79-105 (attn_v); orchestration
 *      rs/nn/attention.rs:85-124 -------------------------------------------
 * q: [n_tok][H][hd]; K, V caches: [S][Hkv][hd] (S = positions incl. the new
 * ones); out: [n_tok][H][hd].
 * P.V (sh/attention.wgsl:96-104): out[d] = sum of p[s] * v[s][d] in one
 * loop over s = 0 .. S-1, one fmaf per step (see the float conventions
 * above); masked positions (p = 0) add exact zeros, so a query is summed over
 * its own positions only. */
void oxo_attention(const float *q, const float *kc, const float *vc, int n_tok,
                   int S, int H, int Hkv, int hd, float *out);
/* The same attention with P.V summed in blocks of pv_block positions in order
 * of s (each block from zero) and the block sums added in block order; the
 * shader's one loop when pv_block <= 0 or pv_block >= S.  NOT the reference
 * order past pv_block positions: a named variant kept so that the tests can
 * show that they tell this association from the reference's (no product path
 * computes it). */
void oxo_attention_pv_blocked(const float *q, const float *kc, const float *vc,
                              int n_tok, int S, int H, int Hkv, int hd,
                              int pv_block, float *out);
/* softmax rows in place order: sh/softmax.wgsl */
void oxo_softmax(const float *x, int rows, int D, float *y);

/* ---- embedding: sh/embedding.wgsl:23-46 -------------------------------- */
void oxo_embedding(const uint32_t *ids, int n_tok, const uint16_t *E, int V,
                   int D, float *out);

/* ---- tied f16 LM head: sh/f32_matmul.wgsl:27-74 ------------------------ */
void oxo_lm_head(const float *h, const uint16_t *E, int V, int D, float *logits);

/* ---- greedy pick (rs/sampling.rs:4-80 with top_k = 1): argmax, lowest
 *      index wins ties --------------------------------------------------- */
int oxo_argmax(const float *x, int n);

/* ---- whole model: rs/nn/model.rs:193-266, rs/nn/transformer.rs:51-75,
 *      rs/nn/attention.rs:85-124, rs/nn/ffn.rs:60-80,
 *      rs/nn/bitlinear.rs:52-97 ------------------------------------------ */
typedef struct {
    const uint8_t *wq, *wk, *wv, *wo, *wgate, *wup, *wdown; /* I2_S rows */
    float sq, sk, sv, so, sgate, sup, sdown;                /* tensor scales */
    const float *attn_norm, *ffn_norm;   /* [D] */
    const float *attn_sub_norm;          /* [H*hd], may be NULL */
    const float *ffn_sub_norm;           /* [F],   may be NULL */
} oxo_layer;

/* Probe sites: oxo_forward hands each intermediate of a layer to the model's
 * probe callback (if set), all rows of the call at once, so that tests can
 * check the composition itself (norm placement, residual order, causality,
 * GQA mapping) and not only the final logits.  Q8 sites are int8 [n][in],
 * SCALE sites f32 [n]; the rest f32 [n][width]. */
enum {
    OXO_SITE_X_IN = 0,      /* residual stream entering the layer      [n][D]   */
    OXO_SITE_ATTN_NORM,     /* input_layernorm output                  [n][D]   */
    OXO_SITE_QKV_Q8,        /* int8 input of q/k/v_proj (one per layer) [n][D]  */
    OXO_SITE_QKV_SCALE,
    OXO_SITE_Q,             /* q after RoPE                            [n][H*hd] */
    OXO_SITE_K,             /* k after RoPE, before any f16 rounding   [n][Hkv*hd] */
    OXO_SITE_V,             /*                                          [n][Hkv*hd] */
    OXO_SITE_ATTN,          /* attention output (input of o_proj)      [n][H*hd] */
    OXO_SITE_O_Q8,          /* int8 input of o_proj (after attn_sub_norm) */
    OXO_SITE_O_SCALE,
    OXO_SITE_O,             /* o_proj output                           [n][D]   */
    OXO_SITE_X_MID,         /* residual after attention                [n][D]   */
    OXO_SITE_FFN_NORM,      /* post_attention_layernorm output         [n][D]   */
    OXO_SITE_GATE,          /* gate_proj output (before the activation) [n][F]  */
    OXO_SITE_UP,            /* up_proj output                          [n][F]   */
    OXO_SITE_DOWN_Q8,       /* int8 input of down_proj (after ffn_sub_norm) */
    OXO_SITE_DOWN_SCALE,
    OXO_SITE_DOWN,          /* down_proj output                        [n][D]   */
    OXO_SITE_X_OUT,         /* residual leaving the layer              [n][D]   */
    OXO_SITE_FINAL,         /* final RMSNorm output, layer = -1        [n][D]   */
    OXO_N_SITES
};
typedef void (*oxo_probe_fn)(void *ud, int layer, int site, const void *data, size_t bytes);

typedef struct {
    int n_layers, D, F, H, Hkv, V, max_seq;
    float eps, rope_theta;
    int kv_f16; /* 1: round K/V to f16 on append (the product's f16 cache) */
    const uint16_t *embed; /* [V][D] f16, tied LM head */
    const float *final_norm;
    const oxo_layer *layers;
    float *kcache, *vcache; /* each [n_layers][max_seq][Hkv][hd] */
    int seq_len;
    oxo_probe_fn probe;     /* optional: intermediates, see OXO_SITE_* */
    void *probe_ud;
    int pv_block;           /* 0: the reference's one-loop P.V; > 0: the named
                               blocked variant (oxo_attention_pv_blocked) */
} oxo_model;

/* Forward n_tok ids at position model->seq_len; writes the last token's
 * logits [V] and advances seq_len.  Returns 0, or -1 if the cache would
 * overflow. */
int oxo_forward(oxo_model *m, const uint32_t *ids, int n_tok, float *logits);

/* ---- OpenMP helpers for the CPU baseline -------------------------------- */
int oxo_num_threads(void);
void oxo_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
