/*
 * oxb_oracle.c — CPU restatement of 0xBitNet's ternary inference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  See oxb_oracle.h for the float
 * conventions and the path legend (sh/, rs/, ts/).  Build with
 * -ffp-contract=off and without -ffast-math: every f32 operation below is a
 * separately rounded IEEE operation, in the order the WGSL shader uses.
 */
#include "oxb_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define WG 256 /* WORKGROUP_SIZE of every reduction shader */

/* ------------------------------------------------------------------------ */
/* f16 <-> f32, bit-level (IEEE 754 binary16).                               */
/* ------------------------------------------------------------------------ */
float oxo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oxo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0));
    }
    if (absx >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absx < 0x38800000u) { /* below the smallest normal: subnormal or 0 */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 -> 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* 14 .. 24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((absx >> 13) - ((127 - 15) << 10));
    uint32_t rem = absx & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

/* ------------------------------------------------------------------------ */
/* exp: Cody-Waite range reduction + degree-7 Taylor polynomial, every step a */
/* fused multiply-add (fmaf: one IEEE rounding), so the same steps give the  */
/* same bits on any IEEE machine with a correctly rounded fma.               */
/* ------------------------------------------------------------------------ */
float oxo_expf(float x) {
    if (x != x) return x;
    if (x < -103.972084f) return 0.0f;
    if (x > 88.7228394f) return INFINITY;
    const float kf = rintf(x * 1.44269502f);   /* round(x / ln2) */
    float r = fmaf(-kf, 0.693145751953125f, x); /* ln2 head */
    r = fmaf(-kf, 1.42860677e-06f, r);          /* ln2 tail */
    float p = fmaf(1.98412701e-04f, r, 1.38888892e-03f); /* 1/7!, 1/6! */
    p = fmaf(p, r, 8.33333377e-03f);           /* 1/5! */
    p = fmaf(p, r, 4.16666679e-02f);           /* 1/4! */
    p = fmaf(p, r, 1.66666672e-01f);           /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)kf);
}

/* ------------------------------------------------------------------------ */
/* The shaders' workgroup reduction: 256 strided partials, then a halving    */
/* tree (sh/rmsnorm.wgsl:41-55, sh/softmax.wgsl:58-71, sh/f32_matmul.wgsl). */
/* ------------------------------------------------------------------------ */
static float tree_sum(float *p /* [WG], clobbered */) {
    for (int stride = WG / 2; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; t++) p[t] = p[t] + p[t + stride];
    return p[0];
}

static float tree_max(float *p) {
    for (int stride = WG / 2; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; t++) p[t] = fmaxf(p[t], p[t + stride]);
    return p[0];
}

/* ------------------------------------------------------------------------ */
/* I2_S                                                                      */
/* ------------------------------------------------------------------------ */
void oxo_i2s_pack_row(const int8_t *w, int K, uint8_t *out) {
    /* ts/i2s-pack.ts:110-138: byte[gp] of block b holds elements
     * b*128 + g*32 + gp at bits (7-2g):(6-2g), code = value + 1. */
    int nblk = (K + 127) / 128;
    for (int b = 0; b < nblk; b++) {
        for (int gp = 0; gp < 32; gp++) {
            uint8_t byte = 0;
            for (int g = 0; g < 4; g++) {
                int k = b * 128 + g * 32 + gp;
                int v = k < K ? w[k] : 0;
                byte |= (uint8_t)((v + 1) << (6 - 2 * g));
            }
            out[b * 32 + gp] = byte;
        }
    }
}

int oxo_i2s_get(const uint8_t *row, int k) {
    /* sh/ternary_gemv.wgsl:58-71 (docs/architecture.md:150-162):
     * block = k/128, group = (k%128)/32, gp = k%32. */
    int blk = k / 128, g = (k % 128) / 32, gp = k % 32;
    uint8_t byte = row[blk * 32 + gp];
    return (int)((byte >> (6 - 2 * g)) & 3u) - 1;
}

void oxo_i2s_unpack_row(const uint8_t *row, int K, int8_t *w) {
    int nblk = K / 128;
    for (int b = 0; b < nblk; b++) {
        const uint8_t *src = row + b * 32;
        int8_t *dst = w + b * 128;
        for (int gp = 0; gp < 32; gp++) {
            uint8_t byte = src[gp];
            dst[gp] = (int8_t)(((byte >> 6) & 3) - 1);
            dst[32 + gp] = (int8_t)(((byte >> 4) & 3) - 1);
            dst[64 + gp] = (int8_t)(((byte >> 2) & 3) - 1);
            dst[96 + gp] = (int8_t)((byte & 3) - 1);
        }
    }
    for (int k = nblk * 128; k < K; k++) w[k] = (int8_t)oxo_i2s_get(row, k);
}

/* Row stride in bytes of an I2_S matrix with K columns: K_packed u32 words,
 * K_packed = ceil(K/16) (rs/nn/bitlinear.rs:46). */
static size_t i2s_row_bytes(int K) { return (size_t)((K + 15) / 16) * 4; }

/* ------------------------------------------------------------------------ */
/* quantize: sh/quantize.wgsl:28-74                                          */
/* ------------------------------------------------------------------------ */
void oxo_quantize(const float *x, int n_tok, int D, int8_t *q, float *scales) {
    for (int t = 0; t < n_tok; t++) {
        const float *row = x + (size_t)t * D;
        float absmax = 0.0f; /* max is exact: the shader's order is immaterial */
        for (int c = 0; c < D; c++) absmax = fmaxf(absmax, fabsf(row[c]));
        float scale = absmax == 0.0f ? 1.0f : absmax / 127.0f;  /* :59 */
        float inv = absmax == 0.0f ? 0.0f : 127.0f / absmax;    /* :68 */
        scales[t] = scale;
        for (int c = 0; c < D; c++) {
            float v = rintf(row[c] * inv); /* WGSL round = half to even */
            int iv = (int)v;
            if (iv < -127) iv = -127;
            if (iv > 127) iv = 127;
            q[(size_t)t * D + c] = (int8_t)iv;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm: sh/rmsnorm.wgsl:27-63                                            */
/* ------------------------------------------------------------------------ */
void oxo_rmsnorm(const float *x, const float *w, int n_tok, int D, float eps,
                 float *y) {
    float p[WG];
    for (int t = 0; t < n_tok; t++) {
        const float *row = x + (size_t)t * D;
        for (int tid = 0; tid < WG; tid++) {
            float s = 0.0f;
            for (int c = tid; c < D; c += WG) {
                float v = row[c];
                float sq = v * v;
                s = s + sq;
            }
            p[tid] = s;
        }
        float sum = tree_sum(p);
        float rms = 1.0f / sqrtf(sum / (float)D + eps); /* inverseSqrt */
        for (int c = 0; c < D; c++) {
            float a = row[c] * rms;
            y[(size_t)t * D + c] = a * w[c];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ternary GEMV / GEMM                                                       */
/* ------------------------------------------------------------------------ */
static int32_t dot_i8(const int8_t *a, const int8_t *b, int K) {
    int32_t acc = 0;
    for (int k = 0; k < K; k++) acc += (int32_t)a[k] * (int32_t)b[k];
    return acc;
}

void oxo_gemv(const uint8_t *W, const int8_t *x, const float *wscale,
              float in_scale, int out_dim, int K, int32_t *acc, float *y) {
    size_t rb = i2s_row_bytes(K);
#pragma omp parallel
    {
        int8_t *w = (int8_t *)malloc((size_t)K + 128);
#pragma omp for schedule(static)
        for (int r = 0; r < out_dim; r++) {
            oxo_i2s_unpack_row(W + (size_t)r * rb, K, w);
            int32_t a = dot_i8(w, x, K); /* exact: order is immaterial */
            if (acc) acc[r] = a;
            /* sh/ternary_gemv.wgsl:94-95: sum * scales[row] * input_scale,
             * evaluated left to right. */
            float s = (float)a * wscale[r];
            y[r] = s * in_scale;
        }
        free(w);
    }
}

void oxo_gemm(const uint8_t *W, const int8_t *X, const float *wscale,
              const float *in_scales, int out_dim, int n_tok, int K,
              int32_t *acc, float *Y) {
    size_t rb = i2s_row_bytes(K);
#pragma omp parallel
    {
        int8_t *w = (int8_t *)malloc((size_t)K + 128);
#pragma omp for schedule(static)
        for (int r = 0; r < out_dim; r++) {
            oxo_i2s_unpack_row(W + (size_t)r * rb, K, w);
            for (int t = 0; t < n_tok; t++) {
                int32_t a = dot_i8(w, X + (size_t)t * K, K);
                if (acc) acc[(size_t)t * out_dim + r] = a;
                /* sh/ternary_gemm.wgsl:132-133: acc * (w_scale * in_scale) */
                float s = wscale[r] * in_scales[t];
                Y[(size_t)t * out_dim + r] = (float)a * s;
            }
        }
        free(w);
    }
}

/* ------------------------------------------------------------------------ */
/* activation / elementwise                                                  */
/* ------------------------------------------------------------------------ */
void oxo_relu2(const float *x, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) {
        float r = fmaxf(0.0f, x[i]); /* sh/activation.wgsl:32-33 */
        y[i] = r * r;
    }
}

void oxo_silu(const float *x, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) y[i] = x[i] / (1.0f + oxo_expf(-x[i])); /* :36 */
}

void oxo_add(const float *a, const float *b, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

void oxo_mul(const float *a, const float *b, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) y[i] = a[i] * b[i];
}

/* ------------------------------------------------------------------------ */
/* RoPE: sh/rope.wgsl:25-56 (interleaved pairs 2i, 2i+1)                     */
/* ------------------------------------------------------------------------ */
void oxo_rope(const float *x, int n_tok, int heads, int hd, int pos_offset,
              float theta_base, float *y) {
    int half = hd / 2;
    for (int t = 0; t < n_tok; t++) {
        float pos = (float)(t + pos_offset);
        for (int h = 0; h < heads; h++) {
            for (int dp = 0; dp < half; dp++) {
                float fe = -2.0f * (float)dp;
                fe = fe / (float)hd;
                float th = pos * powf(theta_base, fe);
                float c = cosf(th), s = sinf(th);
                size_t bi = ((size_t)t * heads + h) * hd + (size_t)dp * 2;
                float x0 = x[bi], x1 = x[bi + 1];
                float a = x0 * c, b = x1 * s;
                float d = x0 * s, e = x1 * c;
                y[bi] = a - b;
                y[bi + 1] = d + e;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* softmax: sh/softmax.wgsl:25-80                                            */
/* ------------------------------------------------------------------------ */
static void softmax_row(const float *in, int D, float *out) {
    float p[WG];
    for (int tid = 0; tid < WG; tid++) {
        float m = -3.402823e+38f;
        for (int c = tid; c < D; c += WG) m = fmaxf(m, in[c]);
        p[tid] = m;
    }
    float row_max = tree_max(p);
    for (int tid = 0; tid < WG; tid++) {
        float s = 0.0f;
        for (int c = tid; c < D; c += WG) s = s + oxo_expf(in[c] - row_max);
        p[tid] = s;
    }
    float inv_sum = 1.0f / tree_sum(p);
    for (int c = 0; c < D; c++) out[c] = oxo_expf(in[c] - row_max) * inv_sum;
}

void oxo_softmax(const float *x, int rows, int D, float *y) {
    for (int r = 0; r < rows; r++)
        softmax_row(x + (size_t)r * D, D, y + (size_t)r * D);
}

/* ------------------------------------------------------------------------ */
/* attention (scores -> softmax -> attn_v)                                   */
/* ------------------------------------------------------------------------ */
void oxo_attention_pv_blocked(const float *q, const float *kc, const float *vc,
                              int n_tok, int S, int H, int Hkv, int hd,
                              int pv_block, float *out) {
    float scale = 1.0f / sqrtf((float)hd); /* rs/nn/attention.rs:206 */
    int group = H / Hkv;
#pragma omp parallel for schedule(static)
    for (int hq = 0; hq < H * n_tok; hq++) {
        int h = hq / n_tok, qp = hq % n_tok;
        int kvh = h / group; /* sh/attention.wgsl:43 */
        float *sc = (float *)malloc(sizeof(float) * (size_t)S);
        float *pr = (float *)malloc(sizeof(float) * (size_t)S);
        const float *qv = q + ((size_t)qp * H + h) * hd;
        for (int kp = 0; kp < S; kp++) { /* sh/attention.wgsl:48-58 */
            const float *kv = kc + ((size_t)kp * Hkv + kvh) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; d++) dot = fmaf(qv[d], kv[d], dot); /* fused: see header */
            int causal = kp > qp + (S - n_tok);
            sc[kp] = causal ? -3.402823e+38f : dot * scale;
        }
        softmax_row(sc, S, pr);
        /* sh/attention.wgsl:96-104: one loop over s for each d.  The masked
         * positions past the query's own (p = 0) add exact zeros and are not
         * visited. */
        const int Sq = qp + (S - n_tok) + 1;
        const int blk = pv_block > 0 ? pv_block : Sq;
        for (int d = 0; d < hd; d++) {
            float total = 0.0f;
            for (int b0 = 0; b0 < Sq; b0 += blk) {
                const int e = b0 + blk < Sq ? b0 + blk : Sq;
                float part = 0.0f;
                for (int s = b0; s < e; s++) /* fused: see header */
                    part = fmaf(pr[s], vc[((size_t)s * Hkv + kvh) * hd + d], part);
                total = b0 == 0 ? part : total + part;
            }
            out[((size_t)qp * H + h) * hd + d] = total;
        }
        free(sc);
        free(pr);
    }
}

void oxo_attention(const float *q, const float *kc, const float *vc, int n_tok,
                   int S, int H, int Hkv, int hd, float *out) {
    oxo_attention_pv_blocked(q, kc, vc, n_tok, S, H, Hkv, hd, 0, out);
}

/* ------------------------------------------------------------------------ */
/* embedding / LM head / argmax                                              */
/* ------------------------------------------------------------------------ */
void oxo_embedding(const uint32_t *ids, int n_tok, const uint16_t *E, int V,
                   int D, float *out) {
    for (int t = 0; t < n_tok; t++)
        for (int d = 0; d < D; d++)
            out[(size_t)t * D + d] =
                ids[t] < (uint32_t)V ? oxo_f16_to_f32(E[(size_t)ids[t] * D + d])
                                     : 0.0f; /* sh/embedding.wgsl:38-45 */
}

void oxo_lm_head(const float *h, const uint16_t *E, int V, int D, float *logits) {
    int Dh = D / 2;
#pragma omp parallel for schedule(static)
    for (int v = 0; v < V; v++) {
        float p[WG];
        const uint16_t *e = E + (size_t)v * D;
        for (int tid = 0; tid < WG; tid++) { /* sh/f32_matmul.wgsl:51-57 */
            float acc = 0.0f;
            for (int dh = tid; dh < Dh; dh += WG) {
                int d = dh * 2; /* fused steps: see header */
                acc = fmaf(h[d], oxo_f16_to_f32(e[d]), acc);
                acc = fmaf(h[d + 1], oxo_f16_to_f32(e[d + 1]), acc);
            }
            p[tid] = acc;
        }
        logits[v] = tree_sum(p);
    }
}

int oxo_argmax(const float *x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

/* ------------------------------------------------------------------------ */
/* whole model                                                               */
/* ------------------------------------------------------------------------ */

static void probe(const oxo_model *m, int layer, int site, const void *data, size_t bytes) {
    if (m->probe) m->probe(m->probe_ud, layer, site, data, bytes);
}

/* rs/nn/bitlinear.rs:52-97: optional RMSNorm (eps hard-coded 1e-5, :112),
 * quantize, then GEMV for one token or GEMM for several.  site_q8 >= 0
 * reports the int8 input and its scales to the probe (sites site_q8 and
 * site_q8 + 1). */
static void bitlinear(const oxo_model *m, int layer, int site_q8, const float *in, int n,
                      int in_dim, int out_dim, const uint8_t *W, float wscale,
                      const float *norm_w, float *out) {
    float *normed = NULL;
    const float *src = in;
    if (norm_w) {
        normed = (float *)malloc(sizeof(float) * (size_t)n * in_dim);
        oxo_rmsnorm(in, norm_w, n, in_dim, 1e-5f, normed);
        src = normed;
    }
    int8_t *q = (int8_t *)malloc((size_t)n * in_dim);
    float *is = (float *)malloc(sizeof(float) * (size_t)n);
    float *ws = (float *)malloc(sizeof(float) * (size_t)out_dim);
    for (int r = 0; r < out_dim; r++) ws[r] = wscale; /* rs/model/loader.rs:131-136 */
    oxo_quantize(src, n, in_dim, q, is);
    if (site_q8 >= 0) {
        probe(m, layer, site_q8, q, (size_t)n * in_dim);
        probe(m, layer, site_q8 + 1, is, sizeof(float) * (size_t)n);
    }
    if (n == 1)
        oxo_gemv(W, q, ws, is[0], out_dim, in_dim, NULL, out);
    else
        oxo_gemm(W, q, ws, is, out_dim, n, in_dim, NULL, out);
    free(ws);
    free(is);
    free(q);
    free(normed);
}

int oxo_forward(oxo_model *m, const uint32_t *ids, int n, float *logits) {
    const int D = m->D, F = m->F, H = m->H, Hkv = m->Hkv;
    const int hd = D / H, kvd = Hkv * hd;
    if (m->seq_len + n > m->max_seq) return -1;
    size_t nD = (size_t)n * D;
    const size_t f4 = sizeof(float);
    float *x = (float *)malloc(f4 * nD);
    float *h = (float *)malloc(f4 * nD);
    float *q = (float *)malloc(f4 * (size_t)n * H * hd);
    float *k = (float *)malloc(f4 * (size_t)n * kvd);
    float *v = (float *)malloc(f4 * (size_t)n * kvd);
    float *qr = (float *)malloc(f4 * (size_t)n * H * hd);
    float *kr = (float *)malloc(f4 * (size_t)n * kvd);
    float *att = (float *)malloc(f4 * (size_t)n * H * hd);
    float *o = (float *)malloc(f4 * nD);
    float *g = (float *)malloc(f4 * (size_t)n * F);
    float *u = (float *)malloc(f4 * (size_t)n * F);

    oxo_embedding(ids, n, m->embed, m->V, D, x); /* rs/nn/model.rs:213 */
    for (int l = 0; l < m->n_layers; l++) {
        const oxo_layer *L = &m->layers[l];
        float *kc = m->kcache + (size_t)l * m->max_seq * kvd;
        float *vc = m->vcache + (size_t)l * m->max_seq * kvd;
        int pos = m->seq_len;
        probe(m, l, OXO_SITE_X_IN, x, f4 * nD);
        /* rs/nn/transformer.rs:51-75 */
        oxo_rmsnorm(x, L->attn_norm, n, D, m->eps, h);
        probe(m, l, OXO_SITE_ATTN_NORM, h, f4 * nD);
        /* rs/nn/attention.rs:98-100: q, k, v each quantize the same input */
        bitlinear(m, l, OXO_SITE_QKV_Q8, h, n, D, H * hd, L->wq, L->sq, NULL, q);
        bitlinear(m, l, -1, h, n, D, kvd, L->wk, L->sk, NULL, k);
        bitlinear(m, l, -1, h, n, D, kvd, L->wv, L->sv, NULL, v);
        oxo_rope(q, n, H, hd, pos, m->rope_theta, qr); /* :103-104 */
        oxo_rope(k, n, Hkv, hd, pos, m->rope_theta, kr);
        probe(m, l, OXO_SITE_Q, qr, f4 * (size_t)n * H * hd);
        probe(m, l, OXO_SITE_K, kr, f4 * (size_t)n * kvd);
        probe(m, l, OXO_SITE_V, v, f4 * (size_t)n * kvd);
        for (size_t i = 0; i < (size_t)n * kvd; i++) { /* append, :182-183 */
            float kv_k = kr[i], kv_v = v[i];
            if (m->kv_f16) {
                kv_k = oxo_f16_to_f32(oxo_f32_to_f16(kv_k));
                kv_v = oxo_f16_to_f32(oxo_f32_to_f16(kv_v));
            }
            kc[(size_t)pos * kvd + i] = kv_k;
            vc[(size_t)pos * kvd + i] = kv_v;
        }
        oxo_attention_pv_blocked(qr, kc, vc, n, pos + n, H, Hkv, hd, m->pv_block, att);
        probe(m, l, OXO_SITE_ATTN, att, f4 * (size_t)n * H * hd);
        bitlinear(m, l, OXO_SITE_O_Q8, att, n, H * hd, D, L->wo, L->so, L->attn_sub_norm, o);
        probe(m, l, OXO_SITE_O, o, f4 * nD);
        oxo_add(x, o, nD, x); /* residual1 */
        probe(m, l, OXO_SITE_X_MID, x, f4 * nD);
        oxo_rmsnorm(x, L->ffn_norm, n, D, m->eps, h);
        probe(m, l, OXO_SITE_FFN_NORM, h, f4 * nD);
        /* rs/nn/ffn.rs:60-80 */
        bitlinear(m, l, -1, h, n, D, F, L->wgate, L->sgate, NULL, g);
        bitlinear(m, l, -1, h, n, D, F, L->wup, L->sup, NULL, u);
        probe(m, l, OXO_SITE_GATE, g, f4 * (size_t)n * F);
        probe(m, l, OXO_SITE_UP, u, f4 * (size_t)n * F);
        oxo_relu2(g, (size_t)n * F, g);
        oxo_mul(g, u, (size_t)n * F, g);
        bitlinear(m, l, OXO_SITE_DOWN_Q8, g, n, F, D, L->wdown, L->sdown, L->ffn_sub_norm, o);
        probe(m, l, OXO_SITE_DOWN, o, f4 * nD);
        oxo_add(x, o, nD, x);
        probe(m, l, OXO_SITE_X_OUT, x, f4 * nD);
    }
    m->seq_len += n; /* rs/nn/model.rs:222 */
    oxo_rmsnorm(x, m->final_norm, n, D, m->eps, h);
    probe(m, -1, OXO_SITE_FINAL, h, f4 * nD);
    oxo_lm_head(h + (size_t)(n - 1) * D, m->embed, m->V, D, logits);

    free(x); free(h); free(q); free(k); free(v); free(qr); free(kr);
    free(att); free(o); free(g); free(u);
    return 0;
}

int oxo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oxo_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
