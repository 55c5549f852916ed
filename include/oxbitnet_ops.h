/*
 * oxbitnet_ops.h — MI355X (gfx950) hot-path entry points of liboxbitnet.
 *
 * Plain C ABI: device pointers, sizes and an opaque stream (a hipStream_t
 * passed as void*, NULL = the default stream).  Every function returns 0 on
 * success and -1 on failure, with the message available from
 * oxb_last_error() on the calling thread.  Shapes the kernels do not support
 * are rejected before launch.
 *
 * Each entry cites the reference routine it replaces (paths relative to
 * packages/rust/crates/oxbitnet/src/ in m96-chan/0xBitNet; sh/ = shaders/).
 *
 * Data formats
 *   I2_S natural:  [N][K/4] bytes, 128-element blocks of 32 bytes, element
 *                  b*128 + g*32 + j at bits (7-2g):(6-2g) of byte b*32 + j,
 *                  code = w + 1 (model/loader.rs:124-137, shaders/ternary_gemv.wgsl:3-10).
 *   I2_S tiled:    the same bytes regrouped into 16-row tiles of 16-byte
 *                  chunks, chunk-major inside a tile (produced once at load
 *                  by oxb_repack_i2s_tiled; consumed by the GEMV/GEMM).
 *   KV cache:      [Hkv][max_seq][128] f16 per layer (the reference keeps
 *                  [max_seq][Hkv][hd] f32, nn/attention.rs:23-48).
 *   decode state:  int32[8] on the device, indices below.
 */
#ifndef OXBITNET_OPS_H
#define OXBITNET_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OXB_ST_POS 0         /* next position (== KV length before the step) */
#define OXB_ST_TOKEN 1       /* current token id (greedy argmax output)      */
#define OXB_ST_NGEN 2        /* LM-head invocations since reset              */
#define OXB_ST_LM_COUNTER 3  /* reserved (kept zero)                         */
#define OXB_ST_HIST_CAP 4    /* capacity of the token history buffer         */
#define OXB_ST_LM_KEY 6      /* internal: ints 6-7, LM-head argmax key (u64) */
#define OXB_STATE_INTS 8

/* Rows (of 128 f16) a cache allocation must extend past its last head's
 * max_seq rows for oxb_attn_decode_head, which reads V in whole 64-row
 * chunks from any chunk start below the cache length. */
#define OXB_KV_PAD_ROWS 64
/* Longest cache of the f32-KV mode (oxb_model_load_kv): its attention holds
 * a score and a probability row per query in LDS. */
#define OXB_KV_F32_MAX_SEQ 16384

/* ---- errors, device memory, streams, events (plumbing) ----------------- */
const char *oxb_last_error(void);
void *oxb_device_malloc(size_t bytes);
int oxb_device_free(void *p);
int oxb_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int oxb_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int oxb_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
int oxb_memset_d(void *dst, int value, size_t bytes, void *stream);
void *oxb_stream_create(void);
int oxb_stream_destroy(void *stream);
int oxb_stream_sync(void *stream);
int oxb_device_sync(void);
void *oxb_event_create(void);
int oxb_event_destroy(void *ev);
int oxb_event_record(void *ev, void *stream);
int oxb_event_sync(void *ev);
float oxb_event_elapsed_ms(void *start, void *stop);
/* Stream capture: replay a fixed launch sequence as one graph (no host cost per
 * launch).  end_capture returns the executable graph, NULL on error.  No
 * counterpart in the reference (wgpu submits command buffers instead). */
int oxb_stream_begin_capture(void *stream);
void *oxb_stream_end_capture(void *stream);
int oxb_graph_launch(void *graph, void *stream);
int oxb_graph_destroy(void *graph);
/* name (NUL-terminated, truncated to len), CU count, peak clock kHz, HBM bytes */
int oxb_device_info(char *name, int len, int *cus, int *clock_khz, size_t *hbm_bytes);

/* ---- load-time layout ---------------------------------------------------- */
/* Natural I2_S [N][K/4] -> tiled layout.  N % 16 == 0, K % 128 == 0.
 * Replaces the raw upload of model/weights.rs:23-69 (no repack there). */
int oxb_repack_i2s_tiled(const void *natural, void *tiled, int N, int K, void *stream);

/* ---- ternary GEMV (decode, one token) ----------------------------------- */
/* y[n] = ((float)acc[n] * wscale[n]) * xscale[0], acc = sum_k w[n][k]*xq[k]
 * exactly in int32; xsum[0] = sum_k xq[k].  acc_out optional.
 * Replaces shaders/ternary_gemv.wgsl:39-97 dispatched by
 * nn/bitlinear.rs:161-205. */
int oxb_gemv_i8(const void *W_tiled, const int8_t *xq, const float *xscale, const int *xsum,
                const float *wscale, int N, int K, float *y, int32_t *acc_out, void *stream);

/* BitLinear for one token: optional RMSNorm (gamma may be NULL) -> absmax int8
 * quantize -> ternary GEMV; residual != 0 adds into y (y += out).
 * acc_out / xq_out / xscale_out optional (for parity checks).
 * Replaces nn/bitlinear.rs:52-97 (n == 1) plus the residual add of
 * nn/transformer.rs:157 / shaders/elementwise.wgsl. */
int oxb_bitlinear_gemv(const void *W_tiled, const float *x, const float *gamma, float eps,
                       const float *wscale, int N, int K, float *y, int residual,
                       int32_t *acc_out, int8_t *xq_out, float *xscale_out, void *stream);

/* Fused gate|up BitLinear (rows interleaved gate0, up0, gate1, up1, ...):
 * h[i] = relu(gate_i)^2 * up_i.  Replaces nn/ffn.rs:60-80 (two BitLinears +
 * shaders/activation.wgsl + shaders/elementwise.wgsl). */
int oxb_bitlinear_gateup(const void *W_tiled, const float *x, const float *gamma, float eps,
                         const float *wscale, int N2, int K, float *h, void *stream);

/* Fused q|k|v BitLinear + RoPE on q and k + f16 KV append at *pos.
 * Replaces nn/attention.rs:97-107,127-184 (three BitLinears, two RoPE
 * dispatches, two cache copies).  rope_cs: [max_seq][hd/2] (cos, sin) f32. */
int oxb_bitlinear_qkv(const void *W_tiled, const float *x, const float *gamma, float eps,
                      const float *wscale, int Dq, int Dkv, int hd, int K, float *q_out,
                      uint16_t *kcache, uint16_t *vcache, int max_seq, const float *rope_cs,
                      const int *pos, void *stream);

/* Host-side RoPE table [max_seq][hd/2] of (cos, sin) f32 with
 * theta = f32(pos) * pow(base, (-2*i) / hd), as shaders/rope.wgsl:43-48
 * computes it per element (built once at load instead of per dispatch). */
int oxb_rope_table(float *cs_host, int max_seq, int hd, float theta_base);

/* ---- prefill ------------------------------------------------------------- */
/* Per-row optional RMSNorm + absmax int8 quantize of [n_rows][D] f32:
 * xq int8, scales f32 [n_rows], sums int32 [n_rows] (sum of q, may be NULL).
 * Replaces shaders/rmsnorm.wgsl + shaders/quantize.wgsl (nn/bitlinear.rs:60-82). */
int oxb_norm_quant_rows(const float *x, const float *gamma, float eps, int n_rows, int D,
                        int8_t *xq, float *scales, int *sums, void *stream);

/* Ternary GEMM on int8 MFMA: Y[t][n] = (float)acc[t][n] * (wscale[n] * xscale[t]).
 * X is the token-tiled int8 layout written by oxb_quantize_rows_tiled:
 * [ceil16(n_tok)/16][K/256][4 planes][4 chunks][16 tokens][16 B], the 16 B of
 * (plane g, chunk kc = 4*stage + c, token) holding x[(kc/2)*128 + g*32 +
 * (kc%2)*16 + 0..15] (N multiple of 32, K of 256).
 * epilogue: 0 store, 1 residual add (Y += ...), 2 gate|up fusion (Y is
 * [n_tok][N/2]), 3 q|k|v + RoPE + KV append (qkv_* arguments used).
 * Replaces shaders/ternary_gemm.wgsl:40-136 dispatched by nn/bitlinear.rs:207-247. */
int oxb_gemm_i8(const void *W_tiled, const int8_t *X, const float *xscale, const int *xsum,
                const float *wscale, int N, int K, int n_tok, float *Y, int32_t *acc_out,
                int epilogue, void *stream);
/* The same GEMM with a workspace, which lets long-K shapes run split over K:
 * more than 64 tokens whose 64 x 64 or 256 x 128 output tiles leave CUs idle
 * (e.g. a 2560 x 6912 down projection over 65-384 prompt tokens), and up to
 * 64 tokens with K >= 8192, where the split gives each workgroup wider
 * feature groups and so fewer re-reads of the activations.  Each tile's (or
 * feature group's) K stages are cut into equal pieces, one workgroup each;
 * the last piece to finish adds the others' int32 partial sums, so the
 * result bits are the same.
 * oxb_gemm_ws_bytes gives the workspace a shape needs (0: the shape runs
 * unsplit, and ws may be NULL); with a smaller or NULL workspace the call runs
 * as oxb_gemm_i8.  The workspace starts with a fixed 16 KB area of arrival
 * counters, which must be zero before its first use (a zero-filled
 * allocation); every call leaves them zero, so one workspace of the largest
 * size needed serves calls of any shapes in turn.  Calls that share a
 * workspace must not run concurrently.  No counterpart in the reference
 * (nn/bitlinear.rs:207-247 dispatches one workgroup per tile). */
size_t oxb_gemm_ws_bytes(int N, int K, int n_tok);
int oxb_gemm_i8_ws(const void *W_tiled, const int8_t *X, const float *xscale, const int *xsum,
                   const float *wscale, int N, int K, int n_tok, float *Y, int32_t *acc_out,
                   int epilogue, void *ws, size_t ws_bytes, void *stream);
int oxb_gemm_qkv(const void *W_tiled, const int8_t *X, const float *xscale, const int *xsum,
                 const float *wscale, int Dq, int Dkv, int hd, int K, int n_tok, int pos0,
                 float *q_out, uint16_t *kcache, uint16_t *vcache, int max_seq,
                 const float *rope_cs, void *stream);

/* ---- attention ------------------------------------------------------------ */
/* Decode attention for one token over L = *pos + 1 cached positions, in the
 * reference's order: scores as 128-term chains in order of d, the softmax in
 * the shader's 256-thread order, and P.V as one chain per output over all L
 * positions in order (sh/attention.wgsl:29-59,79-105, sh/softmax.wgsl:25-80;
 * f32 result identical to the oracle's arithmetic on the f16-rounded cache).
 * Two launches: scores to the buffer, then softmax and P.V.  q, out: [H*128]
 * f32; scores: [H][max_seq] f32 scratch; max_seq <= 6144.  Replaces
 * nn/attention.rs:109-118 (scores, softmax, P.V dispatches). */
int oxb_attn_decode(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                    const int *pos, int H, int Hkv, int hd, int max_seq, float *scores,
                    float *out, void *stream);

/* Decode attention for a batch of independent sequences: sequence z uses
 * q + z*H*128, caches kcache/vcache + z*kv_stride, position pos[z*pos_stride],
 * scores + z*H*max_seq and out + z*H*128; each as oxb_attn_decode. */
int oxb_attn_decode_batch(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                          const int *pos, int pos_stride, size_t kv_stride, int batch, int H,
                          int Hkv, int hd, int max_seq, float *scores, float *out, void *stream);

/* The same, with the V cache also held in position octets (vcache8, a copy
 * the q|k|v projections keep beside the row-major cache in the model): per
 * KV head of a sequence round8(max_seq) x 128 f16, element (position s, dim
 * d) at ((s / 8) * 128 + d) * 8 + s % 8; sequence z's copy at vcache8 +
 * z*kv8_stride.  One 16-byte read gives a P.V chain its dim's next 8
 * positions (the row-major rows hold them 256 bytes apart), for batches of
 * up to 8; larger batches read vcache.  Same result bits.  No counterpart in
 * the reference (its cache is [max_seq][Hkv][hd] f32, nn/attention.rs:23-48). */
int oxb_attn_decode_batch_v8(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                             const uint16_t *vcache8, const int *pos, int pos_stride,
                             size_t kv_stride, size_t kv8_stride, int batch, int H, int Hkv,
                             int hd, int max_seq, float *scores, float *out, void *stream);

/* The same decode attention as one kernel: two 1024-thread workgroups per KV
 * head (one per half of the dims) compute scores, softmax and P.V in LDS (no
 * scores buffer), same result bits.  Faster for short caches (each KV head's
 * scores run on two CUs); H/Hkv <= 4 and the LDS of
 * oxb_attn_decode_fused_supported. */
int oxb_attn_decode_fused_supported(int H, int Hkv, int hd, int max_seq);
int oxb_attn_decode_fused(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                          const int *pos, int H, int Hkv, int hd, int max_seq, float *out,
                          void *stream);

/* The same decode attention in one launch, one workgroup per query head and
 * sequence (grid H x batch), for caches of up to s_max <= 512 positions.
 * Built for latency: every K and V row is loaded before the position is
 * known (clamped to the cache), each thread scores one position with q read
 * from LDS, the softmax runs in the shader's order and waves 0 and 1 run the
 * P.V chains (even and odd dims); same result bits as oxb_attn_decode.  Three
 * kernels: s_max <= 256 with max_seq >= 256 (256 threads), s_max <= 256 with
 * max_seq < 256 (256 threads; reads V in 64-row chunks past the position, so
 * that cache allocation must extend OXB_KV_PAD_ROWS rows past its last head),
 * and s_max <= 512 (512 threads).  Sequence z: q + z*H*128, caches +
 * z*kv_stride, pos[z*pos_stride], out + z*H*128.  Replaces
 * nn/attention.rs:109-118 like oxb_attn_decode; no counterpart of its own in
 * the reference. */
int oxb_attn_decode_head(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                         const int *pos, int pos_stride, size_t kv_stride, int batch, int H,
                         int Hkv, int hd, int max_seq, int s_max, float *out, void *stream);
/* The same with the octet copy of V (as oxb_attn_decode_batch_v8): the
 * 256-position kernel stages the copy's first 32 octets and sums 8 positions
 * per 16-byte read (waves 0 and 1: dims 0-63 and 64-127); the other two
 * kernels read vcache.  Same result bits.  No counterpart in the reference. */
int oxb_attn_decode_head_v8(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                            const uint16_t *vcache8, const int *pos, int pos_stride,
                            size_t kv_stride, size_t kv8_stride, int batch, int H, int Hkv,
                            int hd, int max_seq, int s_max, float *out, void *stream);

/* A decode step's q|k|v BitLinear (as oxb_bitlinear_qkv: attn_norm RMSNorm,
 * int8 quantize, ternary GEMV, RoPE, q to q_out, f16 K/V append at *pos, the
 * V octet copy too) and its attention (as oxb_attn_decode_head_v8 with s_max
 * 256) in one launch.  The workgroups are the GEMV's 16-row tiles; each counts
 * itself on counters[h] for the query heads its rows feed, and the one that
 * completes a head (24 tiles) computes that head's attention, having loaded
 * its K rows and V octets while it ran its tile when it is the head's
 * designated last q tile.  x, gamma: [D] f32 (D 512 or 2560); rope_cs as
 * oxb_bitlinear_qkv; q_out [H*128] f32; caches [Hkv][max_seq][128] f16
 * (max_seq >= 256) and the octet copy; counters [H] ints, zero before the
 * first call and zero again after each call completes (calls on one counter
 * array must not overlap); out [H*128] f32.  Same q, cache contents and
 * result bits as the two calls for *pos < 256; a position from 256 to
 * max_seq - 1 is appended to the caches and out is left as it was.  Replaces
 * nn/attention.rs:97-118 (projections, RoPE, cache copies, attention) for one
 * token; no single counterpart in the reference. */
int oxb_qkv_attn_decode(const void *W_tiled, const float *wscale, const float *x,
                        const float *gamma, float eps, const float *rope_cs, const int *pos,
                        float *q_out, uint16_t *kcache, uint16_t *vcache, uint16_t *vcache8,
                        int *counters, int H, int Hkv, int hd, int D, int max_seq, float *out,
                        void *stream);

/* oxb_attn_decode without the scores buffer and without allocating: the
 * scores live in a static device array of the library (one per device, 1 MiB:
 * H * max_seq <= 262144; larger shapes are rejected), whose address is looked
 * up on the first call on each device.  Same kernels and result bits as
 * oxb_attn_decode.  Calls that overlap on one device share the array and
 * race.  No counterpart in the reference: for callers that cannot allocate
 * device memory (code under hipGraph capture, allocation-free serving loops). */
int oxb_attn_decode_noalloc(const float *q, const uint16_t *kcache, const uint16_t *vcache,
                            const int *pos, int H, int Hkv, int hd, int max_seq, float *out,
                            void *stream);

/* Causal prefill attention for n_tok queries at positions pos0.., same order.
 * q, out: [n_tok][H*128] f32.  Replaces the same three dispatches for n > 1. */
int oxb_attn_prefill(const float *q, const uint16_t *kcache, const uint16_t *vcache, int n_tok,
                     int pos0, int H, int Hkv, int hd, int max_seq, float *out, void *stream);

/* ---- sampling ---------------------------------------------------------------- */
/* One draw of rs/sampling.rs:4-80 over logits[V] (modified in place):
 * repetition penalty over recent[n_recent] (positive logits divided, others
 * multiplied, once per occurrence), temperature (logits * 1/T when T != 1),
 * top-k (values below the k-th largest become -inf; k == 0 or >= V keeps all),
 * softmax, then the first index whose running sum reaches u * sum for the
 * uniform draw u in [0, 1) (V - 1 if none does).  exp is the library's
 * fixed exp (Cody-Waite + degree-7 polynomial, ~1 ulp; the reference's Rust
 * f32::exp is the platform libm's), so the device sampler gives the same
 * token.  The C ABI's generate passes u from its own generator to the device
 * sampler; top_k == 1 without a penalty is the LM head's argmax.
 * Host code, no GPU. */
int32_t oxb_sample_logits(float *logits, size_t V, float temperature, size_t top_k,
                          float repeat_penalty, const int32_t *recent, size_t n_recent, float u);

/* The same draw on the device (sampling.hip): logits[V], recent[n_recent],
 * u (one float) and token (one int) are device pointers; ws is a device
 * workspace of oxb_sample_ws_bytes(V) bytes.  Gives oxb_sample_logits's token
 * for the same logits and u (exp is oxb_expf on both sides) and leaves the
 * logits unchanged.  Replaces the host readback + sample_token of
 * rs/lib.rs:151-167 per generated token. */
size_t oxb_sample_ws_bytes(int V);
int oxb_sample_device(const float *logits, int V, float temperature, size_t top_k,
                      float repeat_penalty, const int32_t *recent, int n_recent, const float *u,
                      int32_t *token, void *ws, size_t ws_bytes, void *stream);

/* ---- tokenizer (host) ------------------------------------------------------- */
/* The tokenizer of a GGUF file from its metadata alone (no weights, no GPU):
 * byte-level BPE over tokenizer.ggml.tokens / .merges as the reference builds
 * it with HF tokenizers, the chat templates and the stop ids.  Replaces
 * rs/tokenizer.rs:22-216 (from_gguf_metadata, encode, decode_one,
 * apply_chat_template).  NULL / -1 on error (oxb_last_error). */
typedef struct oxb_tokenizer oxb_tokenizer;
oxb_tokenizer *oxb_tokenizer_load(const char *path);
void oxb_tokenizer_free(oxb_tokenizer *t);
/* The ids of text (BOS first when add_bos): writes min(count, cap) ids and
 * returns count. */
int oxb_tokenizer_encode(const oxb_tokenizer *t, const char *text, int add_bos, int32_t *ids,
                         int cap);
/* One token as text (UTF-8; invalid byte sequences replaced by U+FFFD):
 * writes at most cap - 1 bytes and a NUL, returns the full length. */
int oxb_tokenizer_decode_one(const oxb_tokenizer *t, int32_t id, char *buf, int cap);
/* apply_chat_template over n messages: writes min(count, cap) ids, returns count. */
int oxb_tokenizer_chat(const oxb_tokenizer *t, const char *const *roles,
                       const char *const *contents, int n, int32_t *ids, int cap);
/* out[0..4] = bos, eos, eot (-1 if absent), im_end (-1 if absent), vocabulary size. */
int oxb_tokenizer_info(const oxb_tokenizer *t, int32_t *out);

/* ---- embedding / LM head --------------------------------------------------- */
/* x[t] = E[ids[t]] (f16 -> f32; out-of-range ids give zeros); ids == NULL reads
 * the decode state's token.  Replaces nn/model.rs:312-352. */
int oxb_embedding(const uint16_t *E, int V, int D, const int *ids, int n_tok, const int *state,
                  float *x, void *stream);

/* Tied embedding [V][D] f16 -> the LM head's row-per-lane layout (64-row
 * tiles, each row's f16 pairs in the order the shader's reduction consumes
 * them).  E_lm holds oxb_lm_bytes(V, D) bytes.  D % 512 == 0, D <= 2560. */
int oxb_repack_lm(const uint16_t *E, void *E_lm, int V, int D, void *stream);
size_t oxb_lm_bytes(int V, int D);

/* Final RMSNorm of x -> tied f16 LM head (E_lm from oxb_repack_lm) -> logits [V]
 * (bit-identical to sh/f32_matmul.wgsl's reduction order) -> greedy argmax
 * (lowest index on ties) written to state[OXB_ST_TOKEN], appended to
 * tok_hist (if state[OXB_ST_HIST_CAP] allows), state[OXB_ST_POS] += advance.
 * state is 8-byte aligned with OXB_ST_LM_COUNTER and OXB_ST_LM_KEY zero
 * (the call leaves them zero; two launches: the head, whose blocks meet in an
 * atomic max on OXB_ST_LM_KEY, then a one-block finish that publishes the
 * token).  Replaces nn/model.rs:226-262,
 * 393-448 plus read_logits (:269-298) and sampling.rs with top_k = 1. */
int oxb_lm_head_argmax(const float *x, const float *gamma, float eps, const void *E_lm, int V,
                       int D, float *logits, int *state, int *tok_hist, int advance,
                       void *stream);
/* The same for n_rows independent rows (x rows x_stride floats apart; row r
 * uses the state block state + r*state_stride and history tok_hist +
 * r*hist_stride; logits [n_rows][V]).  Rows share each pass over the table
 * (4 per pass); each row's logits and token are those of the one-row call. */
int oxb_lm_head_argmax_batch(const float *x, size_t x_stride, const float *gamma, float eps,
                             const void *E_lm, int V, int D, float *logits, int *state,
                             int state_stride, int *tok_hist, int hist_stride, int n_rows,
                             int advance, void *stream);

/* ---- model (ids level) ------------------------------------------------------
 * The ids-level seam the parity and benchmark harnesses drive: the
 * reference's generate_from_ids is private (lib.rs:130) and stops on EOS. */
typedef struct oxb_model oxb_model;

typedef struct oxb_model_info {
    int n_layers, hidden, ffn, heads, kv_heads, head_dim, vocab, max_seq;
    float rms_eps, rope_theta;
    int relu2;           /* 1: ReLU^2 gate (arch "bitnet-25"), 0: SiLU */
    size_t weight_bytes; /* device bytes held by weights */
    int kv_f32;          /* 1: f32 KV cache, 0: f16 */
} oxb_model_info;

/* Parse a GGUF (v2/v3) file, upload and repack.  max_seq <= 0 means 4096
 * (lib.rs:93).  Replaces BitNet::load's model half (lib.rs:77-94,
 * model/loader.rs:75-173, nn/model.rs:42-190). */
oxb_model *oxb_model_load(const char *path, int max_seq);
/* The same with the KV cache type chosen: kv_f32 = 0 stores K/V as f16 (the
 * throughput mode, also oxb_model_load's and oxbitnet_load's default), 1 as
 * f32, the reference's own cache type (nn/attention.rs:23-48: f32 K/V
 * buffers), with which every result is the reference arithmetic's; max_seq
 * <= OXB_KV_F32_MAX_SEQ there, batches (oxb_batch_*) need the f16 cache.
 * oxb_model_load and oxbitnet_load take the type from OXB_KV=f16|f32. */
oxb_model *oxb_model_load_kv(const char *path, int max_seq, int kv_f32);
void oxb_model_free(oxb_model *m);
int oxb_model_get_info(const oxb_model *m, oxb_model_info *out);
/* KV length back to 0 (nn/model.rs:300-310). */
int oxb_model_reset(oxb_model *m);
/* forward(ids): prefill n >= 1 tokens at the current position; writes the
 * last token's logits to logits_host (nullable) and returns the greedy
 * token (the sampled one when oxb_model_set_sampling is on; >= 0) or -1.
 * nn/model.rs:193-298. */
int oxb_model_forward(oxb_model *m, const int32_t *ids, int n, float *logits_host);
/* n_steps greedy decode steps from the current token, each one replay of a
 * captured hipGraph; tokens_out[n_steps] (host).  Returns 0 / -1.  With
 * oxb_model_set_sampling on, each step's token is sampled instead. */
int oxb_model_decode_greedy(oxb_model *m, int n_steps, int32_t *tokens_out);
/* Current KV length. */
int oxb_model_position(const oxb_model *m);
/* Overwrite the current token (host sampling between decode steps). */
int oxb_model_set_token(oxb_model *m, int32_t tok);
/* One decode step from the current token, logits to host (nullable). */
int oxb_model_step(oxb_model *m, float *logits_host);
/* Sampling on the device for the following forwards and steps: after each
 * LM head the token is drawn from the logits as oxb_sample_device does
 * (penalty over the last repeat_last_n tokens of the history since reset,
 * 0: all of them), with u[i] as the draw of the i-th token since reset
 * (n_u <= max_seq + 16), and becomes the current token and history entry.
 * u == NULL turns it off (the LM head's argmax is the token).  The logits
 * (oxb_model_forward / oxb_model_step) stay the model's.  0 / -1. */
int oxb_model_set_sampling(oxb_model *m, float temperature, size_t top_k, float repeat_penalty,
                           size_t repeat_last_n, const float *u, int n_u);

/* ---- batched greedy decode (no counterpart in the reference) --------------
 * B independent sequences (slots) on one loaded model, each with its own KV
 * cache of max_seq positions; a step advances every slot by one token in one
 * hipGraph replay.  Each slot's tokens and logits equal those of the
 * one-sequence engine (oxb_model_forward / oxb_model_step) on its prompt. */
typedef struct oxb_batch oxb_batch;
oxb_batch *oxb_batch_create(oxb_model *m, int batch, int max_seq);
void oxb_batch_free(oxb_batch *b);
/* Prefill n >= 2 prompt tokens into a slot (appended at its position);
 * returns the slot's greedy next token, -1 on error. */
int oxb_batch_prefill(oxb_batch *b, int slot, const int32_t *ids, int n);
/* n_steps greedy steps for all slots; tokens_out [batch][n_steps] (host). */
int oxb_batch_decode_greedy(oxb_batch *b, int n_steps, int32_t *tokens_out);
int oxb_batch_position(const oxb_batch *b, int slot);
/* Logits of the last decode step, [batch][V] (host). */
int oxb_batch_logits(const oxb_batch *b, float *logits_host);

#ifdef __cplusplus
}
#endif
#endif
