// Internal include: the public hot-path ABI plus shared launch helpers.
#pragma once
#include "../../include/oxbitnet_ops.h"

extern "C" int oxb_quantize_rows_tiled(const float *x, const float *gamma, float eps, int n_tok,
                                       int D, void *Xt, float *scales, int *sums, void *stream);

#include <stddef.h>
#include <stdint.h>

namespace oxb {
// Batched-decode helpers (rows are independent single-token steps).
int gemm_rows(const void *W, const int8_t *X, const float *xscale, const int *xsum,
              const float *wscale, int N, int K, int n_tok, float *Y, int epilogue,
              bool gemv_order, void *stream);
int gemm_qkv_rows(const void *W, const int8_t *X, const float *xscale, const int *xsum,
                  const float *wscale, int Dq, int Dkv, int hd, int K, int n_tok,
                  const int *tok_pos, int tok_pos_stride, size_t kv_tok_stride, float *q_out,
                  uint16_t *kcache, uint16_t *vcache, int max_seq, const float *rope_cs,
                  bool gemv_order, void *stream, uint16_t *vcache8 = nullptr,
                  size_t kv8_tok_stride = 0);
// QKV projections that store K/V as f16 bits or, with kv_f32, as f32 (the
// reference's cache type): one token (GEMV, ternary_gemv.hip) or a prefill
// block (GEMM, ternary_gemm.hip).
// vcache8 (optional, f16 cache only): V also written in position octets
// (v8_index), the layout of the long-context decode P.V (attn_decode_v8).
int bitlinear_qkv(const void *W_tiled, const float *x, const float *gamma, float eps,
                  const float *wscale, int Dq, int Dkv, int hd, int K, float *q_out, void *kcache,
                  void *vcache, bool kv_f32, int max_seq, const float *rope_cs, const int *pos,
                  void *stream, uint16_t *vcache8 = nullptr);
int gemm_qkv(const void *W_tiled, const int8_t *X, const float *xscale, const int *xsum,
             const float *wscale, int Dq, int Dkv, int hd, int K, int n_tok, int pos0,
             float *q_out, void *kcache, void *vcache, bool kv_f32, int max_seq,
             const float *rope_cs, void *stream, uint16_t *vcache8 = nullptr);
// Attention over an f32 cache ([Hkv][max_seq][hd]): n_q queries at positions
// pos0 + i, or one query at *pos_ptr when pos_ptr is given (attention.hip).
// Causal prefill attention (oxb_attn_prefill) with the caller's workspace for
// the f32-MFMA kernel's K / V copies: attn_prefill_ws_bytes(Hkv, pos0 + n_q)
// bytes (0: that length runs on the VALU kernel, which needs none).  A
// smaller or null workspace selects the VALU kernel; the results are the same.
size_t attn_prefill_ws_bytes(int Hkv, int s_max);
// the largest such workspace (rows of up to the MFMA kernel's 2368 positions)
size_t attn_prefill_ws_max_bytes(int Hkv);
int attn_prefill(const float *q, const uint16_t *kc, const uint16_t *vc, int n_q, int pos0, int H,
                 int Hkv, int hd, int max_seq, void *ws, size_t ws_bytes, float *out,
                 void *stream);
int attn_f32(const float *q, const float *kcache, const float *vcache, const int *pos_ptr,
             int pos0, int n_q, int H, int Hkv, int hd, int max_seq, float *out, void *stream);
// The token embedding from the LM head's lm-tiled copy of the tied table
// (oxb_repack_lm's layout): rows ids[t * ids_stride], or the decode state's
// token when ids is null (lm_head.hip).
int embedding_lm(const void *E_lm, int V, int D, const int *ids, int ids_stride, const int *state,
                 int n_tok, float *x, void *stream);
// Batched LM head with a workspace of n_rows * D floats (lm_head.hip).
int lm_head_argmax_rows(const float *x, size_t x_stride, const float *gamma, float eps,
                        const void *E, int V, int D, float *logits, int *state, int state_stride,
                        int *tok_hist, int hist_stride, int n_rows, int advance, float *hn,
                        void *stream);
// The fused decode q|k|v BitLinear + attention (attention.hip,
// oxb_qkv_attn_decode) and the shapes it takes.
bool qkv_attn_supported(int D, int H, int Hkv, int hd, int max_seq);
int qkv_attn_decode(const void *W, const float *wscale, const float *x, const float *gamma,
                    float eps, const float *rope, const int *pos, float *q_out, uint16_t *kcache,
                    uint16_t *vcache, uint16_t *vcache8, int *counters, int H, int Hkv, int D,
                    int max_seq, float *out, void *stream);
// Device sampling (sampling.hip).  SampleCtl holds the options of one
// generation; top_k is the one in effect (0: keep all, else 0 < top_k < V).
struct SampleCtl {
    float temperature;
    int top_k;
    float penalty;
    int last_n;   // window: the last last_n tokens before the current one, 0: all
};
size_t sample_ws_bytes(int V);
// Draws one token from logits[V].  The options come from *ctl_dev when it is
// given (read when the kernels run), else from ctl.  With state: the window
// is win[...] (the token history) from state NGEN and last_n, the draw is
// u[NGEN - 1], and the token goes to state TOKEN and win[NGEN - 1] (hist);
// without: window win[0..nwin), draw u[0], token to *out.
int sample_enqueue(const float *logits, int V, const SampleCtl *ctl_dev, SampleCtl ctl,
                   const int *win, int nwin, int *state, int *hist, const float *u, int *out,
                   void *ws, size_t ws_bytes, void *stream);
}  // namespace oxb
