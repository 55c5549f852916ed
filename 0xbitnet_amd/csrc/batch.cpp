// Batched greedy decode: B independent sequences ("slots") advanced one
// token each per step, sharing one pass over the weights.  New relative to
// the reference (which decodes one sequence, rs/lib.rs:130-189); each slot's
// arithmetic is exactly that of a one-sequence decode step (the per-row
// norm/quantize, GEMV-order epilogues, per-slot attention and LM head
// rows), so its tokens and logits equal those of oxb_model_step.
//
// A slot owns its K/V caches ([L][Hkv][max_seq][hd] f16 each, slots
// contiguous), an 8-int state block (position, token, ... as the model's)
// and a token history.  A step is one hipGraph replay.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "model.h"
#include "oxb_common.h"
#include "oxb_kernels.h"

using namespace oxb;

#define B_CHECK(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                         \
            set_error("%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
            return -1;                                                                  \
        }                                                                               \
    } while (0)

struct oxb_batch {
    oxb_model *m = nullptr;
    int B = 0, max_seq = 0, hist_cap = 0;
    size_t layer_kv = 0, slot_kv = 0;     // elements: one layer of one slot, one slot
    size_t layer_kv8 = 0, slot_kv8 = 0;   // the same for the octet copy of V
    uint16_t *kcache = nullptr, *vcache = nullptr, *vcache8 = nullptr;
    int *state = nullptr;                 // [B][OXB_STATE_INTS]
    int *tok_hist = nullptr;              // [B][hist_cap]
    float *rope = nullptr;                // [max_seq][hd/2] (cos, sin)
    float *x = nullptr, *q = nullptr, *attn = nullptr, *h = nullptr;
    float *scores = nullptr, *logits = nullptr, *xscale = nullptr;
    float *hn = nullptr;                  // [B][D] LM-head pair tables (normalised rows)
    int *xsum = nullptr;
    void *X = nullptr;                    // token-tiled int8 rows
    int *pinned = nullptr;
    hipGraphExec_t graph = nullptr;
    std::vector<int> pos, ngen;           // host mirrors per slot
    std::vector<void *> allocs;

    ~oxb_batch() {   // teardown: errors have no caller to go to
        if (graph) (void)hipGraphExecDestroy(graph);
        for (void *p : allocs) (void)hipFree(p);
        if (pinned) (void)hipHostFree(pinned);
    }
    void *dalloc(size_t bytes) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            set_error("hipMalloc(%zu) failed", bytes);
            return nullptr;
        }
        allocs.push_back(p);
        return p;
    }
    int enqueue_step();
    int capture();
};

int oxb_batch::enqueue_step() {
    oxb_model &M = *m;
    void *s = (void *)M.stream;
    const int D = M.D, F = M.F, Dq = M.H * M.hd, Dkv = M.Hkv * M.hd;
    if (embedding_lm(M.embed_lm, M.V, D, state + OXB_ST_TOKEN, OXB_STATE_INTS, nullptr, B, x, s))
        return -1;
    for (int l = 0; l < M.n_layers; ++l) {
        const oxb_model::Layer &L = M.layers[l];
        uint16_t *kc = kcache + l * layer_kv, *vc = vcache + l * layer_kv;
        uint16_t *vc8 = vcache8 + l * layer_kv8;
        if (oxb_quantize_rows_tiled(x, L.attn_norm, M.eps, B, D, X, xscale, xsum, s)) return -1;
        if (gemm_qkv_rows(L.wqkv, (const int8_t *)X, xscale, xsum, L.sqkv, Dq, Dkv, M.hd, D, B,
                          state + OXB_ST_POS, OXB_STATE_INTS, slot_kv, q, kc, vc, max_seq, rope,
                          true, s, vc8, slot_kv8))
            return -1;
        if (oxb_attn_decode_batch_v8(q, kc, vc, vc8, state + OXB_ST_POS, OXB_STATE_INTS, slot_kv,
                                     slot_kv8, B, M.H, M.Hkv, M.hd, max_seq, scores, attn, s))
            return -1;
        // o_proj with attn_sub_norm (eps 1e-5 fixed, nn/bitlinear.rs:112) + residual
        if (oxb_quantize_rows_tiled(attn, L.attn_sub, 1e-5f, B, Dq, X, xscale, xsum, s)) return -1;
        if (gemm_rows(L.wo, (const int8_t *)X, xscale, xsum, L.so, D, Dq, B, x, 1, true, s))
            return -1;
        if (!M.relu2) {
            set_error("unsupported activation: SiLU gate (arch %s)", M.arch.c_str());
            return -1;
        }
        if (oxb_quantize_rows_tiled(x, L.ffn_norm, M.eps, B, D, X, xscale, xsum, s)) return -1;
        if (gemm_rows(L.wgu, (const int8_t *)X, xscale, xsum, L.sgu, 2 * F, D, B, h, 2, true, s))
            return -1;
        if (oxb_quantize_rows_tiled(h, L.ffn_sub, 1e-5f, B, F, X, xscale, xsum, s)) return -1;
        if (gemm_rows(L.wd, (const int8_t *)X, xscale, xsum, L.sd, D, F, B, x, 1, true, s))
            return -1;
    }
    return lm_head_argmax_rows(x, (size_t)D, M.final_norm, M.eps, M.embed_lm, M.V, D, logits,
                               state, OXB_STATE_INTS, tok_hist, hist_cap, B, 1, hn, s);
}

int oxb_batch::capture() {
    if (graph) return 0;
    hipGraph_t g = nullptr;
    B_CHECK(hipStreamSynchronize(m->stream));   // capture on an idle stream only
    B_CHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_step();
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return -1;
    }
    if (e != hipSuccess) {
        set_error("hipStreamEndCapture: %s", hipGetErrorString(e));
        return -1;
    }
    e = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        graph = nullptr;
        set_error("hipGraphInstantiate: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

extern "C" oxb_batch *oxb_batch_create(oxb_model *m, int batch, int max_seq) {
    clear_error();
    if (!m) {
        set_error("model is NULL");
        return nullptr;
    }
    if (m->kv_f32) {
        set_error("batched decode needs the f16 KV cache (model loaded with an f32 cache)");
        return nullptr;
    }
    if (batch < 1 || batch > 1024) {
        set_error("batch %d out of range (1..1024)", batch);
        return nullptr;
    }
    if (max_seq < 2) {
        set_error("max_seq %d too small", max_seq);
        return nullptr;
    }
    if ((size_t)(m->H / m->Hkv) * max_seq * 4 > 96 * 1024) {
        set_error("batch: %d positions exceed the attention LDS budget", max_seq);
        return nullptr;
    }
    oxb_batch *b = new oxb_batch;
    b->m = m;
    b->B = batch;
    b->max_seq = max_seq;
    b->hist_cap = max_seq + 16;
    b->layer_kv = (size_t)m->Hkv * max_seq * m->hd;
    b->slot_kv = b->layer_kv * m->n_layers;
    b->layer_kv8 = (size_t)m->Hkv * v8_head_elems(max_seq, m->hd);
    b->slot_kv8 = b->layer_kv8 * m->n_layers;
    const int D = m->D, F = m->F, Dq = m->H * m->hd;
    const int rows = (batch + 15) & ~15;
    const size_t pad = (size_t)OXB_KV_PAD_ROWS * m->hd;   // per-head attention reads whole V chunks
    b->kcache = (uint16_t *)b->dalloc((b->slot_kv * batch + pad) * 2);
    b->vcache = (uint16_t *)b->dalloc((b->slot_kv * batch + pad) * 2);
    b->vcache8 = (uint16_t *)b->dalloc(b->slot_kv8 * batch * 2);
    b->state = (int *)b->dalloc((size_t)batch * OXB_STATE_INTS * 4);
    b->tok_hist = (int *)b->dalloc((size_t)batch * b->hist_cap * 4);
    b->rope = (float *)b->dalloc((size_t)max_seq * m->hd * 4);
    b->x = (float *)b->dalloc((size_t)batch * D * 4);
    b->q = (float *)b->dalloc((size_t)batch * Dq * 4);
    b->attn = (float *)b->dalloc((size_t)batch * Dq * 4);
    b->h = (float *)b->dalloc((size_t)batch * F * 4);
    b->scores = (float *)b->dalloc((size_t)batch * m->H * max_seq * 4);
    b->logits = (float *)b->dalloc((size_t)batch * m->V * 4);
    b->hn = (float *)b->dalloc((size_t)batch * D * 4);
    b->xscale = (float *)b->dalloc((size_t)rows * 4);
    b->xsum = (int *)b->dalloc((size_t)rows * 4);
    b->X = b->dalloc((size_t)rows * std::max(D, F));
    bool ok = b->kcache && b->vcache && b->vcache8 && b->state && b->tok_hist && b->rope && b->x && b->q &&
              b->attn && b->h && b->scores && b->logits && b->hn && b->xscale &&
              b->xsum && b->X;
    if (ok && hipHostMalloc((void **)&b->pinned, (size_t)batch * OXB_STATE_INTS * 4,
                            hipHostMallocDefault) != hipSuccess) {
        set_error("hipHostMalloc failed");
        ok = false;
    }
    std::vector<float> cs((size_t)max_seq * m->hd);
    if (ok && oxb_rope_table(cs.data(), max_seq, m->hd, m->rope_theta)) ok = false;
    if (ok && hipMemcpy(b->rope, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        set_error("hipMemcpy (rope) failed");
        ok = false;
    }
    if (ok) {
        std::vector<int> st((size_t)batch * OXB_STATE_INTS, 0);
        for (int i = 0; i < batch; ++i) st[(size_t)i * OXB_STATE_INTS + OXB_ST_HIST_CAP] = b->hist_cap;
        if (hipMemcpy(b->state, st.data(), st.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            set_error("hipMemcpy (state) failed");
            ok = false;
        }
    }
    if (!ok) {
        delete b;
        return nullptr;
    }
    b->pos.assign(batch, 0);
    b->ngen.assign(batch, 0);
    return b;
}

extern "C" void oxb_batch_free(oxb_batch *b) {
    if (!b) return;
    (void)hipStreamSynchronize(b->m->stream);   // teardown: nothing to report to
    delete b;
}

extern "C" int oxb_batch_position(const oxb_batch *b, int slot) {
    if (!b || slot < 0 || slot >= b->B) return -1;
    return b->pos[slot];
}

extern "C" int oxb_batch_prefill(oxb_batch *b, int slot, const int32_t *ids, int n) {
    clear_error();
    OXB_REQUIRE(b && ids, "batch or ids is NULL");
    OXB_REQUIRE(slot >= 0 && slot < b->B, "slot %d out of range (batch %d)", slot, b->B);
    OXB_REQUIRE(n >= 2, "batch prefill needs >= 2 tokens (got %d)", n);
    OXB_REQUIRE(b->pos[slot] + n <= b->max_seq, "KV cache overflow: %d + %d > %d", b->pos[slot],
                n, b->max_seq);
    OXB_REQUIRE(b->ngen[slot] + 1 <= b->hist_cap, "token history full");
    oxb_model &M = *b->m;
    int *st = b->state + (size_t)slot * OXB_STATE_INTS;
    const oxb_model::SeqTarget tg{b->kcache + slot * b->slot_kv, b->vcache + slot * b->slot_kv,
                                  b->vcache8 + slot * b->slot_kv8, b->max_seq, b->rope, st,
                                  b->tok_hist + (size_t)slot * b->hist_cap, b->pos[slot]};
    if (M.enqueue_prefill_to(ids, n, tg)) return -1;
    B_CHECK(hipMemcpyAsync(b->pinned, st, OXB_STATE_INTS * 4, hipMemcpyDeviceToHost, M.stream));
    B_CHECK(hipStreamSynchronize(M.stream));
    b->pos[slot] += n;
    b->ngen[slot] += 1;
    return b->pinned[OXB_ST_TOKEN];
}

extern "C" int oxb_batch_decode_greedy(oxb_batch *b, int n_steps, int32_t *tokens_out) {
    clear_error();
    OXB_REQUIRE(b && tokens_out, "batch or output is NULL");
    OXB_REQUIRE(n_steps >= 0, "n_steps %d", n_steps);
    for (int i = 0; i < b->B; ++i) {
        OXB_REQUIRE(b->pos[i] >= 1, "slot %d has no prompt (prefill it first)", i);
        OXB_REQUIRE(b->pos[i] + n_steps <= b->max_seq, "slot %d: KV cache overflow: %d + %d > %d",
                    i, b->pos[i], n_steps, b->max_seq);
        OXB_REQUIRE(b->ngen[i] + n_steps <= b->hist_cap, "slot %d: token history full", i);
    }
    if (b->capture()) return -1;
    hipStream_t s = b->m->stream;
    for (int i = 0; i < n_steps; ++i)
        if (b->m->launch_replay(b->graph, i)) return -1;
    for (int i = 0; i < b->B && n_steps > 0; ++i)
        B_CHECK(hipMemcpyAsync(tokens_out + (size_t)i * n_steps,
                               b->tok_hist + (size_t)i * b->hist_cap + b->ngen[i],
                               (size_t)n_steps * 4, hipMemcpyDeviceToHost, s));
    B_CHECK(hipStreamSynchronize(s));
    for (int i = 0; i < b->B; ++i) {
        b->pos[i] += n_steps;
        b->ngen[i] += n_steps;
    }
    return 0;
}

extern "C" int oxb_batch_logits(const oxb_batch *b, float *logits_host) {
    clear_error();
    OXB_REQUIRE(b && logits_host, "batch or output is NULL");
    B_CHECK(hipMemcpy(logits_host, b->logits, (size_t)b->B * b->m->V * 4, hipMemcpyDeviceToHost));
    return 0;
}
