// Model engine (host side): owns the device weights, caches and the decode
// hipGraph.  Reference: nn/model.rs:42-310, model/loader.rs:75-349.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "gguf.h"
#include "oxb_kernels.h"

struct oxb_model {
    // configuration (model/config.rs:3-48, model/loader.rs:221-291)
    std::string arch;
    int n_layers = 0, D = 0, F = 0, H = 0, Hkv = 0, hd = 0, V = 0, max_seq = 0;
    float eps = 1e-5f, rope_theta = 10000.0f;
    bool relu2 = true;
    size_t weight_bytes = 0;

    struct Layer {
        void *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;  // tiled I2_S
        float *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sd = nullptr; // per-row scales
        float *attn_norm = nullptr, *ffn_norm = nullptr;
        float *attn_sub = nullptr, *ffn_sub = nullptr;  // may be null
    };
    std::vector<Layer> layers;
    void *embed_lm = nullptr;    // the tied f16 table [V][D], in the LM head's layout
    float *final_norm = nullptr;
    float *rope = nullptr;       // [max_seq][hd/2] (cos, sin)
    // [L][Hkv][max_seq][hd]: f16 bits, or f32 when kv_f32 (the reference's
    // cache type, nn/attention.rs:23-48; a parity mode of the engine)
    void *kcache = nullptr, *vcache = nullptr;
    // f16 cache: V again in position octets (v8_index), per layer
    // [Hkv][round8(max_seq) x hd]: the long-context decode P.V reads it
    uint16_t *vcache8 = nullptr;
    bool kv_f32 = false;
    size_t kv_elem_bytes() const { return kv_f32 ? 4 : 2; }

    // decode buffers
    float *x = nullptr, *q = nullptr, *attn = nullptr, *h = nullptr, *scores = nullptr;
    float *logits = nullptr;
    int *state = nullptr, *tok_hist = nullptr;
    int hist_cap = 0;

    // prefill buffers (grown on demand)
    int pf_cap = 0;
    void *pf_ws = nullptr;   // prefill attention's K / V copies (sized at load)
    size_t pf_ws_bytes = 0;
    // the prefill GEMMs' split-K workspace (grown to the largest need met so
    // far; its arrival counters are zero between calls)
    void *gemm_ws = nullptr;
    size_t gemm_ws_bytes = 0;
    float *px = nullptr, *pq = nullptr, *pattn = nullptr, *ph = nullptr, *pscale = nullptr;
    void *pX = nullptr;
    int *psum = nullptr, *pids = nullptr;

    hipStream_t stream = nullptr;
    // Decode attention forms, chosen per step by the cache length S (the
    // position + 1); each has its own step graph.
    //   ATTN_HEAD1 / ATTN_HEAD2: one workgroup per query head, S <= 256 / 512
    //   ATTN_FUSED: two workgroups per KV head, S <= 256
    //   ATTN_SPLIT: scores kernel + P.V kernel, any S
    enum AttnForm { ATTN_HEAD1 = 0, ATTN_HEAD2, ATTN_FUSED, ATTN_SPLIT, ATTN_FORMS };
    // step graphs by [sampling on][attention form]
    hipGraphExec_t graphs[2][ATTN_FORMS] = {};
    // which forms the model uses: 0 per-head kernels up to 512 positions
    // (default), 1 the fused kernel up to 256, 2 the split kernels only
    // (OXB_ATTN=head|fused|split when the model loads; all give the same bits)
    int attn_mode = 0;
    bool qkv_attn = false;   // ATTN_HEAD1 steps as one q|k|v + attention launch
    int *qa_cnt = nullptr;   // its per-head arrival counters [H]
    AttnForm attn_form(int S) const;
    int *pinned = nullptr;      // host-pinned scratch for small readbacks
    int pos = 0;                // host mirror of state[OXB_ST_POS]
    int ngen = 0;               // host mirror of state[OXB_ST_NGEN]

    // device sampling (oxb_model_set_sampling): options and draws in device
    // memory, read by the sampler kernels of every forward and step graph
    bool sampling = false;
    oxb::SampleCtl *samp_ctl = nullptr;   // device
    float *samp_u = nullptr;              // device [hist_cap] draws by token index
    void *samp_ws = nullptr;
    size_t samp_ws_bytes = 0;
    // steps queued ahead of the host (step_async / step_wait): each one's
    // token is copied to pinned[kTokSlot + i % 2] and marked by tok_ev[i % 2]
    static constexpr int kTokSlot = 32;
    hipEvent_t tok_ev[2] = {};
    int tok_issued = 0, tok_read = 0;
    // A run of graph replays (decode_greedy, batch decode) keeps at most
    // 2 * kReplayGroup of them queued: an event marks the end of every group
    // of kReplayGroup, and group g waits for group g - 2 before it is queued.
    static constexpr int kReplayGroup = 4;
    hipEvent_t replay_ev[3] = {};
    int launch_replay(hipGraphExec_t g, int i);   // i: the replay's index in its run

    std::vector<void *> allocations;
    oxb::GgufFile *gguf = nullptr;  // kept for the tokenizer metadata

    ~oxb_model();
    void *dalloc(size_t bytes);
    void dfree(void *p);   // a dalloc allocation no queued work uses any more
    int enqueue_decode_step(AttnForm attn, bool sample);
    int enqueue_sample();   // the sampler over logits (state, history, draws)
    int ensure_prefill(int n);
    int ensure_gemm_ws(int n);
    // one sequence's caches ([L][Hkv][max_seq][hd] each), RoPE table, state
    // block, token history and position
    struct SeqTarget {
        void *kcache, *vcache;   // element type as the model's (kv_f32)
        uint16_t *vcache8;       // the octet copy of V (f16 cache), or null
        int max_seq;
        const float *rope;
        int *state, *tok_hist;
        int pos;
    };
    int enqueue_prefill_to(const int32_t *ids, int n, const SeqTarget &t);
    int enqueue_prefill(const int32_t *ids, int n);
    int capture_graph(AttnForm attn, bool sample);
    // capture the graphs of every step at positions [p0, p1) (on an idle
    // stream, before any of them is replayed)
    int ensure_graphs(int p0, int p1);
    // the graph for a step whose token sits at position p (after ensure_graphs)
    hipGraphExec_t step_graph(int p) const { return graphs[sampling][attn_form(p + 1)]; }
    // One step queued behind the ones already queued (graphs captured by
    // ensure_graphs beforehand), its token read back later by step_wait, at
    // most two ahead.  step_wait returns the oldest queued step's token.
    int step_async();
    int step_wait();
};

namespace oxb {
// Load progress hook used by the C ABI (phase 2 = upload, per tensor).
typedef void (*LoadHook)(int phase, uint64_t loaded, uint64_t total, void *ud);
// kv: 0 f16 cache, 1 f32 cache, -1 from the environment (OXB_KV=f16|f32,
// default f16)
oxb_model *model_load(const char *path, int max_seq, LoadHook hook, void *ud, int kv = -1);
void log_msg(int level, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace oxb
