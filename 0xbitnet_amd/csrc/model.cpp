// Model engine: GGUF load -> device weights, decode step (hipGraph), prefill.
//
// Reference call structure this mirrors (packages/rust/crates/oxbitnet/src):
//   load:    model/loader.rs:75-173 (tensor walk, I2_S scale trailer,
//            F16 -> F32 norms, F16 embedding kept), :185-291 (names, config),
//            nn/model.rs:42-190 (layer assembly, tied head detection).
//   forward: nn/model.rs:193-266 -> nn/transformer.rs:51-75 ->
//            nn/attention.rs:85-124, nn/ffn.rs:60-80, nn/bitlinear.rs:52-97.
// Differences by design: q|k|v and gate|up are fused into one matrix each
// (one quantization of the shared input instead of three / two), weights are
// repacked to the tiled layout, the KV cache is f16, the decode step is one
// hipGraph whose kernels read the position from device memory, and the
// greedy token is reduced on the device.
#include "model.h"

#include <cstdlib>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>

#include "oxb_common.h"

using namespace oxb;

#define M_CHECK(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                         \
            set_error("%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
            return -1;                                                                  \
        }                                                                               \
    } while (0)

oxb_model::~oxb_model() {   // teardown: errors have no caller to go to
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto &row : graphs)
        for (hipGraphExec_t g : row)
            if (g) (void)hipGraphExecDestroy(g);
    for (hipEvent_t e : tok_ev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : replay_ev)
        if (e) (void)hipEventDestroy(e);
    for (void *p : allocations) (void)hipFree(p);
    if (pinned) (void)hipHostFree(pinned);
    if (stream) (void)hipStreamDestroy(stream);
    delete gguf;
}

void oxb_model::dfree(void *p) {
    for (size_t i = 0; i < allocations.size(); ++i)
        if (allocations[i] == p) {
            (void)hipFree(p);
            allocations[i] = allocations.back();
            allocations.pop_back();
            return;
        }
}

void *oxb_model::dalloc(size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) {
        set_error("hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    allocations.push_back(p);
    return p;
}

namespace {

// GGUF name of a tensor given its reference (HF) name: the inverse of
// remap_gguf_name (model/loader.rs:185-219).  Both spellings are accepted.
std::string gguf_layer_name(int i, const char *component) {
    return "blk." + std::to_string(i) + "." + component;
}

struct NameMap {
    const char *gguf;
    const char *hf;
};
const NameMap kLayerNames[] = {
    {"attn_q.weight", "self_attn.q_proj.weight"},
    {"attn_k.weight", "self_attn.k_proj.weight"},
    {"attn_v.weight", "self_attn.v_proj.weight"},
    {"attn_output.weight", "self_attn.o_proj.weight"},
    {"attn_norm.weight", "input_layernorm.weight"},
    {"ffn_norm.weight", "post_attention_layernorm.weight"},
    {"attn_sub_norm.weight", "self_attn.sub_norm.weight"},
    {"ffn_sub_norm.weight", "mlp.sub_norm.weight"},
    {"ffn_up.weight", "mlp.up_proj.weight"},
    {"ffn_down.weight", "mlp.down_proj.weight"},
    {"ffn_gate.weight", "mlp.gate_proj.weight"},
};

const GgufTensor *find_layer(const GgufFile &g, int i, const char *gguf_comp) {
    if (auto *t = g.find(gguf_layer_name(i, gguf_comp))) return t;
    for (auto &nm : kLayerNames)
        if (!strcmp(nm.gguf, gguf_comp))
            return g.find("model.layers." + std::to_string(i) + "." + nm.hf);
    return nullptr;
}

std::string hf_layer_name(int i, const char *gguf_comp) {
    for (auto &nm : kLayerNames)
        if (!strcmp(nm.gguf, gguf_comp))
            return "model.layers." + std::to_string(i) + "." + nm.hf;
    return gguf_layer_name(i, gguf_comp);
}

const GgufTensor *find_global(const GgufFile &g, const char *gguf_name, const char *hf_name) {
    if (auto *t = g.find(gguf_name)) return t;
    return g.find(hf_name);
}

float f16_to_f32_host(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int k = -1;
            do { m <<= 1; k++; } while (!(m & 0x400));
            bits = sign | ((uint32_t)(127 - 15 - k) << 23) | ((m & 0x3ff) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// Norm / small vectors: F32 as is, F16 converted (model/loader.rs:150-153).
bool tensor_to_f32(const GgufFile &g, const GgufTensor &t, std::vector<float> &out) {
    const uint8_t *src = g.base + g.data_offset + t.offset;
    const uint64_t n = t.n_elements();
    out.resize(n);
    if (t.type == GGML_F32) {
        memcpy(out.data(), src, n * 4);
        return true;
    }
    if (t.type == GGML_F16) {
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, src + 2 * i, 2);
            out[i] = f16_to_f32_host(h);
        }
        return true;
    }
    set_error("tensor %s: norm weights must be F32 or F16 (type %u)", t.name.c_str(), t.type);
    return false;
}

struct I2S {
    const uint8_t *rows;  // natural [N][K/4]
    int N, K;
    float scale;
};

bool get_i2s(const GgufFile &g, const GgufTensor *t, const std::string &hf, int K, int N, I2S &out) {
    if (!t) {
        set_error("Missing weight tensor: \"%s\"", hf.c_str());
        return false;
    }
    if (t->type != GGML_I2_S) {
        set_error("tensor %s: ternary linears must be I2_S (GGML type 36), got type %u",
                  t->name.c_str(), t->type);
        return false;
    }
    // GGUF shape is [in, out] (ne0 = K): model/loader.rs:131-133
    if (t->shape.size() < 2 || t->shape[0] != (uint64_t)K || t->shape[1] != (uint64_t)N) {
        set_error("tensor %s: shape [%llu, %llu] does not match [%d, %d]", t->name.c_str(),
                  (unsigned long long)(t->shape.size() > 0 ? t->shape[0] : 0),
                  (unsigned long long)(t->shape.size() > 1 ? t->shape[1] : 0), K, N);
        return false;
    }
    const uint8_t *p = g.base + g.data_offset + t->offset;
    const size_t packed = (t->n_elements() + 3) / 4;
    out.rows = p;
    out.N = N;
    out.K = K;
    memcpy(&out.scale, p + packed, 4);  // first f32 of the 32-byte trailer (:134-136)
    return true;
}

uint32_t meta_u32(const GgufFile &g, const std::string &arch, const char *suffix, uint32_t dflt,
                  bool *found = nullptr) {
    for (const std::string &pre : {arch, std::string("llama"), std::string("bitnet"),
                                   std::string("bitnet-25")}) {
        if (auto *v = g.get(pre + "." + suffix)) {
            if (v->is_int()) {
                if (found) *found = true;
                return (uint32_t)v->u;
            }
        }
    }
    if (found) *found = false;
    return dflt;
}

float meta_f32(const GgufFile &g, const std::string &arch, const char *suffix, float dflt) {
    for (const std::string &pre : {arch, std::string("llama"), std::string("bitnet"),
                                   std::string("bitnet-25")}) {
        if (auto *v = g.get(pre + "." + suffix))
            if (v->kind == GgufValue::F64) return (float)v->f;
    }
    return dflt;
}

}  // namespace

namespace oxb {

static void (*g_log_fn)(int, const char *, size_t, void *) = nullptr;
static void *g_log_ud = nullptr;
static int g_log_min = 2;

void set_log_sink(void (*fn)(int, const char *, size_t, void *), void *ud, int min_level) {
    g_log_fn = fn;
    g_log_ud = ud;
    g_log_min = min_level;
}

void log_msg(int level, const char *fmt, ...) {
    if (!g_log_fn || level < g_log_min) return;
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    int n = vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (n < 0) return;
    g_log_fn(level, buf, (size_t)(n < (int)sizeof buf ? n : (int)sizeof buf - 1), g_log_ud);
}

static int upload_f32(oxb_model *m, const std::vector<float> &v, float **dst) {
    *dst = (float *)m->dalloc(v.size() * 4);
    if (!*dst) return -1;
    M_CHECK(hipMemcpy(*dst, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return 0;
}

// Concatenate row blocks (natural I2_S) into one fused matrix, upload and
// repack it to the tiled layout.  interleave: rows alternate between the two
// parts (gate|up), else parts are stacked (q|k|v).
static int upload_fused(oxb_model *m, const std::vector<I2S> &parts, bool interleave,
                        void *staging, void **out, float **scales) {
    const int K = parts[0].K;
    const size_t rb = (size_t)K / 4;
    int N = 0;
    for (auto &p : parts) N += p.N;
    std::vector<uint8_t> host((size_t)N * rb);
    std::vector<float> sc(N);
    if (interleave) {
        for (int i = 0; i < parts[0].N; ++i)
            for (size_t j = 0; j < parts.size(); ++j) {
                const size_t row = (size_t)i * parts.size() + j;
                memcpy(host.data() + row * rb, parts[j].rows + (size_t)i * rb, rb);
                sc[row] = parts[j].scale;
            }
    } else {
        size_t row = 0;
        for (auto &p : parts) {
            memcpy(host.data() + row * rb, p.rows, (size_t)p.N * rb);
            for (int i = 0; i < p.N; ++i) sc[row + i] = p.scale;
            row += p.N;
        }
    }
    *out = m->dalloc(host.size());
    if (!*out) return -1;
    M_CHECK(hipMemcpy(staging, host.data(), host.size(), hipMemcpyHostToDevice));
    if (oxb_repack_i2s_tiled(staging, *out, N, K, nullptr)) return -1;
    M_CHECK(hipDeviceSynchronize());
    m->weight_bytes += host.size();
    return upload_f32(m, sc, scales);
}

oxb_model *model_load(const char *path, int max_seq, LoadHook hook, void *ud, int kv) {
    std::unique_ptr<oxb_model> m(new oxb_model());
    GgufFile *g = gguf_open(path);
    if (!g) return nullptr;
    m->gguf = g;

    // config_from_gguf_metadata (model/loader.rs:221-291)
    m->arch = "bitnet";
    if (auto *a = g->get("general.architecture"))
        if (a->kind == GgufValue::STR) m->arch = a->s;
    const std::string &arch = m->arch;
    const bool is_b25 = arch == "bitnet-25";
    m->D = (int)meta_u32(*g, arch, "embedding_length", 2560);
    m->n_layers = (int)meta_u32(*g, arch, "block_count", 30);
    m->H = (int)meta_u32(*g, arch, "attention.head_count", 20);
    m->Hkv = (int)meta_u32(*g, arch, "attention.head_count_kv", (uint32_t)m->H);
    bool vfound = false;
    m->V = (int)meta_u32(*g, arch, "vocab_size", 128256, &vfound);
    if (!vfound) {
        if (auto *t = g->get("tokenizer.ggml.tokens"))
            if (t->kind == GgufValue::ARR) m->V = (int)t->arr.size();
    }
    m->F = (int)meta_u32(*g, arch, "feed_forward_length", 6912);
    m->eps = meta_f32(*g, arch, "attention.layer_norm_rms_epsilon", 1e-5f);
    m->rope_theta = meta_f32(*g, arch, "rope.freq_base", is_b25 ? 500000.0f : 10000.0f);
    m->relu2 = is_b25;
    m->max_seq = max_seq > 0 ? max_seq : 4096;  // lib.rs:93
    // Metadata is untrusted: every count must be positive and fit the int
    // arithmetic below, and each layer needs at least nine tensors in the file
    // (seven ternary, two norms), which bounds block_count before anything is
    // sized by it.
    const uint32_t kMaxDim = 1u << 20;
    for (int v : {m->D, m->F, m->H, m->Hkv, m->V, m->n_layers}) {
        if (v <= 0 || (uint32_t)v > kMaxDim) {
            set_error("invalid model metadata: layers %d hidden %d ffn %d heads %d kv_heads %d vocab %d",
                      m->n_layers, m->D, m->F, m->H, m->Hkv, m->V);
            return nullptr;
        }
    }
    if ((size_t)m->n_layers * 9 > g->tensors.size()) {
        set_error("invalid model metadata: block_count %d but the file holds %zu tensors", m->n_layers,
                  g->tensors.size());
        return nullptr;
    }
    m->hd = m->D / m->H;
    const int D = m->D, F = m->F, H = m->H, Hkv = m->Hkv, hd = m->hd;
    const int Dq = H * hd, Dkv = Hkv * hd;
    log_msg(1, "config: arch=%s layers=%d hidden=%d ffn=%d heads=%d kv_heads=%d head_dim=%d vocab=%d",
            arch.c_str(), m->n_layers, m->D, m->F, m->H, m->Hkv, m->hd, m->V);
    if (hd != 128 || D % H != 0) {
        set_error("unsupported shape: head_dim %d (hidden %d / heads %d); the kernels need 128", hd, D, H);
        return nullptr;
    }
    if (D % 512 != 0 || F % 256 != 0 || (H % Hkv) != 0) {
        set_error("unsupported shape: hidden %d must be a multiple of 512, ffn %d of 256, heads %d of kv heads %d",
                  D, F, H, Hkv);
        return nullptr;
    }
    if (find_global(*g, "output.weight", "lm_head.weight")) {
        set_error("unsupported: untied LM head (output.weight); only the tied f16 head is implemented");
        return nullptr;
    }

    // Validate every tensor on the host before touching the device.
    struct LayerSrc {
        I2S q, k, v, o, gt, up, dn;
        const GgufTensor *norm[4];
    };
    static const char *kNormNames[4] = {"attn_norm.weight", "ffn_norm.weight",
                                        "attn_sub_norm.weight", "ffn_sub_norm.weight"};
    const int norm_dim[4] = {D, D, Dq, F};
    std::vector<LayerSrc> src(m->n_layers);
    for (int i = 0; i < m->n_layers; ++i) {
        LayerSrc &ls = src[i];
        if (!get_i2s(*g, find_layer(*g, i, "attn_q.weight"), hf_layer_name(i, "attn_q.weight"), D, Dq, ls.q) ||
            !get_i2s(*g, find_layer(*g, i, "attn_k.weight"), hf_layer_name(i, "attn_k.weight"), D, Dkv, ls.k) ||
            !get_i2s(*g, find_layer(*g, i, "attn_v.weight"), hf_layer_name(i, "attn_v.weight"), D, Dkv, ls.v) ||
            !get_i2s(*g, find_layer(*g, i, "attn_output.weight"), hf_layer_name(i, "attn_output.weight"), Dq, D, ls.o) ||
            !get_i2s(*g, find_layer(*g, i, "ffn_up.weight"), hf_layer_name(i, "ffn_up.weight"), D, F, ls.up) ||
            !get_i2s(*g, find_layer(*g, i, "ffn_down.weight"), hf_layer_name(i, "ffn_down.weight"), F, D, ls.dn) ||
            !get_i2s(*g, find_layer(*g, i, "ffn_gate.weight"), hf_layer_name(i, "ffn_gate.weight"), D, F, ls.gt))
            return nullptr;
        for (int k = 0; k < 4; ++k) {
            ls.norm[k] = find_layer(*g, i, kNormNames[k]);
            if (!ls.norm[k]) {
                if (k < 2) {
                    set_error("Missing weight tensor: \"%s\"", hf_layer_name(i, kNormNames[k]).c_str());
                    return nullptr;
                }
                continue;
            }
            if (ls.norm[k]->n_elements() != (uint64_t)norm_dim[k] ||
                (ls.norm[k]->type != GGML_F32 && ls.norm[k]->type != GGML_F16)) {
                set_error("tensor %s: expected %d F32/F16 elements", ls.norm[k]->name.c_str(), norm_dim[k]);
                return nullptr;
            }
        }
    }
    const GgufTensor *te = find_global(*g, "token_embd.weight", "model.embed_tokens.weight");
    if (!te) {
        set_error("Missing weight tensor: \"model.embed_tokens.weight\"");
        return nullptr;
    }
    if (te->type != GGML_F16 || te->n_elements() != (uint64_t)m->V * D) {
        set_error("token_embd.weight must be F16 [%d, %d]", D, m->V);
        return nullptr;
    }
    const GgufTensor *tn = find_global(*g, "output_norm.weight", "model.norm.weight");
    if (!tn) {
        set_error("Missing weight tensor: \"model.norm.weight\"");
        return nullptr;
    }

    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
        set_error("hipStreamCreate failed (no usable GPU?)");
        return nullptr;
    }
    if (hipHostMalloc((void **)&m->pinned, 64 * sizeof(int), hipHostMallocDefault) != hipSuccess) {
        set_error("hipHostMalloc failed");
        return nullptr;
    }
    for (hipEvent_t &e : m->replay_ev)
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            set_error("hipEventCreate failed");
            return nullptr;
        }
    for (hipEvent_t &e : m->tok_ev)
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            set_error("hipEventCreate failed");
            return nullptr;
        }

    const size_t staging_bytes = (size_t)std::max(Dq + 2 * Dkv, 2 * F) * std::max(D, F) / 4;
    void *staging = m->dalloc(staging_bytes);
    if (!staging) return nullptr;

    const uint64_t total = (uint64_t)m->n_layers + 2;
    m->layers.resize(m->n_layers);
    for (int i = 0; i < m->n_layers; ++i) {
        auto &L = m->layers[i];
        LayerSrc &ls = src[i];
        if (upload_fused(m.get(), {ls.q, ls.k, ls.v}, false, staging, &L.wqkv, &L.sqkv) ||
            upload_fused(m.get(), {ls.o}, false, staging, &L.wo, &L.so) ||
            upload_fused(m.get(), {ls.gt, ls.up}, true, staging, &L.wgu, &L.sgu) ||
            upload_fused(m.get(), {ls.dn}, false, staging, &L.wd, &L.sd))
            return nullptr;
        float **dst[4] = {&L.attn_norm, &L.ffn_norm, &L.attn_sub, &L.ffn_sub};
        for (int k = 0; k < 4; ++k) {
            if (!ls.norm[k]) continue;
            std::vector<float> w;
            if (!tensor_to_f32(*g, *ls.norm[k], w) || upload_f32(m.get(), w, dst[k])) return nullptr;
        }
        if (hook) hook(2, (uint64_t)i + 1, total, ud);
    }
    // embedding (kept f16, model/loader.rs:139-141) and final norm: the tied
    // table is kept once, in the LM head's layout (the embedding gathers its
    // rows from there); the natural copy is staging only
    {
        uint16_t *natural = (uint16_t *)m->dalloc((size_t)m->V * D * 2);
        if (!natural) return nullptr;
        if (hipMemcpy(natural, g->base + g->data_offset + te->offset, (size_t)m->V * D * 2,
                      hipMemcpyHostToDevice) != hipSuccess) {
            set_error("embedding upload failed");
            return nullptr;
        }
        m->embed_lm = m->dalloc(oxb_lm_bytes(m->V, D));
        if (!m->embed_lm || oxb_repack_lm(natural, m->embed_lm, m->V, D, nullptr)) return nullptr;
        if (hipDeviceSynchronize() != hipSuccess) {
            set_error("embedding repack failed");
            return nullptr;
        }
        m->dfree(natural);
        m->weight_bytes += oxb_lm_bytes(m->V, D);
    }
    {
        std::vector<float> w;
        if (!tensor_to_f32(*g, *tn, w) || upload_f32(m.get(), w, &m->final_norm)) return nullptr;
    }
    if (hook) hook(2, total, total, ud);

    {
        std::vector<float> cs((size_t)m->max_seq * (hd / 2) * 2);
        if (oxb_rope_table(cs.data(), m->max_seq, hd, m->rope_theta) ||
            upload_f32(m.get(), cs, &m->rope))
            return nullptr;
    }

    // KV cache and decode buffers (OXB_KV_PAD_ROWS rows of padding past the
    // last head: the per-head decode attention reads whole V chunks)
    if (kv < 0) {
        kv = 0;
        if (const char *env = getenv("OXB_KV")) {
            if (!strcmp(env, "f32")) kv = 1;
            else if (strcmp(env, "f16")) {
                set_error("OXB_KV=%s: expected f16 or f32", env);
                return nullptr;
            }
        }
    }
    m->kv_f32 = kv == 1;
    if (m->kv_f32 && m->max_seq > OXB_KV_F32_MAX_SEQ) {
        set_error("f32 KV cache: max_seq %d beyond %d", m->max_seq, OXB_KV_F32_MAX_SEQ);
        return nullptr;
    }
    const size_t kv_elems = (size_t)m->n_layers * Hkv * m->max_seq * hd + (size_t)OXB_KV_PAD_ROWS * hd;
    const size_t kv_bytes = kv_elems * m->kv_elem_bytes();
    m->kcache = m->dalloc(kv_bytes);
    m->vcache = m->dalloc(kv_bytes);
    const size_t kv8_bytes = m->kv_f32 ? 0 : (size_t)m->n_layers * Hkv * v8_head_elems(m->max_seq, hd) * 2;
    if (kv8_bytes) m->vcache8 = (uint16_t *)m->dalloc(kv8_bytes);
    m->x = (float *)m->dalloc((size_t)D * 4);
    m->q = (float *)m->dalloc((size_t)Dq * 4);
    m->attn = (float *)m->dalloc((size_t)Dq * 4);
    m->h = (float *)m->dalloc((size_t)F * 4);
    m->scores = (float *)m->dalloc((size_t)H * m->max_seq * 4);
    m->logits = (float *)m->dalloc((size_t)m->V * 4);
    m->state = (int *)m->dalloc(OXB_STATE_INTS * 4);
    m->hist_cap = m->max_seq + 16;
    // OXB_QKV_ATTN=1: steps of up to 256 positions run q|k|v + attention as
    // the one launch of oxb_qkv_attn_decode (same bits; slower on MI355X than
    // the two launches, its cross-workgroup hand-off costs more than a launch)
    const char *qa_env = getenv("OXB_QKV_ATTN");
    m->qkv_attn = qa_env && !strcmp(qa_env, "1") &&
                  oxb::qkv_attn_supported(D, H, Hkv, hd, m->max_seq) && m->vcache8;
    // its arrival counters: zero here, zero again after every launch
    if (m->qkv_attn) m->qa_cnt = (int *)m->dalloc((size_t)H * 4);
    if (const char *env = getenv("OXB_ATTN")) {
        if (!strcmp(env, "head")) m->attn_mode = 0;
        else if (!strcmp(env, "fused")) m->attn_mode = 1;
        else if (!strcmp(env, "split")) m->attn_mode = 2;
        else {
            set_error("OXB_ATTN=%s: expected head, fused or split", env);
            return nullptr;
        }
    }
    m->tok_hist = (int *)m->dalloc((size_t)m->hist_cap * 4);
    // the prefill attention's K / V copies, once, for the longest rows any
    // prefill of this model or a batch slot can hand the MFMA kernel
    m->pf_ws_bytes = oxb::attn_prefill_ws_max_bytes(Hkv);
    m->pf_ws = m->dalloc(m->pf_ws_bytes);
    m->samp_ctl = (oxb::SampleCtl *)m->dalloc(sizeof(oxb::SampleCtl));
    m->samp_u = (float *)m->dalloc((size_t)m->hist_cap * 4);
    m->samp_ws_bytes = oxb::sample_ws_bytes(m->V);
    m->samp_ws = m->dalloc(m->samp_ws_bytes);
    if (!m->kcache || !m->vcache || (kv8_bytes && !m->vcache8) || !m->x || !m->q || !m->attn ||
        !m->h || !m->scores ||
        !m->logits || !m->state || !m->tok_hist || !m->pf_ws || !m->samp_ctl || !m->samp_u ||
        !m->samp_ws || (m->qkv_attn && !m->qa_cnt))
        return nullptr;
    if ((m->qa_cnt && hipMemset(m->qa_cnt, 0, (size_t)H * 4) != hipSuccess) ||
        hipMemset(m->kcache, 0, kv_bytes) != hipSuccess ||
        hipMemset(m->vcache, 0, kv_bytes) != hipSuccess ||
        (kv8_bytes && hipMemset(m->vcache8, 0, kv8_bytes) != hipSuccess)) {
        set_error("hipMemset failed");
        return nullptr;
    }
    {
        int st[OXB_STATE_INTS] = {0};
        st[OXB_ST_HIST_CAP] = m->hist_cap;
        if (hipMemcpy(m->state, st, sizeof st, hipMemcpyHostToDevice) != hipSuccess) {
            set_error("state init failed");
            return nullptr;
        }
    }
    if (hipDeviceSynchronize() != hipSuccess) {
        set_error("load: device synchronize failed");
        return nullptr;
    }
    log_msg(2, "%d tensors loaded (%.1f MB of device weights)", (int)g->tensors.size(),
            m->weight_bytes / 1e6);
    return m.release();
}

}  // namespace oxb

// One decode step: embedding of state.token at state.pos -> layers -> LM
// head + argmax (state.token, state.pos += 1).  Every kernel reads the
// position from device memory, so the same launch sequence replays as a graph.
oxb_model::AttnForm oxb_model::attn_form(int S) const {
    if (kv_f32) return ATTN_SPLIT;   // one form (attn_f32) at every length
    if (attn_mode == 0 && S <= 256) return ATTN_HEAD1;
    if (attn_mode == 0 && S <= 512) return ATTN_HEAD2;
    if (attn_mode == 1 && S <= 256 && oxb_attn_decode_fused_supported(H, Hkv, hd, max_seq))
        return ATTN_FUSED;
    return ATTN_SPLIT;
}

int oxb_model::enqueue_sample() {
    return oxb::sample_enqueue(logits, V, samp_ctl, oxb::SampleCtl{}, tok_hist, 0, state,
                               tok_hist, samp_u, nullptr, samp_ws, samp_ws_bytes, stream);
}

int oxb_model::enqueue_decode_step(AttnForm attn, bool sample) {
    void *s = (void *)stream;
    const int Dq = H * hd, Dkv = Hkv * hd;
    int *posp = state + OXB_ST_POS;
    if (oxb::embedding_lm(embed_lm, V, D, nullptr, 0, state, 1, x, s)) return -1;
    const size_t kv_layer = (size_t)Hkv * max_seq * hd * kv_elem_bytes();
    for (int l = 0; l < n_layers; ++l) {
        const Layer &L = layers[l];
        void *kv_k = (char *)kcache + l * kv_layer, *kv_v = (char *)vcache + l * kv_layer;
        uint16_t *kc = (uint16_t *)kv_k, *vc = (uint16_t *)kv_v;
        uint16_t *vc8 = vcache8 ? vcache8 + l * (size_t)Hkv * v8_head_elems(max_seq, hd) : nullptr;
        int rc;
        if (attn == ATTN_HEAD1 && qkv_attn && vc8 && L.attn_norm) {
            // q|k|v BitLinear and the attention in one launch
            rc = oxb::qkv_attn_decode(L.wqkv, L.sqkv, x, L.attn_norm, eps, rope, posp, q, kc, vc,
                                      vc8, qa_cnt, H, Hkv, D, max_seq, this->attn, s);
        } else if (oxb::bitlinear_qkv(L.wqkv, x, L.attn_norm, eps, L.sqkv, Dq, Dkv, hd, D, q, kv_k,
                                      kv_v, kv_f32, max_seq, rope, posp, s, vc8)) {
            return -1;
        } else if (kv_f32)
            rc = oxb::attn_f32(q, (const float *)kv_k, (const float *)kv_v, posp, 0, 1, H, Hkv, hd,
                               max_seq, this->attn, s);
        else switch (attn) {
            case ATTN_HEAD1:
            case ATTN_HEAD2:
                rc = oxb_attn_decode_head_v8(q, kc, vc, vc8, posp, 0, 0, 0, 1, H, Hkv, hd,
                                             max_seq, attn == ATTN_HEAD1 ? 256 : 512, this->attn,
                                             s);
                break;
            case ATTN_FUSED:
                rc = oxb_attn_decode_fused(q, kc, vc, posp, H, Hkv, hd, max_seq, this->attn, s);
                break;
            default:
                rc = oxb_attn_decode_batch_v8(q, kc, vc, vc8, posp, 0, 0, 0, 1, H, Hkv, hd,
                                              max_seq, scores, this->attn, s);
        }
        if (rc) return -1;
        // o_proj with attn_sub_norm (eps 1e-5 fixed, nn/bitlinear.rs:112) + residual
        if (oxb_bitlinear_gemv(L.wo, this->attn, L.attn_sub, 1e-5f, L.so, D, Dq, x, 1, nullptr,
                               nullptr, nullptr, s))
            return -1;
        if (relu2) {
            if (oxb_bitlinear_gateup(L.wgu, x, L.ffn_norm, eps, L.sgu, 2 * F, D, h, s)) return -1;
        } else {
            set_error("unsupported activation: SiLU gate (arch %s)", arch.c_str());
            return -1;
        }
        if (oxb_bitlinear_gemv(L.wd, h, L.ffn_sub, 1e-5f, L.sd, D, F, x, 1, nullptr, nullptr,
                               nullptr, s))
            return -1;
    }
    if (oxb_lm_head_argmax(x, final_norm, eps, embed_lm, V, D, logits, state, tok_hist, 1, s))
        return -1;
    return sample ? enqueue_sample() : 0;
}

int oxb_model::capture_graph(AttnForm attn, bool sample) {
    hipGraphExec_t &slot = graphs[sample][attn];
    if (slot) return 0;
    hipGraph_t g = nullptr;
    // Capture only on an idle stream: no replay of another step graph may
    // still be queued when capture begins, and the kernels' first launches
    // (lazy code-object load, LDS attribute set-up) happen with nothing of
    // this handle in flight.
    M_CHECK(hipStreamSynchronize(stream));
    M_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_decode_step(attn, sample);
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return -1;
    }
    if (e != hipSuccess) {
        set_error("hipStreamEndCapture: %s", hipGetErrorString(e));
        return -1;
    }
    e = hipGraphInstantiate(&slot, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        slot = nullptr;
        set_error("hipGraphInstantiate: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

// Every graph a run of steps will replay is captured before the first of
// them is launched, so a run that crosses from one attention form to the
// next never captures while replays are queued.
int oxb_model::ensure_graphs(int p0, int p1) {
    for (int p = p0; p < p1;) {
        const AttnForm f = attn_form(p + 1);
        if (capture_graph(f, sampling)) return -1;
        while (p < p1 && attn_form(p + 1) == f) ++p;   // the run of positions with this form
    }
    return 0;
}

int oxb_model::ensure_prefill(int n) {
    if (n <= pf_cap) return 0;
    // the buffers of a shorter prefill: released once the work queued on them is done
    if (pf_cap) {
        M_CHECK(hipStreamSynchronize(stream));
        for (void *p : {(void *)px, (void *)pq, (void *)pattn, (void *)ph, (void *)pscale, pX,
                        (void *)psum, (void *)pids})
            dfree(p);
    }
    const int cap = ((n + 63) / 64) * 64;
    const int Dq = H * hd;
    const int Kmax = std::max(D, F);
    float *nx = (float *)dalloc((size_t)cap * D * 4);
    float *nq = (float *)dalloc((size_t)cap * Dq * 4);
    float *na = (float *)dalloc((size_t)cap * Dq * 4);
    float *nh = (float *)dalloc((size_t)cap * F * 4);
    float *ns = (float *)dalloc((size_t)cap * 4);
    void *nX = dalloc((size_t)cap * Kmax);
    int *nsum = (int *)dalloc((size_t)cap * 4);
    int *nids = (int *)dalloc((size_t)cap * 4);
    if (!nx || !nq || !na || !nh || !ns || !nX || !nsum || !nids) return -1;
    px = nx; pq = nq; pattn = na; ph = nh; pscale = ns; pX = nX; psum = nsum; pids = nids;
    pf_cap = cap;
    return 0;
}

// The workspace that lets the prefill's o_proj, gate|up and down GEMMs over n
// tokens run split over K where that pays (e.g. the 2560 x 6912 down
// projection over 65-384 tokens); zero-filled when it grows, and every GEMM
// call leaves its counters zero again.
int oxb_model::ensure_gemm_ws(int n) {
    const int Dq = H * hd;
    const size_t need = std::max({oxb_gemm_ws_bytes(D, Dq, n), oxb_gemm_ws_bytes(2 * F, D, n),
                                  oxb_gemm_ws_bytes(D, F, n)});
    if (need <= gemm_ws_bytes) return 0;
    if (gemm_ws) {   // released once the work queued on it is done
        M_CHECK(hipStreamSynchronize(stream));
        dfree(gemm_ws);
        gemm_ws = nullptr;
        gemm_ws_bytes = 0;
    }
    void *w = dalloc(need);
    if (!w) return -1;
    M_CHECK(hipMemsetAsync(w, 0, need, stream));
    gemm_ws = w;
    gemm_ws_bytes = need;
    return 0;
}

// Prefill n tokens (nn/model.rs:193-266 with n > 1): per-row norm+quantize,
// MFMA GEMMs with fused epilogues, causal attention, then the LM head on the
// last row (advance = n).  The target names the sequence's caches, RoPE
// table, state block and position (the model's own, or a batch slot's).
int oxb_model::enqueue_prefill_to(const int32_t *ids, int n, const SeqTarget &tg) {
    if (ensure_prefill(n) || ensure_gemm_ws(n)) return -1;
    void *s = (void *)stream;
    const int Dq = H * hd, Dkv = Hkv * hd;
    M_CHECK(hipMemcpyAsync(pids, ids, (size_t)n * 4, hipMemcpyHostToDevice, stream));
    if (oxb::embedding_lm(embed_lm, V, D, pids, 1, nullptr, n, px, s)) return -1;
    const size_t kv_layer = (size_t)Hkv * tg.max_seq * hd * kv_elem_bytes();
    for (int l = 0; l < n_layers; ++l) {
        const Layer &L = layers[l];
        void *kc = (char *)tg.kcache + l * kv_layer, *vc = (char *)tg.vcache + l * kv_layer;
        uint16_t *vc8 =
            tg.vcache8 ? tg.vcache8 + l * (size_t)Hkv * v8_head_elems(tg.max_seq, hd) : nullptr;
        if (oxb_quantize_rows_tiled(px, L.attn_norm, eps, n, D, pX, pscale, psum, s)) return -1;
        if (oxb::gemm_qkv(L.wqkv, (const int8_t *)pX, pscale, psum, L.sqkv, Dq, Dkv, hd, D, n,
                          tg.pos, pq, kc, vc, kv_f32, tg.max_seq, tg.rope, s, vc8))
            return -1;
        if (kv_f32 ? oxb::attn_f32(pq, (const float *)kc, (const float *)vc, nullptr, tg.pos, n, H,
                                   Hkv, hd, tg.max_seq, pattn, s)
                   : oxb::attn_prefill(pq, (const uint16_t *)kc, (const uint16_t *)vc, n, tg.pos,
                                       H, Hkv, hd, tg.max_seq, pf_ws, pf_ws_bytes, pattn, s))
            return -1;
        if (oxb_quantize_rows_tiled(pattn, L.attn_sub, 1e-5f, n, Dq, pX, pscale, psum, s)) return -1;
        if (oxb_gemm_i8_ws(L.wo, (const int8_t *)pX, pscale, psum, L.so, D, Dq, n, px, nullptr, 1,
                           gemm_ws, gemm_ws_bytes, s))
            return -1;
        if (oxb_quantize_rows_tiled(px, L.ffn_norm, eps, n, D, pX, pscale, psum, s)) return -1;
        if (!relu2) {
            set_error("unsupported activation: SiLU gate (arch %s)", arch.c_str());
            return -1;
        }
        if (oxb_gemm_i8_ws(L.wgu, (const int8_t *)pX, pscale, psum, L.sgu, 2 * F, D, n, ph, nullptr,
                           2, gemm_ws, gemm_ws_bytes, s))
            return -1;
        if (oxb_quantize_rows_tiled(ph, L.ffn_sub, 1e-5f, n, F, pX, pscale, psum, s)) return -1;
        if (oxb_gemm_i8_ws(L.wd, (const int8_t *)pX, pscale, psum, L.sd, D, F, n, px, nullptr, 1,
                           gemm_ws, gemm_ws_bytes, s))
            return -1;
    }
    return oxb_lm_head_argmax(px + (size_t)(n - 1) * D, final_norm, eps, embed_lm, V, D, logits,
                              tg.state, tg.tok_hist, n, s);
}

int oxb_model::enqueue_prefill(const int32_t *ids, int n) {
    return enqueue_prefill_to(ids, n,
                              SeqTarget{kcache, vcache, vcache8, max_seq, rope, state, tok_hist, pos});
}

// ---------------------------------------------------------------------------
// extern "C" model API (include/oxbitnet_ops.h)
// ---------------------------------------------------------------------------
// RoPE table, computed exactly as shaders/rope.wgsl:43-48 evaluates it:
// theta = f32(pos) * pow(base, (-2 * i) / hd), then cos/sin in f32.
extern "C" int oxb_rope_table(float *cs, int max_seq, int hd, float theta_base) {
    OXB_REQUIRE(cs && max_seq > 0 && hd > 0 && hd % 2 == 0, "rope_table: bad arguments");
    const int half = hd / 2;
    for (int p = 0; p < max_seq; ++p)
        for (int i = 0; i < half; ++i) {
            float fe = -2.0f * (float)i;
            fe = fe / (float)hd;
            const float th = (float)p * powf(theta_base, fe);
            cs[((size_t)p * half + i) * 2] = cosf(th);
            cs[((size_t)p * half + i) * 2 + 1] = sinf(th);
        }
    return 0;
}

extern "C" oxb_model *oxb_model_load(const char *path, int max_seq) {
    clear_error();
    if (!path) {
        set_error("source is NULL");
        return nullptr;
    }
    return model_load(path, max_seq, nullptr, nullptr);
}

extern "C" oxb_model *oxb_model_load_kv(const char *path, int max_seq, int kv_f32) {
    clear_error();
    if (!path) {
        set_error("source is NULL");
        return nullptr;
    }
    if (kv_f32 != 0 && kv_f32 != 1) {
        set_error("kv_f32 must be 0 or 1 (got %d)", kv_f32);
        return nullptr;
    }
    return model_load(path, max_seq, nullptr, nullptr, kv_f32);
}

extern "C" void oxb_model_free(oxb_model *m) { delete m; }

extern "C" int oxb_model_get_info(const oxb_model *m, oxb_model_info *o) {
    OXB_REQUIRE(m && o, "model is NULL");
    o->n_layers = m->n_layers;
    o->hidden = m->D;
    o->ffn = m->F;
    o->heads = m->H;
    o->kv_heads = m->Hkv;
    o->head_dim = m->hd;
    o->vocab = m->V;
    o->max_seq = m->max_seq;
    o->rms_eps = m->eps;
    o->rope_theta = m->rope_theta;
    o->relu2 = m->relu2 ? 1 : 0;
    o->weight_bytes = m->weight_bytes;
    o->kv_f32 = m->kv_f32 ? 1 : 0;
    return 0;
}

static int write_state(oxb_model *m) {
    int *st = m->pinned;
    st[OXB_ST_POS] = m->pos;
    st[OXB_ST_TOKEN] = m->pinned[OXB_ST_TOKEN];
    st[OXB_ST_NGEN] = m->ngen;
    st[OXB_ST_LM_COUNTER] = 0;
    st[OXB_ST_HIST_CAP] = m->hist_cap;
    st[5] = 0;
    st[OXB_ST_LM_KEY] = st[OXB_ST_LM_KEY + 1] = 0;
    M_CHECK(hipMemcpyAsync(m->state, st, OXB_STATE_INTS * 4, hipMemcpyHostToDevice, m->stream));
    M_CHECK(hipStreamSynchronize(m->stream));
    return 0;
}

extern "C" int oxb_model_reset(oxb_model *m) {
    OXB_REQUIRE(m, "model is NULL");
    m->tok_issued = m->tok_read = 0;   // write_state waits for every queued step
    m->pos = 0;
    m->ngen = 0;
    m->pinned[OXB_ST_TOKEN] = 0;
    return write_state(m);
}

extern "C" int oxb_model_position(const oxb_model *m) { return m ? m->pos : -1; }

extern "C" int oxb_model_set_token(oxb_model *m, int32_t tok) {
    OXB_REQUIRE(m, "model is NULL");
    m->pinned[8] = tok;
    M_CHECK(hipMemcpyAsync(m->state + OXB_ST_TOKEN, m->pinned + 8, 4, hipMemcpyHostToDevice,
                           m->stream));
    M_CHECK(hipStreamSynchronize(m->stream));
    return 0;
}

static int read_token(oxb_model *m, float *logits_host) {
    M_CHECK(hipMemcpyAsync(m->pinned + 16, m->state, OXB_STATE_INTS * 4, hipMemcpyDeviceToHost,
                           m->stream));
    if (logits_host)
        M_CHECK(hipMemcpyAsync(logits_host, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost,
                               m->stream));
    M_CHECK(hipStreamSynchronize(m->stream));
    return m->pinned[16 + OXB_ST_TOKEN];
}

extern "C" int oxb_model_step(oxb_model *m, float *logits_host) {
    clear_error();
    OXB_REQUIRE(m, "model is NULL");
    OXB_REQUIRE(m->pos + 1 <= m->max_seq, "KV cache full: position %d of %d", m->pos, m->max_seq);
    if (m->ensure_graphs(m->pos, m->pos + 1)) return -1;
    hipGraphExec_t ge = m->step_graph(m->pos);
    M_CHECK(hipGraphLaunch(ge, m->stream));
    m->pos += 1;
    m->ngen += 1;
    return read_token(m, logits_host);
}

extern "C" int oxb_model_forward(oxb_model *m, const int32_t *ids, int n, float *logits_host) {
    clear_error();
    OXB_REQUIRE(m && ids, "model or ids is NULL");
    OXB_REQUIRE(n > 0, "forward: empty input");
    OXB_REQUIRE(m->pos + n <= m->max_seq, "KV cache overflow: %d + %d > %d", m->pos, n, m->max_seq);
    if (n == 1) {
        if (oxb_model_set_token(m, ids[0])) return -1;
        return oxb_model_step(m, logits_host);
    }
    if (m->enqueue_prefill(ids, n)) return -1;
    if (m->sampling && m->enqueue_sample()) return -1;
    m->pos += n;
    m->ngen += 1;
    return read_token(m, logits_host);
}

extern "C" int oxb_model_set_sampling(oxb_model *m, float temperature, size_t top_k,
                                      float repeat_penalty, size_t repeat_last_n, const float *u,
                                      int n_u) {
    clear_error();
    OXB_REQUIRE(m, "model is NULL");
    if (!u) {
        m->sampling = false;
        return 0;
    }
    OXB_REQUIRE(n_u >= 0 && n_u <= m->hist_cap, "sampling: %d draws (at most %d)", n_u,
                m->hist_cap);
    oxb::SampleCtl c{temperature, (top_k > 0 && top_k < (size_t)m->V) ? (int)top_k : 0,
                     repeat_penalty,
                     repeat_last_n > (size_t)0x7fffffff ? 0x7fffffff : (int)repeat_last_n};
    // the kernels of queued steps may still read the old options and draws
    M_CHECK(hipStreamSynchronize(m->stream));
    M_CHECK(hipMemcpy(m->samp_ctl, &c, sizeof c, hipMemcpyHostToDevice));
    if (n_u) M_CHECK(hipMemcpy(m->samp_u, u, (size_t)n_u * 4, hipMemcpyHostToDevice));
    m->sampling = true;
    return 0;
}

int oxb_model::launch_replay(hipGraphExec_t g, int i) {
    const int grp = i / kReplayGroup;
    if (i % kReplayGroup == 0 && grp >= 2) M_CHECK(hipEventSynchronize(replay_ev[(grp - 2) % 3]));
    M_CHECK(hipGraphLaunch(g, stream));
    if (i % kReplayGroup == kReplayGroup - 1) M_CHECK(hipEventRecord(replay_ev[grp % 3], stream));
    return 0;
}

int oxb_model::step_async() {
    OXB_REQUIRE(tok_issued - tok_read < 2, "two steps already queued");
    OXB_REQUIRE(pos + 1 <= max_seq, "KV cache full: position %d of %d", pos, max_seq);
    if (ensure_graphs(pos, pos + 1)) return -1;
    M_CHECK(hipGraphLaunch(step_graph(pos), stream));
    const int k = tok_issued & 1;
    M_CHECK(hipMemcpyAsync(pinned + kTokSlot + k, state + OXB_ST_TOKEN, 4, hipMemcpyDeviceToHost,
                           stream));
    M_CHECK(hipEventRecord(tok_ev[k], stream));
    ++tok_issued;
    pos += 1;
    ngen += 1;
    return 0;
}

int oxb_model::step_wait() {
    OXB_REQUIRE(tok_read < tok_issued, "no step queued");
    const int k = tok_read & 1;
    M_CHECK(hipEventSynchronize(tok_ev[k]));
    ++tok_read;
    return pinned[kTokSlot + k];
}

extern "C" int oxb_model_decode_greedy(oxb_model *m, int n_steps, int32_t *tokens_out) {
    clear_error();
    OXB_REQUIRE(m && tokens_out, "model or output is NULL");
    OXB_REQUIRE(n_steps >= 0, "n_steps %d", n_steps);
    OXB_REQUIRE(m->pos + n_steps <= m->max_seq, "KV cache overflow: %d + %d > %d", m->pos,
                n_steps, m->max_seq);
    OXB_REQUIRE(m->ngen + n_steps <= m->hist_cap, "token history full");
    const int first = m->ngen;
    if (m->ensure_graphs(m->pos, m->pos + n_steps)) return -1;
    for (int i = 0; i < n_steps; ++i)
        if (m->launch_replay(m->step_graph(m->pos + i), i)) return -1;
    m->pos += n_steps;
    m->ngen += n_steps;
    if (n_steps)
        M_CHECK(hipMemcpyAsync(tokens_out, m->tok_hist + first, (size_t)n_steps * 4,
                               hipMemcpyDeviceToHost, m->stream));
    M_CHECK(hipStreamSynchronize(m->stream));
    return 0;
}
