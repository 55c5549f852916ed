"""The oracle's model composition (oxo_forward) pinned on the CPU.

The kernel-level functions of the oracle are pinned in test_oracle.py; this
file pins how oxo_forward composes them (rs/nn/model.rs:193-266,
rs/nn/transformer.rs:51-75, rs/nn/attention.rs:85-124, rs/nn/ffn.rs:60-80,
rs/nn/bitlinear.rs:52-97) with checks that the mathematics fixes, read
through the oracle's probe sites (OXO_SITE_*):

- all-zero ternary weights make every block the identity, so the logits are
  lm_head(rmsnorm(embedding)) of the separately pinned primitives, bit for bit;
- absmax quantization is invariant to scaling by 2, so doubling a norm's
  gamma leaves the int8 input of the projection right after it unchanged and
  doubles its scale and output exactly; a norm applied anywhere else fails;
- prefill rows are causal: row m of a long prefill equals the last row of a
  prefill of the first m+1 ids, bit for bit (a mask off by one fails);
- prefill(a..y) then decode(z) gives the logits of prefill(a..z) within 1e-3
  (position offset, RoPE position, KV append; the GEMV and GEMM epilogues
  round differently, rs/nn/bitlinear.rs:87-91);
- GQA: query head h reads KV head h // (H / Hkv) (sh/attention.wgsl:43);
- eps: the block norms use the configured eps, the sub-norms 1e-5
  (rs/nn/bitlinear.rs:112).
"""
import numpy as np
import pytest

import oracle as O
from helpers import synth

ZERO_I2S = 0x55  # four codes of 1, i.e. four zero weights


def make_weights(cfg: dict, seed: int, sub_norms: bool = True) -> dict:
    """Random weights in the oracle's naming (as synth writes them)."""
    rng = np.random.default_rng(seed)
    D, F, H, Hkv, V = cfg["D"], cfg["F"], cfg["H"], cfg["Hkv"], cfg["V"]
    hd = D // H
    w = {"model.embed_tokens.weight":
         (rng.standard_normal((V, D)) * 0.02).astype(np.float16).view(np.uint16),
         "model.norm.weight": rng.uniform(0.5, 1.5, D).astype(np.float32)}
    shapes = {"self_attn.q_proj": (H * hd, D), "self_attn.k_proj": (Hkv * hd, D),
              "self_attn.v_proj": (Hkv * hd, D), "self_attn.o_proj": (D, H * hd),
              "mlp.gate_proj": (F, D), "mlp.up_proj": (F, D), "mlp.down_proj": (D, F)}
    for i in range(cfg["n_layers"]):
        p = f"model.layers.{i}"
        for name, (N, K) in shapes.items():
            w[f"{p}.{name}.weight"] = synth.random_i2s(rng, N, K)
            w[f"{p}.{name}.weight_scale"] = synth.master_scale(rng)
        norms = [("input_layernorm", D), ("post_attention_layernorm", D)]
        if sub_norms:
            norms += [("self_attn.sub_norm", H * hd), ("mlp.sub_norm", F)]
        for name, n in norms:
            w[f"{p}.{name}.weight"] = rng.uniform(0.5, 1.5, n).astype(np.float32)
    return w


def small_cfg(**kw) -> dict:
    c = dict(n_layers=2, D=512, F=1024, H=4, Hkv=1, V=300, eps=1e-5, rope_theta=500000.0)
    c.update(kw)
    return c


def run(cfg, w, ids, max_seq=64, kv_f16=True, model=None):
    m = model or O.Model(cfg, w, max_seq=max_seq, kv_f16=kv_f16)
    tr = {}
    logits = m.forward(np.asarray(ids, np.uint32), trace=tr)
    return m, logits, tr


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


IDS = [17, 3, 250, 99, 3, 41, 7, 180, 64]


def test_zero_weights_make_every_block_the_identity():
    cfg = small_cfg()
    w = make_weights(cfg, 1)
    for k in list(w):
        if k.endswith("_proj.weight"):
            w[k] = np.full_like(w[k], ZERO_I2S)
    E = w["model.embed_tokens.weight"]
    m, logits, tr = run(cfg, w, IDS)
    emb = O.embedding(np.array(IDS, np.uint32), E)
    for l in range(cfg["n_layers"]):
        assert np.array_equal(bits(tr[(l, "x_in")]), bits(emb))
        assert not np.any(tr[(l, "o")]) and not np.any(tr[(l, "down")])
        assert np.array_equal(bits(tr[(l, "x_out")]), bits(emb))
    want = O.lm_head(O.rmsnorm(emb[-1:], w["model.norm.weight"], cfg["eps"])[0], E)
    assert np.array_equal(bits(logits), bits(want))
    # a decode step on top: the same identity for the new token
    _, logits2, _ = run(cfg, w, [5], model=m)
    emb5 = O.embedding(np.array([5], np.uint32), E)
    want2 = O.lm_head(O.rmsnorm(emb5, w["model.norm.weight"], cfg["eps"])[0], E)
    assert np.array_equal(bits(logits2), bits(want2))


@pytest.mark.parametrize("n", [1, 9])     # GEMV (decode) and GEMM (prefill) paths
def test_norm_gamma_doubling_pins_each_norm_to_its_projection(n):
    cfg = small_cfg()
    base = make_weights(cfg, 2)
    ids = IDS[:n]
    _, _, t0 = run(cfg, base, ids)
    cases = [  # (gamma doubled, int8/scale site of the projection after it, outputs that double)
        ("self_attn.sub_norm", "o", ["o"]),
        ("mlp.sub_norm", "down", ["down"]),
        ("input_layernorm", "qkv", ["q", "k", "v"]),
        ("post_attention_layernorm", None, ["gate", "up"]),
    ]
    for norm, proj, outs in cases:
        w = dict(base)
        key = f"model.layers.0.{norm}.weight"
        w[key] = (base[key] * np.float32(2)).astype(np.float32)
        _, _, t1 = run(cfg, w, ids)
        if proj:
            assert np.array_equal(t1[(0, f"{proj}_q8")], t0[(0, f"{proj}_q8")]), norm
            assert np.array_equal(bits(t1[(0, f"{proj}_scale")]),
                                  bits(t0[(0, f"{proj}_scale")] * np.float32(2))), norm
        for o in outs:
            assert np.array_equal(bits(t1[(0, o)]), bits(t0[(0, o)] * np.float32(2))), (norm, o)
        # nothing upstream of the norm moved
        upstream = {"self_attn.sub_norm": "attn", "mlp.sub_norm": "gate",
                    "input_layernorm": "x_in", "post_attention_layernorm": "x_mid"}[norm]
        assert np.array_equal(bits(t1[(0, upstream)]), bits(t0[(0, upstream)])), norm


def test_prefill_rows_are_causal():
    cfg = small_cfg()
    w = make_weights(cfg, 3)
    _, _, full = run(cfg, w, IDS)
    for m in (1, 4, len(IDS) - 2):   # m + 1 >= 2 ids: the GEMM path, as in the long prefill
        _, logits, part = run(cfg, w, IDS[:m + 1])
        for (l, site), a in part.items():
            b = full[(l, site)][:m + 1]
            if site.endswith("_q8"):
                assert np.array_equal(a, b), (l, site, m)
            else:
                assert np.array_equal(bits(a), bits(b)), (l, site, m)
        want = O.lm_head(full[(-1, "final")][m], w["model.embed_tokens.weight"])
        assert np.array_equal(bits(logits), bits(want)), m


@pytest.mark.parametrize("kv_f16", [True, False])
def test_prefill_then_decode_matches_one_prefill(kv_f16):
    """Decoding the last ids one at a time after a shorter prefill reproduces
    the long prefill's rows.  At layer 0 the two paths differ only by the
    GEMV/GEMM epilogue rounding (one ulp of q/k/v), so q, k, v and the
    attention output agree to ~1e-6; a decode at the wrong position, with the
    wrong RoPE angle or without its own K/V row is off by far more.  Past
    layer 0 those ulps flip some int8 re-quantizations, which the ternary
    layers amplify (logits move by up to ~1e-2 of max|logit| here), so the
    logits are only compared loosely."""
    cfg = small_cfg(n_layers=3)
    w = make_weights(cfg, 4)
    ids = IDS + [12, 200, 33]
    n0 = 6
    _, ref, full = run(cfg, w, ids, kv_f16=kv_f16)
    m, _, _ = run(cfg, w, ids[:n0], kv_f16=kv_f16)
    steps = []
    for t in ids[n0:]:
        m, logits, tr = run(cfg, w, [t], model=m)
        steps.append(tr)

    def rel(a, b):
        return float(np.abs(a - b).max() / np.abs(b).max())

    for i, tr in enumerate(steps):
        row = n0 + i
        for site, tol in (("q", 1e-6), ("k", 1e-6), ("v", 1e-6), ("attn", 1e-5)):
            assert rel(tr[(0, site)][0], full[(0, site)][row]) <= tol, (i, site)
    scale = float(np.abs(ref).max())
    assert np.abs(logits - ref).max() <= 5e-2 * scale
    assert not np.array_equal(bits(logits), bits(ref))   # GEMV vs GEMM epilogue really differ
    # the same decode at the wrong position (0 instead of n0) is far off at layer 0
    m2, _, _ = run(cfg, w, ids[:n0], kv_f16=kv_f16)
    m2._m.seq_len = 0
    _, _, bad = run(cfg, w, ids[n0:n0 + 1], model=m2)
    assert rel(bad[(0, "q")][0], full[(0, "q")][n0]) > 1e-1
    assert rel(bad[(0, "attn")][0], full[(0, "attn")][n0]) > 1e-2


def test_gqa_query_head_reads_kv_head_h_div_group():
    cfg = small_cfg(H=4, Hkv=2)
    w = make_weights(cfg, 5)
    hd = cfg["D"] // cfg["H"]
    for dead in (0, 1):
        ww = dict(w)
        v = w["model.layers.0.self_attn.v_proj.weight"].copy()
        v[dead * hd:(dead + 1) * hd] = ZERO_I2S
        ww["model.layers.0.self_attn.v_proj.weight"] = v
        _, _, tr = run(cfg, ww, IDS)
        att = tr[(0, "attn")].reshape(len(IDS), cfg["H"], hd)
        for h in range(cfg["H"]):
            if h // (cfg["H"] // cfg["Hkv"]) == dead:
                assert not np.any(att[:, h]), (dead, h)
            else:
                assert np.any(att[:, h]), (dead, h)


def test_eps_of_each_norm():
    cfg = small_cfg(eps=1e-2)   # far from the sub-norms' fixed 1e-5
    w = make_weights(cfg, 6)
    _, logits, tr = run(cfg, w, IDS)
    g = lambda k: w[f"model.layers.0.{k}.weight"]
    assert np.array_equal(bits(tr[(0, "attn_norm")]),
                          bits(O.rmsnorm(tr[(0, "x_in")], g("input_layernorm"), 1e-2)))
    assert np.array_equal(bits(tr[(0, "ffn_norm")]),
                          bits(O.rmsnorm(tr[(0, "x_mid")], g("post_attention_layernorm"), 1e-2)))
    q8, sc = O.quantize(O.rmsnorm(tr[(0, "attn")], g("self_attn.sub_norm"), 1e-5))
    assert np.array_equal(q8, tr[(0, "o_q8")]) and np.array_equal(bits(sc), bits(tr[(0, "o_scale")][:, 0]))
    q8, sc = O.quantize(O.rmsnorm(O.mul(O.relu2(tr[(0, "gate")]), tr[(0, "up")]),
                                  g("mlp.sub_norm"), 1e-5))
    assert np.array_equal(q8, tr[(0, "down_q8")])
    last = cfg["n_layers"] - 1
    assert np.array_equal(bits(tr[(-1, "final")]),
                          bits(O.rmsnorm(tr[(last, "x_out")], w["model.norm.weight"], 1e-2)))


def test_residual_adds_and_missing_sub_norms():
    cfg = small_cfg()
    w = make_weights(cfg, 7, sub_norms=False)
    _, _, tr = run(cfg, w, IDS)
    for l in range(cfg["n_layers"]):
        assert np.array_equal(bits(tr[(l, "x_mid")]), bits(O.add(tr[(l, "x_in")], tr[(l, "o")])))
        assert np.array_equal(bits(tr[(l, "x_out")]), bits(O.add(tr[(l, "x_mid")], tr[(l, "down")])))
        if l + 1 < cfg["n_layers"]:
            assert np.array_equal(bits(tr[(l + 1, "x_in")]), bits(tr[(l, "x_out")]))
        # no sub-norm tensor: the projection quantizes its input directly (bitlinear.rs:60-70)
        q8, _ = O.quantize(tr[(l, "attn")])
        assert np.array_equal(q8, tr[(l, "o_q8")])


def test_kv_cache_rows_hold_roped_k_and_v():
    cfg = small_cfg()
    w = make_weights(cfg, 8)
    hd, Hkv = cfg["D"] // cfg["H"], cfg["Hkv"]
    for kv_f16 in (True, False):
        m, _, tr = run(cfg, w, IDS, kv_f16=kv_f16, max_seq=32)
        kc = m.kcache.reshape(cfg["n_layers"], 32, Hkv * hd)
        vc = m.vcache.reshape(cfg["n_layers"], 32, Hkv * hd)
        for l in range(cfg["n_layers"]):
            k, v = tr[(l, "k")], tr[(l, "v")]
            if kv_f16:
                k = k.astype(np.float16).astype(np.float32)
                v = v.astype(np.float16).astype(np.float32)
            assert np.array_equal(bits(kc[l, :len(IDS)]), bits(k))
            assert np.array_equal(bits(vc[l, :len(IDS)]), bits(v))
            assert not np.any(kc[l, len(IDS):])
