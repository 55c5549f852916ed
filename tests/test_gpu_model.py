"""Whole-model parity on the GPU: the HIP engine (prefill on MFMA GEMMs,
decode as hipGraph replays) against the oracle's restatement of
nn/model.rs:193-266 on the same synthetic GGUF.

Tolerance: logits within 1e-3 of max|logit| (the path's 1e-3 relative
bound); greedy tokens identical except at documented near-ties (top-2 gap
below 1e-3 relative), where the oracle continues from the GPU's token.
The oracle runs with an f16-rounded KV cache like the product; the f32-cache
restatement is compared at the same tolerance.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from helpers import near_tie, oracle_weights, pkg, synth

pytestmark = pytest.mark.gpu


def _close(got, ref, rel=1e-3):
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= rel * scale, f"max err {err} vs {rel} * {scale}"


def _greedy_parity(path, prompt, steps, kv_f16=True, max_seq=None):
    max_seq = max_seq or (len(prompt) + steps + 2)
    m = pkg.Model(path, max_seq=max_seq)
    cfg, w = oracle_weights(path)
    om = O.Model(cfg, w, max_seq=max_seq, kv_f16=kv_f16)
    tok, logits = m.forward(prompt)
    ref = om.forward(prompt.astype(np.uint32))
    _close(logits, ref)
    ties = 0
    toks = [tok]
    for i in range(steps):
        if tok != O.argmax(ref):
            assert near_tie(ref), f"step {i}: gpu {tok} oracle {O.argmax(ref)}"
            ties += 1
        tok, logits = m.step()
        ref = om.forward(np.array([toks[-1]], np.uint32))
        _close(logits, ref)
        toks.append(tok)
    m.close()
    return toks, ties


def test_small_model_prefill_and_64_greedy_steps():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 40).astype(np.int32)
    toks, ties = _greedy_parity(path, prompt, 64)
    assert len(toks) == 65 and ties <= 2


@pytest.mark.skip(reason="the engine stores K/V as f16; the f32-cache mode that matches "
                         "nn/attention.rs:28-29 is not built yet")
def test_small_model_f32_cache_oracle():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 17).astype(np.int32)
    _greedy_parity(path, prompt, 16, kv_f16=False)


def test_graph_decode_matches_stepwise():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 9).astype(np.int32)
    m = pkg.Model(path, max_seq=128)
    t0, _ = m.forward(prompt)
    seq = [m.step(want_logits=False)[0] for _ in range(30)]
    m.reset()
    t1, _ = m.forward(prompt)
    g = m.decode_greedy(30)
    assert t0 == t1 and g.tolist() == seq
    assert m.position == len(prompt) + 30
    # decode_greedy refuses to overflow the cache
    with pytest.raises(pkg.NativeError, match="overflow"):
        m.decode_greedy(1000)
    m.close()


def _decode_logits(path, prompt, steps, max_seq, fused_max_s):
    import os
    old = os.environ.get("OXB_ATTN_FUSED_MAX_S")
    os.environ["OXB_ATTN_FUSED_MAX_S"] = str(fused_max_s)   # read when the model loads
    try:
        m = pkg.Model(path, max_seq=max_seq)
    finally:
        if old is None:
            del os.environ["OXB_ATTN_FUSED_MAX_S"]
        else:
            os.environ["OXB_ATTN_FUSED_MAX_S"] = old
    tok, logits = m.forward(prompt)
    out = [logits]
    toks = [tok]
    for _ in range(steps):
        tok, logits = m.step()
        out.append(logits)
        toks.append(tok)
    m.close()
    return toks, np.stack(out)


def test_fused_and_split_decode_attention_identical():
    """The one-kernel attention graph (short caches) and the two-kernel graph
    give the same bits, including across the switch between them."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab, 500).astype(np.int32)
    t_split, l_split = _decode_logits(path, prompt, 24, 600, 0)
    t_mixed, l_mixed = _decode_logits(path, prompt, 24, 600, 512)
    t_fused, l_fused = _decode_logits(path, prompt, 24, 600, 600)
    assert t_split == t_mixed == t_fused
    assert np.array_equal(l_split.view(np.uint32), l_mixed.view(np.uint32))
    assert np.array_equal(l_split.view(np.uint32), l_fused.view(np.uint32))


def test_single_token_forward_is_decode_path():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    m = pkg.Model(path, max_seq=64)
    cfg_o, w = oracle_weights(path)
    om = O.Model(cfg_o, w, max_seq=64, kv_f16=True)
    for t in (5, 999, 17):
        tok, logits = m.forward(np.array([t], np.int32))
        _close(logits, om.forward(np.array([t], np.uint32)))
    m.close()


@pytest.mark.timeout(600)
def test_bitnet_2b_shape_greedy_64():
    """The 2B-shaped random-init model: 128-token prompt, 64 greedy steps."""
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    prompt = np.random.default_rng(2024).integers(0, synth.BITNET_2B.vocab, 128).astype(np.int32)
    toks, ties = _greedy_parity(path, prompt, 64)
    assert len(toks) == 65 and ties <= 3


def test_c_abi_generate_and_chat_greedy():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    nat = pkg._native
    L = nat.lib()
    progress = []
    opts = L.oxbitnet_default_load_options()
    cb = nat.ProgressFn(lambda p, ud: progress.append((p.contents.phase, p.contents.fraction)))
    opts.on_progress = cb
    h = L.oxbitnet_load(path.encode(), C.byref(opts))
    assert h, L.oxbitnet_error_message()
    assert progress[0][0] == 0 and progress[-1] == (2, 1.0)
    got = []
    tf = nat.TokenFn(lambda t, n, ud: (got.append(C.string_at(t, n)), 0)[1])
    g = L.oxbitnet_default_generate_options()
    g.max_tokens, g.top_k, g.repeat_penalty = 12, 1, 1.0
    assert L.oxbitnet_generate(h, b"hello world", C.byref(g), tf, None) == 0
    assert len(got) == 12
    # stop from the callback after 3 tokens
    n = [0]
    stop = nat.TokenFn(lambda t, k, ud: (n.__setitem__(0, n[0] + 1), 1 if n[0] >= 3 else 0)[1])
    assert L.oxbitnet_generate(h, b"abc", C.byref(g), stop, None) == 0
    assert n[0] == 3
    msgs = (nat.ChatMessage * 2)(nat.ChatMessage(b"system", b"be brief"),
                                 nat.ChatMessage(b"user", b"hi"))
    got.clear()
    assert L.oxbitnet_chat(h, msgs, 2, C.byref(g), tf, None) == 0
    assert len(got) == 12
    # sampling path (top-k 50, temperature 0.8, penalty 1.1) runs and streams
    got.clear()
    g2 = L.oxbitnet_default_generate_options()
    g2.max_tokens = 8
    g2.temperature = 0.8
    assert L.oxbitnet_generate(h, b"xyz", C.byref(g2), tf, None) == 0
    assert len(got) == 8
    L.oxbitnet_free(h)


def test_python_bitnet_api():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    bn = pkg.BitNet.load_sync(path)
    assert repr(bn) == "BitNet(loaded)"
    toks = bn.generate_tokens_sync("hello", max_tokens=6, top_k=1)
    assert len(toks) == 6
    assert bn.generate_sync("hello", max_tokens=6, top_k=1) == "".join(toks)  # greedy, but
    # repeat_penalty 1.1 applies as in the reference binding; identical prompt -> identical text
    n = bn.chat([("user", "hi")], lambda s: None, max_tokens=4, top_k=1)
    assert n == 4
    bn.dispose()
    assert repr(bn) == "BitNet(disposed)"
    with pytest.raises(RuntimeError, match="disposed"):
        bn.generate("x", print)


def test_two_handles_on_two_threads():
    """Two models (each its own stream and graphs) prefilled and decoded from
    two host threads at once give the tokens each gives alone (the C ABI's
    threading contract: one handle per thread, handles independent)."""
    import threading
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    rng = np.random.default_rng(77)
    prompts = [rng.integers(0, cfg.vocab, 30).astype(np.int32) for _ in range(2)]
    models = [pkg.Model(path, max_seq=160) for _ in range(2)]

    def run(i, out):
        m = models[i]
        m.reset()
        t, _ = m.forward(prompts[i], want_logits=False)
        out[i] = [t] + m.decode_greedy(100).tolist()

    alone = [None, None]
    for i in range(2):
        run(i, alone)
    together = [None, None]
    th = [threading.Thread(target=run, args=(i, together)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert together == alone
    for m in models:
        m.close()


@pytest.mark.parametrize("B", [1, 3, 5, 17])
def test_batched_decode_equals_single_sequences(B):
    """Slots decoded together give each slot's one-sequence tokens and logits
    bit for bit (B = 17: two token tiles in the GEMMs, LM head passes 8+8+1;
    B = 5: 4+1)."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    rng = np.random.default_rng(100 + B)
    prompts = [rng.integers(0, cfg.vocab, int(rng.integers(2, 40))).astype(np.int32)
               for _ in range(B)]
    steps = 12
    m = pkg.Model(path, max_seq=128)
    ref_toks, ref_logits = [], []
    for pr in prompts:
        m.reset()
        tok, _ = m.forward(pr, want_logits=False)
        toks = [tok]
        logits = None
        for _ in range(steps):
            tok, logits = m.step()
            toks.append(tok)
        ref_toks.append(toks)
        ref_logits.append(logits)
    b = pkg.Batch(m, B, 96)
    first = [b.prefill(i, pr) for i, pr in enumerate(prompts)]
    got = b.decode_greedy(steps)
    last = b.logits()
    for i in range(B):
        assert [first[i]] + got[i].tolist() == ref_toks[i], f"slot {i}"
        assert np.array_equal(last[i].view(np.uint32), ref_logits[i].view(np.uint32)), f"slot {i}"
        assert b.position(i) == len(prompts[i]) + steps
    with pytest.raises(pkg.NativeError, match="overflow"):
        b.decode_greedy(200)
    b.close()
    m.close()


def test_batch_rejects_unprefilled_slot():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    m = pkg.Model(path, max_seq=64)
    b = pkg.Batch(m, 2, 64)
    b.prefill(0, np.array([1, 2, 3], np.int32))
    with pytest.raises(pkg.NativeError, match="no prompt"):
        b.decode_greedy(1)
    with pytest.raises(pkg.NativeError, match=">= 2 tokens"):
        b.prefill(1, np.array([5], np.int32))
    b.close()
    m.close()
