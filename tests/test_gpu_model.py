"""Whole-model parity on the GPU: the HIP engine (prefill on MFMA GEMMs,
decode as hipGraph replays) against the oracle's restatement of
nn/model.rs:193-266 on the same synthetic GGUF.

The engine computes every reduction in the oracle's order, so its logits are
the oracle's bit for bit (f16-rounded KV cache on both sides) and the greedy
tokens are identical at every step, near-ties included.  Exactness is what
parity means here: in these random-init ternary models a one-ulp change of an
f32 value flips int8 re-quantizations downstream, and 30 layers amplify that
to ~10% of max|logit| (measured on the 2B shape), so a 1e-3 tolerance would
only be met by chance.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from helpers import oracle_weights, pkg, synth

pytestmark = pytest.mark.gpu


def _close(got, ref, rel=1e-3):
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= rel * scale, f"max err {err} vs {rel} * {scale}"


def _same(got, ref, what=""):
    g, r = got.view(np.uint32), ref.view(np.uint32)
    if not np.array_equal(g, r):
        bad = np.count_nonzero(g != r)
        err = float(np.abs(got - ref).max())
        raise AssertionError(f"{what}: {bad} of {got.size} logits differ (max err {err:.3g}, "
                             f"max|ref| {float(np.abs(ref).max()):.3g})")


def _greedy_parity(path, prompt, steps, kv_f16=True, max_seq=None):
    """Prefill + `steps` greedy steps on the GPU and in the oracle: every
    logit bit-equal, every token equal."""
    max_seq = max_seq or (len(prompt) + steps + 2)
    m = pkg.Model(path, max_seq=max_seq, kv="f16" if kv_f16 else "f32")
    cfg, w = oracle_weights(path)
    om = O.Model(cfg, w, max_seq=max_seq, kv_f16=kv_f16)
    tok, logits = m.forward(prompt)
    ref = om.forward(prompt.astype(np.uint32))
    _same(logits, ref, "prefill")
    toks = [tok]
    for i in range(steps):
        assert tok == O.argmax(ref), f"step {i}: gpu {tok} oracle {O.argmax(ref)}"
        tok, logits = m.step()
        ref = om.forward(np.array([toks[-1]], np.uint32))
        _same(logits, ref, f"step {i} (position {len(prompt) + i})")
        toks.append(tok)
    assert tok == O.argmax(ref)
    m.close()
    return toks


def test_small_model_prefill_and_64_greedy_steps():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 40).astype(np.int32)
    toks = _greedy_parity(path, prompt, 64)
    assert len(toks) == 65


# ---- the reference's own cache type (f32 K/V, nn/attention.rs:23-48) -------
def test_small_model_f32_cache_oracle():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 17).astype(np.int32)
    assert len(_greedy_parity(path, prompt, 64, kv_f16=False)) == 65


@pytest.mark.parametrize("n_prompt", [1, 255, 300])
def test_small_model_f32_cache_long_rows(n_prompt):
    """Prompts that end before, at and past 256 positions, then decode to
    position 560: the P.V chains run over every cached position in one loop
    (the f32 cache's attention), bit-equal to the oracle throughout."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng([3, n_prompt]).integers(0, cfg.vocab, n_prompt).astype(np.int32)
    _greedy_parity(path, prompt, 560 - n_prompt if n_prompt < 300 else 40, kv_f16=False,
                   max_seq=600)


def test_f32_cache_prefill_then_decode_equals_oracle_paths():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    ids = np.random.default_rng(6).integers(0, cfg.vocab, 25).astype(np.int32)
    c, w = oracle_weights(path)
    m = pkg.Model(path, max_seq=64, kv="f32")
    assert m.info["kv_f32"] == 1
    for split in (24, 3):
        om = O.Model(c, w, max_seq=64, kv_f16=False)
        m.reset()
        _, lg = m.forward(ids[:split])
        _same(lg, om.forward(ids[:split].astype(np.uint32)), f"prefill {split}")
        for t in ids[split:]:
            _, lg = m.forward(np.array([t], np.int32))
            _same(lg, om.forward(np.array([t], np.uint32)), f"decode after {split}")
    m.close()


def test_f32_cache_is_the_mode_that_ran():
    """The two cache types give different logits (f16 rounding of K/V), the
    f32 ones equal to the oracle's f32 path; a batch needs the f16 cache."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    ids = np.random.default_rng(8).integers(0, cfg.vocab, 30).astype(np.int32)
    out = {}
    for kv in ("f16", "f32"):
        m = pkg.Model(path, max_seq=64, kv=kv)
        out[kv] = m.forward(ids)[1]
        if kv == "f32":
            with pytest.raises(pkg.NativeError, match="f16 KV cache"):
                pkg.Batch(m, 2, 64)
        m.close()
    assert not np.array_equal(out["f16"], out["f32"])
    c, w = oracle_weights(path)
    _same(out["f32"], O.Model(c, w, max_seq=64, kv_f16=False).forward(ids.astype(np.uint32)), "f32")
    with pytest.raises(ValueError):
        pkg.Model(path, kv="bf16")


def test_prefill_then_decode_equals_oracle_paths():
    """prefill(a..y) + decode(z) and prefill(a..z) each equal the oracle's same
    path (the GEMV and GEMM epilogues round differently, so the two paths
    differ from each other, and each must match its own restatement)."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    ids = np.random.default_rng(5).integers(0, cfg.vocab, 25).astype(np.int32)
    c, w = oracle_weights(path)
    m = pkg.Model(path, max_seq=64)
    for split in (24, 20, 2):
        om = O.Model(c, w, max_seq=64, kv_f16=True)
        m.reset()
        _, lg = m.forward(ids[:split])
        _same(lg, om.forward(ids[:split].astype(np.uint32)), f"prefill {split}")
        for t in ids[split:]:
            _, lg = m.forward(np.array([t], np.int32))
            _same(lg, om.forward(np.array([t], np.uint32)), f"decode after {split}")
    m.close()


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


def _decode_logits(path, prompt, steps, max_seq, attn, var="OXB_ATTN"):
    import os
    old = os.environ.get(var)
    os.environ[var] = attn   # read when the model loads
    try:
        m = pkg.Model(path, max_seq=max_seq)
    finally:
        if old is None:
            del os.environ[var]
        else:
            os.environ[var] = old
    tok, logits = m.forward(prompt)
    out = [logits]
    toks = [tok]
    for _ in range(steps):
        tok, logits = m.step()
        out.append(logits)
        toks.append(tok)
    m.close()
    return toks, np.stack(out)


def test_decode_attention_forms_identical():
    """The per-head attention (one and two position groups), the fused
    kernel and the split kernels give the same bits, across the switches
    between them (positions 240 .. 540: 256 and 512 are crossed)."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab, 240).astype(np.int32)
    t_head, l_head = _decode_logits(path, prompt, 300, 600, "head")
    t_fused, l_fused = _decode_logits(path, prompt, 300, 600, "fused")
    t_split, l_split = _decode_logits(path, prompt, 300, 600, "split")
    assert t_split == t_fused == t_head
    assert np.array_equal(l_split.view(np.uint32), l_fused.view(np.uint32))
    assert np.array_equal(l_split.view(np.uint32), l_head.view(np.uint32))


@pytest.mark.parametrize("shape", ["small", "2b"])
def test_fused_qkv_attention_steps_identical(shape):
    """OXB_QKV_ATTN=1 (q|k|v and the attention of steps up to 256 positions
    as one launch, oxb_qkv_attn_decode) gives the default path's tokens and
    logits bits, across position 256 where the steps switch back."""
    cfg = synth.small_config() if shape == "small" else synth.BITNET_2B
    path = synth.cached_gguf(cfg, seed=7 if shape == "small" else 1234)
    n_prompt, steps = (200, 80) if shape == "small" else (230, 40)
    prompt = np.random.default_rng(12).integers(0, cfg.vocab, n_prompt).astype(np.int32)
    t0, l0 = _decode_logits(path, prompt, steps, 320, "0", "OXB_QKV_ATTN")
    t1, l1 = _decode_logits(path, prompt, steps, 320, "1", "OXB_QKV_ATTN")
    assert t0 == t1
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))


def test_single_token_forward_is_decode_path():
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    m = pkg.Model(path, max_seq=64)
    cfg_o, w = oracle_weights(path)
    om = O.Model(cfg_o, w, max_seq=64, kv_f16=True)
    for t in (5, 999, 17):
        tok, logits = m.forward(np.array([t], np.int32))
        _same(logits, om.forward(np.array([t], np.uint32)), f"id {t}")
    m.close()


@pytest.mark.timeout(900)
def test_bitnet_2b_shape_greedy_256():
    """Config 3 end to end: the 2B-shaped random-init model, 128-token prompt,
    256 greedy steps (positions 128..384: the one-kernel attention up to 256
    positions, the 512-row one past it), logits bit-equal to the oracle (P.V
    in the reference's one loop over every position) at every step."""
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    prompt = np.random.default_rng(2024).integers(0, synth.BITNET_2B.vocab, 128).astype(np.int32)
    toks = _greedy_parity(path, prompt, 256)
    assert len(toks) == 257


@pytest.mark.timeout(900)
def test_bitnet_2b_shape_f32_cache_greedy_256():
    """Config 3 with the reference's f32 KV cache: 128-token prompt, 256
    greedy steps, logits bit-equal to the oracle's f32-cache path."""
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    prompt = np.random.default_rng(2024).integers(0, synth.BITNET_2B.vocab, 128).astype(np.int32)
    assert len(_greedy_parity(path, prompt, 256, kv_f16=False)) == 257


@pytest.mark.timeout(900)
def test_bitnet_2b_shape_f32_cache_300_prompt_64_steps():
    """The 2B shape, f32 KV cache, a 300-token prompt (prefill rows past 256
    positions) and 64 greedy steps, bit-equal to the oracle."""
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    prompt = np.random.default_rng(2025).integers(0, synth.BITNET_2B.vocab, 300).astype(np.int32)
    assert len(_greedy_parity(path, prompt, 64, kv_f16=False)) == 65


# ---- long context: 2048-token prefill, then decode (bs 1, 8 and 32) --------
LONG = 2048
LONG_STEPS = 64


def _long_prompt(slot: int) -> np.ndarray:
    return np.random.default_rng([77, slot]).integers(0, synth.BITNET_2B.vocab, LONG).astype(np.int32)


def _oracle_long(path, slot, kv_f16=True):
    """The oracle on slot `slot`'s 2048-token prompt: prefill logits and the
    logits after each of LONG_STEPS greedy steps."""
    cfg, w = oracle_weights(path)
    om = O.Model(cfg, w, max_seq=LONG + LONG_STEPS + 2, kv_f16=kv_f16)
    out = [om.forward(_long_prompt(slot).astype(np.uint32))]
    for _ in range(LONG_STEPS):
        out.append(om.forward(np.array([O.argmax(out[-1])], np.uint32)))
    return out


@pytest.fixture(scope="module")
def long_oracle():
    """(path, {slot: oracle logits}) for slots 0 and 1 (f16 KV cache)."""
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    return path, {0: _oracle_long(path, 0), 1: _oracle_long(path, 1)}


def _long_run(m, slot):
    """Greedy tokens and logits of slot `slot`'s prompt on model m (reset)."""
    m.reset()
    tok, logits = m.forward(_long_prompt(slot))
    out, toks = [logits], [tok]
    for _ in range(LONG_STEPS):
        tok, logits = m.step()
        out.append(logits)
        toks.append(tok)
    return toks, out


def _long_single(path, slot, kv="f16"):
    m = pkg.Model(path, max_seq=LONG + LONG_STEPS + 2, kv=kv)
    try:
        return _long_run(m, slot)
    finally:
        m.close()


@pytest.mark.timeout(900)
def test_bitnet_2b_prefill_2048_and_decode_64(long_oracle):
    """Config 4 at bs 1: 2048-token prefill, then 64 greedy steps (positions
    2048..2112), every logit bit-equal to the oracle."""
    path, ref = long_oracle
    toks, out = _long_single(path, 0)
    _same(out[0], ref[0][0], "2048-token prefill")
    for i in range(LONG_STEPS):
        assert toks[i] == O.argmax(ref[0][i]), f"step {i}"
        _same(out[i + 1], ref[0][i + 1], f"step {i} at position {LONG + i}")


@pytest.mark.timeout(900)
def test_bitnet_2b_f32_cache_prefill_2048_and_decode_64():
    """Config 4 at bs 1 with the reference's f32 KV cache, bit-equal to the
    oracle's f32 path."""
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    ref = _oracle_long(path, 0, kv_f16=False)
    toks, out = _long_single(path, 0, kv="f32")
    _same(out[0], ref[0], "2048-token prefill (f32 cache)")
    for i in range(LONG_STEPS):
        assert toks[i] == O.argmax(ref[i]), f"step {i}"
        _same(out[i + 1], ref[i + 1], f"step {i} at position {LONG + i} (f32 cache)")


@pytest.mark.timeout(900)
@pytest.mark.parametrize("B", [8, 32])
def test_bitnet_2b_batched_decode_after_2048(long_oracle, B):
    """B slots, each prefilled with its own 2048-token prompt, decoded
    together for 64 steps: slots 0 and 1 equal the oracle at every step's
    token and at the last logits, and every slot's tokens and last logits
    equal that sequence decoded alone."""
    path, ref = long_oracle
    m = pkg.Model(path, max_seq=LONG + LONG_STEPS + 2)
    b = pkg.Batch(m, B, 2560)
    first = [b.prefill(i, _long_prompt(i)) for i in range(B)]
    got = b.decode_greedy(LONG_STEPS)
    last = b.logits()
    for z in (0, 1):
        toks = [first[z]] + got[z].tolist()
        assert toks == [O.argmax(r) for r in ref[z]], f"slot {z} vs oracle"
        _same(last[z], ref[z][-1], f"batched slot {z} vs oracle")
    for i in range(2, B):
        toks, lg = _long_run(m, i)
        assert [first[i]] + got[i].tolist() == toks, f"slot {i}"
        _same(last[i], lg[-1], f"slot {i}")
    b.close()
    m.close()


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


@pytest.mark.parametrize("prefix,f16", [("llama", True), ("bitnet", False), ("bitnet-25", True)])
def test_loader_metadata_prefix_and_f16_norms(prefix, f16):
    """model/loader.rs:221-291 reads each hyperparameter under the arch name,
    then llama., bitnet., bitnet-25.; F16 norm tensors are widened to f32
    (:148-151).  Files with the metadata under a fallback prefix and with F16
    norms load and decode bit for bit like the oracle on the same weights."""
    cfg = synth.small_config(meta_prefix=prefix, norm_f16=f16)
    path = synth.cached_gguf(cfg, seed=7)
    prompt = np.random.default_rng(9).integers(0, cfg.vocab, 21).astype(np.int32)
    assert len(_greedy_parity(path, prompt, 8)) == 9


def _token_text(path):
    """decode_one through the host tokenizer (pinned against HF tokenizers in
    test_tokenizer.py): the bytes generate passes to its callback per id."""
    L = pkg._native.lib()
    t = L.oxb_tokenizer_load(path.encode())
    assert t, L.oxb_last_error()
    cache = {}

    def text(i):
        if i not in cache:
            n = L.oxb_tokenizer_decode_one(t, i, None, 0)
            buf = C.create_string_buffer(n + 1)
            L.oxb_tokenizer_decode_one(t, i, buf, n + 1)
            cache[i] = buf.raw[:n]
        return cache[i]
    return text


def _greedy_ids(path, ids, n):
    m = pkg.Model(path, max_seq=64)
    t, _ = m.forward(np.array(ids, np.int32))
    out = [t] + m.decode_greedy(n - 1).tolist()
    m.close()
    return out


def _stream(path, prompt, max_tokens):
    nat = pkg._native
    L = nat.lib()
    h = L.oxbitnet_load(path.encode(), None)
    assert h, L.oxbitnet_error_message()
    got = []
    tf = nat.TokenFn(lambda t, n, ud: (got.append(C.string_at(t, n)), 0)[1])
    g = L.oxbitnet_default_generate_options()
    g.max_tokens, g.top_k, g.repeat_penalty = max_tokens, 1, 1.0
    assert L.oxbitnet_generate(h, prompt.encode(), C.byref(g), tf, None) == 0
    L.oxbitnet_free(h)
    return got


def test_generate_stops_before_eos():
    """rs/lib.rs:175-177: a sampled EOS (or EOT) ends the stream and is not
    emitted.  generate("ab") prefills [BOS, 'a', 'b'] (byte tokens 97, 98);
    files that differ only in their EOS id stop after 0 and 1 tokens when the
    EOS is the first and the second greedy token."""
    base = synth.small_config()
    ids = _greedy_ids(synth.cached_gguf(base, seed=7), [256, 97, 98], 4)
    for k in (0, 1):
        eos = ids[k]
        stops = {eos, 260}   # the file's EOS and <|eot_id|>
        want = next(j for j, t in enumerate(ids) if t in stops)
        path = synth.cached_gguf(synth.small_config(eos=eos), seed=7)
        got = _stream(path, "ab", 10)
        assert len(got) == want <= k, (k, eos, ids, got)


def _penalised_argmax(logits, recent, penalty):
    """rs/sampling.rs:14-24 then top-1: each occurrence in the window divides
    a positive logit (multiplies a negative one) by the penalty, in f32."""
    lg = logits.astype(np.float32).copy()
    p = np.float32(penalty)
    for t in recent:
        lg[t] = lg[t] / p if lg[t] > 0 else lg[t] * p
    return int(np.argmax(lg)), lg


def test_generate_top1_with_penalty_is_the_host_argmax_of_penalised_logits():
    """generate with top_k 1 and repeat penalty 1.1 (the last 64 tokens) streams
    the argmax of the penalised logits that the ids-level engine returns for
    the same ids, step by step; steps whose top two penalised logits tie are
    not expected (the sampler would draw between them)."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    n = 24
    L = pkg._native.lib()
    h = L.oxbitnet_load(path.encode(), None)
    assert h, L.oxbitnet_error_message()
    got = []
    text = _token_text(path)
    tf = pkg._native.TokenFn(lambda t, k, ud: (got.append(C.string_at(t, k)), 0)[1])
    g = L.oxbitnet_default_generate_options()
    g.max_tokens, g.top_k, g.repeat_penalty, g.temperature = n, 1, 1.1, 0.8
    assert L.oxbitnet_generate(h, b"ab", C.byref(g), tf, None) == 0
    L.oxbitnet_free(h)

    m = pkg.Model(path, max_seq=64)
    _, logits = m.forward(np.array([256, 97, 98], np.int32))
    recent, want = [], []
    for _ in range(n):
        t, lg = _penalised_argmax(logits, recent[-64:], 1.1)
        top2 = np.sort(lg)[-2:]
        assert top2[0] < top2[1], "tie at the top: the draw is not determined"
        if t in (257, 260):
            break
        recent.append(t)
        b = text(t)
        if b"\0" not in b:
            want.append(b)
        _, logits = m.forward(np.array([t], np.int32))
    m.close()
    assert got == want


def test_python_binding_greedy_tokens_are_the_engines():
    """BitNet.generate (greedy: top_k 1, no penalty) streams the decoded
    greedy tokens of the ids-level engine for the same prompt ids."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    ids = _greedy_ids(path, [256, 97, 98], 16)
    text = _token_text(path)
    want = []
    for i in ids:
        if i in (257, 260):   # EOS, <|eot_id|>
            break
        b = text(i)
        if b"\0" not in b:   # a token with a NUL is not passed to the callback
            want.append(b.decode("utf-8"))
    bn = pkg.BitNet.load_sync(path)
    got = []
    n = bn.generate("ab", got.append, max_tokens=16, top_k=1, repeat_penalty=1.0)
    bn.dispose()
    assert n == len(got) and got == want


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
