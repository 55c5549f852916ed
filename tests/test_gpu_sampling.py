"""Device sampling (sampling.hip) against the host sampler oxb_sample_logits,
the restatement of rs/sampling.rs:4-80 that test_sampling.py pins: the same
logits, options, window and uniform draw u must give the same token, for
every path of the device code (top-k lists, the dense running sum for k = 0,
k > 256 and ties at the threshold, NaN / inf logits, windows longer than the
LDS stage), and the engine's per-step sampling must give, at every step, the
host sampler's token on the logits it returns.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import ops, pkg, synth

pytestmark = pytest.mark.gpu


def host_sample(logits, temperature, top_k, penalty, recent, u):
    lg = np.ascontiguousarray(logits, np.float32).copy()
    rec = np.ascontiguousarray(recent, np.int32)
    return pkg.lib().oxb_sample_logits(lg.ctypes.data, lg.size, float(temperature), int(top_k),
                                       float(penalty), rec.ctypes.data if rec.size else None,
                                       rec.size, float(u))


class DeviceSampler:
    def __init__(self, V):
        L = ops.lib()
        self.V = V
        self.ws_bytes = L.oxb_sample_ws_bytes(V)
        self.ws = ops.DeviceArray((self.ws_bytes,), np.uint8)
        self.lg = ops.DeviceArray((V,), np.float32)
        self.u = ops.DeviceArray((1,), np.float32)
        self.tok = ops.DeviceArray((1,), np.int32)

    def __call__(self, logits, temperature, top_k, penalty, recent, u):
        L = ops.lib()
        self.lg.upload(np.ascontiguousarray(logits, np.float32))
        self.u.upload(np.array([u], np.float32))
        rec = np.ascontiguousarray(recent, np.int32)
        drec = ops.DeviceArray.from_host(rec) if rec.size else None
        ops.check(L.oxb_sample_device(self.lg.ptr, self.V, float(temperature), int(top_k),
                                      float(penalty), drec.ptr if drec else None, rec.size,
                                      self.u.ptr, self.tok.ptr, self.ws.ptr, self.ws_bytes, None),
                  "sample_device")
        ops.sync()
        out = int(self.tok.download()[0])
        # the device sampler leaves the logits as they were
        assert np.array_equal(self.lg.download().view(np.uint32),
                              np.ascontiguousarray(logits, np.float32).view(np.uint32))
        return out


def _check(ds, logits, T, k, pen, rec, u, what=""):
    want = host_sample(logits, T, k, pen, rec, u)
    got = ds(logits, T, k, pen, rec, u)
    assert got == want, (what, T, k, pen, len(rec), u, got, want)
    return got


def _logits(rng, V, scale=3.0):
    return (rng.standard_normal(V) * scale).astype(np.float32)


@pytest.mark.parametrize("V", [300, 2048, 5000, 128256])
def test_device_sampler_matches_host(V):
    rng = np.random.default_rng(V)
    ds = DeviceSampler(V)
    lg = _logits(rng, V)
    rec = rng.integers(0, V, 40).astype(np.int32)
    rec[5:9] = rec[0]                     # an id penalised five times
    rec[20] = -3                          # out of range: ignored
    rec[21] = V + 7
    for T in (1.0, 0.7, 1.6):
        for k in (0, 1, 2, 50, 256, 257, 1000, V - 1, V, V + 5):
            for pen in (1.0, 1.1, 0.8):
                for u in (0.0, 1e-7, 0.37, 0.999999):
                    _check(ds, lg, T, k, pen, rec if pen != 1.0 else rec[:0], u, "grid")


def test_device_sampler_draw_shares_follow_the_host():
    """Many draws over one distribution: every u of a grid gives the host's
    token (the inverse CDF is a step function of u; the grid crosses every
    step of the top-50 tokens)."""
    V = 128256
    rng = np.random.default_rng(11)
    ds = DeviceSampler(V)
    lg = _logits(rng, V, 2.0)
    lg[:60] += 9.0                       # 60 dominant tokens at the start
    for u in np.linspace(0.0, 0.999, 97):
        _check(ds, lg, 0.9, 50, 1.1, [3, 3, 17], float(u), "shares")


def test_device_sampler_ties_at_the_threshold():
    """Values equal to the k-th largest are kept (sampling.rs:55-59), also
    when one 2048-value block holds more of them than its list of k."""
    V = 10000
    rng = np.random.default_rng(3)
    ds = DeviceSampler(V)
    for levels in (4, 17, 300):
        lg = (rng.integers(0, levels, V) * 0.25).astype(np.float32)
        for k in (1, 3, 50, 256, 600):
            for u in (0.0, 0.2, 0.5, 0.93):
                _check(ds, lg, 1.0, k, 1.0, [], u, f"ties {levels}")
    lg = np.full(V, 1.5, np.float32)     # every value ties
    for k in (1, 50, 0):
        for u in (0.1, 0.6):
            _check(ds, lg, 1.0, k, 1.0, [], u, "all equal")


def test_device_sampler_special_values():
    """NaN or +inf anywhere: the sum is NaN and the draw falls through to
    V - 1; -inf logits are never drawn; temperature 0 gives the host's
    token (V - 1 through inf/NaN logits); -0 equals +0."""
    V = 4100
    rng = np.random.default_rng(5)
    ds = DeviceSampler(V)
    base = _logits(rng, V)
    for idx, val in ((17, np.nan), (4099, np.inf), (2048, -np.inf)):
        lg = base.copy()
        lg[idx] = val
        for k in (0, 10, 300):
            _check(ds, lg, 1.0, k, 1.0, [], 0.5, f"special {val}")
    lg = np.full(V, -np.inf, np.float32)
    _check(ds, lg, 1.0, 5, 1.0, [], 0.5, "all -inf")
    lg = base.copy()
    lg[::7] = -np.inf
    for k in (0, 5, 400):
        _check(ds, lg, 0.8, k, 1.2, [0, 7, 14, 3], 0.77, "some -inf")
    _check(ds, base, 0.0, 50, 1.0, [], 0.4, "T=0")
    lg = np.zeros(V, np.float32)
    lg[1::2] = -0.0
    lg[100] = 1.0
    for k in (1, 2, 3000):
        _check(ds, lg, 1.0, k, 1.0, [], 0.3, "signed zeros")


def test_device_sampler_long_window():
    """A window longer than the kernel's LDS stage (4096 ids) is read in
    place; duplicates still count once per occurrence."""
    V = 6000
    rng = np.random.default_rng(8)
    ds = DeviceSampler(V)
    lg = _logits(rng, V, 1.0)
    lg[:8] = 6.0
    rec = rng.integers(0, 8, 5000).astype(np.int32)   # the top 8 ids, many times each
    for pen in (1.0001, 1.05):
        for u in (0.1, 0.8):
            _check(ds, lg, 1.0, 20, pen, rec, u, "long window")


def test_engine_sampling_matches_host_each_step():
    """oxb_model_set_sampling: prefill and 40 decode steps whose tokens are
    drawn on the device (top-k 20, T 0.9, penalty 1.3 over the last 6 tokens)
    equal the host sampler on the logits each forward returns, with the
    window of lib.rs:156-161 and the draws u[i]."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    m = pkg.Model(path, max_seq=96)
    rng = np.random.default_rng(21)
    u = rng.random(64).astype(np.float32)
    u[3] = 0.0
    T, k, pen, last = 0.9, 20, 1.3, 6
    m.set_sampling(u, temperature=T, top_k=k, repeat_penalty=pen, repeat_last_n=last)
    prompt = rng.integers(0, cfg.vocab, 11).astype(np.int32)
    tok, lg = m.forward(prompt)
    toks = []
    for i in range(41):
        rec = toks[-last:] if last else toks
        want = host_sample(lg, T, k, pen, np.array(rec, np.int32), u[i])
        assert tok == want, (i, tok, want)
        toks.append(tok)
        if i < 40:
            tok, lg = m.step()
    # the steps fed back the drawn tokens: a greedy engine on the same ids
    # gives the same logits at the last step
    m.set_sampling(None)
    m2 = pkg.Model(path, max_seq=96)
    m2.forward(prompt)
    lg2 = None
    for t in toks[:-1]:
        m2.set_token(t)
        _, lg2 = m2.step()
    assert np.array_equal(lg2.view(np.uint32), lg.view(np.uint32))
    m.close()
    m2.close()


def test_engine_sampling_graph_steps():
    """decode through captured graphs with sampling on: the tokens of
    decode_greedy (sampled per step) equal the ones of single steps."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    rng = np.random.default_rng(4)
    u = rng.random(40).astype(np.float32)
    prompt = rng.integers(0, cfg.vocab, 9).astype(np.int32)
    runs = []
    for mode in ("graph", "step"):
        m = pkg.Model(path, max_seq=64)
        m.set_sampling(u, temperature=1.1, top_k=0, repeat_penalty=1.1, repeat_last_n=0)
        t0, _ = m.forward(prompt, want_logits=False)
        if mode == "graph":
            rest = m.decode_greedy(30).tolist()
        else:
            rest = [m.step(want_logits=False)[0] for _ in range(30)]
        runs.append([t0] + rest)
        m.close()
    assert runs[0] == runs[1]


def _generate(path, **opts):
    nat = pkg._native
    L = nat.lib()
    h = L.oxbitnet_load(path.encode(), None)
    assert h, L.oxbitnet_error_message()
    got = []
    tf = nat.TokenFn(lambda t, n, ud: (got.append(C.string_at(t, n)), 0)[1])
    g = L.oxbitnet_default_generate_options()
    for k, v in opts.items():
        setattr(g, k, v)
    assert L.oxbitnet_generate(h, b"hello there", C.byref(g), tf, None) == 0
    L.oxbitnet_free(h)
    return got


def test_generate_with_reference_defaults_streams_tokens():
    """oxbitnet_generate with the reference's defaults (top_k 50, T 1,
    penalty 1.1 over 64) runs on the device sampler and streams up to
    max_tokens pieces; stopping from the callback ends it early."""
    cfg = synth.small_config()
    path = synth.cached_gguf(cfg, seed=7)
    got = _generate(path, max_tokens=24)
    assert 1 <= len(got) <= 24
    nat = pkg._native
    L = nat.lib()
    h = L.oxbitnet_load(path.encode(), None)
    seen = []
    tf = nat.TokenFn(lambda t, n, ud: (seen.append(1), 1 if len(seen) == 3 else 0)[1])
    g = L.oxbitnet_default_generate_options()
    g.max_tokens = 20
    assert L.oxbitnet_generate(h, b"hello there", C.byref(g), tf, None) == 0
    assert len(seen) == 3
    # the handle generates again after an early stop
    g.top_k, g.repeat_penalty, g.max_tokens = 1, 1.0, 6
    seen.clear()
    assert L.oxbitnet_generate(h, b"hello there", C.byref(g), tf, None) == 0
    L.oxbitnet_free(h)
