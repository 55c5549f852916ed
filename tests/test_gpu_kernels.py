"""Parity of each HIP hot-path kernel against the CPU oracle, through the C ABI.

Bars: int8 activations, int32 accumulators and every f32 value the oracle
computes with the same operation sequence are compared bit for bit; the
attention and LM-head sums (different reduction order by design, f16 KV) are
compared with an explicit tolerance, tighter than the 1e-3 relative bound
the path is held to.
"""
import numpy as np
import pytest

import oracle as O
from helpers import ops, synth, ternary

pytestmark = pytest.mark.gpu


def _scale_config1(seed):
    # 1 / mean|m| of a seeded N(0, 0.02) master (the single-GEMV workload)
    m = np.random.default_rng([seed, 99]).standard_normal(1 << 16) * 0.02
    return float(np.float32(1.0 / np.abs(m).mean()))


def _gemv_case(N, K, seed):
    rng = np.random.default_rng(seed)
    w = ternary(rng, N, K)
    Wn = synth.i2s_pack(w)
    x = rng.standard_normal(K).astype(np.float32)
    q, s = O.quantize(x)
    return Wn, q[0], float(s[0])


# K = 4224: 66 chunks of 64, a ragged split over 8 waves; K = 65536: the maximum
@pytest.mark.parametrize("N,K", [(6912, 2560), (16, 128), (48, 384), (2560, 6912), (16, 4224),
                                 (32, 65536)])
def test_gemv_i8_bitexact(N, K):
    Wn, xq, xs = _gemv_case(N, K, seed=N + K)
    ws = np.full(N, _scale_config1(1), np.float32)
    acc_o, y_o = O.gemv(Wn, xq, ws, xs, K)
    Wt = ops.upload_ternary(Wn, K)
    acc, y = ops.gemv_i8(Wt, xq, xs, ws, N, K)
    assert np.array_equal(acc, acc_o)
    assert np.array_equal(y.view(np.uint32), y_o.view(np.uint32))


@pytest.mark.parametrize("N,K", [(28672, 8192), (8192, 28672)])
def test_gemv_i8_sweep_shapes(N, K):
    Wn, xq, xs = _gemv_case(N, K, seed=7)
    ws = np.full(N, 0.75, np.float32)
    acc_o, y_o = O.gemv(Wn, xq, ws, xs, K)
    Wt = ops.upload_ternary(Wn, K)
    acc, y = ops.gemv_i8(Wt, xq, xs, ws, N, K)
    assert np.array_equal(acc, acc_o)
    assert np.array_equal(y, y_o)


def test_gemv_extremes_and_zero():
    K = 28672
    N = 32
    w = np.ones((N, K), np.int8)
    w[1::2] = -1
    w[16:] = 0
    Wt = ops.upload_ternary(synth.i2s_pack(w), K)
    for xv in (127, -127):
        xq = np.full(K, xv, np.int8)
        acc, y = ops.gemv_i8(Wt, xq, 1.0, np.ones(N, np.float32), N, K)
        exp = np.where(np.arange(N) < 16, np.where(np.arange(N) % 2 == 0, 1, -1), 0) * xv * K
        assert np.array_equal(acc, exp)
    # the reference's known answer (ternary-gemv.test.ts:35-53): +-128 at K=128
    w2 = np.zeros((16, 128), np.int8)
    w2[0], w2[1] = 1, -1
    acc, y = ops.gemv_i8(ops.upload_ternary(synth.i2s_pack(w2), 128), np.ones(128, np.int8), 1.0,
                         np.ones(16, np.float32), 16, 128)
    assert acc[:2].tolist() == [128, -128] and y[:2].tolist() == [128.0, -128.0]
    assert not acc[2:].any()


def test_gemv_rejects_bad_shapes():
    Wt = ops.DeviceArray((1024,), np.uint8)
    with pytest.raises(ops.NativeError, match="multiple of 16"):
        ops.gemv_i8(Wt, np.zeros(128, np.int8), 1.0, np.ones(8, np.float32), 8, 128)
    with pytest.raises(ops.NativeError, match="multiple of 128"):
        ops.gemv_i8(Wt, np.zeros(64, np.int8), 1.0, np.ones(16, np.float32), 16, 64)


@pytest.mark.parametrize("K,N,norm,resid", [(2560, 2560, True, True), (6912, 2560, True, True),
                                            (2560, 6912, False, False), (2560, 640, True, False)])
def test_bitlinear_gemv_fused_norm_quant(K, N, norm, resid):
    rng = np.random.default_rng(K * 7 + N)
    w = ternary(rng, N, K)
    Wn = synth.i2s_pack(w)
    x = (rng.standard_normal(K) * 3).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32) if norm else None
    ws = np.full(N, 0.0163, np.float32)
    r = rng.standard_normal(N).astype(np.float32) if resid else None
    # oracle: rs/nn/bitlinear.rs:52-97 (eps 1e-5)
    h = O.rmsnorm(x, g, 1e-5) if norm else x[None]
    q, s = O.quantize(h)
    acc_o, y_o = O.gemv(Wn, q[0], ws, s[0], K)
    if resid:
        y_o = O.add(r, y_o)
    Wt = ops.upload_ternary(Wn, K)
    acc, y, xq, xs = ops.bitlinear_gemv(Wt, x, g, 1e-5, ws, N, K, residual=r)
    assert np.array_equal(xq, q[0])
    assert np.float32(xs) == s[0]
    assert np.array_equal(acc, acc_o)
    assert np.array_equal(y, y_o)


def test_norm_quant_rows_bitexact():
    rng = np.random.default_rng(11)
    for D in (2560, 6912, 16):
        x = (rng.standard_normal((5, D)) * rng.uniform(0.1, 10, (5, 1))).astype(np.float32)
        x[2] = 0.0  # all-zero row: scale 1, q 0 (quantize.test.ts:43-52)
        g = rng.uniform(0.5, 1.5, D).astype(np.float32)
        q, s, sm = ops.norm_quant_rows(x, g, 1e-5)
        qo, so = O.quantize(O.rmsnorm(x, g, 1e-5))
        assert np.array_equal(q, qo) and np.array_equal(s, so)
        assert np.array_equal(sm, qo.astype(np.int64).sum(1))
        q2, s2, _ = ops.norm_quant_rows(x, None, 0.0)
        qo2, so2 = O.quantize(x)
        assert np.array_equal(q2, qo2) and np.array_equal(s2, so2)


def test_gateup_fused_bitexact():
    rng = np.random.default_rng(12)
    K, F = 2560, 6912
    wg, wu = ternary(rng, F, K), ternary(rng, F, K)
    inter = np.empty((2 * F, K), np.int8)
    inter[0::2], inter[1::2] = wg, wu
    ws = np.empty(2 * F, np.float32)
    ws[0::2], ws[1::2] = 0.0151, 0.0172
    x = rng.standard_normal(K).astype(np.float32) * 5
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    q, s = O.quantize(O.rmsnorm(x, g, 1e-5))
    _, yg = O.gemv(synth.i2s_pack(wg), q[0], 0.0151, s[0], K)
    _, yu = O.gemv(synth.i2s_pack(wu), q[0], 0.0172, s[0], K)
    h_o = O.mul(O.relu2(yg), yu)  # rs/nn/ffn.rs:60-80
    h = ops.bitlinear_gateup(ops.upload_ternary(synth.i2s_pack(inter), K), x, g, 1e-5, ws, 2 * F, K)
    assert np.array_equal(h, h_o)


def rope_table(max_seq, hd, theta):
    cs = np.zeros((max_seq, hd // 2, 2), np.float32)
    ops.check(ops.lib().oxb_rope_table(cs.ctypes.data, max_seq, hd, theta), "rope")
    return cs


def test_rope_table_matches_oracle():
    cs = rope_table(300, 128, 500000.0)
    unit = np.zeros((300, 1, 128), np.float32)
    unit[:, :, 0::2] = 1.0
    for p in (0, 1, 17, 299):
        y = O.rope(unit[p].reshape(-1), 1, 1, 128, p, 500000.0).reshape(64, 2)
        assert np.array_equal(cs[p], y), p


def test_qkv_rope_kv_append():
    rng = np.random.default_rng(13)
    K, H, Hkv, hd, S = 2560, 20, 5, 128, 64
    Dq, Dkv = H * hd, Hkv * hd
    wq, wk, wv = ternary(rng, Dq, K), ternary(rng, Dkv, K), ternary(rng, Dkv, K)
    sq, sk, sv = 0.016, 0.017, 0.015
    x = rng.standard_normal(K).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    pos = 37
    # oracle: three BitLinears on the same normed input, RoPE at pos
    h = O.rmsnorm(x, g, 1e-5)
    q8, s8 = O.quantize(h)
    _, q = O.gemv(synth.i2s_pack(wq), q8[0], sq, s8[0], K)
    _, k = O.gemv(synth.i2s_pack(wk), q8[0], sk, s8[0], K)
    _, v = O.gemv(synth.i2s_pack(wv), q8[0], sv, s8[0], K)
    qr = O.rope(q, 1, H, hd, pos, 500000.0)
    kr = O.rope(k, 1, Hkv, hd, pos, 500000.0)
    fused = np.concatenate([wq, wk, wv])
    ws = np.concatenate([np.full(Dq, sq), np.full(Dkv, sk), np.full(Dkv, sv)]).astype(np.float32)
    Wt = ops.upload_ternary(synth.i2s_pack(fused), K)
    dx = ops.DeviceArray.from_host(x)
    dg = ops.DeviceArray.from_host(g)
    dws = ops.DeviceArray.from_host(ws)
    dq = ops.DeviceArray((Dq,), np.float32)
    kc = ops.DeviceArray((Hkv * S * hd,), np.uint16, zero=True)
    vc = ops.DeviceArray((Hkv * S * hd,), np.uint16, zero=True)
    rope = ops.DeviceArray.from_host(rope_table(S, hd, 500000.0))
    dpos = ops.DeviceArray.from_host(np.array([pos], np.int32))
    ops.check(ops.lib().oxb_bitlinear_qkv(Wt.ptr, dx.ptr, dg.ptr, 1e-5, dws.ptr, Dq, Dkv, hd, K,
                                          dq.ptr, kc.ptr, vc.ptr, S, rope.ptr, dpos.ptr, None), "qkv")
    ops.sync()
    assert np.array_equal(dq.download(), qr)
    kh = kc.download().view(np.float16).reshape(Hkv, S, hd)
    vh = vc.download().view(np.float16).reshape(Hkv, S, hd)
    assert np.array_equal(kh[:, pos].reshape(-1), kr.astype(np.float16))
    assert np.array_equal(vh[:, pos].reshape(-1), v.astype(np.float16))
    mask = np.ones(S, bool)
    mask[pos] = False
    assert not kh[:, mask].any() and not vh[:, mask].any()


def _oracle_attn(q, kc16, vc16, n, S, H, Hkv, hd):
    # caches [Hkv][S][hd] f16 -> the reference layout [S][Hkv][hd] f32
    k = kc16[:, :S].astype(np.float32).transpose(1, 0, 2).copy()
    v = vc16[:, :S].astype(np.float32).transpose(1, 0, 2).copy()
    return O.attention(q, k, v, n, S, H, Hkv, hd)


# The two-launch decode attention (scores, then softmax and one P.V chain per
# output over an LDS ring of 64-row V slots): first slot, slot edges (63/64,
# 127/128), the ring wrapping (319/320 with five slots), G = 4, 2, 1 and 8 (two
# groups of four heads per KV head), caches past 4864 rows (three slots),
# lengths not a multiple of 4 (per-element score loads)
@pytest.mark.parametrize("pos,H,Hkv,S", [(0, 20, 5, 512), (63, 20, 5, 512), (64, 20, 5, 512),
                                         (127, 20, 5, 512), (128, 20, 5, 512),
                                         (200, 20, 5, 512), (319, 20, 5, 512), (320, 20, 5, 512),
                                         (511, 20, 5, 512), (300, 8, 8, 4096),
                                         (700, 16, 8, 1024), (4095, 20, 5, 4096), (100, 16, 2, 256),
                                         (1500, 32, 4, 2048), (2599, 20, 5, 2600),
                                         (6143, 20, 5, 6144), (4999, 16, 4, 5000),
                                         (200, 20, 5, 515), (514, 20, 5, 515)])
def test_attn_decode_bitexact(pos, H, Hkv, S):
    rng = np.random.default_rng(pos + H)
    hd = 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = (rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, S, hd)).astype(np.float16)
    out = ops.attn_decode(q, kc, vc, pos, H, Hkv, hd, S)
    ref = _oracle_attn(q, kc, vc, 1, pos + 1, H, Hkv, hd)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_attn_decode_rejects_caches_past_its_lds():
    with pytest.raises(ops.NativeError, match="max_seq"):
        ops.attn_decode(np.zeros(20 * 128, np.float32), np.zeros((5, 6145, 128), np.float16),
                        np.zeros((5, 6145, 128), np.float16), 10, 20, 5, 128, 6145)


def _nan_past(c, pos):
    """Cache rows at and past pos + 1 filled with f16 NaN and +-Inf: no form
    may read a value of them into a result."""
    c = c.copy()
    tail = c[..., pos + 1:, :]
    pat = np.array([0x7e00, 0x7c00, 0xfc00, 0xfe01], np.uint16).view(np.float16)
    tail[...] = np.resize(pat, tail.shape)
    return c


@pytest.mark.parametrize("form,pos,S", [("split", 100, 512), ("split", 300, 700),
                                        ("head", 100, 512), ("head", 255, 512),
                                        ("head", 300, 512), ("head", 20, 64),
                                        ("fused", 100, 512), ("fused", 300, 600),
                                        ("head8", 100, 512), ("head8", 250, 300),
                                        ("head8", 300, 512), ("head8", 400, 404),
                                        ("split8", 100, 512), ("split8", 1000, 1100)])
def test_attn_decode_ignores_nonfinite_rows_past_the_position(form, pos, S):
    """Rows past the position hold NaN/Inf (stale or never-written cache rows
    of a caller): every decode form gives the oracle's bits over the rows it
    may use."""
    H, Hkv, hd = 20, 5, 128
    rng = np.random.default_rng(pos + S)
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = _nan_past((rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16), pos)
    vc = _nan_past(rng.standard_normal((Hkv, S, hd)).astype(np.float16), pos)
    kw = {"head": dict(head=True, s_max=256 if pos < 256 else 512), "fused": dict(fused=True),
          "split": {}, "head8": dict(head=True, s_max=256 if pos < 256 else 512, octets=True),
          "split8": dict(octets=True)}[form]
    out = ops.attn_decode(q, kc, vc, pos, H, Hkv, hd, S, **kw)
    ref = _oracle_attn(q, kc, vc, 1, pos + 1, H, Hkv, hd)
    assert np.isfinite(ref).all()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("pos,H,Hkv,S", [(0, 20, 5, 512), (63, 20, 5, 512), (255, 20, 5, 512),
                                         (256, 20, 5, 512), (300, 20, 5, 408), (511, 20, 5, 512),
                                         (700, 8, 4, 1024), (1500, 20, 5, 4096),
                                         (4095, 20, 5, 4096), (129, 4, 4, 256),
                                         # K chunk pairs (512 rows) and V chunk pairs exactly,
                                         # and one past
                                         (511, 20, 5, 1024), (512, 20, 5, 1024),
                                         (767, 20, 5, 1024), (1023, 20, 5, 1024),
                                         # odd lengths: P.V tails of 1..15 positions
                                         (6, 20, 5, 64), (98, 20, 5, 99)])
def test_attn_decode_fused_bitexact(pos, H, Hkv, S):
    """One-kernel decode attention: same bits as the oracle (and the split path)."""
    assert ops.lib().oxb_attn_decode_fused_supported(H, Hkv, 128, S)
    rng = np.random.default_rng(pos * 7 + H)
    hd = 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = (rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, S, hd)).astype(np.float16)
    out = ops.attn_decode(q, kc, vc, pos, H, Hkv, hd, S, fused=True)
    ref = _oracle_attn(q, kc, vc, 1, pos + 1, H, Hkv, hd)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("pos,H,Hkv,S,s_max", [
    # one position group (up to 256): empty P.V tail, whole and partial chunks
    (0, 20, 5, 512, 256), (3, 20, 5, 512, 256), (63, 20, 5, 512, 256), (64, 20, 5, 512, 256),
    (127, 20, 5, 512, 256), (128, 20, 5, 300, 256), (139, 20, 5, 400, 256),
    (255, 20, 5, 256, 256),
    # 257 .. 512 positions (one chain through both 256-row halves)
    (256, 20, 5, 512, 512), (300, 20, 5, 512, 512), (383, 20, 5, 384, 512),
    (511, 20, 5, 512, 512), (10, 20, 5, 512, 512), (400, 16, 2, 512, 512),
    (290, 8, 8, 300, 512),
    # other GQA groups; short caches (K rows clamped to the cache extent)
    (200, 8, 8, 512, 256), (100, 16, 2, 256, 256), (40, 32, 4, 64, 256), (63, 20, 5, 64, 256),
    (20, 4, 1, 21, 256)])
@pytest.mark.parametrize("octets", [False, True])
def test_attn_decode_head_bitexact(pos, H, Hkv, S, s_max, octets):
    """Per-query-head decode attention: same bits as the oracle, with the
    row-major V and with its octet copy."""
    rng = np.random.default_rng(pos * 11 + H + s_max)
    hd = 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = (rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, S, hd)).astype(np.float16)
    out = ops.attn_decode(q, kc, vc, pos, H, Hkv, hd, S, head=True, s_max=s_max, octets=octets)
    ref = _oracle_attn(q, kc, vc, 1, pos + 1, H, Hkv, hd)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_attn_decode_head_batch_bitexact():
    """The per-head kernel over a batch of sequences (grid y), each its own
    cache and position."""
    B, H, Hkv, S, hd = 5, 20, 5, 448, 128
    rng = np.random.default_rng(97)
    q = rng.standard_normal((B, H * hd)).astype(np.float32)
    kc = (rng.standard_normal((B, Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((B, Hkv, S, hd)).astype(np.float16)
    pos = np.array([447, 0, 255, 256, 100], np.int32)
    st = np.zeros((B, 8), np.int32)
    st[:, 0] = pos
    L = ops.lib()
    pad = np.zeros(ops.KV_PAD_ROWS * hd, np.uint16)
    dq = ops.DeviceArray.from_host(q)
    dk = ops.DeviceArray.from_host(np.concatenate([kc.view(np.uint16).reshape(-1), pad]))
    dv = ops.DeviceArray.from_host(np.concatenate([vc.view(np.uint16).reshape(-1), pad]))
    dst = ops.DeviceArray.from_host(st)
    out = ops.DeviceArray((B, H * hd), np.float32)
    ops.check(L.oxb_attn_decode_head(dq.ptr, dk.ptr, dv.ptr, dst.ptr, 8, Hkv * S * hd, B, H, Hkv,
                                     hd, S, 512, out.ptr, None), "attn_decode_head")
    ops.sync()
    got = out.download()
    for z in range(B):
        ref = _oracle_attn(q[z], kc[z], vc[z], 1, int(pos[z]) + 1, H, Hkv, hd)
        assert np.array_equal(got[z].view(np.uint32), ref.view(np.uint32)), f"slot {z}"
    # the 256-position kernel over the octet copy (positions below 256)
    v8 = ops.v_octets(vc)
    dv8 = ops.DeviceArray.from_host(v8)
    st[:, 0] = np.array([255, 0, 254, 128, 100], np.int32)
    dst.upload(st)
    ops.check(L.oxb_attn_decode_head_v8(dq.ptr, dk.ptr, dv.ptr, dv8.ptr, dst.ptr, 8, Hkv * S * hd,
                                        v8.shape[-1], B, H, Hkv, hd, S, 256, out.ptr, None),
              "attn_decode_head_v8")
    ops.sync()
    got = out.download()
    for z in range(B):
        ref = _oracle_attn(q[z], kc[z], vc[z], 1, int(st[z, 0]) + 1, H, Hkv, hd)
        assert np.array_equal(got[z].view(np.uint32), ref.view(np.uint32)), f"octets, slot {z}"


def test_attn_decode_head_rejects_long_caches():
    with pytest.raises(ops.NativeError, match="s_max"):
        ops.attn_decode(np.zeros(20 * 128, np.float32), np.zeros((5, 600, 128), np.float16),
                        np.zeros((5, 600, 128), np.float16), 599, 20, 5, 128, 600, head=True,
                        s_max=600)


# (28, 20, 5, 3800): both halves per workgroup with its LDS nearly full;
# (28, 20, 5, 3840): one row more than that LDS holds (the per-half kernel)
@pytest.mark.parametrize("B,H,Hkv,S", [(2, 20, 5, 512), (16, 20, 5, 1024), (40, 16, 4, 256),
                                       (9, 8, 8, 512), (8, 16, 8, 2600), (7, 20, 5, 1001),
                                       (32, 20, 5, 2560), (3, 32, 4, 700), (12, 64, 8, 1500),
                                       (10, 16, 8, 300), (28, 20, 5, 3800), (28, 20, 5, 3840)])
def test_attn_decode_batch_bitexact(B, H, Hkv, S):
    """Batched decode attention (per-slot caches and positions): every slot
    equals the oracle."""
    rng = np.random.default_rng(B * 13 + H)
    hd = 128
    q = rng.standard_normal((B, H * hd)).astype(np.float32)
    kc = (rng.standard_normal((B, Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((B, Hkv, S, hd)).astype(np.float16)
    pos = rng.integers(0, S, B).astype(np.int32)
    pos[0] = S - 1
    st = np.zeros((B, 8), np.int32)
    st[:, 0] = pos
    L = ops.lib()
    dq = ops.DeviceArray.from_host(q)
    dk = ops.DeviceArray.from_host(kc.view(np.uint16))
    dv = ops.DeviceArray.from_host(vc.view(np.uint16))
    dst = ops.DeviceArray.from_host(st)
    sc = ops.DeviceArray((B * H * S,), np.float32)
    out = ops.DeviceArray((B, H * hd), np.float32)
    ops.check(L.oxb_attn_decode_batch(dq.ptr, dk.ptr, dv.ptr, dst.ptr, 8, Hkv * S * hd, B, H,
                                      Hkv, hd, S, sc.ptr, out.ptr, None), "attn_decode_batch")
    ops.sync()
    got = out.download()
    # the same with the octet copy of V (read by batches of up to 8)
    v8 = ops.v_octets(vc)
    dv8 = ops.DeviceArray.from_host(v8)
    out8 = ops.DeviceArray((B, H * hd), np.float32)
    ops.check(L.oxb_attn_decode_batch_v8(dq.ptr, dk.ptr, dv.ptr, dv8.ptr, dst.ptr, 8,
                                         Hkv * S * hd, v8.shape[-1], B, H, Hkv, hd, S, sc.ptr,
                                         out8.ptr, None), "attn_decode_batch_v8")
    ops.sync()
    got8 = out8.download()
    for z in range(B):
        ref = _oracle_attn(q[z], kc[z], vc[z], 1, int(pos[z]) + 1, H, Hkv, hd)
        assert np.array_equal(got[z].view(np.uint32), ref.view(np.uint32)), f"slot {z}"
        assert np.array_equal(got8[z].view(np.uint32), ref.view(np.uint32)), f"octets, slot {z}"


@pytest.mark.parametrize("poss", [[0, 127, 128, 2303], [7, 8, 136, 255], [1023, 1024, 129, 15],
                                  [2559, 2047, 2048, 1]])
def test_attn_decode_octets_register_stream_edges(poss):
    """Three or more sequences read V straight into registers (a ring of 16
    octets): every slot at the edges of an octet and of the ring (128
    positions), the first position and the longest cache, bit-equal to the
    oracle."""
    B, H, Hkv, hd, S = len(poss), 20, 5, 128, 2560
    rng = np.random.default_rng(sum(poss))
    q = rng.standard_normal((B, H * hd)).astype(np.float32)
    kc = (rng.standard_normal((B, Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((B, Hkv, S, hd)).astype(np.float16)
    pos = np.array(poss, np.int32)
    st = np.zeros((B, 8), np.int32)
    st[:, 0] = pos
    v8 = ops.v_octets(vc)
    o = v8.reshape(B, Hkv, -1, hd, 8).view(np.float16)
    for z in range(B):   # positions past each slot's own: NaN (never summed)
        for s_ in range(int(pos[z]) + 1, S):
            o[z, :, s_ // 8, :, s_ % 8] = np.nan
    L = ops.lib()
    dq = ops.DeviceArray.from_host(q)
    dk = ops.DeviceArray.from_host(kc.view(np.uint16))
    dv = ops.DeviceArray.from_host(vc.view(np.uint16))
    dv8 = ops.DeviceArray.from_host(v8)
    dst = ops.DeviceArray.from_host(st)
    sc = ops.DeviceArray((B * H * S,), np.float32)
    out = ops.DeviceArray((B, H * hd), np.float32)
    ops.check(L.oxb_attn_decode_batch_v8(dq.ptr, dk.ptr, dv.ptr, dv8.ptr, dst.ptr, 8, Hkv * S * hd,
                                         v8.shape[-1], B, H, Hkv, hd, S, sc.ptr, out.ptr, None),
              "attn_decode_batch_v8")
    ops.sync()
    got = out.download()
    for z in range(B):
        ref = _oracle_attn(q[z], kc[z], vc[z], 1, int(pos[z]) + 1, H, Hkv, hd)
        assert np.array_equal(got[z].view(np.uint32), ref.view(np.uint32)), f"slot {z}"


@pytest.mark.parametrize("S,pos", [(8, 0), (8, 7), (9, 8), (16, 9), (128, 127), (129, 128),
                                   (300, 255), (300, 256), (1000, 999), (2560, 2303),
                                   (4099, 4098), (6144, 6143), (6144, 130)])
def test_attn_decode_octets_ring_edges(S, pos):
    """The octet P.V kernel at the edges of its octets (8 positions) and ring
    slots (128), a cache not a multiple of 8 long and the longest cache:
    bit-equal to the oracle; its entry point also rejects a missing copy."""
    rng = np.random.default_rng(S + 7 * pos)
    H, Hkv, hd = 20, 5, 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = (rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, S, hd)).astype(np.float16)
    L = ops.lib()
    dq = ops.DeviceArray.from_host(q)
    dk = ops.DeviceArray.from_host(kc.view(np.uint16))
    dv = ops.DeviceArray.from_host(vc.view(np.uint16))
    v8 = ops.v_octets(vc)
    # positions past pos in the copy hold NaN: they must never be summed
    o = v8.view(np.float16).reshape(Hkv, -1, hd, 8)
    for s in range(pos + 1, (S + 7) // 8 * 8):
        o[:, s // 8, :, s % 8] = np.nan
    dv8 = ops.DeviceArray.from_host(v8)
    dpos = ops.DeviceArray.from_host(np.array([pos], np.int32))
    sc = ops.DeviceArray((H * S,), np.float32)
    out = ops.DeviceArray((H * hd,), np.float32)
    ops.check(L.oxb_attn_decode_batch_v8(dq.ptr, dk.ptr, dv.ptr, dv8.ptr, dpos.ptr, 0, 0, 0, 1, H,
                                         Hkv, hd, S, sc.ptr, out.ptr, None), "attn v8")
    ops.sync()
    ref = _oracle_attn(q, kc, vc, 1, pos + 1, H, Hkv, hd)
    assert np.array_equal(out.download().view(np.uint32), ref.view(np.uint32))
    assert L.oxb_attn_decode_batch_v8(dq.ptr, dk.ptr, dv.ptr, None, dpos.ptr, 0, 0, 0, 1, H, Hkv,
                                      hd, S, sc.ptr, out.ptr, None) == -1


# The one-launch q|k|v + attention step against the two launches it replaces
# (oxb_bitlinear_qkv, then oxb_attn_decode_head_v8 over the octet copy):
# hidden 512 and 2560, 1 to 4 query heads per KV head, KV heads not a multiple
# of 8 (idle workgroups), first position, octet edges (7 / 8), the last of 256
# positions, caches longer than 256 rows, and a position past 256 (append
# only).  Rows past the position hold NaN / Inf.
@pytest.mark.parametrize("D,H,Hkv,max_seq,pos", [(512, 4, 1, 256, 0), (512, 4, 1, 256, 7),
                                                 (512, 4, 1, 300, 8), (512, 8, 2, 256, 255),
                                                 (512, 9, 9, 256, 50), (2560, 20, 5, 256, 0),
                                                 (2560, 20, 5, 512, 100), (2560, 20, 5, 300, 37),
                                                 (2560, 20, 5, 4096, 255), (2560, 32, 8, 256, 200),
                                                 (2560, 20, 5, 300, 280)])
def test_qkv_attn_decode_matches_two_launches(D, H, Hkv, max_seq, pos):
    rng = np.random.default_rng(D + 31 * pos + H)
    hd = 128
    Dq, Dkv = H * hd, Hkv * hd
    N = Dq + 2 * Dkv
    W = ternary(rng, N, D)
    ws = rng.uniform(0.01, 0.03, N).astype(np.float32)
    x = rng.standard_normal(D).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    kc = (rng.standard_normal((Hkv, max_seq, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, max_seq, hd)).astype(np.float16)
    kc, vc = _nan_past(kc, pos - 1), _nan_past(vc, pos - 1)   # rows pos.. stale
    L = ops.lib()
    Wt = ops.upload_ternary(synth.i2s_pack(W), D)
    dx, dg, dws = (ops.DeviceArray.from_host(a) for a in (x, g, ws))
    rope = ops.DeviceArray.from_host(rope_table(max_seq, hd, 500000.0))
    dpos = ops.DeviceArray.from_host(np.array([pos], np.int32))

    # the two launches
    dq = ops.DeviceArray((Dq,), np.float32)
    rk = ops.DeviceArray.from_host(kc.view(np.uint16))
    rv = ops.DeviceArray.from_host(vc.view(np.uint16))
    ops.check(L.oxb_bitlinear_qkv(Wt.ptr, dx.ptr, dg.ptr, 1e-5, dws.ptr, Dq, Dkv, hd, D, dq.ptr,
                                  rk.ptr, rv.ptr, max_seq, rope.ptr, dpos.ptr, None), "qkv")
    ops.sync()
    kc1 = rk.download().view(np.float16).reshape(Hkv, max_seq, hd)
    vc1 = rv.download().view(np.float16).reshape(Hkv, max_seq, hd)
    if pos < 256:
        want = ops.attn_decode(dq.download(), kc1, vc1, pos, H, Hkv, hd, max_seq, head=True,
                               s_max=256, octets=True)
        ref = _oracle_attn(dq.download(), kc1, vc1, 1, pos + 1, H, Hkv, hd)
        assert np.array_equal(want.view(np.uint32), ref.view(np.uint32))
    else:
        want = np.full(H * hd, 7.5, np.float32)   # the output is left as it was

    # the one launch, twice (its counters are zero again after each)
    cnt = ops.DeviceArray((H,), np.int32, zero=True)
    for rep in range(2):
        fk = ops.DeviceArray.from_host(kc.view(np.uint16))
        fv = ops.DeviceArray.from_host(vc.view(np.uint16))
        fv8 = ops.DeviceArray.from_host(ops.v_octets(vc))
        fq = ops.DeviceArray((Dq,), np.float32)
        out = ops.DeviceArray.from_host(np.full(H * hd, 7.5, np.float32))
        ops.check(L.oxb_qkv_attn_decode(Wt.ptr, dws.ptr, dx.ptr, dg.ptr, 1e-5, rope.ptr, dpos.ptr,
                                        fq.ptr, fk.ptr, fv.ptr, fv8.ptr, cnt.ptr, H, Hkv, hd, D,
                                        max_seq, out.ptr, None), "qkv_attn")
        ops.sync()
        assert not cnt.download().any()
        assert np.array_equal(fq.download().view(np.uint32), dq.download().view(np.uint32))
        assert np.array_equal(out.download().view(np.uint32), want.view(np.uint32)), rep
    assert np.array_equal(fk.download().reshape(-1), kc1.view(np.uint16).reshape(-1))
    assert np.array_equal(fv.download().reshape(-1), vc1.view(np.uint16).reshape(-1))
    assert np.array_equal(fv8.download(), ops.v_octets(vc1))


def test_qkv_attn_decode_rejects_unsupported():
    L = ops.lib()
    for D, H, Hkv, hd, max_seq in ((1024, 8, 2, 128, 256), (2560, 20, 5, 128, 255),
                                   (2560, 20, 5, 64, 256), (2560, 20, 6, 128, 256)):
        rc = L.oxb_qkv_attn_decode(8, 8, 8, 8, 1e-5, 8, 8, 8, 8, 8, 8, 8, H, Hkv, hd, D, max_seq,
                                   8, None)
        assert rc == -1
        assert b"unsupported" in L.oxb_last_error() or b"head_dim" in L.oxb_last_error()


def test_attn_decode_fused_rejects_unsupported():
    L = ops.lib()
    assert not L.oxb_attn_decode_fused_supported(32, 4, 128, 512)     # 8 heads per KV head
    assert not L.oxb_attn_decode_fused_supported(20, 5, 64, 512)      # head_dim 64
    assert not L.oxb_attn_decode_fused_supported(20, 5, 128, 1 << 16)  # LDS
    with pytest.raises(ops.NativeError, match="unsupported shape"):
        ops.attn_decode(np.zeros(32 * 128, np.float32), np.zeros((4, 8, 128), np.float16),
                        np.zeros((4, 8, 128), np.float16), 3, 32, 4, 128, 8, fused=True)


# Rows up to 2368 positions run on the f32-MFMA kernel (16 score rows per
# workgroup: 16/G queries, so for G = 1 and 2 the four rows of one P.V chain
# group have different lengths; ragged last blocks; (0, 257) pairs rows of 256
# and 257 positions; rows shorter than a 16-position batch), longer ones on
# the VALU kernel (G = 4 and 8 take query pairs, G = 1, 2 one query per
# workgroup)
@pytest.mark.parametrize("H,Hkv,S,pos0,n", [(20, 5, 256, 30, 100), (20, 5, 512, 0, 257),
                                            (16, 2, 1200, 900, 31), (8, 8, 300, 5, 40),
                                            (16, 8, 300, 100, 33), (20, 5, 2100, 2040, 9),
                                            (20, 5, 64, 0, 1), (4, 4, 64, 0, 19),
                                            (8, 4, 200, 13, 37), (4, 4, 300, 250, 11),
                                            # 1001 queries over 4 P.V blocks, a lone last query
                                            (20, 5, 1100, 50, 1001),
                                            # the longest rows the MFMA kernel takes
                                            (20, 5, 2368, 2300, 68),
                                            # VALU kernel: rows past 2368 positions
                                            (20, 5, 2600, 2369, 30), (16, 8, 3000, 2900, 17),
                                            (8, 8, 2500, 2450, 11)])
def test_attn_prefill_causal_bitexact(H, Hkv, S, pos0, n):
    rng = np.random.default_rng(21 + n)
    hd = 128
    q = rng.standard_normal((n, H * hd)).astype(np.float32)
    kc = (rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, S, hd)).astype(np.float16)
    out = ops.attn_prefill(q, kc, vc, n, pos0, H, Hkv, hd, S)
    ref = _oracle_attn(q.reshape(-1), kc, vc, n, pos0 + n, H, Hkv, hd).reshape(n, H * hd)
    assert np.array_equal(out, ref)


# n > 64: the DMA-staged 256x128 kernel (8192 x 1024 with one K stage; 8192 x
# 1000 and 8192 x 900 with 10 and 3 stages and a ragged last token tile), the
# LDS-staged kernel at 128x128 (4224, 1024), 128x64 (6912, 512), 64x128 with a
# ragged last token tile (4032, 650), the DMA-staged 64x64 kernel with 4
# buffers (2560 x 512 with 27 stages; 2 and 3 stages, fewer than it prefetches,
# with ragged token tiles) -- and the register-tiled kernel for N % 64 != 0
# (32, 65)
@pytest.mark.parametrize("N,K,n", [(6912, 2560, 512), (2560, 6912, 512), (640, 2560, 7),
                                   (32, 256, 65), (8192, 256, 1024), (4224, 256, 1024),
                                   (4032, 256, 650), (8192, 2560, 1000), (8192, 768, 900),
                                   (2560, 512, 100), (1024, 768, 70),
                                   # n <= 64: the skinny kernel, 1..4 token tiles, 1 or 2
                                   # feature tiles per workgroup, uneven K splits over waves
                                   (2560, 6912, 8), (3840, 2560, 16), (2560, 2560, 32),
                                   (8192, 2560, 40), (8192, 512, 64), (256, 1280, 64),
                                   (96, 256, 1),
                                   # 4 / 2 feature tiles per workgroup at 1-4 token tiles
                                   (16384, 512, 8), (28672, 256, 20), (8192, 1024, 16),
                                   (16384, 512, 40), (28672, 256, 64),
                                   # few tiles for the CUs: one ragged token tile over 27
                                   # K stages; 30 and 40 256x128 tiles' worth; 160 of them
                                   # (5/8 of the CUs) with a ragged last token tile
                                   (2560, 6912, 65), (2560, 2560, 300), (5120, 4096, 200),
                                   (2560, 2560, 2000)])
def test_gemm_mfma_bitexact(N, K, n):
    rng = np.random.default_rng(N + n)
    w = ternary(rng, N, K)
    Wn = synth.i2s_pack(w)
    x = rng.standard_normal((n, K)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    ws = np.full(N, 0.0158, np.float32)
    q, s = O.quantize(O.rmsnorm(x, g, 1e-5))
    acc_o, Y_o = O.gemm(Wn, q, ws, s, K)
    Wt = ops.upload_ternary(Wn, K)
    acc, Y, sc = ops.gemm(Wt, x, g, 1e-5, ws, N, K)
    assert np.array_equal(sc, s)
    assert np.array_equal(acc, acc_o)
    assert np.array_equal(Y, Y_o)


# the split GEMMs' arrival counters: a fixed area at the start of a workspace
CNT_BYTES = 16384


def _tiled_rows(q, s, n, K):
    """The oracle's int8 rows on the device in the GEMM's token-tiled layout
    [n/16][K/256][4 planes][4 chunks][16 tokens][16 B], k = stage*256 +
    (c//2)*128 + g*32 + (c%2)*16 + j (rows this long exceed the fused
    quantizer, D <= 7168); a partial token tile is padded with zero rows
    (scale 1, sum 0), as the device quantizer pads it.  Returns (X, scales,
    sums) device arrays."""
    n16 = (n + 15) // 16 * 16
    qp = np.zeros((n16, K), np.int8)
    qp[:n] = q
    sp = np.ones(n16, np.float32)
    sp[:n] = s
    tiles = qp.reshape(n16 // 16, 16, K // 256, 2, 4, 2, 16).transpose(0, 2, 4, 3, 5, 1, 6)
    return (ops.DeviceArray.from_host(np.ascontiguousarray(tiles).reshape(-1)),
            ops.DeviceArray.from_host(sp),
            ops.DeviceArray.from_host(qp.astype(np.int64).sum(axis=1).astype(np.int32)))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("N,K,n", [(28672, 8192, 8), (28672, 8192, 64), (8192, 28672, 8),
                                   (8192, 28672, 64), (28672, 8192, 512), (8192, 28672, 512),
                                   (28672, 8192, 4096), (8192, 28672, 4096)])
def test_gemm_sweep_shapes_bitexact(N, K, n):
    """The ternary matmul sweep at full size: the skinny kernel (8 and 64
    tokens), the 128x128 LDS-staged or 256x128 DMA-staged kernels (512 and 4096
    tokens, 32 and 112 K stages): int32 accumulators and outputs equal the
    oracle's.  Where the shape splits over K with a workspace (8192 x 28672:
    at 512 tokens 128 tiles in 2 pieces; at 8 and 64 tokens the skinny
    kernel's 128 feature groups in 2 pieces), the split runs too, twice on
    one workspace, with the same results and its counters back at zero."""
    rng = np.random.default_rng(N + K + n)
    w = ternary(rng, N, K)
    Wn = synth.i2s_pack(w)
    x = rng.standard_normal((n, K)).astype(np.float32)
    ws = np.full(N, 0.0131, np.float32)
    q, s = O.quantize(x)
    acc_o, Y_o = O.gemm(Wn, q, ws, s, K)
    L = ops.lib()
    Wt = ops.upload_ternary(Wn, K)
    dX, dsc, dsm = _tiled_rows(q, s, n, K)
    dws = ops.DeviceArray.from_host(ws)
    Y = ops.DeviceArray((n, N), np.float32)
    acc = ops.DeviceArray((n, N), np.int32)
    ops.check(L.oxb_gemm_i8(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, n, Y.ptr, acc.ptr, 0,
                            None), "gemm_i8")
    ops.sync()
    assert np.array_equal(acc.download(), acc_o)
    assert np.array_equal(Y.download(), Y_o)
    wsb = L.oxb_gemm_ws_bytes(N, K, n)
    assert (wsb > 0) == ((N, K) == (8192, 28672) and n <= 512)
    if wsb:
        work = ops.DeviceArray((wsb,), np.uint8, zero=True)
        for _ in range(2):
            Y2 = ops.DeviceArray((n, N), np.float32)
            acc2 = ops.DeviceArray((n, N), np.int32)
            ops.check(L.oxb_gemm_i8_ws(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, n, Y2.ptr,
                                       acc2.ptr, 0, work.ptr, wsb, None), "gemm_i8_ws")
            ops.sync()
            assert np.array_equal(acc2.download(), acc_o)
            assert np.array_equal(Y2.download(), Y_o)
            assert not np.frombuffer(work.download()[:CNT_BYTES].tobytes(), np.int32).any()


@pytest.mark.parametrize("n", [130, 512, 40, 64])
def test_gemm_split_k_epilogues(n):
    """The split-K kernels on 5120 x 8192 with the store, residual and
    gate|up epilogues: 130 tokens on 64 x 64 tiles (240 tiles in 2 pieces of
    16 K stages), 512 on the 256 x 128 tiles (80 tiles in 2 pieces), 40 and
    64 tokens on the skinny kernel (80 feature groups of 64 rows, each in 3
    pieces); ragged token counts (130: a token tile of 2 real rows; 40: of 8)
    included.  Each equals the oracle bit for bit, on two calls sharing one
    workspace, and the arrival counters are zero after each call.  Calls with
    a workspace too small, or none, run unsplit with the same bits."""
    rng = np.random.default_rng(5120 + n)
    N, K = 5120, 8192
    L = ops.lib()
    wsb = L.oxb_gemm_ws_bytes(N, K, n)
    assert wsb > 0
    w = ternary(rng, N, K)
    Wn = synth.i2s_pack(w)
    x = rng.standard_normal((n, K)).astype(np.float32)
    wsc = rng.uniform(0.01, 0.02, N).astype(np.float32)
    q, s = O.quantize(x)
    acc_o, Y_o = O.gemm(Wn, q, wsc, s, K)
    r = rng.standard_normal((n, N)).astype(np.float32)
    want = {0: Y_o, 1: O.add(r, Y_o),
            2: O.mul(O.relu2(Y_o[:, 0::2]), Y_o[:, 1::2])}
    Wt = ops.upload_ternary(Wn, K)
    dX, dsc, dsm = _tiled_rows(q, s, n, K)
    dws = ops.DeviceArray.from_host(wsc)
    work = ops.DeviceArray((wsb,), np.uint8, zero=True)
    for epi in (0, 1, 2):
        for call, (buf, nb) in enumerate([(work, wsb), (work, wsb), (work, wsb - 1), (None, 0)]):
            Y = ops.DeviceArray.from_host(r) if epi == 1 else \
                ops.DeviceArray((n, N // 2 if epi == 2 else N), np.float32)
            acc = ops.DeviceArray((n, N), np.int32)
            ops.check(L.oxb_gemm_i8_ws(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, n, Y.ptr,
                                       acc.ptr, epi, buf.ptr if buf else None, nb, None),
                      "gemm_i8_ws")
            ops.sync()
            assert np.array_equal(acc.download(), acc_o), (epi, call)
            assert np.array_equal(Y.download(), want[epi]), (epi, call)
            assert not np.frombuffer(work.download()[:CNT_BYTES].tobytes(), np.int32).any(), (epi, call)


@pytest.mark.parametrize("n", [512, 65, 8])
def test_gemm_split_k_graph_replays(n):
    """The K splits (8192 x 28672: the 256 x 128 tiles at 512 tokens, the
    64 x 64 tiles at 65, the skinny kernel at 8) captured in a graph of three
    calls on one workspace
    and replayed four times, with eager calls and synchronisations between
    the replays: every replay gives the unsplit kernel's bits (each call's
    last arrival puts its counters back to zero, so no clearing node is
    needed in the graph)."""
    rng = np.random.default_rng(9000 + n)
    N, K = 8192, 28672
    L = ops.lib()
    wsb = L.oxb_gemm_ws_bytes(N, K, n)
    assert wsb > 0
    Wn = synth.i2s_pack(ternary(rng, N, K))
    q, s_ = O.quantize(rng.standard_normal((n, K)).astype(np.float32))
    Wt = ops.upload_ternary(Wn, K)
    dX, dsc, dsm = _tiled_rows(q, s_, n, K)
    dws = ops.DeviceArray.from_host(rng.uniform(0.01, 0.02, N).astype(np.float32))
    work = ops.DeviceArray((wsb,), np.uint8, zero=True)
    ref = ops.DeviceArray((n, N), np.float32)
    ops.check(L.oxb_gemm_i8(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, n, ref.ptr, None, 0,
                            None), "gemm_i8")
    ops.sync()
    want = ref.download()
    outs = [ops.DeviceArray((n, N), np.float32) for _ in range(3)]
    stream = L.oxb_stream_create()
    ops.check(L.oxb_stream_begin_capture(stream), "capture")
    for o in outs:
        ops.check(L.oxb_gemm_i8_ws(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, n, o.ptr, None,
                                   0, work.ptr, wsb, stream), "gemm_i8_ws")
    graph = L.oxb_stream_end_capture(stream)
    assert graph
    try:
        for rep in range(4):
            for o in outs:
                ops.check(L.oxb_memset_d(o.ptr, 0, n * N * 4, stream), "clear")
            ops.check(L.oxb_graph_launch(graph, stream), "replay")
            ops.check(L.oxb_stream_sync(stream), "sync")
            for o in outs:
                assert np.array_equal(o.download(), want), rep
            # an eager split call between the replays, on the same workspace
            ops.check(L.oxb_gemm_i8_ws(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, n,
                                       outs[0].ptr, None, 0, work.ptr, wsb, stream), "gemm_i8_ws")
            ops.check(L.oxb_stream_sync(stream), "sync")
            assert np.array_equal(outs[0].download(), want), rep
            assert not np.frombuffer(work.download()[:CNT_BYTES].tobytes(), np.int32).any(), rep
    finally:
        L.oxb_graph_destroy(graph)
        L.oxb_stream_destroy(stream)


def test_gemm_split_k_forms_share_a_workspace():
    """One workspace serving the three split forms in turn (5120 x 8192: 512
    tokens on 256 x 128 tiles, 130 on 64 x 64 tiles, 40 on the skinny kernel,
    then again in another order): every form keeps its arrival counters in
    the same fixed area, so no form reads another's leftover partial sums as
    counters.  Every call equals the oracle's rows bit for bit."""
    rng = np.random.default_rng(4242)
    N, K, n = 5120, 8192, 512
    L = ops.lib()
    Wn = synth.i2s_pack(ternary(rng, N, K))
    x = rng.standard_normal((n, K)).astype(np.float32)
    wsc = rng.uniform(0.01, 0.02, N).astype(np.float32)
    q, s = O.quantize(x)
    acc_o, Y_o = O.gemm(Wn, q, wsc, s, K)
    Wt = ops.upload_ternary(Wn, K)
    dws = ops.DeviceArray.from_host(wsc)
    rows = (512, 130, 40, 130, 512, 40)
    sizes = [L.oxb_gemm_ws_bytes(N, K, m) for m in rows]
    assert all(sizes)
    work = ops.DeviceArray((max(sizes),), np.uint8, zero=True)
    inputs = {m: _tiled_rows(q[:m], s[:m], m, K) for m in set(rows)}
    for i, m in enumerate(rows):
        dX, dsc, dsm = inputs[m]
        Y = ops.DeviceArray((m, N), np.float32)
        acc = ops.DeviceArray((m, N), np.int32)
        ops.check(L.oxb_gemm_i8_ws(Wt.ptr, dX.ptr, dsc.ptr, dsm.ptr, dws.ptr, N, K, m, Y.ptr,
                                   acc.ptr, 0, work.ptr, max(sizes), None), "gemm_i8_ws")
        ops.sync()
        assert np.array_equal(acc.download(), acc_o[:m]), (i, m)
        assert np.array_equal(Y.download(), Y_o[:m]), (i, m)
        assert not np.frombuffer(work.download()[:CNT_BYTES].tobytes(), np.int32).any(), (i, m)


@pytest.mark.parametrize("n", [40, 41, 130, 600])   # skinny (41: a real and a padding row share a workgroup of the quantizer), 128x64 LDS-staged, 256x128 DMA-staged
def test_gemm_epilogues(n):
    rng = np.random.default_rng(31 + n)
    K, F = 2560, 6912
    wg, wu = ternary(rng, F, K), ternary(rng, F, K)
    inter = np.empty((2 * F, K), np.int8)
    inter[0::2], inter[1::2] = wg, wu
    ws = np.empty(2 * F, np.float32)
    ws[0::2], ws[1::2] = 0.0151, 0.0172
    x = rng.standard_normal((n, K)).astype(np.float32)
    q, s = O.quantize(x)
    _, yg = O.gemm(synth.i2s_pack(wg), q, 0.0151, s, K)
    _, yu = O.gemm(synth.i2s_pack(wu), q, 0.0172, s, K)
    _, H, _ = ops.gemm(ops.upload_ternary(synth.i2s_pack(inter), K), x, None, 0.0, ws, 2 * F, K,
                    epilogue=2)
    assert np.array_equal(H, O.mul(O.relu2(yg), yu))
    # residual
    wd = ternary(rng, K, F)
    h = rng.standard_normal((n, F)).astype(np.float32)
    r = rng.standard_normal((n, K)).astype(np.float32)
    qh, sh = O.quantize(h)
    _, yd = O.gemm(synth.i2s_pack(wd), qh, 0.02, sh, F)
    _, R, _ = ops.gemm(ops.upload_ternary(synth.i2s_pack(wd), F), h, None, 0.0,
                    np.full(K, 0.02, np.float32), K, F, epilogue=1, Y0=r)
    assert np.array_equal(R, O.add(r, yd))


def test_prefill_block_512_tokens():
    """The 512-token prefill block at the 2B shape, chained as the engine runs
    it: RMSNorm (gamma ~ U(0.5, 1.5)) + absmax quantize of X [512, 2560] ~
    N(0, 1), the fused gate|up GEMM (W [6912, 2560] each, seeded uniform
    ternary, per-tensor scales 1/mean|w| of a N(0, 0.02) master) with
    relu^2(gate) * up, the subln RMSNorm + requantize, the down GEMM (W [2560,
    6912]).  Every stage equals the oracle's composition bit for bit."""
    rng = np.random.default_rng(2512)
    M, D, F = 512, 2560, 6912
    wg, wu, wd = ternary(rng, F, D), ternary(rng, F, D), ternary(rng, D, F)
    sg, su, sd = (synth.master_scale(rng) for _ in range(3))
    g1 = rng.uniform(0.5, 1.5, D).astype(np.float32)
    g2 = rng.uniform(0.5, 1.5, F).astype(np.float32)
    x = rng.standard_normal((M, D)).astype(np.float32)
    # oracle: rs/nn/ffn.rs:60-80 on the rs/nn/bitlinear.rs:207-247 path
    q1, s1 = O.quantize(O.rmsnorm(x, g1, 1e-5))
    _, yg = O.gemm(synth.i2s_pack(wg), q1, sg, s1, D)
    _, yu = O.gemm(synth.i2s_pack(wu), q1, su, s1, D)
    h_o = O.mul(O.relu2(yg), yu)
    q2, s2 = O.quantize(O.rmsnorm(h_o, g2, 1e-5))
    acc_o, y_o = O.gemm(synth.i2s_pack(wd), q2, sd, s2, F)
    # device: interleaved gate|up rows, fused epilogue, then the down GEMM
    inter = np.empty((2 * F, D), np.int8)
    inter[0::2], inter[1::2] = wg, wu
    ws = np.empty(2 * F, np.float32)
    ws[0::2], ws[1::2] = sg, su
    _, h, sc1 = ops.gemm(ops.upload_ternary(synth.i2s_pack(inter), D), x, g1, 1e-5, ws, 2 * F, D,
                         epilogue=2)
    assert np.array_equal(sc1, s1)
    assert np.array_equal(h, h_o)
    acc, y, sc2 = ops.gemm(ops.upload_ternary(synth.i2s_pack(wd), F), h, g2, 1e-5,
                           np.full(D, sd, np.float32), D, F)
    assert np.array_equal(sc2, s2)
    assert np.array_equal(acc, acc_o)
    assert np.array_equal(y, y_o)


def test_lm_head_argmax():
    rng = np.random.default_rng(41)
    V, D = 5003, 2560
    E = (rng.standard_normal((V, D)) * 0.02).astype(np.float16)
    x = rng.standard_normal(D).astype(np.float32) * 4
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    logits, tok, st, hist = ops.lm_head_argmax(x, g, 1e-5, E)
    h = O.rmsnorm(x, g, 1e-5)[0]
    ref = O.lm_head(h, E.view(np.uint16))
    assert np.array_equal(logits, ref)  # shader order reproduced: bit-exact
    assert tok == int(np.argmax(logits)) == O.argmax(ref)
    assert st[ops.STATE_POS] == 1 and st[ops.STATE_NGEN] == 1 and st[ops.STATE_LM_COUNTER] == 0
    assert hist[0] == tok


def test_lm_head_tie_lowest_index():
    D, V = 512, 4001
    E = np.zeros((V, D), np.float16)
    E[[17, 2500, 3999], :] = 1.0  # three identical best rows (V not a multiple of 64)
    logits, tok, _, _ = ops.lm_head_argmax(np.ones(D, np.float32), np.ones(D, np.float32), 1e-5, E)
    assert tok == 17


def test_embedding_gather():
    rng = np.random.default_rng(51)
    E = rng.standard_normal((300, 512)).astype(np.float16)
    ids = np.array([0, 299, 300, 5, -1], np.int32)
    x = ops.embedding(E, ids)
    assert np.array_equal(x[0], E[0].astype(np.float32))
    assert np.array_equal(x[1], E[299].astype(np.float32))
    assert not x[2].any() and not x[4].any()  # out of vocab -> zeros (embedding.wgsl:38-45)
    assert np.array_equal(x[3], E[5].astype(np.float32))
