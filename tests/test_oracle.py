"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle (a wrong bit
plane, a dropped term, half-away-from-zero rounding, a transposed operand)
fails: the reference tests' known answers (tests/golden/known_answers.json),
exhaustive/brute-force checks against independent numpy code, and closed
forms of the mathematics.
"""
import json
import math
import os

from fractions import Fraction

import numpy as np
import pytest

import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def np_i2s_decode(packed: np.ndarray, K: int) -> np.ndarray:
    """Independent decode straight from the format description
    (docs/architecture.md:127-162): 32-byte blocks, bit plane g at shift
    6-2g holds elements g*32 .. g*32+31 of the 128-element block, w = code-1."""
    rows = packed.shape[0]
    b = packed.reshape(rows, -1, 32).astype(np.int16)
    planes = [((b >> (6 - 2 * g)) & 3) - 1 for g in range(4)]
    return np.stack(planes, axis=2).reshape(rows, -1)[:, :K].astype(np.int8)


# ---------------------------------------------------------------- f16 ------
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(v)) for v in h], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin]) == np.isnan(ref[~fin]))


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),       # subnormal range
        (rng.standard_normal(2000) * 6e4).astype(np.float32),        # overflow edge
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 2.9802326e-08, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32),
    ])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


def test_expf_within_1ulp_of_double():
    rng = np.random.default_rng(9)
    xs = np.concatenate([rng.uniform(-103, 88, 20000), rng.uniform(-10, 0, 20000),
                         np.array([0.0, -0.0, 1.0, -1.0, 88.7, -87.3, -100.0, 1e-8, -1e-8])])
    xs = xs.astype(np.float32)
    got = np.array([O.expf(float(x)) for x in xs], np.float32)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    ulp = np.maximum(ulp, np.float64(2.0 ** -149))
    err = np.abs(got.astype(np.float64) - ref) / ulp
    assert err.max() <= 1.0, err.max()
    assert O.expf(0.0) == 1.0 and O.expf(-200.0) == 0.0 and O.expf(-3.4e38) == 0.0
    assert O.expf(100.0) == float("inf")


# ---------------------------------------------------------------- I2_S -----
@pytest.mark.parametrize("case", GOLD["i2s_fill_u32"]["cases"])
def test_i2s_known_bytes(case):
    w = np.full(case["K"], case["fill"], np.int8)
    packed = O.i2s_pack(w)
    assert int(packed[0, :4].view("<u4")[0]) == case["u32_0"]


def test_i2s_known_pattern():
    g = GOLD["i2s_pattern"]
    w = np.zeros(g["K"], np.int8)
    for k, v in g["nonzero"].items():
        w[int(k)] = v
    packed = O.i2s_pack(w)
    assert np.array_equal(O.i2s_unpack(packed, g["K"])[0], w)
    # element 0 (group 0, gp 0) sits in bits 7:6 of byte 0: code 0 (-1) ...
    # element 32 (group 1) in bits 5:4 (+1 -> code 2), 64 in 3:2 (-1 -> 0),
    # 96 in 1:0 (+1 -> 2): byte 0 = 0b00_10_00_10.
    assert packed[0, 0] == 0b00100010
    assert packed[0, 1] == 0b10010101  # element 1 = +1 in group 0, rest 0


@pytest.mark.parametrize("K", GOLD["i2s_roundtrip_K"]["K"])
def test_i2s_roundtrip(K):
    rng = np.random.default_rng(K)
    w = rng.integers(-1, 2, size=(3, K)).astype(np.int8)
    packed = O.i2s_pack(w)
    assert np.array_equal(O.i2s_unpack(packed, K), w)
    assert np.array_equal(np_i2s_decode(packed, K), w)
    for k in (0, 31, 32, 95, 127, K - 1):
        assert O.i2s_get(packed[1], k) == w[1, k]


# ---------------------------------------------------------------- quantize -
@pytest.mark.parametrize("case", GOLD["quantize"]["cases"])
def test_quantize_known(case):
    q, s = O.quantize(np.array(case["x"], np.float32))
    np.testing.assert_allclose(s, case["scales"], rtol=GOLD["quantize"]["scale_rtol"])
    if "q" in case:
        assert q.tolist() == case["q"]


def test_quantize_round_half_to_even():
    # absmax = 127 makes inv = 1.0 exactly, so x*inv = x and the .5 ties are
    # exact: WGSL round() goes to even (62.5 -> 62, -63.5 -> -64, 0.5 -> 0,
    # 1.5 -> 2), unlike Math.round in the TS spec (63, -63, 1, 2).
    x = np.array([[127.0, 62.5, -63.5, 0.5, 1.5, -0.5, -2.5, 126.5]], np.float32)
    q, s = O.quantize(x)
    assert q.tolist() == [[127, 62, -64, 0, 2, 0, -2, 126]]
    assert s[0] == np.float32(1.0)


def test_quantize_scale_is_f32_division():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((16, 2560)).astype(np.float32)
    q, s = O.quantize(x)
    am = np.abs(x).max(axis=1)
    assert np.array_equal(s, (am / np.float32(127.0)).astype(np.float32))
    assert np.abs(q).max() == 127
    # each row's absmax element maps to +-127 exactly
    for r in range(16):
        i = int(np.abs(x[r]).argmax())
        assert abs(int(q[r, i])) == 127
    # dequantisation error bound (quantize.test.ts:153-168)
    assert np.all(np.abs(q * s[:, None] - x) <= s[:, None] * 0.5 * (1 + 1e-5))


# ---------------------------------------------------------------- GEMV/GEMM -
def test_gemv_known():
    g = GOLD["gemv"]
    W = O.i2s_pack(np.array([[r] * g["K"] for r in g["rows"]], np.int8))
    x = np.full(g["K"], g["x_fill"], np.int8)
    acc, y = O.gemv(W, x, g["wscale"], g["in_scale"], g["K"])
    assert y.tolist() == g["y"] and acc.tolist() == [int(v) for v in g["y"]]


def test_gemm_known():
    g = GOLD["gemm"]
    W = O.i2s_pack(np.array([[r] * g["K"] for r in g["rows"]], np.int8))
    X = np.full((g["n_tok"], g["K"]), g["x_fill"], np.int8)
    acc, Y = O.gemm(W, X, 1.0, np.ones(g["n_tok"], np.float32), g["K"])
    assert Y.tolist() == g["y"]


def test_gemv_zero_weights_and_bruteforce():
    rng = np.random.default_rng(2)
    N, K = 37, 640
    W0 = O.i2s_pack(np.zeros((N, K), np.int8))
    x = rng.integers(-127, 128, K).astype(np.int8)
    acc, y = O.gemv(W0, x, 1.0, 1.0, K)
    assert not acc.any() and not y.any()
    w = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    W = O.i2s_pack(w)
    acc, y = O.gemv(W, x, 0.37, 0.011, K)
    ref = np_i2s_decode(W, K).astype(np.int64) @ x.astype(np.int64)
    assert np.array_equal(acc, ref)
    # epilogue association: (acc * ws) * is, two f32 roundings
    exp = (acc.astype(np.float32) * np.float32(0.37)) * np.float32(0.011)
    assert np.array_equal(y, exp)


def test_gemm_matches_gemv_rows_and_extremes():
    rng = np.random.default_rng(3)
    N, K, n = 24, 384, 5
    w = rng.integers(-1, 2, size=(N, K)).astype(np.int8)
    W = O.i2s_pack(w)
    X = rng.integers(-127, 128, (n, K)).astype(np.int8)
    isc = rng.uniform(0.01, 0.1, n).astype(np.float32)
    acc, Y = O.gemm(W, X, 2.5, isc, K)
    for t in range(n):
        a1, _ = O.gemv(W, X[t], 2.5, isc[t], K)
        assert np.array_equal(acc[t], a1)
    assert np.array_equal(Y, acc.astype(np.float32) * (np.float32(2.5) * isc[:, None]))
    # extreme accumulator: all +1 weights x all 127 at K = 28672
    K2 = 28672
    W2 = O.i2s_pack(np.ones((1, K2), np.int8))
    a2, _ = O.gemv(W2, np.full(K2, 127, np.int8), 1.0, 1.0, K2)
    assert a2[0] == 127 * K2


def test_bitlinear_constant_known():
    g = GOLD["bitlinear_const"]
    x = np.full((1, g["K"]), g["x_fill"], np.float32)
    q, s = O.quantize(x)
    W = O.i2s_pack(np.full((1, g["K"]), g["row"], np.int8))
    _, y = O.gemv(W, q[0], g["wscale"], s[0], g["K"])
    assert abs(y[0] - g["y"]) < 1e-3


# ---------------------------------------------------------------- norms ----
def test_rmsnorm_closed_form():
    g = GOLD["rmsnorm"]
    x = np.array(g["x"], np.float32)
    y = O.rmsnorm(x, np.ones(4, np.float32), g["eps"])[0]
    rms = math.sqrt(30 / 4 + g["eps"])
    np.testing.assert_allclose(y, np.array(g["x"]) / rms, rtol=g["rtol"])
    y2 = O.rmsnorm(x, np.full(4, 2.0, np.float32), g["eps"])[0]
    np.testing.assert_allclose(y2, 2 * y, rtol=1e-6)
    assert not O.rmsnorm(np.zeros(4, np.float32), np.ones(4, np.float32))[0].any()


def test_rmsnorm_float64_agreement():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 6912)).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, 6912).astype(np.float32)
    y = O.rmsnorm(x, w)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-7)


def test_rmsnorm_uses_strided_tree_order():
    # D = 257: thread 0 owns cols 0 and 256.  With x0^2 = 2^24 a sequential
    # f32 sum loses every later +1 (2^24 + 1 rounds back to 2^24, ties to
    # even).  In the shader's order thread 0 also loses col 256's +1, and the
    # stride-128 step loses p[128] = 1; from stride 64 on, the partials are
    # 2, 4, ..., 128 and add exactly: 2^24 + 2+4+8+16+32+64+128 = 2^24 + 254.
    x = np.ones(257, np.float32)
    x[0] = 4096.0
    seq = np.float32(0)
    for v in x:
        seq = np.float32(seq + np.float32(v * v))
    assert seq == np.float32(2 ** 24)
    y = O.rmsnorm(x, np.ones(257, np.float32), eps=0.0)[0]
    exact = 2.0 ** 24 + 254
    rms_tree = np.float32(1) / np.sqrt(np.float32(np.float32(exact) / np.float32(257)))
    rms_seq = np.float32(1) / np.sqrt(np.float32(seq / np.float32(257)))
    assert rms_tree != rms_seq
    assert y[1] == np.float32(np.float32(1.0) * rms_tree)


# ---------------------------------------------------------------- misc ops -
@pytest.mark.parametrize("case", GOLD["relu2"]["cases"])
def test_relu2_known(case):
    assert O.relu2(np.array(case["x"], np.float32)).tolist() == case["y"]


def test_silu_known():
    g = GOLD["silu"]
    np.testing.assert_allclose(O.silu(np.array(g["x"], np.float32)), g["y"], rtol=g["rtol"], atol=1e-7)


def test_softmax_known():
    g = GOLD["softmax"]
    assert O.softmax(np.array(g["uniform"]["x"], np.float32))[0].tolist() == g["uniform"]["y"]
    y = O.softmax(np.array(g["large"]["x"], np.float32))[0]
    assert np.all(np.isfinite(y)) and abs(y.sum() - 1) < 1e-6
    e = np.exp(np.array([-2.0, -1.0, 0.0]))
    np.testing.assert_allclose(y, e / e.sum(), rtol=1e-6)
    yd = O.softmax(np.array(g["dominant"]["x"], np.float32))
    assert yd.argmax(axis=1).tolist() == g["dominant"]["argmax"]
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 1000)).astype(np.float32)
    y = O.softmax(x)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=1e-5)
    ref = np.exp(x - x.max(1, keepdims=True))
    np.testing.assert_allclose(y, ref / ref.sum(1, keepdims=True), rtol=1e-5)


def test_rope_properties():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(2 * 4 * 8).astype(np.float32)
    # pos 0: identity (rope.test.ts:6-16)
    assert np.array_equal(O.rope(x, 1, 2, 8, 0, 10000.0)[:16], x[:16])
    y = O.rope(x, 2, 4, 8, 3, 500000.0).reshape(-1, 2)
    np.testing.assert_allclose(np.hypot(*y.T), np.hypot(*x.reshape(-1, 2).T), rtol=1e-6)
    # closed form at pos 5, pair 1 of hd 8: theta = 5 * 10000^(-2/8)
    th = 5 * 10000.0 ** (-0.25)
    x0, x1 = x[2], x[3]
    z = O.rope(x[:8], 1, 1, 8, 5, 10000.0)
    np.testing.assert_allclose(z[2:4], [x0 * math.cos(th) - x1 * math.sin(th),
                                        x0 * math.sin(th) + x1 * math.cos(th)], rtol=1e-5, atol=1e-6)


def test_attention_closed_forms():
    g = GOLD["attention_dot"]
    # one key: softmax weight 1 -> output is that V row
    q = np.array(g["q"], np.float32)
    k = np.array(g["k"], np.float32)
    v = np.array([0.5, -1.0, 2.0, 3.0], np.float32)
    out = O.attention(q, k, v, 1, 1, 1, 1, 4)
    assert out.tolist() == v.tolist()
    # two keys, hd 4 (scale 1/2): weights softmax([dot0, dot1] / 2)
    k2 = np.array([g["k"], [1.0, 1.0, 1.0, 1.0]], np.float32)
    v2 = np.array([[1.0, 0, 0, 0], [0, 1.0, 0, 0]], np.float32)
    out = O.attention(q, k2, v2, 1, 2, 1, 1, 4)
    s = np.array([g["dot"], 2.0]) / 2
    p = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    np.testing.assert_allclose(out[:2], p, rtol=1e-6)
    # causal mask with a cache (attention-scores.test.ts:55-77): 4 cached +
    # 2 new; query 0 must not see key 5.  Make key 5's V a marker.
    S, n = 6, 2
    rng = np.random.default_rng(7)
    qq = rng.standard_normal((n, 4)).astype(np.float32)
    kk = rng.standard_normal((S, 4)).astype(np.float32)
    vv = np.zeros((S, 4), np.float32)
    vv[5] = 1000.0
    o = O.attention(qq, kk, vv, n, S, 1, 1, 4).reshape(n, 4)
    assert np.all(o[0] == 0) and np.all(o[1] > 0)
    # GQA: heads 0-1 use kv head 0, heads 2-3 kv head 1 (H=4, Hkv=2)
    kk = rng.standard_normal((1, 2, 4)).astype(np.float32)
    vv = np.array([[[1, 1, 1, 1], [2, 2, 2, 2]]], np.float32)
    o = O.attention(rng.standard_normal((1, 4, 4)).astype(np.float32), kk, vv, 1, 1, 4, 2, 4)
    assert o.reshape(4, 4)[:, 0].tolist() == [1, 1, 2, 2]


def _f32_round(x: Fraction) -> float:
    """An exact rational rounded to the nearest f32 (ties to even), as an
    IEEE single-precision fused multiply-add rounds its exact result."""
    if x == 0:
        return 0.0
    neg, x = x < 0, abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    e = max(e, -126)                      # subnormals share the smallest exponent
    m = x * Fraction(2) ** (23 - e)       # 24 significant bits above the point
    q, r = divmod(m.numerator, m.denominator)
    if 2 * r > m.denominator or (2 * r == m.denominator and q & 1):
        q += 1
    v = float(Fraction(q) * Fraction(2) ** (e - 23))
    return -v if neg else v


def _fma_chain(p, v):
    """sum_s p[s] * v[s] as one f32 fused multiply-add per step, in order of s
    (sh/attention.wgsl:96-104 with each step fused), exactly."""
    acc = 0.0
    for a, b in zip(p, v):
        acc = _f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(acc))
    return acc


@pytest.mark.parametrize("S", [7, 256, 300, 700])
def test_attention_pv_is_one_fused_chain_over_all_positions(S):
    """P.V of the reference is one loop over every position.  With all K rows
    equal every score is the same, so p[s] = exp(0) * (1 / sum) is one known
    f32 value; V holds values whose sum depends on the association (2^24-
    scale terms beside small ones, cancelling across the 256-position mark).
    The oracle's output must be the exact sequential fma chain computed here
    from rationals, for every dim; the blocked variant (256-position blocks)
    must differ from it once S > 256 and equal it up to 256."""
    rng = np.random.default_rng(S)
    hd, H, Hkv = 8, 2, 1
    q = rng.standard_normal((1, H, hd)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, Hkv, hd)).astype(np.float32), S, axis=0)
    v = rng.integers(-9, 10, (S, Hkv, hd)).astype(np.float32) * np.float32(0.125)
    v[0, 0, :] = 2.0 ** 24 * S        # a large first term: later small terms round away
    if S > 256:
        v[256, 0, :] = -(2.0 ** 24) * S   # ... until it cancels at the 256th position
    out = O.attention(q, k, v, 1, S, H, Hkv, hd).reshape(H, hd)
    # p = exp(0) * (1 / sum): the row sum of S exact ones is S in any order
    pval = np.float32(1.0) * (np.float32(1.0) / np.float32(S))
    for d in range(hd):
        want = _fma_chain([pval] * S, v[:, 0, d])
        assert out[0, d] == np.float32(want) and out[1, d] == np.float32(want), d
    blk = O.attention_pv_blocked(q, k, v, 1, S, H, Hkv, hd, 256).reshape(H, hd)
    if S > 256:
        assert np.any(blk != out)
    else:
        assert np.array_equal(blk, out)


@pytest.mark.parametrize("S", [200, 256, 257, 700, 2304])
def test_attention_pv_against_float64(S):
    """The one-loop P.V against float64 attention: within 2e-6 of the sum of
    |p v| terms at every length, 500x inside the path's 1e-3 bound."""
    rng = np.random.default_rng(S)
    hd, H, Hkv = 128, 4, 1
    q = rng.standard_normal((1, H, hd)).astype(np.float32)
    k = (rng.standard_normal((S, Hkv, hd)) * 0.3).astype(np.float32)
    v = rng.standard_normal((S, Hkv, hd)).astype(np.float32)
    out = O.attention(q, k, v, 1, S, H, Hkv, hd).reshape(H, hd)
    sc = (q[0].astype(np.float64) @ k[:, 0].astype(np.float64).T) / np.sqrt(hd)
    p = np.exp(sc - sc.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ref = p @ v[:, 0].astype(np.float64)
    mag = p @ np.abs(v[:, 0].astype(np.float64))
    assert np.abs(out - ref).max() <= 2e-6 * mag.max()
    # a constant V row block is reproduced to rounding: sum_s p[s] * c = c
    vc = np.full((S, Hkv, hd), 0.75, np.float32)
    oc = O.attention(q, k, vc, 1, S, H, Hkv, hd)
    assert np.abs(oc - 0.75).max() <= 1e-5


def test_embedding_known():
    g = GOLD["embedding"]
    E = np.array(g["table"], np.float16).view(np.uint16)
    assert O.embedding(np.array(g["ids"]), E).tolist() == g["out"]


def test_lm_head_known_and_float64():
    for c in GOLD["lm_head"]["cases"]:
        E = np.array(c["E"], np.float16).view(np.uint16)
        assert O.lm_head(np.array(c["h"], np.float32), E).tolist() == c["logits"]
    rng = np.random.default_rng(8)
    E = (rng.standard_normal((300, 2560)) * 0.02).astype(np.float16)
    h = rng.standard_normal(2560).astype(np.float32)
    got = O.lm_head(h, E.view(np.uint16))
    ref = E.astype(np.float64) @ h.astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-5)


def test_argmax_lowest_index_on_ties():
    assert O.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert O.argmax(np.array([-5.0], np.float32)) == 0
