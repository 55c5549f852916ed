"""numpy front-end for the CPU oracle (liboxb_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module.  Each wrapper names the
reference WGSL / Rust routine its C function restates (paths as in
oxb_oracle.h: sh/ = shaders, rs/ = Rust core, ts/ = TS test helpers).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboxb_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_f32p = C.POINTER(C.c_float)
_i8p = C.POINTER(C.c_int8)
_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_i32p = C.POINTER(C.c_int32)


class _Layer(C.Structure):
    _fields_ = [(n, _u8p) for n in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")] + [
        (n, C.c_float) for n in ("sq", "sk", "sv", "so", "sgate", "sup", "sdown")
    ] + [(n, _f32p) for n in ("attn_norm", "ffn_norm", "attn_sub_norm", "ffn_sub_norm")]


ProbeFn = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_size_t)

# probe sites of oxo_forward (oxb_oracle.h, OXO_SITE_*)
SITES = ("x_in", "attn_norm", "qkv_q8", "qkv_scale", "q", "k", "v", "attn", "o_q8", "o_scale",
         "o", "x_mid", "ffn_norm", "gate", "up", "down_q8", "down_scale", "down", "x_out",
         "final")


class _Model(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "D", "F", "H", "Hkv", "V", "max_seq")] + [
        ("eps", C.c_float), ("rope_theta", C.c_float), ("kv_f16", C.c_int),
        ("embed", _u16p), ("final_norm", _f32p), ("layers", C.POINTER(_Layer)),
        ("kcache", _f32p), ("vcache", _f32p), ("seq_len", C.c_int),
        ("probe", ProbeFn), ("probe_ud", C.c_void_p), ("pv_block", C.c_int),
    ]


def _declare(L):
    L.oxo_f16_to_f32.argtypes = [C.c_uint16]
    L.oxo_f16_to_f32.restype = C.c_float
    L.oxo_f32_to_f16.argtypes = [C.c_float]
    L.oxo_f32_to_f16.restype = C.c_uint16
    L.oxo_expf.argtypes = [C.c_float]
    L.oxo_expf.restype = C.c_float
    L.oxo_i2s_pack_row.argtypes = [_i8p, C.c_int, _u8p]
    L.oxo_i2s_get.argtypes = [_u8p, C.c_int]
    L.oxo_i2s_get.restype = C.c_int
    L.oxo_i2s_unpack_row.argtypes = [_u8p, C.c_int, _i8p]
    L.oxo_quantize.argtypes = [_f32p, C.c_int, C.c_int, _i8p, _f32p]
    L.oxo_rmsnorm.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_float, _f32p]
    L.oxo_gemv.argtypes = [_u8p, _i8p, _f32p, C.c_float, C.c_int, C.c_int, _i32p, _f32p]
    L.oxo_gemm.argtypes = [_u8p, _i8p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, _i32p, _f32p]
    for n in ("oxo_relu2", "oxo_silu"):
        getattr(L, n).argtypes = [_f32p, C.c_size_t, _f32p]
    for n in ("oxo_add", "oxo_mul"):
        getattr(L, n).argtypes = [_f32p, _f32p, C.c_size_t, _f32p]
    L.oxo_rope.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _f32p]
    L.oxo_attention.argtypes = [_f32p, _f32p, _f32p] + [C.c_int] * 5 + [_f32p]
    L.oxo_attention_pv_blocked.argtypes = [_f32p, _f32p, _f32p] + [C.c_int] * 6 + [_f32p]
    L.oxo_softmax.argtypes = [_f32p, C.c_int, C.c_int, _f32p]
    L.oxo_embedding.argtypes = [_u32p, C.c_int, _u16p, C.c_int, C.c_int, _f32p]
    L.oxo_lm_head.argtypes = [_f32p, _u16p, C.c_int, C.c_int, _f32p]
    L.oxo_argmax.argtypes = [_f32p, C.c_int]
    L.oxo_argmax.restype = C.c_int
    L.oxo_forward.argtypes = [C.POINTER(_Model), _u32p, C.c_int, _f32p]
    L.oxo_forward.restype = C.c_int
    L.oxo_num_threads.restype = C.c_int
    L.oxo_set_num_threads.argtypes = [C.c_int]


def _p(a: np.ndarray, t):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- f16 ------------------------------------------------------------------
def f16_to_f32(h: int) -> float:
    return lib().oxo_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().oxo_f32_to_f16(f)


def expf(x: float) -> float:
    return lib().oxo_expf(x)


# ---- I2_S -----------------------------------------------------------------
def i2s_pack(w: np.ndarray) -> np.ndarray:
    """[rows, K] int8 ternary -> [rows, ceil(K/128)*32] uint8 (ts/i2s-pack.ts:110-138)."""
    w = _c(np.atleast_2d(w), np.int8)
    rows, K = w.shape
    rb = (K + 127) // 128 * 32
    out = np.zeros((rows, rb), np.uint8)
    for r in range(rows):
        lib().oxo_i2s_pack_row(_p(w[r], _i8p), K, _p(out[r], _u8p))
    return out


def i2s_get(row: np.ndarray, k: int) -> int:
    row = _c(row, np.uint8)
    return lib().oxo_i2s_get(_p(row, _u8p), k)


def i2s_unpack(packed: np.ndarray, K: int) -> np.ndarray:
    packed = _c(np.atleast_2d(packed), np.uint8)
    out = np.zeros((packed.shape[0], K), np.int8)
    for r in range(packed.shape[0]):
        lib().oxo_i2s_unpack_row(_p(packed[r], _u8p), K, _p(out[r], _i8p))
    return out


# ---- kernels ----------------------------------------------------------------
def quantize(x: np.ndarray):
    """sh/quantize.wgsl:28-74 -> (int8 [n, D], scales f32 [n])."""
    x = _c(np.atleast_2d(x), np.float32)
    n, D = x.shape
    q = np.zeros((n, D), np.int8)
    s = np.zeros(n, np.float32)
    lib().oxo_quantize(_p(x, _f32p), n, D, _p(q, _i8p), _p(s, _f32p))
    return q, s


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = _c(np.atleast_2d(x), np.float32)
    w = _c(w, np.float32)
    y = np.zeros_like(x)
    lib().oxo_rmsnorm(_p(x, _f32p), _p(w, _f32p), x.shape[0], x.shape[1], eps, _p(y, _f32p))
    return y


def gemv(W: np.ndarray, x: np.ndarray, wscale, in_scale: float, K: int):
    """sh/ternary_gemv.wgsl:39-97 -> (acc int32 [N], y f32 [N])."""
    W = _c(W, np.uint8)
    N = W.shape[0]
    x = _c(x, np.int8)
    ws = _c(np.broadcast_to(np.float32(wscale), (N,)), np.float32)
    acc = np.zeros(N, np.int32)
    y = np.zeros(N, np.float32)
    lib().oxo_gemv(_p(W, _u8p), _p(x, _i8p), _p(ws, _f32p), float(in_scale), N, K,
                   _p(acc, _i32p), _p(y, _f32p))
    return acc, y


def gemm(W: np.ndarray, X: np.ndarray, wscale, in_scales: np.ndarray, K: int):
    """sh/ternary_gemm.wgsl:40-136 -> (acc int32 [n, N], Y f32 [n, N])."""
    W = _c(W, np.uint8)
    N = W.shape[0]
    X = _c(np.atleast_2d(X), np.int8)
    n = X.shape[0]
    ws = _c(np.broadcast_to(np.float32(wscale), (N,)), np.float32)
    isc = _c(in_scales, np.float32)
    acc = np.zeros((n, N), np.int32)
    Y = np.zeros((n, N), np.float32)
    lib().oxo_gemm(_p(W, _u8p), _p(X, _i8p), _p(ws, _f32p), _p(isc, _f32p), N, n, K,
                   _p(acc, _i32p), _p(Y, _f32p))
    return acc, Y


def relu2(x):
    x = _c(x, np.float32)
    y = np.zeros_like(x)
    lib().oxo_relu2(_p(x, _f32p), x.size, _p(y, _f32p))
    return y


def silu(x):
    x = _c(x, np.float32)
    y = np.zeros_like(x)
    lib().oxo_silu(_p(x, _f32p), x.size, _p(y, _f32p))
    return y


def add(a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    y = np.zeros_like(a)
    lib().oxo_add(_p(a, _f32p), _p(b, _f32p), a.size, _p(y, _f32p))
    return y


def mul(a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    y = np.zeros_like(a)
    lib().oxo_mul(_p(a, _f32p), _p(b, _f32p), a.size, _p(y, _f32p))
    return y


def rope(x, n_tok, heads, hd, pos_offset, theta):
    x = _c(x, np.float32)
    y = np.zeros_like(x)
    lib().oxo_rope(_p(x, _f32p), n_tok, heads, hd, pos_offset, theta, _p(y, _f32p))
    return y


def softmax(x):
    x = _c(np.atleast_2d(x), np.float32)
    y = np.zeros_like(x)
    lib().oxo_softmax(_p(x, _f32p), x.shape[0], x.shape[1], _p(y, _f32p))
    return y


def attention(q, kc, vc, n_tok, S, H, Hkv, hd):
    """sh/attention.wgsl + sh/softmax.wgsl: P.V in one loop over the positions."""
    q, kc, vc = _c(q, np.float32), _c(kc, np.float32), _c(vc, np.float32)
    out = np.zeros(n_tok * H * hd, np.float32)
    lib().oxo_attention(_p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p), n_tok, S, H, Hkv, hd,
                        _p(out, _f32p))
    return out


def attention_pv_blocked(q, kc, vc, n_tok, S, H, Hkv, hd, pv_block):
    """The named non-reference variant: P.V summed in blocks of pv_block
    positions, block sums added in order (identical to attention() while a
    query has at most pv_block positions)."""
    q, kc, vc = _c(q, np.float32), _c(kc, np.float32), _c(vc, np.float32)
    out = np.zeros(n_tok * H * hd, np.float32)
    lib().oxo_attention_pv_blocked(_p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p), n_tok, S, H,
                                   Hkv, hd, pv_block, _p(out, _f32p))
    return out


def embedding(ids, E: np.ndarray):
    ids = _c(ids, np.uint32)
    E = _c(E, np.uint16)
    V, D = E.shape
    out = np.zeros((ids.size, D), np.float32)
    lib().oxo_embedding(_p(ids, _u32p), ids.size, _p(E, _u16p), V, D, _p(out, _f32p))
    return out


def lm_head(h, E: np.ndarray):
    h = _c(h, np.float32)
    E = _c(E, np.uint16)
    V, D = E.shape
    out = np.zeros(V, np.float32)
    lib().oxo_lm_head(_p(h, _f32p), _p(E, _u16p), V, D, _p(out, _f32p))
    return out


def argmax(x) -> int:
    x = _c(x, np.float32)
    return lib().oxo_argmax(_p(x, _f32p), x.size)


def num_threads() -> int:
    return lib().oxo_num_threads()


def set_num_threads(n: int) -> None:
    lib().oxo_set_num_threads(n)


class Model:
    """Oracle model over numpy weight arrays (rs/nn/model.rs:193-266).

    `weights` maps reference tensor names (model.layers.{i}.self_attn.q_proj.weight
    etc., rs/model/loader.rs:185-219) to arrays: I2_S matrices as uint8
    [rows, K/4], their per-tensor scales under "...weight_scale" as float,
    norms as float32, the embedding as uint16 [V, D] (f16 bits)."""

    def __init__(self, cfg: dict, weights: dict, max_seq: int, kv_f16: bool = False,
                 pv_block: int = 0):
        """pv_block 0: the reference's one-loop P.V; > 0: the blocked variant
        (oxo_attention_pv_blocked), which no product path computes."""
        self.cfg = cfg
        self._keep = []
        L = cfg["n_layers"]
        D, H, Hkv = cfg["D"], cfg["H"], cfg["Hkv"]
        hd = D // H
        self._layers = (_Layer * L)()
        for i in range(L):
            p = f"model.layers.{i}"
            lay = self._layers[i]
            for short, name in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"),
                                ("v", "self_attn.v_proj"), ("o", "self_attn.o_proj"),
                                ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                                ("down", "mlp.down_proj")):
                w = self._hold(_c(weights[f"{p}.{name}.weight"], np.uint8))
                setattr(lay, "w" + short, _p(w, _u8p))
                setattr(lay, "s" + short, float(weights[f"{p}.{name}.weight_scale"]))
            for fld, name in (("attn_norm", "input_layernorm"),
                              ("ffn_norm", "post_attention_layernorm"),
                              ("attn_sub_norm", "self_attn.sub_norm"),
                              ("ffn_sub_norm", "mlp.sub_norm")):
                key = f"{p}.{name}.weight"
                if key in weights:
                    setattr(lay, fld, _p(self._hold(_c(weights[key], np.float32)), _f32p))
        self._embed = self._hold(_c(weights["model.embed_tokens.weight"], np.uint16))
        self._fnorm = self._hold(_c(weights["model.norm.weight"], np.float32))
        self.kcache = np.zeros(L * max_seq * Hkv * hd, np.float32)
        self.vcache = np.zeros_like(self.kcache)
        m = _Model()
        m.n_layers, m.D, m.F, m.H, m.Hkv = L, D, cfg["F"], H, Hkv
        m.V, m.max_seq = cfg["V"], max_seq
        m.eps, m.rope_theta, m.kv_f16 = cfg["eps"], cfg["rope_theta"], int(kv_f16)
        m.embed = _p(self._embed, _u16p)
        m.final_norm = _p(self._fnorm, _f32p)
        m.layers = self._layers
        m.kcache, m.vcache = _p(self.kcache, _f32p), _p(self.vcache, _f32p)
        m.seq_len = 0
        m.pv_block = int(pv_block)
        self._m = m

    def _hold(self, a):
        self._keep.append(a)
        return a

    def reset(self):
        self._m.seq_len = 0

    @property
    def seq_len(self) -> int:
        return self._m.seq_len

    def forward(self, ids, trace: dict | None = None) -> np.ndarray:
        """Logits of the last id.  With `trace` (a dict), every probe site of
        every layer is copied into trace[(layer, site_name)] as a numpy array
        with one row per id (int8 for the *_q8 sites, else float32)."""
        ids = _c(ids, np.uint32)
        logits = np.zeros(self.cfg["V"], np.float32)
        n = ids.size

        def on_probe(_ud, layer, site, data, nbytes):
            name = SITES[site]
            dt = np.int8 if name.endswith("_q8") else np.float32
            buf = (C.c_char * nbytes).from_address(data)
            trace[(layer, name)] = np.frombuffer(bytes(buf), dt).reshape(n, -1).copy()

        cb = ProbeFn(on_probe) if trace is not None else ProbeFn()
        self._m.probe = cb
        try:
            rc = lib().oxo_forward(C.byref(self._m), _p(ids, _u32p), n, _p(logits, _f32p))
        finally:
            self._m.probe = ProbeFn()
        if rc != 0:
            raise RuntimeError("oracle: KV cache overflow")
        return logits
