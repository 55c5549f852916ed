"""numpy-level access to the hot-path kernels through the C ABI.

Device memory is owned by DeviceArray (hipMalloc'd by liboxbitnet); every op
launches the HIP kernel on the library's stream and returns host numpy
arrays.  Used by the parity tests and the benchmark.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._native import check, lib, NativeError

STATE_POS, STATE_TOKEN, STATE_NGEN, STATE_LM_COUNTER, STATE_HIST_CAP = 0, 1, 2, 3, 4
STATE_INTS = 8


class DeviceArray:
    """A device allocation with a dtype/shape view for uploads and downloads."""

    def __init__(self, shape, dtype, zero: bool = False):
        self.shape = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = lib().oxb_device_malloc(max(self.nbytes, 16))
        if not self.ptr:
            raise NativeError("oxb_device_malloc failed")
        if zero:
            check(lib().oxb_memset_d(self.ptr, 0, max(self.nbytes, 16), None), "memset")
            sync()

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        check(lib().oxb_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, None), "h2d")

    def download(self, shape=None, dtype=None) -> np.ndarray:
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        shp = shape if shape is not None else self.shape
        out = np.empty(shp, dt)
        assert out.nbytes <= self.nbytes
        check(lib().oxb_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, None), "d2h")
        return out

    def offset(self, nbytes: int) -> int:
        return self.ptr + nbytes

    def free(self) -> None:
        if self.ptr:
            lib().oxb_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync() -> None:
    check(lib().oxb_device_sync(), "device sync")


def device_info() -> dict:
    name = C.create_string_buffer(256)
    cus, clk = C.c_int(), C.c_int()
    mem = C.c_size_t()
    check(lib().oxb_device_info(name, 256, C.byref(cus), C.byref(clk), C.byref(mem)), "device info")
    return {"name": name.value.decode(), "cus": cus.value, "clock_khz": clk.value,
            "hbm_bytes": mem.value}


def _p(x):
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceArray) else x


# ---- layouts -----------------------------------------------------------------
def repack_tiled(W_natural: DeviceArray, N: int, K: int) -> DeviceArray:
    out = DeviceArray((N * K // 4,), np.uint8)
    check(lib().oxb_repack_i2s_tiled(W_natural.ptr, out.ptr, N, K, None), "repack")
    sync()
    return out


def upload_ternary(W_natural: np.ndarray, K: int) -> DeviceArray:
    """Natural I2_S rows [N][K/4] (host) -> tiled device matrix."""
    N = W_natural.shape[0]
    nat = DeviceArray.from_host(np.ascontiguousarray(W_natural, np.uint8).reshape(-1))
    t = repack_tiled(nat, N, K)
    nat.free()
    return t


# ---- kernels -----------------------------------------------------------------
def gemv_i8(Wt: DeviceArray, xq: np.ndarray, xscale: float, wscale: np.ndarray, N: int, K: int):
    """Int8 GEMV: returns (acc int32 [N], y f32 [N])."""
    xq = np.ascontiguousarray(xq, np.int8)
    dx = DeviceArray.from_host(xq)
    ds = DeviceArray.from_host(np.array([xscale], np.float32))
    dsum = DeviceArray.from_host(np.array([int(xq.astype(np.int64).sum())], np.int32))
    dw = DeviceArray.from_host(np.ascontiguousarray(wscale, np.float32))
    y = DeviceArray((N,), np.float32)
    acc = DeviceArray((N,), np.int32)
    check(lib().oxb_gemv_i8(Wt.ptr, dx.ptr, ds.ptr, dsum.ptr, dw.ptr, N, K, y.ptr, acc.ptr, None),
          "gemv_i8")
    sync()
    return acc.download(), y.download()


def bitlinear_gemv(Wt, x: np.ndarray, gamma, eps: float, wscale: np.ndarray, N: int, K: int,
                   residual: np.ndarray | None = None):
    """One-token BitLinear: returns (acc, y, xq, xscale)."""
    dx = DeviceArray.from_host(np.ascontiguousarray(x, np.float32))
    dg = DeviceArray.from_host(np.ascontiguousarray(gamma, np.float32)) if gamma is not None else None
    dw = DeviceArray.from_host(np.ascontiguousarray(wscale, np.float32))
    y = DeviceArray.from_host(np.ascontiguousarray(residual, np.float32)) if residual is not None \
        else DeviceArray((N,), np.float32)
    acc = DeviceArray((N,), np.int32)
    xq = DeviceArray((K,), np.int8)
    xs = DeviceArray((1,), np.float32)
    check(lib().oxb_bitlinear_gemv(Wt.ptr, dx.ptr, _p(dg), eps, dw.ptr, N, K, y.ptr,
                                   1 if residual is not None else 0, acc.ptr, xq.ptr, xs.ptr, None),
          "bitlinear_gemv")
    sync()
    return acc.download(), y.download(), xq.download(), float(xs.download()[0])


def bitlinear_gateup(Wt, x, gamma, eps, wscale, N2, K):
    dx = DeviceArray.from_host(np.ascontiguousarray(x, np.float32))
    dg = DeviceArray.from_host(np.ascontiguousarray(gamma, np.float32)) if gamma is not None else None
    dw = DeviceArray.from_host(np.ascontiguousarray(wscale, np.float32))
    h = DeviceArray((N2 // 2,), np.float32)
    check(lib().oxb_bitlinear_gateup(Wt.ptr, dx.ptr, _p(dg), eps, dw.ptr, N2, K, h.ptr, None),
          "bitlinear_gateup")
    sync()
    return h.download()


def norm_quant_rows(x: np.ndarray, gamma, eps: float):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    n, D = x.shape
    dx = DeviceArray.from_host(x)
    dg = DeviceArray.from_host(np.ascontiguousarray(gamma, np.float32)) if gamma is not None else None
    q = DeviceArray((n, D), np.int8)
    s = DeviceArray((n,), np.float32)
    sm = DeviceArray((n,), np.int32)
    check(lib().oxb_norm_quant_rows(dx.ptr, _p(dg), eps, n, D, q.ptr, s.ptr, sm.ptr, None),
          "norm_quant_rows")
    sync()
    return q.download(), s.download(), sm.download()


def quantize_rows_tiled(x: DeviceArray, gamma, eps: float, n: int, D: int, Xt: DeviceArray,
                        scales: DeviceArray, sums: DeviceArray, stream=None):
    check(lib().oxb_quantize_rows_tiled(x.ptr, _p(gamma), eps, n, D, Xt.ptr, scales.ptr, sums.ptr,
                                        stream), "quantize_rows_tiled")


def gemm(Wt, x: np.ndarray, gamma, eps: float, wscale: np.ndarray, N: int, K: int,
         epilogue: int = 0, Y0: np.ndarray | None = None):
    """Prefill BitLinear on MFMA: (optional RMSNorm) + quantize rows + GEMM.
    Returns (acc int32 [n, N], Y, xscales)."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    n = x.shape[0]
    npad = (n + 63) // 64 * 64
    dx = DeviceArray.from_host(x)
    dg = DeviceArray.from_host(np.ascontiguousarray(gamma, np.float32)) if gamma is not None else None
    Xt = DeviceArray((npad * K,), np.int8, zero=True)
    sc = DeviceArray((npad,), np.float32)
    sm = DeviceArray((npad,), np.int32)
    check(lib().oxb_quantize_rows_tiled(dx.ptr, _p(dg), eps, n, K, Xt.ptr, sc.ptr, sm.ptr, None),
          "quantize_rows_tiled")
    dw = DeviceArray.from_host(np.ascontiguousarray(wscale, np.float32))
    ncol = N // 2 if epilogue == 2 else N
    Y = DeviceArray.from_host(np.ascontiguousarray(Y0, np.float32)) if Y0 is not None \
        else DeviceArray((n, ncol), np.float32)
    acc = DeviceArray((n, N), np.int32)
    check(lib().oxb_gemm_i8(Wt.ptr, Xt.ptr, sc.ptr, sm.ptr, dw.ptr, N, K, n, Y.ptr, acc.ptr,
                            epilogue, None), "gemm_i8")
    sync()
    return acc.download(), Y.download(shape=(n, ncol)), sc.download(shape=(n,))


KV_PAD_ROWS = 64   # include/oxbitnet_ops.h OXB_KV_PAD_ROWS


def _padded_cache(c: np.ndarray, hd: int) -> DeviceArray:
    """A cache on the device with OXB_KV_PAD_ROWS rows of zeros past its end."""
    flat = np.ascontiguousarray(c, np.float16).view(np.uint16).reshape(-1)
    return DeviceArray.from_host(np.concatenate([flat, np.zeros(KV_PAD_ROWS * hd, np.uint16)]))


def v_octets(vc: np.ndarray) -> np.ndarray:
    """V cache rows [..., Hkv, S, hd] (f16) in the decode P.V's octet layout:
    per head round8(S) x hd elements, (position s, dim d) at ((s // 8) * hd +
    d) * 8 + s % 8 (positions past S zero)."""
    vc = np.asarray(vc, np.float16)
    *lead, hkv, S, hd = vc.shape
    S8 = (S + 7) // 8 * 8
    pad = np.zeros((*lead, hkv, S8, hd), np.float16)
    pad[..., :S, :] = vc
    o = pad.reshape(*lead, hkv, S8 // 8, 8, hd).swapaxes(-1, -2)   # [.., oct, hd, 8]
    return np.ascontiguousarray(o).view(np.uint16).reshape(*lead, hkv * S8 * hd)


def attn_decode(q: np.ndarray, kcache: np.ndarray, vcache: np.ndarray, pos: int, H: int, Hkv: int,
                hd: int, max_seq: int, fused: bool = False, head: bool = False, s_max: int = 0,
                octets: bool = False):
    """q [H*hd] f32; caches [Hkv][max_seq][hd] f16; attends over pos+1 positions.
    fused: the one-kernel variant (oxb_attn_decode_fused); head: one workgroup
    per query head (oxb_attn_decode_head, caches padded as it requires);
    octets: with the octet copy of V as well (oxb_attn_decode_head_v8 /
    oxb_attn_decode_batch_v8)."""
    dq = DeviceArray.from_host(np.ascontiguousarray(q, np.float32))
    dk = _padded_cache(kcache, hd)
    dv = _padded_cache(vcache, hd)
    dpos = DeviceArray.from_host(np.array([pos], np.int32))
    out = DeviceArray((H * hd,), np.float32)
    dv8 = DeviceArray.from_host(v_octets(vcache)) if octets else None
    if head and octets:
        check(lib().oxb_attn_decode_head_v8(dq.ptr, dk.ptr, dv.ptr, dv8.ptr, dpos.ptr, 0, 0, 0, 1,
                                            H, Hkv, hd, max_seq, s_max or pos + 1, out.ptr, None),
              "attn_decode_head_v8")
    elif head:
        check(lib().oxb_attn_decode_head(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, 0, 0, 1, H, Hkv, hd,
                                         max_seq, s_max or pos + 1, out.ptr, None),
              "attn_decode_head")
    elif octets:
        sc = DeviceArray((H * max_seq,), np.float32)
        check(lib().oxb_attn_decode_batch_v8(dq.ptr, dk.ptr, dv.ptr, dv8.ptr, dpos.ptr, 0, 0, 0, 1,
                                             H, Hkv, hd, max_seq, sc.ptr, out.ptr, None),
              "attn_decode_batch_v8")
    elif fused:
        check(lib().oxb_attn_decode_fused(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, H, Hkv, hd, max_seq,
                                          out.ptr, None), "attn_decode_fused")
    else:
        sc = DeviceArray((H * max_seq,), np.float32)
        check(lib().oxb_attn_decode(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, H, Hkv, hd, max_seq, sc.ptr,
                                    out.ptr, None), "attn_decode")
    sync()
    return out.download()


def attn_prefill(q: np.ndarray, kcache: np.ndarray, vcache: np.ndarray, n_tok: int, pos0: int,
                 H: int, Hkv: int, hd: int, max_seq: int):
    dq = DeviceArray.from_host(np.ascontiguousarray(q, np.float32))
    dk = DeviceArray.from_host(np.ascontiguousarray(kcache, np.float16).view(np.uint16))
    dv = DeviceArray.from_host(np.ascontiguousarray(vcache, np.float16).view(np.uint16))
    out = DeviceArray((n_tok, H * hd), np.float32)
    check(lib().oxb_attn_prefill(dq.ptr, dk.ptr, dv.ptr, n_tok, pos0, H, Hkv, hd, max_seq, out.ptr,
                                 None), "attn_prefill")
    sync()
    return out.download()


def lm_head_argmax(x: np.ndarray, gamma: np.ndarray, eps: float, E_f16: np.ndarray):
    """Returns (logits [V], token, state)."""
    V, D = E_f16.shape
    dx = DeviceArray.from_host(np.ascontiguousarray(x, np.float32))
    dg = DeviceArray.from_host(np.ascontiguousarray(gamma, np.float32))
    dE0 = DeviceArray.from_host(np.ascontiguousarray(E_f16).view(np.uint16))
    dE = DeviceArray((lib().oxb_lm_bytes(V, D),), np.uint8)
    check(lib().oxb_repack_lm(dE0.ptr, dE.ptr, V, D, None), "repack_lm")
    dE0.free()
    logits = DeviceArray((V,), np.float32)
    st = np.zeros(STATE_INTS, np.int32)
    st[STATE_HIST_CAP] = 4
    dst = DeviceArray.from_host(st)
    hist = DeviceArray((4,), np.int32, zero=True)
    check(lib().oxb_lm_head_argmax(dx.ptr, dg.ptr, eps, dE.ptr, V, D, logits.ptr, dst.ptr,
                                   hist.ptr, 1, None), "lm_head_argmax")
    sync()
    s = dst.download()
    return logits.download(), int(s[STATE_TOKEN]), s, hist.download()


def embedding(E_f16: np.ndarray, ids: np.ndarray):
    V, D = E_f16.shape
    ids = np.ascontiguousarray(ids, np.int32)
    dE = DeviceArray.from_host(np.ascontiguousarray(E_f16).view(np.uint16))
    di = DeviceArray.from_host(ids)
    x = DeviceArray((ids.size, D), np.float32)
    check(lib().oxb_embedding(dE.ptr, V, D, di.ptr, ids.size, None, x.ptr, None), "embedding")
    sync()
    return x.download()
