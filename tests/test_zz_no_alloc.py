"""The allocation-free decode attention (oxb_attn_decode_noalloc): same bits
as oxb_attn_decode with a caller scores buffer, on two calls in a row (the
second smaller, so the static scratch still holds the first call's scores
past the second's), and shapes beyond its scratch rejected."""
import numpy as np
import pytest

from helpers import ops, pkg

pytestmark = pytest.mark.gpu


def _run(L, H, Hkv, S, pos, seed, noalloc):
    rng = np.random.default_rng(seed)
    hd = 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = (rng.standard_normal((Hkv, S, hd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((Hkv, S, hd)).astype(np.float16)
    dq = ops.DeviceArray.from_host(q)
    dk = ops.DeviceArray.from_host(kc.view(np.uint16))
    dv = ops.DeviceArray.from_host(vc.view(np.uint16))
    dpos = ops.DeviceArray.from_host(np.array([pos], np.int32))
    out = ops.DeviceArray((H * hd,), np.float32)
    if noalloc:
        rc = L.oxb_attn_decode_noalloc(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, H, Hkv, hd, S, out.ptr,
                                       None)
    else:
        sc = ops.DeviceArray((H * S,), np.float32)
        rc = L.oxb_attn_decode(dq.ptr, dk.ptr, dv.ptr, dpos.ptr, H, Hkv, hd, S, sc.ptr, out.ptr,
                               None)
    ops.check(rc, "attention")
    ops.sync()
    return out.download()


def test_noalloc_matches_buffer_variant_two_calls():
    L = ops.lib()
    for H, Hkv, S, pos, seed in ((20, 5, 4096, 3000, 1), (8, 2, 700, 311, 2)):
        ref = _run(L, H, Hkv, S, pos, seed, noalloc=False)
        got = _run(L, H, Hkv, S, pos, seed, noalloc=True)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (H, S, pos)


def test_noalloc_rejects_shapes_beyond_its_scratch():
    L = ops.lib()
    z = ops.DeviceArray((16,), np.float32)
    assert L.oxb_attn_decode_noalloc(z.ptr, z.ptr, z.ptr, z.ptr, 64, 8, 128, 8192, z.ptr, None) == -1
    assert "exceed" in pkg._native.last_error()
