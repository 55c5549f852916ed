"""CPU-side checks of the C-ABI library: it loads, exports every symbol the
public headers declare, and its host logic (defaults, argument and GGUF
validation) behaves like the reference's FFI (oxbitnet-ffi/src/lib.rs).
No GPU compute is called here."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

from helpers import ROOT, pkg, synth

nat = pkg._native


def header_functions():
    names = set()
    for h in ("oxbitnet.h", "oxbitnet_ops.h"):
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b((?:oxbitnet|oxb)_\w+)\s*\(", src, re.M):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = nat.lib()
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the ctypes table covers them all
    assert set(names) <= set(nat.SIGNATURES)


def test_default_options_match_reference():
    L = nat.lib()
    o = L.oxbitnet_default_generate_options()
    assert (o.max_tokens, o.top_k, o.repeat_last_n) == (256, 50, 64)
    assert o.temperature == pytest.approx(1.0) and o.repeat_penalty == pytest.approx(1.1)
    lo = L.oxbitnet_default_load_options()
    assert not lo.on_progress and not lo.progress_userdata and not lo.cache_dir
    assert C.sizeof(nat.GenerateOptions) == 40          # LP64 layout of the reference struct
    assert C.sizeof(nat.LoadProgress) == 32
    assert C.sizeof(nat.LoadOptions) == 24


def _err():
    m = nat.lib().oxbitnet_error_message()
    return m.decode() if m else None


def test_load_argument_errors():
    L = nat.lib()
    assert not L.oxbitnet_load(None, None)
    assert _err() == "source must not be NULL"
    assert not L.oxbitnet_load(b"/nonexistent/model.gguf", None)
    assert _err().startswith("IO error")
    assert not L.oxbitnet_load(b"https://example.com/model.gguf", None)
    assert _err().startswith("HTTP error")
    assert not L.oxbitnet_load(b"\xff\xfe", None)
    assert _err().startswith("invalid UTF-8")
    L.oxbitnet_free(None)  # no-op
    assert L.oxbitnet_generate(None, b"hi", None, nat.TokenFn(), None) == -1
    assert _err() == "model must not be NULL"
    assert L.oxbitnet_chat(None, None, 0, None, nat.TokenFn(), None) == -1
    assert _err() == "model must not be NULL"


def test_operator_entry_points_check_arguments_first():
    """Host-side argument checks of the operator entry points return -1 with
    their message before any device call (so this runs without a GPU)."""
    L = nat.lib()
    p = C.c_void_p(64)   # never dereferenced: every call below fails its checks first
    assert L.oxb_attn_decode_batch(p, p, p, p, 8, 0, 1, 20, 5, 128, 300, None, p, None) == -1
    assert _err() == "attention: pos or scores is NULL"
    assert L.oxb_attn_decode_batch(p, p, p, p, 8, 0, 1, 20, 5, 64, 300, p, p, None) == -1
    assert _err() == "attention: head_dim 64 unsupported (128 only)"
    assert L.oxb_attn_decode_batch(p, p, p, p, 8, 0, 1, 20, 6, 128, 300, p, p, None) == -1
    assert _err() == "attention: heads 20 not a multiple of kv heads 6"
    assert L.oxb_attn_decode_batch(p, p, p, p, 8, 100, 2, 20, 5, 128, 300, p, p, None) == -1
    assert _err().startswith("attention: caches of a batch overlap")
    assert L.oxb_attn_decode_batch(p, p, p, p, 8, 0, 1, 20, 5, 128, 6145, p, p, None) == -1
    assert _err() == "attention: max_seq 6145 out of range (1..6144)"
    assert L.oxb_attn_prefill(p, p, p, 10, 95, 20, 5, 128, 100, p, None) == -1
    assert _err() == "prefill attention: bad range"
    assert L.oxb_attn_prefill(p, p, p, 10, 0, 20, 5, 64, 100, p, None) == -1
    assert _err() == "attention: head_dim 64 unsupported (128 only)"
    assert L.oxb_attn_prefill(p, p, p, 10, 0, 24, 8, 128, 100, p, None) == -1
    assert _err() == "attention: GQA group 3 unsupported (1, 2, 4, 8)"
    assert L.oxb_gemm_i8(p, p, p, p, p, 100, 256, 4, p, None, 0, None) == -1
    assert _err() == "ternary GEMM: out_dim 100 must be a multiple of 32"
    assert L.oxb_gemm_i8(p, p, p, p, p, 64, 300, 4, p, None, 0, None) == -1
    assert _err() == "ternary GEMM: in_dim 300 must be a multiple of 256"
    assert L.oxb_gemm_i8_ws(p, p, p, p, p, 64, 300, 4, p, None, 0, None, 0, None) == -1
    assert _err() == "ternary GEMM: in_dim 300 must be a multiple of 256"
    assert L.oxb_quantize_rows_tiled(p, p, 1e-5, 4, 100, p, p, p, None) == -1
    assert _err().startswith("quantize_rows_tiled: D 100 must be a multiple of 256")


def _write(tmp_path, name, data: bytes):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p).encode()


def test_gguf_parse_errors(tmp_path):
    L = nat.lib()
    assert not L.oxbitnet_load(_write(tmp_path, "bad.gguf", b"GGML" + b"\0" * 60), None)
    assert _err() == "Invalid GGUF magic: 0x4c4d4747 (expected 0x46554747)"
    assert not L.oxbitnet_load(_write(tmp_path, "v9.gguf", struct.pack("<IIQQ", 0x46554747, 9, 0, 0)), None)
    assert _err() == "Unsupported GGUF version: 9"
    assert not L.oxbitnet_load(_write(tmp_path, "short.gguf", struct.pack("<II", 0x46554747, 3)), None)
    assert _err().startswith("GGUF parse error: Unexpected EOF")
    kv = synth._s("x") + struct.pack("<I", 77)
    assert not L.oxbitnet_load(_write(tmp_path, "meta.gguf",
                                      struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + kv), None)
    assert _err() == "Unknown GGUF metadata type: 77"
    t = synth._s("w") + struct.pack("<IQQ", 1, 4, 99) + struct.pack("<Q", 0)
    assert not L.oxbitnet_load(_write(tmp_path, "type.gguf",
                                      struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + t), None)
    assert _err() == "Unsupported GGML type: 99"


def test_missing_tensor_error(tmp_path):
    cfg = synth.small_config(n_layers=1, vocab=300)
    path = str(tmp_path / "m.gguf")
    synth.write_gguf(path, cfg, seed=3)
    # drop blk.0.attn_q.weight by renaming it in the file (same length)
    data = bytearray(open(path, "rb").read())
    i = data.find(b"blk.0.attn_q.weight")
    data[i:i + len(b"blk.0.attn_q.weight")] = b"blk.0.attn_Q.weight"
    p2 = _write(tmp_path, "m2.gguf", bytes(data))
    assert not nat.lib().oxbitnet_load(p2, None)
    assert _err() == 'Missing weight tensor: "model.layers.0.self_attn.q_proj.weight"'


def _patch_u32_meta(data: bytes, key: str, value: int) -> bytes:
    """Overwrite the u32 value of metadata `key` in a GGUF image."""
    i = data.find(synth._s(key))
    assert i > 0
    j = i + len(synth._s(key))
    assert struct.unpack_from("<I", data, j)[0] == 4   # GGUF u32
    return data[:j + 4] + struct.pack("<I", value) + data[j + 8:]


def test_corrupt_metadata_is_rejected_before_sizing(tmp_path):
    """Counts read from the file are checked before anything is sized or
    divided by them; malformed lengths are parse errors, not allocations."""
    cfg = synth.small_config(n_layers=1, vocab=300)
    path = str(tmp_path / "m.gguf")
    synth.write_gguf(path, cfg, seed=3)
    data = open(path, "rb").read()
    L = nat.lib()
    a = "bitnet-25"
    for key, val, msg in ((f"{a}.block_count", 0xF0000000, "invalid model metadata"),
                          (f"{a}.block_count", 1000, "invalid model metadata: block_count 1000 but the file holds 13"),
                          (f"{a}.attention.head_count", 0, "invalid model metadata"),
                          (f"{a}.attention.head_count_kv", 0, "invalid model metadata"),
                          (f"{a}.embedding_length", 0x80000000, "invalid model metadata")):
        assert not L.oxbitnet_load(_write(tmp_path, "c.gguf", _patch_u32_meta(data, key, val)), None)
        assert _err().startswith(msg), (key, val, _err())
    hdr = struct.pack("<IIQQ", 0x46554747, 3, 0, 1)
    # string length near 2^64: must not wrap the bounds check
    assert not L.oxbitnet_load(_write(tmp_path, "s.gguf", hdr + struct.pack("<Q", 2**64 - 4)), None)
    assert _err().startswith("GGUF parse error: Unexpected EOF")
    # u32 array claiming more elements than bytes remain
    arr = synth._s("x") + struct.pack("<IIQ", 9, 4, 1 << 40)
    assert not L.oxbitnet_load(_write(tmp_path, "a.gguf", hdr + arr), None)
    assert _err() == "GGUF parse error: array length exceeds file size"
    # arrays nested deeper than any GGUF writer produces
    nest = synth._s("x") + struct.pack("<I", 9) + struct.pack("<IQ", 9, 1) * 6 + struct.pack("<IQ", 4, 0)
    assert not L.oxbitnet_load(_write(tmp_path, "n.gguf", hdr + nest), None)
    assert _err() == "GGUF parse error: arrays nested more than 4 deep"
    # tensor whose element count wraps 2^64
    t = synth._s("w") + struct.pack("<I", 2) + struct.pack("<QQ", 2**33, 2**31) + struct.pack("<IQ", 0, 0)
    assert not L.oxbitnet_load(_write(tmp_path, "t.gguf", struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + t),
                               None)
    assert _err() == "GGUF parse error: tensor w element count exceeds file size"


def test_synthetic_writer_roundtrip(tmp_path):
    import oracle as O
    cfg = synth.small_config(n_layers=1, vocab=300)
    path = str(tmp_path / "s.gguf")
    synth.write_gguf(path, cfg, seed=5)
    meta, t = synth.read_gguf_tensors(path)
    assert meta["general.architecture"] == "bitnet-25"
    assert len(meta["tokenizer.ggml.tokens"]) == 300
    packed, scale = t["blk.0.attn_q.weight"]
    assert packed.shape == (512, 128) and 0.012 < scale < 0.02
    w = synth.i2s_unpack(packed, 512)
    assert set(np.unique(w)) <= {-1, 0, 1}
    # product packer == oracle packer (ts/i2s-pack.ts restatement)
    assert np.array_equal(synth.i2s_pack(w), O.i2s_pack(w))
    assert np.array_equal(O.i2s_unpack(packed, 512), w)
    frac = np.bincount(w.reshape(-1) + 1) / w.size
    assert np.all(np.abs(frac - 1 / 3) < 0.01)
    assert t["token_embd.weight"].shape == (300, 512)


def test_i2s_pack_known_bytes():
    for fill, u32 in ((-1, 0), (1, 0xAAAAAAAA), (0, 0x55555555)):
        b = synth.i2s_pack(np.full((1, 128), fill, np.int8))
        assert int(b[0, :4].view("<u4")[0]) == u32


def _build_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("oxb_build", os.path.join(ROOT, "0xbitnet_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_build_rejects_kernels_with_scratch():
    b = _build_module()
    head = "k.hip:1:1: remark: Function Name: kern [-Rpass-analysis=kernel-resource-usage]\n"
    row = "k.hip:1:1: remark:     {}: {} [-Rpass-analysis=kernel-resource-usage]\n"
    ok = head + row.format("VGPRs", 64) + row.format("ScratchSize [bytes/lane]", 0) + \
        row.format("SGPRs Spill", 12) + row.format("VGPRs Spill", 0) + row.format("Dynamic Stack", "False")
    assert "ScratchSize [bytes/lane]=0" in b._check_resources("k.hip", ok)
    for key, val in (("ScratchSize [bytes/lane]", 80), ("VGPRs Spill", 3), ("Dynamic Stack", "True")):
        with pytest.raises(RuntimeError, match="scratch"):
            b._check_resources("k.hip", head + row.format(key, val))


def test_built_kernels_have_no_private_segment():
    bdir = os.path.join(ROOT, "0xbitnet_amd", "_build")
    srcs = [f for f in os.listdir(os.path.join(ROOT, "0xbitnet_amd", "csrc")) if f.endswith(".hip")]
    reports = [os.path.join(bdir, f + ".o.resources.txt") for f in srcs]
    if not all(os.path.exists(r) for r in reports):
        pytest.skip("library built without resource reports")
    n = 0
    for r in reports:
        for line in open(r):
            n += 1
            assert "ScratchSize [bytes/lane]=0" in line and "VGPRs Spill=0" in line, line
    assert n >= 20


def test_gemm_workspace_sizes():
    """oxb_gemm_ws_bytes (a host computation; 256 CUs assumed without a GPU):
    the split shapes need a workspace (the 16 KB counter area, then one int32
    slot per piece), every other shape and every shape the GEMM rejects none."""
    L = nat.lib()
    c = 16384
    # 8192 x 28672: 128 tiles of 256 x 128 in 2 pieces at 512 tokens, 64 in 4
    # at 256; the skinny kernel's 128 feature groups of 64 rows in 2 pieces at
    # <= 64 tokens; 256 tiles of 64 x 64 in 2 pieces at 65 tokens
    assert L.oxb_gemm_ws_bytes(8192, 28672, 512) == c + 128 * 2 * 256 * 128 * 4
    assert L.oxb_gemm_ws_bytes(8192, 28672, 256) == c + 64 * 4 * 256 * 128 * 4
    assert L.oxb_gemm_ws_bytes(8192, 28672, 8) == c + 128 * 2 * 1 * 4 * 64 * 16
    assert L.oxb_gemm_ws_bytes(8192, 28672, 64) == c + 128 * 2 * 4 * 4 * 64 * 16
    assert L.oxb_gemm_ws_bytes(8192, 28672, 65) == c + 256 * 2 * 64 * 64 * 4
    # the 2B down projection: 80 tiles of 64 x 64 in 3 pieces (9 stages) at
    # 65-128 tokens, 160 in 3 at 256, 240 in 2 at 384; none from 448 tokens
    assert L.oxb_gemm_ws_bytes(2560, 6912, 65) == c + 80 * 3 * 64 * 64 * 4
    assert L.oxb_gemm_ws_bytes(2560, 6912, 128) == c + 80 * 3 * 64 * 64 * 4
    assert L.oxb_gemm_ws_bytes(2560, 6912, 256) == c + 160 * 3 * 64 * 64 * 4
    assert L.oxb_gemm_ws_bytes(2560, 6912, 384) == c + 240 * 2 * 64 * 64 * 4
    for shape in [(2560, 6912, 448), (2560, 6912, 512), (2560, 6912, 1536), (2560, 2560, 128),
                  (13824, 2560, 128), (13824, 2560, 512), (28672, 8192, 64), (5120, 8192, 256),
                  (8192, 28672, 4096), (2560, 2560, 8), (0, 256, 4), (100, 8192, 4),
                  (64, 8200, 4), (8192, 28672, 0)]:
        assert L.oxb_gemm_ws_bytes(*shape) == 0, shape
