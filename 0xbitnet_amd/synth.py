"""Synthetic BitNet models as GGUF files (random init, offline).

Writes the same container the reference loader reads (model/gguf.rs,
model/loader.rs): GGUF v3, arch "bitnet-25", I2_S (GGML type 36) ternary
linears with a 32-byte scale trailer, F32 norms, a tied F16 token embedding,
and tokenizer.ggml.* metadata, so `oxbitnet_load` works with no network.

Random init, per tensor, from numpy PCG64 seeded by (seed, tensor index):
  ternary weights  uniform over {-1, 0, +1};
  per-tensor scale mean|m| of a 65536-sample N(0, 0.02) master (the BitNet
                   dequantisation scale, ~0.016);
  norm gammas      U(0.5, 1.5);
  embedding        N(0, 0.02) in f16.
"""
from __future__ import annotations

import hashlib
import os
import struct
from dataclasses import asdict, dataclass

import numpy as np

GGML_F32, GGML_F16, GGML_I2_S = 0, 1, 36
ALIGN = 32


@dataclass
class Config:
    n_layers: int = 30
    hidden: int = 2560
    ffn: int = 6912
    heads: int = 20
    kv_heads: int = 5
    vocab: int = 128256
    rope_theta: float = 500000.0
    eps: float = 1e-5
    context: int = 4096
    arch: str = "bitnet-25"
    sub_norms: bool = True
    # where the hyperparameters live: "" = under the arch name; the reference
    # loader also reads "llama." / "bitnet." / "bitnet-25." (loader.rs:228-234)
    meta_prefix: str = ""
    norm_f16: bool = False     # norm weights stored F16 (converted on load, loader.rs:148-151)
    eos: int = 257             # tokenizer.ggml.eos_token_id

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


BITNET_2B = Config()


def small_config(**kw) -> Config:
    """A few-layer model with kernel-compatible shapes for tests."""
    base = dict(n_layers=2, hidden=512, ffn=1024, heads=4, kv_heads=1, vocab=1000, context=1024)
    base.update(kw)
    return Config(**base)


# ---- I2_S -------------------------------------------------------------------
def i2s_pack(w: np.ndarray) -> np.ndarray:
    """Ternary [N, K] (values -1/0/+1, K % 128 == 0) -> natural I2_S bytes [N, K/4].

    Byte b*32 + j of a row holds elements b*128 + g*32 + j at bits
    (7-2g):(6-2g) as code = w + 1 (docs/architecture.md:127-162)."""
    w = np.asarray(w)
    N, K = w.shape
    assert K % 128 == 0
    c = (w.astype(np.int16) + 1).astype(np.uint8).reshape(N, K // 128, 4, 32)
    b = (c[:, :, 0] << 6) | (c[:, :, 1] << 4) | (c[:, :, 2] << 2) | c[:, :, 3]
    return b.reshape(N, K // 4)


def i2s_unpack(packed: np.ndarray, K: int) -> np.ndarray:
    N = packed.shape[0]
    b = packed.reshape(N, K // 128, 1, 32).astype(np.int16)
    sh = np.array([6, 4, 2, 0], np.int16).reshape(1, 1, 4, 1)
    return (((b >> sh) & 3) - 1).reshape(N, K).astype(np.int8)


def random_i2s(rng: np.random.Generator, N: int, K: int) -> np.ndarray:
    """Uniform ternary codes packed directly (same distribution as i2s_pack of
    uniform {-1,0,1}), [N, K/4] uint8."""
    c = rng.integers(0, 3, size=(N, K // 128, 4, 32), dtype=np.uint8)
    b = (c[:, :, 0] << 6) | (c[:, :, 1] << 4) | (c[:, :, 2] << 2) | c[:, :, 3]
    return b.reshape(N, K // 4)


def master_scale(rng: np.random.Generator, n: int = 65536, std: float = 0.02) -> float:
    return float(np.float32(np.abs(rng.standard_normal(n) * std).mean()))


# ---- GGUF writer ---------------------------------------------------------------
def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, typ: int, payload: bytes) -> bytes:
    return _s(key) + struct.pack("<I", typ) + payload


def _u32(key, v):
    return _kv(key, 4, struct.pack("<I", v))


def _f32(key, v):
    return _kv(key, 6, struct.pack("<f", v))


def _str(key, v):
    return _kv(key, 8, _s(v))


def _strarr(key, arr):
    return _kv(key, 9, struct.pack("<IQ", 8, len(arr)) + b"".join(_s(a) for a in arr))


def _byte_alphabet():
    out, n = [], 0
    for b in range(256):
        keep = 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255
        out.append(chr(b) if keep else chr(256 + n))
        n += 0 if keep else 1
    return out


SPECIALS = ["<|begin_of_text|>", "<|end_of_text|>", "<|start_header_id|>", "<|end_header_id|>",
            "<|eot_id|>"]


def synthetic_vocab(V: int) -> list[str]:
    """256 byte tokens (GPT-2 alphabet, id = byte), the LLaMA-3 specials, then
    unique letter words with a leading 'Ġ' (space)."""
    toks = _byte_alphabet() + SPECIALS
    i = 0
    while len(toks) < V:
        n, w = i, ""
        while True:
            w = chr(97 + n % 26) + w
            n = n // 26 - 1
            if n < 0:
                break
        toks.append("Ġ" + w)
        i += 1
    return toks[:V]


def _tensor_list(cfg: Config):
    """(name, ggml_type, shape [ne0, ne1], kind) in file order."""
    D, F, hd = cfg.hidden, cfg.ffn, cfg.head_dim
    Dq, Dkv = cfg.heads * hd, cfg.kv_heads * hd
    nt = GGML_F16 if cfg.norm_f16 else GGML_F32
    out = [("token_embd.weight", GGML_F16, [D, cfg.vocab], "embed")]
    for i in range(cfg.n_layers):
        p = f"blk.{i}."
        out += [
            (p + "attn_norm.weight", nt, [D], "norm"),
            (p + "attn_q.weight", GGML_I2_S, [D, Dq], "tern"),
            (p + "attn_k.weight", GGML_I2_S, [D, Dkv], "tern"),
            (p + "attn_v.weight", GGML_I2_S, [D, Dkv], "tern"),
            (p + "attn_output.weight", GGML_I2_S, [Dq, D], "tern"),
            (p + "ffn_norm.weight", nt, [D], "norm"),
            (p + "ffn_gate.weight", GGML_I2_S, [D, F], "tern"),
            (p + "ffn_up.weight", GGML_I2_S, [D, F], "tern"),
            (p + "ffn_down.weight", GGML_I2_S, [F, D], "tern"),
        ]
        if cfg.sub_norms:
            out += [(p + "attn_sub_norm.weight", nt, [Dq], "norm"),
                    (p + "ffn_sub_norm.weight", nt, [F], "norm")]
    out.append(("output_norm.weight", nt, [D], "norm"))
    return out


def _nbytes(typ, shape):
    n = int(np.prod(shape))
    return {GGML_F32: 4 * n, GGML_F16: 2 * n, GGML_I2_S: (n + 3) // 4 + 32}[typ]


def _gen(kind, shape, rng, typ=GGML_F32):
    if kind == "embed":
        D, V = shape
        out = np.empty((V, D), np.float16)
        step = 8192
        for r in range(0, V, step):
            m = min(step, V - r)
            out[r:r + m] = (rng.standard_normal((m, D), dtype=np.float32) * np.float32(0.02))
        return out.tobytes()
    if kind == "norm":
        g = rng.uniform(0.5, 1.5, size=shape[0]).astype(np.float32)
        return (g.astype(np.float16) if typ == GGML_F16 else g).tobytes()
    K, N = shape
    packed = random_i2s(rng, N, K)
    scale = master_scale(rng)
    return packed.tobytes() + struct.pack("<f", scale) * 8


def write_gguf(path: str, cfg: Config = BITNET_2B, seed: int = 1234) -> str:
    """Write a random-init model of shape `cfg`; returns path."""
    tensors = _tensor_list(cfg)
    a = cfg.meta_prefix or cfg.arch
    vocab = synthetic_vocab(cfg.vocab)
    kvs = [
        _str("general.architecture", cfg.arch),
        _str("general.name", "synthetic-bitnet"),
        _u32("general.alignment", ALIGN),
        _u32(f"{a}.block_count", cfg.n_layers),
        _u32(f"{a}.embedding_length", cfg.hidden),
        _u32(f"{a}.feed_forward_length", cfg.ffn),
        _u32(f"{a}.attention.head_count", cfg.heads),
        _u32(f"{a}.attention.head_count_kv", cfg.kv_heads),
        _u32(f"{a}.context_length", cfg.context),
        _u32(f"{a}.vocab_size", cfg.vocab),
        _f32(f"{a}.rope.freq_base", cfg.rope_theta),
        _f32(f"{a}.attention.layer_norm_rms_epsilon", cfg.eps),
        _str("tokenizer.ggml.model", "gpt2"),
        _strarr("tokenizer.ggml.tokens", vocab),
        _u32("tokenizer.ggml.bos_token_id", 256),
        _u32("tokenizer.ggml.eos_token_id", cfg.eos),
    ]
    infos, off = [], 0
    for name, typ, shape, _ in tensors:
        infos.append(_s(name) + struct.pack("<I", len(shape)) +
                     b"".join(struct.pack("<Q", d) for d in shape) + struct.pack("<IQ", typ, off))
        off += _nbytes(typ, shape)
        off = (off + ALIGN - 1) // ALIGN * ALIGN
    header = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kvs)) + b"".join(kvs) + \
        b"".join(infos)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(header)
        f.write(b"\0" * ((-len(header)) % ALIGN))
        for idx, (name, typ, shape, kind) in enumerate(tensors):
            rng = np.random.default_rng([seed, idx])
            data = _gen(kind, shape, rng, typ)
            assert len(data) == _nbytes(typ, shape), name
            f.write(data)
            f.write(b"\0" * ((-len(data)) % ALIGN))
    os.replace(tmp, path)
    return path


def write_tokenizer_gguf(path: str, tokens: list[str], merges: list[str] | None = None,
                         bos: int = 0, eos: int = 1) -> str:
    """A GGUF holding tokenizer metadata only (tokens, optional merges "a b",
    bos/eos ids) and no tensors: what oxb_tokenizer_load reads."""
    kvs = [_str("general.architecture", "bitnet-25"), _str("tokenizer.ggml.model", "gpt2"),
           _strarr("tokenizer.ggml.tokens", tokens), _u32("tokenizer.ggml.bos_token_id", bos),
           _u32("tokenizer.ggml.eos_token_id", eos)]
    if merges is not None:
        kvs.append(_strarr("tokenizer.ggml.merges", merges))
    header = struct.pack("<IIQQ", 0x46554747, 3, 0, len(kvs)) + b"".join(kvs)
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * ((-len(header)) % ALIGN))
    return path


def cached_gguf(cfg: Config = BITNET_2B, seed: int = 1234, directory: str | None = None) -> str:
    """Path of a synthetic model file, written once per (config, seed)."""
    directory = directory or os.environ.get("OXB_MODEL_DIR", "/tmp/oxbitnet_models")
    os.makedirs(directory, exist_ok=True)
    key = "_".join(f"{k}{v}" for k, v in asdict(cfg).items()).replace(".", "p")
    path = os.path.join(directory, f"synth_{seed}_{hashlib.sha1(key.encode()).hexdigest()[:12]}.gguf")
    meta = path + ".cfg"
    if not (os.path.exists(path) and os.path.exists(meta) and open(meta).read() == key):
        write_gguf(path, cfg, seed)
        with open(meta, "w") as f:
            f.write(key)
    return path


# ---- reading back (for harnesses that feed the same weights elsewhere) ------
def read_gguf_tensors(path: str) -> tuple[dict, dict]:
    """Minimal reader for files written here: (metadata, name -> ndarray view).
    I2_S tensors come back as (packed uint8 [N, K/4], scale float)."""
    buf = np.memmap(path, np.uint8, mode="r")
    raw = memoryview(buf)
    off = 0

    def rd(fmt):
        nonlocal off
        v = struct.unpack_from(fmt, raw, off)
        off += struct.calcsize(fmt)
        return v

    def rs():
        (n,) = rd("<Q")
        nonlocal off
        s = bytes(raw[off:off + n]).decode()
        off += n
        return s

    def rv(t):
        if t == 8:
            return rs()
        if t == 9:
            et, n = rd("<IQ")
            return [rv(et) for _ in range(n)]
        fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q",
               11: "<q", 12: "<d"}[t]
        return rd(fmt)[0]

    magic, ver, nt, nkv = rd("<IIQQ")
    assert magic == 0x46554747
    meta = {}
    for _ in range(nkv):
        k = rs()
        (t,) = rd("<I")
        meta[k] = rv(t)
    infos = []
    for _ in range(nt):
        name = rs()
        (nd,) = rd("<I")
        shape = list(rd("<" + "Q" * nd))
        typ, toff = rd("<IQ")
        infos.append((name, shape, typ, toff))
    align = meta.get("general.alignment", 32)
    base = (off + align - 1) // align * align
    out = {}
    for name, shape, typ, toff in infos:
        start = base + toff
        n = int(np.prod(shape))
        if typ == GGML_I2_S:
            K, N = shape
            packed = np.asarray(buf[start:start + n // 4]).reshape(N, K // 4)
            scale = float(np.frombuffer(bytes(buf[start + n // 4:start + n // 4 + 4]), np.float32)[0])
            out[name] = (packed, scale)
        elif typ == GGML_F16:
            out[name] = np.asarray(buf[start:start + 2 * n]).view(np.float16).reshape(shape[::-1])
        else:
            out[name] = np.asarray(buf[start:start + 4 * n]).view(np.float32).reshape(shape[::-1])
    return meta, out
