"""Shared test helpers: import the package (its directory name starts with a
digit), seeded inputs, and the oracle's view of a synthetic GGUF."""
from __future__ import annotations

import importlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

pkg = importlib.import_module("0xbitnet_amd")
ops = importlib.import_module("0xbitnet_amd.ops")
synth = importlib.import_module("0xbitnet_amd.synth")


def ternary(rng, N, K):
    return rng.integers(-1, 2, size=(N, K)).astype(np.int8)


def absmax_quantize_input(rng, K):
    x = rng.standard_normal(K).astype(np.float32)
    return x


def oracle_weights(path: str):
    """(cfg dict, weights dict in the oracle's naming) from a synthetic GGUF."""
    meta, t = synth.read_gguf_tensors(path)
    arch = meta["general.architecture"]

    def get(suffix):   # the loader's prefix order (model/loader.rs:228-234)
        for pre in (arch, "llama", "bitnet", "bitnet-25"):
            if f"{pre}.{suffix}" in meta:
                return meta[f"{pre}.{suffix}"]
        raise KeyError(suffix)

    cfg = dict(n_layers=get("block_count"), D=get("embedding_length"),
               F=get("feed_forward_length"), H=get("attention.head_count"),
               Hkv=get("attention.head_count_kv"), V=get("vocab_size"),
               eps=get("attention.layer_norm_rms_epsilon"), rope_theta=get("rope.freq_base"))
    f32 = lambda a: np.asarray(a).astype(np.float32)   # F16 norms widen exactly
    w = {"model.embed_tokens.weight": t["token_embd.weight"].view(np.uint16),
         "model.norm.weight": f32(t["output_norm.weight"])}
    names = {"attn_q": "self_attn.q_proj", "attn_k": "self_attn.k_proj",
             "attn_v": "self_attn.v_proj", "attn_output": "self_attn.o_proj",
             "ffn_gate": "mlp.gate_proj", "ffn_up": "mlp.up_proj", "ffn_down": "mlp.down_proj"}
    norms = {"attn_norm": "input_layernorm", "ffn_norm": "post_attention_layernorm",
             "attn_sub_norm": "self_attn.sub_norm", "ffn_sub_norm": "mlp.sub_norm"}
    for i in range(cfg["n_layers"]):
        for g, h in names.items():
            packed, scale = t[f"blk.{i}.{g}.weight"]
            w[f"model.layers.{i}.{h}.weight"] = packed
            w[f"model.layers.{i}.{h}.weight_scale"] = scale
        for g, h in norms.items():
            key = f"blk.{i}.{g}.weight"
            if key in t:
                w[f"model.layers.{i}.{h}.weight"] = f32(t[key])
    return cfg, w


def near_tie(logits: np.ndarray, rel: float = 1e-3) -> bool:
    top = np.partition(logits, -2)[-2:]
    return abs(float(top[1] - top[0])) <= rel * max(abs(float(top[1])), 1e-6)
