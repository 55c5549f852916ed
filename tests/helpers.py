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
    a = meta["general.architecture"]
    cfg = dict(n_layers=meta[f"{a}.block_count"], D=meta[f"{a}.embedding_length"],
               F=meta[f"{a}.feed_forward_length"], H=meta[f"{a}.attention.head_count"],
               Hkv=meta[f"{a}.attention.head_count_kv"], V=meta[f"{a}.vocab_size"],
               eps=meta[f"{a}.attention.layer_norm_rms_epsilon"],
               rope_theta=meta[f"{a}.rope.freq_base"])
    w = {"model.embed_tokens.weight": t["token_embd.weight"].view(np.uint16),
         "model.norm.weight": t["output_norm.weight"]}
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
                w[f"model.layers.{i}.{h}.weight"] = t[key]
    return cfg, w


def near_tie(logits: np.ndarray, rel: float = 1e-3) -> bool:
    top = np.partition(logits, -2)[-2:]
    return abs(float(top[1] - top[0])) <= rel * max(abs(float(top[1])), 1e-6)
