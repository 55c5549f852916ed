"""Benchmark: batch-1 greedy decode on the BitNet-b1.58-2B-shaped model.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16]

Workload (random init, synthetic data): 30 layers, hidden 2560, 20 q / 5 kv
heads (head_dim 128), FFN 6912 ReLU^2 gate, I2_S ternary linears, tied f16
embedding/LM head [128256, 2560], f16 KV cache.  A 128-token seeded
random-id prompt is prefilled (untimed), then `steps` greedy decode steps are
timed; each step is one replay of the captured hipGraph (no host work inside
the timed region).  value = decode tokens / second.

The JSON line also carries
  roofline      the ternary GEMV (int8 activations, 2-bit weights) at
                N=8192 x K=28672, M=1, timed with HIP events over launches that
                rotate 16 distinct weight copies (940 MB > the 256 MB MALL);
  gemv_sweep    the same for the other decode/sweep shapes;
  cpu_baseline  the CPU oracle (C restatement of the reference arithmetic,
                OpenMP) decoding on the same model: a bounded sample of
                steps after a short prompt.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_roofline(ops, synth, N: int, K: int, copies: int, iters: int) -> dict:
    """Average duration of the int8 ternary GEMV over `iters` launches that
    rotate through `copies` distinct weight buffers, timed by HIP events on
    the launch stream."""
    L = ops.lib()
    rng = np.random.default_rng([N, K])
    Wn = synth.random_i2s(rng, N, K)
    nat = ops.DeviceArray.from_host(Wn.reshape(-1))
    Ws = [ops.repack_tiled(nat, N, K) for _ in range(copies)]
    nat.free()
    x = rng.standard_normal(K).astype(np.float32)
    xq = np.clip(np.rint(x * (127.0 / np.abs(x).max())), -127, 127).astype(np.int8)
    dx = ops.DeviceArray.from_host(xq)
    ds = ops.DeviceArray.from_host(np.array([np.abs(x).max() / 127], np.float32))
    dsum = ops.DeviceArray.from_host(np.array([int(xq.astype(np.int64).sum())], np.int32))
    dw = ops.DeviceArray.from_host(np.full(N, 0.016, np.float32))
    y = ops.DeviceArray((N,), np.float32)
    stream = L.oxb_stream_create()
    e0, e1 = L.oxb_event_create(), L.oxb_event_create()
    for i in range(copies):  # warm-up
        ops.check(L.oxb_gemv_i8(Ws[i].ptr, dx.ptr, ds.ptr, dsum.ptr, dw.ptr, N, K, y.ptr, None,
                                stream), "gemv")
    ops.check(L.oxb_stream_sync(stream))
    ops.check(L.oxb_event_record(e0, stream))
    for i in range(iters):
        ops.check(L.oxb_gemv_i8(Ws[i % copies].ptr, dx.ptr, ds.ptr, dsum.ptr, dw.ptr, N, K, y.ptr,
                                None, stream), "gemv")
    ops.check(L.oxb_event_record(e1, stream))
    ops.check(L.oxb_event_sync(e1))
    ms = L.oxb_event_elapsed_ms(e0, e1) / iters
    L.oxb_event_destroy(e0)
    L.oxb_event_destroy(e1)
    L.oxb_stream_destroy(stream)
    for w in Ws:
        w.free()
    algo = N * K // 4 + K + 4 * N + 4
    gbs = algo / (ms * 1e-3) / 1e9
    return {"N": N, "K": K, "M": 1, "us": round(ms * 1e3, 3), "GBps": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": algo, "copies": copies}


def cpu_baseline(synth, path: str, prompt: np.ndarray, steps: int) -> dict:
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle as O  # the checker, timed here as the reported CPU baseline
    from helpers import oracle_weights
    cfg, w = oracle_weights(path)
    m = O.Model(cfg, w, max_seq=len(prompt) + steps + 1, kv_f16=True)
    logits = m.forward(prompt)
    tok = O.argmax(logits)
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = O.argmax(m.forward(np.array([tok], np.uint32)))
    dt = time.perf_counter() - t0
    return {"value": round(steps / dt, 3), "unit": "tokens/s", "cores": O.num_threads(),
            "kind": "port",
            "sample": f"{steps} greedy decode steps after a {len(prompt)}-token prompt on the same "
                      f"2B-shape model (C oracle, OpenMP over rows, f16-rounded KV)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--cpu-steps", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the decode path is "
              f"single-device and no multi-GPU figure is produced.", file=sys.stderr)
        return 2

    pkg = importlib.import_module("0xbitnet_amd")
    ops = importlib.import_module("0xbitnet_amd.ops")
    synth = importlib.import_module("0xbitnet_amd.synth")
    info = ops.device_info()
    log(f"device {info['name']} CUs {info['cus']}")

    t = time.time()
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    log(f"model file {path} ({os.path.getsize(path) / 1e9:.2f} GB, {time.time() - t:.1f}s)")
    t = time.time()
    max_seq = args.prompt + args.steps + args.warmup + 8
    model = pkg.Model(path, max_seq=max_seq)
    log(f"loaded in {time.time() - t:.1f}s; weights {model.info['weight_bytes'] / 1e9:.3f} GB")

    rng = np.random.default_rng(2024)
    prompt = rng.integers(0, synth.BITNET_2B.vocab, args.prompt).astype(np.int32)
    L = ops.lib()

    # warm-up run (graph capture, caches), then the timed run from a fresh cache
    model.reset()
    model.forward(prompt, want_logits=False)
    model.decode_greedy(args.warmup)
    model.reset()
    t0 = time.perf_counter()
    model.forward(prompt, want_logits=False)
    prefill_s = time.perf_counter() - t0
    ops.sync()
    t0 = time.perf_counter()
    toks = model.decode_greedy(args.steps)   # replays + one final sync
    dt = time.perf_counter() - t0
    ops.sync()
    tps = args.steps / dt
    log(f"decode {args.steps} steps: {dt * 1e3:.1f} ms -> {tps:.1f} tok/s; prefill "
        f"{args.prompt} tok {prefill_s * 1e3:.1f} ms; first tokens {toks[:8].tolist()}")

    # roofline of the ternary GEMV (the north-star shape) and the sweep
    roof = gemv_roofline(ops, synth, 8192, 28672, copies=16, iters=400)
    log(f"gemv 8192x28672: {roof['us']} us, {roof['GBps']} GB/s ({roof['frac'] * 100:.1f}% of peak)")
    sweep = []
    if not args.no_sweep:
        for N, K in ((28672, 8192), (6912, 2560), (3840, 2560), (13824, 2560), (2560, 6912)):
            r = gemv_roofline(ops, synth, N, K, copies=max(4, (600 << 20) // (N * K // 4)),
                              iters=400)
            sweep.append(r)
            log(f"gemv {N}x{K}: {r['us']} us {r['GBps']} GB/s")

    cpu = None
    if not args.no_cpu:
        t = time.time()
        cpu = cpu_baseline(synth, path, prompt[:8].astype(np.uint32), args.cpu_steps)
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads ({time.time() - t:.1f}s)")

    # bytes per decode step at the mean KV length of the timed run
    cfg = synth.BITNET_2B
    Lmean = args.prompt + args.steps / 2
    step_bytes = (model.info["weight_bytes"] + cfg.n_layers * 2 * cfg.kv_heads * 128 * 2 * Lmean
                  + 4 * (cfg.hidden * 2))
    line = {
        "metric": "decode tok/s bs=1 (2B shape); ternary GEMV HBM GB/s vs peak",
        "value": round(tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xternary/f16",
        "data": "synthetic (random-init weights, seeded random prompt ids)",
        "config": {"workload": "BitNet-b1.58-2B-shape batch-1 greedy decode: 30 layers, hidden "
                               "2560, 20q/5kv heads, FFN 6912, vocab 128256, 128-token prompt",
                   "prompt_tokens": args.prompt, "decode_tokens": args.steps,
                   "kv_cache": "f16", "parallelism": "none (1 GPU)"},
        "decode_step_GBps": round(step_bytes * tps / 1e9, 1),
        "decode_step_frac": round(step_bytes * tps / 1e9 / HBM_PEAK_GBS, 4),
        "prefill_ms": round(prefill_s * 1e3, 2),
        "roofline": {"bound": "hbm", "achieved": roof["GBps"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": roof["frac"], "traffic": None,
                     "kernel": "gemv_kernel<PRO_INT8,EPI_STORE> N=8192 K=28672 M=1",
                     "bytes_per_launch": roof["bytes"], "us_per_launch": roof["us"]},
        "gemv_sweep": sweep,
        "cpu_baseline": cpu,
        "device": info["name"],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
