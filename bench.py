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
                N=8192 x K=28672, M=1: 400 launches that rotate 16 distinct
                weight copies (940 MB > the 256 MB MALL), captured as one
                graph and timed with HIP events (median of 5 replays);
  gemv_sweep    the same for the other decode/sweep shapes;
  gemm_sweep    the ternary GEMM on int8 MFMA at M = 8 .. 4096 tokens for
                both sweep shapes (TOPS, and GB/s of the algorithmic bytes);
  prefill_block the 512-token prefill block: RMSNorm + quantize, fused
                gate|up GEMM with relu^2 * up, subln + requantize, down GEMM;
  long_context  2048-token prefill, then greedy decode up to 2560 cached
                positions at batch 1, 8 and 32 (independent sequences);
  cpu_baseline  the CPU oracle (C restatement of the reference arithmetic,
                OpenMP) decoding on the same model: a bounded sample of
                steps after the same 128-token prompt, with the host CPU's
                name and the reference's two other CPU legs (WGSL on
                lavapipe, bitnet.cpp) recorded as unavailable.

    python bench.py --roofline-only [--calib-mib 256]

runs only the 8192 x 28672 GEMV (plus, with --calib-mib, one device copy of
that many MiB, the calibration kernel for the FETCH_SIZE / WRITE_SIZE
counters) -- the command the rocprofv3 --pmc runs profile.

    python bench.py --long-context-only [--lc-batches 1,8,32] [--lc-steps 512]

runs only the long-context section.
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


def measured_traffic() -> int | None:
    """HBM bytes per launch of the 8192x28672 GEMV from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (copy-kernel calibrated)."""
    path = os.path.join(ROOT, "profiles", "gemv_8192x28672_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def gemv_roofline(ops, synth, N: int, K: int, copies: int, iters: int) -> dict:
    """Average duration of the int8 ternary GEMV over `iters` launches that
    rotate through `copies` distinct weight buffers, captured as one graph
    (so the host's per-call cost does not set the rate) and timed by HIP
    events on the launch stream; the median of 5 replays."""
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
    ops.check(L.oxb_stream_begin_capture(stream), "capture")
    for i in range(iters):
        ops.check(L.oxb_gemv_i8(Ws[i % copies].ptr, dx.ptr, ds.ptr, dsum.ptr, dw.ptr, N, K, y.ptr,
                                None, stream), "gemv")
    graph = L.oxb_stream_end_capture(stream)
    if not graph:
        ops.check(-1, "capture")
    ops.check(L.oxb_graph_launch(graph, stream))   # warm-up replay
    ops.check(L.oxb_stream_sync(stream))
    reps = []
    for _ in range(5):   # median of 5 replays (single replays vary by ~+-3%)
        ops.check(L.oxb_event_record(e0, stream))
        ops.check(L.oxb_graph_launch(graph, stream))
        ops.check(L.oxb_event_record(e1, stream))
        ops.check(L.oxb_event_sync(e1))
        reps.append(L.oxb_event_elapsed_ms(e0, e1) / iters)
    ms = float(np.median(reps))
    L.oxb_graph_destroy(graph)
    L.oxb_event_destroy(e0)
    L.oxb_event_destroy(e1)
    L.oxb_stream_destroy(stream)
    for w in Ws:
        w.free()
    algo = N * K // 4 + K + 4 * N + 4
    gbs = algo / (ms * 1e-3) / 1e9
    return {"N": N, "K": K, "M": 1, "us": round(ms * 1e3, 3), "GBps": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": algo, "copies": copies}


MFMA_I8_PEAK_TOPS = 5000.0


def _timed(L, stream, fn, iters: int, reps: int = 3) -> float:
    """Mean ms per call of fn(i) over iters calls on `stream`: the calls are
    captured as one graph (fn(0) runs once before, uncaptured), replayed
    once to warm up, then timed with HIP events; the median of `reps`."""
    e0, e1 = L.oxb_event_create(), L.oxb_event_create()
    fn(0)
    ops_check = _native_check(L)
    ops_check(L.oxb_stream_sync(stream))
    ops_check(L.oxb_stream_begin_capture(stream))
    for i in range(iters):
        fn(i)
    graph = L.oxb_stream_end_capture(stream)
    if not graph:
        ops_check(-1)
    ops_check(L.oxb_graph_launch(graph, stream))
    ops_check(L.oxb_stream_sync(stream))
    times = []
    for _ in range(reps):
        ops_check(L.oxb_event_record(e0, stream))
        ops_check(L.oxb_graph_launch(graph, stream))
        ops_check(L.oxb_event_record(e1, stream))
        ops_check(L.oxb_event_sync(e1))
        times.append(L.oxb_event_elapsed_ms(e0, e1) / iters)
    L.oxb_graph_destroy(graph)
    L.oxb_event_destroy(e0)
    L.oxb_event_destroy(e1)
    return float(np.median(times))


def _native_check(L):
    def check(rc):
        if rc != 0:
            raise RuntimeError(L.oxb_last_error().decode())
    return check


def _host_tiles(rng, M: int, K: int):
    """int8 activations of M seeded N(0,1) rows (per-token absmax, RNE, +-127)
    in the GEMM's token-tiled layout [Mpad/16][K/256][4 planes][4 chunks][16 tokens][16],
    plane g of chunk kc = 4*stage + c holding k = (kc//2)*128 + g*32 + (kc%2)*16 + j;
    returns (tiles, scales, sums) with rows past M zero (scale 1, sum 0)."""
    mpad = (M + 63) // 64 * 64
    x = rng.standard_normal((M, K)).astype(np.float32)
    am = np.abs(x).max(axis=1, keepdims=True)
    q = np.clip(np.rint(x * (np.float32(127.0) / am)), -127, 127).astype(np.int8)
    Q = np.zeros((mpad, K), np.int8)
    Q[:M] = q
    # k = stage*256 + (c//2)*128 + g*32 + (c%2)*16 + j
    t = Q.reshape(mpad // 16, 16, K // 256, 2, 4, 2, 16).transpose(0, 2, 4, 3, 5, 1, 6)
    sc = np.ones(mpad, np.float32)
    sc[:M] = (am[:, 0] / np.float32(127.0)).astype(np.float32)
    sm = np.zeros(mpad, np.int32)
    sm[:M] = q.astype(np.int64).sum(axis=1)
    return np.ascontiguousarray(t).reshape(-1), sc, sm


def gemm_sweep(ops, synth, N: int, K: int, M: int, copies: int, iters: int) -> dict:
    """Ternary GEMM (int8 MFMA, int32 accumulate, f32 epilogue) at M tokens."""
    L = ops.lib()
    rng = np.random.default_rng([N, K, M])
    nat = ops.DeviceArray.from_host(synth.random_i2s(rng, N, K).reshape(-1))
    Ws = [ops.repack_tiled(nat, N, K) for _ in range(copies)]
    nat.free()
    stream = L.oxb_stream_create()
    ht, hs, hm = _host_tiles(rng, M, K)
    Xt, sc, sm = (ops.DeviceArray.from_host(a) for a in (ht, hs, hm))
    dw = ops.DeviceArray.from_host(np.full(N, 0.016, np.float32))
    Y = ops.DeviceArray((M, N), np.float32)
    # the split-K workspace where the shape splits (counters zero-filled)
    wsb = L.oxb_gemm_ws_bytes(N, K, M)
    work = ops.DeviceArray((wsb,), np.uint8, zero=True) if wsb else None

    def run(i):
        ops.check(L.oxb_gemm_i8_ws(Ws[i % copies].ptr, Xt.ptr, sc.ptr, sm.ptr, dw.ptr, N, K, M,
                                   Y.ptr, None, 0, work.ptr if work else None, wsb, stream),
                  "gemm")
    ms = _timed(L, stream, run, iters)
    L.oxb_stream_destroy(stream)
    for b in Ws + [Xt, sc, sm, dw, Y] + ([work] if work else []):
        b.free()
    ops_n = 2.0 * M * N * K
    algo = N * K // 4 + M * K + 4 * M * N + 4
    tops = ops_n / (ms * 1e-3) / 1e12
    gbs = algo / (ms * 1e-3) / 1e9
    return {"N": N, "K": K, "M": M, "us": round(ms * 1e3, 2), "TOPS": round(tops, 2),
            "frac_mfma": round(tops / MFMA_I8_PEAK_TOPS, 4), "GBps": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "bytes": algo, "copies": copies,
            "split_k_ws_bytes": wsb}


def prefill_block(ops, synth, M: int = 512, iters: int = 20) -> dict:
    """RMSNorm + quantize -> gate|up GEMM (relu^2 * up fused) -> subln +
    requantize -> down GEMM, on M tokens of the 2B shape."""
    L = ops.lib()
    cfg = synth.BITNET_2B
    D, F = cfg.hidden, cfg.ffn
    rng = np.random.default_rng(512)
    nat = ops.DeviceArray.from_host(synth.random_i2s(rng, 2 * F, D).reshape(-1))
    Wgu = ops.repack_tiled(nat, 2 * F, D)
    nat.free()
    nat = ops.DeviceArray.from_host(synth.random_i2s(rng, D, F).reshape(-1))
    Wd = ops.repack_tiled(nat, D, F)
    nat.free()
    g1 = ops.DeviceArray.from_host(rng.uniform(0.5, 1.5, D).astype(np.float32))
    g2 = ops.DeviceArray.from_host(rng.uniform(0.5, 1.5, F).astype(np.float32))
    s1 = ops.DeviceArray.from_host(np.full(2 * F, 0.016, np.float32))
    s2 = ops.DeviceArray.from_host(np.full(D, 0.016, np.float32))
    stream = L.oxb_stream_create()
    mpad = (M + 63) // 64 * 64
    x = ops.DeviceArray.from_host(rng.standard_normal((M, D)).astype(np.float32))
    X1 = ops.DeviceArray((mpad * D,), np.int8, zero=True)
    X2 = ops.DeviceArray((mpad * F,), np.int8, zero=True)
    sc = ops.DeviceArray((mpad,), np.float32)
    sm = ops.DeviceArray((mpad,), np.int32)
    h = ops.DeviceArray((M, F), np.float32)
    y = ops.DeviceArray((M, D), np.float32)
    # the split-K workspaces (none of the block's shapes splits at 512 tokens)
    wb1, wb2 = L.oxb_gemm_ws_bytes(2 * F, D, M), L.oxb_gemm_ws_bytes(D, F, M)
    work = ops.DeviceArray((max(wb1, wb2),), np.uint8, zero=True) if max(wb1, wb2) else None
    wp = work.ptr if work else None

    def run(_):
        ops.check(L.oxb_quantize_rows_tiled(x.ptr, g1.ptr, 1e-5, M, D, X1.ptr, sc.ptr, sm.ptr,
                                            stream), "q1")
        ops.check(L.oxb_gemm_i8_ws(Wgu.ptr, X1.ptr, sc.ptr, sm.ptr, s1.ptr, 2 * F, D, M, h.ptr,
                                   None, 2, wp, wb1, stream), "gateup")
        ops.check(L.oxb_quantize_rows_tiled(h.ptr, g2.ptr, 1e-5, M, F, X2.ptr, sc.ptr, sm.ptr,
                                            stream), "q2")
        ops.check(L.oxb_gemm_i8_ws(Wd.ptr, X2.ptr, sc.ptr, sm.ptr, s2.ptr, D, F, M, y.ptr, None,
                                   0, wp, wb2, stream), "down")
    ms = _timed(L, stream, run, iters)
    L.oxb_stream_destroy(stream)
    for b in (Wgu, Wd, g1, g2, s1, s2, x, X1, X2, sc, sm, h, y) + ((work,) if work else ()):
        b.free()
    ops_n = 2.0 * M * (2 * F) * D + 2.0 * M * D * F
    tops = ops_n / (ms * 1e-3) / 1e12
    return {"M": M, "ms": round(ms, 4), "ops": int(ops_n), "TOPS": round(tops, 2),
            "frac_mfma": round(tops / MFMA_I8_PEAK_TOPS, 4),
            "kernels": "quantize_rows_tiled, gemm gate|up (relu^2*up), quantize_rows_tiled "
                       "(subln), gemm down"}


def long_context(pkg, synth, path: str, prompt_len: int = 2048, steps: int = 512,
                 batches=(1, 8, 32)) -> dict:
    """2048-token prefill (per sequence), then greedy decode to 2560 cached
    positions at batch 1 (one-sequence engine) and 8 / 32 (batched engine,
    independent seeded prompts)."""
    import importlib as _il
    ops = _il.import_module("0xbitnet_amd.ops")
    max_seq = prompt_len + steps + 8
    m = pkg.Model(path, max_seq=max_seq)
    out = {"prompt_tokens": prompt_len, "decode_tokens": steps, "kv_positions_max": prompt_len + steps}
    if 1 in batches:   # the one-sequence engine: timed prefill, then its decode below
        rng = np.random.default_rng(4096)
        prompt = rng.integers(0, synth.BITNET_2B.vocab, prompt_len).astype(np.int32)
        # warm-up at the full length: graph capture, code paths and the prefill
        # buffers, which the engine sizes on the first prompt this long
        m.forward(prompt, want_logits=False)
        m.decode_greedy(4)
        pfs = []
        for _ in range(5):   # median of 5 timed prefills; the last one's cache is decoded below
            m.reset()
            ops.sync()
            t0 = time.perf_counter()
            m.forward(prompt, want_logits=False)
            ops.sync()
            pfs.append(time.perf_counter() - t0)
        pf = float(np.median(pfs))
        out.update({"prefill_ms": round(pf * 1e3, 2), "prefill_tok_s": round(prompt_len / pf, 1),
                    "prefill_ms_runs": [round(x * 1e3, 2) for x in pfs]})
    rows = []
    for B in batches:
        if B == 1:
            t0 = time.perf_counter()
            m.decode_greedy(steps)
            ops.sync()
            dt = time.perf_counter() - t0
        else:
            b = pkg.Batch(m, B, max_seq)
            for i in range(B):
                p_i = np.random.default_rng([4096, i]).integers(0, synth.BITNET_2B.vocab,
                                                                 prompt_len).astype(np.int32)
                b.prefill(i, p_i)
            b.decode_greedy(2)                      # graph capture
            t0 = time.perf_counter()
            b.decode_greedy(steps - 2)
            ops.sync()
            dt = (time.perf_counter() - t0) * steps / (steps - 2)
            b.close()
        rows.append({"batch": B, "decode_tok_s": round(B * steps / dt, 1),
                     "ms_per_step": round(dt * 1e3 / steps, 3)})
        log(f"long context bs={B}: {B * steps / dt:.1f} tok/s ({dt * 1e3 / steps:.3f} ms/step)")
    m.close()
    out["decode"] = rows
    return out


def calib_copy(ops, mib: int) -> None:
    """One device-to-device copy of `mib` MiB: the reference kernel whose
    FETCH_SIZE / WRITE_SIZE readings scale the counters to bytes."""
    L = ops.lib()
    n = mib << 20
    a = ops.DeviceArray((n,), np.uint8, zero=True)
    b = ops.DeviceArray((n,), np.uint8)
    ops.check(L.oxb_memcpy_d2d(b.ptr, a.ptr, n, None), "calib copy")
    ops.sync()
    a.free()
    b.free()


def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# The reference's other CPU legs for this workload, neither of which can run
# here: both would need software that is not on the machine and cannot be
# fetched.
OTHER_CPU_LEGS = {
    "wgsl_lavapipe": {
        "status": "unavailable",
        "reason": "0xBitNet's own WGSL shaders on a CPU Vulkan adapter (Mesa lavapipe) through "
                  "wgpu 26 need a Rust toolchain, the wgpu crates and a lavapipe ICD; none is "
                  "installed and there is no network"},
    "bitnet_cpp": {
        "status": "unavailable",
        "reason": "bitnet.cpp's I2_S kernels come from the reference's vendor/BitNet git "
                  "submodule, which is not vendored (empty directory); there is no network"},
}


def cpu_baseline(synth, path: str, prompt: np.ndarray, steps: int) -> dict:
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle as O  # the checker, timed here as the reported CPU baseline
    from helpers import oracle_weights
    cfg, w = oracle_weights(path)
    m = O.Model(cfg, w, max_seq=len(prompt) + steps + 1, kv_f16=True)
    t0 = time.perf_counter()
    logits = m.forward(prompt)
    prefill_s = time.perf_counter() - t0
    tok = O.argmax(logits)
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = O.argmax(m.forward(np.array([tok], np.uint32)))
    dt = time.perf_counter() - t0
    return {"value": round(steps / dt, 3), "unit": "tokens/s", "cores": O.num_threads(),
            "kind": "port", "cpu": cpu_model_name(),
            "sample": f"{steps} greedy decode steps after the same {len(prompt)}-token prompt on "
                      f"the same 2B-shape model (C oracle, OpenMP over rows, f16-rounded KV)",
            "prefill_ms": round(prefill_s * 1e3, 1),
            "other_cpu_legs": OTHER_CPU_LEGS}


def cpu_kernels(synth) -> list:
    """The oracle's GEMV / GEMM on the host cores at the ternary-matmul configs:
    6912x2560 M=1 (the FFN up-projection GEMV) and 28672x8192 at M = 1, 8, 64;
    the same algorithmic bytes and ops as the GPU figures."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # the checker, timed here as the reported CPU baseline
    rng = np.random.default_rng(5)
    out = []
    for N, K, M, reps in ((6912, 2560, 1, 50), (28672, 8192, 1, 20), (28672, 8192, 8, 5),
                          (28672, 8192, 64, 3)):
        Wn = synth.i2s_pack(rng.integers(-1, 2, size=(N, K)).astype(np.int8))
        X = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
        sc = np.full(M, 0.01, np.float32)
        run = ((lambda: O.gemv(Wn, X[0], 0.0158, 0.01, K)) if M == 1
               else (lambda: O.gemm(Wn, X, 0.0158, sc, K)))
        run()
        t0 = time.perf_counter()
        for _ in range(reps):
            run()
        dt = (time.perf_counter() - t0) / reps
        nbytes = N * K // 4 + M * K + 4 * M * N + 4
        out.append({"N": N, "K": K, "M": M, "us": round(dt * 1e6, 1),
                    "GBps": round(nbytes / dt / 1e9, 2), "GOPS": round(2 * M * N * K / dt / 1e9, 2),
                    "cores": O.num_threads()})
        log(f"cpu {N}x{K} M={M}: {dt * 1e3:.2f} ms {out[-1]['GBps']} GB/s {out[-1]['GOPS']} GOPS")
    return out


def decode_breakdown(ops, synth, pos: int = 139) -> dict:
    """The decode step's kernels at the 2B shape, rebuilt from the operator
    ABI with 30 layers of their own (zero-coded) weights and caches, each
    kind timed as a graph of its 30 launches (cold weights, so HBM latency
    as in the model), then the whole chain (30 x q|k|v, attention, o_proj,
    gate|up, down) and the LM head (final norm + tied head + argmax, its
    finishing kernel included).  Per-launch microseconds include the launch
    gap of a graph; the attention runs at `pos` + 1 cached positions."""
    L = ops.lib()
    cfg = synth.BITNET_2B
    nl, D, F, H, Hkv, hd, V = cfg.n_layers, cfg.hidden, cfg.ffn, cfg.heads, cfg.kv_heads, 128, cfg.vocab
    Dq, Dkv, max_seq = H * hd, Hkv * hd, 4096
    lay = []
    for _ in range(nl):
        lay.append({k: ops.DeviceArray((n * kk // 4,), np.uint8, zero=True)
                    for k, n, kk in (("qkv", Dq + 2 * Dkv, D), ("o", D, Dq), ("gu", 2 * F, D),
                                     ("down", D, F))})
    kvl = Hkv * max_seq * hd
    kc = ops.DeviceArray((nl * kvl + 64 * hd,), np.uint16, zero=True)
    vc = ops.DeviceArray((nl * kvl + 64 * hd,), np.uint16, zero=True)
    kvl8 = Hkv * ((max_seq + 7) // 8 * 8) * hd   # the octet copy of V the model's attention reads
    vc8 = ops.DeviceArray((nl * kvl8,), np.uint16, zero=True)
    rng = np.random.default_rng(5)
    x = ops.DeviceArray.from_host(rng.standard_normal(D).astype(np.float32))
    ones = ops.DeviceArray.from_host(np.ones(2 * F, np.float32))
    ws = ops.DeviceArray.from_host(np.full(2 * F, 0.016, np.float32))
    q, att = ops.DeviceArray((Dq,), np.float32), ops.DeviceArray((Dq,), np.float32)
    hbuf = ops.DeviceArray((F,), np.float32)
    cs = np.zeros(max_seq * hd, np.float32)
    ops.check(L.oxb_rope_table(cs.ctypes.data, max_seq, hd, cfg.rope_theta), "rope")
    rope = ops.DeviceArray.from_host(cs)
    state = ops.DeviceArray.from_host(np.array([pos, 0, 0, 0, 1 << 20, 0, 0, 0], np.int32))
    hist = ops.DeviceArray((1 << 20,), np.int32, zero=True)
    E = ops.DeviceArray((L.oxb_lm_bytes(V, D),), np.uint8, zero=True)
    logits = ops.DeviceArray((V,), np.float32)
    stream = L.oxb_stream_create()
    kv_b = kvl * 2

    def qkv(l):
        ops.check(L.oxb_bitlinear_qkv(lay[l]["qkv"].ptr, x.ptr, ones.ptr, 1e-5, ws.ptr, Dq, Dkv, hd, D,
                                      q.ptr, kc.ptr + l * kv_b, vc.ptr + l * kv_b, max_seq, rope.ptr,
                                      state.ptr, stream), "qkv")

    def attn(l):
        ops.check(L.oxb_attn_decode_head_v8(q.ptr, kc.ptr + l * kv_b, vc.ptr + l * kv_b,
                                            vc8.ptr + l * kvl8 * 2, state.ptr, 0, 0, 0, 1, H, Hkv,
                                            hd, max_seq, 256, att.ptr, stream), "attention")

    def o(l):
        ops.check(L.oxb_bitlinear_gemv(lay[l]["o"].ptr, att.ptr, ones.ptr, 1e-5, ws.ptr, D, Dq, x.ptr,
                                       1, None, None, None, stream), "o_proj")

    def gu(l):
        ops.check(L.oxb_bitlinear_gateup(lay[l]["gu"].ptr, x.ptr, ones.ptr, 1e-5, ws.ptr, 2 * F, D,
                                         hbuf.ptr, stream), "gate|up")

    def down(l):
        ops.check(L.oxb_bitlinear_gemv(lay[l]["down"].ptr, hbuf.ptr, ones.ptr, 1e-5, ws.ptr, D, F,
                                       x.ptr, 1, None, None, None, stream), "down")

    def lm(_):   # advance 0: the position stays put across replays
        ops.check(L.oxb_lm_head_argmax(x.ptr, ones.ptr, 1e-5, E.ptr, V, D, logits.ptr, state.ptr,
                                       hist.ptr, 0, stream), "lm head")

    out = {"positions": pos + 1}
    for name, fn in (("qkv", qkv), ("attention", attn), ("o_proj", o), ("gate_up", gu),
                     ("down", down)):
        out[name + "_us"] = round(_timed(L, stream, fn, nl) * 1e3, 2)
    out["lm_head_us"] = round(_timed(L, stream, lm, 4) * 1e3, 1)

    def chain(_):
        for l in range(nl):
            qkv(l), attn(l), o(l), gu(l), down(l)
        lm(0)
    out["layers_and_lm_head_us"] = round(_timed(L, stream, chain, 1) * 1e3, 1)
    L.oxb_stream_destroy(stream)
    for a in [kc, vc, vc8, x, ones, ws, q, att, hbuf, rope, state, hist, E, logits] + \
             [b for d in lay for b in d.values()]:
        a.free()
    return out


def gemm_extras(ops, synth) -> dict:
    """The ternary GEMM sweep (28672x8192 and 8192x28672 at M = 8 .. 4096) and
    the 512-token prefill block."""
    gs = []
    for N, K in ((28672, 8192), (8192, 28672)):
        for M in (8, 64, 512, 4096):
            copies = 8 if M <= 64 else 2
            r = gemm_sweep(ops, synth, N, K, M, copies=copies, iters=40 if M < 4096 else 10)
            gs.append(r)
            log(f"gemm {N}x{K} M={M}: {r['us']} us {r['TOPS']} TOPS {r['GBps']} GB/s")
    pb = prefill_block(ops, synth)
    log(f"prefill block M=512: {pb['ms']} ms {pb['TOPS']} TOPS")
    return {"gemm_sweep": gs, "prefill_block": pb}


def generate_surface(pkg, model, path: str, max_tokens: int = 128) -> dict:
    """Tokens/s of the C ABI's streaming generate (oxbitnet_generate,
    rs/lib.rs:130-189) on the same file, as a user of include/oxbitnet.h sees
    it: greedy options (top_k 1, penalty 1: the LM head's argmax) and the
    reference's defaults (top_k 50, T 1, penalty 1.1 over the last 64 tokens:
    drawn on the device).  One warm-up call (graph capture), then one timed
    call each; the rate is taken between the first and the last token the
    callback receives (the decode steps), the call's wall time is reported
    beside it (prefill and tokenizer included).  The ids-level greedy decode
    (oxb_model_decode_greedy) over the same positions is timed for the
    ratio."""
    import ctypes as C
    nat = pkg._native
    L = nat.lib()
    h = L.oxbitnet_load(path.encode(), None)
    if not h:
        raise RuntimeError(L.oxbitnet_error_message())
    prompt = b"The quick brown fox jumps over the lazy dog; generate some more text."
    out = {}
    try:
        for name, (top_k, penalty) in (("greedy", (1, 1.0)), ("reference_defaults", (50, 1.1))):
            g = L.oxbitnet_default_generate_options()
            g.max_tokens, g.top_k, g.repeat_penalty = max_tokens, top_k, penalty
            stamps = []
            tf = nat.TokenFn(lambda t, n, ud: (stamps.append(time.perf_counter()), 0)[1])
            if L.oxbitnet_generate(h, prompt, C.byref(g), tf, None) != 0:
                raise RuntimeError(L.oxbitnet_error_message())
            stamps.clear()
            t0 = time.perf_counter()
            if L.oxbitnet_generate(h, prompt, C.byref(g), tf, None) != 0:
                raise RuntimeError(L.oxbitnet_error_message())
            wall = time.perf_counter() - t0
            n = len(stamps)
            rate = (n - 1) / (stamps[-1] - stamps[0]) if n > 2 else None
            out[name] = {"tokens": n, "tok_s": round(rate, 2) if rate else None,
                         "call_ms": round(wall * 1e3, 2), "top_k": top_k,
                         "repeat_penalty": penalty, "temperature": 1.0, "repeat_last_n": 64}
    finally:
        L.oxbitnet_free(h)
    # the same positions through the ids-level engine: a prompt of the same
    # length, then max_tokens - 1 greedy steps as one run of graph replays
    tok = L.oxb_tokenizer_load(path.encode())
    n_prompt = L.oxb_tokenizer_encode(tok, prompt, 1, None, 0)
    L.oxb_tokenizer_free(tok)
    ids = np.random.default_rng(5).integers(0, model.vocab, n_prompt).astype(np.int32)
    model.reset()
    model.forward(ids, want_logits=False)
    model.decode_greedy(max_tokens - 1)
    model.reset()
    model.forward(ids, want_logits=False)
    t0 = time.perf_counter()
    model.decode_greedy(max_tokens - 1)
    ref = (max_tokens - 1) / (time.perf_counter() - t0)
    for v in out.values():
        v["decode_greedy_tok_s"] = round(ref, 2)
        v["vs_decode_greedy"] = round(v["tok_s"] / ref, 4) if v["tok_s"] else None
    out["prompt_tokens"] = n_prompt
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--cpu-steps", type=int, default=160)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the GEMM sweep, prefill block and long-context runs")
    ap.add_argument("--roofline-only", action="store_true")
    ap.add_argument("--calib-mib", type=int, default=0)
    ap.add_argument("--long-context-only", action="store_true",
                    help="run only the long-context section (2048-token prefill, decode at the "
                         "batch sizes of --lc-batches)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="run only the ternary GEMM sweep and the 512-token prefill block")
    ap.add_argument("--gemm-shape", default="",
                    help="N,K,M: time only the ternary GEMM at that shape (the command the "
                         "GEMM rocprofv3 --pmc runs profile)")
    ap.add_argument("--decode-only", action="store_true",
                    help="stop after the decode measurement (the command the decode counter "
                         "profiles run), logging each phase")
    ap.add_argument("--no-generate", action="store_true",
                    help="skip the oxbitnet_generate (C ABI streaming) timing")
    ap.add_argument("--gen-tokens", type=int, default=128)
    ap.add_argument("--lc-batches", default="1,8,32")
    ap.add_argument("--lc-steps", type=int, default=512)
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
    if args.gemm_only:
        print(json.dumps(gemm_extras(ops, synth)), flush=True)
        return 0
    if args.gemm_shape:
        N, K, M = (int(v) for v in args.gemm_shape.split(","))
        r = gemm_sweep(ops, synth, N, K, M, copies=2, iters=10)
        log(f"gemm {N}x{K} M={M}: {r['us']} us {r['TOPS']} TOPS")
        print(json.dumps({"gemm": r}), flush=True)
        return 0
    if args.roofline_only:
        roof = gemv_roofline(ops, synth, 8192, 28672, copies=16, iters=400)
        if args.calib_mib:
            calib_copy(ops, args.calib_mib)
        print(json.dumps({"roofline_gemv": roof, "calib_copy_mib": args.calib_mib}), flush=True)
        return 0

    t = time.time()
    path = synth.cached_gguf(synth.BITNET_2B, seed=1234)
    log(f"model file {path} ({os.path.getsize(path) / 1e9:.2f} GB, {time.time() - t:.1f}s)")
    if args.long_context_only:
        lc = long_context(pkg, synth, path, steps=args.lc_steps,
                          batches=tuple(int(b) for b in args.lc_batches.split(",")))
        print(json.dumps({"long_context": lc}), flush=True)
        return 0
    t = time.time()
    # the context the C ABI loads with (rs/lib.rs:93: 4096), or more if the run needs it
    max_seq = max(4096, args.prompt + args.steps + args.warmup + 8)
    model = pkg.Model(path, max_seq=max_seq)
    log(f"loaded in {time.time() - t:.1f}s; weights {model.info['weight_bytes'] / 1e9:.3f} GB")

    rng = np.random.default_rng(2024)
    prompt = rng.integers(0, synth.BITNET_2B.vocab, args.prompt).astype(np.int32)
    L = ops.lib()

    # warm-up run (graph capture, caches), then the timed run from a fresh cache
    model.reset()
    model.forward(prompt, want_logits=False)
    if args.decode_only:
        log("warm-up prefill done")
    model.decode_greedy(args.warmup)
    if args.decode_only:
        log(f"warm-up decode ({args.warmup} steps) done")
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
    if args.decode_only:
        print(json.dumps({"decode_tok_s": round(tps, 2), "steps": args.steps,
                          "prompt": args.prompt}), flush=True)
        return 0

    gen = None
    if not args.no_generate:
        gen = generate_surface(pkg, model, path, args.gen_tokens)
        for k in ("greedy", "reference_defaults"):
            v = gen[k]
            log(f"oxbitnet_generate {k}: {v['tokens']} tokens, {v['tok_s']} tok/s "
                f"({v['call_ms']} ms per call); decode_greedy {v['decode_greedy_tok_s']} tok/s")

    # roofline of the ternary GEMV (8192 x 28672, M = 1) and the sweep
    roof = gemv_roofline(ops, synth, 8192, 28672, copies=16, iters=400)
    log(f"gemv 8192x28672: {roof['us']} us, {roof['GBps']} GB/s ({roof['frac'] * 100:.1f}% of peak)")
    sweep = []
    if not args.no_sweep:
        for N, K in ((28672, 8192), (6912, 2560), (3840, 2560), (13824, 2560), (2560, 6912)):
            r = gemv_roofline(ops, synth, N, K, copies=max(4, (600 << 20) // (N * K // 4)),
                              iters=400)
            sweep.append(r)
            log(f"gemv {N}x{K}: {r['us']} us {r['GBps']} GB/s")

    extra = {}
    if not args.no_extra:
        db = decode_breakdown(ops, synth)
        log(f"decode kernels at {db['positions']} positions: " +
            ", ".join(f"{k} {v}" for k, v in db.items() if k.endswith("_us")))
        extra["decode_kernels"] = db
        extra.update(gemm_extras(ops, synth))
        lc = long_context(pkg, synth, path)
        log(f"long context: prefill {lc['prefill_ms']} ms")
        extra["long_context"] = lc

    cpu = None
    if not args.no_cpu:
        t = time.time()
        cpu = cpu_baseline(synth, path, prompt.astype(np.uint32), args.cpu_steps)
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads ({time.time() - t:.1f}s)")
        extra["cpu_kernels"] = cpu_kernels(synth)

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
        "generate": gen,
        "roofline": {"bound": "hbm", "achieved": roof["GBps"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": roof["frac"], "traffic": measured_traffic(),
                     "kernel": "gemv_kernel<PRO_INT8,EPI_STORE> N=8192 K=28672 M=1",
                     "bytes_per_launch": roof["bytes"], "us_per_launch": roof["us"]},
        "gemv_sweep": sweep,
        **extra,
        "cpu_baseline": cpu,
        "device": info["name"],
        "hbm_gib": round(info["hbm_bytes"] / 2**30, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
