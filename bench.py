"""Benchmark of the MI355X decode hot path (one GPU).

Workload: one decode step of a random-init Qwen2.5-1.5B
shaped model (28 layers, Q4_K_M-style weights, tied Q6_K LM head, 2048-token
fp16 KV prefix, on-device top-k 40) captured as one hipGraph.  A "step" is one
replay of that graph; ``value`` is batch-1 decode tokens/s with every input
resident in HBM.  The same line carries the batch-16 step, the quant-GEMV
bandwidth of configs 0/1 on a cold (> 256 MB MALL) rotating weight pool, the
roofline of the dominant kernel and a CPU baseline (the NumPy oracle on the
host cores, bounded sample).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "quant GEMV HBM GB/s (% peak); decode tok/s 1.5B-shape at batch 1/16"
HBM_PEAK_GBPS = 8000.0


def _events(hip):
    return hip.event_create(), hip.event_create()


def time_graph(hip, ex, steps, warmup):
    ex.build_decode_graph()
    ex.replay(warmup)
    hip.synchronize()
    e0, e1 = _events(hip)
    t0 = time.perf_counter()
    hip.event_record(e0)
    ex.replay(steps)
    hip.event_record(e1)
    ms = hip.event_elapsed_ms(e0, e1)
    hip.synchronize()
    wall = time.perf_counter() - t0
    return ms / steps, wall


def prefill_bench(hip, model, n=2048, chunk=512, trials=3, profile_runs=0):
    """Multi-token prefill of an n-token synthetic prompt into sequence 0 of a
    batch-1 executor, chunks of `chunk` columns (vte_amd.core.prefill), timed
    with HIP events around the whole prompt; median of `trials` after one
    untimed run.  With profile_runs > 0: only that many untimed runs (for
    rocprofv3 kernel traces)."""
    from vte_amd.core.hip_graph_executor import HIPGraphExecutor
    from vte_amd.core.prefill import PrefillRunner
    ex = HIPGraphExecutor(hip, model, batch_size=1, max_seq=n + 256)
    runner = PrefillRunner(ex, chunk=chunk)
    prompt = [int(t) for t in np.random.default_rng(0).integers(0, model.cfg.vocab, n)]
    try:
        runner.prefill(prompt, seq=0, start=0)
        if profile_runs:
            for i in range(profile_runs):
                runner.prefill(prompt, seq=0, start=0)
                print(f"profile-prefill: run {i + 1}/{profile_runs}", flush=True)
            return None
        times = []
        for _ in range(trials):
            e0, e1 = _events(hip)
            hip.event_record(e0)
            runner.prefill(prompt, seq=0, start=0)
            hip.event_record(e1)
            hip.synchronize()
            times.append(hip.event_elapsed_ms(e0, e1))
        ms = float(np.median(times))
        return {"prompt": n, "chunk": chunk, "ms": round(ms, 3), "tok_s": round(n / (ms * 1e-3), 1)}
    finally:
        runner.close()
        ex.close()


def time_classes(hip, ex, classes, reps=20):
    """Average time of the launches of ``classes`` in one step, measured with
    HIP events on the executor's stream around replays of a graph holding only
    those launches (same buffers and shapes as the full step)."""
    g, ge = ex.capture_classes(classes)
    try:
        hip.graph_launch(ge)
        hip.synchronize()
        e0, e1 = _events(hip)
        hip.event_record(e0)
        for _ in range(reps):
            hip.graph_launch(ge)
        hip.event_record(e1)
        ms = hip.event_elapsed_ms(e0, e1) / reps
    finally:
        hip.graph_exec_destroy(ge)
        hip.graph_destroy(g)
    return ms


def step_breakdown(hip, ex, prefix, reps=20):
    """Per launch class: launches per step, time per step (us) and GB/s."""
    cfg = ex.cfg
    algo = ex.class_algorithmic_bytes()
    algo["attn"] += cfg.n_layers * ex.B * (prefix + 1) * cfg.n_kv * cfg.head_dim * 2 * 2
    n = {"embed": 1, "attn_in": cfg.n_layers, "attn": cfg.n_layers, "o_proj": cfg.n_layers, "ffn_in": cfg.n_layers,
         "down": cfg.n_layers, "lm_head": 1, "topk": 1}
    out = {}
    for c in ex.FUSED_CLASSES:
        ms = time_classes(hip, ex, [c], reps)
        out[c] = {"launches": n[c], "us_per_step": round(ms * 1e3, 2), "algo_bytes": int(algo[c]),
                  "GBps": round(algo[c] / (ms * 1e-3) / 1e9, 1)}
    return out


MV_CLASSES = ["attn_in", "o_proj", "ffn_in", "down", "lm_head"]


def fused_mv_roofline(hip, ex, reps=20):
    """Roofline of the step's dominant kernel, fused_mv_kernel: every
    quantised mat-vec launch of a batch-1 step (28 norm+QKV+RoPE+append, 28
    o-proj+residual, 28 norm+gate/up+SwiGLU, 28 down+residual, 1 norm+LM
    head): algorithmic bytes per launch over the average launch duration (HIP
    events on the executor's stream around replays of a graph of exactly
    those launches)."""
    algo = ex.class_algorithmic_bytes()
    launches = 4 * ex.cfg.n_layers + 1
    per_launch_bytes = sum(algo[c] for c in MV_CLASSES) / launches
    ms = time_classes(hip, ex, MV_CLASSES, reps) / launches
    gbps = per_launch_bytes / (ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "fused_mv_decode_b1_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
            "kernel": "fused_mv_kernel (all %d quantised mat-vec launches of the batch-1 step)" % launches,
            "avg_launch_us": round(ms * 1e3, 3), "algo_bytes_per_launch": int(per_launch_bytes)}


def persistent_roofline(hip, ex_p, layer_bytes, lm_head_ms, reps=20):
    """Roofline of the default batch-1 step's dominant kernel,
    decode_persistent_kernel (every layer of the step in one launch):
    algorithmic bytes of the layers (weights + the KV rows read and appended)
    over its duration = HIP-event time of the step's ``decode`` node (the
    persistent launch + the LM-head launch) minus the LM-head launch timed
    alone on the per-node graph (same kernel, same shapes)."""
    ms = time_classes(hip, ex_p, ["decode"], reps) - lm_head_ms
    gbps = layer_bytes / (ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_persistent_b1_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
            "kernel": "decode_persistent_kernel (all %d layers of the batch-1 step, one launch)" % ex_p.cfg.n_layers,
            "avg_launch_us": round(ms * 1e3, 3), "algo_bytes_per_launch": int(layer_bytes),
            "timing": "HIP events around graph replays of the decode node, minus the LM-head launch"}


def mfma_b16_roofline(hip, ex, reps=20):
    """Roofline of the batch-16 step's dominant kernel, the gate/up + SwiGLU
    MFMA launch (fused_mm_kernel, 28 per step): algorithmic bytes per launch
    (gate and up weights + the 16 normalised activation columns read + the 16
    SwiGLU columns written) over the average launch duration, HIP events on
    the executor's stream around replays of a graph of the step's 28 launches
    (same buffers and shapes as the step)."""
    cfg, B, K = ex.cfg, ex.B, ex.K
    from vte_amd import synthetic as syn
    per_launch = [syn.matrix_bytes(lw["gate_fmt"], cfg.ffn, cfg.hidden) + syn.matrix_bytes(lw["up_fmt"], cfg.ffn,
                  cfg.hidden) + B * 2 * (cfg.hidden + cfg.ffn) for lw in ex.layers]
    hip.synchronize()
    hip.stream_begin_capture()
    try:
        for lw in ex.layers:
            K.ffn_in(ex.xn, None, cfg.eps, lw["gate"], lw["up"], lw["gate_fmt"], ex.a, B, cfg.hidden, cfg.ffn,
                     stream=hip.stream)
    finally:
        g = hip.stream_end_capture()
    ge = hip.graph_instantiate(g)
    try:
        hip.graph_launch(ge)
        hip.synchronize()
        e0, e1 = _events(hip)
        hip.event_record(e0)
        for _ in range(reps):
            hip.graph_launch(ge)
        hip.event_record(e1)
        ms = hip.event_elapsed_ms(e0, e1) / reps / len(ex.layers)
    finally:
        hip.graph_exec_destroy(ge)
        hip.graph_destroy(g)
    algo = sum(per_launch) / len(per_launch)
    gbps = algo / (ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "fused_mm_gateup_b16_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
            "kernel": "fused_mm_kernel<2, 1, 6> (gate/up + SwiGLU on MFMA, 28 launches of the batch-16 step)",
            "avg_launch_us": round(ms * 1e3, 3), "algo_bytes_per_launch": int(algo),
            "timing": "HIP events around graph replays of the step's 28 gate/up launches"}


def time_greedy(hip, ex, steps, start_pos):
    """Greedy decoding with the token fed back on the device (generate_greedy):
    wall time per step of one call of ``steps`` steps, tokens read at the end."""
    ex.generate_greedy([1] * ex.B, [start_pos] * ex.B, steps)  # captures its graph
    t0 = time.perf_counter()
    ex.generate_greedy([1] * ex.B, [start_pos] * ex.B, steps)
    return (time.perf_counter() - t0) / steps


def time_e2e(hip, ex, steps, start_pos):
    """Per-token loop as a caller runs it: stage token/offset, replay, read top-k, sample."""
    from vte_amd.core.sampler import Sampler
    rng = np.random.default_rng(0)
    toks = [1] * ex.B
    t0 = time.perf_counter()
    for s in range(steps):
        ex.execute_decode_batch(toks, [start_pos + s] * ex.B)
        vals, idx = ex.read_topk()
        toks = [Sampler.sample_candidates(vals[b], idx[b], 0.7, 0.9, rng) for b in range(ex.B)]
    return (time.perf_counter() - t0) / steps


def gemv_bench(hip, K, fmt, n, k, launches=200, pool_bytes=768 << 20, mfma_batch=0, in_dtype="f32"):
    """Average kernel time over a rotating cold pool; returns dict with GB/s.
    Activations fp32 (the BASELINE configs) or fp16 (as inside the decode step);
    the output is fp32."""
    from vte_amd import synthetic as syn
    from vte_amd.bridge import DeviceArray
    raw = syn.random_matrix(fmt, np.random.default_rng(42), n, k)
    copies = max(2, int(np.ceil(pool_bytes / raw.nbytes)))
    pool = DeviceArray(hip, copies * raw.nbytes + 256, np.uint8, f"pool_{fmt}")
    first = DeviceArray.from_numpy(hip, raw, "w0")
    stride = raw.nbytes
    for c in range(copies):
        hip.memcpy_device_to_device(pool.ptr + c * stride, first.ptr, stride)
    M = max(1, mfma_batch)
    xdt = np.float32 if in_dtype == "f32" else np.float16
    x = DeviceArray.from_numpy(hip, np.random.default_rng(1).standard_normal((M, k)).astype(xdt), "x")
    y = DeviceArray(hip, (M, n), np.float32, "y")
    run = (lambda w: K.gemm_mfma(fmt, x, w, y, M, k, n, in_dtype=in_dtype, stream=hip.stream)) if mfma_batch else \
          (lambda w: K.gemv(fmt, x, w, y, M, k, n, in_dtype=in_dtype, stream=hip.stream))
    # launches captured into one graph (as inside the decode step), each on the
    # next cold copy of the weights
    hip.synchronize()
    hip.stream_begin_capture()
    for i in range(launches):
        run(pool.ptr + (i % copies) * stride)
    graph = hip.stream_end_capture()
    gexec = hip.graph_instantiate(graph)
    hip.graph_launch(gexec)
    hip.synchronize()
    e0, e1 = _events(hip)
    hip.event_record(e0)
    hip.graph_launch(gexec)
    hip.event_record(e1)
    ms = hip.event_elapsed_ms(e0, e1) / launches
    hip.graph_exec_destroy(gexec)
    hip.graph_destroy(graph)
    algo = raw.nbytes + M * k * np.dtype(xdt).itemsize + M * n * 4
    for d in (pool, first, x, y):
        d.free()
    return {"shape": f"{n}x{k}", "fmt": fmt, "batch": M, "x": in_dtype, "us": round(ms * 1e3, 3),
            "algo_bytes": int(algo), "GBps": round(algo / (ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(algo / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}


def attn_bench(hip, K, ctx, split=None, B=1, fused=False, launches=40):
    """Split-KV decode attention (12q/2kv, hd 128, fp16 KV) over a cold set of
    KV caches, graph-captured launches.  Algorithmic bytes: KV = B*ctx*1024 B.
    split None: the dispatcher's choice for this context and batch."""
    from vte_amd.bridge import DeviceArray
    from vte_amd.core.split_kv_attention import choose_split
    n_q, n_kv, D = 12, 2, 128
    if split is None:
        split = choose_split(ctx, B, n_kv, hip.get_num_cus())
    per_seq = ctx * n_kv * D
    copies = max(2, int(np.ceil((512 << 20) / (2 * 2 * B * per_seq))))
    kc = [DeviceArray(hip, B * per_seq, np.float16, "kc") for _ in range(copies)]
    vc = [DeviceArray(hip, B * per_seq, np.float16, "vc") for _ in range(copies)]
    for i in range(copies):
        K.fill_normal_f16(kc[i], B * per_seq, 10 + i, 0.5, stream=hip.stream)
        K.fill_normal_f16(vc[i], B * per_seq, 100 + i, 0.5, stream=hip.stream)
    q = DeviceArray.from_numpy(hip, np.random.default_rng(0).standard_normal((B, n_q, D)).astype(np.float16), "q")
    offs = DeviceArray.from_numpy(hip, np.full(B, ctx - 1, np.int32), "offs")
    ms_ = (ctx + split - 1) // split
    pm = DeviceArray(hip, B * n_q * ms_, np.float32, "pm")
    pl = DeviceArray(hip, B * n_q * ms_, np.float32, "pl")
    po = DeviceArray(hip, B * n_q * ms_ * (2 * (D + 2) if fused else D), np.float32, "po")
    po.zero()
    out = DeviceArray(hip, B * n_q * D, np.float16, "out")
    ctr = DeviceArray(hip, 1 + B * n_kv, np.int32, "ctr")
    ctr.zero()
    hip.synchronize()
    hip.stream_begin_capture()
    for i in range(launches):
        K.attn_split_kv(q, kc[i % copies], vc[i % copies], pm, pl, po, out, B, n_q, n_kv, D, 1 / np.sqrt(D), offs,
                        per_seq, split, ms_, dtype="f16", counters=ctr if fused else None, stream=hip.stream)
    g = hip.stream_end_capture()
    ge = hip.graph_instantiate(g)
    hip.graph_launch(ge)
    hip.synchronize()
    e0, e1 = _events(hip)
    hip.event_record(e0)
    hip.graph_launch(ge)
    hip.event_record(e1)
    ms = hip.event_elapsed_ms(e0, e1) / launches
    hip.graph_exec_destroy(ge)
    hip.graph_destroy(g)
    for d in kc + vc + [q, offs, pm, pl, po, out, ctr]:
        d.free()
    algo = B * ctx * 1024
    return {"ctx": ctx, "batch": B, "split": split, "fused_combine": fused, "us": round(ms * 1e3, 3),
            "kv_bytes": algo, "GBps": round(algo / (ms * 1e-3) / 1e9, 1)}


def _host_info():
    """CPU model, core count and the NumPy BLAS backend with its thread count."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas, threads = "unknown", int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    try:
        from threadpoolctl import threadpool_info
        for pool in threadpool_info():
            if pool.get("user_api") == "blas":
                blas = f"{pool.get('internal_api')} {pool.get('version')}"
                threads = int(pool.get("num_threads", threads))
                break
    except Exception:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "blas": blas, "blas_threads": threads}


def _stats(ts):
    ts = sorted(ts)
    return {"median": round(float(np.median(ts)), 6), "min": round(ts[0], 6), "max": round(ts[-1], 6),
            "trials": len(ts)}


def cpu_baseline(trials=5):
    """The NumPy oracle (the reference's CPU arithmetic restated, oracle/) on the
    host cores, bounded samples of the same workloads, >= 3 trials each:

    * decode step: the full 28-layer 1.5B-shaped forward at position 2048,
      fp32 GEMVs, float32 GQA attention (math_refs.py:30-62), the LM head and
      a top-40 selection per row, with the dequantised weights of every layer
      cached once outside the timed region (vte/compiler/dequantizer.py) ->
      tok/s at batch 1 (``value``, 5 trials) and 16 (3 trials);
    * quant GEMV configs 0/1: dequantisation and the fp32 mat-vec timed
      separately (the pattern of tools/validate_gemv_q6k_header_fix.py:63-64);
    * split-KV attention configs 2 and 3b: float32 softmax(q K^T / sqrt(128)) V
      per KV head group.
    """
    from oracle import dequant as odq
    from oracle import step as ost
    from oracle.attention import attention_gqa_f32
    from vte_amd import synthetic as syn
    from vte_amd.core.model_config import QWEN25_1P5B
    from vte_amd.core.weights import SyntheticQwen2
    info = _host_info()
    t_start = time.perf_counter()
    cfg = QWEN25_1P5B.with_(max_seq=2304)
    model = SyntheticQwen2(cfg, seed=0)
    rng = np.random.default_rng(0)
    out = {}
    cache = {}
    # one random KV prefix shared by every layer (the timing does not depend on its values)
    k16 = (0.5 * rng.standard_normal((16, 2304, 2, 128), np.float32)).astype(np.float16)
    v16 = (0.5 * rng.standard_normal((16, 2304, 2, 128), np.float32)).astype(np.float16)
    for B, nt in ((1, trials), (16, max(3, trials - 2))):
        ks, vs = [k16[:B]] * cfg.n_layers, [v16[:B]] * cfg.n_layers
        toks, pos = list(range(1, B + 1)), [2048] * B
        # untimed: dequantises every layer and the LM head once (cached), and warms the pages
        ost.decode_step(model, toks, pos, ks, vs, cache, attn="f32")
        steps = []
        for _ in range(nt):
            s = time.perf_counter()
            logits = ost.decode_step(model, toks, pos, ks, vs, cache, attn="f32")
            np.argpartition(logits, -40, axis=1)[:, -40:]
            steps.append(time.perf_counter() - s)
        out[B] = {"tok_s": _stats([B / t for t in steps]), "step_s": _stats(steps)}
    del cache, k16, v16
    gemv = []
    for fmt, n, k, _ in GEMV_CONFIGS[:4]:
        raw = syn.random_matrix(fmt, np.random.default_rng(42), n, k)
        x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
        nt = trials if n * k < 50_000_000 else max(3, trials - 2)
        td, tm = [], []
        for _ in range(nt):
            s = time.perf_counter()
            w = odq.dequantize_matrix(fmt, raw, n, k)
            td.append(time.perf_counter() - s)
            s = time.perf_counter()
            w @ x
            tm.append(time.perf_counter() - s)
        del w
        algo = raw.nbytes + 4 * (n + k)
        gemv.append({"shape": f"{n}x{k}", "fmt": fmt, "dequant_ms": _stats([1e3 * t for t in td]),
                     "matvec_ms": _stats([1e3 * t for t in tm]),
                     "total_ms_median": round(1e3 * (float(np.median(td)) + float(np.median(tm))), 3),
                     "GBps_median": round(algo / (float(np.median(td)) + float(np.median(tm))) / 1e9, 2)})
    attn = []
    for ctx in (512, 4096, 32768):
        q = rng.standard_normal((12, 128)).astype(np.float32)
        kc = (0.5 * rng.standard_normal((ctx, 2, 128))).astype(np.float16)
        vc = (0.5 * rng.standard_normal((ctx, 2, 128))).astype(np.float16)
        ts = []
        for _ in range(trials):
            s = time.perf_counter()
            attention_gqa_f32(q, kc, vc, ctx, 1 / np.sqrt(128))
            ts.append(time.perf_counter() - s)
        attn.append({"ctx": ctx, "ms": _stats([1e3 * t for t in ts])})
    # config 3b: 16 sequences of U[128, 8192] cached rows
    lens = np.random.default_rng(16).integers(128, 8193, 16)
    qs = rng.standard_normal((16, 12, 128)).astype(np.float32)
    kcs = [(0.5 * rng.standard_normal((n, 2, 128))).astype(np.float16) for n in lens]
    vcs = [(0.5 * rng.standard_normal((n, 2, 128))).astype(np.float16) for n in lens]
    ts = []
    for _ in range(trials):
        s = time.perf_counter()
        for b in range(16):
            attention_gqa_f32(qs[b], kcs[b], vcs[b], int(lens[b]), 1 / np.sqrt(128))
        ts.append(time.perf_counter() - s)
    attn.append({"ctx": "ragged B16 U[128,8192]", "rows": int(lens.sum()), "ms": _stats([1e3 * t for t in ts])})
    return {"value": out[1]["tok_s"]["median"], "unit": "tok/s", "cores": info["blas_threads"], "kind": "port",
            "sample": "NumPy oracle (oracle/) on the host: decode step = 28 of 28 layers (fp32 GEMVs, float32 "
                      "GQA attention) + LM head + top-40 at position 2048, dequant cached; batch 1 "
                      f"{trials} trials, batch 16 {max(3, trials - 2)} (median); GEMV configs 0/1 dequant and "
                      "mat-vec separately; attention configs 2 and 3b (float32)",
            "tok_s_b1": out[1]["tok_s"], "tok_s_b16": out[16]["tok_s"], "gemv": gemv, "attention": attn,
            "host": info, "wall_s": round(time.perf_counter() - t_start, 1)}


def hbm_copy_bandwidth(hip, nbytes=1 << 30, reps=10):
    """Device-to-device copy of nbytes (read + write), median GB/s of (2 x nbytes) / time."""
    from vte_amd.bridge import DeviceArray
    a = DeviceArray(hip, nbytes, np.uint8, "copy_src")
    b = DeviceArray(hip, nbytes, np.uint8, "copy_dst")
    a.zero()
    hip.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = _events(hip)
        hip.event_record(e0)
        hip.memcpy_device_to_device(b.ptr, a.ptr, nbytes)
        hip.event_record(e1)
        hip.synchronize()
        ts.append(hip.event_elapsed_ms(e0, e1))
    a.free()
    b.free()
    return round(2 * nbytes / (float(np.median(ts)) * 1e-3) / 1e9, 1)


def profile_step(B, steps, prefix=2048, classes=None, persistent=False):
    """Kernel-trace / counter workload: one plain device-to-device copy of
    256 MiB (reads and writes exactly 256 MiB: the scale of FETCH_SIZE and
    WRITE_SIZE), then ``steps`` replays of the batch-B decode-step graph, or
    of a graph of only the launch classes ``classes`` (the same graph that
    ``time_classes`` times)."""
    from vte_amd.bridge import DeviceArray, HIPRuntime
    from vte_amd.core.hip_graph_executor import HIPGraphExecutor
    from vte_amd.core.model_config import QWEN25_1P5B
    from vte_amd.core.weights import SyntheticQwen2
    hip = HIPRuntime()
    if not hip.initialize():
        raise SystemExit("HIP initialisation failed")
    a = DeviceArray(hip, 256 << 20, np.uint8, "calib_src")
    b = DeviceArray(hip, 256 << 20, np.uint8, "calib_dst")
    a.zero()
    hip.synchronize()
    hip.memcpy_device_to_device(b.ptr, a.ptr, 256 << 20)
    hip.synchronize()
    a.free()
    b.free()
    ex = HIPGraphExecutor(hip, SyntheticQwen2(QWEN25_1P5B, seed=0), batch_size=B, max_seq=prefix + 256,
                          persistent=persistent)
    ex.fill_kv_prefix(seed=B)
    ex._update_staging_buffers([1] * B, [prefix] * B)
    if classes:
        g, ge = ex.capture_classes(classes)
        replay = lambda: hip.graph_launch(ge)
    else:
        ex.build_decode_graph()
        replay = lambda: ex.replay(1)
    for i in range(steps):
        replay()
        # one replay in flight at a time: the profiler's per-dispatch records
        # stay bounded (thousands of unsynchronised graph dispatches have
        # crashed rocprofv3's kernel tracing)
        hip.synchronize()
        if i % 10 == 0:
            print(f"profile-step: batch {B}, step {i}/{steps}", flush=True)
    hip.synchronize()
    if classes:
        hip.graph_exec_destroy(ge)
        hip.graph_destroy(g)
    ex.close()
    hip.cleanup()


GEMV_CONFIGS = [("q4_k", 8960, 1536, 0), ("q6_k", 1536, 8960, 0), ("q6_k", 151936, 1536, 0),
                ("q8_0", 2048, 2048, 0), ("q4_k", 8960, 1536, 16)]


# (fmt, N, K) of the per-launch method: the reference's own shape (Q4_K
# FFN-down 1536x8960, tools/bench_gemv_q4k_bandwidth.py:66-67) and configs 0/1
REFMETHOD_SHAPES = [("q4_k", 1536, 8960), ("q4_k", 8960, 1536), ("q6_k", 1536, 8960), ("q6_k", 151936, 1536),
                    ("q8_0", 2048, 2048)]
SYMBOL = {"q4_k": "gemv_q4k_kernel", "q6_k": "gemv_q6k_kernel", "q8_0": "gemv_q8_0_kernel"}


def gemv_reference_method(hip, K, shapes=REFMETHOD_SHAPES, iters=500, warmup=300, trials=5):
    """The reference's GEMV bandwidth method (tools/bench_gemv_q4k_bandwidth.py
    run_trial, :166-200): every launch bracketed by its own pair of events
    (launches issued one at a time from the host, so none overlaps the next),
    a 300-launch warm-up, 500 timed launches over a rotating cold pool, the
    event time of an empty kernel subtracted as the dispatch floor, and the
    GEMV's corrected bandwidth divided by that of a plain read of the same
    rows with the GEMV ABI's geometry (one 64-thread block per row,
    ``vte_read_rows_kernel``); median / min / max over 5 trials.  Timed for
    the reference-ABI code-object symbol (fp16 I/O, grid (N, 1), block 64) and
    for the C-ABI mat-vec that the decode step uses (fp16 I/O)."""
    import ctypes
    import statistics
    from vte_amd import synthetic as syn
    from vte_amd.bridge import DeviceArray
    from vte_amd.kernels import HSACO_PATH
    _, f_null = hip.load_kernel(str(HSACO_PATH), "vte_null_kernel")
    _, f_read = hip.load_kernel(str(HSACO_PATH), "vte_read_rows_kernel")
    ev = [(hip.event_create(), hip.event_create()) for _ in range(iters)]

    def timed(launch):
        for i in range(warmup):
            launch(i)
        hip.synchronize()
        for i in range(iters):
            hip.event_record(ev[i][0])
            launch(i)
            hip.event_record(ev[i][1])
        hip.synchronize()
        return sum(hip.event_elapsed_ms(a, b) for a, b in ev) / iters

    out = []
    for fmt, n, k in shapes:
        raw = syn.random_matrix(fmt, np.random.default_rng(42), n, k)
        wbytes = raw.nbytes
        copies = max(2, int(np.ceil((640 << 20) / wbytes)), 40 if wbytes * 40 <= (1 << 30) else 2)
        pool = DeviceArray(hip, copies * wbytes + 256, np.uint8, "refm_pool")
        first = DeviceArray.from_numpy(hip, raw, "refm_w0")
        for c in range(copies):
            hip.memcpy_device_to_device(pool.ptr + c * wbytes, first.ptr, wbytes)
        x = DeviceArray.from_numpy(hip, np.random.default_rng(1).standard_normal((1, k)).astype(np.float16), "refm_x")
        y = DeviceArray(hip, (1, n), np.float16, "refm_y")
        sink = DeviceArray(hip, (n,), np.uint32, "refm_sink")
        _, f_gemv = hip.load_kernel(str(HSACO_PATH), SYMBOL[fmt])
        rb = wbytes // n
        w = lambda i: pool.ptr + (i % copies) * wbytes

        def l_null(i):
            hip.launch_kernel(f_null, (1, 1, 1), (1, 1, 1), [], expected_args=0)

        def l_read(i):
            hip.launch_kernel(f_read, (n, 1, 1), (64, 1, 1),
                              [ctypes.c_void_p(w(i)), ctypes.c_void_p(sink.ptr), ctypes.c_int(rb)], expected_args=3)

        def l_ref(i):
            hip.launch_kernel(f_gemv, (n, 1, 1), (64, 1, 1),
                              [ctypes.c_void_p(x.ptr), ctypes.c_void_p(w(i)), ctypes.c_void_p(y.ptr), ctypes.c_int(1),
                               ctypes.c_int(1), ctypes.c_int(k), ctypes.c_int(n), ctypes.c_void_p(None),
                               ctypes.c_void_p(None), ctypes.c_float(1.0)], expected_args=10)

        def l_capi(i):
            K.gemv(fmt, x, w(i), y, 1, k, n, in_dtype="f16", out_dtype="f16", stream=hip.stream)

        rows = {"null_us": [], "read_us": [], "ref_abi_us": [], "capi_us": []}
        for _ in range(trials):
            for key, fn in (("null_us", l_null), ("read_us", l_read), ("ref_abi_us", l_ref), ("capi_us", l_capi)):
                rows[key].append(timed(fn) * 1e3)
        r = {"shape": f"{n}x{k}", "fmt": fmt, "weight_bytes": int(wbytes), "cold_copies": copies}
        for key, v in rows.items():
            r[key] = round(statistics.median(v), 3)
        for name in ("read", "ref_abi", "capi"):
            gb = [wbytes / max(t - z, 1e-3) / 1e3 for t, z in zip(rows[name + "_us"], rows["null_us"])]
            r[name + "_GBps_corrected"] = round(statistics.median(gb), 1)
        for name in ("ref_abi", "capi"):
            ratio = [(rd - z) / max(t - z, 1e-3) for t, rd, z in
                     zip(rows[name + "_us"], rows["read_us"], rows["null_us"])]
            r[name + "_vs_read"] = {"median": round(statistics.median(ratio), 4), "min": round(min(ratio), 4),
                                    "max": round(max(ratio), 4)}
        r["capi_frac_hbm_peak_corrected"] = round(r["capi_GBps_corrected"] / HBM_PEAK_GBPS, 4)
        out.append(r)
        for d in (pool, first, x, y, sink):
            d.free()
    for a, b in ev:
        hip.event_destroy(a)
        hip.event_destroy(b)
    return out


def gemv_configs(hip, K, launches=200):
    """Quant-GEMV configs 0/1 and the batch-16 MFMA GEMM (config 3a), cold pools."""
    out = []
    for fmt, n, k, mb in GEMV_CONFIGS:
        big = n * k > 50_000_000
        out.append(gemv_bench(hip, K, fmt, n, k, launches=50 if big else launches,
                              pool_bytes=(600 << 20) if big else (768 << 20), mfma_batch=mb))
    return out


def profile_configs():
    """rocprofv3 workload: calibration copy, GEMV configs, attention configs."""
    from vte_amd.bridge import DeviceArray, HIPRuntime
    from vte_amd.kernels import kernels
    hip = HIPRuntime()
    if not hip.initialize():
        raise SystemExit("HIP initialisation failed")
    a = DeviceArray(hip, 256 << 20, np.uint8, "calib_src")
    b = DeviceArray(hip, 256 << 20, np.uint8, "calib_dst")
    a.zero()
    hip.synchronize()
    hip.memcpy_device_to_device(b.ptr, a.ptr, 256 << 20)
    hip.synchronize()
    a.free()
    b.free()
    K = kernels()
    for r in gemv_configs(hip, K, launches=100):
        print("profile-gemv:", json.dumps(r), flush=True)
    for ctx, B in ((512, 1), (4096, 1), (32768, 1), (2049, 1), (2049, 16)):
        print("profile-attn:", json.dumps(attn_bench(hip, K, ctx, B=B)), flush=True)
    hip.cleanup()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="skip the batch-16 step and GEMV sweep")
    ap.add_argument("--profile-step", type=int, default=0, metavar="B",
                    help="profiling run only: a 256 MiB calibration copy, then --steps replays of the batch-B "
                         "step graph (for rocprofv3 kernel traces and counters)")
    ap.add_argument("--profile-prefill", type=int, default=0, metavar="R",
                    help="profiling run only: R untimed 2048-token prefills (chunks of 512)")
    ap.add_argument("--profile-gemv", action="store_true",
                    help="profiling run only: a 256 MiB calibration copy, then the quant-GEMV configs 0/1 "
                         "(Q4_K 8960x1536, Q6_K 1536x8960 and 151936x1536, Q8_0 2048x2048) and the batch-16 "
                         "MFMA GEMM over cold rotating pools, and the split-KV attention configs 2/3b")
    ap.add_argument("--profile-gemv-reference", action="store_true",
                    help="profiling run only: the reference's per-launch GEMV method (reference-ABI symbols, the "
                         "C-ABI mat-vec, the read baseline and the empty kernel) over its five shapes, one trial")
    ap.add_argument("--profile-persistent", action="store_true",
                    help="with --profile-step 1: the persistent form of the step (the default batch-1 step; "
                         "without this flag the per-node graph is profiled)")
    ap.add_argument("--profile-classes", default="", metavar="C1,C2",
                    help="with --profile-step: replay only these launch classes (e.g. attn_in,ffn_in,lm_head)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only (no multi-GPU path is built); "
                                   "--gpus must be 1"}))
        sys.exit(2)
    if args.profile_gemv:
        profile_configs()
        return
    if args.profile_gemv_reference:
        from vte_amd.bridge import HIPRuntime
        from vte_amd.kernels import kernels
        hip = HIPRuntime()
        if not hip.initialize():
            raise SystemExit("HIP initialisation failed")
        for r in gemv_reference_method(hip, kernels(), iters=200, warmup=50, trials=1):
            print("profile-gemv-reference:", json.dumps(r), flush=True)
        hip.cleanup()
        return
    if args.profile_step:
        profile_step(args.profile_step, args.steps,
                     classes=[c for c in args.profile_classes.split(",") if c] or None,
                     persistent=args.profile_persistent)
        return

    from vte_amd.bridge import HIPRuntime
    from vte_amd.core.hip_graph_executor import HIPGraphExecutor
    from vte_amd.core.model_config import QWEN25_1P5B
    from vte_amd.core.weights import SyntheticQwen2
    from vte_amd.kernels import kernels

    hip = HIPRuntime()
    if not hip.initialize():
        print(json.dumps({"error": "HIP initialisation failed"}))
        sys.exit(1)
    K = kernels()
    t_gen = time.perf_counter()
    model = SyntheticQwen2(QWEN25_1P5B, seed=0)
    t_gen = time.perf_counter() - t_gen
    if args.profile_prefill:
        prefill_bench(hip, model, profile_runs=args.profile_prefill)
        hip.cleanup()
        return
    wbytes = model.weight_bytes()
    prefix = 2048
    result = {}
    cfg = QWEN25_1P5B
    kv_layer_bytes = cfg.n_layers * (prefix + 1) * cfg.n_kv * cfg.head_dim * 2 * 2  # K and V rows read + appended
    # the per-node graph of the batch-1 step: its own timing (for comparison),
    # the per-class breakdown, the fused mat-vec roofline and the LM-head time
    ex = HIPGraphExecutor(hip, model, batch_size=1, max_seq=prefix + 256, persistent=False)
    ex.fill_kv_prefix(seed=1)
    ex._update_staging_buffers([1], [prefix])
    ms_g, _ = time_graph(hip, ex, max(20, args.steps // 2), args.warmup)
    ex._update_staging_buffers([1], [prefix])
    roof_mv = fused_mv_roofline(hip, ex)
    breakdown = step_breakdown(hip, ex, prefix)
    algo = ex.class_algorithmic_bytes()
    layer_bytes = sum(algo[c] for c in ("attn_in", "attn", "o_proj", "ffn_in", "down")) + kv_layer_bytes
    lm_head_ms = breakdown["lm_head"]["us_per_step"] * 1e-3
    ex.close()
    graph_b1 = {"ms_per_step": round(ms_g, 4), "tok_s": round(1e3 / ms_g, 2)}
    roof = roof16 = None
    for B in ([1] if args.quick else [1, 16]):
        ex = HIPGraphExecutor(hip, model, batch_size=B, max_seq=prefix + 256)  # batch 1: the persistent step
        ex.fill_kv_prefix(seed=B)
        ex._update_staging_buffers([1] * B, [prefix] * B)
        ms, wall = time_graph(hip, ex, args.steps, args.warmup)
        e2e = time_e2e(hip, ex, 20, prefix)
        greedy = time_greedy(hip, ex, 64, prefix)
        if B == 1:
            assert ex.persistent, "the batch-1 step of this model runs the persistent kernel"
            ex._update_staging_buffers([1] * B, [prefix] * B)
            roof = persistent_roofline(hip, ex, layer_bytes, lm_head_ms)
            status = ex.decode_status()
            if status:
                raise RuntimeError(f"persistent decode step error flags {status:#x}")
        else:
            roof16 = mfma_b16_roofline(hip, ex)
        kv_read = cfg.n_layers * (prefix + 1) * cfg.n_kv * cfg.head_dim * 2 * 2 * B
        step_bytes = wbytes + kv_read
        result[B] = {"ms_per_step": ms, "tok_s": B / (ms * 1e-3), "wall_s": wall, "e2e_ms_per_step": e2e * 1e3,
                     "greedy_ms_per_step": greedy * 1e3,
                     "step_bytes": step_bytes, "step_GBps": step_bytes / (ms * 1e-3) / 1e9}
        ex.close()

    gemv = [] if args.quick else gemv_configs(hip, K)
    gemv_refm = [] if args.quick else gemv_reference_method(hip, K)
    attn = []
    if not args.quick:
        for ctx in (512, 4096, 32768):
            attn.append(attn_bench(hip, K, ctx))
        attn.append(attn_bench(hip, K, 2049))
        attn.append(attn_bench(hip, K, 2049, fused=True))
        attn.append(attn_bench(hip, K, 2049, B=16))
    prefill = None if args.quick else prefill_bench(hip, model)
    cpu = None if args.no_cpu else cpu_baseline()
    r1 = result[1]
    line = {
        "metric": METRIC, "value": round(r1["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r1["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k/q6_k weights, f16 activations, f32 accumulate",
        "data": "synthetic (random-init Q4_K_M-style weights, random fp16 KV prefix)",
        "config": {"workload": "config4: Qwen2.5-1.5B-shape decode step as one hipGraph (embedding, the "
                               "persistent 28-layer kernel, norm + LM head, top-k), batch 1, 2048-token fp16 "
                               "KV prefix, on-device top-k 40",
                   "layers": 28, "hidden": 1536, "ffn": 8960, "heads": "12q/2kv x128", "vocab": 151936,
                   "kv_prefix": prefix, "batch": 1},
        "step_GBps_b1": round(r1["step_GBps"], 1),
        "step_frac_hbm_b1": round(r1["step_GBps"] / HBM_PEAK_GBPS, 4),
        "e2e_tok_s_b1": round(1e3 / r1["e2e_ms_per_step"], 2),
        "greedy_tok_s_b1": round(1e3 / r1["greedy_ms_per_step"], 2),
        "weight_gen_s": round(t_gen, 1),
    }
    if 16 in result:
        r16 = result[16]
        line.update({"tok_s_b16": round(r16["tok_s"], 2), "ms_per_step_b16": round(r16["ms_per_step"], 4),
                     "step_GBps_b16": round(r16["step_GBps"], 1),
                     "e2e_tok_s_b16": round(16e3 / r16["e2e_ms_per_step"], 2),
                     "greedy_tok_s_b16": round(16e3 / r16["greedy_ms_per_step"], 2)})
    line["graph_b1"] = graph_b1  # the same step as a graph of per-node launches (VTE_PERSISTENT=0)
    if gemv:
        line["gemv"] = gemv
        line["gemv_reference_method"] = gemv_refm
    if attn:
        line["attention"] = attn
    if prefill:
        line["prefill"] = prefill
    line["hbm_copy_GBps"] = hbm_copy_bandwidth(hip)
    line["hbm_peak_GBps"] = HBM_PEAK_GBPS
    line["roofline"] = roof
    if roof16:
        line["roofline_b16"] = roof16
    line["roofline_graph_fused_mv"] = roof_mv
    line["step_breakdown_b1"] = breakdown
    if cpu:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    hip.cleanup()


if __name__ == "__main__":
    main()
