#!/usr/bin/env python3
"""bench.py -- paged decode attention at the Llama-3-8B shape on one MI355X.

Workload (the metric's config): 32 query heads,
8 KV heads, head_dim 128, bf16 Q/K/V ~ N(0, 1); 64 sequences with context
lengths uniform in [512, 4096] (seed 2); block size 16; block tables are
disjoint slices of a seeded permutation of a 20000-block pool.

One step = what the engine does per layer for this batch
(crates/engine/src/model.rs:309-319): write_kv of the 64 new tokens
(reshape_and_cache), then decode_attention over ctx + 1 keys per sequence
(split-K kernel + reduce kernel).  Steps alternate between two pool layers
(2.6 GB) so that the 256 MB MALL cannot serve one step's KV from the last.

value = algorithmic decode bytes per step / step time, in GB/s, where the
algorithmic bytes are every key's K and V once per KV head (bf16), the q and
out rows, and the block-table entries.  attention_rows_per_s = 64 / step
time: one layer's decode attention rows per second (not model tokens).
roofline.achieved = the same bytes / the split-K kernel's average duration,
timed live with HIP events around each launch.

The default run prints that cfg2 line with three nested records for the
north_star's other targets, each with its own roofline and CPU baseline:
"cfg5" (prefix-shared decode at the Llama-3-70B layer shape, HBM roofline on
the unique bytes), "cfg3" (chunked prefill, bf16 MFMA roofline on the
causal-aware FLOPs) and "cfg4" (the full 32-layer mixed step of the
Llama-3-8B-shaped model: model tokens/s and decode tokens/s, the metric's
"tokens/s", with the GEMMs' MFMA roofline and per-kernel ms per step).
--config cfg3 / cfg5 / cfg4 / cfg4a print one config's full line instead;
--headline-only drops the nested records.
"""
import argparse
import ctypes
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

METRIC = "paged decode attn HBM GB/s (% of peak) + tokens/s, Llama-3-8B shape, 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def _load_package():
    import __graft_entry__ as g
    return g._load_package()


def cpu_info():
    model = platform.processor() or ""
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, avail


def cpu_threads(rows, args):
    """Threads for the CPU baseline: every CPU this process may run on (its
    affinity), within the job's CPU share when the environment states one
    (OMP_NUM_THREADS: the GPU box allots 16 CPUs to a one-GPU job and sets it
    to 16), and at most one per row (the reference's CPU attention is parallel
    over rows only, attention.rs:54-71, rayon's default pool).  Returns (used,
    available by affinity, share or None)."""
    _, avail = cpu_info()
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "") or 0) or None
    except ValueError:
        share = None
    n = avail if share is None else min(avail, share)
    if args.cpu_threads:
        n = min(n, args.cpu_threads)
    return max(1, min(n, rows)), avail, share


def profile_record(kernel, workload):
    """The committed rocprofv3 --pmc record (profiles/*.json) for this kernel
    and workload, or None.  A record counts only while the kernel source it
    was measured on is unchanged (sha256 prefix of the source file)."""
    import hashlib
    for p in sorted((ROOT / "profiles").glob("*.json")):
        try:
            rec = json.loads(p.read_text())
        except (OSError, ValueError):
            continue
        if rec.get("kernel") != kernel or rec.get("workload") != workload:
            continue
        src = ROOT / rec.get("source", "")
        if not src.is_file():
            continue
        if hashlib.sha256(src.read_bytes()).hexdigest()[:16] != rec.get("source_sha256_16"):
            continue
        return rec
    return None


def traffic_record(kernel, workload):
    """Counter-measured HBM bytes per launch (FETCH_SIZE and WRITE_SIZE,
    scaled by a device copy's readings), or None."""
    rec = profile_record(kernel, workload)
    return rec.get("hbm_bytes_per_launch") if rec else None


# Under sustained bf16 MFMA load the GPU's clocks take tens of milliseconds to
# settle: the first ~150 calls of the cfg3 prefill step run at 270-340 us,
# later ones at ~245 us, call after call.  The MFMA-bound configs therefore
# run their step for this long before the warmup and the timed steps, so
# that they report the sustained rate.  (The HBM-bound decode step runs at its
# steady rate from the second call.)
MFMA_SETTLE_S = 0.25


def settle(torch, fn, seconds):
    """Run fn(i) until `seconds` of wall time have passed (GPU synchronized)."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        fn(i)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return i


def time_steps(torch, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def bench_decode(vo, W, orc, args, cfg):
    import torch
    heads, kvh, hd, bs = cfg["heads"], 8, 128, 16
    ctx = cfg["ctx"]
    layers = args.layers
    backend = vo.HipBackend(device=0, max_seqs=len(ctx), max_rows=W.FILL_ROWS,
                            max_table_entries=cfg["num_blocks"], max_query_heads=heads)
    wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=bs, num_blocks=cfg["num_blocks"], context_lens=ctx, seed=cfg["seed"],
                 num_layers=layers, fill_layers=list(range(layers)),
                 shared_prefix=cfg.get("shared_prefix", 0),
                 shared_count=cfg.get("shared_count", 0), keep_host=not args.no_cpu)
    S = len(ctx)
    out = torch.empty_like(wl.q)
    # The step's metadata crosses to the device once (as in a real step, where
    # all layers share it); the ops below then take raw C-ABI arguments.
    backend.write_kv(wl.pool, 0, wl.k_new, wl.v_new, wl.meta)
    meta_h = backend.step_meta(wl.pool).handle
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lib = vo.lib
    kp, vp = ctypes.c_void_p(wl.k_new.data_ptr()), ctypes.c_void_p(wl.v_new.data_ptr())
    qp, op = ctypes.c_void_p(wl.q.data_ptr()), ctypes.c_void_p(out.data_ptr())
    width = kvh * hd

    def step(i):
        layer = i % layers
        if args.unfused:
            rc = lib.vo_write_kv(wl.pool.handle, layer, kp, vp, S, width, meta_h, stream)
            rc |= lib.vo_decode_attention(qp, S, heads * hd, wl.pool.handle, layer, meta_h, op,
                                          stream)
        else:
            # The same two ops as one call (one launch where the step allows it).
            rc = lib.vo_decode_attention_write_kv(qp, S, heads * hd, kp, vp, width,
                                                  wl.pool.handle, layer, meta_h, op, stream)
        if rc:
            raise RuntimeError(f"C-ABI call failed: {rc}")

    sec = time_steps(torch, step, args.steps, args.warmup)
    # Per-kernel durations, live, over a second timed pass with event timing on.
    vo.profile_reset()
    vo.enable_profiling(True)
    sec_prof = time_steps(torch, step, args.steps, 0)
    vo.enable_profiling(False)
    prof = vo.profile()

    nbytes = wl.decode_bytes()
    # HBM bytes: each physical block once (equal to nbytes unless rows alias a
    # shared prefix, whose blocks are then read from HBM once and hit in cache).
    ubytes = wl.decode_unique_bytes()
    gbs = nbytes / sec / 1e9
    split = prof.get("decode_splitk", {})
    split_s = split.get("avg_ms", 0.0) / 1e3
    achieved = ubytes / split_s / 1e9 if split_s else None
    workload_name = cfg["name"]
    traffic = traffic_record("decode_splitk", workload_name)
    line = {
        "metric": METRIC if cfg["name"].startswith("cfg2") else cfg["metric"],
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": workload_name,
            "seqs": S, "query_heads": heads, "kv_heads": kvh, "head_dim": hd, "block_size": bs,
            "pool_blocks": cfg["num_blocks"], "context": cfg["ctx_desc"],
            "keys_total": int(wl.row_num_keys().sum()),
            "step": ("write_kv(new tokens) + decode_attention (split-K + reduce)" +
                     (", two calls" if args.unfused else
                      ", one call: vo_decode_attention_write_kv")),
            "layers_rotated": layers,
            "split_keys": int(os.environ.get("VO_DECODE_SPLIT", "2048")),  # the backend's default
        },
        # One layer's decode attention: S rows per step (model tokens/s are
        # the cfg4 record's).
        "attention_rows_per_s": round(S / sec, 1),
        # HBM bytes move once per physical block, so the fraction of peak is
        # taken on the unique bytes (equal to the algorithmic bytes when no
        # block is shared, as in cfg2).
        "pct_of_hbm_peak": round(100.0 * ubytes / sec / 1e9 / HBM_PEAK_GBS, 2),
        "algorithmic_bytes_per_step": nbytes,
        "unique_bytes_per_step": ubytes,
        "kernels_us": {k: round(v["avg_ms"] * 1e3, 2) for k, v in prof.items()},
        "ms_per_step_event_timed": round(sec_prof * 1e3, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_splitk",
            "achieved": round(achieved, 1) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": traffic,
            "bytes": "unique (each physical block once)",
            "achieved_logical": round(nbytes / split_s / 1e9, 1) if split_s else None,
        },
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(orc, W, wl, nbytes, args)
    return line


def cpu_baseline(orc, W, wl, nbytes, args):
    """The oracle (C restatement of the reference's CPU attention, row-parallel
    like rayon) on the same workload: the whole decode_attention of the step,
    repeated until about args.cpu_seconds have passed."""
    model, _ = cpu_info()
    threads, avail, share = cpu_threads(wl.rows, args)
    pool = W.oracle_pool(orc, wl)
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while True:
        t0 = time.perf_counter()
        W.oracle_attention(orc, wl, pool=pool, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() >= t_end or len(times) >= 2000:
            break
    med = float(np.median(times))
    t0 = time.perf_counter()
    W.oracle_attention(orc, wl, pool=pool, threads=1)
    single = time.perf_counter() - t0
    S = wl.rows
    return {
        "value": round(nbytes / med / 1e9, 2),
        "unit": "GB/s",
        "attention_rows_per_s": round(S / med, 2),
        "ms_per_step": round(med * 1e3, 2),
        "single_thread_ms_per_step": round(single * 1e3, 2),
        "cores": threads,
        "cores_available": avail,
        "cpu_share": share,
        "kind": "port",
        "cpu": model,
        "sample": (f"full decode_attention of the same step ({S} rows, f32 oracle on the bf16 "
                   f"inputs), median of {len(times)} runs; same algorithmic-byte definition"),
    }


def cpu_baseline_model(orc, W, cfg, ctx, new, args):
    """The oracle's Llama layer (model.rs:269-356 restated in C) on a bounded
    sample of the cfg4 step: one decoder layer for 32 of its 1280 rows -- 8
    decode rows (the step's first 8 sequences, their cached contexts) and 24
    rows of a prefill chunk (positions 2024..2047 of the chunk whose context
    is 1536) -- with f32 weights ~ N(0, 0.02), plus the LM head for 8 rows.
    Scaled linearly to the step: 32 layers x 1280 rows and 258 LM-head rows
    (the GEMMs, 94% of the reference's CPU time, scale with rows)."""
    model_name, _ = cpu_info()
    threads, avail, share = cpu_threads(32, args)
    rng = np.random.default_rng(14)
    H, F, V, hd = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.head_dim
    KVH, NH = cfg.num_key_value_heads, cfg.num_attention_heads
    qd, kvd = NH * hd, KVH * hd

    def nrm(o, i):
        return (rng.standard_normal((o, i), np.float32) * np.float32(0.02)).astype(np.float32)

    L = dict(wq=nrm(qd, H), wk=nrm(kvd, H), wv=nrm(kvd, H), wo=nrm(H, qd), w_gate=nrm(F, H),
             w_up=nrm(F, H), w_down=nrm(H, F), norm=np.ones(H, np.float32))
    embed = nrm(V, H)
    dec = [int(c) for c in ctx[:8]]
    chunk_ctx, chunk_rows = 1536 + 512 - 24, 24
    seqs = [(c, 1) for c in dec] + [(chunk_ctx, chunk_rows)]
    bs = 16
    nblk = [-(-(c + n) // bs) for c, n in seqs]
    perm = rng.permutation(sum(nblk)).astype(np.uint32)
    tables, at = [], 0
    for b in nblk:
        tables.append(perm[at:at + b])
        at += b
    pool = orc.Pool(1, sum(nblk), bs, KVH, hd)
    for (c, _), t in zip(seqs, tables):
        if c:
            slots = [int(t[p // bs]) * bs + p % bs for p in range(c)]
            pool.write_kv(0, rng.standard_normal((c, kvd), np.float32),
                          rng.standard_normal((c, kvd), np.float32), slots)
    meta = orc.prefill_meta([(c, n, t) for (c, n), t in zip(seqs, tables)], bs)
    inv = orc.rope_inv_freq(hd, cfg.rope_theta, **cfg.rope_scaling)
    cos, sin = orc.rope_table(inv, 8192 + 1024)
    rows = len(meta["positions"])
    x = rng.standard_normal((rows, H), np.float32)
    eps = np.float32(cfg.rms_norm_eps)

    def layer():
        n = orc.rmsnorm(x, L["norm"], eps)
        q = orc.rope_apply(orc.matmul(n, L["wq"], threads), meta["positions"], cos, sin)
        k = orc.rope_apply(orc.matmul(n, L["wk"], threads), meta["positions"], cos, sin)
        v = orc.matmul(n, L["wv"], threads)
        pool.write_kv(0, k, v, meta["slot_mapping"])
        a = pool.attention(q, 0, tables, meta["row_seq"], meta["row_num_keys"], threads)
        h = orc.add(x, orc.matmul(a, L["wo"], threads))
        n = orc.rmsnorm(h, L["norm"], eps)
        act = orc.silu_mul(orc.matmul(n, L["w_gate"], threads), orc.matmul(n, L["w_up"], threads))
        return orc.add(h, orc.matmul(act, L["w_down"], threads))

    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while True:
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() >= t_end or len(times) >= 50:
            break
    t_layer = float(np.median(times))
    t0 = time.perf_counter()
    orc.argmax(orc.matmul(orc.rmsnorm(x[:8], L["norm"], eps), embed, threads))
    t_head = time.perf_counter() - t0
    step = cfg.num_hidden_layers * t_layer * (1280 / rows) + t_head * (258 / 8)
    return {
        "value": round(1280 / step, 2), "unit": "tokens/s", "cores": threads,
        "cores_available": avail, "cpu_share": share, "kind": "port",
        "cpu": model_name, "est_ms_per_step": round(step * 1e3, 1),
        "sample": (f"one decoder layer for {rows} of the step's 1280 rows (8 decode rows with "
                   f"their contexts, 24 rows of the 1536-context chunk) and the LM head for 8 "
                   f"rows, f32 oracle, median of {len(times)} layer runs; scaled to 32 layers x "
                   f"1280 rows + 258 LM-head rows"),
    }


def bench_prefill(vo, W, orc, args):
    import torch
    heads, kvh, hd, bs = 32, 8, 128, 16
    ctx = W.cfg3_context_lens()
    backend = vo.HipBackend(device=0, max_seqs=8, max_rows=W.FILL_ROWS, max_table_entries=12000,
                            max_query_heads=heads)
    wl = W.build(vo, backend, kind="prefill", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=bs, num_blocks=12000, context_lens=ctx, num_new=[512] * 8, seed=3,
                 keep_host=not args.no_cpu)
    out = torch.empty_like(wl.q)

    def step(i):
        backend.write_kv(wl.pool, 0, wl.k_new, wl.v_new, wl.meta)
        backend.prefill_attention(wl.q, wl.pool, 0, wl.meta, out=out)

    settled = settle(torch, step, MFMA_SETTLE_S)
    n = max(20, args.steps // 2)
    sec = time_steps(torch, step, n, 5)
    vo.profile_reset()
    vo.enable_profiling(True)
    time_steps(torch, step, n, 0)
    vo.enable_profiling(False)
    prof = vo.profile()
    flops = wl.attention_flops()
    kern = max(prof.items(), key=lambda kv: kv[1]["total_ms"])
    k_s = kern[1]["avg_ms"] / 1e3
    workload = "cfg3: 8 seqs x 512-row chunk, ctx U[0,8192] seed 3"
    rec = profile_record(kern[0], workload) or {}
    return {
        "metric": "chunked prefill attention TFLOP/s (causal-aware), Llama-3-8B shape, 1 GPU",
        "value": round(flops / sec / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "step": "write_kv + prefill_attention"},
        "steps": n, "warmup": 5, "settle": {"seconds": MFMA_SETTLE_S, "steps": settled},
        "kernels_us": {k: round(v["avg_ms"] * 1e3, 2) for k, v in prof.items()},
        "roofline": {"bound": "mfma", "kernel": kern[0],
                     "achieved": round(flops / k_s / 1e12, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / k_s / 1e12 / BF16_PEAK_TFLOPS, 4),
                     "traffic": rec.get("hbm_bytes_per_launch"),
                     # Cycles the MFMA pipe was busy / all cycles, from the
                     # committed counter record (SQ_VALU_MFMA_BUSY_CYCLES).
                     "mfma_busy": rec.get("mfma_busy_frac")},
        "cpu_baseline": None if args.no_cpu else cpu_baseline_prefill(orc, W, wl, args),
    }


def cpu_baseline_prefill(orc, W, wl, args):
    """The oracle's prefill_attention (the reference's CPU attention restated
    in C, row-parallel) on a bounded sample of the cfg3 step: every 8th row of
    the 4096 (512 rows, the same positions in every sequence), repeated for
    about args.cpu_seconds.  Reported as causal-aware TFLOP/s of the sampled
    rows, the unit of the GPU figure; the whole step would take 8x as long."""
    model, _ = cpu_info()
    rows = np.arange(0, wl.rows, 8)
    threads, avail, share = cpu_threads(len(rows), args)
    pool = W.oracle_pool(orc, wl)
    flops = int(wl.row_num_keys()[rows].sum()) * wl.heads * 4 * wl.head_dim
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while True:
        t0 = time.perf_counter()
        W.oracle_attention(orc, wl, pool=pool, rows=rows, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() >= t_end or len(times) >= 200:
            break
    med = float(np.median(times))
    return {
        "value": round(flops / med / 1e12, 4), "unit": "TFLOP/s",
        "est_ms_per_step": round(med * 1e3 * wl.rows / len(rows), 1),
        "cores": threads, "cores_available": avail, "cpu_share": share, "kind": "port",
        "cpu": model,
        "sample": (f"prefill_attention of {len(rows)} of the step's {wl.rows} rows (every 8th, "
                   f"f32 oracle on the bf16 inputs), median of {len(times)} runs; causal-aware "
                   f"FLOPs of those rows; est_ms_per_step scales by rows"),
    }


def bench_mixed(vo, W, orc, args):
    """BASELINE config 4's attention step: 256 decode sequences (lognormal
    context, median 1024) + two 512-row chunks in one write_kv +
    prefill_attention call (the decode rows run on the split-K kernel, the
    chunks on the MFMA prefill kernel)."""
    import torch
    heads, kvh, hd, bs = 32, 8, 128, 16
    ctx, new = W.cfg4_attention_lens()
    backend = vo.HipBackend(device=0, max_seqs=len(ctx), max_rows=W.FILL_ROWS,
                            max_table_entries=30000, max_query_heads=heads)
    wl = W.build(vo, backend, kind="prefill", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=bs, num_blocks=30000, context_lens=ctx, num_new=new, seed=4,
                 num_layers=args.layers, fill_layers=list(range(args.layers)), keep_host=False)
    out = torch.empty_like(wl.q)

    def step(i):
        layer = i % args.layers
        backend.write_kv(wl.pool, layer, wl.k_new, wl.v_new, wl.meta)
        backend.prefill_attention(wl.q, wl.pool, layer, wl.meta, out=out)

    settle(torch, step, MFMA_SETTLE_S)
    sec = time_steps(torch, step, args.steps, args.warmup)
    vo.profile_reset()
    vo.enable_profiling(True)
    time_steps(torch, step, args.steps, 0)
    vo.enable_profiling(False)
    prof = vo.profile()
    dec = int((np.asarray(new) == 1).sum())
    return {
        "metric": "mixed continuous-batching attention step (cfg4 shape), 1 GPU",
        "value": round(wl.rows / sec, 1), "unit": "tokens/s", "n_gpus": 1,
        "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg4 attention: 256 decode (lognormal median 1024, sigma 1, "
                               "clip [128, 8192], seed 4) + 2 x 512-row chunks (ctx 0, 1536)",
                   "step": "write_kv + prefill_attention (one call, mixed rows)",
                   "decode_row_routing": os.environ.get("VO_PREFILL_DECODE_ROWS", "1") != "0"},
        "decode_tokens_per_s": round(dec / sec, 1),
        "kernels_us": {k: round(v["avg_ms"] * 1e3, 2) for k, v in prof.items()},
    }


def bench_model(vo, W, orc, args):
    """one full mixed continuous-batching step of a
    random-init Llama-3-8B-shaped model (32 layers, hidden 4096, 32q/8kv heads,
    head_dim 128, FFN 14336, vocab 128256, theta 500000), bf16 weights
    ~ N(0, 0.02) drawn on the GPU: 256 decode sequences (context lognormal,
    median 1024, clipped to [128, 8192]) plus two 512-token prefill chunks in
    one step (1280 rows).  One step = Llama::forward (model.rs:269-356) through
    the C ABI: embed, 32 x (rmsnorm, QKV GEMM, fused RoPE + cache write,
    attention, O GEMM + residual, rmsnorm, gate/up GEMM, silu_mul, down GEMM +
    residual), last-row rmsnorm, LM head GEMM, argmax with its host copy."""
    import importlib
    import torch
    M = importlib.import_module("vllm_oxide_amd.model")
    cfg = W.llama3_8b_config(args.model_layers)
    hd, H, F, V = cfg.head_dim, cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    ctx, new = W.cfg4_attention_lens()
    S, T = len(ctx), int(np.sum(new))
    backend = vo.HipBackend(device=0, max_seqs=S, max_rows=W.FILL_ROWS,
                            max_table_entries=30000, max_query_heads=cfg.num_attention_heads)
    num_blocks = 30000
    wl = W.build(vo, backend, kind="prefill", heads=cfg.num_attention_heads,
                 kv_heads=cfg.num_key_value_heads, head_dim=hd, block_size=16,
                 num_blocks=num_blocks, context_lens=ctx, num_new=new, seed=4,
                 num_layers=cfg.num_hidden_layers, fill_layers=range(cfg.num_hidden_layers),
                 keep_host=False)
    del wl.ctx_kv[:]
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(44)

    def nrm(o, i):
        return (torch.randn((o, i), generator=gen, device="cuda:0", dtype=torch.float32)
                * 0.02).to(torch.bfloat16)

    ones = torch.ones(H, dtype=torch.bfloat16, device="cuda:0")
    weights = dict(embed=nrm(V, H), final_norm=ones, layers=[
        dict(attn_norm=ones, wq=nrm(qd, H), wk=nrm(kvd, H), wv=nrm(kvd, H), wo=nrm(H, qd),
             mlp_norm=ones, w_gate=nrm(F, H), w_up=nrm(F, H), w_down=nrm(H, F))
        for _ in range(cfg.num_hidden_layers)])
    mc = M.ModelConfig(H, F, cfg.num_hidden_layers, cfg.num_attention_heads,
                       cfg.num_key_value_heads, V, cfg.max_position_embeddings,
                       cfg.rms_norm_eps, cfg.rope_theta, dict(cfg.rope_scaling))
    ec = M.EngineConfig(max_batch_tokens=T, max_seqs=S, max_model_len=8192 + 1024,
                        block_size=16, num_blocks=num_blocks)
    model = M.Llama(backend, mc, ec, weights)
    del weights
    torch.cuda.empty_cache()
    tokens = [int(t) for t in np.random.default_rng(4).integers(0, V, T)]

    def step(i):
        model.prefill(wl.pool, tokens, wl.meta)

    sec = time_steps(torch, step, args.steps, args.warmup)
    vo.profile_reset()
    vo.enable_profiling(True)
    prof_steps = max(3, min(args.steps, 10))
    time_steps(torch, step, prof_steps, 0)
    vo.enable_profiling(False)
    prof = vo.profile()
    L = cfg.num_hidden_layers
    gemm_flops = (L * 2 * T * H * (qd + 2 * kvd + qd + 2 * F + F) + 2 * S * H * V)
    mm = prof.get("matmul", {"avg_ms": float("nan"), "calls": 0})
    mm_ms_step = mm["avg_ms"] * mm["calls"] / prof_steps
    achieved = gemm_flops / (mm_ms_step * 1e-3) / 1e12
    return {
        "metric": "full mixed continuous-batching step tokens/s (Llama-3-8B shape, cfg4), 1 GPU",
        "value": round(T / sec, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights N(0, 0.02), random token ids and cached K/V)",
        "config": {"workload": f"cfg4: Llama-3-8B shape, {L} layers, 256 decode (lognormal median "
                               "1024, sigma 1, clip [128, 8192], seed 4) + 2 x 512-token "
                               "prefill chunks (ctx 0, 1536); 1280 rows; block 16",
                   "step": "Llama::forward through the C ABI incl. argmax host copy"},
        "decode_tokens_per_s": round(256 / sec, 1),
        "roofline": {"bound": "mfma", "kernel": "hipBLASLt GEMMs (sum)",
                     "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
        "gemm_tflop_per_step": round(gemm_flops / 1e12, 3),
        "kernels_ms_per_step": {k: round(v["avg_ms"] * v["calls"] / prof_steps, 4)
                                for k, v in sorted(prof.items(),
                                                   key=lambda kv: -kv[1]["avg_ms"] * kv[1]["calls"])},
        "cpu_baseline": None if args.no_cpu else cpu_baseline_model(orc, W, cfg, ctx, new, args),
    }


def bench_model_decode(vo, W, orc, args):
    """Decode-only steps of the random-init Llama-3-8B-shaped model: S
    sequences (context lognormal, median 1024, clipped to [128, 8192]) each
    add one token per step; one step = Llama::decode through the C ABI,
    argmax included.  Prints one line per batch size in --decode-batches."""
    import importlib
    import torch
    M = importlib.import_module("vllm_oxide_amd.model")
    cfg = W.llama3_8b_config(args.model_layers)
    hd, H, F, V = cfg.head_dim, cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    batches = [int(b) for b in args.decode_batches.split(",")]
    S_max = max(batches)
    ctx, _ = W.cfg4_attention_lens(num_decode=S_max, chunk_ctx=())
    backend = vo.HipBackend(device=0, max_seqs=S_max, max_rows=W.FILL_ROWS,
                            max_table_entries=40000, max_query_heads=cfg.num_attention_heads)
    num_blocks = int(sum(-(-(int(c) + 1) // 16) for c in ctx)) + 64
    wl = W.build(vo, backend, kind="decode", heads=cfg.num_attention_heads,
                 kv_heads=cfg.num_key_value_heads, head_dim=hd, block_size=16,
                 num_blocks=num_blocks, context_lens=ctx, seed=5,
                 num_layers=cfg.num_hidden_layers, fill_layers=range(cfg.num_hidden_layers),
                 keep_host=False)
    del wl.ctx_kv[:]
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(45)

    def nrm(o, i):
        return (torch.randn((o, i), generator=gen, device="cuda:0", dtype=torch.float32)
                * 0.02).to(torch.bfloat16)

    ones = torch.ones(H, dtype=torch.bfloat16, device="cuda:0")
    weights = dict(embed=nrm(V, H), final_norm=ones, layers=[
        dict(attn_norm=ones, wq=nrm(qd, H), wk=nrm(kvd, H), wv=nrm(kvd, H), wo=nrm(H, qd),
             mlp_norm=ones, w_gate=nrm(F, H), w_up=nrm(F, H), w_down=nrm(H, F))
        for _ in range(cfg.num_hidden_layers)])
    mc = M.ModelConfig(H, F, cfg.num_hidden_layers, cfg.num_attention_heads,
                       cfg.num_key_value_heads, V, cfg.max_position_embeddings,
                       cfg.rms_norm_eps, cfg.rope_theta, dict(cfg.rope_scaling))
    ec = M.EngineConfig(max_batch_tokens=S_max, max_seqs=S_max, max_model_len=8192 + 1024,
                        block_size=16, num_blocks=num_blocks)
    model = M.Llama(backend, mc, ec, weights)
    del weights
    torch.cuda.empty_cache()
    lines = []
    for S in batches:
        meta = vo.DecodeMeta.new([vo.DecodeSeq(int(ctx[s]), wl.tables[s]) for s in range(S)], 16)
        tokens = [int(t) for t in np.random.default_rng(S).integers(0, V, S)]

        def step(i):
            model.decode(wl.pool, tokens, meta)

        sec = time_steps(torch, step, args.steps, args.warmup)
        t0 = time.perf_counter()
        for _ in range(5):
            model.enqueue(wl.pool, tokens, meta, False)
        host = (time.perf_counter() - t0) / 5
        torch.cuda.synchronize()
        vo.profile_reset()
        vo.enable_profiling(True)
        time_steps(torch, step, 5, 0)
        vo.enable_profiling(False)
        prof = vo.profile()
        kernels = {k: round(v["avg_ms"] * v["calls"] / 5, 4)
                   for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["total_ms"])}
        graph_ms = None
        if args.graph:
            graph = model.capture_decode(wl.pool, tokens, meta)
            eager = model.decode(wl.pool, tokens, meta, want_logits=True)
            replay = graph.run(tokens, meta, want_logits=True)
            if replay.tokens != eager.tokens or not np.array_equal(replay.logits, eager.logits):
                raise SystemExit(f"graph replay differs from the eager step at {S} sequences")
            gsec = time_steps(torch, lambda i: graph.run(tokens, meta), args.steps, args.warmup)
            graph_ms = round(gsec * 1e3, 3)
            backend.step_meta(wl.pool).unfix_launch()
        lines.append({
            "metric": "Llama-3-8B-shape decode step, 1 GPU", "value": round(S / sec, 1),
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True, "dtype": "bf16",
            "data": "synthetic (random-init weights N(0, 0.02), random cached K/V)",
            "config": {"workload": f"decode, {S} sequences, context lognormal median 1024 "
                                   f"(seed 4), {cfg.num_hidden_layers} layers"},
            "host_enqueue_ms_per_step": round(host * 1e3, 3),
            "graph_ms_per_step": graph_ms,
            "kernels_ms_per_step": kernels,
            "graph_tokens_per_s": round(S / (graph_ms * 1e-3), 1) if graph_ms else None})
    return lines


def bench_rope_write(vo, W, orc, args):
    """The layer step before attention (model.rs:307-311): rope(q); rope(k);
    write_kv(k, v) as three launches, against the fused rope_write_kv, at the
    decode (cfg2, 64 rows) and prefill (cfg3, 4096 rows) shapes."""
    import torch
    heads, kvh, hd, bs = 32, 8, 128, 16
    table = vo.RopeTable(hd, 500000.0, 16384)
    res = {}
    for name, ctx, new in (("decode_64_rows", W.cfg2_context_lens(), None),
                           ("prefill_4096_rows", W.cfg3_context_lens(), [512] * 8)):
        kind = "decode" if new is None else "prefill"
        backend = vo.HipBackend(device=0, max_seqs=len(ctx), max_rows=W.FILL_ROWS,
                                max_table_entries=20000, max_query_heads=heads)
        wl = W.build(vo, backend, kind=kind, heads=heads, kv_heads=kvh, head_dim=hd,
                     block_size=bs, num_blocks=20000, context_lens=ctx, num_new=new, seed=7,
                     keep_host=False)
        q, k, v = wl.q.clone(), wl.k_new.clone(), wl.v_new.clone()

        def unfused(i):
            backend.rope(table, q, wl.pool, wl.meta, hd)
            backend.rope(table, k, wl.pool, wl.meta, hd)
            backend.write_kv(wl.pool, 0, k, v, wl.meta)

        def fused(i):
            backend.rope_write_kv(wl.pool, 0, table, q, k, v, wl.meta)

        t_u = time_steps(torch, unfused, args.steps, args.warmup)
        t_f = time_steps(torch, fused, args.steps, args.warmup)
        rows = wl.rows
        nbytes = rows * (heads * hd * 2 * 2 + kvh * hd * 2 * 2 * 2)
        res[name] = {"rows": rows, "unfused_us": round(t_u * 1e6, 2), "fused_us": round(t_f * 1e6, 2),
                     "fused_gbs": round(nbytes / t_f / 1e9, 1)}
    return {"metric": "rope(q) + rope(k) + write_kv, fused vs three launches, 1 GPU",
            "value": res["prefill_4096_rows"]["fused_us"], "unit": "us", "n_gpus": 1,
            "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "Llama-3-8B shape: 32 q heads, 8 KV heads, head_dim 128, "
                                   "theta 500000 llama3 scaling", "shapes": res}}


def nested_record(line):
    """The fields of a config's own line that the headline line nests."""
    keep = ("metric", "value", "unit", "ms_per_step", "pct_of_hbm_peak", "attention_rows_per_s",
            "decode_tokens_per_s", "kernels_us", "kernels_ms_per_step", "roofline",
            "cpu_baseline", "algorithmic_bytes_per_step", "unique_bytes_per_step",
            "gemm_tflop_per_step", "steps", "warmup", "settle")
    out = {k: line[k] for k in keep if k in line}
    out["workload"] = line["config"]["workload"]
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=2, help="pool layers to rotate over")
    ap.add_argument("--config", default="cfg2",
                    choices=["cfg2", "cfg3", "cfg4", "cfg4a", "cfg5", "decode", "rope", "all"])
    ap.add_argument("--decode-batches", default="1,16,64,256",
                    help="--config decode: batch sizes (sequences per step)")
    ap.add_argument("--graph", action="store_true",
                    help="--config decode: also time the step replayed as a HIP graph")
    ap.add_argument("--model-layers", type=int, default=32,
                    help="cfg4: decoder layers (32 = Llama-3-8B)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--unfused", action="store_true",
                    help="decode lines: time write_kv and decode_attention as two calls instead "
                         "of vo_decode_attention_write_kv")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="cap on the CPU baseline's threads (0: every CPU of the job's share)")
    ap.add_argument("--headline-only", action="store_true",
                    help="default config: print the cfg2 line without the nested cfg3 and cfg5 "
                         "records")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (scales the HBM byte "
                         "counters of rocprofv3 --pmc)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build runs "
              f"the paged-attention path on a single MI355X and has no multi-GPU mode.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        n = 1 << 30
        src = torch.ones(n // 2, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": n, "bytes_written": n, "launches": 5}))
        return

    vo = _load_package()
    import oracle as orc
    import workloads as W

    cfg2 = dict(name="cfg2: isolated paged decode, Llama-3-8B shape", heads=32,
                ctx=W.cfg2_context_lens(), seed=2, num_blocks=20000,
                ctx_desc="U[512, 4096], seed 2, keys = ctx + 1")
    cfg5 = dict(name="cfg5: prefix-shared decode, Llama-3-70B layer shape", heads=64,
                ctx=W.cfg5_context_lens(), seed=5, num_blocks=40000, shared_prefix=4096,
                shared_count=64,
                ctx_desc="64 x (4096 shared + U[256,1024]) + 1 x 32768, seed 5",
                metric="prefix-shared decode attn GB/s (logical bytes), Llama-3-70B layer")
    lines = []
    if args.config == "cfg2" and not args.headline_only:
        # The headline (cfg2) line, with the other north_star targets nested:
        # cfg5's prefix-shared decode, cfg3's chunked prefill and cfg4's full
        # model step (the metric's tokens/s).
        line = bench_decode(vo, W, orc, args, cfg2)
        line["cfg5"] = nested_record(bench_decode(vo, W, orc, args, cfg5))
        line["cfg3"] = nested_record(bench_prefill(vo, W, orc, args))
        torch.cuda.empty_cache()
        line["cfg4"] = nested_record(bench_model(vo, W, orc, args))
        lines.append(line)
    elif args.config in ("cfg2", "all"):
        lines.append(bench_decode(vo, W, orc, args, cfg2))
    if args.config in ("cfg5", "all"):
        lines.append(bench_decode(vo, W, orc, args, cfg5))
    if args.config in ("cfg3", "all"):
        lines.append(bench_prefill(vo, W, orc, args))
    if args.config in ("cfg4a", "all"):
        lines.append(bench_mixed(vo, W, orc, args))
    if args.config in ("cfg4", "all"):
        lines.append(bench_model(vo, W, orc, args))
    if args.config == "decode":
        lines.extend(bench_model_decode(vo, W, orc, args))
    if args.config in ("rope", "all"):
        lines.append(bench_rope_write(vo, W, orc, args))
    for line in lines:
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
