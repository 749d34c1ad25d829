"""Headline benchmark: paged decode KV-read GB/s (+ tokens/s) at Qwen3-0.6B KV
shapes, batch 128.

One step = one decode step of the hot path: upload the batch metadata (block
tables, positions, slots) once, then for each of 28 layers append one token's
K/V per sequence through the slot mapping and run paged GQA decode attention
over every sequence's full context. Context lengths start uniform in
[1024, 8192] (seeded) and grow by one token per step; pages are handed out in
a seeded random order so tables are non-contiguous. K/V/Q are synthetic
N(0,1) bf16 already resident in HBM when timing starts.

The default run then appends bounded legs of the other GPU configs under
"legs" (config 2: 2,000 decode launches; the same layer over one 32,768-token
row: 2,000 launches; config 4: 5 prefill steps at the 2,008-token prefix;
config 5: the first 1,000 churn steps), each with its own
roofline and CPU baseline; the line's "value" stays config 3's. --no-legs
skips them.

Prints one JSON line (see the keys below). --gpus N > 1 is refused: this
build measures one GPU.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
# HBM bytes per launch of the dominant kernel, from rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes scaled by a known-size copy (measure/rocprof_summary.py
# traffic writes these files from those passes)
TRAFFIC_FILES = {
    "config3": os.path.join(ROOT, "profiles", "append_decode_config3_traffic.json"),
    "config2": os.path.join(ROOT, "profiles", "decode_config2_traffic.json"),
}
LAYERS, BATCH, KV_HEADS, Q_HEADS, HEAD_DIM, BLOCK = 28, 128, 8, 16, 128, 16
CTX_LO, CTX_HI = 1024, 8192


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# pool element types bench.py measures: bf16 (the BASELINE configs) and f32
# (the reference's own storage type)
ELEM_BYTES = {"bf16": 2, "f32": 4}
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3}  # MI355X dense matrix peaks


def pool_types(dtype):
    """(torch dtype, ckv code, oracle code) of a pool of element type `dtype`."""
    import torch

    from chibillm_amd import ckv
    from oracle import oracle as orc

    if dtype == "f32":
        return torch.float32, ckv.F32, orc.F32
    return torch.bfloat16, ckv.BF16, orc.BF16


def host_values(orc, a, code):
    """float32 samples as the oracle's host array of element type `code`."""
    return np.asarray(a, np.float32) if code == orc.F32 else orc.from_f32(a, code)


def traffic_bytes(workload, kernel):
    """Measured HBM bytes per launch of `kernel` if a counter summary exists."""
    try:
        with open(TRAFFIC_FILES[workload]) as fh:
            data = json.load(fh)
    except (OSError, KeyError):
        return None
    entry = data.get("kernels", {}).get(kernel)
    return None if entry is None else int(entry["hbm_bytes_per_launch"])


# ---- CPU baseline (the oracle: a C restatement of the reference path) ----------------

BOX_CPU_SHARE = 16  # host threads one GPU's box gives a job, whatever os.cpu_count() shows


def baseline_threads(args):
    return args.cpu_threads or min(os.cpu_count() or 1, BOX_CPU_SHARE)


def cpu_model():
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def median_seconds(fn, runs):
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def host_decode_batch(lengths, seed, dtype="bf16"):
    """One layer of K/V of element type `dtype` on the host for rows of
    `lengths` tokens on permuted pages, and queries of that type: the oracle's
    attention over them. The pages hold a tiled block of N(0,1) values (the
    timing does not depend on the values)."""
    from oracle import oracle as orc

    code = orc.F32 if dtype == "f32" else orc.BF16
    gen = np.random.default_rng(seed)
    F = KV_HEADS * HEAD_DIM
    pages = [math.ceil(n / BLOCK) for n in lengths]
    n_pages = sum(pages)
    block = host_values(orc, gen.standard_normal(1 << 22, np.float32), code)
    reps = -(-(n_pages * BLOCK * F) // block.size)
    kc = np.tile(block, reps)[:n_pages * BLOCK * F]
    vc = np.roll(kc, 12345)
    q = host_values(orc, gen.standard_normal((len(lengths), Q_HEADS * HEAD_DIM), np.float32),
                    code)
    perm = gen.permutation(n_pages).astype(np.uint32)
    offsets = np.cumsum([0] + pages[:-1])
    return orc.Attention((1, n_pages, BLOCK, KV_HEADS, HEAD_DIM), kc, vc, code, q, code,
                         [n - 1 for n in lengths], perm, offsets, pages, Q_HEADS, 0,
                         1 / math.sqrt(HEAD_DIM))


_CPU_DECODE_CACHE = {}


def cpu_decode_baseline(lengths, threads, runs, with_step=False, dtype="bf16"):
    """The CPU path of one decode step at these lengths, timed on this host
    (median of `runs` each): decode attention over one layer on `threads`
    threads and on one thread (oracle/oracle.c, the restated
    paged_attention_f32 with fp32 accumulation), and with_step: the append of
    one K/V row per sequence into a layer (store_kv) and the host work of the
    step, block_manager reservations plus prepare_paged_batch. A run that asks
    twice for the same inputs (the default run's config-3 line and its config-5
    leg) times them once."""
    key = (tuple(lengths), threads, runs, with_step, dtype)
    if key not in _CPU_DECODE_CACHE:
        _CPU_DECODE_CACHE[key] = _cpu_decode_baseline(lengths, threads, runs, with_step, dtype)
    return dict(_CPU_DECODE_CACHE[key], legs_ms=dict(_CPU_DECODE_CACHE[key]["legs_ms"]))


def _cpu_decode_baseline(lengths, threads, runs, with_step, dtype):
    from oracle import oracle as orc

    F = KV_HEADS * HEAD_DIM
    code = orc.F32 if dtype == "f32" else orc.BF16
    layer_bytes = sum(lengths) * F * 2 * ELEM_BYTES[dtype]
    att = host_decode_batch(lengths, 1, dtype)
    all_s = median_seconds(lambda: att.online_threads(threads), runs)
    single_s = median_seconds(lambda: att.online_threads(1), runs)
    out = {
        "value": round(layer_bytes / all_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "threads": threads,
        "cores_total": os.cpu_count(),
        "cpu_model": cpu_model(),
        "median_of": runs,
        "single_thread": {"value": round(layer_bytes / single_s / 1e9, 3), "unit": "GB/s"},
        "legs_ms": {"decode_attention_per_layer": round(all_s * 1e3, 3),
                    "decode_attention_per_layer_single_thread": round(single_s * 1e3, 3)},
    }
    del att
    if with_step:
        rows = len(lengths)
        gen = np.random.default_rng(2)
        k = host_values(orc, gen.standard_normal((rows, F), np.float32), code)
        pages = sum(math.ceil((n + 1) / BLOCK) for n in lengths) + 1
        kc = np.zeros(pages * BLOCK * F, k.dtype)
        vc = np.zeros_like(kc)
        slots = gen.permutation(pages * BLOCK)[:rows].astype(np.uint32)
        reps = 100
        append_s = median_seconds(
            lambda: [orc.store_kv(kc, vc, k, k, slots, 0, pages * BLOCK) for _ in range(reps)],
            runs) / reps

        def host_steps():
            step = orc.DecodeStepHost(lengths, pages + rows, BLOCK,
                                      math.ceil(max(lengths) / BLOCK) + 2)
            t0 = time.perf_counter()
            step.step()
            return time.perf_counter() - t0

        host_s = statistics.median(host_steps() for _ in range(runs))
        out["legs_ms"]["append_store_kv_per_layer"] = round(append_s * 1e3, 4)
        out["legs_ms"]["block_manager_and_prepare_paged_batch_per_step"] = round(host_s * 1e3, 4)
    return out


def calibration_copy(ctx):
    """A copy of known size for scaling the HBM counters: ckv_copy_blocks of 1024
    pages of 32 KiB, keys and values (64 MiB read, 64 MiB written)."""
    from chibillm_amd import ckv

    calib = ckv.Pool(ctx, 1, 2048, BLOCK, KV_HEADS, HEAD_DIM, ckv.BF16)
    calib.copy_blocks(np.arange(1024), np.arange(1024, 2048))
    ctx.sync()
    calib.close()
    log("calibration copy: 1024 pages x 32 KiB, keys + values = 64 MiB read, 64 MiB written")


# ---- config 2: single-layer decode attention -----------------------------------------

CONFIG2_BATCH, CONFIG2_POOL = 32, 65536
LONG_ROW_TOKENS = 32768
CONFIG2_LO, CONFIG2_HI = 256, 4096


def bench_config2(args, long_row=False):
    """one layer, batch 32, contexts U[256, 4096], 16-token
    pages from a seeded permutation of a 65,536-page pool. A step is one
    ckv_decode_attention call (one decode launch; the rows the plan cuts into
    chunks are merged by their last chunk) over the uploaded batch; one event
    pair on the launch stream brackets the timed steps (an event pair per 55 us
    step would add its own gaps). long_row (--workload longrow): the same over
    one row of 32,768 tokens, the single long row split-K exists for."""
    import torch

    from chibillm_amd import ckv

    steps = 2000 if args.steps == 20 else args.steps
    device = torch.device("cuda:0")
    gen = np.random.default_rng(args.seed)
    lengths = [int(x) for x in gen.integers(CONFIG2_LO, CONFIG2_HI + 1, CONFIG2_BATCH)]
    if long_row:
        lengths = [LONG_ROW_TOKENS]
    batch = len(lengths)
    perm = gen.permutation(CONFIG2_POOL).astype(np.uint32)
    pages = [math.ceil(n / BLOCK) for n in lengths]
    flat = perm[:sum(pages)]
    offsets = np.cumsum([0] + pages[:-1])
    F = KV_HEADS * HEAD_DIM
    tdt, code, _ = pool_types(args.dtype)
    es = ELEM_BYTES[args.dtype]
    ctx = ckv.Context(0, stream=torch.cuda.current_stream())
    if args.calibrate_copy:
        calibration_copy(ctx)
    tgen = torch.Generator(device=device)
    tgen.manual_seed(args.seed)
    elems = CONFIG2_POOL * BLOCK * F
    keys = torch.empty(elems, dtype=tdt, device=device).normal_(generator=tgen)
    values = torch.empty(elems, dtype=tdt, device=device).normal_(generator=tgen)
    pool = ckv.Pool(ctx, 1, CONFIG2_POOL, BLOCK, KV_HEADS, HEAD_DIM, code, keys, values)
    q = torch.randn(batch, Q_HEADS * HEAD_DIM, generator=tgen, device=device).to(tdt)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    pool.upload(flat, offsets, pages, [n - 1 for n in lengths])
    split_pages, items, records = pool.decode_plan()
    name = "longrow" if long_row else "config2"
    log(f"{name}: {sum(lengths)} tokens, plan: {split_pages} pages per workgroup or chunk, "
        f"{items} row segments, {records} records")
    for _ in range(args.warmup * 10):
        pool.decode(0, q, Q_HEADS, scale, out)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        pool.decode(0, q, Q_HEADS, scale, out)
    end.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    launch_ms = start.elapsed_time(end) / steps
    kv_bytes = sum(lengths) * F * 2 * es
    per_launch = kv_bytes + 2 * batch * Q_HEADS * HEAD_DIM * es + 4 * sum(pages)
    achieved = per_launch / (launch_ms / 1e3) / 1e9
    if long_row:
        metric = ("paged decode KV-read GB/s (% HBM peak), Qwen3-0.6B KV, one layer, one row of "
                  f"{LONG_ROW_TOKENS} tokens")
        workload = (f"longrow: single-layer paged GQA decode attention over one row of "
                    f"{LONG_ROW_TOKENS} tokens, pages from a seeded permutation of a 65,536-page "
                    "pool")
    else:
        metric = "paged decode KV-read GB/s (% HBM peak), Qwen3-0.6B KV, one layer, batch 32"
        workload = ("config2: single-layer paged GQA decode attention, batch 32, context "
                    "U[256,4096], pages from a seeded permutation of a 65,536-page pool")
    if args.dtype != "bf16":
        metric += f", {args.dtype} pages"
        workload += f"; {args.dtype} pages (BASELINE's config is bf16)"
    result = {
        "metric": metric,
        "value": round(kv_bytes / (launch_ms / 1e3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup * 10,
        "ms_per_step": round(launch_ms, 5),
        "wall_ms_per_step": round(elapsed * 1e3 / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic N(0,1) K/V/Q, seeded lengths and page permutation",
        "config": {
            "workload": workload,
            "batch": batch, "kv_heads": KV_HEADS, "q_heads": Q_HEADS,
            "head_dim": HEAD_DIM, "block_size": BLOCK, "pool_pages": CONFIG2_POOL,
            "tokens": sum(lengths), "plan": {"pages_per_workgroup": split_pages,
                                             "segments": items, "records": records},
        },
        "hbm_frac": round(kv_bytes / (launch_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "kernel": "paged_attention_decode (decode_wg_kernel, cut rows merged in-launch)",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (None if long_row or args.dtype != "bf16"
                        else traffic_bytes("config2", "decode")),
            "avg_launch_us": round(launch_ms * 1e3, 3),
            "algorithmic_bytes_per_launch": int(per_launch),
        },
        "cpu_baseline": None,
    }
    pool.close()
    del keys, values
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        threads = baseline_threads(args)
        log(f"CPU baseline on {threads} threads")
        base = cpu_decode_baseline(lengths, threads, runs=5, dtype=args.dtype)
        base["sample"] = (f"the whole workload: oracle/oracle.c decode attention (restated "
                          f"paged_attention_f32, fp32 accumulate) over the same {batch} "
                          f"rows ({sum(lengths)} tokens, {kv_bytes / 1e9:.3f} GB of "
                          f"{args.dtype} K/V), "
                          f"median of 5 runs on {threads} threads and 5 on one")
        result["cpu_baseline"] = base
    return result


# ---- config 3: the 28-layer decode step (headline) -----------------------------------

def bench_config3(args):
    import torch

    from chibillm_amd import ckv

    device = torch.device("cuda:0")
    gen = np.random.default_rng(args.seed)
    lengths = gen.integers(CTX_LO, CTX_HI + 1, BATCH).astype(np.int64)
    profile_steps = min(args.steps, 5)
    total_steps = args.warmup + args.steps + profile_steps
    max_len = lengths + total_steps
    pages_needed = [math.ceil(n / BLOCK) for n in max_len]
    n_pool = sum(pages_needed) + 64
    perm = gen.permutation(n_pool).astype(np.uint32)
    F = KV_HEADS * HEAD_DIM
    max_pages = max(pages_needed)

    # per-sequence table regions of the flat table; pages appear as needed
    flat = np.zeros(BATCH * max_pages, np.uint32)
    owned = [0] * BATCH
    next_free = 0

    def ensure_pages(s, tokens):
        nonlocal next_free
        need = math.ceil(tokens / BLOCK)
        while owned[s] < need:
            flat[s * max_pages + owned[s]] = perm[next_free]
            next_free += 1
            owned[s] += 1

    for s in range(BATCH):
        ensure_pages(s, int(lengths[s]))

    tdt, code, _ = pool_types(args.dtype)
    es = ELEM_BYTES[args.dtype]
    kv_gb = LAYERS * n_pool * BLOCK * F * 2 * es / 1e9
    log(f"pool {n_pool} pages x {LAYERS} layers = {kv_gb:.1f} GB K+V; "
        f"context tokens {int(lengths.sum())}")
    ctx = ckv.Context(0, stream=torch.cuda.current_stream())
    if args.calibrate_copy:
        calibration_copy(ctx)
    elems = LAYERS * n_pool * BLOCK * F
    keys = torch.empty(elems, dtype=tdt, device=device)
    values = torch.empty(elems, dtype=tdt, device=device)
    tgen = torch.Generator(device=device)
    tgen.manual_seed(args.seed)
    t0 = time.perf_counter()
    step = 1 << 30
    for buf in (keys, values):
        for i in range(0, elems, step):
            buf[i:i + step].normal_(generator=tgen)
    torch.cuda.synchronize()
    log(f"filled K/V with N(0,1) in {time.perf_counter() - t0:.1f} s")
    pool = ckv.Pool(ctx, LAYERS, n_pool, BLOCK, KV_HEADS, HEAD_DIM, code, keys, values)

    q = torch.randn(LAYERS, BATCH, Q_HEADS * HEAD_DIM, generator=tgen, device=device).to(tdt)
    k_new = torch.randn(LAYERS, BATCH, F, generator=tgen, device=device).to(tdt)
    v_new = torch.randn(LAYERS, BATCH, F, generator=tgen, device=device).to(tdt)
    out = torch.empty(LAYERS, BATCH, Q_HEADS * HEAD_DIM, dtype=tdt, device=device)
    gate = (torch.randn(LAYERS, BATCH, Q_HEADS * HEAD_DIM, generator=tgen, device=device)
            .to(tdt) if args.gate else None)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    offsets = np.arange(BATCH, dtype=np.uint32) * max_pages

    def one_step(start=None, end=None):
        positions = lengths.copy()  # the new token's position
        for s in range(BATCH):
            ensure_pages(s, int(positions[s]) + 1)
        slots = [int(flat[s * max_pages + p // BLOCK]) * BLOCK + p % BLOCK
                 for s, p in enumerate(positions)]
        pool.upload(flat, offsets, owned, positions, slots)
        if start is not None:
            start.record()
        for layer in range(LAYERS):
            if args.no_fuse:
                pool.append(layer, k_new[layer], v_new[layer])
                pool.decode(layer, q[layer], Q_HEADS, scale, out[layer])
            elif args.rope:
                pool.rope_append_decode(layer, k_new[layer], v_new[layer], q[layer], Q_HEADS,
                                        scale, ROPE_THETA, out[layer],
                                        gate=gate[layer] if args.gate else None)
            elif args.gate:
                pool.append_decode_gated(layer, k_new[layer], v_new[layer], q[layer], Q_HEADS,
                                         scale, gate[layer], out[layer])
            else:
                pool.append_decode(layer, k_new[layer], v_new[layer], q[layer], Q_HEADS, scale,
                                   out[layer])
        if end is not None:
            end.record()
        attended = positions + 1
        lengths[:] = attended
        return int(attended.sum()), int(sum(math.ceil(a / BLOCK) for a in attended))

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} steps done")

    # the timed region: whole steps, no per-launch timing; one event pair per
    # step on the launch stream brackets its 28 launches (after the upload)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    tokens_attended = pages_read = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        toks, pages = one_step(starts[i], ends[i])
        tokens_attended += toks
        pages_read += pages
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    launches_ms = sum(a.elapsed_time(b) for a, b in zip(starts, ends))
    log(f"timed {args.steps} steps in {elapsed:.3f} s")

    # a separate, profiled pass: per-kernel times from events around every launch
    dominant = ("paged_attention_decode" if args.no_fuse
                else "rope_append_decode" if args.rope else "append_decode")
    ctx.profile(True)
    ctx.profile_reset()
    for _ in range(profile_steps):
        one_step()
    kernels = {name: ctx.profile_query(name)
               for name in (dominant, "paged_attention_merge", "store_kv")}
    ctx.profile(False)

    kv_row_bytes = F * 2 * es  # K + V, all KV heads
    kv_bytes = LAYERS * tokens_attended * kv_row_bytes
    value = kv_bytes / elapsed / 1e9
    ms_per_step = elapsed * 1e3 / args.steps
    # algorithmic bytes of one launch (one layer): KV of every attended token,
    # Q and O, the table entries read, and (fused) the new K/V rows written
    appended = 0 if args.no_fuse else BATCH * kv_row_bytes
    qo_rows = 3 if args.gate else 2  # Q and O, and the gate when it is read
    per_launch = (tokens_attended * kv_row_bytes + pages_read * 4
                  + args.steps * (qo_rows * BATCH * Q_HEADS * HEAD_DIM * es + appended)) / args.steps
    launches = LAYERS * args.steps * (2 if args.no_fuse else 1)
    avg_launch_s = launches_ms / launches / 1e3
    achieved = per_launch / (launches_ms / (LAYERS * args.steps) / 1e3) / 1e9
    result = {
        "metric": "paged decode KV-read GB/s (% HBM peak) + tokens/s, Qwen3-0.6B KV, batch 128"
                  + ("" if args.dtype == "bf16" else f", {args.dtype} pages"),
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic N(0,1) K/V/Q, seeded lengths and page order",
        "config": {
            "workload": "config3: 28-layer decode step (append 1 token/seq/layer + paged GQA "
                        "decode attention), batch 128, context U[1024,8192] growing 1/step",
            "launches": "two per layer (ckv_append, ckv_decode_attention)" if args.no_fuse
                        else ("one per layer (ckv_rope_append_decode: queries and new keys "
                              "rotated in the kernel, Qwen3 theta 1e6"
                              + (", sigmoid gate" if args.gate else "") + ")") if args.rope
                        else ("one per layer (ckv_append_decode_gated: sigmoid gate in the "
                              "epilogue)" if args.gate else "one per layer (ckv_append_decode)"),
            "layers": LAYERS, "batch": BATCH, "kv_heads": KV_HEADS, "q_heads": Q_HEADS,
            "head_dim": HEAD_DIM, "block_size": BLOCK, "pool_pages": n_pool,
            "kv_pool_gb": round(kv_gb, 2),
            "mean_context": round(tokens_attended / args.steps / BATCH, 1),
        },
        "tokens_per_s": round(BATCH * args.steps / elapsed, 1),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "launch_ms_per_step": round(launches_ms / args.steps, 4),
        "kernels_ms_per_step_profiled_pass": {
            name: round(ms / max(profile_steps, 1), 4) for name, (ms, _) in kernels.items()},
        "roofline": {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes("config3", dominant) if args.dtype == "bf16" else None,
            "avg_launch_us": round(avg_launch_s * 1e6, 2),
            "algorithmic_bytes_per_launch": int(per_launch),
            "timing": "one event pair per step around its 28 launches, launch gaps included",
        },
        "cpu_baseline": None,
    }
    if args.dtype != "bf16":
        result["config"]["workload"] += f"; {args.dtype} pages (BASELINE's config is bf16)"
    pool.close()
    del keys, values
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        threads = baseline_threads(args)
        log(f"CPU baseline on {threads} threads")
        base_lengths = [int(x) for x in np.random.default_rng(args.seed).integers(
            CTX_LO, CTX_HI + 1, BATCH)]
        base = cpu_decode_baseline(base_lengths, threads, runs=5, with_step=True,
                                   dtype=args.dtype)
        legs = base["legs_ms"]
        step_ms = (LAYERS * (legs["decode_attention_per_layer"]
                             + legs["append_store_kv_per_layer"])
                   + legs["block_manager_and_prepare_paged_batch_per_step"])
        base["step_ms"] = round(step_ms, 2)
        base["tokens_per_s"] = round(BATCH / (step_ms / 1e3), 1)
        base["sample"] = (f"one layer of the workload, scaled by {LAYERS}: oracle/oracle.c decode "
                          f"attention (restated paged_attention_f32, fp32 accumulate) over the "
                          f"{BATCH} rows ({sum(base_lengths)} tokens, "
                          f"{sum(base_lengths) * F * 2 * es / 1e9:.2f} GB of {args.dtype} K/V per "
                          f"layer), "
                          f"store_kv of the {BATCH} new rows, and the step's block_manager + "
                          f"prepare_paged_batch; median of 5 runs each, on {threads} threads "
                          f"and on one")
        result["cpu_baseline"] = base
    return result

ROPE_THETA = 1e6  # Qwen3-0.6B rope_theta
PREFILL_SEQS, PREFILL_CHUNK = 64, 512


def prefill_flops(prefix, chunk, seqs):
    """Causal attention FLOPs of one layer: QK^T and PV, 2 FLOPs per MAC each,
    over the keys each row attends (prefix + its own position + 1)."""
    keys = sum(prefix + i + 1 for i in range(chunk))
    return 4 * HEAD_DIM * Q_HEADS * seqs * keys


def prefill_cpu_baseline(threads, prefix, runs=5, dtype="bf16"):
    """Oracle causal attention (restated paged_flash_attention_prefill_f32
    maths, fp32) on bounded samples of one layer: 4 sequences x 256 chunk rows
    on `threads` threads and 1 sequence x 128 rows on one thread, median of
    `runs` each."""
    from oracle import oracle as orc

    code = orc.F32 if dtype == "f32" else orc.BF16

    def sample(seqs, rows, seed):
        gen = np.random.default_rng(seed)
        F = KV_HEADS * HEAD_DIM
        pages = math.ceil((prefix + rows) / BLOCK)
        n_pages = pages * seqs
        kc = host_values(orc, gen.standard_normal(n_pages * BLOCK * F, np.float32), code)
        vc = host_values(orc, gen.standard_normal(n_pages * BLOCK * F, np.float32), code)
        q = host_values(orc, gen.standard_normal((seqs * rows, Q_HEADS * HEAD_DIM), np.float32),
                        code)
        table = gen.permutation(n_pages).astype(np.uint32)
        positions = [prefix + i for _ in range(seqs) for i in range(rows)]
        offsets = [s * pages for s in range(seqs) for _ in range(rows)]
        return orc.Attention((1, n_pages, BLOCK, KV_HEADS, HEAD_DIM), kc, vc, code, q,
                             code, positions, table, offsets, [pages] * len(positions),
                             Q_HEADS, 0, 1 / math.sqrt(HEAD_DIM))

    big, small = sample(4, 256, 2), sample(1, 128, 3)
    all_s = median_seconds(lambda: big.online_threads(threads), runs)
    single_s = median_seconds(lambda: small.online_threads(1), runs)
    flops, flops1 = prefill_flops(prefix, 256, 4), prefill_flops(prefix, 128, 1)
    return {
        "value": round(flops / all_s / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": threads,
        "kind": "port",
        "threads": threads,
        "cores_total": os.cpu_count(),
        "cpu_model": cpu_model(),
        "median_of": runs,
        "single_thread": {"value": round(flops1 / single_s / 1e9, 3), "unit": "GFLOP/s"},
        "sample": (f"oracle/oracle.c causal attention over paged {dtype} K/V, fp32 accumulate, one "
                   f"layer: 4 sequences x 256 rows at positions {prefix}..{prefix + 255} "
                   f"({flops / 1e9:.1f} GFLOP) on {threads} threads, and 1 x 128 rows "
                   f"({flops1 / 1e9:.1f} GFLOP) on one; median of {runs} runs each"),
    }


def bench_config4(args):
    """64 sequences share one prefix held once as pages; each step restores it
    for every sequence (shared full pages; a copy-on-write copy of a partial
    tail page, all layers, one ckv_copy_blocks), uploads the chunk's metadata,
    then per layer appends the 512-row chunks and runs the MFMA prefill."""
    import torch

    from chibillm_amd import ckv

    device = torch.device("cuda:0")
    prefix, S, C = args.prefix, args.sequences, PREFILL_CHUNK
    F = KV_HEADS * HEAD_DIM
    full = prefix // BLOCK
    partial = prefix % BLOCK != 0
    prefix_pages = math.ceil(prefix / BLOCK)
    own = math.ceil((prefix + C) / BLOCK) - full
    n_pool = prefix_pages + S * own + 16
    perm = np.random.default_rng(args.seed).permutation(n_pool).astype(np.uint32)
    prefix_table = perm[:prefix_pages]
    tables = [np.concatenate([prefix_table[:full],
                              perm[prefix_pages + s * own:prefix_pages + (s + 1) * own]])
              for s in range(S)]
    flat = np.concatenate(tables).astype(np.uint32)
    positions = np.tile(np.arange(prefix, prefix + C, dtype=np.uint32), S)
    offsets = np.repeat(np.arange(S, dtype=np.uint32) * len(tables[0]), C)
    lengths = np.full(S * C, len(tables[0]), np.uint32)
    slots = np.array([int(t[p // BLOCK]) * BLOCK + p % BLOCK
                      for t in tables for p in range(prefix, prefix + C)], np.uint32)
    cow_src = [int(prefix_table[full])] * S if partial else []
    cow_dst = [int(t[full]) for t in tables] if partial else []

    ctx = ckv.Context(0, stream=torch.cuda.current_stream())
    tdt, code, _ = pool_types(args.dtype)
    es = ELEM_BYTES[args.dtype]
    elems = LAYERS * n_pool * BLOCK * F
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed)
    keys = torch.empty(elems, dtype=tdt, device=device).normal_(generator=gen)
    values = torch.empty(elems, dtype=tdt, device=device).normal_(generator=gen)
    pool = ckv.Pool(ctx, LAYERS, n_pool, BLOCK, KV_HEADS, HEAD_DIM, code, keys, values)
    rows = S * C
    q = torch.randn(LAYERS, rows, Q_HEADS * HEAD_DIM, generator=gen, device=device).to(tdt)
    k_new = torch.randn(LAYERS, rows, F, generator=gen, device=device).to(tdt)
    v_new = torch.randn(LAYERS, rows, F, generator=gen, device=device).to(tdt)
    out = torch.empty(LAYERS, rows, Q_HEADS * HEAD_DIM, dtype=tdt, device=device)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    log(f"config4: prefix {prefix} ({prefix_pages} shared pages, tail copy: {partial}), "
        f"{S} x {C}-row chunks, pool {n_pool} pages x {LAYERS} layers")

    def one_step():
        if partial:
            pool.copy_blocks(cow_src, cow_dst)
        pool.upload(flat, offsets, lengths, positions, slots)
        for layer in range(LAYERS):
            if args.rope:
                pool.rope(q[layer], q[layer], Q_HEADS, ROPE_THETA)
                pool.rope_append(layer, k_new[layer], v_new[layer], ROPE_THETA)
            else:
                pool.append(layer, k_new[layer], v_new[layer])
            pool.prefill(layer, q[layer], Q_HEADS, scale, out[layer])

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    ctx.profile(True)
    ctx.profile_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernels = {}
    for name in ("paged_attention_prefill", "store_kv", "copy_blocks", "rope", "rope_append"):
        ms, n = ctx.profile_query(name)
        kernels[name] = (ms, n)
    ctx.profile(False)
    prefill_ms, prefill_n = kernels["paged_attention_prefill"]
    avg_s = prefill_ms / prefill_n / 1e3
    flops = prefill_flops(prefix, C, S)
    achieved = flops / avg_s / 1e12
    ms_per_step = elapsed * 1e3 / args.steps
    peak = MFMA_PEAK_TFLOPS[args.dtype]
    result = {
        "metric": "chunked-prefill attention TFLOP/s (MFMA) + tokens/s, Qwen3-0.6B KV, "
                  f"{S} sequences x {C}-token chunks over a shared prefix"
                  + ("" if args.dtype == "bf16" else f", {args.dtype} pages"),
        "value": round(LAYERS * flops * args.steps / elapsed / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic N(0,1) K/V/Q, seeded page order",
        "config": {
            "workload": f"config4: {S} sequences share a {prefix}-token prefix (refcounted "
                        f"pages, copy-on-write tail: {partial}); each appends and prefills a "
                        f"{C}-row causal chunk over prefix + chunk, {LAYERS} layers per step",
            "layers": LAYERS, "sequences": S, "chunk": C, "prefix": prefix,
            "kv_heads": KV_HEADS, "q_heads": Q_HEADS, "head_dim": HEAD_DIM,
            "block_size": BLOCK, "pool_pages": n_pool,
        },
        "tokens_per_s": round(S * C * args.steps / elapsed, 1),
        "kernels_ms_per_step": {k: round(v[0] / args.steps, 4) for k, v in kernels.items()},
        "roofline": {
            "kernel": "paged_attention_prefill",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": None,
            "avg_launch_us": round(avg_s * 1e6, 2),
            "algorithmic_flops_per_launch": flops,
        },
        "cpu_baseline": None,
    }
    if args.dtype != "bf16":
        result["config"]["workload"] += f"; {args.dtype} pages (BASELINE's config is bf16)"
    if args.rope:
        # the fused append's algorithmic bytes: key and value rows read, page
        # rows written, positions and slots
        ms, n = kernels["rope_append"]
        per = rows * (4 * F * es + 8)
        result["rope_append"] = {"avg_launch_us": round(ms / n * 1e3, 2),
                                 "bytes_per_launch": per,
                                 "achieved_gbs": round(per / (ms / n / 1e3) / 1e9, 2)}
        # the queries' rotation in place: query rows read and written, positions
        ms, n = kernels["rope"]
        per = rows * (2 * Q_HEADS * HEAD_DIM * es + 4)
        result["rope"] = {"avg_launch_us": round(ms / n * 1e3, 2), "bytes_per_launch": per,
                          "achieved_gbs": round(per / (ms / n / 1e3) / 1e9, 2)}
        result["config"]["workload"] += "; keys rotated inside the append, queries by ckv_rope"
    pool.close()
    del keys, values, q, k_new, v_new, out
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        threads = baseline_threads(args)
        log(f"CPU baseline on {threads} threads")
        result["cpu_baseline"] = prefill_cpu_baseline(threads, prefix, dtype=args.dtype)
    return result


PCIE5_X16_GBS = 64.0  # PCIe 5.0 x16, one direction


def bench_spill(args):
    """A cached prefix leaving HBM and coming back: config 4's 2,008-token
    prefix (28 layers, 16-token pages in seeded order) exported to pinned host
    memory in the packed [layer, token, kv_head, feature] layout and imported
    into other pages (ckv_checkpoint_export / ckv_checkpoint_import), one of
    each per step; the bytes cross PCIe once each way."""
    import torch

    from chibillm_amd import ckv

    device = torch.device("cuda:0")
    tokens = args.prefix
    F = KV_HEADS * HEAD_DIM
    pages = math.ceil(tokens / BLOCK)
    n_pool = 2 * pages + 16
    perm = np.random.default_rng(args.seed).permutation(n_pool).astype(np.uint32)
    src, dst = perm[:pages], perm[pages:2 * pages]
    ctx = ckv.Context(0, stream=torch.cuda.current_stream())
    elems = LAYERS * n_pool * BLOCK * F
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed)
    keys = torch.empty(elems, dtype=torch.bfloat16, device=device).normal_(generator=gen)
    values = torch.empty(elems, dtype=torch.bfloat16, device=device).normal_(generator=gen)
    pool = ckv.Pool(ctx, LAYERS, n_pool, BLOCK, KV_HEADS, HEAD_DIM, ckv.BF16, keys, values)
    packed = LAYERS * tokens * F * 2  # bytes per tensor
    hk = ctx.host_alloc(packed)
    hv = ctx.host_alloc(packed)
    log(f"spill: {tokens}-token prefix, {LAYERS} layers, {2 * packed / 2**20:.1f} MiB each way")

    def one_step():
        pool.checkpoint_export(src, tokens, hk, hv)
        pool.checkpoint_import(dst, tokens, hk, hv)

    for _ in range(args.warmup):
        one_step()
    ctx.sync()
    ctx.profile(True)
    ctx.profile_reset()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    kernels = {name: ctx.profile_query(name) for name in ("checkpoint_export", "checkpoint_import")}
    ctx.profile(False)
    moved = 2 * 2 * packed  # keys + values, down and up
    gbs = moved * args.steps / elapsed / 1e9
    result = {
        "metric": "prefix spill round trip (export to pinned host + import), GB/s over PCIe",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V, seeded page order",
        "config": {
            "workload": f"spill: a {tokens}-token prefix of {LAYERS} layers exported to pinned "
                        "host memory (packed layout) and imported into other pages, per step",
            "layers": LAYERS, "tokens": tokens, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM,
            "block_size": BLOCK, "bytes_each_way": 2 * packed,
        },
        "kernels_ms_per_step": {k: round(v[0] / args.steps, 4) for k, v in kernels.items()},
        # the two directions run one after the other on one stream, so the
        # bytes over the whole step time are the rate of the active direction
        "roofline": {
            "kernel": "checkpoint export + import (DMA over PCIe)",
            "bound": "pcie",
            "achieved": round(gbs, 2),
            "peak": PCIE5_X16_GBS,
            "unit": "GB/s (one direction at a time)",
            "frac": round(gbs / PCIE5_X16_GBS, 4),
            "traffic": None,
        },
        "cpu_baseline": None,
    }
    ctx.host_free(hk)
    ctx.host_free(hv)
    pool.close()
    return result


CHURN_STEPS = 5000


def bench_config5(args):
    """The churn trace runs in the C++ driver (chibillm_amd/bin/churn): the
    scheduler, refcounted pages and a 160 GB device pool, one engine step per
    scheduler step. --steps sets the trace length (default 5000 when the
    default 20 is given); warmup does not apply to a trace. The trace runs
    twice: once plain, timed as a whole (the line's value, steps/s and HBM
    fraction), and once with every launch bracketed by HIP events (the
    per-kernel times and the roofline's average launch), since those events
    add their own gaps to the steps."""
    import subprocess

    steps = CHURN_STEPS if args.steps == 20 else args.steps
    driver = os.path.join(ROOT, "chibillm_amd", "bin", "churn")
    if not os.path.exists(driver):
        raise SystemExit(f"{driver} is not built: run __graft_entry__.build()")

    def run_trace(*extra):
        cmd = [driver, "--steps", str(steps), "--seed", str(args.seed), *extra]
        log("config5: " + " ".join(cmd))
        proc = subprocess.run(cmd, capture_output=True, text=True)
        sys.stderr.write(proc.stderr)
        if proc.returncode != 0:
            raise SystemExit(f"churn driver failed ({proc.returncode})")
        return json.loads(proc.stdout.strip().splitlines()[-1])

    trace = run_trace()
    profiled = run_trace("--profile")
    for key in ("prefill_tokens", "decode_tokens", "decode_step_bytes"):
        if profiled[key] != trace[key]:
            raise SystemExit(f"the profiled trace differs from the plain one in {key}")
    decode_ms, decode_n = profiled["kernels_ms"]["append_decode"]
    decode_s = decode_ms / 1e3
    achieved = trace["decode_step_bytes"] / decode_s / 1e9 if decode_s else 0.0
    result = {
        "metric": "continuous-batching churn: tokens/s, steps/s and HBM fraction, Qwen3-0.6B KV, "
                  "28 layers, 160 GB page pool, live batch <= 512",
        "value": trace["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 0,
        "ms_per_step": round(trace["seconds"] * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/Q rows; seeded Poisson(8) arrivals, lognormal prompt "
                "(median 512, sigma 1, [16, 16384]) and output (median 256, sigma 1, [1, 4096])",
        "config": {
            "workload": "config5: churn trace through the C++ scheduler and page allocator; each "
                        "step uploads the batch tables and runs append + paged attention for 28 "
                        "layers (prefill tiles or fused decode)",
            "pool_pages": trace["pool_pages"], "max_live": 512, "max_batch_tokens": 2048,
            "prefill_chunk": 512,
        },
        "steps_per_s": trace["steps_per_s"],
        "hbm_frac": trace["hbm_frac"],
        "hbm_gbs": trace["hbm_gbs"],
        "trace": {k: trace[k] for k in ("prefill_tokens", "decode_tokens", "prefill_steps",
                                        "decode_steps", "arrived", "admitted", "finished",
                                        "pending_at_end", "peak_live")},
        "kernels_ms_per_step_profiled_pass": {k: round(v[0] / steps, 4)
                                              for k, v in profiled["kernels_ms"].items()},
        "profiled_pass_steps_per_s": profiled["steps_per_s"],
        "roofline": {
            "kernel": "append_decode",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": round(decode_ms * 1e3 / max(decode_n, 1), 2),
            "algorithmic_bytes_per_launch": int(trace["decode_step_bytes"] / max(decode_n, 1)),
            "timing": "the profiled pass's HIP events around each fused decode launch",
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        threads = baseline_threads(args)
        log(f"CPU baseline on {threads} threads")
        base_lengths = [int(x) for x in np.random.default_rng(args.seed).integers(
            CTX_LO, CTX_HI + 1, BATCH)]
        base = cpu_decode_baseline(base_lengths, threads, runs=5, with_step=True)
        legs = base["legs_ms"]
        step_ms = (LAYERS * (legs["decode_attention_per_layer"]
                             + legs["append_store_kv_per_layer"])
                   + legs["block_manager_and_prepare_paged_batch_per_step"])
        base["kv_read_gbs"] = base["value"]
        base["value"] = round(BATCH / (step_ms / 1e3), 1)
        base["unit"] = "tokens/s"
        base["sample"] = (f"a decode step of {BATCH} rows at U[{CTX_LO},{CTX_HI}] tokens, the "
                          f"dominant work of the trace, one layer scaled by {LAYERS}: "
                          f"oracle/oracle.c decode attention, store_kv and the step's "
                          f"block_manager + prepare_paged_batch; median of 5 runs each on "
                          f"{threads} threads (attention also on one)")
        result["cpu_baseline"] = base
    return result


CEILING_POOL = 65536  # pages of 16 tokens x 2 KiB per tensor: 2 GiB each for K and V
CEILING_PAGES_PER_ROW = 288  # config 3's mean row: 4,600 tokens


def bench_ceiling(args):
    """What the part itself allows, measured by libckv_probes.so: one pass over an
    8 GiB buffer with plain and with nontemporal 16-byte loads; the decode's page
    pattern without its arithmetic (a seeded permutation of a 65,536-page K and V
    pool read as config 3's rows, one workgroup per 288 pages and kv head reading
    that head's 256 bytes of every token row, or one per 36 pages reading whole
    2 KiB rows, and the same over pages in pool order; 8, 10 or 16 waves, one,
    two or any number of workgroups per compute unit); and
    back-to-back bf16 32x32x16 products, one 8-wave workgroup per compute unit.
    Each figure is the best of its settings, timed with one event pair around
    `reps` launches after two untimed ones."""
    import torch

    from measure import probes

    device = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    handle = stream.cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(4, dtype=torch.int32, device=device)

    def timed(launch, reps):
        for _ in range(2):
            launch()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            launch()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps / 1e3  # seconds per launch

    # streaming reads
    buf = torch.empty(8 << 30, dtype=torch.uint8, device=device)
    reads = {}
    for nt in (False, True):
        for per_cu in (8, 16, 32, 64):
            grid = cus * per_cu
            s = timed(lambda: probes.read(buf, nt, grid, sink, handle), 10)
            reads[f"{'nontemporal' if nt else 'plain'}_grid{grid}"] = round(buf.numel() / s / 1e9, 1)
    del buf
    torch.cuda.empty_cache()
    best_plain = max(v for k, v in reads.items() if k.startswith("plain"))
    best_nt = max(v for k, v in reads.items() if k.startswith("nontemporal"))
    log(f"streaming reads GB/s: {reads}")

    # the decode's page pattern
    page_bytes = BLOCK * KV_HEADS * HEAD_DIM * 2
    row_bytes = KV_HEADS * HEAD_DIM * 2
    keys = torch.empty(CEILING_POOL * page_bytes, dtype=torch.uint8, device=device)
    values = torch.empty_like(keys)
    gen = np.random.default_rng(args.seed)
    permuted = torch.from_numpy(gen.permutation(CEILING_POOL).astype(np.int32)).to(device)
    ordered = torch.arange(CEILING_POOL, dtype=torch.int32, device=device)
    patterns = {}
    for order, plist in (("permuted", permuted), ("pool_order", ordered)):
        for name, slice_bytes, per_wg in (("head_slice", HEAD_DIM * 2, CEILING_PAGES_PER_ROW),
                                          ("whole_rows", row_bytes,
                                           CEILING_PAGES_PER_ROW // KV_HEADS)):
            best = (0.0, None)
            # waves per workgroup x workgroups per compute unit (an LDS reservation caps
            # them; 0: as many as the registers allow)
            for waves in (8, 10, 16):
                for per_cu in (1, 2, 0):
                    lds = 160 * 1024 // per_cu - 1024 if per_cu else 0
                    s = timed(lambda: probes.pages(keys, values, CEILING_POOL, plist, page_bytes,
                                                   row_bytes, slice_bytes, per_wg, waves, lds,
                                                   sink, handle), 20)
                    gbs = round(2 * CEILING_POOL * page_bytes / s / 1e9, 1)
                    if gbs > best[0]:
                        best = (gbs, f"{waves} waves, {per_cu or 'any'} per CU")
            patterns[f"{order}_{name}"] = {"gbs": best[0], "best_setting": best[1]}
    del keys, values
    torch.cuda.empty_cache()
    log(f"page pattern GB/s: {patterns}")

    # matrix cores
    mfma = {}
    iters = 20000
    for chains in (1, 2, 4):
        s = timed(lambda: probes.mfma(iters, chains, 8, cus, sink, handle), 3)
        flops = cus * 8 * chains * iters * 32 * 32 * 16 * 2
        mfma[f"chains{chains}"] = round(flops / s / 1e12, 1)
    log(f"bf16 MFMA TFLOP/s: {mfma}")

    return {
        "metric": "hardware ceilings: HBM read GB/s (best streaming pass), page-pattern reads, "
                  "bf16 MFMA TFLOP/s",
        "value": best_nt,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": 10,
        "warmup": 2,
        "ms_per_step": round((8 << 30) / best_nt / 1e6, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "uninitialised device buffers (only the loads are measured)",
        "config": {"workload": "ceiling: streaming reads of 8 GiB, the decode's page pattern "
                               "over a 65,536-page pool, back-to-back bf16 MFMA",
                   "compute_units": cus},
        "roofline": {"kernel": "probe_read_kernel (nontemporal)", "bound": "hbm",
                     "achieved": best_nt, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(best_nt / HBM_PEAK_GBS, 4), "traffic": None},
        "streaming_read_gbs": reads,
        "best_plain_read_gbs": best_plain,
        "page_pattern_gbs": patterns,
        "mfma_bf16_tflops": mfma,
        "mfma_frac_of_2500": round(max(mfma.values()) / 2500.0, 4),
        "cpu_baseline": None,
    }


# The default run's other BASELINE configs, each bounded so the whole run stays
# near two minutes: (name, overrides of the command line, what the leg is)
LEGS = (
    ("config2", {"steps": 2000, "warmup": 3},
     "one decode launch over config 2's batch per step, 2,000 timed steps"),
    ("longrow", {"steps": 2000, "warmup": 3},
     "one decode launch over a single 32,768-token row (config 2's layer and pool) per step, "
     "2,000 timed steps"),
    ("config4", {"steps": 5, "warmup": 1, "prefix": 2008, "sequences": PREFILL_SEQS},
     "5 timed steps of config 4 at the 2,008-token prefix (copy-on-write tail)"),
    ("config5", {"steps": 1000},
     "the first 1,000 steps of config 5's churn trace (ramp-up to the live cap included)"),
)
# keys every line carries that a leg would only repeat
LEG_DROP = ("n_gpus", "higher_is_better", "scaling", "vs_baseline", "dtype")


def run_legs(args):
    """Configs 2, 4 and 5 after the headline config 3 (and config 2's layer
    over one long row), each with its own roofline and CPU baseline, so one
    default run measures every BASELINE config with a GPU workload. A leg's
    `value` is that config's own metric."""
    legs = {}
    for name, overrides, what in LEGS:
        sub = argparse.Namespace(**vars(args))
        for key, val in overrides.items():
            setattr(sub, key, val)
        sub.calibrate_copy = sub.gate = sub.rope = sub.no_fuse = False
        log(f"leg {name}: {what}")
        t0 = time.perf_counter()
        fn = {"config2": bench_config2, "longrow": lambda a: bench_config2(a, long_row=True),
              "config4": bench_config4, "config5": bench_config5}[name]
        res = fn(sub)
        leg = {k: v for k, v in res.items() if k not in LEG_DROP}
        leg["leg"] = what
        leg["wall_s"] = round(time.perf_counter() - t0, 2)
        legs[name] = leg
    return legs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one ckv_copy_blocks of 1024 pages (64 MiB read + 64 MiB "
                         "written), the known-size copy the HBM counters are scaled by")
    ap.add_argument("--no-fuse", action="store_true",
                    help="append and decode as two launches instead of ckv_append_decode")
    ap.add_argument("--workload",
                    choices=["config2", "config3", "config4", "config5", "spill", "longrow", "ceiling"],
                    default="config3",
                    help="config3 (default): the headline decode step; config2: one layer of "
                         "decode attention, batch 32 (a step is one launch, default 2000 "
                         "steps); longrow: the same over one 32,768-token row; config4: chunked "
                         "prefill of 64 sequences over a shared prefix (MFMA tiles); config5: "
                         "the continuous-batching churn trace (C++ scheduler driver); spill: "
                         "a cached prefix exported to host memory and imported back; ceiling: the "
                         "part's own streaming-read, page-pattern and MFMA rates (probes)")
    ap.add_argument("--gate", action="store_true",
                    help="config3: the Qwen3.5 sigmoid gate applied in the decode epilogue "
                         "(ckv_append_decode_gated)")
    ap.add_argument("--rope", action="store_true",
                    help="config3: queries and new keys rotated inside the fused decode "
                         "(ckv_rope_append_decode); config4: rotate the chunk's keys inside the "
                         "append (ckv_rope_append) and the queries in place (ckv_rope); Qwen3 "
                         "theta 1e6")
    ap.add_argument("--prefix", type=int, default=2008,
                    help="config4 shared prefix tokens (2008 leaves a partial tail page, "
                         "so every sequence copies it on write; 2000 does not); spill: the "
                         "prefix moved")
    ap.add_argument("--sequences", type=int, default=PREFILL_SEQS,
                    help="config4 sequences (default 64, BASELINE's config); fewer make a "
                         "launch too small to fill the GPU, which splits each tile's keys "
                         "between workgroups (e.g. --sequences 1 --prefix 8000)")
    ap.add_argument("--dtype", choices=["bf16", "f32"], default="bf16",
                    help="config2, config3, config4: the pools' element type (bf16, the "
                         "BASELINE configs; f32, the reference's storage type); an f32 run "
                         "appends no legs")
    ap.add_argument("--no-legs", action="store_true",
                    help="config3: skip the bounded config 2, 4 and 5 legs the default run "
                         "appends to its line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    if args.sequences < 1:
        print("--sequences must be at least 1", file=sys.stderr)
        sys.exit(2)
    if args.dtype != "bf16" and args.workload not in ("config2", "config3", "config4"):
        print(f"--dtype {args.dtype}: config2, config3 and config4 only", file=sys.stderr)
        sys.exit(2)
    if args.workload == "config2":
        result = bench_config2(args)
    elif args.workload == "longrow":
        result = bench_config2(args, long_row=True)
    elif args.workload == "config4":
        result = bench_config4(args)
    elif args.workload == "config5":
        result = bench_config5(args)
    elif args.workload == "spill":
        result = bench_spill(args)
    elif args.workload == "ceiling":
        result = bench_ceiling(args)
    else:
        result = bench_config3(args)
        if not args.no_legs and args.dtype == "bf16":
            result["legs"] = run_legs(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
