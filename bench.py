"""Headline benchmark: paged decode KV-read GB/s (+ tokens/s) at Qwen3-0.6B KV
shapes, batch 128.

One step = one decode step of the hot path: upload the batch metadata (block
tables, positions, slots) once, then for each of 28 layers append one token's
K/V per sequence through the slot mapping and run paged GQA decode attention
over every sequence's full context. Context lengths start uniform in
[1024, 8192] (seeded) and grow by one token per step; pages are handed out in
a seeded random order so tables are non-contiguous. K/V/Q are synthetic
N(0,1) bf16 already resident in HBM when timing starts.

Prints one JSON line (see the keys below). --gpus N > 1 is refused: this
build measures one GPU.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
# HBM bytes per launch of the dominant kernel, from rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes scaled by a known-size copy (written by those passes)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "append_decode_config3_traffic.json")
LAYERS, BATCH, KV_HEADS, Q_HEADS, HEAD_DIM, BLOCK = 28, 128, 8, 16, 128, 16
CTX_LO, CTX_HI = 1024, 8192


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_bytes(kernel):
    """Measured HBM bytes per launch of `kernel` if a counter summary exists."""
    try:
        with open(TRAFFIC_FILE) as fh:
            data = json.load(fh)
    except OSError:
        return None
    entry = data.get("kernels", {}).get(kernel)
    return None if entry is None else int(entry["hbm_bytes_per_launch"])


def cpu_baseline(threads, budget_s=10.0):
    """Oracle decode attention (the CPU restatement of the reference kernel,
    fp32 accumulation) on a bounded sample of the workload: the full batch of
    128 sequences at the same length distribution, bf16 K/V of one layer,
    attended layer after layer until about `budget_s` seconds have passed (at
    most 28 layers). The K/V pages hold a tiled block of N(0,1) values: the
    timing does not depend on the values."""
    from oracle import oracle as orc

    gen = np.random.default_rng(1)
    rows = BATCH
    lengths = [int(x) for x in gen.integers(CTX_LO, CTX_HI + 1, rows)]
    F = KV_HEADS * HEAD_DIM
    pages = [math.ceil(n / BLOCK) for n in lengths]
    n_pages = sum(pages)
    block = orc.from_f32(gen.standard_normal(1 << 22, np.float32), orc.BF16)
    reps = -(-(n_pages * BLOCK * F) // block.size)
    kc = np.tile(block, reps)[:n_pages * BLOCK * F]
    vc = np.roll(kc, 12345)
    q = orc.from_f32(gen.standard_normal((rows, Q_HEADS * HEAD_DIM), np.float32), orc.BF16)
    perm = gen.permutation(n_pages).astype(np.uint32)
    offsets = np.cumsum([0] + pages[:-1])
    att = orc.Attention((1, n_pages, BLOCK, KV_HEADS, HEAD_DIM), kc, vc, orc.BF16, q, orc.BF16,
                        [n - 1 for n in lengths], perm, offsets, pages, Q_HEADS, 0,
                        1 / math.sqrt(HEAD_DIM))
    layer_bytes = sum(lengths) * F * 2 * 2
    layers = 0
    t0 = time.perf_counter()
    while layers < LAYERS and (layers == 0 or time.perf_counter() - t0 < budget_s):
        att.online_threads(threads)
        layers += 1
    dt = time.perf_counter() - t0
    one = orc.Attention((1, n_pages, BLOCK, KV_HEADS, HEAD_DIM), kc, vc, orc.BF16, q[:4],
                        orc.BF16, [n - 1 for n in lengths[:4]], perm, offsets[:4], pages[:4],
                        Q_HEADS, 0, 1 / math.sqrt(HEAD_DIM))
    t1 = time.perf_counter()
    one.online_threads(1)
    dt1 = time.perf_counter() - t1
    single_gbs = sum(lengths[:4]) * F * 4 / dt1 / 1e9
    return {
        "value": round(layers * layer_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/oracle.c decode attention (restated paged_attention_f32, fp32 "
                   f"accumulate) over {rows} sequences ({sum(lengths)} tokens, "
                   f"{layer_bytes / 1e9:.2f} GB of bf16 K/V per layer) x {layers} layers in "
                   f"{dt:.1f} s on {threads} threads; single-thread {single_gbs:.3f} GB/s on 4 "
                   f"of them"),
    }


def bench_config3(args):
    import torch

    from chibillm_amd import ckv
    from oracle import oracle as orc  # seeded lengths / page order only

    device = torch.device("cuda:0")
    rng = orc.Mt64(args.seed)
    lengths = np.array([rng.uniform_int(CTX_LO, CTX_HI) for _ in range(BATCH)], np.int64)
    total_steps = args.warmup + args.steps
    max_len = lengths + total_steps
    pages_needed = [math.ceil(n / BLOCK) for n in max_len]
    n_pool = sum(pages_needed) + 64
    perm = rng.permutation(n_pool)
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

    kv_gb = LAYERS * n_pool * BLOCK * F * 2 * 2 / 1e9
    log(f"pool {n_pool} pages x {LAYERS} layers = {kv_gb:.1f} GB K+V; "
        f"context tokens {int(lengths.sum())}")
    ctx = ckv.Context(0, stream=torch.cuda.current_stream())
    if args.calibrate_copy:
        calib = ckv.Pool(ctx, 1, 2048, BLOCK, KV_HEADS, HEAD_DIM, ckv.BF16)
        calib.copy_blocks(np.arange(1024), np.arange(1024, 2048))
        ctx.sync()
        calib.close()
        log("calibration copy: 1024 pages x 32 KiB, keys + values = 64 MiB read, 64 MiB written")
    elems = LAYERS * n_pool * BLOCK * F
    keys = torch.empty(elems, dtype=torch.bfloat16, device=device)
    values = torch.empty(elems, dtype=torch.bfloat16, device=device)
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed)
    t0 = time.perf_counter()
    step = 1 << 30
    for buf in (keys, values):
        for i in range(0, elems, step):
            buf[i:i + step].normal_(generator=gen)
    torch.cuda.synchronize()
    log(f"filled K/V with N(0,1) in {time.perf_counter() - t0:.1f} s")
    pool = ckv.Pool(ctx, LAYERS, n_pool, BLOCK, KV_HEADS, HEAD_DIM, ckv.BF16, keys, values)

    q = torch.randn(LAYERS, BATCH, Q_HEADS * HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    k_new = torch.randn(LAYERS, BATCH, F, generator=gen, device=device).to(torch.bfloat16)
    v_new = torch.randn(LAYERS, BATCH, F, generator=gen, device=device).to(torch.bfloat16)
    out = torch.empty(LAYERS, BATCH, Q_HEADS * HEAD_DIM, dtype=torch.bfloat16, device=device)
    gate = (torch.randn(LAYERS, BATCH, Q_HEADS * HEAD_DIM, generator=gen, device=device)
            .to(torch.bfloat16) if args.gate else None)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    offsets = np.arange(BATCH, dtype=np.uint32) * max_pages

    def one_step():
        positions = lengths.copy()  # the new token's position
        for s in range(BATCH):
            ensure_pages(s, int(positions[s]) + 1)
        slots = [int(flat[s * max_pages + p // BLOCK]) * BLOCK + p % BLOCK
                 for s, p in enumerate(positions)]
        pool.upload(flat, offsets, owned, positions, slots)
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
        attended = positions + 1
        lengths[:] = attended
        return int(attended.sum()), int(sum(math.ceil(a / BLOCK) for a in attended))

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} steps done")

    ctx.profile(True)
    ctx.profile_reset()
    tokens_attended = pages_read = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks, pages = one_step()
        tokens_attended += toks
        pages_read += pages
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    dominant = ("paged_attention_decode" if args.no_fuse
                else "rope_append_decode" if args.rope else "append_decode")
    decode_ms, decode_n = ctx.profile_query(dominant)
    merge_ms, merge_n = ctx.profile_query("paged_attention_merge")
    store_ms, store_n = ctx.profile_query("store_kv")
    ctx.profile(False)
    log(f"timed {args.steps} steps in {elapsed:.3f} s")

    kv_row_bytes = F * 2 * 2  # K + V, bf16, all KV heads
    kv_bytes = LAYERS * tokens_attended * kv_row_bytes
    value = kv_bytes / elapsed / 1e9
    ms_per_step = elapsed * 1e3 / args.steps
    # algorithmic bytes of one launch (one layer): KV of every attended token,
    # Q and O, the table entries read, and (fused) the new K/V rows written
    appended = 0 if args.no_fuse else BATCH * kv_row_bytes
    qo_rows = 3 if args.gate else 2  # Q and O, and the gate when it is read
    per_launch = (tokens_attended * kv_row_bytes + pages_read * 4
                  + args.steps * (qo_rows * BATCH * Q_HEADS * HEAD_DIM * 2 + appended)) / args.steps
    decode_avg_s = decode_ms / decode_n / 1e3
    achieved = per_launch / decode_avg_s / 1e9
    result = {
        "metric": "paged decode KV-read GB/s (% HBM peak) + tokens/s, Qwen3-0.6B KV, batch 128",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
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
        "kernels_ms_per_step": {
            dominant: round(decode_ms / args.steps, 4),
            "paged_attention_merge": round(merge_ms / args.steps, 4),
            "store_kv": round(store_ms / args.steps, 4),
        },
        "roofline": {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes(dominant),
            "avg_launch_us": round(decode_avg_s * 1e6, 2),
            "algorithmic_bytes_per_launch": int(per_launch),
        },
        "cpu_baseline": None,
    }
    pool.close()
    del keys, values
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        log(f"CPU baseline on {threads} threads")
        result["cpu_baseline"] = cpu_baseline(threads)
    return result

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
ROPE_THETA = 1e6  # Qwen3-0.6B rope_theta
PREFILL_SEQS, PREFILL_CHUNK = 64, 512


def prefill_flops(prefix, chunk, seqs):
    """Causal attention FLOPs of one layer: QK^T and PV, 2 FLOPs per MAC each,
    over the keys each row attends (prefix + its own position + 1)."""
    keys = sum(prefix + i + 1 for i in range(chunk))
    return 4 * HEAD_DIM * Q_HEADS * seqs * keys


def prefill_cpu_baseline(threads, prefix):
    """Oracle causal attention (restated paged_flash_attention_prefill_f32 maths,
    fp32) on a bounded sample: 4 sequences x 256 chunk rows of one layer."""
    from oracle import oracle as orc

    gen = np.random.default_rng(2)
    seqs, rows = 4, 256
    F = KV_HEADS * HEAD_DIM
    pages = math.ceil((prefix + rows) / BLOCK)
    n_pages = pages * seqs
    kc = orc.from_f32(gen.standard_normal(n_pages * BLOCK * F, np.float32), orc.BF16)
    vc = orc.from_f32(gen.standard_normal(n_pages * BLOCK * F, np.float32), orc.BF16)
    q = orc.from_f32(gen.standard_normal((seqs * rows, Q_HEADS * HEAD_DIM), np.float32),
                     orc.BF16)
    table = gen.permutation(n_pages).astype(np.uint32)
    positions = [prefix + i for _ in range(seqs) for i in range(rows)]
    offsets = [s * pages for s in range(seqs) for _ in range(rows)]
    att = orc.Attention((1, n_pages, BLOCK, KV_HEADS, HEAD_DIM), kc, vc, orc.BF16, q, orc.BF16,
                        positions, table, offsets, [pages] * len(positions), Q_HEADS, 0,
                        1 / math.sqrt(HEAD_DIM))
    t0 = time.perf_counter()
    att.online_threads(threads)
    dt = time.perf_counter() - t0
    flops = prefill_flops(prefix, rows, seqs)
    return {
        "value": round(flops / dt / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/oracle.c causal attention over paged bf16 K/V, fp32 accumulate: "
                   f"1 layer x {seqs} sequences x {rows} rows at positions {prefix}.."
                   f"{prefix + rows - 1} ({flops / 1e9:.1f} GFLOP) in {dt:.2f} s on "
                   f"{threads} threads"),
    }


def bench_config4(args):
    """64 sequences share one prefix held once as pages; each step restores it
    for every sequence (shared full pages; a copy-on-write copy of a partial
    tail page, all layers, one ckv_copy_blocks), uploads the chunk's metadata,
    then per layer appends the 512-row chunks and runs the MFMA prefill."""
    import torch

    from chibillm_amd import ckv
    from oracle import oracle as orc  # seeded page order only

    device = torch.device("cuda:0")
    prefix, S, C = args.prefix, PREFILL_SEQS, PREFILL_CHUNK
    F = KV_HEADS * HEAD_DIM
    full = prefix // BLOCK
    partial = prefix % BLOCK != 0
    prefix_pages = math.ceil(prefix / BLOCK)
    own = math.ceil((prefix + C) / BLOCK) - full
    n_pool = prefix_pages + S * own + 16
    perm = orc.Mt64(args.seed).permutation(n_pool)
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
    elems = LAYERS * n_pool * BLOCK * F
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed)
    keys = torch.empty(elems, dtype=torch.bfloat16, device=device).normal_(generator=gen)
    values = torch.empty(elems, dtype=torch.bfloat16, device=device).normal_(generator=gen)
    pool = ckv.Pool(ctx, LAYERS, n_pool, BLOCK, KV_HEADS, HEAD_DIM, ckv.BF16, keys, values)
    rows = S * C
    q = torch.randn(LAYERS, rows, Q_HEADS * HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    k_new = torch.randn(LAYERS, rows, F, generator=gen, device=device).to(torch.bfloat16)
    v_new = torch.randn(LAYERS, rows, F, generator=gen, device=device).to(torch.bfloat16)
    out = torch.empty(LAYERS, rows, Q_HEADS * HEAD_DIM, dtype=torch.bfloat16, device=device)
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
    result = {
        "metric": "chunked-prefill attention TFLOP/s (MFMA) + tokens/s, Qwen3-0.6B KV, "
                  "64 sequences x 512-token chunks over a shared prefix",
        "value": round(LAYERS * flops * args.steps / elapsed / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
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
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "avg_launch_us": round(avg_s * 1e6, 2),
            "algorithmic_flops_per_launch": flops,
        },
        "cpu_baseline": None,
    }
    if args.rope:
        # the fused append's algorithmic bytes: key and value rows read, page
        # rows written, positions and slots
        ms, n = kernels["rope_append"]
        per = rows * (4 * F * 2 + 8)
        result["rope_append"] = {"avg_launch_us": round(ms / n * 1e3, 2),
                                 "bytes_per_launch": per,
                                 "achieved_gbs": round(per / (ms / n / 1e3) / 1e9, 2)}
        result["config"]["workload"] += "; keys rotated inside the append, queries by ckv_rope"
    pool.close()
    del keys, values, q, k_new, v_new, out
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        log(f"CPU baseline on {threads} threads")
        result["cpu_baseline"] = prefill_cpu_baseline(threads, prefix)
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
    from oracle import oracle as orc  # seeded page order only

    device = torch.device("cuda:0")
    tokens = args.prefix
    F = KV_HEADS * HEAD_DIM
    pages = math.ceil(tokens / BLOCK)
    n_pool = 2 * pages + 16
    perm = orc.Mt64(args.seed).permutation(n_pool)
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
    default 20 is given); warmup does not apply to a trace."""
    import subprocess

    steps = CHURN_STEPS if args.steps == 20 else args.steps
    driver = os.path.join(ROOT, "chibillm_amd", "bin", "churn")
    if not os.path.exists(driver):
        raise SystemExit(f"{driver} is not built: run __graft_entry__.build()")
    cmd = [driver, "--steps", str(steps), "--seed", str(args.seed), "--profile"]
    log("config5: " + " ".join(cmd))
    proc = subprocess.run(cmd, capture_output=True, text=True)
    sys.stderr.write(proc.stderr)
    if proc.returncode != 0:
        raise SystemExit(f"churn driver failed ({proc.returncode})")
    trace = json.loads(proc.stdout.strip().splitlines()[-1])
    decode_ms, decode_n = trace["kernels_ms"]["append_decode"]
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
        "kernels_ms_per_step": {k: round(v[0] / steps, 4) for k, v in trace["kernels_ms"].items()},
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
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        log(f"CPU baseline on {threads} threads")
        base = cpu_baseline(threads)
        base["sample"] = "decode attention, the dominant work of the trace: " + base["sample"]
        result["cpu_baseline"] = base
    return result


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
    ap.add_argument("--workload", choices=["config3", "config4", "config5", "spill"],
                    default="config3",
                    help="config3 (default): the headline decode step; config4: chunked "
                         "prefill of 64 sequences over a shared prefix (MFMA tiles); config5: "
                         "the continuous-batching churn trace (C++ scheduler driver); spill: "
                         "a cached prefix exported to host memory and imported back")
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
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    if args.workload == "config4":
        result = bench_config4(args)
    elif args.workload == "config5":
        result = bench_config5(args)
    elif args.workload == "spill":
        result = bench_spill(args)
    else:
        result = bench_config3(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
