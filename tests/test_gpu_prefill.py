"""Chunked-prefill attention on the matrix cores (ckv_prefill_attention /
ckv_attention with query tiles) against the CPU oracle: causal attention of
each chunk row over its sequence's prefix + chunk through the block table,
within 2e-2 abs + 1e-2 rel (bf16/fp16 storage, fp32 accumulation).

The shared-prefix case follows config 4's shape at a reduced batch: sequences
share the prefix's full pages, each takes a copy-on-write copy of a partial
tail page, appends its chunk and attends over prefix + chunk."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import assert_close, new_context, new_pool, to_dev, to_f32, to_host

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def scale():
    return float(np.float32(1 / math.sqrt(D)))


def pages_for(tokens):
    return -(-tokens // 16)


@pytest.mark.parametrize("prefix", [2000, 2008])
def test_shared_prefix_chunks_with_copy_on_write_tail(ctx, prefix):
    print(f"shared prefix {prefix}", flush=True)
    H, Hq, S, C = 8, 16, 3, 300
    F = H * D
    rng = orc.Mt64(40 + prefix)
    prefix_pages = pages_for(prefix)
    partial = prefix % 16 != 0
    full = prefix // 16
    own = pages_for(prefix + C) - full  # each sequence's private pages (tail copy first)
    blocks = prefix_pages + S * own + 5
    geom = (1, blocks, 16, H, D)
    pool, kd, vd = new_pool(ctx, geom, orc.BF16)
    slot_count = blocks * 16
    kc = np.zeros(slot_count * F, np.uint16)
    vc = np.zeros_like(kc)

    # the prefix, written once through the append path
    prefix_table = np.arange(prefix_pages, dtype=np.uint32)
    pk = rng.normal(prefix * F, orc.BF16).reshape(prefix, F)
    pv = rng.normal(prefix * F, orc.BF16).reshape(prefix, F)
    slots = [orc.slot(prefix_table, p, 16) for p in range(prefix)]
    pool.upload(prefix_table, [0] * prefix, [prefix_pages] * prefix, list(range(prefix)), slots)
    pool.append(0, to_dev(pk, orc.BF16), to_dev(pv, orc.BF16))
    orc.store_kv(kc, vc, pk, pv, slots, 0, slot_count)

    # per-sequence tables: shared full pages, then private pages
    tables = []
    for s in range(S):
        mine = prefix_pages + s * own + np.arange(own, dtype=np.uint32)
        tables.append(np.concatenate([prefix_table[:full], mine]).astype(np.uint32))
    if partial:  # copy-on-write of the shared tail page into each sequence's first own page
        src = [int(prefix_table[full])] * S
        dst = [int(t[full]) for t in tables]
        pool.copy_blocks(src, dst)
        orc.copy_blocks(kc, vc, geom, src, dst)

    # each sequence appends its chunk, then attends
    positions, offsets, lengths, slots, ks, vs = [], [], [], [], [], []
    flat = np.concatenate(tables)
    at = 0
    for t in tables:
        positions += list(range(prefix, prefix + C))
        offsets += [at] * C
        lengths += [len(t)] * C
        slots += [orc.slot(t, p, 16) for p in range(prefix, prefix + C)]
        at += len(t)
        ks.append(rng.normal(C * F, orc.BF16).reshape(C, F))
        vs.append(rng.normal(C * F, orc.BF16).reshape(C, F))
    ks, vs = np.concatenate(ks), np.concatenate(vs)
    q = rng.normal(S * C * Hq * D, orc.BF16).reshape(S * C, Hq * D)
    pool.upload(flat, offsets, lengths, positions, slots)
    pool.append(0, to_dev(ks, orc.BF16), to_dev(vs, orc.BF16))
    orc.store_kv(kc, vc, ks, vs, slots, 0, slot_count)
    ctx.sync()
    assert np.array_equal(to_host(kd, orc.BF16), kc)
    assert np.array_equal(to_host(vd, orc.BF16), vc)

    expected = orc.Attention(geom, kc, vc, orc.BF16, q, orc.BF16, positions, flat, offsets,
                             lengths, Hq, 0, scale()).online_threads(8)
    qd = to_dev(q, orc.BF16)
    for name in ("attention", "prefill"):
        out = torch.full_like(qd, float("nan"))
        getattr(pool, name)(0, qd, Hq, scale(), out)
        ctx.sync()
        assert_close(to_f32(out), expected, what=f"{name}, prefix {prefix}")
    pool.close()


# (first position, rows) per sequence: single rows, rows across page and
# 32-key block edges, tiles longer than one workgroup's share, a chunk
# starting mid-page, and decode rows of other sequences in the same batch
RAGGED = [(0, 1), (0, 40), (5, 300), (100, 33), (16, 257), (1000, 64), (700, 1), (63, 2)]


@pytest.mark.parametrize("waves", [None, "8"])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16, orc.F32])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_ragged_tiles_every_group_size(ctx, group, code, waves, monkeypatch):
    """Every route (auto, prefill, decode form) against the oracle; f32 pages
    (the reference's storage dtype, fp32 products on the matrix cores) within
    1e-5 abs + 1e-4 rel, and their prefill takes the MFMA kernel (one
    paged_attention_prefill launch). This batch is too small to give every
    compute unit an 8-wave workgroup, so 16-bit pools with GQA groups up to 4
    take 4-wave workgroups by default; waves "8" forces the 8-wave kernel."""
    if waves:
        monkeypatch.setenv("CKV_PREFILL_WAVES", waves)
    print(f"ragged tiles group {group} dtype {code} waves {waves}", flush=True)
    H = 2
    Hq = H * group
    F = H * D
    rng = orc.Mt64(7 * group + code)
    lengths_tok = [start + n for start, n in RAGGED]
    total_pages = sum(pages_for(n) for n in lengths_tok)
    blocks = total_pages + 7
    perm = rng.permutation(blocks)
    geom = (2, blocks, 16, H, D)
    slot_count = blocks * 16
    kc = rng.normal(2 * slot_count * F, code)  # every slot finite, layer 1 used
    vc = rng.normal(2 * slot_count * F, code)
    tables, at = [], 0
    for n in lengths_tok:
        tables.append(perm[at:at + pages_for(n)])
        at += pages_for(n)
    flat = np.concatenate(tables)
    positions, offsets, lengths = [], [], []
    at = 0
    for (start, n), t in zip(RAGGED, tables):
        positions += list(range(start, start + n))
        offsets += [at] * n
        lengths += [len(t)] * n
        at += len(t)
    rows = len(positions)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    pool, kd, vd = new_pool(ctx, geom, code)
    kd.copy_(to_dev(kc, code))
    vd.copy_(to_dev(vc, code))
    pool.upload(flat, offsets, lengths, positions)
    expected = orc.Attention(geom, kc, vc, code, q, code, positions, flat, offsets, lengths, Hq,
                             1, scale()).online_threads(8)
    qd = to_dev(q, code)
    tol = dict(atol=1e-5, rtol=1e-4) if code == orc.F32 else {}
    for name in ("attention", "prefill", "decode"):
        out = torch.full_like(qd, float("nan"))
        ctx.sync()
        ctx.profile(True)
        ctx.profile_reset()
        getattr(pool, name)(1, qd, Hq, scale(), out)
        ctx.sync()
        launches = ctx.profile_query("paged_attention_prefill")[1]
        ctx.profile(False)
        assert launches == (0 if name == "decode" else 1), (name, launches)
        assert_close(to_f32(out), expected, what=f"{name}, group {group}", **tol)
    pool.close()


# (first position, rows): tiles whose last key block is block 7, 8, ..., 16, so
# the 8-wave kernel's steady loop (pairs of blocks while kb + 8 < n_blocks)
# runs zero to four times and leaves each possible remainder to the checked
# iterations, in both halves of the workgroup
BOUNDARIES = [(250, 6), (270, 18), (300, 20), (330, 22), (360, 24), (400, 16), (420, 28),
              (470, 10), (500, 12), (520, 24)]


@pytest.mark.parametrize("waves", [None, "8"])
@pytest.mark.parametrize("group", [2, 4])
def test_steady_loop_boundaries(ctx, group, waves, monkeypatch):
    """Tiles of 8 to 17 key blocks through the prefill kernel against the
    oracle (bf16)."""
    if waves:
        monkeypatch.setenv("CKV_PREFILL_WAVES", waves)
    print(f"steady-loop boundaries group {group} waves {waves}", flush=True)
    code = orc.BF16
    H = 2
    Hq = H * group
    F = H * D
    rng = orc.Mt64(91 + group)
    lengths_tok = [start + n for start, n in BOUNDARIES]
    blocks = sum(pages_for(n) for n in lengths_tok) + 3
    perm = rng.permutation(blocks)
    geom = (1, blocks, 16, H, D)
    slot_count = blocks * 16
    kc = rng.normal(slot_count * F, code)
    vc = rng.normal(slot_count * F, code)
    tables, at = [], 0
    for n in lengths_tok:
        tables.append(perm[at:at + pages_for(n)])
        at += pages_for(n)
    flat = np.concatenate(tables)
    positions, offsets, lengths = [], [], []
    at = 0
    for (start, n), t in zip(BOUNDARIES, tables):
        positions += list(range(start, start + n))
        offsets += [at] * n
        lengths += [len(t)] * n
        at += len(t)
    rows = len(positions)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    pool, kd, vd = new_pool(ctx, geom, code)
    kd.copy_(to_dev(kc, code))
    vd.copy_(to_dev(vc, code))
    pool.upload(flat, offsets, lengths, positions)
    expected = orc.Attention(geom, kc, vc, code, q, code, positions, flat, offsets, lengths, Hq,
                             0, scale()).online_threads(8)
    qd = to_dev(q, code)
    out = torch.full_like(qd, float("nan"))
    pool.prefill(0, qd, Hq, scale(), out)
    ctx.sync()
    assert_close(to_f32(out), expected, what=f"boundaries, group {group}, waves {waves}")
    pool.close()


# a long chunk over a long prefix (three tiles, the last of one row), a short
# sequence beside it, and a chunk that starts at position 0
LONG = [(3000, 513), (40, 200), (0, 130)]
_long_expected = {}


@pytest.mark.parametrize("split", [None, "1", "3", "8", "8/1"])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16, orc.F32])
@pytest.mark.parametrize("group", [1, 4])
def test_key_split_of_small_launches(ctx, group, code, split, monkeypatch):
    """A launch too small to fill the GPU splits each long tile's key blocks
    between up to 8 workgroups (16-bit pools in 4-wave workgroups, f32 pools
    in the fp32 kernel's 8-wave ones), and the last of them to finish folds every
    range's (max, denominator, accumulator) record; the result matches the
    oracle for every split (None: the launch's own choice, "1": no split,
    "3": ranges of uneven length, "8/1": ranges down to one 32-key block, so
    that some ranges lie wholly after some of their rows' positions and carry
    a -inf maximum that must weigh nothing), is the same bit for bit on a
    second call (the arrival counters are left at zero), and is one
    paged_attention_prefill launch."""
    if split:
        n, _, least = split.partition("/")
        monkeypatch.setenv("CKV_PREFILL_SPLIT", n)
        if least:
            monkeypatch.setenv("CKV_PREFILL_SPLIT_MIN", least)
    print(f"key split group {group} dtype {code} split {split}", flush=True)
    H = 2
    Hq = H * group
    F = H * D
    rng = orc.Mt64(11 * group + code)
    lengths_tok = [start + n for start, n in LONG]
    total_pages = sum(pages_for(n) for n in lengths_tok)
    blocks = total_pages + 3
    perm = rng.permutation(blocks)
    geom = (1, blocks, 16, H, D)
    slot_count = blocks * 16
    kc = rng.normal(slot_count * F, code)
    vc = rng.normal(slot_count * F, code)
    tables, at = [], 0
    for n in lengths_tok:
        tables.append(perm[at:at + pages_for(n)])
        at += pages_for(n)
    flat = np.concatenate(tables)
    positions, offsets, lengths = [], [], []
    at = 0
    for (start, n), t in zip(LONG, tables):
        positions += list(range(start, start + n))
        offsets += [at] * n
        lengths += [len(t)] * n
        at += len(t)
    rows = len(positions)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    pool, kd, vd = new_pool(ctx, geom, code)
    kd.copy_(to_dev(kc, code))
    vd.copy_(to_dev(vc, code))
    pool.upload(flat, offsets, lengths, positions)
    key = (group, code)
    if key not in _long_expected:
        _long_expected[key] = orc.Attention(geom, kc, vc, code, q, code, positions, flat, offsets,
                                            lengths, Hq, 0, scale()).online_threads(8)
    expected = _long_expected[key]
    qd = to_dev(q, code)
    tol = dict(atol=1e-5, rtol=1e-4) if code == orc.F32 else {}
    outs = []
    for _ in range(2):
        out = torch.full_like(qd, float("nan"))
        ctx.sync()
        ctx.profile(True)
        ctx.profile_reset()
        pool.prefill(0, qd, Hq, scale(), out)
        ctx.sync()
        launches = ctx.profile_query("paged_attention_prefill")[1]
        ctx.profile(False)
        assert launches == 1, launches
        assert_close(to_f32(out), expected, what=f"split {split}, group {group}", **tol)
        outs.append(out)
    bits = torch.int32 if code == orc.F32 else torch.int16
    assert torch.equal(outs[0].view(bits), outs[1].view(bits))
    pool.close()


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_layer_beyond_4_gib_takes_64_bit_page_addresses(ctx, code):
    """A pool whose layer spans more than 4 GiB per tensor (140,000 bf16 or
    70,000 f32 pages of 32 or 64 KiB) makes the kernels address pages with
    64-bit arithmetic; two sequences whose pages lie above the 4 GiB line (one
    of them interleaved with pages below it) attend over 1,000 tokens with
    200-row chunks through the prefill and decode forms, checked against the
    oracle over a compact copy of the pages used."""
    H, Hq, n, chunk = 8, 16, 1000, 200
    F = H * D
    es = 4 if code == orc.F32 else 2
    blocks = 140_000 * 2 // es
    assert blocks * 16 * F * es > 1 << 32
    rng = orc.Mt64(77)
    n_pages = pages_for(n)
    high = np.arange(blocks - n_pages, blocks, dtype=np.uint32)  # byte offsets past 4 GiB
    mixed = np.empty(n_pages, np.uint32)
    mixed[0::2] = np.arange(5, 5 + len(mixed[0::2]), dtype=np.uint32)
    mixed[1::2] = np.arange(blocks - 3 * n_pages, blocks - 3 * n_pages + len(mixed[1::2]),
                            dtype=np.uint32)
    tables = [high, mixed]
    ks = [rng.normal(n * F, code).reshape(n, F) for _ in tables]
    vs = [rng.normal(n * F, code).reshape(n, F) for _ in tables]
    print(f"prefill over a {blocks}-page layer ({blocks * 16 * F * es / 2**30:.2f} GiB per "
          f"tensor), dtype {code}", flush=True)
    pool, _, _ = new_pool(ctx, (1, blocks, 16, H, D), code)
    for t, k, v in zip(tables, ks, vs):
        slots = [orc.slot(t, p, 16) for p in range(n)]
        pool.upload(t, [0] * n, [len(t)] * n, list(range(n)), slots)
        pool.append(0, to_dev(k, code), to_dev(v, code))
    positions = list(range(n - chunk, n)) * 2
    offsets = [0] * chunk + [n_pages] * chunk
    lengths = [n_pages] * (2 * chunk)
    rows = len(positions)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    pool.upload(np.concatenate(tables), offsets, lengths, positions)
    # the oracle over a compact pool: page j of sequence s renumbered s * n_pages + j
    kc = np.zeros(2 * n_pages * 16 * F, ks[0].dtype)
    vc = np.zeros_like(kc)
    for s_i, (k, v) in enumerate(zip(ks, vs)):
        compact = np.arange(s_i * n_pages, (s_i + 1) * n_pages, dtype=np.uint32)
        slots = [orc.slot(compact, p, 16) for p in range(n)]
        orc.store_kv(kc, vc, k, v, slots, 0, 2 * n_pages * 16)
    flat_c = np.arange(2 * n_pages, dtype=np.uint32)
    expected = orc.Attention((1, 2 * n_pages, 16, H, D), kc, vc, code, q, code, positions,
                             flat_c, offsets, lengths, Hq, 0, scale()).online_threads(8)
    qd = to_dev(q, code)
    tol = dict(atol=1e-5, rtol=1e-4) if code == orc.F32 else {}
    for name in ("prefill", "attention", "decode"):
        out = torch.full_like(qd, float("nan"))
        getattr(pool, name)(0, qd, Hq, scale(), out)
        ctx.sync()
        assert_close(to_f32(out), expected, what=f"{name} over a {blocks}-page layer", **tol)
    pool.close()
    del pool
    torch.cuda.empty_cache()


@pytest.mark.parametrize("scale_value", [-0.125, 0.0])
def test_non_positive_scale_matches_the_oracle(ctx, scale_value):
    """softmax(q.k * scale) for scale <= 0 (the reference takes any scale): the
    prefill route hands such batches to the decode form, which scales every
    score before taking maxima; a 40-row chunk of one sequence against the
    oracle."""
    H, Hq, n, chunk = 2, 4, 300, 40
    F = H * D
    rng = orc.Mt64(91)
    table = rng.permutation(pages_for(n) + 3)[:pages_for(n)].astype(np.uint32)
    blocks = pages_for(n) + 3
    k = rng.normal(n * F, orc.BF16).reshape(n, F)
    v = rng.normal(n * F, orc.BF16).reshape(n, F)
    pool, _, _ = new_pool(ctx, (1, blocks, 16, H, D), orc.BF16)
    pool.upload(table, [0] * n, [len(table)] * n, list(range(n)),
                [orc.slot(table, p, 16) for p in range(n)])
    pool.append(0, to_dev(k, orc.BF16), to_dev(v, orc.BF16))
    positions = list(range(n - chunk, n))
    pool.upload(table, [0] * chunk, [len(table)] * chunk, positions)
    q = rng.normal(chunk * Hq * D, orc.BF16).reshape(chunk, Hq * D)
    kc = np.zeros(blocks * 16 * F, np.uint16)
    vc = np.zeros_like(kc)
    orc.store_kv(kc, vc, k, v, [orc.slot(table, p, 16) for p in range(n)], 0, blocks * 16)
    expected = orc.Attention((1, blocks, 16, H, D), kc, vc, orc.BF16, q, orc.BF16, positions,
                             table, [0] * chunk, [len(table)] * chunk, Hq, 0,
                             scale_value).online_threads(8)
    qd = to_dev(q, orc.BF16)
    for name in ("prefill", "attention"):
        out = torch.full_like(qd, float("nan"))
        getattr(pool, name)(0, qd, Hq, scale_value, out)
        ctx.sync()
        assert_close(to_f32(out), expected, what=f"{name}, scale {scale_value}")
    pool.close()
