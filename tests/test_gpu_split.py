"""The fast decode kernel over rows the batch plan cuts into page chunks (the
split-K of paged_attention_partial_f32 / paged_attention_reduce_f32,
src/metal/kernels/attention.metal:446-615, for any row): single long rows, the
records across consecutive launches, and the fused append, all against
the CPU oracle within 2e-2 abs + 1e-2 rel and the unfused pair bit for bit.
Also the host checks that keep the fused append and the RoPE tables in bounds."""
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import (assert_close, force_plan, new_context, new_pool, to_dev, to_f32,
                            to_host)
from tests.test_gpu_parity import compact_oracle, fill_by_append

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1 / math.sqrt(128)))


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def rows_case(seed, lengths, H=8):
    """Seeded K/V rows and queries for rows of `lengths` tokens on permuted pages."""
    rng = orc.Mt64(seed)
    B = sum(-(-n // 16) for n in lengths) + 7
    perm = rng.permutation(B)
    tables, at = [], 0
    for n in lengths:
        tables.append(perm[at:at + -(-n // 16)])
        at += len(tables[-1])
    F = H * 128
    ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    q = rng.normal(len(lengths) * 2 * H * 128, orc.BF16).reshape(len(lengths), -1)
    return B, tables, ks, vs, q


def fused_and_unfused(ctx, lengths, B, tables, ks, vs, q, H=8, layers=1, layer=0):
    """The last token of every row appended by ckv_append_decode in one pool and
    by ckv_append + ckv_decode_attention in another; returns both outputs and
    both pools' tensors."""
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    outs, caches, plans = [], [], []
    for fused in (True, False):
        pool, keys, values = new_pool(ctx, (layers, B, 16, H, 128), orc.BF16, fill=float("nan"))
        fill_by_append(pool, [n - 1 for n in lengths], tables, [k[:-1] for k in ks],
                       [v[:-1] for v in vs], layer=layer)
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        plans.append(pool.decode_plan())
        k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
        v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
        out = torch.full((len(lengths), 2 * H * 128), float("nan"), dtype=torch.bfloat16,
                         device="cuda")
        if fused:
            pool.append_decode(layer, k_new, v_new, to_dev(q, orc.BF16), 2 * H, SCALE, out)
        else:
            pool.append(layer, k_new, v_new)
            pool.decode(layer, to_dev(q, orc.BF16), 2 * H, SCALE, out)
        ctx.sync()
        outs.append(out)
        caches.append((keys, values))
        pool.close()
    assert plans[0] == plans[1]
    return outs, caches, plans[0]


@pytest.mark.parametrize("lengths", [[5000], [40960], [40960, 300, 7], [32768, 32768]])
def test_long_rows_cut_into_chunks(ctx, lengths):
    """Rows far longer than a compute unit's share of the batch: the default
    plan cuts them into chunks over every compute unit. The fused step equals
    append-then-decode bit for bit (pages and outputs; unwritten slots hold
    NaN), and the oracle within tolerance."""
    print(f"long rows {lengths}", flush=True)
    B, tables, ks, vs, q = rows_case(41 + len(lengths), lengths)
    outs, caches, (span, items, records) = fused_and_unfused(ctx, lengths, B, tables, ks, vs, q)
    assert span > 0 and records > 0, "a long row must be cut"
    pages = [-(-n // 16) for n in lengths]
    assert items >= sum(-(-p // span) for p in pages)
    assert torch.equal(caches[0][0].view(torch.int16), caches[1][0].view(torch.int16))
    assert torch.equal(caches[0][1].view(torch.int16), caches[1][1].view(torch.int16))
    assert torch.equal(outs[0], outs[1])
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(outs[0]), expected, what=f"rows {lengths} (chunks of {span} pages)")


@pytest.mark.parametrize("split", ["b3", "b25", "b400"])
def test_fused_append_in_balanced_workgroups(ctx, split, monkeypatch):
    """The fused append + decode with the batch dealt out 3, 25 or 400 pages
    to a workgroup over 40 rows of 1-700 tokens: a workgroup attends to
    several rows (and row pieces) in turn and appends a row's new token when
    it reaches the row's last page. Fused equals append-then-decode bit for
    bit (pages and outputs), and the oracle within tolerance."""
    force_plan(monkeypatch, split)
    print(f"fused balanced {split}", flush=True)
    rng = np.random.default_rng(5)
    lengths = [int(n) for n in rng.integers(1, 701, size=40)]
    B, tables, ks, vs, q = rows_case(95, lengths)
    outs, caches, (span, items, records) = fused_and_unfused(ctx, lengths, B, tables, ks, vs, q)
    assert span == int(split[1:]) and items >= len(lengths)
    assert torch.equal(caches[0][0].view(torch.int16), caches[1][0].view(torch.int16))
    assert torch.equal(caches[0][1].view(torch.int16), caches[1][1].view(torch.int16))
    assert torch.equal(outs[0], outs[1])
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(outs[0]), expected, what=f"40 rows, plan {split}")


@pytest.mark.parametrize("split", ["1", "2", "7", "b1", "b7", "b40", "b1000"])
def test_tiny_chunks_and_chunk_boundaries(ctx, split, monkeypatch):
    """Chunks of 1, 2 and 7 pages over rows ending on, just past and inside
    page and chunk boundaries, at every GQA group size of the fast kernel;
    rows shorter than a chunk are not cut. Also the balanced plan with 1, 7,
    40 and 1000 pages to a workgroup: workgroups that take several whole rows
    and row pieces one after another (all rows in one workgroup at 1000)."""
    force_plan(monkeypatch, split)
    lengths = [1, 16, 17, 32, 33, 112, 113, 127, 500, 1999]
    for group in (1, 2, 4, 8):
        H = 16 // group if group < 8 else 2
        q_heads = H * group
        rng = orc.Mt64(70 + group + int(split.lstrip("b")))
        B = sum(-(-n // 16) for n in lengths) + 3
        perm = rng.permutation(B)
        tables, at = [], 0
        for n in lengths:
            tables.append(perm[at:at + -(-n // 16)])
            at += len(tables[-1])
        F = H * 128
        ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
        vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
        q = rng.normal(len(lengths) * q_heads * 128, orc.BF16).reshape(len(lengths), -1)
        pool, _, _ = new_pool(ctx, (1, B, 16, H, 128), orc.BF16)
        fill_by_append(pool, lengths, tables, ks, vs)
        flat = np.concatenate(tables)
        offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
        pool.upload(flat, offsets, [len(t) for t in tables], [n - 1 for n in lengths])
        span, items, records = pool.decode_plan()
        pages = [-(-n // 16) for n in lengths]
        if split.startswith("b"):  # balanced: whole rows and row pieces per workgroup
            assert span == int(split[1:]) and items >= len(lengths)
        else:
            assert span == int(split)
            assert records == sum(-(-p // span) for p in pages if p > span)
        out = torch.empty(len(lengths), q_heads * 128, dtype=torch.bfloat16, device="cuda")
        pool.decode(0, to_dev(q, orc.BF16), q_heads, SCALE, out)
        expected = compact_oracle((H, 128), lengths, tables, ks, vs, q, q_heads)
        assert_close(to_f32(out), expected, what=f"group {group}, chunks of {split} pages")
        pool.close()
    ctx.sync()


def test_records_reused_between_launches(ctx, monkeypatch):
    """Consecutive launches over one batch and over a second, smaller batch
    reuse the partial records: every launch's output equals the oracle, so no
    launch reads a record an earlier launch left behind."""
    monkeypatch.setenv("CKV_DECODE_SPLIT", "5")
    lengths = [3000, 700, 64, 2500]
    B, tables, ks, vs, q = rows_case(90, lengths)
    pool, _, _ = new_pool(ctx, (3, B, 16, 8, 128), orc.BF16)
    for layer in range(3):
        fill_by_append(pool, lengths, tables, ks, vs, layer=layer)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    pool.upload(flat, offsets, [len(t) for t in tables], [n - 1 for n in lengths])
    qd = to_dev(q, orc.BF16)
    for layer in (0, 1, 2, 1, 0):
        out = torch.empty(len(lengths), 2048, dtype=torch.bfloat16, device="cuda")
        pool.decode(layer, qd, 16, SCALE, out)
        assert_close(to_f32(out), expected, what=f"layer {layer}")
    # a smaller batch (the first two rows, shorter positions) on the same pool
    short = [1500, 700]
    pool.upload(flat, offsets[:2], [len(t) for t in tables[:2]], [n - 1 for n in short])
    out = torch.empty(2, 2048, dtype=torch.bfloat16, device="cuda")
    pool.decode(2, qd[:2], 16, SCALE, out)
    expected2 = compact_oracle((8, 128), short, tables[:2], [k[:1500] for k in ks[:1]] + [ks[1]],
                               [v[:1500] for v in vs[:1]] + [vs[1]], q[:2], 16)
    assert_close(to_f32(out), expected2, what="smaller batch")
    ctx.sync()
    pool.close()


def test_back_to_back_launches_are_bit_identical(ctx):
    """200 launches over one cut batch (32 rows of U[256, 4096] tokens, the
    default plan), queued with no synchronisation between them: the merge of a
    row happens in whichever of its chunks arrives last, and the records and
    arrival counters are reused launch after launch, yet the fold order is
    fixed, so every output equals the first bit for bit, and the first equals
    the oracle."""
    rng = np.random.default_rng(11)
    lengths = [int(n) for n in rng.integers(256, 4097, size=32)]
    B, tables, ks, vs, q = rows_case(91, lengths)
    pool, _, _ = new_pool(ctx, (1, B, 16, 8, 128), orc.BF16)
    fill_by_append(pool, lengths, tables, ks, vs)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    pool.upload(flat, offsets, [len(t) for t in tables], [n - 1 for n in lengths])
    span, items, records = pool.decode_plan()
    assert span > 0 and records > 0
    qd = to_dev(q, orc.BF16)
    outs = [torch.empty(len(lengths), 2048, dtype=torch.bfloat16, device="cuda")
            for _ in range(200)]
    for out in outs:
        pool.decode(0, qd, 16, SCALE, out)
    ctx.sync()
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(outs[0]), expected, what="first launch")
    first = outs[0].view(torch.int16)
    for i, out in enumerate(outs[1:], 1):
        assert torch.equal(out.view(torch.int16), first), f"launch {i} differs from the first"
    pool.close()


def test_config3_shape_layer_plan_not_cut(ctx):
    """Batch 128 with rows of 1K-8K tokens fills every compute unit with whole
    rows: the default plan does not cut them (one workgroup per row and kv head)."""
    rng = orc.Mt64(0)
    lengths = [rng.uniform_int(1024, 8192) for _ in range(128)]
    pages = [-(-n // 16) for n in lengths]
    B = sum(pages) + 1
    pool = ckv.Pool(ctx, 1, B, 16, 8, 128, ckv.BF16)
    flat = np.arange(sum(pages), dtype=np.uint32)
    offsets = np.cumsum([0] + pages[:-1])
    pool.upload(flat, offsets, pages, [n - 1 for n in lengths])
    assert pool.decode_plan() == (0, 128, 0)
    pool.close()


def test_patch_of_a_rows_own_page_unfuses_the_append(ctx):
    """A table patch that moves the page holding a row's position (a
    copy-on-write after the upload) leaves the uploaded slot in place: the
    token goes to the uploaded slot and the attention reads the patched page,
    as store_kv then paged_attention would, whether or not the fused kernel
    could apply. Compared with the unfused pair and with the oracle."""
    lengths = [40, 77, 300]
    B, tables, ks, vs, q = rows_case(17, lengths)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    # row 1's own page moves to a fresh page holding a copy of its first tokens
    own = int(offsets[1]) + positions[1] // 16
    fresh = min(set(range(B)) - set(int(x) for x in flat))  # a page no table holds
    results = []
    for fused in (True, False):
        pool, keys, values = new_pool(ctx, (1, B, 16, 8, 128), orc.BF16)
        fill_by_append(pool, [n - 1 for n in lengths], tables, [k[:-1] for k in ks],
                       [v[:-1] for v in vs])
        pool.copy_blocks([int(flat[own])], [fresh])
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        pool.patch([own], [fresh])
        k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
        v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
        out = torch.empty(3, 2048, dtype=torch.bfloat16, device="cuda")
        if fused:
            pool.append_decode(0, k_new, v_new, to_dev(q, orc.BF16), 16, SCALE, out)
        else:
            pool.append(0, k_new, v_new)
            pool.decode(0, to_dev(q, orc.BF16), 16, SCALE, out)
        ctx.sync()
        results.append((out, to_host(keys, orc.BF16), to_host(values, orc.BF16)))
        pool.close()
    assert torch.equal(results[0][0], results[1][0])
    assert np.array_equal(results[0][1], results[1][1])
    assert np.array_equal(results[0][2], results[1][2])
    # the oracle: every row's table after the patch; row 1's last token was
    # stored in the old page, so the patched page holds no token at position 76
    patched = flat.copy()
    patched[own] = fresh
    kc, vc = results[0][1], results[0][2]
    expected = orc.Attention((1, B, 16, 8, 128), kc, vc, orc.BF16, q, orc.BF16, positions,
                             patched, offsets, [len(t) for t in tables], 16, 0,
                             SCALE).online_threads(8)
    assert_close(to_f32(results[0][0]), expected, what="patched own page")
    # and the appended token is at the uploaded slot
    F = 1024
    assert np.array_equal(kc[slots[1] * F:(slots[1] + 1) * F], ks[1][-1])


def test_rope_width_beyond_the_frequency_table_is_rejected(ctx):
    """A pool with 2048-wide heads: a rotary width above 1024 is refused on
    the host (invalid_head_dimension) before any launch."""
    pool = ckv.Pool(ctx, 1, 2, 16, 1, 2048, ckv.BF16)
    pool.upload([0, 1], [0], [2], [3], slots=[3])
    x = torch.zeros(1, 2048, dtype=torch.bfloat16, device="cuda")
    for call in (lambda: pool.rope(x, x, 1, 1e4),
                 lambda: pool.rope_append(0, x, x, 1e4),
                 lambda: pool.rope_append_decode(0, x, x, x, 1, 0.1, 1e4, x.clone()),
                 lambda: pool.rope(x, x, 1, 1e4, rotary_dim=1026)):
        with pytest.raises(ckv.CkvError) as e:
            call()
        assert e.value.name == "tensor_op.invalid_head_dimension"
    pool.rope(x, x, 1, 1e4, rotary_dim=1024)  # the largest width accepted
    ctx.sync()
    pool.close()
