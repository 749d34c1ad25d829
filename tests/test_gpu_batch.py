"""Device-resident sequence tables and device-expanded batches
(ckv_seq_tables_reserve / ckv_seq_tables_update / ckv_batch_upload): the
prepare_paged_batch loop of src/model_batch.cc:127-204 run on the device.

Parity is two-sided. Against ckv_tables_upload given the same tables as a
flat array (offsets seq * pages_per_sequence, lengths the tables' lengths,
the slots of prepare_paged_batch computed on the host): appended pages,
prefill and decode outputs bit-exact. Against the oracle with the
reference's own metadata layout (every item's block table concatenated):
appends bit-exact, attention within 2e-2 abs + 1e-2 rel."""
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import (assert_close, force_plan, new_context, new_pool, to_dev, to_f32,
                            to_host)

pytestmark = pytest.mark.gpu

BS, H, D, HQ = 16, 8, 128, 16
F = H * D
SCALE = float(np.float32(1 / math.sqrt(D)))


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def random_pools(ctx, geom, count, seed):
    """`count` pools over identical random caches (bf16)."""
    torch.manual_seed(seed)
    n = int(np.prod(geom))
    k = torch.randn(n, device="cuda").to(torch.bfloat16)
    v = torch.randn(n, device="cuda").to(torch.bfloat16)
    out = []
    for _ in range(count):
        kk, vv = k.clone(), v.clone()
        out.append((ckv.Pool(ctx, *geom, ckv.BF16, kk, vv), kk, vv))
    return out


class Tables:
    """Host mirror of the sequence tables: what a caller tracks to send deltas."""

    def __init__(self, pool, max_seqs, cap):
        self.pool, self.cap = pool, cap
        self.tables = [[] for _ in range(max_seqs)]
        pool.reserve_sequences(max_seqs, cap)

    def set(self, seq, table):
        old = self.tables[seq]
        idx = [i for i, b in enumerate(table) if i >= len(old) or old[i] != b]
        self.pool.update_sequences([seq] * len(idx), idx, [table[i] for i in idx],
                                   [seq], [len(table)])
        self.tables[seq] = list(table)

    def flat(self):
        """The arena as one flat table (unset entries are page 0)."""
        arena = np.zeros(len(self.tables) * self.cap, np.uint32)
        for s, t in enumerate(self.tables):
            arena[s * self.cap:s * self.cap + len(t)] = t
        return arena


def host_rows(items, tables, cap):
    """Per-row metadata of a batch: the arena layout ckv_batch_upload expands
    to, and the reference's layout (each item's table concatenated)."""
    offsets, lengths, positions, slots = [], [], [], []
    ref_table, ref_offsets = [], []
    for seq, first, count in items:
        t = tables[seq]
        ref_at = len(ref_table)
        ref_table += t
        for p in range(first, first + count):
            offsets.append(seq * cap)
            lengths.append(len(t))
            positions.append(p)
            slots.append(orc.slot(t, p, BS))
            ref_offsets.append(ref_at)
    return (offsets, lengths, positions, slots), (np.array(ref_table, np.uint32), ref_offsets)


def upload_items(pool, items, with_slots=True):
    s, f, c = zip(*items)
    pool.upload_batch(s, f, c, with_slots)


def test_batch_upload_equals_host_upload_prefill_decode_append(ctx):
    """Mixed batch: decode rows, a fresh prompt chunk, a chunk continuing a
    cached prefix, and one sequence split over two consecutive items."""
    geom = (2, 256, BS, H, D)
    (pa, ka, va), (pb, kb, vb) = random_pools(ctx, geom, 2, seed=1)
    rng = orc.Mt64(21)
    perm = [int(x) for x in rng.permutation(256)]
    cap = 24
    # sequence -> tokens after this batch; pages taken from a permutation
    totals = {0: 48, 1: 34, 2: 101, 3: 41, 4: 256, 5: 13}
    tables = {}
    at = 0
    for s, n in totals.items():
        pages = -(-n // BS)
        tables[s] = perm[at:at + pages]
        at += pages
    items = [(1, 33, 1), (0, 0, 48), (2, 100, 1), (3, 16, 25), (4, 255, 1), (5, 7, 3), (5, 10, 3)]

    mirror = Tables(pb, 8, cap)
    for s, t in tables.items():
        mirror.set(s, t)
    (offsets, lengths, positions, slots), (ref_table, ref_offsets) = host_rows(items, tables, cap)
    rows = len(positions)
    pa.upload(mirror.flat(), offsets, lengths, positions, slots)
    upload_items(pb, items)

    kr = orc.Mt64(5).normal(rows * F, orc.BF16).reshape(rows, F)
    vr = orc.Mt64(6).normal(rows * F, orc.BF16).reshape(rows, F)
    q = orc.Mt64(7).normal(rows * HQ * D, orc.BF16).reshape(rows, HQ * D)
    outs = []
    for pool in (pa, pb):
        pool.append(1, to_dev(kr, orc.BF16), to_dev(vr, orc.BF16))
        pre = torch.empty(rows, HQ * D, dtype=torch.bfloat16, device="cuda")
        dec = torch.empty_like(pre)
        pool.prefill(1, to_dev(q, orc.BF16), HQ, SCALE, pre)
        pool.decode(1, to_dev(q, orc.BF16), HQ, SCALE, dec)
        outs.append((pre, dec))
    ctx.sync()
    assert torch.equal(ka, kb) and torch.equal(va, vb), "device slots differ from host slots"
    assert torch.equal(outs[0][0], outs[1][0]), "prefill differs"
    assert torch.equal(outs[0][1], outs[1][1]), "decode differs"

    # the oracle over the reference's metadata layout
    kc, vc = to_host(kb, orc.BF16), to_host(vb, orc.BF16)
    expected = orc.Attention(geom, kc, vc, orc.BF16, q, orc.BF16, positions, ref_table,
                             ref_offsets, lengths, HQ, 1, SCALE).online()
    assert_close(to_f32(outs[1][0]), expected, what="prefill vs oracle")
    assert_close(to_f32(outs[1][1]), expected, what="decode vs oracle")
    pa.close()
    pb.close()


@pytest.mark.parametrize("plan", [None, "2", "b2", "b9"])
def test_decode_steps_with_growing_tables_and_fused_append(ctx, plan, monkeypatch):
    """A decode loop: each step appends one token per sequence (the fused
    append + decode launch), sequences cross page boundaries and take new
    pages, one finishes and its row is reused; only table deltas are sent.
    Also with the rows cut into 2-page chunks and with the balanced plan of 2
    and 9 pages to a workgroup (several rows and row pieces per workgroup)
    over the device-expanded batch."""
    force_plan(monkeypatch, plan)
    geom = (1, 128, BS, H, D)
    (pa, ka, va), (pb, kb, vb) = random_pools(ctx, geom, 2, seed=2)
    cap = 8
    mirror = Tables(pb, 4, cap)
    free = list(range(127, -1, -1))
    lengths = {0: 14, 1: 31, 2: 1, 3: 60}
    tables = {s: [free.pop() for _ in range(-(-n // BS))] for s, n in lengths.items()}
    for step in range(6):
        if step == 3:  # sequence 2 finishes; a new one takes its row
            free += tables[2]
            lengths[2], tables[2] = 5, [free.pop()]
        # this step appends the token at position lengths[s]
        for s in lengths:
            if lengths[s] // BS >= len(tables[s]):
                tables[s].append(free.pop())
            mirror.set(s, tables[s])
        items = [(s, lengths[s], 1) for s in (3, 0, 2, 1)]
        (offsets, lens, positions, slots), _ = host_rows(items, tables, cap)
        pa.upload(mirror.flat(), offsets, lens, positions, slots)
        upload_items(pb, items)
        kn = orc.Mt64(100 + step).normal(4 * F, orc.BF16).reshape(4, F)
        vn = orc.Mt64(200 + step).normal(4 * F, orc.BF16).reshape(4, F)
        q = orc.Mt64(300 + step).normal(4 * HQ * D, orc.BF16).reshape(4, HQ * D)
        outs = []
        for pool in (pa, pb):
            out = torch.empty(4, HQ * D, dtype=torch.bfloat16, device="cuda")
            pool.append_decode(0, to_dev(kn, orc.BF16), to_dev(vn, orc.BF16),
                               to_dev(q, orc.BF16), HQ, SCALE, out)
            outs.append(out)
        ctx.sync()
        assert torch.equal(ka, kb) and torch.equal(va, vb), f"step {step}: pages differ"
        assert torch.equal(outs[0], outs[1]), f"step {step}: attention differs"
        for s in lengths:
            lengths[s] += 1
    # the last step against the oracle
    (_, lens, positions, _), (ref_table, ref_offsets) = host_rows(
        [(s, lengths[s] - 1, 1) for s in (3, 0, 2, 1)], tables, cap)
    expected = orc.Attention(geom, to_host(kb, orc.BF16), to_host(vb, orc.BF16), orc.BF16, q,
                             orc.BF16, positions, ref_table, ref_offsets, lens, HQ, 0,
                             SCALE).online()
    assert_close(to_f32(outs[1]), expected, what="decode step vs oracle")
    pa.close()
    pb.close()


def test_copy_on_write_update_redirects_the_batch(ctx):
    """A copy-on-write replacement of one shared page (copy_blocks, then the
    sequence's table entry redirected) reaches the device as a single entry."""
    geom = (1, 16, BS, H, D)
    (pool, keys, values), = random_pools(ctx, geom, 1, seed=3)
    mirror = Tables(pool, 2, 4)
    mirror.set(0, [3, 9, 4])
    mirror.set(1, [3, 9, 11])  # shares two pages with sequence 0
    pool.copy_blocks([9], [12])
    mirror.set(1, [3, 12, 11])  # sequence 1's private copy of page 9
    upload_items(pool, [(0, 20, 1), (1, 20, 1)])
    k = orc.Mt64(8).normal(2 * F, orc.BF16).reshape(2, F)
    pool.append(0, to_dev(k, orc.BF16), to_dev(k, orc.BF16))
    ctx.sync()
    got = to_host(keys, orc.BF16).reshape(16, BS, F)
    assert np.array_equal(got[9, 4], k[0]) and np.array_equal(got[12, 4], k[1])
    pool.close()


def test_sequence_table_validation_codes(ctx):
    (pool, _, _), = random_pools(ctx, (1, 8, BS, H, D), 1, seed=4)
    with pytest.raises(ckv.CkvError) as e:
        pool.upload_batch([0], [0], [1])
    assert e.value.code == 403  # before reserve
    with pytest.raises(ckv.CkvError) as e:
        pool.update_sequences([0], [0], [1])
    assert e.value.code == 403
    with pytest.raises(ckv.CkvError) as e:
        pool.reserve_sequences(0, 4)
    assert e.value.code == 400
    pool.reserve_sequences(2, 4)
    cases = [
        (dict(seq=[2], index=[0], block=[1]), "tensor_op.block_table_range_out_of_bounds"),
        (dict(seq=[0], index=[4], block=[1]), "tensor_op.block_table_range_out_of_bounds"),
        (dict(seq=[0], index=[0], block=[8]), "tensor_op.cache_block_out_of_range"),
        (dict(len_seq=[1], length=[5]), "tensor_op.block_table_range_out_of_bounds"),
        (dict(len_seq=[2], length=[1]), "tensor_op.block_table_range_out_of_bounds"),
    ]
    for kwargs, name in cases:
        with pytest.raises(ckv.CkvError) as e:
            pool.update_sequences(**kwargs)
        assert e.value.name == name, kwargs
    pool.update_sequences([0, 0], [0, 1], [5, 6], [0], [2])
    for items, code in [([(0, 32, 1)], 123),  # position 32 needs a third page
                        ([(1, 0, 1)], 123),   # sequence 1 has no pages
                        ([(2, 0, 1)], 123),   # beyond max_sequences
                        ([(0, 0, 0)], 400)]:  # an item with no tokens
        with pytest.raises(ckv.CkvError) as e:
            upload_items(pool, items)
        assert e.value.code == code, items
    upload_items(pool, [(0, 0, 32)])
    with pytest.raises(ckv.CkvError) as e:  # the batch indexes the arena
        pool.patch([0], [1])
    assert e.value.code == 400
    pool.upload([5, 6], [0], [2], [3])
    pool.patch([0], [1])  # a host-uploaded batch is patchable again
    ctx.sync()
    pool.close()


def test_batch_edge_cases_long_items_empty_batch_gather_and_rope(ctx):
    """A 600-row prompt chunk (three query tiles), an empty batch, gather and
    RoPE through the sequence tables, all against the host-uploaded equivalent."""
    geom = (1, 96, BS, H, D)
    (pa, ka, va), (pb, kb, vb) = random_pools(ctx, geom, 2, seed=9)
    cap = 48
    mirror = Tables(pb, 3, cap)
    tables = {0: list(range(3, 3 + 40)), 1: list(range(50, 52)), 2: [90]}
    for s, t in tables.items():
        mirror.set(s, t)
    items = [(0, 10, 600), (1, 20, 1), (2, 3, 2)]
    (offsets, lengths, positions, slots), (ref_table, ref_offsets) = host_rows(items, tables, cap)
    rows = len(positions)
    pa.upload(mirror.flat(), offsets, lengths, positions, slots)
    upload_items(pb, items)
    q = orc.Mt64(4).normal(rows * HQ * D, orc.BF16).reshape(rows, HQ * D)
    outs = []
    for pool in (pa, pb):
        out = torch.empty(rows, HQ * D, dtype=torch.bfloat16, device="cuda")
        pool.attention(0, to_dev(q, orc.BF16), HQ, SCALE, out)  # shared tiles: prefill
        rq = to_dev(q, orc.BF16)
        pool.rope(rq, rq, HQ, 1e6)
        outs.append((out, rq))
    ctx.sync()
    assert torch.equal(outs[0][0], outs[1][0]), "prefill over three tiles differs"
    assert torch.equal(outs[0][1], outs[1][1]), "rope positions differ"
    expected = orc.Attention(geom, to_host(kb, orc.BF16), to_host(vb, orc.BF16), orc.BF16, q,
                             orc.BF16, positions, ref_table, ref_offsets, lengths, HQ, 0,
                             SCALE).online_threads(8)
    assert_close(to_f32(outs[1][0]), expected, what="600-row chunk vs oracle")
    # gather of sequence 0's first 610 tokens through the arena row
    n_tok = 610
    ga = [torch.empty(n_tok * F, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    gb = [torch.empty(n_tok * F, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    pa.gather(0, 0, 40, n_tok, ga[0], ga[1])
    pb.gather(0, 0, 40, n_tok, gb[0], gb[1])
    ctx.sync()
    assert torch.equal(ga[0], gb[0]) and torch.equal(ga[1], gb[1])
    # an empty batch uploads and attends nothing
    pb.upload_batch([], [], [], True)
    assert pb.decode(0, torch.empty(0, HQ * D, dtype=torch.bfloat16, device="cuda"), HQ, SCALE,
                     torch.empty(0, HQ * D, dtype=torch.bfloat16, device="cuda")) is None
    pa.close()
    pb.close()
