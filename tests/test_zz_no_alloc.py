"""ckv_append_decode_noalloc (the decode step for callers that cannot allocate:
its partial records go to the library's fixed per-GPU scratch array) against
ckv_append_decode through the C ABI: the same pages and outputs bit for bit,
on two calls in a row, the second with a smaller batch, and the oracle within
2e-2 abs + 1e-2 rel. Also what it refuses instead of allocating."""
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import assert_close, new_context, new_pool, to_dev, to_f32
from tests.test_gpu_parity import compact_oracle, fill_by_append

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1 / math.sqrt(128)))


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def batch(seed, lengths, B):
    rng = orc.Mt64(seed)
    perm = rng.permutation(B)
    tables, at = [], 0
    for n in lengths:
        tables.append(perm[at:at + -(-n // 16)])
        at += len(tables[-1])
    F = 8 * 128
    ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    q = rng.normal(len(lengths) * 2048, orc.BF16).reshape(len(lengths), -1)
    return tables, ks, vs, q


def test_noalloc_equals_append_decode_on_two_calls(ctx):
    """Call 1: six rows of 1 to 20,000 tokens (the plan cuts the long ones into
    chunks, so the scratch records are used); call 2: three shorter rows on
    another layer. Each call's pages and output equal ckv_append_decode's bit
    for bit; the outputs are within tolerance of the oracle."""
    calls = [([20000, 9000, 300, 17, 1, 4100], 0, 101), ([6000, 2500, 33], 1, 202)]
    B = sum(-(-n // 16) for n in calls[0][0]) + sum(-(-n // 16) for n in calls[1][0]) + 8
    pools = [new_pool(ctx, (2, B, 16, 8, 128), orc.BF16, fill=float("nan")) for _ in range(2)]
    for lengths, layer, seed in calls:
        print(f"noalloc call: rows {lengths}, layer {layer}", flush=True)
        tables, ks, vs, q = batch(seed, lengths, B)
        flat = np.concatenate(tables)
        offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
        positions = [n - 1 for n in lengths]
        slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
        outs = []
        for which, (pool, _, _) in enumerate(pools):
            fill_by_append(pool, [n - 1 for n in lengths], tables, [k[:-1] for k in ks],
                           [v[:-1] for v in vs], layer=layer)
            pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
            span, _, records = pool.decode_plan()
            assert span > 0 and records > 0, "the batch must use the scratch records"
            k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
            v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
            out = torch.full((len(lengths), 2048), float("nan"), dtype=torch.bfloat16,
                             device="cuda")
            args = (layer, k_new, v_new, to_dev(q, orc.BF16), 16, SCALE, out)
            if which == 0:
                pool.append_decode(*args)
            else:
                pool.append_decode_noalloc(*args)
            ctx.sync()
            outs.append(out)
        assert torch.equal(outs[0], outs[1]), "noalloc output differs from ckv_append_decode"
        for a, b in zip(pools[0][1:], pools[1][1:]):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "pages differ"
        expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
        assert_close(to_f32(outs[1]), expected, what=f"noalloc rows {lengths}")
    for pool, _, _ in pools:
        pool.close()


def test_noalloc_back_to_back_calls_are_bit_identical(ctx):
    """100 queued ckv_append_decode_noalloc calls over one cut batch (the same
    new token appended to the same slot each time, which leaves the pages as
    they were): the merge of every cut row reuses the array's records and
    arrival counters call after call, and every output equals the first bit
    for bit."""
    lengths = [12000, 5000, 700, 64]
    B = sum(-(-n // 16) for n in lengths) + 4
    tables, ks, vs, q = batch(303, lengths, B)
    pool, _, _ = new_pool(ctx, (1, B, 16, 8, 128), orc.BF16)
    fill_by_append(pool, [n - 1 for n in lengths], tables, [k[:-1] for k in ks],
                   [v[:-1] for v in vs])
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    pool.upload(flat, offsets, [len(t) for t in tables], positions,
                [orc.slot(t, p, 16) for t, p in zip(tables, positions)])
    span, _, records = pool.decode_plan()
    assert span > 0 and records > 0
    k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
    v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
    qd = to_dev(q, orc.BF16)
    outs = [torch.empty(len(lengths), 2048, dtype=torch.bfloat16, device="cuda")
            for _ in range(100)]
    for out in outs:
        pool.append_decode_noalloc(0, k_new, v_new, qd, 16, SCALE, out)
    ctx.sync()
    first = outs[0].view(torch.int16)
    for i, out in enumerate(outs[1:], 1):
        assert torch.equal(out.view(torch.int16), first), f"call {i} differs from the first"
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(outs[0]), expected, what="first noalloc call")
    pool.close()


def test_noalloc_makes_no_allocation(ctx):
    """The library's own count of device and pinned allocations and frees
    (ckv_debug_allocations) does not move across ckv_append_decode_noalloc
    calls, the first of them on a pool on which no allocating decode ever ran
    (so its partial-record and arrival-counter buffers do not exist), while
    one ckv_append_decode on the same batch allocates them."""
    lengths = [15000, 6000, 90]
    B = sum(-(-n // 16) for n in lengths) + 4
    tables, ks, vs, q = batch(404, lengths, B)
    pool, _, _ = new_pool(ctx, (1, B, 16, 8, 128), orc.BF16)
    fill_by_append(pool, [n - 1 for n in lengths], tables, [k[:-1] for k in ks],
                   [v[:-1] for v in vs])
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    pool.upload(flat, offsets, [len(t) for t in tables], positions,
                [orc.slot(t, p, 16) for t, p in zip(tables, positions)])
    span, _, records = pool.decode_plan()
    assert span > 0 and records > 0, "the batch must use the scratch records"
    k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
    v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
    qd = to_dev(q, orc.BF16)
    out = torch.empty(len(lengths), 2048, dtype=torch.bfloat16, device="cuda")
    ctx.sync()
    before = ctx.allocations()
    for _ in range(3):
        pool.append_decode_noalloc(0, k_new, v_new, qd, 16, SCALE, out)
    ctx.sync()
    assert ctx.allocations() == before, "ckv_append_decode_noalloc allocated"
    first = out.clone()
    pool.append_decode(0, k_new, v_new, qd, 16, SCALE, out)
    ctx.sync()
    assert ctx.allocations() > before, "the allocating decode made its scratch buffers"
    assert torch.equal(out, first)
    pool.close()


def test_noalloc_refuses_a_tiled_batch_whatever_ran_before(ctx):
    """A batch with a multi-row query tile is refused even after
    ckv_decode_plan derived its decode plan (the refusal depends on the
    batch, not on the calls made on it)."""
    q = torch.zeros(4, 2048, dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros(4, 1024, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    pool, _, _ = new_pool(ctx, (1, 64, 16, 8, 128), orc.BF16)
    pool.upload([0, 1], [0] * 4, [2] * 4, [3, 4, 5, 6], slots=[3, 4, 5, 6])
    pool.decode_plan()
    with pytest.raises(ckv.CkvError) as e:
        pool.append_decode_noalloc(0, kv, kv, q, 16, SCALE, out)
    assert e.value.name == "ckv.invalid_argument" and "query tiles" in str(e.value)
    pool.decode(0, q, 16, SCALE, out)  # an allocating decode launch on it
    with pytest.raises(ckv.CkvError) as e:
        pool.append_decode_noalloc(0, kv, kv, q, 16, SCALE, out)
    assert e.value.name == "ckv.invalid_argument" and "query tiles" in str(e.value)
    ctx.sync()
    pool.close()


def test_noalloc_refuses_instead_of_allocating(ctx, monkeypatch):
    """A batch of multi-row query tiles (no decode plan uploaded), a pool of
    64-feature heads (the generic kernel's geometry) and a plan whose records
    exceed the 16 MiB array are refused with invalid_argument; nothing is
    launched."""
    q = torch.zeros(4, 2048, dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros(4, 1024, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    pool, _, _ = new_pool(ctx, (1, 2100, 16, 8, 128), orc.BF16)
    # four rows of one sequence at consecutive positions: a prefill tile
    pool.upload([0, 1], [0] * 4, [2] * 4, [3, 4, 5, 6], slots=[3, 4, 5, 6])
    with pytest.raises(ckv.CkvError) as e:
        pool.append_decode_noalloc(0, kv, kv, q, 16, SCALE, out)
    assert e.value.name == "ckv.invalid_argument" and "query tiles" in str(e.value)
    # four rows of 8,000 tokens cut into 1-page chunks: 2,000 records x 16 q
    # heads x 528 bytes > 16 MiB
    monkeypatch.setenv("CKV_DECODE_SPLIT", "1")
    flat = np.arange(2000, dtype=np.uint32)
    pool.upload(flat, [0, 500, 1000, 1500], [500] * 4, [7999] * 4,
                slots=[(500 * r + 499) * 16 + 15 for r in range(4)])
    assert pool.decode_plan()[2] == 2000
    with pytest.raises(ckv.CkvError) as e:
        pool.append_decode_noalloc(0, kv, kv, q, 16, SCALE, out)
    assert e.value.name == "ckv.invalid_argument" and "16 MiB" in str(e.value)
    monkeypatch.delenv("CKV_DECODE_SPLIT")
    pool.close()
    narrow, _, _ = new_pool(ctx, (1, 4, 16, 8, 64), orc.BF16)
    narrow.upload([0, 1, 2, 3], [0, 1, 2, 3], [1] * 4, [0] * 4, slots=[0, 16, 32, 48])
    qn = torch.zeros(4, 16 * 64, dtype=torch.bfloat16, device="cuda")
    kn = torch.zeros(4, 8 * 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ckv.CkvError) as e:
        narrow.append_decode_noalloc(0, kn, kn, qn, 16, SCALE, torch.empty_like(qn))
    assert e.value.name == "ckv.invalid_argument" and "head_dim 128" in str(e.value)
    ctx.sync()
    narrow.close()
