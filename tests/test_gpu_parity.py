"""Parity of the HIP path (through the C ABI) with the CPU oracle on the same
inputs: append / gather / page copies / checkpoints bit-exact, attention within
2e-2 abs + 1e-2 rel (the reference's own known-answer tests at their stated
tolerances). Runs on the MI355X only."""
import functools
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.golden import config1
from tests.gpu_util import (approx, assert_close, force_plan, new_context, new_pool, to_dev,
                            to_f32, to_host)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


# ---- append ------------------------------------------------------------------------

@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
def test_store_kv_writes_rows_into_selected_slots(ctx, code):
    # tests/tensor_ops_test.cc:610-633 (cache L2 B2 bs2 H1 D2, slots {1, 3}, layer 1)
    pool, keys, values = new_pool(ctx, (2, 2, 2, 1, 2), code, fill=-1.0)
    pool.upload([0, 1], [0, 0], [2, 2], [0, 0], slots=[1, 3])
    k = to_dev(orc.from_f32(np.array([[1, 2], [3, 4]]), code), code)
    v = to_dev(orc.from_f32(np.array([[5, 6], [7, 8]]), code), code)
    pool.append(1, k, v)
    ctx.sync()
    assert to_f32(keys).tolist() == [-1] * 10 + [1, 2, -1, -1, 3, 4]
    assert to_f32(values).tolist() == [-1] * 10 + [5, 6, -1, -1, 7, 8]


def test_store_kv_validation_codes(ctx):
    # tests/tensor_ops_test.cc:635-691 (the checks that exist at this boundary)
    pool, _, _ = new_pool(ctx, (2, 2, 2, 1, 2), orc.F32)
    k = torch.zeros(2, 2, device="cuda")
    with pytest.raises(ckv.CkvError) as e:
        pool.append(0, k, k)
    assert e.value.code == 403  # nothing uploaded yet
    pool.upload([0, 1], [0, 0], [2, 2], [0, 0], slots=[0, 1])
    with pytest.raises(ckv.CkvError) as e:
        pool.append(0, k, k, rows=1)
    assert e.value.name == "tensor_op.cache_slot_count_mismatch"
    with pytest.raises(ckv.CkvError) as e:
        pool.append(2, k, k)
    assert e.value.name == "tensor_op.cache_layer_out_of_range"
    with pytest.raises(ckv.CkvError) as e:
        pool.upload([0, 1], [0, 0], [2, 2], [0, 0], slots=[0, 4])
    assert e.value.name == "tensor_op.cache_slot_out_of_range"


def test_attention_metadata_validation_codes(ctx):
    # tests/tensor_ops_test.cc:986-1099 (host checks of the table metadata)
    pool, _, _ = new_pool(ctx, (2, 2, 2, 1, 2), orc.F32)
    with pytest.raises(ckv.CkvError) as e:  # missing required block
        pool.upload([0], [0], [1], [2])
    assert e.value.name == "tensor_op.block_table_range_out_of_bounds"
    with pytest.raises(ckv.CkvError) as e:  # range outside the flattened table
        pool.upload([0, 1], [1], [2], [0])
    assert e.value.name == "tensor_op.block_table_range_out_of_bounds"
    with pytest.raises(ckv.CkvError) as e:  # physical block out of range
        pool.upload([2], [0], [1], [0])
    assert e.value.name == "tensor_op.cache_block_out_of_range"
    pool.upload([0], [0], [1], [0])
    q = torch.zeros(1, 2, device="cuda")
    out = torch.zeros(1, 2, device="cuda")
    with pytest.raises(ckv.CkvError) as e:
        pool.decode(0, q, 0, 1.0, out)
    assert e.value.name == "tensor_op.invalid_head_count"
    with pytest.raises(ckv.CkvError) as e:
        pool.decode(2, q, 1, 1.0, out)
    assert e.value.name == "tensor_op.cache_layer_out_of_range"
    with pytest.raises(ckv.CkvError) as e:
        pool.decode(0, q, 1, 1.0, out, rows=2)
    assert e.value.name == "tensor_op.position_count_mismatch"
    gqa, _, _ = new_pool(ctx, (1, 1, 1, 2, 2), orc.F32)
    gqa.upload([0], [0], [1], [0])
    with pytest.raises(ckv.CkvError) as e:
        gqa.decode(0, torch.zeros(1, 6, device="cuda"), 3, 1.0, torch.zeros(1, 6, device="cuda"))
    assert e.value.name == "tensor_op.invalid_kv_head_mapping"


def test_pool_geometry_codes_and_offsets(ctx):
    # tests/metal_kv_cache_test.cc:64-101
    for geom, name in [((0, 3, 4, 2, 8), "kv_cache.invalid_layer_count"),
                       ((2, 0, 4, 2, 8), "kv_cache.invalid_block_count"),
                       ((2, 3, 0, 2, 8), "kv_cache.invalid_block_size"),
                       ((2, 3, 4, 0, 8), "kv_cache.invalid_kv_head_count"),
                       ((2, 3, 4, 2, 0), "kv_cache.invalid_head_dimension"),
                       ((2**64 - 1, 3, 4, 2, 8), "kv_cache.layout_size_overflow")]:
        with pytest.raises(ckv.CkvError) as e:
            ckv.Pool(ctx, *geom, ckv.F32)
        assert e.value.name == name
    pool = ckv.Pool(ctx, 2, 3, 4, 2, 8, ckv.F32)
    k, v, n = pool.buffers()
    assert n == 384 * 4 and k and v and k != v
    offsets = [pool.element_offset(*c) for c in [(0, 0, 0, 0, 0), (0, 0, 0, 0, 1), (0, 0, 0, 1, 0),
                                                 (0, 0, 1, 0, 0), (0, 1, 0, 0, 0), (1, 0, 0, 0, 0),
                                                 (1, 2, 3, 1, 7)]]
    assert offsets == [0, 1, 8, 16, 64, 192, 383]
    for coords, name in [((2, 0, 0, 0, 0), "layer"), ((0, 3, 0, 0, 0), "block"),
                         ((0, 0, 4, 0, 0), "token_offset"), ((0, 0, 0, 2, 0), "kv_head"),
                         ((0, 0, 0, 0, 8), "head_feature")]:
        with pytest.raises(ckv.CkvError) as e:
            pool.element_offset(*coords)
        assert e.value.name == f"kv_cache.{name}_out_of_range"
    pool.close()


# ---- attention known answers ------------------------------------------------------------

def run_attention(ctx, geom, keys, values, q, positions, table, offsets, lengths, q_heads,
                  layer=0, code=orc.F32):
    pool, kd, vd = new_pool(ctx, geom, code)
    kd.copy_(to_dev(keys, code))
    vd.copy_(to_dev(values, code))
    pool.upload(table, offsets, lengths, positions)
    qd = to_dev(q, code)
    scale = float(np.float32(1.0 / math.sqrt(geom[4])))
    outs = {}
    for name in ("decode", "prefill", "attention"):
        out = torch.full_like(qd, float("nan"))
        getattr(pool, name)(layer, qd, q_heads, scale, out)
        outs[name] = to_f32(out)
    ctx.sync()
    pool.close()
    return outs


def test_decode_closed_form_through_page_table(ctx):
    # tests/tensor_ops_test.cc:693-735
    keys = np.array([1, 1, 0, 0, 1, 0, 0, 1] + [0] * 8, np.float32)
    values = np.array([30, 3, 0, 0, 10, 1, 20, 2] + [0] * 8, np.float32)
    outs = run_attention(ctx, (2, 2, 2, 1, 2), keys, values, np.array([[1, 0, 0, 1]], np.float32),
                         [2], [1, 0], [0], [2], 2)
    e = math.exp(1 / math.sqrt(2))
    d = 2 * e + 1
    expected = [(40 * e + 20) / d, (4 * e + 2) / d, (10 + 50 * e) / d, (1 + 5 * e) / d]
    for name, out in outs.items():
        assert approx(out[0], expected, 1e-5), name


def test_prefill_tiles_known_answer(ctx):
    # tests/tensor_ops_test.cc:737-822
    geom = (1, 2, 2, 1, 2)
    keys = np.array([0.25, 0.75, -0.5, 1.0, 1.0, 0.0, 0.5, -0.25], np.float32)
    values = np.array([30, 3, 40, 4, 10, 1, 20, 2], np.float32)
    q = np.array([1.0, 0.5, -0.5, 1.0, 0.25, 1.0, 1.0, -0.25, -0.5, 0.75, 0.5, 0.5, 1.0, -1.0,
                  -0.25, 0.75], np.float32).reshape(4, 4)
    args = ([0, 1, 2, 3], [1, 0], [0] * 4, [2] * 4)
    expected = orc.Attention(geom, keys, values, orc.F32, q, orc.F32, *args, 2, 0,
                             1 / math.sqrt(2)).reference()
    for name, out in run_attention(ctx, geom, keys, values, q, *args, 2).items():
        assert approx(out, expected, 1e-5), name


def test_prefill_merges_key_tiles_across_cached_prefix(ctx):
    # tests/tensor_ops_test.cc:824-870
    values = np.array([[t, 2 * t] for t in range(32)], np.float32).ravel()
    outs = run_attention(ctx, (1, 2, 16, 1, 2), np.zeros(64, np.float32), values,
                         np.ones((8, 2), np.float32), list(range(16, 24)), [0, 1], [0] * 8,
                         [2] * 8, 1)
    for name, out in outs.items():
        for r in range(8):
            assert approx(out[r], [(16 + r) / 2, 16 + r], 1e-5), name


def test_split_decode_combines_chunks(ctx):
    # tests/tensor_ops_test.cc:941-984: mean of (t, 2t) over 0..128 = (64, 128)
    values = np.array([[t, 2 * t] for t in range(144)], np.float32).ravel()
    outs = run_attention(ctx, (1, 9, 16, 1, 2), np.zeros(288, np.float32), values,
                         np.ones((1, 2), np.float32), [128], list(range(9)), [0], [9], 1)
    for name, out in outs.items():
        assert approx(out[0], [64, 128], 1e-5), name


@pytest.mark.parametrize("dim", [129, 192, 256, 257])
def test_wide_heads_ragged_batch(ctx, dim):
    # tests/tensor_ops_test.cc:872-939 (rel 3e-5 against a double reference)
    rows, heads, kv_heads = 5, 4, 2
    geom = (2, 6, 16, kv_heads, dim)
    n = 2 * 6 * 16 * kv_heads * dim
    i = np.arange(n, dtype=np.float32)
    keys = np.sin(i * np.float32(0.17)).astype(np.float32)
    values = np.cos(i * np.float32(0.11)).astype(np.float32)
    q = (20 * np.sin(np.arange(rows * heads * dim, dtype=np.float32) * np.float32(0.13))
         ).astype(np.float32).reshape(rows, -1)
    args = ([17, 18, 7, 32, 9], [4, 1, 5, 3, 0, 2], [0, 0, 3, 3, 0], [3] * rows)
    expected = orc.Attention(geom, keys, values, orc.F32, q, orc.F32, *args, heads, 1,
                             1 / math.sqrt(dim)).reference()
    for name, out in run_attention(ctx, geom, keys, values, q, *args, heads, layer=1).items():
        assert approx(out, expected, 3e-5, 1.0), name


# ---- token-by-token fp16 appends + one decode step ----------------------

def test_config1_fp16_appends_bit_exact_and_decode_within_tolerance(ctx):
    steps, q, tables = config1.generate()
    L, B, bs, H, D = config1.GEOMETRY
    pool, keys, values = new_pool(ctx, config1.GEOMETRY, orc.F16)
    for active, t, ks, vs, step_tables in steps:
        flat, offsets, lengths, positions, slots = config1.step_metadata(step_tables, active, t)
        pool.upload(flat, offsets, lengths, positions, slots)
        pool.append(0, to_dev(ks, orc.F16), to_dev(vs, orc.F16))
    kc, vc = config1.oracle_cache(steps)
    assert np.array_equal(to_host(keys, orc.F16), kc)
    assert np.array_equal(to_host(values, orc.F16), vc)

    flat, offsets, lengths, positions = config1.decode_metadata(tables)
    pool.upload(flat, offsets, lengths, positions)
    F = H * D
    for s, n in enumerate(config1.LENGTHS):  # gather = the rows drawn for the sequence
        gk = torch.empty(n, F, dtype=torch.float16, device="cuda")
        gv = torch.empty_like(gk)
        pool.gather(0, int(offsets[s]), lengths[s], n, gk, gv)
        drawn_k = np.stack([st[2][st[0].index(s)] for st in steps if s in st[0]])
        drawn_v = np.stack([st[3][st[0].index(s)] for st in steps if s in st[0]])
        assert np.array_equal(to_host(gk, orc.F16), drawn_k)
        assert np.array_equal(to_host(gv, orc.F16), drawn_v)

    online, reference = config1.oracle_attention(kc, vc, q, tables)
    qd = to_dev(q, orc.F16)
    for name in ("decode", "attention", "prefill"):
        out = torch.empty_like(qd)
        getattr(pool, name)(0, qd, config1.Q_HEADS, config1.SCALE, out)
        assert_close(to_f32(out), online, what=f"{name} vs oracle online")
        assert_close(to_f32(out), reference, what=f"{name} vs double reference")
    ctx.sync()


# ---- single-layer bf16 decode over a permuted 65,536-page pool -----------

@functools.lru_cache(maxsize=2)
def config2_inputs(seed=0, batch=32):
    rng = orc.Mt64(seed)
    lengths = [rng.uniform_int(256, 4096) for _ in range(batch)]
    perm = rng.permutation(65536)
    tables, at = [], 0
    for n in lengths:
        pages = -(-n // 16)
        tables.append(perm[at:at + pages])
        at += pages
    F = 8 * 128
    ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    q = rng.normal(batch * 16 * 128, orc.BF16).reshape(batch, 16 * 128)
    return lengths, tables, ks, vs, q


def compact_oracle(geom_h_d, lengths, tables, ks, vs, q, q_heads, positions=None,
                   code=orc.BF16, threads=8):
    """Oracle attention over a compact host pool holding only the pages in use
    (page ids renumbered in table order; the attention result depends only on
    the values reached through the tables)."""
    H, D = geom_h_d
    F = H * D
    n_pages = sum(len(t) for t in tables)
    kc = np.zeros(n_pages * 16 * F, np.float32 if code == orc.F32 else np.uint16)
    vc = np.zeros_like(kc)
    flat, offsets, at = [], [], 0
    for n, t, k, v in zip(lengths, tables, ks, vs):
        compact = np.arange(at, at + len(t), dtype=np.uint32)
        offsets.append(at)
        flat.append(compact)
        slots = [int(compact[p // 16]) * 16 + p % 16 for p in range(n)]
        orc.store_kv(kc, vc, k, v, slots, 0, n_pages * 16)
        at += len(t)
    flat = np.concatenate(flat)
    positions = [n - 1 for n in lengths] if positions is None else positions
    att = orc.Attention((1, n_pages, 16, H, D), kc, vc, code, q, code, positions, flat, offsets,
                        [len(t) for t in tables], q_heads, 0, float(np.float32(1 / math.sqrt(D))))
    return att.online_threads(threads)


def fill_by_append(pool, lengths, tables, ks, vs, layer=0, code=orc.BF16):
    """Writes every sequence's rows through ckv_append, one sequence per call."""
    for n, t, k, v in zip(lengths, tables, ks, vs):
        slots = [orc.slot(t, p, 16) for p in range(n)]
        pool.upload(t, [0] * n, [len(t)] * n, list(range(n)), slots)
        pool.append(layer, to_dev(k, code), to_dev(v, code))


@pytest.mark.parametrize("split", [None, "0", "4", "17", "64", "b9", "b300"])
def test_config2_bf16_decode_over_permuted_pages(ctx, split, monkeypatch):
    """Config 2 through the fast decode kernel: the batch plan's default
    (rows of up to 256 pages on 256 compute units: the batch's pages dealt out
    evenly to the workgroups, rows cut where a workgroup's share ends), no
    cut, forced chunks of 4, 17 and 64 pages, and 9 or 300 pages to a
    workgroup; each checked against the oracle and against the plan the
    library reports."""
    force_plan(monkeypatch, split)
    lengths, tables, ks, vs, q = config2_inputs()
    pool, _, _ = new_pool(ctx, (1, 65536, 16, 8, 128), orc.BF16)
    fill_by_append(pool, lengths, tables, ks, vs)
    # gather of every sequence returns its rows bit for bit
    for n, t, k, v in zip(lengths[:4], tables, ks, vs):
        pool.upload(t, [0], [len(t)], [n - 1])
        gk = torch.empty(n, 1024, dtype=torch.bfloat16, device="cuda")
        gv = torch.empty_like(gk)
        pool.gather(0, 0, len(t), n, gk, gv)
        assert np.array_equal(to_host(gk, orc.BF16), k)
        assert np.array_equal(to_host(gv, orc.BF16), v)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    pool.upload(flat, offsets, [len(t) for t in tables], [n - 1 for n in lengths])
    span, items, records = pool.decode_plan()
    pages = [-(-n // 16) for n in lengths]
    if split == "0":
        assert (span, items, records) == (0, 32, 0)
    elif split is None or split.startswith("b"):
        # balanced: a workgroup's share is `span` pages or fewer
        assert span == (int(split[1:]) if split else span) and span > 0
        assert items >= 32 and records > 0, "some row must be cut"
    else:
        assert span == int(split)
        assert items == sum(-(-p // span) for p in pages)
        assert records == sum(-(-p // span) for p in pages if p > span)
        assert records > 0, "some row must be cut into several chunks"
    out = torch.empty(32, 16 * 128, dtype=torch.bfloat16, device="cuda")
    pool.decode(0, to_dev(q, orc.BF16), 16, float(np.float32(1 / math.sqrt(128))), out)
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(out), expected, what=f"config 2 decode (split {split})")
    ctx.sync()
    pool.close()


def misaligned(rows, width):
    """A contiguous bf16 [rows, width] view 2 bytes past a 16-byte boundary:
    the fast decode kernel needs 16-byte aligned queries and outputs, so such
    views take the generic split-KV kernel."""
    base = torch.empty(rows * width + 8, dtype=torch.bfloat16, device="cuda")
    view = base[1:1 + rows * width].view(rows, width)
    assert view.data_ptr() % 16 == 2
    return view


@pytest.mark.parametrize("chunk", ["32", "4096"])
def test_config2_generic_split_kv_chunks(ctx, chunk, monkeypatch):
    """Config 2 through the generic kernel (misaligned queries and output):
    token chunks of 32 cut every row (256..4096 tokens) into 8..128 partials
    merged by the merge launch; chunks of 4096 leave every row whole."""
    monkeypatch.setenv("CKV_DECODE_CHUNK", chunk)
    lengths, tables, ks, vs, q = config2_inputs(seed=11, batch=12)
    pool, _, _ = new_pool(ctx, (1, 65536, 16, 8, 128), orc.BF16)
    fill_by_append(pool, lengths, tables, ks, vs)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    pool.upload(flat, offsets, [len(t) for t in tables], [n - 1 for n in lengths])
    qd = misaligned(len(lengths), 16 * 128)
    qd.copy_(to_dev(q, orc.BF16))
    out = misaligned(len(lengths), 16 * 128)
    ctx.profile(True)
    ctx.profile_reset()
    pool.decode(0, qd, 16, float(np.float32(1 / math.sqrt(128))), out)
    _, merges = ctx.profile_query("paged_attention_merge")
    ctx.profile(False)
    assert merges == (1 if chunk == "32" else 0), "chunks of 32 tokens need the merge launch"
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(out), expected, what=f"generic decode (chunk {chunk})")
    ctx.sync()
    pool.close()


@pytest.mark.parametrize("waves", ["1", "3", "12"])
def test_decode_wave_counts_and_long_rows(ctx, waves, monkeypatch):
    """The fused decode kernel at forced wave counts. A wave walks every W-th
    page of its row in runs of 64 (one table read per run): at one wave the
    5,000-token row takes five runs. Rows end on, just past and inside page
    boundaries. The fused step equals append-then-decode bit for bit and the
    oracle within tolerance."""
    monkeypatch.setenv("CKV_DECODE_WAVES", waves)
    rng = orc.Mt64(23)
    lengths = [5000, 1, 16, 17, 1025, 2049, 300]
    B = sum(-(-n // 16) for n in lengths) + 5
    perm = rng.permutation(B)
    tables, at = [], 0
    for n in lengths:
        tables.append(perm[at:at + -(-n // 16)])
        at += len(tables[-1])
    F = 8 * 128
    ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    q = rng.normal(len(lengths) * 16 * 128, orc.BF16).reshape(len(lengths), -1)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    scale = float(np.float32(1 / math.sqrt(128)))
    pools, outs = [], []
    for fused in (True, False):
        pool, keys, values = new_pool(ctx, (1, B, 16, 8, 128), orc.BF16, fill=float("nan"))
        fill_by_append(pool, [n - 1 for n in lengths], tables,
                       [k[:-1] for k in ks], [v[:-1] for v in vs])
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
        v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
        out = torch.empty(len(lengths), 16 * 128, dtype=torch.bfloat16, device="cuda")
        if fused:
            pool.append_decode(0, k_new, v_new, to_dev(q, orc.BF16), 16, scale, out)
        else:
            pool.append(0, k_new, v_new)
            pool.decode(0, to_dev(q, orc.BF16), 16, scale, out)
        pools.append((pool, keys, values))
        outs.append(out)
    ctx.sync()
    # slots never written hold NaN: nothing past a row's last token reaches the output
    assert torch.equal(pools[0][1].view(torch.int16), pools[1][1].view(torch.int16))
    assert torch.equal(pools[0][2].view(torch.int16), pools[1][2].view(torch.int16))
    assert torch.equal(outs[0], outs[1])
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(outs[0]), expected, what=f"{waves} waves")
    for pool, _, _ in pools:
        pool.close()


@pytest.mark.parametrize("group,waves", [(2, None), (2, "3"), (4, None)])
def test_decode_large_batch_many_units_per_cu(ctx, group, waves, monkeypatch):
    """96 rows of 1 to 700 tokens: several (row, kv head) units per compute
    unit, at the default and a forced wave count, with eight and with four KV
    heads. Unwritten slots hold NaN. The fused step equals append-then-decode
    bit for bit and the oracle within tolerance."""
    if waves:
        monkeypatch.setenv("CKV_DECODE_WAVES", waves)
    rng = orc.Mt64(31 + group)
    rows = 96
    lengths = [rng.uniform_int(1, 700) for _ in range(rows - 4)] + [16, 17, 32, 1]
    H = 16 // group
    q_heads = H * group
    F = H * 128
    B = sum(-(-n // 16) for n in lengths) + 5
    perm = rng.permutation(B)
    tables, at = [], 0
    for n in lengths:
        tables.append(perm[at:at + -(-n // 16)])
        at += len(tables[-1])
    ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
    q = rng.normal(rows * q_heads * 128, orc.BF16).reshape(rows, -1)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    scale = float(np.float32(1 / math.sqrt(128)))
    pools, outs = [], []
    for fused in (True, False):
        pool, keys, values = new_pool(ctx, (1, B, 16, H, 128), orc.BF16, fill=float("nan"))
        fill_by_append(pool, [n - 1 for n in lengths], tables,
                       [k[:-1] for k in ks], [v[:-1] for v in vs])
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
        v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
        out = torch.empty(rows, q_heads * 128, dtype=torch.bfloat16, device="cuda")
        if fused:
            pool.append_decode(0, k_new, v_new, to_dev(q, orc.BF16), q_heads, scale, out)
        else:
            pool.append(0, k_new, v_new)
            pool.decode(0, to_dev(q, orc.BF16), q_heads, scale, out)
        pools.append((pool, keys, values))
        outs.append(out)
    ctx.sync()
    assert torch.equal(pools[0][1].view(torch.int16), pools[1][1].view(torch.int16))
    assert torch.equal(pools[0][2].view(torch.int16), pools[1][2].view(torch.int16))
    assert torch.equal(outs[0], outs[1])
    expected = compact_oracle((H, 128), lengths, tables, ks, vs, q, q_heads)
    assert_close(to_f32(outs[0]), expected, what=f"group {group}, waves {waves}")
    for pool, _, _ in pools:
        pool.close()


def test_edge_positions_and_gqa_groups(ctx):
    """Single-token rows, rows ending exactly on page and chunk boundaries, and
    every GQA group size the fast kernel specialises."""
    rng = orc.Mt64(9)
    lengths = [1, 16, 17, 32, 33, 64, 257, 1024, 1025]
    B = sum(-(-n // 16) for n in lengths) + 3
    perm = rng.permutation(B)
    tables, at = [], 0
    for n in lengths:
        tables.append(perm[at:at + -(-n // 16)])
        at += len(tables[-1])
    for group in (1, 2, 4, 8):
        H = 16 // group if group < 8 else 2
        q_heads = H * group
        F = H * 128
        ks = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
        vs = [rng.normal(n * F, orc.BF16).reshape(n, F) for n in lengths]
        q = rng.normal(len(lengths) * q_heads * 128, orc.BF16).reshape(len(lengths), -1)
        pool, _, _ = new_pool(ctx, (1, B, 16, H, 128), orc.BF16)
        fill_by_append(pool, lengths, tables, ks, vs)
        flat = np.concatenate(tables)
        offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
        pool.upload(flat, offsets, [len(t) for t in tables], [n - 1 for n in lengths])
        out = torch.empty(len(lengths), q_heads * 128, dtype=torch.bfloat16, device="cuda")
        pool.decode(0, to_dev(q, orc.BF16), q_heads, float(np.float32(1 / math.sqrt(128))), out)
        expected = compact_oracle((H, 128), lengths, tables, ks, vs, q, q_heads)
        assert_close(to_f32(out), expected, what=f"group {group}")
        pool.close()
    ctx.sync()


# ---- f32 pools (the reference's storage dtype) through the fast decode ------------------------

@pytest.mark.parametrize("split", [None, "0", "3"])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_f32_decode_append_decode_and_noalloc(ctx, group, split, monkeypatch):
    """f32 pages through the fast decode kernel (1, 2 or 4 q heads per kv head
    in one pass; 8 in two passes of 4 heads): rows of 1 to 1,025 tokens ending
    on and past page boundaries, under the default plan, with no cut and with
    chunks of 3 pages. ckv_append_decode (fused), ckv_append then
    ckv_decode_attention, and the no-allocation entry point leave the same
    pages and outputs bit for bit; outputs within 1e-5 abs + 1e-4 rel of the
    oracle (f32 storage and f32 arithmetic on both sides)."""
    print(f"f32 decode group {group} split {split}", flush=True)
    force_plan(monkeypatch, split)
    rng = orc.Mt64(40 + group)
    lengths = [1, 16, 17, 32, 33, 257, 1024, 1025]
    B = sum(-(-n // 16) for n in lengths) + 3
    perm = rng.permutation(B)
    tables, at = [], 0
    for n in lengths:
        tables.append(perm[at:at + -(-n // 16)])
        at += len(tables[-1])
    H = 16 // group if group < 8 else 2
    q_heads = H * group
    F = H * 128
    ks = [rng.normal(n * F, orc.F32).reshape(n, F) for n in lengths]
    vs = [rng.normal(n * F, orc.F32).reshape(n, F) for n in lengths]
    q = rng.normal(len(lengths) * q_heads * 128, orc.F32).reshape(len(lengths), -1)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    k_new = to_dev(np.stack([k[-1] for k in ks]), orc.F32)
    v_new = to_dev(np.stack([v[-1] for v in vs]), orc.F32)
    qd = to_dev(q, orc.F32)
    scale = float(np.float32(1 / math.sqrt(128)))
    outs, caches = [], []
    for how in ("fused", "pair", "noalloc"):
        pool, kd, vd = new_pool(ctx, (1, B, 16, H, 128), orc.F32, fill=float("nan"))
        cached = [(n - 1, t, k[:-1], v[:-1]) for n, t, k, v in zip(lengths, tables, ks, vs) if n > 1]
        fill_by_append(pool, *zip(*cached), code=orc.F32)
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        out = torch.full((len(lengths), q_heads * 128), float("nan"), device="cuda")
        if how == "fused":
            pool.append_decode(0, k_new, v_new, qd, q_heads, scale, out)
        elif how == "pair":
            pool.append(0, k_new, v_new)
            pool.decode(0, qd, q_heads, scale, out)
        else:
            pool.append_decode_noalloc(0, k_new, v_new, qd, q_heads, scale, out)
        ctx.sync()
        outs.append(out)
        caches.append((kd.clone(), vd.clone()))
        pool.close()
    for other, cache in zip(outs[1:], caches[1:]):
        assert torch.equal(outs[0], other)
        # bit patterns: pages never written hold the NaN fill
        for a, b in zip(caches[0], cache):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    expected = compact_oracle((H, 128), lengths, tables, ks, vs, q, q_heads, code=orc.F32)
    assert_close(to_f32(outs[0]), expected, atol=1e-5, rtol=1e-4,
                 what=f"f32 group {group} split {split}")


# ---- pages: copies, checkpoints, table patches ----------------------------------------------

def test_copy_blocks_bit_exact_and_aliasing_rejected(ctx):
    geom = (3, 10, 16, 2, 8)
    pool, keys, values = new_pool(ctx, geom, orc.BF16)
    rng = np.random.default_rng(7)
    kc = rng.integers(0, 2**16, keys.numel(), dtype=np.uint16)
    vc = rng.integers(0, 2**16, keys.numel(), dtype=np.uint16)
    keys.copy_(to_dev(kc, orc.BF16))
    values.copy_(to_dev(vc, orc.BF16))
    pool.copy_blocks([1, 4, 9], [7, 2, 0])
    orc.copy_blocks(kc, vc, geom, [1, 4, 9], [7, 2, 0])
    assert np.array_equal(to_host(keys, orc.BF16), kc)
    assert np.array_equal(to_host(values, orc.BF16), vc)
    for src, dst, name in [([1, 2], [3, 3], "tensor_op.unsupported_aliasing"),
                           ([1, 2], [2, 5], "tensor_op.unsupported_aliasing"),
                           ([10], [3], "tensor_op.cache_block_out_of_range")]:
        with pytest.raises(ckv.CkvError) as e:
            pool.copy_blocks(src, dst)
        assert e.value.name == name
    pool.close()


def test_checkpoint_pack_and_restore_known_answer(ctx):
    # tests/metal_kv_cache_test.cc:103-142
    geom = (2, 3, 4, 2, 8)
    pool, keys, values = new_pool(ctx, geom, orc.F32)
    k = np.arange(1, 385, dtype=np.float32)
    v = np.arange(1001, 1385, dtype=np.float32)
    keys.copy_(torch.from_numpy(k))
    values.copy_(torch.from_numpy(v))
    pk = torch.zeros(2 * 5 * 16, device="cuda")
    pv = torch.zeros_like(pk)
    pool.checkpoint_pack([2, 0], 5, pk, pv)
    keys.zero_()
    values.zero_()
    pool.checkpoint_unpack([0, 1], 5, pk, pv)
    rk, rv = to_f32(keys), to_f32(values)
    for layer in range(2):
        for token in range(8):
            for f in range(16):
                dest = layer * 192 + token * 16 + f
                orig = layer * 192 + [2, 0][token // 4] * 64 + (token % 4) * 16 + f
                assert rk[dest] == (k[orig] if token < 5 else 0)
                assert rv[dest] == (v[orig] if token < 5 else 0)
    for blocks, tokens in (([3], 1), ([2, 0], 9), ([2], 5), ([2, 0], 0)):
        with pytest.raises(ckv.CkvError) as e:
            pool.checkpoint_pack(blocks, tokens, pk, pv)
        assert e.value.name == "state.invalid_reservation"
    pool.close()


def test_table_patch_equals_reupload(ctx):
    lengths, tables, ks, vs, q = config2_inputs(seed=3, batch=6)
    pool, _, _ = new_pool(ctx, (1, 65536, 16, 8, 128), orc.BF16)
    fill_by_append(pool, lengths, tables, ks, vs)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    # upload a wrong table, then patch it into the right one on the device
    wrong = flat.copy()
    idx = np.arange(0, flat.size, 3)
    wrong[idx] = (wrong[idx] + 1) % 65536
    pool.upload(wrong, offsets, [len(t) for t in tables], positions)
    pool.patch(idx, flat[idx])
    qd = to_dev(q, orc.BF16)
    scale = float(np.float32(1 / math.sqrt(128)))
    patched = torch.empty(6, 2048, dtype=torch.bfloat16, device="cuda")
    pool.decode(0, qd, 16, scale, patched)
    pool.upload(flat, offsets, [len(t) for t in tables], positions)
    fresh = torch.empty_like(patched)
    pool.decode(0, qd, 16, scale, fresh)
    ctx.sync()
    assert torch.equal(patched, fresh)
    with pytest.raises(ckv.CkvError) as e:
        pool.patch([flat.size], [0])
    assert e.value.name == "tensor_op.block_table_range_out_of_bounds"
    with pytest.raises(ckv.CkvError) as e:
        pool.patch([0], [65536])
    assert e.value.name == "tensor_op.cache_block_out_of_range"
    pool.close()


# ---- fused append + decode ------------------------------------------------------------------

def test_append_decode_equals_append_then_decode(ctx):
    lengths, tables, ks, vs, q = config2_inputs(seed=5, batch=12)
    geom = (2, 65536, 16, 8, 128)
    pools = []
    for _ in range(2):
        pool, keys, values = new_pool(ctx, geom, orc.BF16)
        # every token but the last is already cached
        fill_by_append(pool, [n - 1 for n in lengths], tables,
                       [k[:-1] for k in ks], [v[:-1] for v in vs], layer=1)
        pools.append((pool, keys, values))
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    k_new = to_dev(np.stack([k[-1] for k in ks]), orc.BF16)
    v_new = to_dev(np.stack([v[-1] for v in vs]), orc.BF16)
    qd = to_dev(q, orc.BF16)
    scale = float(np.float32(1 / math.sqrt(128)))
    outs = []
    for i, (pool, _, _) in enumerate(pools):
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        out = torch.empty(len(lengths), 16 * 128, dtype=torch.bfloat16, device="cuda")
        if i == 0:
            pool.append_decode(1, k_new, v_new, qd, 16, scale, out)
        else:
            pool.append(1, k_new, v_new)
            pool.decode(1, qd, 16, scale, out)
        outs.append(out)
    ctx.sync()
    assert torch.equal(pools[0][1], pools[1][1]) and torch.equal(pools[0][2], pools[1][2])
    assert torch.equal(outs[0], outs[1])
    expected = compact_oracle((8, 128), lengths, tables, ks, vs, q, 16)
    assert_close(to_f32(outs[0]), expected, what="append_decode vs oracle")
    for pool, _, _ in pools:
        pool.close()


def _own_page_case():
    """Row 0 appends position 20 into page 9 (its table [3, 9]); row 1 appends
    position 40 into page 6 and attends positions 0..40 through [5, x, 6], so
    with x = 9 it reads (as its positions 16..31) the page row 0 writes: such
    a batch must take store_kv then paged_attention."""
    rng = orc.Mt64(29)
    F = 1024
    k = [rng.normal(21 * F, orc.BF16).reshape(21, F), rng.normal(41 * F, orc.BF16).reshape(41, F)]
    v = [rng.normal(21 * F, orc.BF16).reshape(21, F), rng.normal(41 * F, orc.BF16).reshape(41, F)]
    q = rng.normal(2 * 2048, orc.BF16).reshape(2, 2048)
    return k, v, q


def _fused_launches(ctx, run):
    """Runs `run` with profiling on; (fused launches, store_kv launches)."""
    ctx.sync()
    ctx.profile(True)
    ctx.profile_reset()
    run()
    ctx.sync()
    fused = ctx.profile_query("append_decode")[1]
    stores = ctx.profile_query("store_kv")[1]
    ctx.profile(False)
    return fused, stores


@pytest.mark.parametrize("how", ["upload", "patch", "sequence_tables"])
def test_append_decode_unfused_when_another_row_reads_an_own_page(ctx, how):
    """A row's own page (where the fused append writes its token) reached
    through another row's table entry: set by ckv_tables_upload, by a later
    ckv_tables_patch, or through sequence tables and ckv_batch_upload, the
    batch leaves the fused path, and its outputs equal store_kv followed by
    paged_attention bit for bit."""
    k, v, q = _own_page_case()
    geom = (1, 16, 16, 8, 128)
    scale = float(np.float32(1 / math.sqrt(128)))
    t0 = np.array([3, 9], np.uint32)
    clash = np.array([5, 9, 6], np.uint32)
    clean = np.array([5, 11, 6], np.uint32)
    positions = [20, 40]
    slots = [orc.slot(t0, 20, 16), orc.slot(clash, 40, 16)]
    outs = []
    for which in range(2):
        pool, _, _ = new_pool(ctx, geom, orc.BF16)
        fill_by_append(pool, [40], [clash], [k[1][:40]], [v[1][:40]])
        fill_by_append(pool, [20], [t0], [k[0][:20]], [v[0][:20]])
        k_new = to_dev(np.stack([k[0][20], k[1][40]]), orc.BF16)
        v_new = to_dev(np.stack([v[0][20], v[1][40]]), orc.BF16)
        out = torch.empty(2, 2048, dtype=torch.bfloat16, device="cuda")
        if how == "sequence_tables":
            pool.reserve_sequences(2, 4)
            pool.update_sequences(seq=[0, 0, 1, 1, 1], index=[0, 1, 0, 1, 2],
                                  block=[3, 9, 5, 9, 6], len_seq=[0, 1], length=[2, 3])
            pool.upload_batch([0, 1], positions, [1, 1])
        elif how == "upload":
            pool.upload(np.concatenate([t0, clash]), [0, 2], [2, 3], positions, slots)
        else:  # a clean batch, then row 1's second entry patched onto page 9
            pool.upload(np.concatenate([t0, clean]), [0, 2], [2, 3], positions, slots)
            pool.patch([3], [9])
        if which == 0:
            fused, stores = _fused_launches(ctx, lambda: pool.append_decode(
                0, k_new, v_new, to_dev(q, orc.BF16), 16, scale, out))
            assert fused == 0 and stores == 1, (how, fused, stores)
        else:
            pool.append(0, k_new, v_new)
            pool.decode(0, to_dev(q, orc.BF16), 16, scale, out)
        ctx.sync()
        outs.append(out)
        pool.close()
    assert torch.equal(outs[0], outs[1])


def test_append_decode_stays_fused_without_a_shared_own_page(ctx):
    """The same batch with row 1's second entry on a page of its own keeps the
    fused launch."""
    k, v, q = _own_page_case()
    pool, _, _ = new_pool(ctx, (1, 16, 16, 8, 128), orc.BF16)
    t0 = np.array([3, 9], np.uint32)
    t1 = np.array([5, 11, 6], np.uint32)
    pool.upload(np.concatenate([t0, t1]), [0, 2], [2, 3], [20, 40],
                [orc.slot(t0, 20, 16), orc.slot(t1, 40, 16)])
    out = torch.empty(2, 2048, dtype=torch.bfloat16, device="cuda")
    fused, stores = _fused_launches(ctx, lambda: pool.append_decode(
        0, to_dev(np.stack([k[0][20], k[1][40]]), orc.BF16),
        to_dev(np.stack([v[0][20], v[1][40]]), orc.BF16), to_dev(q, orc.BF16), 16,
        float(np.float32(1 / math.sqrt(128))), out))
    assert fused == 1 and stores == 0
    pool.close()


def test_append_decode_falls_back_when_rows_share_a_sequence(ctx):
    # two rows of one sequence (positions 40 and 41) cannot be fused: the
    # second row attends to the token the first row appends
    rng = orc.Mt64(13)
    geom = (1, 8, 16, 8, 128)
    F = 1024
    table = [5, 2, 7]
    k = rng.normal(42 * F, orc.BF16).reshape(42, F)
    v = rng.normal(42 * F, orc.BF16).reshape(42, F)
    q = rng.normal(2 * 2048, orc.BF16).reshape(2, 2048)
    pool, _, _ = new_pool(ctx, geom, orc.BF16)
    fill_by_append(pool, [40], [np.array(table, np.uint32)], [k[:40]], [v[:40]])
    pool.upload(table, [0, 0], [3, 3], [40, 41], [orc.slot(table, 40, 16), orc.slot(table, 41, 16)])
    out = torch.empty(2, 2048, dtype=torch.bfloat16, device="cuda")
    pool.append_decode(0, to_dev(k[40:], orc.BF16), to_dev(v[40:], orc.BF16),
                       to_dev(q, orc.BF16), 16, float(np.float32(1 / math.sqrt(128))), out)
    expected = compact_oracle((8, 128), [41, 42], [np.array(table, np.uint32)] * 2, [k[:41], k],
                              [v[:41], v], q, 16)
    assert_close(to_f32(out), expected, what="append_decode fallback")
    ctx.sync()
    pool.close()
