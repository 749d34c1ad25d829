"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each test restates one of the reference's own known-answer tests (file:line
cited), a closed form, an exhaustive enumeration, or an independent library
routine (numpy, torch, libstdc++). CPU only.
"""
import math
import shutil
import subprocess
import tempfile

import numpy as np
import pytest
import torch

from oracle import oracle as orc


def approx(actual, expected, eps, scale=0.0):
    """doctest::Approx(expected).epsilon(eps).scale(scale), elementwise."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    tol = eps * (scale + np.maximum(np.abs(a), np.abs(e)))
    return bool(np.all(np.abs(a - e) <= tol))


# ---- bf16 / fp16 ---------------------------------------------------------------

def bits_of(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def float_of(bits: int) -> float:
    return float(np.array([bits], dtype=np.uint32).view(np.float32)[0])


def test_bf16_known_answers():
    # tests/tensor_test.cc:47-69
    L = orc.lib()
    assert L.orc_bf16_to_f32(0x0000) == 0.0
    assert L.orc_bf16_to_f32(0x3F80) == 1.0
    assert L.orc_bf16_to_f32(0xC020) == -2.5
    assert L.orc_bf16_from_f32(1.0) == 0x3F80
    assert L.orc_bf16_from_f32(-2.5) == 0xC020
    assert L.orc_bf16_from_f32(float_of(0x3F808000)) == 0x3F80  # tie rounds to even (down)
    assert L.orc_bf16_from_f32(float_of(0x3F818000)) == 0x3F82  # tie rounds to even (up)
    assert math.isinf(L.orc_bf16_to_f32(L.orc_bf16_from_f32(float("inf"))))
    assert math.isnan(L.orc_bf16_to_f32(L.orc_bf16_from_f32(float("nan"))))


def test_bf16_exhaustive_round_trip_and_torch_agreement():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.to_f32(bits, orc.BF16)
    assert np.array_equal(f.view(np.uint32), bits.astype(np.uint32) << 16)
    back = orc.from_f32(f, orc.BF16)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(back[nan] & 0x40)  # NaNs come back quiet
    # torch rounds f32 -> bf16 to nearest even: an independent implementation
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32),
                        (rng.integers(0, 2**32, 200000, dtype=np.uint64)
                         .astype(np.uint32).view(np.float32))])
    x = x[np.isfinite(x)]
    ours = orc.from_f32(x, orc.BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_exhaustive_round_trip_and_numpy_agreement():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.to_f32(bits, orc.F16)
    # numpy's binary16 -> binary32 widening is exact: an independent decoder
    assert np.array_equal(f.view(np.uint32), bits.view(np.float16).astype(np.float32)
                          .view(np.uint32))
    back = orc.from_f32(f, orc.F16)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(back[nan] & 0x200)
    # narrowing: numpy rounds to nearest even, including subnormals, ties and overflow
    rng = np.random.default_rng(2)
    mags = rng.uniform(-27.0, 17.0, 400000)
    x = (np.sign(rng.standard_normal(mags.size)) * np.exp2(mags)).astype(np.float32)
    ties = (bits[(bits & 0x7C00) != 0x7C00].view(np.float16).astype(np.float32)
            .view(np.uint32) + np.uint32(1 << 12)).view(np.float32)  # exact halfway points
    x = np.concatenate([x, ties, np.array([65504, 65519.99, 65520, 1e9, 2.0**-25,
                                           2.0**-25 * 1.0000001, 2.0**-26], np.float32)])
    ours = orc.from_f32(x, orc.F16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ---- seeded inputs ---------------------------------------------------------------

def test_mt19937_64_standard_check_value():
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed
    # std::mt19937_64 (seed 5489) produces 9981545732273789042.
    rng = orc.Mt64(5489)
    for _ in range(9999):
        rng.next()
    assert rng.next() == 9981545732273789042


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_mt19937_64_matches_libstdcxx():
    src = r"""
    #include <cstdio>
    #include <random>
    int main() {
        for (unsigned long long seed : {0ULL, 1ULL, 12345ULL, 0xFFFFFFFFFFFFFFFFULL}) {
            std::mt19937_64 g(seed);
            for (int i = 0; i < 700; ++i) std::printf("%llu\n", (unsigned long long)g());
        }
    }"""
    with tempfile.TemporaryDirectory() as d:
        with open(f"{d}/m.cc", "w") as fh:
            fh.write(src)
        subprocess.run(["g++", "-O1", "-o", f"{d}/m", f"{d}/m.cc"], check=True)
        expected = [int(v) for v in subprocess.run([f"{d}/m"], check=True, capture_output=True,
                                                   text=True).stdout.split()]
    ours = []
    for seed in (0, 1, 12345, 0xFFFFFFFFFFFFFFFF):
        rng = orc.Mt64(seed)
        ours += [rng.next() for _ in range(700)]
    assert ours == expected


def test_normal_draws_are_standard_normal():
    from scipy import stats
    z = orc.Mt64(0).normal(200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1.0) < 0.01
    assert stats.kstest(z, "norm").pvalue > 1e-3
    # consecutive outputs (cos / sin of one pair) are uncorrelated
    assert abs(np.corrcoef(z[0::2], z[1::2])[0, 1]) < 0.01
    # 16-bit draws are the RNE rounding of the f32 draws
    assert np.array_equal(orc.Mt64(0).normal(1000, orc.BF16),
                          orc.from_f32(orc.Mt64(0).normal(1000), orc.BF16))


def test_permutation_is_a_permutation():
    p = orc.Mt64(7).permutation(65536)
    assert np.array_equal(np.sort(p), np.arange(65536))
    assert not np.array_equal(p, np.arange(65536))


# ---- page allocator ----------------------------------------------------------------

def test_block_manager_validates_geometry():
    # tests/block_manager_test.cc:6-14
    with pytest.raises(ValueError, match="invalid_block_count"):
        orc.BlockManager(0, 16)
    with pytest.raises(ValueError, match="invalid_block_size"):
        orc.BlockManager(4, 0)
    with pytest.raises(ValueError, match="too_many_blocks"):
        orc.BlockManager(2**32 + 1, 16)


def test_block_manager_grows_at_block_boundaries_and_releases_fifo():
    # tests/block_manager_test.cc:16-37
    s = orc.BlockManager(4, 2)
    assert s.reserve(1, 3) is None
    assert s.table(1).size == 2 and s.free_count() == 2
    assert s.reserve(1, 4) is None and s.free_count() == 2
    assert s.reserve(1, 5) is None and s.table(1).size == 3
    assert s.reserve(2, 2) is None and s.table(2)[0] == 3
    s.release(1)
    assert s.table(1).size == 0 and s.free_count() == 3
    s.release(1)
    assert s.free_count() == 3
    assert s.reserve(3, 1) is None
    assert s.table(3)[0] == 0 and s.table(2)[0] == 3


def test_block_manager_failed_reservation_is_atomic():
    # tests/block_manager_test.cc:39-50
    s = orc.BlockManager(2, 2)
    assert s.reserve(1, 2) is None
    assert s.reserve(2, 3) == "capacity_exhausted"
    assert s.table(2).size == 0
    assert s.reserve(1, 5) == "capacity_exhausted"
    assert s.table(1).size == 1 and s.free_count() == 1
    assert s.reserve(2, 0) == "invalid_reservation"


def test_slots_cover_each_page_once_in_logical_order():
    rng = np.random.default_rng(3)
    for block_size in (1, 2, 16):
        table = rng.permutation(64)[:9].astype(np.uint32)
        slots = [orc.slot(table, p, block_size) for p in range(9 * block_size)]
        assert len(set(slots)) == len(slots)
        pages = [s // block_size for s in slots]
        assert pages == [int(table[p // block_size]) for p in range(len(slots))]
        assert [s % block_size for s in slots] == [p % block_size for p in range(len(slots))]
        assert orc.slot(table, 9 * block_size, block_size) is None  # beyond the table


# ---- cache addressing ---------------------------------------------------------------

def test_prepare_paged_batch_rows_follow_the_closed_form():
    """src/model_batch.cc:127-204 restated: per row, slot = table[p / bs] * bs +
    p % bs (brute force over every position of a fragmented table), the item's
    offset in the flat table and its table length; the flat table is the
    items' tables concatenated."""
    rng = np.random.default_rng(4)
    for block_size in (1, 2, 16):
        tables = [rng.permutation(64)[:n].astype(np.uint32) for n in (3, 1, 7)]
        counts = [3 * block_size, block_size, 7 * block_size]
        positions = np.concatenate([np.arange(c) for c in counts]).astype(np.uint32)
        got = orc.prepare_paged_batch(counts, tables, positions, 10**6, 64, block_size)
        assert got is not None
        flat, slots, offsets, lengths = got
        assert flat.tolist() == np.concatenate(tables).tolist()
        row = 0
        for i, (t, c) in enumerate(zip(tables, counts)):
            for p in range(c):
                assert slots[row] == int(t[p // block_size]) * block_size + p % block_size
                assert offsets[row] == sum(len(x) for x in tables[:i])
                assert lengths[row] == len(t)
                row += 1


def test_prepare_paged_batch_rejects_inconsistent_batches():
    """The checks of src/model_batch.cc:132-192, each on its own."""
    ok = dict(token_counts=[2], tables=[[3, 4]], positions=[16, 17], max_positions=64,
              block_count=8, block_size=16)
    assert orc.prepare_paged_batch(**ok) is not None
    for change in (dict(token_counts=[]), dict(block_size=0), dict(block_count=0),
                   dict(token_counts=[0], positions=[]), dict(tables=[[]]),
                   dict(tables=[[3, 8]]),            # entry >= block_count
                   dict(positions=[16, 64]),         # position >= max_positions
                   dict(positions=[16, 32])):        # logical block past the table
        args = dict(ok)
        args.update(change)
        if change.get("token_counts") == []:
            args["tables"], args["positions"] = [], []
        assert orc.prepare_paged_batch(**args) is None, change


def test_decode_step_host_matches_block_manager_and_slots():
    """One decode step's host work equals block_manager reserve(len + 1) per
    sequence (FIFO pages) followed by the slot closed form at position len."""
    lengths = [1, 15, 16, 17, 40, 300]
    step = orc.DecodeStepHost(lengths, 200, 16, 32)
    step.step()
    bm = orc.BlockManager(200, 16, len(lengths))
    for s, n in enumerate(lengths):
        assert bm.reserve(s, n) is None
    for s, n in enumerate(lengths):
        assert bm.reserve(s, n + 1) is None
    tables = [bm.table(s) for s in range(len(lengths))]
    assert step.flat[:sum(len(t) for t in tables)].tolist() == np.concatenate(tables).tolist()
    assert step.slots.tolist() == [orc.slot(t, n, 16) for t, n in zip(tables, lengths)]
    assert step.row_lengths.tolist() == [len(t) for t in tables]
    assert step.lengths.tolist() == [n + 1 for n in lengths]


def test_element_offsets_follow_layout_order():
    # tests/metal_kv_cache_test.cc:82-101, geometry (L2, B3, bs4, H2, D8)
    g = (2, 3, 4, 2, 8)
    assert orc.element_offset(g, 0, 0, 0, 0, 0) == 0
    assert orc.element_offset(g, 0, 0, 0, 0, 1) == 1
    assert orc.element_offset(g, 0, 0, 0, 1, 0) == 8
    assert orc.element_offset(g, 0, 0, 1, 0, 0) == 16
    assert orc.element_offset(g, 0, 1, 0, 0, 0) == 64
    assert orc.element_offset(g, 1, 0, 0, 0, 0) == 192
    assert orc.element_offset(g, 1, 2, 3, 1, 7) == 383
    # kv_cache_errc: layer 7, block 8, token 9, head 10, feature 11
    assert orc.element_offset(g, 2, 0, 0, 0, 0) == -7
    assert orc.element_offset(g, 0, 3, 0, 0, 0) == -8
    assert orc.element_offset(g, 0, 0, 4, 0, 0) == -9
    assert orc.element_offset(g, 0, 0, 0, 2, 0) == -10
    assert orc.element_offset(g, 0, 0, 0, 0, 8) == -11


# ---- append / gather -----------------------------------------------------------------

@pytest.mark.parametrize("dtype", [orc.F32, orc.BF16, orc.F16])
def test_store_kv_writes_rows_into_selected_slots(dtype):
    # tests/tensor_ops_test.cc:610-633: cache (L2, B2, bs2, H1, D2), slots {1, 3}, layer 1
    kc = orc.from_f32(np.full(16, -1.0), dtype)
    vc = orc.from_f32(np.full(16, -1.0), dtype)
    keys = orc.from_f32(np.array([[1, 2], [3, 4]]), dtype)
    values = orc.from_f32(np.array([[5, 6], [7, 8]]), dtype)
    orc.store_kv(kc, vc, keys, values, [1, 3], layer=1, slot_count=4)
    assert list(orc.to_f32(kc, dtype)) == [-1] * 10 + [1, 2, -1, -1, 3, 4]
    assert list(orc.to_f32(vc, dtype)) == [-1] * 10 + [5, 6, -1, -1, 7, 8]
    # attention.metal:19-22: a slot beyond the cache is skipped
    before = kc.copy()
    orc.store_kv(kc, vc, keys, values, [4, 9], layer=1, slot_count=4)
    assert np.array_equal(kc, before)


def test_gather_inverts_store_through_a_fragmented_table():
    rng = np.random.default_rng(4)
    L, B, bs, F = 3, 40, 16, 24
    kc = np.zeros(L * B * bs * F, np.uint16)
    vc = np.zeros_like(kc)
    table = rng.permutation(B)[:5].astype(np.uint32)
    n = 70
    keys = rng.integers(0, 2**16, (n, F), dtype=np.uint16)
    values = rng.integers(0, 2**16, (n, F), dtype=np.uint16)
    slots = [orc.slot(table, p, bs) for p in range(n)]
    orc.store_kv(kc, vc, keys, values, slots, layer=2, slot_count=B * bs)
    gk, gv = orc.gather(kc, vc, table, n, 2, B * bs, bs, F)
    assert np.array_equal(gk, keys) and np.array_equal(gv, values)
    # nothing outside the table's pages of layer 2 was written
    view = kc.reshape(L, B, bs * F)
    untouched = np.ones((L, B), bool)
    untouched[2, table] = False
    assert not view[untouched].any()


# ---- attention -------------------------------------------------------------------------

def _all_paths(att: orc.Attention):
    return {"online": att.online(), "split": att.split(64), "prefill": att.prefill(),
            "threads": att.online_threads(3), "reference": att.reference()}


def test_decode_attention_closed_form_gqa_and_page_order():
    # tests/tensor_ops_test.cc:693-735: cache (L2, B2, bs2, H1, D2), table {1, 0},
    # position 2, two q heads share the KV head.
    keys = np.array([1, 1, 0, 0, 1, 0, 0, 1] + [0] * 8, np.float32)
    values = np.array([30, 3, 0, 0, 10, 1, 20, 2] + [0] * 8, np.float32)
    att = orc.Attention((2, 2, 2, 1, 2), keys, values, orc.F32,
                        np.array([[1, 0, 0, 1]], np.float32), orc.F32, [2], [1, 0], [0], [2],
                        q_heads=2, layer=0, scale=1 / math.sqrt(2))
    e = math.exp(1 / math.sqrt(2))
    d = 2 * e + 1
    expected = [(40 * e + 20) / d, (4 * e + 2) / d, (10 + 50 * e) / d, (1 + 5 * e) / d]
    for name, out in _all_paths(att).items():
        assert approx(out[0], expected, 1e-5), name


def test_gqa_maps_consecutive_q_heads_to_one_kv_head():
    # Hq 4 over Hkv 2: V is 1.0 for KV head 0 and 2.0 for KV head 1, so the
    # output is (1, 1, 2, 2) per head. head % Hkv would give (1, 2, 1, 2).
    L, B, bs, H, D = 1, 4, 4, 2, 8
    rng = np.random.default_rng(5)
    keys = rng.standard_normal(L * B * bs * H * D).astype(np.float32)
    values = np.zeros((L, B, bs, H, D), np.float32)
    values[..., 0, :] = 1.0
    values[..., 1, :] = 2.0
    q = rng.standard_normal((3, 4 * D)).astype(np.float32)
    att = orc.Attention((L, B, bs, H, D), keys, values.ravel(), orc.F32, q, orc.F32,
                        [5, 6, 0], [2, 0, 3], [0, 0, 2], [2, 2, 1], 4, 0, 1 / math.sqrt(D))
    expected = np.repeat([1.0, 1.0, 2.0, 2.0], D)
    for name, out in _all_paths(att).items():
        assert approx(out, np.tile(expected, (3, 1)), 1e-6), name


def _dense_sdpa(geom, keys, values, q, positions, table, offsets, q_heads, layer, scale):
    """torch scaled_dot_product_attention over K/V gathered densely by table."""
    L, B, bs, H, D = geom
    kc = torch.from_numpy(np.asarray(keys, np.float64).reshape(L, B * bs, H, D))
    vc = torch.from_numpy(np.asarray(values, np.float64).reshape(L, B * bs, H, D))
    qt = torch.from_numpy(np.asarray(q, np.float64)).reshape(len(positions), q_heads, D)
    out = torch.zeros(len(positions), q_heads, D, dtype=torch.float64)
    for r, p in enumerate(positions):
        tokens = np.arange(p + 1)
        slots = np.asarray(table)[offsets[r] + tokens // bs] * bs + tokens % bs
        k = kc[layer, slots].permute(1, 0, 2)  # [H, T, D]
        v = vc[layer, slots].permute(1, 0, 2)
        k = k.repeat_interleave(q_heads // H, dim=0)
        v = v.repeat_interleave(q_heads // H, dim=0)
        out[r] = torch.nn.functional.scaled_dot_product_attention(
            qt[r][:, None, :], k, v, scale=float(np.float32(scale)))[:, 0, :]
    return out.reshape(len(positions), -1).numpy()


def test_prefill_tiles_match_causal_library_attention():
    # tests/tensor_ops_test.cc:737-822: logical tokens 0..3 live in block 1 then block 0
    keys = np.array([0.25, 0.75, -0.5, 1.0, 1.0, 0.0, 0.5, -0.25], np.float32)
    values = np.array([30, 3, 40, 4, 10, 1, 20, 2], np.float32)
    q = np.array([1.0, 0.5, -0.5, 1.0, 0.25, 1.0, 1.0, -0.25, -0.5, 0.75, 0.5, 0.5, 1.0,
                  -1.0, -0.25, 0.75], np.float32).reshape(4, 4)
    geom = (1, 2, 2, 1, 2)
    att = orc.Attention(geom, keys, values, orc.F32, q, orc.F32, [0, 1, 2, 3], [1, 0],
                        [0] * 4, [2] * 4, 2, 0, 1 / math.sqrt(2))
    starts, lens, shared = orc.query_tiles(att.pos, att.off, att.len)
    assert shared and list(starts) == [0] and list(lens) == [4]
    expected = _dense_sdpa(geom, keys, values, q, [0, 1, 2, 3], [1, 0], [0] * 4, 2, 0,
                           1 / math.sqrt(2))
    for name, out in _all_paths(att).items():
        assert approx(out, expected, 1e-5), name


def test_prefill_merges_key_tiles_across_a_cached_prefix():
    # tests/tensor_ops_test.cc:824-870: K = 0 gives uniform weights, so row p
    # averages V over 0..p: (p/2, p).
    geom = (1, 2, 16, 1, 2)
    values = np.array([[t, 2 * t] for t in range(32)], np.float32).ravel()
    att = orc.Attention(geom, np.zeros(64, np.float32), values, orc.F32,
                        np.ones((8, 2), np.float32), orc.F32, list(range(16, 24)), [0, 1],
                        [0] * 8, [2] * 8, 1, 0, 1 / math.sqrt(2))
    for name, out in _all_paths(att).items():
        for r in range(8):
            p = 16 + r
            assert approx(out[r], [p / 2, p], 1e-5), name


def test_split_decode_combines_context_chunks():
    # tests/tensor_ops_test.cc:941-984: position 128 over 9 pages, K = 0:
    # mean of (t, 2t) over t = 0..128 inclusive is (64, 128).
    geom = (1, 9, 16, 1, 2)
    values = np.array([[t, 2 * t] for t in range(144)], np.float32).ravel()
    att = orc.Attention(geom, np.zeros(288, np.float32), values, orc.F32,
                        np.ones((1, 2), np.float32), orc.F32, [128], list(range(9)), [0], [9],
                        1, 0, 1 / math.sqrt(2))
    for name, out in _all_paths(att).items():
        assert approx(out[0], [64, 128], 1e-5), name


@pytest.mark.parametrize("dim", [129, 192, 256, 257])
def test_wide_heads_ragged_batch_match_double_reference(dim):
    # tests/tensor_ops_test.cc:872-939
    rows, heads, kv_heads = 5, 4, 2
    geom = (2, 6, 16, kv_heads, dim)
    n = 2 * 6 * 16 * kv_heads * dim
    i = np.arange(n, dtype=np.float32)
    keys = np.sin(i * np.float32(0.17)).astype(np.float32)
    values = np.cos(i * np.float32(0.11)).astype(np.float32)
    q = (20 * np.sin(np.arange(rows * heads * dim, dtype=np.float32) * np.float32(0.13))
         ).astype(np.float32).reshape(rows, -1)
    pos, tables, offsets = [17, 18, 7, 32, 9], [4, 1, 5, 3, 0, 2], [0, 0, 3, 3, 0]
    att = orc.Attention(geom, keys, values, orc.F32, q, orc.F32, pos, tables, offsets,
                        [3] * rows, heads, 1, 1 / math.sqrt(dim))
    paths = _all_paths(att)
    expected = paths.pop("reference")
    library = _dense_sdpa(geom, keys, values, q, pos, tables, offsets, heads, 1,
                          1 / math.sqrt(dim))
    assert approx(expected, library, 1e-9, 1.0)
    for name, out in paths.items():
        assert approx(out, expected, 3e-5, 1.0), name


@pytest.mark.parametrize("dtype", [orc.BF16, orc.F16])
def test_16bit_caches_convert_exactly(dtype):
    # a 16-bit cache is read as its exact f32 value: the result equals the f32
    # path on the widened arrays, bit for bit
    rng = orc.Mt64(11)
    geom = (1, 8, 16, 2, 128)
    n = 8 * 16 * 2 * 128
    k16, v16 = rng.normal(n, dtype), rng.normal(n, dtype)
    q16 = rng.normal(3 * 4 * 128, dtype).reshape(3, -1)
    args = ([100, 31, 0], [3, 1, 7, 2, 0, 5, 4, 6], [0, 0, 7], [7, 7, 1], 4, 0,
            1 / math.sqrt(128))
    a16 = orc.Attention(geom, k16, v16, dtype, q16, dtype, *args)
    a32 = orc.Attention(geom, orc.to_f32(k16, dtype), orc.to_f32(v16, dtype), orc.F32,
                        orc.to_f32(q16, dtype), orc.F32, *args)
    assert np.array_equal(a16.online(), a32.online())


def test_query_tiles_partition_rows_into_maximal_runs():
    rng = np.random.default_rng(6)
    positions, offsets, lengths = [], [], []
    for s in range(40):
        n = int(rng.integers(1, 20))
        start = int(rng.integers(0, 50))
        positions += list(range(start, start + n))
        offsets += [s * 4] * n
        lengths += [4] * n
    starts, lens, shared = orc.query_tiles(positions, offsets, lengths)
    assert shared
    assert starts[0] == 0 and np.all(starts[1:] == np.cumsum(lens)[:-1])
    assert lens.sum() == len(positions) and lens.max() <= 8
    for s, n in zip(starts, lens):
        rows = range(s, s + n)
        assert all(offsets[r] == offsets[s] and lengths[r] == lengths[s] for r in rows)
        assert all(positions[r] == positions[s] + (r - s) for r in rows)
        e = s + n
        if n < 8 and e < len(positions):
            assert (offsets[e] != offsets[s] or lengths[e] != lengths[s]
                    or positions[e] != positions[e - 1] + 1)
    # decode rows of different sequences never share a tile
    _, lens, shared = orc.query_tiles([5, 9, 100], [0, 4, 8], [4, 4, 4])
    assert not shared and list(lens) == [1, 1, 1]


# ---- checkpoints and page copies -----------------------------------------------------

def test_checkpoint_remaps_pages_and_copies_only_the_committed_tail():
    # tests/metal_kv_cache_test.cc:103-142, geometry (L2, B3, bs4, H2, D8)
    g = (2, 3, 4, 2, 8)
    n = 2 * 3 * 4 * 2 * 8
    keys = np.arange(1, n + 1, dtype=np.float32)
    packed = np.zeros(2 * 5 * 16, np.float32)  # checkpoint_bytes(5) / 2 / sizeof(float)
    orc.copy_prefix(keys, packed, [2, 0], g, 5, restore=False)
    restored = np.zeros(n, np.float32)
    orc.copy_prefix(restored, packed, [0, 1], g, 5, restore=True)
    for layer in range(2):
        for token in range(8):
            for f in range(16):
                dest = layer * 192 + token * 16 + f
                orig = layer * 192 + [2, 0][token // 4] * 64 + (token % 4) * 16 + f
                assert restored[dest] == (keys[orig] if token < 5 else 0)


def test_copy_blocks_duplicates_pages_bit_for_bit():
    g = (3, 10, 16, 2, 8)
    rng = np.random.default_rng(7)
    kc = rng.integers(0, 2**16, 3 * 10 * 16 * 16, dtype=np.uint16)
    vc = rng.integers(0, 2**16, kc.size, dtype=np.uint16)
    k0, v0 = kc.copy(), vc.copy()
    orc.copy_blocks(kc, vc, g, [1, 4], [7, 2])
    kv, k0v = kc.reshape(3, 10, -1), k0.reshape(3, 10, -1)
    assert np.array_equal(kv[:, 7], k0v[:, 1]) and np.array_equal(kv[:, 2], k0v[:, 4])
    assert np.array_equal(vc.reshape(3, 10, -1)[:, 7], v0.reshape(3, 10, -1)[:, 1])
    others = [b for b in range(10) if b not in (7, 2)]
    assert np.array_equal(kv[:, others], k0v[:, others])


# ---- rotary position embedding ---------------------------------------------------------

def test_rope_rotates_split_half_pairs_known_answer():
    # tests/tensor_ops_test.cc:426-469: two heads of 4, positions {0, 1}, theta 1e4
    x = np.tile(np.arange(1, 9, dtype=np.float32), (2, 1))
    out = orc.rope(x, orc.F32, 2, [0, 1], 10000.0)
    fc, fs, sc, ss = math.cos(1.0), math.sin(1.0), math.cos(0.01), math.sin(0.01)
    expected = [1, 2, 3, 4, 5, 6, 7, 8,
                1 * fc - 3 * fs, 2 * sc - 4 * ss, 3 * fc + 1 * fs, 4 * sc + 2 * ss,
                5 * fc - 7 * fs, 6 * sc - 8 * ss, 7 * fc + 5 * fs, 8 * sc + 6 * ss]
    assert approx(out.ravel(), expected, 1e-5)


def test_partial_rope_rotates_only_the_prefix():
    # tests/tensor_ops_test.cc:471-511: rotary widths 8 and 4 of 8-wide heads, theta 100
    values = (np.arange(32, dtype=np.float32) - 8).reshape(2, 16)
    for rotary in (8, 4, 8, 4):
        expected = values.copy()
        for row in range(2):
            for head in range(2):
                for pair in range(rotary // 2):
                    a = head * 8 + pair
                    b = a + rotary // 2
                    angle = np.float32(1 + row * 2) * np.float32(100.0) ** np.float32(
                        -2.0 * pair / rotary)
                    expected[row, a] = values[row, a] * math.cos(angle) - values[row, b] * math.sin(angle)
                    expected[row, b] = values[row, b] * math.cos(angle) + values[row, a] * math.sin(angle)
        assert approx(orc.rope(values, orc.F32, 2, [1, 3], 100.0, rotary), expected, 1e-5)
    for invalid in (3, 10):
        with pytest.raises(ValueError):
            orc.rope(values, orc.F32, 2, [1, 3], 100.0, invalid)
    for theta in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError):
            orc.rope(values, orc.F32, 2, [1, 3], theta)


def test_rope_frequencies_and_invariants():
    # inverse frequencies theta^(-2p/rotary) in float (src/metal/metal_kernels.mm:186-191)
    f = orc.rope_frequencies(1e6, 128)
    assert f[0] == 1.0 and f.size == 64
    assert np.allclose(f, 1e6 ** (-2.0 * np.arange(64) / 128), rtol=1e-6)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 4 * 128)).astype(np.float32)
    # position 0 is the identity; every pair keeps its length; a rotation by
    # p followed by the inverse angle returns the input
    assert np.array_equal(orc.rope(x, orc.F32, 4, [0] * 5, 1e6), x)
    pos = [1, 17, 300, 4096, 16383]
    y = orc.rope(x, orc.F32, 4, pos, 1e6)
    xr, yr = x.reshape(5, 4, 2, 64), y.reshape(5, 4, 2, 64)
    assert np.allclose(np.hypot(xr[:, :, 0], xr[:, :, 1]), np.hypot(yr[:, :, 0], yr[:, :, 1]),
                       rtol=1e-5, atol=1e-6)
    angles = np.float32(np.array(pos, np.float32)[:, None]) * f[None, :]
    c, s = np.cos(angles)[:, None, :], np.sin(angles)[:, None, :]
    back0 = yr[:, :, 0] * c + yr[:, :, 1] * s
    back1 = yr[:, :, 1] * c - yr[:, :, 0] * s
    assert np.allclose(back0, xr[:, :, 0], atol=1e-4) and np.allclose(back1, xr[:, :, 1], atol=1e-4)
    # 16-bit rows: rotate in float, round to nearest even (bf16 of the f32 result)
    xb = orc.from_f32(x, orc.BF16)
    yb = orc.rope(xb, orc.BF16, 4, pos, 1e6)
    assert np.array_equal(yb, orc.from_f32(orc.rope(orc.to_f32(xb, orc.BF16), orc.F32, 4, pos,
                                                    1e6), orc.BF16))


# ---- the attention-output gate -------------------------------------------------

def test_sigmoid_mul_known_answer():
    # tests/tensor_ops_test.cc:513-539: gate {0, 1, -1, 2, -1000, 1000, 0, -2} on
    # query {1..8}; sigmoid(+-1000) is exactly 1 and 0
    gate = np.array([0, 1, -1, 2, -1000, 1000, 0, -2], np.float32)
    query = np.arange(1, 9, dtype=np.float32)
    got = orc.sigmoid_mul(gate, query, orc.F32)
    expected = [0.5, 2 / (1 + math.exp(-1)), 3 / (1 + math.exp(1)), 4 / (1 + math.exp(-2)),
                0.0, 6.0, 3.5, 8 / (1 + math.exp(2))]
    assert approx(got, expected, 1e-5)
    assert got[4] == 0.0 and got[5] == 6.0


def test_sigmoid_mul_against_torch_and_rounding():
    # an independent routine: torch.sigmoid in float64, then one rounding to
    # the storage type; 16-bit results within one unit in the last place
    rng = np.random.default_rng(5)
    g = rng.normal(0, 4, 4096).astype(np.float32)
    x = rng.normal(0, 1, 4096).astype(np.float32)
    ref = torch.sigmoid(torch.from_numpy(g).double()) * torch.from_numpy(x).double()
    got = orc.sigmoid_mul(g, x, orc.F32)
    assert np.allclose(got, ref.numpy(), rtol=4e-7, atol=1e-30)
    for code in (orc.BF16, orc.F16):
        gb, xb = orc.from_f32(g, code), orc.from_f32(x, code)
        ref16 = (torch.sigmoid(torch.from_numpy(orc.to_f32(gb, code)).double())
                 * torch.from_numpy(orc.to_f32(xb, code)).double()).numpy()
        got16 = orc.sigmoid_mul(gb, xb, code)
        expect_bits = orc.from_f32(ref16.astype(np.float32), code)
        a = got16.astype(np.int32)
        b = expect_bits.astype(np.int32)
        a = np.where(a & 0x8000, -(a & 0x7FFF), a)
        b = np.where(b & 0x8000, -(b & 0x7FFF), b)
        assert np.abs(a - b).max() <= 1
