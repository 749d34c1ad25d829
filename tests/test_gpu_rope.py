"""Rotary position embedding on the device (ckv_rope) and its fusion with the
KV append (ckv_rope_append), against the reference's known answers
(tests/tensor_ops_test.cc:426-560) and the oracle restatement of rope_f32.

Rotation is floating point: rotated rows are checked within one unit in the
last place of the storage type against the oracle (and within 2e-2 abs +
1e-2 rel); the appended values and the slot placement are bit-exact, and the
fused launch equals rope followed by append bit for bit."""
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import (assert_close, approx, force_plan, new_context, new_pool, to_dev,
                            to_f32, to_host)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def ulps(a_bits, b_bits, code):
    """Distance in units in the last place between two arrays of 16-bit patterns."""
    a = np.asarray(a_bits, np.uint16).astype(np.int32)
    b = np.asarray(b_bits, np.uint16).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


def test_rope_known_answer_split_half_pairs(ctx):
    # tests/tensor_ops_test.cc:426-469: heads 2 x 4, positions {0, 1}, theta 1e4
    pool, _, _ = new_pool(ctx, (1, 1, 2, 2, 4), orc.F32)
    pool.upload([0], [0, 0], [1, 1], [0, 1])
    x = torch.tensor([list(range(1, 9))] * 2, dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    pool.rope(x, out, 2, 10000.0)
    fc, fs, sc, ss = math.cos(1.0), math.sin(1.0), math.cos(0.01), math.sin(0.01)
    expected = [1, 2, 3, 4, 5, 6, 7, 8,
                1 * fc - 3 * fs, 2 * sc - 4 * ss, 3 * fc + 1 * fs, 4 * sc + 2 * ss,
                5 * fc - 7 * fs, 6 * sc - 8 * ss, 7 * fc + 5 * fs, 8 * sc + 6 * ss]
    assert approx(to_f32(out).ravel(), expected, 1e-5)
    pool.close()


def test_partial_rope_in_and_out_of_place(ctx):
    # tests/tensor_ops_test.cc:471-511: heads 2 x 8, positions {1, 3}, theta 100
    pool, _, _ = new_pool(ctx, (1, 2, 4, 2, 8), orc.F32)
    pool.upload([0], [0, 0], [1, 1], [1, 3])
    values = (np.arange(32, dtype=np.float32) - 8).reshape(2, 16)
    x = torch.from_numpy(values).cuda()
    for rotary in (8, 4, 8, 4):
        expected = orc.rope(values, orc.F32, 2, [1, 3], 100.0, rotary)
        out = torch.empty_like(x)
        pool.rope(x, out, 2, 100.0, rotary)
        assert approx(to_f32(out), expected, 1e-5)
        inplace = x.clone()
        pool.rope(inplace, inplace, 2, 100.0, rotary)
        assert approx(to_f32(inplace), expected, 1e-5)
    pool.close()


def test_rope_validation_codes(ctx):
    # tests/tensor_ops_test.cc:542-560 (the checks that exist at this boundary)
    pool, _, _ = new_pool(ctx, (1, 2, 4, 2, 8), orc.F32)
    x = torch.zeros(2, 16, device="cuda")
    with pytest.raises(ckv.CkvError) as e:
        pool.rope(x, x, 2, 100.0)
    assert e.value.code == 403  # nothing uploaded
    pool.upload([0], [0, 0], [1, 1], [1, 3])
    cases = [
        (dict(heads=2, theta=100.0, rows=1), "tensor_op.position_count_mismatch"),
        (dict(heads=0, theta=100.0), "tensor_op.invalid_head_count"),
        (dict(heads=2, theta=100.0, rotary_dim=3), "tensor_op.invalid_head_dimension"),
        (dict(heads=2, theta=100.0, rotary_dim=10), "tensor_op.invalid_head_dimension"),
        (dict(heads=2, theta=0.0), "tensor_op.invalid_rope_theta"),
        (dict(heads=2, theta=-1.0), "tensor_op.invalid_rope_theta"),
        (dict(heads=2, theta=float("inf")), "tensor_op.invalid_rope_theta"),
        (dict(heads=2, theta=float("nan")), "tensor_op.invalid_rope_theta"),
        # the row count is checked before the head count, as the reference does
        (dict(heads=0, theta=0.0, rows=1), "tensor_op.position_count_mismatch"),
    ]
    for kwargs, name in cases:
        with pytest.raises(ckv.CkvError) as e:
            pool.rope(x, x, **kwargs)
        assert e.value.name == name, kwargs
    k = torch.zeros(2, 16, device="cuda")
    with pytest.raises(ckv.CkvError) as e:  # append checks come first
        pool.rope_append(0, k, k, 100.0)
    assert e.value.code == 403
    pool.upload([0], [0, 0], [1, 1], [1, 3], slots=[0, 1])
    with pytest.raises(ckv.CkvError) as e:
        pool.rope_append(1, k, k, 100.0)
    assert e.value.name == "tensor_op.cache_layer_out_of_range"
    with pytest.raises(ckv.CkvError) as e:
        pool.rope_append(0, k, k, -2.0)
    assert e.value.name == "tensor_op.invalid_rope_theta"
    pool.close()


@pytest.mark.parametrize("code,rotary", [(orc.BF16, 0), (orc.F16, 0), (orc.F32, 0),
                                         (orc.BF16, 64)])
def test_rope_append_matches_rope_then_store(ctx, code, rotary):
    """Qwen3-0.6B KV rows (8 heads x 128, theta 1e6) at positions up to 16 K,
    scattered through a permuted table; full width (the 128-bit path for
    16-bit rows) and a partial rotary width (the per-pair path)."""
    print(f"rope_append dtype {code} rotary {rotary}", flush=True)
    rng = orc.Mt64(17 + code)
    H, D, bs, B = 8, 128, 16, 96
    F = H * D
    rows = 300
    positions = [rng.uniform_int(0, 16383) for _ in range(rows - 4)] + [0, 1, 4095, 16383]
    perm = rng.permutation(B * bs)  # distinct slots, any order
    slots = perm[:rows]
    k = rng.normal(rows * F, code).reshape(rows, F)
    v = rng.normal(rows * F, code).reshape(rows, F)
    q = rng.normal(rows * 16 * D, code).reshape(rows, 16 * D)

    pool, kd, vd = new_pool(ctx, (2, B, bs, H, D), code, fill=0.0)
    # rope and append read only positions and slots; one 1024-entry table
    # (valid page ids, repeated) covers every position
    table = np.arange(1024) % B
    pool.upload(table, [0] * rows, [1024] * rows, positions, slots)
    pool.rope_append(1, to_dev(k, code), to_dev(v, code), 1e6, rotary)
    ctx.sync()
    got_k, got_v = to_host(kd, code), to_host(vd, code)

    # oracle: rope the key rows, then store_kv
    rk = orc.rope(k, code, H, positions, 1e6, rotary)
    kc = np.zeros_like(got_k)
    vc = np.zeros_like(got_v)
    orc.store_kv(kc, vc, rk, v, slots, 1, B * bs)
    assert np.array_equal(got_v, vc), "values must land bit-exact"
    if code == orc.F32:
        assert_close(got_k, kc, atol=1e-5, rtol=1e-5, what="rotated keys (f32)")
    else:
        d = ulps(got_k, kc, code)
        assert d.max() <= 1, f"rotated keys off by {d.max()} ulp"
        assert_close(orc.to_f32(got_k, code), orc.to_f32(kc, code), what="rotated keys")

    # the fused launch equals ckv_rope followed by ckv_append, bit for bit
    pool2, kd2, vd2 = new_pool(ctx, (2, B, bs, H, D), code, fill=0.0)
    pool2.upload(table, [0] * rows, [1024] * rows, positions, slots)
    kr = to_dev(k, code)
    pool2.rope(kr, kr, H, 1e6, rotary)
    pool2.append(1, kr, to_dev(v, code))
    ctx.sync()
    assert np.array_equal(to_host(kd2, code), got_k)
    assert np.array_equal(to_host(vd2, code), got_v)

    # queries: 16 heads through ckv_rope against the oracle
    qd = to_dev(q, code)
    qo = torch.empty_like(qd)
    pool.rope(qd, qo, 16, 1e6, rotary)
    ctx.sync()
    rq = orc.rope(q, code, 16, positions, 1e6, rotary)
    if code == orc.F32:
        assert_close(to_host(qo, code), rq, atol=1e-5, rtol=1e-5, what="rotated queries (f32)")
    else:
        assert ulps(to_host(qo, code), rq, code).max() <= 1
    pool.close()
    pool2.close()


def gated_f32(expected, gate_bits, code):
    g = orc.to_f32(gate_bits, code).astype(np.float64) if code != orc.F32 else gate_bits
    return expected * (1.0 / (1.0 + np.exp(-np.asarray(g, np.float64))))


def decode_rows(rng, code, batch, H, Hq, bs=16, D=128):
    """Decode rows over permuted pages (the new token is each row's last),
    including rows of 1, 16 and 17 tokens."""
    lengths = [1, 16, 17] + [rng.uniform_int(1, 3000) for _ in range(batch - 3)]
    pages = [-(-n // bs) for n in lengths]
    blocks = sum(pages) + 5
    perm = rng.permutation(blocks)
    tables, at = [], 0
    for p in pages:
        tables.append(perm[at:at + p])
        at += p
    F = H * D
    case = dict(
        geom=(1, blocks, bs, H, D), flat=np.concatenate(tables),
        offsets=np.cumsum([0] + pages[:-1]), pages=pages,
        positions=[n - 1 for n in lengths],
        kc=rng.normal(blocks * bs * F, code), vc=rng.normal(blocks * bs * F, code),
        q=rng.normal(batch * Hq * D, code).reshape(batch, Hq * D),
        kn=rng.normal(batch * F, code).reshape(batch, F),
        vn=rng.normal(batch * F, code).reshape(batch, F))
    case["slots"] = [orc.slot(t, p, bs) for t, p in zip(tables, case["positions"])]
    return case


@pytest.mark.parametrize("code,group,rotary,gated,split", [
    (orc.BF16, 2, 0, False, None), (orc.F16, 2, 0, False, None), (orc.BF16, 1, 64, False, None),
    (orc.BF16, 8, 32, False, None), (orc.BF16, 2, 0, True, None), (orc.F16, 4, 16, True, None),
    (orc.BF16, 2, 48, False, None), (orc.F32, 2, 0, True, None), (orc.BF16, 2, 0, True, "2"),
    (orc.F16, 4, 32, False, "3"), (orc.BF16, 2, 0, True, "b6"), (orc.F16, 1, 64, False, "b2")])
def test_rope_append_decode_equals_unfused_sequence(ctx, code, group, rotary, gated, split,
                                                   monkeypatch):
    """ckv_rope_append_decode (the fused decode kernel rotating queries and the
    new keys in registers; rotary 48 and f32 take the unfused form) against
    ckv_rope + ckv_rope_append + the attention, and against the oracle
    (rope_f32, store_kv, paged attention, gate). Values land bit-exact; a
    rotated 16-bit element may differ by one unit in the last place between the
    two kernels that rotate it (each is within one of the oracle), so rotated
    keys are compared within one ulp and outputs within the attention tolerance
    (the unfused form's own outputs are compared bit for bit: same kernels)."""
    print(f"rope_append_decode dtype {code} group {group} rotary {rotary} gated {gated} "
          f"split {split}", flush=True)
    # rows cut into chunks of `split` pages, or dealt out a few pages to a
    # workgroup ("b"): the chunk that merges applies the gate
    force_plan(monkeypatch, split)
    rng = orc.Mt64(60 + 7 * group + code + rotary + gated)
    H = 8 if group <= 2 else 2
    Hq = H * group
    D, batch, theta = 128, 24, 1e6
    c = decode_rows(rng, code, batch, H, Hq)
    gate = rng.normal(batch * Hq * D, code).reshape(batch, Hq * D) if gated else None
    scale = float(np.float32(1 / math.sqrt(D)))
    outs, caches = [], []
    for fused in (True, False):
        pool, kd, vd = new_pool(ctx, c["geom"], code)
        kd.copy_(to_dev(c["kc"], code))
        vd.copy_(to_dev(c["vc"], code))
        pool.upload(c["flat"], c["offsets"], c["pages"], c["positions"], c["slots"])
        qd, knd, vnd = to_dev(c["q"], code), to_dev(c["kn"], code), to_dev(c["vn"], code)
        gd = to_dev(gate, code) if gated else None
        out = torch.full((batch, Hq * D), float("nan"), dtype=qd.dtype, device="cuda")
        if fused:
            pool.rope_append_decode(0, knd, vnd, qd, Hq, scale, theta, out, rotary, gd)
        else:
            qr = torch.empty_like(qd)
            pool.rope(qd, qr, Hq, theta, rotary)
            pool.rope_append(0, knd, vnd, theta, rotary)
            if gated:
                pool.attention_gated(0, qr, Hq, scale, gd, out)
            else:
                pool.attention(0, qr, Hq, scale, out)
        ctx.sync()
        assert np.array_equal(to_host(qd, code), c["q"]), "queries must not be modified"
        assert np.array_equal(to_host(knd, code), c["kn"]), "keys must not be modified"
        outs.append(to_host(out, code))
        caches.append((to_host(kd, code), to_host(vd, code)))
        pool.close()
    assert np.array_equal(caches[0][1], caches[1][1]), "values differ from ckv_rope_append"
    fused_path = code != orc.F32 and rotary in (0, 16, 32, 64, 128)
    if fused_path:
        assert ulps(caches[0][0], caches[1][0], code).max() <= 1, "keys vs ckv_rope_append"
        assert_close(orc.to_f32(outs[0], code), orc.to_f32(outs[1], code),
                     what="fused vs unfused sequence")
    else:  # the unfused form runs the very same kernels
        assert np.array_equal(caches[0][0], caches[1][0])
        assert np.array_equal(outs[0], outs[1])

    rk = orc.rope(c["kn"], code, H, c["positions"], theta, rotary)
    want_k, want_v = c["kc"].copy(), c["vc"].copy()
    orc.store_kv(want_k, want_v, rk, c["vn"], c["slots"], 0, c["geom"][1] * 16)
    assert np.array_equal(caches[0][1], want_v), "values must land bit-exact"
    if code == orc.F32:
        assert_close(caches[0][0], want_k, atol=1e-5, rtol=1e-5, what="rotated keys (f32)")
    else:
        assert ulps(caches[0][0], want_k, code).max() <= 1
    rq = orc.rope(c["q"], code, Hq, c["positions"], theta, rotary)
    expected = orc.Attention(c["geom"], caches[0][0], caches[0][1], code, rq, code,
                             c["positions"], c["flat"], c["offsets"], c["pages"], Hq, 0,
                             scale).online_threads(8)
    if gated:
        expected = gated_f32(expected, gate, code)
    got = outs[0] if code == orc.F32 else orc.to_f32(outs[0], code)
    assert_close(got, expected, what="rope_append_decode vs oracle")


def test_rope_append_decode_validation_codes(ctx):
    D = 128
    pool, kd, vd = new_pool(ctx, (1, 4, 16, 2, D), orc.BF16)
    q = torch.zeros(2, 4 * D, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(2, 2 * D, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(ckv.CkvError) as e:
        pool.rope_append_decode(0, k, k, q, 4, 0.1, 1e4, out)
    assert e.value.code == 403  # nothing uploaded
    pool.upload([0, 1, 2, 3], [0, 2], [2, 2], [20, 5], slots=[20, 37])
    cases = [
        (dict(rows=1), "tensor_op.cache_slot_count_mismatch"),
        (dict(layer=1), "tensor_op.cache_layer_out_of_range"),
        (dict(q_heads=3), "tensor_op.invalid_kv_head_mapping"),
        (dict(theta=0.0), "tensor_op.invalid_rope_theta"),
        (dict(theta=float("nan")), "tensor_op.invalid_rope_theta"),
        (dict(rotary_dim=3), "tensor_op.invalid_head_dimension"),
        (dict(rotary_dim=256), "tensor_op.invalid_head_dimension"),
        (dict(gate=q), "tensor_op.unsupported_aliasing"),
    ]
    for kwargs, name in cases:
        args = dict(layer=0, q_heads=4, theta=1e4, rotary_dim=0, gate=None, rows=None)
        args.update(kwargs)
        with pytest.raises(ckv.CkvError) as e:
            pool.rope_append_decode(args["layer"], k, k, q, args["q_heads"], 0.1, args["theta"],
                                    out, args["rotary_dim"], args["gate"], args["rows"])
        assert e.value.name == name, kwargs
    pool.close()
