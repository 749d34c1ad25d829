"""The attention output's consumer: the Qwen3.5 sigmoid gate
(src/qwen/qwen_layer.cc:183-206: split_heads -> paged_attention ->
sigmoid_mul(gate, attended, attended)).

ckv_sigmoid_mul is checked against the reference's known answer
(tests/tensor_ops_test.cc:513-539) and the oracle (within one unit in the last
place for 16-bit storage). The gated attention forms (the gate applied in the
decode, split-K merge and MFMA prefill epilogues) are checked against the
oracle's attention followed by the gate in float, within 2e-2 abs + 1e-2 rel,
and against the unfused pair (attention, then ckv_sigmoid_mul)."""
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import (assert_close, force_plan, new_context, new_pool, to_dev, to_f32,
                            to_host, torch_dtype)

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def gate_f32(expected, gate_bits, code):
    g = orc.to_f32(gate_bits, code).astype(np.float64) if code != orc.F32 else gate_bits
    return expected * (1.0 / (1.0 + np.exp(-np.asarray(g, np.float64))))


def ulps(a, b):
    a = np.asarray(a, np.uint16).astype(np.int32)
    b = np.asarray(b, np.uint16).astype(np.int32)
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


def test_sigmoid_mul_known_answer_and_oracle(ctx):
    # tests/tensor_ops_test.cc:513-539, in place as the reference calls it
    gate = torch.tensor([[0, 1, -1, 2], [-1000, 1000, 0, -2]], dtype=torch.float32, device="cuda")
    query = torch.arange(1, 9, dtype=torch.float32, device="cuda").reshape(2, 4)
    ctx.sigmoid_mul(gate, query, query)
    ctx.sync()
    expected = [0.5, 2 / (1 + math.exp(-1)), 3 / (1 + math.exp(1)), 4 / (1 + math.exp(-2)),
                0.0, 6.0, 3.5, 8 / (1 + math.exp(2))]
    got = to_f32(query).ravel()
    assert np.allclose(got, expected, rtol=1e-5, atol=0)
    assert got[4] == 0.0 and got[5] == 6.0
    rng = orc.Mt64(3)
    # 16-byte vectors (n a multiple of 8), a scalar tail (n % 8 == 3), and views one
    # element off 16-byte alignment (the per-element kernel)
    for code in (orc.BF16, orc.F16):
        for n, off in ((5000, 0), (5003, 0), (4999, 1)):
            g = orc.from_f32(4 * orc.to_f32(rng.normal(n + off, code), code), code)
            x = rng.normal(n + off, code)
            out = torch.empty_like(to_dev(x, code))[off:]
            ctx.sigmoid_mul(to_dev(g, code)[off:], to_dev(x, code)[off:], out)
            ctx.sync()
            got = to_host(out, code)
            assert ulps(got, orc.sigmoid_mul(g[off:], x[off:], code)).max() <= 1, (code, n, off)
    for n, off in ((4003, 0), (4001, 1)):  # f32: 4 a vector, and unaligned
        g = 4 * rng.normal(n + off, orc.F32).astype(np.float32)
        x = rng.normal(n + off, orc.F32).astype(np.float32)
        gd, xd = torch.from_numpy(g).cuda()[off:], torch.from_numpy(x).cuda()[off:]
        out = torch.empty_like(xd)
        ctx.sigmoid_mul(gd, xd, out)
        ctx.sync()
        ref = x[off:] / (1 + np.exp(-g[off:].astype(np.float64)))
        assert np.allclose(out.cpu().numpy(), ref, rtol=4e-6, atol=1e-30), (n, off)
    with pytest.raises(ckv.CkvError) as e:
        ctx.sigmoid_mul(gate, query, query, dtype=7)
    assert e.value.name == "tensor_op.unsupported_dtype"


def decode_case(seed, batch=24):
    rng = orc.Mt64(seed)
    lengths = [rng.uniform_int(1, 3000) for _ in range(batch)]
    pages = [-(-n // 16) for n in lengths]
    blocks = sum(pages) + 5
    perm = rng.permutation(blocks)
    tables, at = [], 0
    for p in pages:
        tables.append(perm[at:at + p])
        at += p
    return rng, lengths, tables, blocks


def shifted(t, aligned):
    """t itself, or a copy one element past a 16-byte boundary."""
    if aligned:
        return t
    base = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    view = base[1:1 + t.numel()].view(t.shape)
    view.copy_(t)
    assert view.data_ptr() % 16 != 0
    return view


@pytest.mark.parametrize("aligned", [True, False])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16, orc.F32])
def test_gated_decode_matches_oracle_and_unfused(ctx, code, aligned):
    """Every pool dtype through the fast decode kernel's gated epilogue, and
    through the generic split-K path with the merge (misaligned queries and
    output: the gate in both of its epilogues)."""
    print(f"gated decode dtype {code} aligned {aligned}", flush=True)
    rng, lengths, tables, blocks = decode_case(11 + code)
    H, Hq = 8, 16
    F = H * D
    geom = (1, blocks, 16, H, D)
    kc = rng.normal(blocks * 16 * F, code)
    vc = rng.normal(blocks * 16 * F, code)
    rows = len(lengths)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    gate = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    scale = float(np.float32(1 / math.sqrt(D)))
    pool, kd, vd = new_pool(ctx, geom, code)
    kd.copy_(to_dev(kc, code))
    vd.copy_(to_dev(vc, code))
    pool.upload(flat, offsets, [len(t) for t in tables], positions)
    qd, gd = shifted(to_dev(q, code), aligned), shifted(to_dev(gate, code), aligned)
    gated = shifted(torch.full_like(qd, float("nan")), aligned)
    pool.attention_gated(0, qd, Hq, scale, gd, gated)
    plain = shifted(torch.full_like(qd, float("nan")), aligned)
    pool.attention(0, qd, Hq, scale, plain)
    unfused = torch.empty_like(plain)
    ctx.sigmoid_mul(gd, plain, unfused)
    ctx.sync()
    expected = orc.Attention(geom, kc, vc, code, q, code, positions, flat, offsets,
                             [len(t) for t in tables], Hq, 0, scale).online_threads(8)
    want = gate_f32(expected, gate, code)
    assert_close(to_f32(gated), want, what="gated decode vs oracle")
    assert_close(to_f32(gated), to_f32(unfused), what="fused gate vs unfused")
    pool.close()


@pytest.mark.parametrize("group,code", [(2, orc.BF16), (8, orc.BF16), (2, orc.F32), (8, orc.F32)])
def test_gated_prefill_tiles(ctx, group, code):
    """Ragged tiles through the MFMA prefill kernels' gated epilogues (bf16
    and f32 pages)."""
    print(f"gated prefill group {group} dtype {code}", flush=True)
    rng = orc.Mt64(40 + group)
    H = 2
    Hq = H * group
    F = H * D
    spans = [(0, 40), (5, 300), (1000, 64), (700, 1), (16, 257)]
    ends = [s + n for s, n in spans]
    pages = [-(-n // 16) for n in ends]
    blocks = sum(pages) + 3
    perm = rng.permutation(blocks)
    geom = (1, blocks, 16, H, D)
    kc = rng.normal(blocks * 16 * F, code)
    vc = rng.normal(blocks * 16 * F, code)
    tables, at = [], 0
    for p in pages:
        tables.append(perm[at:at + p])
        at += p
    flat = np.concatenate(tables)
    positions, offsets, lengths, at = [], [], [], 0
    for (start, n), t in zip(spans, tables):
        positions += list(range(start, start + n))
        offsets += [at] * n
        lengths += [len(t)] * n
        at += len(t)
    rows = len(positions)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    gate = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    scale = float(np.float32(1 / math.sqrt(D)))
    pool, kd, vd = new_pool(ctx, geom, code)
    kd.copy_(to_dev(kc, code))
    vd.copy_(to_dev(vc, code))
    pool.upload(flat, offsets, lengths, positions)
    qd, gd = to_dev(q, code), to_dev(gate, code)
    gated = torch.full_like(qd, float("nan"))
    pool.attention_gated(0, qd, Hq, scale, gd, gated)  # shared tiles: the prefill kernel
    ctx.sync()
    expected = orc.Attention(geom, kc, vc, code, q, code, positions, flat, offsets, lengths, Hq,
                             0, scale).online_threads(8)
    assert_close(to_f32(gated), gate_f32(expected, gate, code), what="gated prefill vs oracle")
    pool.close()


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
@pytest.mark.parametrize("split", [None, "3", "b5"])
def test_append_decode_gated_equals_fused_pair(ctx, split, code, monkeypatch):
    """The decode step's fused append + attention with the gate, bf16 and f32
    pages: pages bit-exact with ckv_append_decode, output within tolerance of
    the oracle; also with every row cut into chunks of 3 pages and with the
    batch dealt out 5 pages to a workgroup (the gate applied by the chunk that
    merges)."""
    print(f"append_decode_gated dtype {code} split {split}", flush=True)
    force_plan(monkeypatch, split)
    rng, lengths, tables, blocks = decode_case(5, batch=16)
    H, Hq = 8, 16
    F = H * D
    geom = (1, blocks, 16, H, D)
    kc = rng.normal(blocks * 16 * F, code)
    vc = rng.normal(blocks * 16 * F, code)
    rows = len(lengths)
    q = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    gate = rng.normal(rows * Hq * D, code).reshape(rows, Hq * D)
    k_new = rng.normal(rows * F, code).reshape(rows, F)
    v_new = rng.normal(rows * F, code).reshape(rows, F)
    flat = np.concatenate(tables)
    offsets = np.cumsum([0] + [len(t) for t in tables[:-1]])
    positions = [n - 1 for n in lengths]
    slots = [orc.slot(t, p, 16) for t, p in zip(tables, positions)]
    scale = float(np.float32(1 / math.sqrt(D)))
    outs, caches = [], []
    for gated in (True, False):
        pool, kd, vd = new_pool(ctx, geom, code)
        kd.copy_(to_dev(kc, code))
        vd.copy_(to_dev(vc, code))
        pool.upload(flat, offsets, [len(t) for t in tables], positions, slots)
        out = torch.full((rows, Hq * D), float("nan"), dtype=torch_dtype(code), device="cuda")
        if gated:
            pool.append_decode_gated(0, to_dev(k_new, code), to_dev(v_new, code),
                                     to_dev(q, code), Hq, scale, to_dev(gate, code), out)
        else:
            pool.append_decode(0, to_dev(k_new, code), to_dev(v_new, code), to_dev(q, code),
                               Hq, scale, out)
        ctx.sync()
        outs.append(to_f32(out))
        caches.append((to_host(kd, code), to_host(vd, code)))
        pool.close()
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])
    kc2, vc2 = caches[0]
    expected = orc.Attention(geom, kc2, vc2, code, q, code, positions, flat, offsets,
                             [len(t) for t in tables], Hq, 0, scale).online_threads(8)
    assert_close(outs[0], gate_f32(expected, gate, code), what="append_decode_gated vs oracle")
    assert_close(outs[1], expected, what="append_decode vs oracle")


def test_gate_validation_codes(ctx):
    pool, kd, vd = new_pool(ctx, (1, 4, 16, 2, D), orc.BF16)
    torch.manual_seed(1)
    kd.copy_(torch.randn(kd.numel(), device="cuda").to(torch.bfloat16))
    vd.copy_(torch.randn(vd.numel(), device="cuda").to(torch.bfloat16))
    pool.upload([0, 1], [0], [2], [20])
    q = torch.zeros(1, 4 * D, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(ckv.CkvError) as e:
        pool.attention_gated(0, q, 4, 0.1, None, out)
    assert e.value.code == 400  # the gate is required
    with pytest.raises(ckv.CkvError) as e:
        pool.attention_gated(0, q, 4, 0.1, out, out)
    assert e.value.name == "tensor_op.unsupported_aliasing"
    with pytest.raises(ckv.CkvError) as e:
        pool.attention_gated(0, q, 4, 0.1, q, out)
    assert e.value.name == "tensor_op.unsupported_aliasing"
    g = torch.zeros_like(q)
    with pytest.raises(ckv.CkvError) as e:  # the attention checks follow
        pool.attention_gated(0, q, 3, 0.1, g, out)
    assert e.value.name == "tensor_op.invalid_kv_head_mapping"
    q.copy_(torch.randn(q.shape, device="cuda").to(torch.bfloat16))
    pool.attention_gated(0, q, 4, 0.1, g, out)  # sigmoid(0) = 1/2: half the attention, exactly
    plain = torch.empty_like(q)
    pool.attention(0, q, 4, 0.1, plain)
    ctx.sync()
    assert np.array_equal(to_f32(out), to_f32(plain) * 0.5)
    pool.close()
