"""Prefix checkpoints in host memory (ckv_checkpoint_export / ckv_checkpoint_import):
the packed [layer, token, kv_head, feature] layout of metal_kv_cache::checkpoint
(src/metal/metal_kv_cache.cc:14-35, :225-253) written to and read from host
buffers. Bit-exact: against the reference's checkpoint known answer
(tests/metal_kv_cache_test.cc:103-142), against the oracle's copy_prefix, and
against ckv_checkpoint_pack of the same pages."""
import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import new_context, new_pool, to_dev, to_f32, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def test_export_import_known_answer_pageable(ctx):
    # tests/metal_kv_cache_test.cc:103-142 through host memory: pages {2, 0},
    # 5 tokens, restored into pages {0, 1}
    geom = (2, 3, 4, 2, 8)
    pool, keys, values = new_pool(ctx, geom, orc.F32)
    k = np.arange(1, 385, dtype=np.float32)
    v = np.arange(1001, 1385, dtype=np.float32)
    keys.copy_(torch.from_numpy(k))
    values.copy_(torch.from_numpy(v))
    hk = np.zeros(2 * 5 * 16, np.float32)
    hv = np.zeros_like(hk)
    pool.checkpoint_export([2, 0], 5, hk, hv)
    ctx.sync()
    for layer in range(2):
        for token in range(5):
            orig = layer * 192 + [2, 0][token // 4] * 64 + (token % 4) * 16
            row = (layer * 5 + token) * 16
            assert np.array_equal(hk[row:row + 16], k[orig:orig + 16])
            assert np.array_equal(hv[row:row + 16], v[orig:orig + 16])
    keys.zero_()
    values.zero_()
    pool.checkpoint_import([0, 1], 5, hk, hv)
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
            pool.checkpoint_export(blocks, tokens, hk, hv)
        assert e.value.name == "state.invalid_reservation"
    with pytest.raises(ValueError):
        pool.checkpoint_export([2, 0], 5, hk[::2], hv)
    pool.close()


def test_export_in_layer_chunks_equals_device_pack_and_oracle(ctx):
    """28 layers x 4,000 tokens of Qwen3-0.6B KV (219 MiB per tensor): the
    transfer runs in 64 MiB layer groups through pinned memory; a partial
    tail page; pages in permuted order; import into other pages."""
    L, B, bs, H, D = 28, 520, 16, 8, 128
    F = H * D
    tokens = 4000
    pages = -(-tokens // bs)
    rng = orc.Mt64(31)
    perm = [int(x) for x in rng.permutation(B)]
    src, dst = perm[:pages], perm[pages:2 * pages]
    print(f"export/import {L} layers x {tokens} tokens", flush=True)
    torch.manual_seed(7)
    n = L * B * bs * F
    keys = torch.randn(n, device="cuda").to(torch.bfloat16)
    values = torch.randn(n, device="cuda").to(torch.bfloat16)
    pool = ckv.Pool(ctx, L, B, bs, H, D, ckv.BF16, keys, values)
    packed = L * tokens * F
    hk = ctx.host_alloc(packed * 2).view(np.uint16)
    hv = ctx.host_alloc(packed * 2).view(np.uint16)
    pool.checkpoint_export(src, tokens, hk, hv)
    dk = torch.empty(packed, dtype=torch.bfloat16, device="cuda")
    dv = torch.empty_like(dk)
    pool.checkpoint_pack(src, tokens, dk, dv)
    ctx.sync()
    assert np.array_equal(hk, to_host(dk, orc.BF16)), "export != device pack (keys)"
    assert np.array_equal(hv, to_host(dv, orc.BF16)), "export != device pack (values)"
    kc = to_host(keys, orc.BF16)
    expected = np.zeros(packed, np.uint16)
    orc.copy_prefix(kc, expected, src, (L, B, bs, H, D), tokens, False)
    assert np.array_equal(hk, expected), "export != oracle copy_prefix"

    before_k = kc.copy()
    before_v = to_host(values, orc.BF16)
    pool.checkpoint_import(dst, tokens, hk, hv)
    ctx.sync()
    after_k, after_v = to_host(keys, orc.BF16), to_host(values, orc.BF16)
    want_k, want_v = before_k.copy(), before_v.copy()
    orc.copy_prefix(want_k, hk, dst, (L, B, bs, H, D), tokens, True)
    orc.copy_prefix(want_v, hv, dst, (L, B, bs, H, D), tokens, True)
    assert np.array_equal(after_k, want_k), "import != oracle restore (keys)"
    assert np.array_equal(after_v, want_v), "import != oracle restore (values)"
    ctx.host_free(hk.view(np.uint8))
    ctx.host_free(hv.view(np.uint8))
    pool.close()
