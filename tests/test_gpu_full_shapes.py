"""BASELINE configs 3 and 4 at their real shapes, checked against the CPU oracle
(the reference's own check of append + attention inside the layer loop,
tests/qwen_weights_test.cc:1045-1205, at the benchmark's sizes):

- config 3: a 28-layer pool of ~36,900 pages (67.7 GB of bf16 K/V), batch 128
  with contexts U[1024, 8192]; the fused append + decode on layers 0 and 27
  (byte offsets past 32 GB); appended rows bit-exact, outputs within
  2e-2 abs + 1e-2 rel of the oracle over K/V indexed out of the pool tensors
  through the tables (not read back by the library);
- config 4: 64 sequences x 512-row chunks over a shared 2,000- or 2,008-token
  prefix (the 2,008 tail page copied on write for every sequence) at layer 27
  of a 28-layer pool; the copied pages bit-exact, appended rows bit-exact,
  four sequences' 2,048 rows within tolerance of the oracle."""
import math

import numpy as np
import pytest
import torch

from chibillm_amd import ckv
from oracle import oracle as orc
from tests.gpu_util import assert_close, new_context, to_f32, to_host
from tests.test_gpu_parity import compact_oracle

pytestmark = pytest.mark.gpu

L, H, D, HQ, BS = 28, 8, 128, 16, 16
F = H * D
SCALE = float(np.float32(1 / math.sqrt(D)))
ORACLE_THREADS = 16


@pytest.fixture(scope="module")
def ctx():
    c = new_context()
    yield c
    c.sync()
    c.close()


def random_pool(ctx, blocks, seed):
    """A 28-layer bf16 pool over N(0,1) torch tensors, filled a GiB at a time."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    n = L * blocks * BS * F
    tensors = []
    for _ in range(2):
        t = torch.empty(n, dtype=torch.bfloat16, device="cuda")
        for i in range(0, n, 1 << 30):
            t[i:i + (1 << 30)].normal_(generator=gen)
        tensors.append(t)
    pool = ckv.Pool(ctx, L, blocks, BS, H, D, ckv.BF16, tensors[0], tensors[1])
    return pool, tensors[0], tensors[1], gen


def rows_from_pool(keys, values, blocks, layer, table, n_tokens):
    """A sequence's first n_tokens of one layer, indexed out of the pool's
    torch tensors through its block table (slot = table[p / 16] * 16 + p % 16):
    the library's own read-back path is not involved."""
    p = np.arange(n_tokens)
    slots = torch.from_numpy(table[p // BS].astype(np.int64) * BS + p % BS).to("cuda")
    k3 = keys.view(L, blocks * BS, F)
    v3 = values.view(L, blocks * BS, F)
    return to_host(k3[layer, slots], orc.BF16), to_host(v3[layer, slots], orc.BF16)


def test_config3_full_shape_append_decode_layers_0_and_27(ctx):
    rng = np.random.default_rng(0)
    lengths = [int(x) for x in rng.integers(1024, 8193, 128)]  # tokens cached before the step
    positions = lengths  # the new token's position: each row attends 0..len
    pages = [math.ceil((n + 1) / BS) for n in lengths]
    blocks = sum(pages) + 64
    perm = rng.permutation(blocks).astype(np.uint32)
    tables = np.split(perm[:sum(pages)], np.cumsum(pages)[:-1])
    flat = perm[:sum(pages)]
    offsets = np.cumsum([0] + pages[:-1]).astype(np.uint32)
    slots = [int(t[p // BS]) * BS + p % BS for t, p in zip(tables, positions)]
    print(f"config 3: {blocks} pages x {L} layers, {sum(lengths)} cached tokens", flush=True)
    pool, keys, values, gen = random_pool(ctx, blocks, 3)
    pool.upload(flat, offsets, pages, positions, slots)
    assert pool.decode_plan() == (0, 128, 0)  # whole rows: one workgroup per (row, kv head)
    k3 = keys.view(L, blocks * BS, F)
    v3 = values.view(L, blocks * BS, F)
    for layer in (0, L - 1):
        print(f"config 3: layer {layer}", flush=True)
        k_new = torch.randn(128, F, generator=gen, device="cuda").to(torch.bfloat16)
        v_new = torch.randn(128, F, generator=gen, device="cuda").to(torch.bfloat16)
        q = torch.randn(128, HQ * D, generator=gen, device="cuda").to(torch.bfloat16)
        out = torch.full((128, HQ * D), float("nan"), dtype=torch.bfloat16, device="cuda")
        pool.append_decode(layer, k_new, v_new, q, HQ, SCALE, out)
        ctx.sync()
        slot_idx = torch.tensor(slots, dtype=torch.long, device="cuda")
        assert torch.equal(k3[layer, slot_idx].view(torch.int16), k_new.view(torch.int16))
        assert torch.equal(v3[layer, slot_idx].view(torch.int16), v_new.view(torch.int16))
        # the oracle's K/V: each row's cached tokens indexed out of the pool
        # tensors, then the new token's row as drawn (appended bit-exact above)
        k_host, v_host = to_host(k_new, orc.BF16), to_host(v_new, orc.BF16)
        ks, vs = [], []
        for s in range(128):
            ck, cv = rows_from_pool(keys, values, blocks, layer, tables[s], positions[s])
            ks.append(np.concatenate([ck, k_host[s:s + 1]]))
            vs.append(np.concatenate([cv, v_host[s:s + 1]]))
        expected = compact_oracle((H, D), [p + 1 for p in positions], tables, ks, vs,
                                  to_host(q, orc.BF16), HQ, threads=ORACLE_THREADS)
        assert_close(to_f32(out), expected, what=f"config 3 layer {layer}")
        del ks, vs
    pool.close()
    del keys, values
    torch.cuda.empty_cache()


def prefill_oracle(seq_rows, tables, prefix, chunk, q_rows):
    """Oracle causal attention of each listed sequence's chunk rows over its
    prefix + chunk (a compact host pool, pages renumbered)."""
    n_tok = prefix + chunk
    n_pages = sum(len(t) for t in tables)
    kc = np.zeros(n_pages * BS * F, np.uint16)
    vc = np.zeros_like(kc)
    offsets, at = [], 0
    for (k, v), t in zip(seq_rows, tables):
        compact = np.arange(at, at + len(t), dtype=np.uint32)
        orc.store_kv(kc, vc, k, v, [int(compact[p // BS]) * BS + p % BS for p in range(n_tok)],
                     0, n_pages * BS)
        offsets.append(at)
        at += len(t)
    positions = [prefix + i for _ in tables for i in range(chunk)]
    row_offsets = [o for o in offsets for _ in range(chunk)]
    row_lengths = [len(t) for t in tables for _ in range(chunk)]
    att = orc.Attention((1, n_pages, BS, H, D), kc, vc, orc.BF16, q_rows, orc.BF16, positions,
                        np.arange(n_pages, dtype=np.uint32), row_offsets, row_lengths, HQ, 0,
                        SCALE)
    return att.online_threads(ORACLE_THREADS)


@pytest.mark.parametrize("prefix", [2000, 2008])
def test_config4_full_shape_prefill_layer_27(ctx, prefix):
    seqs, chunk = 64, 512
    full = prefix // BS
    partial = prefix % BS != 0
    prefix_pages = math.ceil(prefix / BS)
    own = math.ceil((prefix + chunk) / BS) - full
    blocks = prefix_pages + seqs * own + 16
    perm = np.random.default_rng(4).permutation(blocks).astype(np.uint32)
    prefix_table = perm[:prefix_pages]
    tables = [np.concatenate([prefix_table[:full],
                              perm[prefix_pages + s * own:prefix_pages + (s + 1) * own]])
              for s in range(seqs)]
    tlen = len(tables[0])
    print(f"config 4: prefix {prefix}, {blocks} pages x {L} layers", flush=True)
    pool, keys, values, gen = random_pool(ctx, blocks, 5)
    if partial:  # the shared tail page, copied on write into every sequence's own page
        src = [int(prefix_table[full])] * seqs
        dst = [int(t[full]) for t in tables]
        pool.copy_blocks(src, dst)
        ctx.sync()
        kp = keys.view(L, blocks, BS * F)
        vp = values.view(L, blocks, BS * F)
        d = torch.tensor(dst, dtype=torch.long, device="cuda")
        assert torch.equal(kp[:, d].view(torch.int16),
                           kp[:, src[0]:src[0] + 1].expand(-1, seqs, -1).view(torch.int16))
        assert torch.equal(vp[:, d].view(torch.int16),
                           vp[:, src[0]:src[0] + 1].expand(-1, seqs, -1).view(torch.int16))
    flat = np.concatenate(tables)
    positions = np.tile(np.arange(prefix, prefix + chunk, dtype=np.uint32), seqs)
    offsets = np.repeat(np.arange(seqs, dtype=np.uint32) * tlen, chunk)
    slots = [int(t[p // BS]) * BS + p % BS for t in tables for p in range(prefix, prefix + chunk)]
    rows = seqs * chunk
    pool.upload(flat, offsets, np.full(rows, tlen, np.uint32), positions, slots)
    layer = L - 1
    k_new = torch.randn(rows, F, generator=gen, device="cuda").to(torch.bfloat16)
    v_new = torch.randn(rows, F, generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn(rows, HQ * D, generator=gen, device="cuda").to(torch.bfloat16)
    out = torch.full((rows, HQ * D), float("nan"), dtype=torch.bfloat16, device="cuda")
    pool.append(layer, k_new, v_new)
    pool.prefill(layer, q, HQ, SCALE, out)
    ctx.sync()
    k3 = keys.view(L, blocks * BS, F)
    slot_idx = torch.tensor(slots, dtype=torch.long, device="cuda")
    assert torch.equal(k3[layer, slot_idx].view(torch.int16), k_new.view(torch.int16))
    assert torch.equal(values.view(L, blocks * BS, F)[layer, slot_idx].view(torch.int16),
                       v_new.view(torch.int16))
    checked = [0, 21, 42, 63]
    # the oracle's K/V: the prefix indexed out of the pool tensors through each
    # sequence's table (the copied tail page included), the chunk as drawn
    kn = to_host(k_new, orc.BF16).reshape(seqs, chunk, F)
    vn = to_host(v_new, orc.BF16).reshape(seqs, chunk, F)
    gathered = []
    for s in checked:
        pk, pv = rows_from_pool(keys, values, blocks, layer, tables[s], prefix)
        gathered.append((np.concatenate([pk, kn[s]]), np.concatenate([pv, vn[s]])))
    q_host = to_host(q, orc.BF16).reshape(seqs, chunk, HQ * D)
    expected = prefill_oracle(gathered, [tables[s] for s in checked], prefix, chunk,
                              np.concatenate([q_host[s] for s in checked]))
    got = to_f32(out).reshape(seqs, chunk, HQ * D)
    assert_close(np.concatenate([got[s] for s in checked]), expected,
                 what=f"config 4 prefix {prefix}, sequences {checked}")
    pool.close()
    del keys, values
    torch.cuda.empty_cache()
