"""BASELINE config 1 inputs, drawn exactly as stated there.

One layer of Qwen3-0.6B KV (8 KV heads x head_dim 128, 16 q heads), fp16,
16-token pages from a FIFO page allocator of 107 pages (the page ids do not
depend on the pool size without releases). Sequences of 37/128/513/1000
tokens are appended token by token, round-robin: at step t every sequence
with length > t reserves t+1 tokens and draws its K row then its V row from
N(0,1) (mt19937_64, seed 0, Box-Muller; oracle.h). After the last step one Q
row per sequence is drawn (16 heads x 128) and one decode step runs at
position length-1 with scale 1/sqrt(128).
"""
import numpy as np

from oracle import oracle as orc

LENGTHS = (37, 128, 513, 1000)
GEOMETRY = (1, 107, 16, 8, 128)  # layers, blocks, block_size, kv_heads, head_dim
Q_HEADS = 16
DTYPE = orc.F16
SCALE = float(np.float32(1.0 / np.sqrt(128.0)))


def generate():
    L, B, bs, H, D = GEOMETRY
    F = H * D
    rng = orc.Mt64(0)
    pages = orc.BlockManager(B, bs)
    steps = []  # per step: (seq ids, positions, K rows, V rows, tables snapshot)
    for t in range(max(LENGTHS)):
        active = [s for s in range(len(LENGTHS)) if LENGTHS[s] > t]
        ks, vs = [], []
        for s in active:
            assert pages.reserve(s, t + 1) is None
            ks.append(rng.normal(F, DTYPE))
            vs.append(rng.normal(F, DTYPE))
        tables = [pages.table(s) for s in range(len(LENGTHS))]
        steps.append((active, t, np.stack(ks), np.stack(vs), tables))
    q = rng.normal(len(LENGTHS) * Q_HEADS * D, DTYPE).reshape(len(LENGTHS), Q_HEADS * D)
    tables = [pages.table(s) for s in range(len(LENGTHS))]
    return steps, q, tables


def step_metadata(tables, active, t):
    """Flat table, per-row offsets/lengths/positions and slots for one append step."""
    flat = np.concatenate(tables).astype(np.uint32)
    starts = np.cumsum([0] + [len(x) for x in tables[:-1]])
    offsets = [int(starts[s]) for s in active]
    lengths = [len(tables[s]) for s in active]
    positions = [t] * len(active)
    slots = [orc.slot(tables[s], t, GEOMETRY[2]) for s in active]
    return flat, offsets, lengths, positions, slots


def oracle_cache(steps):
    """The KV pool after every append, by the oracle's store_kv."""
    L, B, bs, H, D = GEOMETRY
    n = L * B * bs * H * D
    kc = np.zeros(n, np.uint16)
    vc = np.zeros(n, np.uint16)
    for active, t, ks, vs, tables in steps:
        _, _, _, _, slots = step_metadata(tables, active, t)
        orc.store_kv(kc, vc, ks, vs, slots, 0, B * bs)
    return kc, vc


def decode_metadata(tables):
    flat = np.concatenate(tables).astype(np.uint32)
    offsets = np.cumsum([0] + [len(x) for x in tables[:-1]]).astype(np.uint32)
    lengths = [len(x) for x in tables]
    positions = [n - 1 for n in LENGTHS]
    return flat, offsets, lengths, positions


def oracle_attention(kc, vc, q, tables):
    flat, offsets, lengths, positions = decode_metadata(tables)
    att = orc.Attention(GEOMETRY, kc, vc, DTYPE, q, DTYPE, positions, flat, offsets, lengths,
                        Q_HEADS, 0, SCALE)
    return att.online(), att.reference()
