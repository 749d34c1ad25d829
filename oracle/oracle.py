"""ctypes view of liboracle.so, the CPU oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, as the checker. The product package
(chibillm_amd) never imports this module.

Every function mirrors one C function of oracle.h, which cites the reference
lines it restates. Arrays are numpy; 16-bit element types travel as uint16 bit
patterns, f32 as float32.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

F32, BF16, F16 = 0, 1, 2
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_size_t = C.c_size_t
_u16 = C.c_uint16
_u32p = C.POINTER(C.c_uint32)
_vp = C.c_void_p


class Geometry(C.Structure):
    _fields_ = [("layers", _size_t), ("blocks", _size_t), ("block_size", _size_t),
                ("kv_heads", _size_t), ("head_dim", _size_t)]


class _AttnArgs(C.Structure):
    _fields_ = [("g", C.POINTER(Geometry)), ("key_cache", _vp), ("value_cache", _vp),
                ("cache_dtype", C.c_int), ("queries", _vp), ("q_dtype", C.c_int),
                ("positions", _u32p), ("table", _u32p), ("table_entries", _size_t),
                ("offsets", _u32p), ("lengths", _u32p), ("rows", _size_t),
                ("q_heads", _size_t), ("layer", _size_t), ("scale", C.c_float)]


class _Mt64(C.Structure):
    _fields_ = [("state", C.c_uint64 * 312), ("index", _size_t)]


def lib() -> C.CDLL:
    """Load liboracle.so (built by `make -C oracle`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing: run `make -C oracle`")
        L = C.CDLL(_LIB_PATH)
        L.orc_bf16_from_f32.restype = _u16
        L.orc_bf16_from_f32.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [_u16]
        L.orc_f16_from_f32.restype = _u16
        L.orc_f16_from_f32.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [_u16]
        L.orc_convert_from_f32.argtypes = [_vp, _vp, _size_t, C.c_int]
        L.orc_convert_to_f32.argtypes = [_vp, _vp, _size_t, C.c_int]
        L.orc_mt64_seed.argtypes = [C.POINTER(_Mt64), C.c_uint64]
        L.orc_mt64_next.restype = C.c_uint64
        L.orc_mt64_next.argtypes = [C.POINTER(_Mt64)]
        L.orc_uniform.restype = C.c_double
        L.orc_uniform.argtypes = [C.POINTER(_Mt64)]
        L.orc_fill_normal.argtypes = [C.POINTER(_Mt64), _vp, _size_t, C.c_int]
        L.orc_permutation.argtypes = [C.POINTER(_Mt64), _u32p, _size_t]
        L.orc_uniform_int.restype = C.c_uint64
        L.orc_uniform_int.argtypes = [C.POINTER(_Mt64), C.c_uint64, C.c_uint64]
        L.orc_bm_make.argtypes = [_size_t, _size_t, _size_t, C.POINTER(_vp)]
        L.orc_bm_destroy.argtypes = [_vp]
        L.orc_bm_reserve.argtypes = [_vp, _size_t, _size_t]
        L.orc_bm_release.argtypes = [_vp, _size_t]
        L.orc_bm_free_count.restype = _size_t
        L.orc_bm_free_count.argtypes = [_vp]
        L.orc_bm_table.restype = _size_t
        L.orc_bm_table.argtypes = [_vp, _size_t, _u32p, _size_t]
        L.orc_slot.argtypes = [_u32p, _size_t, C.c_uint32, C.c_uint32, _u32p]
        _szp = C.POINTER(_size_t)
        L.orc_prepare_paged_batch.argtypes = [_size_t, _u32p, _u32p, _szp, _u32p, _u32p,
                                              _size_t, _size_t, _size_t, _u32p, _u32p, _u32p,
                                              _u32p]
        L.orc_decode_step_host.argtypes = [_vp, _size_t, _u32p, _u32p, _szp, _u32p, _u32p,
                                           _u32p, _u32p, _u32p, _u32p, _size_t, _size_t]
        L.orc_element_offset.argtypes = [C.POINTER(Geometry), _size_t, _size_t, _size_t,
                                         _size_t, _size_t, C.POINTER(_size_t)]
        L.orc_store_kv.argtypes = [_vp, _vp, _vp, _vp, _u32p, _size_t, _size_t, _size_t,
                                   _size_t, _size_t]
        L.orc_gather.argtypes = [_vp, _vp, _u32p, _size_t, _size_t, _size_t, _size_t,
                                 _size_t, _size_t, _vp, _vp]
        for name in ("orc_attention_online", "orc_attention_reference"):
            getattr(L, name).argtypes = [C.POINTER(_AttnArgs), _vp]
        L.orc_attention_split.argtypes = [C.POINTER(_AttnArgs), _size_t, _vp]
        L.orc_attention_prefill_tiles.argtypes = [C.POINTER(_AttnArgs), _u32p, _u32p,
                                                  _size_t, _vp]
        L.orc_attention_online_threads.argtypes = [C.POINTER(_AttnArgs), _vp, C.c_int]
        L.orc_query_tiles.restype = _size_t
        L.orc_query_tiles.argtypes = [_u32p, _u32p, _u32p, _size_t, _u32p, _u32p,
                                      C.POINTER(C.c_int)]
        L.orc_copy_prefix.argtypes = [_vp, _vp, _u32p, C.POINTER(Geometry), _size_t, _size_t,
                                      C.c_int]
        L.orc_copy_blocks.argtypes = [_vp, _vp, C.POINTER(Geometry), _u32p, _u32p, _size_t,
                                      _size_t]
        L.orc_rope_frequencies.argtypes = [C.c_float, _size_t, _vp]
        L.orc_sigmoid_mul.argtypes = [_vp, _vp, _vp, _size_t, C.c_int]
        L.orc_sigmoid_mul.restype = None
        L.orc_rope.argtypes = [_vp, _vp, C.c_int, _size_t, _size_t, _size_t, _u32p, C.c_float,
                               _size_t]
        _lib = L
    return _lib


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


def _p32(a: np.ndarray):
    return a.ctypes.data_as(_u32p)


def _np_dtype(dtype: int):
    return np.float32 if dtype == F32 else np.uint16


# ---- conversions -----------------------------------------------------------

def from_f32(x, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=_np_dtype(dtype))
    lib().orc_convert_from_f32(x.ctypes.data, out.ctypes.data, x.size, dtype)
    return out


def to_f32(x, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=_np_dtype(dtype))
    out = np.empty(x.shape, dtype=np.float32)
    lib().orc_convert_to_f32(x.ctypes.data, out.ctypes.data, x.size, dtype)
    return out


# ---- seeded inputs -----------------------------------------------------------

class Mt64:
    """std::mt19937_64 with the normal / permutation draws of oracle.h."""

    def __init__(self, seed: int):
        self._s = _Mt64()
        lib().orc_mt64_seed(C.byref(self._s), seed)

    def next(self) -> int:
        return lib().orc_mt64_next(C.byref(self._s))

    def uniform(self) -> float:
        return lib().orc_uniform(C.byref(self._s))

    def normal(self, n: int, dtype: int = F32) -> np.ndarray:
        out = np.empty(n, dtype=_np_dtype(dtype))
        lib().orc_fill_normal(C.byref(self._s), out.ctypes.data, n, dtype)
        return out

    def permutation(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint32)
        lib().orc_permutation(C.byref(self._s), _p32(out), n)
        return out

    def uniform_int(self, lo: int, hi: int) -> int:
        return lib().orc_uniform_int(C.byref(self._s), lo, hi)


# ---- pages, slots, offsets ----------------------------------------------------

class BlockManager:
    """FIFO page allocator (src/block_manager.cc:5-64) over dense sequence ids."""

    def __init__(self, block_count: int, block_size: int, max_sequences: int = 64):
        h = _vp()
        status = lib().orc_bm_make(block_count, block_size, max_sequences, C.byref(h))
        if status:
            raise ValueError(["", "invalid_block_count", "invalid_block_size",
                              "too_many_blocks"][status])
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_bm_destroy(self._h)
            self._h = None

    def reserve(self, seq: int, tokens: int) -> str | None:
        status = lib().orc_bm_reserve(self._h, seq, tokens)
        return [None, "capacity_exhausted", "invalid_reservation"][status]

    def release(self, seq: int) -> None:
        lib().orc_bm_release(self._h, seq)

    def free_count(self) -> int:
        return lib().orc_bm_free_count(self._h)

    def table(self, seq: int) -> np.ndarray:
        n = lib().orc_bm_table(self._h, seq, None, 0)
        out = np.empty(n, dtype=np.uint32)
        lib().orc_bm_table(self._h, seq, _p32(out), n)
        return out


def slot(table, position: int, block_size: int) -> int | None:
    t = _u32(table)
    out = C.c_uint32()
    if lib().orc_slot(_p32(t), t.size, position, block_size, C.byref(out)):
        return None
    return out.value


def prepare_paged_batch(token_counts, tables, positions, max_positions: int,
                        block_count: int, block_size: int):
    """src/model_batch.cc:127-204: (flat table, slots, offsets, lengths), or None
    for inconsistent_batch. tables: one block table per item."""
    counts = _u32(token_counts)
    lens = _u32([len(t) for t in tables])
    flat_in = _u32(np.concatenate([np.asarray(t, np.uint32) for t in tables])
                   if len(tables) and lens.sum() else [])
    starts = np.ascontiguousarray(np.cumsum([0] + [len(t) for t in tables[:-1]]),
                                  dtype=np.uintp) if len(tables) else np.zeros(0, np.uintp)
    pos = _u32(positions)
    rows = int(counts.sum()) if counts.size else 0
    flat = np.zeros(max(int(lens.sum()), 1), np.uint32)
    slots, offsets, lengths = (np.zeros(max(rows, 1), np.uint32) for _ in range(3))
    status = lib().orc_prepare_paged_batch(
        counts.size, _p32(counts), _p32(flat_in), starts.ctypes.data_as(C.POINTER(_size_t)),
        _p32(lens), _p32(pos), max_positions, block_count, block_size, _p32(flat),
        _p32(slots), _p32(offsets), _p32(lengths))
    if status:
        return None
    return flat[:int(lens.sum())], slots[:rows], offsets[:rows], lengths[:rows]


class DecodeStepHost:
    """One decode step's host work for n sequences (orc_decode_step_host): the
    block_manager reservation of one more token per sequence, then
    prepare_paged_batch over one row per sequence. Buffers sized for
    max_pages pages per sequence."""

    def __init__(self, lengths, block_count: int, block_size: int, max_pages: int):
        n = len(lengths)
        self.bm = BlockManager(block_count, block_size, n)
        self.n, self.block_count, self.block_size = n, block_count, block_size
        self.lengths = _u32(lengths).copy()
        for s in range(n):  # the sequences' current tokens
            if self.bm.reserve(s, int(self.lengths[s])):
                raise ValueError("pool too small")
        cap = n * max_pages
        self.tables = np.zeros(cap, np.uint32)
        self.start = np.zeros(n, np.uintp)
        self.table_len, self.counts = np.zeros(n, np.uint32), np.zeros(n, np.uint32)
        self.flat = np.zeros(cap, np.uint32)
        self.slots, self.offsets, self.row_lengths = (np.zeros(n, np.uint32) for _ in range(3))

    def step(self) -> None:
        status = lib().orc_decode_step_host(
            self.bm._h, self.n, _p32(self.lengths), _p32(self.tables),
            self.start.ctypes.data_as(C.POINTER(_size_t)), _p32(self.table_len),
            _p32(self.counts), _p32(self.flat), _p32(self.slots), _p32(self.offsets),
            _p32(self.row_lengths), self.block_count, self.block_size)
        if status:
            raise RuntimeError("decode step host work failed")


def element_offset(geom: tuple, layer, block, token, head, feature):
    """Returns the offset, or the kv_cache_errc value as a negative int."""
    g = Geometry(*geom)
    out = _size_t()
    status = lib().orc_element_offset(C.byref(g), layer, block, token, head, feature,
                                      C.byref(out))
    return -status if status else out.value


# ---- append / gather / copies --------------------------------------------------

def store_kv(key_cache: np.ndarray, value_cache: np.ndarray, keys: np.ndarray,
             values: np.ndarray, slots, layer: int, slot_count: int) -> None:
    s = _u32(slots)
    rows, features = keys.shape
    lib().orc_store_kv(key_cache.ctypes.data, value_cache.ctypes.data,
                       np.ascontiguousarray(keys).ctypes.data,
                       np.ascontiguousarray(values).ctypes.data, _p32(s), rows, features,
                       layer, slot_count, keys.dtype.itemsize)


def gather(key_cache, value_cache, table, n_tokens: int, layer: int, slot_count: int,
           block_size: int, features: int):
    t = _u32(table)
    ok = np.empty((n_tokens, features), dtype=key_cache.dtype)
    ov = np.empty((n_tokens, features), dtype=key_cache.dtype)
    lib().orc_gather(key_cache.ctypes.data, value_cache.ctypes.data, _p32(t), n_tokens, layer,
                     slot_count, block_size, features, key_cache.dtype.itemsize,
                     ok.ctypes.data, ov.ctypes.data)
    return ok, ov


def copy_prefix(paged: np.ndarray, packed: np.ndarray, blocks, geom: tuple, tokens: int,
                restore: bool) -> None:
    b = _u32(blocks)
    g = Geometry(*geom)
    lib().orc_copy_prefix(paged.ctypes.data, packed.ctypes.data, _p32(b), C.byref(g), tokens,
                          paged.dtype.itemsize, 1 if restore else 0)


def copy_blocks(key_cache, value_cache, geom: tuple, src, dst) -> None:
    s, d = _u32(src), _u32(dst)
    g = Geometry(*geom)
    lib().orc_copy_blocks(key_cache.ctypes.data, value_cache.ctypes.data, C.byref(g), _p32(s),
                          _p32(d), s.size, key_cache.dtype.itemsize)


# ---- rotary position embedding ---------------------------------------------------

def sigmoid_mul(gate: np.ndarray, x: np.ndarray, dtype: int) -> np.ndarray:
    """sigmoid_mul (src/tensor/tensor_ops.cc:289-296): x * sigmoid(gate) in float,
    arrays of `dtype` (float32 or 16-bit bit patterns), rounded once."""
    g = np.ascontiguousarray(gate, dtype=_np_dtype(dtype))
    a = np.ascontiguousarray(x, dtype=_np_dtype(dtype))
    assert g.shape == a.shape
    out = np.empty_like(a)
    lib().orc_sigmoid_mul(g.ctypes.data, a.ctypes.data, out.ctypes.data, a.size, dtype)
    return out


def rope_frequencies(theta: float, rotary_dim: int) -> np.ndarray:
    out = np.empty(max(rotary_dim // 2, 1), dtype=np.float32)
    lib().orc_rope_frequencies(theta, rotary_dim, out.ctypes.data)
    return out[:rotary_dim // 2]


def rope(rows_in: np.ndarray, dtype: int, heads: int, positions, theta: float,
         rotary_dim: int = 0) -> np.ndarray:
    """rope_f32 on [rows, heads*head_dim] rows of `dtype` (float32 or 16-bit bit patterns)."""
    x = np.ascontiguousarray(rows_in)
    rows, width = x.shape
    out = np.empty_like(x)
    p = _u32(positions)
    if lib().orc_rope(x.ctypes.data, out.ctypes.data, dtype, rows, heads, width // heads,
                      _p32(p), theta, rotary_dim):
        raise ValueError("invalid rope arguments")
    return out


# ---- attention -------------------------------------------------------------------

class Attention:
    """Bundles one attention problem; arrays are kept alive by this object."""

    def __init__(self, geom: tuple, key_cache, value_cache, cache_dtype: int, queries,
                 q_dtype: int, positions, table, offsets, lengths, q_heads: int, layer: int,
                 scale: float):
        self.geom = Geometry(*geom)
        self.kc = np.ascontiguousarray(key_cache)
        self.vc = np.ascontiguousarray(value_cache)
        self.q = np.ascontiguousarray(queries)
        self.pos, self.tab = _u32(positions), _u32(table)
        self.off, self.len = _u32(offsets), _u32(lengths)
        self.rows, self.q_heads, self.D = self.pos.size, q_heads, geom[4]
        self.args = _AttnArgs(C.pointer(self.geom), self.kc.ctypes.data, self.vc.ctypes.data,
                              cache_dtype, self.q.ctypes.data, q_dtype, _p32(self.pos),
                              _p32(self.tab), self.tab.size, _p32(self.off), _p32(self.len),
                              self.rows, q_heads, layer, scale)

    def _out(self, dtype):
        return np.zeros((self.rows, self.q_heads * self.D), dtype=dtype)

    def online(self) -> np.ndarray:
        out = self._out(np.float32)
        if lib().orc_attention_online(C.byref(self.args), out.ctypes.data):
            raise ValueError("invalid attention metadata")
        return out

    def reference(self) -> np.ndarray:
        out = self._out(np.float64)
        if lib().orc_attention_reference(C.byref(self.args), out.ctypes.data):
            raise ValueError("invalid attention metadata")
        return out

    def split(self, chunk: int = 64) -> np.ndarray:
        out = self._out(np.float32)
        if lib().orc_attention_split(C.byref(self.args), chunk, out.ctypes.data):
            raise ValueError("invalid attention metadata")
        return out

    def prefill(self) -> np.ndarray:
        starts, lens, _ = query_tiles(self.pos, self.off, self.len)
        out = self._out(np.float32)
        if lib().orc_attention_prefill_tiles(C.byref(self.args), _p32(starts), _p32(lens),
                                             starts.size, out.ctypes.data):
            raise ValueError("invalid attention metadata")
        return out

    def online_threads(self, threads: int) -> np.ndarray:
        out = self._out(np.float32)
        if lib().orc_attention_online_threads(C.byref(self.args), out.ctypes.data, threads):
            raise ValueError("invalid attention metadata")
        return out


def query_tiles(positions, offsets, lengths):
    p, o, l = _u32(positions), _u32(offsets), _u32(lengths)
    starts = np.empty(max(p.size, 1), dtype=np.uint32)
    lens = np.empty(max(p.size, 1), dtype=np.uint32)
    shared = C.c_int()
    n = lib().orc_query_tiles(_p32(p), _p32(o), _p32(l), p.size, _p32(starts), _p32(lens),
                              C.byref(shared))
    return starts[:n].copy(), lens[:n].copy(), bool(shared.value)
