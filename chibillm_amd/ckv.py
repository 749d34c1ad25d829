"""ctypes binding of libckv.so (include/ckv.h).

This is the Python-side FFI a host program would use for the paged KV-cache +
attention path; it mirrors the C ABI one-to-one. Device arrays are passed as
torch tensors (or raw device addresses); host metadata as numpy/sequence
arrays of u32. PyTorch only provides device memory and the stream.

There is no CPU fallback: if libckv.so is missing or the device is absent,
every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libckv.so")

F32, BF16, F16 = 0, 1, 2
_lib = None

_sz = C.c_size_t
_vp = C.c_void_p
_u32p = C.POINTER(C.c_uint32)
_i = C.c_int

# (name, restype, argtypes) for every declaration of include/ckv.h
_SIGNATURES = [
    ("ckv_abi_version", _i, []),
    ("ckv_error_name", C.c_char_p, [_i]),
    ("ckv_last_error", C.c_char_p, [_vp]),
    ("ckv_context_create", _i, [_i, C.POINTER(_vp)]),
    ("ckv_context_destroy", _i, [_vp]),
    ("ckv_context_set_stream", _i, [_vp, _vp]),
    ("ckv_context_stream", _vp, [_vp]),
    ("ckv_context_own_stream", _vp, [_vp]),
    ("ckv_sync", _i, [_vp]),
    ("ckv_device_alloc", _i, [_vp, _sz, C.POINTER(_vp)]),
    ("ckv_device_free", _i, [_vp, _vp]),
    ("ckv_host_alloc", _i, [_vp, _sz, C.POINTER(_vp)]),
    ("ckv_host_free", _i, [_vp, _vp]),
    ("ckv_copy_to_device", _i, [_vp, _vp, _vp, _sz]),
    ("ckv_copy_to_host", _i, [_vp, _vp, _vp, _sz]),
    ("ckv_profile_enable", _i, [_vp, _i]),
    ("ckv_profile_query", _i, [_vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    ("ckv_profile_reset", _i, [_vp]),
    ("ckv_pool_create", _i, [_vp, _sz, _sz, _sz, _sz, _sz, _i, C.POINTER(_vp)]),
    ("ckv_pool_wrap", _i, [_vp, _sz, _sz, _sz, _sz, _sz, _i, _vp, _vp, C.POINTER(_vp)]),
    ("ckv_pool_destroy", _i, [_vp]),
    ("ckv_pool_buffers", _i, [_vp, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_sz)]),
    ("ckv_element_offset", _i, [_vp, _sz, _sz, _sz, _sz, _sz, C.POINTER(_sz)]),
    ("ckv_tables_upload", _i, [_vp, _u32p, _sz, _u32p, _u32p, _u32p, _u32p, _sz]),
    ("ckv_tables_patch", _i, [_vp, _u32p, _u32p, _sz]),
    ("ckv_seq_tables_reserve", _i, [_vp, _sz, _sz]),
    ("ckv_seq_tables_update", _i, [_vp, _u32p, _u32p, _u32p, _sz, _u32p, _u32p, _sz]),
    ("ckv_batch_upload", _i, [_vp, _u32p, _u32p, _u32p, _sz, _i]),
    ("ckv_decode_plan", _i, [_vp, _u32p, _u32p, _u32p]),
    ("ckv_debug_allocations", _i, [_vp, C.POINTER(C.c_uint64)]),
    ("ckv_append", _i, [_vp, _sz, _vp, _vp, _sz]),
    ("ckv_gather", _i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp]),
    ("ckv_decode_attention", _i, [_vp, _sz, _vp, _sz, C.c_float, _vp, _sz]),
    ("ckv_append_decode", _i, [_vp, _sz, _vp, _vp, _vp, _sz, C.c_float, _vp, _sz]),
    ("ckv_append_decode_noalloc", _i, [_vp, _sz, _vp, _vp, _vp, _sz, C.c_float, _vp, _sz]),
    ("ckv_prefill_attention", _i, [_vp, _sz, _vp, _sz, C.c_float, _vp, _sz]),
    ("ckv_attention", _i, [_vp, _sz, _vp, _sz, C.c_float, _vp, _sz]),
    ("ckv_rope", _i, [_vp, _vp, _vp, _sz, C.c_float, _sz, _sz]),
    ("ckv_rope_append", _i, [_vp, _sz, _vp, _vp, C.c_float, _sz, _sz]),
    ("ckv_rope_append_decode", _i, [_vp, _sz, _vp, _vp, _vp, _sz, C.c_float, C.c_float, _sz,
                                    _vp, _vp, _sz]),
    ("ckv_copy_blocks", _i, [_vp, _u32p, _u32p, _sz]),
    ("ckv_checkpoint_pack", _i, [_vp, _u32p, _sz, _sz, _vp, _vp]),
    ("ckv_checkpoint_unpack", _i, [_vp, _u32p, _sz, _sz, _vp, _vp]),
    ("ckv_attention_gated", _i, [_vp, _sz, _vp, _sz, C.c_float, _vp, _vp, _sz]),
    ("ckv_append_decode_gated", _i, [_vp, _sz, _vp, _vp, _vp, _sz, C.c_float, _vp, _vp, _sz]),
    ("ckv_sigmoid_mul", _i, [_vp, _i, _vp, _vp, _vp, _sz]),
    ("ckv_checkpoint_export", _i, [_vp, _u32p, _sz, _sz, _vp, _vp]),
    ("ckv_checkpoint_import", _i, [_vp, _u32p, _sz, _sz, _vp, _vp]),
]
SYMBOLS = [name for name, _, _ in _SIGNATURES]


def load() -> C.CDLL:
    """Load libckv.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        lib = C.CDLL(LIB_PATH)
        for name, res, args in _SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class CkvError(RuntimeError):
    def __init__(self, code: int, detail: str = ""):
        self.code = code
        self.name = load().ckv_error_name(code).decode()
        super().__init__(f"{self.name} ({code})" + (f": {detail}" if detail else ""))


def error_name(code: int) -> str:
    return load().ckv_error_name(code).decode()


def _dtype_code(dtype) -> int:
    import torch
    table = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}
    if isinstance(dtype, int):
        return dtype
    return table[dtype]


def torch_dtype(code: int):
    import torch
    return {F32: torch.float32, BF16: torch.bfloat16, F16: torch.float16}[code]


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if not x.is_cuda:
        raise ValueError("device arrays must be GPU tensors")
    if not x.is_contiguous():
        raise ValueError("device arrays must be contiguous")
    return x.data_ptr()


def _host(a: np.ndarray) -> int:
    if not isinstance(a, np.ndarray) or not a.flags.c_contiguous or not a.flags.writeable:
        raise ValueError("host buffers must be writeable contiguous numpy arrays")
    return a.ctypes.data


def _u32(a) -> Optional[np.ndarray]:
    if a is None:
        return None
    return np.ascontiguousarray(np.asarray(a), dtype=np.uint32)


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(_u32p)


class Context:
    """A device and the stream ckv enqueues on (ckv_context)."""

    def __init__(self, device: int = 0, stream=None):
        lib = load()
        h = _vp()
        rc = lib.ckv_context_create(device, C.byref(h))
        if rc:
            raise CkvError(rc, "context creation")
        self.handle = h
        self.device = device
        if stream is not None:
            self.set_stream(stream)

    def check(self, rc: int) -> None:
        if rc:
            raise CkvError(rc, load().ckv_last_error(self.handle).decode())

    def set_stream(self, stream) -> None:
        """stream: a torch.cuda.Stream or a raw hipStream_t address; 0 / None is
        the null stream (torch's default stream)."""
        raw = getattr(stream, "cuda_stream", stream)
        self.check(load().ckv_context_set_stream(self.handle, raw or None))

    def own_stream(self) -> int:
        return load().ckv_context_own_stream(self.handle) or 0

    def sync(self) -> None:
        self.check(load().ckv_sync(self.handle))

    def allocations(self) -> int:
        """Device and pinned host allocations and frees the library has made on
        this context (ckv_debug_allocations)."""
        n = C.c_uint64()
        self.check(load().ckv_debug_allocations(self.handle, C.byref(n)))
        return n.value

    def host_alloc(self, nbytes: int) -> np.ndarray:
        """Pinned host memory (ckv_host_alloc) as a uint8 numpy array; freed by
        host_free (which waits for the stream) or when the context closes."""
        ptr = _vp()
        self.check(load().ckv_host_alloc(self.handle, nbytes, C.byref(ptr)))
        buf = (C.c_uint8 * nbytes).from_address(ptr.value)
        arr = np.frombuffer(buf, dtype=np.uint8)
        self._pinned = getattr(self, "_pinned", {})
        self._pinned[arr.ctypes.data] = ptr.value
        return arr

    def host_free(self, arr: np.ndarray) -> None:
        ptr = self._pinned.pop(arr.ctypes.data)
        self.check(load().ckv_host_free(self.handle, ptr))

    def sigmoid_mul(self, gate, inputs, output, dtype=None) -> None:
        """output = inputs * sigmoid(gate), elementwise (ckv_sigmoid_mul)."""
        code = _dtype_code(dtype if dtype is not None else inputs.dtype)
        self.check(load().ckv_sigmoid_mul(self.handle, code, _ptr(gate), _ptr(inputs),
                                          _ptr(output), inputs.numel()))

    def profile(self, enabled: bool = True) -> None:
        self.check(load().ckv_profile_enable(self.handle, 1 if enabled else 0))

    def profile_query(self, kernel: str):
        ms, n = C.c_double(), C.c_uint64()
        self.check(load().ckv_profile_query(self.handle, kernel.encode(), C.byref(ms),
                                            C.byref(n)))
        return ms.value, n.value

    def profile_reset(self) -> None:
        self.check(load().ckv_profile_reset(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            for ptr in getattr(self, "_pinned", {}).values():
                load().ckv_host_free(self.handle, ptr)
            self._pinned = {}
            load().ckv_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Pool:
    """Paged K/V tensors [layer, block, token, kv_head, feature] (ckv_pool)."""

    def __init__(self, ctx: Context, layers: int, blocks: int, block_size: int, kv_heads: int,
                 head_dim: int, dtype=BF16, keys=None, values=None):
        lib = load()
        self.ctx = ctx
        self.geometry = (layers, blocks, block_size, kv_heads, head_dim)
        self.dtype = _dtype_code(dtype)
        h = _vp()
        if keys is None:
            rc = lib.ckv_pool_create(ctx.handle, layers, blocks, block_size, kv_heads, head_dim,
                                     self.dtype, C.byref(h))
        else:
            rc = lib.ckv_pool_wrap(ctx.handle, layers, blocks, block_size, kv_heads, head_dim,
                                   self.dtype, _ptr(keys), _ptr(values), C.byref(h))
        ctx.check(rc)
        self.handle = h
        self._keep = (keys, values)

    @property
    def features(self) -> int:
        return self.geometry[3] * self.geometry[4]

    def buffers(self):
        k, v, n = _vp(), _vp(), _sz()
        self.ctx.check(load().ckv_pool_buffers(self.handle, C.byref(k), C.byref(v), C.byref(n)))
        return k.value, v.value, n.value

    def element_offset(self, layer, block, token, head, feature) -> int:
        out = _sz()
        rc = load().ckv_element_offset(self.handle, layer, block, token, head, feature,
                                       C.byref(out))
        if rc:
            raise CkvError(rc)
        return out.value

    def upload(self, table: Sequence[int], offsets, lengths, positions, slots=None) -> None:
        t, o, l, p, s = (_u32(table), _u32(offsets), _u32(lengths), _u32(positions),
                         _u32(slots))
        self.ctx.check(load().ckv_tables_upload(self.handle, _p(t), t.size, _p(o), _p(l), _p(p),
                                                _p(s), p.size))

    def patch(self, idx, val) -> None:
        i, v = _u32(idx), _u32(val)
        self.ctx.check(load().ckv_tables_patch(self.handle, _p(i), _p(v), i.size))

    def reserve_sequences(self, max_sequences: int, pages_per_sequence: int) -> None:
        """Device arena of per-sequence block tables (ckv_seq_tables_reserve)."""
        self.ctx.check(load().ckv_seq_tables_reserve(self.handle, max_sequences,
                                                     pages_per_sequence))

    def update_sequences(self, seq=(), index=(), block=(), len_seq=(), length=()) -> None:
        """entry (seq[i], index[i]) = block[i]; table length of len_seq[j] = length[j]."""
        s, i, b, ls, ln = (_u32(seq), _u32(index), _u32(block), _u32(len_seq), _u32(length))
        self.ctx.check(load().ckv_seq_tables_update(self.handle, _p(s), _p(i), _p(b), s.size,
                                                    _p(ls), _p(ln), ls.size))

    def upload_batch(self, seq, first_position, token_count, with_slots: bool = True) -> None:
        """Batch of items (sequence, first position, token count) over the
        sequence tables; rows are expanded on the device (ckv_batch_upload)."""
        s, f, c = _u32(seq), _u32(first_position), _u32(token_count)
        self.ctx.check(load().ckv_batch_upload(self.handle, _p(s), _p(f), _p(c), s.size,
                                               1 if with_slots else 0))

    def decode_plan(self):
        """(pages per chunk, work items, partial records) of the current batch's
        fast decode plan (ckv_decode_plan); pages per chunk 0 = one chunk per row."""
        span, items, records = C.c_uint32(), C.c_uint32(), C.c_uint32()
        self.ctx.check(load().ckv_decode_plan(self.handle, C.byref(span), C.byref(items),
                                              C.byref(records)))
        return span.value, items.value, records.value

    def append(self, layer: int, keys, values, rows: Optional[int] = None) -> None:
        rows = keys.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_append(self.handle, layer, _ptr(keys), _ptr(values), rows))

    def gather(self, layer: int, table_offset: int, table_length: int, n_tokens: int,
               out_keys, out_values) -> None:
        self.ctx.check(load().ckv_gather(self.handle, layer, table_offset, table_length, n_tokens,
                                         _ptr(out_keys), _ptr(out_values)))

    def _attend(self, fn, layer, queries, q_heads, scale, output, rows):
        rows = queries.shape[0] if rows is None else rows
        self.ctx.check(fn(self.handle, layer, _ptr(queries), q_heads, scale, _ptr(output), rows))

    def decode(self, layer, queries, q_heads, scale, output, rows=None) -> None:
        self._attend(load().ckv_decode_attention, layer, queries, q_heads, scale, output, rows)

    def append_decode(self, layer, keys, values, queries, q_heads, scale, output,
                      rows=None) -> None:
        rows = queries.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_append_decode(self.handle, layer, _ptr(keys), _ptr(values),
                                                _ptr(queries), q_heads, scale, _ptr(output),
                                                rows))

    def append_decode_noalloc(self, layer, keys, values, queries, q_heads, scale, output,
                              rows=None) -> None:
        """ckv_append_decode without allocating (ckv_append_decode_noalloc)."""
        rows = queries.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_append_decode_noalloc(self.handle, layer, _ptr(keys),
                                                        _ptr(values), _ptr(queries), q_heads,
                                                        scale, _ptr(output), rows))

    def prefill(self, layer, queries, q_heads, scale, output, rows=None) -> None:
        self._attend(load().ckv_prefill_attention, layer, queries, q_heads, scale, output, rows)

    def attention(self, layer, queries, q_heads, scale, output, rows=None) -> None:
        self._attend(load().ckv_attention, layer, queries, q_heads, scale, output, rows)

    def attention_gated(self, layer, queries, q_heads, scale, gate, output, rows=None) -> None:
        """output = attention * sigmoid(gate) (ckv_attention_gated)."""
        rows = queries.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_attention_gated(self.handle, layer, _ptr(queries), q_heads,
                                                  scale, _ptr(gate), _ptr(output), rows))

    def append_decode_gated(self, layer, keys, values, queries, q_heads, scale, gate, output,
                            rows=None) -> None:
        rows = queries.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_append_decode_gated(self.handle, layer, _ptr(keys),
                                                      _ptr(values), _ptr(queries), q_heads,
                                                      scale, _ptr(gate), _ptr(output), rows))

    def rope(self, inputs, outputs, heads: int, theta: float, rotary_dim: int = 0,
             rows: Optional[int] = None) -> None:
        rows = inputs.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_rope(self.handle, _ptr(inputs), _ptr(outputs), heads, theta,
                                       rotary_dim, rows))

    def rope_append(self, layer: int, keys, values, theta: float, rotary_dim: int = 0,
                    rows: Optional[int] = None) -> None:
        rows = keys.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_rope_append(self.handle, layer, _ptr(keys), _ptr(values),
                                              theta, rotary_dim, rows))

    def rope_append_decode(self, layer: int, keys, values, queries, q_heads: int, scale: float,
                           theta: float, output, rotary_dim: int = 0, gate=None,
                           rows: Optional[int] = None) -> None:
        """rope(queries), rope(keys) + append, decode attention (* sigmoid(gate)) in one
        call (ckv_rope_append_decode)."""
        rows = queries.shape[0] if rows is None else rows
        self.ctx.check(load().ckv_rope_append_decode(
            self.handle, layer, _ptr(keys), _ptr(values), _ptr(queries), q_heads, scale, theta,
            rotary_dim, None if gate is None else _ptr(gate), _ptr(output), rows))

    def copy_blocks(self, src, dst) -> None:
        s, d = _u32(src), _u32(dst)
        self.ctx.check(load().ckv_copy_blocks(self.handle, _p(s), _p(d), s.size))

    def checkpoint_pack(self, blocks, tokens: int, packed_keys, packed_values) -> None:
        b = _u32(blocks)
        self.ctx.check(load().ckv_checkpoint_pack(self.handle, _p(b), b.size, tokens,
                                                  _ptr(packed_keys), _ptr(packed_values)))

    def checkpoint_unpack(self, blocks, tokens: int, packed_keys, packed_values) -> None:
        b = _u32(blocks)
        self.ctx.check(load().ckv_checkpoint_unpack(self.handle, _p(b), b.size, tokens,
                                                    _ptr(packed_keys), _ptr(packed_values)))

    def checkpoint_export(self, blocks, tokens: int, host_keys: np.ndarray,
                          host_values: np.ndarray) -> None:
        """Packed prefix into host memory (numpy arrays, pinned from
        Context.host_alloc or pageable); read them only after ctx.sync()."""
        b = _u32(blocks)
        self.ctx.check(load().ckv_checkpoint_export(self.handle, _p(b), b.size, tokens,
                                                    _host(host_keys), _host(host_values)))

    def checkpoint_import(self, blocks, tokens: int, host_keys: np.ndarray,
                          host_values: np.ndarray) -> None:
        b = _u32(blocks)
        self.ctx.check(load().ckv_checkpoint_import(self.handle, _p(b), b.size, tokens,
                                                    _host(host_keys), _host(host_values)))

    def close(self) -> None:
        if getattr(self, "handle", None):
            load().ckv_pool_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
