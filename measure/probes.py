"""ctypes binding of libckv_probes.so (measure/probes.hip): the
hardware-ceiling probes that `bench.py --workload ceiling` runs. They are not
part of the libckv boundary. Raises if the library has not been built."""
import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libckv_probes.so")
_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (__graft_entry__.build())")
        lib = C.CDLL(LIB_PATH)
        vp, u32, sz = C.c_void_p, C.c_uint32, C.c_size_t
        lib.ckv_probe_read.argtypes = [vp, sz, C.c_int, u32, vp, vp]
        lib.ckv_probe_pages.argtypes = [vp, vp, u32, vp, u32, u32, u32, u32, u32, u32, u32, vp, vp]
        lib.ckv_probe_mfma.argtypes = [u32, u32, u32, u32, vp, vp]
        for f in (lib.ckv_probe_read, lib.ckv_probe_pages, lib.ckv_probe_mfma):
            f.restype = C.c_int
        _lib = lib
    return _lib


def _check(code, what):
    if code != 0:
        raise RuntimeError(f"{what} failed with hipError {code}")


def read(src, nontemporal, grid, sink, stream):
    """One pass over the device tensor `src` with 16-byte loads."""
    _check(load().ckv_probe_read(src.data_ptr(), src.numel() * src.element_size(),
                                 int(bool(nontemporal)), grid, sink.data_ptr(), stream),
           "ckv_probe_read")


def pages(keys, values, pool_pages, page_list, page_bytes, row_bytes, slice_bytes, per_wg,
          waves, lds_bytes, sink, stream):
    """The decode's page reads over the device uint32 tensor `page_list`."""
    _check(load().ckv_probe_pages(keys.data_ptr(), values.data_ptr(), pool_pages,
                                  page_list.data_ptr(), page_list.numel(), page_bytes, row_bytes,
                                  slice_bytes, per_wg, waves, lds_bytes, sink.data_ptr(), stream),
           "ckv_probe_pages")


def mfma(iters, chains, waves, grid, sink, stream):
    """Back-to-back bf16 32x32x16 products: grid x waves x chains x iters of them."""
    _check(load().ckv_probe_mfma(iters, chains, waves, grid, sink.data_ptr(), stream),
           "ckv_probe_mfma")
