"""MI355X-native paged KV-cache + attention path for chibillm.

libckv.so (HIP kernels for gfx950 + the C ABI of include/ckv.h) is the
product; chibillm_amd.ckv is its Python binding and chibillm_amd/host the C++
host layer (block_manager, scheduler, prefix_cache, model_batch, model state)
built on the same ABI.
"""
from . import ckv  # noqa: F401

__all__ = ["ckv"]
