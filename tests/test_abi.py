"""The C-ABI library loads and exports exactly what include/ckv.h declares.
CPU only: no compute call is made."""
import os
import re
import subprocess
import sys

import pytest

from chibillm_amd import ckv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ckv_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    declared = declared_functions("ckv.h")
    assert declared, "no declarations parsed"
    out = subprocess.run(["nm", "-D", "--defined-only", ckv.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [name for name in declared if name not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # the Python binding covers the whole ABI
    assert sorted(ckv.SYMBOLS) == declared
    lib = ckv.load()
    for name in declared:
        assert getattr(lib, name)


def test_abi_version_and_error_names_match_the_reference_strings():
    lib = ckv.load()
    assert lib.ckv_abi_version() == 1
    # src/tensor/tensor_ops.h:50-86, src/metal/metal_kv_cache.h:57-70, src/model_state.h:17-28
    expected = {
        0: "ok",
        107: "tensor_op.invalid_rank",
        114: "tensor_op.position_count_mismatch",
        118: "tensor_op.cache_slot_count_mismatch",
        120: "tensor_op.cache_layer_out_of_range",
        121: "tensor_op.cache_slot_out_of_range",
        123: "tensor_op.block_table_range_out_of_bounds",
        124: "tensor_op.cache_block_out_of_range",
        126: "tensor_op.invalid_kv_head_mapping",
        128: "tensor_op.unsupported_aliasing",
        200: "kv_cache.invalid_layer_count",
        205: "kv_cache.layout_size_overflow",
        211: "kv_cache.head_feature_out_of_range",
        300: "state.capacity_exhausted",
        301: "state.invalid_reservation",
        403: "ckv.no_tables",
        999: "ckv.unknown_error",
    }
    for code, name in expected.items():
        assert ckv.error_name(code) == name


def test_header_compiles_as_c_and_cxx():
    for compiler, flag in (("gcc", "-std=c11"), ("g++", "-std=c++17")):
        src = '#include "ckv.h"\nint main(void) { return ckv_abi_version() == CKV_ABI_VERSION ? 0 : 1; }\n'
        r = subprocess.run([compiler, flag, "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                            "-x", "c" if compiler == "gcc" else "c++", "-"], input=src, text=True,
                           capture_output=True)
        assert r.returncode == 0, r.stderr


def test_probe_library_loads_and_rejects_bad_geometry():
    """libckv_probes.so (bench.py --workload ceiling) exports its three probes and
    refuses, before any launch, what its kernels do not cover."""
    import ctypes as C

    from measure import probes

    lib = probes.load()
    invalid = 1  # hipErrorInvalidValue
    buf = C.c_void_p(256)  # never dereferenced: every call below fails its checks
    assert lib.ckv_probe_read(None, 16, 1, 1, buf, None) == invalid
    assert lib.ckv_probe_read(C.c_void_p(264), 16, 1, 1, buf, None) == invalid  # unaligned
    assert lib.ckv_probe_read(buf, 17, 1, 1, buf, None) == invalid  # not whole 16-byte loads
    assert lib.ckv_probe_read(buf, 16, 1, 0, buf, None) == invalid  # empty grid
    # slice of 96 bytes does not divide a 2 KiB row; 16 rows x 8 chunks is not a multiple of 256
    args = [buf, buf, 64, buf, 64, 32768, 2048]
    assert lib.ckv_probe_pages(*args, 96, 8, 10, 0, buf, None) == invalid
    assert lib.ckv_probe_pages(*args, 128, 8, 10, 0, buf, None) == invalid
    assert lib.ckv_probe_pages(*args, 256, 8, 17, 0, buf, None) == invalid  # 17 waves
    assert lib.ckv_probe_pages(*args, 256, 8, 10, 160 * 1024 + 1, buf, None) == invalid
    assert lib.ckv_probe_pages(buf, buf, 0, buf, 64, 32768, 2048, 256, 8, 10, 0, buf,
                               None) == invalid
    assert lib.ckv_probe_mfma(10, 3, 8, 1, buf, None) == invalid  # chains 1, 2 or 4
    assert lib.ckv_probe_mfma(10, 1, 0, 1, buf, None) == invalid
