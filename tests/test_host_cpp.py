"""Runs the C++ host-layer test programs (tests/cpp) built into chibillm_amd/bin.

host_tests restates the reference's scheduler, block manager, model batch,
prefix cache and engine tests on the CPU; host_gpu_tests runs the KV cache,
tensor-op and shared-prefix tests through libckv on the device.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "chibillm_amd", "bin")


def _run(name: str, timeout: int) -> None:
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built: run __graft_entry__.build()")
    proc = subprocess.run([path], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout[-4000:])
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert " 0 failed checks" in proc.stdout


def test_host_layer_cpu():
    _run("host_tests", 120)


@pytest.mark.gpu
def test_host_layer_gpu():
    _run("host_gpu_tests", 100)
