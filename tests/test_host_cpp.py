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


@pytest.mark.gpu
def test_churn_driver_runs_a_short_trace():
    """The config-5 driver end to end at a small size: the scheduler admits,
    runs and retires sequences over the device KV path without errors."""
    import json

    path = os.path.join(BIN, "churn")
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built: run __graft_entry__.build()")
    proc = subprocess.run([path, "--steps", "300", "--pool-gb", "4", "--layers", "2",
                           "--max-live", "64"], capture_output=True, text=True, timeout=100)
    assert proc.returncode == 0, proc.stderr[-2000:]
    trace = json.loads(proc.stdout.strip().splitlines()[-1])
    assert trace["prefill_steps"] > 0 and trace["decode_steps"] > 0
    assert trace["finished"] > 0 and trace["rejected"] == 0
    assert trace["peak_live"] <= 64
    assert trace["prefill_tokens"] + trace["decode_tokens"] > 0
