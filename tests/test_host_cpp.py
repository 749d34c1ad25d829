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


def test_decode_planner_cpu():
    """libckv's fast decode planner on the CPU (tests/cpp/plan_tests.cc): every
    plan covers each row's pages once, its workgroups' entries link up, and
    the balanced plan evens out the work."""
    _run("plan_tests", 120)


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


def _prefill_oracle(H, D, HQ, k, v, q, first_position):
    """Oracle causal attention of `q`'s rows (consecutive positions from
    first_position) over one sequence's K/V, stored on a compact table."""
    import math

    import numpy as np

    from oracle import oracle as orc

    n = k.shape[0]
    pages = math.ceil(n / 16)
    F = H * D
    kc = np.zeros(pages * 16 * F, np.uint16)
    vc = np.zeros_like(kc)
    table = np.arange(pages, dtype=np.uint32)
    orc.store_kv(kc, vc, k, v, list(range(n)), 0, pages * 16)
    rows = q.shape[0]
    att = orc.Attention((1, pages, 16, H, D), kc, vc, orc.BF16, q, orc.BF16,
                        [first_position + r for r in range(rows)], table, [0] * rows,
                        [pages] * rows, HQ, 0, float(np.float32(1 / math.sqrt(D))))
    return att.online_threads(8)


@pytest.mark.gpu
def test_churn_full_size_checked_trace(tmp_path):
    """BASELINE config 5 at its real size (160 GB pool, 28 layers, live batch
    512), the whole 5,000-step trace under --check. Every layer appends and attends its
    own K/V/Q rows, and every step takes them from a different window, so a
    read of the wrong layer, a stale step or a misplaced row changes what is
    compared. Every 500 steps the page accounting holds (each live sequence's
    pages held once, reference counts summing to the pages in tables, free +
    used = pool) and sampled sequences' K/V, packed back from every layer,
    equal the rows the trace appended for them (the driver stops at the first
    failure with status 3). Eight rows of one decode step and one prefill
    chunk are checked here at layers 0 and 27 against the oracle, over K/V
    regenerated on the host from the rows the trace appended (not read back
    from the pool), within 2e-2 abs + 1e-2 rel."""
    import json

    import numpy as np

    from oracle import oracle as orc
    from tests.gpu_util import assert_close
    from tests.test_gpu_parity import compact_oracle

    path = os.path.join(BIN, "churn")
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built: run __graft_entry__.build()")
    steps = 5000
    print(f"churn --check: {steps} steps, 160 GB, 28 layers", flush=True)
    proc = subprocess.run([path, "--steps", str(steps), "--check", str(tmp_path), "--check-every",
                           "500", "--dump-after", "2500"], capture_output=True, text=True,
                          timeout=300)
    print(proc.stderr[-3000:])
    assert proc.returncode == 0, proc.stderr[-3000:]
    trace = json.loads(proc.stdout.strip().splitlines()[-1])
    assert trace["pool_pages"] == 87193
    assert trace["check"]["checks"] == 11
    assert trace["check"]["dumped_decode"] and trace["check"]["dumped_prefill"]
    assert trace["check"]["kv_tokens_checked"] > 0
    assert trace["decode_steps"] > 0 and trace["finished"] > 0 and trace["rejected"] == 0

    meta = json.loads((tmp_path / "decode_rows.json").read_text())
    H, D, HQ = meta["kv_heads"], meta["head_dim"], meta["q_heads"]
    rows = meta["rows"]
    lengths = [r["position"] + 1 for r in rows]
    assert meta["layers"] == [0, 27]
    outs = {}
    for layer in meta["layers"]:
        q = np.fromfile(tmp_path / f"dq_{layer}.bin", np.uint16).reshape(len(rows), HQ * D)
        out = np.fromfile(tmp_path / f"dout_{layer}.bin", np.uint16).reshape(len(rows), HQ * D)
        ks = [np.fromfile(tmp_path / f"dk_{layer}_{i}.bin", np.uint16).reshape(n, H * D)
              for i, n in enumerate(lengths)]
        vs = [np.fromfile(tmp_path / f"dv_{layer}_{i}.bin", np.uint16).reshape(n, H * D)
              for i, n in enumerate(lengths)]
        tables = [np.zeros(-(-n // 16), np.uint32) for n in lengths]
        expected = compact_oracle((H, D), lengths, tables, ks, vs, q, HQ)
        assert_close(orc.to_f32(out, orc.BF16), expected,
                     what=f"layer {layer} decode rows of sequences {[r['seq'] for r in rows]}")
        outs[layer] = out
    # the layers' data differ, so their outputs must too
    assert not np.array_equal(outs[0], outs[27])

    pre = json.loads((tmp_path / "prefill_rows.json").read_text())
    count, n = pre["rows"], pre["tokens"]
    assert pre["first_position"] + count == n
    print(f"prefill chunk: sequence {pre['seq']}, {count} rows over {n} tokens", flush=True)
    for layer in pre["layers"]:
        k = np.fromfile(tmp_path / f"pk_{layer}.bin", np.uint16).reshape(n, H * D)
        v = np.fromfile(tmp_path / f"pv_{layer}.bin", np.uint16).reshape(n, H * D)
        q = np.fromfile(tmp_path / f"pq_{layer}.bin", np.uint16).reshape(count, HQ * D)
        out = np.fromfile(tmp_path / f"pout_{layer}.bin", np.uint16).reshape(count, HQ * D)
        expected = _prefill_oracle(H, D, HQ, k, v, q, pre["first_position"])
        assert_close(orc.to_f32(out, orc.BF16), expected,
                     what=f"layer {layer} prefill chunk of sequence {pre['seq']}")
