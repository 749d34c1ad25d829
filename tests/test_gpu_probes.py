"""The hardware-ceiling probes of libckv_probes.so (bench.py --workload ceiling) at
small sizes: each launches, completes, and leaves its sink untouched (the probes
only read; the sink is written only if a reduction equals a constant that the
all-zero inputs here cannot produce)."""
import numpy as np
import pytest
import torch

from measure import probes

pytestmark = pytest.mark.gpu


def test_probes_run_and_write_nothing():
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    buf = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    for nt in (False, True):
        probes.read(buf, nt, 1024, sink, stream)
    pool_pages, page_bytes, row_bytes = 256, 32768, 2048
    keys = torch.zeros(pool_pages * page_bytes, dtype=torch.uint8, device=dev)
    values = torch.zeros_like(keys)
    order = torch.from_numpy(np.random.default_rng(0).permutation(pool_pages).astype(np.int32)).to(dev)
    for slice_bytes, per_wg in ((256, 36), (2048, 5)):
        for waves, lds in ((10, 0), (8, 80 * 1024)):
            probes.pages(keys, values, pool_pages, order, page_bytes, row_bytes, slice_bytes,
                         per_wg, waves, lds, sink, stream)
    for chains in (1, 2, 4):
        probes.mfma(16, chains, 8, 4, sink, stream)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sink).item() == 0
