"""Helpers for the GPU parity tests: device <-> numpy moves and tolerance checks.

The oracle keeps 16-bit values as uint16 bit patterns; these helpers move them
to torch bf16/fp16 device tensors bit-for-bit and back.
"""
import numpy as np
import torch

from chibillm_amd import ckv
from oracle import oracle as orc

ATOL, RTOL = 2e-2, 1e-2  # attention within 2e-2 abs / 1e-2 rel


def torch_dtype(code):
    return {orc.F32: torch.float32, orc.BF16: torch.bfloat16, orc.F16: torch.float16}[code]


def to_dev(array, code, device="cuda"):
    a = np.ascontiguousarray(array)
    if code == orc.F32:
        return torch.from_numpy(a.astype(np.float32)).to(device)
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch_dtype(code)).to(device)


def to_host(t, code):
    t = t.detach().contiguous()
    if code == orc.F32:
        return t.float().cpu().numpy()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def to_f32(t):
    return t.detach().float().cpu().numpy()


def new_context():
    return ckv.Context(0, stream=torch.cuda.current_stream())


def new_pool(ctx, geom, code, fill=0.0):
    L, B, bs, H, D = geom
    n = L * B * bs * H * D
    keys = torch.full((n,), fill, dtype=torch_dtype(code), device="cuda")
    values = torch.full((n,), fill, dtype=torch_dtype(code), device="cuda")
    return ckv.Pool(ctx, L, B, bs, H, D, code, keys, values), keys, values


def assert_close(got, expected, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    excess = np.abs(got - expected) - (atol + rtol * np.abs(expected))
    worst = float(excess.max()) if excess.size else 0.0
    assert worst <= 0, (f"{what}: max |got-expected| beyond tolerance by {worst:.3g} "
                        f"(max abs err {np.abs(got - expected).max():.3g})")


def approx(got, expected, eps, scale=0.0):
    """doctest::Approx(expected).epsilon(eps).scale(scale), elementwise."""
    a = np.asarray(got, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return bool(np.all(np.abs(a - e) <= eps * (scale + np.maximum(np.abs(a), np.abs(e)))))


def force_plan(monkeypatch, split):
    """Forces the fast decode's batch plan: None keeps the default, "N" cuts
    every row into fixed chunks of N pages (CKV_DECODE_SPLIT; "0": no cut),
    "bN" deals the batch's pages out N to a workgroup (CKV_DECODE_BALANCE), so
    a workgroup may take several rows and row pieces."""
    if split is None:
        return
    if split.startswith("b"):
        monkeypatch.setenv("CKV_DECODE_BALANCE", split[1:])
    else:
        monkeypatch.setenv("CKV_DECODE_SPLIT", split)
