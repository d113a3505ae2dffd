"""Shared test setup: repo root on sys.path, the package registered as
``specdec_nanovllm_amd``, the ``gpu`` marker, and helpers that move tensors
between torch (device) and the numpy oracle (host)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def to_np(t):
    """Device/host tensor -> numpy; bf16 becomes float32 values (exact)."""
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy()
    return t.numpy()


def bits16(t):
    """16-bit tensor -> numpy uint16 bit patterns (for bit-exact checks)."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_close_attn(got, ref, atol=2e-3, rtol=1e-2, what=""):
    """Attention tolerance: |got - ref| <= atol + rtol * |ref| elementwise."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    excess = np.abs(got - ref) - (atol + rtol * np.abs(ref))
    worst = np.unravel_index(np.argmax(excess), excess.shape) if excess.size else None
    assert excess.size == 0 or excess.max() <= 0, (
        f"{what}: max excess {excess.max():.3g} at {worst}: got {got[worst]:.6g} "
        f"ref {ref[worst]:.6g}")
