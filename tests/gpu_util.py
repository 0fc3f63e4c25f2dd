"""Helpers for the GPU parity tests (they call the HIP path through the
package's C-ABI bindings and check it against the CPU oracle)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

# Tolerances (rel-L2) of the path: fp32 inputs, and bf16 inputs with fp32
# accumulation.
TOL_F32 = 1e-5
TOL_BF16 = 1e-2


def need_gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import burn_dragon_amd as bd
    if not bd.supports_backend():
        pytest.skip("device is not gfx950")
    return torch


def announce(*parts):
    """Names the case before a GPU step (a fault would end the process)."""
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def dev(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def host(t):
    return t.detach().float().cpu().numpy()


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b.ravel())
    return float(np.linalg.norm((a - b).ravel()) / den) if den > 0 else float(np.linalg.norm(a))
