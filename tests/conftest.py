"""Test configuration: the `gpu` marker, package import, parity helpers."""
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
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


def rel_l2(a, b):
    """||a - b||_2 / ||b||_2 (the parity metric for fp32 tensors)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


def max_rel(a, b):
    """max|a - b| / max|b|."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    mb = np.abs(b).max() if b.size else 0.0
    return float(np.abs(a - b).max() / (mb if mb > 0 else 1.0)) if a.size else 0.0


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a HIP device")
    return torch.device("cuda:0")


_hip = None


def d2h(ptr, shape, dtype=np.float32):
    """Copy a raw device buffer to a new host array (hipMemcpy D2H)."""
    import ctypes
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
    out = np.empty(shape, dtype)
    assert _hip.hipDeviceSynchronize() == 0
    rc = _hip.hipMemcpy(out.ctypes.data, ptr, out.nbytes, 2)   # hipMemcpyDeviceToHost
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out


def masked_slots_zeroed(out, mask):
    """The trainer's own forward output: it runs the option scorer only on
    legal options (their masked scores never reach the loss), so masked
    slots read 0 — except in rows with no legal option, scored in full."""
    out = np.array(out, dtype=np.float32, copy=True)
    mask = np.asarray(mask) != 0
    A = mask.shape[1]
    rows = mask.any(axis=1)
    sl = out[:, :A]
    sl[rows[:, None] & ~mask] = 0.0
    return out
