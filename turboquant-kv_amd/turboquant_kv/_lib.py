"""Loads the native libraries built by turboquant-kv_amd/build.py.

There is no fallback: if the libraries are missing, or an op gets a tensor that
is not on a HIP device, the call raises.
"""

from __future__ import annotations

import os
import threading

import torch

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
HIP_LIB = os.path.join(LIB_DIR, "libturboquant_hip.so")
TORCH_LIB = os.path.join(LIB_DIR, "libturboquant_torch.so")

_lock = threading.Lock()
_loaded = False


def load() -> None:
    """Register torch.ops.turboquant (idempotent)."""
    global _loaded
    if _loaded:
        return
    with _lock:
        if _loaded:
            return
        if not (os.path.exists(HIP_LIB) and os.path.exists(TORCH_LIB)):
            raise RuntimeError(
                "turboquant_kv: the gfx950 kernel library is not built "
                f"(expected {TORCH_LIB}); run `python turboquant-kv_amd/build.py`")
        torch.ops.load_library(TORCH_LIB)
        _loaded = True


def ops():
    """The `turboquant` torch.ops namespace, loading the library on first use."""
    load()
    return torch.ops.turboquant


def require_device(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(
            f"turboquant_kv: {name} must be a tensor on a HIP device; this MI355X build "
            "has no CPU kernels")


def require_tensor(t: torch.Tensor, name: str) -> None:
    """The five reference schemas run on HIP-device tensors (gfx950 kernels) and on CPU
    tensors (their CPU kernels, as the reference registers): any tensor is accepted."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"turboquant_kv: {name} must be a torch.Tensor")
