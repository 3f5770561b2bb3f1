"""Loader of libsparton_torch.so: the sparton_eager torch ops (C++, csrc/sparton_torch.cpp).

They are the modules' eager training paths -- SpartonHead, SpartonMLMTransform and the SPLADE
loss -- with their autograd in C++, on the same C ABI as everything else (include/sparton.h).
Under torch.compile the modules call the torch.library ops of ops.py / transform.py / loss.py
instead (those carry the fake kernels). There is no fallback: a missing library raises,
naming the build command.
"""
from __future__ import annotations

import os
import threading

import torch

from . import _lib

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(_HERE, "libsparton_torch.so")
_lock = threading.Lock()
_ops = None


def lib_path() -> str:
    return os.environ.get("SPARTON_TORCH_LIB", DEFAULT_LIB)


def load():
    """torch.ops.sparton_eager, loading the library once (after the C ABI it links to)."""
    global _ops
    if _ops is not None:
        return _ops
    with _lock:
        if _ops is None:
            _lib.load()  # libsparton_hip.so first: checks its ABI version
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(
                    f"sparton: torch op library not found at {path}. Build it with "
                    "`python -m sparton_amd.build` (hipcc for the kernels, g++ for the ops).")
            torch.ops.load_library(path)
            _ops = torch.ops.sparton_eager
    return _ops
