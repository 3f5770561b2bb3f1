"""ctypes binding of libsparton_hip.so (the C ABI in include/sparton.h).

The library is loaded after torch, so its libamdhip64.so.7 dependency resolves to
the HIP runtime torch already loaded: streams and device pointers from torch are
valid in the library. There is no fallback: if the library is missing the first
call raises, telling the user how to build it.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be imported first: see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(_HERE, "libsparton_hip.so")
ABI_VERSION = 10

# enum sparton_dtype / sparton_mask_dtype (include/sparton.h)
DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
F32_SPLIT = 0x100  # SPARTON_F32_SPLIT


def fwd_dtype_code(dtype):
    """The forward's dtype argument: fp32 follows torch's float32 matmul precision, as the
    reference's GEMM does (it sets 'high' at import, sparton_kernel.py:14): 'high' and
    'medium' take the bf16 hi/lo split (SPARTON_F32_SPLIT), 'highest' exact fp32."""
    code = DTYPE_CODE[dtype]
    if dtype == torch.float32 and torch.get_float32_matmul_precision() != "highest":
        code |= F32_SPLIT
    return code
MASK_CODE = {
    torch.int64: 0,
    torch.int32: 1,
    torch.bool: 2,
    torch.uint8: 2,
    torch.float32: 3,
    torch.bfloat16: 4,
    torch.float16: 5,
}

EXPORTED_SYMBOLS = (
    "sparton_fwd",
    "sparton_fwd_profile",
    "sparton_fwd_workspace_bytes",
    "sparton_fwd_noalloc",
    "sparton_fwd_noalloc_max_workspace",
    "sparton_bwd",
    "sparton_bwd_workspace_bytes",
    "sparton_transform_fwd",
    "sparton_transform_bwd",
    "sparton_transform_workspace_bytes",
    "sparton_transform_dz_chunks",
    "sparton_transform_chunk_sum",
    "sparton_loss_fwd",
    "sparton_loss_bwd",
    "sparton_loss_bwd_terms",
    "sparton_loss_workspace_bytes",
    "sparton_mfma_probe",
    "sparton_strerror",
    "sparton_limits",
    "sparton_abi_version",
)

_lock = threading.Lock()
_lib = None

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


def lib_path() -> str:
    return os.environ.get("SPARTON_HIP_LIB", DEFAULT_LIB)


def load() -> ctypes.CDLL:
    """Load (once) and type the C ABI. Raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"sparton: HIP library not found at {path}. Build it with "
                "`python -m sparton_amd.build` (hipcc, --offload-arch=gfx950).")
        L = ctypes.CDLL(path)
        L.sparton_fwd.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, _vp,
                                  _i64, _i64, _i64, _i64, ctypes.c_int, _vp, ctypes.c_size_t, _vp]
        L.sparton_fwd.restype = ctypes.c_int
        L.sparton_fwd_profile.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, _vp,
                                          _i64, _i64, _i64, _i64, ctypes.c_int, _vp, ctypes.c_size_t,
                                          _vp, ctypes.POINTER(ctypes.c_float)]
        L.sparton_fwd_profile.restype = ctypes.c_int
        L.sparton_fwd_noalloc.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, _vp,
                                          _i64, _i64, _i64, _i64, ctypes.c_int, _vp]
        L.sparton_fwd_noalloc.restype = ctypes.c_int
        L.sparton_fwd_noalloc_max_workspace.argtypes = []
        L.sparton_fwd_noalloc_max_workspace.restype = ctypes.c_size_t
        L.sparton_fwd_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, ctypes.c_int]
        L.sparton_fwd_workspace_bytes.restype = ctypes.c_size_t
        L.sparton_bwd.argtypes = [_vp, _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _vp, _vp, _vp,
                                  _vp, _vp, ctypes.c_int, _vp, ctypes.c_size_t, _i64, _i64, _i64,
                                  _i64, ctypes.c_int, _vp]
        L.sparton_bwd.restype = ctypes.c_int
        L.sparton_bwd_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
        L.sparton_bwd_workspace_bytes.restype = ctypes.c_size_t
        L.sparton_transform_workspace_bytes.argtypes = [_i64, _i64]
        L.sparton_transform_workspace_bytes.restype = ctypes.c_size_t
        L.sparton_transform_fwd.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp,
                                            _i64, _i64, ctypes.c_int, _vp]
        L.sparton_transform_fwd.restype = ctypes.c_int
        L.sparton_transform_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                            _vp, ctypes.c_size_t, _i64, _i64, ctypes.c_int, _vp]
        L.sparton_transform_bwd.restype = ctypes.c_int
        L.sparton_transform_dz_chunks.argtypes = [_vp, _vp, _i64, _i64, _i64, ctypes.c_int, _vp]
        L.sparton_transform_dz_chunks.restype = ctypes.c_int
        L.sparton_transform_chunk_sum.argtypes = [_vp, _vp, _i64, _i64, ctypes.c_int, _vp]
        L.sparton_transform_chunk_sum.restype = ctypes.c_int
        L.sparton_loss_workspace_bytes.argtypes = [_i64, _i64, _i64]
        L.sparton_loss_workspace_bytes.restype = ctypes.c_size_t
        L.sparton_loss_fwd.argtypes = [_vp, _vp, _i64, _i64, _i64, ctypes.c_float, ctypes.c_float,
                                       ctypes.c_float, ctypes.c_float, _vp, _vp, _vp, ctypes.c_size_t,
                                       ctypes.c_int, _vp]
        L.sparton_loss_fwd.restype = ctypes.c_int
        L.sparton_loss_bwd.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, ctypes.c_float,
                                       ctypes.c_float, ctypes.c_float, _vp, _vp, ctypes.c_int, _vp]
        L.sparton_loss_bwd.restype = ctypes.c_int
        L.sparton_loss_bwd_terms.argtypes = [_vp, _vp, _vp, ctypes.POINTER(_vp), _i64, _i64, _i64,
                                             ctypes.c_float, ctypes.c_float, ctypes.c_float, _vp, _vp,
                                             ctypes.c_int, _vp]
        L.sparton_loss_bwd_terms.restype = ctypes.c_int
        L.sparton_mfma_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]
        L.sparton_mfma_probe.restype = ctypes.c_int
        L.sparton_strerror.argtypes = [ctypes.c_int]
        L.sparton_strerror.restype = ctypes.c_char_p
        L.sparton_limits.argtypes = [ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
        L.sparton_limits.restype = None
        L.sparton_abi_version.argtypes = []
        L.sparton_abi_version.restype = ctypes.c_int
        got = L.sparton_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"sparton: {path} has ABI version {got}, expected {ABI_VERSION}; rebuild it")
        _lib = L
        return L


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().sparton_strerror(rc).decode()
        raise RuntimeError(f"sparton: {what} failed with status {rc}: {msg}")


def limits() -> tuple[int, int]:
    s, b = _i64(), _i64()
    load().sparton_limits(ctypes.byref(s), ctypes.byref(b))
    return s.value, b.value


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
