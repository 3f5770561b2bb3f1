"""sparton_fwd_noalloc (the forward with its workspace in a static device array) against
sparton_fwd with a caller workspace: bitwise equal, on two calls in a row, the second with a
smaller input of another dtype, mask type and bias setting."""
import ctypes

import pytest
import torch

from sparton_amd import _lib
from _parity import check_fwd, say
from test_gpu_parity import make_case

pytestmark = pytest.mark.gpu


def run_noalloc(H, W, b, m):
    L = _lib.load()
    B, S, D = H.shape
    V = W.shape[0]
    reps = torch.full((B, V), float("nan"), dtype=H.dtype, device=H.device)
    idx = torch.full((B, V), -7, dtype=torch.int32, device=H.device)
    r32 = torch.full((B, V), float("nan"), dtype=torch.float32, device=H.device)
    rc = L.sparton_fwd_noalloc(H.data_ptr(), W.data_ptr(), _lib.ptr(b), m.data_ptr(),
                               _lib.MASK_CODE[m.dtype], reps.data_ptr(), idx.data_ptr(),
                               r32.data_ptr(), B, S, D, V, _lib.DTYPE_CODE[H.dtype],
                               torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "sparton_fwd_noalloc")
    return reps, idx, r32


@pytest.mark.parametrize("cases", [[
    ("bf16", 32, 256, 768, 30522, True, "int64"),   # config 2's shape, then a smaller one
    ("fp16", 3, 100, 64, 1000, False, "holes"),
]])
def test_fwd_noalloc_matches_fwd(cases, device):
    for case in cases:
        say(f"noalloc forward, case {case}")
        H, W, b, m, _ = make_case(*case)
        Hd, Wd, md = H.to(device), W.to(device), m.to(device)
        bd = None if b is None else b.to(device)
        ref = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, md)
        got = run_noalloc(Hd, Wd, bd, md)
        torch.cuda.synchronize()
        for a, c in zip(ref, got):
            assert torch.equal(a, c)
        if case[1] * case[4] <= 10 ** 5:
            n, bad = check_fwd(H, W, b, m, got[0], got[1])
            say(f"  checked {n} entries against the oracle, {bad} near-ties")
