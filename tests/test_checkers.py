"""The full-size GPU checkers of tests/_parity.py, run on the CPU against the oracle's own
outputs: they must accept correct results and reject planted mistakes (an argmax moved off
a near-tie, reps scaled, a zero rep with a nonzero index, a dW row gathered from the wrong
batch row, a dropped exp(-reps) factor). The GPU tests use the same functions on device
tensors."""
import torch

import oracle
from _parity import check_dw_identity_gpu, check_fwd_full_gpu
from sparton_amd.workloads import WORKLOADS, make_inputs


def _case(seed=5):
    w = WORKLOADS[2].scaled(B=3, S=24, D=40, V=300)
    inp = make_inputs(w, seed=seed)
    M, I, ref = oracle.fused_fwd_ref(inp.hidden, inp.weight, inp.bias, inp.mask)
    reps = ref.to(w.dtype)
    return inp, reps, I.to(torch.int32), ref


def test_fwd_checker_accepts_oracle_outputs():
    inp, reps, idx, _ = _case()
    n, bad = check_fwd_full_gpu(inp.hidden, inp.weight, inp.bias, inp.mask, reps, idx, chunk=128)
    assert n == reps.numel() and bad == 0


def test_fwd_checker_rejects_planted_mistakes():
    inp, reps, idx, ref = _case()
    H, W, b, m = inp.hidden, inp.weight, inp.bias, inp.mask
    pos = (ref > 0.05).nonzero()
    bb, vv = (int(t) for t in pos[0])
    # an argmax moved to a position whose logit is clearly below the max
    S = H.shape[1]
    xs = torch.stack([oracle.logit_at(H, W, b, m, torch.full_like(idx.long(), s)) for s in range(S)], 1)
    lo = int(torch.argmin(xs[bb, :, vv]))
    moved = idx.clone()
    moved[bb, vv] = lo
    try:
        check_fwd_full_gpu(H, W, b, m, reps, moved, chunk=128)
        raise RuntimeError("a moved argmax was accepted")
    except AssertionError:
        pass
    scaled = (reps.float() * 1.05).to(reps.dtype)
    try:
        check_fwd_full_gpu(H, W, b, m, scaled, idx, chunk=128)
        raise RuntimeError("scaled reps were accepted")
    except AssertionError:
        pass
    zeros = ref == 0
    if bool(zeros.any()):
        zb, zv = (int(t) for t in zeros.nonzero()[0])
        nz = idx.clone()
        nz[zb, zv] = 1
        try:
            check_fwd_full_gpu(H, W, b, m, reps, nz, chunk=128)
            raise RuntimeError("a zero rep with a nonzero index was accepted")
        except AssertionError:
            pass


def test_dw_checker_accepts_oracle_and_rejects_mistakes():
    inp, reps, idx, ref = _case()
    H, W, b, m, G = inp.hidden, inp.weight, inp.bias, inp.mask, inp.grad
    r32 = ref.float()
    _, dW, _ = oracle.fused_bwd_ref(G, r32, idx, H, W, True, m)
    worst = check_dw_identity_gpu(G, r32, idx, H, m, dW.float(), chunk=64)
    assert worst <= 1.0
    # gathered from the next batch row
    Hs = torch.roll(H, 1, dims=0)
    _, dW_bad, _ = oracle.fused_bwd_ref(G, r32, idx, Hs, W, True, m)
    try:
        check_dw_identity_gpu(G, r32, idx, H, m, dW_bad.float(), chunk=64)
        raise RuntimeError("a dW gathered from the wrong batch row was accepted")
    except AssertionError:
        pass
    # exp(-reps) dropped: g' = G m[b, I] where reps > 0
    _, dW_noexp, _ = oracle.fused_bwd_ref(G, torch.where(r32 > 0, torch.full_like(r32, 1e-30), r32),
                                          idx, H, W, True, m)
    try:
        check_dw_identity_gpu(G, r32, idx, H, m, dW_noexp.float(), chunk=64)
        raise RuntimeError("a dW without exp(-reps) was accepted")
    except AssertionError:
        pass
