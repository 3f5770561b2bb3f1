"""Comparison helpers for the GPU parity tests (HIP path vs the CPU oracle).

Tolerances (from the task's statement of the bar):
  reps vs the fp64 oracle on the same rounded inputs: rtol 1e-2, atol 1e-3.
  argmax: a zero rep carries index 0 (the reference initialises (max, idx) to (0, 0),
      sparton_kernel.py:112-114). Elsewhere the index is exact, except documented
      near-ties: an index is accepted when the oracle's logit at it is within tau of the
      oracle max M, where tau is derived from the two ways the GPU's choice can differ:
        * the kernel's tie precision: its integer keys keep each logit with its 5 low
          mantissa bits replaced by the row, so values within KEY_REL = 2^-18 relative
          of each other tie and the lowest s wins;
        * fp32 accumulation: each logit is a D-term fp32 dot product plus bias, times the
          mask, so |computed - exact| <= gamma_{D+2} * (sum_d |h_d w_d| + |bias|) * |m|
          with gamma_n = n * 2^-24, for the GPU's candidate and the oracle's alike.
      tau = KEY_REL * |M| + gamma_{D+2} * (A(idx) + A(I)) + 4 * 2^-24 * |M|, A(s) being the
      absolute-value sum above at position s. Under the fp32 bf16-split mode (torch's 'high'
      float32 matmul precision) each product is within SPLIT_REL = 3 * 2^-16 relative of the
      exact one, which adds SPLIT_REL * (A(idx) + A(I)).
  backward vs the oracle evaluated at the GPU's own reps/argmax: rtol 1e-4,
      atol 1e-5 (both sum exact products of the same rounded inputs; the GPU sums
      in fp32, the oracle in fp64).
  end-to-end vs the torch head (fp32 autograd): rtol 1e-2, atol 1e-3, on rows
      that no near-tie moved.
"""
import sys

import torch

import oracle

F64 = torch.float64
KEY_REL = 2.0 ** -18      # tie precision of the forward kernel's integer keys
U32 = 2.0 ** -24          # fp32 unit roundoff
SPLIT_REL = 3 * 2.0 ** -16  # a product's error as bf16 hi*hi + hi*lo + lo*hi
FWD_TOL = dict(rtol=1e-2, atol=1e-3)
BWD_TOL = dict(rtol=1e-4, atol=1e-5)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check_fwd(H, W, b, m, reps, idx, cols=None, split=False):
    """H, W, b, m: CPU tensors in the run dtype. reps/idx: GPU outputs (any device).
    cols: optional LongTensor of vocab columns to check (full check when None).
    split: the outputs come from the fp32 bf16-split mode (wider tie band).
    Returns (n_checked, n_index_mismatch)."""
    reps, idx = reps.cpu(), idx.cpu().long()
    if cols is not None:
        W, reps, idx = W[cols], reps[:, cols], idx[:, cols]
        b = None if b is None else b[cols]
    M, I, ref = oracle.fused_fwd_ref(H, W, b, m)
    torch.testing.assert_close(reps.to(F64), ref, **FWD_TOL)
    S = H.shape[1]
    assert int(idx.min()) >= 0 and int(idx.max()) < max(S, 1), "argmax out of range"
    zero = reps == 0
    assert bool((idx[zero] == 0).all()), (
        f"{int((idx[zero] != 0).sum())} zero reps carry a nonzero argmax (must be 0)")
    bad = idx != I
    n_bad = int(bad.sum())
    if n_bad:
        # a positive GPU max at another position: that position's exact logit must be
        # within tau of the exact max
        pos = bad & (reps != 0)
        x_at = oracle.logit_at(H, W, b, m, idx)
        near = x_at >= M - tie_band(H, W, b, m, idx, I, M, split)
        assert bool(near[pos].all()), (
            f"{int((~near & pos).sum())} argmax entries are not near-ties; first at "
            f"{(~near & pos).nonzero()[:5].tolist()}")
        # no positive GPU logit (index 0) where the oracle has one: its max must be
        # within the error band of 0
        zb = bad & (reps == 0)
        small = M <= tie_band(H, W, b, m, I, I, M, split)
        assert bool(small[zb].all()), (
            f"{int((~small & zb).sum())} zero reps where the exact max is clearly positive")
    return reps.numel(), n_bad


def tie_band(H, W, b, m, idx_a, idx_b, M, split=False):
    """tau[b,v] for two competing positions idx_a, idx_b (see the module docstring)."""
    D = H.shape[-1]
    gam = (D + 2) * U32 + (SPLIT_REL if split else 0.0)
    Ha, Wa = H.abs(), W.abs()
    ma = m if m.dtype == torch.bool else m.abs()
    ba = None if b is None else b.abs()
    A = oracle.logit_at(Ha, Wa, ba, ma, idx_a) + oracle.logit_at(Ha, Wa, ba, ma, idx_b)
    return KEY_REL * M.abs() + gam * A + 4 * U32 * M.abs()


def check_bwd_isolated(H, W, b, m, G, reps, idx, dH, dW, db):
    """Backward kernels against the oracle's closed form at the GPU's reps/argmax."""
    rH, rW, rb = oracle.fused_bwd_ref(G, reps.cpu(), idx.cpu(), H, W, b is not None, m)
    torch.testing.assert_close(dH.cpu().to(F64), rH, **BWD_TOL)
    torch.testing.assert_close(dW.cpu().to(F64), rW, **BWD_TOL)
    if b is not None:
        torch.testing.assert_close(db.cpu().to(F64), rb, **BWD_TOL)
    return rH, rW, rb


U64 = 2.0 ** -53          # fp64 unit roundoff


def check_fwd_full_gpu(Hd, Wd, bd, md, reps, idx, split=False, chunk=None):
    """Every (b, v) of a full-size forward against logits recomputed on the GPU by a library
    routine: V-chunked float64 GEMMs (torch.matmul), x = (H W^T + b) * m, M = max(0, max_s x)
    and its index. reps within FWD_TOL of log1p(M); a zero rep carries index 0; an index that
    differs from the recomputed one must be a near-tie: the recomputed logit at it lies within
    tau of M, tau as in check_fwd, widened by the float64 GEMM's own bound
    (D+2) * 2^-53 * (A(idx) + A(I)). Returns (n_checked, n_index_mismatch)."""
    B, S, D = Hd.shape
    V = Wd.shape[0]
    if chunk is None:
        chunk = max(256, min(8192, (1 << 27) // max(1, B * S * 8)))
    gam = (D + 2) * U32 + (D + 2) * U64 + (SPLIT_REL if split else 0.0)
    H64 = Hd.reshape(B * S, D).double()
    Ha = H64.abs()
    m64 = md.double()
    ma = m64.abs()
    reps, idx = reps.double(), idx.long()
    n_bad = 0
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        C = v1 - v0
        Wc = Wd[v0:v1].double()
        X = (H64 @ Wc.t()).view(B, S, C)
        A = (Ha @ Wc.abs().t()).view(B, S, C)
        if bd is not None:
            bc = bd[v0:v1].double()
            X += bc
            A += bc.abs()
        X *= m64[:, :, None]
        A *= ma[:, :, None]
        M, I = X.max(dim=1)
        M = M.clamp_min(0.0)
        I = torch.where(M > 0, I, torch.zeros_like(I))
        r, ix = reps[:, v0:v1], idx[:, v0:v1]
        torch.testing.assert_close(r, torch.log1p(M), **FWD_TOL)
        assert int(ix.min()) >= 0 and int(ix.max()) < max(S, 1), "argmax out of range"
        zero = r == 0
        assert bool((ix[zero] == 0).all()), (
            f"cols {v0}..{v1}: {int((ix[zero] != 0).sum())} zero reps carry a nonzero argmax")
        bad = ix != I
        nb = int(bad.sum())
        if nb:
            x_at = X.gather(1, ix.view(B, 1, C)).view(B, C)
            A_at = A.gather(1, ix.view(B, 1, C)).view(B, C)
            A_I = A.gather(1, I.view(B, 1, C)).view(B, C)
            tau = KEY_REL * M.abs() + gam * (A_at + A_I) + 4 * U32 * M.abs()
            pos = bad & (r != 0)
            near = x_at >= M - tau
            assert bool(near[pos].all()), (
                f"cols {v0}..{v1}: {int((~near & pos).sum())} argmax entries are not near-ties")
            zb = bad & (r == 0)
            small = M <= KEY_REL * M.abs() + gam * 2 * A_I + 4 * U32 * M.abs()
            assert bool(small[zb].all()), (
                f"cols {v0}..{v1}: {int((~small & zb).sum())} zero reps where the max is clearly positive")
        n_bad += nb
    return B * V, n_bad


def check_dw_identity_gpu(Gd, reps32, idx, Hd, md, dW, chunk=None):
    """Every row of dW against the identity dW[v,:] = sum_b g'[b,v] H[b, I[b,v], :], with
    g' = G exp(-reps) m[b,I] where reps > 0, evaluated in float64 on the GPU at the GPU's own
    reps and argmax. The kernel sums B products in fp32 from a g' with one expf, so
    |dW - ref| <= (B + 8) * 2^-24 * sum_b |g' H| elementwise."""
    B, S, D = Hd.shape
    V = dW.shape[0]
    if chunk is None:
        chunk = max(64, (1 << 27) // max(1, B * D * 8))
    r = reps32.double()
    ix = idx.long()
    mI = md.double().gather(1, ix)
    gp = torch.where(r > 0, Gd.double() * torch.exp(-r), torch.zeros_like(r)) * mI
    H64 = Hd.double()
    rows = torch.arange(B, device=Hd.device).view(B, 1)
    worst = 0.0
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        Hg = H64[rows, ix[:, v0:v1]]                      # [B, C, D]
        g = gp[:, v0:v1, None]
        ref = (g * Hg).sum(0)
        bound = (B + 8) * U32 * (g.abs() * Hg.abs()).sum(0)
        err = (dW[v0:v1].double() - ref).abs()
        ok = err <= bound + 1e-30
        assert bool(ok.all()), (
            f"dW rows {v0}..{v1}: {int((~ok).sum())} elements off the identity; worst "
            f"{float((err - bound).max()):.3e} above the bound")
        worst = max(worst, float((err / (bound + 1e-30)).max()))
    return worst
