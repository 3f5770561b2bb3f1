"""CPU oracle of the SpartonHead path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this
module, and only as the checker (or as the timed CPU baseline). The product path
(sparton_amd) never imports it: device tensors go to the HIP kernels or raise.

Contents, each restating the reference (paths relative to the reference repo):
  torch_head          training/model.py:56-62 -- the repo's own torch head, the
                      correctness reference and CPU baseline named by the task.
  torch_head_chunked  the same, evaluated per V chunk (max over S is independent
                      per v, so the result is identical) to bound memory.
  fused_fwd_ref       src/sparton/sparton_kernel.py:85-168 + :226-253 semantics:
                      mask multiplies (:147), running max starts at 0 with idx 0
                      (:112-114), lowest s wins ties (:151-156), reps = log1p(M).
  logit_at            x[b, idx[b,v], v] for any index map (near-tie classification).
  fused_bwd_ref       src/sparton/sparton_kernel.py:473-565 closed form:
                      g' = G*exp(-reps) where reps > 0 (:531), dbias = sum_b g' (:536),
                      dW[v] = sum_b g' H[b, I] (:554-557), dH[b, I] += g' W[v] (:559-561),
                      times mask[b, I] (the torch head's factor; 1 for 0/1 masks).
  brute_fwd/brute_bwd pure-Python loops of the same formulas for tiny shapes; they
                      share no code with the tensor versions above.

How each function is pinned (tests/test_oracle.py): brute force on tiny shapes,
fp64 torch.autograd.gradcheck of torch_head, torch_head autograd == fused_bwd_ref
when argmaxes are unique, closed-form known-answer cases (W=0, all-masked rows,
S=1, one-hot), and invariants (V-permutation, appended masked positions,
V-chunking, sum identities). There are no reference-held golden vectors.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F


def torch_head(hidden, weight, bias, mask):
    """reps = log1p(relu((H W^T + b) * mask)).max(dim=1).values  (training/model.py:56-62)."""
    logits = F.linear(hidden, weight, bias)
    return torch.log1p(torch.relu(logits * mask.unsqueeze(-1))).max(dim=1).values


def torch_head_chunked(hidden, weight, bias, mask, v_chunk: int = 4096):
    """torch_head evaluated over V chunks; identical values, O(B*S*v_chunk) memory."""
    outs = []
    for v0 in range(0, weight.shape[0], v_chunk):
        b = None if bias is None else bias[v0:v0 + v_chunk]
        outs.append(torch_head(hidden, weight[v0:v0 + v_chunk], b, mask))
    return torch.cat(outs, dim=1)


def _auto_chunk(B, S, V, bytes_per=8, budget=1 << 28):
    return max(1, min(V, budget // max(1, B * S * bytes_per)))


def fused_fwd_ref(hidden, weight, bias, mask, acc=torch.float64, v_chunk: Optional[int] = None):
    """(M [B,V], I [B,V] int64, reps [B,V]) in `acc` precision on the given (already
    rounded) inputs. M = max(0, max_s x), I = lowest s with x == M if M > 0 else 0."""
    B, S, D = hidden.shape
    V = weight.shape[0]
    h = hidden.to(acc)
    m = mask.to(acc)
    v_chunk = v_chunk or _auto_chunk(B, S, V)
    M = torch.empty(B, V, dtype=acc)
    I = torch.empty(B, V, dtype=torch.int64)
    s_idx = torch.arange(S).view(1, S, 1)
    for v0 in range(0, V, v_chunk):
        w = weight[v0:v0 + v_chunk].to(acc)
        x = h @ w.T
        if bias is not None:
            x = x + bias[v0:v0 + v_chunk].to(acc)
        x = x * m.unsqueeze(-1)
        xm = x.max(dim=1).values
        first = torch.where(x == xm.unsqueeze(1), s_idx, S).min(dim=1).values
        Mc = torch.clamp(xm, min=0)
        M[:, v0:v0 + v_chunk] = Mc
        I[:, v0:v0 + v_chunk] = torch.where(Mc > 0, first, torch.zeros_like(first))
    return M, I, torch.log1p(M)


def logit_at(hidden, weight, bias, mask, idx, acc=torch.float64, v_chunk: int = 2048):
    """x[b, idx[b,v], v] = (H[b,idx] . W[v] + bias[v]) * mask[b, idx]  in `acc`."""
    B, S, D = hidden.shape
    V = weight.shape[0]
    idx = idx.long()
    out = torch.empty(B, V, dtype=acc)
    bidx = torch.arange(B).view(B, 1)
    for v0 in range(0, V, v_chunk):
        ii = idx[:, v0:v0 + v_chunk]
        hg = hidden[bidx, ii].to(acc)                      # [B, C, D]
        x = (hg * weight[v0:v0 + v_chunk].to(acc).unsqueeze(0)).sum(-1)
        if bias is not None:
            x = x + bias[v0:v0 + v_chunk].to(acc)
        out[:, v0:v0 + v_chunk] = x * mask[bidx, ii].to(acc)
    return out


def grad_coeff(grad, reps, idx, mask, acc=torch.float64):
    """g'[b,v] = G * exp(-reps) * mask[b, I] where reps > 0, else 0 (sparton_kernel.py:531)."""
    B = grad.shape[0]
    r = reps.to(acc)
    mI = mask[torch.arange(B).view(B, 1), idx.long()].to(acc)
    return torch.where(r > 0, grad.to(acc) * torch.exp(-r), torch.zeros_like(r)) * mI


def fused_bwd_ref(grad, reps, idx, hidden, weight, has_bias: bool, mask, acc=torch.float64,
                  chunk: int = 1 << 15, with_dW: bool = True):
    """(dH [B,S,D], dW [V,D] or None, dbias [V] or None) in `acc` (closed-form sparse
    backward). Sums run over the entries with g' != 0 only (index_add_ in fp64), in
    chunks of `chunk` entries to bound memory; zero entries contribute nothing."""
    B, S, D = hidden.shape
    V = weight.shape[0]
    gp = grad_coeff(grad, reps, idx, mask, acc)
    dbias = gp.sum(0) if has_bias else None
    nz = gp.nonzero()
    bb, vv = nz[:, 0], nz[:, 1]
    g = gp[bb, vv].unsqueeze(-1)
    ss = idx.long()[bb, vv]
    dW = torch.zeros(V, D, dtype=acc) if with_dW else None
    dH = torch.zeros(B * S, D, dtype=acc)
    for c0 in range(0, nz.shape[0], chunk):
        sl = slice(c0, c0 + chunk)
        if with_dW:
            dW.index_add_(0, vv[sl], g[sl] * hidden[bb[sl], ss[sl]].to(acc))
        dH.index_add_(0, bb[sl] * S + ss[sl], g[sl] * weight[vv[sl]].to(acc))
    return dH.view(B, S, D), dW, dbias


# ---------------------------------------------------------------------------
# Pure-Python loops (tiny shapes only): no tensor ops, no shared code.

def _tolist(t):
    return None if t is None else t.double().tolist() if t.is_floating_point() else t.tolist()


def brute_fwd(hidden, weight, bias, mask):
    """Lists M, I, reps following sparton_kernel.py:112-161 step by step: running
    max starts at 0 with index 0 and is replaced only on a strictly larger value
    while s increases, which keeps the lowest s among equal maxima."""
    H, Wl, bl, ml = _tolist(hidden), _tolist(weight), _tolist(bias), _tolist(mask)
    B, S, D = len(H), len(H[0]), len(H[0][0])
    V = len(Wl)
    M = [[0.0] * V for _ in range(B)]
    I = [[0] * V for _ in range(B)]
    for b in range(B):
        for v in range(V):
            best, arg = 0.0, 0
            for s in range(S):
                dot = 0.0
                for d in range(D):
                    dot += H[b][s][d] * Wl[v][d]
                x = (dot + (bl[v] if bl is not None else 0.0)) * float(ml[b][s])
                if x > best:
                    best, arg = x, s
            M[b][v], I[b][v] = best, arg
    reps = [[math.log1p(x) for x in row] for row in M]
    return M, I, reps


def brute_bwd(grad, reps, idx, hidden, weight, has_bias, mask):
    """Lists dH, dW, dbias by explicit loops over (b, v, d)."""
    G, R, Il, H, Wl, ml = (_tolist(grad), _tolist(reps), _tolist(idx), _tolist(hidden),
                           _tolist(weight), _tolist(mask))
    B, S, D = len(H), len(H[0]), len(H[0][0])
    V = len(Wl)
    dH = [[[0.0] * D for _ in range(S)] for _ in range(B)]
    dW = [[0.0] * D for _ in range(V)]
    db = [0.0] * V
    for b in range(B):
        for v in range(V):
            r = R[b][v]
            if not r > 0:
                continue
            s = Il[b][v]
            g = G[b][v] * math.exp(-r) * float(ml[b][s])
            db[v] += g
            for d in range(D):
                dW[v][d] += g * H[b][s][d]
                dH[b][s][d] += g * Wl[v][d]
    return dH, dW, (db if has_bias else None)
