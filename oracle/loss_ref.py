"""CPU restatement of the SPLADE training loss -- test infrastructure, not product code.

Follows the reference's training/train.py:
  info_nce_loss         :73-77  scores = q d^T / T, cross entropy against labels arange(Bq)
  l1_regularization     :80-82  mean over rows of sum_v |reps|
  flops_regularization  :85-87  mean over v of (sum over rows of reps)^2
  get_reg_weight        :90-94  linear warm-up of a regulariser weight
  compute_loss          :164-197 total = CE + w_l1 (L1 q + L1 d) + w_flops (FL q + FL d)
in float64 numpy, with the gradients written out analytically.

Parity pinning (tests/test_loss_oracle.py):
  * closed forms: InfoNCE of scores c I (CE = log(1 + (Bd-1) e^{-c/T})), uniform scores
    (CE = log Bd), L1 and FLOPS of matrices whose sums are known by construction;
  * the gradients against central finite differences of the loss, and against torch
    autograd (float64, CPU) of the same formulas -- an independent differentiation;
  * invariants: the CE gradient rows of q sum to zero against constant d columns, shift
    invariance of the softmax, scaling laws L1(a x) = a L1(x), FL(a x) = a^2 FL(x).
"""
import numpy as np


def info_nce(q, d, temperature=1.0):
    """train.py:73-77. q [Bq,V], d [Bd,V], Bq <= Bd."""
    s = q.astype(np.float64) @ d.astype(np.float64).T / temperature
    m = s.max(axis=1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(s - m).sum(axis=1))
    return float(np.mean(lse - s[np.arange(s.shape[0]), np.arange(s.shape[0])]))


def info_nce_grad(q, d, temperature=1.0):
    """(dCE/dq, dCE/dd) = (P d, P^T q), P = (softmax(S) - I) / (Bq T)."""
    q64, d64 = q.astype(np.float64), d.astype(np.float64)
    s = q64 @ d64.T / temperature
    e = np.exp(s - s.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    p[np.arange(s.shape[0]), np.arange(s.shape[0])] -= 1.0
    p /= s.shape[0] * temperature
    return p @ d64, p.T @ q64


def l1(x):
    """train.py:80-82."""
    return float(np.mean(np.abs(x.astype(np.float64)).sum(axis=-1)))


def l1_grad(x):
    return np.sign(x.astype(np.float64)) / x.shape[0]


def flops(x):
    """train.py:85-87."""
    return float(np.mean(x.astype(np.float64).sum(axis=0) ** 2))


def flops_grad(x):
    cs = x.astype(np.float64).sum(axis=0)
    return np.broadcast_to(2.0 * cs / x.shape[1], x.shape).copy()


def reg_weight(step, warmup_steps, target):
    """train.py:90-94."""
    if warmup_steps <= 0:
        return target
    return target * min(1.0, step / warmup_steps)


def splade_loss(q, d, temperature=1.0, w_ce=1.0, w_l1=0.0, w_flops=0.0):
    """(total, CE, L1 q, L1 d, FL q, FL d) as in compute_loss (:178-197); d may be None."""
    ce = info_nce(q, d, temperature) if d is not None else 0.0
    l1q, flq = l1(q), flops(q)
    l1d = l1(d) if d is not None else 0.0
    fld = flops(d) if d is not None else 0.0
    total = w_ce * ce + w_l1 * (l1q + l1d) + w_flops * (flq + fld)
    return np.array([total, ce, l1q, l1d, flq, fld])


def splade_loss_grad(q, d, grad_out, temperature=1.0, w_ce=1.0, w_l1=0.0, w_flops=0.0):
    """Gradients of sum_k grad_out[k] * splade_loss(...)[k] with respect to q and d."""
    g = np.asarray(grad_out, dtype=np.float64)
    gq = (g[0] * w_l1 + g[2]) * l1_grad(q) + (g[0] * w_flops + g[4]) * flops_grad(q)
    if d is None:
        return gq, None
    cq, cd = info_nce_grad(q, d, temperature)
    gq = gq + (g[0] * w_ce + g[1]) * cq
    gd = ((g[0] * w_ce + g[1]) * cd + (g[0] * w_l1 + g[3]) * l1_grad(d)
          + (g[0] * w_flops + g[5]) * flops_grad(d))
    return gq, gd
