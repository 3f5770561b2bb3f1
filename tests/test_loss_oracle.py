"""Pin the SPLADE loss oracle (oracle/loss_ref.py, restating training/train.py:73-94,164-197)
before trusting it as the checker of the HIP loss kernels.

Each function is checked against something other than its own formula: closed forms,
central finite differences, float64 torch autograd on the CPU (an independent
differentiation of the same expressions), and invariants. The last test plants plausible
mistakes in copies of the oracle and shows that these checks catch them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import loss_ref as L


def scaled_identity(n_rows, V, c):
    x = np.zeros((n_rows, V))
    x[np.arange(n_rows), np.arange(n_rows)] = math.sqrt(c)
    return x


@pytest.mark.parametrize("Bq,Bd,c,T", [(4, 4, 2.0, 1.0), (3, 7, 5.0, 0.5), (1, 1, 1.0, 2.0), (8, 16, 0.1, 0.05)])
def test_info_nce_closed_form(Bq, Bd, c, T):
    """S = c I / T: every row has one score c/T on its label and Bd - 1 zeros."""
    V = 20
    q, d = scaled_identity(Bq, V, c), scaled_identity(Bd, V, c)
    want = math.log(1.0 + (Bd - 1) * math.exp(-c / T))
    assert L.info_nce(q, d, T) == pytest.approx(want, rel=1e-12)


def test_info_nce_uniform_scores_and_shift():
    rng = np.random.default_rng(0)
    d = rng.random((6, 30))
    assert L.info_nce(np.zeros((4, 30)), d) == pytest.approx(math.log(6), rel=1e-12)
    # adding one vector u to every document row adds q_i . u to the whole row i of S
    q = rng.random((4, 30))
    u = rng.random(30)
    assert L.info_nce(q, d + u, 0.7) == pytest.approx(L.info_nce(q, d, 0.7), rel=1e-10)


def test_l1_and_flops_known_sums():
    V = 11
    a = np.array([0.5, 2.0, 0.0, 3.25])
    x = np.repeat(a[:, None], V, axis=1)             # row b is a_b everywhere
    assert L.l1(x) == pytest.approx(a.sum() * V / len(a), rel=1e-12)
    assert L.flops(x) == pytest.approx(a.sum() ** 2, rel=1e-12)   # every column sums to sum(a)
    y = np.zeros((3, V))
    y[:, 2] = [1.0, 2.0, 4.0]                         # one active column
    assert L.flops(y) == pytest.approx(49.0 / V, rel=1e-12)
    assert L.l1(y) == pytest.approx(7.0 / 3, rel=1e-12)
    assert L.l1(2.5 * x) == pytest.approx(2.5 * L.l1(x), rel=1e-12)
    assert L.flops(2.5 * x) == pytest.approx(6.25 * L.flops(x), rel=1e-12)


def test_reg_weight():
    assert L.reg_weight(0, 100, 1e-3) == 0.0
    assert L.reg_weight(50, 100, 1e-3) == pytest.approx(5e-4)
    assert L.reg_weight(500, 100, 1e-3) == 1e-3
    assert L.reg_weight(7, 0, 1e-3) == 1e-3


def _case(Bq, Bd, V, seed):
    rng = np.random.default_rng(seed)
    q = rng.random((Bq, V)) * 2.0 + 0.05                 # reps >= 0, away from 0 for the FD
    d = rng.random((Bd, V)) * 2.0 + 0.05 if Bd else None
    return q, d


def _total(q, d, g, T, w):
    return float(np.dot(g, L.splade_loss(q, d, T, *w)))


def _fd_grads(q, d, g, T, w, h=1e-6):
    """Central finite differences of sum_k g[k] * splade_loss(q, d)[k]."""
    out = []
    for x in (q, d):
        if x is None:
            out.append(None)
            continue
        num = np.zeros_like(x)
        for idx in np.ndindex(*x.shape):
            x[idx] += h
            fp = _total(q, d, g, T, w)
            x[idx] -= 2 * h
            fm = _total(q, d, g, T, w)
            x[idx] += h
            num[idx] = (fp - fm) / (2 * h)
        out.append(num)
    return out


def _fd_agrees(grads, fd):
    return all(a is None or np.allclose(a, b, rtol=1e-6, atol=1e-8) for a, b in zip(grads, fd))


@pytest.mark.parametrize("Bq,Bd", [(3, 5), (4, 4), (2, 0)])
def test_grad_matches_finite_differences(Bq, Bd):
    V, T, w = 9, 0.6, (1.0, 0.3, 0.7)
    q, d = _case(Bq, Bd, V, seed=Bq * 10 + Bd)
    g = np.array([1.0, 0.2, -0.4, 0.5, 0.9, -1.1])
    gq, gd = L.splade_loss_grad(q, d, g, T, *w)
    fq, fdd = _fd_grads(q, d, g, T, w)
    np.testing.assert_allclose(gq, fq, rtol=1e-6, atol=1e-8)
    if gd is not None:
        np.testing.assert_allclose(gd, fdd, rtol=1e-6, atol=1e-8)


def test_grad_matches_torch_autograd_float64():
    """The same expressions differentiated by torch autograd (float64, CPU), with exact
    zeros in the reps: abs has gradient 0 there, as torch's sign(0) = 0."""
    rng = np.random.default_rng(5)
    q = rng.random((6, 40)) * (rng.random((6, 40)) > 0.5)
    d = rng.random((8, 40)) * (rng.random((8, 40)) > 0.5)
    T, w = 0.25, (1.0, 1e-2, 3e-2)
    tq = torch.tensor(q, requires_grad=True)
    td = torch.tensor(d, requires_grad=True)
    s = tq @ td.t() / T
    ce = torch.nn.functional.cross_entropy(s, torch.arange(6))
    l1q, l1d = tq.abs().sum(-1).mean(), td.abs().sum(-1).mean()
    flq, fld = (tq.sum(0) ** 2).mean(), (td.sum(0) ** 2).mean()
    total = w[0] * ce + w[1] * (l1q + l1d) + w[2] * (flq + fld)
    parts = torch.stack([total, ce, l1q, l1d, flq, fld])
    np.testing.assert_allclose(L.splade_loss(q, d, T, *w), parts.detach().numpy(), rtol=1e-12)
    g = torch.tensor([1.0, 0.5, -2.0, 0.25, 3.0, -0.75], dtype=torch.float64)
    (parts * g).sum().backward()
    gq, gd = L.splade_loss_grad(q, d, g.numpy(), T, *w)
    np.testing.assert_allclose(gq, tq.grad.numpy(), rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(gd, td.grad.numpy(), rtol=1e-10, atol=1e-14)


def test_ce_gradient_rows_orthogonal_to_constant_columns():
    """sum_j P[i,j] = 0 for every row, so dCE/dq is orthogonal to any column direction that
    is constant over the documents; here: the documents share column 0."""
    rng = np.random.default_rng(2)
    q, d = rng.random((4, 10)), rng.random((6, 10))
    d[:, 0] = 0.37
    gq, _ = L.info_nce_grad(q, d, 0.5)
    np.testing.assert_allclose(gq[:, 0], 0.0, atol=1e-14)


def test_planted_mistakes_are_caught(monkeypatch):
    """Plausible slips planted in copies of the oracle's gradient pieces fail the
    finite-difference check that the real ones pass."""
    q, d = _case(3, 5, 7, seed=11)
    T, w = 0.4, (1.0, 0.1, 0.1)
    g = np.array([1.0, 0.0, 0.0, 0.0, 0.0, 0.0])
    fd = _fd_grads(q, d, g, T, w)
    good_nce, good_fl = L.info_nce_grad, L.flops_grad

    def nce_no_temperature(q_, d_, t_):                 # dropped the 1/T
        return good_nce(q_, d_, 1.0)

    def nce_variant(axis, one_hot):
        def grad(q_, d_, t_):
            s_ = q_ @ d_.T / t_
            e = np.exp(s_ - s_.max(axis=axis, keepdims=True))
            p = e / e.sum(axis=axis, keepdims=True)
            if one_hot:
                p[np.arange(q_.shape[0]), np.arange(q_.shape[0])] -= 1.0
            p /= q_.shape[0] * t_
            return p @ d_, p.T @ q_
        return grad

    def flops_mean_over_rows(x):                        # mean over b instead of over v
        return np.broadcast_to(2.0 * x.sum(axis=0) / x.shape[0], x.shape).copy()

    assert _fd_agrees(L.splade_loss_grad(q, d, g, T, *w), fd)
    for name, fn in (("info_nce_grad", nce_no_temperature),
                     ("info_nce_grad", nce_variant(axis=0, one_hot=True)),   # softmax over queries
                     ("info_nce_grad", nce_variant(axis=1, one_hot=False)),  # label term dropped
                     ("flops_grad", flops_mean_over_rows)):
        with monkeypatch.context() as m:
            m.setattr(L, name, fn)
            assert not _fd_agrees(L.splade_loss_grad(q, d, g, T, *w), fd), name
    assert L.info_nce_grad is good_nce and L.flops_grad is good_fl
