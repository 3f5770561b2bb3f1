"""GPU parity of the fused SPLADE loss (training/train.py:73-94,164-197) against the float64
CPU oracle (oracle/loss_ref.py, pinned by tests/test_loss_oracle.py) on the same rounded
inputs, and against the reference's torch formulas in fp32 autograd on the GPU.

Tolerances: the six scalars rtol 1e-4 vs float64 (fp32 accumulation over up to 30522
columns is the only difference); the gradients, returned in the reps dtype, within one
rounding of that dtype relative to their largest magnitude (fp32 2e-5, fp16 2e-3,
bf16 1e-2)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import sparton_amd
from oracle import loss_ref
from sparton_amd import loss as sl
from _parity import say

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}
GRAD_TOL = {"fp32": 2e-5, "fp16": 2e-3, "bf16": 1e-2}
OUT_TOL = dict(rtol=1e-4, atol=1e-7)


def reps_like(B, V, dt, seed, density=0.3):
    """Head-like reps: log1p(relu(x)) with about `density` of the entries nonzero."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, V, generator=g) + (torch.rand(B, V, generator=g) < density).float() * 1.5 - 1.0
    return torch.log1p(torch.relu(x)).to(DT[dt])


def torch_reference(q, d, T, w_l1, w_fl):
    """The reference's functions (train.py:73-87) in fp32 autograd."""
    s = q @ d.t() / T
    ce = F.cross_entropy(s, torch.arange(q.shape[0], device=q.device))
    l1q, l1d = q.abs().sum(-1).mean(), d.abs().sum(-1).mean()
    flq, fld = (q.sum(0) ** 2).mean(), (d.sum(0) ** 2).mean()
    return torch.stack([ce + w_l1 * (l1q + l1d) + w_fl * (flq + fld), ce, l1q, l1d, flq, fld])


def close_rel(a, ref, tol, what):
    a, ref = a.detach().double().cpu(), torch.as_tensor(ref).double()
    err = (a - ref).abs().max().item()
    scale = ref.abs().max().item() + 1e-30
    assert err <= tol * scale, f"{what}: max error {err:.3e} vs {tol:.1e} x {scale:.3e}"


CASES = [  # dtype, Bq, Bd, V, T, w_l1, w_flops
    ("bf16", 32, 32, 30522, 1.0, 1e-4, 1e-4),     # config 2: train.py defaults
    ("fp32", 8, 16, 1000, 0.05, 0.3, 0.2),
    ("fp16", 1, 1, 7, 2.0, 1.0, 1.0),
    ("bf16", 64, 64, 5000, 0.5, 1e-2, 1e-3),      # the largest batch of these kernels
    ("fp32", 37, 70, 2049, 1.0, 0.1, 0.05),       # ragged rows and a partial last slice
    ("bf16", 64, 64, 64, 0.7, 0.5, 0.5),          # one slice
    ("fp32", 5, 0, 333, 1.0, 1.0, 1.0),           # query reps only (no documents)
]


@pytest.mark.parametrize("dt,Bq,Bd,V,T,w_l1,w_fl", CASES,
                         ids=[f"{c[0]}-{c[1]}x{c[2]}-V{c[3]}" for c in CASES])
def test_loss_matches_oracle(dt, Bq, Bd, V, T, w_l1, w_fl, device):
    say(f"loss {dt} Bq={Bq} Bd={Bd} V={V}")
    q = reps_like(Bq, V, dt, seed=Bq + V)
    d = reps_like(Bd, V, dt, seed=Bd + 2 * V) if Bd else None
    qd = q.to(device).requires_grad_()
    dd = d.to(device).requires_grad_() if d is not None else None
    out, probs = torch.ops.sparton.splade_loss_fwd(qd, dd, T, 1.0, w_l1, w_fl)
    g = torch.tensor([1.0, 0.3, -0.5, 0.25, 2.0, -1.5], device=device)
    out.backward(g)
    torch.cuda.synchronize()
    qn = q.double().numpy()
    dn = d.double().numpy() if d is not None else None
    want = loss_ref.splade_loss(qn, dn, T, 1.0, w_l1, w_fl)
    np.testing.assert_allclose(out.detach().double().cpu().numpy(), want, **OUT_TOL)
    gq, gd = loss_ref.splade_loss_grad(qn, dn, g.double().cpu().numpy(), T, 1.0, w_l1, w_fl)
    assert qd.grad.dtype == q.dtype
    close_rel(qd.grad, gq, GRAD_TOL[dt], "dq")
    if d is not None:
        close_rel(dd.grad, gd, GRAD_TOL[dt], "dd")
    say(f"  total {out[0].item():.6f} (oracle {want[0]:.6f})")


LARGE_CASES = [  # dtype, Bq, Bd, V
    ("fp32", 200, 200, 700),
    ("bf16", 150, 300, 2000),
    ("fp16", 129, 0, 500),        # query reps only
    ("bf16", 512, 512, 30522),    # config 2's vocabulary, 16x its batch
    ("fp32", 129, 1000, 4099),    # ragged tiles and chunks
    ("fp16", 300, 300, 31),       # fewer columns than one slice
    ("bf16", 1, 700, 3000),       # one query, many documents
    ("bf16", 65, 128, 5000),      # just past the slice-staged kernels
    ("fp32", 40, 65, 1000),       # documents alone past them
]


@pytest.mark.parametrize("dt,Bq,Bd,V", LARGE_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}-V{c[3]}" for c in LARGE_CASES])
def test_loss_large_batches_match_oracle(dt, Bq, Bd, V, device):
    """More than 64 rows on a side: the GEMM kernels (split-vocabulary score GEMM, per-slice
    statistics, row softmax; a backward that forms both gradients tile by tile), on the bf16 /
    fp16 matrix cores for 16-bit reps and the fp32 ones for fp32 reps. Values and gradients against the float64 oracle, weighting the six terms as the
    kernel test does, through splade_loss (the eager C++ op) and the single-term functions."""
    say(f"loss large batch {dt} Bq={Bq} Bd={Bd} V={V}")
    T, w_l1, w_fl = 0.5, 1e-2, 1e-3
    q = reps_like(Bq, V, dt, seed=Bq + V)
    d = reps_like(Bd, V, dt, seed=Bd + 2 * V) if Bd else None
    qd = q.to(device).requires_grad_()
    dd = d.to(device).requires_grad_() if d is not None else None
    res = sl.splade_loss(qd, dd, T, w_l1, w_fl)
    g = [1.0, 0.3, -0.5, 0.25, 2.0, -1.5] if Bd else [1.0, 0.0, -0.5, 0.0, 2.0, 0.0]
    sum(w * t for w, t in zip(g, res) if w != 0.0).backward()
    torch.cuda.synchronize()
    qn = q.double().numpy()
    dn = d.double().numpy() if d is not None else None
    want = loss_ref.splade_loss(qn, dn, T, 1.0, w_l1, w_fl)
    np.testing.assert_allclose(torch.stack(list(res)).detach().double().cpu().numpy(), want, **OUT_TOL)
    gq, gd = loss_ref.splade_loss_grad(qn, dn, np.array(g), T, 1.0, w_l1, w_fl)
    assert qd.grad.dtype == q.dtype
    close_rel(qd.grad, gq, GRAD_TOL[dt], "dq")
    if d is not None:
        close_rel(dd.grad, gd, GRAD_TOL[dt], "dd")
    np.testing.assert_allclose(sl.l1_regularization(qd).item(), want[2], rtol=1e-4)
    np.testing.assert_allclose(sl.flops_regularization(qd).item(), want[4], rtol=1e-4)
    say(f"  total {res.total.item():.6f} (oracle {want[0]:.6f})")


@pytest.mark.parametrize("dt,Bq,Bd,V", [("bf16", 300, 400, 5000), ("fp16", 130, 257, 3001),
                                         ("bf16", 1, 129, 64)])
def test_loss_large_batch_16bit_mfma_matches_fp32_mfma(dt, Bq, Bd, V, device, monkeypatch):
    """16-bit reps: the score GEMM on the 16-bit MFMA (exact products) and, for bf16, the
    gradients' products with P in two bf16 parts, against the same kernels on the fp32 MFMA
    (SPARTON_LOSS_MFMA16=0): the six terms within fp32 summation-order differences, the
    gradients within one rounding of the reps' dtype."""
    say(f"loss large batch 16-bit MFMA vs fp32 MFMA {dt} Bq={Bq} Bd={Bd} V={V}")
    q = reps_like(Bq, V, dt, seed=7).to(device)
    d = reps_like(Bd, V, dt, seed=8).to(device)
    out = []
    for mode in ("1", "0"):
        monkeypatch.setenv("SPARTON_LOSS_MFMA16", mode)
        qs, ds = q.clone().requires_grad_(), d.clone().requires_grad_()
        res = sl.splade_loss(qs, ds, 0.6, 1e-3, 1e-3)
        (res.total + 0.5 * res.contrastive).backward()
        torch.cuda.synchronize()
        out.append((torch.stack(list(res)).detach().double(), qs.grad.float(), ds.grad.float()))
    (s16, gq16, gd16), (s32, gq32, gd32) = out
    torch.testing.assert_close(s16, s32, rtol=1e-5, atol=1e-7)
    tol = {"bf16": 2 ** -7, "fp16": 2 ** -10}[dt]
    for a, b in ((gq16, gq32), (gd16, gd32)):
        scale = b.abs().max().item() + 1e-30
        assert (a - b).abs().max().item() <= tol * scale, (a - b).abs().max().item() / scale


def test_loss_large_batch_deterministic_and_paths_agree(device):
    """The large-batch kernels are bitwise reproducible, and the custom op (what torch.compile
    traces) and the eager C++ op run the same kernels."""
    q = reps_like(300, 5000, "bf16", seed=31).to(device)
    d = reps_like(400, 5000, "bf16", seed=32).to(device)
    runs = []
    for _ in range(2):
        qs, ds = q.clone().requires_grad_(), d.clone().requires_grad_()
        res = sl.splade_loss(qs, ds, 0.7, 1e-3, 1e-3)
        res.total.backward()
        runs.append((torch.stack(list(res)).detach(), qs.grad, ds.grad))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    qs, ds = q.clone().requires_grad_(), d.clone().requires_grad_()
    out, _ = torch.ops.sparton.splade_loss_fwd(qs, ds, 0.7, 1.0, 1e-3, 1e-3)
    out[0].backward()
    assert torch.equal(out.detach(), runs[0][0])
    assert torch.equal(qs.grad, runs[0][1]) and torch.equal(ds.grad, runs[0][2])


def test_loss_matches_torch_formulas_fp32(device):
    """Against train.py's own expressions (F.cross_entropy etc.) in fp32 autograd."""
    q = reps_like(16, 4000, "fp32", seed=1).to(device)
    d = reps_like(24, 4000, "fp32", seed=2).to(device)
    T, w_l1, w_fl = 0.3, 1e-3, 2e-3
    qr, dr = q.clone().requires_grad_(), d.clone().requires_grad_()
    ref = torch_reference(qr, dr, T, w_l1, w_fl)
    ref[0].backward()
    qs, ds = q.clone().requires_grad_(), d.clone().requires_grad_()
    res = sl.splade_loss(qs, ds, T, w_l1, w_fl)
    res.total.backward()
    torch.testing.assert_close(torch.stack(list(res)), ref.detach(), rtol=1e-4, atol=1e-6)
    close_rel(qs.grad, qr.grad.cpu(), 1e-4, "dq")
    close_rel(ds.grad, dr.grad.cpu(), 1e-4, "dd")
    # the single-term functions, as the reference names them
    torch.testing.assert_close(sl.info_nce_loss(q, d, T), ref[1].detach(), rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(sl.l1_regularization(q), ref[2].detach(), rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(sl.flops_regularization(d), ref[5].detach(), rtol=1e-4, atol=1e-6)


def test_loss_zero_reps(device):
    """All-zero reps: uniform scores (CE = log Bd), no L1 or FLOPS, and zero gradients."""
    q = torch.zeros(4, 300, device=device, requires_grad=True)
    d = torch.zeros(6, 300, device=device, requires_grad=True)
    res = sl.splade_loss(q, d, 1.0, 1.0, 1.0)
    res.total.backward()
    assert res.contrastive.item() == pytest.approx(np.log(6), rel=1e-6)
    assert res.l1_q.item() == 0 and res.flops_d.item() == 0
    assert torch.count_nonzero(q.grad) == 0 and torch.count_nonzero(d.grad) == 0


def test_loss_deterministic_and_modes_agree(device):
    q = reps_like(32, 30522, "bf16", seed=7).to(device)
    d = reps_like(32, 30522, "bf16", seed=8).to(device)
    runs = []
    for _ in range(2):
        qs, ds = q.clone().requires_grad_(), d.clone().requires_grad_()
        res = sl.splade_loss(qs, ds, 1.0, 1e-4, 1e-4)
        res.total.backward()
        runs.append((torch.stack(list(res)).detach(), qs.grad, ds.grad))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    # the custom-op path (what torch.compile traces) runs the same kernels
    qs, ds = q.clone().requires_grad_(), d.clone().requires_grad_()
    out, _ = torch.ops.sparton.splade_loss_fwd(qs, ds, 1.0, 1.0, 1e-4, 1e-4)
    out[0].backward()
    assert torch.equal(out.detach(), runs[0][0]) and torch.equal(qs.grad, runs[0][1])


@pytest.mark.parametrize("dt,Bq,Bd,V", [("bf16", 32, 32, 30522), ("fp32", 5, 9, 333), ("fp16", 3, 0, 100)])
def test_loss_terms_backward_equals_six_vector_backward(dt, Bq, Bd, V, device):
    """The eager op returns the six terms as separate tensors and passes the backward only
    the gradients of the terms used (NULL for the others); the custom op returns one
    six-vector whose gradient autograd assembles. Any combination of terms must give the
    same gradients, bitwise."""
    say(f"loss terms backward {dt} {Bq}x{Bd}x{V}")
    q = reps_like(Bq, V, dt, seed=11).to(device)
    d = reps_like(Bd, V, dt, seed=12).to(device) if Bd else None
    wts = [1.0, 0.5, 0.0, 2.0, 1.0, 0.0] if Bd else [1.0, 0.0, 0.25, 0.0, 3.0, 0.0]
    grads = []
    for path in ("terms", "vector"):
        qs = q.clone().requires_grad_()
        ds = d.clone().requires_grad_() if Bd else None
        if path == "terms":
            res = list(sl.splade_loss(qs, ds, 0.7, 0.1, 0.2))
        else:
            out, _ = torch.ops.sparton.splade_loss_fwd(qs, ds, 0.7, 1.0, 0.1, 0.2)
            res = list(out.unbind(0))
        sum(w * t for w, t in zip(wts, res) if w != 0.0).backward()
        grads.append((qs.grad.clone(), ds.grad.clone() if Bd else None))
    torch.cuda.synchronize()
    assert torch.equal(grads[0][0], grads[1][0])
    if Bd:
        assert torch.equal(grads[0][1], grads[1][1])


def test_head_then_loss_trains(device):
    """SpartonHead reps of queries and documents -> splade_training_loss -> backward."""
    torch.manual_seed(0)
    head = sparton_amd.SpartonHead(3000, 128, use_bias=True).to(device)
    hq = torch.randn(8, 16, 128, device=device)
    hd = torch.randn(8, 48, 128, device=device)
    mq = torch.ones(8, 16, dtype=torch.long, device=device)
    md = torch.ones(8, 48, dtype=torch.long, device=device)
    md[:, 40:] = 0
    res = sl.splade_training_loss(head(hq, mq), head(hd, md), step=5000)
    res.total.backward()
    torch.cuda.synchronize()
    assert torch.isfinite(res.total) and head.weight.grad is not None
    assert torch.isfinite(head.weight.grad).all() and head.weight.grad.abs().sum() > 0


def test_loss_opcheck_and_compile(device):
    q = reps_like(4, 200, "fp32", seed=3).to(device)
    d = reps_like(6, 200, "fp32", seed=4).to(device)
    torch.library.opcheck(torch.ops.sparton.splade_loss_fwd, (q, d, 0.5, 1.0, 0.1, 0.1),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))

    def f(a, b):
        return sl.splade_loss(a, b, 0.5, 0.1, 0.1).total

    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    torch.testing.assert_close(cf(q, d), f(q, d))


def test_loss_probs_not_differentiable(device):
    q = reps_like(4, 100, "fp32", seed=9).to(device).requires_grad_()
    d = reps_like(4, 100, "fp32", seed=10).to(device).requires_grad_()
    out, probs = torch.ops.sparton.splade_loss_fwd(q, d, 1.0, 1.0, 0.0, 0.0)
    assert out.requires_grad and not probs.requires_grad
