"""GPU parity of the MLM transform (dense -> gelu -> LayerNorm, training/model.py:14-40):
the fused HIP epilogues around hipBLASLt GEMMs against a plain PyTorch fp32 reference
of the same op, forward and backward. The reference is computed in fp32 on the GPU from
the same (rounded) inputs; the tolerances below are written per dtype."""
import pytest
import torch
import torch.nn.functional as F

import sparton_amd  # noqa: F401  (registers the ops)
from sparton_amd import SpartonMLMTransform
from _parity import say

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}
# Max error relative to the reference's max magnitude. z = x W^T is rounded to the
# compute dtype once (as a bf16/fp16 GEMM output), which bounds the low-precision paths.
TOL = {"fp32": 2e-5, "bf16": 2.5e-2, "fp16": 4e-3}


def reference(x, w, b, g, bt, eps):
    """fp32 torch: LayerNorm(gelu(x W^T + b)), exact gelu."""
    return F.layer_norm(F.gelu(F.linear(x.float(), w.float(), b.float())), (x.shape[-1],),
                        g.float(), bt.float(), eps)


def case(dt, shape, D, seed=0, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, D, generator=gen) * scale).to(DT[dt])
    w = (torch.randn(D, D, generator=gen) / D ** 0.5).to(DT[dt])
    b = torch.randn(D, generator=gen) * 0.1
    g = 1.0 + 0.1 * torch.randn(D, generator=gen)
    bt = 0.1 * torch.randn(D, generator=gen)
    dy = torch.randn(*shape, D, generator=gen).to(DT[dt])
    return x, w, b, g, bt, dy


def close(a, ref, tol, what):
    a, ref = a.float(), ref.float()
    err = (a - ref).abs().max().item()
    scale = ref.abs().max().item() + 1e-30
    assert err <= tol * scale, f"{what}: max error {err:.3e} vs {tol:.1e} x {scale:.3e}"
    return err / scale


CASES = [
    ("bf16", (32, 256), 768, 1e-12),   # BERT-base at config 2's shape
    ("fp16", (8, 512), 768, 1e-12),    # config 3's shape
    ("fp32", (5, 7), 64, 1e-5),
    ("bf16", (3, 33), 1024, 1e-5),     # BERT-large / XLM-R large width, ragged rows
    ("fp16", (100,), 3072, 1e-5),      # the largest D the kernels take
    ("fp32", (2, 3), 4, 1e-12),        # one partial pass
    ("bf16", (1, 1), 12, 1e-5),
    ("fp32", (2050,), 768, 1e-12),     # 2 rows per backward wave, last workgroup partial
    ("fp16", (16411,), 256, 1e-5),     # 9 rows per wave, ragged
    ("bf16", (4133,), 1540, 1e-5),     # wide rows (4-wave backward), partial last pass
    ("fp32", (9, 64), 2048, 1e-12),    # wide rows, full passes
    ("bf16", (64, 512), 768, 1e-12),   # M = 32768: dW as 16 row chunks
    ("bf16", (16, 512), 1024, 1e-5),   # BERT-large width, dW as 8 row chunks
    ("fp16", (300,), 1500, 1e-5),      # wide rows, lanes past the row end in the 6th pass
    ("bf16", (2, 40), 3000, 1e-5),     # widest passes, the last one partial
]


@pytest.mark.parametrize("dt,shape,D,eps", CASES, ids=[f"{c[0]}-{'x'.join(map(str, c[1]))}-{c[2]}" for c in CASES])
def test_transform_matches_torch_fp32(dt, shape, D, eps, device):
    say(f"transform {dt} {shape} D={D}")
    x, w, b, g, bt, dy = case(dt, shape, D)
    x, w, b, g, bt, dy = (t.to(device) for t in (x, w, b, g, bt, dy))
    xr = x.float().clone().requires_grad_()
    wr, br, gr, btr = (t.float().clone().requires_grad_() for t in (w, b, g, bt))
    yr = reference(xr, wr, br, gr, btr, eps)
    yr.backward(dy.float())

    xs = x.clone().requires_grad_()
    ws, bs, gs, bts = w.clone().requires_grad_(), b.clone().requires_grad_(), g.clone().requires_grad_(), bt.clone().requires_grad_()
    y, z, mean, rstd = torch.ops.sparton.mlm_transform_fwd(xs, ws, bs, gs, bts, eps)
    y.backward(dy)
    torch.cuda.synchronize()
    tol = TOL[dt]
    assert y.dtype == x.dtype and y.shape == x.shape
    e = close(y, yr, tol, "y")
    close(xs.grad, xr.grad, 2 * tol, "dx")
    close(ws.grad, wr.grad, 2 * tol, "dW")
    close(bs.grad, br.grad, 2 * tol, "d dense bias")
    close(gs.grad, gr.grad, 2 * tol, "d ln weight")
    close(bts.grad, btr.grad, 2 * tol, "d ln bias")
    say(f"  y rel err {e:.2e}")


def test_transform_row_statistics(device):
    """mean and 1/std are those of gelu(z + b) per row (the backward recomputes xhat from them)."""
    x, w, b, g, bt, _ = case("fp32", (16,), 256, seed=3)
    x, w, b, g, bt = (t.to(device) for t in (x, w, b, g, bt))
    _, z, mean, rstd = torch.ops.sparton.mlm_transform_fwd(x, w, b, g, bt, 1e-5)
    u = F.gelu(z.float() + b)
    torch.testing.assert_close(mean, u.mean(-1), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(rstd, torch.rsqrt(u.var(-1, unbiased=False) + 1e-5), rtol=1e-4, atol=1e-5)


def test_transform_deterministic(device):
    x, w, b, g, bt, dy = (t.to(device) for t in case("bf16", (32, 256), 768, seed=1))
    outs = []
    for _ in range(2):
        y, z, mean, rstd = torch.ops.sparton.mlm_transform_fwd(x, w, b, g, bt, 1e-12)
        grads = torch.ops.sparton.mlm_transform_bwd(dy, x, w, z, b, g, mean, rstd)
        outs.append([t.clone() for t in (y, mean, rstd) + tuple(grads)])
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


def test_transform_module_autograd_and_autocast(device):
    """SpartonMLMTransform over shared nn.Linear / nn.LayerNorm parameters (fp32 masters)
    matches the same modules evaluated by torch, in fp32 and under bf16 autocast."""
    torch.manual_seed(0)
    dense = torch.nn.Linear(768, 768).to(device)
    ln = torch.nn.LayerNorm(768, eps=1e-12).to(device)
    m = SpartonMLMTransform(dense, ln)
    x = torch.randn(4, 64, 768, device=device)
    y = m(x)
    ref = ln(F.gelu(dense(x)))
    close(y, ref, 2e-5, "fp32 module")
    # A random upstream gradient: y.sum() alone would give dense gradients that cancel to
    # roundoff, since LayerNorm's backward removes each row's mean and xhat component.
    dy = torch.randn_like(y)
    params = [dense.weight, dense.bias, ln.weight, ln.bias]
    g = torch.autograd.grad(y, params, dy)
    gr = torch.autograd.grad(ref, params, dy)
    for a, r, n in zip(g, gr, ("dW", "d dense bias", "d ln weight", "d ln bias")):
        assert a.dtype == torch.float32
        close(a, r, 1e-4, n)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ya = m(x)
    assert ya.dtype == torch.bfloat16
    close(ya, ref, 3e-2, "bf16 autocast module")
    # the module's autograd function and the custom ops run the same kernels: bitwise equal
    vecs = [dense.bias, ln.weight, ln.bias]
    y_op = torch.ops.sparton.mlm_transform_fwd(x, dense.weight, *vecs, 1e-12)[0]
    g_op = torch.autograd.grad(y_op, params, dy)
    assert torch.equal(y_op, y)
    for a, b in zip(g_op, g):
        assert torch.equal(a, b)


def test_transform_feeds_the_head(device):
    """The transform's output is the head's hidden input: transform -> SpartonHead trains."""
    torch.manual_seed(0)
    dense = torch.nn.Linear(256, 256).to(device)
    ln = torch.nn.LayerNorm(256, eps=1e-12).to(device)
    head = sparton_amd.SpartonHead(500, 256, use_bias=True).to(device)
    x = torch.randn(2, 16, 256, device=device, requires_grad=True)
    mask = torch.ones(2, 16, dtype=torch.long, device=device)
    mask[1, 10:] = 0
    reps = head(SpartonMLMTransform(dense, ln)(x), mask)
    reps.sum().backward()
    torch.cuda.synchronize()
    for t in (x.grad, dense.weight.grad, ln.weight.grad, head.weight.grad):
        assert t is not None and torch.isfinite(t).all()
    assert x.grad.abs().sum() > 0


def test_transform_opcheck(device):
    x, w, b, g, bt, dy = (t.to(device) for t in case("fp32", (3, 5), 64, seed=2))
    torch.library.opcheck(torch.ops.sparton.mlm_transform_fwd, (x, w, b, g, bt, 1e-5),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))


def test_weight_grad_chunk_kernels(device):
    """The chunked dW pieces on their own: the K-contiguous chunks of dz and the ordered
    chunk sum, against torch; and dW itself against one fp32 GEMM."""
    from sparton_amd import _lib
    from sparton_amd.transform import _weight_grad, _wgrad_chunks
    L = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for dt, M, D in (("bf16", 8192, 768), ("fp16", 4096, 1024), ("bf16", 32768, 256)):
        C = _wgrad_chunks(M, D, DT[dt])
        assert C in (4, 8, 16)
        gen = torch.Generator(device=device).manual_seed(M + D)
        dz = torch.randn(M, D, device=device, generator=gen).to(DT[dt])
        x = torch.randn(M, D, device=device, generator=gen).to(DT[dt])
        dzt = torch.empty(C, D, M // C, dtype=DT[dt], device=device)
        assert L.sparton_transform_dz_chunks(dz.data_ptr(), dzt.data_ptr(), M, D, C, 1 if dt == "bf16" else 2, stream) == 0
        assert torch.equal(dzt, dz.view(C, M // C, D).transpose(1, 2))
        part = torch.randn(C, D * D, device=device, generator=gen)
        out = torch.empty(D * D, dtype=torch.float32, device=device)
        assert L.sparton_transform_chunk_sum(part.data_ptr(), out.data_ptr(), C, D * D, 0, stream) == 0
        want = part[0].clone()
        for c in range(1, C):
            want += part[c]
        assert torch.equal(out, want)  # same order, same fp32 additions
        dw = _weight_grad(L, dz, x, M, D)
        ref = dz.float().t() @ x.float()
        close(dw, ref, 2 ** -8, f"dW {dt} M={M} D={D}")
        assert torch.equal(_weight_grad(L, dz, x, M, D), dw)


def test_transform_auxiliary_outputs_not_differentiable(device):
    """z, mean and 1/std exist for the backward: autograd does not track them, and a loss
    that uses only y gives the same gradients whatever else is read."""
    x, w, b, g, bt, dy = (t.to(device) for t in case("fp32", (6,), 64, seed=4))
    x.requires_grad_()
    y, z, mean, rstd = torch.ops.sparton.mlm_transform_fwd(x, w, b, g, bt, 1e-5)
    assert y.requires_grad and not (z.requires_grad or mean.requires_grad or rstd.requires_grad)
