"""The SPLADE training loss on SpartonHead's reps, fused on the GPU.

Reference: training/train.py -- info_nce_loss (:73-77), l1_regularization (:80-82),
flops_regularization (:85-87), get_reg_weight (:90-94) and their combination in
compute_loss (:164-197):

    total = CE(q, d, T) + w_l1 (L1(q) + L1(d)) + w_flops (FL(q) + FL(d))

The reference evaluates these as a dozen small torch ops over the [B, V] reps (the score
GEMM, softmax/cross entropy, abs, two sums per regulariser, squares, means). Here one HIP
pass reads q and d once and produces the partial scores and sums per 64-column vocabulary
slice, a fixed-order reduction and a one-workgroup finish give the six scalars, and one HIP
pass writes both gradients. Everything accumulates in fp32 (the reference's score GEMM
runs in the reps dtype), deterministically. Device tensors only, like the head.

    sparton::splade_loss_fwd(q, d?, temperature, w_ce, w_l1, w_flops)
        -> (out[6] fp32 = (total, CE, L1 q, L1 d, FLOPS q, FLOPS d), probs [Bq, Bd] fp32)
    sparton::splade_loss_bwd(grad_out[6], q, d?, probs, w_ce, w_l1, w_flops) -> (dq, dd)

Batches of up to 64 rows on each side take the slice-staged kernels above. Larger batches
take GEMM-shaped HIP kernels on the matrix cores (16-bit reps on the bf16/fp16 MFMA, whose
products are exact in fp32; fp32 reps on the fp32 MFMA): a split-vocabulary score GEMM with a
fixed-order sum of its partials, per-slice row and column statistics, a row softmax, and a
backward that recomputes each vocabulary slice's column sums and forms both gradients tile by
tile (sparton_loss.hip). Limits: 1 <= Bq <= Bd when documents are given (the labels
arange(Bq) index d's rows); the C ABI reports sizes past its int offsets as unsupported.
"""
from __future__ import annotations

from typing import NamedTuple, Optional, Tuple

import torch
from torch import Tensor

from . import _eager, _lib

SMALL_MAX_ROWS = 64    # rows per side taken by the slice-staged kernels (the library's own rule); larger batches take the GEMM kernels
_FLOAT_DTYPES = tuple(_lib.DTYPE_CODE)


class SpladeLossOutput(NamedTuple):
    """The scalars compute_loss (train.py:178-197) forms and logs: total is what it
    back-propagates, the others are the terms it adds up (each differentiable too)."""
    total: Tensor
    contrastive: Tensor
    l1_q: Tensor
    l1_d: Tensor
    flops_q: Tensor
    flops_d: Tensor


def _check(q: Tensor, d: Optional[Tensor], op: str) -> Tuple[int, int, int]:
    if not q.is_cuda:
        raise RuntimeError(f"{op} only supports ROCm/HIP device tensors (got device {q.device})")
    if q.dim() != 2 or q.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"{op}: query reps must be a 2-D float tensor [B, V], got {q.dtype} {tuple(q.shape)}")
    Bq, V = q.shape
    Bd = 0
    if d is not None:
        if d.dim() != 2 or d.dtype != q.dtype or d.shape[1] != V or d.device != q.device:
            raise ValueError(f"{op}: document reps must be [B, {V}] {q.dtype} on {q.device}, got "
                             f"{d.dtype} {tuple(d.shape)} on {d.device}")
        Bd = d.shape[0]
        if Bq > Bd:
            raise ValueError(f"{op}: {Bq} queries but {Bd} documents; the labels arange(Bq) "
                             "index the documents, so Bq <= Bd")
    if Bq < 1 or V < 1:
        raise ValueError(f"{op}: needs at least one query row and V >= 1, got Bq={Bq} V={V}")
    return Bq, Bd, V


def _fwd_impl(q: Tensor, d: Optional[Tensor], temperature: float, w_ce: float, w_l1: float,
              w_flops: float) -> Tuple[Tensor, Tensor]:
    op = "sparton::splade_loss_fwd"
    Bq, Bd, V = _check(q, d, op)
    if d is not None and not temperature > 0.0:
        raise ValueError(f"{op}: temperature must be > 0, got {temperature}")
    q = q.contiguous()
    d = d.contiguous() if d is not None else None
    out = torch.empty((6,), dtype=torch.float32, device=q.device)
    probs = torch.empty((Bq, Bd), dtype=torch.float32, device=q.device)
    L = _lib.load()
    nbytes = int(L.sparton_loss_workspace_bytes(Bq, Bd, V))
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = L.sparton_loss_fwd(q.data_ptr(), d.data_ptr() if d is not None else None, Bq, Bd, V,
                                float(temperature), float(w_ce), float(w_l1), float(w_flops),
                                out.data_ptr(), probs.data_ptr() if Bd else None, ws.data_ptr(),
                                nbytes, _lib.DTYPE_CODE[q.dtype],
                                torch.cuda.current_stream(q.device).cuda_stream)
    _lib.check(rc, op)
    return out, probs


def _bwd_impl(grad_out: Tensor, q: Tensor, d: Optional[Tensor], probs: Tensor, w_ce: float,
              w_l1: float, w_flops: float) -> Tuple[Tensor, Tensor]:
    op = "sparton::splade_loss_bwd"
    Bq, Bd, V = _check(q, d, op)
    q = q.contiguous()
    d = d.contiguous() if d is not None else None
    g = grad_out.to(device=q.device, dtype=torch.float32).contiguous()
    dq = torch.empty_like(q)
    dd = torch.empty_like(d) if d is not None else q.new_empty((0, V))
    L = _lib.load()
    with torch.cuda.device(q.device):
        rc = L.sparton_loss_bwd(q.data_ptr(), d.data_ptr() if d is not None else None,
                                probs.data_ptr() if Bd else None, g.data_ptr(), Bq, Bd, V,
                                float(w_ce), float(w_l1), float(w_flops), dq.data_ptr(),
                                dd.data_ptr() if d is not None else None, _lib.DTYPE_CODE[q.dtype],
                                torch.cuda.current_stream(q.device).cuda_stream)
    _lib.check(rc, op)
    return dq, dd


@torch.library.custom_op("sparton::splade_loss_fwd", mutates_args=())
def splade_loss_fwd(q: Tensor, d: Optional[Tensor], temperature: float, w_ce: float, w_l1: float,
                    w_flops: float) -> Tuple[Tensor, Tensor]:
    """(out[6], probs): out = (total, CE, L1 q, L1 d, FLOPS q, FLOPS d) in fp32; probs =
    (softmax(S) - I) / (Bq T), which the backward uses."""
    return _fwd_impl(q, d, temperature, w_ce, w_l1, w_flops)


@splade_loss_fwd.register_fake
def _(q, d, temperature, w_ce, w_l1, w_flops):
    Bd = d.shape[0] if d is not None else 0
    return q.new_empty((6,), dtype=torch.float32), q.new_empty((q.shape[0], Bd), dtype=torch.float32)


@torch.library.custom_op("sparton::splade_loss_bwd", mutates_args=())
def splade_loss_bwd(grad_out: Tensor, q: Tensor, d: Optional[Tensor], probs: Tensor, w_ce: float,
                    w_l1: float, w_flops: float) -> Tuple[Tensor, Tensor]:
    """(dq, dd) in the reps dtype; dd is [0, V] when d is None."""
    return _bwd_impl(grad_out, q, d, probs, w_ce, w_l1, w_flops)


@splade_loss_bwd.register_fake
def _(grad_out, q, d, probs, w_ce, w_l1, w_flops):
    return torch.empty_like(q), (torch.empty_like(d) if d is not None else q.new_empty((0, q.shape[1])))


def _setup_context(ctx, inputs, output):
    q, d, temperature, w_ce, w_l1, w_flops = inputs
    _out, probs = output
    ctx.has_d = d is not None
    ctx.w = (w_ce, w_l1, w_flops)
    ctx.mark_non_differentiable(probs)  # kept for the backward only
    ctx.save_for_backward(q, d if d is not None else q.new_empty(0), probs)


def _backward(ctx, g_out, _g_probs):
    q, d, probs = ctx.saved_tensors
    if g_out is None:  # out did not reach the loss
        return None, None, None, None, None, None
    dq, dd = torch.ops.sparton.splade_loss_bwd(g_out, q, d if ctx.has_d else None, probs, *ctx.w)
    return dq, (dd if ctx.has_d else None), None, None, None, None


splade_loss_fwd.register_autograd(_backward, setup_context=_setup_context)


def _run(q: Tensor, d: Optional[Tensor], temperature: float, w_ce: float, w_l1: float,
         w_flops: float) -> Tuple[Tensor, ...]:
    """The six terms (total, CE, L1(q), L1(d), FL(q), FL(d)) as separate scalars."""
    if torch.compiler.is_compiling() or not q.is_cuda:
        out, _ = torch.ops.sparton.splade_loss_fwd(q, d, temperature, w_ce, w_l1, w_flops)
        return out.unbind(0)
    # eager: the C++ op (autograd in C++), the same implementation as the custom ops; its six
    # outputs are separate, so backpropagating one term materialises no gradients of the
    # others
    _check(q, d, "splade_loss")
    if d is not None and not temperature > 0.0:
        raise ValueError(f"splade_loss: temperature must be > 0, got {temperature}")
    return _eager.load().splade_loss(q, d, float(temperature), float(w_ce), float(w_l1), float(w_flops))


def splade_loss(query_reps: Tensor, doc_reps: Optional[Tensor], temperature: float = 1.0,
                lambda_l1: float = 0.0, lambda_flops: float = 0.0) -> SpladeLossOutput:
    """InfoNCE + weighted L1 and FLOPS regularisers of both sides in one fused pass
    (train.py:178-197 with the weights already warmed up, see get_reg_weight)."""
    return SpladeLossOutput(*_run(query_reps, doc_reps, temperature, 1.0, lambda_l1, lambda_flops))


def info_nce_loss(query_reps: Tensor, doc_reps: Tensor, temperature: float = 1.0) -> Tensor:
    """In-batch negatives contrastive loss (train.py:73-77)."""
    return _run(query_reps, doc_reps, temperature, 1.0, 0.0, 0.0)[0]


def l1_regularization(reps: Tensor) -> Tensor:
    """mean_b sum_v |reps| (train.py:80-82)."""
    return _run(reps, None, 1.0, 0.0, 1.0, 0.0)[0]


def flops_regularization(reps: Tensor) -> Tensor:
    """mean_v (sum_b reps)^2 (train.py:85-87)."""
    return _run(reps, None, 1.0, 0.0, 0.0, 1.0)[0]


def get_reg_weight(current_step: int, warmup_steps: int, target_lambda: float) -> float:
    """Linear warm-up from 0 to target_lambda (train.py:90-94)."""
    if warmup_steps <= 0:
        return target_lambda
    return target_lambda * min(1.0, current_step / warmup_steps)


def splade_training_loss(query_reps: Tensor, doc_reps: Tensor, step: int, temperature: float = 1.0,
                         lambda_l1: float = 1e-4, lambda_flops: float = 1e-4,
                         reg_warmup_steps: int = 10000) -> SpladeLossOutput:
    """compute_loss's loss (train.py:164-197) at a training step: the warmed-up weights, then
    splade_loss. Defaults are LSRTrainingArguments' (train.py:50-66)."""
    return splade_loss(query_reps, doc_reps, temperature,
                       get_reg_weight(step, reg_warmup_steps, lambda_l1),
                       get_reg_weight(step, reg_warmup_steps, lambda_flops))
