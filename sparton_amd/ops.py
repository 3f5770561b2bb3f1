"""torch.library custom ops of the SpartonHead path, backed by libsparton_hip.so.

Same op names, argument order and outputs as the reference's
(src/sparton/sparton_kernel.py:643-707):
  sparton::fused_sparton_fwd(hidden, embed, bias, mask) -> (scores, idx)
  sparton::fused_sparton_bwd(grad_out, max_scores, max_idx, hidden, embed, bias, mask)
      -> (hidden_grad, embed_grad, bias_grad)   all float32
plus fake kernels (for torch.compile tracing) and the autograd registration.
Differences: `idx` is int32 (it never leaves the op pair), `bias` may be None in
the backward too (bias_grad is then an empty tensor and autograd gets None), and
an inference-only op `sparton::fused_sparton_encode` skips the index store, and
`sparton::fused_sparton_fwd_train` (what SpartonHead trains through) also returns
the unrounded fp32 reps that its backward `sparton::fused_sparton_bwd_train` uses;
that backward writes the gradients in the parameters' dtype.

Device tensors go to the HIP kernels and nowhere else: there is no CPU or
fallback path. CPU tensors raise, like the reference's `assert hidden.is_cuda`
(:650, :673).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib

_FLOAT_DTYPES = tuple(_lib.DTYPE_CODE)


def _require_device(t: Tensor, op: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{op} only supports ROCm/HIP device tensors (got device {t.device})")


def _dense(t: Optional[Tensor]) -> Optional[Tensor]:
    """Row-major, unit inner stride, 16-byte aligned base (what the C ABI requires)."""
    if t is None:
        return None
    t = t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


def _validate(hidden: Tensor, embed: Tensor, bias: Optional[Tensor], mask: Tensor, op: str):
    if hidden.dim() != 3:
        raise ValueError(f"{op}: hidden must be [B,S,D], got shape {tuple(hidden.shape)}")
    if embed.dim() != 2 or embed.shape[1] != hidden.shape[2]:
        raise ValueError(f"{op}: embed must be [V,D] with D={hidden.shape[2]}, got {tuple(embed.shape)}")
    B, S, D = hidden.shape
    V = embed.shape[0]
    if bias is not None and tuple(bias.shape) != (V,):
        raise ValueError(f"{op}: bias must be [V]=[{V}], got {tuple(bias.shape)}")
    if tuple(mask.shape) != (B, S):
        raise ValueError(f"{op}: mask must be [B,S]=[{B},{S}], got {tuple(mask.shape)}")
    if hidden.dtype not in _FLOAT_DTYPES:
        raise TypeError(f"{op}: hidden dtype {hidden.dtype} not supported (float32/bfloat16/float16)")
    if embed.dtype != hidden.dtype or (bias is not None and bias.dtype != hidden.dtype):
        raise TypeError(f"{op}: hidden, embed and bias must share one dtype, got "
                        f"{hidden.dtype}/{embed.dtype}/{None if bias is None else bias.dtype}")
    if mask.dtype not in _lib.MASK_CODE:
        raise TypeError(f"{op}: mask dtype {mask.dtype} not supported")
    for t in (embed, bias, mask):
        if t is not None and t.device != hidden.device:
            raise ValueError(f"{op}: all tensors must be on {hidden.device}, got {t.device}")
    if (D * hidden.element_size()) % 16 != 0:
        raise ValueError(f"{op}: hidden_dim D={D} must be a multiple of {16 // hidden.element_size()} "
                         f"for {hidden.dtype} (SpartonHead pads it automatically)")
    return B, S, D, V


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _fwd_impl(hidden: Tensor, embed: Tensor, bias: Optional[Tensor], mask: Tensor,
              with_idx: bool, with_f32: bool, op: str):
    B, S, D, V = _validate(hidden, embed, bias, mask, op)
    _require_device(hidden, op)
    hidden, embed, bias, mask = _dense(hidden), _dense(embed), _dense(bias), _dense(mask)
    dev = hidden.device
    reps = torch.empty((B, V), dtype=hidden.dtype, device=dev)
    idx = torch.empty((B, V), dtype=torch.int32, device=dev) if with_idx else None
    reps32 = torch.empty((B, V), dtype=torch.float32, device=dev) if with_f32 else None
    L = _lib.load()
    dt = _lib.fwd_dtype_code(hidden.dtype)
    ws_bytes = int(L.sparton_fwd_workspace_bytes(B, S, D, V, dt))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = L.sparton_fwd(hidden.data_ptr(), embed.data_ptr(), _lib.ptr(bias), mask.data_ptr(),
                           _lib.MASK_CODE[mask.dtype], reps.data_ptr(), _lib.ptr(idx),
                           _lib.ptr(reps32), B, S, D, V, dt, ws.data_ptr(), ws_bytes,
                           _stream(dev))
    _lib.check(rc, op)
    return reps, idx, reps32


@torch.library.custom_op("sparton::fused_sparton_fwd", mutates_args=())
def fused_sparton_fwd(hidden: Tensor, embed: Tensor, bias: Optional[Tensor],
                      mask: Tensor) -> Tuple[Tensor, Tensor]:
    """reps[B,V] (hidden dtype) and argmax-over-S idx[B,V] (int32).

    Replaces fused_sparton_fwd_op (src/sparton/sparton_kernel.py:643-652)."""
    reps, idx, _ = _fwd_impl(hidden, embed, bias, mask, True, False, "sparton::fused_sparton_fwd")
    return reps, idx


@fused_sparton_fwd.register_fake
def _(hidden, embed, bias, mask):
    B, S, D = hidden.shape
    V = embed.shape[0]
    return hidden.new_empty((B, V)), hidden.new_empty((B, V), dtype=torch.int32)


@torch.library.custom_op("sparton::fused_sparton_fwd_train", mutates_args=())
def fused_sparton_fwd_train(hidden: Tensor, embed: Tensor, bias: Optional[Tensor],
                            mask: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """(reps [B,V] hidden dtype, idx [B,V] int32, reps_f32 [B,V] float32) from one kernel.

    The training forward of SpartonHead: its autograd keeps the unrounded reps_f32 for
    the backward's exp(-reps) (sparton_kernel.py:531 uses the rounded scores), so the
    gradients match the fp32 torch head instead of inheriting bf16/fp16 rounding."""
    reps, idx, reps32 = _fwd_impl(hidden, embed, bias, mask, True, True,
                                  "sparton::fused_sparton_fwd_train")
    return reps, idx, reps32


@fused_sparton_fwd_train.register_fake
def _(hidden, embed, bias, mask):
    B, S, D = hidden.shape
    V = embed.shape[0]
    return (hidden.new_empty((B, V)), hidden.new_empty((B, V), dtype=torch.int32),
            hidden.new_empty((B, V), dtype=torch.float32))


@torch.library.custom_op("sparton::fused_sparton_encode", mutates_args=())
def fused_sparton_encode(hidden: Tensor, embed: Tensor, bias: Optional[Tensor],
                         mask: Tensor) -> Tensor:
    """Inference-only forward: reps[B,V] without the argmax store.

    Serves the no-grad path (training/model.py:141-144, SpladeModel.encode) that the
    reference's dead no-index kernel targeted (src/sparton/sparton_kernel.py:262-394)."""
    reps, _, _ = _fwd_impl(hidden, embed, bias, mask, False, False, "sparton::fused_sparton_encode")
    return reps


@fused_sparton_encode.register_fake
def _(hidden, embed, bias, mask):
    return hidden.new_empty((hidden.shape[0], embed.shape[0]))


def bwd_workspace_bytes(B: int, S: int, D: int, V: int) -> int:
    return int(_lib.load().sparton_bwd_workspace_bytes(B, S, D, V))


def _bwd_impl(grad_out, max_scores, max_idx, hidden, embed, bias, mask, grad_dtype, op):
    B, S, D, V = _validate(hidden, embed, bias, mask, op)
    _require_device(grad_out, op)
    if tuple(max_scores.shape) != (B, V) or max_scores.dtype not in (hidden.dtype, torch.float32):
        raise ValueError(f"{op}: max_scores must be [{B},{V}] {hidden.dtype} or float32, "
                         f"got {tuple(max_scores.shape)} {max_scores.dtype}")
    if tuple(max_idx.shape) != (B, V) or max_idx.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{op}: max_idx must be [{B},{V}] int32 (or int64), got "
                         f"{tuple(max_idx.shape)} {max_idx.dtype}")
    if max_idx.dtype == torch.int64:
        # The reference's ops exchange int64 indices (sparton_kernel.py:658-667); accept them,
        # range-checked (this reads the tensor on the host) and narrowed to the int32 the
        # kernels take.
        if max_idx.numel() and (int(max_idx.min()) < 0 or int(max_idx.max()) >= max(S, 1)):
            raise ValueError(f"{op}: max_idx values must lie in [0, {S})")
        max_idx = max_idx.to(torch.int32)
    if tuple(grad_out.shape) != (B, V):
        raise ValueError(f"{op}: grad_out must be [{B},{V}], got {tuple(grad_out.shape)}")
    grad_out = _dense(grad_out.to(hidden.dtype))
    max_scores, max_idx = _dense(max_scores), _dense(max_idx)
    hidden, embed, bias, mask = _dense(hidden), _dense(embed), _dense(bias), _dense(mask)
    dev = hidden.device
    d_hidden = torch.empty((B, S, D), dtype=grad_dtype, device=dev)
    d_embed = torch.empty((V, D), dtype=grad_dtype, device=dev)
    d_bias = torch.empty((V if bias is not None else 0,), dtype=grad_dtype, device=dev)
    L = _lib.load()
    ws_bytes = int(L.sparton_bwd_workspace_bytes(B, S, D, V))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = L.sparton_bwd(grad_out.data_ptr(), max_scores.data_ptr(),
                           _lib.DTYPE_CODE[max_scores.dtype], max_idx.data_ptr(), mask.data_ptr(),
                           _lib.MASK_CODE[mask.dtype], hidden.data_ptr(), embed.data_ptr(),
                           d_hidden.data_ptr(), d_embed.data_ptr(),
                           d_bias.data_ptr() if bias is not None else None,
                           _lib.DTYPE_CODE[grad_dtype], ws.data_ptr(), ws_bytes, B, S, D, V,
                           _lib.DTYPE_CODE[hidden.dtype], _stream(dev))
    _lib.check(rc, op)
    return d_hidden, d_embed, d_bias


@torch.library.custom_op("sparton::fused_sparton_bwd", mutates_args=())
def fused_sparton_bwd(grad_out: Tensor, max_scores: Tensor, max_idx: Tensor, hidden: Tensor,
                      embed: Tensor, bias: Optional[Tensor],
                      mask: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """(dH [B,S,D], dW [V,D], dbias [V] or [0]) in float32.

    Replaces fused_sparton_bwd_op (src/sparton/sparton_kernel.py:663-685)."""
    return _bwd_impl(grad_out, max_scores, max_idx, hidden, embed, bias, mask, torch.float32,
                     "sparton::fused_sparton_bwd")


@fused_sparton_bwd.register_fake
def _(grad_out, max_scores, max_idx, hidden, embed, bias, mask):
    return (torch.empty_like(hidden, dtype=torch.float32),
            torch.empty_like(embed, dtype=torch.float32),
            hidden.new_empty((embed.shape[0] if bias is not None else 0,), dtype=torch.float32))


@torch.library.custom_op("sparton::fused_sparton_bwd_train", mutates_args=())
def fused_sparton_bwd_train(grad_out: Tensor, max_scores: Tensor, max_idx: Tensor,
                            hidden: Tensor, embed: Tensor, bias: Optional[Tensor],
                            mask: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """The backward of fused_sparton_fwd_train: gradients in hidden's dtype, each rounded
    once from its fp32 sum (the values autograd's cast of fp32 gradients would give,
    without the extra pass over dW and dH)."""
    return _bwd_impl(grad_out, max_scores, max_idx, hidden, embed, bias, mask, hidden.dtype,
                     "sparton::fused_sparton_bwd_train")


@fused_sparton_bwd_train.register_fake
def _(grad_out, max_scores, max_idx, hidden, embed, bias, mask):
    return (torch.empty_like(hidden), torch.empty_like(embed),
            hidden.new_empty((embed.shape[0] if bias is not None else 0,)))


def _setup_context(ctx, inputs, output):
    hidden, embed, bias, mask = inputs
    scores, idx = output
    ctx.save_for_backward(scores, idx, hidden, embed, bias, mask)


def _backward(ctx, grad_scores, grad_idx):
    # grad_idx is ignored: the index output is not differentiable.
    scores, idx, hidden, embed, bias, mask = ctx.saved_tensors
    d_hidden, d_embed, d_bias = torch.ops.sparton.fused_sparton_bwd(
        grad_scores, scores, idx, hidden, embed, bias, mask)
    return d_hidden, d_embed, (d_bias if bias is not None else None), None


fused_sparton_fwd.register_autograd(_backward, setup_context=_setup_context)


def _setup_context_train(ctx, inputs, output):
    hidden, embed, bias, mask = inputs
    _scores, idx, scores32 = output
    ctx.mark_non_differentiable(idx, scores32)
    ctx.set_materialize_grads(False)  # no zero tensors for the two index/aux outputs
    ctx.save_for_backward(scores32, idx, hidden, embed, bias, mask)


def _backward_train(ctx, grad_scores, grad_idx, grad_scores32):
    scores32, idx, hidden, embed, bias, mask = ctx.saved_tensors
    if grad_scores is None:
        return None, None, None, None
    d_hidden, d_embed, d_bias = torch.ops.sparton.fused_sparton_bwd_train(
        grad_scores, scores32, idx, hidden, embed, bias, mask)
    return d_hidden, d_embed, (d_bias if bias is not None else None), None


fused_sparton_fwd_train.register_autograd(_backward_train, setup_context=_setup_context_train)
