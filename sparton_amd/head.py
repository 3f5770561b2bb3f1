"""SpartonHead: the nn.Module surface of the reference, on the HIP ops.

Mirrors src/sparton/sparton_kernel.py:710-746: same constructor, parameters
(`weight` [V,D], optional `bias` [V]), `tie_weights`, `load`, `init_parameters`
and `forward(hidden_states, attention_mask) -> reps [B,V]`, so that
training/model.py:72-85 (ProjectionSparton) uses it unchanged.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from . import ops  # noqa: F401  (registers torch.ops.sparton.*)


class _AutocastTrainFn(torch.autograd.Function):
    """Training forward/backward under autocast with fp32 parameters (the usual
    mixed-precision setup: fp32 master weights, bf16/fp16 compute).

    The forward casts W, bias and H to the compute dtype and runs the training kernels on
    them, as the plain path does. The backward writes dH, dW and dbias in fp32 straight from
    the kernels' fp32 sums, so dW reaches the fp32 master without autograd's cast pass
    (read a [V,D] 16-bit gradient, write it again as fp32) and without being rounded to
    16 bits on the way."""

    @staticmethod
    def forward(ctx, hidden, weight, bias, mask, dt, pad, cast):
        # cast(t): the compute-dtype (zero-padded) copy of a parameter, reused while unchanged
        w = cast(weight, dt, pad, "weight")
        b = cast(bias, dt, 0, "bias") if bias is not None else None
        h = hidden.to(dt)
        if pad:
            h = F.pad(h, (0, pad))
        reps, idx, reps32 = ops._fwd_impl(h, w, b, mask, True, True,
                                          "sparton::fused_sparton_fwd_train")
        ctx.save_for_backward(reps32, idx, h, w, b, mask)
        ctx.hidden_dtype, ctx.D, ctx.has_bias = hidden.dtype, hidden.shape[-1], bias is not None
        return reps

    @staticmethod
    def backward(ctx, grad_reps):
        reps32, idx, h, w, b, mask = ctx.saved_tensors
        d_h, d_w, d_b = ops._bwd_impl(grad_reps, reps32, idx, h, w, b, mask, torch.float32,
                                      "sparton::fused_sparton_bwd")
        if d_h.shape[-1] != ctx.D:  # drop the zero padding columns
            d_h, d_w = d_h[..., :ctx.D], d_w[:, :ctx.D]
        return (d_h.to(ctx.hidden_dtype), d_w, d_b if ctx.has_bias else None, None, None, None, None)


class _CastCache:
    """Compute-dtype copies of fp32 parameters for the autocast path, reused while the
    parameter is unchanged, so the head's calls between two optimizer steps (train.py calls
    it for queries and for documents, training/train.py:165-172) share one cast of W.

    A copy is keyed on the parameter's storage address, its version counter, dtype and
    padding: an in-place update (an optimizer step, load(), copy_) bumps the version counter,
    re-binding (tie_weights) changes the address, and either makes the next call cast again.
    Writes through `param.data` are not versioned by torch and are not seen: update
    parameters in place under torch.no_grad() instead."""

    def __init__(self):
        self._entries = {}

    def __call__(self, t, dt, pad, slot):
        key = (t.data_ptr(), t._version, tuple(t.shape), dt, pad)
        hit = self._entries.get(slot)
        if hit is not None and hit[0] == key:
            return hit[1]
        with torch.no_grad():
            v = t.detach().to(dt)
            if pad:
                v = F.pad(v, (0, pad))
        self._entries[slot] = (key, v)
        return v

    def clear(self):
        self._entries.clear()


class SpartonHead(nn.Module):
    def __init__(self, vocab_size, hidden_dim, use_bias=False):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(vocab_size, hidden_dim))
        if use_bias:
            self.bias = nn.Parameter(torch.empty(vocab_size))
        else:
            self.register_parameter("bias", None)
        self.init_parameters()
        self._cast_cache = _CastCache()

    def tie_weights(self, decoder):
        """Share the MLM decoder's parameters (sparton_kernel.py:721-723)."""
        self.weight = decoder.weight
        self.bias = decoder.bias

    def load(self, weights_dict):
        """Copy `weight` (and `bias` if both sides have one) (sparton_kernel.py:725-734)."""
        with torch.no_grad():
            self.weight.copy_(weights_dict["weight"])
            if self.bias is not None and "bias" in weights_dict:
                self.bias.copy_(weights_dict["bias"])
            else:
                print("no bias")

    def init_parameters(self):
        """Kaiming-uniform(a=sqrt(5)) weight, U(+-1/sqrt(fan_in)) bias (sparton_kernel.py:736-741)."""
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in, _ = nn.init._calculate_fan_in_and_fan_out(self.weight)
            bound = 1 / math.sqrt(fan_in) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, hidden_states, attention_mask):
        hidden, weight, bias = hidden_states, self.weight, self.bias
        dev = hidden.device.type
        # The reference leaves autocast to leak into its torch.compile'd GEMM; the HIP
        # op does not see autocast, so apply the autocast dtype here explicitly.
        if dev in ("cuda", "cpu") and torch.is_autocast_enabled(dev):
            dt = torch.get_autocast_dtype(dev)
            if (dt in (torch.bfloat16, torch.float16) and weight.dtype == torch.float32
                    and (bias is None or bias.dtype == torch.float32)
                    and torch.is_grad_enabled() and not torch.compiler.is_compiling()
                    and (hidden.requires_grad or weight.requires_grad
                         or (bias is not None and bias.requires_grad))):
                pad = (-hidden.shape[-1]) % (128 // torch.finfo(dt).bits)  # 16-byte chunks
                return _AutocastTrainFn.apply(hidden, weight, bias, attention_mask, dt, pad,
                                              self._cast_cache)
            if (weight.dtype == torch.float32 and not torch.compiler.is_compiling()
                    and not (torch.is_grad_enabled() and weight.requires_grad)):
                weight = self._cast_cache(weight, dt, 0, "weight")  # inference: reuse the cast copy
                bias = self._cast_cache(bias, dt, 0, "bias") if bias is not None else None
            else:
                weight = weight.to(dt)
                bias = bias.to(dt) if bias is not None else None
            hidden = hidden.to(dt)
        elif weight.dtype != hidden.dtype:
            weight = weight.to(hidden.dtype)
            bias = bias.to(hidden.dtype) if bias is not None else None
        # The kernels read 16-byte chunks along D; zero columns change no dot product.
        step = 16 // hidden.element_size()
        pad = (-hidden.shape[-1]) % step
        if pad:
            hidden, weight = F.pad(hidden, (0, pad)), F.pad(weight, (0, pad))
        needs_grad = torch.is_grad_enabled() and (
            hidden.requires_grad or weight.requires_grad or (bias is not None and bias.requires_grad))
        if needs_grad:
            scores, _idx, _scores32 = torch.ops.sparton.fused_sparton_fwd_train(
                hidden, weight, bias, attention_mask)
            return scores
        return torch.ops.sparton.fused_sparton_encode(hidden, weight, bias, attention_mask)
