"""SpartonHead: the nn.Module surface of the reference, on the HIP ops.

Mirrors src/sparton/sparton_kernel.py:710-746: same constructor, parameters
(`weight` [V,D], optional `bias` [V]), `tie_weights`, `load`, `init_parameters`
and `forward(hidden_states, attention_mask) -> reps [B,V]`, so that
training/model.py:72-85 (ProjectionSparton) uses it unchanged.
"""
from __future__ import annotations

import math
import weakref

import torch
import torch.nn.functional as F
from torch import nn

from . import _eager, ops  # ops registers torch.ops.sparton.*


class _CastCache:
    """Compute-dtype copies of fp32 parameters for the autocast path, reused while the
    parameter is unchanged, so the head's calls between two optimizer steps (train.py calls
    it for queries and for documents, training/train.py:165-172) share one cast of W.

    A copy is tied to the parameter object itself (a weak reference, so a new tensor that
    reuses a freed address is a different key), its storage address, its version counter,
    dtype and padding: an in-place update (an optimizer step, load(), copy_) bumps the version
    counter, re-binding (tie_weights) changes the object, and either makes the next call cast
    again. Training also drops every copy when a backward runs through the head (a hook on
    the output's gradient): whatever updates the parameters after that backward -- including
    optimizers that write through `param.data`, which torch does not version -- is seen by
    the next forward. Inference calls with no backward in between keep their copy: update
    parameters in place under torch.no_grad() (versioned) rather than through `.data`."""

    def __init__(self):
        self._entries = {}

    def __call__(self, t, dt, pad, slot):
        key = (t.data_ptr(), t._version, tuple(t.shape), dt, pad)
        hit = self._entries.get(slot)
        if hit is not None and hit[0] == key and hit[2]() is t:
            return hit[1]
        with torch.no_grad():
            v = t.detach().to(dt)
            if pad:
                v = F.pad(v, (0, pad))
        self._entries[slot] = (key, v, weakref.ref(t))
        return v

    def clear(self):
        self._entries.clear()

    def clear_on_backward(self, out):
        """Drop the copies when the gradient of `out` is computed (the backward that precedes
        the optimizer step); returns `out`."""
        entries = self._entries

        def hook(grad):
            entries.clear()

        out.register_hook(hook)
        return out


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
        eager = hidden.is_cuda and not torch.compiler.is_compiling()
        # The reference leaves autocast to leak into its torch.compile'd GEMM; the HIP
        # op does not see autocast, so apply the autocast dtype here explicitly.
        if dev in ("cuda", "cpu") and torch.is_autocast_enabled(dev):
            dt = torch.get_autocast_dtype(dev)
            if (eager and dt in (torch.bfloat16, torch.float16) and weight.dtype == torch.float32
                    and (bias is None or bias.dtype == torch.float32)
                    and torch.is_grad_enabled()
                    and (hidden.requires_grad or weight.requires_grad
                         or (bias is not None and bias.requires_grad))):
                # Mixed-precision training: the kernels run on the cached compute-dtype copies
                # and write fp32 gradients straight to the masters (C++ autograd).
                pad = (-hidden.shape[-1]) % (128 // torch.finfo(dt).bits)  # 16-byte chunks
                wc = self._cast_cache(weight, dt, pad, "weight")
                bc = self._cast_cache(bias, dt, 0, "bias") if bias is not None else None
                _check_autocast(hidden, weight, bias, attention_mask, wc)
                out = _eager.load().head_train_autocast(hidden, weight, bias, attention_mask,
                                                        wc, bc, pad)
                return self._cast_cache.clear_on_backward(out)
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
        if eager:
            # C++ ops (autograd in C++): the same kernels as the torch.library ops below
            ops._validate(hidden, weight, bias, attention_mask, "SpartonHead")
            E = _eager.load()
            if needs_grad:
                return E.head_train(hidden, weight, bias, attention_mask)
            return E.head_encode(hidden, weight, bias, attention_mask)
        if needs_grad:
            scores, _idx, _scores32 = torch.ops.sparton.fused_sparton_fwd_train(
                hidden, weight, bias, attention_mask)
            return scores
        return torch.ops.sparton.fused_sparton_encode(hidden, weight, bias, attention_mask)


def _check_autocast(hidden, weight, bias, mask, weight_c):
    """The checks of ops._validate for the mixed-precision path (fp32 hidden and masters,
    16-bit padded weight copy)."""
    op = "SpartonHead"
    if hidden.dim() != 3 or weight.dim() != 2 or weight.shape[1] != hidden.shape[2]:
        raise ValueError(f"{op}: hidden must be [B,S,D] and weight [V,D], got "
                         f"{tuple(hidden.shape)} and {tuple(weight.shape)}")
    B, S, _ = hidden.shape
    V = weight.shape[0]
    if bias is not None and tuple(bias.shape) != (V,):
        raise ValueError(f"{op}: bias must be [V]=[{V}], got {tuple(bias.shape)}")
    if tuple(mask.shape) != (B, S):
        raise ValueError(f"{op}: mask must be [B,S]=[{B},{S}], got {tuple(mask.shape)}")
    if mask.dtype not in ops._lib.MASK_CODE:
        raise TypeError(f"{op}: mask dtype {mask.dtype} not supported")
    for t in (weight, bias, mask, weight_c):
        if t is not None and t.device != hidden.device:
            raise ValueError(f"{op}: all tensors must be on {hidden.device}, got {t.device}")
