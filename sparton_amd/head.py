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


class SpartonHead(nn.Module):
    def __init__(self, vocab_size, hidden_dim, use_bias=False):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(vocab_size, hidden_dim))
        if use_bias:
            self.bias = nn.Parameter(torch.empty(vocab_size))
        else:
            self.register_parameter("bias", None)
        self.init_parameters()

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
            hidden, weight = hidden.to(dt), weight.to(dt)
            bias = bias.to(dt) if bias is not None else None
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
