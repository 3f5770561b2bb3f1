"""The five benchmark/parity workloads and their seeded synthetic inputs.

Shapes and distributions are BASELINE.json's configs (they are not in the
reference, which ships no benchmark). Inputs are drawn on the CPU with a
torch.Generator seeded by the config index, in float32, then cast to the config
dtype, in this fixed order:
    lengths, hidden, weight, bias, grad values, grad keep-mask.
The attention mask is int64 and right-padded (mask[b, :len_b] = 1), as a
tokenizer emits it (training/train.py:122-123).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch


@dataclass(frozen=True)
class Workload:
    index: int
    name: str
    B: int
    S: int
    D: int
    V: int
    dtype: torch.dtype
    h_scale: float = 1.0
    w_std: float = 0.02
    bias: Optional[Tuple[float, float]] = (0.0, 0.02)  # (mean, std); None = use_bias=False
    lengths: Tuple[int, int] = (1, 1)                   # inclusive uniform range
    full_rows: int = 0                                  # leading rows forced to length S
    grad_density: float = 1.0                           # Bernoulli keep-rate of G

    @property
    def tokens(self) -> int:
        return self.B * self.S

    def scaled(self, **kw) -> "Workload":
        """Same distributions at other sizes (CPU-sized parity cases); lengths and
        full_rows are clamped into the new S and B."""
        d = dict(self.__dict__)
        d.update(kw)
        lo, hi = d["lengths"]
        d["lengths"] = (max(1, min(lo, d["S"])), max(1, min(hi, d["S"])))
        d["full_rows"] = min(d["full_rows"], d["B"])
        return Workload(**d)


WORKLOADS = {
    1: Workload(1, "plumbing-fp32", 2, 32, 768, 30522, torch.float32,
                bias=(0.0, 0.02), lengths=(8, 32), grad_density=1.0),
    2: Workload(2, "bert-base-bf16", 32, 256, 768, 30522, torch.bfloat16,
                bias=(-0.5, 0.1), lengths=(32, 256), grad_density=0.05),
    3: Workload(3, "long-doc-fp16", 8, 512, 768, 30522, torch.float16,
                bias=(-0.5, 0.1), lengths=(64, 512), full_rows=4, grad_density=0.05),
    4: Workload(4, "xlmr-bf16", 32, 256, 768, 250002, torch.bfloat16,
                bias=(0.0, 0.0), lengths=(16, 256), grad_density=0.05),
    5: Workload(5, "llm-bf16", 16, 512, 4096, 128256, torch.bfloat16,
                h_scale=0.5, w_std=0.01, bias=None, lengths=(128, 512), grad_density=0.05),
}

# The configuration the headline metric is quoted on (BASELINE.json metric: B32 S256 V30522 bf16).
HEADLINE = 2


@dataclass
class Inputs:
    hidden: torch.Tensor
    weight: torch.Tensor
    bias: Optional[torch.Tensor]
    mask: torch.Tensor
    grad: torch.Tensor
    lengths: torch.Tensor = field(default=None)

    def to(self, device) -> "Inputs":
        mv = lambda t: None if t is None else t.to(device)
        return Inputs(mv(self.hidden), mv(self.weight), mv(self.bias), mv(self.mask),
                      mv(self.grad), self.lengths)


def make_inputs(w: Workload, seed: Optional[int] = None, device="cpu") -> Inputs:
    g = torch.Generator().manual_seed(w.index if seed is None else seed)
    lo, hi = w.lengths
    lengths = torch.randint(lo, hi + 1, (w.B,), generator=g)
    if w.full_rows:
        lengths[: w.full_rows] = w.S
    hidden = torch.randn(w.B, w.S, w.D, generator=g) * w.h_scale
    weight = torch.randn(w.V, w.D, generator=g) * w.w_std
    bias = None
    if w.bias is not None:
        bias = torch.randn(w.V, generator=g) * w.bias[1] + w.bias[0]
    gval = torch.rand(w.B, w.V, generator=g)
    if w.grad_density < 1.0:
        keep = torch.rand(w.B, w.V, generator=g) < w.grad_density
        gval = gval * keep
    mask = (torch.arange(w.S)[None, :] < lengths[:, None]).to(torch.int64)
    cast = lambda t: None if t is None else t.to(w.dtype)
    inp = Inputs(cast(hidden), cast(weight), cast(bias), mask, cast(gval), lengths)
    return inp.to(device) if str(device) != "cpu" else inp
