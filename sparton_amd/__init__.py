"""MI355X (gfx950) implementation of the SpartonHead forward and backward.

`SpartonHead` and the ops `torch.ops.sparton.fused_sparton_fwd/_bwd/_encode` run
on hand-written HIP kernels in libsparton_hip.so (C ABI: include/sparton.h).
`SpartonMLMTransform` (ops `sparton::mlm_transform_fwd/_bwd`) is the dense + gelu +
LayerNorm step that produces the head's input, its GEMMs in hipBLASLt and the rest fused.
`sparton_amd.loss` is the SPLADE training loss on the head's reps (InfoNCE + L1 + FLOPS
regularisers, ops `sparton::splade_loss_fwd/_bwd`), fused into two HIP passes.
Importing the package registers the ops; the library itself is loaded on first use
and raises if it has not been built (`python -m sparton_amd.build`).
"""
from .head import SpartonHead
from . import ops
from . import transform
from .transform import SpartonMLMTransform
from . import loss
from .loss import splade_loss

__all__ = ["SpartonHead", "SpartonMLMTransform", "ops", "transform", "loss", "splade_loss"]
