"""MI355X (gfx950) implementation of the SpartonHead forward and backward.

`SpartonHead` and the ops `torch.ops.sparton.fused_sparton_fwd/_bwd/_encode` run
on hand-written HIP kernels in libsparton_hip.so (C ABI: include/sparton.h).
`SpartonMLMTransform` (ops `sparton::mlm_transform_fwd/_bwd`) is the dense + gelu +
LayerNorm step that produces the head's input, its GEMMs in hipBLASLt and the rest fused.
Importing the package registers the ops; the library itself is loaded on first use
and raises if it has not been built (`python -m sparton_amd.build`).
"""
from .head import SpartonHead
from . import ops
from . import transform
from .transform import SpartonMLMTransform

__all__ = ["SpartonHead", "SpartonMLMTransform", "ops", "transform"]
