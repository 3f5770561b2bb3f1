"""The MLM transform in front of SpartonHead: dense (D x D) -> gelu (erf) -> LayerNorm.

Reference: training/model.py:14-40 (BERT's cls.predictions.transform; RoBERTa's lm_head
dense, gelu and layer_norm), applied to the backbone's hidden states just before the
head (:56-58). Its output is the head's `hidden` input.

The two D x D GEMMs (x W^T forward; dz W and dz^T x backward) are plain library GEMMs
(hipBLASLt through torch, on the current stream). Everything fused around them runs in
libsparton_hip.so: bias + gelu + LayerNorm with the row statistics (sparton_transform_fwd),
and the LayerNorm and gelu backward with deterministic column sums for the LayerNorm and
dense-bias gradients (sparton_transform_bwd). Device tensors only, like the head.

    sparton::mlm_transform_fwd(x, weight, dense_bias, ln_weight, ln_bias, eps)
        -> (y, z, mean, rstd)        y in x's dtype; z = x W^T, mean and 1/std are kept for
                                     the backward and are not differentiable
    sparton::mlm_transform_bwd(dy, x, weight, z, dense_bias, ln_weight, mean, rstd)
        -> (dx, d_weight, d_dense_bias, d_ln_weight, d_ln_bias)
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _eager, _lib

_FLOAT_DTYPES = tuple(_lib.DTYPE_CODE)


def _check(x: Tensor, weight: Tensor, vecs, op: str) -> int:
    if not x.is_cuda:
        raise RuntimeError(f"{op} only supports ROCm/HIP device tensors (got device {x.device})")
    D = x.shape[-1]
    if weight.dim() != 2 or tuple(weight.shape) != (D, D):
        raise ValueError(f"{op}: weight must be [D,D]=[{D},{D}], got {tuple(weight.shape)}")
    if x.dtype not in _FLOAT_DTYPES or weight.dtype != x.dtype:
        raise TypeError(f"{op}: x and weight must share a float dtype, got {x.dtype}/{weight.dtype}")
    for v in vecs:
        if tuple(v.shape) != (D,) or v.dtype != torch.float32:
            raise ValueError(f"{op}: bias and LayerNorm vectors must be float32 [{D}], got "
                             f"{v.dtype} {tuple(v.shape)}")
    for t in (weight,) + tuple(vecs):
        if t.device != x.device:
            raise ValueError(f"{op}: all tensors must be on {x.device}, got {t.device}")
    if D % 4 != 0 or D > 3072:
        raise ValueError(f"{op}: hidden size {D} must be a multiple of 4 and at most 3072")
    return D


def _fwd_impl(x: Tensor, weight: Tensor, dense_bias: Tensor, ln_weight: Tensor,
              ln_bias: Tensor, eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    op = "sparton::mlm_transform_fwd"
    D = _check(x, weight, (dense_bias, ln_weight, ln_bias), op)
    x2 = x.reshape(-1, D)
    z = F.linear(x2, weight)  # hipBLASLt
    M = z.shape[0]
    y = torch.empty_like(z)
    mean = torch.empty((M,), dtype=torch.float32, device=x.device)
    rstd = torch.empty((M,), dtype=torch.float32, device=x.device)
    L = _lib.load()
    vb, vg, vt = dense_bias.contiguous(), ln_weight.contiguous(), ln_bias.contiguous()
    with torch.cuda.device(x.device):
        rc = L.sparton_transform_fwd(z.data_ptr(), vb.data_ptr(), vg.data_ptr(), vt.data_ptr(),
                                     float(eps), y.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                                     M, D, _lib.DTYPE_CODE[x.dtype],
                                     torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, op)
    return y.view(x.shape), z, mean, rstd


@torch.library.custom_op("sparton::mlm_transform_fwd", mutates_args=())
def mlm_transform_fwd(x: Tensor, weight: Tensor, dense_bias: Tensor, ln_weight: Tensor,
                      ln_bias: Tensor, eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """y = LayerNorm(gelu(x W^T + b)) (x's dtype), with z = x W^T and each row's mean and
    1/std, which the backward uses."""
    return _fwd_impl(x, weight, dense_bias, ln_weight, ln_bias, eps)


@mlm_transform_fwd.register_fake
def _(x, weight, dense_bias, ln_weight, ln_bias, eps):
    D = x.shape[-1]
    M = x.numel() // D if D else 0
    return (x.new_empty(x.shape), x.new_empty((M, D)), x.new_empty((M,), dtype=torch.float32),
            x.new_empty((M,), dtype=torch.float32))


def _bwd_impl(dy: Tensor, x: Tensor, weight: Tensor, z: Tensor, dense_bias: Tensor,
              ln_weight: Tensor, mean: Tensor, rstd: Tensor
              ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    op = "sparton::mlm_transform_bwd"
    D = _check(x, weight, (dense_bias, ln_weight), op)
    x2 = x.reshape(-1, D)
    M = x2.shape[0]
    dy2 = dy.reshape(-1, D).to(x.dtype).contiguous()
    dz = torch.empty_like(z)
    dg = torch.empty((D,), dtype=torch.float32, device=x.device)
    dbt = torch.empty_like(dg)
    dbd = torch.empty_like(dg)
    L = _lib.load()
    nbytes = int(L.sparton_transform_workspace_bytes(M, D))
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=x.device)
    vb, vg = dense_bias.contiguous(), ln_weight.contiguous()
    with torch.cuda.device(x.device):
        rc = L.sparton_transform_bwd(dy2.data_ptr(), z.data_ptr(), vb.data_ptr(), vg.data_ptr(),
                                     mean.data_ptr(), rstd.data_ptr(), dz.data_ptr(), dg.data_ptr(),
                                     dbt.data_ptr(), dbd.data_ptr(), ws.data_ptr(), nbytes, M, D,
                                     _lib.DTYPE_CODE[x.dtype],
                                     torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(rc, op)
    dx = torch.mm(dz, weight)        # hipBLASLt
    dw = _weight_grad(L, dz, x2, M, D)
    return dx.view(x.shape), dw, dbd, dg, dbt


def _wgrad_chunks(M: int, D: int, dtype: torch.dtype) -> int:
    """Row chunks C of the batched dW GEMM, or 0 for one plain GEMM. Measured on MI355X at
    D = 768 bf16, dz^T x as one hipBLASLt GEMM takes 28 / 50 / 187 us at M = 4096 / 8192 /
    32768 (a D x D output is too few tiles for K = M); C = 4 / 8 / 16 chunks take 15 / 20 / 57
    us for the batched GEMM."""
    if dtype not in (torch.bfloat16, torch.float16) or M < 2048 or D % 64:
        return 0
    C = 4 if M <= 4096 else (8 if M <= 16384 else 16)
    return C if M % (C * 64) == 0 else 0


def _weight_grad(L, dz: Tensor, x2: Tensor, M: int, D: int) -> Tensor:
    """dW = dz^T x2. Split into C row chunks: dz's chunks transposed to K-contiguous [D, M/C]
    (HIP), one batched GEMM with fp32 outputs (hipBLASLt; x2's chunks are views), and the C
    products summed in chunk order and cast once (HIP): deterministic, one rounding."""
    C = _wgrad_chunks(M, D, dz.dtype)
    if C == 0:
        return torch.mm(dz.t(), x2)  # hipBLASLt (what F.linear's weight gradient does)
    code = _lib.DTYPE_CODE[dz.dtype]
    stream = torch.cuda.current_stream(dz.device).cuda_stream
    dzt = torch.empty((C, D, M // C), dtype=dz.dtype, device=dz.device)
    with torch.cuda.device(dz.device):
        _lib.check(L.sparton_transform_dz_chunks(dz.data_ptr(), dzt.data_ptr(), M, D, C, code, stream),
                   "sparton_transform_dz_chunks")
    part = torch.bmm(dzt, x2.contiguous().view(C, M // C, D), out_dtype=torch.float32)
    dw = torch.empty((D, D), dtype=dz.dtype, device=dz.device)
    with torch.cuda.device(dz.device):
        _lib.check(L.sparton_transform_chunk_sum(part.data_ptr(), dw.data_ptr(), C, D * D, code, stream),
                   "sparton_transform_chunk_sum")
    return dw


@torch.library.custom_op("sparton::mlm_transform_bwd", mutates_args=())
def mlm_transform_bwd(dy: Tensor, x: Tensor, weight: Tensor, z: Tensor, dense_bias: Tensor,
                      ln_weight: Tensor, mean: Tensor, rstd: Tensor
                      ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dx, d_weight, d_dense_bias, d_ln_weight, d_ln_bias); dx and d_weight in x's dtype,
    the vectors in float32."""
    return _bwd_impl(dy, x, weight, z, dense_bias, ln_weight, mean, rstd)


@mlm_transform_bwd.register_fake
def _(dy, x, weight, z, dense_bias, ln_weight, mean, rstd):
    D = x.shape[-1]
    v = dense_bias.new_empty((D,))
    return x.new_empty(x.shape), weight.new_empty(weight.shape), v, v.clone(), v.clone()


def _setup_context(ctx, inputs, output):
    x, weight, dense_bias, ln_weight, ln_bias, eps = inputs
    _y, z, mean, rstd = output
    ctx.mark_non_differentiable(z, mean, rstd)  # kept for the backward only
    ctx.save_for_backward(x, weight, z, dense_bias, ln_weight, mean, rstd)


def _backward(ctx, dy, _dz, _dmean, _drstd):
    x, weight, z, dense_bias, ln_weight, mean, rstd = ctx.saved_tensors
    if dy is None:  # y did not reach the loss
        return None, None, None, None, None, None
    dx, dw, dbd, dg, dbt = torch.ops.sparton.mlm_transform_bwd(dy, x, weight, z, dense_bias,
                                                              ln_weight, mean, rstd)
    return dx, dw, dbd, dg, dbt, None


mlm_transform_fwd.register_autograd(_backward, setup_context=_setup_context)


def _is_erf_gelu(act) -> bool:
    """torch's F.gelu / nn.GELU() without the tanh approximation, or transformers'
    GELUActivation (hidden_act "gelu" or "gelu_python", both the erf form)."""
    if act is F.gelu:
        return True
    if isinstance(act, nn.GELU):
        return act.approximate == "none"
    return type(act).__name__ == "GELUActivation"


class SpartonMLMTransform(nn.Module):
    """Drop-in for the transform: shares the parameters of an existing dense (nn.Linear
    D x D) and LayerNorm, e.g. BERT's `cls.predictions.transform.dense` and `.LayerNorm` or
    RoBERTa's `lm_head.dense` and `.layer_norm` (training/model.py:14-40)."""

    def __init__(self, dense: nn.Linear, layer_norm: nn.LayerNorm):
        super().__init__()
        D = dense.in_features
        if dense.out_features != D or dense.bias is None:
            raise ValueError("dense must be a square nn.Linear with bias")
        if tuple(layer_norm.normalized_shape) != (D,) or not layer_norm.elementwise_affine:
            raise ValueError(f"layer_norm must be an affine LayerNorm over {D}")
        self.dense = dense
        self.layer_norm = layer_norm

    @classmethod
    def from_hf(cls, transform: nn.Module) -> "SpartonMLMTransform":
        """From BERT's BertPredictionHeadTransform (dense, transform_act_fn, LayerNorm) or a
        module with `dense` and `layer_norm` (the RoBERTa wrapper of training/model.py:25-34,
        whose activation is transformers' erf gelu). The kernels compute the exact (erf) gelu,
        so a BERT transform configured with another activation is refused."""
        act = getattr(transform, "transform_act_fn", None)
        if act is not None and not _is_erf_gelu(act):
            raise ValueError(f"SpartonMLMTransform computes the exact (erf) gelu; this transform's "
                             f"activation is {act!r}")
        ln = getattr(transform, "LayerNorm", None) or getattr(transform, "layer_norm")
        return cls(transform.dense, ln)

    def forward(self, x: Tensor) -> Tensor:
        weight = self.dense.weight
        dev = x.device.type
        if dev in ("cuda", "cpu") and torch.is_autocast_enabled(dev):
            dt = torch.get_autocast_dtype(dev)
            x, weight = x.to(dt), weight.to(dt)
        elif weight.dtype != x.dtype:
            weight = weight.to(x.dtype)
        args = (x, weight, self.dense.bias.float(), self.layer_norm.weight.float(),
                self.layer_norm.bias.float(), float(self.layer_norm.eps))
        if torch.compiler.is_compiling() or not x.is_cuda:  # the registered op: fake + autograd
            return torch.ops.sparton.mlm_transform_fwd(*args)[0]
        # eager: the C++ op (autograd in C++), the same implementation as the custom ops
        _check(args[0], args[1], args[2:5], "SpartonMLMTransform")
        return _eager.load().mlm_transform(*args)
