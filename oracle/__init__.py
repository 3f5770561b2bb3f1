"""CPU oracle for the SpartonHead path -- test infrastructure, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
package, and only as the checker or as the timed CPU baseline. Parity status of
each function and how it is pinned is listed in oracle/sparton_ref.py (the head) and
oracle/loss_ref.py (the SPLADE loss on its reps).
"""
from .sparton_ref import (brute_bwd, brute_fwd, fused_bwd_ref, fused_fwd_ref, grad_coeff,
                          logit_at, torch_head, torch_head_chunked)

from . import loss_ref

__all__ = ["brute_bwd", "brute_fwd", "fused_bwd_ref", "fused_fwd_ref", "grad_coeff", "logit_at",
           "torch_head", "torch_head_chunked", "loss_ref"]
