"""kda_bt16 -- KDA (Kimi Delta Attention) BT=16 chunked forward for MI355X.

Public surface of ``/root/reference/src/kda_bt16/__init__.py:1-16``:
``kda_bt16_fwd`` and ``kda_bt16_debug`` with the same signatures.  The raw
Triton kernels the reference also exports are replaced by
``kda_bt16_stage_launchers`` (stage-1 / stage-2 launch closures over the
HIP library); ``kda_bt16_kernel_fused`` raises NotImplementedError.

Beyond the reference: the backward (``kda_bt16_bwd``, and autograd through
``kda_bt16_fwd`` / ``chunk_kda``); ``kda_recurrent_fwd`` (token-by-token recurrence in
fp32, the decode step and an on-GPU gold) and ``kda_decode_step``; FLA's
``chunk_kda`` / ``fused_recurrent_kda`` calling convention (``kda_bt16.fla``)
and a per-function backend dispatch that registers these kernels
(``kda_bt16.dispatch``).
"""

from . import dispatch
from .fla import chunk_kda, fused_recurrent_kda
from .kernels import (
    forward_choice,
    fused_abort_count,
    kda_bt16_bwd,
    kda_bt16_debug,
    kda_bt16_fwd,
    kda_bt16_kernel_fused,
    kda_bt16_stage_launchers,
    kda_decode_step,
    kda_recurrent_fwd,
    set_backward_recompute,
)

__all__ = [
    "kda_bt16_fwd",
    "kda_bt16_bwd",
    "kda_bt16_debug",
    "kda_bt16_kernel_fused",
    "kda_bt16_stage_launchers",
    "kda_recurrent_fwd",
    "kda_decode_step",
    "set_backward_recompute",
    "forward_choice",
    "fused_abort_count",
    "chunk_kda",
    "fused_recurrent_kda",
    "dispatch",
]
__version__ = "0.1.0"
