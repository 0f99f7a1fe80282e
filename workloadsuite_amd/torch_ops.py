"""torch.library registrations of the SSD forward and of the fused layer span.

The reference harness may wrap a workload in ``torch.compile(fullgraph=False)``
(bench.py:185 of ShouyangDong/WorkloadSuite).  A ctypes call is opaque to the
tracer and breaks the graph; as registered ops, ``ssd_forward`` and
``ssd_layer`` are traced as single nodes (``fullgraph=True`` works), with fake
implementations that give the output shapes.  The real implementations call
``workloadsuite_amd.ssd`` and keep its behaviour: HIP tensors only, no CPU
fallback, the same argument checks.

    torch.ops.workloadsuite_amd.ssd_forward(X, A, B, C, chunk_size, dt, initial_states,
                                             return_final_states, state_dtype) -> (Y, final)
    torch.ops.workloadsuite_amd.ssd_layer(x, z, B, C, dt, conv_weight, conv_bias, dt_bias,
                                           A_log, D, chunk_size, nheads) -> y

``final`` is the [b, h, P, N] float32 state after the last chunk, or an empty
tensor when ``return_final_states`` is False (a registered op returns tensors
only).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ssd as _ssd

_NS = "workloadsuite_amd"


@torch.library.custom_op(f"{_NS}::ssd_forward", mutates_args=())
def ssd_forward_op(X: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, chunk_size: int,
                   dt: Optional[torch.Tensor], initial_states: Optional[torch.Tensor], return_final_states: bool,
                   state_dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    if return_final_states:
        return _ssd.ssd_forward(X, A, B, C, chunk_size, dt=dt, initial_states=initial_states,
                                return_final_states=True, state_dtype=state_dtype)
    Y = _ssd.ssd_forward(X, A, B, C, chunk_size, dt=dt, initial_states=initial_states, state_dtype=state_dtype)
    return Y, X.new_empty((0,), dtype=torch.float32)


@ssd_forward_op.register_fake
def _(X, A, B, C, chunk_size, dt, initial_states, return_final_states, state_dtype):
    b, L, h, P = X.shape
    N = B.shape[-1]
    Y = X.new_empty((b, L, h, P))
    final = X.new_empty((b, h, P, N) if return_final_states else (0,), dtype=torch.float32)
    return Y, final


@torch.library.custom_op(f"{_NS}::ssd_layer", mutates_args=())
def ssd_layer_op(x: torch.Tensor, z: torch.Tensor, B: torch.Tensor, C: torch.Tensor, dt: torch.Tensor,
                 conv_weight: torch.Tensor, conv_bias: Optional[torch.Tensor], dt_bias: torch.Tensor,
                 A_log: torch.Tensor, D: Optional[torch.Tensor], chunk_size: int, nheads: int) -> torch.Tensor:
    return _ssd.ssd_layer(x, z, B, C, dt, conv_weight, conv_bias, dt_bias, A_log, D, chunk_size, nheads)


@ssd_layer_op.register_fake
def _(x, z, B, C, dt, conv_weight, conv_bias, dt_bias, A_log, D, chunk_size, nheads):
    return x.new_empty(x.shape)
