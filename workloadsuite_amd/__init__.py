"""MI355X-native Mamba-2 SSD forward (drop-in for the hot path of
ShouyangDong/WorkloadSuite ``workloads/mamba/model_ref.py``).

    from workloadsuite_amd import ssd_forward
    Y = ssd_forward(X, A, B, C, chunk_size=256)

Kernels live in ``libssd.so`` (built by ``python -m workloadsuite_amd.build``);
the C ABI is ``include/ssd.h``.
"""

from . import torch_ops  # noqa: F401,E402  (torch.ops.workloadsuite_amd.ssd_forward / ssd_layer)
from .ssd import (SSDError, chunk_cumsum, chunk_prep, chunk_scan, chunk_state, chunk_state_passing, decode_step,
                  layer_prep, ssd_core, ssd_forward, ssd_layer, state_passing, workspace_bytes)

__all__ = ["ssd_forward", "ssd_core", "chunk_cumsum", "chunk_prep", "chunk_state", "state_passing",
           "chunk_state_passing", "chunk_scan",
           "decode_step", "layer_prep", "ssd_layer", "workspace_bytes", "SSDError"]
