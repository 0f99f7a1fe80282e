"""Drop-in workload module for the SSD forward: ``Model``, ``get_inputs()``,
``get_init_inputs()``.

The reference harness loads a workload module by path and calls
``Model(*get_init_inputs())``, ``.eval()``, then ``model(*get_inputs())``
under ``torch.inference_mode()`` (ShouyangDong/WorkloadSuite bench.py:217-233;
contract in README.md:26-29).  Tensors are created without an explicit
device, so the harness's ``torch.set_default_device`` (bench.py:390) decides
where they live.  This module keeps that contract for the SSD core of
``workloads/mamba/model_ref.py`` (MR:123-162); the forward runs in libssd's
HIP kernels.

The module-level defaults are the first benchmark configuration (C1: batch 16,
seqlen 128, 8 heads, head_dim 64, d_state 16, block_len 64, fp32, A/B/C/X all
N(0,1)), with A, B and C held as parameters and X as the input.
``CONFIGS`` (re-exported from ``configs``) lists the other shapes; use
``build_workload(name)`` for seeded parameters and inputs of any of them.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .configs import CONFIGS, SSDConfig, make_inputs
from . import torch_ops  # noqa: F401  (registers torch.ops.workloadsuite_amd.*)

__all__ = ["Model", "get_inputs", "get_init_inputs", "build_workload", "CONFIGS"]


class Model(nn.Module):
    """SSD forward with A (log-decay), B and C as parameters; forward(X) -> Y.

    A: [batch, seqlen, n_heads] fp32;  B, C: [batch, seqlen, n_groups, d_state];
    X: [batch, seqlen, n_heads, d_head].  ``n_groups`` defaults to ``n_heads``
    (B and C per head, as in C1).  With ``return_final_state`` the forward
    returns (Y, final_state [batch, n_heads, d_head, d_state] fp32).
    """

    def __init__(self, batch_size: int, seq_length: int, n_heads: int, d_head: int, d_state: int,
                 block_len: int = 64, n_groups: int | None = None, dtype: torch.dtype = torch.float32,
                 return_final_state: bool = False, state_dtype: torch.dtype = torch.float32):
        super().__init__()
        g = n_heads if n_groups is None else n_groups
        if n_heads % g != 0:
            raise ValueError("n_heads must be divisible by n_groups")
        self.batch_size, self.seq_length = batch_size, seq_length
        self.n_heads, self.d_head, self.d_state, self.n_groups = n_heads, d_head, d_state, g
        self.block_len = block_len
        self.return_final_state = return_final_state
        self.state_dtype = state_dtype
        self.A = nn.Parameter(torch.randn(batch_size, seq_length, n_heads, dtype=torch.float32))
        self.B = nn.Parameter(torch.randn(batch_size, seq_length, g, d_state).to(dtype))
        self.C = nn.Parameter(torch.randn(batch_size, seq_length, g, d_state).to(dtype))

    def forward(self, X: torch.Tensor, initial_states: torch.Tensor | None = None):
        # the registered op, so that torch.compile traces it as one node
        Y, final = torch.ops.workloadsuite_amd.ssd_forward(X, self.A, self.B, self.C, self.block_len, None,
                                                           initial_states, self.return_final_state,
                                                           self.state_dtype)
        return (Y, final) if self.return_final_state else Y


# ----- module-level defaults: configuration C1 -----
_C1 = CONFIGS["C1"]
batch_size = _C1.batch
seq_length = _C1.seqlen
n_heads = _C1.nheads
d_head = _C1.headdim
d_state = _C1.dstate
block_len = _C1.chunk


def get_inputs():
    return [torch.randn(batch_size, seq_length, n_heads, d_head)]


def get_init_inputs():
    return [batch_size, seq_length, n_heads, d_head, d_state, block_len]


def build_workload(name_or_cfg, device="cuda", seed: int = 0, state_dtype=torch.float32):
    """(model, inputs) for a named configuration with seeded synthetic values.

    Parameters and inputs come from ``configs.make_inputs`` (draw order X, A,
    B, C, initial state), so the oracle can be fed the very same tensors.
    """
    cfg: SSDConfig = CONFIGS[name_or_cfg] if isinstance(name_or_cfg, str) else name_or_cfg
    inp = make_inputs(cfg, seed=seed, device=device)
    model = Model(cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.chunk,
                  n_groups=cfg.ngroups, dtype=cfg.dtype, return_final_state=cfg.final_state,
                  state_dtype=state_dtype).to(device)
    with torch.no_grad():
        model.A.copy_(inp["A"])
        model.B.copy_(inp["B"])
        model.C.copy_(inp["C"])
    inputs = [inp["X"]] + ([inp["init"]] if inp["init"] is not None else [])
    return model.eval(), inputs
