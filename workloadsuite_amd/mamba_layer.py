"""Full-layer drop-in for ``workloads/mamba/model_ref.py`` (MR): ``SSDLayer``,
``Model``, ``get_inputs()``, ``get_init_inputs()`` with MR's exact
constructor signatures, parameter names, shapes and dtypes (MR:13-66,
165-196), so a reference ``state_dict`` loads unchanged and the reference
harness (bench.py:104-115, 217-233) runs this module as it runs MR.

The SSD core (MR:112, ``_ssd_core``, MR:123-162) runs in libssd's HIP kernels
through ``ssd_forward``: B and C are passed per group (no GQA ``repeat``,
MR:97-99), the chunking rearranges (MR:105-110, 115) disappear because the
kernels take ``[b, L, ...]`` tensors with strides, and dt scales x inside the
kernels in float32 (MR:144 multiplies in float16).  The glue around the core
-- RMSNorm, the two projections, the depthwise causal conv, SiLU, softplus,
the skip and the gate (MR:70-121) -- stays on PyTorch-ROCm (hipBLASLt/rocBLAS
GEMMs and elementwise kernels), in MR's float16.

Differences from MR a caller can observe: the core accumulates in float32 and
keeps the per-chunk states in float32 (MR rounds intermediates to float16 at
MR:145, 148, 155, 160), so outputs agree with MR to float16 rounding, not bit
for bit.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .ssd import ssd_forward

__all__ = ["SSDLayer", "Model", "get_inputs", "get_init_inputs"]


class SSDLayer(nn.Module):
    """One Mamba-2 SSD block; same signature and parameters as MR:13-66."""

    def __init__(self, d_model: int, n_heads: int, d_state: int, d_head: int, n_groups: int,
                 block_len: int = 64, conv_kernel: int = 4):
        super().__init__()
        if n_heads % n_groups != 0:
            raise ValueError("n_heads must be divisible by n_groups")
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_state = d_state
        self.d_head = d_head
        self.n_groups = n_groups
        self.block_len = block_len
        self.d_inner = n_heads * d_head
        # in_proj output order: x, z (gate), B, C, dt (MR:41-47)
        self.d_proj = 2 * self.d_inner + 2 * n_groups * d_state + n_heads
        f16 = torch.float16
        self.in_proj = nn.Linear(d_model, self.d_proj, bias=False, dtype=f16)
        self.conv1d = nn.Conv1d(self.d_inner, self.d_inner, kernel_size=conv_kernel, padding=conv_kernel - 1,
                                groups=self.d_inner, bias=True, dtype=f16)
        self.A_log = nn.Parameter(torch.log(torch.arange(1, n_heads + 1, dtype=torch.float32)))
        self.D = nn.Parameter(torch.ones(n_heads, dtype=f16))
        self.dt_bias = nn.Parameter(torch.zeros(n_heads, dtype=f16) - 4.0)
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False, dtype=f16)
        self.norm = nn.RMSNorm(d_model, dtype=f16)

    def forward(self, u: torch.Tensor) -> torch.Tensor:
        b, L, _ = u.shape
        if L % self.block_len != 0:
            raise ValueError(f"seqlen {L} is not a multiple of block_len {self.block_len}")
        h, P, g, N = self.n_heads, self.d_head, self.n_groups, self.d_state
        zxbcdt = self.in_proj(self.norm(u))
        x, z, B, C, dt = torch.split(zxbcdt, [self.d_inner, self.d_inner, g * N, g * N, h], dim=-1)
        # causal depthwise conv over time, then SiLU; [b, L, d_inner] with unit stride on d
        x = F.silu(self.conv1d(x.transpose(1, 2))[..., :L]).transpose(1, 2).contiguous()
        X = x.view(b, L, h, P)
        dt = F.softplus(dt + self.dt_bias)
        A_dt = -torch.exp(self.A_log) * dt.float()
        Y = ssd_forward(X, A_dt, B.view(b, L, g, N), C.view(b, L, g, N), self.block_len, dt=dt.float())
        Y = Y + X * self.D.view(1, 1, -1, 1)
        Y = Y.reshape(b, L, self.d_inner) * F.silu(z)
        return self.out_proj(Y)


class Model(nn.Module):
    """Stacked SSD layers with residuals and a final RMSNorm (MR:165-203)."""

    def __init__(self, d_model: int, n_layers: int, n_heads: int, d_state: int, d_head: int, n_groups: int,
                 block_len: int = 64, conv_kernel: int = 4):
        super().__init__()
        self.d_model = d_model
        self.n_layers = n_layers
        self.layers = nn.ModuleList([
            SSDLayer(d_model=d_model, n_heads=n_heads, d_state=d_state, d_head=d_head, n_groups=n_groups,
                     block_len=block_len, conv_kernel=conv_kernel)
            for _ in range(n_layers)
        ])
        self.final_norm = nn.RMSNorm(d_model, dtype=torch.float16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = x + layer(x)
        return self.final_norm(x)


# ----- module-level configuration: MR's production config (MR:209-221) -----
d_model = 2048
n_layers = 24
n_heads = 128
d_state = 128
d_head = 64
n_groups = 8
block_len = 64
conv_kernel = 4

batch_size = 8
seq_length = 2048


def get_inputs():
    return [torch.randn(batch_size, seq_length, d_model, dtype=torch.float16)]


def get_init_inputs():
    return [d_model, n_layers, n_heads, d_state, d_head, n_groups, block_len, conv_kernel]
