"""Workload shapes for the SSD forward and their seeded synthetic inputs.

C1..C5 are the benchmark configurations of this build; R0 is the shape of the
reference workload's defaults (``workloads/mamba/model_ref.py:211-221``:
d_model 2048, 128 heads, d_state 128, d_head 64, 8 groups, block_len 64,
batch 8, seqlen 2048).

Distributions ("mamba2"): X ~ N(0,1); B, C ~ N(0,1)/sqrt(N);
A = -softplus(N(-2,1)) * exp(N(0,0.5)) (negative log-decays, 0.5 read as the
standard deviation); initial state ~ N(0, 0.1) (0.1 read as the standard
deviation).  "normal": every input N(0,1) (C1).

Draw order from one seeded generator: X, A's two normals, B, C, initial state.
Inputs are drawn in float32 and then rounded to the config dtype; A and the
states stay float32.
"""

from __future__ import annotations

import dataclasses
import math

import torch


@dataclasses.dataclass(frozen=True)
class SSDConfig:
    name: str
    batch: int
    seqlen: int
    nheads: int
    headdim: int
    dstate: int
    chunk: int
    ngroups: int
    dtype: torch.dtype
    dist: str = "mamba2"          # "mamba2" or "normal"
    init_state: bool = False      # draw a seeded initial state
    final_state: bool = False     # return the final state as well

    @property
    def nchunks(self) -> int:
        return self.seqlen // self.chunk

    @property
    def tokens(self) -> int:
        return self.batch * self.seqlen

    def scaled(self, **changes) -> "SSDConfig":
        return dataclasses.replace(self, **changes)


CONFIGS = {
    "C1": SSDConfig("C1", 16, 128, 8, 64, 16, 64, 8, torch.float32, dist="normal"),
    "C2": SSDConfig("C2", 8, 2048, 24, 64, 128, 64, 1, torch.float32),
    "C3": SSDConfig("C3", 4, 4096, 80, 64, 128, 256, 1, torch.bfloat16, final_state=True),
    "C4": SSDConfig("C4", 1, 65536, 80, 64, 128, 256, 1, torch.bfloat16, final_state=True),
    "C5": SSDConfig("C5", 64, 512, 64, 64, 64, 128, 8, torch.float32, init_state=True,
                    final_state=True),
    "R0": SSDConfig("R0", 8, 2048, 128, 64, 128, 64, 8, torch.float16),
}

HEADLINE = "C3"


def make_inputs(cfg: SSDConfig, seed: int = 0, device="cpu", a_scale: float = 1.0):
    """Seeded synthetic inputs for ``cfg``.

    Returns dict(X, A, B, C, init) on ``device``; ``init`` is None unless the
    config draws an initial state.  ``a_scale`` multiplies A (stress inputs with
    weak decay).  With device != "cpu" the numbers are drawn by the device's
    own generator (faster for the large configs); either way every consumer of
    the returned tensors sees identical values.
    """
    gen = torch.Generator(device=device).manual_seed(seed)
    b, L, h, P, N, g = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    f32 = dict(dtype=torch.float32, device=device, generator=gen)
    X = torch.randn(b, L, h, P, **f32)
    if cfg.dist == "normal":
        A = torch.randn(b, L, h, **f32)
        Bm = torch.randn(b, L, g, N, **f32)
        Cm = torch.randn(b, L, g, N, **f32)
    else:
        a1 = torch.randn(b, L, h, **f32)
        a2 = torch.randn(b, L, h, **f32)
        A = -torch.nn.functional.softplus(a1 - 2.0) * torch.exp(0.5 * a2)
        Bm = torch.randn(b, L, g, N, **f32) / math.sqrt(N)
        Cm = torch.randn(b, L, g, N, **f32) / math.sqrt(N)
    init = torch.randn(b, h, P, N, **f32) * 0.1 if cfg.init_state else None
    A = A * a_scale
    return dict(X=X.to(cfg.dtype), A=A, B=Bm.to(cfg.dtype), C=Cm.to(cfg.dtype), init=init)


def tolerance(dtype: torch.dtype) -> float:
    """rtol = atol for the parity checks: 1e-4 for fp32, 2e-2 for 16-bit inputs."""
    return 1e-4 if dtype == torch.float32 else 2e-2
