"""CPU oracle for the full Mamba-2 layer and model -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker.  The product
(``workloadsuite_amd.mamba_layer``) never calls it.

Reference: ``workloads/mamba/model_ref.py`` ("MR") in ShouyangDong/WorkloadSuite:
``SSDLayer.forward`` (MR:68-121) around the SSD core, and ``Model.forward``
(MR:200-203).  Restated from the mathematics of each step, in one compute dtype
(float64 by default) instead of MR's float16 parameters and activations:

  rms_norm        MR:72, 199       u / sqrt(mean(u^2) + eps) * weight; eps is
                                   torch's default for nn.RMSNorm in float16
                                   (finfo(float16).eps), as MR builds it
  in_proj         MR:75            u W^T, split into x, z, B, C, dt (MR:76-80)
  causal conv     MR:83-86         depthwise, kernel k, k-1 zeros of left
                                   padding, plus bias; then SiLU
  dt              MR:94            softplus(dt + dt_bias)
  A_dt            MR:102-103       -exp(A_log) * dt
  SSD core        MR:112           ssd_oracle.ssd_chunked with dt scaling X
  skip + gate     MR:116-119       (Y + x * D) * SiLU(z), then out_proj
  model           MR:200-203       x <- x + layer(x) for each layer, final norm

Parameters are passed as a dict of tensors named like MR's state_dict
(``in_proj.weight``, ``conv1d.weight``, ``conv1d.bias``, ``A_log``, ``D``,
``dt_bias``, ``out_proj.weight``, ``norm.weight``), so the same values feed
this oracle and the HIP module.

Pinning (``tests/test_layer.py``): the elementwise steps and the conv are
checked against torch's own float64 library routines (``F.rms_norm``,
``F.silu``, ``F.softplus``, ``F.conv1d``), and the whole layer against the same
layer composed from those routines, ``F.linear`` and the sequential-scan SSD
(``ssd_oracle.ssd_sequential``, independent of the chunked core used here).
"""

from __future__ import annotations

import numpy as np
import torch

from . import ssd_oracle

RMS_EPS_F16 = float(np.finfo(np.float16).eps)


def rms_norm(u: torch.Tensor, weight: torch.Tensor, eps: float = RMS_EPS_F16) -> torch.Tensor:
    ms = (u * u).mean(dim=-1, keepdim=True)
    return u / torch.sqrt(ms + eps) * weight


def silu(v: torch.Tensor) -> torch.Tensor:
    return v / (1.0 + torch.exp(-v))


def softplus(v: torch.Tensor, threshold: float = 20.0) -> torch.Tensor:
    # log(1 + e^v) without overflow, and v itself above the threshold, as
    # torch.nn.functional.softplus (MR:94) documents
    smooth = torch.clamp(v, min=0.0) + torch.log1p(torch.exp(-v.abs()))
    return torch.where(v > threshold, v, smooth)


def causal_depthwise_conv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """x [b, L, d]; weight [d, 1, k]; bias [d] -> [b, L, d]:
    out[t, ch] = bias[ch] + sum_j weight[ch, 0, j] * x[t - (k - 1) + j, ch] (x = 0 before t = 0)."""
    b, L, d = x.shape
    k = weight.shape[-1]
    out = bias.reshape(1, 1, d).expand(b, L, d).clone()
    for j in range(k):
        shift = k - 1 - j                       # tap j looks back `shift` tokens
        if shift >= L:
            continue
        out[:, shift:, :] += weight[:, 0, j].reshape(1, 1, d) * x[:, : L - shift, :]
    return out


def layer_forward(u: torch.Tensor, p: dict, n_heads: int, d_state: int, d_head: int, n_groups: int,
                  block_len: int, dtype=torch.float64) -> torch.Tensor:
    """One SSD layer (MR:68-121) on u [b, L, d_model]."""
    u = u.to(dtype)
    P = {k: v.to(dtype) for k, v in p.items()}
    b, L, _ = u.shape
    d_inner = n_heads * d_head
    gn = n_groups * d_state
    un = rms_norm(u, P["norm.weight"])
    proj = un @ P["in_proj.weight"].T
    x, z, B, C, dt = torch.split(proj, [d_inner, d_inner, gn, gn, n_heads], dim=-1)
    x = silu(causal_depthwise_conv(x, P["conv1d.weight"], P["conv1d.bias"]))
    X = x.reshape(b, L, n_heads, d_head)
    Bm = B.reshape(b, L, n_groups, d_state)
    Cm = C.reshape(b, L, n_groups, d_state)
    dt = softplus(dt + P["dt_bias"])
    A_dt = -torch.exp(P["A_log"]) * dt
    Y, _ = ssd_oracle.ssd_chunked(X, A_dt, Bm, Cm, block_len, dt=dt, dtype=dtype)
    Y = Y + X * P["D"].reshape(1, 1, -1, 1)
    Y = Y.reshape(b, L, d_inner) * silu(z)
    return Y @ P["out_proj.weight"].T


def model_forward(x: torch.Tensor, layers: list, final_norm_weight: torch.Tensor, n_heads: int, d_state: int,
                  d_head: int, n_groups: int, block_len: int, dtype=torch.float64) -> torch.Tensor:
    """Stacked layers with residuals and a final norm (MR:200-203)."""
    h = x.to(dtype)
    for p in layers:
        h = h + layer_forward(h, p, n_heads, d_state, d_head, n_groups, block_len, dtype)
    return rms_norm(h, final_norm_weight.to(dtype))
