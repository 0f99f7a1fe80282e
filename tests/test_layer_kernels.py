"""The layer around the SSD core (workloads/mamba/model_ref.py:76-118, "MR")
on the GPU, piece by piece, against the float64 layer oracle:

  layer_prep   causal depthwise conv + SiLU, softplus(dt + dt_bias),
               A_dt = -exp(A_log) dt and its chunk cumsum (MR:83-103)
  chunk_scan   with the skip + gate epilogue (Y + x D) * silu(z) (MR:116-118),
               on the generic kernel and the chunk-256 persistent one
  ssd_layer    the whole span from in_proj's output slices to out_proj's input

Tolerances (|a-e| <= atol + rtol|e|): f32 1e-4; 16-bit 2e-2 for values that
pass through 16-bit storage or MFMA operands (X, y).  dt and the cumsum are
float32 functions of exact 16-bit inputs, so they are held to 1e-4 for every
dtype.
"""

import pytest
import torch

from oracle import layer_oracle as LO
from oracle import ssd_oracle as O
from state_plans import k2_k3_f16s
from workloadsuite_amd import ssd as S
from workloadsuite_amd.configs import tolerance

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def say(*a):
    print("CASE", *a, flush=True)


def close(actual, expected, tol):
    torch.testing.assert_close(actual.detach().double().cpu(), expected.double().cpu(), rtol=tol, atol=tol)


def layer_case(dtype, b=2, L=256, h=4, P=64, g=2, N=64, k=4, pad=0, seed=0):
    """in_proj's output [b, L, pad + d_proj] (x, z, B, C, dt after `pad` unused
    columns) and the layer parameters, float32 master values rounded to dtype."""
    gen = torch.Generator().manual_seed(seed)
    d_inner = h * P
    d_proj = 2 * d_inner + 2 * g * N + h
    r = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    proj = r(b, L, pad + d_proj)
    proj[..., pad + 2 * d_inner:pad + 2 * d_inner + 2 * g * N] *= N ** -0.5   # B, C
    proj = proj.to(dtype)
    prm = {
        "conv_w": (r(d_inner, 1, k) * 0.5).to(dtype),
        "conv_b": (r(d_inner) * 0.1).to(dtype),
        "dt_bias": (torch.rand(h, generator=gen) * 2.0 - 3.0).to(dtype),
        "A_log": torch.rand(h, generator=gen) * 2.0 - 1.0,
        "D": 1.0 + 0.1 * r(h),
    }
    return proj, prm


def split(proj, h, P, g, N, pad=0):
    d_inner = h * P
    x, z, B, C, dt = torch.split(proj[..., pad:], [d_inner, d_inner, g * N, g * N, h], dim=-1)
    b, L = proj.shape[:2]
    return x, z, B.view(b, L, g, N), C.view(b, L, g, N), dt


def ref_prep(x, dt, prm, Q, h, P):
    """float64 oracle of the prep: X [b, L, h, P], dt, A_dt, Acs, decay."""
    b, L, _ = x.shape
    X = LO.silu(LO.causal_depthwise_conv(x.double(), prm["conv_w"].double(), prm["conv_b"].double()))
    dtr = LO.softplus(dt.double() + prm["dt_bias"].double())
    A = -torch.exp(prm["A_log"].double()) * dtr
    Acs, dec = O.chunk_cumsum(A, Q)
    return X.reshape(b, L, h, P), dtr, A, Acs, dec


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k", [1, 2, 3, 4])
@pytest.mark.parametrize("pad", [0, 1])
def test_layer_prep_matches_oracle(dtype, k, pad):
    """pad = 1 shifts every slice off 16-byte alignment: the conv then runs
    one channel per lane instead of 16-byte vectors."""
    say("layer_prep", dtype, k, pad)
    h, P, g, N, Q = 4, 64, 2, 64, 64
    proj, prm = layer_case(dtype, h=h, P=P, g=g, N=N, k=k, pad=pad)
    x, z, B, C, dt = split(proj, h, P, g, N, pad)
    X, dto, Acs, dec = S.layer_prep(x.to(DEV), dt.to(DEV), prm["conv_w"].to(DEV), prm["conv_b"].to(DEV),
                                    prm["dt_bias"].to(DEV), prm["A_log"].to(DEV), Q, h)
    rX, rdt, _, rAcs, rdec = ref_prep(x, dt, prm, Q, h, P)
    assert X.dtype == dtype and X.is_contiguous() and dto.dtype == torch.float32
    close(X, rX, tolerance(dtype))
    close(dto, rdt, 1e-4)
    close(Acs, rAcs, 1e-4)
    close(dec, rdec, 1e-4)


def test_layer_prep_without_conv_bias_and_long_sequence():
    say("layer_prep no bias, L=4096")
    h, P, g, N, Q = 2, 64, 1, 64, 256
    proj, prm = layer_case(torch.float16, b=1, L=4096, h=h, P=P, g=g, N=N)
    x, z, B, C, dt = split(proj, h, P, g, N)
    X, dto, Acs, dec = S.layer_prep(x.to(DEV), dt.to(DEV), prm["conv_w"].to(DEV), None, prm["dt_bias"].to(DEV),
                                    prm["A_log"].to(DEV), Q, h)
    prm0 = dict(prm, conv_b=torch.zeros_like(prm["conv_b"]))
    rX, rdt, _, rAcs, rdec = ref_prep(x, dt, prm0, Q, h, P)
    close(X, rX, 2e-2)
    close(Acs, rAcs, 1e-4)


def gated_ref(X, A, B, C, dt, Q, D, z):
    Y, _ = O.ssd_chunked(X.double(), A, B.double(), C.double(), Q, dt=dt)
    out = Y
    if D is not None:
        out = out + X.double() * D.double().reshape(1, 1, -1, 1)
    if z is not None:
        out = out * LO.silu(z.double())
    return out


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q,N,use_prep", [(64, 64, False), (64, 128, False), (256, 64, True), (256, 128, True),
                                          (256, 128, False)])
@pytest.mark.parametrize("epi", ["D+z", "D", "z"])
def test_chunk_scan_epilogue(dtype, Q, N, use_prep, epi):
    """K4 with the fused skip and gate against the float64 chunked core plus
    (Y + x D) * silu(z).  Q = 256 with 16-bit inputs and prep runs the
    persistent kernel's epilogue variant (split states, as the layer does);
    without prep the generic kernel's."""
    say("k4 epilogue", dtype, Q, N, use_prep, epi)
    gen = torch.Generator().manual_seed(5)
    b, h, g, P, nc = 2, 8, 2, 64, 3
    L = Q * nc
    X = torch.randn(b, L, h, P, generator=gen).to(dtype)
    B = (torch.randn(b, L, g, N, generator=gen) * N ** -0.5).to(dtype)
    C = (torch.randn(b, L, g, N, generator=gen) * N ** -0.5).to(dtype)
    dt = torch.rand(b, L, h, generator=gen) * 0.5 + 0.05
    A = -(torch.rand(h, generator=gen) + 0.2) * dt
    D = 1.0 + 0.1 * torch.randn(h, generator=gen) if "D" in epi else None
    z = torch.randn(b, L, h, P, generator=gen).to(dtype) if "z" in epi else None
    ref = gated_ref(X, A.double(), B, C, dt.double(), Q, D, z)
    Xd, Bd, Cd, dtd = X.to(DEV), B.to(DEV), C.to(DEV), dt.to(DEV)
    Acs, dec = S.chunk_cumsum(A.to(DEV), Q)
    prep = S.chunk_prep(Bd, Cd, Q) if use_prep else None
    if use_prep and dtype != torch.float32:
        assert prep is not None
    st = S.chunk_state(Xd, Bd, Acs, dt=dtd, prep=prep)
    split_st = dtype if prep is not None else None
    S_in, _ = S.state_passing(st, dec, split=split_st)
    Y = S.chunk_scan(Xd, Bd, Cd, Acs, S_in, dt=dtd, prep=prep, split=split_st is not None,
                     D=None if D is None else D.to(DEV), z=None if z is None else z.to(DEV))
    close(Y, ref, tolerance(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q,N,g,L", [(64, 128, 2, 128), (64, 128, 2, 512), (128, 64, 4, 768), (256, 128, 1, 512),
                                     (256, 64, 2, 512)])
def test_ssd_layer_matches_oracle(dtype, Q, N, g, L):
    """One C-ABI call from in_proj's output slices to out_proj's input.  With
    16-bit inputs and L % 256 == 0 the core runs at chunk 256 whatever the
    block_len; the oracle evaluates MR's chunking at Q."""
    say("ssd_layer", dtype, Q, N, g, L)
    h, P = 8, 64
    proj, prm = layer_case(dtype, b=2, L=L, h=h, P=P, g=g, N=N)
    x, z, B, C, dt = split(proj, h, P, g, N)
    pd = proj.to(DEV)
    xd, zd, Bd, Cd, dtd = split(pd, h, P, g, N)
    y = S.ssd_layer(xd, zd, Bd, Cd, dtd, prm["conv_w"].to(DEV), prm["conv_b"].to(DEV), prm["dt_bias"].to(DEV),
                    prm["A_log"].to(DEV), prm["D"].to(DEV), Q, h)
    assert y.shape == x.shape and y.dtype == dtype
    rX, rdt, rA, _, _ = ref_prep(x, dt, prm, Q, h, P)
    b = x.shape[0]
    ref = gated_ref(rX, rA, B, C, rdt, Q, prm["D"], z.reshape(b, L, h, P)).reshape(b, L, h * P)
    close(y, ref, tolerance(dtype))


def test_chunk_scan_epilogue_rejects_mismatched_gate():
    say("epilogue shape error")
    X = torch.zeros(1, 64, 2, 64, device=DEV)
    B = torch.zeros(1, 64, 1, 16, device=DEV)
    Acs, _ = S.chunk_cumsum(torch.zeros(1, 64, 2, device=DEV), 64)
    st = torch.zeros(1, 1, 2, 64, 16, device=DEV)
    with pytest.raises(ValueError, match="z must match"):
        S.chunk_scan(X, B, B, Acs, st, z=torch.zeros(1, 64, 2, 32, device=DEV))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,g,h", [(128, 2, 8), (64, 4, 8), (128, 4, 64)])
def test_ssd_layer_equals_its_kernels_one_by_one(dtype, N, g, h):
    """ssd_layer (conv, then K1's layer variant inside K0's launch, K0 writing
    CB^T in the input type for K4's epilogue variant) against the public
    entry points called one by one: bit-identical."""
    say("ssd_layer == kernels", dtype, N, g, h)
    P, Q, L, b = 64, 256, 512, 2
    proj, prm = layer_case(dtype, b=b, L=L, h=h, P=P, g=g, N=N)
    pd = proj.to(DEV)
    x, z, B, C, dt = split(pd, h, P, g, N)
    dev = {k: v.to(DEV) for k, v in prm.items()}
    y = S.ssd_layer(x, z, B, C, dt, dev["conv_w"], dev["conv_b"], dev["dt_bias"], dev["A_log"], dev["D"], 64, h)
    X, dto, Acs, dec = S.layer_prep(x, dt, dev["conv_w"], dev["conv_b"], dev["dt_bias"], dev["A_log"], Q, h)
    prep = S.chunk_prep(B, C, Q)
    # the layer hands S_in to chunk_scan as f16 rows with per-row scales (the
    # local states as f16 rows too where chunk_state and state_passing run as
    # separate launches)
    S_in, _ = k2_k3_f16s(X, B, Acs, dec, dt=dto, prep=prep)
    yk = S.chunk_scan(X, B, C, Acs, S_in, dt=dto, prep=prep, split="f16s", D=dev["D"], z=z.reshape(b, L, h, P))
    torch.cuda.synchronize()
    assert torch.equal(y, yk.reshape(b, L, h * P))


def _random_layer_cases(n, seed=23):
    """Seeded shapes for the fused span: dtype, chunk, state size, groups,
    heads per group, batch, chunks, conv width and a column offset of the
    slices inside in_proj's output."""
    gen = torch.Generator().manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=gen))]  # noqa: E731
    cases = []
    for k in range(n):
        dtype = DTYPES[k % 3]
        Q, N, g = pick([64, 128, 256]), pick([32, 64, 128]), pick([1, 2, 4])
        h = g * pick([1, 2, 3])
        b, nc = pick([1, 2]), pick([1, 2, 3])
        cases.append((k, dtype, Q, N, g, h, b, Q * nc, pick([2, 3, 4]), pick([0, 8])))
    return cases


@pytest.mark.parametrize("k,dtype,Q,N,g,h,b,L,kw,pad", _random_layer_cases(12))
def test_random_layer_shapes_vs_oracle(k, dtype, Q, N, g, h, b, L, kw, pad):
    say("random ssd_layer", k, dtype, Q, N, g, h, b, L, kw, pad)
    P = 64
    proj, prm = layer_case(dtype, b=b, L=L, h=h, P=P, g=g, N=N, k=kw, pad=pad, seed=200 + k)
    x, z, B, C, dt = split(proj, h, P, g, N, pad)
    xd, zd, Bd, Cd, dtd = split(proj.to(DEV), h, P, g, N, pad)
    y = S.ssd_layer(xd, zd, Bd, Cd, dtd, prm["conv_w"].to(DEV), prm["conv_b"].to(DEV), prm["dt_bias"].to(DEV),
                    prm["A_log"].to(DEV), prm["D"].to(DEV), Q, h)
    rX, rdt, rA, _, _ = ref_prep(x, dt, prm, Q, h, P)
    ref = gated_ref(rX, rA, B, C, rdt, Q, prm["D"], z.reshape(b, L, h, P)).reshape(b, L, h * P)
    close(y, ref, tolerance(dtype))
