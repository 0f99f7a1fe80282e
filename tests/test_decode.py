"""Decode (one token of the recurrence on the [b, h, P, N] state) against
the float64 sequential-scan oracle (oracle/ssd_oracle.py ``ssd_sequential``,
the per-token form of workloads/mamba/model_ref.py:152-161).

Tolerances: f32 1e-4; 16-bit inputs 2e-2 (y is rounded to the input type;
the state stays f32 and is held to 1e-4 relative to its scale, or 2e-3 where
the forward that produced it passed its local states as f16 rows: chunk 256
without the state chain, half an f16 ulp of each row's largest local
state)."""

import numpy as np
import pytest
import torch

from oracle import layer_oracle as LO
from oracle import ssd_oracle as O
from state_plans import f16_local
from workloadsuite_amd import ssd as S
from workloadsuite_amd.configs import tolerance

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def say(*a):
    print("CASE", *a, flush=True)


def close(actual, expected, tol):
    expected = torch.as_tensor(np.asarray(expected)) if not isinstance(expected, torch.Tensor) else expected
    torch.testing.assert_close(actual.detach().double().cpu(), expected.double().cpu(), rtol=tol, atol=tol)


def inputs(dtype, b, L, h, g, N, seed):
    gen = torch.Generator().manual_seed(seed)
    X = torch.randn(b, L, h, 64, generator=gen).to(dtype)
    B = (torch.randn(b, L, g, N, generator=gen) * N ** -0.5).to(dtype)
    C = (torch.randn(b, L, g, N, generator=gen) * N ** -0.5).to(dtype)
    dt = torch.rand(b, L, h, generator=gen) * 0.5 + 0.05
    A = -(torch.rand(h, generator=gen) + 0.2) * dt
    return X, A, B, C, dt


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("N,g", [(16, 4), (32, 1), (64, 2), (128, 1), (128, 8)])
def test_decode_continues_the_forward(dtype, N, g):
    """ssd_forward over L tokens, then one decode step: the step's y and the
    new state equal the sequential recurrence over L + 1 tokens."""
    say("decode after forward", dtype, N, g)
    b, h, Q = 2, 8, 64
    L = 2 * Q
    X, A, B, C, dt = inputs(dtype, b, L + 1, h, g, N, seed=1)
    Ys, fs = O.ssd_sequential(X, A, B, C, dt=dt)
    d = lambda t: t.to(DEV)  # noqa: E731
    _, state = S.ssd_forward(d(X[:, :L]), d(A[:, :L]), d(B[:, :L]), d(C[:, :L]), Q, dt=d(dt[:, :L]),
                             return_final_states=True)
    y = S.decode_step(state, d(X[:, L]), d(B[:, L]), d(C[:, L]), d(A[:, L]), dt=d(dt[:, L]))
    assert y.dtype == dtype and y.shape == (b, h, 64)
    close(y, Ys[:, L], tolerance(dtype))
    scale = float(np.abs(fs).max())
    close(state / scale, fs / scale, 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_decode_from_zero_state_equals_the_sequence(dtype):
    """K decode steps from a zero state reproduce every y_t of the sequence."""
    say("decode K steps", dtype)
    b, h, g, N, K = 3, 4, 2, 64, 12
    X, A, B, C, dt = inputs(dtype, b, K, h, g, N, seed=2)
    Ys, fs = O.ssd_sequential(X, A, B, C, dt=dt)
    state = torch.zeros(b, h, 64, N, device=DEV)
    for t in range(K):
        y = S.decode_step(state, X[:, t].to(DEV), B[:, t].to(DEV), C[:, t].to(DEV), A[:, t].to(DEV),
                          dt=dt[:, t].to(DEV))
        close(y, Ys[:, t], tolerance(dtype))
    close(state, fs, 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_epilogue_and_unit_dt(dtype):
    """Skip and gate on the step's y (MR:116-118); dt None means 1."""
    say("decode epilogue", dtype)
    b, h, g, N = 2, 6, 3, 128
    X, A, B, C, _ = inputs(dtype, b, 1, h, g, N, seed=3)
    init = torch.randn(b, h, 64, N, generator=torch.Generator().manual_seed(4)) * 0.3
    Ys, fs = O.ssd_sequential(X, A, B, C, initial_states=init)
    D = torch.rand(h) + 0.5
    z = torch.randn(b, h, 64).to(dtype)
    ref = (torch.from_numpy(Ys[:, 0]) + X[:, 0].double() * D.double()[None, :, None]) * LO.silu(z.double())
    state = init.clone().to(DEV)
    y = S.decode_step(state, X[:, 0].to(DEV), B[:, 0].to(DEV), C[:, 0].to(DEV), A[:, 0].to(DEV),
                      D=D.to(DEV), z=z.to(DEV))
    close(y, ref, tolerance(dtype))
    close(state, fs, 1e-4)


def test_decode_rejects_bad_arguments_on_the_host():
    lib = S._lib.load()
    import ctypes
    d = S._lib.dims(2, 1, 8, 64, 64, 3, 1)      # 8 heads over 3 groups
    s2 = (ctypes.c_int64 * 2)(512, 64)
    fake = ctypes.c_void_p(0x100000)
    args = (fake, fake, s2, fake, s2, fake, s2, fake, None, s2, fake, s2, None, None)
    assert lib.ssd_decode_step(ctypes.byref(d), 1, *args) == -4
    d = S._lib.dims(2, 1, 8, 64, 48, 2, 1)
    assert lib.ssd_decode_step(ctypes.byref(d), 1, *args) == -7
    d = S._lib.dims(2, 1, 8, 64, 64, 2, 1)
    assert lib.ssd_decode_step(ctypes.byref(d), 1, ctypes.c_void_p(0x100008), *args[1:]) == -10
    assert lib.ssd_decode_step(ctypes.byref(d), 1, None, *args[1:]) == -1
    with pytest.raises(ValueError, match="float32"):
        S.decode_step(torch.zeros(1, 2, 64, 16, dtype=torch.float16), torch.zeros(1, 2, 64), torch.zeros(1, 1, 16),
                      torch.zeros(1, 1, 16), torch.zeros(1, 2))


def _random_decode_cases(n, seed=31):
    gen = torch.Generator().manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=gen))]  # noqa: E731
    cases = []
    for k in range(n):
        g = pick([1, 2, 4])
        cases.append((k, DTYPES[k % 3], pick([64, 128, 256]), pick([16, 64, 128]), g, g * pick([1, 2, 3]), pick([1, 3])))
    return cases


@pytest.mark.gpu
@pytest.mark.parametrize("k,dtype,Q,N,g,h,b", _random_decode_cases(9))
def test_decode_several_steps_after_forward(k, dtype, Q, N, g, h, b):
    """ssd_forward over one chunk, then four decode steps in a row on the
    returned state: every step's y and the last state equal the sequential
    recurrence over the whole sequence."""
    say("decode steps after forward", k, dtype, Q, N, g, h, b)
    steps = 4
    X, A, B, C, dt = inputs(dtype, b, Q + steps, h, g, N, seed=300 + k)
    Ys, fs = O.ssd_sequential(X, A, B, C, dt=dt)
    d = lambda t: t.to(DEV)  # noqa: E731
    _, state = S.ssd_forward(d(X[:, :Q]), d(A[:, :Q]), d(B[:, :Q]), d(C[:, :Q]), Q, dt=d(dt[:, :Q]),
                             return_final_states=True)
    for s in range(Q, Q + steps):
        y = S.decode_step(state, d(X[:, s]), d(B[:, s]), d(C[:, s]), d(A[:, s]), dt=d(dt[:, s]))
        close(y, Ys[:, s], tolerance(dtype))
    scale = float(np.abs(fs).max())
    f16l = dtype != torch.float32 and Q == 256 and N in (64, 128) and f16_local(b * h, N)
    close(state / scale, fs / scale, 2e-3 if f16l else 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_full_size_sampled(dtype):
    """One decode step at C3's head shape with 256 batch rows (the largest
    shape bench.py --decode times: 20480 workgroups, a 671 MB state), with the
    skip and gate: sampled (batch, head) pairs against the float64 per-token
    update state' = exp(a) state + dt x B^T, y = (C . state' + D x) silu(z)
    (MR:152-161's per-token form, MR:116-118's epilogue), and every other
    state row unchanged in its update rule (checked through the state's
    checksum over all rows: sum state' = exp(a) sum state + dt (sum x)(sum B))."""
    say("decode full size", dtype)
    b, h, P, N, g = 256, 80, 64, 128, 1
    gen = torch.Generator(device=DEV).manual_seed(7)
    state = torch.randn(b, h, P, N, device=DEV, generator=gen)
    x = torch.randn(b, h, P, device=DEV, generator=gen).to(dtype)
    z = torch.randn(b, h, P, device=DEV, generator=gen).to(dtype)
    Bm = (torch.randn(b, g, N, device=DEV, generator=gen) * N ** -0.5).to(dtype)
    Cm = (torch.randn(b, g, N, device=DEV, generator=gen) * N ** -0.5).to(dtype)
    a = -torch.rand(b, h, device=DEV, generator=gen) * 0.2
    dt = torch.rand(b, h, device=DEV, generator=gen) * 0.5 + 0.05
    D = torch.randn(h, device=DEV, generator=gen)
    s0 = state.double()
    # per-(b, h) checksums of the state before the step, for the size-independent check
    sum0 = s0.sum(dim=(2, 3))
    y = S.decode_step(state, x, Bm, Cm, a, dt=dt, D=D, z=z)
    torch.cuda.synchronize()
    ea = torch.exp(a.double())
    xs, Bs = x.double(), Bm.double()
    # every row: sum_p,n state' = exp(a) sum state + dt (sum_p x)(sum_n B)
    want = ea * sum0 + dt.double() * xs.sum(-1) * Bs[:, 0].sum(-1)[:, None]
    got = state.double().sum(dim=(2, 3))
    scale = float(s0.abs().sum(dim=(2, 3)).max())
    assert float((got - want).abs().max()) <= 1e-5 * scale
    # sampled pairs in full, in float64
    pick = torch.Generator().manual_seed(11)
    bs = torch.randint(b, (12,), generator=pick).tolist()
    hs = torch.randint(h, (12,), generator=pick).tolist()
    for bi, hi in zip(bs, hs):
        sn = ea[bi, hi] * s0[bi, hi] + dt[bi, hi].double() * xs[bi, hi][:, None] * Bs[bi, 0][None, :]
        close(state[bi, hi], sn, 1e-5)
        zz = z[bi, hi].double()
        yr = (sn @ Cm[bi, 0].double() + D[hi].double() * xs[bi, hi]) * zz * torch.sigmoid(zz)
        close(y[bi, hi], yr, tolerance(dtype))
