"""GPU parity: libssd's HIP kernels against the CPU oracle on identical inputs.

Tolerances (``torch.testing.assert_close`` semantics |a-e| <= atol + rtol|e|):
  f32 inputs                      rtol = atol = 1e-4
  bf16 / f16 inputs (f32 accum.)  rtol = atol = 2e-2
  f32 forwards compared with the whole oracle (C1, the random shapes, the
  C1 model surface): element-wise max(1e-4 + 1e-4|e|, 2 K u32 Yabs[e]), the
  strict bound or the forward-error bound of the element's sum, K calibrated
  on the float32 evaluation of the reference algorithm (tests/parity_bounds.py).
  C1's log-decays are N(0,1), i.e. half of them positive, so |Y| reaches
  ~4e13 through cancelling terms and even that float32 evaluation misses the
  strict 1e-4 on ~0.05% of the elements; the strict bound binds on ~95% of
  them and the bound is below |Y| on all but ~10 of 1.05 M.

Each test prints the case it runs before touching the GPU.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ssd_oracle as O
from parity_bounds import check_within, f32_reference_bounds
from state_plans import f16_local, k2_k3_f16s
from workloadsuite_amd import ssd as S
from workloadsuite_amd.configs import CONFIGS, make_inputs, tolerance
from workloadsuite_amd.mamba_ssd import build_workload

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def say(*a):
    print("CASE", *a, flush=True)


def small_case(dtype, Q, N, b=2, nc=2, h=4, g=2, seed=0, a_scale=1.0, dist="mamba2", init=False):
    cfg = CONFIGS["C2"].scaled(batch=b, seqlen=Q * nc, nheads=h, dstate=N, chunk=Q, ngroups=g, dtype=dtype,
                               dist=dist, init_state=init)
    return cfg, make_inputs(cfg, seed=seed, a_scale=a_scale)


def to_dev(inp):
    return {k: (None if v is None else v.to(DEV)) for k, v in inp.items()}


def assert_close(actual, expected, tol, atol=None):
    actual = actual.detach().double().cpu()
    expected = torch.as_tensor(np.asarray(expected)) if not isinstance(expected, torch.Tensor) else expected
    torch.testing.assert_close(actual, expected.double().cpu(), rtol=tol, atol=tol if atol is None else atol)


# ---------------------------------------------------------------------------
# per-kernel parity
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("Q", [64, 128, 256])
@pytest.mark.parametrize("h", [1, 5, 16, 24])
def test_k1_chunk_cumsum(Q, h):
    say("k1", Q, h)
    cfg, inp = small_case(torch.float32, Q, 16, h=h, g=1, nc=3)
    Acs, decay = S.chunk_cumsum(inp["A"].to(DEV), Q)
    rAcs, rdecay = O.chunk_cumsum(inp["A"].double(), Q)
    assert_close(Acs, rAcs, 1e-5)
    assert_close(decay, rdecay, 1e-5)


def test_k1_strided_input():
    say("k1 strided")
    A = torch.randn(2, 256, 40).to(DEV)[:, :, ::2]          # head stride 2
    Acs, decay = S.chunk_cumsum(A, 128)
    rAcs, rdecay = O.chunk_cumsum(A.cpu().double(), 128)
    assert_close(Acs, rAcs, 1e-5)
    assert_close(decay, rdecay, 1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q", [64, 128, 256])
@pytest.mark.parametrize("N", [16, 32, 64, 128])
def test_k2_chunk_state(dtype, Q, N):
    say("k2", dtype, Q, N)
    cfg, inp = small_case(dtype, Q, N)
    rAcs, _ = O.chunk_cumsum(inp["A"].double(), Q)
    S_ref = O.chunk_state(inp["X"].double(), inp["B"].double(), rAcs)
    d = to_dev(inp)
    states = S.chunk_state(d["X"], d["B"], rAcs.float().to(DEV))
    assert_close(states, S_ref, tolerance(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Q,N", [(64, 128), (64, 64), (128, 64), (128, 128)])
def test_k2_16bit_inputs_keep_f32_accuracy(dtype, Q, N):
    """chunk_state with 16-bit inputs and f32 states at chunk 64 / 128: the
    weighted x goes through the MFMA as a hi + lo pair of the input type, so
    the states match the float64 oracle on the same (exactly converted)
    inputs to f32 accumulation accuracy.  Tolerance 3e-5 of max|S| (64-128
    f32 products per element); with hi alone the error is ~2e-4 of max|S|.
    With dt, chunk 64 / 128 x d_state 64 / 128 (the 4-n-tile and 8-n-tile
    operand reads), 3 chunks of 5 heads in 1 group."""
    say("k2 16-bit accuracy", dtype, Q, N)
    cfg, inp = small_case(dtype, Q, N, b=1, nc=3, h=5, g=1)
    dt = torch.rand(1, 3 * Q, 5, generator=torch.Generator().manual_seed(7)) + 0.5
    rAcs, _ = O.chunk_cumsum(inp["A"].double(), Q)
    S_ref = O.chunk_state(inp["X"].double(), inp["B"].double(), rAcs, dt=dt.double())
    d = to_dev(inp)
    states = S.chunk_state(d["X"], d["B"], rAcs.float().to(DEV), dt=dt.to(DEV))
    assert_close(states, S_ref, 0.0, atol=3e-5 * S_ref.abs().max().item())


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("init", [False, True])
@pytest.mark.parametrize("nc", [1, 7, 16, 33])
def test_k3_state_passing(state_dtype, init, nc):
    say("k3", state_dtype, init, nc)
    g = torch.Generator().manual_seed(nc)
    local = torch.randn(2, nc, 3, 64, 128, generator=g).to(state_dtype)
    decay = torch.rand(2, 3, nc, generator=g)
    s0 = torch.randn(2, 3, 64, 128, generator=g) if init else None
    S_in, final = S.state_passing(local.to(DEV), decay.to(DEV), None if s0 is None else s0.to(DEV))
    rS, rfinal = O.state_passing(local.double(), decay.double(), None if s0 is None else s0.double())
    tol = 1e-5 if state_dtype == torch.float32 else 1e-2
    assert_close(S_in, rS, tol)
    assert_close(final, rfinal, 1e-5)


@pytest.mark.parametrize("N", [64, 128])
@pytest.mark.parametrize("init", [False, True])
def test_k3_f16s_format(N, init):
    """state_passing's f16s handover: row p of each state holds N f16 values v
    and the scales array a power of two s with max|v| in [2^14, 2^15]; v s is
    the f32 S_in to within f16 rounding (half an f16 ulp of the row's scale)."""
    say("k3 f16s", N, init)
    g = torch.Generator().manual_seed(N)
    local = torch.randn(2, 5, 3, 64, N, generator=g) * torch.logspace(-3, 3, 64).reshape(1, 1, 1, 64, 1)
    decay = torch.rand(2, 3, 5, generator=g)
    s0 = torch.randn(2, 3, 64, N, generator=g) if init else None
    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    ref, rfinal = S.state_passing(local.to(DEV), dev(decay), dev(s0))
    got, final = S.state_passing(local.to(DEV), dev(decay), dev(s0), split="f16s")
    torch.cuda.synchronize()
    assert torch.equal(final, rfinal)
    v = got.states.view(torch.float16)[..., :N].double().cpu()
    sc = got.scales.double().cpu()
    assert torch.equal(torch.exp2(torch.log2(sc).round()), sc)   # powers of two
    vmax = v.abs().amax(-1)
    live = vmax > 0
    # (a row maximum just below 2^15 may round up to it)
    bad = live & ~((vmax >= 2.0 ** 14) & (vmax <= 2.0 ** 15))
    assert not bad.any(), f"row maxima outside [2^14, 2^15]: {vmax[bad][:8].tolist()} scales {sc[bad][:8].tolist()}"
    dec = v * sc[..., None]
    r = ref.double().cpu()
    assert ((dec - r).abs() <= sc[..., None] * 2.0 ** 3 * (1 + 1e-9)).all()   # half an f16 ulp at 2^14..2^15


def _check_f16_rows(v, sc, ref):
    """f16 row values v [.., R, M] with power-of-two row scales sc [.., R]:
    row maxima in [2^14, 2^15] and v sc within half an f16 ulp of the row's
    scale of the f32 reference."""
    assert torch.equal(torch.exp2(torch.log2(sc).round()), sc)   # powers of two
    vmax = v.abs().amax(-1)
    live = vmax > 0
    # (a row maximum just below 2^15 may round up to it)
    bad = live & ~((vmax >= 2.0 ** 14) & (vmax <= 2.0 ** 15))
    assert not bad.any(), f"row maxima outside [2^14, 2^15]: {vmax[bad][:8].tolist()} scales {sc[bad][:8].tolist()}"
    assert ((v * sc[..., None] - ref).abs() <= sc[..., None] * 2.0 ** 3 * (1 + 1e-9)).all()


def _f16_local_case(dtype, N, nc, h=40, g=2, seed=3):
    """Inputs at chunk 256 whose local state rows span 6 decades (x scaled per
    column p), with dt; 2 * nc * h items, more than the CUs for nc >= 4."""
    cfg, inp = small_case(dtype, 256, N, b=2, nc=nc, h=h, g=g, seed=seed)
    d = to_dev(inp)
    col = torch.logspace(-3, 3, 64, device=DEV).to(dtype)
    X = (d["X"] * col).contiguous()
    dt = torch.rand(2, nc * 256, h, generator=torch.Generator().manual_seed(seed)).to(DEV) + 0.5
    Acs, dec = S.chunk_cumsum(d["A"], 256)
    return X, d["B"], d["C"], Acs, dec, dt


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N", [64, 128])
def test_k2_f16s_local_format(dtype, N):
    """chunk_state(..., state_dtype="f16s") at chunk 256: row p of each local
    state holds N f16 values v in the first half of its f32 slots, and the
    item's packed scales a power of two s per row and 16-column tile with
    max|v| over the tile row in [2^14, 2^15]; v s is chunk_state's f32 local
    state to within half an f16 ulp of the tile's scale.  With and without
    chunk_prep's operands and dt."""
    say("k2 f16s local", dtype, N)
    X, B, C, Acs, _, dt = _f16_local_case(dtype, N, nc=5)
    prep = S.chunk_prep(B, C, 256)
    for pr in (None, prep):
        for dtv in (None, dt):
            ref = S.chunk_state(X, B, Acs, dt=dtv, prep=pr)
            got = S.chunk_state(X, B, Acs, dt=dtv, prep=pr, state_dtype="f16s")
            assert isinstance(got, S.F16SLocalStates)
            torch.cuda.synchronize()
            v = got.states.view(torch.float16)[..., :N].double().cpu()
            sc = got.scales().double().cpu()
            tiles = lambda t: t.unflatten(-1, (N // 16, 16))  # noqa: E731  [.., P, N/16, 16]
            _check_f16_rows(tiles(v), sc, tiles(ref.double().cpu()))
            assert torch.allclose(got.decode().double().cpu(), v * sc.repeat_interleave(16, -1))


@pytest.mark.parametrize("N", [64, 128])
@pytest.mark.parametrize("nc,init", [(5, False), (12, True), (3, True)])
def test_k3_f16s_local_input(N, nc, init):
    """state_passing on f16 local states (chunk_state's "f16s") gives bit for
    bit what it gives on their f32 values, which f16 value times a power of two
    is exactly: S_in as "f16s" and the final state (chains of 3, 5, 12 chunks:
    both load paths)."""
    say("k3 f16s local", N, nc, init)
    X, B, C, Acs, dec, dt = _f16_local_case(torch.bfloat16, N, nc=nc, h=6, g=3)
    loc = S.chunk_state(X, B, Acs, dt=dt, state_dtype="f16s")
    s0 = torch.randn(2, 6, 64, N, generator=torch.Generator().manual_seed(nc)).to(DEV) if init else None
    got, fin = S.state_passing(loc, dec, s0, split="f16s")
    ref, rfin = S.state_passing(loc.decode(), dec, s0, split="f16s")
    torch.cuda.synchronize()
    assert torch.equal(fin, rfin)
    assert torch.equal(got.scales, ref.scales)
    assert torch.equal(got.states.view(torch.float16)[..., :N], ref.states.view(torch.float16)[..., :N])
    assert torch.equal(loc.scales(), S.chunk_state(X, B, Acs, dt=dt, state_dtype="f16s").scales())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q", [64, 128, 256])
@pytest.mark.parametrize("N", [16, 32, 64, 128])
def test_k4_chunk_scan(dtype, Q, N):
    say("k4", dtype, Q, N)
    cfg, inp = small_case(dtype, Q, N, nc=3)
    rAcs, rdecay = O.chunk_cumsum(inp["A"].double(), Q)
    S_local = O.chunk_state(inp["X"].double(), inp["B"].double(), rAcs)
    S_in, _ = O.state_passing(S_local, rdecay)
    Y_ref = O.chunk_scan(inp["X"].double(), inp["B"].double(), inp["C"].double(), rAcs, S_in)
    d = to_dev(inp)
    Y = S.chunk_scan(d["X"], d["B"], d["C"], rAcs.float().to(DEV), S_in.float().to(DEV))
    assert Y.dtype == dtype
    assert_close(Y, Y_ref, tolerance(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Q,N,use_dt,init", [(64, 128, True, True), (64, 64, False, False), (128, 64, True, False)])
def test_k4_f16s_states_at_chunk_64_128(dtype, Q, N, use_dt, init):
    """chunk_scan on S_in handed over as "f16s" (f16 rows, a power-of-two
    scale per row) at chunk 64 / 128, where the 16-bit kernel reads them: the
    y of chunk_scan on the same states decoded to f32 (C rounded to f16 with
    a power-of-two scale per row is exact for these inputs, so only the f32
    summation order differs: one rounding of the output type), and the
    oracle's within the 16-bit tolerance.  Groups of 4 heads over 2 head
    slices, 5 chunks."""
    say("k4 f16s", dtype, Q, N, use_dt, init)
    cfg, inp = small_case(dtype, Q, N, b=2, nc=5, h=8, g=2, init=init)
    d = to_dev(inp)
    dt = torch.rand(2, 5 * Q, 8, generator=torch.Generator().manual_seed(5)) + 0.5 if use_dt else None
    dtd = None if dt is None else dt.to(DEV)
    Acs, dec = S.chunk_cumsum(d["A"], Q)
    st = S.chunk_state(d["X"], d["B"], Acs, dt=dtd)
    S_f, _ = S.state_passing(st, dec, d["init"], split="f16s")
    Yf = S.chunk_scan(d["X"], d["B"], d["C"], Acs, S_f, dt=dtd, split="f16s")
    Yd = S.chunk_scan(d["X"], d["B"], d["C"], Acs, S_f.decode(), dt=dtd)
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    assert_close(Yf, Yd.float(), eps, atol=eps * Yd.float().abs().max().item())
    Ys, _ = O.ssd_sequential(inp["X"], inp["A"], inp["B"], inp["C"], dt=dt, initial_states=inp["init"])
    assert_close(Yf, Ys, tolerance(dtype))


@pytest.mark.parametrize("Q", [64, 256])
def test_k4_masked_exponent_is_never_evaluated(Q):
    """A = -4|N(0,1)|: every causal decay exp(Acs[l]-Acs[s]), s <= l, is <= 1,
    while the masked entries above the diagonal have exponents up to ~+800
    (exp overflows to inf in f32).  A kernel that multiplies by the mask after
    exp produces inf * 0 = nan; the result must instead be finite and match.

    Tolerance: the segsum is a difference of two f32 cumsums that reach ~-200
    (Q=64) / ~-800 (Q=256), as in the reference (MR:135-139), so the f32
    evaluation of the reference algorithm itself misses the f64 result by
    ~3e-4 / ~1.2e-3 here: the element-wise f32 bound of tests/parity_bounds.py."""
    say("k4 masked exponent", Q)
    cfg, inp = small_case(torch.float32, Q, 32, dist="normal", nc=2)
    inp["A"] = -4.0 * inp["A"].abs()
    rAcs, _ = O.chunk_cumsum(inp["A"].double(), Q)
    assert (rAcs[..., 0, None] - rAcs).max() > 100  # the masked exponents do overflow f32
    Y, _, allowed, _, _ = f32_reference_bounds(inp["X"], inp["A"], inp["B"], inp["C"], Q)
    Yg = S.ssd_forward(*[inp[k].to(DEV) for k in ("X", "A", "B", "C")], Q)
    assert torch.isfinite(Yg).all()
    check_within(Yg, Y, allowed)


def test_positive_log_decay_within_f32_range():
    """A ~ N(0,1) (half the log-decays positive, as in C1) at a chunk where the
    growing terms stay inside the f32 range."""
    say("positive decay")
    cfg, inp = small_case(torch.float32, 64, 16, dist="normal", nc=2, h=8, g=8)
    Y, _, allowed, _, _ = f32_reference_bounds(inp["X"], inp["A"], inp["B"], inp["C"], 64)
    Yg = S.ssd_forward(*[inp[k].to(DEV) for k in ("X", "A", "B", "C")], 64)
    assert torch.isfinite(Yg).all()
    check_within(Yg, Y, allowed)


# ---------------------------------------------------------------------------
# whole forward: small shapes with every option, against the fp64 sequential scan
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q,N,h,g", [(64, 16, 8, 8), (64, 128, 6, 1), (128, 64, 16, 8), (256, 128, 4, 1),
                                     (256, 32, 6, 3)])
@pytest.mark.parametrize("opts", ["plain", "dt+init", "weak-decay"])
def test_forward_vs_sequential(dtype, Q, N, h, g, opts):
    say("fwd", dtype, Q, N, h, g, opts)
    init = opts == "dt+init"
    cfg, inp = small_case(dtype, Q, N, b=2, nc=3, h=h, g=g, init=init,
                          a_scale=1e-3 if opts == "weak-decay" else 1.0)
    dt = torch.rand(2, 3 * Q, h, generator=torch.Generator().manual_seed(5)) + 0.5 if init else None
    Ys, fs = O.ssd_sequential(inp["X"], inp["A"], inp["B"], inp["C"], dt=dt, initial_states=inp["init"])
    d = to_dev(inp)
    Y, final = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], Q, dt=None if dt is None else dt.to(DEV),
                             initial_states=d["init"], return_final_states=True)
    tol = tolerance(dtype)
    assert_close(Y, Ys, tol)
    assert_close(final, fs, tol)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q,N", [(64, 16), (64, 32), (128, 16), (128, 32)])
@pytest.mark.parametrize("nc,h,g,opts", [(2, 8, 8, "plain"), (3, 6, 2, "dt+init"), (16, 4, 1, "dt+init"),
                                         (17, 2, 1, "dt+init"), (1, 3, 3, "init")])
def test_small_state_forward(dtype, Q, N, nc, h, g, opts):
    """d_state 16 / 32 at chunk 64 / 128 with up to 16 chunks per chain: the
    whole forward as one launch (one workgroup per (b, h) chain, f32 state in
    LDS); 17 chunks take the four-kernel path.  Against the fp64 sequential
    scan (Y and the final state), 2e-2 for 16-bit inputs; f32 inputs with
    N(0,1) log-decays (as C1) against the element-wise f32 bound."""
    say("small-state fwd", dtype, Q, N, nc, h, g, opts)
    init = "init" in opts
    dist = "normal" if dtype == torch.float32 and opts == "plain" else "mamba2"
    cfg, inp = small_case(dtype, Q, N, b=2, nc=nc, h=h, g=g, init=init, dist=dist)
    dt = torch.rand(2, nc * Q, h, generator=torch.Generator().manual_seed(6)) + 0.5 if "dt" in opts else None
    d = to_dev(inp)
    Y, final = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], Q, dt=None if dt is None else dt.to(DEV),
                             initial_states=d["init"], return_final_states=True)
    torch.cuda.synchronize()
    if dist == "normal":
        Yr, fr, aY, af, stats = f32_reference_bounds(inp["X"], inp["A"], inp["B"], inp["C"], Q)
        check_within(Y, Yr, aY)
        check_within(final, fr, af, "final")
        return
    Ys, fs = O.ssd_sequential(inp["X"], inp["A"], inp["B"], inp["C"], dt=dt, initial_states=inp["init"])
    tol = tolerance(dtype)
    assert_close(Y, Ys, tol)
    assert_close(final, fs, tol)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Q,N", [(64, 16), (64, 32), (128, 16)])
def test_small_state_forward_one_workgroup_per_chain(dtype, Q, N):
    """The one-launch forward with at least twice as many (b, h) chains as
    CUs (32 x 16 = 512 on 256 CUs): one workgroup per chain instead of two
    halves of P.  Against the fp64 sequential scan, with dt and an initial
    state."""
    say("small-state fwd, whole chains", dtype, Q, N)
    b, h, g, nc = 32, 16, 4, 3
    cfg, inp = small_case(dtype, Q, N, b=b, nc=nc, h=h, g=g, init=True)
    dt = torch.rand(b, nc * Q, h, generator=torch.Generator().manual_seed(7)) + 0.5
    d = to_dev(inp)
    Y, final = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], Q, dt=dt.to(DEV), initial_states=d["init"],
                             return_final_states=True)
    torch.cuda.synchronize()
    Ys, fs = O.ssd_sequential(inp["X"], inp["A"], inp["B"], inp["C"], dt=dt, initial_states=inp["init"])
    tol = tolerance(dtype)
    assert_close(Y, Ys, tol)
    assert_close(final, fs, tol)


def test_forward_bf16_states():
    say("fwd bf16 states")
    cfg, inp = small_case(torch.bfloat16, 256, 128, b=2, nc=4, h=4, g=1, init=True)
    Ys, fs = O.ssd_sequential(inp["X"], inp["A"], inp["B"], inp["C"], initial_states=inp["init"])
    d = to_dev(inp)
    Y, final = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], 256, initial_states=d["init"],
                             return_final_states=True, state_dtype=torch.bfloat16)
    assert_close(Y, Ys, 2e-2)
    assert_close(final, fs, 2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,h,g,use_dt", [(128, 24, 2, False), (64, 12, 3, True), (128, 10, 5, True)])
def test_forward_equals_kernel_by_kernel(dtype, N, h, g, use_dt):
    """ssd_forward (chunk_prep's precomputed group operands) against the four
    public kernels called one by one (each CU rebuilds them): bit-identical.
    More items than CUs and few heads per group, so ranges cross groups."""
    say("fwd == kernels", dtype, N, h, g, use_dt)
    cfg, inp = small_case(dtype, 256, N, b=4, nc=16, h=h, g=g)
    d = to_dev(inp)
    dt = torch.rand(4, 16 * 256, h, device=DEV) + 0.5 if use_dt else None
    # the forward handing S_in over as (hi, lo) pairs: the same values as f32 S_in
    Y, final = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], 256, dt=dt, return_final_states=True,
                             state_format="split")
    Acs, dec = S.chunk_cumsum(d["A"], 256)
    st = S.chunk_state(d["X"], d["B"], Acs, dt=dt)
    S_in, fin = S.state_passing(st, dec)
    Yk = S.chunk_scan(d["X"], d["B"], d["C"], Acs, S_in, dt=dt)
    prep = S.chunk_prep(d["B"], d["C"], 256)
    assert prep is not None
    assert torch.equal(S.chunk_state(d["X"], d["B"], Acs, dt=dt, prep=prep), st)
    Yp = S.chunk_scan(d["X"], d["B"], d["C"], Acs, S_in, dt=dt, prep=prep)
    # the forward's own K3 -> K4 hand-over: S_in stored as (hi, lo) pairs
    S_sp, fin_sp = S.state_passing(st, dec, split=dtype)
    Ys = S.chunk_scan(d["X"], d["B"], d["C"], Acs, S_sp, dt=dt, prep=prep, split=True)
    # the default forward hands S_in over as f16 rows with per-row scales (and
    # here, with chunk_state and state_passing as separate launches, passes
    # the local states as f16 rows too)
    assert f16_local(4 * h, N)
    Yf, final_f = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], 256, dt=dt, return_final_states=True)
    S_f, fin_f = k2_k3_f16s(d["X"], d["B"], Acs, dec, dt=dt, prep=prep)
    Yfk = S.chunk_scan(d["X"], d["B"], d["C"], Acs, S_f, dt=dt, prep=prep, split="f16s")
    torch.cuda.synchronize()
    assert torch.equal(Y, Yk)
    assert torch.equal(Yp, Yk)
    assert torch.equal(Ys, Yk)
    assert torch.equal(final, fin)
    assert torch.equal(fin_sp, fin)
    assert torch.equal(Yf, Yfk)
    assert torch.equal(final_f, fin_f)


# ---------------------------------------------------------------------------
# benchmark configurations at full size
# ---------------------------------------------------------------------------

def _slice_inputs(inp, batches, heads, ngroups, nheads):
    """Inputs restricted to some batches and heads, with B/C given per head."""
    r = nheads // ngroups
    grp = torch.tensor([hh // r for hh in heads])
    hs = torch.tensor(heads)
    bs = torch.tensor(batches)
    cpu = lambda t: t.cpu()  # noqa: E731
    X = cpu(inp["X"])[bs][:, :, hs]
    A = cpu(inp["A"])[bs][:, :, hs]
    B = cpu(inp["B"])[bs][:, :, grp]
    C = cpu(inp["C"])[bs][:, :, grp]
    init = None if inp["init"] is None else cpu(inp["init"])[bs][:, hs]
    return X, A, B, C, init


@pytest.mark.parametrize("name,batches,heads", [
    ("C1", None, None),
    ("C2", [0, 7], list(range(24))),
    ("C3", [0, 3], [0, 41, 79]),
    ("C4", [0], [0, 40, 79]),
    ("C5", [0, 63], list(range(64))),
    ("R0", [0, 7], [0, 17, 63, 64, 127]),
])
def test_config_full_size(name, batches, heads):
    cfg = CONFIGS[name]
    say("config", name, cfg)
    gen_dev = DEV if cfg.seqlen * cfg.batch * cfg.nheads > 2e6 else "cpu"
    inp = to_dev(make_inputs(cfg, seed=0, device=gen_dev))
    out = S.ssd_forward(inp["X"], inp["A"], inp["B"], inp["C"], cfg.chunk, initial_states=inp["init"],
                        return_final_states=True)
    torch.cuda.synchronize()
    Y, final = out
    assert Y.shape == inp["X"].shape and Y.dtype == cfg.dtype
    assert torch.isfinite(Y).all() and torch.isfinite(final).all()
    if batches is None:
        # C1: the whole output, element-wise bound (module docstring)
        X, A, B, C = (inp[k].cpu() for k in ("X", "A", "B", "C"))
        Yr, fr, aY, af, stats = f32_reference_bounds(X, A, B, C, cfg.chunk)
        print("C1 bound", stats, flush=True)
        assert stats["Y"]["within_10x_strict"] > 0.99 and stats["Y"]["bound_below_abs"] > 0.999
        check_within(Y, Yr, aY)
        check_within(final, fr, af, "final")
        return
    X, A, B, C, init = _slice_inputs(inp, batches, heads, cfg.ngroups, cfg.nheads)
    Yr, fr = O.ssd_chunked(X, A, B, C, cfg.chunk, initial_states=init)
    bs, hs = torch.tensor(batches), torch.tensor(heads)
    Yg = Y.cpu()[bs][:, :, hs]
    fg = final.cpu()[bs][:, hs]
    tol = tolerance(cfg.dtype)
    assert_close(Yg, Yr, tol)
    assert_close(fg, fr, tol)


def mr_regime_inputs(cfg, seed):
    """R0-shaped inputs in MR's own parameter regime (MR:61-63, 94, 102-103):
    A = -(1..h) (A_log = log(1..h)), dt = softplus(dt_raw - 4) with dt_raw,
    x, B and C ~ N(0, 1/3) (in_proj's default-initialised outputs on a
    unit-RMS input; x a conv + SiLU output of the same scale), so per-token
    log-decays A dt reach ~-2.3 at head 127 and the in-chunk cumsums ~-150 at
    block_len 64 (~-600 at 256).  f16 like MR.  Returns X, A_dt, B, C, dt
    on the GPU."""
    b, L, h, P, N, g = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    gen = torch.Generator(device=DEV).manual_seed(seed)
    sd = 3 ** -0.5
    X = (torch.randn(b, L, h, P, device=DEV, generator=gen) * sd).half()
    Bm = (torch.randn(b, L, g, N, device=DEV, generator=gen) * sd).half()
    Cm = (torch.randn(b, L, g, N, device=DEV, generator=gen) * sd).half()
    dt_raw = (torch.randn(b, L, h, device=DEV, generator=gen) * sd).half()
    dt = torch.nn.functional.softplus(dt_raw.float() - 4.0)
    A = -torch.arange(1, h + 1, device=DEV, dtype=torch.float32)
    return X, A * dt, Bm, Cm, dt


# every group (16 heads each), both ends of A = -(1..128)
R0_HEADS = [0, 17, 34, 51, 68, 85, 102, 127]


def _check_mr_regime(Y, final, X, A, B, C, dt, heads, batches, block_len, ngroups, nheads):
    bs, hs = torch.tensor(batches), torch.tensor(heads)
    grp = torch.tensor([hh // (nheads // ngroups) for hh in heads])
    cpu = lambda t: t.cpu()[bs]  # noqa: E731
    Yr, fr = O.ssd_chunked(cpu(X)[:, :, hs], cpu(A)[:, :, hs], cpu(B)[:, :, grp], cpu(C)[:, :, grp], block_len,
                           dt=cpu(dt)[:, :, hs])
    assert torch.isfinite(Y).all() and torch.isfinite(final).all()
    assert_close(Y.cpu()[bs][:, :, hs], Yr, 2e-2)
    assert_close(final.cpu()[bs][:, hs], fr, 2e-2)


def test_full_r0_forward_at_block_len_64_in_the_reference_regime():
    """R0 (batch 8, seqlen 2048, 128 heads, d_state 128, 8 groups, MR's
    block_len 64, f16) through ssd_forward with MR's own A and dt (see
    mr_regime_inputs) and B / C per group, the form INTEGRATION's
    "better" binding passes: the library runs it at chunk 256 (the
    persistent kernels, in-chunk log-decay sums to ~-600).  Sampled heads
    of every group on two batches against the float64 oracle at block_len
    64, 2e-2, Y and the final state."""
    cfg = CONFIGS["R0"]
    say("R0 forward, MR regime", cfg)
    X, A, B, C, dt = mr_regime_inputs(cfg, seed=21)
    assert S.forward_chunk(cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups, 64,
                           torch.float16) == 256
    Y, final = S.ssd_forward(X, A, B, C, 64, dt=dt, return_final_states=True)
    torch.cuda.synchronize()
    _check_mr_regime(Y, final, X, A, B, C, dt, R0_HEADS, [0, 7], 64, cfg.ngroups, cfg.nheads)


def test_full_r0_ssd_core_on_the_block_64_kernels_in_the_reference_regime():
    """The same inputs through ssd_core with MR's own argument layout
    (chunked tensors, B / C repeated per head, MR:97-110): with one group
    per head the chunk-256 workspace would be the larger one, so the library
    runs MR's block_len 64 itself -- the f32-state chain (f16 rows handed to
    chunk_scan) and the 16-bit chunk_scan for f32 states, with in-chunk
    log-decay sums to ~-150.  Sampled heads of every group, 2e-2."""
    cfg = CONFIGS["R0"]
    say("R0 ssd_core, MR regime", cfg)
    b, L, h, P, N, g, Q = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups, 64
    X, A, B, C, dt = mr_regime_inputs(cfg, seed=21)
    assert S.forward_chunk(b, L, h, P, N, h, Q, torch.float16) == Q
    r = h // g
    chunk = lambda t: t.reshape(b, L // Q, Q, *t.shape[2:])  # noqa: E731
    Brep = B.repeat_interleave(r, dim=2)
    Crep = C.repeat_interleave(r, dim=2)
    Yc = S.ssd_core(chunk(X), chunk(Brep), chunk(Crep), chunk(dt), chunk(A), b)
    del Brep, Crep
    torch.cuda.synchronize()
    Y = Yc.reshape(b, L, h, P)
    bs, hs = torch.tensor([0, 7]), torch.tensor(R0_HEADS)
    grp = torch.tensor([hh // r for hh in R0_HEADS])
    cpu = lambda t: t.cpu()[bs]  # noqa: E731
    Yr, _ = O.ssd_chunked(cpu(X)[:, :, hs], cpu(A)[:, :, hs], cpu(B)[:, :, grp], cpu(C)[:, :, grp], Q,
                          dt=cpu(dt)[:, :, hs])
    assert torch.isfinite(Y).all()
    assert_close(Y.cpu()[bs][:, :, hs], Yr, 2e-2)


def forward_by_kernels(X, A, B, C, Q, dt=None, initial_states=None):
    """The 16-bit forward at exactly chunk Q (64 / 128) through the per-kernel
    entry points, as ssd_forward runs that chunk: K1, K2 + K3 handing S_in
    over as f16 rows ("f16s"), K4 -> (Y, final state)."""
    Acs, decay = S.chunk_cumsum(A, Q)
    S_in, final = S.chunk_state_passing(X, B, Acs, decay, dt=dt, initial_states=initial_states, split="f16s")
    return S.chunk_scan(X, B, C, Acs, S_in, dt=dt, split="f16s"), final


@pytest.mark.parametrize("name", ["C3", "C4"])
def test_full_size_chunk_invariance_and_state_linearity(name):
    """Size-independent properties of the whole forward at the full config
    size (the oracle is too slow there): the chunked SSD computes one linear
    recurrence whatever the chunk length (MR:152-161), so the chunk-256
    persistent path (state chain, chunk_scan's persistent kernel) and the
    chunk-64 kernels agree; and Y is linear in the initial state,
    Y(X, S0) = Y(X, 0) + Y(0, S0), as is the final state.  Tolerances are the
    16-bit one relative to each output's scale (every Y is rounded to bf16
    once)."""
    cfg = CONFIGS[name]
    say("full-size properties", name)
    inp = to_dev(make_inputs(cfg, seed=3, device=DEV))
    X, A, B, C = inp["X"], inp["A"], inp["B"], inp["C"]
    gen = torch.Generator(device=DEV).manual_seed(4)
    S0 = 0.1 * torch.randn(cfg.batch, cfg.nheads, cfg.headdim, cfg.dstate, device=DEV, generator=gen)
    Y256, f256 = S.ssd_forward(X, A, B, C, 256, return_final_states=True)
    # ssd_forward itself runs these 16-bit shapes at chunk 256 for any block
    # length: the chunk-64 kernels one by one (f32-state chain, 16-bit chunk_scan)
    Y64, f64 = forward_by_kernels(X, A, B, C, 64)
    Yi, fi = S.ssd_forward(X, A, B, C, 256, initial_states=S0, return_final_states=True)
    Y0, f0 = S.ssd_forward(torch.zeros_like(X), A, B, C, 256, initial_states=S0, return_final_states=True)
    torch.cuda.synchronize()
    tol = tolerance(cfg.dtype)
    scale = Y256.float().abs().max().item()
    fscale = f256.abs().max().item()
    assert torch.isfinite(Y256).all() and torch.isfinite(f256).all()
    assert_close(Y64, Y256.float(), tol, atol=tol * scale)
    assert_close(f64, f256, tol, atol=tol * fscale)
    assert_close(Yi, Y256.float() + Y0.float(), tol, atol=tol * scale)
    assert_close(fi, f256 + f0, tol, atol=tol * fscale)


def test_long_context_weak_decay_recurrence():
    """C4 shape with A scaled by 1e-3: 256 chunks of carried state dominate."""
    cfg = CONFIGS["C4"]
    say("C4 weak decay")
    inp = to_dev(make_inputs(cfg, seed=1, device=DEV, a_scale=1e-3))
    Y, final = S.ssd_forward(inp["X"], inp["A"], inp["B"], inp["C"], cfg.chunk, return_final_states=True)
    X, A, B, C, _ = _slice_inputs(inp, [0], [5, 66], 1, cfg.nheads)
    Yr, fr = O.ssd_chunked(X, A, B, C, cfg.chunk)
    hs = torch.tensor([5, 66])
    assert_close(Y.cpu()[:, :, hs], Yr, 2e-2)
    assert_close(final.cpu()[:, hs], fr, 2e-2)


# ---------------------------------------------------------------------------
# properties of the launch path
# ---------------------------------------------------------------------------

def test_bitwise_deterministic():
    say("determinism")
    inp = to_dev(make_inputs(CONFIGS["C3"].scaled(batch=1, seqlen=1024), seed=2))
    a = S.ssd_forward(inp["X"], inp["A"], inp["B"], inp["C"], 256)
    b = S.ssd_forward(inp["X"], inp["A"], inp["B"], inp["C"], 256)
    assert torch.equal(a, b)


def test_runs_on_callers_stream():
    say("side stream")
    inp = to_dev(make_inputs(CONFIGS["C2"].scaled(batch=2, seqlen=512), seed=3))
    ref = S.ssd_forward(inp["X"], inp["A"], inp["B"], inp["C"], 64)
    side = torch.cuda.Stream()   # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y = S.ssd_forward(inp["X"], inp["A"], inp["B"], inp["C"], 64)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


def test_strided_views_like_the_reference_layer():
    """x as a transposed conv-output view and B/C as slices of an in_proj output (MR:76-91)."""
    say("strided views")
    b, L, h, P, g, N = 2, 256, 4, 64, 2, 64
    gen = torch.Generator().manual_seed(9)
    conv_out = torch.randn(b, h * P, L, generator=gen)                 # [b, d, l]
    X = conv_out.transpose(1, 2).unflatten(2, (h, P))                   # inner stride L, not 1
    proj = torch.randn(b, L, 3 * g * N + 8, generator=gen)             # row stride not contiguous in g*N
    B = proj[:, :, g * N:2 * g * N].unflatten(2, (g, N))
    C = proj[:, :, 2 * g * N:3 * g * N].unflatten(2, (g, N))
    A = -torch.rand(b, L, h, generator=gen)
    Yr, _ = O.ssd_chunked(X, A, B, C, 64)
    Y = S.ssd_forward(X.to(DEV), A.to(DEV), B.to(DEV), C.to(DEV), 64)
    assert_close(Y, Yr, 1e-4)


def test_library_errors_surface_as_exceptions():
    say("errors")
    X = torch.zeros(1, 96, 2, 64, device=DEV)
    A = torch.zeros(1, 96, 2, device=DEV)
    B = torch.zeros(1, 96, 1, 48, device=DEV)
    with pytest.raises(S.SSDError, match="d_state"):
        S.ssd_forward(X, A, B, B, 32)
    with pytest.raises(ValueError, match="multiple"):
        S.ssd_forward(X, A, B, B, 64)


@pytest.mark.parametrize("name", ["C1", "C5"])
def test_model_surface(name):
    say("model", name)
    model, inputs = build_workload(name, device=DEV)
    with torch.inference_mode():
        out = model(*inputs)
    Y = out[0] if isinstance(out, tuple) else out
    cfg = CONFIGS[name]
    args = (inputs[0][:1].cpu(), model.A[:1].detach().cpu(), model.B[:1].detach().cpu(), model.C[:1].detach().cpu(),
            cfg.chunk)
    init = inputs[1][:1].cpu() if len(inputs) > 1 else None
    if name == "C1":
        Yr, _, allowed, _, _ = f32_reference_bounds(*args, init=init)
        check_within(Y[:1], Yr, allowed)
    else:
        Yr, _ = O.ssd_chunked(*args, initial_states=init)
        assert_close(Y[:1], Yr, 1e-4)


def test_ssd_core_takes_the_reference_arguments():
    """MR:123-162's own argument layout: chunked [b, c, l, ...] tensors, B/C
    repeated per head, X unscaled with dt separate, f16 data (the reference's
    dtype) -- against the sequential scan."""
    say("ssd_core reference layout")
    b, c, l, h, p, n, g = 2, 3, 64, 8, 64, 32, 2
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(b, c * l, h, p, generator=gen).half()
    Bg = (torch.randn(b, c * l, g, n, generator=gen) / math.sqrt(n)).half()
    Cg = (torch.randn(b, c * l, g, n, generator=gen) / math.sqrt(n)).half()
    dt = torch.nn.functional.softplus(torch.randn(b, c * l, h, generator=gen) - 1.0)
    A = -torch.rand(h, generator=gen) - 0.5
    A_dt = A * dt
    Brep = Bg.repeat_interleave(h // g, dim=2)
    Crep = Cg.repeat_interleave(h // g, dim=2)
    chunk = lambda t: t.reshape(b, c, l, *t.shape[2:])  # noqa: E731
    Y = S.ssd_core(chunk(x).to(DEV), chunk(Brep).to(DEV), chunk(Crep).to(DEV), chunk(dt).to(DEV),
                   chunk(A_dt).to(DEV), b)
    assert Y.shape == (b, c, l, h, p) and Y.dtype == torch.float16
    Ys, _ = O.ssd_sequential(x, A_dt, Bg, Cg, dt=dt)
    assert_close(Y.reshape(b, c * l, h, p), Ys, 2e-2)


# ---------------------------------------------------------------------------
# seeded random shapes: every launch plan against the oracle
# ---------------------------------------------------------------------------

def _random_cases(n, seed=11):
    rng = np.random.default_rng(seed)
    cases = []
    for k in range(n):
        dtype = [torch.float32, torch.bfloat16, torch.float16][k % 3]
        Q = int(rng.choice([64, 128, 256]))
        N = int(rng.choice([16, 32, 64, 128]))
        g = int(rng.choice([1, 2, 4]))
        h = g * int(rng.integers(1, 6))
        if k % 5 == 4 and dtype != torch.float32:
            Q, N, h = 256, 128, 160   # 2 x 160 = 320 chains: the state chain's mixed plan at 256 CUs
        b = int(rng.integers(1, 3))
        nc = int(rng.integers(1, 4))
        cases.append((k, dtype, Q, N, g, h, b, nc, bool(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    return cases


@pytest.mark.parametrize("k,dtype,Q,N,g,h,b,nc,use_dt,use_init", _random_cases(20))
def test_random_shapes_vs_oracle(k, dtype, Q, N, g, h, b, nc, use_dt, use_init):
    """Seeded random shapes (dtype, chunk, d_state, groups, heads, batch,
    chunks, dt, initial state) through ssd_forward against the chunked
    oracle, Y and the final state."""
    say("random", k, dtype, Q, N, g, h, b, nc, use_dt, use_init)
    cfg = CONFIGS["C2"].scaled(batch=b, seqlen=Q * nc, nheads=h, dstate=N, chunk=Q, ngroups=g, dtype=dtype,
                               init_state=use_init)
    inp = make_inputs(cfg, seed=100 + k)
    gen = torch.Generator().manual_seed(200 + k)
    dt = (torch.rand(b, Q * nc, h, generator=gen) + 0.1) if use_dt else None
    d = to_dev(inp)
    Y, final = S.ssd_forward(d["X"], d["A"], d["B"], d["C"], Q, dt=None if dt is None else dt.to(DEV),
                             initial_states=d["init"], return_final_states=True)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        Yr, fr, aY, af, _ = f32_reference_bounds(inp["X"], inp["A"], inp["B"], inp["C"], Q, dt=dt, init=inp["init"])
        check_within(Y, Yr, aY)
        check_within(final, fr, af, "final")
        return
    Yr, fr = O.ssd_chunked(inp["X"], inp["A"], inp["B"], inp["C"], Q, dt=dt, initial_states=inp["init"])
    tol = tolerance(dtype)
    assert_close(Y, Yr, tol)
    assert_close(final, fr, tol)


def _sweep_cases(n, seed=2024):
    """Wider seeded random shapes than _random_cases: up to 8 groups and 8
    heads per group, 96-320 heads at chunk 256 / d_state 128 (the state
    chain's plans), 1-3 batch rows, 1-6 chunks, the split hand-over and the
    allocation-free entry point (where its array holds the workspace)."""
    rng = np.random.default_rng(seed)
    cases = []
    for k in range(n):
        dtype = [torch.float32, torch.bfloat16, torch.float16][k % 3]
        Q = int(rng.choice([64, 128, 256]))
        N = int(rng.choice([16, 32, 64, 128]))
        g = int(rng.choice([1, 2, 4, 8]))
        h = g * int(rng.integers(1, 9))
        if k % 7 == 3 and dtype != torch.float32:
            Q, N, h = 256, 128, int(rng.choice([96, 160, 200, 320]))
        b, nc = int(rng.integers(1, 4)), int(rng.integers(1, 7))
        if b * h * Q * nc > 400_000:
            nc = max(1, 400_000 // (b * h * Q))
        use_dt, use_init = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        split = dtype != torch.float32 and rng.integers(0, 4) == 0
        noalloc = bool(rng.integers(0, 5) == 0) and b * h * nc * 64 * N * 8 < (128 << 20)
        cases.append((k, dtype, Q, N, g, h, b, nc, use_dt, use_init, bool(split), noalloc))
    return cases


@pytest.mark.parametrize("k,dtype,Q,N,g,h,b,nc,use_dt,use_init,split,noalloc", _sweep_cases(120))
def test_random_forward_sweep(k, dtype, Q, N, g, h, b, nc, use_dt, use_init, split, noalloc):
    """ssd_forward (or ssd_forward_noalloc) on seeded random shapes against
    the chunked oracle, Y and the final state, with the checks of
    test_random_shapes_vs_oracle."""
    say("sweep", k, dtype, Q, N, g, h, b, nc, use_dt, use_init, split, noalloc)
    cfg = CONFIGS["C2"].scaled(batch=b, seqlen=Q * nc, nheads=h, dstate=N, chunk=Q, ngroups=g, dtype=dtype,
                               init_state=use_init)
    inp = make_inputs(cfg, seed=5000 + k)
    gen = torch.Generator().manual_seed(7000 + k)
    dt = (torch.rand(b, Q * nc, h, generator=gen) + 0.1) if use_dt else None
    d = to_dev(inp)
    fwd = S.ssd_forward_noalloc if noalloc else S.ssd_forward
    Y, final = fwd(d["X"], d["A"], d["B"], d["C"], Q, dt=None if dt is None else dt.to(DEV),
                   initial_states=d["init"], return_final_states=True, state_format="split" if split else None)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        Yr, fr, aY, af, _ = f32_reference_bounds(inp["X"], inp["A"], inp["B"], inp["C"], Q, dt=dt, init=inp["init"])
        check_within(Y, Yr, aY)
        check_within(final, fr, af, "final")
        return
    Yr, fr = O.ssd_chunked(inp["X"], inp["A"], inp["B"], inp["C"], Q, dt=dt, initial_states=inp["init"])
    tol = tolerance(dtype)
    assert_close(Y, Yr, tol)
    assert_close(final, fr, tol)
