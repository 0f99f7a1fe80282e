"""The chunk-256 forward (and the f32 forward at chunk 64 / 128, at the end
of this file) runs chunk_state and state_passing as one launch
(each workgroup walks one (batch, head) chain of chunks with the running
state in registers, workloads/mamba/model_ref.py:144-157) when the chains
keep every CU about equally busy: at least 3/4 of the busiest CU's chains on
the average CU.  Between one and two chains per CU it runs one whole chain
per CU and the remaining chains in segments whose local states
state_passing finishes.  The shapes here have 192-256 chains (one per CU on
a 256-CU MI355X), 640 (three per CU) or 300-360 (the mixed plan).  It must give exactly what the two kernels
give one after the other: ssd_forward against the public per-kernel entry
points, bit for bit (Y and the final state), with and without dt and an
initial state, both 16-bit types, both dstates, several groups, for both
formats in which state_passing hands f32 states to chunk_scan (hi/lo pairs,
"split"; f16 rows with a power-of-two scale per row, "f16s", the default).
With "f16s" the local states that cross HBM (chunk_state then
state_passing; the mixed plan's segments) go as f16 rows, so the per-kernel
reference passes each chain's local states in the format the forward uses
for it (tests/state_plans.py).
The per-kernel path itself is held to the oracle by the parity tests."""

import pytest
import torch

from state_plans import chain_plan, k2_k3_f16s
from workloadsuite_amd import ssd as S

pytestmark = pytest.mark.gpu

DEV = "cuda"


def takes_chain(chains):
    return chain_plan(chains) is not None


FORMATS = ["split", "f16s"]


def kernels_one_by_one(X, A, B, C, dt, init, fmt, Q=256):
    """K1, K0, K2, K3 (handing S_in over in `fmt`), K4 through their own entry points."""
    Acs, decay = S.chunk_cumsum(A, Q)
    prep = S.chunk_prep(B, C, Q)
    if fmt == "f16s":
        # f32 local states where the forward runs the state chain, f16 rows
        # where it runs chunk_state then state_passing (d_state 64 here)
        S_in, fk = k2_k3_f16s(X, B, Acs, decay, dt=dt, prep=prep, initial_states=init)
    else:
        st = S.chunk_state(X, B, Acs, dt=dt, prep=prep)
        S_in, fk = S.state_passing(st, decay, initial_states=init, split=X.dtype)
    Yk = S.chunk_scan(X, B, C, Acs, S_in, dt=dt, prep=prep, split=True if fmt == "split" else "f16s")
    return Yk, fk


def handover_bytes(S_in, fmt):
    """The bytes of handed-over states that carry data: all of them for
    "split"; for "f16s" (S.F16SStates) the f16 half of each row and the row
    scales."""
    if fmt != "f16s":
        return S_in.view(torch.uint8)
    N = S_in.states.shape[-1]
    return torch.cat([S_in.states.view(torch.float16)[..., :N].contiguous().view(torch.uint8).reshape(-1),
                      S_in.scales.contiguous().view(torch.uint8).reshape(-1)])


def case(dtype, b, L, h, P, N, g, seed):
    gen = torch.Generator().manual_seed(seed)
    X = torch.randn(b, L, h, P, generator=gen).to(dtype)
    A = -torch.rand(b, L, h, generator=gen) * 0.2
    B = (torch.randn(b, L, g, N, generator=gen) * N ** -0.5).to(dtype)
    C = (torch.randn(b, L, g, N, generator=gen) * N ** -0.5).to(dtype)
    dt = torch.rand(b, L, h, generator=gen) + 0.1
    init = torch.randn(b, h, P, N, generator=gen)
    return [t.to(DEV) for t in (X, A, B, C, dt, init)]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,g,h", [(128, 1, 96), (64, 2, 128), (128, 4, 112)])
@pytest.mark.parametrize("with_dt,with_init", [(True, True), (False, False), (True, False)])
def test_forward_equals_kernels_one_by_one(dtype, N, g, h, with_dt, with_init, fmt):
    b, L, P, Q = 2, 1280, 64, 256
    print("CASE chain", dtype, N, g, h, with_dt, with_init, fmt, flush=True)
    if not takes_chain(b * h):
        pytest.skip("this device's CU count sends the shape to chunk_state then state_passing")
    X, A, B, C, dt, init = case(dtype, b, L, h, P, N, g, seed=N + g + h)
    dt = dt if with_dt else None
    init = init if with_init else None
    Y, final = S.ssd_forward(X, A, B, C, Q, dt=dt, initial_states=init, return_final_states=True, state_format=fmt)
    Yk, fk = kernels_one_by_one(X, A, B, C, dt, init, fmt, Q)
    torch.cuda.synchronize()
    assert torch.equal(final, fk)
    assert torch.equal(Y, Yk)


@pytest.mark.parametrize("fmt", FORMATS)
def test_single_chunk_and_many_chains(fmt):
    """One chunk per chain (the loop body runs once) and more chains than the
    GPU holds at once."""
    for (b, L, h) in [(2, 256, 100), (4, 512, 160)]:
        print("CASE chain shape", b, L, h, fmt, flush=True)
        if not takes_chain(b * h):
            pytest.skip("this device's CU count sends the shape to chunk_state then state_passing")
        X, A, B, C, dt, init = case(torch.bfloat16, b, L, h, 64, 128, 1, seed=L + h)
        Y, final = S.ssd_forward(X, A, B, C, 256, dt=dt, initial_states=init, return_final_states=True,
                                 state_format=fmt)
        Yk, fk = kernels_one_by_one(X, A, B, C, dt, init, fmt)
        torch.cuda.synchronize()
        assert torch.equal(final, fk)
        assert torch.equal(Y, Yk)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,h,L,g", [(2, 160, 1280, 1), (3, 120, 2048, 4), (1, 300, 256, 2), (2, 150, 4096, 2)])
def test_mixed_plan_equals_kernels_one_by_one(dtype, b, h, L, g, fmt):
    """Whole chains, segments of the remaining chains (ragged last segment
    with 5 chunks, a single chunk, 16 chunks), state_passing over those
    chains only, with an initial state and the final state."""
    print("CASE chain mixed", dtype, b, h, L, g, fmt, flush=True)
    if chain_plan(b * h) != "mixed":
        pytest.skip("this device's CU count does not give the mixed plan for this shape")
    X, A, B, C, dt, init = case(dtype, b, L, h, 64, 128, g, seed=b * h + L)
    Y, final = S.ssd_forward(X, A, B, C, 256, dt=dt, initial_states=init, return_final_states=True,
                             state_format=fmt)
    Yk, fk = kernels_one_by_one(X, A, B, C, dt, init, fmt)
    torch.cuda.synchronize()
    assert torch.equal(final, fk)
    assert torch.equal(Y, Yk)


@pytest.mark.parametrize("b,h,L", [(2, 128, 1280), (2, 160, 1280), (1, 24, 512)])
@pytest.mark.parametrize("split", [torch.bfloat16, "f16s", None])
def test_chunk_state_passing_entry_point(b, h, L, split):
    """ssd_chunk_state_passing (whole chains, the mixed plan, or chunk_state
    then state_passing, by shape) against the two entry points it stands for,
    bit for bit (with f16 local states for "f16s" where the two run as
    separate launches); also without split (f32 S_in, always two launches)."""
    print("CASE chunk_state_passing", b, h, L, split, flush=True)
    X, A, B, C, dt, init = case(torch.bfloat16, b, L, h, 64, 128, 2, seed=h + L)
    Acs, decay = S.chunk_cumsum(A, 256)
    prep = S.chunk_prep(B, C, 256)
    S_in, final = S.chunk_state_passing(X, B, Acs, decay, dt=dt, prep=prep, initial_states=init, split=split)
    if split == "f16s":
        # the local states as the forward passes them at this shape (f16 rows
        # where chunk_state then state_passing run)
        S_ref, f_ref = k2_k3_f16s(X, B, Acs, decay, dt=dt, prep=prep, initial_states=init)
    else:
        st = S.chunk_state(X, B, Acs, dt=dt, prep=prep)
        S_ref, f_ref = S.state_passing(st, decay, initial_states=init, split=split)
    torch.cuda.synchronize()
    assert torch.equal(final, f_ref)
    fmt = "f16s" if split == "f16s" else "split"
    assert torch.equal(handover_bytes(S_in, fmt), handover_bytes(S_ref, fmt))


# ---------------------------------------------------------------------------
# f32 inputs and states (chunk 64 / 128): K2 + K3 always run as one launch
# where chunk x d_state <= 8192
# ---------------------------------------------------------------------------

F32_SHAPES = [
    # (b, L, h, N, g, Q): 192 chains of 32 chunks (C2-like), many short chains
    # with groups (C5-like), one chunk per chain, chunk 128 x d_state 128
    # (no one-launch form: chunk_state then state_passing)
    (2, 2048, 24, 128, 1, 64),
    (8, 512, 64, 64, 8, 128),
    (3, 128, 20, 64, 4, 128),
    (2, 640, 6, 128, 3, 64),
    (1, 512, 4, 128, 2, 128),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,L,h,N,g,Q", F32_SHAPES)
@pytest.mark.parametrize("with_dt,with_init", [(True, True), (False, False), (False, True)])
def test_f32_chain_entry_point(b, L, h, N, g, Q, with_dt, with_init, dtype):
    """ssd_chunk_state_passing with f32 states against chunk_state then
    state_passing: S_in and the final state bit for bit (f32 inputs, and
    16-bit inputs at chunk 64 / 128, which the same f32-MFMA kernels take)."""
    print("CASE f32 chain", dtype, b, L, h, N, g, Q, with_dt, with_init, flush=True)
    X, A, B, C, dt, init = case(dtype, b, L, h, 64, N, g, seed=L + h + N)
    dt = dt if with_dt else None
    init = init if with_init else None
    Acs, decay = S.chunk_cumsum(A, Q)
    S_in, final = S.chunk_state_passing(X, B, Acs, decay, dt=dt, initial_states=init)
    st = S.chunk_state(X, B, Acs, dt=dt)
    S_ref, f_ref = S.state_passing(st, decay, initial_states=init)
    torch.cuda.synchronize()
    assert torch.equal(final, f_ref)
    assert torch.equal(S_in, S_ref)


@pytest.mark.parametrize("b,L,h,N,g,Q", F32_SHAPES[:3])
def test_f32_forward_equals_kernels_one_by_one(b, L, h, N, g, Q):
    """ssd_forward on f32 inputs (the one-launch state chain) against K1, K2,
    K3 and K4 through their own entry points: Y and the final state bit for bit."""
    print("CASE f32 forward", b, L, h, N, g, Q, flush=True)
    X, A, B, C, dt, init = case(torch.float32, b, L, h, 64, N, g, seed=3 * L + h)
    Y, final = S.ssd_forward(X, A, B, C, Q, dt=dt, initial_states=init, return_final_states=True)
    Acs, decay = S.chunk_cumsum(A, Q)
    st = S.chunk_state(X, B, Acs, dt=dt)
    S_in, fk = S.state_passing(st, decay, initial_states=init)
    Yk = S.chunk_scan(X, B, C, Acs, S_in, dt=dt)
    torch.cuda.synchronize()
    assert torch.equal(final, fk)
    assert torch.equal(Y, Yk)


def _f16_halves(s):
    """The f16 values of f16s states (the first half of each f32 row)."""
    return s.states.view(torch.float16)[..., :s.states.shape[-1]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,L,h,N,g,Q", F32_SHAPES)
@pytest.mark.parametrize("with_dt,with_init", [(True, True), (False, False)])
def test_chain_f16s_entry_point(b, L, h, N, g, Q, with_dt, with_init, dtype):
    """16-bit inputs at chunk 64 / 128 with S_in handed over as "f16s" (f16
    rows, a power-of-two scale per row): ssd_chunk_state_passing (the chain,
    whose 4 waves per state row exchange the row maxima through LDS) against
    chunk_state then state_passing(split="f16s"): the f16 values, the row
    scales and the final state bit for bit."""
    print("CASE chain f16s", dtype, b, L, h, N, g, Q, with_dt, with_init, flush=True)
    X, A, B, C, dt, init = case(dtype, b, L, h, 64, N, g, seed=L + h + N + 1)
    dt = dt if with_dt else None
    init = init if with_init else None
    Acs, decay = S.chunk_cumsum(A, Q)
    S_in, final = S.chunk_state_passing(X, B, Acs, decay, dt=dt, initial_states=init, split="f16s")
    st = S.chunk_state(X, B, Acs, dt=dt)
    S_ref, f_ref = S.state_passing(st, decay, initial_states=init, split="f16s")
    torch.cuda.synchronize()
    assert torch.equal(final, f_ref)
    assert torch.equal(S_in.scales, S_ref.scales)
    assert torch.equal(_f16_halves(S_in), _f16_halves(S_ref))


# 16-bit shapes that ssd_forward runs at their own chunk: F32_SHAPES[:4] with
# seqlens that 256 does not divide (16-bit inputs at chunk 64 / 128 with
# seqlen % 256 == 0 run at chunk 256: test_routed_forward_is_the_chunk_256_forward)
B16_FORWARD_SHAPES = [
    (2, 2112, 24, 128, 1, 64),
    (8, 640, 64, 64, 8, 128),
    (3, 128, 20, 64, 4, 128),
    (2, 640, 6, 128, 3, 64),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,L,h,N,g,Q", B16_FORWARD_SHAPES)
def test_16bit_forward_f16s_equals_kernels_one_by_one(b, L, h, N, g, Q, dtype):
    """ssd_forward on 16-bit inputs at chunk 64 / 128 hands S_in to the 16-bit
    chunk_scan as "f16s": Y and the final state bit for bit against K1, K2 + K3
    (split="f16s") and K4 (split="f16s") through their own entry points."""
    print("CASE 16-bit forward f16s", dtype, b, L, h, N, g, Q, flush=True)
    assert S.forward_chunk(b, L, h, 64, N, g, Q, dtype) == Q
    X, A, B, C, dt, init = case(dtype, b, L, h, 64, N, g, seed=5 * L + h)
    Y, final = S.ssd_forward(X, A, B, C, Q, dt=dt, initial_states=init, return_final_states=True)
    Acs, decay = S.chunk_cumsum(A, Q)
    S_in, fk = S.chunk_state_passing(X, B, Acs, decay, dt=dt, initial_states=init, split="f16s")
    Yk = S.chunk_scan(X, B, C, Acs, S_in, dt=dt, split="f16s")
    torch.cuda.synchronize()
    assert torch.equal(final, fk)
    assert torch.equal(Y, Yk)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,L,h,N,g,Q", [(2, 2048, 24, 128, 1, 64), (8, 512, 64, 64, 4, 128),
                                         (1, 1024, 32, 128, 8, 64)])
def test_routed_forward_is_the_chunk_256_forward(b, L, h, N, g, Q, dtype):
    """16-bit inputs at chunk 64 / 128 with seqlen % 256 == 0 and d_state
    64 / 128: ssd_forward runs them at chunk 256 (the library's
    ssd_forward_chunk), so Y and the final state are those of the chunk-256
    call bit for bit; the no-alloc entry point runs them the same way."""
    print("CASE routed forward", dtype, b, L, h, N, g, Q, flush=True)
    assert S.forward_chunk(b, L, h, 64, N, g, Q, dtype) == 256
    X, A, B, C, dt, init = case(dtype, b, L, h, 64, N, g, seed=7 * L + h)
    Y, final = S.ssd_forward(X, A, B, C, Q, dt=dt, initial_states=init, return_final_states=True)
    Y256, f256 = S.ssd_forward(X, A, B, C, 256, dt=dt, initial_states=init, return_final_states=True)
    Yn, fn = S.ssd_forward_noalloc(X, A, B, C, Q, dt=dt, initial_states=init, return_final_states=True)
    torch.cuda.synchronize()
    assert torch.equal(Y, Y256) and torch.equal(final, f256)
    assert torch.equal(Yn, Y256) and torch.equal(fn, f256)
