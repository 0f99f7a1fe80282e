"""How ssd_forward runs K2 + K3 at a shape, restated for the tests that
compare it with the public per-kernel entry points (GPU only).

At chunk 256 with 16-bit inputs the forward runs chunk_state and
state_passing as one state-chain launch when the (batch, head) chains keep
every CU about equally busy (at least 3/4 of the busiest CU's chains on the
average CU), a mixed plan between one and two chains per CU (one whole
chain per CU, the remaining chains in segments whose local states
state_passing finishes), and otherwise the two kernels one after the other.
The chain keeps each local state in registers as f32; where S_in goes to
chunk_scan as "f16s", the local states that do cross HBM (the two kernels,
the mixed plan's segments) go as f16 rows with per-tile scales
(chunk_state(..., state_dtype="f16s")).  The chain's f16s store needs
d_state 128."""

import torch

from workloadsuite_amd import ssd as S


def chain_plan(chains):
    """The library's dispatch rule (chunk_state_chain_plan) on this device:
    "whole" (every chain in one workgroup), "mixed" (one whole chain per CU,
    the rest in segments finished by state_passing) or None (chunk_state then
    state_passing)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_cu = -(-chains // cus)
    if 4 * chains >= 3 * per_cu * cus:
        return "whole"
    if cus < chains < 2 * cus:
        return "mixed"
    return None


def f16_local_mask(chains, N):
    """Per chain b * nheads + h: True where the forward with the f16s hand-over
    passes the chain's local states through HBM as f16 rows."""
    plan = chain_plan(chains) if N == 128 else None
    if plan is None:
        return [True] * chains
    if plan == "whole":
        return [False] * chains
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return [bh >= cus for bh in range(chains)]


def f16_local(chains, N):
    """True where some chain's local states cross HBM as f16 rows."""
    return any(f16_local_mask(chains, N))


def k2_k3_f16s(X, B, Acs, decay, dt=None, prep=None, initial_states=None):
    """chunk_state then state_passing with S_in as "f16s", each chain's local
    states in the format the forward passes them in at this shape (chunk 256,
    16-bit inputs, prep given as the forward computes it): (F16SStates, final)."""
    b, h = X.shape[0], X.shape[2]
    mask = f16_local_mask(b * h, B.shape[-1])
    run = lambda **kw: S.state_passing(S.chunk_state(X, B, Acs, dt=dt, prep=prep, **kw), decay,  # noqa: E731
                                       initial_states=initial_states, split="f16s")
    if all(mask):
        return run(state_dtype="f16s")
    if not any(mask):
        return run()
    (s16, f16), (s32, f32) = run(state_dtype="f16s"), run()
    m = torch.tensor(mask, device=X.device).reshape(b, h)
    states = torch.where(m[:, None, :, None, None], s16.states, s32.states)
    scales = torch.where(m[:, None, :, None], s16.scales, s32.scales)
    final = None if f16 is None else torch.where(m[:, :, None, None], f16, f32)
    return S.F16SStates(states, scales), final
