"""The Python wrappers reject operands the C ABI would read without a size
(per-kernel entry points take raw pointers): wrong shapes and dtypes of
states, Acs, prep buffers, and parameters on another device.  Every case
raises on the host before any kernel is launched."""

import pytest
import torch

from workloadsuite_amd import ssd as S

pytestmark = pytest.mark.gpu

DEV = "cuda"


def operands(dtype=torch.bfloat16, b=1, L=512, h=2, P=64, g=1, N=64, Q=256):
    X = torch.zeros(b, L, h, P, dtype=dtype, device=DEV)
    B = torch.zeros(b, L, g, N, dtype=dtype, device=DEV)
    Acs = torch.zeros(b, h, L // Q, Q, device=DEV)
    states = torch.zeros(b, L // Q, h, P, N, device=DEV)
    return X, B, Acs, states


def test_chunk_scan_rejects_wrong_states():
    print("CASE chunk_scan states checks", flush=True)
    X, B, Acs, states = operands()
    with pytest.raises(ValueError, match="states must be"):
        S.chunk_scan(X, B, B, Acs, states[:, :, :1])                     # too few heads
    with pytest.raises(ValueError, match="states must be"):
        S.chunk_scan(X, B, B, Acs, states.to(torch.bfloat16), split=True)  # split needs f32 rows
    with pytest.raises(ValueError, match="unsupported state dtype"):
        S.chunk_scan(X, B, B, Acs, states.to(torch.float16))
    with pytest.raises(ValueError, match="Acs must be"):
        S.chunk_scan(X, B, B, Acs[:, :, :1], states)
    with pytest.raises(ValueError, match="split states"):
        S.chunk_scan(X.float(), B.float(), B.float(), Acs, states, split=True)


def test_prep_buffer_must_fit():
    print("CASE prep size checks", flush=True)
    X, B, Acs, states = operands()
    small = torch.zeros(16, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="prep must be"):
        S.chunk_scan(X, B, B, Acs, states, prep=small)
    with pytest.raises(ValueError, match="prep must be"):
        S.chunk_state(X, B, Acs, prep=small)


def test_state_passing_rejects_wrong_decay_and_init():
    print("CASE state_passing checks", flush=True)
    _, _, _, states = operands()
    decay = torch.ones(1, 2, 2, device=DEV)
    with pytest.raises(ValueError, match="chunk_decay must be"):
        S.state_passing(states, decay[:, :1])
    with pytest.raises(ValueError, match="initial_states must be"):
        S.state_passing(states, decay, torch.zeros(1, 2, 64, 32, device=DEV))


def test_decode_step_rejects_host_parameters():
    print("CASE decode_step device checks", flush=True)
    b, h, P, N, g = 2, 4, 64, 64, 1
    state = torch.zeros(b, h, P, N, device=DEV)
    x = torch.zeros(b, h, P, dtype=torch.bfloat16, device=DEV)
    Bm = torch.zeros(b, g, N, dtype=torch.bfloat16, device=DEV)
    a = torch.zeros(b, h, device=DEV)
    with pytest.raises(ValueError, match="HIP devices only"):
        S.decode_step(state, x, Bm, Bm, a, D=torch.ones(h))              # D on the host
    with pytest.raises(ValueError, match="HIP devices only"):
        S.decode_step(state, x, Bm, Bm, a, z=torch.zeros(b, h, P, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="D must have"):
        S.decode_step(state, x, Bm, Bm, a, D=torch.ones(h + 1, device=DEV))
