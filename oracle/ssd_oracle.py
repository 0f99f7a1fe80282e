"""CPU oracle for the Mamba-2 SSD forward -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed
CPU baseline).  The product path (``workloadsuite_amd``) never calls it; it
fails loudly when its HIP library is missing.

Reference: ``workloads/mamba/model_ref.py`` ("MR") in ShouyangDong/WorkloadSuite.
The reference's hot path is ``SSDLayer._ssd_core`` (MR:123-162).  That function
is fp16-only as written (it hard-casts four intermediates to float16 at MR:145,
148, 155, 160), so this restatement lifts those casts to one compute dtype
(float64 for parity, float32 for the timed CPU baseline).  Everything else
follows the reference's algorithm:

  chunk_cumsum   MR:135-136, MR:150   intra-chunk prefix sum of the log-decays
  segsum_decay   MR:139-141           L[l,s] = exp(Acs[l]-Acs[s]) for s<=l else 0
  chunk_state    MR:144, MR:148-149   S_local = B^T (decay_to_end * dt * X)
  state_passing  MR:152-157           exclusive recurrence over chunks
  chunk_scan     MR:143-145, 160-162  Y = (L*CB^T) (dt*X) + exp(Acs) C S_in
  ssd_chunked    MR:123-162           composition of the above
  ssd_sequential (closed form)        h_t = e^{a_t} h_{t-1} + (dt_t x_t) B_t^T,
                                      y_t = h_t C_t  -- the recurrence the chunked
                                      algorithm factorises (SSD duality)

Layouts are the ones the HIP library uses (they differ from MR only by the
order of the state axes, see ``state_passing``):

  X  [b, L, h, P]        A (= A*dt, the log-decay) [b, L, h]
  B, C [b, L, g, N]      dt [b, L, h] (optional, None means dt == 1)
  Acs [b, h, c, Q]       chunk_decay [b, h, c]
  states [b, c, h, P, N] initial/final state [b, h, P, N]

Head i reads group i // (h // g) of B and C, which is what MR's
``repeat(B, "b l g n -> b l (g r) n")`` (MR:97-99) produces.

Pinning (what checks this oracle, ``tests/test_oracle.py``): the reference
holds no golden vectors for this path, so every function is pinned by
mathematics -- the fp64 sequential scan (an O(L) recurrence written
independently of the chunked factorisation), brute-force loops on tiny inputs,
closed forms (A == 0 gives prefix sums; one state dimension with B = C = 1 gives
a discounted cumulative sum), the segsum semigroup identity, chunk-size
invariance, initial-state linearity, and einops itself (the library MR calls)
for the group broadcast and the chunk layout.  Every function below has at
least one such check; none is "parity unpinned".
"""

from __future__ import annotations

import numpy as np
import torch

__all__ = [
    "expand_groups",
    "chunk_cumsum",
    "segsum_decay",
    "chunk_state",
    "state_passing",
    "chunk_scan",
    "ssd_chunked",
    "ssd_sequential",
]


def expand_groups(T: torch.Tensor, nheads: int) -> torch.Tensor:
    """[b, L, g, N] -> [b, L, h, N]; head i reads group i // (h // g) (MR:97-99)."""
    g = T.shape[2]
    if nheads % g != 0:
        raise ValueError("n_heads must be divisible by n_groups")
    return T.repeat_interleave(nheads // g, dim=2)


def _chunked(T: torch.Tensor, Q: int) -> torch.Tensor:
    """[b, L, ...] -> [b, c, Q, ...] with position = chunk*Q + offset (MR:106-110)."""
    b, L = T.shape[:2]
    if L % Q != 0:
        raise ValueError(f"seqlen {L} is not a multiple of chunk size {Q}")
    return T.reshape(b, L // Q, Q, *T.shape[2:])


def chunk_cumsum(A: torch.Tensor, Q: int):
    """Intra-chunk inclusive prefix sum of the log-decays (MR:135-136) and the
    per-chunk total decay exp(Acs[..., -1]) (MR:150).

    A [b, L, h] -> Acs [b, h, c, Q], chunk_decay [b, h, c].
    """
    Ac = _chunked(A, Q)                                   # [b, c, Q, h]
    Acs = torch.cumsum(Ac, dim=2).permute(0, 3, 1, 2)     # [b, h, c, Q]
    return Acs.contiguous(), torch.exp(Acs[..., -1])


def segsum_decay(Acs: torch.Tensor) -> torch.Tensor:
    """L[..., l, s] = exp(Acs[l] - Acs[s]) for s <= l, else 0 (MR:139-141).

    The causal mask is applied to the exponent (``-inf``) before ``exp`` so that
    positive log-decays above the diagonal cannot overflow into inf * 0.
    """
    Q = Acs.shape[-1]
    diff = Acs[..., :, None] - Acs[..., None, :]
    causal = torch.ones(Q, Q, dtype=torch.bool).tril()
    return torch.exp(diff.masked_fill(~causal, float("-inf")))


def _scaled_x(X: torch.Tensor, dt) -> torch.Tensor:
    """X * dt (MR:144); dt None means the dt-free form the benchmark configs use."""
    return X if dt is None else X * dt[..., None]


def chunk_state(X, B, Acs, dt=None):
    """Per-chunk local state (MR:148-149):
    S_local[b,c,h,p,n] = sum_l X[l,p] * dt[l] * exp(Acs[Q-1] - Acs[l]) * B[l,n].

    MR stores this as [b,c,h,N,P]; this oracle (and the HIP library) keeps the
    state as [.., P, N] so that the final state comes out as [b, h, P, N].
    """
    b, L, h, P = X.shape
    Q = Acs.shape[-1]
    Xc = _chunked(_scaled_x(X, dt), Q)                    # [b, c, Q, h, P]
    Bc = _chunked(expand_groups(B, h), Q)                 # [b, c, Q, h, N]
    decay_to_end = torch.exp(Acs[..., -1:] - Acs)         # [b, h, c, Q]
    w = decay_to_end.permute(0, 2, 3, 1)                  # [b, c, Q, h]
    return torch.einsum("bclhp,bclh,bclhn->bchpn", Xc, w, Bc)


def state_passing(S_local, chunk_decay, initial_states=None):
    """Exclusive recurrence over chunks (MR:152-157):
    S_in[0] = init (zeros in MR:153), S_in[c+1] = chunk_decay[c] * S_in[c] + S_local[c].

    Returns (S_in [b,c,h,P,N], final [b,h,P,N]); ``final`` is the state after the
    last chunk, which MR computes and discards (MR:156).
    """
    b, c, h, P, N = S_local.shape
    state = (torch.zeros(b, h, P, N, dtype=S_local.dtype)
             if initial_states is None else initial_states.to(S_local.dtype).clone())
    S_in = torch.empty_like(S_local)
    for i in range(c):
        S_in[:, i] = state
        state = chunk_decay[:, :, i, None, None] * state + S_local[:, i]
    return S_in, state


def chunk_scan(X, B, C, Acs, S_in, dt=None):
    """Intra-chunk output plus state-to-output term (MR:139-145, 160-162):
    Y[l,p] = sum_{s<=l} exp(Acs[l]-Acs[s]) (C_l . B_s) dt_s X[s,p]
             + exp(Acs[l]) sum_n C[l,n] S_in[p,n].
    Processed one chunk at a time so the [b,h,Q,Q] decay stays bounded.
    """
    b, L, h, P = X.shape
    Q = Acs.shape[-1]
    nc = L // Q
    Xc = _chunked(_scaled_x(X, dt), Q)                    # [b, c, Q, h, P]
    Bc = _chunked(expand_groups(B, h), Q)
    Cc = _chunked(expand_groups(C, h), Q)
    Y = torch.empty(b, nc, Q, h, P, dtype=Xc.dtype)
    for i in range(nc):
        Lmat = segsum_decay(Acs[:, :, i])                 # [b, h, Q, Q]
        CB = torch.einsum("blhn,bshn->bhls", Cc[:, i], Bc[:, i])
        y_diag = torch.einsum("bhls,bshp->blhp", Lmat * CB, Xc[:, i])
        decay_from_start = torch.exp(Acs[:, :, i]).permute(0, 2, 1)    # [b, Q, h]
        y_off = torch.einsum("blhn,bhpn->blhp", Cc[:, i], S_in[:, i]) * decay_from_start[..., None]
        Y[:, i] = y_diag + y_off
    return Y.reshape(b, L, h, P)


def ssd_chunked(X, A, B, C, chunk_size, dt=None, initial_states=None, dtype=torch.float64):
    """Whole chunked SSD forward (MR:123-162) in one compute dtype on the CPU.

    Inputs are upcast to ``dtype`` first (bf16/fp16 inputs keep their rounded
    values).  Returns (Y [b,L,h,P], final_state [b,h,P,N]).
    """
    cast = lambda t: None if t is None else t.detach().to("cpu", dtype)  # noqa: E731
    X, A, B, C, dt, init = map(cast, (X, A, B, C, dt, initial_states))
    Acs, decay = chunk_cumsum(A, chunk_size)
    S_local = chunk_state(X, B, Acs, dt)
    S_in, final = state_passing(S_local, decay, init)
    Y = chunk_scan(X, B, C, Acs, S_in, dt)
    return Y, final


def ssd_sequential(X, A, B, C, dt=None, initial_states=None):
    """fp64 O(L) linear recurrence that the chunked algorithm factorises:

        h_t = exp(a_t) h_{t-1} + (dt_t x_t) B_t^T      h_{-1} = init (or 0)
        y_t = h_t C_t

    with h_t [b,h,P,N].  Written in numpy, independently of the chunked path.
    Returns (Y [b,L,h,P], final_state [b,h,P,N]) as float64 numpy arrays.
    """
    f64 = lambda t: None if t is None else np.asarray(t.detach().cpu().double().numpy() if isinstance(t, torch.Tensor) else t, dtype=np.float64)  # noqa: E731
    X, A, B, C, dt, init = map(f64, (X, A, B, C, dt, initial_states))
    b, L, h, P = X.shape
    g, N = B.shape[2], B.shape[3]
    grp = np.arange(h) // (h // g)
    state = np.zeros((b, h, P, N)) if init is None else init.copy()
    Y = np.empty((b, L, h, P))
    for t in range(L):
        xt = X[:, t] if dt is None else X[:, t] * dt[:, t, :, None]     # [b, h, P]
        Bt = B[:, t][:, grp]                                             # [b, h, N]
        Ct = C[:, t][:, grp]
        state = np.exp(A[:, t])[:, :, None, None] * state + xt[..., :, None] * Bt[..., None, :]
        Y[:, t] = np.einsum("bhpn,bhn->bhp", state, Ct)
    return Y, state
