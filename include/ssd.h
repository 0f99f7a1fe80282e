/*
 * libssd -- MI355X (gfx950) Mamba-2 SSD forward, C ABI.
 *
 * Replaces the hot path of ShouyangDong/WorkloadSuite
 * workloads/mamba/model_ref.py ("MR"): SSDLayer._ssd_core (MR:123-162), which
 * its only caller SSDLayer.forward invokes at MR:112.  The reference is pure
 * Python/PyTorch, so it has no FFI of its own; these entry points are what a
 * ctypes (or cffi / pybind) binding of that function binds.  The Python side
 * that mirrors _ssd_core is workloadsuite_amd/ssd.py.
 *
 * Conventions
 *   - Every pointer is a device pointer (HIP device memory) unless noted.
 *   - Strides are in ELEMENTS; the innermost dimension must have stride 1.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Every kernel is
 *     launched on it; nothing synchronises the host.
 *   - Except ssd_forward_noalloc, no entry point allocates or frees device
 *     memory or keeps a pointer past the call: the caller owns every buffer,
 *     workspaces included.  ssd_forward_noalloc's workspace is a static
 *     __device__ array of SSD_NOALLOC_SCRATCH_BYTES (256 MiB) in the
 *     library's code object, so every device on which any libssd kernel
 *     loads holds it from then until the process ends, whether or not the
 *     process ever calls ssd_forward_noalloc.
 *   - Return value: 0 on success, a negative SSD_ERR_* for invalid arguments
 *     (checked on the host before any launch), a positive hipError_t when a
 *     launch fails.  ssd_strerror() names both.  No exit/abort in the library.
 *   - Thread-safe and re-entrant.  Host-side state: a per-device cache of the
 *     CU count (the state chain's launch plan), and ssd_forward_noalloc's
 *     per-device cache of its array's device address (behind a mutex; stale
 *     after hipDeviceReset).  Calls of ssd_forward_noalloc that overlap on
 *     one device race on its array.
 *   - Operands copied to LDS 16 bytes at a time (x, bmat, cmat, a_cumsum,
 *     states, initial / final states) need 16-byte aligned bases and rows;
 *     SSD_ERR_MISALIGNED otherwise.
 *
 * Layouts (b batch, L seqlen, h heads, P headdim, N dstate, g groups,
 *          Q chunk, c = L / Q chunks):
 *   x, y          [b, L, h, P]  dtype (f32 / bf16 / f16)
 *   a             [b, L, h]     f32   log-decay per token and head, A*dt
 *   bmat, cmat    [b, L, g, N]  dtype; head i reads group i / (h / g)
 *   dt            [b, L, h]     f32   optional (NULL means dt == 1)
 *   a_cumsum      [b, h, c, Q]  f32   contiguous (workspace)
 *   chunk_decay   [b, h, c]     f32   contiguous (workspace)
 *   states        [b, c, h, P, N] state dtype, contiguous (workspace)
 *   initial/final [b, h, P, N]  f32   contiguous, optional
 */
#ifndef WORKLOADSUITE_AMD_SSD_H
#define WORKLOADSUITE_AMD_SSD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSD_ABI_VERSION 8

/* Element types.  The SPLIT and F16S values are storage formats of the
 * per-chunk states only, all laid out in the f32 states buffer
 * [b, c, h, P, N] (4 bytes per state):
 *   SPLIT: each f32 state as the 16-bit pair hi = round(v), lo = round(v - hi)
 *     of the inputs' type, stored per 8 consecutive states as [hi x8 | lo x8].
 *   F16S: each state row p (N states) as N f16 values v / 2^e in the first half
 *     of the row's f32 slots, and the scale 2^e (f32) in a separate array
 *     state_scales [b, c, h, P]; e is chosen per row so that the row's largest
 *     |v| lies in [2^14, 2^15] (f16's 11-bit significand; MR:155 itself stores
 *     the states in float16).
 *   F16S_LOCAL: the local states (K2's output) as f16 values in the first
 *     halves of the rows, as F16S, but with a scale 2^e per row p and
 *     16-column tile t (the tile row's largest |v| in [2^14, 2^15]) kept in
 *     the states buffer: the P x N/16 scales of an item [P][N], in (p, t)
 *     order k = p N/16 + t, packed into the second halves (unused by the f16
 *     values) of its first rows, scale k as the f32 in slot N/2 + k % (N/2)
 *     of row k / (N/2).
 * ssd_state_passing and ssd_chunk_state_passing write SPLIT and F16S from f32
 * (or F16S_LOCAL) local states; ssd_chunk_scan reads them, for 16-bit inputs
 * at chunk 256 and dstate 64 / 128 (F16S with dstate 128 for the one-launch
 * state chain), as MFMA operands without converting them, and reads F16S for
 * 16-bit inputs at chunk 64 / 128, dstate 64 / 128, chunk x dstate <= 8192,
 * without the epilogue.  ssd_chunk_state writes F16S_LOCAL for 16-bit inputs
 * at chunk 256 and dstate 64 / 128.  ssd_forward hands the states to
 * chunk_scan as F16S wherever that applies (state_dtype SSD_DTYPE_F32), or in
 * the format state_dtype names (at chunk 256; a SPLIT state_dtype at chunk
 * 64 / 128 hands over plain f32).
 * Where the forward runs chunk_state and state_passing as separate launches
 * with an F16S hand-over (16-bit inputs at chunk 256 outside the one-launch
 * state chain, and the chain's segments), the local states cross HBM as
 * F16S_LOCAL; the chain keeps them in f32 registers.  So the forward's last
 * bits depend on the launch plan, which depends on batch x heads and the
 * device's CU count: results are not bitwise invariant to batch slicing.
 * state_dtype SPLIT (at chunk 256) keeps every local state in f32. */
enum {
  SSD_DTYPE_F32 = 0,
  SSD_DTYPE_BF16 = 1,
  SSD_DTYPE_F16 = 2,
  SSD_STATE_SPLIT_BF16 = 3,
  SSD_STATE_SPLIT_F16 = 4,
  SSD_STATE_F16S = 5,
  SSD_STATE_F16S_LOCAL = 6,
};

/* Status codes (negative: rejected on the host before any launch). */
enum {
  SSD_OK = 0,
  SSD_ERR_NULL_POINTER = -1,
  SSD_ERR_BAD_SHAPE = -2,            /* a dimension is < 1                     */
  SSD_ERR_SEQLEN_NOT_DIVISIBLE = -3, /* L % Q != 0 (MR:106-110 would raise)    */
  SSD_ERR_HEADS_NOT_DIVISIBLE = -4,  /* h % g != 0 (MR:37-38 raises)           */
  SSD_ERR_UNSUPPORTED_DTYPE = -5,
  SSD_ERR_UNSUPPORTED_HEADDIM = -6,  /* P != 64                                */
  SSD_ERR_UNSUPPORTED_DSTATE = -7,   /* N not in {16, 32, 64, 128}             */
  SSD_ERR_UNSUPPORTED_CHUNK = -8,    /* Q not in {64, 128, 256}                */
  SSD_ERR_BAD_STRIDE = -9,           /* innermost stride != 1, or negative     */
  SSD_ERR_MISALIGNED = -10,          /* vector-loaded rows not 16-byte aligned */
  SSD_ERR_WORKSPACE_TOO_SMALL = -11,
  SSD_ERR_TOO_LARGE = -12,           /* a grid dimension would overflow        */
  SSD_ERR_UNSUPPORTED_CONV = -13,    /* conv kernel width not in 1..4          */
};

/* Problem dimensions. */
typedef struct ssd_dims {
  int64_t batch;   /* b */
  int64_t seqlen;  /* L, a multiple of chunk */
  int64_t nheads;  /* h, a multiple of ngroups */
  int64_t headdim; /* P */
  int64_t dstate;  /* N */
  int64_t ngroups; /* g */
  int64_t chunk;   /* Q (MR's block_len) */
} ssd_dims;

/* ABI version of the loaded library (SSD_ABI_VERSION). */
int ssd_abi_version(void);

/* Static, NUL-terminated description of a status code. */
const char* ssd_strerror(int status);

/* Host-only validation of dims + dtype; no device call.  Replaces the shape
 * errors MR raises (MR:37-38 ValueError, MR:106-110 einops error). */
int ssd_check_dims(const ssd_dims* d, int dtype);

/* Bytes of workspace ssd_forward needs: a_cumsum, chunk_decay, the
 * per-chunk states (state_dtype: SSD_DTYPE_F32 or SSD_DTYPE_BF16), for f32
 * states at the shapes where a 16-bit chunk_scan reads F16S (chunk 256, or
 * chunk 64 / 128 with chunk x dstate <= 8192; dstate 64 / 128) their row
 * scales [b, c, h, P] f32, and ssd_chunk_prep_bytes(d), each region 256-byte
 * aligned.  256 where ssd_forward runs the whole forward as one launch and
 * uses no workspace (f32 states, dstate 16 / 32, chunk 64 / 128 with chunk x
 * dstate <= 2048, at most 16 chunks).  0 when dims are invalid. */
size_t ssd_workspace_bytes(const ssd_dims* d, int state_dtype);

/* K1 -- intra-chunk cumsum of the log-decays and the per-chunk total decay.
 * Replaces MR:135-136 (torch.cumsum + rearrange) and MR:150 (exp of the last
 * cumsum).  a_strides: element strides of a over [b, L, h]. */
int ssd_chunk_cumsum(const ssd_dims* d, const float* a, const int64_t a_strides[3],
                     float* a_cumsum, float* chunk_decay, void* stream);

/* K0 -- per-(batch, chunk, group) operands of the chunk-256 kernels for
 * 16-bit inputs: C.B^T over each chunk (MR:143) in the register order
 * ssd_chunk_scan keeps it in, and B in the order ssd_chunk_state keeps it in.
 * Optional: K2 / K4 given prep = NULL rebuild them on every CU that meets a
 * group, which costs a chain of dependent loads per group.
 * ssd_chunk_prep_bytes is 0 for shapes without that path (chunk != 256 or
 * dstate not 64 / 128); ssd_chunk_prep then returns SSD_OK and writes
 * nothing, as it does for f32 inputs.  prep: device memory, 256-byte
 * aligned.  MR forms C.B^T inside its einsum (MR:143); there is no separate
 * reference interface for this stage. */
size_t ssd_chunk_prep_bytes(const ssd_dims* d);
int ssd_chunk_prep(const ssd_dims* d, int dtype,
                   const void* bmat, const int64_t b_strides[4],
                   const void* cmat, const int64_t c_strides[4],
                   void* prep, size_t prep_bytes, void* stream);

/* K2 -- per-chunk local states
 *   states[b,c,h,p,n] = sum_l x[l,p] dt[l] exp(Acs[Q-1]-Acs[l]) bmat[l,n].
 * Replaces MR:144 (X*dt) and MR:148-149 (decay_to_end and the 3-operand
 * einsum).  MR's [.., N, P] state is stored here as [.., P, N].
 * state_dtype: SSD_DTYPE_F32 / BF16, or SSD_STATE_F16S_LOCAL (16-bit inputs at
 * chunk 256, dstate 64 / 128; the f32 local states rounded to f16 rows with
 * their row scale, for ssd_state_passing with SSD_STATE_F16S_LOCAL).
 * prep: NULL, or ssd_chunk_prep's output for the same d, dtype and bmat. */
int ssd_chunk_state(const ssd_dims* d, int dtype,
                    const void* x, const int64_t x_strides[4],
                    const void* bmat, const int64_t b_strides[4],
                    const float* dt, const int64_t dt_strides[3],
                    const float* a_cumsum, void* states, int state_dtype,
                    const void* prep, void* stream);

/* K3 -- inter-chunk recurrence, in place: on entry states[c] holds chunk c's
 * local state, on exit the state entering chunk c:
 *   S_in[0] = initial (or 0), S_in[c+1] = chunk_decay[c] S_in[c] + S_local[c].
 * Replaces the Python loop at MR:152-157.  final_states (optional) receives
 * the state after the last chunk, which MR computes and discards (MR:156).
 * state_scales: [b, c, h, P] f32, written for SSD_STATE_F16S (NULL otherwise);
 * the same argument of ssd_chunk_state_passing and ssd_chunk_scan.
 * state_dtype names S_in's format; the local states are f32 for the SPLIT
 * formats and F16S, else of state_dtype.  SSD_STATE_F16S_LOCAL: the local
 * states in that format (ssd_chunk_state's), S_in written as SSD_STATE_F16S
 * with state_scales (dstate 64 / 128). */
int ssd_state_passing(const ssd_dims* d, void* states, int state_dtype, float* state_scales,
                      const float* chunk_decay, const float* initial_states,
                      float* final_states, void* stream);

/* K2 then K3 as ssd_forward runs them: on return states holds S_in (the
 * state entering each chunk, [b, c, h, P, N]) in state_dtype, exactly as
 * ssd_chunk_state (f32 local states for the SPLIT formats and F16S, else
 * state_dtype) followed by ssd_state_passing would leave it.  For a SPLIT
 * state_dtype of the inputs' type or F16S with prep (chunk 256), and for f32
 * states (or F16S with 16-bit inputs) at chunk 64 / 128 and dstate 64 / 128
 * (chunk x dstate <= 8192), the two stages run as one launch (at chunk 256,
 * wherever that is faster on the device): each (b, h) chain of chunks keeps
 * its running state in registers and the local states are never stored.
 * Where F16S's two stages run as separate launches (16-bit inputs at chunk
 * 256) they pass the local states as SSD_STATE_F16S_LOCAL, half the bytes of
 * f32: the result is then that of ssd_chunk_state with SSD_STATE_F16S_LOCAL
 * followed by ssd_state_passing with SSD_STATE_F16S_LOCAL, and differs from
 * the one-launch result by the local states' f16 rounding.
 * Replaces MR:144-157 (X*dt, decay_to_end, block_state, the state loop).
 * a_cumsum, chunk_decay: ssd_chunk_cumsum's outputs; prep as for
 * ssd_chunk_state; initial_states / final_states as for ssd_state_passing. */
int ssd_chunk_state_passing(const ssd_dims* d, int dtype,
                            const void* x, const int64_t x_strides[4],
                            const void* bmat, const int64_t b_strides[4],
                            const float* dt, const int64_t dt_strides[3],
                            const float* a_cumsum, const float* chunk_decay,
                            const void* prep, const float* initial_states,
                            void* states, int state_dtype, float* state_scales,
                            float* final_states, void* stream);

/* Skip and gate of SSDLayer.forward (MR:116-118), applied by ssd_chunk_scan
 * to y in float32 before its single rounding to the output dtype:
 *   y[l,p] = (y_ssd[l,p] + D[h] x[l,p]) * silu(z[l,p]),  silu(v) = v / (1 + e^-v)
 * D: [h] f32, or NULL (no skip term).  z: [b, L, h, P] of the input dtype
 * with element strides z_strides (unit stride over P), or NULL (no gate). */
typedef struct ssd_epilogue {
  const float* D;
  const void* z;
  int64_t z_strides[4];
} ssd_epilogue;

/* K4 -- fused chunk scan: writes y once,
 *   y[l,p] = sum_{s<=l} exp(Acs[l]-Acs[s]) (C_l.B_s) dt[s] x[s,p]
 *            + exp(Acs[l]) sum_n C[l,n] states[c][p,n].
 * Replaces MR:139-145 (segsum, mask, C.B^T, Y_diag), MR:160-161 (Y_off) and
 * MR:162 (the sum).
 * prep: NULL, or ssd_chunk_prep's output for the same d, dtype, bmat, cmat.
 * epilogue: NULL (y as above, MR's _ssd_core), or the layer's skip and gate
 * (MR:116-118) fused into the same write of y. */
int ssd_chunk_scan(const ssd_dims* d, int dtype,
                   const void* x, const int64_t x_strides[4],
                   const void* bmat, const int64_t b_strides[4],
                   const void* cmat, const int64_t c_strides[4],
                   const float* dt, const int64_t dt_strides[3],
                   const float* a_cumsum, const void* states, int state_dtype,
                   const float* state_scales,
                   void* y, const int64_t y_strides[4],
                   const void* prep, const ssd_epilogue* epilogue, void* stream);

/* Whole SSD forward (K1, K0, K2, K3, K4 on one stream): the replacement for
 * SSDLayer._ssd_core (MR:123-162).  Launches, all on `stream`: at chunk 256
 * with 16-bit inputs K1 + K0 as one launch, then K2 + K3 as one state-chain
 * launch (the chain's mixed plan adds K3 over the chains it leaves as
 * segments) or K2 then K3 where the chains are too few, then K4: three or
 * four.  At chunk 64 / 128 with f32 states, dstate 64 / 128 and chunk x
 * dstate <= 8192: K1, the f32-state chain, K4.  With f32 states, dstate
 * 16 / 32, chunk x dstate <= 2048 and at most 16 chunks: the whole forward in
 * one launch.  Otherwise one launch per stage.  workspace must hold
 * ssd_workspace_bytes(d, state_dtype) bytes, 256-byte aligned (or that of
 * the chunk ssd_forward_chunk reports).  d->chunk is MR's block_len and only
 * has to divide L: for 16-bit inputs with f32 states (SSD_DTYPE_F32 or
 * SSD_STATE_F16S), L % 256 == 0 and dstate 64 / 128, a chunk of 64 or 128
 * runs at 256 unless that workspace would be larger than the caller's
 * chunk's (see ssd_forward_chunk).  Every chunking evaluates the same linear
 * recurrence (MR:152-161), so this changes rounding only. */
/* The chunk length ssd_forward (and ssd_forward_noalloc) runs d at for this
 * dtype and state_dtype: d->chunk, or 256 where the rule above applies; 0
 * for invalid dims.  Host-only.  No counterpart in the reference (its
 * block_len is the chunk); for callers that size the workspace at the chunk
 * actually run or time its kernels one by one. */
int64_t ssd_forward_chunk(const ssd_dims* d, int dtype, int state_dtype);

int ssd_forward(const ssd_dims* d, int dtype,
                const void* x, const int64_t x_strides[4],
                const float* a, const int64_t a_strides[3],
                const void* bmat, const int64_t b_strides[4],
                const void* cmat, const int64_t c_strides[4],
                const float* dt, const int64_t dt_strides[3],
                const float* initial_states,
                void* y, const int64_t y_strides[4],
                float* final_states,
                void* workspace, size_t workspace_bytes, int state_dtype,
                void* stream);

/* Decode: one token of the recurrence (the per-token form of MR:152-161),
 * in place on a [b, h, P, N] f32 state such as ssd_forward's final_states:
 *   state[b,h,p,n] = exp(a[b,h]) state[b,h,p,n] + dt[b,h] x[b,h,p] bmat[b,g,n]
 *   y[b,h,p]       = sum_n cmat[b,g,n] state[b,h,p,n]
 * with head h reading group h / (nheads / ngroups), then the optional
 * epilogue (skip D x, gate silu(z)).  MR has no single-token path; this is the
 * consumer of the final state it computes (MR:156).  d->seqlen and d->chunk
 * are not used.  x, y: [b, h, P] of dtype, element strides {batch, head}
 * (unit stride over P).  bmat, cmat: [b, g, N] of dtype, strides {batch,
 * group} (unit over N).  a, dt: [b, h] f32 with strides ad_strides {batch,
 * head}; dt NULL means 1.  state: contiguous, 16-byte aligned.  The
 * epilogue's z is [b, h, P] with z_strides[0] (batch) and z_strides[2]
 * (head); z_strides[1] is not used. */
int ssd_decode_step(const ssd_dims* d, int dtype, float* state,
                    const void* x, const int64_t x_strides[2],
                    const void* bmat, const int64_t b_strides[2],
                    const void* cmat, const int64_t c_strides[2],
                    const float* a, const float* dt, const int64_t ad_strides[2],
                    void* y, const int64_t y_strides[2],
                    const ssd_epilogue* epilogue, void* stream);

/* ---- the layer around the SSD core (SSDLayer.forward, MR:68-121) ---- */

/* Parameters of one layer, as MR's module holds them (MR:41-66).  Device
 * pointers; conv_w, conv_b and dt_bias are of the layer's dtype (MR: f16). */
typedef struct ssd_layer_params {
  int64_t conv_kernel;  /* k, 1..4 (MR default 4) */
  const void* conv_w;   /* conv1d.weight [h*P, 1, k], contiguous */
  const void* conv_b;   /* conv1d.bias [h*P], or NULL */
  const void* dt_bias;  /* [h] */
  const float* A_log;   /* [h] f32; A = -exp(A_log) (MR:102) */
  const float* D;       /* [h] f32 skip weight, or NULL (no skip term) */
} ssd_layer_params;

/* Pre-SSD prep (MR:83-103) in two launches:
 *   x_out[b,l,h,p] = silu(conv_b[d] + sum_j conv_w[d,j] x_in[b, l-(k-1)+j, d]),
 *                    d = h P + p, x_in = 0 before l = 0 (causal conv1d, MR:83-86)
 *   dt_out[b,l,h]  = softplus(dt_in[b,l,h] + dt_bias[h])          (MR:94)
 *   a_cumsum, chunk_decay as ssd_chunk_cumsum of A_dt = -exp(A_log[h]) dt  (MR:102-103)
 * x_in [b, L, h*P] and dt_in [b, L, h] are of dtype (MR: strided slices of
 * in_proj's output) with element strides x_strides / dt_strides (unit stride
 * over the last dim); x_out [b, L, h, P] dtype and dt_out [b, L, h] f32 are
 * contiguous.  softplus is log(1 + e^v), and v itself above 20 (torch's
 * threshold).  Accumulates and activates in float32, rounds x once. */
int ssd_layer_prep(const ssd_dims* d, int dtype, const ssd_layer_params* prm,
                   const void* x_in, const int64_t x_strides[3],
                   const void* dt_in, const int64_t dt_strides[3],
                   void* x_out, float* dt_out, float* a_cumsum, float* chunk_decay,
                   void* stream);

/* Workspace of ssd_layer_forward: x_out, dt_out, then ssd_workspace_bytes
 * (f32 states) at the chunk the core runs at, each 256-byte aligned; 0 when
 * dims are invalid. */
size_t ssd_layer_workspace_bytes(const ssd_dims* d, int dtype);

/* SSDLayer.forward between its two projections (MR:76-118): from in_proj's
 * output slices x_in [b, L, h*P], z [b, L, h*P], bmat/cmat [b, L, g, N] and
 * dt_in [b, L, h] (all of dtype, any strides with unit innermost stride) to
 * out_proj's input y [b, L, h*P]:
 *   ssd_layer_prep, then the SSD core (K0, K2, K3, K4 of ssd_forward), with
 *   the skip D x and the gate silu(z) fused into K4's write of y.
 * z_strides / y_strides are over [b, L, h*P].  d->chunk is MR's block_len
 * and only has to divide L: for 16-bit inputs with L % 256 == 0 and dstate
 * 64 / 128 the core runs at chunk 256, whose result equals every other
 * chunking's up to rounding (the chunked SSD evaluates one linear recurrence,
 * MR:152-161) and whose per-chunk states take a quarter of the memory. */
int ssd_layer_forward(const ssd_dims* d, int dtype, const ssd_layer_params* prm,
                      const void* x_in, const int64_t x_strides[3],
                      const void* z, const int64_t z_strides[3],
                      const void* bmat, const int64_t b_strides[4],
                      const void* cmat, const int64_t c_strides[4],
                      const void* dt_in, const int64_t dt_strides[3],
                      void* y, const int64_t y_strides[3],
                      void* workspace, size_t workspace_bytes, void* stream);

/* ssd_forward without a workspace argument: the workspace is a static
 * __device__ array of SSD_NOALLOC_SCRATCH_BYTES in libssd's code object, so
 * the call itself allocates nothing.  The array is reserved on every device
 * where the code object loads (any libssd kernel launch loads it), until the
 * process ends, whether or not ssd_forward_noalloc is ever called.  Its
 * device address is looked up once per device (hipGetSymbolAddress) and
 * cached on the host; after a hipDeviceReset that cache is stale.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as ssd_forward otherwise,
 * at the chunk ssd_forward_chunk reports; the caller still provides every
 * input and output.  When the workspace of the whole call is larger than the
 * array, the batch runs in slices whose workspace fits; a shape whose single
 * batch element needs more returns SSD_ERR_WORKSPACE_TOO_SMALL before any
 * launch.  All calls on one device share that device's array: calls that
 * overlap on one device (other streams, other threads) race, so the caller
 * serialises them. */
#define SSD_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int ssd_forward_noalloc(const ssd_dims* d, int dtype,
                        const void* x, const int64_t x_strides[4],
                        const float* a, const int64_t a_strides[3],
                        const void* bmat, const int64_t b_strides[4],
                        const void* cmat, const int64_t c_strides[4],
                        const float* dt, const int64_t dt_strides[3],
                        const float* initial_states,
                        void* y, const int64_t y_strides[4],
                        float* final_states, int state_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WORKLOADSUITE_AMD_SSD_H */
