// C ABI of libssd (declared in include/ssd.h): host-side validation and
// dispatch to the four kernels.  Nothing here allocates or synchronises, and
// nothing is kept between calls but a per-device cache of the CU count; every
// kernel goes to the caller's stream.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstdint>

#include "../../include/ssd.h"
#include "ssd_launch.h"

namespace {

using ssd::ChunkPrepArgs;
using ssd::ChunkScanArgs;
using ssd::ChunkStateArgs;
using ssd::ConvArgs;
using ssd::CumsumArgs;
using ssd::StatePassingArgs;

constexpr size_t kWsAlign = 256;

size_t elem_size(int dtype) { return dtype == SSD_DTYPE_F32 ? 4 : 2; }

bool valid_dtype(int dtype) {
  return dtype == SSD_DTYPE_F32 || dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16;
}

// f32 inputs keep f32 states; 16-bit inputs may use f32 or bf16 states.
bool valid_state_dtype(int dtype, int state_dtype) {
  if (state_dtype == SSD_DTYPE_F32) return true;
  return state_dtype == SSD_DTYPE_BF16 && dtype != SSD_DTYPE_F32;
}

// The 16-bit type of a SPLIT state storage, 0 for the others.
int split_of(int state_dtype) {
  if (state_dtype == SSD_STATE_SPLIT_BF16) return SSD_DTYPE_BF16;
  if (state_dtype == SSD_STATE_SPLIT_F16) return SSD_DTYPE_F16;
  return 0;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A handover format of f32 states (SPLIT or F16S): stored in the f32 layout.
bool f32_layout(int state_dtype) { return split_of(state_dtype) != 0 || state_dtype == SSD_STATE_F16S; }

int check_dims_impl(const ssd_dims* d, int dtype) {
  if (!d) return SSD_ERR_NULL_POINTER;
  if (d->batch < 1 || d->seqlen < 1 || d->nheads < 1 || d->headdim < 1 || d->dstate < 1 ||
      d->ngroups < 1 || d->chunk < 1)
    return SSD_ERR_BAD_SHAPE;
  if (d->seqlen % d->chunk != 0) return SSD_ERR_SEQLEN_NOT_DIVISIBLE;
  if (d->nheads % d->ngroups != 0) return SSD_ERR_HEADS_NOT_DIVISIBLE;
  if (!valid_dtype(dtype)) return SSD_ERR_UNSUPPORTED_DTYPE;
  if (d->headdim != 64) return SSD_ERR_UNSUPPORTED_HEADDIM;
  if (d->dstate != 16 && d->dstate != 32 && d->dstate != 64 && d->dstate != 128)
    return SSD_ERR_UNSUPPORTED_DSTATE;
  if (d->chunk != 64 && d->chunk != 128 && d->chunk != 256) return SSD_ERR_UNSUPPORTED_CHUNK;
  const int64_t nchunks = d->seqlen / d->chunk;
  // Kernels index workgroups and (batch, chunk, head) triples in 32-bit ints.
  if (d->batch > INT_MAX / nchunks || d->batch * nchunks > INT_MAX / d->nheads) return SSD_ERR_TOO_LARGE;
  return SSD_OK;
}

// A strided [.., inner] operand read with 16-byte vector loads.
int check_vec_operand(const void* p, const int64_t* strides, int n, int dtype) {
  if (!p || !strides) return SSD_ERR_NULL_POINTER;
  if (strides[n - 1] != 1) return SSD_ERR_BAD_STRIDE;
  for (int k = 0; k < n - 1; ++k)
    if (strides[k] < 0) return SSD_ERR_BAD_STRIDE;
  if (!aligned16(p)) return SSD_ERR_MISALIGNED;
  const int64_t es = (int64_t)elem_size(dtype);
  for (int k = 0; k < n - 1; ++k)
    if ((strides[k] * es) % 16 != 0) return SSD_ERR_MISALIGNED;
  return SSD_OK;
}

// A strided f32 operand read with scalar loads ([b, L, h]).
int check_scalar_operand(const void* p, const int64_t* strides, int n) {
  if (!p || !strides) return SSD_ERR_NULL_POINTER;
  for (int k = 0; k < n; ++k)
    if (strides[k] < 0) return SSD_ERR_BAD_STRIDE;
  if ((reinterpret_cast<uintptr_t>(p) & 3u) != 0) return SSD_ERR_MISALIGNED;
  return SSD_OK;
}

// The output y [b, L, h, P] is written 4 elements at a time: unit inner
// stride, non-negative strides, 4-element aligned base and row strides.
int check_output(const void* y, const int64_t* strides, int dtype) {
  if (!y || !strides) return SSD_ERR_NULL_POINTER;
  if (strides[3] != 1) return SSD_ERR_BAD_STRIDE;
  const int64_t es = (int64_t)elem_size(dtype), align = 4 * es;
  for (int k = 0; k < 3; ++k) {
    if (strides[k] < 0) return SSD_ERR_BAD_STRIDE;
    if ((strides[k] * es) % align != 0) return SSD_ERR_MISALIGNED;
  }
  if ((int64_t)(reinterpret_cast<uintptr_t>(y) % (uintptr_t)align) != 0) return SSD_ERR_MISALIGNED;
  return SSD_OK;
}

int hip_status(hipError_t e) { return e == hipSuccess ? SSD_OK : (int)e; }

size_t round_up(size_t v) { return (v + kWsAlign - 1) / kWsAlign * kWsAlign; }

struct WsLayout {
  size_t acs, decay, states, scales, prep, total;
};

// chunk_prep's outputs only exist for the persistent kernels' shapes
bool prep_shape(const ssd_dims* d) { return d->chunk == 256 && (d->dstate == 64 || d->dstate == 128); }
// The chunk-64 / 128 shapes whose 16-bit chunk_scan reads f16s states
bool f16s_small_shape(const ssd_dims* d) {
  return (d->chunk == 64 || d->chunk == 128) && (d->dstate == 64 || d->dstate == 128) && d->chunk * d->dstate <= 8192;
}

// prep buffer: the CB^T fragments, then (256-byte aligned) the B^T fragments
size_t prep_cb_region(const ssd_dims* d) {
  const int64_t groups = d->batch * (d->seqlen / d->chunk) * d->ngroups;
  return round_up(ssd::chunk_prep_cb_bytes(groups));
}
size_t prep_bytes(const ssd_dims* d) {
  if (!prep_shape(d)) return 0;
  const int64_t groups = d->batch * (d->seqlen / d->chunk) * d->ngroups;
  return prep_cb_region(d) + round_up(ssd::chunk_prep_bt_bytes(groups, (int)d->dstate));
}

WsLayout ws_layout(const ssd_dims* d, int state_dtype) {
  const size_t nchunks = (size_t)(d->seqlen / d->chunk);
  const size_t bhc = (size_t)d->batch * d->nheads * nchunks;
  WsLayout w;
  w.acs = 0;
  w.decay = round_up(bhc * (size_t)d->chunk * sizeof(float));
  w.states = w.decay + round_up(bhc * sizeof(float));
  w.scales = w.states + round_up(bhc * (size_t)d->headdim * d->dstate * elem_size(state_dtype));
  // the row scales of f16s-handed-over states (only with f32 states, at the
  // shapes where a 16-bit chunk_scan reads them)
  const size_t scales =
      state_dtype == SSD_DTYPE_F32 && (prep_shape(d) || f16s_small_shape(d)) ? bhc * (size_t)d->headdim * sizeof(float) : 0;
  w.prep = w.scales + round_up(scales);
  w.total = w.prep + prep_bytes(d);
  return w;
}

ChunkPrepArgs make_prep_args(const ssd_dims* d, const void* bmat, const int64_t b_strides[4], const void* cmat,
                             const int64_t c_strides[4], void* prep) {
  ChunkPrepArgs pa;
  pa.bm = bmat;
  pa.sbb = b_strides[0];
  pa.sbl = b_strides[1];
  pa.sbg = b_strides[2];
  pa.cm = cmat;
  pa.scb = c_strides[0];
  pa.scl = c_strides[1];
  pa.scg = c_strides[2];
  pa.batch = (int)d->batch;
  pa.nchunks = (int)(d->seqlen / d->chunk);
  pa.ngroups = (int)d->ngroups;
  pa.dstate = (int)d->dstate;
  pa.chunk = (int)d->chunk;
  pa.cbf = reinterpret_cast<float*>(prep);
  pa.btf = static_cast<char*>(prep) + prep_cb_region(d);
  return pa;
}

StatePassingArgs make_sp_args(const ssd_dims* d, void* states, const float* chunk_decay,
                              const float* initial_states, float* final_states) {
  StatePassingArgs p;
  p.states = states;
  p.decay = chunk_decay;
  p.init = initial_states;
  p.final_state = final_states;
  p.batch = (int)d->batch;
  p.nchunks = (int)(d->seqlen / d->chunk);
  p.nheads = (int)d->nheads;
  p.headdim = (int)d->headdim;
  p.dstate = (int)d->dstate;
  return p;
}

// The CB^T / B^T fragments inside a prep buffer (null when there is none).
const float* prep_cbf(const void* prep) { return static_cast<const float*>(prep); }
const void* prep_btf(const ssd_dims* d, const void* prep) {
  return prep ? static_cast<const char*>(prep) + prep_cb_region(d) : nullptr;
}

// A 16-bit input with a prepared shape: ssd_chunk_prep has work to do.
bool prep_applies(const ssd_dims* d, int dtype) {
  return prep_shape(d) && (dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16);
}

ChunkStateArgs make_state_args(const ssd_dims* d, const void* x, const int64_t x_strides[4], const void* bmat,
                               const int64_t b_strides[4], const float* dt, const int64_t dt_strides[3],
                               const float* a_cumsum, void* states) {
  ChunkStateArgs p;
  p.x = x;
  p.sxb = x_strides[0];
  p.sxl = x_strides[1];
  p.sxh = x_strides[2];
  p.bm = bmat;
  p.sbb = b_strides[0];
  p.sbl = b_strides[1];
  p.sbg = b_strides[2];
  p.dt = dt;
  p.sdb = dt ? dt_strides[0] : 0;
  p.sdl = dt ? dt_strides[1] : 0;
  p.sdh = dt ? dt_strides[2] : 0;
  p.acs = a_cumsum;
  p.states = states;
  p.batch = (int)d->batch;
  p.nchunks = (int)(d->seqlen / d->chunk);
  p.nheads = (int)d->nheads;
  p.ngroups = (int)d->ngroups;
  p.dstate = (int)d->dstate;
  p.chunk = (int)d->chunk;
  return p;
}

ChunkScanArgs make_scan_args(const ssd_dims* d, const void* x, const int64_t x_strides[4], const void* bmat,
                             const int64_t b_strides[4], const void* cmat, const int64_t c_strides[4],
                             const float* dt, const int64_t dt_strides[3], const float* a_cumsum,
                             const void* states, void* y, const int64_t y_strides[4]) {
  ChunkScanArgs p;
  p.x = x;
  p.sxb = x_strides[0];
  p.sxl = x_strides[1];
  p.sxh = x_strides[2];
  p.bm = bmat;
  p.sbb = b_strides[0];
  p.sbl = b_strides[1];
  p.sbg = b_strides[2];
  p.cm = cmat;
  p.scb = c_strides[0];
  p.scl = c_strides[1];
  p.scg = c_strides[2];
  p.dt = dt;
  p.sdb = dt ? dt_strides[0] : 0;
  p.sdl = dt ? dt_strides[1] : 0;
  p.sdh = dt ? dt_strides[2] : 0;
  p.acs = a_cumsum;
  p.states = states;
  p.y = y;
  p.syb = y_strides[0];
  p.syl = y_strides[1];
  p.syh = y_strides[2];
  p.batch = (int)d->batch;
  p.nchunks = (int)(d->seqlen / d->chunk);
  p.nheads = (int)d->nheads;
  p.ngroups = (int)d->ngroups;
  p.dstate = (int)d->dstate;
  p.chunk = (int)d->chunk;
  return p;
}

// The epilogue's operands: D any f32 array, z a [b, L, h, P] operand of the
// input dtype with unit inner stride (read per element, or 16 bytes at a
// time where aligned).
int check_epilogue(const ssd_epilogue* e, int dtype) {
  if (!e) return SSD_OK;
  if (e->D && (reinterpret_cast<uintptr_t>(e->D) & 3u) != 0) return SSD_ERR_MISALIGNED;
  if (e->z) {
    if (e->z_strides[3] != 1) return SSD_ERR_BAD_STRIDE;
    for (int k = 0; k < 3; ++k)
      if (e->z_strides[k] < 0) return SSD_ERR_BAD_STRIDE;
    if ((reinterpret_cast<uintptr_t>(e->z) % elem_size(dtype)) != 0) return SSD_ERR_MISALIGNED;
  }
  return SSD_OK;
}

void set_epilogue(ChunkScanArgs& p, const ssd_epilogue* e) {
  if (!e) return;
  p.dskip = e->D;
  p.z = e->z;
  if (e->z) {
    p.szb = e->z_strides[0];
    p.szl = e->z_strides[1];
    p.szh = e->z_strides[2];
  }
}

CumsumArgs make_cumsum_args(const ssd_dims* d, const float* a, const int64_t a_strides[3], float* acs,
                            float* decay) {
  CumsumArgs p;
  p.a = a;
  p.sab = a_strides[0];
  p.sal = a_strides[1];
  p.sah = a_strides[2];
  p.acs = acs;
  p.decay = decay;
  p.batch = (int)d->batch;
  p.nchunks = (int)(d->seqlen / d->chunk);
  p.nheads = (int)d->nheads;
  p.chunk = (int)d->chunk;
  return p;
}

// K1 (when k1 is given; together with K0 in one launch where K0 applies), K0,
// K2, K3, K4 of one forward.  Without k1, K1's outputs are already in the
// workspace.  Operands are validated by the caller.
// K2 then K3 (local states in the f32 / bf16 state_dtype, or as f16 rows
// where K3 writes F16S from the chunk-256 K2's output; pa.split_dtype set:
// S_in written as hi/lo pairs), as one chain launch where that is faster.
int run_state_passing(const ssd_dims* d, int dtype, const ChunkStateArgs& sa, const StatePassingArgs& pa,
                      int state_dtype, hipStream_t s) {
  int rc;
  // f32: K2 and K3 as one launch wherever it applies (forward 12% faster at
  // C2's 192 chains of 32 chunks, 7% at C5's 4096 chains of 4)
  if (state_dtype == SSD_DTYPE_F32 && ssd::chunk_state_chain_f32_supported(sa, dtype, pa))
    return hip_status(ssd::launch_chunk_state_chain_f32(sa, pa, dtype, s));
  ssd::ChainPlan plan = (pa.split_dtype || pa.f16s) ? ssd::chunk_state_chain_plan(sa, dtype) : ssd::ChainPlan{0, 1, 1};
  if (pa.f16s && sa.dstate != 128) plan = ssd::ChainPlan{0, 1, 1};  // the chain's f16s store needs d_state 128
  if (plan.nfull > 0) {
    // K2 and K3 as one launch: the local states stay in registers (same bits);
    // chains beyond nfull leave local states that K3 finishes
    if ((rc = hip_status(ssd::launch_chunk_state_chain(sa, pa, plan, dtype, s)))) return rc;
    const int64_t chains = d->batch * d->nheads;
    if (plan.nfull < chains) {
      StatePassingArgs rest = pa;
      rest.bh_begin = plan.nfull;
      rest.bh_count = (int)(chains - plan.nfull);
      // (the segments leave f16 local states where S_in goes out as f16s)
      if ((rc = hip_status(ssd::launch_state_passing(rest, pa.f16s ? SSD_STATE_F16S_LOCAL : state_dtype, s)))) return rc;
    }
    return SSD_OK;
  }
  if (pa.f16s && ssd::chunk_state_persistent_supported(sa, dtype)) {
    // S_in goes to chunk_scan as f16 rows: the local states cross HBM as f16
    // rows too (SSD_STATE_F16S_LOCAL, half the bytes of f32 in K2's writes
    // and K3's reads)
    if ((rc = hip_status(ssd::launch_chunk_state(sa, dtype, SSD_STATE_F16S_LOCAL, s)))) return rc;
    return hip_status(ssd::launch_state_passing(pa, SSD_STATE_F16S_LOCAL, s));
  }
  if ((rc = hip_status(ssd::launch_chunk_state(sa, dtype, state_dtype, s)))) return rc;
  return hip_status(ssd::launch_state_passing(pa, state_dtype, s));
}

// The format in which the forward hands f32 states from K3 to K4: 0 (plain
// f32 or bf16 states), SSD_STATE_F16S or a SPLIT value.  The chunk-256
// persistent chunk_scan reads both handover formats; the 16-bit chunk_scan at
// chunk 64 / 128 reads F16S (a SPLIT request there hands over plain f32).
int handover_format(const ssd_dims* d, int dtype, int state_dtype, const ChunkScanArgs& ca, const float* scales) {
  if (!f32_layout(state_dtype) && state_dtype != SSD_DTYPE_F32) return 0;
  const bool f16s = state_dtype == SSD_DTYPE_F32 || state_dtype == SSD_STATE_F16S;
  if (prep_applies(d, dtype) && ssd::chunk_scan_persistent_supported(ca, dtype)) return f16s ? SSD_STATE_F16S : state_dtype;
  if (f16s && f16s_small_shape(d)) {
    ChunkScanArgs fa = ca;
    fa.f16s = true;
    fa.sscale = scales;
    if (ssd::chunk_scan_b16_supported(fa, dtype, SSD_DTYPE_F32)) return SSD_STATE_F16S;
  }
  return 0;
}

int run_core(const ssd_dims* d, int dtype, const CumsumArgs* k1, const void* x, const int64_t x_strides[4],
             const void* bmat, const int64_t b_strides[4], const void* cmat, const int64_t c_strides[4],
             const float* dt, const int64_t dt_strides[3], const float* initial_states, void* y,
             const int64_t y_strides[4], float* final_states, char* ws, const WsLayout& w, int state_dtype,
             const ssd_epilogue* epi, hipStream_t s) {
  int rc;
  float* acs = reinterpret_cast<float*>(ws + w.acs);
  float* decay = reinterpret_cast<float*>(ws + w.decay);
  void* states = ws + w.states;
  ChunkStateArgs sa = make_state_args(d, x, x_strides, bmat, b_strides, dt, dt_strides, acs, states);
  ChunkScanArgs ca = make_scan_args(d, x, x_strides, bmat, b_strides, cmat, c_strides, dt, dt_strides, acs, states,
                                    y, y_strides);
  set_epilogue(ca, epi);
  // K0: the persistent kernels' per-group operands, once per (b, c, group)
  if (prep_applies(d, dtype)) {
    void* prep = ws + w.prep;
    ChunkPrepArgs pa = make_prep_args(d, bmat, b_strides, cmat, c_strides, prep);
    // the epilogue variant of K4 keeps CB^T in the input type: K0 writes it so
    ca.cbf = prep_cbf(prep);
    pa.cb16 = epi && ssd::chunk_scan_persistent_supported(ca, dtype);
    ca.cb16 = pa.cb16;
    if ((rc = hip_status(k1 ? ssd::launch_chunk_prologue(pa, *k1, dtype, s) : ssd::launch_chunk_prep(pa, dtype, s))))
      return rc;
    sa.btf = prep_btf(d, prep);
    ca.cbf = prep_cbf(prep);
  } else if (k1) {
    if ((rc = hip_status(ssd::launch_chunk_cumsum(*k1, s)))) return rc;
  }
  // f32 states for a 16-bit chunk_scan that reads the handover formats: K3
  // (or the state chain) hands them over as f16 with per-row scales (the
  // default), or at chunk 256 as its hi/lo operand pairs when state_dtype
  // asks for that format
  StatePassingArgs pa = make_sp_args(d, states, decay, initial_states, final_states);
  float* scales = reinterpret_cast<float*>(ws + w.scales);
  const int handover = handover_format(d, dtype, state_dtype, ca, scales);
  if (handover == SSD_STATE_F16S) {
    pa.f16s = 1;
    ca.f16s = true;
    pa.sscale = scales;
    ca.sscale = pa.sscale;
  } else if (handover) {
    pa.split_dtype = dtype;
    ca.presplit = true;
  }
  const int sd = f32_layout(state_dtype) ? SSD_DTYPE_F32 : state_dtype;
  if ((rc = run_state_passing(d, dtype, sa, pa, sd, s))) return rc;
  return hip_status(ssd::launch_chunk_scan(ca, dtype, sd, s));
}

// ---- the layer around the core ----

// The chunk length the layer's core runs at.  The chunked SSD's output does
// not depend on the chunk length (every chunking evaluates the same linear
// recurrence, MR:152-161); MR's block_len only has to divide L.  With 16-bit
// inputs chunk 256 runs the persistent kernels and stores a quarter of the
// per-chunk states of chunk 64 (at MR's shape those states are most of the
// core's HBM traffic), so the layer uses it whenever L and dstate allow.
ssd_dims layer_core_dims(const ssd_dims* d, int dtype) {
  ssd_dims e = *d;
  if ((dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16) && d->seqlen % 256 == 0 &&
      (d->dstate == 64 || d->dstate == 128))
    e.chunk = 256;
  return e;
}

// The chunk length ssd_forward runs at (dims already validated).  As for the
// layer, MR's block_len only has to divide L.  16-bit inputs with f32 states
// (handed to chunk_scan as f16 rows), L % 256 == 0 and dstate 64 / 128 run a
// chunk of 64 or 128 at 256: the persistent kernels, with a quarter of the
// per-chunk states.  Not when that workspace would be the larger one (many
// groups: chunk_prep's per-group operands then outgrow the states saved), so
// a workspace sized by ssd_workspace_bytes for the caller's chunk always
// suffices.  The SPLIT / bf16 state formats keep the caller's chunk.
ssd_dims forward_dims(const ssd_dims* d, int dtype, int state_dtype) {
  ssd_dims e = *d;
  const bool b16 = dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16;
  const bool f32_states = state_dtype == SSD_DTYPE_F32 || state_dtype == SSD_STATE_F16S;
  if (b16 && f32_states && (d->chunk == 64 || d->chunk == 128) && d->seqlen % 256 == 0 &&
      (d->dstate == 64 || d->dstate == 128)) {
    ssd_dims c = *d;
    c.chunk = 256;
    if (ws_layout(&c, SSD_DTYPE_F32).total <= ws_layout(d, SSD_DTYPE_F32).total) e = c;
  }
  return e;
}

// ssd_forward's one-launch path for small states and short chains (f32
// states; the shapes ssd_small_supported takes)
bool small_forward(const ssd_dims* d, int state_dtype) {
  return state_dtype == SSD_DTYPE_F32 &&
         ssd::ssd_small_supported(d->batch, d->nheads, d->headdim, d->dstate, d->chunk, d->seqlen / d->chunk);
}

struct LayerWs {
  size_t xo, dto, core, total;
  WsLayout cw;
};

LayerWs layer_ws(const ssd_dims* d, int dtype) {
  LayerWs w;
  const size_t tokens = (size_t)d->batch * d->seqlen;
  w.xo = 0;
  w.dto = round_up(tokens * d->nheads * d->headdim * elem_size(dtype));
  w.core = w.dto + round_up(tokens * d->nheads * sizeof(float));
  const ssd_dims e = layer_core_dims(d, dtype);
  w.cw = ws_layout(&e, SSD_DTYPE_F32);
  w.total = w.core + w.cw.total;
  return w;
}

int check_layer_params(const ssd_layer_params* prm) {
  if (!prm) return SSD_ERR_NULL_POINTER;
  if (prm->conv_kernel < 1 || prm->conv_kernel > 4) return SSD_ERR_UNSUPPORTED_CONV;
  if (!prm->conv_w || !prm->dt_bias || !prm->A_log) return SSD_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(prm->A_log) & 3u) != 0 ||
      (prm->D && (reinterpret_cast<uintptr_t>(prm->D) & 3u) != 0))
    return SSD_ERR_MISALIGNED;
  return SSD_OK;
}

// A [b, L, inner] operand read per element (or per vector where aligned).
int check_rows3(const void* p, const int64_t* strides, int dtype) {
  if (!p || !strides) return SSD_ERR_NULL_POINTER;
  if (strides[2] != 1) return SSD_ERR_BAD_STRIDE;
  if (strides[0] < 0 || strides[1] < 0) return SSD_ERR_BAD_STRIDE;
  if ((reinterpret_cast<uintptr_t>(p) % elem_size(dtype)) != 0) return SSD_ERR_MISALIGNED;
  return SSD_OK;
}

// Grid limits of the conv and cumsum launches.
int check_layer_grid(const ssd_dims* d) {
  const int64_t runs = (d->seqlen + 31) / 32;
  if (d->batch > 65535 || (runs + 3) / 4 > 65535) return SSD_ERR_TOO_LARGE;
  return SSD_OK;
}

// K1's layer variant: dt = softplus(dt_raw + dt_bias), A_dt = -exp(A_log) dt, then the cumsum.
CumsumArgs make_raw_cumsum_args(const ssd_dims* d, int dtype, const ssd_layer_params* prm, const void* dt_in,
                                const int64_t dt_strides[3], float* dt_out, float* acs, float* decay) {
  CumsumArgs ca;
  ca.a = nullptr;
  ca.sab = ca.sal = ca.sah = 0;
  ca.acs = acs;
  ca.decay = decay;
  ca.batch = (int)d->batch;
  ca.nchunks = (int)(d->seqlen / d->chunk);
  ca.nheads = (int)d->nheads;
  ca.chunk = (int)d->chunk;
  ca.dt_raw = dt_in;
  ca.srb = dt_strides[0];
  ca.srl = dt_strides[1];
  ca.srh = dt_strides[2];
  ca.dt_bias = prm->dt_bias;
  ca.a_log = prm->A_log;
  ca.dt_out = dt_out;
  ca.raw_dtype = dtype;
  return ca;
}

int launch_conv(const ssd_dims* d, int dtype, const ssd_layer_params* prm, const void* x_in,
                const int64_t x_strides[3], void* x_out, hipStream_t s) {
  ConvArgs cv;
  cv.x = x_in;
  cv.sxb = x_strides[0];
  cv.sxl = x_strides[1];
  cv.w = prm->conv_w;
  cv.bias = prm->conv_b;
  cv.y = x_out;
  cv.batch = (int)d->batch;
  cv.seqlen = (int)d->seqlen;
  cv.channels = (int)(d->nheads * d->headdim);
  cv.kwidth = (int)prm->conv_kernel;
  return hip_status(ssd::launch_conv_silu(cv, dtype, s));
}

int launch_layer_prep(const ssd_dims* d, int dtype, const ssd_layer_params* prm, const void* x_in,
                      const int64_t x_strides[3], const void* dt_in, const int64_t dt_strides[3], void* x_out,
                      float* dt_out, float* acs, float* decay, hipStream_t s) {
  int rc;
  if ((rc = launch_conv(d, dtype, prm, x_in, x_strides, x_out, s))) return rc;
  return hip_status(
      ssd::launch_chunk_cumsum(make_raw_cumsum_args(d, dtype, prm, dt_in, dt_strides, dt_out, acs, decay), s));
}

}  // namespace

namespace ssd {

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < kMaxDevices) {
    const int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < kMaxDevices) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace ssd

extern "C" {

int ssd_abi_version(void) { return SSD_ABI_VERSION; }

const char* ssd_strerror(int status) {
  switch (status) {
    case SSD_OK: return "success";
    case SSD_ERR_NULL_POINTER: return "null pointer argument";
    case SSD_ERR_BAD_SHAPE: return "every dimension must be >= 1";
    case SSD_ERR_SEQLEN_NOT_DIVISIBLE: return "seqlen must be a multiple of the chunk size";
    case SSD_ERR_HEADS_NOT_DIVISIBLE: return "n_heads must be divisible by n_groups";
    case SSD_ERR_UNSUPPORTED_DTYPE:
      return "unsupported dtype or state format (f32, bf16, f16; bf16 states and the SPLIT / F16S formats need "
             "16-bit inputs, and the formats chunk 256 with dstate 64 or 128)";
    case SSD_ERR_UNSUPPORTED_HEADDIM: return "unsupported head_dim (must be 64)";
    case SSD_ERR_UNSUPPORTED_DSTATE: return "unsupported d_state (16, 32, 64 or 128)";
    case SSD_ERR_UNSUPPORTED_CHUNK: return "unsupported chunk size (64, 128 or 256)";
    case SSD_ERR_BAD_STRIDE: return "innermost stride must be 1 and strides non-negative";
    case SSD_ERR_MISALIGNED: return "vector-loaded operands need 16-byte aligned rows and buffers";
    case SSD_ERR_WORKSPACE_TOO_SMALL: return "workspace too small (see ssd_workspace_bytes)";
    case SSD_ERR_TOO_LARGE: return "problem too large for 32-bit workgroup indexing";
    case SSD_ERR_UNSUPPORTED_CONV: return "unsupported conv kernel width (1 to 4)";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown ssd status";
}

int ssd_check_dims(const ssd_dims* d, int dtype) { return check_dims_impl(d, dtype); }

size_t ssd_workspace_bytes(const ssd_dims* d, int state_dtype) {
  if (check_dims_impl(d, SSD_DTYPE_BF16) != SSD_OK) return 0;
  // the one-launch forward of small states uses no workspace
  if (small_forward(d, state_dtype)) return kWsAlign;
  if (f32_layout(state_dtype)) state_dtype = SSD_DTYPE_F32;
  if (state_dtype != SSD_DTYPE_F32 && state_dtype != SSD_DTYPE_BF16) return 0;
  return ws_layout(d, state_dtype).total;
}

int64_t ssd_forward_chunk(const ssd_dims* d, int dtype, int state_dtype) {
  if (check_dims_impl(d, dtype) != SSD_OK) return 0;
  return forward_dims(d, dtype, state_dtype).chunk;
}

int ssd_chunk_cumsum(const ssd_dims* d, const float* a, const int64_t a_strides[3],
                     float* a_cumsum, float* chunk_decay, void* stream) {
  int rc = check_dims_impl(d, SSD_DTYPE_F32);
  if (rc) return rc;
  if ((rc = check_scalar_operand(a, a_strides, 3))) return rc;
  if (!a_cumsum || !chunk_decay) return SSD_ERR_NULL_POINTER;
  return hip_status(ssd::launch_chunk_cumsum(make_cumsum_args(d, a, a_strides, a_cumsum, chunk_decay),
                                            (hipStream_t)stream));
}

size_t ssd_chunk_prep_bytes(const ssd_dims* d) {
  if (check_dims_impl(d, SSD_DTYPE_BF16) != SSD_OK) return 0;
  return prep_bytes(d);
}

int ssd_chunk_prep(const ssd_dims* d, int dtype, const void* bmat, const int64_t b_strides[4], const void* cmat,
                   const int64_t c_strides[4], void* prep, size_t prep_bytes_given, void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  if ((rc = check_vec_operand(bmat, b_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(cmat, c_strides, 4, dtype))) return rc;
  if (!prep_applies(d, dtype)) return SSD_OK;
  if (!prep) return SSD_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(prep) % kWsAlign) != 0) return SSD_ERR_MISALIGNED;
  if (prep_bytes_given < prep_bytes(d)) return SSD_ERR_WORKSPACE_TOO_SMALL;
  return hip_status(ssd::launch_chunk_prep(make_prep_args(d, bmat, b_strides, cmat, c_strides, prep), dtype,
                                           (hipStream_t)stream));
}

int ssd_chunk_state(const ssd_dims* d, int dtype, const void* x, const int64_t x_strides[4],
                    const void* bmat, const int64_t b_strides[4], const float* dt,
                    const int64_t dt_strides[3], const float* a_cumsum, void* states,
                    int state_dtype, const void* prep, void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  const bool f16l = state_dtype == SSD_STATE_F16S_LOCAL;
  if (!valid_state_dtype(dtype, state_dtype) && !f16l) return SSD_ERR_UNSUPPORTED_DTYPE;
  if ((rc = check_vec_operand(x, x_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(bmat, b_strides, 4, dtype))) return rc;
  if (dt && (rc = check_scalar_operand(dt, dt_strides, 3))) return rc;
  if (!a_cumsum || !states) return SSD_ERR_NULL_POINTER;
  // the kernels copy a_cumsum to LDS 16 bytes at a time
  if (!aligned16(states) || !aligned16(a_cumsum)) return SSD_ERR_MISALIGNED;
  if (prep && (reinterpret_cast<uintptr_t>(prep) % kWsAlign) != 0) return SSD_ERR_MISALIGNED;
  ChunkStateArgs p = make_state_args(d, x, x_strides, bmat, b_strides, dt, dt_strides, a_cumsum, states);
  // f16 local states: the chunk-256 kernel for 16-bit inputs only
  if (f16l && !ssd::chunk_state_persistent_supported(p, dtype)) return SSD_ERR_UNSUPPORTED_DTYPE;
  if (prep_applies(d, dtype)) p.btf = prep_btf(d, prep);
  return hip_status(ssd::launch_chunk_state(p, dtype, state_dtype, (hipStream_t)stream));
}

int ssd_state_passing(const ssd_dims* d, void* states, int state_dtype, float* state_scales,
                      const float* chunk_decay, const float* initial_states, float* final_states, void* stream) {
  int rc = check_dims_impl(d, SSD_DTYPE_BF16);
  if (rc) return rc;
  const int split = split_of(state_dtype);
  const bool f16l = state_dtype == SSD_STATE_F16S_LOCAL;  // F16S_LOCAL in, F16S out
  const bool f16s = state_dtype == SSD_STATE_F16S || f16l;
  if (state_dtype != SSD_DTYPE_F32 && state_dtype != SSD_DTYPE_BF16 && !split && !f16s)
    return SSD_ERR_UNSUPPORTED_DTYPE;
  if (f16s && d->dstate != 64 && d->dstate != 128) return SSD_ERR_UNSUPPORTED_DSTATE;
  if (!states || !chunk_decay || (f16s && !state_scales)) return SSD_ERR_NULL_POINTER;
  if (f16s && (reinterpret_cast<uintptr_t>(state_scales) & 3u)) return SSD_ERR_MISALIGNED;
  if (!aligned16(states) || (initial_states && !aligned16(initial_states)) ||
      (final_states && !aligned16(final_states)))
    return SSD_ERR_MISALIGNED;
  StatePassingArgs p = make_sp_args(d, states, chunk_decay, initial_states, final_states);
  p.split_dtype = split;
  p.f16s = f16s ? 1 : 0;
  p.sscale = f16s ? state_scales : nullptr;
  return hip_status(ssd::launch_state_passing(p, f16l ? SSD_STATE_F16S_LOCAL : f32_layout(state_dtype) ? SSD_DTYPE_F32 : state_dtype,
                                              (hipStream_t)stream));
}

int ssd_chunk_state_passing(const ssd_dims* d, int dtype, const void* x, const int64_t x_strides[4],
                            const void* bmat, const int64_t b_strides[4], const float* dt,
                            const int64_t dt_strides[3], const float* a_cumsum, const float* chunk_decay,
                            const void* prep, const float* initial_states, void* states, int state_dtype,
                            float* state_scales, float* final_states, void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  const int split = split_of(state_dtype);
  const bool f16s = state_dtype == SSD_STATE_F16S;
  if (f16s ? (dtype == SSD_DTYPE_F32 || (d->dstate != 64 && d->dstate != 128))
           : split ? split != dtype : !valid_state_dtype(dtype, state_dtype))
    return SSD_ERR_UNSUPPORTED_DTYPE;
  if ((rc = check_vec_operand(x, x_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(bmat, b_strides, 4, dtype))) return rc;
  if (dt && (rc = check_scalar_operand(dt, dt_strides, 3))) return rc;
  if (!a_cumsum || !chunk_decay || !states || (f16s && !state_scales)) return SSD_ERR_NULL_POINTER;
  if (!aligned16(states) || !aligned16(a_cumsum) || (initial_states && !aligned16(initial_states)) ||
      (final_states && !aligned16(final_states)) || (f16s && (reinterpret_cast<uintptr_t>(state_scales) & 3u)))
    return SSD_ERR_MISALIGNED;
  if (prep && (reinterpret_cast<uintptr_t>(prep) % kWsAlign) != 0) return SSD_ERR_MISALIGNED;
  ChunkStateArgs sa = make_state_args(d, x, x_strides, bmat, b_strides, dt, dt_strides, a_cumsum, states);
  if (prep_applies(d, dtype)) sa.btf = prep_btf(d, prep);
  StatePassingArgs pa = make_sp_args(d, states, chunk_decay, initial_states, final_states);
  pa.split_dtype = split;
  pa.f16s = f16s ? 1 : 0;
  pa.sscale = f16s ? state_scales : nullptr;
  return run_state_passing(d, dtype, sa, pa, f32_layout(state_dtype) ? SSD_DTYPE_F32 : state_dtype,
                           (hipStream_t)stream);
}

int ssd_chunk_scan(const ssd_dims* d, int dtype, const void* x, const int64_t x_strides[4],
                   const void* bmat, const int64_t b_strides[4], const void* cmat,
                   const int64_t c_strides[4], const float* dt, const int64_t dt_strides[3],
                   const float* a_cumsum, const void* states, int state_dtype, const float* state_scales,
                   void* y, const int64_t y_strides[4], const void* prep, const ssd_epilogue* epilogue,
                   void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  const int split = split_of(state_dtype);
  const bool f16s = state_dtype == SSD_STATE_F16S;
  if (!valid_state_dtype(dtype, state_dtype) && !(split && split == dtype) && !(f16s && dtype != SSD_DTYPE_F32))
    return SSD_ERR_UNSUPPORTED_DTYPE;
  if ((rc = check_vec_operand(x, x_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(bmat, b_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(cmat, c_strides, 4, dtype))) return rc;
  if (dt && (rc = check_scalar_operand(dt, dt_strides, 3))) return rc;
  if (!a_cumsum || !states || (f16s && !state_scales)) return SSD_ERR_NULL_POINTER;
  // a_cumsum and the states are copied to LDS 16 bytes at a time
  if (!aligned16(a_cumsum) || !aligned16(states)) return SSD_ERR_MISALIGNED;
  if (f16s && (reinterpret_cast<uintptr_t>(state_scales) & 3u)) return SSD_ERR_MISALIGNED;
  if ((rc = check_output(y, y_strides, dtype))) return rc;
  if ((rc = check_epilogue(epilogue, dtype))) return rc;
  if (prep && (reinterpret_cast<uintptr_t>(prep) % kWsAlign) != 0) return SSD_ERR_MISALIGNED;
  ChunkScanArgs p = make_scan_args(d, x, x_strides, bmat, b_strides, cmat, c_strides, dt, dt_strides, a_cumsum,
                                   states, y, y_strides);
  set_epilogue(p, epilogue);
  if (prep_applies(d, dtype)) p.cbf = prep_cbf(prep);
  if (split || f16s) {
    // the chunk-256 kernel reads both handover formats, the 16-bit kernel at
    // chunk 64 / 128 reads f16s
    p.presplit = split != 0;
    p.f16s = f16s;
    p.sscale = f16s ? state_scales : nullptr;
    if (!(prep_applies(d, dtype) && ssd::chunk_scan_persistent_supported(p, dtype)) &&
        !ssd::chunk_scan_b16_supported(p, dtype, SSD_DTYPE_F32))
      return SSD_ERR_UNSUPPORTED_DTYPE;
  }
  return hip_status(ssd::launch_chunk_scan(p, dtype, f32_layout(state_dtype) ? SSD_DTYPE_F32 : state_dtype,
                                           (hipStream_t)stream));
}

int ssd_forward(const ssd_dims* d, int dtype, const void* x, const int64_t x_strides[4], const float* a,
                const int64_t a_strides[3], const void* bmat, const int64_t b_strides[4],
                const void* cmat, const int64_t c_strides[4], const float* dt,
                const int64_t dt_strides[3], const float* initial_states, void* y,
                const int64_t y_strides[4], float* final_states, void* workspace,
                size_t workspace_bytes, int state_dtype, void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  const int split = split_of(state_dtype);
  if (!valid_state_dtype(dtype, state_dtype) && !(split && split == dtype) &&
      !(state_dtype == SSD_STATE_F16S && dtype != SSD_DTYPE_F32))
    return SSD_ERR_UNSUPPORTED_DTYPE;
  if (!workspace) return SSD_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(workspace) % kWsAlign) != 0) return SSD_ERR_MISALIGNED;
  // the chunk the forward runs at (never a larger workspace than d's own)
  const ssd_dims e = forward_dims(d, dtype, state_dtype);
  d = &e;
  const bool small = small_forward(d, state_dtype);
  const WsLayout w = ws_layout(d, f32_layout(state_dtype) ? SSD_DTYPE_F32 : state_dtype);
  if (workspace_bytes < (small ? kWsAlign : w.total)) return SSD_ERR_WORKSPACE_TOO_SMALL;
  // Validate every operand before the first launch, so a bad argument never
  // leaves a partially computed result behind.
  if ((rc = check_scalar_operand(a, a_strides, 3))) return rc;
  if ((rc = check_vec_operand(x, x_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(bmat, b_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(cmat, c_strides, 4, dtype))) return rc;
  if (dt && (rc = check_scalar_operand(dt, dt_strides, 3))) return rc;
  if ((rc = check_output(y, y_strides, dtype))) return rc;
  if ((initial_states && !aligned16(initial_states)) || (final_states && !aligned16(final_states)))
    return SSD_ERR_MISALIGNED;

  // small states and short chains: the whole forward in one launch, the
  // states kept in f32 (the workspace is not used)
  if (small) {
    ssd::SmallArgs sm;
    sm.x = x;
    sm.sxb = x_strides[0];
    sm.sxl = x_strides[1];
    sm.sxh = x_strides[2];
    sm.a = a;
    sm.sab = a_strides[0];
    sm.sal = a_strides[1];
    sm.sah = a_strides[2];
    sm.bm = bmat;
    sm.sbb = b_strides[0];
    sm.sbl = b_strides[1];
    sm.sbg = b_strides[2];
    sm.cm = cmat;
    sm.scb = c_strides[0];
    sm.scl = c_strides[1];
    sm.scg = c_strides[2];
    sm.dt = dt;
    sm.sdb = dt ? dt_strides[0] : 0;
    sm.sdl = dt ? dt_strides[1] : 0;
    sm.sdh = dt ? dt_strides[2] : 0;
    sm.init = initial_states;
    sm.final_state = final_states;
    sm.y = y;
    sm.syb = y_strides[0];
    sm.syl = y_strides[1];
    sm.syh = y_strides[2];
    sm.batch = (int)d->batch;
    sm.nchunks = (int)(d->seqlen / d->chunk);
    sm.nheads = (int)d->nheads;
    sm.ngroups = (int)d->ngroups;
    sm.dstate = (int)d->dstate;
    sm.chunk = (int)d->chunk;
    return hip_status(ssd::launch_ssd_small(sm, dtype, (hipStream_t)stream));
  }

  char* ws = static_cast<char*>(workspace);
  const CumsumArgs k1 = make_cumsum_args(d, a, a_strides, reinterpret_cast<float*>(ws + w.acs),
                                         reinterpret_cast<float*>(ws + w.decay));
  return run_core(d, dtype, &k1, x, x_strides, bmat, b_strides, cmat, c_strides, dt, dt_strides, initial_states, y,
                  y_strides, final_states, ws, w, state_dtype, nullptr, (hipStream_t)stream);
}

int ssd_decode_step(const ssd_dims* d, int dtype, float* state, const void* x, const int64_t x_strides[2],
                    const void* bmat, const int64_t b_strides[2], const void* cmat, const int64_t c_strides[2],
                    const float* a, const float* dt, const int64_t ad_strides[2], void* y,
                    const int64_t y_strides[2], const ssd_epilogue* epilogue, void* stream) {
  if (!d) return SSD_ERR_NULL_POINTER;
  ssd_dims one = *d;  // the sequence dimensions do not apply to one token
  one.seqlen = one.chunk = 64;
  int rc = check_dims_impl(&one, dtype);
  if (rc) return rc;
  if (d->batch * d->nheads > INT_MAX) return SSD_ERR_TOO_LARGE;
  if (!state || !x || !x_strides || !bmat || !b_strides || !cmat || !c_strides || !a || !ad_strides || !y ||
      !y_strides)
    return SSD_ERR_NULL_POINTER;
  for (const int64_t* st : {x_strides, b_strides, c_strides, ad_strides, y_strides})
    if (st[0] < 0 || st[1] < 0) return SSD_ERR_BAD_STRIDE;
  if (!aligned16(state)) return SSD_ERR_MISALIGNED;
  const uintptr_t es = elem_size(dtype);
  for (const void* q : {x, bmat, cmat, static_cast<const void*>(y)})
    if (reinterpret_cast<uintptr_t>(q) % es != 0) return SSD_ERR_MISALIGNED;
  if ((reinterpret_cast<uintptr_t>(a) & 3u) != 0 || (dt && (reinterpret_cast<uintptr_t>(dt) & 3u) != 0))
    return SSD_ERR_MISALIGNED;
  if (epilogue) {
    if (epilogue->D && (reinterpret_cast<uintptr_t>(epilogue->D) & 3u) != 0) return SSD_ERR_MISALIGNED;
    if (epilogue->z) {
      if (epilogue->z_strides[0] < 0 || epilogue->z_strides[2] < 0 || epilogue->z_strides[3] != 1)
        return SSD_ERR_BAD_STRIDE;
      if (reinterpret_cast<uintptr_t>(epilogue->z) % es != 0) return SSD_ERR_MISALIGNED;
    }
  }
  ssd::DecodeArgs p;
  p.state = state;
  p.x = x;
  p.sxb = x_strides[0];
  p.sxh = x_strides[1];
  p.bm = bmat;
  p.sbb = b_strides[0];
  p.sbg = b_strides[1];
  p.cm = cmat;
  p.scb = c_strides[0];
  p.scg = c_strides[1];
  p.a = a;
  p.dt = dt;
  p.sab = ad_strides[0];
  p.sah = ad_strides[1];
  p.y = y;
  p.syb = y_strides[0];
  p.syh = y_strides[1];
  if (epilogue) {
    p.dskip = epilogue->D;
    p.z = epilogue->z;
    p.szb = epilogue->z_strides[0];
    p.szh = epilogue->z_strides[2];
  }
  p.batch = (int)d->batch;
  p.nheads = (int)d->nheads;
  p.ngroups = (int)d->ngroups;
  p.dstate = (int)d->dstate;
  return hip_status(ssd::launch_decode_step(p, dtype, (hipStream_t)stream));
}

int ssd_layer_prep(const ssd_dims* d, int dtype, const ssd_layer_params* prm, const void* x_in,
                   const int64_t x_strides[3], const void* dt_in, const int64_t dt_strides[3], void* x_out,
                   float* dt_out, float* a_cumsum, float* chunk_decay, void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  if ((rc = check_layer_params(prm))) return rc;
  if ((rc = check_layer_grid(d))) return rc;
  if ((rc = check_rows3(x_in, x_strides, dtype))) return rc;
  if (!dt_in || !dt_strides) return SSD_ERR_NULL_POINTER;
  for (int k = 0; k < 3; ++k)
    if (dt_strides[k] < 0) return SSD_ERR_BAD_STRIDE;
  if ((reinterpret_cast<uintptr_t>(dt_in) % elem_size(dtype)) != 0) return SSD_ERR_MISALIGNED;
  if (!x_out || !dt_out || !a_cumsum || !chunk_decay) return SSD_ERR_NULL_POINTER;
  if (!aligned16(x_out) || (reinterpret_cast<uintptr_t>(dt_out) & 3u) != 0) return SSD_ERR_MISALIGNED;
  return launch_layer_prep(d, dtype, prm, x_in, x_strides, dt_in, dt_strides, x_out, dt_out, a_cumsum,
                           chunk_decay, (hipStream_t)stream);
}

size_t ssd_layer_workspace_bytes(const ssd_dims* d, int dtype) {
  if (check_dims_impl(d, dtype) != SSD_OK) return 0;
  return layer_ws(d, dtype).total;
}

int ssd_layer_forward(const ssd_dims* d, int dtype, const ssd_layer_params* prm, const void* x_in,
                      const int64_t x_strides[3], const void* z, const int64_t z_strides[3], const void* bmat,
                      const int64_t b_strides[4], const void* cmat, const int64_t c_strides[4], const void* dt_in,
                      const int64_t dt_strides[3], void* y, const int64_t y_strides[3], void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc = check_dims_impl(d, dtype);
  if (rc) return rc;
  if ((rc = check_layer_params(prm))) return rc;
  if ((rc = check_layer_grid(d))) return rc;
  if (!workspace) return SSD_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(workspace) % kWsAlign) != 0) return SSD_ERR_MISALIGNED;
  const LayerWs w = layer_ws(d, dtype);
  if (workspace_bytes < w.total) return SSD_ERR_WORKSPACE_TOO_SMALL;
  // every operand is checked before the first launch
  if ((rc = check_rows3(x_in, x_strides, dtype))) return rc;
  if ((rc = check_rows3(z, z_strides, dtype))) return rc;
  if (!dt_in || !dt_strides) return SSD_ERR_NULL_POINTER;
  for (int k = 0; k < 3; ++k)
    if (dt_strides[k] < 0) return SSD_ERR_BAD_STRIDE;
  if ((reinterpret_cast<uintptr_t>(dt_in) % elem_size(dtype)) != 0) return SSD_ERR_MISALIGNED;
  if ((rc = check_vec_operand(bmat, b_strides, 4, dtype))) return rc;
  if ((rc = check_vec_operand(cmat, c_strides, 4, dtype))) return rc;
  if (!y || !y_strides) return SSD_ERR_NULL_POINTER;
  const int64_t P = d->headdim;
  const int64_t ys4[4] = {y_strides[0], y_strides[1], y_strides[2] * P, y_strides[2]};
  if ((rc = check_output(y, ys4, dtype))) return rc;

  char* ws = static_cast<char*>(workspace);
  void* x_out = ws + w.xo;
  float* dt_out = reinterpret_cast<float*>(ws + w.dto);
  char* core = ws + w.core;
  const hipStream_t s = (hipStream_t)stream;
  const ssd_dims e = layer_core_dims(d, dtype);
  d = &e;
  // conv, then K1's layer variant inside the core's first launch (with K0 where it applies)
  if ((rc = launch_conv(d, dtype, prm, x_in, x_strides, x_out, s))) return rc;
  const CumsumArgs k1 = make_raw_cumsum_args(d, dtype, prm, dt_in, dt_strides, dt_out,
                                             reinterpret_cast<float*>(core + w.cw.acs),
                                             reinterpret_cast<float*>(core + w.cw.decay));
  const int64_t h = d->nheads, L = d->seqlen;
  const int64_t xs4[4] = {L * h * P, h * P, P, 1};
  const int64_t dts[3] = {L * h, h, 1};
  ssd_epilogue epi;
  epi.D = prm->D;
  epi.z = z;
  epi.z_strides[0] = z_strides[0];
  epi.z_strides[1] = z_strides[1];
  epi.z_strides[2] = P * z_strides[2];
  epi.z_strides[3] = z_strides[2];
  return run_core(d, dtype, &k1, x_out, xs4, bmat, b_strides, cmat, c_strides, dt_out, dts, nullptr, y, ys4,
                  nullptr, core, w.cw, SSD_DTYPE_F32, &epi, s);
}

}  // extern "C"
