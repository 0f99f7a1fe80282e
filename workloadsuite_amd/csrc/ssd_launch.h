// Internal launcher interface between the C ABI (ssd_api.cpp) and the kernel
// translation units.  Arguments are already validated; launchers only pick a
// template instantiation, size the grid and launch on `stream`.  They return
// the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssd {

struct CumsumArgs {
  const float* a;
  int64_t sab, sal, sah;  // element strides of a [b, L, h]
  float* acs;             // [b, h, c, Q]
  float* decay;           // [b, h, c]
  int batch, nchunks, nheads, chunk;
  // Optional (the layer's prep): a = -exp(a_log[h]) softplus(dt_raw + dt_bias[h])
  // is formed here, and that dt written to dt_out ([b, L, h] f32, contiguous);
  // `a` is then unused.  dt_raw and dt_bias are of raw_dtype.
  const void* dt_raw = nullptr;
  int64_t srb = 0, srl = 0, srh = 0;
  const void* dt_bias = nullptr;
  const float* a_log = nullptr;
  float* dt_out = nullptr;
  int raw_dtype = 0;
};

// Causal depthwise conv1d of width kwidth over the sequence, plus bias, then
// SiLU (ssd_layer_prep.hip): y [b, L, channels] contiguous from x [b, L,
// channels] (unit channel stride); w [channels, kwidth], bias [channels] or null.
struct ConvArgs {
  const void* x;
  int64_t sxb, sxl;
  const void* w;
  const void* bias;
  void* y;
  int batch, seqlen, channels, kwidth;
};
hipError_t launch_conv_silu(const ConvArgs& a, int dtype, hipStream_t stream);

struct ChunkStateArgs {
  const void* x;
  int64_t sxb, sxl, sxh;  // x [b, L, h, P], unit stride over P
  const void* bm;
  int64_t sbb, sbl, sbg;  // bmat [b, L, g, N], unit stride over N
  const float* dt;        // optional [b, L, h]
  int64_t sdb, sdl, sdh;
  const float* acs;       // [b, h, c, Q]
  void* states;           // [b, c, h, P, N]
  int batch, nchunks, nheads, ngroups, dstate, chunk;
  const void* btf = nullptr;  // optional chunk_prep B^T fragments (persistent kernel)
};

struct StatePassingArgs {
  void* states;           // [b, c, h, P, N], in place
  const float* decay;     // [b, h, c]
  const float* init;      // optional [b, h, P, N]
  float* final_state;     // optional [b, h, P, N]
  int batch, nchunks, nheads, headdim, dstate;
  // 0, or SSD_DTYPE_BF16 / F16: f32 S_in is written as chunk_scan's hi/lo
  // operand pairs of that type (chunk-256 forward path only)
  int split_dtype = 0;
  // S_in written as f16 with a power-of-two scale per state row
  // (SSD_STATE_F16S, in place in the f32 layout; chunk-256 forward path only)
  int f16s = 0;
  float* sscale = nullptr;  // f16s: the row scales [b, c, h, P]
  // chains (b * nheads + h) [bh_begin, bh_begin + bh_count) only; bh_count 0: all
  int bh_begin = 0, bh_count = 0;
};

struct ChunkScanArgs {
  const void* x;
  int64_t sxb, sxl, sxh;
  const void* bm;
  int64_t sbb, sbl, sbg;
  const void* cm;
  int64_t scb, scl, scg;
  const float* dt;
  int64_t sdb, sdl, sdh;
  const float* acs;       // [b, h, c, Q]
  const void* states;     // [b, c, h, P, N] (state entering each chunk)
  void* y;
  int64_t syb, syl, syh;  // y [b, L, h, P], unit stride over P
  int batch, nchunks, nheads, ngroups, dstate, chunk;
  const float* cbf = nullptr;  // optional chunk_prep CB^T fragments (persistent kernel)
  bool cb16 = false;           // ... rounded to the input type (the epilogue variant reads those)
  bool presplit = false;       // f32 states already split by state_passing (split_dtype)
  bool f16s = false;           // states in the SSD_STATE_F16S format (state_passing's f16s output)
  const float* sscale = nullptr;  // ... and their row scales [b, c, h, P]
  // optional epilogue: y = (y + dskip[h] x) * silu(z)
  const float* dskip = nullptr;  // [h]
  const void* z = nullptr;       // [b, L, h, P], unit stride over P
  int64_t szb = 0, szl = 0, szh = 0;
};

// Decode: one token of the recurrence on a [b, h, P, N] f32 state (ssd_decode.hip).
struct DecodeArgs {
  float* state;           // [b, h, P, N] contiguous, in place
  const void* x;          // [b, h, P]
  int64_t sxb, sxh;
  const void* bm;         // [b, g, N]
  int64_t sbb, sbg;
  const void* cm;
  int64_t scb, scg;
  const float* a;         // [b, h] log-decay A dt
  const float* dt;        // [b, h] or null (1); same strides as a
  int64_t sab, sah;
  void* y;                // [b, h, P]
  int64_t syb, syh;
  const float* dskip = nullptr;  // [h] or null
  const void* z = nullptr;       // [b, h, P] or null
  int64_t szb = 0, szh = 0;
  int batch, nheads, ngroups, dstate;
};
hipError_t launch_decode_step(const DecodeArgs& a, int dtype, hipStream_t stream);

// K0 -- per-(b, c, group) operands of the chunk-256 persistent kernels
// (ssd_chunk_prep.hip): CB^T blocks for chunk_scan, B^T fragments for chunk_state.
struct ChunkPrepArgs {
  const void* bm;
  int64_t sbb, sbl, sbg;
  const void* cm;
  int64_t scb, scl, scg;
  int batch, nchunks, ngroups, dstate, chunk;
  float* cbf;  // chunk_prep_cb_bytes(batch * nchunks * ngroups)
  void* btf;   // chunk_prep_bt_bytes(batch * nchunks * ngroups, dstate)
  // CB^T rounded to the input type (half of chunk_prep_cb_bytes), for chunk_scan's epilogue variant
  bool cb16 = false;
};
size_t chunk_prep_cb_bytes(int64_t groups);
size_t chunk_prep_bt_bytes(int64_t groups, int dstate);
hipError_t launch_chunk_prep(const ChunkPrepArgs& a, int dtype, hipStream_t stream);
// K0 and K1 (chunk 256; from A, or the layer variant from raw dt) in one
// launch: bit-identical to launching launch_chunk_prep and
// launch_chunk_cumsum one after the other.
hipError_t launch_chunk_prologue(const ChunkPrepArgs& a, const CumsumArgs& ca, int dtype, hipStream_t stream);

// Compute units of the current device (cached per device id after the first
// query; 0 when the query fails).
int device_cu_count();

// Workgroups for a persistent kernel that loops over `items` work items:
// every workgroup slot the kernel's occupancy allows on the device's CUs,
// capped by the item count.  `kernel` is the __global__ function.
template <typename K>
int persistent_grid(K kernel, int threads, int items) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel), threads, 0) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int cus = device_cu_count();
  const long slots = (long)(cus > 0 ? cus : 256) * per_cu;
  return (int)(slots < items ? slots : items);
}

// dtype / state_dtype use the SSD_DTYPE_* values of include/ssd.h.
hipError_t launch_chunk_cumsum(const CumsumArgs& a, hipStream_t stream);
hipError_t launch_chunk_state(const ChunkStateArgs& a, int dtype, int state_dtype, hipStream_t stream);
hipError_t launch_state_passing(const StatePassingArgs& a, int state_dtype, hipStream_t stream);
hipError_t launch_chunk_scan(const ChunkScanArgs& a, int dtype, int state_dtype, hipStream_t stream);

// chunk_state's persistent kernel for 16-bit inputs at chunk 256
// (ssd_chunk_state_q256.hip); launch_chunk_state dispatches to it when supported.
bool chunk_state_persistent_supported(const ChunkStateArgs& a, int dtype);
hipError_t launch_chunk_state_persistent(const ChunkStateArgs& a, int dtype, int state_dtype, hipStream_t stream);

// K2 and K3 of the chunk-256 forward in one launch (ssd_chunk_state_q256.hip):
// one workgroup per (b, h) chain walks the chunks in order with the running
// state in registers and writes S_in as chunk_scan's hi/lo pairs (sp.split_dtype ==
// dtype); the per-chunk local states never reach memory.  Needs chunk_prep's
// B^T fragments (a.btf).  Bit-identical to launch_chunk_state with f32 states
// followed by launch_state_passing.
bool chunk_state_chain_supported(const ChunkStateArgs& a, int dtype);
// Chains [0, nfull) run whole; each later chain runs as seg_per_chain
// workgroups of seg_len chunks that write f32 local states, and
// launch_state_passing over chains [nfull, b*h) (bh_begin / bh_count) then
// finishes them.  nfull == 0: the launch is not worth it on this device for
// this shape; run launch_chunk_state then launch_state_passing instead.
struct ChainPlan {
  int nfull, seg_per_chain, seg_len;
};
ChainPlan chunk_state_chain_plan(const ChunkStateArgs& a, int dtype);
hipError_t launch_chunk_state_chain(const ChunkStateArgs& a, const StatePassingArgs& sp, const ChainPlan& plan,
                                    int dtype, hipStream_t stream);

// chunk_scan's persistent kernel for 16-bit inputs at chunk 256
// (ssd_chunk_scan_q256.hip); launch_chunk_scan dispatches to it when supported.
bool chunk_scan_persistent_supported(const ChunkScanArgs& a, int dtype);
hipError_t launch_chunk_scan_persistent(const ChunkScanArgs& a, int dtype, int state_dtype, hipStream_t stream);

// chunk_scan for f32 inputs and states at chunk 64 / 128, d_state 64 / 128,
// without the layer epilogue (ssd_chunk_scan_f32.hip): C.B^T once per
// (b, c, group); launch_chunk_scan dispatches to it when supported.
bool chunk_scan_f32_supported(const ChunkScanArgs& a, int dtype, int state_dtype);
// chunk_state for f32 states at chunk 64 / 128, d_state 64 / 128, f32 or
// 16-bit inputs (ssd_chunk_state_f32.hip: f32 MFMAs, or 16-bit MFMAs with the
// weighted x as hi/lo pairs): B once per (b, c, group); launch_chunk_state
// dispatches to it when supported.
bool chunk_state_f32_supported(const ChunkStateArgs& a, int dtype, int state_dtype);
hipError_t launch_chunk_state_f32(const ChunkStateArgs& a, int dtype, hipStream_t stream);
// ... and K2 + K3 as one launch for f32 states (one workgroup per (b, h)
// chain, S_in written in place of the local states in the f32 layout, or for
// 16-bit inputs as f16s with sp.sscale): bit-identical to
// launch_chunk_state_f32 followed by launch_state_passing.
bool chunk_state_chain_f32_supported(const ChunkStateArgs& a, int dtype, const StatePassingArgs& sp);
hipError_t launch_chunk_state_chain_f32(const ChunkStateArgs& a, const StatePassingArgs& sp, int dtype, hipStream_t stream);
hipError_t launch_chunk_scan_f32(const ChunkScanArgs& a, hipStream_t stream);
// chunk_scan for 16-bit inputs with f32 states (plain, or f16s with
// a.sscale) at chunk 64 / 128, d_state 64 / 128, without the layer epilogue
// (ssd_chunk_scan_b16.hip): the f32 kernel's decomposition on 16-bit MFMAs;
// launch_chunk_scan dispatches to it when supported.
bool chunk_scan_b16_supported(const ChunkScanArgs& a, int dtype, int state_dtype);
hipError_t launch_chunk_scan_b16(const ChunkScanArgs& a, int dtype, hipStream_t stream);

// The whole forward in one launch for small states and short chains
// (ssd_small.hip): d_state 16 / 32, chunk 64 / 128, at most kSmallMaxChunks
// chunks per chain, f32 states kept in LDS; one workgroup per (b, h) chain.
constexpr int64_t kSmallMaxChunks = 16;
struct SmallArgs {
  const void* x;
  int64_t sxb, sxl, sxh;  // x [b, L, h, P], unit stride over P
  const float* a;
  int64_t sab, sal, sah;  // A (log-decay A dt) [b, L, h]
  const void* bm;
  int64_t sbb, sbl, sbg;  // bmat [b, L, g, N]
  const void* cm;
  int64_t scb, scl, scg;  // cmat [b, L, g, N]
  const float* dt;        // optional [b, L, h]
  int64_t sdb, sdl, sdh;
  const float* init;      // optional [b, h, P, N]
  float* final_state;     // optional [b, h, P, N]
  void* y;
  int64_t syb, syl, syh;  // y [b, L, h, P], unit stride over P
  int batch, nchunks, nheads, ngroups, dstate, chunk;
};
bool ssd_small_supported(int64_t batch, int64_t nheads, int64_t headdim, int64_t dstate, int64_t chunk, int64_t nchunks);
hipError_t launch_ssd_small(const SmallArgs& a, int dtype, hipStream_t stream);

}  // namespace ssd
