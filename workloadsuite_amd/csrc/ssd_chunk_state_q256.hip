// K2 -- chunk_state, persistent variant for 16-bit inputs at chunk 256 (the
// Mamba-2-2.7B layer shape).  Same result as the generic kernel in
// ssd_chunk_state.hip (workloads/mamba/model_ref.py:144, 148-149):
//   S[p, n] = sum_l x[l, p] dt[l] exp(Acs[Q-1] - Acs[l]) B[l, n]
// stored as states[b, c, h, p, n].
//
// Work decomposition.  Workgroups of 8 waves loop over contiguous ranges of
// (b, c, h) items, heads fastest, so a workgroup's items share (b, c) and
// usually the group of B.  The product is computed transposed,
//   S^T[n, p] = sum_l (B^T[n, l] w[l]) x[l, p],   w[l] = exp(Acs[Q-1]-Acs[l]) dt[l],
// so that each lane ends with 4 consecutive n of one p (16-byte stores).
//   * B is per group: wave w owns one 16-wide n tile and keeps its B^T
//     fragments for the whole chunk in registers, loaded only when the group
//     changes.  Per item the weight w[l] is applied to them in registers and
//     the product is split into a hi + lo pair of the input type, so the
//     weighting keeps ~16 significant bits through the MFMA.
//   * x comes straight from row-major x in LDS through the transposing read
//     ds_read_b64_tr_b16 (x^T is never staged).
// Data movement.  The next item's x, Acs (and dt) are copied global -> LDS by
// global_load_lds into the second of two LDS buffers while the current item
// computes; x rows are XOR-swizzled by 16-byte piece at copy time so the
// transposing reads are free of bank conflicts.  After the copy lands the
// weights w[l] are tabulated in LDS once per item.  States are stored at the
// start of the next item so the store latency overlaps its compute.
//
// Traffic per item: x 32 KB + Acs 1 KB read, states 32 KB (f32) written; B
// once per group.  HBM bound at this shape.
//
// F16L (SSD_STATE_F16S_LOCAL): the 16 states of row p in n tile t are stored
// as f16 values v / 2^e in the first half of the row's f32 slots, e chosen
// per (p, t) so that the tile row's largest |v| lies in [2^14, 2^15], and the
// item's P x N/16 scales 2^e (f32) packed into the second halves of its
// first rows -- 18 KB written per item instead of 32 KB, in whole cache lines
// (MR:148-149 itself forms the states in the inputs' 16-bit type and MR:155
// stores them in float16).  A tile row lies in one wave (lanes i, i + 16,
// i + 32, i + 48 hold its 16 states), so its maximum takes two lane swaps.
// Two p tiles are stored together: lane groups g, g + 1 swap halves of their
// values, so that each lane writes 8 consecutive f16 (one 16-byte store per
// lane and tile pair instead of two 8-byte ones).
#include <climits>
#include <type_traits>

#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kQ = 256;
constexpr int kNW = 8;               // waves per half workgroup
constexpr int kHalves = 2;           // two items in flight per workgroup
constexpr int kThreads = 64 * kNW * kHalves;
constexpr int kKS = kQ / 32;         // 32-token K steps
constexpr int kXBlocks = kQ / 8;     // 1 KB copy blocks of x (8 rows of 64 x 16-bit)

struct Item {
  int b, c, h, grp;
  int hg;  // head within the group
};

__device__ __forceinline__ Item item_of(const ChunkStateArgs& p, int it) {
  Item r;
  r.h = it % p.nheads;
  const int bc = it / p.nheads;
  r.c = bc % p.nchunks;
  r.b = bc / p.nchunks;
  const int hpg = p.nheads / p.ngroups;
  r.grp = r.h / hpg;
  r.hg = r.h - r.grp * hpg;
  return r;
}

// The item after r in (b, c, h) order, heads fastest: item_of(it + 1)
// without its integer divisions (hpg = heads per group).
__device__ __forceinline__ Item next_item(const ChunkStateArgs& p, Item r, int hpg) {
  ++r.h;
  if (++r.hg == hpg) {
    r.hg = 0;
    ++r.grp;
  }
  if (r.h == p.nheads) {
    r.h = r.grp = r.hg = 0;
    if (++r.c == p.nchunks) {
      r.c = 0;
      ++r.b;
    }
  }
  return r;
}

// SSD_STATE_F16S_LOCAL store of one lane's local states of two p tiles: rows
// row0 (tile 2u) and row0 + 16 (tile 2u + 1), columns 16 nt + 4 g .. + 3 of
// the [P][N] item at `item` (f32 layout), 4 values each.  The 16 states of a
// row in n tile nt are in lanes i, i + 16, i + 32, i + 48 (i = row % 16) of
// the wave: their largest magnitude takes two lane swaps, and sets the tile
// row's power-of-two scale (largest |v| in [2^14, 2^15]).  Lane groups g,
// g + 1 (g even) then swap halves so that each lane writes 8 consecutive f16
// (one 16-byte store): the even group tile 2u's row, the odd one tile
// 2u + 1's.
template <int N>
__device__ __forceinline__ void store_f16l(float* item, int row0, int nt, int g, f32x4 v0, f32x4 v1) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x2 hw[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const f32x4 v = s ? v1 : v0;
    float m = abs_max4(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = nn_max(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = nn_max(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
    const int e = m > 0.f ? min(max(__builtin_amdgcn_frexp_expf(m) - 15, -100), 100) : 0;
    f16x4 hv;
#pragma unroll
    for (int k = 0; k < 4; ++k) hv[k] = (f16)__builtin_ldexpf(v[k], -e);
    hw[s] = __builtin_bit_cast(u32x2, hv);
    if (g == 0) item[f16l_scale_slot<N>(row0 + 16 * s, nt)] = __builtin_ldexpf(1.f, e);
  }
  const auto w0 = __builtin_amdgcn_permlane16_swap(hw[0][0], hw[1][0], false, false);
  const auto w1 = __builtin_amdgcn_permlane16_swap(hw[0][1], hw[1][1], false, false);
  const int row = row0 + 16 * (g & 1);
  *reinterpret_cast<u32x4*>(reinterpret_cast<f16*>(item + (int64_t)row * N) + 16 * nt + 4 * (g & ~1)) =
      u32x4{w0[0], w1[0], w0[1], w1[1]};
}

template <typename S> struct StateStore;
template <> struct StateStore<float> {
  __device__ static void store(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <> struct StateStore<bf16> {
  __device__ static void store(bf16* p, f32x4 v) {
    bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
    *reinterpret_cast<bf16x4*>(p) = o;
  }
};


template <typename T, typename S, int NK, bool HAS_DT, bool PREP, bool F16L>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
void chunk_state_q256_kernel(ChunkStateArgs p) {
  constexpr int N = 32 * NK;        // dstate (64 or 128)
  constexpr int NTILE = N / 16;     // n tiles
  constexpr int PTW = NTILE / 2;    // p tiles per wave (4 for N=128, 2 for N=64)
  static_assert(!F16L || std::is_same<S, float>::value, "f16 local states live in the f32 layout");
  // [half][buffer]: each half's current item and its next one (in flight)
  __shared__ __attribute__((aligned(1024))) T xr[kHalves][2][kQ * kP];
  __shared__ __attribute__((aligned(16))) float ar[kHalves][2][kQ];
  __shared__ __attribute__((aligned(16))) float dr[kHalves][HAS_DT ? 2 : 1][HAS_DT ? kQ : 4];
  __shared__ __attribute__((aligned(16))) float wr[kHalves][kQ];  // w[l] of each half's current item

  const int tid = threadIdx.x, htid = tid & 511, lane = tid & 63;
  const int half = __builtin_amdgcn_readfirstlane(tid >> 9);        // wave-uniform
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 7);  // wave within the half
  __builtin_assume(wave < kNW);
  const int g = lane >> 4, i = lane & 15;
  const int nitems = p.batch * p.nchunks * p.nheads;
  // consecutive item ranges (which share B and C) go to one XCD's L2
  const int lb = xcd_remap(blockIdx.x, gridDim.x);
  const int it0 = (int)((int64_t)lb * nitems / gridDim.x);
  const int it1 = (int)((int64_t)(lb + 1) * nitems / gridDim.x);
  if (it0 >= it1) return;
  const int nt = wave % NTILE, pt0 = (wave / NTILE) * PTW;  // this wave's n tile and first p tile

  // ---- per-lane offsets (fixed for the kernel) ----
  // x operand via transposing reads: rows 4 g + i/4 (+ 16, + 32 ks), columns 16 pt + 4 (i % 4), swizzled.
  int xoff[PTW];
  {
    const int r = 4 * g + (i >> 2), x7 = r & 7;
#pragma unroll
    for (int q = 0; q < PTW; ++q) {
      const int pt = pt0 + q;
      xoff[q] = r * kP + 8 * ((2 * pt + ((i & 3) >> 1)) ^ x7) + 4 * (i & 1);
    }
  }
  const int64_t xcopy = (int64_t)(lane >> 3) * p.sxl + 8 * ((lane & 7) ^ (lane >> 3));
  // states [p][n]: row 16 pt + i, columns 16 nt + 4 g .. + 3
  const int srow = (16 * pt0 + i) * N + 16 * nt + 4 * g;

  // Part m (0..3) of one item's copy into this half's buffer b: x block
  // wave + 8 m; part 0 also Acs (and dt).  Parts are issued between compute
  // steps, so a wave's vector memory queue never holds up its MFMAs for a
  // whole item's copy.
  // (LDS destinations as integer offsets from the __shared__ objects: no
  // generic -> LDS pointer conversion per copy)
  const uint32_t xr_lds = lds_offset(&xr[0][0][0]), ar_lds = lds_offset(&ar[0][0][0]);
  const uint32_t dr_lds = lds_offset(&dr[0][0][0]);
  auto issue_copy_part = [&](const Item& r, int b, int m) __attribute__((always_inline)) {
    const int64_t l0 = (int64_t)r.c * kQ;
    const int hb = 2 * half + b;  // [half][buffer]
    const T* xg = reinterpret_cast<const T*>(p.x) + r.b * p.sxb + l0 * p.sxl + r.h * p.sxh + xcopy;
    {
      const int blk = wave + kNW * m;
      dma16_at(xg + (int64_t)(8 * blk) * p.sxl, xr_lds + (uint32_t)((hb * kQ * kP + blk * 512) * (int)sizeof(T)));
    }
    if (m != 0) return;
    if (wave == kNW - 1) {
      const float* ag = p.acs + (((int64_t)r.b * p.nheads + r.h) * p.nchunks + r.c) * kQ;
      dma16_at(ag + 4 * lane, ar_lds + (uint32_t)(hb * kQ * 4));
    }
    if constexpr (HAS_DT) {
      if (wave < kQ / 64) {
        const float* dg = p.dt + r.b * p.sdb + r.h * p.sdh;
        dma4_at(dg + (l0 + 64 * wave + lane) * p.sdl, dr_lds + (uint32_t)((hb * kQ + 64 * wave) * 4));
      }
    }
  };

  // w[l] = exp(Acs[Q-1] - Acs[l]) dt[l] of the item in this half's buffer b
  auto tabulate = [&](int b) __attribute__((always_inline)) {
    for (int l = htid; l < kQ; l += 512) {
      float w = __builtin_amdgcn_exp2f((ar[half][b][kQ - 1] - ar[half][b][l]) * kLog2e);
      if constexpr (HAS_DT) w *= dr[half][b][l];
      wr[half][l] = w;
    }
  };

  // ---- per-group registers: B^T fragments of this wave's n tile, one per K step ----
  frag8<T> bt[kKS];
  auto load_group = [&](const Item& r) __attribute__((always_inline)) {
    int lane_o = lane;
    asm volatile("" : "+v"(lane_o));  // opaque: per-group address math, not hoisted
    const int go = lane_o >> 4, io = lane_o & 15;
    if constexpr (PREP) {
      // chunk_prep's fragments: one 16-byte load per K step
      const frag8<T>* bf = reinterpret_cast<const frag8<T>*>(p.btf) +
                           ((((int64_t)r.b * p.nchunks + r.c) * p.ngroups + r.grp) * NTILE + nt) * (kKS * 64) + lane_o;
#pragma unroll
      for (int ks = 0; ks < kKS; ++ks) bt[ks] = bf[ks * 64];
      return;
    }
    const int64_t l0 = (int64_t)r.c * kQ;
    const T* bg = reinterpret_cast<const T*>(p.bm) + r.b * p.sbb + l0 * p.sbl + r.grp * p.sbg + 16 * nt + io;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) bt[ks][j] = bg[(int64_t)(32 * ks + slot_token(go, j)) * p.sbl];
  };

  // ---- one item from this half's LDS buffer b into the state registers ----
  f32x4 acc[PTW];
  // step(ks) runs before K step ks.
  auto compute = [&](int b, auto step) __attribute__((always_inline)) {
    const T* xb = xr[half][b];
    const float* wh = wr[half];
#pragma unroll
    for (int q = 0; q < PTW; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      set_prio(3 - ks / 2);  // waves behind in the item go first
      step(ks);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(wh + 32 * ks + 4 * g);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(wh + 32 * ks + 16 + 4 * g);
      frag8<T> hi, lo;
      split_weighted<T>(bt[ks], w0, w1, hi, lo);
#pragma unroll
      for (int q = 0; q < PTW; ++q) {
        const T* a0 = xb + xoff[q] + (32 * ks) * kP;
        const frag8<T> xfr = join<T>(lds_read_tr(a0), lds_read_tr(a0 + 16 * kP));
        acc[q] = mma(hi, xfr, acc[q]);
        acc[q] = mma(lo, xfr, acc[q]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  f32x4 st_prev[PTW];
  // store k of the previous item's states: tile q = k, or with F16L the tile
  // pair (2k, 2k + 1)
  constexpr int NSTORE = F16L ? PTW / 2 : PTW;
  auto store_state = [&](const Item& r, int k) __attribute__((always_inline)) {
    S* sg = reinterpret_cast<S*>(p.states) + (((int64_t)r.b * p.nchunks + r.c) * p.nheads + r.h) * (int64_t)(kP * N);
    if constexpr (F16L) {
      store_f16l<N>(reinterpret_cast<float*>(sg), 16 * (pt0 + 2 * k) + i, nt, g, st_prev[2 * k], st_prev[2 * k + 1]);
    } else {
      StateStore<S>::store(sg + srow + 16 * N * k, st_prev[k]);
    }
  };

  // The two halves take alternate items of the range (half h: it0 + h,
  // it0 + h + 2, ...) and run in lockstep, one barrier pair per step, so
  // they finish together.  Per step and half: compute the current item while
  // the next one's copy and the previous one's state stores are issued
  // between its K steps; then wait for the copy, publish it, tabulate its
  // weights, and publish those.
  const int nsteps = (it1 - it0 + 1) / 2;
  const int hpg = p.nheads / p.ngroups;
  Item cur = item_of(p, it0 + half), prev = cur;
  const bool any = it0 + half < it1;
  if (any) {
#pragma unroll
    for (int m = 0; m < kXBlocks / kNW; ++m) issue_copy_part(cur, 0, m);
    load_group(cur);
  }
  dma_wait();
  __syncthreads();
  if (any) tabulate(0);
  __syncthreads();
  for (int k = 0; k < nsteps; ++k) {
    const int it = it0 + half + 2 * k;
    const int bc = k & 1, bn = bc ^ 1;
    const bool active = it < it1, has_next = it + 2 < it1;
    const Item nxt = has_next ? next_item(p, next_item(p, cur, hpg), hpg) : cur;
    const bool has_prev = k > 0;
    if (active) {
      // copy parts in steps 0..3, the previous item's state stores after them
      compute(bc, [&](int ks) __attribute__((always_inline)) {
        if (ks < kXBlocks / kNW) {
          if (has_next) issue_copy_part(nxt, bn, ks);
        } else if (ks - kXBlocks / kNW < NSTORE) {
          if (has_prev) store_state(prev, ks - kXBlocks / kNW);
        }
      });
#pragma unroll
      for (int q = 0; q < PTW; ++q) st_prev[q] = acc[q];
      prev = cur;
    }
    // the next item's copy, issued before this step's PTW state stores, must
    // have landed; the stores may still be in flight (F16L: PTW more stores of
    // the tile scales, part of which this wait then covers)
    if (active && has_prev) vm_wait<PTW>();
    else dma_wait();
    __syncthreads();
    if (has_next) {
      tabulate(bn);
      if (nxt.b != cur.b || nxt.c != cur.c || nxt.grp != cur.grp) {
        load_group(nxt);
        // complete before the next item's copies are issued: the compiler's
        // wait before the first use would also count those copies
        dma_wait();
      }
      cur = nxt;
    }
    __syncthreads();
  }
  if (any) {
#pragma unroll
    for (int k = 0; k < NSTORE; ++k) store_state(prev, k);
  }
}

template <typename T, typename S, int NK, bool F16L = false>
hipError_t launch_nk(const ChunkStateArgs& a, hipStream_t stream) {
  auto kern = a.dt ? (a.btf ? chunk_state_q256_kernel<T, S, NK, true, true, F16L> : chunk_state_q256_kernel<T, S, NK, true, false, F16L>)
                   : (a.btf ? chunk_state_q256_kernel<T, S, NK, false, true, F16L> : chunk_state_q256_kernel<T, S, NK, false, false, F16L>);
  const int items = a.batch * a.nchunks * a.nheads;
  const int grid = persistent_grid(kern, kThreads, items);
  kern<<<dim3((unsigned)grid), dim3(kThreads), 0, stream>>>(a);
  return hipGetLastError();
}

template <typename T, typename S, bool F16L = false>
hipError_t launch_ts(const ChunkStateArgs& a, hipStream_t stream) {
  switch (a.dstate) {
    case 64: return launch_nk<T, S, 2, F16L>(a, stream);
    case 128: return launch_nk<T, S, 4, F16L>(a, stream);
    default: return hipErrorInvalidValue;
  }
}


// ---- K2 + K3 in one launch: chunk_state with the state recurrence ----
//
// One workgroup (8 waves, the wave layout of one half above) per (b, h)
// chain walks the chunks in order.  Per chunk it computes the chunk's local
// state exactly as chunk_state_q256_kernel does, then advances the running
// state held in registers, h <- h * decay[c] + local (workloads/mamba/
// model_ref.py:152-157), after storing the state entering the chunk, S_in[c],
// as chunk_scan's hi/lo operand pairs (the layout of state_passing's split
// kernel).  The per-chunk local states never reach memory: per chunk the
// chain reads x (32 KB) and writes S_in (32 KB) instead of K2's 32 KB write
// plus K3's 32 KB read and 32 KB write.  Same arithmetic in the same order
// as K2 then K3 (f32 local state, one f32 FMA per element and chunk), so the
// result is bit-identical.
//
// Pipelining per chunk step: the next chunk's x, Acs and dt copies are
// issued in K steps 0-3, and each B^T fragment of the next chunk is loaded
// into its register as soon as the current chunk's weighting has consumed
// it, so the per-chunk group operands arrive under the current chunk's
// compute.  The chunk's S_in stores go out after all of that (storing them
// at the start of the step instead costs 7-12%: later waits for the B^T
// fragments then also wait for those stores).
//
// Workgroups [0, plan.nfull) walk one whole chain each (chains 0 .. nfull -
// 1).  Each of the rest takes plan.seg_len chunks of one of the remaining
// chains (chains nfull, nfull + 1, ...; plan.seg_per_chain segments each;
// both ranges dealt out XCD by XCD, xcd_remap) and writes those
// chunks' local states, exactly as chunk_state would (f32, or with the f16s
// hand-over its f16 rows, SSD_STATE_F16S_LOCAL), for state_passing to
// finish: with 1.25 chains per CU the whole chains take one workgroup slot
// of every CU and the segments the second.
template <typename T, int NK, bool HAS_DT, bool F16S>
__global__ __launch_bounds__(64 * kNW) __attribute__((amdgpu_waves_per_eu(4)))
void chunk_state_chain_kernel(ChunkStateArgs p, StatePassingArgs sp, ChainPlan plan) {
  constexpr int N = 32 * NK;
  constexpr int NTILE = N / 16;
  constexpr int PTW = NTILE / 2;
  static_assert(!F16S || NTILE == kNW, "the f16s store has one n tile per wave");
  __shared__ __attribute__((aligned(1024))) T xr[2][kQ * kP];
  __shared__ __attribute__((aligned(16))) float ar[2][kQ];
  __shared__ __attribute__((aligned(16))) float dr[HAS_DT ? 2 : 1][HAS_DT ? kQ : 4];
  __shared__ __attribute__((aligned(16))) float wr[kQ];
  // F16S: each wave's largest |state| per row p over its n tile, for the
  // state entering the current chunk and the next one ([parity][p][wave])
  __shared__ __attribute__((aligned(16))) float rmx[2][F16S ? kP : 1][kNW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave < kNW);
  const int g = lane >> 4, i = lane & 15;
  const bool local = (int)blockIdx.x >= plan.nfull;  // workgroup-uniform
  // Neighbouring chains (the heads of one batch row, which share B and its
  // group's B^T fragments) go to one XCD's L2: workgroups are dealt to the
  // XCDs in turn, so without the remap every fragment is fetched by all of
  // them.  Whole chains and segments are remapped separately.
  int bh = 0, c0 = 0, c1 = p.nchunks;  // chain b * nheads + h, chunks [c0, c1)
  if (!local) {
    bh = xcd_remap((int)blockIdx.x, plan.nfull);
  } else {
    const int sg = xcd_remap((int)blockIdx.x - plan.nfull, (int)gridDim.x - plan.nfull);
    bh = plan.nfull + sg / plan.seg_per_chain;
    c0 = (sg % plan.seg_per_chain) * plan.seg_len;
    c1 = min(c0 + plan.seg_len, p.nchunks);
    if (c0 >= c1) return;  // the whole workgroup, before any barrier
  }
  const int h = bh % p.nheads, b = bh / p.nheads;
  const int grp = h / (p.nheads / p.ngroups);
  const int nt = wave % NTILE, pt0 = (wave / NTILE) * PTW;
  const bool odd = g & 1;

  int xoff[PTW];
  {
    const int r = 4 * g + (i >> 2), x7 = r & 7;
#pragma unroll
    for (int q = 0; q < PTW; ++q) {
      const int pt = pt0 + q;
      xoff[q] = r * kP + 8 * ((2 * pt + ((i & 3) >> 1)) ^ x7) + 4 * (i & 1);
    }
  }
  const int64_t xcopy = (int64_t)(lane >> 3) * p.sxl + 8 * ((lane & 7) ^ (lane >> 3));
  // this lane's states: row 16 pt + i, columns 16 nt + 4 g .. + 3 of the [P][N] state
  const int srow = (16 * pt0 + i) * N + 16 * nt + 4 * g;
  const T* xchain = reinterpret_cast<const T*>(p.x) + b * p.sxb + h * p.sxh + xcopy;
  const float* achain = p.acs + (int64_t)bh * p.nchunks * kQ;
  const float* dchain = HAS_DT ? p.dt + b * p.sdb + h * p.sdh : nullptr;

  const uint32_t xr_lds = lds_offset(&xr[0][0]), ar_lds = lds_offset(&ar[0][0]);
  const uint32_t dr_lds = lds_offset(&dr[0][0]);
  // part m (0..3) of chunk c's copy into buffer bs
  auto issue_copy_part = [&](int c, int bs, int m) __attribute__((always_inline)) {
    const int64_t l0 = (int64_t)c * kQ;
    const int blk = wave + kNW * m;
    dma16_at(xchain + (l0 + 8 * blk) * p.sxl, xr_lds + (uint32_t)((bs * kQ * kP + blk * 512) * (int)sizeof(T)));
    if (m != 0) return;
    if (wave == kNW - 1) dma16_at(achain + (int64_t)c * kQ + 4 * lane, ar_lds + (uint32_t)(bs * kQ * 4));
    if constexpr (HAS_DT) {
      if (wave < kQ / 64) dma4_at(dchain + (l0 + 64 * wave + lane) * p.sdl, dr_lds + (uint32_t)((bs * kQ + 64 * wave) * 4));
    }
  };
  auto tabulate = [&](int bs) __attribute__((always_inline)) {
    if (tid < kQ) {
      float w = __builtin_amdgcn_exp2f((ar[bs][kQ - 1] - ar[bs][tid]) * kLog2e);
      if constexpr (HAS_DT) w *= dr[bs][tid];
      wr[tid] = w;
    }
  };
  // chunk_prep's B^T fragments of chunk c, this wave's n tile
  auto btf_of = [&](int c) __attribute__((always_inline)) {
    return reinterpret_cast<const frag8<T>*>(p.btf) +
           ((((int64_t)b * p.nchunks + c) * p.ngroups + grp) * NTILE + nt) * (kKS * 64) + lane;
  };

  // running state: S_in of the current chunk
  f32x4 st[PTW];
#pragma unroll
  for (int q = 0; q < PTW; ++q)
    st[q] = sp.init && !local ? *reinterpret_cast<const f32x4*>(sp.init + (int64_t)bh * (kP * N) + srow + 16 * N * q)
                              : f32x4{0.f, 0.f, 0.f, 0.f};

  // S_in of chunk c, as [hi x8 | lo x8] of T per 8 consecutive states: lane
  // pairs (g, g ^ 1) swap halves so that the even-g lane stores the 8 hi and
  // the odd-g lane the 8 lo values, each at its own f32 state address.
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  auto store_sin = [&](int c, int q) __attribute__((always_inline)) {
    // from the f32 state (opaque: no fusing of the recurrence's fma into the rounding)
    f32x4 v = st[q];
    asm volatile("" : "+v"(v));
    vec4<T> hi, lo;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hi[k] = from_f32<T>(v[k]);
      lo[k] = from_f32<T>(v[k] - to_f32<T>(hi[k]));
    }
    const u32x2 hw = __builtin_bit_cast(u32x2, hi), lw = __builtin_bit_cast(u32x2, lo);
    const u32x2 give = odd ? hw : lw, keep = odd ? lw : hw;
    u32x2 got;
    got[0] = (uint32_t)__shfl_xor((int)give[0], 16);
    got[1] = (uint32_t)__shfl_xor((int)give[1], 16);
    const u32x4 out = odd ? u32x4{got[0], got[1], keep[0], keep[1]} : u32x4{keep[0], keep[1], got[0], got[1]};
    float* sg = reinterpret_cast<float*>(sp.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * (int64_t)(kP * N);
    *reinterpret_cast<u32x4*>(sg + srow + 16 * N * q) = out;
  };
  // F16S (SSD_STATE_F16S): S_in[c] as f16 rows with a power-of-two scale per
  // row p (row p's N f16 values in the first half of its f32 slots, the scale
  // in sp.sscale[b, c, h, p]).  The row's largest |state| spans all waves (one
  // n tile each): every wave publishes its own per-row maximum into rmx[par]
  // once the state is final, and after the next barrier each lane reads the 8
  // maxima of its 4 rows.
  auto publish_rowmax = [&](int par) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < PTW; ++q) {
      float m = abs_max4(st[q]);
      // across the lane groups g (lanes i, i + 16, i + 32, i + 48): swap with
      // the neighbouring 16-lane row, then with the other 32-lane half
      {
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
        m = nn_max(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
        m = nn_max(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
      }
      if (g == 0) rmx[par][16 * (pt0 + q) + i][wave] = m;
    }
  };
  auto store_sin_f16s = [&](int c, int par) __attribute__((always_inline)) {
    float* item = reinterpret_cast<float*>(sp.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * (int64_t)(kP * N);
    // one p-tile pair (2u, 2u + 1) at a time: lane groups g, g + 1 (g even)
    // swap halves, so the even group holds columns 16 nt + 4 g .. + 7 of tile
    // 2u's row and the odd one those of tile 2u + 1's row (one 16-byte store each)
#pragma unroll
    for (int u = 0; u < PTW / 2; ++u) {
      u32x2 hw[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int q = 2 * u + s, row = 16 * (pt0 + q) + i;
        const f32x4 m0 = *reinterpret_cast<const f32x4*>(&rmx[par][row][0]);
        const f32x4 m1 = *reinterpret_cast<const f32x4*>(&rmx[par][row][4]);
        const float m = nn_max(nn_max(nn_max(m0[0], m0[1]), nn_max(m0[2], m0[3])),
                               nn_max(nn_max(m1[0], m1[1]), nn_max(m1[2], m1[3])));
        const int e = m > 0.f ? min(max(__builtin_amdgcn_frexp_expf(m) - 15, -100), 100) : 0;
        f32x4 v = st[q];
        asm volatile("" : "+v"(v));  // from the f32 state (no fusing of the recurrence into the rounding)
        f16x4 hv;
#pragma unroll
        for (int k = 0; k < 4; ++k) hv[k] = (f16)__builtin_ldexpf(v[k], -e);
        hw[s] = __builtin_bit_cast(u32x2, hv);
        if (wave == 0 && g == 0)
          sp.sscale[(((int64_t)b * p.nchunks + c) * p.nheads + h) * kP + row] = __builtin_ldexpf(1.f, e);
      }
      const auto w0 = __builtin_amdgcn_permlane16_swap(hw[0][0], hw[1][0], false, false);
      const auto w1 = __builtin_amdgcn_permlane16_swap(hw[0][1], hw[1][1], false, false);
      const int row = 16 * (pt0 + 2 * u + (odd ? 1 : 0)) + i;
      *reinterpret_cast<u32x4*>(reinterpret_cast<f16*>(item + (int64_t)row * N) + 16 * nt + 4 * (g & ~1)) =
          u32x4{w0[0], w1[0], w0[1], w1[1]};
    }
  };

  // a segment's local state of chunk c in chunk_state's layout: f32, or with
  // the f16s hand-over as chunk_state's f16 rows (SSD_STATE_F16S_LOCAL) for
  // state_passing to finish
  auto store_local = [&](int c) __attribute__((always_inline)) {
    float* sg = reinterpret_cast<float*>(sp.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * (int64_t)(kP * N);
    if constexpr (F16S) {
#pragma unroll
      for (int u = 0; u < PTW / 2; ++u) store_f16l<N>(sg, 16 * (pt0 + 2 * u) + i, nt, g, st[2 * u], st[2 * u + 1]);
    } else {
#pragma unroll
      for (int q = 0; q < PTW; ++q) *reinterpret_cast<f32x4*>(sg + srow + 16 * N * q) = st[q];
    }
  };

  frag8<T> bt[kKS];
  {
    const frag8<T>* bf = btf_of(c0);
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) bt[ks] = bf[ks * 64];
  }
#pragma unroll
  for (int m = 0; m < kXBlocks / kNW; ++m) issue_copy_part(c0, 0, m);
  if constexpr (F16S) {
    if (!local) publish_rowmax(c0 & 1);
  }
  dma_wait();
  __syncthreads();
  tabulate(0);
  __syncthreads();

  for (int c = c0; c < c1; ++c) {
    const int bc = (c - c0) & 1, bn = bc ^ 1;
    const bool has_next = c + 1 < c1;
    const float dec = sp.decay[(int64_t)bh * p.nchunks + c];
    const frag8<T>* bnext = btf_of(has_next ? c + 1 : c);
    const T* xb = xr[bc];
    f32x4 acc[PTW];
#pragma unroll
    for (int q = 0; q < PTW; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      set_prio(3 - ks / 2);
      if (ks < kXBlocks / kNW && has_next) issue_copy_part(c + 1, bn, ks);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(wr + 32 * ks + 4 * g);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(wr + 32 * ks + 16 + 4 * g);
      frag8<T> hi, lo;
      split_weighted<T>(bt[ks], w0, w1, hi, lo);
      bt[ks] = bnext[ks * 64];  // (the last chunk reloads its own: no branch, no register copies)
#pragma unroll
      for (int q = 0; q < PTW; ++q) {
        const T* a0 = xb + xoff[q] + (32 * ks) * kP;
        const frag8<T> xfr = join<T>(lds_read_tr(a0), lds_read_tr(a0 + 16 * kP));
        acc[q] = mma(hi, xfr, acc[q]);
        acc[q] = mma(lo, xfr, acc[q]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the chunk's stores go out after every load of the step; the wait
    // leaves only them in flight (the next chunk's copies and B^T fragments
    // have landed)
    if (local) {
#pragma unroll
      for (int q = 0; q < PTW; ++q) st[q] = acc[q];
      store_local(c);
    } else if constexpr (F16S) {
      store_sin_f16s(c, c & 1);
#pragma unroll
      for (int q = 0; q < PTW; ++q) st[q] = st[q] * dec + acc[q];
      publish_rowmax((c + 1) & 1);
    } else {
#pragma unroll
      for (int q = 0; q < PTW; ++q) store_sin(c, q);
#pragma unroll
      for (int q = 0; q < PTW; ++q) st[q] = st[q] * dec + acc[q];
    }
    vm_wait<PTW>();
    __syncthreads();
    if (has_next) tabulate(bn);
    __syncthreads();
  }
  if (!local && sp.final_state) {
#pragma unroll
    for (int q = 0; q < PTW; ++q)
      *reinterpret_cast<f32x4*>(sp.final_state + (int64_t)bh * (kP * N) + srow + 16 * N * q) = st[q];
  }
}

template <typename T, int NK>
hipError_t launch_chain_nk(const ChunkStateArgs& a, const StatePassingArgs& sp, const ChainPlan& plan,
                           hipStream_t stream) {
  constexpr bool kF16S = 32 * NK / 16 == kNW;  // the f16s store needs one n tile per wave (d_state 128)
  if (sp.f16s && (!kF16S || !sp.sscale)) return hipErrorInvalidValue;
  auto kern = sp.f16s ? (a.dt ? chunk_state_chain_kernel<T, NK, true, kF16S> : chunk_state_chain_kernel<T, NK, false, kF16S>)
                      : (a.dt ? chunk_state_chain_kernel<T, NK, true, false> : chunk_state_chain_kernel<T, NK, false, false>);
  const int64_t rest = (int64_t)a.batch * a.nheads - plan.nfull;
  const unsigned grid = (unsigned)(plan.nfull + rest * plan.seg_per_chain);
  kern<<<dim3(grid), dim3(64 * kNW), 0, stream>>>(a, sp, plan);
  return hipGetLastError();
}

}  // namespace

bool chunk_state_persistent_supported(const ChunkStateArgs& a, int dtype) {
  return a.chunk == kQ && (a.dstate == 64 || a.dstate == 128) &&
         (dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16);
}

hipError_t launch_chunk_state_persistent(const ChunkStateArgs& a, int dtype, int state_dtype, hipStream_t stream) {
  if (state_dtype == SSD_DTYPE_F32) {
    if (dtype == SSD_DTYPE_BF16) return launch_ts<bf16, float>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_ts<f16, float>(a, stream);
  } else if (state_dtype == SSD_STATE_F16S_LOCAL) {
    if (dtype == SSD_DTYPE_BF16) return launch_ts<bf16, float, true>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_ts<f16, float, true>(a, stream);
  } else if (state_dtype == SSD_DTYPE_BF16) {
    if (dtype == SSD_DTYPE_BF16) return launch_ts<bf16, bf16>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_ts<f16, bf16>(a, stream);
  }
  return hipErrorInvalidValue;
}

bool chunk_state_chain_supported(const ChunkStateArgs& a, int dtype) {
  return chunk_state_persistent_supported(a, dtype) && a.btf != nullptr;
}

ChainPlan chunk_state_chain_plan(const ChunkStateArgs& a, int dtype) {
  ChainPlan none{0, 1, 1};
  if (!chunk_state_chain_supported(a, dtype)) return none;
  // One workgroup per chain, up to two per CU.  The launch saves K3's pass
  // over the states but runs each chain's chunks in sequence, so it pays off
  // only when the chains keep every CU equally busy.  With fewer chains than
  // CUs the idle CUs are lost (C4, 80 chains of 256 chunks: 31% slower than
  // K2 then K3).  Measured on MI355X (forward, chunk 256): 7-14% faster
  // wherever the average CU holds at least 3/4 of the busiest CU's chains.
  const int64_t chains = (int64_t)a.batch * a.nheads;
  const int n = device_cu_count();
  const int64_t cus = n > 0 ? n : 256;
  const int64_t per_cu = (chains + cus - 1) / cus;
  if (4 * chains >= 3 * per_cu * cus) return ChainPlan{(int)chains, 1, a.nchunks};
  // Between one and two chains per CU (C3: 320 chains on 256 CUs) the CUs
  // holding a second chain would set the time.  One whole chain per CU, and
  // the remaining chains in segments that fill the second slots; their local
  // states go to state_passing, which then runs over those chains only.
  if (chains > cus && chains < 2 * cus) {
    const int64_t rest = chains - cus;
    const int64_t want = cus / rest > 1 ? cus / rest : 1;  // segments per chain
    const int seg_len = (int)((a.nchunks + want - 1) / want);
    const int segs = (a.nchunks + seg_len - 1) / seg_len;
    return ChainPlan{(int)cus, segs, seg_len};
  }
  return none;
}

hipError_t launch_chunk_state_chain(const ChunkStateArgs& a, const StatePassingArgs& sp, const ChainPlan& plan,
                                    int dtype, hipStream_t stream) {
  const int64_t chains = (int64_t)a.batch * a.nheads;
  if (!chunk_state_chain_supported(a, dtype) || (sp.f16s ? sp.split_dtype != 0 : sp.split_dtype != dtype) ||
      plan.nfull < 1 || plan.nfull > chains ||
      plan.seg_per_chain < 1 || plan.seg_len < 1 || (int64_t)plan.seg_per_chain * plan.seg_len < a.nchunks ||
      plan.nfull + (chains - plan.nfull) * plan.seg_per_chain > INT_MAX)
    return hipErrorInvalidValue;
  if (dtype == SSD_DTYPE_BF16)
    return a.dstate == 64 ? launch_chain_nk<bf16, 2>(a, sp, plan, stream) : launch_chain_nk<bf16, 4>(a, sp, plan, stream);
  return a.dstate == 64 ? launch_chain_nk<f16, 2>(a, sp, plan, stream) : launch_chain_nk<f16, 4>(a, sp, plan, stream);
}

}  // namespace ssd
