// K3 -- state_passing: the inter-chunk recurrence, in place.
//
// Replaces the Python loop of workloads/mamba/model_ref.py:152-157:
//   states.append(h); h = h * chunk_decay[:, i] + block_state[:, i]
// On entry states[b, c, h] holds chunk c's local state (K2's output); on exit
// it holds the state entering chunk c (S_in).  h starts at the optional
// initial state (zeros in MR:153) and the state after the last chunk -- which
// MR computes and drops -- goes to final_state.
//
// Sequential over chunks, parallel over batch x head x P x N: one thread owns
// 4 consecutive state elements (one 16-byte vector for f32 states), keeps the
// running state in registers and streams the chunks.  Each step's local-state
// load does not depend on the running state, so U chunks of loads are issued
// before the U dependent FMAs and stores -- the loads run ahead of the FMA
// chain, and the next batch's loads are in flight while a batch is stored.
// Threads of a workgroup cover consecutive elements of one (b, h)
// state, so every load and store is a fully coalesced 16-byte access.
// Pure streaming: HBM traffic per chunk is one read and one write of the
// state, the roofline bound is HBM bandwidth.
#include <type_traits>

#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {


template <typename S> struct StateIO;
// Local states are read once.  Long chains read them with non-temporal loads
// (a read-only stream of 16-byte nt loads reaches ~7.0 TB/s on MI355X against
// ~6.3 TB/s for plain loads; K3 over 256 chunks gains ~3%); chains shorter
// than two load batches use plain loads (nt loads made the 4-chunk C5 shape
// 25% slower).  S_in is stored normally: chunk_scan reads it next and finds
// part of it still cached.
template <bool NT> __device__ __forceinline__ f32x4 load_state(const float* p) {
  return NT ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p)) : *reinterpret_cast<const f32x4*>(p);
}

template <> struct StateIO<float> {
  template <bool NT = false>
  __device__ static f32x4 load(const float* p) { return load_state<NT>(p); }
  __device__ static void store(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <> struct StateIO<bf16> {
  template <bool NT = false>
  __device__ static f32x4 load(const bf16* p) {
    bf16x4 v = NT ? __builtin_nontemporal_load(reinterpret_cast<const bf16x4*>(p)) : *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
  __device__ static void store(bf16* p, f32x4 v) {
    bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
    *reinterpret_cast<bf16x4*>(p) = o;
  }
};

// The recurrence over all chunks for one thread's 4 state elements, software
// pipelined: the loads of the next kUnroll chunks are issued before the
// current kUnroll chunks' stores and FMAs, so each thread always has a batch
// of loads in flight (two register batches used in turn: no copies between
// them, which would wait for the loads).  load(c) returns chunk c's local
// state, store(c, v) writes S_in[c] = v; dec[c] is chunk c's decay.
template <int kUnroll = 8, typename V, typename LoadF, typename StoreF>
__device__ __forceinline__ V run_chain(int nchunks, const float* __restrict__ dec, V st, LoadF load,
                                       StoreF store) {
  V la[kUnroll], lb[kUnroll];
  float da[kUnroll], db[kUnroll];
  // In the main loop the loads are unconditional (past the last chunk they
  // re-read it and the value is unused): with no branches around them the
  // compiler's vmcnt waits count exactly, and waiting for one batch leaves the
  // other in flight.  Chains shorter than two batches load only their chunks.
  auto fetch = [&](int c0, V* l, float* d, bool all) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (all || c0 + u < nchunks) {
        const int c = min(c0 + u, nchunks - 1);
        l[u] = all ? load(c, std::true_type()) : load(c, std::false_type());
        d[u] = dec[c];
      }
    }
  };
  auto advance = [&](int c0, const V* l, const float* d, bool all) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (all || c0 + u < nchunks) {
        store(c0 + u, st);
        st = st * d[u] + l[u];
      }
    }
  };
  int c0 = 0;
  if (nchunks >= 2 * kUnroll) {
    fetch(0, la, da, true);
    for (; c0 + 2 * kUnroll <= nchunks; c0 += 2 * kUnroll) {
      fetch(c0 + kUnroll, lb, db, true);
      advance(c0, la, da, true);
      fetch(c0 + 2 * kUnroll, la, da, true);
      advance(c0 + kUnroll, lb, db, true);
    }
  } else {
    fetch(0, la, da, false);
  }
  if (c0 < nchunks) {  // the last 1 .. 2 kUnroll - 1 chunks; la holds chunks c0 ..
    fetch(c0 + kUnroll, lb, db, false);
    advance(c0, la, da, false);
    advance(c0 + kUnroll, lb, db, false);
  }
  return st;
}

template <typename S>
__global__ __launch_bounds__(256) void state_passing_kernel(StatePassingArgs p) {
  const int64_t PN = (int64_t)p.headdim * p.dstate;
  const int vec_per_bh = (int)(PN / 4);
  const int blocks_per_bh = (vec_per_bh + 255) / 256;
  const int bh = p.bh_begin + (int)blockIdx.x / blocks_per_bh;  // b * nheads + h
  const int v = (blockIdx.x % blocks_per_bh) * 256 + threadIdx.x;
  if (v >= vec_per_bh) return;
  const int h = bh % p.nheads, b = bh / p.nheads;

  S* base = reinterpret_cast<S*>(p.states) + ((int64_t)b * p.nchunks * p.nheads + h) * PN + 4 * (int64_t)v;
  const int64_t cstride = (int64_t)p.nheads * PN;  // elements between chunks
  const float* dec = p.decay + (int64_t)bh * p.nchunks;

  f32x4 st = p.init ? *reinterpret_cast<const f32x4*>(p.init + (int64_t)bh * PN + 4 * (int64_t)v)
                    : f32x4{0.f, 0.f, 0.f, 0.f};
  st = run_chain(
      p.nchunks, dec, st,
      [&](int c, auto nt) { return StateIO<S>::template load<decltype(nt)::value>(base + c * cstride); },
      [&](int c, f32x4 val) { StateIO<S>::store(base + c * cstride, val); });
  if (p.final_state) *reinterpret_cast<f32x4*>(p.final_state + (int64_t)bh * PN + 4 * (int64_t)v) = st;
}

// f32 states handed to the chunk-256 chunk_scan: S_in is written as that
// kernel's MFMA operands -- every 8 consecutive states (32 bytes) become
// [hi x8 | lo x8] of T, hi = T(v), lo = T(v - hi) -- so chunk_scan does not
// split it again per item.  The recurrence and final_state stay f32.
// Thread mapping as in state_passing_kernel (4 states, one 16-byte load per
// chunk); lane pairs then swap halves so that the even lane stores the 8 hi
// and the odd lane the 8 lo values of their 8 states: 16 contiguous bytes per
// lane, 1 KB per wave store.
template <typename T>
__global__ __launch_bounds__(256) void state_passing_split_kernel(StatePassingArgs p) {
  const int64_t PN = (int64_t)p.headdim * p.dstate;
  const int vec_per_bh = (int)(PN / 4);
  const int blocks_per_bh = (vec_per_bh + 255) / 256;
  const int bh = p.bh_begin + (int)blockIdx.x / blocks_per_bh;
  const int v = (blockIdx.x % blocks_per_bh) * 256 + threadIdx.x;
  if (v >= vec_per_bh) return;  // vec_per_bh is a multiple of 256: whole waves leave together
  const int h = bh % p.nheads, b = bh / p.nheads;
  const bool odd = threadIdx.x & 1;

  float* base = reinterpret_cast<float*>(p.states) + ((int64_t)b * p.nchunks * p.nheads + h) * PN + 4 * (int64_t)v;
  const int64_t cstride = (int64_t)p.nheads * PN;
  const float* dec = p.decay + (int64_t)bh * p.nchunks;

  f32x4 st = p.init ? *reinterpret_cast<const f32x4*>(p.init + (int64_t)bh * PN + 4 * (int64_t)v)
                    : f32x4{0.f, 0.f, 0.f, 0.f};
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  auto store_split = [&](int c, f32x4 val) {
    // the split starts from the f32 state: opaque, so that the compiler cannot
    // fuse the recurrence's fma with the rounding to T (one rounding instead of
    // two would change hi in rare cases)
    asm volatile("" : "+v"(val));
    vec4<T> hi, lo;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hi[k] = from_f32<T>(val[k]);
      lo[k] = from_f32<T>(val[k] - to_f32<T>(hi[k]));
    }
    const u32x2 hw = __builtin_bit_cast(u32x2, hi), lw = __builtin_bit_cast(u32x2, lo);
    // even lane keeps its hi and receives the odd lane's hi; odd lane the reverse for lo
    const u32x2 give = odd ? hw : lw, keep = odd ? lw : hw;
    u32x2 got;
    got[0] = (uint32_t)__builtin_amdgcn_mov_dpp((int)give[0], 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
    got[1] = (uint32_t)__builtin_amdgcn_mov_dpp((int)give[1], 0xB1, 0xF, 0xF, false);
    const u32x4 out = odd ? u32x4{got[0], got[1], keep[0], keep[1]} : u32x4{keep[0], keep[1], got[0], got[1]};
    // the pair's 32 bytes start at the even lane's 16: hi at +0, lo at +16
    *reinterpret_cast<u32x4*>(base + c * cstride) = out;
  };
  st = run_chain(
      p.nchunks, dec, st,
      [&](int c, auto nt) { return StateIO<float>::template load<decltype(nt)::value>(base + c * cstride); },
      store_split);
  if (p.final_state) *reinterpret_cast<f32x4*>(p.final_state + (int64_t)bh * PN + 4 * (int64_t)v) = st;
}

// The maximum of m over each aligned group of G lanes (G = 8 or 16, within
// one DPP row), with DPP moves (no LDS round trip): two quad permutations,
// then the half-row and row mirrors.
template <int G>
__device__ __forceinline__ float row_max(float m) {
  static_assert(G == 8 || G == 16 || G == 32, "lane group");
  auto dpp = [](float v, int ctrl) __attribute__((always_inline)) {
    switch (ctrl) {
      case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad 1,0,3,2
      case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad 2,3,0,1
      case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
      default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
    }
  };
  m = nn_max(m, dpp(m, 0));
  m = nn_max(m, dpp(m, 1));
  m = nn_max(m, dpp(m, 2));
  if constexpr (G >= 16) m = nn_max(m, dpp(m, 3));
  if constexpr (G == 32) {
    // with the neighbouring 16-lane row
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = nn_max(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  }
  return m;
}

// f32 states handed to the chunk-256 chunk_scan as f16 with a power-of-two
// scale per state row (SSD_STATE_F16S), the f16 values written in place in
// the f32 layout: row p of an item (N f32 slots) gets its N f16 values,
// v / 2^e, in its first half, and 2^e goes to sscale[item][p]; e is chosen
// so that the row's largest |v| lies in [2^14, 2^15].  Each thread owns SPT
// consecutive states of a row (16-byte loads per chunk, one 2 SPT-byte
// store); the N/SPT threads of a row (one wave holds whole rows) find the
// row's largest magnitude with DPP moves (and a 16-lane row swap for 32
// threads).  Every load of a row precedes, in the wave's instruction order,
// the stores into that row, so the in-place writes never overtake a read.
// The recurrence and final_state stay f32.
// F16L: the local states arrive as SSD_STATE_F16S_LOCAL (chunk_state's f16
// rows, a scale per 16-column tile of each row packed into the second halves
// of the item's first rows): each thread reads its SPT f16 values (the slots
// its S_in values then overwrite; SPT divides 16) and their tile's scale,
// which no store touches; f16 value times a power of two is exact in f32.
template <int N, int SPT, int UNROLL, bool F16L>
__global__ __launch_bounds__(256) void state_passing_f16s_kernel(StatePassingArgs p) {
  constexpr int TPR = N / SPT;  // threads per row (SPT = 4 or 8 states per thread)
  typedef typename std::conditional<SPT == 8, f32x8, f32x4>::type V;
  typedef typename std::conditional<SPT == 8, f16x8, f16x4>::type H;
  const int64_t PN = (int64_t)p.headdim * N;
  const int vec_per_bh = (int)(PN / SPT);
  const int blocks_per_bh = (vec_per_bh + 255) / 256;
  const int bh = p.bh_begin + (int)blockIdx.x / blocks_per_bh;
  const int v = (blockIdx.x % blocks_per_bh) * 256 + threadIdx.x;
  if (v >= vec_per_bh) return;  // vec_per_bh is a multiple of 256: whole waves leave together
  const int h = bh % p.nheads, b = bh / p.nheads;
  const int row = v / TPR, col = SPT * (v % TPR);

  float* base = reinterpret_cast<float*>(p.states) + ((int64_t)b * p.nchunks * p.nheads + h) * PN;
  const int64_t cstride = (int64_t)p.nheads * PN;
  const float* dec = p.decay + (int64_t)bh * p.nchunks;
  float* elem = base + SPT * (int64_t)v;                     // this thread's f32 states
  f16* hrow = reinterpret_cast<f16*>(base + (int64_t)row * N) + col;  // its f16 slots
  // the row's scale: sscale[b, c, h, row], chunks p.nheads * headdim apart
  float* srow = p.sscale + ((int64_t)b * p.nchunks * p.nheads + h) * p.headdim + row;
  const int64_t sstride = (int64_t)p.nheads * p.headdim;

  // SPT consecutive floats from p (16-byte loads), non-temporal or not
  auto loadv = [](const float* src, auto nt) __attribute__((always_inline)) {
    const f32x4* q = reinterpret_cast<const f32x4*>(src);
    V r;
#pragma unroll
    for (int h = 0; h < SPT / 4; ++h) {
      const f32x4 x = decltype(nt)::value ? __builtin_nontemporal_load(q + h) : q[h];
#pragma unroll
      for (int k = 0; k < 4; ++k) r[4 * h + k] = x[k];
    }
    return r;
  };
  V st;
  if (p.init) {
    st = loadv(p.init + (int64_t)bh * PN + SPT * (int64_t)v, std::false_type());
  } else {
#pragma unroll
    for (int k = 0; k < SPT; ++k) st[k] = 0.f;
  }
  auto store_f16s = [&](int c, V val) {
    asm volatile("" : "+v"(val));  // from the f32 state (no fusing of the recurrence into the rounding)
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < SPT; ++k) m = __builtin_elementwise_maximum(m, fabsf(val[k]));
    m = row_max<TPR>(m);
    const int e = m > 0.f ? min(max(__builtin_amdgcn_frexp_expf(m) - 15, -100), 100) : 0;
    H hv;
#pragma unroll
    for (int k = 0; k < SPT; ++k) hv[k] = (f16)__builtin_ldexpf(val[k], -e);
    // non-temporal: S_in is read once, by chunk_scan after this launch (C4's
    // forward 884 -> 875 us; C3's, whose K3 covers only the mixed plan's
    // segment chains, unchanged)
    __builtin_nontemporal_store(hv, reinterpret_cast<H*>(hrow + c * 2 * cstride));
    if (col == 0) srow[c * sstride] = __builtin_ldexpf(1.f, e);
  };
  // F16L: this thread's SPT f16 local values of chunk c times the row's scale
  static_assert(16 % SPT == 0, "a thread's states lie in one 16-column tile");
  const float* rscale = base + f16l_scale_slot<N>(row, col / 16);
  auto loadh = [&](int c, auto nt) __attribute__((always_inline)) {
    const H* q = reinterpret_cast<const H*>(hrow + c * 2 * cstride);
    const H hv = decltype(nt)::value ? __builtin_nontemporal_load(q) : *q;
    const float sc = rscale[c * cstride];
    V r;
#pragma unroll
    for (int k = 0; k < SPT; ++k) r[k] = (float)hv[k] * sc;
    return r;
  };
  if constexpr (F16L) {
    st = run_chain<UNROLL>(p.nchunks, dec, st, loadh, store_f16s);
  } else {
    st = run_chain<UNROLL>(p.nchunks, dec, st, [&](int c, auto nt) { return loadv(elem + c * cstride, nt); }, store_f16s);
  }
  if (p.final_state) {
    float* fo = p.final_state + (int64_t)bh * PN + SPT * (int64_t)v;
#pragma unroll
    for (int h = 0; h < SPT / 4; ++h)
      *reinterpret_cast<f32x4*>(fo + 4 * h) = f32x4{st[4 * h], st[4 * h + 1], st[4 * h + 2], st[4 * h + 3]};
  }
}

}  // namespace

hipError_t launch_state_passing(const StatePassingArgs& a, int state_dtype, hipStream_t stream) {
  const int64_t PN = (int64_t)a.headdim * a.dstate;
  const int64_t all = (int64_t)a.batch * a.nheads;
  if (a.bh_begin < 0 || a.bh_count < 0 || a.bh_begin + (int64_t)a.bh_count > all) return hipErrorInvalidValue;
  const int64_t chains = a.bh_count > 0 ? a.bh_count : all - a.bh_begin;
  if (a.f16s) {
    // 8 states per thread (two 16-byte loads of f32 local states or one of f16
    // ones, one 16-byte f16 store per chunk) in batches of 2 chunks: 76 VGPRs.
    // Against 4 states per thread in batches of 4 (MI355X, rotated buffers
    // beyond the Infinity Cache): C3 (f32 local states in) 52.5 -> 51.0 us,
    // 0.646 of HBM peak, where a hand-written stream at the same 2 : 1 read /
    // write mix with plain stores reaches 0.633 and with non-temporal ones
    // 0.670 (bench.py --hbm-probe); C4 (f16 local states in) 164 -> 161 us.
    constexpr int spt = 8, unroll = 2;
    const bool f16l = state_dtype == SSD_STATE_F16S_LOCAL;
    if ((state_dtype != SSD_DTYPE_F32 && !f16l) || a.split_dtype != 0 || !a.sscale || (PN / spt) % 256 != 0)
      return hipErrorInvalidValue;
    const dim3 grid((unsigned)(chains * ((PN / spt + 255) / 256)));
    if (a.dstate == 128) {
      if (f16l) state_passing_f16s_kernel<128, spt, unroll, true><<<grid, 256, 0, stream>>>(a);
      else state_passing_f16s_kernel<128, spt, unroll, false><<<grid, 256, 0, stream>>>(a);
    } else if (a.dstate == 64) {
      if (f16l) state_passing_f16s_kernel<64, spt, unroll, true><<<grid, 256, 0, stream>>>(a);
      else state_passing_f16s_kernel<64, spt, unroll, false><<<grid, 256, 0, stream>>>(a);
    } else {
      return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (a.split_dtype != 0) {
    if (state_dtype != SSD_DTYPE_F32 || PN % 8 != 0) return hipErrorInvalidValue;
    if (PN % 256 != 0) return hipErrorInvalidValue;  // whole waves per (b, h)
    const dim3 grid((unsigned)(chains * ((PN / 4 + 255) / 256)));
    if (a.split_dtype == SSD_DTYPE_BF16) state_passing_split_kernel<bf16><<<grid, 256, 0, stream>>>(a);
    else if (a.split_dtype == SSD_DTYPE_F16) state_passing_split_kernel<f16><<<grid, 256, 0, stream>>>(a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
  }
  const int64_t blocks_per_bh = (PN / 4 + 255) / 256;
  const dim3 grid((unsigned)(chains * blocks_per_bh));
  if (state_dtype == SSD_DTYPE_F32) {
    state_passing_kernel<float><<<grid, 256, 0, stream>>>(a);
  } else if (state_dtype == SSD_DTYPE_BF16) {
    state_passing_kernel<bf16><<<grid, 256, 0, stream>>>(a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ssd
