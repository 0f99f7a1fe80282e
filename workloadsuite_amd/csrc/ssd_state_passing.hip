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
// chain.  Threads of a workgroup cover consecutive elements of one (b, h)
// state, so every load and store is a fully coalesced 16-byte access.
// Pure streaming: HBM traffic per chunk is one read and one write of the
// state, the roofline bound is HBM bandwidth.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kUnroll = 8;

template <typename S> struct StateIO;
template <> struct StateIO<float> {
  __device__ static f32x4 load(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
  __device__ static void store(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <> struct StateIO<bf16> {
  __device__ static f32x4 load(const bf16* p) {
    bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
  __device__ static void store(bf16* p, f32x4 v) {
    bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
    *reinterpret_cast<bf16x4*>(p) = o;
  }
};

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
  for (int c0 = 0; c0 < p.nchunks; c0 += kUnroll) {
    f32x4 loc[kUnroll];
    float d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (c0 + u < p.nchunks) {
        loc[u] = StateIO<S>::load(base + (c0 + u) * cstride);
        d[u] = dec[c0 + u];
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (c0 + u < p.nchunks) {
        StateIO<S>::store(base + (c0 + u) * cstride, st);
        st = st * d[u] + loc[u];
      }
    }
  }
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
  for (int c0 = 0; c0 < p.nchunks; c0 += kUnroll) {
    f32x4 loc[kUnroll];
    float d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (c0 + u < p.nchunks) {
        loc[u] = *reinterpret_cast<const f32x4*>(base + (c0 + u) * cstride);
        d[u] = dec[c0 + u];
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (c0 + u < p.nchunks) {
        vec4<T> hi, lo;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          hi[k] = from_f32<T>(st[k]);
          lo[k] = from_f32<T>(st[k] - to_f32<T>(hi[k]));
        }
        const u32x2 hw = __builtin_bit_cast(u32x2, hi), lw = __builtin_bit_cast(u32x2, lo);
        // even lane keeps its hi and receives the odd lane's hi; odd lane the reverse for lo
        const u32x2 give = odd ? hw : lw, keep = odd ? lw : hw;
        u32x2 got;
        got[0] = (uint32_t)__builtin_amdgcn_mov_dpp((int)give[0], 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
        got[1] = (uint32_t)__builtin_amdgcn_mov_dpp((int)give[1], 0xB1, 0xF, 0xF, false);
        const u32x4 out = odd ? u32x4{got[0], got[1], keep[0], keep[1]} : u32x4{keep[0], keep[1], got[0], got[1]};
        // the pair's 32 bytes start at the even lane's 16: hi at +0, lo at +16
        *reinterpret_cast<u32x4*>(base + (c0 + u) * cstride) = out;
        st = st * d[u] + loc[u];
      }
    }
  }
  if (p.final_state) *reinterpret_cast<f32x4*>(p.final_state + (int64_t)bh * PN + 4 * (int64_t)v) = st;
}

}  // namespace

hipError_t launch_state_passing(const StatePassingArgs& a, int state_dtype, hipStream_t stream) {
  const int64_t PN = (int64_t)a.headdim * a.dstate;
  const int64_t all = (int64_t)a.batch * a.nheads;
  if (a.bh_begin < 0 || a.bh_count < 0 || a.bh_begin + (int64_t)a.bh_count > all) return hipErrorInvalidValue;
  const int64_t chains = a.bh_count > 0 ? a.bh_count : all - a.bh_begin;
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
