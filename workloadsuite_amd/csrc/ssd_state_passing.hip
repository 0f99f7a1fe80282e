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
  const int bh = blockIdx.x / blocks_per_bh;  // b * nheads + h
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

}  // namespace

hipError_t launch_state_passing(const StatePassingArgs& a, int state_dtype, hipStream_t stream) {
  const int64_t PN = (int64_t)a.headdim * a.dstate;
  const int64_t blocks_per_bh = (PN / 4 + 255) / 256;
  const dim3 grid((unsigned)((int64_t)a.batch * a.nheads * blocks_per_bh));
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
