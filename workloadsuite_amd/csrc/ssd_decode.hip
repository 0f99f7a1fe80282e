// Decode: one token of the SSD recurrence, in place on the [b, h, P, N] f32
// state that ssd_forward returns as its final state.  The per-token form of
// workloads/mamba/model_ref.py:152-161 (MR's chunk recurrence with a chunk
// of one token):
//   state[p, n] = exp(a) state[p, n] + dt x[p] B[n]
//   y[p]        = sum_n C[n] state[p, n]        (then the optional skip / gate)
//
// One workgroup (4 waves) per (batch, head); wave w owns state rows
// 16 w .. 16 w + 15.  A row of N f32 is spread over N/4 lanes (16 bytes
// each), so one wave instruction covers 64 / (N/4) rows; every lane keeps its
// 4 values of B and C in registers, and y[p] is a butterfly sum over the
// row's lanes.  The state is read and written once: 8 bytes per element,
// memory bound (the launch itself dominates at small batch x heads).
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;

template <typename T, int N>
__global__ __launch_bounds__(256) void decode_step_kernel(DecodeArgs p) {
  constexpr int LPR = N / 4;        // lanes per state row
  constexpr int RPI = 64 / LPR;     // rows per wave instruction
  constexpr int ITERS = 16 / RPI;   // instructions per wave (16 rows)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int bh = blockIdx.x;
  const int h = bh % p.nheads, b = bh / p.nheads;
  const int grp = h / (p.nheads / p.ngroups);
  const int n4 = 4 * (lane % LPR), rsub = lane / LPR;

  const T* bg = static_cast<const T*>(p.bm) + (int64_t)b * p.sbb + (int64_t)grp * p.sbg + n4;
  const T* cg = static_cast<const T*>(p.cm) + (int64_t)b * p.scb + (int64_t)grp * p.scg + n4;
  float bv[4], cv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    bv[k] = to_f32<T>(bg[k]);
    cv[k] = to_f32<T>(cg[k]);
  }
  const float da = expf(p.a[(int64_t)b * p.sab + (int64_t)h * p.sah]);
  const float dt = p.dt ? p.dt[(int64_t)b * p.sab + (int64_t)h * p.sah] : 1.f;
  const T* xg = static_cast<const T*>(p.x) + (int64_t)b * p.sxb + (int64_t)h * p.sxh;
  T* yg = static_cast<T*>(p.y) + (int64_t)b * p.syb + (int64_t)h * p.syh;
  float* sg = p.state + ((int64_t)b * p.nheads + h) * (int64_t)(kP * N);
  const float dsk = p.dskip ? p.dskip[h] : 0.f;
  const T* zg = p.z ? static_cast<const T*>(p.z) + (int64_t)b * p.szb + (int64_t)h * p.szh : nullptr;
  f32x4 st[ITERS];
  float xv[ITERS], zr[ITERS];

  // every load of the wave's rows first (ITERS 16-byte state loads in flight
  // per lane instead of one round trip per row), then the updates and stores.
  // The state streams through once per step: non-temporal loads and stores
  // (batch 256 at C3's head shape: 251 -> 227 us per step, batch 4 5.9 -> 5.6)
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int row = 16 * wave + RPI * it + rsub;
    st[it] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sg + row * N + n4));
    xv[it] = to_f32<T>(xg[row]);
    if (zg) zr[it] = to_f32<T>(zg[row]);
  }
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int row = 16 * wave + RPI * it + rsub;
    const float u = dt * xv[it];
    f32x4 ns;
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ns[k] = da * st[it][k] + u * bv[k];
      part += cv[k] * ns[k];
    }
    __builtin_nontemporal_store(ns, reinterpret_cast<f32x4*>(sg + row * N + n4));
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
    if (lane % LPR == 0) {
      float v = part + dsk * xv[it];
      if (zg) v *= zr[it] / (1.f + expf(-zr[it]));
      yg[row] = from_f32<T>(v);
    }
  }
}

template <typename T>
hipError_t launch_t(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.batch * a.nheads));
  switch (a.dstate) {
    case 16: decode_step_kernel<T, 16><<<grid, 256, 0, stream>>>(a); break;
    case 32: decode_step_kernel<T, 32><<<grid, 256, 0, stream>>>(a); break;
    case 64: decode_step_kernel<T, 64><<<grid, 256, 0, stream>>>(a); break;
    case 128: decode_step_kernel<T, 128><<<grid, 256, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_step(const DecodeArgs& a, int dtype, hipStream_t stream) {
  switch (dtype) {
    case SSD_DTYPE_F32: return launch_t<float>(a, stream);
    case SSD_DTYPE_BF16: return launch_t<bf16>(a, stream);
    case SSD_DTYPE_F16: return launch_t<f16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ssd
