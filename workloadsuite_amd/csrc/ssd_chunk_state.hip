// K2 -- chunk_state: per-chunk local state on MFMA.
//
// Replaces workloads/mamba/model_ref.py:144 (X * dt) and MR:148-149:
//   decay_to_end = exp(A_cumsum[..., -1:] - A_cumsum)
//   block_state  = einsum("bclhn, bchl, bclhp -> bchnp", B, decay_to_end, X*dt)
// computing, per (batch, chunk, head),
//   S[p, n] = sum_l (w[l] x[l, p]) B[l, n],   w[l] = exp(Acs[Q-1] - Acs[l]) dt[l]
// and storing it as states[b, c, h, p, n] (MR's [n, p] order transposed, so
// the state comes out in the [b, h, P, N] layout of the final state).
//
// One workgroup (4 waves) per (b, c, h); 5120 workgroups at the 2.7B layer
// shape.  The contraction runs over the chunk's tokens l, which is the strided
// axis of both x [l, p] and B [l, n] in HBM, so 64-token blocks of both are
// staged through LDS transposed (x^T with the decay weight folded in,
// B^T), giving each MFMA lane 8 consecutive tokens per 16-byte LDS read.
// Output tiles: 4 p-tiles x N/16 n-tiles of 16x16, split over the 4 waves.
// For 16-bit inputs the decay-weighted x is staged as a bf16/f16 hi + lo pair
// and both parts go through the MFMA against the exact B: the weighting is
// then carried to ~2^-16 relative instead of one 2^-9 rounding, at no cost in
// time because the kernel is bound by HBM, not by the doubled MFMA work.
// Arithmetic intensity at Q=256, N=128 is ~62 flop/byte (bf16 x in, f32 state
// out) against a bf16 ridge of ~315: HBM bound.  Workgroup ids are remapped so
// the heads of one chunk run on one XCD and share the B tile through its L2.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kLB = 64;  // tokens per staged block

template <typename T, typename S, int NT>
__global__ __launch_bounds__(256) void chunk_state_kernel(ChunkStateArgs p) {
  constexpr int N = 16 * NT;
  constexpr int PAD = 16 / sizeof(T);
  constexpr int LDP = kLB + PAD;
  constexpr bool SPLIT = sizeof(T) == 2;
  __shared__ float w_l[256];
  __shared__ __attribute__((aligned(16))) T xt[kP * LDP];
  __shared__ __attribute__((aligned(16))) T xt_lo[SPLIT ? kP * LDP : 8];
  __shared__ __attribute__((aligned(16))) T bt[N * LDP];

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int nblocks = p.batch * p.nchunks * p.nheads;
  const int blk = xcd_remap(blockIdx.x, nblocks);
  const int h = blk % p.nheads;
  const int bc = blk / p.nheads;
  const int c = bc % p.nchunks, b = bc / p.nchunks;
  const int grp = h / (p.nheads / p.ngroups);
  const int Q = p.chunk;
  const int64_t l0 = (int64_t)c * Q;

  const T* xg = reinterpret_cast<const T*>(p.x) + b * p.sxb + l0 * p.sxl + h * p.sxh;
  const T* bg = reinterpret_cast<const T*>(p.bm) + b * p.sbb + l0 * p.sbl + grp * p.sbg;
  const float* acs = p.acs + (((int64_t)b * p.nheads + h) * p.nchunks + c) * Q;

  const float last = acs[Q - 1];
  for (int l = tid; l < Q; l += 256) {
    float w = exp2f((last - acs[l]) * kLog2e);
    if (p.dt) w *= p.dt[b * p.sdb + (l0 + l) * p.sdl + h * p.sdh];
    w_l[l] = w;
  }

  constexpr int PTW = NT >= 2 ? 2 : 1;       // p-tiles per wave
  constexpr int NTW = NT >= 2 ? NT / 2 : 1;  // n-tiles per wave
  const int pt0 = NT >= 2 ? 2 * (wave & 1) : wave;
  const int nt0 = NT >= 2 ? (wave >> 1) * NTW : 0;

  f32x4 acc[PTW][NTW];
#pragma unroll
  for (int a = 0; a < PTW; ++a)
#pragma unroll
    for (int n = 0; n < NTW; ++n) acc[a][n] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int lb = 0; lb < Q; lb += kLB) {
    __syncthreads();
    if constexpr (SPLIT)
      stage_transposed_split<T, kLB, kP, 256>(xg + lb * p.sxl, p.sxl, xt, xt_lo, LDP, w_l + lb, tid);
    else
      stage_transposed<T, kLB, kP, 256>(xg + lb * p.sxl, p.sxl, xt, LDP, w_l + lb, tid);
    stage_transposed<T, kLB, N, 256>(bg + lb * p.sbl, p.sbl, bt, LDP, nullptr, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kLB / 32; ++ks) {
      frag8<T> af[PTW], bf[NTW];
#pragma unroll
      for (int a = 0; a < PTW; ++a) af[a] = load8<T>(xt + (16 * (pt0 + a) + i) * LDP + 32 * ks + 8 * g);
#pragma unroll
      for (int n = 0; n < NTW; ++n) bf[n] = load8<T>(bt + (16 * (nt0 + n) + i) * LDP + 32 * ks + 8 * g);
#pragma unroll
      for (int a = 0; a < PTW; ++a)
#pragma unroll
        for (int n = 0; n < NTW; ++n) acc[a][n] = mma(af[a], bf[n], acc[a][n]);
      if constexpr (SPLIT) {
#pragma unroll
        for (int a = 0; a < PTW; ++a) af[a] = load8<T>(xt_lo + (16 * (pt0 + a) + i) * LDP + 32 * ks + 8 * g);
#pragma unroll
        for (int a = 0; a < PTW; ++a)
#pragma unroll
          for (int n = 0; n < NTW; ++n) acc[a][n] = mma(af[a], bf[n], acc[a][n]);
      }
    }
  }

  S* sg = reinterpret_cast<S*>(p.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * (kP * N);
#pragma unroll
  for (int a = 0; a < PTW; ++a)
#pragma unroll
    for (int n = 0; n < NTW; ++n)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int pp = 16 * (pt0 + a) + 4 * g + jj, nn = 16 * (nt0 + n) + i;
        sg[pp * N + nn] = (S)acc[a][n][jj];
      }
}

template <typename T, typename S>
hipError_t launch_t(const ChunkStateArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.batch * a.nchunks * a.nheads));
  switch (a.dstate) {
    case 16: chunk_state_kernel<T, S, 1><<<grid, 256, 0, stream>>>(a); break;
    case 32: chunk_state_kernel<T, S, 2><<<grid, 256, 0, stream>>>(a); break;
    case 64: chunk_state_kernel<T, S, 4><<<grid, 256, 0, stream>>>(a); break;
    case 128: chunk_state_kernel<T, S, 8><<<grid, 256, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_chunk_state(const ChunkStateArgs& a, int dtype, int state_dtype, hipStream_t stream) {
  if (chunk_state_persistent_supported(a, dtype)) return launch_chunk_state_persistent(a, dtype, state_dtype, stream);
  if (chunk_state_f32_supported(a, dtype, state_dtype)) return launch_chunk_state_f32(a, dtype, stream);
  if (state_dtype == SSD_DTYPE_F32) {
    if (dtype == SSD_DTYPE_F32) return launch_t<float, float>(a, stream);
    if (dtype == SSD_DTYPE_BF16) return launch_t<bf16, float>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_t<f16, float>(a, stream);
  } else if (state_dtype == SSD_DTYPE_BF16) {
    if (dtype == SSD_DTYPE_BF16) return launch_t<bf16, bf16>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_t<f16, bf16>(a, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ssd
