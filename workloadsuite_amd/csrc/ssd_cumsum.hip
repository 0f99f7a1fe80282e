// K1 -- chunk_cumsum: intra-chunk inclusive prefix sum of the log-decays and
// the per-chunk total decay.
//
// Replaces workloads/mamba/model_ref.py:135-136 (torch.cumsum over the chunk
// axis + rearrange to [b, c, h, l]) and MR:150 (chunk_decay = exp of the last
// cumsum).  Output layout: Acs [b, h, c, Q] contiguous along Q, the layout K2
// and K4 read.
//
// One workgroup (4 waves) per (batch, chunk, tile of 16 heads).  The tile of A
// [Q tokens x 16 heads] is read with 16 consecutive heads per row segment and
// transposed through LDS; each wave then scans one head at a time: every lane
// sums Q/64 consecutive tokens serially, a wavefront inclusive scan of the
// lane totals (DPP/permute shuffles, log2(64) steps) gives each lane its
// offset.  HBM traffic is one read of A and one write of Acs: memory bound,
// about 8 bytes per token and head.
//
// Layer variant (RAW = true): the tile is formed from in_proj's raw dt
// instead of A (MR:94, 102-103): dt = softplus(dt_raw + dt_bias[h]) in
// float32 (written out, [b, L, h], for K2 / K4), A_dt = -exp(A_log[h]) dt.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kHeadTile = 16;

__device__ __forceinline__ float wave_inclusive_scan(float v, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float t = __shfl_up(v, off, kWave);
    if (lane >= off) v += t;
  }
  return v;
}

// log(1 + e^v), and v itself above 20 (torch.nn.functional.softplus's
// default threshold, as MR:94 calls it)
__device__ __forceinline__ float softplus(float v) { return v > 20.f ? v : log1pf(expf(v)); }

template <int Q, typename R, bool RAW>
__global__ __launch_bounds__(256) void chunk_cumsum_kernel(CumsumArgs p) {
  constexpr int PER = Q / kWave;  // tokens per lane
  __shared__ float tile[kHeadTile][Q + 1];

  const int htiles = (p.nheads + kHeadTile - 1) / kHeadTile;
  int blk = blockIdx.x;
  const int ht = blk % htiles;
  blk /= htiles;
  const int c = blk % p.nchunks;
  const int b = blk / p.nchunks;
  const int h0 = ht * kHeadTile;
  const int nh = min(kHeadTile, p.nheads - h0);

  if constexpr (RAW) {
    const R* src = static_cast<const R*>(p.dt_raw) + (int64_t)b * p.srb + (int64_t)c * Q * p.srl + (int64_t)h0 * p.srh;
    const R* bias = static_cast<const R*>(p.dt_bias) + h0;
    float* dto = p.dt_out + ((int64_t)b * p.nchunks * Q + (int64_t)c * Q) * p.nheads + h0;
    for (int e = threadIdx.x; e < Q * kHeadTile; e += 256) {
      const int l = e / kHeadTile, hh = e % kHeadTile;
      float a = 0.f;
      if (hh < nh) {
        const float dt = softplus(to_f32<R>(src[(int64_t)l * p.srl + (int64_t)hh * p.srh]) + to_f32<R>(bias[hh]));
        dto[(int64_t)l * p.nheads + hh] = dt;
        a = -expf(p.a_log[h0 + hh]) * dt;
      }
      tile[hh][l] = a;
    }
  } else {
    const float* src = p.a + (int64_t)b * p.sab + (int64_t)c * Q * p.sal + (int64_t)h0 * p.sah;
    for (int e = threadIdx.x; e < Q * kHeadTile; e += 256) {
      const int l = e / kHeadTile, hh = e % kHeadTile;
      tile[hh][l] = hh < nh ? src[(int64_t)l * p.sal + (int64_t)hh * p.sah] : 0.f;
    }
  }
  __syncthreads();

  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int hh = wave; hh < nh; hh += 4) {
    float v[PER];
    float run = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      run += tile[hh][lane * PER + k];
      v[k] = run;
    }
    const float incl = wave_inclusive_scan(run, lane);
    float excl = __shfl_up(incl, 1, kWave);
    if (lane == 0) excl = 0.f;
    const int64_t bhc = ((int64_t)b * p.nheads + h0 + hh) * p.nchunks + c;
    float* dst = p.acs + bhc * Q + lane * PER;
#pragma unroll
    for (int k = 0; k < PER; ++k) dst[k] = v[k] + excl;
    if (lane == kWave - 1) p.decay[bhc] = expf(v[PER - 1] + excl);
  }
}

template <typename R, bool RAW>
hipError_t launch_q(const CumsumArgs& a, hipStream_t stream) {
  const int htiles = (a.nheads + kHeadTile - 1) / kHeadTile;
  const dim3 grid((unsigned)((int64_t)a.batch * a.nchunks * htiles));
  switch (a.chunk) {
    case 64: chunk_cumsum_kernel<64, R, RAW><<<grid, 256, 0, stream>>>(a); break;
    case 128: chunk_cumsum_kernel<128, R, RAW><<<grid, 256, 0, stream>>>(a); break;
    case 256: chunk_cumsum_kernel<256, R, RAW><<<grid, 256, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_chunk_cumsum(const CumsumArgs& a, hipStream_t stream) {
  if (!a.dt_raw) return launch_q<float, false>(a, stream);
  switch (a.raw_dtype) {
    case SSD_DTYPE_F32: return launch_q<float, true>(a, stream);
    case SSD_DTYPE_BF16: return launch_q<bf16, true>(a, stream);
    case SSD_DTYPE_F16: return launch_q<f16, true>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ssd
