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
#include "ssd_device.h"
#include "ssd_launch.h"

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

template <int Q>
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

  const float* src = p.a + (int64_t)b * p.sab + (int64_t)c * Q * p.sal + (int64_t)h0 * p.sah;
  for (int e = threadIdx.x; e < Q * kHeadTile; e += 256) {
    const int l = e / kHeadTile, hh = e % kHeadTile;
    tile[hh][l] = hh < nh ? src[(int64_t)l * p.sal + (int64_t)hh * p.sah] : 0.f;
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

}  // namespace

hipError_t launch_chunk_cumsum(const CumsumArgs& a, hipStream_t stream) {
  const int htiles = (a.nheads + kHeadTile - 1) / kHeadTile;
  const dim3 grid((unsigned)((int64_t)a.batch * a.nchunks * htiles));
  switch (a.chunk) {
    case 64: chunk_cumsum_kernel<64><<<grid, 256, 0, stream>>>(a); break;
    case 128: chunk_cumsum_kernel<128><<<grid, 256, 0, stream>>>(a); break;
    case 256: chunk_cumsum_kernel<256><<<grid, 256, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ssd
