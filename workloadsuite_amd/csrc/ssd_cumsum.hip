// K1 -- chunk_cumsum: intra-chunk inclusive prefix sum of the log-decays and
// the per-chunk total decay.
//
// Replaces workloads/mamba/model_ref.py:135-136 (torch.cumsum over the chunk
// axis + rearrange to [b, c, h, l]) and MR:150 (chunk_decay = exp of the last
// cumsum).  Output layout: Acs [b, h, c, Q] contiguous along Q, the layout K2
// and K4 read.  One workgroup (4 waves) per (batch, chunk, tile of 16 heads);
// the work itself is in ssd_cumsum_body.h, shared with the forward's combined
// K1 + K0 launch.  HBM traffic is one read of A and one write of Acs: memory
// bound, about 8 bytes per token and head.
#include "ssd_cumsum_body.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

template <int Q, typename R, bool RAW>
__global__ __launch_bounds__(256) void chunk_cumsum_kernel(CumsumArgs p) {
  __shared__ CumsumTile<Q> tile;
  cumsum_load<Q, R, RAW>(p, blockIdx.x, threadIdx.x, tile);
  __syncthreads();
  cumsum_scan<Q>(p, blockIdx.x, threadIdx.x / kWave, threadIdx.x % kWave, tile);
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
