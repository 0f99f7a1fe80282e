// K1's body (the intra-chunk cumsum of the log-decays and the chunk decay,
// workloads/mamba/model_ref.py:135-136, 150) as device functions on a
// caller-provided LDS tile, so that both K1's own kernel (ssd_cumsum.hip) and
// the forward's combined K1 + K0 launch (ssd_chunk_prep.hip) run the same code
// and give bit-identical results.
//
// One block of work = (batch, chunk, tile of kHeadTile heads), done by 256
// threads (4 waves): the [Q tokens x 16 heads] tile of A is read with 16
// consecutive heads per row segment and transposed through LDS; each wave
// then scans one head at a time: every lane sums Q/64 consecutive tokens
// serially, a wavefront inclusive scan of the lane totals (log2(64) shuffle
// steps) gives each lane its offset.
//
// Layer variant (RAW = true): the tile is formed from in_proj's raw dt
// instead of A (MR:94, 102-103): dt = softplus(dt_raw + dt_bias[h]) in
// float32 (written out, [b, L, h], for K2 / K4), A_dt = -exp(A_log[h]) dt.
#pragma once

#include "ssd_device.h"
#include "ssd_launch.h"

namespace ssd {

constexpr int kHeadTile = 16;

template <int Q> using CumsumTile = float[kHeadTile][Q + 1];

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

__host__ __device__ __forceinline__ int cumsum_blocks(const CumsumArgs& p) {
  return p.batch * p.nchunks * ((p.nheads + kHeadTile - 1) / kHeadTile);
}

// Phase 1 of block blk: the tile, by threads t = 0..255 (a barrier follows).
template <int Q, typename R, bool RAW>
__device__ __forceinline__ void cumsum_load(const CumsumArgs& p, int blk, int t, CumsumTile<Q>& tile) {
  const int htiles = (p.nheads + kHeadTile - 1) / kHeadTile;
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
    for (int e = t; e < Q * kHeadTile; e += 256) {
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
    for (int e = t; e < Q * kHeadTile; e += 256) {
      const int l = e / kHeadTile, hh = e % kHeadTile;
      tile[hh][l] = hh < nh ? src[(int64_t)l * p.sal + (int64_t)hh * p.sah] : 0.f;
    }
  }
}

// Phase 2 of block blk, after the barrier: wave w4 (0..3) scans heads w4, w4 + 4, ...
template <int Q>
__device__ __forceinline__ void cumsum_scan(const CumsumArgs& p, int blk, int w4, int lane, CumsumTile<Q>& tile) {
  constexpr int PER = Q / kWave;  // tokens per lane
  const int htiles = (p.nheads + kHeadTile - 1) / kHeadTile;
  const int ht = blk % htiles;
  blk /= htiles;
  const int c = blk % p.nchunks;
  const int b = blk / p.nchunks;
  const int h0 = ht * kHeadTile;
  const int nh = min(kHeadTile, p.nheads - h0);
  for (int hh = w4; hh < nh; hh += 4) {
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

}  // namespace ssd
