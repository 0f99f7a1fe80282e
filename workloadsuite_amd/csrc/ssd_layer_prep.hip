// Pre-SSD prep of the Mamba-2 layer, x half: causal depthwise conv1d over the
// sequence, plus bias, then SiLU (workloads/mamba/model_ref.py:83-86):
//   y[b, l, d] = silu(bias[d] + sum_{j<k} w[d, j] x[b, l - (k-1) + j, d]),
//   x = 0 before l = 0,  silu(v) = v / (1 + e^-v)
// MR forms this as transpose -> nn.Conv1d(padding k-1) -> slice [:L] -> SiLU
// -> transpose; here it is one pass that reads x where in_proj left it (a
// strided slice of its output, channels contiguous) and writes the [b, L, h, P]
// operand K2 and K4 read (contiguous).  float32 accumulation and activation,
// one rounding to the output type.
//
// Each lane owns one 16-byte vector of channels (V of them) and walks a run
// of kRun consecutive tokens, keeping the k-1 previous rows of its channels
// in registers, so every input row is read once per run plus a (k-1)-row
// halo; a wave covers 64 adjacent vectors (1 KB of each row for 16-bit
// types).  HBM traffic: one read of x and one write of y, 4 bytes per element
// for 16-bit types -- memory bound.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kRun = 64;       // tokens per lane
constexpr int kBatchRows = 8;  // rows per batch; the next batch's loads are in flight during this one's math
constexpr int kWavesPerBlock = 4;

template <typename T, int V>
struct Row {
  T v[V];
};

template <typename T, int V>
__device__ __forceinline__ Row<T, V> load_row(const T* p) {
  Row<T, V> r;
  if constexpr (V * sizeof(T) == 16) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<u32x4*>(r.v) = *reinterpret_cast<const u32x4*>(p);
  } else {
#pragma unroll
    for (int e = 0; e < V; ++e) r.v[e] = p[e];
  }
  return r;
}

template <typename T, int V>
__device__ __forceinline__ void store_row(T* p, const Row<T, V>& r) {
  if constexpr (V * sizeof(T) == 16) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<u32x4*>(p) = *reinterpret_cast<const u32x4*>(r.v);
  } else {
#pragma unroll
    for (int e = 0; e < V; ++e) p[e] = r.v[e];
  }
}

__device__ __forceinline__ float silu(float v) {
  return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * v));
}

// grid: (channel vectors / 64 rounded up) x (runs / kWavesPerBlock rounded up) x batch
template <typename T, int V, int K>
__global__ __launch_bounds__(64 * kWavesPerBlock) void conv_silu_kernel(ConvArgs p) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar registers
  const int nvec = p.channels / V;
  const int cv = blockIdx.x * 64 + lane;
  const int run = blockIdx.y * kWavesPerBlock + wave;
  const int b = blockIdx.z;
  const int l0 = run * kRun;
  if (cv >= nvec || l0 >= p.seqlen) return;
  const int d0 = cv * V;

  float w[K][V], bias[V];
  {
    // the lane's V x K weights are contiguous: 16-byte loads where they fill them
    const T* wg = static_cast<const T*>(p.w) + (int64_t)d0 * K;
    const T* bg = static_cast<const T*>(p.bias);
    constexpr int WV = 16 / sizeof(T);
    if constexpr ((V * K) % WV == 0 && V * sizeof(T) == 16) {
#pragma unroll
      for (int q = 0; q < V * K / WV; ++q) {
        const Row<T, WV> r = load_row<T, WV>(wg + q * WV);
#pragma unroll
        for (int u = 0; u < WV; ++u) w[(q * WV + u) % K][(q * WV + u) / K] = to_f32<T>(r.v[u]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
#pragma unroll
        for (int j = 0; j < K; ++j) w[j][e] = to_f32<T>(wg[e * K + j]);
    }
#pragma unroll
    for (int e = 0; e < V; ++e) bias[e] = bg ? to_f32<T>(bg[d0 + e]) : 0.f;
  }
  const T* xg = static_cast<const T*>(p.x) + (int64_t)b * p.sxb + d0;
  T* yg = static_cast<T*>(p.y) + ((int64_t)b * p.seqlen) * p.channels + d0;

  // window[j] = row l - (K-1) + j for j < K-1 (zeros before the sequence start)
  float win[K > 1 ? K - 1 : 1][V];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int l = l0 - (K - 1) + j;
    if (l >= 0) {
      const Row<T, V> r = load_row<T, V>(xg + (int64_t)l * p.sxl);
#pragma unroll
      for (int e = 0; e < V; ++e) win[j][e] = to_f32<T>(r.v[e]);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) win[j][e] = 0.f;
    }
  }

  const int nrows = min(kRun, p.seqlen - l0);
  Row<T, V> nxt[kBatchRows];
  auto load_batch = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < kBatchRows; ++t)
      if (t0 + t < nrows) nxt[t] = load_row<T, V>(xg + (int64_t)(l0 + t0 + t) * p.sxl);
  };
  load_batch(0);
  for (int t0 = 0; t0 < nrows; t0 += kBatchRows) {
    Row<T, V> in[kBatchRows];
#pragma unroll
    for (int t = 0; t < kBatchRows; ++t) in[t] = nxt[t];
    if (t0 + kBatchRows < nrows) load_batch(t0 + kBatchRows);
#pragma unroll
    for (int t = 0; t < kBatchRows; ++t) {
      if (t0 + t >= nrows) break;
      Row<T, V> out;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float cur = to_f32<T>(in[t].v[e]);
        float acc = bias[e];
#pragma unroll
        for (int j = 0; j < K - 1; ++j) acc += w[j][e] * win[j][e];
        acc += w[K - 1][e] * cur;
        out.v[e] = from_f32<T>(silu(acc));
#pragma unroll
        for (int j = 0; j + 1 < K - 1; ++j) win[j][e] = win[j + 1][e];
        if constexpr (K > 1) win[K - 2][e] = cur;
      }
      store_row<T, V>(yg + (int64_t)(l0 + t0 + t) * p.channels, out);
    }
  }
}

template <typename T, int V>
hipError_t launch_tv(const ConvArgs& a, hipStream_t stream) {
  const int nvec = a.channels / V;
  const int runs = (a.seqlen + kRun - 1) / kRun;
  const dim3 grid((unsigned)((nvec + 63) / 64), (unsigned)((runs + kWavesPerBlock - 1) / kWavesPerBlock),
                  (unsigned)a.batch);
  const dim3 block(64 * kWavesPerBlock);
  switch (a.kwidth) {
    case 1: conv_silu_kernel<T, V, 1><<<grid, block, 0, stream>>>(a); break;
    case 2: conv_silu_kernel<T, V, 2><<<grid, block, 0, stream>>>(a); break;
    case 3: conv_silu_kernel<T, V, 3><<<grid, block, 0, stream>>>(a); break;
    case 4: conv_silu_kernel<T, V, 4><<<grid, block, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// 16-byte vectors when x rows, y rows, the weights and the channel count
// allow them, else one channel per lane.
template <typename T>
hipError_t launch_t(const ConvArgs& a, hipStream_t stream) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = a.channels % V == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15u) == 0 &&
                   (a.sxb * (int64_t)sizeof(T)) % 16 == 0 &&
                   (a.sxl * (int64_t)sizeof(T)) % 16 == 0;
  return vec ? launch_tv<T, V>(a, stream) : launch_tv<T, 1>(a, stream);
}

}  // namespace

hipError_t launch_conv_silu(const ConvArgs& a, int dtype, hipStream_t stream) {
  switch (dtype) {
    case SSD_DTYPE_F32: return launch_t<float>(a, stream);
    case SSD_DTYPE_BF16: return launch_t<bf16>(a, stream);
    case SSD_DTYPE_F16: return launch_t<f16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ssd
