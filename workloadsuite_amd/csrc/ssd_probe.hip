// Streaming probes: the HBM rate this device reaches for a given read / write
// mix and access width, the ceiling against which the state-passing kernel
// (K3) is judged.  A measurement aid for bench.py --hbm-probe, built into
// libssd_probe.so; no counterpart in the reference and not part of the SSD
// forward's ABI (include/ssd.h).
//
// K3 with f32 local states and the f16s hand-over reads 4 bytes and writes 2
// bytes per state (plus a 4-byte scale per 128-state row): reads : writes =
// 2 : 1.  The probe reads n_read f32 (16-byte loads, plain or non-temporal)
// and writes one f16 per f32 read (the value rounded), so its traffic has
// K3's mix.  kind:
//   0  16-byte loads, 8-byte stores (one f16x4 per load; K3's own widths)
//   1  16-byte loads, 16-byte stores (one f16x8 per two loads)
//   2  copy: 16-byte loads, 16-byte stores of the same f32 values (1 : 1)
// flags: bit 0 non-temporal loads, bit 1 non-temporal stores, bit 2 eight
// independent 16-byte vectors per thread per iteration (else four).
// Grid-stride over 16-byte vectors; n_read a multiple of 8, base pointers
// 16-byte aligned (checked on the host).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ssd_device.h"

namespace {

using ssd::f16;
using ssd::f16x4;
using ssd::f16x8;
using ssd::f32x4;

template <bool NT>
__device__ __forceinline__ f32x4 ld(const f32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}

template <bool NT, typename V>
__device__ __forceinline__ void st(V* p, V v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <int KIND, bool NT, bool NTS, int UNROLL>
__global__ __launch_bounds__(256) void stream_probe_kernel(const float* __restrict__ src, void* __restrict__ dst,
                                                           int64_t nvec) {
  const f32x4* s = reinterpret_cast<const f32x4*>(src);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (KIND == 1) {
    // pairs of 16-byte vectors -> one 16-byte f16x8 store
    const int64_t npair = nvec / 2;
    f16x8* d = reinterpret_cast<f16x8*>(dst);
    for (int64_t base = t0; base < npair; base += stride * UNROLL) {
      f32x4 a[UNROLL], b[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t k = base + u * stride;
        if (k < npair) {
          a[u] = ld<NT>(s + 2 * k);
          b[u] = ld<NT>(s + 2 * k + 1);
        }
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t k = base + u * stride;
        if (k < npair) {
          f16x8 o;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            o[j] = (f16)a[u][j];
            o[4 + j] = (f16)b[u][j];
          }
          st<NTS>(d + k, o);
        }
      }
    }
  } else {
    for (int64_t base = t0; base < nvec; base += stride * UNROLL) {
      f32x4 a[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t k = base + u * stride;
        if (k < nvec) a[u] = ld<NT>(s + k);
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t k = base + u * stride;
        if (k < nvec) {
          if constexpr (KIND == 0) {
            f16x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = (f16)a[u][j];
            st<NTS>(reinterpret_cast<f16x4*>(dst) + k, o);
          } else {
            st<NTS>(reinterpret_cast<f32x4*>(dst) + k, a[u]);
          }
        }
      }
    }
  }
}

template <int KIND, bool NT, bool NTS>
hipError_t launch(const float* src, void* dst, int64_t nvec, int blocks, bool u8, hipStream_t s) {
  if (u8) stream_probe_kernel<KIND, NT, NTS, 8><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(src, dst, nvec);
  else stream_probe_kernel<KIND, NT, NTS, 4><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(src, dst, nvec);
  return hipGetLastError();
}

template <int KIND>
hipError_t launch_kind(const float* src, void* dst, int64_t nvec, int blocks, int flags, hipStream_t s) {
  const bool u8 = flags & 4;
  switch (flags & 3) {
    case 0: return launch<KIND, false, false>(src, dst, nvec, blocks, u8, s);
    case 1: return launch<KIND, true, false>(src, dst, nvec, blocks, u8, s);
    case 2: return launch<KIND, false, true>(src, dst, nvec, blocks, u8, s);
    default: return launch<KIND, true, true>(src, dst, nvec, blocks, u8, s);
  }
}

}  // namespace

// src: n_read f32 (16-byte aligned); dst: n_read f16 for kinds 0 / 1, n_read
// f32 for kind 2 (16-byte aligned).  blocks: workgroups of 256 threads (0: 8
// per CU).  Returns 0, -1 for invalid arguments, or a hipError_t.
extern "C" int ssd_stream_probe(const float* src, void* dst, int64_t n_read, int kind, int flags, int blocks,
                                void* stream) {
  if (!src || !dst || n_read <= 0 || n_read % 8 != 0 || kind < 0 || kind > 2 || blocks < 0 || flags < 0 || flags > 7)
    return -1;
  if ((reinterpret_cast<uintptr_t>(src) & 15u) || (reinterpret_cast<uintptr_t>(dst) & 15u)) return -1;
  if (blocks == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return -1;
    blocks = 8 * cus;
  }
  const int64_t nvec = n_read / 4;
  const hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (kind == 0) e = launch_kind<0>(src, dst, nvec, blocks, flags, s);
  else if (kind == 1) e = launch_kind<1>(src, dst, nvec, blocks, flags, s);
  else e = launch_kind<2>(src, dst, nvec, blocks, flags, s);
  return e == hipSuccess ? 0 : (int)e;
}
