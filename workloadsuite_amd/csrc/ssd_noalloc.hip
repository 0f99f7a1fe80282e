// ssd_forward_noalloc: the whole SSD forward with its workspace in a
// library-owned device array instead of a caller-provided buffer, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).  No counterpart in the
// reference (its forward allocates through PyTorch).
//
// The workspace (Acs, chunk decays, per-chunk states, chunk_prep's operands)
// lives in `scratch`, a file-scope __device__ array of kScratchBytes.  Each
// device the library runs on holds its own copy, from the code object's load
// until the process ends.  Host code never passes `scratch` itself to a
// kernel (on the host the name is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, taken once per device with
// that device current and cached here.
//
// The array lives in the code object's data segment: it is reserved on every
// device where libssd's code object loads, from then until the process ends,
// whether or not this entry point is ever called.
//
// When one call's workspace does not fit, the batch is processed in slices
// whose workspace does; a shape whose single batch element needs more than
// kScratchBytes is rejected (SSD_ERR_WORKSPACE_TOO_SMALL) before anything is
// launched.  Nothing in the workspace has to start at zero: every region is
// written before it is read within a call.  All calls on one device share
// that device's array, so calls that overlap on one device (other streams,
// other host threads) race; callers serialise them.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <vector>

#include "../../include/ssd.h"

namespace {

constexpr size_t kScratchBytes = size_t(256) << 20;  // SSD_NOALLOC_SCRATCH_BYTES

__device__ __align__(256) unsigned char scratch[kScratchBytes];

static_assert(kScratchBytes == SSD_NOALLOC_SCRATCH_BYTES, "header and library agree on the scratch size");

std::mutex g_mu;
std::vector<void*> g_ptr;  // per device id: scratch's device address, or null before the first call

// scratch's address on the current device (looked up on the first call per device).
int scratch_of_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lock(g_mu);
  if (dev < 0) return (int)hipErrorInvalidDevice;
  if ((size_t)dev >= g_ptr.size()) g_ptr.resize((size_t)dev + 1, nullptr);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return SSD_OK;
}

size_t elem_bytes(int dtype) { return dtype == SSD_DTYPE_F32 ? 4 : 2; }

template <typename T>
T* advance(T* p, int64_t elems, size_t es) {
  return p ? reinterpret_cast<T*>(reinterpret_cast<uintptr_t>(p) + (uintptr_t)(elems * (int64_t)es)) : p;
}

}  // namespace

extern "C" int ssd_forward_noalloc(const ssd_dims* d, int dtype, const void* x, const int64_t x_strides[4],
                                   const float* a, const int64_t a_strides[3], const void* bmat,
                                   const int64_t b_strides[4], const void* cmat, const int64_t c_strides[4],
                                   const float* dt, const int64_t dt_strides[3], const float* initial_states,
                                   void* y, const int64_t y_strides[4], float* final_states, int state_dtype,
                                   void* stream) {
  int rc = ssd_check_dims(d, dtype);
  if (rc) return rc;
  if (!x || !x_strides || !a || !a_strides || !bmat || !b_strides || !cmat || !c_strides || !y || !y_strides ||
      (dt && !dt_strides))
    return SSD_ERR_NULL_POINTER;
  // the chunk ssd_forward runs at (the routing depends on the shape's ratios,
  // not on the batch; every slice below is run at it explicitly)
  ssd_dims e = *d;
  e.chunk = ssd_forward_chunk(d, dtype, state_dtype);
  if (e.chunk == 0) return SSD_ERR_UNSUPPORTED_DTYPE;
  d = &e;
  const size_t need = ssd_workspace_bytes(d, state_dtype);
  if (need == 0) return SSD_ERR_UNSUPPORTED_DTYPE;
  // the largest batch slice whose workspace fits
  int64_t slice = d->batch;
  ssd_dims sd = *d;
  if (need > kScratchBytes) {
    sd.batch = 1;
    const size_t one = ssd_workspace_bytes(&sd, state_dtype);
    if (one == 0 || one > kScratchBytes) return SSD_ERR_WORKSPACE_TOO_SMALL;
    slice = 1;
    while (slice < d->batch) {
      sd.batch = slice + 1;
      if (ssd_workspace_bytes(&sd, state_dtype) > kScratchBytes) break;
      ++slice;
    }
  }
  void* ws = nullptr;
  if ((rc = scratch_of_current_device(&ws))) return rc;
  const size_t es = elem_bytes(dtype);
  const int64_t PN = d->headdim * d->dstate;
  for (int64_t b0 = 0; b0 < d->batch; b0 += slice) {
    sd = *d;
    sd.batch = b0 + slice <= d->batch ? slice : d->batch - b0;
    // every operand is indexed from its batch element b0 by its batch stride;
    // initial / final states are contiguous [b, h, P, N]
    rc = ssd_forward(&sd, dtype, advance(x, b0 * x_strides[0], es), x_strides, advance(a, b0 * a_strides[0], 4),
                     a_strides, advance(bmat, b0 * b_strides[0], es), b_strides,
                     advance(cmat, b0 * c_strides[0], es), c_strides,
                     dt ? advance(dt, b0 * dt_strides[0], 4) : nullptr, dt_strides,
                     advance(initial_states, b0 * d->nheads * PN, 4), advance(y, b0 * y_strides[0], es), y_strides,
                     advance(final_states, b0 * d->nheads * PN, 4), ws, kScratchBytes, state_dtype, stream);
    if (rc) return rc;
  }
  return SSD_OK;
}
