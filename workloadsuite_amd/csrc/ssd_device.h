// Device-side building blocks shared by the SSD kernels (gfx950 / CDNA4).
//
// MFMA fragments.  Every matrix product in this library is expressed with the
// 16x16 MFMA shape and an 8-element-per-lane operand fragment:
//   lane = 16*g + i  (g = lane group 0..3, i = 0..15)
//   A operand: lane holds A[row = i][k-slot (g, j)], j = 0..7
//   B operand: lane holds B[k-slot (g, j)][col = i]
//   D (f32x4): lane holds D[row = 4*g + jj][col = i], jj = 0..3
// For bf16/f16 one v_mfma_f32_16x16x32_{bf16,f16} consumes the fragment
// (k-slot (g, j) is K index 8*g + j); for f32 eight v_mfma_f32_16x16x4_f32
// consume it, instruction j pairing A and B slot (g, j) across the 4 lane
// groups.  Which logical index a k-slot stands for is the caller's choice, as
// long as the A and B fragments agree -- the kernels use that freedom to feed
// an MFMA result (D layout, 4 consecutive rows per lane) straight back in as
// an A operand without an LDS round trip.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssd {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

template <typename T> struct VecT;
template <> struct VecT<float> { typedef f32x8 v8; typedef f32x4 v4; };
template <> struct VecT<bf16> { typedef bf16x8 v8; typedef bf16x4 v4; };
template <> struct VecT<f16> { typedef f16x8 v8; typedef f16x4 v4; };
template <typename T> using frag8 = typename VecT<T>::v8;
template <typename T> using vec4 = typename VecT<T>::v4;

// ---------------------------------------------------------------------------
// MFMA wrappers: D += A * B over one 8-slot fragment.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f32x8 a, f32x8 b, f32x4 c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

// ---------------------------------------------------------------------------
// Conversions (round to nearest even).
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }
template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }

// chunk_state's weighted B^T operand as a hi + lo pair of T: v = b w,
// hi = T(v), lo = T(b w - float(hi)), the residual formed exactly by one
// fma.  Pairs of elements take one packed conversion each way (for bf16 hi's
// f32 value is read back from its bits): fewer instructions than converting
// one value at a time, same values.
// MIX (f16): the product b w is formed as an fma with an opaque -0 addend
// (the same value as the product; the compiler would turn a literal -0 back
// into a multiply), so that it takes the f16 b as it is (v_fma_mix_f32)
// instead of converting it first -- one register more, which the chunk-256
// state chain does not have to spare.
template <typename T, bool MIX = false>
__device__ __forceinline__ void split_weighted(const frag8<T>& b, f32x4 w0, f32x4 w1, frag8<T>& hi, frag8<T>& lo) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  constexpr bool kMix = MIX && std::is_same<T, f16>::value;
  float nz = -0.f;
  if constexpr (kMix) asm("" : "+v"(nz));
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const float wa = j < 4 ? w0[j] : w1[j - 4], wb = j < 4 ? w0[j + 1] : w1[j - 3];
    const float b0 = (float)b[j], b1 = (float)b[j + 1];
    const float v0 = kMix ? __builtin_fmaf(b0, wa, nz) : b0 * wa;
    const float v1 = kMix ? __builtin_fmaf(b1, wb, nz) : b1 * wb;
    const t2 h = __builtin_convertvector((f32x2{v0, v1}), t2);
    f32x2 hf;
    if constexpr (std::is_same<T, bf16>::value) {
      const uint32_t hu = __builtin_bit_cast(uint32_t, h);
      hf = f32x2{__uint_as_float(hu << 16), __uint_as_float(hu & 0xffff0000u)};
    } else {
      hf = __builtin_convertvector(h, f32x2);
    }
    const t2 l = __builtin_convertvector((f32x2{__builtin_fmaf(b0, wa, -hf[0]), __builtin_fmaf(b1, wb, -hf[1])}), t2);
    hi[j] = h[0];
    hi[j + 1] = h[1];
    lo[j] = l[0];
    lo[j + 1] = l[1];
  }
}

// Larger of two non-negative floats (magnitudes, or maxima of magnitudes)
// as an unsigned integer max of their bits: for non-negative IEEE values the
// order of the bit patterns is the numeric order, so a finite result is
// fmaxf's, without the quieting max(x, x) the compiler puts in front of
// fmaxf for a value read from memory or moved across lanes (a NaN, whose bits
// lie above infinity's, wins where fmaxf would drop it).
__device__ __forceinline__ float nn_max(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// Largest magnitude of v's elements (IEEE maximum: v_maximum3_f32 with abs
// modifiers, two instructions for four values; fmaxf on an MFMA result or an
// opaque value would quiet each input first, and it drops a NaN that
// maximum keeps).
__device__ __forceinline__ float abs_max4(f32x4 v) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(fabsf(v[0]), fabsf(v[1])),
                                       __builtin_elementwise_maximum(fabsf(v[2]), fabsf(v[3])));
}

// SSD_STATE_F16S_LOCAL: the f32 slot, within a [P][N] item, that holds the
// scale of row p's n tile t (columns 16 t .. 16 t + 15) -- the item's
// P x N/16 scales, in (p, t) order, packed into the second halves (unused by
// the f16 values) of its first rows.
template <int N> __device__ __forceinline__ int f16l_scale_slot(int p, int t) {
  const int k = p * (N / 16) + t;
  return (k / (N / 2)) * N + N / 2 + k % (N / 2);
}

template <typename T> __device__ __forceinline__ frag8<T> zero_frag() {
  frag8<T> z;
#pragma unroll
  for (int j = 0; j < 8; ++j) z[j] = (T)0.0f;
  return z;
}

// v if keep, else zeros (a per-lane select, no branch).
template <typename T> __device__ __forceinline__ frag8<T> select_frag(bool keep, frag8<T> v) {
  typedef uint32_t u32v __attribute__((ext_vector_type(sizeof(frag8<T>) / 4)));
  u32v w = __builtin_bit_cast(u32v, v);
#pragma unroll
  for (int j = 0; j < (int)(sizeof(frag8<T>) / 4); ++j) w[j] = keep ? w[j] : 0u;
  return __builtin_bit_cast(frag8<T>, w);
}

// 16-byte vector loads/stores.  p must be 16-byte aligned.
template <typename T> __device__ __forceinline__ frag8<T> load8(const T* p);
template <> __device__ __forceinline__ f32x8 load8<float>(const float* p) {
  f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
  f32x8 r;
  r.lo = lo;
  r.hi = hi;
  return r;
}
template <> __device__ __forceinline__ bf16x8 load8<bf16>(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
template <> __device__ __forceinline__ f16x8 load8<f16>(const f16* p) {
  return *reinterpret_cast<const f16x8*>(p);
}

template <typename T> __device__ __forceinline__ void store8(T* p, frag8<T> v);
template <> __device__ __forceinline__ void store8<float>(float* p, f32x8 v) {
  *reinterpret_cast<f32x4*>(p) = v.lo;
  *reinterpret_cast<f32x4*>(p + 4) = v.hi;
}
template <> __device__ __forceinline__ void store8<bf16>(bf16* p, bf16x8 v) {
  *reinterpret_cast<bf16x8*>(p) = v;
}
template <> __device__ __forceinline__ void store8<f16>(f16* p, f16x8 v) {
  *reinterpret_cast<f16x8*>(p) = v;
}

// 4-element load (8 bytes for 16-bit types, 16 bytes for f32); p aligned to that.
template <typename T> __device__ __forceinline__ vec4<T> load4(const T* p) {
  return *reinterpret_cast<const vec4<T>*>(p);
}
template <typename T> __device__ __forceinline__ void store4(T* p, vec4<T> v) {
  *reinterpret_cast<vec4<T>*>(p) = v;
}

template <typename T> __device__ __forceinline__ frag8<T> join(vec4<T> lo, vec4<T> hi) {
  frag8<T> r;
  r.lo = lo;
  r.hi = hi;
  return r;
}

// ---------------------------------------------------------------------------
// gfx950 LDS transfer primitives.
// ---------------------------------------------------------------------------
template <typename V> using lds_ptr = __attribute__((address_space(3))) V*;

// Transposing 8-byte LDS read (ds_read_b64_tr_b16).  Within each group of 16
// lanes, lane j returns element (j % 4) of the 8-byte chunks addressed by
// lanes 4r + j/4 of its group, r = 0..3.  So if lane k of a group addresses
// the 4 consecutive columns c0 + 4(k%4) .. +3 of row r0 + k/4 of a row-major
// 16-bit matrix, lane j receives column c0 + j of rows r0 .. r0+3: a 4 x 16
// block read transposed, as an MFMA operand wants it.
__device__ __forceinline__ bf16x4 lds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_ptr<bf16x4>)(const_cast<bf16*>(p)));
}
__device__ __forceinline__ f16x4 lds_read_tr(const f16* p) {
  typedef __fp16 fp16x4_builtin __attribute__((ext_vector_type(4)));  // the builtin's element type
  const fp16x4_builtin r =
      __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_ptr<fp16x4_builtin>)(const_cast<f16*>(p)));
  return __builtin_bit_cast(f16x4, r);
}

// Asynchronous global -> LDS copy (global_load_lds_dwordx4 / _dword): lane k
// reads 16 (or 4) bytes at its own global address g and the hardware writes
// them to lds_base + 16k (or + 4k); lds_base is taken from the first lane
// (it must be wave-uniform).  The copy is counted by vmcnt: wait with
// dma_wait() before the barrier that publishes the data.
//
// Issued through inline asm (M0 saved and restored around it) rather than
// __builtin_amdgcn_global_load_lds: the compiler then does not track the
// copy, and so cannot place conservative vmcnt(0) waits before unrelated LDS
// reads of the other buffer -- which would serialise the copy of the next
// work item with the compute of the current one.  The price is that the
// caller owns the wait.  Callers must not have compiler-issued global loads
// in flight alongside an outstanding copy (their partial vmcnt waits would
// not count it).
__device__ __forceinline__ uint32_t lds_offset(const void* lds) {
  return (uint32_t)(uintptr_t)(lds_ptr<const void>)lds;
}
// As dma16, with the LDS destination given as an LDS offset (lds_offset() of
// a __shared__ object plus a byte offset), wave-uniform.
__device__ __forceinline__ void dma16_at(const void* g, uint32_t lds_off) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_off))
      : "memory");
}
__device__ __forceinline__ void dma16(const void* g, void* lds_base) { dma16_at(g, lds_offset(lds_base)); }
__device__ __forceinline__ void dma4_at(const void* g, uint32_t lds_off) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_off))
      : "memory");
}
__device__ __forceinline__ void dma4(const void* g, void* lds_base) { dma4_at(g, lds_offset(lds_base)); }
// s_waitcnt vmcnt(0): every vector memory operation of this wave has completed.
__device__ __forceinline__ void dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt vmcnt(N): all but this wave's N most recent vector memory
// operations have completed (the count retires in issue order), e.g. copies
// issued before N stores, without waiting for the stores.
template <int N> __device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  // vmcnt is split over bits [3:0] and [15:14]
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// s_setprio with a value known after unrolling (the builtin takes an
// immediate).  Kernels whose waves meet at a barrier every item raise the
// priority of the waves that are behind in the item -- the hardware otherwise
// favours the oldest waves, and the youngest finish their item alone.
__device__ __forceinline__ void set_prio(int prio) {
  switch (prio) {
    case 3: __builtin_amdgcn_s_setprio(3); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    default: __builtin_amdgcn_s_setprio(0); break;
  }
}

// MFMA K slot j of lane group g stands for token 4 g + j (j < 4) or 16 + 4 g + j - 4
// (j >= 4) of a 32-token step: the rows a pair of transposing reads delivers.
__device__ __forceinline__ int slot_token(int g, int j) { return (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4)); }

// ---------------------------------------------------------------------------
// Workgroup -> tile mapping.  Hardware dispatches workgroup ids round-robin
// over the 8 XCDs (id % 8), each with its own L2.  The remap hands every XCD a
// contiguous range of logical tile ids, so tiles that share operands (the
// heads of one chunk share B and C when ngroups is small) meet in one L2.
// Bijective for any nblocks.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  const int per = nblocks / kXcds, rem = nblocks % kXcds;
  const int x = bid % kXcds, k = bid / kXcds;
  const int start = x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
  return start + k;
}

// ---------------------------------------------------------------------------
// Stage a ROWS x COLS tile of a row-major global matrix (unit column stride)
// into LDS transposed, dst[col * ldp + row], optionally scaling row r by
// scale[r] (an LDS or global array indexed from the tile's first row).
// Work unit: 4 rows x (16 / sizeof(T)) columns per thread -- one 16-byte load
// per row, one 4-element LDS store per column.  Requires ROWS % 4 == 0,
// COLS % (16 / sizeof(T)) == 0, ldp % 4 == 0 and 16-byte aligned rows.
// ---------------------------------------------------------------------------
template <typename T, int ROWS, int COLS, int NTHREADS>
__device__ __forceinline__ void stage_transposed(const T* __restrict__ src, int64_t row_stride,
                                                 T* __restrict__ dst, int ldp,
                                                 const float* scale, int tid) {
  constexpr int V = 16 / sizeof(T);
  constexpr int CU = COLS / V;
  constexpr int UNITS = (ROWS / 4) * CU;
#pragma unroll
  for (int u0 = 0; u0 < UNITS; u0 += NTHREADS) {
    const int u = u0 + tid;
    if (UNITS % NTHREADS == 0 || u < UNITS) {
      const int cu = u % CU, r4 = u / CU;
      const int row = 4 * r4, col = V * cu;
      float v[4][V];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const T* p = src + (int64_t)(row + rr) * row_stride + col;
        if constexpr (sizeof(T) == 4) {
          f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
          for (int k = 0; k < V; ++k) v[rr][k] = x[k];
        } else {
          frag8<T> x = load8<T>(p);
#pragma unroll
          for (int k = 0; k < V; ++k) v[rr][k] = to_f32<T>(x[k]);
        }
        if (scale) {
          const float s = scale[row + rr];
#pragma unroll
          for (int k = 0; k < V; ++k) v[rr][k] *= s;
        }
      }
#pragma unroll
      for (int k = 0; k < V; ++k) {
        vec4<T> o;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o[rr] = from_f32<T>(v[rr][k]);
        store4<T>(dst + (col + k) * ldp + row, o);
      }
    }
  }
}

// As stage_transposed, for 16-bit T, writing the scaled value v as two
// T-valued parts: hi = round(v) to dst_hi and lo = round(v - hi) to dst_lo.
// hi + lo carries ~16 significant bits, so an MFMA pair (hi, lo) against an
// exact 16-bit operand reproduces the f32-scaled product to ~2^-16 relative
// instead of the 2^-9 of a single rounding.
template <typename T, int ROWS, int COLS, int NTHREADS>
__device__ __forceinline__ void stage_transposed_split(const T* __restrict__ src, int64_t row_stride,
                                                       T* __restrict__ dst_hi, T* __restrict__ dst_lo,
                                                       int ldp, const float* scale, int tid) {
  static_assert(sizeof(T) == 2, "split staging is for 16-bit element types");
  constexpr int V = 8;
  constexpr int CU = COLS / V;
  constexpr int UNITS = (ROWS / 4) * CU;
#pragma unroll
  for (int u0 = 0; u0 < UNITS; u0 += NTHREADS) {
    const int u = u0 + tid;
    if (UNITS % NTHREADS == 0 || u < UNITS) {
      const int cu = u % CU, r4 = u / CU;
      const int row = 4 * r4, col = V * cu;
      float v[4][V];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const frag8<T> x = load8<T>(src + (int64_t)(row + rr) * row_stride + col);
        const float s = scale ? scale[row + rr] : 1.f;
#pragma unroll
        for (int k = 0; k < V; ++k) v[rr][k] = to_f32<T>(x[k]) * s;
      }
#pragma unroll
      for (int k = 0; k < V; ++k) {
        vec4<T> hi, lo;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          hi[rr] = from_f32<T>(v[rr][k]);
          lo[rr] = from_f32<T>(v[rr][k] - to_f32<T>(hi[rr]));
        }
        store4<T>(dst_hi + (col + k) * ldp + row, hi);
        store4<T>(dst_lo + (col + k) * ldp + row, lo);
      }
    }
  }
}

// Stage ROWS x COLS rows unchanged (dst[row * ldp + col]); columns >= ncols_valid
// are zero-filled (padding of the contraction dimension).
template <typename T, int ROWS, int COLS, int NTHREADS>
__device__ __forceinline__ void stage_rows(const T* __restrict__ src, int64_t row_stride,
                                           T* __restrict__ dst, int ldp, int ncols_valid, int tid) {
  constexpr int V = 16 / sizeof(T);
  constexpr int CU = COLS / V;
  constexpr int UNITS = ROWS * CU;
#pragma unroll
  for (int u0 = 0; u0 < UNITS; u0 += NTHREADS) {
    const int u = u0 + tid;
    if (UNITS % NTHREADS == 0 || u < UNITS) {
      const int cu = u % CU, row = u / CU;
      const int col = V * cu;
      if (col < ncols_valid) {
        const T* p = src + (int64_t)row * row_stride + col;
        if constexpr (sizeof(T) == 4) {
          *reinterpret_cast<f32x4*>(dst + row * ldp + col) = *reinterpret_cast<const f32x4*>(p);
        } else {
          store8<T>(dst + row * ldp + col, load8<T>(p));
        }
      } else {
        if constexpr (sizeof(T) == 4) {
          *reinterpret_cast<f32x4*>(dst + row * ldp + col) = f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
          store8<T>(dst + row * ldp + col, zero_frag<T>());
        }
      }
    }
  }
}

}  // namespace ssd
