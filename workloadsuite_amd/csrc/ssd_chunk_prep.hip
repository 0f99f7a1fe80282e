// K0 -- chunk_prep: the per-(batch, chunk, group) register operands of the
// chunk-256 persistent kernels, computed once per group instead of on every
// CU that meets the group (there they cost a chain of dependent global loads
// before the first item can start).
//   cbf  CB^T[s, l] = C_l . B_s over the causal 16x16 sub-tiles
//        (workloads/mamba/model_ref.py:143, the C . B^T einsum), f32, in the
//        D-fragment order chunk_scan keeps in registers: wave w, step k
//        (row tile w's s block k for k < w/2 + 1, else row tile 15-w's s block
//        8-k), sub-tile st, lane.  Sub-tiles above the diagonal are 0.
//        With cb16 the same values are written rounded to T, [step][lane]
//        16 bytes (both sub-tiles), for chunk_scan's epilogue variant, which
//        holds CB^T in T.
//   btf  the B^T MFMA operands of chunk_state (MR:148 contracts over the
//        chunk's tokens): n tile nt, 32-token step ks, lane (g, i) holds
//        B[32 ks + slot_token(g, j)][16 nt + i] for j = 0..7.
// One workgroup per (b, c, g): B of the chunk is copied to LDS (rows
// XOR-swizzled by 16-byte piece so the 16 rows of an operand read hit
// distinct banks) and each wave loads the C rows of its two row tiles into
// registers; each wave then forms its CB^T blocks with the same MFMA
// sequence as chunk_scan's own fallback, so both give bit-identical values.
// 64 KB of LDS (N = 128) lets two workgroups share a CU.
//
// The forward launches K0 and K1 (ssd_cumsum_body.h) together: the first
// workgroups of the grid do two K1 blocks each (one per 256 threads), the
// rest K0, on the same LDS.  Both are short and independent; together they
// fill the GPU that K0's few workgroups alone leave mostly idle, and one
// kernel boundary goes away.
#include <cstdint>

#include "ssd_cumsum_body.h"
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kQ = 256;
constexpr int kNW = 8;
constexpr int kThreads = 64 * kNW;
constexpr int kNPair = kQ / 32 + 1;  // CB^T steps per wave (two row tiles)

template <int NK> constexpr int prep_lds_bytes() { return kQ * (64 * NK); }  // B rows

// K0 for group bcg = (b * nchunks + c) * ngroups + grp, on lds (prep_lds_bytes, 1 KB aligned).
template <typename T, int NK>
__device__ __forceinline__ void prep_body(const ChunkPrepArgs& p, int bcg, unsigned char* lds) {
  constexpr int N = 32 * NK;
  constexpr int RB = N * 2;      // bytes per B / C row
  constexpr int PPR = RB / 16;   // 16-byte pieces per row
  constexpr int RPD = 1024 / RB; // rows per 64-lane copy
  constexpr int NTILE = N / 16;
  unsigned char* bl = lds;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int g = lane >> 4, i = lane & 15;
  const int grp = bcg % p.ngroups, bc = bcg / p.ngroups;
  const int c = bc % p.nchunks, b = bc / p.nchunks;
  auto sw = [](int r) __attribute__((always_inline)) { return PPR >= 16 ? (r & 15) : ((r >> 1) & 7); };

  // ---- B of the chunk -> LDS (copy d moves rows RPD d .. RPD d + RPD - 1);
  // this wave's C rows straight into registers ----
  const int64_t l0 = (int64_t)c * kQ;
  const T* bg = reinterpret_cast<const T*>(p.bm) + (int64_t)b * p.sbb + l0 * p.sbl + (int64_t)grp * p.sbg;
  const T* cg = reinterpret_cast<const T*>(p.cm) + (int64_t)b * p.scb + l0 * p.scl + (int64_t)grp * p.scg;
  const uint32_t bl_lds = lds_offset(bl);
  for (int d = wave; d < kQ / RPD; d += kNW) {
    const int r = d * RPD + lane / PPR;
    const int piece = (lane % PPR) ^ sw(r);
    dma16_at(bg + (int64_t)r * p.sbl + 8 * piece, bl_lds + (uint32_t)(d * 1024));
  }
  const int ta = wave, tb = 15 - wave, KA = ta / 2 + 1;
  frag8<T> cf[2][NK];
#pragma unroll
  for (int kc = 0; kc < NK; ++kc) {
    cf[0][kc] = load8<T>(cg + (int64_t)(16 * ta + i) * p.scl + 8 * (4 * kc + g));
    cf[1][kc] = load8<T>(cg + (int64_t)(16 * tb + i) * p.scl + 8 * (4 * kc + g));
  }
  dma_wait();
  __syncthreads();

  // 8 consecutive elements (piece pc) of row r
  auto rd = [&](const unsigned char* base, int r, int pc) __attribute__((always_inline)) {
    return *reinterpret_cast<const frag8<T>*>(base + r * RB + 16 * (pc ^ sw(r)));
  };

  // ---- CB^T blocks of wave w's row tiles ta = w and tb = 15 - w ----
  f32x4* out = reinterpret_cast<f32x4*>(p.cbf) + (int64_t)(bcg * kNW + wave) * kNPair * 2 * 64 + lane;
#pragma unroll
  for (int k = 0; k < kNPair; ++k) {
    const bool first = k < KA;
    const int t = first ? ta : tb, sb = first ? k : kNPair - 1 - k;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) d = mma(rd(bl, 32 * sb + 16 * st + i, 4 * kc + g), first ? cf[0][kc] : cf[1][kc], d);
      const bool live = 2 * sb + st <= t;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) d[jj] = live ? d[jj] : 0.f;
      if (p.cb16) {
        // [k][lane] 16 bytes: sub-tile 0's 4 values, then sub-tile 1's, in T
        vec4<T>* o16 = reinterpret_cast<vec4<T>*>(p.cbf) + ((int64_t)(bcg * kNW + wave) * kNPair * 64 + lane) * 2;
        o16[k * 64 * 2 + st] = __builtin_convertvector(d, vec4<T>);
      } else {
        out[(k * 2 + st) * 64] = d;
      }
    }
  }

  // ---- B^T fragments of chunk_state, fragment f = nt * 8 + ks ----
  frag8<T>* bt_out = reinterpret_cast<frag8<T>*>(p.btf) + (int64_t)bcg * NTILE * 8 * 64 + lane;
  for (int f = wave; f < NTILE * 8; f += kNW) {
    const int nt = f / 8, ks = f % 8, n = 16 * nt + i;
    frag8<T> v;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 32 * ks + slot_token(g, j);
      v[j] = *reinterpret_cast<const T*>(bl + r * RB + 16 * ((n >> 3) ^ sw(r)) + 2 * (n & 7));
    }
    bt_out[f * 64] = v;
  }
}

template <typename T, int NK>
__global__ __launch_bounds__(kThreads) void chunk_prep_kernel(ChunkPrepArgs p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[prep_lds_bytes<NK>()];
  prep_body<T, NK>(p, blockIdx.x, lds);
}

// K0's B rows or two K1 tiles
template <int NK> constexpr int prologue_lds_bytes() {
  return prep_lds_bytes<NK>() > (int)(2 * sizeof(CumsumTile<kQ>)) ? prep_lds_bytes<NK>() : (int)(2 * sizeof(CumsumTile<kQ>));
}

// Two K1 blocks (chunk 256) per workgroup for the first nk1 workgroups, then
// K0.  K1's short, latency-bound blocks are dispatched first, so that they
// run beside K0's workgroups instead of after them when K0 fills the GPU.
template <typename T, int NK, typename R, bool RAW>
__global__ __launch_bounds__(kThreads) void chunk_prologue_kernel(ChunkPrepArgs p, CumsumArgs ca, int nk1) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[prologue_lds_bytes<NK>()];
  if ((int)blockIdx.x >= nk1) {
    prep_body<T, NK>(p, (int)blockIdx.x - nk1, lds);
    return;
  }
  const int half = threadIdx.x >> 8, t = threadIdx.x & 255;
  const int blk = 2 * (int)blockIdx.x + half;
  CumsumTile<kQ>& tile = *reinterpret_cast<CumsumTile<kQ>*>(lds + half * sizeof(CumsumTile<kQ>));
  const bool valid = blk < cumsum_blocks(ca);
  if (valid) cumsum_load<kQ, R, RAW>(ca, blk, t, tile);
  __syncthreads();
  if (valid) cumsum_scan<kQ>(ca, blk, t / kWave, t % kWave, tile);
}

template <typename T>
hipError_t launch_t(const ChunkPrepArgs& a, hipStream_t stream) {
  const unsigned grid = (unsigned)(a.batch * a.nchunks * a.ngroups);
  switch (a.dstate) {
    case 64: chunk_prep_kernel<T, 2><<<grid, kThreads, 0, stream>>>(a); break;
    case 128: chunk_prep_kernel<T, 4><<<grid, kThreads, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, typename R, bool RAW>
hipError_t launch_prologue_t(const ChunkPrepArgs& a, const CumsumArgs& ca, hipStream_t stream) {
  const int nprep = a.batch * a.nchunks * a.ngroups;
  const int nk1 = (cumsum_blocks(ca) + 1) / 2;
  const unsigned grid = (unsigned)(nprep + nk1);
  switch (a.dstate) {
    case 64: chunk_prologue_kernel<T, 2, R, RAW><<<grid, kThreads, 0, stream>>>(a, ca, nk1); break;
    case 128: chunk_prologue_kernel<T, 4, R, RAW><<<grid, kThreads, 0, stream>>>(a, ca, nk1); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

size_t chunk_prep_cb_bytes(int64_t groups) { return (size_t)groups * kNW * kNPair * 2 * 64 * sizeof(f32x4); }
size_t chunk_prep_bt_bytes(int64_t groups, int dstate) { return (size_t)groups * (dstate / 16) * 8 * 64 * 16; }

hipError_t launch_chunk_prep(const ChunkPrepArgs& a, int dtype, hipStream_t stream) {
  if (a.chunk != kQ) return hipErrorInvalidValue;
  if (dtype == SSD_DTYPE_BF16) return launch_t<bf16>(a, stream);
  if (dtype == SSD_DTYPE_F16) return launch_t<f16>(a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_chunk_prologue(const ChunkPrepArgs& a, const CumsumArgs& ca, int dtype, hipStream_t stream) {
  if (a.chunk != kQ || ca.chunk != kQ) return hipErrorInvalidValue;
  // the layer variant's raw dt has the inputs' type
  if (ca.dt_raw && ca.raw_dtype != dtype) return hipErrorInvalidValue;
  if (dtype == SSD_DTYPE_BF16)
    return ca.dt_raw ? launch_prologue_t<bf16, bf16, true>(a, ca, stream) : launch_prologue_t<bf16, float, false>(a, ca, stream);
  if (dtype == SSD_DTYPE_F16)
    return ca.dt_raw ? launch_prologue_t<f16, f16, true>(a, ca, stream) : launch_prologue_t<f16, float, false>(a, ca, stream);
  return hipErrorInvalidValue;
}

}  // namespace ssd
