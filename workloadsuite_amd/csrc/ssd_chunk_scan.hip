// K4 -- chunk_scan: fused intra-chunk (diagonal) and state-to-output
// (off-diagonal) terms on MFMA, writing y once.
//
// Replaces workloads/mamba/model_ref.py:139-145 (segsum decay L, causal mask,
// M = C.B^T, Y_diag = (L*M) X*dt), MR:160-161 (Y_off = exp(Acs) C.state) and
// MR:162 (Y_diag + Y_off):
//   y[l, p] = sum_{s<=l} exp(Acs[l]-Acs[s]) (C_l . B_s) dt[s] x[s, p]
//             + exp(Acs[l]) sum_n C[l, n] S_in[p, n]
// The [Q, Q] decay and C.B^T matrices never leave registers.
//
// Tiling.  One workgroup (4 waves) per (b, c, h).  The chunk's Q rows form
// Q/16 row tiles of 16; wave w owns the interleaved tiles w, w+4, w+8, ... so
// the causal triangle's work is balanced across waves.  Per wave:
//   * C fragments of its rows stay in registers for the whole chunk; they are
//     the A operand of C.S^T and the B operand of (C.B^T)^T.
//   * Y_off: D[l, p] = C[l, :] . S_in[p, :] from an LDS copy of S_in, then
//     each row is scaled by exp(Acs[l]).  For 16-bit inputs with f32 states,
//     S_in is staged as a hi + lo pair of the input type and both parts go
//     through the MFMA: the state keeps ~16 significant bits instead of the
//     8 of one bf16 rounding (the state is the largest term of y when the
//     decay is weak).
//   * Diagonal, 32 tokens s at a time (LDS-staged B rows and x^T with dt
//     folded in, shared by the 4 waves): the MFMA computes the transposed
//     block CB^T[s, l], whose D layout puts 4 consecutive s of one l in each
//     lane -- exactly an A-operand fragment of the next product once the
//     decay exp2(log2e (Acs[l]-Acs[s])) and the causal mask (s <= l, applied
//     by selection so positive log-decays above the diagonal cannot overflow
//     into inf*0) are applied and the values rounded to the input type.
//     Fully masked 16x16 blocks are skipped.
//   * y rows are written once, in the input dtype; the layer's skip D x and
//     gate silu(z) (MR:116-118), when given, are applied in float32 first.
// Workgroup ids are remapped so the heads of one chunk run on one XCD.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kSB = 32;  // tokens s per diagonal step

// f32 at d_state 128 with chunk 128 / 256 holds 64 / 128 VGPRs of C
// fragments alone: one workgroup per CU (one wave per SIMD, whose full
// register file the compiler may then use) instead of two, and no scratch.
template <typename T, int NK, int RT> constexpr int scan_blocks_per_cu() {
  return sizeof(T) == 4 && NK * RT >= 8 ? 1 : 2;
}

template <typename T, typename S, int NK, int RT>
__global__ __launch_bounds__(256, (scan_blocks_per_cu<T, NK, RT>())) void chunk_scan_kernel(ChunkScanArgs p) {
  constexpr int Q = 64 * RT;
  constexpr int NP = 32 * NK;                 // dstate padded to the MFMA K step
  constexpr int PAD = 16 / sizeof(T);
  constexpr int LDS_S = NP + PAD;             // S_in rows [p][n]
  constexpr int LDS_B = NP + PAD;             // B rows [s][n]
  constexpr int LDS_X = kSB + PAD;            // x^T rows [p][s]
  constexpr bool SPLIT = sizeof(T) == 2 && sizeof(S) == 4;
  __shared__ float acs_l[Q];                  // Acs * log2(e)
  __shared__ __attribute__((aligned(16))) T st_lds[kP * LDS_S];
  __shared__ __attribute__((aligned(16))) T st_lo_lds[SPLIT ? kP * LDS_S : 8];
  __shared__ __attribute__((aligned(16))) T bs_lds[kSB * LDS_B];
  __shared__ __attribute__((aligned(16))) T xt_lds[kP * LDS_X];
  __shared__ float dt_l[Q];

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int N = p.dstate;
  const int nblocks = p.batch * p.nchunks * p.nheads;
  const int blk = xcd_remap(blockIdx.x, nblocks);
  const int h = blk % p.nheads;
  const int bc = blk / p.nheads;
  const int c = bc % p.nchunks, b = bc / p.nchunks;
  const int grp = h / (p.nheads / p.ngroups);
  const int64_t l0 = (int64_t)c * Q;

  const T* xg = reinterpret_cast<const T*>(p.x) + b * p.sxb + l0 * p.sxl + h * p.sxh;
  const T* bg = reinterpret_cast<const T*>(p.bm) + b * p.sbb + l0 * p.sbl + grp * p.sbg;
  const T* cg = reinterpret_cast<const T*>(p.cm) + b * p.scb + l0 * p.scl + grp * p.scg;
  const float* acs = p.acs + (((int64_t)b * p.nheads + h) * p.nchunks + c) * Q;
  const S* sg = reinterpret_cast<const S*>(p.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * (kP * N);
  T* yg = reinterpret_cast<T*>(p.y) + b * p.syb + l0 * p.syl + h * p.syh;

  // ---- chunk-wide LDS: log2-scaled Acs, dt, S_in (as T, zero padded to NP) ----
  for (int q = tid; q < Q; q += 256) {
    acs_l[q] = acs[q] * kLog2e;
    dt_l[q] = p.dt ? p.dt[b * p.sdb + (l0 + q) * p.sdl + h * p.sdh] : 1.f;
  }
  for (int e = tid; e < kP * (NP / 4); e += 256) {
    const int pp = e / (NP / 4), n4 = 4 * (e % (NP / 4));
    vec4<T> o, lo;
    if (n4 < N) {
      const S* src = sg + pp * N + n4;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float v = (float)src[k];
        o[k] = from_f32<T>(v);
        lo[k] = from_f32<T>(v - to_f32<T>(o[k]));
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = lo[k] = (T)0.f;
    }
    store4<T>(st_lds + pp * LDS_S + n4, o);
    if constexpr (SPLIT) store4<T>(st_lo_lds + pp * LDS_S + n4, lo);
  }

  // ---- C fragments of this wave's row tiles (rows 16*t + i, t = wave + 4r) ----
  frag8<T> cf[RT][NK];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int row = 16 * (wave + 4 * r) + i;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) {
      const int n0 = 32 * kc + 8 * g;
      cf[r][kc] = n0 < N ? load8<T>(cg + row * p.scl + n0) : zero_frag<T>();
    }
  }
  __syncthreads();

  // ---- off-diagonal: acc[l, p] = exp(Acs[l]) * sum_n C[l, n] S_in[p, n] ----
  f32x4 acc[RT][4];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) acc[r][pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) {
      const frag8<T> sf = load8<T>(st_lds + (16 * pt + i) * LDS_S + 32 * kc + 8 * g);
#pragma unroll
      for (int r = 0; r < RT; ++r) acc[r][pt] = mma(cf[r][kc], sf, acc[r][pt]);
      if constexpr (SPLIT) {
        const frag8<T> sl = load8<T>(st_lo_lds + (16 * pt + i) * LDS_S + 32 * kc + 8 * g);
#pragma unroll
        for (int r = 0; r < RT; ++r) acc[r][pt] = mma(cf[r][kc], sl, acc[r][pt]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int t = wave + 4 * r;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float e = exp2f(acs_l[16 * t + 4 * g + jj]);
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) acc[r][pt][jj] *= e;
    }
  }

  // ---- diagonal: 32 tokens s per step ----
  for (int sb = 0; sb < Q / kSB; ++sb) {
    __syncthreads();
    stage_rows<T, kSB, NP, 256>(bg + (int64_t)(kSB * sb) * p.sbl, p.sbl, bs_lds, LDS_B, N, tid);
    stage_transposed<T, kSB, kP, 256>(xg + (int64_t)(kSB * sb) * p.sxl, p.sxl, xt_lds, LDS_X,
                                      p.dt ? dt_l + kSB * sb : nullptr, tid);
    __syncthreads();

    // Row tile t needs this step iff 32*sb <= 16*t + 15, i.e. sb <= t / 2.
    const int t_last = wave + 4 * (RT - 1);
    if (sb > t_last / 2) continue;  // wave-uniform

    frag8<T> bfr[2][NK];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int kc = 0; kc < NK; ++kc)
        bfr[st][kc] = load8<T>(bs_lds + (16 * st + i) * LDS_B + 32 * kc + 8 * g);
    frag8<T> xfr[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
      const T* rowp = xt_lds + (16 * pt + i) * LDS_X;
      xfr[pt] = join<T>(load4<T>(rowp + 4 * g), load4<T>(rowp + 16 + 4 * g));
    }

#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int t = wave + 4 * r;
      if (sb > t / 2) continue;  // wave-uniform
      const int l = 16 * t + i;   // this lane's column of CB^T
      const float al = acs_l[l];
      f32x4 cb[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        cb[st] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (kSB * sb + 16 * st <= 16 * t + 15) {  // not entirely above the diagonal
#pragma unroll
          for (int kc = 0; kc < NK; ++kc) cb[st] = mma(bfr[st][kc], cf[r][kc], cb[st]);
        }
      }
      frag8<T> af;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int s = kSB * sb + 16 * st + 4 * g + jj;
          const float v = s <= l ? cb[st][jj] * exp2f(al - acs_l[s]) : 0.f;
          af[4 * st + jj] = from_f32<T>(v);
        }
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) acc[r][pt] = mma(af, xfr[pt], acc[r][pt]);
    }
  }

  // ---- write y[l, p], with the layer's skip and gate (MR:116-118) when given ----
  const float dsk = p.dskip ? p.dskip[h] : 0.f;
  const T* zg = p.z ? reinterpret_cast<const T*>(p.z) + b * p.szb + l0 * p.szl + h * p.szh : nullptr;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int t = wave + 4 * r;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int64_t row = 16 * t + 4 * g + jj;
      T* yrow = yg + row * p.syl;
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        float v = acc[r][pt][jj];
        if (p.dskip) v += dsk * to_f32<T>(xg[row * p.sxl + 16 * pt + i]);
        if (zg) {
          const float zv = to_f32<T>(zg[row * p.szl + 16 * pt + i]);
          v *= zv / (1.f + expf(-zv));
        }
        yrow[16 * pt + i] = from_f32<T>(v);
      }
    }
  }
}

template <typename T, typename S, int NK>
hipError_t launch_q(const ChunkScanArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.batch * a.nchunks * a.nheads));
  switch (a.chunk) {
    case 64: chunk_scan_kernel<T, S, NK, 1><<<grid, 256, 0, stream>>>(a); break;
    case 128: chunk_scan_kernel<T, S, NK, 2><<<grid, 256, 0, stream>>>(a); break;
    case 256: chunk_scan_kernel<T, S, NK, 4><<<grid, 256, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, typename S>
hipError_t launch_t(const ChunkScanArgs& a, hipStream_t stream) {
  switch (a.dstate) {
    case 16:
    case 32: return launch_q<T, S, 1>(a, stream);
    case 64: return launch_q<T, S, 2>(a, stream);
    case 128: return launch_q<T, S, 4>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_chunk_scan(const ChunkScanArgs& a, int dtype, int state_dtype, hipStream_t stream) {
  if (chunk_scan_persistent_supported(a, dtype)) return launch_chunk_scan_persistent(a, dtype, state_dtype, stream);
  // f16s: also the 16-bit kernel at chunk 64 / 128; the hi/lo pairs: the persistent kernel only
  if (chunk_scan_b16_supported(a, dtype, state_dtype)) return launch_chunk_scan_b16(a, dtype, stream);
  if (a.f16s || a.presplit) return hipErrorInvalidValue;
  if (chunk_scan_f32_supported(a, dtype, state_dtype)) return launch_chunk_scan_f32(a, stream);
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
