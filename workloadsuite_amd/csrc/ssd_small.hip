// The whole SSD forward in one launch for small states and short chains
// (d_state 16 / 32, chunk 64 / 128, a few chunks per chain; C1 is 16 x 8
// chains of 2 chunks at d_state 16): one workgroup of 4 waves per (b, h)
// chain walks its chunks in order with the chunk's operands, the decay table
// and the running state in LDS, all arithmetic in f32.  Per chunk, as K1-K4
// compute it (workloads/mamba/model_ref.py:135-162):
//   Acs[l]   = sum_{k<=l} A[k]                    (MR:135-136; K1's scan order)
//   W[l][s]  = exp(Acs[l] - Acs[s]) dt[s] (C_l . B_s) for s <= l, else 0
//                                                 (MR:139-144; 0 by selection above the diagonal)
//   y[l][p]  = sum_{s<=l} W[l][s] x[s][p] + exp(Acs[l]) sum_n C[l][n] S[p][n]
//                                                 (MR:145, 160-162)
//   S[p][n] <- exp(Acs[Q-1]) S[p][n] + sum_l x[l][p] dt[l] exp(Acs[Q-1] - Acs[l]) B[l][n]
//                                                 (MR:148-157)
// with S the state entering the chunk (the initial state, or zero, first),
// and the state after the last chunk to final_state.  One launch and no
// workspace traffic, where the four-kernel path would spend most of its time
// in launch gaps: at these shapes each kernel moves a few MB.
//
// Each chunk: the next chunk's x, B, C, A and dt are loaded into registers
// while the current one computes (issued after the scan), and written to LDS
// (as f32, x transposed) after it.  The three products run on f32 MFMAs
// (v_mfma_f32_16x16x4f32, 16 x 16 tiles, K in blocks of 16: lane (g, i) of
// instruction j supplies A[i][4 g + j] and B[4 g + j][i], read as one 16-byte
// piece per operand and block; D holds rows 4 g + jj, column i):
//   W = C.B^T on the causal 16 x 16 tiles, then the decay and the mask;
//   y = W.x (over s, causal blocks only) + exp(Acs) (C.S^T), wave w taking
//       row tiles w and Q/16 - 1 - w (equal causal work);
//   S = exp(Acs[Q-1]) S + x^T.Bw, Bw = B exp(Acs[Q-1] - Acs) dt.
#include <climits>

#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kT = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A 16-byte piece of T as floats (4 for f32, 8 for 16-bit types).
template <typename T>
__device__ __forceinline__ void unpack(u32x4 raw, float* out) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = __uint_as_float(raw[k]);
  } else {
    const frag8<T> v = __builtin_bit_cast(frag8<T>, raw);
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = to_f32<T>(v[k]);
  }
}

__device__ __forceinline__ f32x4 mfma4(f32x4 a, f32x4 b, f32x4 c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

// PS workgroups per chain, each taking kP / PS of the head dimension (p) for
// y and the state (C.B^T is formed by each): PS = 2 where the chains alone
// would leave CUs idle.
template <typename T, int N, int Q, int PS>
__global__ __launch_bounds__(kT) void ssd_small_kernel(SmallArgs p) {
  constexpr int PP = kP / PS;                         // p columns of this workgroup
  constexpr int QT = PP / 16;                         // p tiles
  constexpr int VPP = 16 / (int)sizeof(T);            // values per 16-byte piece
  constexpr int XPR = PP / VPP;                       // pieces per x row (this workgroup's columns)
  constexpr int XPT = Q * XPR / kT;                   // x pieces per thread
  constexpr int BPR = N / VPP;                        // pieces per B / C row
  constexpr int BPT = (Q * BPR + kT - 1) / kT;        // B (and C) pieces per thread (the last partly idle)
  constexpr int R = Q / 16;                           // 16-row tiles of the chunk
  constexpr int QS = Q + 4, NS = N + 4;               // padded LDS row strides (16-byte aligned)
  constexpr int PER = Q / kWave;                      // scan: tokens per lane
  constexpr int NT = N / 16;                          // n tiles
  static_assert(XPT * kT == Q * XPR && (R == 4 || R == 8) && (QT == 2 || QT == 4), "thread mappings");

  __shared__ __attribute__((aligned(16))) float xt[PP][QS];   // x transposed [p][l] (this workgroup's p)
  __shared__ __attribute__((aligned(16))) float bs[Q][NS];    // B [s][n]
  __shared__ __attribute__((aligned(16))) float cs[Q][NS];    // C [l][n]
  __shared__ __attribute__((aligned(16))) float bwt[N][QS];   // (B exp(Acs[Q-1] - Acs) dt) transposed [n][l]
  __shared__ __attribute__((aligned(16))) float wl[Q][QS];    // W [l][s] (0 above the diagonal)
  __shared__ __attribute__((aligned(16))) float ss[PP][NS];   // the state entering the chunk [p][n] (its p)
  __shared__ __attribute__((aligned(16))) float araw[Q], dts[Q], acl[Q], wend[Q];  // A, dt, Acs log2(e), end weights

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int bh = blockIdx.x / PS, pc0 = PP * (blockIdx.x % PS);  // chain, first p column
  const int h = bh % p.nheads, b = bh / p.nheads;
  const int grp = h / (p.nheads / p.ngroups);
  const T* xg = static_cast<const T*>(p.x) + b * p.sxb + h * p.sxh + pc0;
  const T* bg = static_cast<const T*>(p.bm) + b * p.sbb + grp * p.sbg;
  const T* cg = static_cast<const T*>(p.cm) + b * p.scb + grp * p.scg;
  const float* ag = p.a + b * p.sab + h * p.sah;
  const float* dg = p.dt ? p.dt + b * p.sdb + h * p.sdh : nullptr;

  // ---- one chunk's operands: global -> registers -> LDS ----
  u32x4 xr[XPT], br[BPT], cr[BPT];
  float ar = 0.f, dr = 1.f;
  auto fetch = [&](int c) __attribute__((always_inline)) {
    const int64_t l0 = (int64_t)c * Q;
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int e = t + kT * k, r = e / XPR, q = e % XPR;
      xr[k] = *reinterpret_cast<const u32x4*>(xg + (l0 + r) * p.sxl + VPP * q);
    }
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      const int e = t + kT * k, r = e / BPR, q = e % BPR;
      if (e < Q * BPR) {
        br[k] = *reinterpret_cast<const u32x4*>(bg + (l0 + r) * p.sbl + VPP * q);
        cr[k] = *reinterpret_cast<const u32x4*>(cg + (l0 + r) * p.scl + VPP * q);
      }
    }
    if (t < Q) {
      ar = ag[(l0 + t) * p.sal];
      dr = dg ? dg[(l0 + t) * p.sdl] : 1.f;
    }
  };
  auto stage = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int e = t + kT * k, r = e / XPR, q = e % XPR;
      float v[VPP];
      unpack<T>(xr[k], v);
#pragma unroll
      for (int j = 0; j < VPP; ++j) xt[VPP * q + j][r] = v[j];
    }
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      const int e = t + kT * k, r = e / BPR, q = e % BPR;
      if (e < Q * BPR) {
        float v[VPP], u[VPP];
        unpack<T>(br[k], v);
        unpack<T>(cr[k], u);
#pragma unroll
        for (int j = 0; j < VPP; j += 4) {
          *reinterpret_cast<f32x4*>(&bs[r][VPP * q + j]) = f32x4{v[j], v[j + 1], v[j + 2], v[j + 3]};
          *reinterpret_cast<f32x4*>(&cs[r][VPP * q + j]) = f32x4{u[j], u[j + 1], u[j + 2], u[j + 3]};
        }
      }
    }
    if (t < Q) {
      araw[t] = ar;
      dts[t] = dr;
    }
  };
  auto ld4 = [](const float* q) __attribute__((always_inline)) { return *reinterpret_cast<const f32x4*>(q); };

  // ---- the state entering the first chunk ----
  const bool init = p.init != nullptr;
  for (int e = t; e < PP * N; e += kT) {
    const int pp = e / N, n = e % N;
    ss[pp][n] = init ? p.init[(int64_t)bh * kP * N + (int64_t)pc0 * N + e] : 0.f;
  }
  bool has_state = init;  // workgroup-uniform: S != 0 (else the off-diagonal term is skipped)

  fetch(0);
  stage();
  __syncthreads();
  for (int c = 0; c < p.nchunks; ++c) {
    // Acs as K1 scans it: PER consecutive tokens per lane, then a wavefront
    // scan of the lane totals; kept times log2(e) for exp2
    if (wave == 0) {
      float v[PER];
      float run = 0.f;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        run += araw[lane * PER + k];
        v[k] = run;
      }
      float incl = run;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const float u = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += u;
      }
      float excl = __shfl_up(incl, 1, kWave);
      if (lane == 0) excl = 0.f;
      const float last = __shfl(v[PER - 1] + excl, kWave - 1, kWave) * kLog2e;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int l = lane * PER + k;
        const float al = (v[k] + excl) * kLog2e;
        acl[l] = al;
        wend[l] = exp2f(last - al) * dts[l];
      }
    }
    __syncthreads();
    if (c + 1 < p.nchunks) fetch(c + 1);  // lands while this chunk computes

    // W on the causal 16 x 16 tiles (row tile r, column tile cc <= r): C.B^T
    // over n, then exp(Acs[l] - Acs[s]) dt[s]; above the diagonal the entries
    // are 0 by selection, so an exponent that overflows there (positive
    // log-decays) is discarded, never multiplied into W
    for (int tau = wave; tau < R * (R + 1) / 2; tau += 4) {
      int r = 0;
      while ((r + 1) * (r + 2) / 2 <= tau) ++r;
      const int cc = tau - r * (r + 1) / 2;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int nb = 0; nb < NT; ++nb)
        acc = mfma4(ld4(&cs[16 * r + i][16 * nb + 4 * g]), ld4(&bs[16 * cc + i][16 * nb + 4 * g]), acc);
      const int s = 16 * cc + i;
      const float as = acl[s], ds = dts[s];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int l = 16 * r + 4 * g + jj;
        wl[l][s] = s <= l ? acc[jj] * exp2f(acl[l] - as) * ds : 0.f;
      }
    }
    // B weighted to the chunk end, transposed, for the state update
    for (int e = t; e < Q * N; e += kT) {
      const int l = e / N, n = e % N;
      bwt[n][l] = bs[l][n] * wend[l];
    }
    __syncthreads();

    // y: row tiles w and R - 1 - w; with R = 4 the two waves of a row-tile
    // pair split the workgroup's QT column tiles (p) between them
    {
      T* yg = static_cast<T*>(p.y) + b * p.syb + h * p.syh + ((int64_t)c * Q) * p.syl + pc0;
      constexpr int QPW = R == 4 ? QT / 2 : QT;  // p tiles per (wave, row tile)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int r = half ? R - 1 - wave : wave;
        const int q0 = R == 4 ? QPW * half : 0;
        f32x4 acc[QPW], off[QPW];
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) acc[qq] = off[qq] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int sb = 0; sb <= r; ++sb) {
          const f32x4 wv = ld4(&wl[16 * r + i][16 * sb + 4 * g]);
#pragma unroll
          for (int qq = 0; qq < QPW; ++qq) acc[qq] = mfma4(wv, ld4(&xt[16 * (q0 + qq) + i][16 * sb + 4 * g]), acc[qq]);
        }
        if (has_state) {
#pragma unroll
          for (int nb = 0; nb < NT; ++nb) {
            const f32x4 cv = ld4(&cs[16 * r + i][16 * nb + 4 * g]);
#pragma unroll
            for (int qq = 0; qq < QPW; ++qq) off[qq] = mfma4(cv, ld4(&ss[16 * (q0 + qq) + i][16 * nb + 4 * g]), off[qq]);
          }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int l = 16 * r + 4 * g + jj;
          const float el = exp2f(acl[l]);
          T* yrow = yg + (int64_t)l * p.syl;
#pragma unroll
          for (int qq = 0; qq < QPW; ++qq)
            yrow[16 * (q0 + qq) + i] = from_f32<T>(has_state ? fmaf(el, off[qq][jj], acc[qq][jj]) : acc[qq][jj]);
        }
      }
    }

    // the state entering the next chunk: tiles (p tile q, n tile m), K = l
    {
      const float dend = exp2f(acl[Q - 1]);
      constexpr int TS = QT * NT;           // state tiles
      constexpr int TPW = (TS + 3) / 4;     // per wave
      f32x4 snew[TPW];
#pragma unroll
      for (int k = 0; k < TPW; ++k) {
        const int tile = wave + 4 * k, q = tile % QT, m = tile / QT;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (tile < TS) {
#pragma unroll 4
          for (int lb = 0; lb < R; ++lb)
            acc = mfma4(ld4(&xt[16 * q + i][16 * lb + 4 * g]), ld4(&bwt[16 * m + i][16 * lb + 4 * g]), acc);
          if (has_state) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) acc[jj] = fmaf(ss[16 * q + 4 * g + jj][16 * m + i], dend, acc[jj]);
          }
        }
        snew[k] = acc;
      }
      __syncthreads();  // every read of this chunk's S, x, B, C and tables is done
#pragma unroll
      for (int k = 0; k < TPW; ++k) {
        const int tile = wave + 4 * k, q = tile % QT, m = tile / QT;
        if (tile < TS) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int pp = 16 * q + 4 * g + jj, n = 16 * m + i;
            ss[pp][n] = snew[k][jj];
            if (c + 1 == p.nchunks && p.final_state)
              p.final_state[(int64_t)bh * kP * N + (int64_t)(pc0 + pp) * N + n] = snew[k][jj];
          }
        }
      }
      if (c + 1 < p.nchunks) stage();
    }
    has_state = true;
    __syncthreads();
  }
}

// Two workgroups per chain (halves of p) while the chains fill fewer than
// two workgroups per CU: C1's 128 chains then use all 256 CUs.
template <typename T, int N, int Q>
hipError_t launch_tnq(const SmallArgs& a, hipStream_t stream) {
  const int64_t chains = (int64_t)a.batch * a.nheads;
  const int cus = device_cu_count();
  if (chains < 2 * (int64_t)(cus > 0 ? cus : 256)) {
    ssd_small_kernel<T, N, Q, 2><<<dim3((unsigned)(2 * chains)), dim3(kT), 0, stream>>>(a);
  } else {
    ssd_small_kernel<T, N, Q, 1><<<dim3((unsigned)chains), dim3(kT), 0, stream>>>(a);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const SmallArgs& a, hipStream_t stream) {
  if (a.dstate == 16) return a.chunk == 64 ? launch_tnq<T, 16, 64>(a, stream) : launch_tnq<T, 16, 128>(a, stream);
  return launch_tnq<T, 32, 64>(a, stream);
}

}  // namespace

bool ssd_small_supported(int64_t batch, int64_t nheads, int64_t headdim, int64_t dstate, int64_t chunk, int64_t nchunks) {
  // (chunk 128 x d_state 32 would need more than the 160 KB of LDS)
  return headdim == kP && (dstate == 16 || dstate == 32) && (chunk == 64 || chunk == 128) && chunk * dstate <= 2048 &&
         nchunks >= 1 && nchunks <= kSmallMaxChunks && 2 * batch * nheads <= INT_MAX;
}

hipError_t launch_ssd_small(const SmallArgs& a, int dtype, hipStream_t stream) {
  if (!ssd_small_supported(a.batch, a.nheads, kP, a.dstate, a.chunk, a.nchunks)) return hipErrorInvalidValue;
  if (dtype == SSD_DTYPE_F32) return launch_t<float>(a, stream);
  if (dtype == SSD_DTYPE_BF16) return launch_t<bf16>(a, stream);
  if (dtype == SSD_DTYPE_F16) return launch_t<f16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace ssd
