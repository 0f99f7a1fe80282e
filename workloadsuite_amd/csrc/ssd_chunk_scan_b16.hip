// K4 -- chunk_scan for 16-bit inputs with f32 states (plain f32, or the
// SSD_STATE_F16S hand-over: f16 rows with a power-of-two scale per row) at
// chunk 64 / 128 and d_state 64 / 128 (MR's own block_len 64 at the
// production layer shape).
// Same result as the generic kernel in ssd_chunk_scan.hip up to rounding
// (workloads/mamba/model_ref.py:139-145, 160-162):
//   y[l, p] = sum_{s<=l} exp(Acs[l]-Acs[s]) (C_l . B_s) dt[s] x[s, p]
//             + exp(Acs[l]) sum_n C[l, n] S_in[p, n]
//
// Work decomposition as in the f32 kernel (ssd_chunk_scan_f32.hip): C.B^T
// does not depend on the head (MR:97-99 repeats B and C over the heads of a
// group before MR:143 contracts them), so one workgroup of 8 waves takes one
// (b, c, group) -- or a slice of its heads when there are few groups -- forms
// the causal C.B^T sub-tiles of its rows once, in registers, and walks the
// heads with x, Acs and dt copied global -> LDS one head ahead (two buffers)
// and S_in into one buffer, copied under the diagonal part of the previous
// head once its off-diagonal part has read it: 49 KB of LDS at d_state 128,
// two workgroups per CU (double-buffered S_in, 81 KB and one per CU, was 12%
// slower).  Wave w owns row tiles t (chunk 64: t = w % 4 for w < 4, 3 - w % 4
// above; chunk 128: w % 4 and 7 - w % 4) and p tiles 2 (w / 4), 2 (w / 4) + 1.
//
// The products run on 16x16x32 MFMAs of the input type, as in the chunk-256
// kernel (ssd_chunk_scan_q256.hip):
//   * C.B^T once per slice, from B rows staged in LDS and C fragments in
//     registers, kept as f32 D fragments (4 consecutive s per lane);
//   * the off-diagonal S_in . C^T: each head's f32 S_in is split in LDS, once,
//     into a hi + lo pair of the input type (~16 significant bits through the
//     MFMA: hi = round(v), lo = round(v - hi)), two MFMAs per K step; f16s
//     S_in is read as it lies (half the bytes) on one f16 MFMA per K step,
//     with the C rows held as f16 times a power of two per row and both
//     scales applied to the f32 result;
//   * the diagonal x^T . (decay . C.B^T): x^T straight from row-major x in LDS
//     through ds_read_b64_tr_b16 (rows XOR-swizzled by 16-byte piece at copy
//     time), the weighted C.B^T block rounded to the input type once.
// The accumulators hold y^T (4 consecutive p of one token per lane, 8-byte y
// stores).
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kNW = 8;
constexpr int kThreads = 64 * kNW;

template <typename T, int NK, int RT, bool HAS_DT, bool F16S>
__global__ __launch_bounds__(kThreads) void chunk_scan_b16_kernel(ChunkScanArgs p, int hs, int slices) {
  constexpr int Q = 64 * RT;
  constexpr int N = 32 * NK;
  // S_in rows as stored: N f32 values, or (F16S) the N f16 values in the
  // first half of the row's f32 slots and a scale per row
  constexpr int SRB = F16S ? N * 2 : N * 4;  // bytes per S_in row in LDS
  constexpr int SPR = SRB / 16;              // 16-byte pieces per S_in row
  constexpr int XPW = Q * kP * 2 / 1024 / kNW;  // x copies (1 KB = 8 rows) per wave and head
  constexpr int SPW = kP * SRB / 1024 / kNW;    // S_in copies per wave and head
  constexpr int BPR = N * 2 / 16;            // 16-byte pieces per B row
  constexpr int BPW = Q * N * 2 / 1024 / kNW;   // B copies per wave (once per slice)
  constexpr int NSB = 2 * RT;                // 32-token s blocks of the chunk
  static_assert(XPW >= 1 && SPW >= 1 && BPW >= 1, "copies per wave");
  // S_in's buffer also stages the chunk's B rows (Q N 2 bytes) once per slice
  constexpr int SSB = kP * SRB > Q * N * 2 ? kP * SRB : Q * N * 2;
  __shared__ __attribute__((aligned(1024))) T xs[2][Q * kP];
  __shared__ __attribute__((aligned(1024))) float ss[SSB / 4];
  __shared__ __attribute__((aligned(16))) float scl[F16S ? kP : 4];  // F16S: the row scales of S_in
  __shared__ __attribute__((aligned(16))) float al[2][Q];
  __shared__ __attribute__((aligned(16))) float dl[HAS_DT ? 2 : 1][HAS_DT ? Q : 4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, i = lane & 15;
  const int ph = wave >> 2, rg = RT == 1 && ph ? 3 - (wave & 3) : wave & 3;
  int trow[RT];
  trow[0] = rg;
  if constexpr (RT == 2) trow[1] = 7 - rg;

  // ---- unit: (b, c, group, head slice) ----
  const int u = blockIdx.x;
  const int slice = u % slices, bcg = u / slices;
  const int grp = bcg % p.ngroups, bc = bcg / p.ngroups;
  const int c = bc % p.nchunks, b = bc / p.nchunks;
  const int hpg = p.nheads / p.ngroups;
  const int h0 = grp * hpg + slice * hs;
  const int h1 = min(h0 + hs, (grp + 1) * hpg);
  if (h0 >= h1) return;  // the whole workgroup, before any barrier
  const int64_t l0 = (int64_t)c * Q;

  const T* xg0 = reinterpret_cast<const T*>(p.x) + b * p.sxb + l0 * p.sxl;
  const T* bg = reinterpret_cast<const T*>(p.bm) + b * p.sbb + l0 * p.sbl + grp * p.sbg;
  const T* cg = reinterpret_cast<const T*>(p.cm) + b * p.scb + l0 * p.scl + grp * p.scg;
  T* yg0 = reinterpret_cast<T*>(p.y) + b * p.syb + l0 * p.syl;

  // ---- per-head copies: x, Acs, dt into buffer bf, S_in into its buffer ----
  // x rows s (64 elements, 8 pieces): copy block blk holds rows 8 blk ..
  // 8 blk + 7, piece k of row s at slot k ^ (s & 7).
  const uint32_t xs_lds = lds_offset(&xs[0][0]), ss_lds = lds_offset(&ss[0]);
  const uint32_t al_lds = lds_offset(&al[0][0]), dl_lds = lds_offset(&dl[0][0]);
  const int64_t xcopy = (int64_t)(lane >> 3) * p.sxl + 8 * ((lane & 7) ^ (lane >> 3));
  auto issue_head = [&](int h, int bf) __attribute__((always_inline)) {
    const T* xg = xg0 + h * p.sxh + xcopy;
#pragma unroll
    for (int m = 0; m < XPW; ++m) {
      const int blk = wave + kNW * m;
      dma16_at(xg + (int64_t)(8 * blk) * p.sxl, xs_lds + (uint32_t)((bf * Q * kP) * 2 + blk * 1024));
    }
    if (wave == kNW - 1 && lane < Q / 4) {
      const float* ag = p.acs + (((int64_t)b * p.nheads + h) * p.nchunks + c) * Q;
      dma16_at(ag + 4 * lane, al_lds + (uint32_t)(bf * Q * 4));
    }
    if constexpr (HAS_DT) {
      if (wave >= kNW - 1 - Q / 64 && wave < kNW - 1) {
        const int part = wave - (kNW - 1 - Q / 64);
        const float* dg = p.dt + b * p.sdb + h * p.sdh;
        dma4_at(dg + (l0 + 64 * part + lane) * p.sdl, dl_lds + (uint32_t)((bf * Q + 64 * part) * 4));
      }
    }
  };
  // S_in of head h into its (single) buffer: piece k of row r at slot
  // k ^ ssw(r).  F16S: the 16 rows one operand read takes then lie on
  // distinct banks (256-byte rows: r & 15; 128-byte rows, two per bank
  // window: (r / 2) & 7); f32: r & 7
  auto ssw = [](int r) __attribute__((always_inline)) {
    if constexpr (!F16S) return r & 7;
    else if constexpr (SPR >= 16) return r & 15;
    else return (r >> 1) & 7;
  };
  const uint32_t scl_lds = lds_offset(&scl[0]);
  auto issue_sin = [&](int h) __attribute__((always_inline)) {
    const int64_t item = ((int64_t)b * p.nchunks + c) * p.nheads + h;
    const unsigned char* sg = reinterpret_cast<const unsigned char*>(reinterpret_cast<const float*>(p.states) + item * (kP * N));
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
      const int blk = wave + kNW * m, r = blk * (64 / SPR) + lane / SPR, pc = (lane % SPR) ^ ssw(r);
      dma16_at(sg + r * (N * 4) + 16 * pc, ss_lds + (uint32_t)(blk * 1024));
    }
    if constexpr (F16S) {
      if (wave == 0) dma4_at(p.sscale + item * kP + lane, scl_lds);
    }
  };
  // f32 S_in -> MFMA operand pairs in place: each 32-byte pair
  // of pieces (8 states) becomes [hi x8 | lo x8] of T (all threads; a barrier
  // publishes it)
  auto convert = [&]() __attribute__((always_inline)) {
    for (int v = tid; v < kP * (N / 8); v += kThreads) {
      const int row = v / (N / 8), q = v % (N / 8);
      float* ph_ = &ss[row * N + 4 * ((2 * q) ^ (row & 7))];
      float* pl_ = &ss[row * N + 4 * ((2 * q + 1) ^ (row & 7))];
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(ph_);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(pl_);
      frag8<T> hi, lo;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        hi[k] = from_f32<T>(v0[k]);
        lo[k] = from_f32<T>(v0[k] - to_f32<T>(hi[k]));
        hi[4 + k] = from_f32<T>(v1[k]);
        lo[4 + k] = from_f32<T>(v1[k] - to_f32<T>(hi[4 + k]));
      }
      *reinterpret_cast<frag8<T>*>(ph_) = hi;
      *reinterpret_cast<frag8<T>*>(pl_) = lo;
    }
  };
  issue_head(h0, 0);
  // B rows of the chunk (N elements of T, piece k of row s at slot k ^ (s %
  // BPR) so that the 16 rows one C.B^T operand read takes hit distinct banks)
  // into S_in's buffer, free until the first head's S_in is copied
  const uint32_t bt_lds = ss_lds;
#pragma unroll
  for (int m = 0; m < BPW; ++m) {
    const int blk = wave + kNW * m, r = blk * (64 / BPR) + lane / BPR, pc = (lane % BPR) ^ (r % BPR);
    dma16_at(bg + r * p.sbl + 8 * pc, bt_lds + (uint32_t)(blk * 1024));
  }

  // ---- per slice: C fragments and raw C.B^T sub-tiles of this wave's rows ----
  frag8<T> cf[RT][NK];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) cf[r][kc] = load8<T>(cg + (16 * trow[r] + i) * p.scl + 32 * kc + 8 * g);
  dma_wait();
  __syncthreads();
  const T* bt = reinterpret_cast<const T*>(&ss[0]);
  // cbr[r][sb][st][jj] = C.B^T[s = 32 sb + 16 st + 4 g + jj][l = 16 t + i]
  f32x4 cbr[RT][NSB][2];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int t = trow[r];
#pragma unroll
    for (int sb = 0; sb < (r == 0 ? 2 : NSB); ++sb)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
        if (32 * sb + 16 * st <= 16 * t) {  // not entirely above the diagonal (wave-uniform)
          const int row = 32 * sb + 16 * st + i;
#pragma unroll
          for (int kc = 0; kc < NK; ++kc) {
            const frag8<T> bf8 = *reinterpret_cast<const frag8<T>*>(bt + row * N + 8 * ((4 * kc + g) ^ (row % BPR)));
            d = mma(bf8, cf[r][kc], d);
          }
        }
        cbr[r][sb][st] = d;
      }
  }
  // F16S: the off-diagonal product runs on f16 MFMAs, so each C row l of the
  // wave's tiles is held as f16 scaled by a power of two 2^-e (its largest
  // element then lies in [2^14, 2^15): bf16 values convert exactly), and
  // cs[r] = 2^e undoes it with the decay factor of row l
  float cs[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) cs[r] = 1.f;
  if constexpr (F16S && !std::is_same<T, f16>::value) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      // largest |value| from the bf16 bit patterns (sign cleared, the order
      // of non-negative bf16 values is that of their bits)
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      uint32_t mb = 0;
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) {
        const auto w = __builtin_bit_cast(u32x4, cf[r][kc]);
#pragma unroll
        for (int j = 0; j < 4; ++j) mb = max(mb, max(w[j] & 0x7fffu, (w[j] >> 16) & 0x7fffu));
      }
      float m = __uint_as_float(min(mb, 0x7f80u) << 16);  // a NaN counts as inf, as in every lane
      // the row's 4 lane groups (lanes i, i + 16, i + 32, i + 48)
      m = nn_max(m, __shfl_xor(m, 16));
      m = nn_max(m, __shfl_xor(m, 32));
      const int e = m > 0.f ? min(max(__builtin_amdgcn_frexp_expf(m) - 15, -100), 100) : 0;
      cs[r] = __builtin_ldexpf(1.f, e);
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) {
        f16x8 hv;
#pragma unroll
        for (int j = 0; j < 8; ++j) hv[j] = (f16)__builtin_ldexpf(to_f32<T>(cf[r][kc][j]), -e);
        cf[r][kc] = __builtin_bit_cast(frag8<T>, hv);
      }
    }
  }
  __syncthreads();  // B's buffer takes the first head's S_in from here on
  issue_sin(h0);
  dma_wait();
  __syncthreads();
  if constexpr (!F16S) {
    convert();
    __syncthreads();
  }

  // x^T operand of p tile pt (via ds_read_b64_tr_b16): rows 4 g + i / 4
  // (+ 16, + 32 sb), columns 16 pt + 4 (i % 4), swizzled
  int xoff[2];
  {
    const int r = 4 * g + (i >> 2), x7 = r & 7;
#pragma unroll
    for (int e = 0; e < 2; ++e) xoff[e] = r * kP + 8 * ((2 * (2 * ph + e) + ((i & 3) >> 1)) ^ x7) + 4 * (i & 1);
  }

  f32x4 acc[RT][2];
  int hprev = -1;
  // y of head hy from acc (y^T: rows p = 16 pt + 4 g + jj, columns l = 16 t + i)
  auto store_y = [&](int hy) __attribute__((always_inline)) {
    T* yg = yg0 + hy * p.syh;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        vec4<T> o;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) o[jj] = from_f32<T>(acc[r][e][jj]);
        *reinterpret_cast<vec4<T>*>(yg + (int64_t)(16 * trow[r] + i) * p.syl + 16 * (2 * ph + e) + 4 * g) = o;
      }
  };

  for (int h = h0; h < h1; ++h) {
    const int bf = (h - h0) & 1;
    // the previous head's y, then the next head's copies: the wait at the end
    // of this head covers both
    if (hprev >= 0) store_y(hprev);
    if (h + 1 < h1) issue_head(h + 1, bf ^ 1);
    hprev = h;
    const T* xb = xs[bf];
    const unsigned char* sb_ = reinterpret_cast<const unsigned char*>(&ss[0]);
    const float* ab = al[bf];

    // ---- off-diagonal: acc[p, l] = exp(Acs[l]) sum_n S_in[p, n] C[l, n] ----
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int e = 0; e < 2; ++e) acc[r][e] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < NK; ++kc)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        // states 32 kc + 8 g .. + 7 of row p = 16 pt + i (pair q = 4 kc + g):
        // F16S, piece q of the f16 row; else the hi and lo of pair q at
        // pieces 2 q and 2 q + 1
        const int row = 16 * (2 * ph + e) + i, q = 4 * kc + g;
        const unsigned char* srow = sb_ + row * SRB;
        if constexpr (F16S) {
          const f16x8 a = *reinterpret_cast<const f16x8*>(srow + 16 * (q ^ ssw(row)));
#pragma unroll
          for (int r = 0; r < RT; ++r) acc[r][e] = mma(a, __builtin_bit_cast(f16x8, cf[r][kc]), acc[r][e]);
        } else {
          const frag8<T> hi = *reinterpret_cast<const frag8<T>*>(srow + 16 * ((2 * q) ^ ssw(row)));
          const frag8<T> lo = *reinterpret_cast<const frag8<T>*>(srow + 16 * ((2 * q + 1) ^ ssw(row)));
#pragma unroll
          for (int r = 0; r < RT; ++r) {
            acc[r][e] = mma(hi, cf[r][kc], acc[r][e]);
            acc[r][e] = mma(lo, cf[r][kc], acc[r][e]);
          }
        }
      }
    // F16S: rows p carry their S_in row scale (4 consecutive p per lane),
    // columns l the C row scale
    f32x4 sc[2] = {f32x4{1.f, 1.f, 1.f, 1.f}, f32x4{1.f, 1.f, 1.f, 1.f}};
    if constexpr (F16S) {
#pragma unroll
      for (int e = 0; e < 2; ++e) sc[e] = *reinterpret_cast<const f32x4*>(&scl[16 * (2 * ph + e) + 4 * g]);
    }
    // every wave is done with S_in: the next head's comes in under the diagonal
    __syncthreads();
    if (h + 1 < h1) issue_sin(h + 1);
    // log2(e) Acs[l] of this lane's token l = 16 t + i in each row tile
    float all[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      all[r] = ab[16 * trow[r] + i] * kLog2e;
      const float e = __builtin_amdgcn_exp2f(all[r]) * cs[r];
#pragma unroll
      for (int ee = 0; ee < 2; ++ee) acc[r][ee] *= F16S ? sc[ee] * e : f32x4{e, e, e, e};
    }

    // ---- diagonal: 32 tokens s per block; row tile t needs blocks sb <= t / 2 ----
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      if (sb > trow[RT - 1] / 2) continue;  // wave-uniform
      frag8<T> xf[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const T* a0 = xb + xoff[e] + (32 * sb) * kP;
        xf[e] = join<T>(lds_read_tr(a0), lds_read_tr(a0 + 16 * kP));
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (r == 0 && sb >= 2) continue;  // row tiles w % 4 need at most two blocks
        const int t = trow[r];
        if (sb > t / 2) continue;  // wave-uniform
        f32x8 wv;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int sub = 2 * sb + st;  // 16-token sub-tile of s
          if (sub > t) {                // wholly above the diagonal (wave-uniform)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) wv[4 * st + jj] = 0.f;
            continue;
          }
          const int s0 = 16 * sub + 4 * g;
          const f32x4 as = *reinterpret_cast<const f32x4*>(ab + s0);
          f32x4 ds = f32x4{1.f, 1.f, 1.f, 1.f};
          if constexpr (HAS_DT) ds = *reinterpret_cast<const f32x4*>(&dl[bf][s0]);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float v = cbr[r][sb][st][jj] * __builtin_amdgcn_exp2f(__builtin_fmaf(as[jj], -kLog2e, all[r])) * ds[jj];
            // on the diagonal sub-tile s <= l is 4 g + jj <= i; selection, not
            // a product with the mask: exp2 of a positive log-decay above the
            // diagonal may be inf
            wv[4 * st + jj] = sub < t || 4 * g + jj <= i ? v : 0.f;
          }
        }
        const frag8<T> af = __builtin_convertvector(wv, frag8<T>);
#pragma unroll
        for (int e = 0; e < 2; ++e) acc[r][e] = mma(xf[e], af, acc[r][e]);
      }
    }
    dma_wait();
    __syncthreads();
    if (!F16S && h + 1 < h1) {
      convert();
      __syncthreads();
    }
  }
  store_y(hprev);
}

template <typename T, int NK, int RT>
hipError_t launch_qn(const ChunkScanArgs& a, hipStream_t stream) {
  const int hpg = a.nheads / a.ngroups;
  const int64_t bcg = (int64_t)a.batch * a.nchunks * a.ngroups;
  // slices of a group's heads: enough workgroups for every CU, C.B^T
  // formed as few times as that allows
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  int slices = (int)((cus + bcg - 1) / bcg);
  if (slices > hpg) slices = hpg;
  if (slices < 1) slices = 1;
  const int hs = (hpg + slices - 1) / slices;
  slices = (hpg + hs - 1) / hs;
  const int64_t grid = bcg * slices;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  auto kern = a.f16s ? (a.dt ? chunk_scan_b16_kernel<T, NK, RT, true, true> : chunk_scan_b16_kernel<T, NK, RT, false, true>)
                     : (a.dt ? chunk_scan_b16_kernel<T, NK, RT, true, false> : chunk_scan_b16_kernel<T, NK, RT, false, false>);
  kern<<<dim3((unsigned)grid), dim3(kThreads), 0, stream>>>(a, hs, slices);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const ChunkScanArgs& a, hipStream_t stream) {
  if (a.chunk == 64) return a.dstate == 64 ? launch_qn<T, 2, 1>(a, stream) : launch_qn<T, 4, 1>(a, stream);
  if (a.chunk == 128 && a.dstate == 64) return launch_qn<T, 2, 2>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool chunk_scan_b16_supported(const ChunkScanArgs& a, int dtype, int state_dtype) {
  return (dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16) && state_dtype == SSD_DTYPE_F32 &&
         (a.chunk == 64 || a.chunk == 128) && (a.dstate == 64 || a.dstate == 128) && a.chunk * a.dstate <= 8192 &&
         !a.dskip && !a.z && !a.presplit && !a.cbf && (!a.f16s || a.sscale);
}

hipError_t launch_chunk_scan_b16(const ChunkScanArgs& a, int dtype, hipStream_t stream) {
  if (dtype == SSD_DTYPE_BF16) return launch_t<bf16>(a, stream);
  if (dtype == SSD_DTYPE_F16) return launch_t<f16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace ssd
