// K4 -- chunk_scan for f32 inputs and f32 states at chunk 64 / 128 and
// d_state 64 / 128 (the Mamba-2-130M shape and the grouped short-sequence
// shape).  Same result as the generic kernel in ssd_chunk_scan.hip
// (workloads/mamba/model_ref.py:139-145, 160-162):
//   y[l, p] = sum_{s<=l} exp(Acs[l]-Acs[s]) (C_l . B_s) dt[s] x[s, p]
//             + exp(Acs[l]) sum_n C[l, n] S_in[p, n]
//
// C.B^T does not depend on the head (MR:97-99 repeats B and C over the heads
// of a group before MR:143 contracts them), so one workgroup takes one
// (b, c, group) -- or a slice of its heads when there are few groups -- and
// forms the causal C.B^T sub-tiles once, in registers, for all of them.  At
// f32 the MFMA is 1/16 of the 16-bit rate and C.B^T is 40% (chunk 64,
// d_state 128) to 50% (chunk 128, d_state 64) of a head's MFMA work.
//
// Work decomposition: 8 waves; wave w owns row tiles t (rows 16 t .. 16 t +
// 15 of the chunk) -- at chunk 64 t = w % 4 for w < 4 and 3 - w % 4 above
// (so the two waves of each SIMD together hold three diagonal blocks), at
// chunk 128 t = w % 4 and 7 - w % 4 (five blocks for every wave) -- and p
// tiles 2 (w / 4) and 2 (w / 4) + 1.  Per wave and for the whole slice of
// heads: C fragments of its rows (the B operand of S.C^T and of C.B^T) and
// the raw C.B^T sub-tiles [s][l] of its rows in the D layout (4 consecutive s
// per lane), which with the decay, the causal mask and dt applied are
// directly the B operand of the diagonal product.  S_in and x are the A
// operands, so the accumulators hold y^T: each lane holds 4 consecutive p of
// one token and writes them as one 16-byte store.  The chunk's B rows reach
// the C.B^T products through LDS (one global -> LDS copy per slice, waited
// for once) rather than as global loads per sub-tile.
// Per head, x [s][p] and S_in [p][n] of the head are copied global -> LDS
// (global_load_lds, rows XOR-swizzled by 16-byte piece so the operand reads
// are free of bank conflicts) one head ahead, with Acs and dt.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kNW = 8;
constexpr int kThreads = 64 * kNW;

template <int NK, int RT, bool HAS_DT>
__global__ __launch_bounds__(kThreads) void chunk_scan_f32_kernel(ChunkScanArgs p, int hs, int slices) {
  constexpr int Q = 64 * RT;
  constexpr int N = 32 * NK;
  constexpr int SPR = N / 4;            // 16-byte pieces per S_in row
  constexpr int XPW = Q * kP / 256 / kNW;   // x copies (1 KB) per wave and head
  constexpr int SPW = kP * N / 256 / kNW;   // S_in copies per wave and head
  // s blocks of 32 that row tile set r can need: t <= 3 (r = 0) needs 2, t <= 7 needs 4
  constexpr int NSB = 2 * RT;
  __shared__ __attribute__((aligned(1024))) float xs[2][Q * kP];
  __shared__ __attribute__((aligned(1024))) float ss[2][kP * N];
  __shared__ __attribute__((aligned(16))) float al[2][Q];
  __shared__ __attribute__((aligned(16))) float dl[HAS_DT ? 2 : 1][HAS_DT ? Q : 4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, i = lane & 15;
  // the two waves of SIMD s (w = s, s + 4) take row groups s and 3 - s, so
  // every SIMD holds the same number of diagonal blocks at chunk 64
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

  const float* xg0 = reinterpret_cast<const float*>(p.x) + b * p.sxb + l0 * p.sxl;
  const float* bg = reinterpret_cast<const float*>(p.bm) + b * p.sbb + l0 * p.sbl + grp * p.sbg;
  const float* cg = reinterpret_cast<const float*>(p.cm) + b * p.scb + l0 * p.scl + grp * p.scg;
  float* yg0 = reinterpret_cast<float*>(p.y) + b * p.syb + l0 * p.syl;

  // ---- per-head copies into buffer bf ----
  // x rows r (64 floats, 16 pieces): piece k of the copy lands at piece k of
  // row r and holds global piece k ^ 4((r >> 2) & 3); S_in rows r (N floats):
  // global piece k ^ (r & 7).
  const uint32_t xs_lds = lds_offset(&xs[0][0]), ss_lds = lds_offset(&ss[0][0]);
  const uint32_t al_lds = lds_offset(&al[0][0]), dl_lds = lds_offset(&dl[0][0]);
  auto issue_head = [&](int h, int bf) __attribute__((always_inline)) {
    const float* xg = xg0 + h * p.sxh;
#pragma unroll
    for (int m = 0; m < XPW; ++m) {
      const int blk = wave + kNW * m, r = 4 * blk + (lane >> 4), pc = (lane & 15) ^ (4 * ((r >> 2) & 3));
      dma16_at(xg + r * p.sxl + 4 * pc, xs_lds + (uint32_t)((bf * Q * kP + blk * 256) * 4));
    }
    const float* sg = reinterpret_cast<const float*>(p.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * (kP * N);
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
      const int blk = wave + kNW * m, r = blk * (64 / SPR) + lane / SPR, pc = (lane % SPR) ^ (r & 7);
      dma16_at(sg + r * N + 4 * pc, ss_lds + (uint32_t)((bf * kP * N + blk * 256) * 4));
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
  issue_head(h0, 0);
  // B rows of the chunk (N floats, pieces swizzled as S_in's) into the second
  // copy buffer -- x's when N <= 64, else S_in's (then Q = 64): Q N floats
  // either way -- free until the first head issues the second head's copies
  constexpr bool kBinX = N <= kP;
  constexpr int BPW = Q * N / 256 / kNW;
  const uint32_t bt_lds = kBinX ? xs_lds + Q * kP * 4 : ss_lds + kP * N * 4;
#pragma unroll
  for (int m = 0; m < BPW; ++m) {
    const int blk = wave + kNW * m, r = blk * (64 / SPR) + lane / SPR, pc = (lane % SPR) ^ (r & 7);
    dma16_at(bg + r * p.sbl + 4 * pc, bt_lds + (uint32_t)(blk * 1024));
  }

  // ---- per slice: C fragments and raw C.B^T sub-tiles of this wave's rows ----
  frag8<float> cf[RT][NK];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) cf[r][kc] = load8<float>(cg + (16 * trow[r] + i) * p.scl + 32 * kc + 8 * g);
  dma_wait();
  __syncthreads();
  const float* bt = kBinX ? xs[1] : ss[1];
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
#pragma unroll
          for (int kc = 0; kc < NK; ++kc) {
            const int row = 32 * sb + 16 * st + i, pc = 8 * kc + 2 * g;
            const float* brow = bt + row * N;
            frag8<float> bf8;
            bf8.lo = *reinterpret_cast<const f32x4*>(brow + 4 * (pc ^ (row & 7)));
            bf8.hi = *reinterpret_cast<const f32x4*>(brow + 4 * ((pc + 1) ^ (row & 7)));
            d = mma(bf8, cf[r][kc], d);
          }
        }
        cbr[r][sb][st] = d;
      }
  }
  __syncthreads();  // B's buffer takes the second head's copies from here on

  f32x4 acc[RT][2];
  int hprev = -1;
  // y of head hy from acc, which holds y^T (the S_in / x side is the MFMA's
  // A operand): rows p = 16 pt + 4 g + jj, columns l = 16 t + i, so each lane
  // writes 4 consecutive p of one token
  auto store_y = [&](int hy) __attribute__((always_inline)) {
    float* yg = yg0 + hy * p.syh;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        *reinterpret_cast<f32x4*>(yg + (int64_t)(16 * trow[r] + i) * p.syl + 16 * (2 * ph + e) + 4 * g) = acc[r][e];
  };

  for (int h = h0; h < h1; ++h) {
    const int bf = (h - h0) & 1;
    // the previous head's y, then the next head's copies: the wait at the end
    // of this head covers both
    if (hprev >= 0) store_y(hprev);
    if (h + 1 < h1) issue_head(h + 1, bf ^ 1);
    hprev = h;
    const float* xb = xs[bf];
    const float* sb_ = ss[bf];
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
        const int row = 16 * (2 * ph + e) + i, pc = 8 * kc + 2 * g;
        const float* srow = sb_ + row * N;
        frag8<float> sf;
        sf.lo = *reinterpret_cast<const f32x4*>(srow + 4 * (pc ^ (row & 7)));
        sf.hi = *reinterpret_cast<const f32x4*>(srow + 4 * ((pc + 1) ^ (row & 7)));
#pragma unroll
        for (int r = 0; r < RT; ++r) acc[r][e] = mma(sf, cf[r][kc], acc[r][e]);
      }
    // log2(e) Acs[l] of this lane's token l = 16 t + i in each row tile
    float all[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      all[r] = ab[16 * trow[r] + i] * kLog2e;
      const float e = __builtin_amdgcn_exp2f(all[r]);
#pragma unroll
      for (int ee = 0; ee < 2; ++ee) acc[r][ee] *= e;
    }

    // ---- diagonal: 32 tokens s per block; row tile t needs blocks sb <= t / 2 ----
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      if (sb > trow[RT - 1] / 2) continue;  // wave-uniform
      // x[s][16 pt + i] for s = 32 sb + 16 st + 4 g + jj (slot j = 4 st + jj),
      // shared by the row tiles that need the block
      frag8<float> xf[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int pt = 2 * ph + e;
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int s = 32 * sb + 16 * st + 4 * g + jj;
            xf[e][4 * st + jj] = xb[s * kP + 4 * ((4 * pt + (i >> 2)) ^ (4 * ((s >> 2) & 3))) + (i & 3)];
          }
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (r == 0 && sb >= 2) continue;  // row tiles w % 4 need at most two blocks
        const int t = trow[r];
        if (sb > t / 2) continue;  // wave-uniform
        frag8<float> af;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int sub = 2 * sb + st;  // 16-token sub-tile of s
          if (sub > t) {                // wholly above the diagonal (wave-uniform)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) af[4 * st + jj] = 0.f;
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
            af[4 * st + jj] = sub < t || 4 * g + jj <= i ? v : 0.f;
          }
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          if (2 * sb + 1 > t) {
            // the block's second 16 tokens lie wholly above the diagonal (their
            // slots of af are zero): only the first half's MFMAs, same sums
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[r][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[e][j], af[j], acc[r][e], 0, 0, 0);
          } else {
            acc[r][e] = mma(xf[e], af, acc[r][e]);
          }
        }
      }
    }
    dma_wait();
    __syncthreads();
  }
  store_y(hprev);
}

template <int NK, int RT>
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
  auto kern = a.dt ? chunk_scan_f32_kernel<NK, RT, true> : chunk_scan_f32_kernel<NK, RT, false>;
  kern<<<dim3((unsigned)grid), dim3(kThreads), 0, stream>>>(a, hs, slices);
  return hipGetLastError();
}

}  // namespace

bool chunk_scan_f32_supported(const ChunkScanArgs& a, int dtype, int state_dtype) {
  // chunk 128 with d_state 128 needs more than the 256 VGPRs of two waves per SIMD
  return dtype == SSD_DTYPE_F32 && state_dtype == SSD_DTYPE_F32 && (a.chunk == 64 || a.chunk == 128) &&
         (a.dstate == 64 || a.dstate == 128) && a.chunk * a.dstate <= 8192 && !a.dskip && !a.z && !a.f16s &&
         !a.presplit && !a.cbf;
}

hipError_t launch_chunk_scan_f32(const ChunkScanArgs& a, hipStream_t stream) {
  if (a.chunk == 64) return a.dstate == 64 ? launch_qn<2, 1>(a, stream) : launch_qn<4, 1>(a, stream);
  if (a.chunk == 128 && a.dstate == 64) return launch_qn<2, 2>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace ssd
