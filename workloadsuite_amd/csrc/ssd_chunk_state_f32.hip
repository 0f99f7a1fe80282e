// K2 -- chunk_state for f32 states at chunk 64 / 128 and d_state 64 / 128
// (the Mamba-2-130M shape, the grouped short-sequence shape, and MR's own
// block_len 64 with 16-bit inputs).  Inputs of type T (f32, bf16 or f16) are
// staged as they are.  f32 inputs: every product is an f32 MFMA on the
// inputs' exact values.  16-bit inputs: 16x16x32 MFMAs of the input type,
// B exact and the weighted x as a hi + lo pair (kstep below).  Same result
// as the generic kernel in ssd_chunk_state.hip up to its 16-bit rounding of
// the weighted operand (workloads/mamba/model_ref.py:144, 148-149):
//   S[p, n] = sum_l (w[l] x[l, p]) B[l, n],   w[l] = exp(Acs[Q-1] - Acs[l]) dt[l]
// stored as states[b, c, h, p, n].
//
// B does not depend on the head (MR:97-99 repeats it over the heads of a
// group), so one workgroup takes one (b, c, group) -- or a slice of its heads
// when there are few groups -- and keeps the B operand of its output tiles in
// registers for all of them; per head only x (and Acs, dt) move, copied
// global -> LDS one head ahead (global_load_lds, rows XOR-swizzled by 16-byte
// piece so the column reads of the A operand are free of bank conflicts).
// The weight w[l] is applied in f32 as the x operand is read (for 16-bit
// inputs the product is then split into the hi + lo pair).
//
// Work decomposition: 8 waves; wave w owns p tiles 2 (w % 2), 2 (w % 2) + 1
// and n tiles [(w / 2) N / 64, (w / 2 + 1) N / 64).  K index slot (g, j) of
// K step ks is token l = 32 ks + 16 (j / 4) + 4 g + j % 4 in both operands.
// B is the MFMA's A operand and the weighted x its B operand, so the
// accumulators hold S^T: each lane holds 4 consecutive n of one p and stores
// them as one 16-byte store.
#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kNW = 8;
constexpr int kThreads = 64 * kNW;

// Staged rows of x and B: 16-byte pieces of EPP = 16 / sizeof(T) elements,
// piece k of row l stored at piece k ^ swz_x(l).  f32: a fragment read takes
// one column of rows 4 g + jj (g = 0..3), and the XOR moves those 4 rows to 4
// different 64-byte bank groups.  16-bit: the operands come through
// transposing reads (tr_operand), in which 32 lanes take 32 bytes (a pair of
// pieces) of each of 8 consecutive rows; the XOR (a multiple of 2, so pairs
// stay whole) puts those 8 row segments on distinct banks (rows of >= 256
// bytes: 2 (l & 7); rows of 128 bytes, two per 256-byte bank window: the
// window half l & 1 and 2 ((l / 2) & 3)).
template <typename T> __device__ __forceinline__ int swz_x(int l, int cols) {
  if constexpr (sizeof(T) == 4) return 4 * ((l >> 2) & 3);
  else return cols * 2 >= 256 ? 2 * (l & 7) : 2 * ((l >> 1) & 3);
}
// element offset of x / B element (l, col) in a staged block of rows of `cols` elements
template <typename T> __device__ __forceinline__ int swz_off(int l, int col, int cols) {
  constexpr int EPP = 16 / (int)sizeof(T);
  return l * cols + EPP * ((col / EPP) ^ swz_x<T>(l, cols)) + col % EPP;
}
// global -> LDS copy blk (1 KB, 64 lanes x 16 bytes) of rows of `cols`
// elements of T, rows ld elements apart, into dst + 1 KB blk (piece k of row
// r from piece k ^ swz_x(r) of the global row)
template <typename T>
__device__ __forceinline__ void stage_rows(const T* src, int64_t ld, int cols, int blk, uint32_t dst, int lane) {
  const int ppr = cols * (int)sizeof(T) / 16, r = blk * (64 / ppr) + lane / ppr, pc = (lane % ppr) ^ swz_x<T>(r, cols);
  dma16_at(src + r * ld + (16 / (int)sizeof(T)) * pc, dst + (uint32_t)(blk * 1024));
}
// 16-bit inputs: the MFMA operand of K step ks for column c0 + i (c0 a
// multiple of 16) from a staged block of rows of `cols` elements, as two
// transposing reads: lane (i, g) addresses row 32 ks + 4 g + i / 4 (then 16
// rows on), columns c0 + 4 (i % 4) .. + 3, and receives column c0 + i of
// rows 4 g .. 4 g + 3 -- K slot j holds token 32 ks + 16 (j / 4) + 4 g + j % 4,
// the slot order of the element-wise reads (ds_read_b64_tr_b16, as chunk_scan
// reads x^T)
template <typename T>
__device__ __forceinline__ frag8<T> tr_operand(const T* blk, int ks, int c0, int cols, int g, int i) {
  const int r = 32 * ks + 4 * g + (i >> 2), c = c0 + 4 * (i & 3);
  return join<T>(lds_read_tr(blk + swz_off<T>(r, c, cols)), lds_read_tr(blk + swz_off<T>(r + 16, c, cols)));
}

// w[l] = exp(Acs[Q-1] - Acs[l]) dt[l] from Acs[l], log2(e) Acs[Q-1] and dt[l]
// (exp2 of a non-positive argument for decaying chunks; results below f32's
// normal range flush to 0)
__device__ __forceinline__ float chunk_weight(float acs_l, float last_log2, float dt_l) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(acs_l, -kLog2e, last_log2)) * dt_l;
}

// The B operand fragments as the MFMA takes them: f32 values for f32 inputs,
// the inputs' own 16-bit values otherwise.
template <typename T> using BFrag = typename std::conditional<std::is_same<T, float>::value, frag8<float>, frag8<T>>::type;

// One K step of S^T += B^T (w x) for one p tile: x is this lane's 8 tokens of
// column p (K slots in the B fragment's order) and w their weights.  f32
// inputs: the f32 products on 16x16x4 f32 MFMAs.  16-bit inputs: the
// weighted x split into a hi + lo pair of the input type (hi = round(x w),
// lo = round(x w - hi), ~16 significant bits through the MFMA) on two
// 16x16x32 MFMAs of that type, B exact.
template <typename T>
__device__ __forceinline__ f32x4 kstep(const BFrag<T>& bf, const frag8<T>& x, const float* w, f32x4 acc) {
  if constexpr (std::is_same<T, float>::value) {
    frag8<float> xf;
#pragma unroll
    for (int j = 0; j < 8; ++j) xf[j] = x[j] * w[j];
    return mma(bf, xf, acc);
  } else {
    frag8<T> hi, lo;
    split_weighted<T, true>(x, f32x4{w[0], w[1], w[2], w[3]}, f32x4{w[4], w[5], w[6], w[7]}, hi, lo);
    acc = mma(bf, hi, acc);
    return mma(bf, lo, acc);
  }
}

template <typename T, int NK, int RT, bool HAS_DT>
__global__ __launch_bounds__(kThreads) void chunk_state_f32_kernel(ChunkStateArgs p, int hs, int slices) {
  constexpr int Q = 64 * RT;
  constexpr int N = 32 * NK;
  constexpr int ES = (int)sizeof(T);
  constexpr int KS = Q / 32;             // K steps of 32 tokens
  constexpr int NTW = N / 64;            // n tiles per wave
  constexpr int XPW = Q * kP * ES / 1024 / kNW;  // x copies (1 KB) per wave and head
  constexpr int BPW = Q * N * ES / 1024 / kNW;   // B copies per wave
  // x buffers 0 and 1, then room for B (staged once, over buffer 1)
  constexpr int LDS_E = 2 * Q * kP > Q * kP + Q * N ? 2 * Q * kP : Q * kP + Q * N;
  __shared__ __attribute__((aligned(1024))) T lds[LDS_E];
  __shared__ __attribute__((aligned(16))) float al[2][Q];
  __shared__ __attribute__((aligned(16))) float dl[HAS_DT ? 2 : 1][HAS_DT ? Q : 4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, i = lane & 15;
  const int pp = wave & 1, nt0 = (wave >> 1) * NTW;

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
  const uint32_t lds_base = lds_offset(&lds[0]);
  const uint32_t al_lds = lds_offset(&al[0][0]), dl_lds = lds_offset(&dl[0][0]);

  auto issue_head = [&](int h, int bf) __attribute__((always_inline)) {
    const T* xg = xg0 + h * p.sxh;
#pragma unroll
    for (int m = 0; m < XPW; ++m) stage_rows<T>(xg, p.sxl, kP, wave + kNW * m, lds_base + (uint32_t)(bf * Q * kP * ES), lane);
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

  // ---- per slice: B operands of this wave's n tiles, via LDS ----
  issue_head(h0, 0);
#pragma unroll
  for (int m = 0; m < BPW; ++m) stage_rows<T>(bg, p.sbl, N, wave + kNW * m, lds_base + (uint32_t)(Q * kP * ES), lane);
  dma_wait();
  __syncthreads();
  BFrag<T> bfr[NTW][KS];
  {
    const T* bl = lds + Q * kP;
#pragma unroll
    for (int n = 0; n < NTW; ++n)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (std::is_same<T, float>::value) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            bfr[n][ks][j] = bl[swz_off<T>(32 * ks + 16 * (j >> 2) + 4 * g + (j & 3), 16 * (nt0 + n) + i, N)];
        } else {
          bfr[n][ks] = tr_operand<T>(bl, ks, 16 * (nt0 + n), N, g, i);
        }
      }
  }
  __syncthreads();  // B's LDS is x buffer 1 from here on

  f32x4 acc[2][NTW];
  int hprev = -1;
  // states[b, c, h, p, n] of head hst from acc, which holds S^T (B is the
  // MFMA's A operand): rows n = 16 nt + 4 g + jj, columns p = 16 pt + i, so
  // each lane writes 4 consecutive n of one p as one 16-byte store
  auto store_states = [&](int hst) __attribute__((always_inline)) {
    float* sg = reinterpret_cast<float*>(p.states) + (((int64_t)b * p.nchunks + c) * p.nheads + hst) * (kP * N);
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int n = 0; n < NTW; ++n)
        *reinterpret_cast<f32x4*>(sg + (16 * (2 * pp + a) + i) * N + 16 * (nt0 + n) + 4 * g) = acc[a][n];
  };

  for (int h = h0; h < h1; ++h) {
    const int bf = (h - h0) & 1;
    // the previous head's states, then the next head's copies: the wait at
    // the end of this head covers both
    if (hprev >= 0) store_states(hprev);
    if (h + 1 < h1) issue_head(h + 1, bf ^ 1);
    hprev = h;
    const T* xb = lds + bf * Q * kP;
    const float* ab = al[bf];
    const float last = ab[Q - 1] * kLog2e;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int n = 0; n < NTW; ++n) acc[a][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      // w[l] of this lane's 8 tokens
      float w[8];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int l = 32 * ks + 16 * st + 4 * g;
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(ab + l);
        f32x4 d4 = f32x4{1.f, 1.f, 1.f, 1.f};
        if constexpr (HAS_DT) d4 = *reinterpret_cast<const f32x4*>(&dl[bf][l]);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) w[4 * st + jj] = chunk_weight(a4[jj], last, d4[jj]);
      }
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        frag8<T> xr;
        if constexpr (std::is_same<T, float>::value) {
          const int col = 16 * (2 * pp + a) + i;
#pragma unroll
          for (int j = 0; j < 8; ++j) xr[j] = xb[swz_off<T>(32 * ks + 16 * (j >> 2) + 4 * g + (j & 3), col, kP)];
        } else {
          xr = tr_operand<T>(xb, ks, 16 * (2 * pp + a), kP, g, i);
        }
#pragma unroll
        for (int n = 0; n < NTW; ++n) acc[a][n] = kstep<T>(bfr[n][ks], xr, w, acc[a][n]);
      }
    }
    dma_wait();
    __syncthreads();
  }
  store_states(hprev);
}

// K2 + K3 in one launch for f32 inputs and f32 states: one workgroup per
// (b, h) chain walks the chunks in order (DB: the next chunk's copies run
// under the current chunk's compute; otherwise each chunk's copies are
// waited for, and a second workgroup per CU covers that latency), computes each chunk's local state
// exactly as chunk_state_f32_kernel does (same operands, same MFMA and FMA
// order), and advances the running state held in registers,
// h <- h * decay[c] + local (workloads/mamba/model_ref.py:152-157) -- the
// same f32 FMA per element and chunk as state_passing -- after storing the
// state entering the chunk, S_in[c], in the f32 states layout.  The local
// states never reach memory.  x and B of the next chunk are copied
// global -> LDS while the current chunk computes; the chains of one group's
// heads run on one XCD and share B through its L2.
// F16S (16-bit inputs, DB): S_in[c] goes out as SSD_STATE_F16S, f16 rows
// with a power-of-two scale per row p, rounded exactly as state_passing's
// f16s store rounds them; a row's N states lie in 4 waves, which exchange
// their row maxima through LDS (written at the end of the previous chunk,
// two buffers).
template <typename T, int NK, int RT, bool HAS_DT, bool DB, bool F16S>
__global__ __launch_bounds__(kThreads) void chunk_state_chain_f32_kernel(ChunkStateArgs p, StatePassingArgs sp) {
  constexpr int Q = 64 * RT;
  constexpr int N = 32 * NK;
  constexpr int ES = (int)sizeof(T);
  constexpr int KS = Q / 32;
  constexpr int NTW = N / 64;
  constexpr int XPW = Q * kP * ES / 1024 / kNW;
  constexpr int BPW = Q * N * ES / 1024 / kNW;
  constexpr int NBUF = DB ? 2 : 1;
  __shared__ __attribute__((aligned(1024))) T xs[NBUF][Q * kP];
  __shared__ __attribute__((aligned(1024))) T bs[NBUF][Q * N];
  __shared__ __attribute__((aligned(16))) float al[NBUF][Q];
  __shared__ __attribute__((aligned(16))) float dl[HAS_DT ? NBUF : 1][HAS_DT ? Q : 4];
  static_assert(!F16S || DB, "the f16s store needs the double-buffered loop");
  // F16S: the largest |S_in| of row p over n quarter k (waves 2 k, 2 k + 1)
  __shared__ float rmax[F16S ? 2 : 1][F16S ? 4 * kP : 1];
  // each wave's copy of the current chunk's weights w[l] (written and read by
  // that wave only)
  __shared__ __attribute__((aligned(16))) float wl[kNW][Q];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, i = lane & 15;
  const int pp = wave & 1, nt0 = (wave >> 1) * NTW;
  // consecutive chains (the heads of a group) on one XCD
  const int bh = __builtin_amdgcn_readfirstlane(xcd_remap(blockIdx.x, gridDim.x));
  const int h = bh % p.nheads, b = bh / p.nheads;
  const int grp = h / (p.nheads / p.ngroups);

  const T* xg = reinterpret_cast<const T*>(p.x) + b * p.sxb + h * p.sxh;
  const T* bg = reinterpret_cast<const T*>(p.bm) + b * p.sbb + grp * p.sbg;
  const float* dg = HAS_DT ? p.dt + b * p.sdb + h * p.sdh : nullptr;
  const uint32_t xs_lds = lds_offset(&xs[0][0]), bs_lds = lds_offset(&bs[0][0]);
  const uint32_t al_lds = lds_offset(&al[0][0]), dl_lds = lds_offset(&dl[0][0]);
  auto issue_chunk = [&](int c, int bf) __attribute__((always_inline)) {
    const int64_t l0 = (int64_t)c * Q;
#pragma unroll
    for (int m = 0; m < XPW; ++m) stage_rows<T>(xg + l0 * p.sxl, p.sxl, kP, wave + kNW * m, xs_lds + (uint32_t)(bf * Q * kP * ES), lane);
#pragma unroll
    for (int m = 0; m < BPW; ++m) stage_rows<T>(bg + l0 * p.sbl, p.sbl, N, wave + kNW * m, bs_lds + (uint32_t)(bf * Q * N * ES), lane);
    if (wave == kNW - 1 && lane < Q / 4) {
      const float* ag = p.acs + ((int64_t)bh * p.nchunks + c) * Q;
      dma16_at(ag + 4 * lane, al_lds + (uint32_t)(bf * Q * 4));
    }
    if constexpr (HAS_DT) {
      if (wave >= kNW - 1 - Q / 64 && wave < kNW - 1) {
        const int part = wave - (kNW - 1 - Q / 64);
        dma4_at(dg + (l0 + 64 * part + lane) * p.sdl, dl_lds + (uint32_t)((bf * Q + 64 * part) * 4));
      }
    }
  };

  // running state: S_in of the current chunk in the accumulators' S^T
  // layout, rows n = 16 nt + 4 g + jj, columns p = 16 pt + i (4 consecutive n
  // of one p per lane)
  const int64_t PN = (int64_t)kP * N;
  auto sidx = [&](int a, int n) __attribute__((always_inline)) { return (16 * (2 * pp + a) + i) * N + 16 * (nt0 + n) + 4 * g; };
  f32x4 st[2][NTW];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int n = 0; n < NTW; ++n)
      st[a][n] = sp.init ? *reinterpret_cast<const f32x4*>(sp.init + bh * PN + sidx(a, n)) : f32x4{0.f, 0.f, 0.f, 0.f};
  // F16S: this wave's part of the row maxima of the running state (lanes
  // i, i + 16, i + 32, i + 48 hold row p's 16 n of each of its n tiles; two
  // lane swaps in the VALU, each lane keeping the larger of its value and
  // the swapped one)
  auto put_rmax = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      float m = 0.f;
#pragma unroll
      for (int n = 0; n < NTW; ++n)
#pragma unroll
        for (int k = 0; k < 4; ++k) m = __builtin_elementwise_maximum(m, fabsf(st[a][n][k]));
      const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
      m = nn_max(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
      const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
      m = nn_max(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
      if (g == 0) rmax[buf][(wave >> 1) * kP + 16 * (2 * pp + a) + i] = m;
    }
  };
  if constexpr (F16S) put_rmax(0);
  if constexpr (DB) {
    issue_chunk(0, 0);
    dma_wait();
    __syncthreads();
  }

  // the chain's decays, 64 chunks at a time: lane k holds decay[c0 + k]
  float decv = 0.f;
  constexpr int kStores = 2 * NTW;  // S_in stores per lane and chunk
  for (int c = 0; c < p.nchunks; ++c) {
    // decay[c] from the lanes' block, loaded (and waited for) before this
    // chunk's copies are issued, so that wait does not include them
    if ((c & 63) == 0) decv = c + lane < p.nchunks ? sp.decay[(int64_t)bh * p.nchunks + c + lane] : 0.f;
    const float dec = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, decv), c & 63));
    // DB: the next chunk's copies run under this chunk's compute; otherwise
    // this chunk's copies are waited for here (other workgroups on the CU
    // cover the latency).  S_in[c] -- the running state as the chunk begins
    // -- is stored after the copies are issued, so the waits for the copies
    // (vmcnt retires in issue order) leave the stores in flight.
    const int bf = DB ? (c & 1) : 0;
    float* sg = reinterpret_cast<float*>(sp.states) + (((int64_t)b * p.nchunks + c) * p.nheads + h) * PN;
    if constexpr (DB) {
      if (c + 1 < p.nchunks) issue_chunk(c + 1, bf ^ 1);
    } else {
      issue_chunk(c, 0);
    }
    if constexpr (F16S) {
      // row p's f16 values in the first half of its f32 slots, its scale in
      // sscale[b, c, h, p] (written by the lanes of n quarter 0)
      const float* rm = rmax[c & 1];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int pr = 16 * (2 * pp + a) + i;
        const float m = nn_max(nn_max(rm[pr], rm[kP + pr]), nn_max(rm[2 * kP + pr], rm[3 * kP + pr]));
        const int e = m > 0.f ? min(max(__builtin_amdgcn_frexp_expf(m) - 15, -100), 100) : 0;
#pragma unroll
        for (int n = 0; n < NTW; ++n) {
          f16x4 hv;
#pragma unroll
          for (int k = 0; k < 4; ++k) hv[k] = (f16)__builtin_ldexpf(st[a][n][k], -e);
          *reinterpret_cast<f16x4*>(reinterpret_cast<f16*>(sg + pr * N) + 16 * (nt0 + n) + 4 * g) = hv;
        }
        if (nt0 == 0 && g == 0)
          sp.sscale[(((int64_t)b * p.nchunks + c) * p.nheads + h) * kP + pr] = __builtin_ldexpf(1.f, e);
      }
    } else {
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int n = 0; n < NTW; ++n) *reinterpret_cast<f32x4*>(sg + sidx(a, n)) = st[a][n];
    }
    if constexpr (!DB) {
      vm_wait<kStores>();
      __syncthreads();
    }
    const T* xb = xs[bf];
    const T* bl = bs[bf];
    const float* ab = al[bf];
    const float last = ab[Q - 1] * kLog2e;
    // 16-bit inputs, and f32 inputs with several workgroups per CU: the
    // chunk's weights, token 64 k + lane by each lane, into this wave's copy
    // (the same values as forming each lane's 8 weights per K step, which f32
    // inputs with one workgroup per CU still do: there the LDS round trip
    // would lie on the chain's critical path, C2 110 -> 119 us)
    constexpr bool kWaveWeights = !std::is_same<T, float>::value || !DB;
    float* wv = wl[wave];
    if constexpr (kWaveWeights) {
#pragma unroll
      for (int k = 0; k < Q / 64; ++k) {
        const int l = 64 * k + lane;
        wv[l] = chunk_weight(ab[l], last, HAS_DT ? dl[bf][l] : 1.f);
      }
    }
    f32x4 acc[2][NTW];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int n = 0; n < NTW; ++n) acc[a][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float w[8];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int l = 32 * ks + 16 * s2 + 4 * g;
        if constexpr (kWaveWeights) {
          const f32x4 w4 = *reinterpret_cast<const f32x4*>(wv + l);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) w[4 * s2 + jj] = w4[jj];
        } else {
          const f32x4 a4 = *reinterpret_cast<const f32x4*>(ab + l);
          f32x4 d4 = f32x4{1.f, 1.f, 1.f, 1.f};
          if constexpr (HAS_DT) d4 = *reinterpret_cast<const f32x4*>(&dl[bf][l]);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) w[4 * s2 + jj] = chunk_weight(a4[jj], last, d4[jj]);
        }
      }
      BFrag<T> bfr[NTW];
#pragma unroll
      for (int n = 0; n < NTW; ++n) {
        if constexpr (std::is_same<T, float>::value) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            bfr[n][j] = bl[swz_off<T>(32 * ks + 16 * (j >> 2) + 4 * g + (j & 3), 16 * (nt0 + n) + i, N)];
        } else {
          bfr[n] = tr_operand<T>(bl, ks, 16 * (nt0 + n), N, g, i);
        }
      }
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        frag8<T> xr;
        if constexpr (std::is_same<T, float>::value) {
          const int col = 16 * (2 * pp + a) + i;
#pragma unroll
          for (int j = 0; j < 8; ++j) xr[j] = xb[swz_off<T>(32 * ks + 16 * (j >> 2) + 4 * g + (j & 3), col, kP)];
        } else {
          xr = tr_operand<T>(xb, ks, 16 * (2 * pp + a), kP, g, i);
        }
#pragma unroll
        for (int n = 0; n < NTW; ++n) acc[a][n] = kstep<T>(bfr[n], xr, w, acc[a][n]);
      }
    }
    // the recurrence (state_passing's f32 FMA)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int n = 0; n < NTW; ++n) st[a][n] = st[a][n] * dec + acc[a][n];
    if constexpr (F16S) put_rmax((c + 1) & 1);
    // DB: the next chunk's copies have landed (the stores may still be in
    // flight); either way every wave is done with this chunk's buffer
    if constexpr (DB) vm_wait<kStores>();
    __syncthreads();
  }
  if (sp.final_state) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int n = 0; n < NTW; ++n) *reinterpret_cast<f32x4*>(sp.final_state + bh * PN + sidx(a, n)) = st[a][n];
  }
}

template <typename T, int NK, int RT>
hipError_t launch_chain_qn(const ChunkStateArgs& a, const StatePassingArgs& sp, hipStream_t stream) {
  const int64_t chains = (int64_t)a.batch * a.nheads;
  if (chains > INT32_MAX) return hipErrorInvalidValue;
  // two chunks of x and B in LDS (one workgroup per CU at f32) while chains
  // are fewer than two per CU; with more, one chunk (two workgroups per CU,
  // each covering the other's copy latency): C2 (192 chains of 32 chunks) 7%
  // faster double-buffered, C5 (4096 chains of 4) 3% faster single-buffered.
  // 16-bit inputs always double-buffer: their two chunks (48 KB at chunk 64,
  // d_state 128) still leave room for two workgroups per CU (R0's core, 1024
  // chains of 32 chunks: 404 -> 378 us)
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const bool db = chains < 2 * (int64_t)cus || !std::is_same<T, float>::value;
  if constexpr (!std::is_same<T, float>::value) {
    if (sp.f16s) {
      auto kern = a.dt ? chunk_state_chain_f32_kernel<T, NK, RT, true, true, true> : chunk_state_chain_f32_kernel<T, NK, RT, false, true, true>;
      kern<<<dim3((unsigned)chains), dim3(kThreads), 0, stream>>>(a, sp);
      return hipGetLastError();
    }
  }
  auto kern = db ? (a.dt ? chunk_state_chain_f32_kernel<T, NK, RT, true, true, false> : chunk_state_chain_f32_kernel<T, NK, RT, false, true, false>)
                 : (a.dt ? chunk_state_chain_f32_kernel<T, NK, RT, true, false, false> : chunk_state_chain_f32_kernel<T, NK, RT, false, false, false>);
  kern<<<dim3((unsigned)chains), dim3(kThreads), 0, stream>>>(a, sp);
  return hipGetLastError();
}

template <typename T, int NK, int RT>
hipError_t launch_qn(const ChunkStateArgs& a, hipStream_t stream) {
  const int hpg = a.nheads / a.ngroups;
  const int64_t bcg = (int64_t)a.batch * a.nchunks * a.ngroups;
  // slices of a group's heads: enough workgroups for every CU, B loaded as
  // few times as that allows
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  int slices = (int)((cus + bcg - 1) / bcg);
  if (slices > hpg) slices = hpg;
  if (slices < 1) slices = 1;
  const int hs = (hpg + slices - 1) / slices;
  slices = (hpg + hs - 1) / hs;
  const int64_t grid = bcg * slices;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  auto kern = a.dt ? chunk_state_f32_kernel<T, NK, RT, true> : chunk_state_f32_kernel<T, NK, RT, false>;
  kern<<<dim3((unsigned)grid), dim3(kThreads), 0, stream>>>(a, hs, slices);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_chain_t(const ChunkStateArgs& a, const StatePassingArgs& sp, hipStream_t stream) {
  if (a.chunk == 64) return a.dstate == 64 ? launch_chain_qn<T, 2, 1>(a, sp, stream) : launch_chain_qn<T, 4, 1>(a, sp, stream);
  if (a.chunk == 128 && a.dstate == 64) return launch_chain_qn<T, 2, 2>(a, sp, stream);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_t(const ChunkStateArgs& a, hipStream_t stream) {
  if (a.chunk == 64) return a.dstate == 64 ? launch_qn<T, 2, 1>(a, stream) : launch_qn<T, 4, 1>(a, stream);
  return a.dstate == 64 ? launch_qn<T, 2, 2>(a, stream) : launch_qn<T, 4, 2>(a, stream);
}

}  // namespace

bool chunk_state_f32_supported(const ChunkStateArgs& a, int dtype, int state_dtype) {
  return (dtype == SSD_DTYPE_F32 || dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16) &&
         state_dtype == SSD_DTYPE_F32 && (a.chunk == 64 || a.chunk == 128) && (a.dstate == 64 || a.dstate == 128);
}

bool chunk_state_chain_f32_supported(const ChunkStateArgs& a, int dtype, const StatePassingArgs& sp) {
  // two chunks of x and B in LDS: chunk x d_state up to 8192; S_in as f16s
  // for 16-bit inputs
  return chunk_state_f32_supported(a, dtype, SSD_DTYPE_F32) && a.chunk * a.dstate <= 8192 && !sp.split_dtype &&
         (!sp.f16s || (dtype != SSD_DTYPE_F32 && sp.sscale)) && sp.bh_begin == 0 &&
         (sp.bh_count == 0 || sp.bh_count == a.batch * a.nheads);
}

hipError_t launch_chunk_state_chain_f32(const ChunkStateArgs& a, const StatePassingArgs& sp, int dtype, hipStream_t stream) {
  if (dtype == SSD_DTYPE_BF16) return launch_chain_t<bf16>(a, sp, stream);
  if (dtype == SSD_DTYPE_F16) return launch_chain_t<f16>(a, sp, stream);
  return launch_chain_t<float>(a, sp, stream);
}

hipError_t launch_chunk_state_f32(const ChunkStateArgs& a, int dtype, hipStream_t stream) {
  if (dtype == SSD_DTYPE_BF16) return launch_t<bf16>(a, stream);
  if (dtype == SSD_DTYPE_F16) return launch_t<f16>(a, stream);
  return launch_t<float>(a, stream);
}

}  // namespace ssd
