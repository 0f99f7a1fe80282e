// K4 -- chunk_scan, persistent variant for 16-bit inputs at chunk 256 (the
// Mamba-2-2.7B layer shape).  Same result as the generic kernel in
// ssd_chunk_scan.hip (workloads/mamba/model_ref.py:139-145, 160-162):
//   y[l, p] = sum_{s<=l} exp(Acs[l]-Acs[s]) (C_l . B_s) dt[s] x[s, p]
//             + exp(Acs[l]) sum_n C[l, n] S_in[p, n]
//
// Work decomposition.  One workgroup of 8 waves per CU loops over a
// contiguous range of (b, c, h) items, heads fastest, so consecutive items
// share (b, c) and usually the group of B and C.
//   * C . B^T depends on (b, c, group) only.  Wave w owns row tiles w and
//     15-w (16 rows each; every wave then has 17 causal 16x16 blocks in 9
//     32-token s blocks) and keeps their CB^T blocks in registers as f32 MFMA
//     D fragments, recomputed only when the group changes (B and C are read
//     from global memory then; they are shared by all heads of the group and
//     sit in L2).
//   * Per item two products remain, computed transposed, D = Y^T[p, l], so
//     each lane ends with 4 consecutive p of one row (8-byte y stores):
//       off-diagonal  Y^T = exp(Acs[l]) S_in[p, :] . C[l, :]
//       diagonal      Y^T += x^T[p, s] (exp(Acs[l]-Acs[s]) dt[s] CB^T[s, l])
//     The weighted CB^T block is a D fragment with 4 consecutive s of one l
//     per lane, i.e. already the B operand of the diagonal MFMA.  Below the
//     diagonal the decay factors around the last token r of each 32-token s
//     block, exp(Acs[l]-Acs[r]) exp(Acs[r]-Acs[s]) (both <= 1 for decaying
//     A): one exp per lane and block plus a per-item table of the second
//     factor, instead of one exp per element.  The block that crosses the
//     diagonal keeps the exact per-element form, masked before its exponent
//     can overflow.
//   * x^T operands come straight from row-major x in LDS through the
//     transposing read ds_read_b64_tr_b16.  S_in arrives, by default, as f16
//     rows with a power-of-two scale per row (SSD_STATE_F16S, written so by
//     state_passing or the state chain): one f16 MFMA per K step reads it as
//     it lies, with C's rows held as f16 times their own power of two and
//     both scales applied to the f32 result.  With state_format "split" it
//     arrives as 16-bit (hi, lo) pairs of the input type (two MFMAs per K
//     step, ~16 significant bits); plain f32 S_in is split so in LDS once per
//     item.
// Data movement.  The next item's x, S_in, Acs and dt are copied global ->
// LDS by global_load_lds (no VGPRs held) into the second of two LDS buffers
// while the current item computes; one wait + barrier per item publishes
// them.  x rows and S_in rows are XOR-swizzled by 16-byte piece at copy time
// (the copy picks each lane's global address), so the transposing reads of x
// and the row reads of S_in are free of bank conflicts.  Every operand read
// uses a per-lane base computed once plus a compile-time offset.  y is stored
// at the end of each item, 16 bytes per lane.
//
// Traffic per item: x 32 KB + S_in 16 KB (f16s; 32 KB as hi / lo pairs or
// f32) + its row scales 256 B + Acs 1 KB read, y 32 KB written; B and C (or
// chunk_prep's C.B^T fragments) per group from L2.
//
// Layer epilogue (EPI, with dt and chunk_prep's operands): y = (y + D[h] x)
// * silu(z) (MR:116-118) before y's one rounding.  D x reads x from the
// item's LDS block; z (32 KB more per item) is loaded into registers once the
// off-diagonal part is done, in the layout of the y stores.
#include <climits>
#include <cstdint>
#include <type_traits>

#include "ssd_device.h"
#include "ssd_launch.h"
#include "../../include/ssd.h"

namespace ssd {

namespace {

constexpr int kP = 64;
constexpr int kQ = 256;
constexpr int kNT = kQ / 16;         // row tiles
constexpr int kNW = kNT / 2;         // waves: wave w owns row tiles w and kNT-1-w
constexpr int kThreads = 64 * kNW;
constexpr int kNPair = kNT / 2 + 1;  // 32-token s blocks per wave, both tiles
constexpr int kXBlocks = kQ / 8;     // 1 KB copy blocks of x (8 rows of 64 x 16-bit)

// Kernel arguments with 32-bit element strides (offsets are still formed in
// 64 bits): fewer scalar registers stay live across the item loop than with
// the int64 ChunkScanArgs.  The launcher checks that every stride fits.
struct ScanArgs32 {
  const void* x;
  const void* bm;
  const void* cm;
  const float* dt;
  const float* acs;
  const void* states;
  void* y;
  const float* cbf;  // chunk_prep's CB^T fragments, or null
  const float* sscale;  // F16S: the row scales of the states [b, c, h, P]
  int cb16;          // ... rounded to T (the epilogue variant)
  int presplit;      // f32 S_in already stored as [hi x8 | lo x8] pairs
  const float* dskip;  // epilogue: skip weights [h], or null
  const void* z;       // epilogue: gate [b, L, h, P], or null
  int sxb, sxl, sxh, sbb, sbl, sbg, scb, scl, scg, sdb, sdl, sdh, syb, syl, syh, szb, szl, szh;
  int batch, nchunks, nheads, ngroups, dstate;
};

struct Item {
  int b, c, h, grp;
  int hg;  // head within the group
};

// State storage tag: f32 states handed over as f16 with a power-of-two scale
// per state row p (SSD_STATE_F16S): row p of an item (N f32 slots) holds N
// f16 values in its first half; the row scales are a separate [b, c, h, P]
// array.
struct f16s_t {};
template <typename S> struct StateElem { typedef S type; };
template <> struct StateElem<f16s_t> { typedef f16 type; };

// CB^T blocks of one 32-token s block (two 16x16 sub-tiles st) as MFMA D
// fragments: f32, or rounded to T where the registers are needed elsewhere
// (the epilogue variant's z values).
template <typename T, bool NARROW>
struct CbStep {
  f32x4 v[2];
  __device__ __forceinline__ void set(int st, f32x4 d) { v[st] = d; }
  __device__ __forceinline__ f32x4 get(int st) const { return v[st]; }
};
template <typename T>
struct CbStep<T, true> {
  vec4<T> v[2];
  __device__ __forceinline__ void set(int st, f32x4 d) { v[st] = __builtin_convertvector(d, vec4<T>); }
  __device__ __forceinline__ f32x4 get(int st) const { return __builtin_convertvector(v[st], f32x4); }
};

__device__ __forceinline__ Item item_of(const ScanArgs32& p, int it) {
  Item r;
  r.h = it % p.nheads;
  const int bc = it / p.nheads;
  r.c = bc % p.nchunks;
  r.b = bc / p.nchunks;
  const int hpg = p.nheads / p.ngroups;
  r.grp = r.h / hpg;
  r.hg = r.h - r.grp * hpg;
  return r;
}

// The item after r in (b, c, h) order, heads fastest: item_of(it + 1)
// without its integer divisions (hpg = heads per group).
__device__ __forceinline__ Item next_item(const ScanArgs32& p, Item r, int hpg) {
  ++r.h;
  if (++r.hg == hpg) {
    r.hg = 0;
    ++r.grp;
  }
  if (r.h == p.nheads) {
    r.h = r.grp = r.hg = 0;
    if (++r.c == p.nchunks) {
      r.c = 0;
      ++r.b;
    }
  }
  return r;
}

template <typename T, typename S, int NK, bool HAS_DT, bool PREP, bool EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void chunk_scan_q256_kernel(ScanArgs32 p) {
  constexpr int N = 32 * NK;                      // dstate (64 or 128)
  constexpr bool F16S = std::is_same<S, f16s_t>::value;  // f16 rows with a per-row scale
  constexpr bool SPLIT = std::is_same<S, float>::value;  // f32 states become a hi/lo pair
  typedef typename StateElem<S>::type SE;          // element type of the stored states
  // global layout: row stride GRS and item stride of the states, in SE elements
  constexpr int GRS = F16S ? 2 * N : N;
  // S_in rows in LDS: RB bytes, PPR 16-byte pieces, unpadded; piece c of row
  // r sits at slot c ^ ssw(r), which spreads the 16 rows that one operand
  // read touches over distinct banks.  One 64-lane copy moves RPD rows.
  constexpr int RB = N * (int)sizeof(SE);
  constexpr int PPR = RB / 16;
  constexpr int RPD = 1024 / RB;
  constexpr int SCOPIES = kP / RPD / kNW;         // S_in copies per wave and item
  static_assert(PPR >= 8 && SCOPIES >= 1 && SCOPIES <= 4, "S_in row shape");
  auto ssw = [](int r) __attribute__((always_inline)) { return PPR >= 16 ? (r & 15) : ((r >> 1) & 7); };
  // Two buffers of each: the current item's and the next item's (in flight).
  __shared__ __attribute__((aligned(1024))) T xr[2][kQ * kP];
  __shared__ __attribute__((aligned(1024))) unsigned char sr[2][kP * RB];
  __shared__ __attribute__((aligned(16))) float dr[HAS_DT ? 2 : 1][HAS_DT ? kQ : 4];
  // Each wave's own copy of the next item's Acs, and its tables of the
  // current item (a wave writes and reads only its own, so they need no
  // barrier): [0] Acs * log2(e); [1] G[s] =
  // exp(Acs[r] - Acs[s]), r the last token of s's 32-token block (the decay
  // of the blocks below the diagonal factors as exp(Acs[l] - Acs[r]) * G[s]).
  __shared__ __attribute__((aligned(16))) float ar[kNW][kQ];
  __shared__ __attribute__((aligned(16))) float wt[kNW][2][kQ];
  // F16S: the per-row scales of S_in, current and next item
  __shared__ __attribute__((aligned(16))) float scl[2][F16S ? kP : 4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  __builtin_assume(wave < kNW);  // lets the tile-range tests below fold
  const int g = lane >> 4, i = lane & 15;
  const int nitems = p.batch * p.nchunks * p.nheads;
  // consecutive item ranges (which share B and C) go to one XCD's L2
  const int lb = xcd_remap(blockIdx.x, gridDim.x);
  const int it0 = (int)((int64_t)lb * nitems / gridDim.x);
  const int it1 = (int)((int64_t)(lb + 1) * nitems / gridDim.x);
  if (it0 >= it1) return;
  const int ta = wave, tb = kNT - 1 - wave;
  const int KA = ta / 2 + 1;  // s blocks of tile ta; tile tb has the other kNPair - KA

  // ---- per-lane LDS offsets of the MFMA operands (fixed for the kernel) ----
  int xoff[4];  // x^T operand: rows 4g + i/4 (+ 32 sb + 16 h), columns 16 pt + 4 (i % 4), swizzled
  // S_in operand, row 16 pt + i, K step kc (32 states): piece CPK kc + lp of
  // the row, lp = 2 g (+1 for lo) when split, else g.  The slot
  // (CPK kc + lp) ^ ssw(i) = (CPK (kc % NKB) ^ lp ^ ssw(i)) + 16 (kc / NKB)
  // leaves NKB lane bases per half (byte offsets; + 16 pt RB per column tile).
  constexpr int CPK = SPLIT ? 8 : 4;
  constexpr int NKB = NK < 16 / CPK ? NK : 16 / CPK;
  constexpr int NH = SPLIT ? 2 : 1;
  int sbase[NKB][NH];
  {
    const int r = 4 * g + (i >> 2), x7 = r & 7;
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) xoff[pt] = r * kP + 8 * ((2 * pt + ((i & 3) >> 1)) ^ x7) + 4 * (i & 1);
#pragma unroll
    for (int k = 0; k < NKB; ++k)
#pragma unroll
      for (int h = 0; h < NH; ++h) sbase[k][h] = i * RB + 16 * ((CPK * k) ^ ((SPLIT ? 2 * g + h : g) ^ ssw(i)));
  }


  // ---- per-lane parts of the copy and store addresses (fixed for the kernel) ----
  // x copy: lane reads row (lane / 8) of its 8-row block, piece (lane % 8) ^ (lane / 8).
  const int64_t xcopy = (int64_t)(lane >> 3) * p.sxl + 8 * ((lane & 7) ^ (lane >> 3));
  // y store: a lane holds p 16 pt + 4 g .. + 3 of row 16 t + i for every
  // column tile pt; lane rows g, g ^ 1 swap halves of the column-tile pairs
  // (0, 1) and (2, 3), after which each lane holds 8 consecutive p starting
  // at 32 pair + ycol of its row (16-byte stores, 64 contiguous bytes per
  // row and instruction).
  const int ycol = 8 * (g >> 1) + 16 * (g & 1);
  // S_in copy: lane k fills slot k % PPR of row RPD d + k / PPR, i.e. reads
  // piece (k % PPR) ^ ssw(row); the row's ssw depends on d only through the
  // wave (RPD d = RPD wave mod 16).
  const int scopy = (lane / PPR) * GRS + ((lane % PPR) ^ ssw(wave * RPD + lane / PPR)) * (16 / (int)sizeof(SE));


  // ---- global -> LDS copy of one item's x, S_in, Acs (and dt) into buffer b ----
  // LDS offsets of the buffer arrays (from the __shared__ objects themselves,
  // so that no generic -> LDS pointer conversion is needed per copy).
  const uint32_t xr_lds = lds_offset(&xr[0][0]), sr_lds = lds_offset(&sr[0][0]);
  const uint32_t ar_lds = lds_offset(&ar[0][0]), dr_lds = lds_offset(&dr[0][0]);
  const uint32_t scl_lds = lds_offset(&scl[0][0]);

  // Part `part` (0..3) of one item's copy: x block rows 64 part + 8 wave ..,
  // S_in rows 16 part + wave and + 8; part 0 also copies Acs (and dt).  The
  // parts are issued between compute steps, so that a wave's vector-memory
  // queue never holds up its MFMAs for a whole item's copy.
  auto issue_copy_part = [&](const Item& r, int b, int part) __attribute__((always_inline)) {
    // opaque buffer index: the LDS destinations are formed per item instead of
    // being hoisted for both buffers (which would pin ~30 scalar registers)
    b = __builtin_amdgcn_readfirstlane(b);
    asm volatile("" : "+s"(b));
    const int64_t l0 = (int64_t)r.c * kQ;
    const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)r.b * p.sxb + l0 * p.sxl + (int64_t)r.h * p.sxh + xcopy;
    // x: copy block blk holds rows 8 blk .. 8 blk + 7; row s keeps piece c at slot c ^ (s & 7).
    {
      const int blk = wave + kNW * part;
      dma16_at(xg + (int64_t)(8 * blk) * p.sxl, xr_lds + (uint32_t)(b * kQ * kP * (int)sizeof(T) + blk * 1024));
    }
    // S_in: copy d = wave + 8 part moves rows RPD d .. RPD d + RPD - 1 (1 KB).
    const int64_t item = ((int64_t)r.b * p.nchunks + r.c) * p.nheads + r.h;
    if (part < SCOPIES) {
      const SE* sg = reinterpret_cast<const SE*>(p.states) + item * (int64_t)(kP * GRS) + scopy;
      const int d = wave + kNW * part;
      dma16_at(sg + d * RPD * GRS, sr_lds + (uint32_t)(b * kP * RB + d * 1024));
    }
    if constexpr (F16S) {
      // the item's 64 row scales (256 contiguous bytes)
      if (part == 1 && wave == 0) dma4_at(p.sscale + item * kP + lane, scl_lds + (uint32_t)(b * kP * 4));
    }
    if (part == 0) {
      const float* ag = p.acs + (((int64_t)r.b * p.nheads + r.h) * p.nchunks + r.c) * kQ;
      dma16_at(ag + 4 * lane, ar_lds + (uint32_t)(wave * kQ * 4));
    }
    if constexpr (HAS_DT) {
      if (part == 0 && wave < kQ / 64) {
        const float* dg = p.dt + (int64_t)r.b * p.sdb + (int64_t)r.h * p.sdh;
        dma4_at(dg + (l0 + 64 * wave + lane) * p.sdl, dr_lds + (uint32_t)(b * kQ * 4 + 256 * wave));
      }
    }
  };
  static_assert(kXBlocks == 4 * kNW, "four copy parts cover x");


  // ---- once the copy of the next item has landed ----
  // This wave's tables of the item, from its own copy of Acs (no barrier).
  auto tables = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int e = lane; e < kQ; e += 64) {
      const float a = ar[wave][e] * kLog2e, a_end = ar[wave][e | 31] * kLog2e;
      wt[wave][0][e] = a;
      wt[wave][1][e] = __builtin_amdgcn_exp2f(a_end - a);
    }
  };
  // S_in -> MFMA operand type, by all waves (a barrier publishes it).  f32
  // S_in: each 32-byte pair of pieces (8 states) becomes [hi x8 | lo x8] of T
  // in place, unless state_passing already stored it so; bf16 S_in with f16
  // inputs: converted to f16 in place.
  constexpr bool kBf16ToF16 = !SPLIT && !F16S && !std::is_same<S, T>::value;
  const bool must_convert = SPLIT ? !p.presplit : kBf16ToF16;
  auto convert = [&](int b) __attribute__((always_inline)) {
    if constexpr (SPLIT) {
      for (int u = tid; u < kP * (N / 8); u += kThreads) {
        // pair q = pieces 2q, 2q+1 (8 states) -> hi at piece 2q's slot, lo at 2q+1's
        const int row = u / (N / 8), q = u % (N / 8), sw = ssw(row);
        unsigned char* ph = sr[b] + row * RB + 16 * ((2 * q) ^ sw);
        unsigned char* pl = sr[b] + row * RB + 16 * ((2 * q + 1) ^ sw);
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(ph);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(pl);
        frag8<T> hi, lo;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          hi[k] = from_f32<T>(v0[k]);
          lo[k] = from_f32<T>(v0[k] - to_f32<T>(hi[k]));
          hi[4 + k] = from_f32<T>(v1[k]);
          lo[4 + k] = from_f32<T>(v1[k] - to_f32<T>(hi[4 + k]));
        }
        *reinterpret_cast<frag8<T>*>(ph) = hi;
        *reinterpret_cast<frag8<T>*>(pl) = lo;
      }
    } else if constexpr (kBf16ToF16) {
      for (int u = tid; u < kP * PPR; u += kThreads) {
        unsigned char* pr = sr[b] + 16 * u;
        const frag8<SE> v = *reinterpret_cast<const frag8<SE>*>(pr);
        frag8<T> o;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = from_f32<T>(to_f32<SE>(v[k]));
        *reinterpret_cast<frag8<T>*>(pr) = o;
      }
    }
  };

  // ---- per-group registers: C fragments of both tiles and their CB^T blocks ----
  frag8<T> cf[2][NK];
  CbStep<T, EPI> cbc[kNPair];
  // F16S: the off-diagonal product runs on f16 MFMAs, so each C row l of the
  // two tiles is held as f16 scaled by a power of two 2^-e (its largest
  // element then lies in [2^14, 2^15): bf16 values convert exactly), and
  // cs[t] = 2^e undoes it with the decay factor of row l.
  float cs[2] = {1.f, 1.f};
  auto c_to_f16 = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // largest |value| from the bf16 bit patterns (sign cleared, the order
      // of non-negative bf16 values is that of their bits): no f32
      // temporaries live across the row's 8 NK values (called for bf16 only)
      float m = 0.f;
      if constexpr (std::is_same<T, bf16>::value) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        uint32_t mb = 0;
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
          const auto w = __builtin_bit_cast(u32x4, cf[t][kc]);
#pragma unroll
          for (int j = 0; j < 4; ++j) mb = max(mb, max(w[j] & 0x7fffu, (w[j] >> 16) & 0x7fffu));
        }
        m = __uint_as_float(min(mb, 0x7f80u) << 16);  // a NaN counts as inf, as in every lane
      }
      // the row's 4 lane groups (lanes i, i + 16, i + 32, i + 48)
      m = nn_max(m, __shfl_xor(m, 16));
      m = nn_max(m, __shfl_xor(m, 32));
      const int e = m > 0.f ? min(max(__builtin_amdgcn_frexp_expf(m) - 15, -100), 100) : 0;
      cs[t] = __builtin_ldexpf(1.f, e);
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) {
        f16x8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (f16)__builtin_ldexpf(to_f32<T>(cf[t][kc][j]), -e);
        cf[t][kc] = __builtin_bit_cast(frag8<T>, h);
      }
    }
  };
  auto load_group = [&](int it) __attribute__((always_inline)) {
    int lane_o = lane;
    asm volatile("" : "+v"(lane_o));
    const int g = lane_o >> 4, i = lane_o & 15;
    const Item r = item_of(p, it);
    const int64_t l0 = (int64_t)r.c * kQ;
    const T* cg = reinterpret_cast<const T*>(p.cm) + (int64_t)r.b * p.scb + l0 * p.scl + (int64_t)r.grp * p.scg;
    const T* bg = reinterpret_cast<const T*>(p.bm) + (int64_t)r.b * p.sbb + l0 * p.sbl + (int64_t)r.grp * p.sbg;
#pragma unroll
    for (int kc = 0; kc < NK; ++kc) {
      cf[0][kc] = load8<T>(cg + (int64_t)(16 * ta + i) * p.scl + 32 * kc + 8 * g);
      cf[1][kc] = load8<T>(cg + (int64_t)(16 * tb + i) * p.scl + 32 * kc + 8 * g);
    }
    if constexpr (PREP) {
      // precomputed by chunk_prep in this order: one round of independent loads
      const int64_t wbase = (((int64_t)r.b * p.nchunks + r.c) * p.ngroups + r.grp) * kNW + wave;
      if constexpr (EPI) {
        if (p.cb16) {
          // rounded to T by chunk_prep already (the same values CbStep would hold)
          const frag8<T>* cb = reinterpret_cast<const frag8<T>*>(p.cbf) + wbase * (kNPair * 64) + lane_o;
#pragma unroll
          for (int k = 0; k < kNPair; ++k) {
            const frag8<T> v = cb[k * 64];
            cbc[k].v[0] = v.lo;
            cbc[k].v[1] = v.hi;
          }
          if constexpr (F16S && !std::is_same<T, f16>::value) c_to_f16();
          return;
        }
      }
      const f32x4* cb = reinterpret_cast<const f32x4*>(p.cbf) + wbase * (kNPair * 2 * 64) + lane_o;
#pragma unroll
      for (int k = 0; k < kNPair; ++k)
#pragma unroll
        for (int st = 0; st < 2; ++st) cbc[k].set(st, cb[(k * 2 + st) * 64]);
      if constexpr (F16S && !std::is_same<T, f16>::value) c_to_f16();
      return;
    }
    // One 32-token s block (two 16x16 sub-tiles) per step; every row lies in
    // the chunk, so all loads of a step issue together, and a sub-tile
    // entirely above the diagonal is zeroed after its MFMAs.
#pragma unroll
    for (int k = 0; k < kNPair; ++k) {
      // cbc[k]: tile ta's s block k for k < KA, else tile tb's s block kNPair-1-k
      // (reverse order, so step j of either tile sits at a compile-time index)
      const bool first = k < KA;
      const int t = first ? ta : tb, sb = first ? k : kNPair - 1 - k;
      frag8<T> cfx[NK];
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) cfx[kc] = first ? cf[0][kc] : cf[1][kc];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        // one 16-row sub-tile of B at a time (fewer registers live beside
        // the CB^T blocks; this path runs once per group)
        frag8<T> bfr[NK];
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) bfr[kc] = load8<T>(bg + (int64_t)(32 * sb + 16 * st + i) * p.sbl + 32 * kc + 8 * g);
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) d = mma(bfr[kc], cfx[kc], d);
        const bool live = 2 * sb + st <= t;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) d[jj] = live ? d[jj] : 0.f;
        cbc[k].set(st, d);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (F16S && !std::is_same<T, f16>::value) c_to_f16();
  };

  // ---- one item from LDS buffer b into packed y registers ----
  // Both row tiles together: the off-diagonal reads each S_in fragment once
  // for both, and diagonal step j of the two tiles shares one 32-token s
  // block, so its x^T fragments and G factors are read once and feed two
  // independent MFMA chains.
  vec4<T> ypk[2][4];
  // With the layer's epilogue: y in f32 until the gate, and the gate's z
  // values of the item (loaded once the off-diagonal part is done, in the
  // layout store_y writes y in).
  f32x4 yf[2][4];
  frag8<T> zv[2][2];
  // off_step(pt) runs before off-diagonal step pt.
  auto compute = [&](int b, const Item& r, auto off_step) __attribute__((always_inline)) {
    const T* xb = xr[b];
    const unsigned char* sbuf = sr[b];
    const float* ab = wt[wave][0];
    const float* gb = wt[wave][1];
    const float* db = dr[HAS_DT ? b : 0];
    const int KB = kNPair - KA;
    float al[2];
    al[0] = ab[16 * ta + i];  // Acs[l] * log2(e) of this lane's row in each tile
    al[1] = ab[16 * tb + i];
    f32x4 acc[2][4];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) acc[s2][pt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // off-diagonal: acc[s2][pt] = S_in[p, :] . C[l, :], then * exp(Acs[l])
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
      off_step(pt);
#pragma unroll
      for (int kc = 0; kc < NK; ++kc) {
        const unsigned char* q = sbuf + 16 * pt * RB + 256 * (kc / NKB);
        if constexpr (F16S) {
          const f16x8 a = *reinterpret_cast<const f16x8*>(q + sbase[kc % NKB][0]);
          acc[0][pt] = mma(a, __builtin_bit_cast(f16x8, cf[0][kc]), acc[0][pt]);
          acc[1][pt] = mma(a, __builtin_bit_cast(f16x8, cf[1][kc]), acc[1][pt]);
          continue;
        }
        const frag8<T> hi = *reinterpret_cast<const frag8<T>*>(q + sbase[kc % NKB][0]);
        acc[0][pt] = mma(hi, cf[0][kc], acc[0][pt]);
        acc[1][pt] = mma(hi, cf[1][kc], acc[1][pt]);
        if constexpr (SPLIT) {
          const frag8<T> lo = *reinterpret_cast<const frag8<T>*>(q + sbase[kc % NKB][NH - 1]);
          acc[0][pt] = mma(lo, cf[0][kc], acc[0][pt]);
          acc[1][pt] = mma(lo, cf[1][kc], acc[1][pt]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // bound how far LDS reads are hoisted (register pressure)
    }
    if constexpr (F16S) {
      // rows p of the off-diagonal tiles carry their S_in row scale, columns
      // l the C row scale and exp(Acs[l])
      // (one column tile's scales at a time: fewer live registers)
      float e[2];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) e[s2] = __builtin_amdgcn_exp2f(al[s2]) * cs[s2];
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(&scl[b][16 * pt + 4 * g]);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) acc[s2][pt] *= sc * e[s2];
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const float e = __builtin_amdgcn_exp2f(al[s2]);
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) acc[s2][pt] *= e;
      }
    }
    if constexpr (EPI) {
      if (p.z) {
        const T* zg = reinterpret_cast<const T*>(p.z) + (int64_t)r.b * p.szb + ((int64_t)r.c * kQ) * p.szl +
                      (int64_t)r.h * p.szh + ycol;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int pp = 0; pp < 2; ++pp)
            zv[s2][pp] = load8<T>(zg + (int64_t)(16 * (s2 ? tb : ta) + i) * p.szl + 32 * pp);
      }
    }

    // weighted CB^T block of one tile and s block as an MFMA operand; only
    // the block that crosses the diagonal needs the causal mask.
    auto weights = [&](int s2, int sb, const CbStep<T, EPI>& cbs, bool on_diag, const f32x4* gs)
                       __attribute__((always_inline)) {
      const f32x4 cb[2] = {cbs.get(0), cbs.get(1)};
      frag8<T> af;
      if (on_diag) {
        // The causal-mask predicates depend only on the lane: from an opaque
        // lane id they are evaluated per item instead of being hoisted out of
        // the item loop as ~60 live 64-bit lane masks.
        int lane_o = lane;
        asm volatile("" : "+v"(lane_o));
        const int go = lane_o >> 4, l = 16 * (s2 ? tb : ta) + (lane_o & 15);
        // Exact decay, masked before it can overflow above the diagonal.  The
        // sub-tile of rows 16 t .. 16 t + 15 crosses the diagonal; for even t
        // the other one lies wholly above it (zero), for odd t wholly below
        // it (no mask needed).
        const bool odd = ((s2 ? tb : ta) & 1) != 0;  // wave-uniform
        f32x8 wv;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          if (!odd && st == 1) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) wv[4 + jj] = 0.f;
            continue;
          }
          const f32x4 as = *reinterpret_cast<const f32x4*>(ab + 32 * sb + 16 * st + 4 * g);
          f32x4 ds = f32x4{1.f, 1.f, 1.f, 1.f};
          if constexpr (HAS_DT) ds = *reinterpret_cast<const f32x4*>(db + 32 * sb + 16 * st + 4 * g);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            float w = __builtin_amdgcn_exp2f(al[s2] - as[jj]) * cb[st][jj];
            if constexpr (HAS_DT) w *= ds[jj];
            const bool below = odd && st == 0;
            wv[4 * st + jj] = (below || 32 * sb + 16 * st + 4 * go + jj <= l) ? w : 0.f;
          }
        }
        af = __builtin_convertvector(wv, frag8<T>);
      } else {
        // below the diagonal: exp(Acs[l] - Acs[s]) = exp(Acs[l] - Acs[r]) G[s]
        const float fl = __builtin_amdgcn_exp2f(al[s2] - ab[32 * sb + 31]);
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) af[4 * st + jj] = from_f32<T>(cb[st][jj] * (fl * gs[st][jj]));
      }
      return af;
    };

    // diagonal, step j: s block j of tile ta (j < KA) and of tile tb (j < KB)
#pragma unroll
    for (int j = 0; j < kNPair - 1; ++j) {
      const bool do_a = j < KA, do_b = j < KB;  // wave-uniform
      if (!do_b) continue;                       // KB >= KA: nothing left for either tile
      f32x4 gs[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        gs[st] = *reinterpret_cast<const f32x4*>(gb + 32 * j + 16 * st + 4 * g);
        if constexpr (HAS_DT) gs[st] *= *reinterpret_cast<const f32x4*>(db + 32 * j + 16 * st + 4 * g);
      }
      frag8<T> xfr[4];
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        const T* a0 = xb + xoff[pt] + (32 * j) * kP;
        xfr[pt] = join<T>(lds_read_tr(a0), lds_read_tr(a0 + 16 * kP));
      }
      {
        const frag8<T> af = weights(1, j, cbc[kNPair - 1 - j], j == KB - 1, gs);
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) acc[1][pt] = mma(xfr[pt], af, acc[1][pt]);
      }
      if (do_a) {
        const frag8<T> af = weights(0, j, cbc[j], j == KA - 1, gs);
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) acc[0][pt] = mma(xfr[pt], af, acc[0][pt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EPI) {
      // skip term D x[l, p], x from this item's LDS block (row l, piece
      // 2 pt + g / 2 at its swizzled slot, half g % 2)
      if (p.dskip) {
        const float dsk = p.dskip[r.h];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int l = 16 * (s2 ? tb : ta) + i;
#pragma unroll
          for (int pt = 0; pt < 4; ++pt) {
            const vec4<T> xv = load4<T>(xb + l * kP + 8 * ((2 * pt + (g >> 1)) ^ (l & 7)) + 4 * (g & 1));
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) acc[s2][pt][jj] += dsk * to_f32<T>(xv[jj]);
          }
        }
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) yf[s2][pt] = acc[s2][pt];
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) ypk[s2][pt][jj] = from_f32<T>(acc[s2][pt][jj]);
    }
  };

  // y of item r from ypk: lane rows g, g ^ 1 swap halves of the column-tile
  // pairs, then each lane stores 8 consecutive p (16 bytes) of its row.
  auto store_y = [&](const Item& r) __attribute__((always_inline)) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    T* yg = reinterpret_cast<T*>(p.y) + (int64_t)r.b * p.syb + ((int64_t)r.c * kQ) * p.syl + (int64_t)r.h * p.syh;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      T* yrow = yg + (int64_t)(16 * (s2 ? tb : ta) + i) * p.syl + ycol;
      if constexpr (EPI) {
        // the same exchange on f32 values, then the gate, then one rounding
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          // one named swap per word (a loop over the words, assigning vector
          // elements, lost all but the first swap in compilation)
          const u32x4 a = __builtin_bit_cast(u32x4, yf[s2][2 * pp]);
          const u32x4 c = __builtin_bit_cast(u32x4, yf[s2][2 * pp + 1]);
          const auto w0 = __builtin_amdgcn_permlane16_swap(a[0], c[0], false, false);
          const auto w1 = __builtin_amdgcn_permlane16_swap(a[1], c[1], false, false);
          const auto w2 = __builtin_amdgcn_permlane16_swap(a[2], c[2], false, false);
          const auto w3 = __builtin_amdgcn_permlane16_swap(a[3], c[3], false, false);
          f32x8 v;
          v.lo = __builtin_bit_cast(f32x4, u32x4{w0[0], w1[0], w2[0], w3[0]});
          v.hi = __builtin_bit_cast(f32x4, u32x4{w0[1], w1[1], w2[1], w3[1]});
          if (p.z) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float zf = to_f32<T>(zv[s2][pp][k]);
              v[k] *= zf * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * zf));
            }
          }
          store8<T>(yrow + 32 * pp, __builtin_convertvector(v, frag8<T>));
        }
        continue;
      }
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const u32x2 a = __builtin_bit_cast(u32x2, ypk[s2][2 * pp]);
        const u32x2 c = __builtin_bit_cast(u32x2, ypk[s2][2 * pp + 1]);
        // row g even keeps tile 2pp and takes the odd row's half of it; row g
        // odd takes the even row's half of tile 2pp+1 and keeps its own
        const auto w0 = __builtin_amdgcn_permlane16_swap(a[0], c[0], false, false);
        const auto w1 = __builtin_amdgcn_permlane16_swap(a[1], c[1], false, false);
        *reinterpret_cast<u32x4*>(yrow + 32 * pp) = u32x4{w0[0], w1[0], w0[1], w1[1]};
      }
    }
  };

  // Per item: compute it while the next item's copy is issued between its
  // steps, store its y; then wait for the copy, form this wave's tables of
  // the next item (from its own copy of Acs) and publish the copy (the one
  // barrier per item).
  Item cur = item_of(p, it0);
#pragma unroll
  for (int part = 0; part < 4; ++part) issue_copy_part(cur, 0, part);
  load_group(it0);
  dma_wait();
  tables();
  __syncthreads();
  if (must_convert) {
    convert(0);
    __syncthreads();
  }
  const int hpg = p.nheads / p.ngroups;
  for (int it = it0; it < it1; ++it) {
    const int bc = (it - it0) & 1, bn = bc ^ 1;
    const bool has_next = it + 1 < it1;
    const Item nxt = has_next ? next_item(p, cur, hpg) : cur;
    compute(bc, cur, [&](int pt) __attribute__((always_inline)) {
      if (has_next) issue_copy_part(nxt, bn, pt);
    });
    store_y(cur);
    // the copy has landed; this item's 4 y stores may still be in flight
    vm_wait<4>();
    if (has_next) tables();
    __syncthreads();
    if (has_next) {
      if (must_convert) {
        convert(bn);
        __syncthreads();
      }
      if (nxt.b != cur.b || nxt.c != cur.c || nxt.grp != cur.grp) {
        load_group(it + 1);
        // complete before the next item's copies are issued: the compiler's
        // wait before the first use would also count those copies
        dma_wait();
      }
      cur = nxt;
    }
  }
}

bool fits_i32(int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; }

ScanArgs32 narrow(const ChunkScanArgs& a) {
  ScanArgs32 n;
  n.x = a.x;
  n.bm = a.bm;
  n.cm = a.cm;
  n.dt = a.dt;
  n.acs = a.acs;
  n.states = a.states;
  n.y = a.y;
  n.cbf = a.cbf;
  n.sscale = a.sscale;
  n.cb16 = a.cb16 ? 1 : 0;
  n.presplit = a.presplit ? 1 : 0;
  n.dskip = a.dskip;
  n.z = a.z;
  n.szb = (int)a.szb, n.szl = (int)a.szl, n.szh = (int)a.szh;
  n.sxb = (int)a.sxb, n.sxl = (int)a.sxl, n.sxh = (int)a.sxh;
  n.sbb = (int)a.sbb, n.sbl = (int)a.sbl, n.sbg = (int)a.sbg;
  n.scb = (int)a.scb, n.scl = (int)a.scl, n.scg = (int)a.scg;
  n.sdb = (int)a.sdb, n.sdl = (int)a.sdl, n.sdh = (int)a.sdh;
  n.syb = (int)a.syb, n.syl = (int)a.syl, n.syh = (int)a.syh;
  n.batch = a.batch, n.nchunks = a.nchunks, n.nheads = a.nheads, n.ngroups = a.ngroups, n.dstate = a.dstate;
  return n;
}

template <typename T, typename S, int NK>
hipError_t launch_nk(const ChunkScanArgs& a, hipStream_t stream) {
  // the epilogue variant exists for the layer's path only (dt and prep given)
  const bool epi = a.dskip || a.z;
  auto kern = epi ? chunk_scan_q256_kernel<T, S, NK, true, true, true>
              : a.dt ? (a.cbf ? chunk_scan_q256_kernel<T, S, NK, true, true, false>
                              : chunk_scan_q256_kernel<T, S, NK, true, false, false>)
                     : (a.cbf ? chunk_scan_q256_kernel<T, S, NK, false, true, false>
                              : chunk_scan_q256_kernel<T, S, NK, false, false, false>);
  const int items = a.batch * a.nchunks * a.nheads;
  const int grid = persistent_grid(kern, kThreads, items);
  kern<<<dim3((unsigned)grid), dim3(kThreads), 0, stream>>>(narrow(a));
  return hipGetLastError();
}

template <typename T, typename S>
hipError_t launch_ts(const ChunkScanArgs& a, hipStream_t stream) {
  switch (a.dstate) {
    case 64: return launch_nk<T, S, 2>(a, stream);
    case 128: return launch_nk<T, S, 4>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool chunk_scan_persistent_supported(const ChunkScanArgs& a, int dtype) {
  // dstate 16 / 32 stay on the generic kernel (this one spills registers there).
  for (int64_t st : {a.sxb, a.sxl, a.sxh, a.sbb, a.sbl, a.sbg, a.scb, a.scl, a.scg, a.sdb, a.sdl, a.sdh, a.syb,
                     a.syl, a.syh, a.szb, a.szl, a.szh})
    if (!fits_i32(st)) return false;
  // y is written (and z read) 16 bytes per lane
  if (reinterpret_cast<uintptr_t>(a.y) % 16 != 0 || a.syb % 8 != 0 || a.syl % 8 != 0 || a.syh % 8 != 0) return false;
  if (a.dskip || a.z) {
    if (!a.dt || !a.cbf) return false;
    if (a.z && (reinterpret_cast<uintptr_t>(a.z) % 16 != 0 || a.szb % 8 != 0 || a.szl % 8 != 0 || a.szh % 8 != 0))
      return false;
  }
  return a.chunk == kQ && (a.dstate == 64 || a.dstate == 128) &&
         (dtype == SSD_DTYPE_BF16 || dtype == SSD_DTYPE_F16);
}

hipError_t launch_chunk_scan_persistent(const ChunkScanArgs& a, int dtype, int state_dtype, hipStream_t stream) {
  if (a.f16s) {
    if (!a.sscale) return hipErrorInvalidValue;
    if (dtype == SSD_DTYPE_BF16) return launch_ts<bf16, f16s_t>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_ts<f16, f16s_t>(a, stream);
    return hipErrorInvalidValue;
  }
  if (state_dtype == SSD_DTYPE_F32) {
    if (dtype == SSD_DTYPE_BF16) return launch_ts<bf16, float>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_ts<f16, float>(a, stream);
  } else if (state_dtype == SSD_DTYPE_BF16) {
    if (dtype == SSD_DTYPE_BF16) return launch_ts<bf16, bf16>(a, stream);
    if (dtype == SSD_DTYPE_F16) return launch_ts<f16, bf16>(a, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ssd
