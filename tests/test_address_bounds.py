"""CPU-side bounds check of the kernels' per-lane global and LDS address
arithmetic at the C1-C5 and R0 shapes (no GPU).

The persistent and DMA-staged kernels form every global address from an item
base (batch, chunk, head or group) plus a per-lane offset (wave, lane, copy
part, loop step), and the global -> LDS copies (global_load_lds) write 16 or
4 bytes per lane at a wave-uniform LDS base.  A wrong lane formula would read
or write outside a tensor or an LDS buffer, which on the GPU is a memory
fault, not a test failure.  Each check below restates one kernel's formulas
in numpy, evaluates them over every workgroup, wave, lane and loop step the
launch runs at a shape, and asserts that every element touched lies inside
its tensor (as an index in range in each dimension, which also holds for
strided views) and every LDS byte inside its buffer.

Kernels per shape: C3, C4 and the R0 layer span (16-bit, chunk 256) run
chunk_prep, the persistent chunk_state / chunk_scan and the state chain; C2
and C5 (f32, chunk 64 / 128) the f32 chunk_scan, chunk_state and chain, and
R0's core (16-bit inputs at chunk 64) the same chunk_state and chain on
16-bit staged rows and the 16-bit chunk_scan for f32 states (also checked at
chunk 128, d_state 64); every shape runs state_passing.  C1 (d_state 16) runs
the generic kernels, whose staging loops bound every row and column by the
shape explicitly (ssd_device.h stage_rows / stage_transposed) instead of by
lane arithmetic.

The restatements are pinned to the source: each check first asserts that
the lines it restates still read as below in the kernel file
(whitespace-normalised), so a change to a kernel's address arithmetic fails
here until the check is updated with it.
"""

import pathlib
import re

import numpy as np
import pytest

SRC = pathlib.Path(__file__).resolve().parent.parent / "workloadsuite_amd" / "csrc"
CUS = 256  # MI355X

# (batch, seqlen, nheads, headdim, dstate, chunk, ngroups, 16-bit inputs)
SHAPES = {
    "C1": (16, 128, 8, 64, 16, 64, 8, False),
    "C2": (8, 2048, 24, 64, 128, 64, 1, False),
    "C3": (4, 4096, 80, 64, 128, 256, 1, True),
    "C4": (1, 65536, 80, 64, 128, 256, 1, True),
    "C5": (64, 512, 64, 64, 64, 128, 8, False),
    "R0": (8, 2048, 128, 64, 128, 64, 8, True),        # the module's core at chunk 64
    "R0-layer": (8, 2048, 128, 64, 128, 256, 8, True),  # the layer span at chunk 256
    # MR's _ssd_core arguments (B / C repeated per head, MR:97-99): one group
    # per head, which ssd_forward keeps at chunk 64
    "R0-repeated": (8, 2048, 128, 64, 128, 64, 128, True),
}

_src_cache = {}


def pin(fname, *snippets):
    """The kernel file still contains each restated line."""
    if fname not in _src_cache:
        _src_cache[fname] = re.sub(r"\s+", " ", (SRC / fname).read_text())
    text = _src_cache[fname]
    for s in snippets:
        assert re.sub(r"\s+", " ", s) in text, f"{fname} no longer contains: {s}"


def inside(name, idx, lo, hi):
    """lo <= idx < hi for every element (idx: array of indices touched)."""
    idx = np.asarray(idx)
    assert idx.size > 0, name
    mn, mx = int(idx.min()), int(idx.max())
    assert lo <= mn and mx < hi, f"{name}: touches [{mn}, {mx}], allowed [{lo}, {hi})"


def f16l_scale_slot(p, t, N):
    """ssd_device.h f16l_scale_slot: the item slot of the scale of row p's n tile t."""
    pin("ssd_device.h", "const int k = p * (N / 16) + t;", "return (k / (N / 2)) * N + N / 2 + k % (N / 2);")
    k = p * (N // 16) + t
    return (k // (N // 2)) * N + N // 2 + k % (N // 2)


def lanes():
    """(wave, lane) grids of an 8-wave workgroup, shapes [8, 1] and [1, 64]."""
    return np.arange(8)[:, None], np.arange(64)[None, :]


def xcd_remap(bid, n):
    """ssd_device.h: xcd_remap (8 XCDs, workgroups dispatched round-robin)."""
    per, rem = n // 8, n % 8
    x, k = bid % 8, bid // 8
    start = np.where(x < rem, x * (per + 1), rem * (per + 1) + (x - rem) * per)
    return start + k


def test_xcd_remap_is_a_permutation():
    pin("ssd_device.h",
        "const int per = nblocks / kXcds, rem = nblocks % kXcds;",
        "const int x = bid % kXcds, k = bid / kXcds;",
        "const int start = x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;",
        "return start + k;")
    for n in list(range(1, 300)) + [1024, 2047, 2048, 20480, 65536 + 3]:
        m = xcd_remap(np.arange(n), n)
        assert np.array_equal(np.sort(m), np.arange(n)), n


@pytest.mark.parametrize("nitems", [1, 7, 320, 5120, 20480, 8192, 16384])
def test_persistent_item_ranges_partition_the_items(nitems):
    """it0 = lb * n / grid, it1 = (lb + 1) * n / grid over every grid size a
    persistent launch can take (one up to two workgroups per CU, capped by the
    item count): the ranges lie in [0, n) and cover it exactly once."""
    pin("ssd_chunk_scan_q256.hip",
        "const int it0 = (int)((int64_t)lb * nitems / gridDim.x);",
        "const int it1 = (int)((int64_t)(lb + 1) * nitems / gridDim.x);")
    for grid in sorted({min(nitems, g) for g in (1, 3, CUS, 2 * CUS, 3 * CUS)}):
        lb = xcd_remap(np.arange(grid), grid)
        it0, it1 = lb * nitems // grid, (lb + 1) * nitems // grid
        inside("it0", it0, 0, nitems)
        inside("it1", it1, 1, nitems + 1)
        cover = np.zeros(nitems, np.int64)
        for a, b in zip(it0, it1):
            cover[a:b] += 1
        assert (cover == 1).all()


def items(B, L, H, Q):
    """item_of(it) for every item: (b, c, h) arrays, heads fastest."""
    nc = L // Q
    it = np.arange(B * nc * H)
    h = it % H
    bc = it // H
    return bc // nc, bc % nc, h


# ---------------------------------------------------------------------------
# chunk-256 persistent chunk_scan (ssd_chunk_scan_q256.hip)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["C3", "C4", "R0-layer"])
@pytest.mark.parametrize("fmt", ["f16s", "split", "bf16"])
def test_chunk_scan_q256_addresses(name, fmt):
    B, L, H, P, N, Q, G, _ = SHAPES[name]
    assert Q == 256 and P == 64
    pin("ssd_chunk_scan_q256.hip",
        "const int64_t xcopy = (int64_t)(lane >> 3) * p.sxl + 8 * ((lane & 7) ^ (lane >> 3));",
        "const int blk = wave + kNW * part;",
        "dma16_at(xg + (int64_t)(8 * blk) * p.sxl, xr_lds + (uint32_t)(b * kQ * kP * (int)sizeof(T) + blk * 1024));",
        "const int scopy = (lane / PPR) * GRS + ((lane % PPR) ^ ssw(wave * RPD + lane / PPR)) * (16 / (int)sizeof(SE));",
        "const int d = wave + kNW * part;",
        "dma16_at(sg + d * RPD * GRS, sr_lds + (uint32_t)(b * kP * RB + d * 1024));",
        "if (part == 1 && wave == 0) dma4_at(p.sscale + item * kP + lane, scl_lds + (uint32_t)(b * kP * 4));",
        "dma16_at(ag + 4 * lane, ar_lds + (uint32_t)(wave * kQ * 4));",
        "dma4_at(dg + (l0 + 64 * wave + lane) * p.sdl, dr_lds + (uint32_t)(b * kQ * 4 + 256 * wave));",
        "const int ycol = 8 * (g >> 1) + 16 * (g & 1);",
        "T* yrow = yg + (int64_t)(16 * (s2 ? tb : ta) + i) * p.syl + ycol;",
        "*reinterpret_cast<u32x4*>(yrow + 32 * pp) = u32x4{w0[0], w1[0], w0[1], w1[1]};",
        "store8<T>(yrow + 32 * pp, __builtin_convertvector(v, frag8<T>));",
        "const int ta = wave, tb = kNT - 1 - wave;",
        "cf[0][kc] = load8<T>(cg + (int64_t)(16 * ta + i) * p.scl + 32 * kc + 8 * g);",
        "const int64_t wbase = (((int64_t)r.b * p.nchunks + r.c) * p.ngroups + r.grp) * kNW + wave;",
        "const f32x4* cb = reinterpret_cast<const f32x4*>(p.cbf) + wbase * (kNPair * 2 * 64) + lane_o;",
        "cbc[k].set(st, cb[(k * 2 + st) * 64]);",
        "const frag8<T>* cb = reinterpret_cast<const frag8<T>*>(p.cbf) + wbase * (kNPair * 64) + lane_o;",
        "zv[s2][pp] = load8<T>(zg + (int64_t)(16 * (s2 ? tb : ta) + i) * p.szl + 32 * pp);")
    wave, lane = lanes()
    g, i = lane >> 4, lane & 15
    parts = np.arange(4)[:, None, None]
    b, c, h = items(B, L, H, Q)
    nc = L // Q
    inside("item b", b, 0, B)
    inside("item c", c, 0, nc)
    inside("item h", h, 0, H)
    # x copy: 8 elements of row l0 + 8 blk + lane / 8 from column 8 ((lane % 8) ^ (lane / 8))
    blk = wave + 8 * parts
    inside("x rows in the chunk", 8 * blk + (lane >> 3), 0, Q)
    xcol = 8 * ((lane & 7) ^ (lane >> 3))
    inside("x columns", np.concatenate([xcol, xcol + 7], None), 0, P)
    inside("x LDS (2 buffers of Q x P x 2 bytes)", 1 * Q * P * 2 + blk * 1024 + 16 * lane + 15, 0, 2 * Q * P * 2)
    # S_in copy (states [b, c, h, P, N] in SE elements, rows of GRS)
    es, grs = {"f16s": (2, 2 * N), "split": (4, N), "bf16": (2, N)}[fmt]
    rb = N * es
    ppr, rpd = rb // 16, 1024 // rb
    scopies = P // rpd // 8
    ssw = (lambda r: r & 15) if ppr >= 16 else (lambda r: (r >> 1) & 7)
    d = wave + 8 * np.arange(scopies)[:, None, None]
    srow = rpd * d + lane // ppr
    spiece = (lane % ppr) ^ ssw(wave * rpd + lane // ppr)
    inside("S_in rows", srow, 0, P)
    inside("S_in pieces within the stored row", spiece, 0, ppr)   # ppr * 16 bytes = the row's data
    inside("S_in element within the row slot", spiece * (16 // es) + 16 // es - 1, 0, grs)
    inside("S_in LDS", 1 * P * rb + d * 1024 + 16 * lane + 15, 0, 2 * P * rb)
    # the ssw the copy uses (from the wave) is the row's own
    assert (ssw(wave * rpd + lane // ppr) == ssw(srow)).all()
    # scales, Acs, dt
    inside("scales per item", lane, 0, P)
    inside("Acs of the item", 4 * lane + 3, 0, Q)
    inside("Acs LDS (one copy per wave)", wave * Q * 4 + 16 * lane + 15, 0, 8 * Q * 4)
    dwave = np.arange(4)[:, None]
    inside("dt rows in the chunk", 64 * dwave + lane, 0, Q)
    inside("dt LDS", 1 * Q * 4 + 256 * dwave + 4 * lane + 3, 0, 2 * Q * 4)
    # y stores (and the epilogue's z loads): rows 16 t + i, 8 columns from ycol + 32 pp
    t = np.stack([wave, 15 - wave])
    inside("y / z rows", 16 * t + i, 0, Q)
    ycol = 8 * (g >> 1) + 16 * (g & 1)
    pp = np.arange(2)[:, None, None]
    inside("y / z columns", ycol + 32 * pp + 7, 0, P)
    # C fragments (rows 16 t + i, columns 32 kc + 8 g .. + 7)
    kc = np.arange(N // 32)[:, None, None]
    inside("C columns", 32 * kc + 8 * g + 7, 0, N)
    # chunk_prep's CB^T fragments: f32x4 index wbase * (9 * 2 * 64) + lane + (2 k + st) * 64
    groups = B * nc * G
    wbase = (np.arange(groups)[:, None] * 8 + np.arange(8)[None, :]).max()
    k = np.arange(9)[:, None, None, None]
    st = np.arange(2)[None, :, None, None]
    cb32 = wbase * (9 * 2 * 64) + lane + (k * 2 + st) * 64
    inside("CB^T f32 fragments", cb32, 0, groups * 8 * 9 * 2 * 64)
    cb16 = wbase * (9 * 64) + lane + k * 64
    inside("CB^T 16-bit fragments (16-byte units)", cb16, 0, groups * 8 * 9 * 2 * 64 // 2)


# ---------------------------------------------------------------------------
# chunk-256 persistent chunk_state and the state chain (ssd_chunk_state_q256.hip)
# ---------------------------------------------------------------------------

def chain_plan(chains, nchunks):
    """chunk_state_chain_plan on a 256-CU device: (nfull, seg_per_chain, seg_len)."""
    pin("ssd_chunk_state_q256.hip",
        "if (4 * chains >= 3 * per_cu * cus) return ChainPlan{(int)chains, 1, a.nchunks};",
        "const int64_t want = cus / rest > 1 ? cus / rest : 1;  // segments per chain",
        "const int seg_len = (int)((a.nchunks + want - 1) / want);",
        "const int segs = (a.nchunks + seg_len - 1) / seg_len;",
        "return ChainPlan{(int)cus, segs, seg_len};")
    per_cu = -(-chains // CUS)
    if 4 * chains >= 3 * per_cu * CUS:
        return chains, 1, nchunks
    if CUS < chains < 2 * CUS:
        rest = chains - CUS
        want = max(CUS // rest, 1)
        seg_len = -(-nchunks // want)
        return CUS, -(-nchunks // seg_len), seg_len
    return None


@pytest.mark.parametrize("name", ["C3", "C4", "R0-layer"])
def test_chunk_state_q256_and_chain_addresses(name):
    B, L, H, P, N, Q, G, _ = SHAPES[name]
    nc = L // Q
    NT = N // 16
    NK = N // 32
    PTW = NT // 2
    pin("ssd_chunk_state_q256.hip",
        "const int nt = wave % NTILE, pt0 = (wave / NTILE) * PTW;",
        "const int srow = (16 * pt0 + i) * N + 16 * nt + 4 * g;",
        "const int blk = wave + kNW * m;",
        "dma16_at(xg + (int64_t)(8 * blk) * p.sxl, xr_lds + (uint32_t)((hb * kQ * kP + blk * 512) * (int)sizeof(T)));",
        "dma16_at(xchain + (l0 + 8 * blk) * p.sxl, xr_lds + (uint32_t)((bs * kQ * kP + blk * 512) * (int)sizeof(T)));",
        "if (wave == kNW - 1) dma16_at(achain + (int64_t)c * kQ + 4 * lane, ar_lds + (uint32_t)(bs * kQ * 4));",
        "if (wave < kQ / 64) dma4_at(dchain + (l0 + 64 * wave + lane) * p.sdl, dr_lds + (uint32_t)((bs * kQ + 64 * wave) * 4));",
        "((((int64_t)b * p.nchunks + c) * p.ngroups + grp) * NTILE + nt) * (kKS * 64) + lane;",
        "const frag8<T>* bnext = btf_of(has_next ? c + 1 : c);",
        "const int row = 16 * (pt0 + 2 * u + (odd ? 1 : 0)) + i;",
        "*reinterpret_cast<u32x4*>(reinterpret_cast<f16*>(item + (int64_t)row * N) + 16 * nt + 4 * (g & ~1)) =",
        "sp.sscale[(((int64_t)b * p.nchunks + c) * p.nheads + h) * kP + row] = __builtin_ldexpf(1.f, e);",
        "const int row = row0 + 16 * (g & 1);",
        "store_f16l<N>(reinterpret_cast<float*>(sg), 16 * (pt0 + 2 * k) + i, nt, g, st_prev[2 * k], st_prev[2 * k + 1]);",
        "for (int u = 0; u < PTW / 2; ++u) store_f16l<N>(sg, 16 * (pt0 + 2 * u) + i, nt, g, st[2 * u], st[2 * u + 1]);",
        "bh = xcd_remap((int)blockIdx.x, plan.nfull);",
        "const int sg = xcd_remap((int)blockIdx.x - plan.nfull, (int)gridDim.x - plan.nfull);",
        "bh = plan.nfull + sg / plan.seg_per_chain;",
        "c0 = (sg % plan.seg_per_chain) * plan.seg_len;",
        "c1 = min(c0 + plan.seg_len, p.nchunks);",
        "if (c0 >= c1) return;  // the whole workgroup, before any barrier",
        "if (g == 0) item[f16l_scale_slot<N>(row0 + 16 * s, nt)] = __builtin_ldexpf(1.f, e);")
    wave, lane = lanes()
    g, i = lane >> 4, lane & 15
    nt, pt0 = wave % NT, (wave // NT) * PTW
    q = np.arange(PTW)[:, None, None]
    # state tiles: rows 16 (pt0 + q) + i, columns 16 nt + 4 g .. + 3 (f32 [P][N])
    inside("state rows", 16 * (pt0 + q) + i, 0, P)
    inside("state columns", 16 * nt + 4 * g + 3, 0, N)
    inside("f16s: f16 columns in the row's first half", 16 * nt + 4 * g + 3, 0, N)
    inside("f16s scales rows", 16 * (pt0 + q) + i, 0, P)
    # 16-byte stores of a tile pair (2u, 2u + 1): row of tile 2u + (g & 1),
    # columns 16 nt + 4 (g & ~1) .. + 7, 16-byte aligned in the row's f16 half
    u = np.arange(PTW // 2)[:, None, None]
    prow = 16 * (pt0 + 2 * u + (g & 1)) + i
    pcol = 16 * nt + 4 * (g & ~1)
    inside("pair store rows", prow, 0, P)
    inside("pair store columns (f16)", pcol + 7, 0, N)
    assert ((pcol * 2) % 16 == 0).all()
    # every (row, column) of the item written exactly once by the 8 waves' pair stores
    seen = np.zeros((P, N), np.int64)
    for wv in range(8):
        ntw, pt0w = wv % NT, (wv // NT) * PTW
        for uu in range(PTW // 2):
            for ln in range(64):
                gg, ii = ln >> 4, ln & 15
                r = 16 * (pt0w + 2 * uu + (gg & 1)) + ii
                c0 = 16 * ntw + 4 * (gg & ~1)
                seen[r, c0:c0 + 8] += 1
    if NT == 8:  # the f16s chain store needs one n tile per wave (d_state 128)
        assert (seen == 1).all()
    # K2's f16 local states: f16 columns in the row's first half, the tile
    # scales packed into the second halves of the item's first rows (every
    # (row, tile)'s slot distinct, none in an f16 half)
    inside("f16 local: f16 slots (f32 units)", (16 * nt + 4 * g + 3) // 2, 0, N // 2)
    pp_, tt_ = np.meshgrid(np.arange(P), np.arange(NT), indexing="ij")
    slot = f16l_scale_slot(pp_, tt_, N)
    inside("f16 local: scale slots in the item", slot, 0, P * N)
    assert len(set(slot.ravel().tolist())) == P * NT and ((slot % N) >= N // 2).all()
    inside("f16 local: the store's tile", nt, 0, NT)
    # x copy parts, Acs, dt: as chunk_scan's (8-row blocks blk = wave + 8 m, m < 4)
    blk = wave + 8 * np.arange(4)[:, None, None]
    inside("x rows in the chunk", 8 * blk + (lane >> 3), 0, Q)
    inside("chain x LDS (2 buffers)", 1 * Q * P * 2 + blk * 512 * 2 + 16 * lane + 15, 0, 2 * Q * P * 2)
    inside("persistent x LDS ([2 halves][2 buffers])", 3 * Q * P * 2 + blk * 512 * 2 + 16 * lane + 15, 0, 4 * Q * P * 2)
    inside("Acs", 4 * lane + 3, 0, Q)
    inside("dt", 64 * np.arange(4)[:, None] + lane, 0, Q)
    # B^T fragments: ((bcg * NTILE + nt) * 8 + ks) * 64 + lane frag8 units
    groups = B * nc * G
    ks = np.arange(8)[:, None, None]
    inside("B^T fragments", ((groups - 1) * NT + nt) * (8 * 64) + ks * 64 + lane, 0, groups * NT * 8 * 64)
    # the chain's workgroups: whole chains and segments, the chunks each walks
    chains = B * H
    plan = chain_plan(chains, nc)
    if plan is None:
        return
    nfull, spc, seg_len = plan
    grid = nfull + (chains - nfull) * spc
    blocks = np.arange(grid)
    local = blocks >= nfull
    # whole chains and segments are each dealt out XCD by XCD
    sg = np.where(local, xcd_remap(np.maximum(blocks - nfull, 0), max(grid - nfull, 1)), 0)
    bh = np.where(local, nfull + sg // spc, xcd_remap(np.minimum(blocks, nfull - 1), nfull))
    c0 = np.where(local, (sg % spc) * seg_len, 0)
    c1 = np.where(local, np.minimum(c0 + seg_len, nc), nc)
    live = c0 < c1
    inside("chain bh", bh[live], 0, chains)
    inside("chain first chunk", c0[live], 0, nc)
    inside("chain end chunk", c1[live], 1, nc + 1)
    # every chunk of every chain walked exactly once
    cover = np.zeros((chains, nc), np.int64)
    for a, s, e in zip(bh[live], c0[live], c1[live]):
        cover[a, s:e] += 1
    assert (cover == 1).all()
    # K2-then-K3 tail of the mixed plan: state_passing over chains [nfull, chains)
    if nfull < chains:
        inside("state_passing chains", np.arange(nfull, chains), 0, chains)


# ---------------------------------------------------------------------------
# chunk_prep (ssd_chunk_prep.hip)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["C3", "C4", "R0-layer"])
def test_chunk_prep_addresses(name):
    B, L, H, P, N, Q, G, _ = SHAPES[name]
    pin("ssd_chunk_prep.hip",
        "constexpr int RB = N * 2;",
        "constexpr int RPD = 1024 / RB;",
        "for (int d = wave; d < kQ / RPD; d += kNW) {",
        "const int r = d * RPD + lane / PPR;",
        "const int piece = (lane % PPR) ^ sw(r);",
        "dma16_at(bg + (int64_t)r * p.sbl + 8 * piece, bl_lds + (uint32_t)(d * 1024));",
        "const int ta = wave, tb = 15 - wave, KA = ta / 2 + 1;",
        "cf[0][kc] = load8<T>(cg + (int64_t)(16 * ta + i) * p.scl + 8 * (4 * kc + g));",
        "f32x4* out = reinterpret_cast<f32x4*>(p.cbf) + (int64_t)(bcg * kNW + wave) * kNPair * 2 * 64 + lane;",
        "frag8<T>* bt_out = reinterpret_cast<frag8<T>*>(p.btf) + (int64_t)bcg * NTILE * 8 * 64 + lane;",
        "for (int f = wave; f < NTILE * 8; f += kNW) {")
    rb = 2 * N
    ppr, rpd = rb // 16, 1024 // rb
    sw = (lambda r: r & 15) if ppr >= 16 else (lambda r: (r >> 1) & 7)
    wave, lane = lanes()
    g, i = lane >> 4, lane & 15
    d = np.arange(Q // rpd)
    r = d[:, None] * rpd + lane // ppr
    inside("B rows", r, 0, Q)
    inside("B elements", 8 * ((lane % ppr) ^ sw(r)) + 7, 0, N)
    inside("B LDS", d[:, None] * 1024 + 16 * lane + 15, 0, Q * rb)
    inside("C rows", 16 * np.stack([wave, 15 - wave]) + i, 0, Q)
    inside("C columns", 8 * (4 * np.arange(N // 32)[:, None, None] + g) + 7, 0, N)
    groups = B * (L // Q) * G
    bcg = groups - 1
    k = np.arange(9)[:, None, None, None]
    st = np.arange(2)[None, :, None, None]
    inside("CB^T out", (bcg * 8 + wave) * 9 * 2 * 64 + lane + (k * 2 + st) * 64, 0, groups * 8 * 9 * 2 * 64)
    f = np.arange(N // 16 * 8)[:, None]
    inside("B^T out", bcg * (N // 16) * 8 * 64 + lane + f * 64, 0, groups * (N // 16) * 8 * 64)


# ---------------------------------------------------------------------------
# f32 chunk_scan and chunk_state / state chain at chunk 64 / 128
# (ssd_chunk_scan_f32.hip, ssd_chunk_state_f32.hip)
# ---------------------------------------------------------------------------

def f32_units(B, L, H, Q, G):
    """launch_qn's units (b, c, group, head slice) and their heads."""
    pin("ssd_chunk_scan_f32.hip",
        "int slices = (int)((cus + bcg - 1) / bcg);",
        "const int hs = (hpg + slices - 1) / slices;",
        "slices = (hpg + hs - 1) / hs;",
        "const int h0 = grp * hpg + slice * hs;",
        "const int h1 = min(h0 + hs, (grp + 1) * hpg);")
    hpg = H // G
    bcg = B * (L // Q) * G
    slices = min(max(-(-CUS // bcg), 1), hpg)
    hs = -(-hpg // slices)
    slices = -(-hpg // hs)
    u = np.arange(bcg * slices)
    slice_, bcgi = u % slices, u // slices
    grp = bcgi % G
    h0 = grp * hpg + slice_ * hs
    h1 = np.minimum(h0 + hs, (grp + 1) * hpg)
    cover = np.zeros((bcg, H), np.int64)
    for k, a, e in zip(bcgi, h0, h1):
        cover[k, a:e] += 1
    # every (b, c) sees every head exactly once, within its group's heads
    assert (cover.reshape(B * (L // Q), G, H).sum(1) == 1).all()
    return h0, h1


@pytest.mark.parametrize("name", ["C2", "C5", "R0", "R0-repeated"])
def test_f32_kernel_addresses(name):
    B, L, H, P, N, Q, G, _ = SHAPES[name]
    assert P == 64 and Q in (64, 128) and N in (64, 128)
    f32_units(B, L, H, Q, G)
    RT = Q // 64
    pin("ssd_chunk_scan_f32.hip",
        "const int blk = wave + kNW * m, r = 4 * blk + (lane >> 4), pc = (lane & 15) ^ (4 * ((r >> 2) & 3));",
        "dma16_at(xg + r * p.sxl + 4 * pc, xs_lds + (uint32_t)((bf * Q * kP + blk * 256) * 4));",
        "const int blk = wave + kNW * m, r = blk * (64 / SPR) + lane / SPR, pc = (lane % SPR) ^ (r & 7);",
        "dma16_at(sg + r * N + 4 * pc, ss_lds + (uint32_t)((bf * kP * N + blk * 256) * 4));",
        "if (wave == kNW - 1 && lane < Q / 4) {",
        "dma16_at(ag + 4 * lane, al_lds + (uint32_t)(bf * Q * 4));",
        "const int part = wave - (kNW - 1 - Q / 64);",
        "dma4_at(dg + (l0 + 64 * part + lane) * p.sdl, dl_lds + (uint32_t)((bf * Q + 64 * part) * 4));",
        "*reinterpret_cast<f32x4*>(yg + (int64_t)(16 * trow[r] + i) * p.syl + 16 * (2 * ph + e) + 4 * g) = acc[r][e];",
        "const int ph = wave >> 2, rg = RT == 1 && ph ? 3 - (wave & 3) : wave & 3;",
        "cf[r][kc] = load8<float>(cg + (16 * trow[r] + i) * p.scl + 32 * kc + 8 * g);",
        "const uint32_t bt_lds = kBinX ? xs_lds + Q * kP * 4 : ss_lds + kP * N * 4;",
        "dma16_at(bg + r * p.sbl + 4 * pc, bt_lds + (uint32_t)(blk * 1024));",
        "const int row = 32 * sb + 16 * st + i, pc = 8 * kc + 2 * g;",
        "bf8.hi = *reinterpret_cast<const f32x4*>(brow + 4 * ((pc + 1) ^ (row & 7)));")
    pin("ssd_chunk_state_f32.hip",
        "if constexpr (sizeof(T) == 4) return 4 * ((l >> 2) & 3);",
        "else return cols * 2 >= 256 ? 2 * (l & 7) : 2 * ((l >> 1) & 3);",
        "return l * cols + EPP * ((col / EPP) ^ swz_x<T>(l, cols)) + col % EPP;",
        "const int ppr = cols * (int)sizeof(T) / 16, r = blk * (64 / ppr) + lane / ppr, pc = (lane % ppr) ^ swz_x<T>(r, cols);",
        "const int r = 32 * ks + 4 * g + (i >> 2), c = c0 + 4 * (i & 3);",
        "return join<T>(lds_read_tr(blk + swz_off<T>(r, c, cols)), lds_read_tr(blk + swz_off<T>(r + 16, c, cols)));",
        "bfr[n][ks] = tr_operand<T>(bl, ks, 16 * (nt0 + n), N, g, i);",
        "bfr[n] = tr_operand<T>(bl, ks, 16 * (nt0 + n), N, g, i);",
        "xr = tr_operand<T>(xb, ks, 16 * (2 * pp + a), kP, g, i);",
        "dma16_at(src + r * ld + (16 / (int)sizeof(T)) * pc, dst + (uint32_t)(blk * 1024));",
        "constexpr int XPW = Q * kP * ES / 1024 / kNW;",
        "constexpr int BPW = Q * N * ES / 1024 / kNW;",
        "*reinterpret_cast<f32x4*>(sg + (16 * (2 * pp + a) + i) * N + 16 * (nt0 + n) + 4 * g) = acc[a][n];",
        "return (16 * (2 * pp + a) + i) * N + 16 * (nt0 + n) + 4 * g;",
        "*reinterpret_cast<f32x4*>(sg + sidx(a, n)) = st[a][n];",
        "*reinterpret_cast<const f32x4*>(sp.init + bh * PN + sidx(a, n))",
        "*reinterpret_cast<f32x4*>(sp.final_state + bh * PN + sidx(a, n)) = st[a][n];",
        "const int pp = wave & 1, nt0 = (wave >> 1) * NTW;",
        "__shared__ float rmax[F16S ? 2 : 1][F16S ? 4 * kP : 1];",
        "if (g == 0) rmax[buf][(wave >> 1) * kP + 16 * (2 * pp + a) + i] = m;",
        "const float* rm = rmax[c & 1];",
        "const int pr = 16 * (2 * pp + a) + i;",
        "const float m = nn_max(nn_max(rm[pr], rm[kP + pr]), nn_max(rm[2 * kP + pr], rm[3 * kP + pr]));",
        "*reinterpret_cast<f16x4*>(reinterpret_cast<f16*>(sg + pr * N) + 16 * (nt0 + n) + 4 * g) = hv;",
        "sp.sscale[(((int64_t)b * p.nchunks + c) * p.nheads + h) * kP + pr] = __builtin_ldexpf(1.f, e);")
    wave, lane = lanes()
    g, i = lane >> 4, lane & 15
    # x copies (chunk_scan, chunk_state, chain): 1 KB = 4 rows of 64 floats
    xpw = Q * P // 256 // 8
    blk = wave + 8 * np.arange(xpw)[:, None, None]
    r = 4 * blk + (lane >> 4)
    inside("x rows", r, 0, Q)
    inside("x floats", 4 * ((lane & 15) ^ (4 * ((r >> 2) & 3))) + 3, 0, P)
    inside("x LDS", (1 * Q * P + blk * 256) * 4 + 16 * lane + 15, 0, 2 * Q * P * 4)
    # S_in copies (chunk_scan): rows of N floats, SPR pieces
    spr = N // 4
    spw = P * N // 256 // 8
    sblk = wave + 8 * np.arange(spw)[:, None, None]
    sr = sblk * (64 // spr) + lane // spr
    inside("S_in rows", sr, 0, P)
    inside("S_in floats", 4 * ((lane % spr) ^ (sr & 7)) + 3, 0, N)
    inside("S_in LDS", (1 * P * N + sblk * 256) * 4 + 16 * lane + 15, 0, 2 * P * N * 4)
    # B copies (chunk_scan): rows of N floats, SPR pieces, into x's second
    # buffer when N <= 64, else S_in's (Q = 64 there); C.B^T reads rows
    # 32 sb + 16 st + i < Q
    bpw = Q * N // 256 // 8
    tblk = wave + 8 * np.arange(bpw)[:, None, None]
    tr = tblk * (64 // spr) + lane // spr
    inside("chunk_scan B rows", tr, 0, Q)
    inside("chunk_scan B floats", 4 * ((lane % spr) ^ (tr & 7)) + 3, 0, N)
    if N <= P:
        inside("chunk_scan B LDS (x buffer 1)", Q * P * 4 + tblk * 1024 + 16 * lane + 15, Q * P * 4, 2 * Q * P * 4)
    else:
        assert Q == 64
        inside("chunk_scan B LDS (S_in buffer 1)", P * N * 4 + tblk * 1024 + 16 * lane + 15, P * N * 4, 2 * P * N * 4)
    sb_, st_ = np.arange(2 * RT)[:, None, None, None], np.arange(2)[None, :, None, None]
    inside("chunk_scan B fragment rows", 32 * sb_ + 16 * st_ + i, 0, Q)
    bpc = 8 * np.arange(N // 32)[:, None, None, None] + 2 * g[..., None] + np.arange(2)
    inside("chunk_scan B fragment floats", 4 * (bpc[..., None] ^ np.arange(8)) + 3, 0, N)
    # x and B copies of chunk_state and the chain (stage_rows), for f32 and
    # 16-bit inputs: rows of `cols` elements in 16-byte pieces, piece k of row
    # r from piece k ^ swz_x(r); operand reads at swz_off (f32: element-wise;
    # 16-bit: the transposing reads' 4-element runs, below)
    for es in (4, 2):
        epp = 16 // es
        lds_e = max(2 * Q * P, Q * P + Q * N)
        for cols, name in ((P, "x"), (N, "B")):
            if es == 4:
                swx = lambda r: 4 * ((r >> 2) & 3)  # noqa: E731
            elif cols * 2 >= 256:
                swx = lambda r: 2 * (r & 7)  # noqa: E731
            else:
                swx = lambda r: 2 * ((r >> 1) & 3)  # noqa: E731
            ppr = cols * es // 16
            ncp = Q * cols * es // 1024
            assert ncp % 8 == 0, (name, es)
            cblk = wave + 8 * np.arange(ncp // 8)[:, None, None]
            cr = cblk * (64 // ppr) + lane // ppr
            inside(f"{name} rows ({es}-byte)", cr, 0, Q)
            inside(f"{name} elements ({es}-byte)", epp * ((lane % ppr) ^ swx(cr)) + epp - 1, 0, cols)
            inside(f"{name} LDS buffer ({es}-byte)", cblk * 1024 + 16 * lane + 15, 0, Q * cols * es)
            if name == "B":
                inside("chunk_state B staging LDS", Q * P * es + cblk * 1024 + 16 * lane + 15, 0, lds_e * es)
            l_ = 32 * np.arange(Q // 32)[:, None, None, None] + 16 * (np.arange(8)[None, :, None, None] >> 2) + 4 * g + (np.arange(8)[None, :, None, None] & 3)
            col = np.arange(cols)[:, None, None, None, None]
            off = l_ * cols + epp * ((col // epp) ^ swx(l_)) + col % epp
            inside(f"{name} operand reads ({es}-byte)", off, 0, Q * cols)
            inside(f"{name} piece swizzle ({es}-byte)", swx(np.arange(Q)), 0, ppr)
            if es == 2:
                # transposing reads: rows 32 ks + 4 g + i / 4 (+ 16), 4 elements
                # from column c0 + 4 (i % 4), c0 = 16 t for the operand's column tile
                ks_ = np.arange(Q // 32)[:, None, None, None]
                t_ = np.arange(cols // 16)[:, None, None]
                r_ = 32 * ks_ + 4 * g + (i >> 2)
                c_ = 16 * t_ + 4 * (i & 3)
                for rr in (r_, r_ + 16):
                    inside(f"{name} tr rows", rr, 0, Q)
                    o = rr * cols + epp * ((c_ // epp) ^ swx(rr)) + c_ % epp
                    inside(f"{name} tr elements", o + 3, 0, Q * cols)
                    assert ((c_ % epp) + 3 < epp).all()     # 4 elements within one piece
                # 8 consecutive rows' 32-byte segments (lanes 0-31 or 32-63 of
                # one read) on distinct 8-byte bank slots of a 256-byte window
                for t in range(cols // 16):
                    for r0 in range(0, Q, 8):
                        rows = np.arange(r0, r0 + 8)[:, None]
                        cc = 16 * t + 4 * np.arange(4)[None, :]
                        byte = 2 * (rows * cols + epp * ((cc // epp) ^ swx(rows)) + cc % epp)
                        assert len(set((byte % 256 // 8).ravel().tolist())) == 32, (name, t, r0)
    # Acs and dt copies
    inside("Acs (lanes < Q / 4)", 4 * np.arange(Q // 4) + 3, 0, Q)
    part = np.arange(Q // 64)[:, None]
    inside("dt", 64 * part + lane, 0, Q)
    # y stores (4 floats): rows 16 t + i (t from the wave's row group), columns 16 (2 ph + e) + 4 g .. + 3
    ph = wave >> 2
    rg = np.where((RT == 1) & (ph > 0), 3 - (wave & 3), wave & 3)
    trow = [rg] + ([7 - rg] if RT == 2 else [])
    jj = np.arange(4)[:, None, None]
    for t in trow:
        inside("y rows", 16 * t + i, 0, Q)
        inside("C rows", 16 * t + i, 0, Q)
    inside("y columns", 16 * (2 * ph + np.arange(2)[:, None, None]) + 4 * g + 3, 0, P)
    inside("C / B columns", 32 * np.arange(N // 32)[:, None, None] + 8 * g + 7, 0, N)
    # state stores, init and final state loads / stores (chunk_state f32,
    # chain; 4 floats): rows 16 (2 pp + a) + i, columns 16 (nt0 + n) + 4 g .. + 3
    pp, nt0 = wave & 1, (wave >> 1) * (N // 64)
    a = np.arange(2)[:, None, None, None]
    n = np.arange(N // 64)[None, :, None, None]
    inside("state rows", 16 * (2 * pp + a) + i, 0, P)
    inside("state columns", 16 * (nt0 + n) + 4 * g + 3, 0, N)
    # the chain's f16s S_in (16-bit inputs): 4 f16 at f16 column 16 (nt0 + n)
    # + 4 g of row pr, inside the row's first half (2 N bytes of its 4 N);
    # row maxima: quarter wave / 2 of row pr, every (quarter, row) written
    # by exactly one lane (g == 0) and the 4 quarters read for each row
    pr = 16 * (2 * pp + a) + i
    inside("f16s S_in f16 columns", 16 * (nt0 + n) + 4 * g + 3, 0, N)
    slots = ((wave >> 1) * P + pr)[..., :16]                   # the lanes with g == 0
    assert sorted(slots.ravel().tolist()) == list(range(4 * P))
    inside("row maxima read", 3 * P + pr, 0, 4 * P)
    inside("row scale (quarter 0, g == 0)", pr, 0, P)


# ---------------------------------------------------------------------------
# chunk_scan for 16-bit inputs with f32 states (ssd_chunk_scan_b16.hip)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("f16s", [False, True])
@pytest.mark.parametrize("Q,N", [(64, 128), (64, 64), (128, 64)])
def test_chunk_scan_b16_addresses(Q, N, f16s):
    """f16s: S_in as f16 rows (the first half of each f32 row) with a scale
    per row, read as they lie; otherwise f32 rows split in LDS into hi / lo
    pairs.  Either way S_in's buffer first stages the chunk's B rows."""
    P, RT = 64, Q // 64
    pin("ssd_chunk_scan_b16.hip",
        "constexpr int SRB = F16S ? N * 2 : N * 4;",
        "constexpr int SPR = SRB / 16;",
        "constexpr int XPW = Q * kP * 2 / 1024 / kNW;",
        "constexpr int SPW = kP * SRB / 1024 / kNW;",
        "constexpr int BPR = N * 2 / 16;",
        "constexpr int BPW = Q * N * 2 / 1024 / kNW;",
        "constexpr int SSB = kP * SRB > Q * N * 2 ? kP * SRB : Q * N * 2;",
        "__shared__ __attribute__((aligned(1024))) T xs[2][Q * kP];",
        "__shared__ __attribute__((aligned(1024))) float ss[SSB / 4];",
        "__shared__ __attribute__((aligned(16))) float scl[F16S ? kP : 4];",
        "const int64_t xcopy = (int64_t)(lane >> 3) * p.sxl + 8 * ((lane & 7) ^ (lane >> 3));",
        "dma16_at(xg + (int64_t)(8 * blk) * p.sxl, xs_lds + (uint32_t)((bf * Q * kP) * 2 + blk * 1024));",
        "if constexpr (!F16S) return r & 7;",
        "else if constexpr (SPR >= 16) return r & 15;",
        "else return (r >> 1) & 7;",
        "const int blk = wave + kNW * m, r = blk * (64 / SPR) + lane / SPR, pc = (lane % SPR) ^ ssw(r);",
        "dma16_at(sg + r * (N * 4) + 16 * pc, ss_lds + (uint32_t)(blk * 1024));",
        "if (wave == 0) dma4_at(p.sscale + item * kP + lane, scl_lds);",
        "const int row = v / (N / 8), q = v % (N / 8);",
        "float* ph_ = &ss[row * N + 4 * ((2 * q) ^ (row & 7))];",
        "float* pl_ = &ss[row * N + 4 * ((2 * q + 1) ^ (row & 7))];",
        "const int blk = wave + kNW * m, r = blk * (64 / BPR) + lane / BPR, pc = (lane % BPR) ^ (r % BPR);",
        "dma16_at(bg + r * p.sbl + 8 * pc, bt_lds + (uint32_t)(blk * 1024));",
        "const frag8<T> bf8 = *reinterpret_cast<const frag8<T>*>(bt + row * N + 8 * ((4 * kc + g) ^ (row % BPR)));",
        "cf[r][kc] = load8<T>(cg + (16 * trow[r] + i) * p.scl + 32 * kc + 8 * g);",
        "for (int e = 0; e < 2; ++e) xoff[e] = r * kP + 8 * ((2 * (2 * ph + e) + ((i & 3) >> 1)) ^ x7) + 4 * (i & 1);",
        "const T* a0 = xb + xoff[e] + (32 * sb) * kP;",
        "const int row = 16 * (2 * ph + e) + i, q = 4 * kc + g;",
        "const unsigned char* srow = sb_ + row * SRB;",
        "const f16x8 a = *reinterpret_cast<const f16x8*>(srow + 16 * (q ^ ssw(row)));",
        "const frag8<T> hi = *reinterpret_cast<const frag8<T>*>(srow + 16 * ((2 * q) ^ ssw(row)));",
        "const frag8<T> lo = *reinterpret_cast<const frag8<T>*>(srow + 16 * ((2 * q + 1) ^ ssw(row)));",
        "for (int e = 0; e < 2; ++e) sc[e] = *reinterpret_cast<const f32x4*>(&scl[16 * (2 * ph + e) + 4 * g]);",
        "*reinterpret_cast<vec4<T>*>(yg + (int64_t)(16 * trow[r] + i) * p.syl + 16 * (2 * ph + e) + 4 * g) = o;",
        "const int ph = wave >> 2, rg = RT == 1 && ph ? 3 - (wave & 3) : wave & 3;")
    wave, lane = lanes()
    g, i = lane >> 4, lane & 15
    srb = 2 * N if f16s else 4 * N          # bytes of an S_in row in LDS
    spr = srb // 16
    ssb = max(P * srb, Q * N * 2)            # S_in's buffer, which also stages B

    def ssw(r):
        if not f16s:
            return r & 7
        return r & 15 if spr >= 16 else (r >> 1) & 7
    # x copies: 1 KB blocks of 8 rows of 64 16-bit elements
    xpw = Q * P * 2 // 1024 // 8
    blk = wave + 8 * np.arange(xpw)[:, None, None]
    xr = 8 * blk + (lane >> 3)
    inside("x rows", xr, 0, Q)
    inside("x elements", 8 * ((lane & 7) ^ (lane >> 3)) + 7, 0, P)
    inside("x LDS (2 buffers)", 1 * Q * P * 2 + blk * 1024 + 16 * lane + 15, 0, 2 * Q * P * 2)
    # S_in copies: rows of srb bytes (f16s: the f16 half of each 4 N-byte row)
    spw = P * srb // 1024 // 8
    assert spw >= 1
    sblk = wave + 8 * np.arange(spw)[:, None, None]
    sr = sblk * (64 // spr) + lane // spr
    inside("S_in rows", sr, 0, P)
    inside("S_in pieces", (lane % spr) ^ ssw(sr), 0, spr)
    inside("S_in bytes of the row", 16 * ((lane % spr) ^ ssw(sr)) + 15, 0, srb)
    inside("S_in LDS", sblk * 1024 + 16 * lane + 15, 0, ssb)
    assert P * srb == 1024 * 8 * spw            # the copies cover every row once
    if f16s:
        inside("S_in row scales (wave 0)", lane, 0, P)
    else:
        # in-place conversion: pair q of row `row`, pieces (2 q) ^ (row & 7) and (2 q + 1) ^ (row & 7)
        v = np.arange(P * (N // 8))
        row, q = v // (N // 8), v % (N // 8)
        inside("S_in convert floats", row * N + 4 * np.maximum((2 * q) ^ (row & 7), (2 * q + 1) ^ (row & 7)) + 3,
               0, P * N)
        assert (ssw(row) == (row & 7)).all()       # the copies' swizzle
    # B copies (N 16-bit elements per row, BPR pieces) into S_in's buffer
    bpr = N * 2 // 16
    bpw = Q * N * 2 // 1024 // 8
    bblk = wave + 8 * np.arange(bpw)[:, None, None]
    br = bblk * (64 // bpr) + lane // bpr
    inside("B rows", br, 0, Q)
    inside("B elements", 8 * ((lane % bpr) ^ (br % bpr)) + 7, 0, N)
    inside("B LDS (in S_in's buffer)", bblk * 1024 + 16 * lane + 15, 0, ssb)
    # C.B^T operand reads: rows 32 sb + 16 st + i < Q, pieces (4 kc + g) ^ (row % BPR)
    kc = np.arange(N // 32)[:, None, None, None]
    rowb = 32 * np.arange(2 * RT)[:, None, None] + 16 * np.arange(2)[:, None] + i
    inside("C.B^T B rows", rowb, 0, Q)
    inside("C.B^T B elements", 8 * ((4 * kc + g.reshape(1, 1, 1, 64)) ^ (rowb[None] % bpr)) + 7, 0, N)
    # C fragments and y stores: rows 16 t + i, t from the wave's row group
    ph = wave >> 2
    rg = np.where((RT == 1) & (ph > 0), 3 - (wave & 3), wave & 3)
    trow = [rg] + ([7 - rg] if RT == 2 else [])
    for t in trow:
        inside("C / y rows", 16 * t + i, 0, Q)
    inside("C columns", 32 * kc + 8 * g + 7, 0, N)
    inside("y columns", 16 * (2 * ph + np.arange(2)[:, None, None]) + 4 * g + 3, 0, P)
    # S_in operand reads: f16s piece q, else the hi / lo pieces 2 q, 2 q + 1
    e_ = np.arange(2)[:, None, None, None]
    srow_ = 16 * (2 * ph[..., None] + e_) + i[..., None]
    qq = 4 * np.arange(N // 32)[:, None, None, None, None] + g[..., None]
    inside("S_in operand rows", srow_, 0, P)
    piece = qq ^ ssw(srow_) if f16s else np.maximum((2 * qq) ^ ssw(srow_), (2 * qq + 1) ^ ssw(srow_))
    inside("S_in operand bytes", 16 * piece + 15, 0, srb)
    if f16s:
        # the 16 lanes of one read (one g) hit 16 distinct 16-byte bank slots
        slot = (((srow_ * srb + 16 * (qq ^ ssw(srow_))) % 256) // 16)[..., 0]   # [kc, e, wave, lane]
        for k in range(slot.shape[0]):
            for e in range(2):
                for gg in range(4):
                    got = slot[k, e, :, 16 * gg:16 * gg + 16]
                    assert all(len(set(r.tolist())) == 16 for r in got), (k, e, gg)
        inside("row scale reads", 16 * (2 * ph + np.arange(2)[:, None, None]) + 4 * g + 3, 0, P)
    # x^T operand reads (ds_read_b64_tr_b16, 4 elements): rows 4 g + i / 4 + 16 h + 32 sb,
    # columns 8 ((2 pt + (i & 3) / 2) ^ (row & 7)) + 4 (i & 1) .. + 3
    r4 = 4 * g + (i >> 2)
    pt = 2 * ph[..., None] + e_
    col = 8 * ((2 * pt + ((i & 3) >> 1)) ^ (r4 & 7)) + 4 * (i & 1)
    inside("x^T columns", col + 3, 0, P)
    inside("x^T rows", r4 + 16 + 32 * (2 * RT - 1), 0, Q)


# ---------------------------------------------------------------------------
# state_passing (ssd_state_passing.hip)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", list(SHAPES))
def test_state_passing_addresses(name):
    B, L, H, P, N, Q, G, _ = SHAPES[name]
    pin("ssd_state_passing.hip",
        "const int bh = p.bh_begin + (int)blockIdx.x / blocks_per_bh;",
        "const int v = (blockIdx.x % blocks_per_bh) * 256 + threadIdx.x;",
        "if (v >= vec_per_bh) return;",
        "const int row = v / TPR, col = SPT * (v % TPR);",
        "float* elem = base + SPT * (int64_t)v;",
        "__builtin_nontemporal_store(hv, reinterpret_cast<H*>(hrow + c * 2 * cstride));",
        "constexpr int spt = 8, unroll = 2;",
        "const int c = min(c0 + u, nchunks - 1);",
        "const float* rscale = base + f16l_scale_slot<N>(row, col / 16);",
        "const H* q = reinterpret_cast<const H*>(hrow + c * 2 * cstride);",
        "const float sc = rscale[c * cstride];")
    PN = P * N
    nc = L // Q
    chains = B * H
    for per_thread in (4, 8):  # f32 / split kernels (4) and the f16s kernel (spt)
        vec = PN // per_thread
        bpb = -(-vec // 256)
        blocks = np.arange(chains * bpb)
        bh = blocks // bpb
        v = (blocks % bpb)[:, None] * 256 + np.arange(256)[None, :]
        v = v[v < vec]
        inside("chains", bh, 0, chains)
        inside("state elements of a chain", per_thread * v + per_thread - 1, 0, PN)
        if N in (64, 128):
            tpr = N // per_thread
            row, col = v // tpr, per_thread * (v % tpr)
            inside("f16s rows", row, 0, P)
            inside("f16s f16 columns (the row's first half)", col + per_thread - 1, 0, N)
            # f16 local states in: the same f16 slots, and the row's packed scale
            inside("f16 local scale slot", f16l_scale_slot(row, col // 16, N), 0, PN)
            assert ((col + per_thread - 1) // 16 == col // 16).all()
    # the chunk index every (clamped) load of the pipelined chain uses (batches of 2, 4 or 8)
    for unroll in (2, 4, 8):
        for nchunks in sorted({1, 2, 7, 16, 17, nc}):
            c0 = np.arange(0, nchunks + 2 * unroll, unroll)
            c = np.minimum(c0[:, None] + np.arange(unroll)[None, :], nchunks - 1)
            inside("chain chunk", c, 0, nchunks)


# ---------------------------------------------------------------------------
# the one-launch forward for small states (ssd_small.hip)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("es", [4, 2])
@pytest.mark.parametrize("Q,N", [(64, 16), (64, 32), (128, 16)])
@pytest.mark.parametrize("PS", [1, 2])
def test_small_forward_addresses(Q, N, PS, es):
    """Every LDS index of each phase inside its array, every global column
    inside the workgroup's p range (two workgroups per chain take halves of
    p), and each workgroup's y, state and final-state writes a partition of
    its part; C1's shape and the other supported (chunk, d_state) pairs, f32
    and 16-bit inputs."""
    pin("ssd_small.hip",
        "constexpr int PP = kP / PS;",
        "constexpr int QT = PP / 16;",
        "constexpr int XPR = PP / VPP;",
        "constexpr int XPT = Q * XPR / kT;",
        "constexpr int BPT = (Q * BPR + kT - 1) / kT;",
        "const int bh = blockIdx.x / PS, pc0 = PP * (blockIdx.x % PS);",
        "const int e = t + kT * k, r = e / XPR, q = e % XPR;",
        "xr[k] = *reinterpret_cast<const u32x4*>(xg + (l0 + r) * p.sxl + VPP * q);",
        "for (int j = 0; j < VPP; ++j) xt[VPP * q + j][r] = v[j];",
        "acc = mfma4(ld4(&cs[16 * r + i][16 * nb + 4 * g]), ld4(&bs[16 * cc + i][16 * nb + 4 * g]), acc);",
        "wl[l][s] = s <= l ? acc[jj] * exp2f(acl[l] - as) * ds : 0.f;",
        "constexpr int QPW = R == 4 ? QT / 2 : QT;",
        "const int r = half ? R - 1 - wave : wave;",
        "const int q0 = R == 4 ? QPW * half : 0;",
        "for (int sb = 0; sb <= r; ++sb) {",
        "yrow[16 * (q0 + qq) + i] = from_f32<T>(",
        "const int tile = wave + 4 * k, q = tile % QT, m = tile / QT;",
        "acc = mfma4(ld4(&xt[16 * q + i][16 * lb + 4 * g]), ld4(&bwt[16 * m + i][16 * lb + 4 * g]), acc);",
        "p.final_state[(int64_t)bh * kP * N + (int64_t)(pc0 + pp) * N + n] = snew[k][jj];",
        "ss[pp][n] = init ? p.init[(int64_t)bh * kP * N + (int64_t)pc0 * N + e] : 0.f;")
    P, T = 64, 256
    PP, VPP = P // PS, 16 // es
    QT, XPR, BPR = PP // 16, PP // VPP, N // VPP
    XPT, BPT = Q * XPR // T, -(-(Q * BPR) // T)
    R, QS, NS, NT = Q // 16, Q + 4, N + 4, N // 16
    assert XPT * T == Q * XPR
    lds_bytes = 4 * (PP * QS + 2 * Q * NS + N * QS + Q * QS + PP * NS + 4 * Q)
    assert lds_bytes <= 160 * 1024
    t = np.arange(T)
    lane, wave = t % 64, t // 64
    g, i = lane // 16, lane % 16
    # x pieces: rows and global columns (pc0 + ...) of this workgroup
    e = (t[None, :] + T * np.arange(XPT)[:, None]).ravel()
    r, q = e // XPR, e % XPR
    inside("x rows", r, 0, Q)
    inside("x columns of the part", VPP * q + VPP - 1, 0, PP)
    eb = (t[None, :] + T * np.arange(BPT)[:, None]).ravel()
    eb = eb[eb < Q * BPR]
    inside("B / C rows", eb // BPR, 0, Q)
    inside("B / C columns", VPP * (eb % BPR) + VPP - 1, 0, N)
    # W tiles (causal), y tiles, state tiles
    taus = np.arange(R * (R + 1) // 2)
    rr = np.array([max(k for k in range(R) if k * (k + 1) // 2 <= tau) for tau in taus])
    cc = taus - rr * (rr + 1) // 2
    assert (cc <= rr).all() and len(set(zip(rr, cc))) == len(taus)
    QPW = QT // 2 if R == 4 else QT
    covered = np.zeros((Q, PP), np.int64)
    for w in range(4):
        for half in range(2):
            row_t = R - 1 - w if half else w
            q0 = QPW * half if R == 4 else 0
            for qq in range(QPW):
                col = 16 * (q0 + qq) + np.arange(16)
                inside("y p tiles", col, 0, PP)
                for gg in range(4):
                    for jj in range(4):
                        covered[16 * row_t + 4 * gg + jj, col] += 1
    assert (covered == 1).all(), "every y element of the part written once"
    TS = QT * NT
    st = np.zeros((PP, N), np.int64)
    for w in range(4):
        for k in range(-(-TS // 4)):
            tile = w + 4 * k
            if tile < TS:
                qt, m = tile % QT, tile // QT
                for gg in range(4):
                    for jj in range(4):
                        st[16 * qt + 4 * gg + jj, 16 * m + np.arange(16)] += 1
    assert (st == 1).all(), "every state element of the part written once"
    # init / final: the part's rows of the [P, N] state
    ei = np.arange(PP * N)
    for pc0 in range(0, P, PP):
        inside("state element", pc0 * N + ei, 0, P * N)
