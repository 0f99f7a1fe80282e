"""CPU-only checks of the C ABI: the library loads, exports every symbol
include/ssd.h declares, and rejects invalid arguments on the host before any
device call (the failure handling of the path, forced from the host)."""

import ctypes
import os
import re

import pytest
import torch

from workloadsuite_amd import _lib
from workloadsuite_amd import ssd as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ssd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(ssd_[a-z_]+)\s*\(", text, flags=re.M)))


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    declared = header_functions()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.ssd_abi_version() == _lib.SSD_ABI_VERSION


def d(**kw):
    base = dict(batch=2, seqlen=256, nheads=8, headdim=64, dstate=64, ngroups=2, chunk=64)
    base.update(kw)
    return _lib.SSDDims(*[base[k] for k in ("batch", "seqlen", "nheads", "headdim", "dstate", "ngroups", "chunk")])


@pytest.mark.parametrize("kw,code", [
    (dict(), 0),
    (dict(seqlen=100), -3),
    (dict(nheads=6, ngroups=4), -4),
    (dict(headdim=32), -6),
    (dict(dstate=48), -7),
    (dict(dstate=256), -7),
    (dict(chunk=32, seqlen=64), -8),
    (dict(batch=0), -2),
    (dict(chunk=0), -2),
])
def test_check_dims_codes(kw, code):
    lib = _lib.load()
    dims = d(**kw)
    assert lib.ssd_check_dims(ctypes.byref(dims), _lib.DTYPE_BF16) == code


def test_check_dims_dtype_and_null():
    lib = _lib.load()
    dims = d()
    assert lib.ssd_check_dims(ctypes.byref(dims), 7) == -5
    assert lib.ssd_check_dims(None, 0) == -1


def test_strerror_names_every_code():
    lib = _lib.load()
    for code in range(-12, 1):
        msg = lib.ssd_strerror(code).decode()
        assert msg and "unknown" not in msg
    assert "unknown" in lib.ssd_strerror(-99).decode()


def test_workspace_bytes_layout():
    lib = _lib.load()
    dims = d()
    n32 = lib.ssd_workspace_bytes(ctypes.byref(dims), _lib.DTYPE_F32)
    n16 = lib.ssd_workspace_bytes(ctypes.byref(dims), _lib.DTYPE_BF16)
    bhc = 2 * 8 * 4
    states32 = bhc * 64 * 64 * 4
    assert n32 >= bhc * 64 * 4 + bhc * 4 + states32 and n32 % 256 == 0
    # f32 states also carry the f16s hand-over's row scales ([b, c, h, P] f32,
    # read by the 16-bit chunk_scan at chunk 64 / 128)
    assert n32 - n16 == states32 // 2 + bhc * 64 * 4
    bad = d(seqlen=100)
    assert lib.ssd_workspace_bytes(ctypes.byref(bad), _lib.DTYPE_F32) == 0
    # chunk 256, dstate 128: also chunk_prep's CB^T fragments (8 waves x 9 steps
    # x 2 sub-tiles x 1 KB) and B^T fragments (8 n tiles x 8 steps x 1 KB) per group
    big = d(seqlen=1024, chunk=256, dstate=128, ngroups=2)
    groups = 2 * 4 * 2
    base = 2 * 8 * 4 * (256 * 4 + 4 + 64 * 128 * 4)
    assert lib.ssd_workspace_bytes(ctypes.byref(big), _lib.DTYPE_F32) >= base + groups * (144 + 64) * 1024


def test_entry_points_reject_null_and_bad_strides_before_launch():
    lib = _lib.load()
    dims = d()
    s4 = (ctypes.c_int64 * 4)(256 * 8 * 64, 8 * 64, 64, 1)
    s3 = (ctypes.c_int64 * 3)(256 * 8, 8, 1)
    bs4 = (ctypes.c_int64 * 4)(256 * 2 * 64, 2 * 64, 64, 1)
    fake = ctypes.c_void_p(0x100000)  # never dereferenced: validation fails first
    # null x
    assert lib.ssd_chunk_state(ctypes.byref(dims), 1, None, s4, fake, bs4, None, None, fake, fake, 0, None, None) == -1
    # inner stride != 1
    bad = (ctypes.c_int64 * 4)(256 * 8 * 64, 8 * 64, 1, 8)
    assert lib.ssd_chunk_state(ctypes.byref(dims), 1, fake, bad, fake, bs4, None, None, fake, fake, 0, None, None) == -9
    # misaligned base pointer
    mis = ctypes.c_void_p(0x100002)
    assert lib.ssd_chunk_state(ctypes.byref(dims), 1, mis, s4, fake, bs4, None, None, fake, fake, 0, None, None) == -10
    # row stride not a multiple of 16 bytes
    odd = (ctypes.c_int64 * 4)(256 * 8 * 64, 8 * 64 + 3, 64, 1)
    assert lib.ssd_chunk_state(ctypes.byref(dims), 1, fake, odd, fake, bs4, None, None, fake, fake, 0, None, None) == -10
    # bf16 states with f32 inputs are not supported
    assert lib.ssd_chunk_state(ctypes.byref(dims), 0, fake, s4, fake, bs4, None, None, fake, fake, 1, None, None) == -5
    # workspace too small / misaligned
    assert lib.ssd_forward(ctypes.byref(dims), 1, fake, s4, fake, s3, fake, bs4, fake, bs4, None, None, None,
                           fake, s4, None, fake, 16, 0, None) == -11
    assert lib.ssd_forward(ctypes.byref(dims), 1, fake, s4, fake, s3, fake, bs4, fake, bs4, None, None, None,
                           fake, s4, None, ctypes.c_void_p(0x100010), 1 << 30, 0, None) == -10
    # chunk_prep: nothing to do for f32 inputs or chunk 64; otherwise checked like a workspace
    big = d(seqlen=512, chunk=256, dstate=128)
    n = lib.ssd_chunk_prep_bytes(ctypes.byref(big))
    assert n > 0 and lib.ssd_chunk_prep_bytes(ctypes.byref(dims)) == 0
    assert lib.ssd_chunk_prep(ctypes.byref(big), 0, fake, bs4, fake, bs4, None, 0, None) == 0
    assert lib.ssd_chunk_prep(ctypes.byref(dims), 1, fake, bs4, fake, bs4, None, 0, None) == 0
    assert lib.ssd_chunk_prep(ctypes.byref(big), 1, fake, bs4, fake, bs4, None, n, None) == -1
    assert lib.ssd_chunk_prep(ctypes.byref(big), 1, fake, bs4, fake, bs4, ctypes.c_void_p(0x100010), n, None) == -10
    assert lib.ssd_chunk_prep(ctypes.byref(big), 1, fake, bs4, fake, bs4, fake, n - 256, None) == -11
    # state passing: misaligned initial state
    assert lib.ssd_state_passing(ctypes.byref(dims), fake, 0, None, fake, ctypes.c_void_p(0x100004), None, None) == -10
    # the f16s format needs its scales array (and a shape the chunk-256 kernels take)
    big256 = _lib.SSDDims(1, 512, 8, 64, 128, 1, 256)
    assert lib.ssd_state_passing(ctypes.byref(big256), fake, 5, None, fake, None, None, None) == -1
    assert lib.ssd_state_passing(ctypes.byref(big256), fake, 5, ctypes.c_void_p(0x100002), fake, None, None, None) == -10
    small_n = _lib.SSDDims(1, 512, 8, 64, 32, 1, 256)
    assert lib.ssd_state_passing(ctypes.byref(small_n), fake, 5, fake, fake, None, None, None) == -7
    # chunk_state + state_passing in one entry point: the same operand checks, plus the decay and
    # the split format's type (the inputs' own)
    csp = lib.ssd_chunk_state_passing
    assert csp(ctypes.byref(dims), 1, None, s4, fake, bs4, None, None, fake, fake, None, None, fake, 0, None, None, None) == -1
    assert csp(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, None, None, None, fake, 0, None, None, None) == -1
    assert csp(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, fake, None, None, None, 0, None, None, None) == -1
    assert csp(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, fake, None, None,
               ctypes.c_void_p(0x100004), 0, None, None, None) == -10
    assert csp(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, fake, None, None, fake, 0, None,
               ctypes.c_void_p(0x100004), None) == -10
    # split pairs of the other 16-bit type, or of f32 inputs: unsupported
    assert csp(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, fake, None, None, fake,
               _lib.STATE_SPLIT_F16, None, None, None) == -5
    assert csp(ctypes.byref(dims), 0, fake, s4, fake, bs4, None, None, fake, fake, None, None, fake,
               _lib.STATE_SPLIT_BF16, None, None, None) == -5
    # the f16s format needs its scales array
    assert csp(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, fake, None, None, fake,
               _lib.STATE_F16S, None, None, None) == -1
    assert csp(ctypes.byref(dims), 1, fake, bad, fake, bs4, None, None, fake, fake, None, None, fake, 0, None, None, None) == -9


def test_python_op_refuses_cpu_tensors_instead_of_falling_back():
    X = torch.zeros(1, 64, 2, 64)
    A = torch.zeros(1, 64, 2)
    B = torch.zeros(1, 64, 1, 16)
    with pytest.raises(ValueError, match="HIP devices only"):
        S.ssd_forward(X, A, B, B, 64)


@pytest.mark.parametrize("kw,msg", [
    (dict(L=96), "multiple of chunk"),
    (dict(h=3, g=2), "divisible by n_groups"),
    (dict(bdtype=torch.float16), "dtype"),
])
def test_python_op_shape_errors_mirror_reference(kw, msg):
    L, h, g = kw.get("L", 128), kw.get("h", 4), kw.get("g", 2)
    X = torch.zeros(1, L, h, 64)
    A = torch.zeros(1, L, h)
    B = torch.zeros(1, L, g, 16, dtype=kw.get("bdtype", torch.float32))
    with pytest.raises(ValueError, match=msg):
        S.ssd_forward(X, A, B, B, 64)


def test_unsupported_dstate_raises_library_error():
    with pytest.raises(S.SSDError, match="d_state"):
        S.workspace_bytes(1, 64, 2, 64, 48, 1, 64)


def test_layer_entry_points_validate_on_the_host():
    lib = _lib.load()
    dims = d()
    fake = ctypes.c_void_p(0x100000)
    s3 = (ctypes.c_int64 * 3)(256 * 1000, 1000, 1)
    bs4 = (ctypes.c_int64 * 4)(256 * 1000, 1000, 64, 1)
    prm = _lib.SSDLayerParams(5, 0x100000, 0, 0x100000, 0x100000, 0)
    args = (fake, s3, fake, s3, fake, fake, fake, fake, None)
    assert lib.ssd_layer_prep(ctypes.byref(dims), 2, ctypes.byref(prm), *args) == -13
    prm.conv_kernel = 0
    assert lib.ssd_layer_prep(ctypes.byref(dims), 2, ctypes.byref(prm), *args) == -13
    prm.conv_kernel = 4
    prm.conv_w = None
    assert lib.ssd_layer_prep(ctypes.byref(dims), 2, ctypes.byref(prm), *args) == -1
    prm.conv_w = 0x100000
    assert lib.ssd_layer_prep(ctypes.byref(dims), 2, None, *args) == -1
    # x_out must be 16-byte aligned for the kernels that read it
    assert lib.ssd_layer_prep(ctypes.byref(dims), 2, ctypes.byref(prm), fake, s3, fake, s3,
                              ctypes.c_void_p(0x100008), fake, fake, fake, None) == -10
    # bad x stride
    bad = (ctypes.c_int64 * 3)(256 * 1000, 1000, 2)
    assert lib.ssd_layer_prep(ctypes.byref(dims), 2, ctypes.byref(prm), fake, bad, fake, s3,
                              fake, fake, fake, fake, None) == -9
    # workspace: x (f16) and dt (f32) ahead of the core's f32-state workspace,
    # which is sized at chunk 256 for 16-bit inputs when L allows it
    n = lib.ssd_layer_workspace_bytes(ctypes.byref(dims), 2)
    tokens = 2 * 256
    core = d(chunk=256)
    assert n == tokens * 8 * 64 * 2 + tokens * 8 * 4 + lib.ssd_workspace_bytes(ctypes.byref(core), 0)
    f32 = lib.ssd_layer_workspace_bytes(ctypes.byref(dims), 0)
    assert f32 == tokens * 8 * 64 * 4 + tokens * 8 * 4 + lib.ssd_workspace_bytes(ctypes.byref(dims), 0)
    odd = d(seqlen=320)
    assert lib.ssd_layer_workspace_bytes(ctypes.byref(odd), 2) == (
        2 * 320 * 8 * 64 * 2 + 2 * 320 * 8 * 4 + lib.ssd_workspace_bytes(ctypes.byref(odd), 0))
    ys = (ctypes.c_int64 * 3)(256 * 512, 512, 1)
    fwd = lambda ws, nb: lib.ssd_layer_forward(ctypes.byref(dims), 2, ctypes.byref(prm), fake, s3, fake, s3,  # noqa: E731
                                               fake, bs4, fake, bs4, fake, s3, fake, ys, ws, nb, None)
    assert fwd(fake, n - 1) == -11
    assert fwd(ctypes.c_void_p(0x100010), n) == -10
    assert fwd(None, n) == -1
    prm.conv_kernel = 7
    assert fwd(fake, n) == -13


def test_build_rejects_kernels_with_scratch():
    """build.py reads hipcc's per-kernel resource remarks and names every
    kernel that spills registers to scratch (the build then fails)."""
    from workloadsuite_amd import build
    text = "\n".join([
        "a.hip:1:1: remark: Function Name: _Zspill [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark: Function Name: _Zclean [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build._spills(text) == [("_Zspill", 12)]
    assert "-Rpass-analysis=kernel-resource-usage" in build.RESOURCE_FLAGS


def test_forward_chunk_routes_16bit_small_chunks_to_256():
    """ssd_forward_chunk: the chunk ssd_forward runs at.  16-bit inputs with
    f32 states (or F16S), L % 256 == 0 and dstate 64 / 128 run chunk 64 / 128
    at 256, unless that workspace would be the larger one (B and C given per
    head, as MR's _ssd_core passes them after the repeat: chunk_prep's
    per-group operands then outgrow the states saved)."""
    lib = _lib.load()
    q = lambda dtype, sd=_lib.DTYPE_F32, **kw: lib.ssd_forward_chunk(ctypes.byref(r0(**kw)), dtype, sd)  # noqa: E731
    assert q(_lib.DTYPE_F16) == 256 and q(_lib.DTYPE_BF16) == 256
    assert q(_lib.DTYPE_F16, _lib.STATE_F16S) == 256
    assert q(_lib.DTYPE_F16, chunk=128) == 256 and q(_lib.DTYPE_F16, chunk=256) == 256
    assert q(_lib.DTYPE_F32) == 64                                   # no chunk-256 f32 path
    assert q(_lib.DTYPE_F16, seqlen=2048 + 64) == 64                 # L % 256 != 0
    assert q(_lib.DTYPE_F16, dstate=32) == 64                        # not a persistent-kernel shape
    assert q(_lib.DTYPE_F16, _lib.DTYPE_BF16) == 64                  # bf16 states keep the chunk
    assert q(_lib.DTYPE_F16, _lib.STATE_SPLIT_F16) == 64             # so does the split format
    assert q(_lib.DTYPE_F16, ngroups=128) == 64                      # per-head B / C (MR's _ssd_core)
    assert q(_lib.DTYPE_F16, seqlen=100) == 0                        # invalid dims
    # routed only where the chunk-256 workspace is not larger than the caller's
    for g in (1, 8, 32, 64, 128):
        dims = r0(ngroups=g)
        d256 = r0(ngroups=g, chunk=256)
        n64 = lib.ssd_workspace_bytes(ctypes.byref(dims), _lib.DTYPE_F32)
        n256 = lib.ssd_workspace_bytes(ctypes.byref(d256), _lib.DTYPE_F32)
        assert lib.ssd_forward_chunk(ctypes.byref(dims), _lib.DTYPE_F16, 0) == (256 if n256 <= n64 else 64)


def r0(**kw):
    """R0's dims (MR's defaults: batch 8, seqlen 2048, 128 heads, d_state 128, 8 groups, block_len 64)."""
    base = dict(batch=8, seqlen=2048, nheads=128, headdim=64, dstate=128, ngroups=8, chunk=64)
    base.update(kw)
    return _lib.SSDDims(*[base[k] for k in ("batch", "seqlen", "nheads", "headdim", "dstate", "ngroups", "chunk")])


def test_forward_workspace_check_uses_the_chunk_it_runs_at():
    """A routed forward accepts a workspace sized for chunk 256 (smaller than
    chunk 64's) and rejects one byte less; rejected on the host before any launch."""
    lib = _lib.load()
    dims = r0()
    n256 = lib.ssd_workspace_bytes(ctypes.byref(r0(chunk=256)), _lib.DTYPE_F32)
    assert n256 < lib.ssd_workspace_bytes(ctypes.byref(dims), _lib.DTYPE_F32)
    s4 = (ctypes.c_int64 * 4)(2048 * 128 * 64, 128 * 64, 64, 1)
    s3 = (ctypes.c_int64 * 3)(2048 * 128, 128, 1)
    bs4 = (ctypes.c_int64 * 4)(2048 * 8 * 128, 8 * 128, 128, 1)
    fake = ctypes.c_void_p(0x100000)
    # every operand valid but y misaligned: the workspace check passes first at n256
    rc = lib.ssd_forward(ctypes.byref(dims), _lib.DTYPE_F16, fake, s4, fake, s3, fake, bs4, fake, bs4, None, None,
                         None, ctypes.c_void_p(0x100002), s4, None, fake, n256, 0, None)
    assert rc == -10
    rc = lib.ssd_forward(ctypes.byref(dims), _lib.DTYPE_F16, fake, s4, fake, s3, fake, bs4, fake, bs4, None, None,
                         None, fake, s4, None, fake, n256 - 1, 0, None)
    assert rc == -11


def test_per_kernel_entry_points_reject_misaligned_cumsum_and_states():
    """a_cumsum and the states are copied to LDS 16 bytes at a time: a base
    that is only 4-byte aligned is rejected (SSD_ERR_MISALIGNED) on the host."""
    lib = _lib.load()
    dims = d()
    s4 = (ctypes.c_int64 * 4)(256 * 8 * 64, 8 * 64, 64, 1)
    bs4 = (ctypes.c_int64 * 4)(256 * 2 * 64, 2 * 64, 64, 1)
    ys4 = (ctypes.c_int64 * 4)(256 * 8 * 64, 8 * 64, 64, 1)
    fake = ctypes.c_void_p(0x100000)
    mis = ctypes.c_void_p(0x100004)
    # ssd_chunk_state: a_cumsum, then states
    assert lib.ssd_chunk_state(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, mis, fake, 0, None, None) == -10
    assert lib.ssd_chunk_state(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, fake, mis, 0, None, None) == -10
    # ssd_chunk_state_passing: a_cumsum
    assert lib.ssd_chunk_state_passing(ctypes.byref(dims), 1, fake, s4, fake, bs4, None, None, mis, fake, None, None,
                                       fake, 0, None, None, None) == -10
    # ssd_chunk_scan: a_cumsum, then states
    scan = lambda acs, st: lib.ssd_chunk_scan(ctypes.byref(dims), 1, fake, s4, fake, bs4, fake, bs4, None, None,  # noqa: E731
                                              acs, st, 0, None, fake, ys4, None, None, None)
    assert scan(mis, fake) == -10
    assert scan(fake, mis) == -10


def test_forward_chunk_keeps_the_chunk_where_chunk_prep_outweighs_the_states_saved():
    """C5-like 16-bit shape (8 groups, d_state 64, chunk 128): chunk_prep's
    per-group operands at chunk 256 take more than the halved states save,
    so the forward keeps chunk 128; with 4 groups it runs at 256."""
    lib = _lib.load()
    keep = _lib.SSDDims(8, 512, 64, 64, 64, 8, 128)
    move = _lib.SSDDims(8, 512, 64, 64, 64, 4, 128)
    assert lib.ssd_forward_chunk(ctypes.byref(keep), _lib.DTYPE_BF16, 0) == 128
    assert lib.ssd_forward_chunk(ctypes.byref(move), _lib.DTYPE_BF16, 0) == 256


def test_one_launch_forward_needs_no_workspace():
    """d_state 16 / 32 at chunk 64 / 128 (chunk x d_state <= 2048) with at most
    16 chunks and f32 states: ssd_forward runs as one launch and uses no
    workspace, so ssd_workspace_bytes reports 256; bf16 states, 17 chunks or
    chunk 128 x d_state 32 keep the four-kernel workspace."""
    lib = _lib.load()
    def ws(sd=_lib.DTYPE_F32, **kw):
        dims = dict(batch=16, seqlen=128, nheads=8, headdim=64, dstate=16, ngroups=8, chunk=64)
        dims.update(kw)
        return lib.ssd_workspace_bytes(ctypes.byref(_lib.SSDDims(*[dims[k] for k in (
            "batch", "seqlen", "nheads", "headdim", "dstate", "ngroups", "chunk")])), sd)

    assert ws() == 256                                   # C1
    assert ws(dstate=32) == 256 and ws(chunk=128, seqlen=256) == 256
    assert ws(seqlen=64 * 16) == 256 and ws(seqlen=64 * 17) > 256
    assert ws(_lib.DTYPE_BF16) > 256
    assert ws(dstate=32, chunk=128, seqlen=256) > 256
    assert ws(dstate=64) > 256
