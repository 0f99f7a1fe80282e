"""Builds libssd.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m workloadsuite_amd.build [-v]

Each source compiles to an object in ``workloadsuite_amd/_build`` (in
parallel), then one shared library is linked next to this file.  hipcc
cross-compiles for gfx950 without a GPU present.
"""

from __future__ import annotations

import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libssd.so")
ARCH = "gfx950"

SOURCES = [
    "ssd_api.cpp",
    "ssd_cumsum.hip",
    "ssd_chunk_prep.hip",
    "ssd_chunk_state.hip",
    "ssd_chunk_state_q256.hip",
    "ssd_chunk_state_f32.hip",
    "ssd_state_passing.hip",
    "ssd_chunk_scan.hip",
    "ssd_chunk_scan_b16.hip",
    "ssd_chunk_scan_q256.hip",
    "ssd_chunk_scan_f32.hip",
    "ssd_layer_prep.hip",
    "ssd_decode.hip",
    "ssd_noalloc.hip",
    "ssd_small.hip",
]

# The streaming probe behind bench.py --hbm-probe: its own library, outside
# the SSD forward's ABI.
PROBE_SOURCES = ["ssd_probe.hip"]
PROBE_LIB = os.path.join(PKG, "libssd_probe.so")

# Packed FP32 VALU forms are disabled: hipcc -O3 would otherwise emit
# v_pk_{add,mul,fma}_f32 from plain float code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-Wall", "-Werror", "-Wno-unused-function"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libssd)")


# Every kernel keeps its registers: the compiler's per-kernel resource remarks
# are read and a kernel with scratch (spilled registers) fails the build.
RESOURCE_FLAGS = ["-Rpass-analysis=kernel-resource-usage"]


def _spills(text: str) -> list:
    """(kernel, bytes per lane) for every kernel whose remarks report scratch."""
    out, name = [], None
    for ln in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", ln)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", ln)
        if m and name and int(m.group(1)) > 0:
            out.append((name, int(m.group(1))))
    return out


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *RESOURCE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    text = res.stdout + res.stderr
    # The host pass does not know the packed-fp32 target feature; drop that
    # note, and the resource remarks (checked below).
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in text.splitlines() if noise not in ln and "kernel-resource-usage" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
    spills = _spills(text)
    if spills:
        raise RuntimeError(f"{src}: kernels spill registers to scratch (bytes per lane): {spills}")
    if verbose and msgs:
        print("\n".join(msgs))
    return obj


def _link(objs, lib, verbose):
    tmp = lib + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    """Compile every source, link libssd.so (and the probe library); returns libssd's path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    _link(objs[:len(SOURCES)], LIB, verbose)
    _link(objs[len(SOURCES):], PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
