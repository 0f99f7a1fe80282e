#!/usr/bin/env python3
"""Benchmark of the MI355X SSD forward (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3]
                    [--state-dtype f32|bf16] [--no-cpu-baseline]
    python bench.py --layer [--steps K] [--warmup W]
    python bench.py --decode [--decode-batches 4,64,256]

A step is one SSD forward (K1 cumsum and K0 chunk_prep in one launch -> K2
chunk_state and K3 state_passing, one launch per (b, h) chain where that is
faster -> K4 chunk_scan) over one batch of synthetic inputs already resident in HBM, at
the Mamba-2-2.7B layer shape by default (C3: batch 4, seqlen 4096, 80 heads,
head_dim 64, d_state 128, chunk 256, 1 group, bf16 X/B/C, fp32 A, final state
returned).  Prints ONE JSON line.

Timing follows the reference harness (ShouyangDong/WorkloadSuite
bench.py:138-170): warmup, then device-synchronised timing of K steps.  The
order is each kernel's average launch duration, K forwards timed one by one
(per-step median / mean / p90 / p99), then the W warmup steps and the K timed
forwards: a fresh process's first tens of forwards run up to 15% slower, and
the measurements before the timed region bring the GPU to its steady state.
Kernel durations are measured live with HIP events on the
stream the kernels run on (torch's current stream), and the dominant kernel's
algorithmic bytes (or flops) per launch over that duration give
``roofline.achieved``.  ``cpu_baseline`` times the CPU oracle's float32
restatement of the reference einsum path on a bounded sample (one batch
element of the same config) on this host's cores.

``--layer`` instead times one full Mamba-2 layer at the reference module's
production shape (workloads/mamba/model_ref.py:209-221: batch 8, seqlen 2048,
d_model 2048, 128 heads, d_state 128, 8 groups, block_len 64, fp16, random
weights): the whole ``SSDLayer.forward``, and separately the span between
its two projections, once as libssd's single ``ssd_layer`` call and once as
PyTorch glue (conv1d, SiLU, softplus, skip, gate) around ``ssd_forward``.
It prints one JSON line of its own; the headline line above is unaffected.

``--decode`` times one decode step (``ssd_decode_step``, one token of the
recurrence in place on the f32 state) at C3's head shape for a few batch
sizes, with the state's HBM bytes per step over the step's device time.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from workloadsuite_amd import ssd as S  # noqa: E402
from workloadsuite_amd.configs import CONFIGS, HEADLINE, make_inputs  # noqa: E402

METRIC = "SSD fwd tokens/s + MFMA%/HBM% of peak at Mamba-2-2.7B layer, 1 MI355X"
PEAK_HBM_GBS = 8000.0                      # MI355X HBM3E
PEAK_TFLOPS = {torch.bfloat16: 2500.0, torch.float16: 2500.0, torch.float32: 157.3}   # dense MFMA
DTYPE_NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def esize(dt):
    return torch.tensor([], dtype=dt).element_size()


def kernel_model(cfg, state_dtype, handover=None, local_f16=False, cb_in_scan=True):
    """Algorithmic HBM bytes and MFMA flops per launch of each kernel.

    Bytes count every operand read once and every result written once at its
    storage type (B and C per group, not per head); the states entering each
    chunk at the format K3 hands them to K4 in (``handover`` "f16s": 2 bytes
    per state plus a 4-byte scale per state row; otherwise the state dtype,
    the (hi, lo) pairs taking 4 bytes); the local states between chunk_state
    and state_passing at the state dtype, or (``local_f16``) as f16 with a
    4-byte scale per row and 16-column tile.  Flops count useful work: the
    causal triangle T_Q = Q(Q+1)/2 of the intra-chunk products, with C.B^T
    formed once per (batch, chunk, group) as the kernels form it -- inside
    chunk_scan (``cb_in_scan``), or in chunk_prep where that runs (16-bit
    inputs at chunk 256), and then not in chunk_scan.  ``flops_cb_per_head``
    of chunk_scan is the reference algorithm's count (C.B^T per head after
    the GQA repeat, MR:97-99, 143), kept as a separately labelled figure.
    """
    b, L, h, P, N, Q, g = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.chunk, cfg.ngroups
    c = L // Q
    es, ss = esize(cfg.dtype), esize(state_dtype)
    x = b * L * h * P * es
    bc = b * L * g * N * es
    a = b * L * h * 4
    acs = b * h * c * Q * 4
    dec = b * h * c * 4
    st = b * c * h * (P * N * 2 + P * (N // 16) * 4) if local_f16 else b * c * h * P * N * ss
    sin = b * c * h * (P * N * 2 + P * 4) if handover == "f16s" else st
    fin = b * h * P * N * 4 if cfg.final_state else 0
    init = b * h * P * N * 4 if cfg.init_state else 0
    TQ = Q * (Q + 1) // 2
    cb_frag = b * c * g * 8 * 9 * 2 * 64 * 16       # chunk_prep's CB^T fragments (f32)
    bt_frag = b * c * g * (N // 16) * 8 * 64 * 16   # and B^T fragments (16-bit)
    return {
        "chunk_cumsum": dict(bytes=a + acs + dec, flops=b * L * h),
        "chunk_prep": dict(bytes=2 * bc + cb_frag + bt_frag, flops=2 * b * c * g * TQ * N),
        "chunk_state": dict(bytes=x + bc + acs + st, flops=2 * b * c * h * Q * P * N),
        "state_passing": dict(bytes=st + sin + dec + fin + init, flops=2 * b * c * h * P * N),
        # K2 + K3 as the forward runs them: x in, S_in out; the local states are not counted
        "chunk_state_passing": dict(bytes=x + bc + acs + dec + sin + fin + init, flops=2 * b * c * h * (Q + 1) * P * N),
        "chunk_scan": dict(bytes=x + 2 * bc + acs + sin + x,
                           flops=b * c * h * (2 * TQ * P + 2 * Q * N * P) + (b * c * g * 2 * TQ * N if cb_in_scan else 0),
                           flops_cb_per_head=b * c * h * (2 * TQ * N + 2 * TQ * P + 2 * Q * N * P)),
    }


def takes_small_path(cfg, state_dtype):
    """ssd_forward's one-launch path for small states and short chains
    (ssd_small_supported in the library): f32 states, d_state 16 / 32,
    chunk 64 / 128, at most 16 chunks per chain."""
    return (state_dtype == torch.float32 and cfg.dstate in (16, 32) and cfg.chunk in (64, 128)
            and cfg.nchunks <= 16)


def small_chunk_shape(cfg):
    """chunk 64 / 128, d_state 64 / 128, chunk x d_state <= 8192: the shapes of
    the f32-state chain and of the 16-bit chunk_scan for f32 states."""
    return cfg.chunk in (64, 128) and cfg.dstate in (64, 128) and cfg.chunk * cfg.dstate <= 8192


def handover_format(cfg, state_dtype, prep, state_format):
    """The format ssd_forward hands f32 S_in to K4 in (handover_format in the
    library): at chunk 256 with 16-bit inputs "f16s", or the inputs' (hi, lo)
    pairs with --state-format split; at the small-chunk shapes with 16-bit
    inputs "f16s" (a split request hands over plain f32 there); else None."""
    if state_dtype != torch.float32 or cfg.dtype == torch.float32:
        return None
    if prep is not None:
        return cfg.dtype if state_format == "split" else "f16s"
    if small_chunk_shape(cfg) and state_format != "split":
        return "f16s"
    return None


def takes_state_chain(cfg, split, state_dtype):
    """ssd_forward's dispatch for K2 + K3: at chunk 64 / 128 the f32-state
    chain wherever its shape allows; at chunk 256 with a hand-over format
    (chunk_state_chain_plan in the library) one state-chain launch when the
    (batch, head) chains keep every CU about equally busy (at least 3/4 of the
    busiest CU's chains on the average CU) or number between one and two per
    CU (d_state 128 for "f16s"); otherwise chunk_state then state_passing."""
    if cfg.chunk != 256:
        return state_dtype == torch.float32 and small_chunk_shape(cfg)
    if split is None or (split == "f16s" and cfg.dstate != 128):
        return False
    chains = cfg.batch * cfg.nheads
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_cu = -(-chains // cus)
    return 4 * chains >= 3 * per_cu * cus or cus < chains < 2 * cus


def end_to_end_model(cfg):
    """F_min / B_min per forward: inputs read once, outputs written once; CB per group."""
    b, L, h, P, N, Q, g = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.chunk, cfg.ngroups
    c = L // Q
    es = esize(cfg.dtype)
    TQ = Q * (Q + 1) // 2
    flops = b * c * (g * 2 * TQ * N + h * (2 * TQ * P + 4 * Q * N * P + 2 * N * P))
    byts = 2 * b * L * h * P * es + 2 * b * L * g * N * es + b * L * h * 4
    byts += b * h * P * N * 4 * (int(cfg.final_state) + int(cfg.init_state))
    return flops, byts


def profiled_traffic(cfg, kernel):
    """HBM bytes per launch of `kernel` as measured with rocprofv3 FETCH_SIZE /
    WRITE_SIZE (scaled by a copy of known size) and committed under
    profiles/ssd_forward_<config>.md as a line ``traffic_bytes_per_launch
    <kernel>: <bytes>``; (None, None) when there is no such measurement."""
    path = os.path.join(ROOT, "profiles", f"ssd_forward_{cfg.name}.md")
    if not os.path.exists(path):
        return None, None
    key = f"traffic_bytes_per_launch {kernel}:"
    for line in open(path):
        if line.startswith(key):
            return int(line[len(key):].strip()), os.path.relpath(path, ROOT)
    return None, None


def profiled_mfma(cfg, kernel):
    """MFMA instructions per launch of `kernel` (rocprofv3 SQ_INSTS_MFMA) and
    the flops one of them performs, as committed under
    profiles/ssd_forward_<config>.md in lines ``mfma_instructions_per_launch
    <kernel>: <n>`` and ``mfma_flops_per_instruction <kernel>: <f>``;
    None when there is no such measurement."""
    path = os.path.join(ROOT, "profiles", f"ssd_forward_{cfg.name}.md")
    if not os.path.exists(path):
        return None
    got = {}
    for line in open(path):
        for key in ("mfma_instructions_per_launch", "mfma_flops_per_instruction"):
            k = f"{key} {kernel}:"
            if line.startswith(k):
                got[key] = int(line[len(k):].strip())
    if len(got) != 2:
        return None
    return got["mfma_instructions_per_launch"] * got["mfma_flops_per_instruction"]


def summarize(samples):
    """median / mean / p90 / p99 of per-step times (ms), quantiles by nearest
    rank on the sorted samples, index round(q (n - 1)) (the reference
    harness's convention, bench.py:123-135 of ShouyangDong/WorkloadSuite)."""
    srt = sorted(samples)

    def q(x):
        return srt[min(len(srt) - 1, max(0, round(x * (len(srt) - 1))))]

    return {"median_ms": round(statistics.median(srt), 5), "mean_ms": round(statistics.mean(srt), 5),
            "p90_ms": round(q(0.90), 5), "p99_ms": round(q(0.99), 5), "runs": len(srt)}


def step_stats(fn, runs):
    """Per-call device time of fn(): an event pair around each of `runs`
    back-to-back calls on the current stream."""
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(runs)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return summarize([a.elapsed_time(b) for a, b in ev])


def time_launches(fn, reps):
    """Average device time (ms) of fn() over reps back-to-back calls.

    A device-side sleep is queued first so the host can enqueue all calls
    before the device reaches the start event: the events then bracket device
    work only, not host launch latency.  The sleep is doubled and the calls
    timed again while the host's enqueue outlasts it (fn may be several
    Python-level launches).
    """
    sleep = getattr(torch.cuda, "_sleep", None)
    cycles = 20_000_000
    while True:
        torch.cuda.synchronize()
        s0, start, end = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        s0.record()
        if sleep is not None:
            sleep(cycles)
        start.record()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        host_ms = (time.perf_counter() - t0) * 1e3
        end.record()
        end.synchronize()
        if sleep is None or host_ms < 0.8 * s0.elapsed_time(start) or cycles >= 1_600_000_000:
            return start.elapsed_time(end) / reps
        cycles *= 2


def cpu_baseline(cfg, budget_s=12.0, max_runs=30):
    """The oracle's float32 restatement of the reference einsum path (MR:123-162)
    on one batch element of cfg, on this host's CPU cores."""
    from oracle import ssd_oracle as O

    sample = cfg.scaled(batch=1)
    inp = make_inputs(sample, seed=0)
    torch.set_float32_matmul_precision("highest")
    args = (inp["X"], inp["A"], inp["B"], inp["C"], sample.chunk)
    kw = dict(initial_states=inp["init"], dtype=torch.float32)
    O.ssd_chunked(*args, **kw)  # warmup
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        O.ssd_chunked(*args, **kw)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": sample.tokens / med,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{cfg.name} with batch 1 of {cfg.batch} ({sample.tokens} tokens, all {cfg.nheads} heads); "
                   f"oracle/ssd_oracle.py ssd_chunked in torch float32 on CPU (inputs rounded to "
                   f"{DTYPE_NAMES[cfg.dtype]} first), median of {len(times)} runs, "
                   f"{torch.get_num_threads()} intra-op threads, os.cpu_count()={os.cpu_count()}"),
        "ms_per_forward": med * 1e3,
    }


def hbm_probe(args):
    """The streaming probes of libssd_probe.so (csrc/ssd_probe.hip): read
    args.hbm_probe MiB of f32 with 16-byte loads and write one f16 per f32
    read (state_passing's 2 : 1 read / write mix, 8-byte or 16-byte stores),
    or copy them (1 : 1); plain or non-temporal loads and stores, 4 or 8
    vectors in flight per thread, 4 / 8 / 16 workgroups of 256 threads per
    CU.  Two source / destination pairs are used in turn, together well
    beyond the 256 MB Infinity Cache.  Reports every variant, the best per
    mix, and torch's own device copy for reference."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "workloadsuite_amd", "libssd_probe.so"))
    lib.ssd_stream_probe.restype = ctypes.c_int
    lib.ssd_stream_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    n = (args.hbm_probe << 20) // 4
    src = [torch.rand(n, device=dev) for _ in range(2)]
    dst = [torch.empty(n, dtype=torch.float32, device=dev) for _ in range(2)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {"hbm_probe_read_bytes": 4 * n, "peak_GB_s": PEAK_HBM_GBS, "reps": args.kernel_reps, "probes": {},
           "best": {}}
    mixes = {0: "2:1 mix, f16x4 stores", 1: "2:1 mix, f16x8 stores", 2: "copy 1:1"}
    for kind in (0, 1, 2):
        for flags in range(8):
            for per_cu in (4, 8, 16):
                k = [0]

                def launch():
                    i = k[0] % 2
                    k[0] += 1
                    rc = lib.ssd_stream_probe(ctypes.c_void_p(src[i].data_ptr()), ctypes.c_void_p(dst[i].data_ptr()),
                                              n, kind, flags, per_cu * cus, stream)
                    if rc:
                        raise RuntimeError(f"ssd_stream_probe failed: {rc}")

                launch()
                ms = time_launches(launch, args.kernel_reps)
                moved = 4 * n + (4 * n if kind == 2 else 2 * n)
                gbs = moved / (ms * 1e-3) / 1e9
                name = (f"{mixes[kind]}, {'nt' if flags & 1 else 'plain'} loads, {'nt' if flags & 2 else 'plain'} "
                        f"stores, {8 if flags & 4 else 4} in flight, {per_cu} WG/CU")
                out["probes"][name] = {"ms": round(ms, 5), "GB_s": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
                best = out["best"].get(mixes[kind])
                if best is None or gbs > best["GB_s"]:
                    out["best"][mixes[kind]] = {"variant": name, "GB_s": round(gbs, 1),
                                                "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
    k = [0]

    def torch_copy():
        i = k[0] % 2
        k[0] += 1
        dst[i].copy_(src[i])

    torch_copy()
    ms = time_launches(torch_copy, args.kernel_reps)
    gbs = 8 * n / (ms * 1e-3) / 1e9
    out["torch_copy"] = {"ms": round(ms, 5), "GB_s": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
    print(json.dumps(out), flush=True)


def layer_bench(args):
    import torch.nn.functional as F

    from workloadsuite_amd import mamba_layer as ML

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    torch.manual_seed(0)
    d_model, _, h, N, P, g, Q, k = ML.get_init_inputs()
    b, L = ML.batch_size, ML.seq_length
    layer = ML.SSDLayer(d_model, h, N, P, g, block_len=Q, conv_kernel=k).to(dev).eval()
    u = torch.randn(b, L, d_model, dtype=torch.float16, device=dev)
    d_inner = h * P
    with torch.inference_mode():
        zxbcdt = layer.in_proj(layer.norm(u))
        x, z, B, C, dt = torch.split(zxbcdt, [d_inner, d_inner, g * N, g * N, h], dim=-1)
        Bv, Cv = B.view(b, L, g, N), C.view(b, L, g, N)

        def fused():
            return S.ssd_layer(x, z, Bv, Cv, dt, layer.conv1d.weight, layer.conv1d.bias, layer.dt_bias,
                               layer.A_log, layer.D, Q, h)

        def glue():
            xx = F.silu(layer.conv1d(x.transpose(1, 2))[..., :L]).transpose(1, 2).contiguous()
            X = xx.view(b, L, h, P)
            dtt = F.softplus(dt + layer.dt_bias)
            Y = S.ssd_forward(X, -torch.exp(layer.A_log) * dtt.float(), Bv, Cv, Q, dt=dtt.float())
            Y = Y + X * layer.D.view(1, 1, -1, 1)
            return Y.reshape(b, L, d_inner) * F.silu(z)

        def whole():
            return layer(u)

        diff = (fused().float() - glue().float()).abs().max().item()
        res = {}
        for name, fn in (("layer", whole), ("span_fused", fused), ("span_torch_glue", glue)):
            for _ in range(args.warmup):
                fn()
            res[name] = time_launches(fn, args.steps)
    tokens = b * L
    out = {
        "metric": "Mamba-2 SSD layer forward tokens/s (one layer, model_ref.py production shape), 1 MI355X",
        "value": round(tokens / (res["layer"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["layer"], 5),
        "higher_is_better": True,
        "dtype": "f16",
        "data": "synthetic (u ~ N(0,1); module's default init)",
        "config": {"workload": "mamba2-layer R0", "batch": b, "seqlen": L, "d_model": d_model, "nheads": h,
                   "headdim": P, "dstate": N, "ngroups": g, "chunk": Q, "conv_kernel": k},
        "span_ms": {"ssd_layer (fused)": round(res["span_fused"], 5),
                    "torch glue + ssd_forward": round(res["span_torch_glue"], 5)},
        "span_max_abs_diff": diff,
    }
    print(json.dumps(out), flush=True)


def decode_bench(args):
    """One decode step (ssd_decode_step: one token of the recurrence, in place
    on the [b, h, P, N] f32 state) at C3's head shape for each batch size in
    args.decode_batches.  Algorithmic bytes per step: the state read and
    written once (8 bytes per element), x and y (P values per head), B and C
    (N per group), a and dt (f32 per head).  Two states are used in turn, so
    that from 64 batch rows on (2 x 168 MB) the state does not stay in the
    256 MB Infinity Cache between steps."""
    cfg = CONFIGS[HEADLINE]
    h, P, N, g, dt_ = cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups, cfg.dtype
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    es = esize(dt_)
    rows = []
    for b in args.decode_batches:
        states = [torch.randn(b, h, P, N, device=dev, generator=gen) for _ in range(2)]
        x = torch.randn(b, h, P, device=dev, generator=gen).to(dt_)
        Bm = torch.randn(b, g, N, device=dev, generator=gen).to(dt_)
        Cm = torch.randn(b, g, N, device=dev, generator=gen).to(dt_)
        a = -torch.rand(b, h, device=dev, generator=gen) * 0.1
        dt = torch.rand(b, h, device=dev, generator=gen) * 0.1
        k = [0]

        def step():
            i = k[0] % 2
            k[0] += 1
            return S.decode_step(states[i], x, Bm, Cm, a, dt)

        step()
        ms = time_launches(step, args.kernel_reps)
        nbytes = b * h * P * N * 8 + 2 * b * h * P * es + 2 * b * g * N * es + 2 * b * h * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append({"batch": b, "us_per_step": round(ms * 1e3, 2), "tokens_per_s": round(b / (ms * 1e-3), 1),
                     "algorithmic_bytes": nbytes, "GB_s": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)})
        del states
    out = {
        "metric": "SSD decode step (one token, in place on the f32 state), 1 MI355X",
        "dtype": DTYPE_NAMES[dt_] + " inputs, f32 state",
        "data": "synthetic",
        "config": {"workload": "decode at C3's head shape", "nheads": h, "headdim": P, "dstate": N, "ngroups": g},
        "reps": args.kernel_reps,
        "roofline_peak_GB_s": PEAK_HBM_GBS,
        "steps": rows,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default=HEADLINE, choices=sorted(CONFIGS))
    ap.add_argument("--state-dtype", default="f32", choices=["f32", "bf16"])
    ap.add_argument("--state-format", default=None, choices=["split", "f16s"],
                    help="how f32 states reach chunk_scan (default: the library's choice, f16s for 16-bit inputs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=30)
    ap.add_argument("--layer", action="store_true",
                    help="time one full layer at the reference module's production shape instead")
    ap.add_argument("--decode", action="store_true",
                    help="time one decode step (ssd_decode_step) at C3's head shape instead, per batch size")
    ap.add_argument("--decode-batches", type=lambda v: [int(t) for t in v.split(",")], default=[4, 64, 256],
                    metavar="B1,B2,..", help="batch sizes for --decode (default 4,64,256)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="only run a plain device-to-device copy of MB MiB (5 times) and exit: the "
                         "reference point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    ap.add_argument("--hbm-probe", type=int, default=0, metavar="MB",
                    help="only time the hand-written streaming probes (libssd_probe.so) reading MB MiB of f32 "
                         "at state_passing's read / write mix (and a copy), with and without non-temporal "
                         "loads, and exit with one JSON line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path. The SSD forward "
              "shards over batch x heads with no communication, so N GPUs would each run this "
              "single-GPU workload on 1/N of the heads.", file=sys.stderr)
        sys.exit(2)

    if args.layer:
        layer_bench(args)
        return

    if args.hbm_probe:
        hbm_probe(args)
        return

    if args.decode:
        decode_bench(args)
        return

    if args.copy_probe:
        n = args.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": 5}), flush=True)
        return

    cfg = CONFIGS[args.config]
    state_dtype = torch.float32 if args.state_dtype == "f32" else torch.bfloat16
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = make_inputs(cfg, seed=0, device=dev)
    X, A, B, C, init = inp["X"], inp["A"], inp["B"], inp["C"], inp["init"]
    # the chunk ssd_forward runs this config at (16-bit inputs at chunk 64 /
    # 128 run at 256 where seqlen and d_state allow): the kernels are timed,
    # and their traffic modelled, at that chunk
    run_chunk = S.forward_chunk(cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups, cfg.chunk,
                                cfg.dtype, state_dtype, args.state_format)
    kcfg = cfg.scaled(chunk=run_chunk)

    # ---- per-kernel device time, each kernel on its real inputs ----
    Acs, decay = S.chunk_cumsum(A, kcfg.chunk)
    prep = S.chunk_prep(B, C, kcfg.chunk)
    states = S.chunk_state(X, B, Acs, state_dtype=state_dtype, prep=prep)
    # as in ssd_forward: with 16-bit inputs and f32 states, K3 hands S_in to K4
    # as f16 rows with a power-of-two scale per row ("f16s"), or at chunk 256
    # as 16-bit (hi, lo) pairs with --state-format split
    split = handover_format(kcfg, state_dtype, prep, args.state_format)
    # where the forward runs chunk_state then state_passing with the f16s
    # hand-over at chunk 256, the local states cross HBM as f16 rows: time
    # those variants
    local_f16 = split == "f16s" and prep is not None and not takes_state_chain(kcfg, split, state_dtype)
    if local_f16:
        states = S.chunk_state(X, B, Acs, state_dtype="f16s", prep=prep).states
    S_in, _ = S.state_passing(S.F16SLocalStates(states) if local_f16 else states, decay, init, split=split)
    # K3 is timed in place on its own buffers, re-applying the recurrence to
    # their contents on every launch: the same traffic and instructions (nothing
    # in the kernel depends on the values, which stop being meaningful).  The
    # launches rotate over enough buffers (at least two, at least 512 MB in
    # all: twice the MI355X's 256 MB Infinity Cache) that each launch reads
    # states that are no longer cached.
    nbuf = max(2, -(-512 * 2**20 // states.numel() // states.element_size()))
    sp_bufs = [states.clone() for _ in range(nbuf)]
    sp_scales = torch.empty(states.shape[:4], dtype=torch.float32, device=dev) if split == "f16s" else None
    sp_next = [0]

    def sp_launch():
        buf = sp_bufs[sp_next[0] % nbuf]
        sp_next[0] += 1
        return S.state_passing_(buf, decay, init, sp_final, split=split, scales=sp_scales, f16_local=local_f16)

    sp_final = torch.empty(cfg.batch, cfg.nheads, cfg.headdim, cfg.dstate, device=dev) if cfg.final_state else None
    kfn = {
        "chunk_cumsum": lambda: S.chunk_cumsum(A, kcfg.chunk),
        "chunk_prep": lambda: S.chunk_prep(B, C, kcfg.chunk),
        "chunk_state": lambda: S.chunk_state(X, B, Acs, state_dtype="f16s" if local_f16 else state_dtype, prep=prep),
        "state_passing": sp_launch,
        "chunk_state_passing": lambda: S.chunk_state_passing(X, B, Acs, decay, prep=prep, initial_states=init,
                                                             return_final_states=cfg.final_state, split=split,
                                                             state_dtype=state_dtype),
        "chunk_scan": lambda: S.chunk_scan(X, B, C, Acs, S_in, prep=prep,
                                           split="f16s" if split == "f16s" else split is not None),
    }
    if prep is None:
        del kfn["chunk_prep"]
    small = takes_small_path(kcfg, state_dtype)
    if small:
        # the forward is one launch (ssd_small): time it, with the forward's
        # minimum bytes and flops; the four stages' entry points are not what
        # it runs
        kfn = {"ssd_small": lambda: S.ssd_forward(X, A, B, C, cfg.chunk, initial_states=init,
                                                  return_final_states=cfg.final_state, state_dtype=state_dtype,
                                                  state_format=args.state_format)}
    model = kernel_model(kcfg, state_dtype, split if isinstance(split, str) else None, local_f16,
                         cb_in_scan=prep is None)
    f_min, b_min = end_to_end_model(cfg)
    model["ssd_small"] = dict(bytes=b_min, flops=f_min)
    kernels = {}
    pre_launches = 0

    def kernel_entry(name, ms):
        m = model[name]
        gbs = m["bytes"] / (ms * 1e-3) / 1e9
        tfs = m["flops"] / (ms * 1e-3) / 1e12
        t_hbm = m["bytes"] / (PEAK_HBM_GBS * 1e9)
        t_mfma = m["flops"] / (PEAK_TFLOPS[cfg.dtype] * 1e12)
        e = {
            "ms": round(ms, 5), "bytes": m["bytes"], "flops": m["flops"],
            "GB_s": round(gbs, 1), "TFLOP_s": round(tfs, 2),
            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "mfma_frac": round(tfs / PEAK_TFLOPS[cfg.dtype], 4),
            "bound": "hbm" if t_hbm >= t_mfma else "mfma",
        }
        if "flops_cb_per_head" in m:
            e["flops_cb_per_head"] = m["flops_cb_per_head"]
            e["mfma_frac_cb_per_head"] = round(m["flops_cb_per_head"] / (ms * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype], 4)
        executed = profiled_mfma(cfg, name)
        if executed is not None:
            # the flops the MFMA instructions of one launch perform (rocprofv3
            # SQ_INSTS_MFMA), over this run's time
            e["mfma_executed_frac"] = round(executed / (ms * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype], 4)
        return e

    # each kernel alone, back to back on its own inputs
    for name, fn in kfn.items():
        fn()
        kernels[name] = kernel_entry(name, time_launches(fn, args.kernel_reps))
        pre_launches += 1 + args.kernel_reps
    # the dominant kernel among those the forward runs: K2 + K3 as it runs them
    # (chunk_state_passing), K4, K1 and K0 -- not the standalone chunk_state
    # and state_passing rows, which stand in for it only as a breakdown
    dom = max((k for k in kernels if k not in ("chunk_state", "state_passing")), key=lambda k: kernels[k]["ms"])
    kd = kernels[dom]
    if kd["bound"] == "hbm":
        roof = {"bound": "hbm", "achieved": kd["GB_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": kd["hbm_frac"]}
    else:
        roof = {"bound": "mfma", "achieved": kd["TFLOP_s"], "peak": PEAK_TFLOPS[cfg.dtype], "unit": "TFLOP/s",
                "frac": kd["mfma_frac"]}
    roof["kernel"] = dom
    if roof["bound"] == "mfma":
        roof["flops_basis"] = "useful: causal triangle, C.B^T once per (batch, chunk, group)"
        if "mfma_executed_frac" in kd:
            roof["mfma_executed_frac"] = kd["mfma_executed_frac"]
    roof["traffic"], roof["traffic_source"] = profiled_traffic(cfg, dom)

    # ---- K forwards timed one by one: per-step median / mean / p90 / p99 ----
    # A fresh process's first ~60 forwards run slower (C3, per 20 steps after
    # the first 20: 223-242, 214-224, 212-217, then 210-213 us): the per-kernel
    # times above and these statistics come before the headline's W warmup
    # and K timed steps, and carry most of that ramp.
    def step():
        return S.ssd_forward(X, A, B, C, cfg.chunk, initial_states=init,
                             return_final_states=cfg.final_state, state_dtype=state_dtype,
                             state_format=args.state_format)

    stats = step_stats(step, args.steps)
    pre_launches_forwards = args.steps

    # ---- the headline: W warmup steps, then K whole forwards back to back ----
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dev_ms = ev0.elapsed_time(ev1) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    tokens_per_s = cfg.tokens * args.steps / wall

    roof_tps = min(PEAK_TFLOPS[cfg.dtype] * 1e12 / (f_min / cfg.tokens), PEAK_HBM_GBS * 1e9 / (b_min / cfg.tokens))

    out = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAMES[cfg.dtype],
        "data": "synthetic (seeded: X~N(0,1), B,C~N(0,1)/sqrt(N), A=-softplus(N(-2,1))*exp(N(0,.5)))",
        "config": {"workload": f"mamba2-ssd-forward {cfg.name}" + (" (Mamba-2-2.7B layer)" if cfg.name == "C3" else ""),
                   "batch": cfg.batch, "seqlen": cfg.seqlen, "nheads": cfg.nheads, "headdim": cfg.headdim,
                   "dstate": cfg.dstate, "chunk": cfg.chunk, "chunk_run": run_chunk, "ngroups": cfg.ngroups,
                   "inputs": f"{DTYPE_NAMES[cfg.dtype]} X/B/C, f32 A", "state_storage": args.state_dtype,
                   "state_handover": split if isinstance(split, str) else ("split" if split is not None else None),
                   "local_states": ("in LDS (one-launch forward)" if small else "f16 rows" if local_f16 else
                                    "in registers (state chain)" if takes_state_chain(kcfg, split, state_dtype)
                                    else args.state_dtype),
                   "final_state": cfg.final_state, "initial_state": cfg.init_state},
        "device_ms_per_step": round(dev_ms, 5),
        "step_stats": stats,
        # what ran on the GPU in this process before the timed region: the
        # per-kernel timing launches, the step_stats forwards, then the
        # warmup forwards
        "pre_timing": {"kernel_launches": pre_launches, "step_stats_forwards": pre_launches_forwards,
                       "warmup_forwards": args.warmup,
                       "effective_warmup_forwards": pre_launches_forwards + args.warmup},
        "roofline": roof,
        "end_to_end": {"F_min_per_token": f_min / cfg.tokens, "B_min_per_token": b_min / cfg.tokens,
                       "roofline_tokens_per_s": roof_tps, "frac": round(tokens_per_s / roof_tps, 4)},
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
