#!/usr/bin/env python3
"""MoE-layer throughput of the MI355X MoE feed-forward path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-extra] [--no-cpu]

A step is one pass of the MoE block over one batch of synthetic input, with
all weights and inputs resident in HBM, through 16 distinct, independently
seeded layers (16 layers exceed the 256 MB last-level cache, so weights
stream from HBM as they do across a model's layers).

The metric names two configurations, both measured in every default run:
  olmoe_decode_t1 (the headline, `value`): 1 token through the OLMoE MoE block
  (hidden 2048, 64 experts, top-8, intermediate 1024, 4-bit affine g=64
  experts, bf16 scales/biases). `value` = MoE-layer tok/s = tokens x layers /
  step time; `roofline` is its gate/up kernel against 8 TB/s of HBM.
  olmoe_prefill_t4096_zipf: 4096 tokens with Zipf(1.1)-skewed routing,
  reported in `metric_configs` (the last key of the line) with its layer and
  gate/up kernel against the 2.5 PFLOP/s dense bf16 MFMA peak.

The other workloads (decode batch 8 over 16 layers, prefill 512, Granite
prefill 2048 and decode 32, 8-bit and f16 variants) are measured in the same
run; `workloads` holds their per-layer latency, tok/s and roofline fraction
(HBM for decode, bf16 MFMA for prefill). Each workload's step is also replayed
from a HIP graph; the replay is used when its output equals the eager step's
bit for bit. --report PATH writes the full per-workload record as JSON.

"cpu_baseline" is the oracle's MLX-semantics CPU block on the host cores over
a bounded sample of the headline workload (cycling through its 16 distinct
layers so the host's last-level cache does not hold the weights), with all
cores and with one thread; every other workload the CPU block runs (bf16
storage, dense router) carries its own bounded sample (`cpu_tok_per_s` with
all cores, at least 3 whole layers from 2048 tokens; `cpu_tok_per_s_1thread`).

Kernel durations (`us_per_launch`, `gateup_us`, `down_us`) are the kernels' own:
the stage profiler launches each stage's main kernel with events bound to its
dispatch, the timestamps a rocprofv3 kernel trace reports. The events
bracketing each stage of the eager profiled steps are only in the full
`--report` record (`stages_us`): they also hold the host's submission gaps
between the instrumented launches.
"""
from __future__ import annotations

import argparse
import json
import re
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "MoE-layer tok/s: decode b=1 & prefill 4096; % HBM BW / % MFMA peak"
HEADLINE = "olmoe_decode_t1"
PREFILL_METRIC = "olmoe_prefill_t4096_zipf"


def is_decode(w) -> bool:
    """Workloads on the decode kernels, bounded by HBM: the named decode
    workloads, and batch-size sweep points (olmoe_t<N>, granite_t<N>) of at
    most 256 routes."""
    sweep = re.match(r"^(olmoe|granite)_t[0-9]+$", w.name) is not None
    return w.name in DECODE or (sweep and w.tokens * w.geometry.top_k <= 256)
DECODE = {"olmoe_decode_t1", "olmoe_decode_t8_x16", "granite_decode_t32", "olmoe_decode_t8_x16_int8",
          "olmoe_decode_t8_x16_f16"}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default=HEADLINE)
    p.add_argument("--no-extra", action="store_true", help="measure the headline workload only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=8.0)
    p.add_argument("--report", default=None, help="write the full per-workload record (JSON) here")
    p.add_argument("--deterministic", action="store_true",
                   help="pass TFM_FLAG_DETERMINISTIC (every path already reduces routes in k order)")
    p.add_argument("--pmc-summary", default=None, metavar="DIR",
                   help="only summarise the rocprofv3 counter CSVs under DIR (mean per dispatch of "
                        "every counter, per kernel) as JSON and exit")
    p.add_argument("--linear-only", action="store_true",
                   help="measure the dense affine linear shapes only and print them")
    p.add_argument("--pmc-copy", type=int, default=0, metavar="MIB",
                   help="only run 5 device-to-device copies of MIB MiB (a kernel of known traffic, to "
                        "calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return p.parse_args()


def pmc_summary(root: str):
    """Per kernel (name up to its argument list): dispatch count and the mean
    over its dispatches of every counter in the rocprofv3 --pmc CSV output
    under `root` (Counter_Value summed over the CSV rows of one dispatch)."""
    import csv
    import glob
    from collections import defaultdict

    sums = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(set)
    for path in glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                k = row.get("Kernel_Name", "?").split("(")[0]
                disp[k].add(row.get("Dispatch_Id"))
                sums[k][row["Counter_Name"]] += float(row["Counter_Value"])
    out = {k: {"dispatches": len(disp[k]), **{c: v / len(disp[k]) for c, v in sorted(sums[k].items())}}
           for k in sums}
    # The kernel sources the counters were read from (measured_traffic keys a
    # figure to its kernel's source file).
    here = os.path.dirname(os.path.abspath(__file__))
    out["source_sha16"] = {os.path.relpath(p, here): source_sha16(os.path.relpath(p, here))
                           for p in sorted(glob.glob(os.path.join(here, "trifuse_amd", "csrc", "*.hip")))}
    print(json.dumps(out, indent=1), flush=True)


def pmc_copy(mib: int, reps: int = 5):
    """Copies of a known size: under rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE)
    each copy dispatch reads and writes exactly `mib` MiB, so counter /
    (mib * 1024) is the counter's scale in KiB per KiB moved."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {mib} MiB x {reps}", flush=True)


def cpu_info():
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return model, cores


class Runner:
    """Resident weights/input of one workload and its step function."""

    def __init__(self, name, device, deterministic=False):
        import torch

        from trifuse_amd import moe as tmoe
        from trifuse_amd import workload as wl

        self.torch = torch
        self.wl = wl.get_workload(name)
        g = self.wl.geometry
        self.geom = g
        # Rotate through TIMING_LAYERS distinct layers so weights come from HBM,
        # not from the last-level cache (a single layer is 28-226 MB).
        self.nlayers = max(self.wl.layers, wl.TIMING_LAYERS)
        self.layers = wl.workload_layers(self.wl, device, self.nlayers)
        self.weights = [tmoe.ExpertWeights.from_layer(l) for l in self.layers]
        self.x = wl.workload_x(self.wl).to(device)
        self.block = tmoe.MoEBlock(g.hidden, g.intermediate, g.experts, g.top_k, route=g.route,
                                   bits=self.wl.bits, dtype=self.wl.torch_dtype, router=self.wl.router)
        self.block.workspace(self.wl.tokens, device)
        self.y = None
        self.deterministic = deterministic

    def step(self):
        for w in self.weights:
            self.y = self.block.forward(self.x, w, deterministic=self.deterministic)

    def route_stats(self):
        """Per layer, from the GPU's own routing: distinct experts routed and
        the share of routes taken by the four busiest experts (cached)."""
        if getattr(self, "_route_stats", None) is None:
            U, top4 = [], []
            for w in self.weights:
                _, idx, _ = self.block.forward(self.x, w, return_routes=True)
                counts = self.torch.bincount(idx.reshape(-1).long(), minlength=self.geom.experts)
                U.append(int((counts > 0).sum()))
                top4.append(float(counts.sort(descending=True).values[:4].sum()) / float(counts.sum()))
            self._route_stats = (U, top4)
        return self._route_stats

    def distinct_experts(self):
        """Distinct experts routed per layer, from the GPU's own routing."""
        return self.route_stats()[0]

    def time_steps(self, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            self.step()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            self.step()
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return start.elapsed_time(end) / steps, wall * 1e3 / steps

    def graph_time(self, steps, warmup):
        """The step captured once in a HIP graph (torch.cuda.CUDAGraph) and
        replayed: the GPU-side step time without per-launch host work.
        Returns (ms per step, replayed output == eager output bit for bit)."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step()  # warm the allocator on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.step()
        y_graph = self.y  # written by every replay
        self.step()
        torch.cuda.synchronize()
        y_eager = self.y.clone()
        for _ in range(max(1, warmup)):
            graph.replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(y_graph, y_eager))
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        del graph
        return ms, same

    def stage_times(self, steps):
        from trifuse_amd.moe import StageProfiler

        prof = StageProfiler(capacity=steps * len(self.weights) * 6 + 16)
        with prof:
            for _ in range(steps):
                self.step()
        self.torch.cuda.synchronize()
        out = {}
        for s in prof.STAGES:
            ms, n = prof.stage(s)
            if n:
                out[s] = {"us_per_launch": ms * 1e3 / n, "launches": n}
            kms, kn = prof.stage_kernel(s)
            if n and kn:
                out[s]["kernel_us_per_launch"] = kms * 1e3 / kn
        prof.close()
        return out


def workload_report(r: Runner, ms_per_step: float, wall_ms: float, stages, graph=None):
    from trifuse_amd import workload as wl

    g, T, L = r.geom, r.wl.tokens, r.nlayers
    U = r.distinct_experts()
    per_layer_ms = ms_per_step / L
    bytes_step = sum(wl.algorithmic_bytes(g, T, u, r.wl.bits, r.wl.router == "affine") for u in U)
    flops_step = wl.algorithmic_flops(g, T) * L
    gbs = bytes_step / (ms_per_step * 1e-3) / 1e9
    tflops = flops_step / (ms_per_step * 1e-3) / 1e12
    bound = "hbm" if is_decode(r.wl) else "mfma"
    rep = {
        "description": r.wl.description,
        "bits": r.wl.bits, "dtype": r.wl.dtype, "router": r.wl.router,
        "tokens": T, "layers_per_step": L,
        "per_layer_us": per_layer_ms * 1e3,
        "tok_per_s": T * L / (ms_per_step * 1e-3),
        "wall_ms_per_step": wall_ms,
        "distinct_experts_per_layer": U if L <= 4 else [min(U), sum(U) / len(U), max(U)],
        "alg_bytes_per_step": bytes_step,
        "alg_flops_per_step": flops_step,
        "hbm_GBs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
        "mfma_TFLOPs": tflops, "mfma_frac": tflops / BF16_PEAK_TFLOPS,
        "bound": bound,
        "stages_us": {k: round(v["us_per_launch"], 3) for k, v in stages.items()},
        "stages_kernel_us": {k: round(v["kernel_us_per_launch"], 3) for k, v in stages.items()
                             if "kernel_us_per_launch" in v},
    }
    if graph is not None:
        gms, same = graph
        rep["graph_per_layer_us"] = gms / L * 1e3
        rep["graph_tok_per_s"] = T * L / (gms * 1e-3)
        rep["graph_matches_eager"] = same
    return rep


def gemv_gateup_label(g, T: int, bits: int) -> str:
    """The decode GEMV path's gate/up kernel: with at least 4096 gate/up
    workgroups (row-unit blocks x active-slot bound) the library publishes a
    slot table and runs gemv_kernel, else decode_gateup_kernel groups the
    routes in every workgroup (TFM_DECODE_GROUPING overrides, as in the
    library)."""
    o = os.environ.get("TFM_DECODE_GROUPING")
    if o in ("slots", "workgroup"):
        slots = o == "slots"
    else:
        nch = g.hidden // 32
        lg = 4 if nch <= 4 else 8 if nch <= 8 else 16 if nch <= 16 else 32 if nch <= 32 else 64
        ur = 4 * (64 // lg)
        upe = (g.intermediate + ur - 1) // ur
        slots = (upe + 1) // 2 * min(T * g.top_k, g.experts) >= 4096
    return "gemv_kernel<gateup>" if slots else "decode_gateup_kernel"


def dominant_roofline(r: Runner, stages):
    """Roofline object for the gate/up kernel (the largest share of bytes and FLOPs)."""
    from trifuse_amd import workload as wl

    g, T = r.geom, r.wl.tokens
    st = stages["gateup"]
    # The kernel's own duration (dispatch timestamps, as a kernel trace
    # reports it); the bracketing events add the launch and cache-release gap.
    kus = st.get("kernel_us_per_launch", st["us_per_launch"])
    dur_s = kus * 1e-6
    timing = {"us_per_launch": kus,
              "timing": "kernel dispatch timestamps (hipExtLaunchKernelGGL events)"
              if "kernel_us_per_launch" in st else "events around the launch"}
    U = r.distinct_experts()
    H, I = g.hidden, g.intermediate
    gu_bytes_expert = 2 * (I * H * r.wl.bits // 8 + 2 * (I * H // 64) * 2)
    R = T * g.top_k
    # The library's decode path choice: the streaming kernels at 1 to 3
    # tokens while the token rows fit their prologue, and for 8-bit codes
    # wherever they fit; the decode GEMV kernels (4-bit codes, bf16 or half
    # storage) from 4 tokens up to E + 40 routes (at most 176); else the
    # grouped GEMM.
    gemv = R <= min(176, g.experts + 40) and r.wl.bits == 4
    fits = (R <= 256 and g.experts <= 64 and T * (H // 32) <= 1024 and
            T * (H // 32) * 68 + R * 4 <= 65536 and  # staged x rows in LDS
            H % 512 == 0 and 512 <= H <= 2048 and I % 512 == 0 and 512 <= I <= 2048)
    streaming = fits and (T <= 3 or r.wl.bits != 4)
    gemv = gemv and not (fits and T <= 3)
    # 4-bit weights with inputs up to 2048 wide (a multiple of 128) run the
    # weights-in-registers grouped GEMM, everything else the LDS-dequant one
    wr = r.wl.bits == 4 and H <= 2048 and H % 128 == 0
    gemm_label = "ggemm_wr_kernel<gateup>" if wr else "ggemm_kernel<gateup>"
    if is_decode(r.wl):
        # Per launch: routed experts' gate+up Q/S/B, x rows in, h rows out.
        per_launch = sum(u * gu_bytes_expert + T * H * 2 + T * g.top_k * I * 2 for u in U) / len(U)
        # With TFM_DS_PREFETCH=1 the gate/up kernel of 1 to 3 tokens (T*K
        # <= 24) also copies the routed experts' down Q/S/B from HBM for the
        # fused down+combine kernel: those bytes are then moved by this kernel.
        dn_bytes_expert = H * I * r.wl.bits // 8 + 2 * (H * I // 64) * 2
        pf_on = os.environ.get("TFM_DS_PREFETCH") == "1"
        prefetch = (sum(U) / len(U) * dn_bytes_expert) if (pf_on and streaming and T <= 3 and R <= 24) else 0.0
        achieved = (per_launch + prefetch) / dur_s / 1e9
        label = "ds_gateup_kernel" if streaming else gemv_gateup_label(g, T, r.wl.bits) if gemv else gemm_label
        return {"kernel": label,
                "bound": "hbm", "achieved": achieved,
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                "traffic": None, "alg_bytes_per_launch": per_launch + prefetch,
                "prefetch_bytes_per_launch": prefetch,
                "frac_gateup_bytes_only": per_launch / dur_s / 1e9 / HBM_PEAK_GBS, **timing}
    flops = wl.gemm_flops(g, T * g.top_k, "gateup")
    achieved = flops / dur_s / 1e12
    return {"kernel": gemm_label, "bound": "mfma",
            "achieved": achieved,
            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": achieved / BF16_PEAK_TFLOPS,
            "traffic": None, "alg_flops_per_launch": flops, **timing}


def source_sha16(rel: str):
    """First 16 hex digits of the SHA-256 of a repository file, or None."""
    import hashlib

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), rel)
    try:
        with open(path, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()[:16]
    except OSError:
        return None


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of the dominant (gate/up) kernel from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summaries (the JSON blocks of
    profiles/pmc_*.md), or None. A summary counts only for the kernel the
    workload runs today and only while the kernel's source file hashes as it
    did when the counters were read (its "source" and "source_sha16" keys), so
    that a changed kernel never inherits an old figure."""
    import glob
    import re

    here = os.path.dirname(os.path.abspath(__file__))
    for path in sorted(glob.glob(os.path.join(here, "profiles", "pmc_*.md"))):
        with open(path) as f:
            text = f.read()
        for block in re.findall(r"```json\n(.*?)\n```", text, re.S):
            try:
                d = json.loads(block)
            except ValueError:
                continue
            e = d.get(workload)
            if not isinstance(e, dict) or e.get("kernel") != kernel:
                continue
            src, sha = e.get("source"), e.get("source_sha16")
            if src and sha and source_sha16(src) == sha:
                return e.get("traffic_bytes")
    return None


def _host_layers(r: Runner, n: int):
    """Host (numpy) copies of the runner's first n layers for the CPU block."""
    import numpy as np

    class NpLayer:
        pass

    out = []
    for lay in r.layers[:n]:
        nl = NpLayer()
        for name in ("gate_q", "gate_s", "gate_b", "up_q", "up_s", "up_b", "down_q", "down_s", "down_b"):
            t = getattr(lay, name).cpu()
            setattr(nl, name, t.numpy() if t.dtype == r.torch.int32 else t.view(r.torch.int16).numpy())
        router = lay.router.cpu().view(r.torch.int16).numpy()
        lb = None if lay.logit_bias is None else lay.logit_bias.cpu().numpy()
        out.append((nl, router, lb))
    return out, r.x.cpu().view(r.torch.int16).numpy().view(np.uint16)


def _cpu_rate(r: Runner, host, x, seconds: float, threads: int, min_layers: int):
    """Whole layers of the CPU block, cycling through `host`, until `seconds`
    have elapsed and at least `min_layers` layers ran. Returns
    (tok/s, layers, seconds, threads used)."""
    import oracle

    T = r.wl.tokens
    layers, elapsed, used = 0, 0.0, threads
    while elapsed < seconds or layers < min_layers:
        nl, router, lb = host[layers % len(host)]
        t0 = time.perf_counter()
        _, _, _, used = oracle.moe_block_cpu(x, nl, r.geom.route, router, lb, top_k=r.geom.top_k,
                                             threads=threads)
        elapsed += time.perf_counter() - t0
        layers += 1
    return T * layers / elapsed, layers, elapsed, used


def cpu_baseline(r: Runner, seconds: float, one_thread_seconds: float, min_layers: int = 1,
                 nlayers: int = 16):
    """The oracle's MLX-semantics CPU block on the host cores over a bounded
    sample of the same workload: whole layers, cycling through `nlayers`
    distinct layers (so the host's last-level cache does not serve the
    weights), with every core and then with one thread."""
    model, cores = cpu_info()
    host, x = _host_layers(r, min(nlayers, len(r.layers)))
    rate, layers, elapsed, used = _cpu_rate(r, host, x, seconds, min(cores, 64), min_layers)
    out = {"value": rate, "unit": "tok/s", "cores": used, "kind": "port",
           "sample": f"{layers} layer passes x {r.wl.tokens} tokens of {r.wl.name}, cycling over "
                     f"{len(host)} distinct layers, {elapsed:.1f} s, {used} OpenMP threads on "
                     f"{cores} cores of {model}",
           "per_layer_ms": elapsed / layers * 1e3}
    if one_thread_seconds > 0:
        rate1, layers1, elapsed1, _ = _cpu_rate(r, host, x, one_thread_seconds, 1, 1)
        out["threads_1"] = {"value": rate1, "layers": layers1, "seconds": round(elapsed1, 2),
                            "per_layer_ms": elapsed1 / layers1 * 1e3}
    return out


def has_cpu_block(w) -> bool:
    """The oracle's CPU block runs bf16 storage with the dense router."""
    return w.dtype == "bf16" and w.router == "dense"


def workload_cpu_baseline(r: Runner):
    """A bounded CPU-block sample of one workload: all cores over at least 2 s
    (at least 3 whole layers from 2048 tokens), then one thread over at least
    1 s (one whole layer from 2048 tokens), cycling over 3 distinct layers."""
    big = r.wl.tokens >= 2048
    return cpu_baseline(r, 2.0, 1.0, min_layers=3 if big else 1, nlayers=3)


def measure(name, dev, args, steps, warmup, deterministic):
    """Eager, stage and HIP-graph timings of one workload."""
    r = Runner(name, dev, deterministic)
    ms, wall = r.time_steps(steps, warmup)
    st = r.stage_times(max(10, min(steps, 50)))
    gr = r.graph_time(steps, warmup)
    rep = workload_report(r, ms, wall, st, gr)
    rep["roofline_gateup"] = dominant_roofline(r, st)
    gms, same = gr
    rep["step_mode"] = "hip_graph" if same else "eager"
    rep["best_per_layer_us"] = (gms if same else ms) / r.nlayers * 1e3
    rep["best_tok_per_s"] = r.wl.tokens * r.nlayers / ((gms if same else ms) * 1e-3)
    return r, rep


# Dense affine linear shapes (quantized_matmul behind NativeLinearWeight,
# MLXNativeLinear.h:42-48): OLMoE's q/k/v/o projections and its router as a
# 4-bit affine matrix, at one token and at 512.
LINEAR_SHAPES = {"olmoe_qproj": (2048, 2048), "olmoe_router": (64, 2048)}
LINEAR_TOKENS = (1, 512)


def measure_dense_linear(dev, calls: int = 256):
    """tfm_affine_qmm per call, replayed from a HIP graph of `calls` calls that
    rotate over distinct weight matrices (at least 512 MB of them where the
    matrix is large enough, so that the Infinity Cache does not serve the
    weights; the router's 73 KB matrices total 19 MB and stay cached)."""
    import torch
    from trifuse_amd import moe as tmoe
    from trifuse_amd import workload as wl

    out = {}
    for name, (N, K) in LINEAR_SHAPES.items():
        wbytes = N * K // 2 + 2 * (N * (K // 64)) * 2
        nsets = max(1, min(calls, -(-(512 << 20) // wbytes)))
        q = wl.packed_nibbles((nsets, N, K // 8), 70 + N, dev)
        s = wl.uniform_scales((nsets, N, K // 64), 71 + N, dev)
        b = (s.float() * -8.0).to(torch.bfloat16)
        for T in LINEAR_TOKENS:
            x = wl.normal_bf16((T, K), 1.0, 72 + T).to(dev)
            def run():
                for i in range(calls):
                    tmoe.native_affine_qmm(x, q[i % nsets], s[i % nsets], b[i % nsets], 64, 4)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                run()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run()
            graph.replay()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            t0.record()
            for _ in range(reps):
                graph.replay()
            t1.record()
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) * 1e3 / (reps * calls)
            del graph
            nbytes = wbytes + T * K * 2 + T * N * 2
            flops = 2.0 * T * N * K
            out[f"{name}_t{T}"] = {"n_out": N, "k_in": K, "tokens": T, "us_per_call": round(us, 3),
                                   "weight_sets": nsets, "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                   "mfma_frac": round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                                   "path": "GEMV" if T <= 176 else "grouped GEMM",
                                   "timing": "HIP graph replay of consecutive calls"}
            log(f"[bench] dense linear {name} T={T}: {us:.2f} us per call")
        del q, s, b
        torch.cuda.empty_cache()
    return out


def layer_frac(rep):
    """Roofline fraction of the whole layer at the reported (best) step time."""
    frac = rep["hbm_frac"] if rep["bound"] == "hbm" else rep["mfma_frac"]
    return frac * rep["per_layer_us"] / rep["best_per_layer_us"]


def compact(name, rep):
    """Short per-workload summary for the output line: kernel durations are
    the kernels' own (dispatch timestamps), as a kernel trace reports them."""
    ru = rep["roofline_gateup"]
    out = {"per_layer_us": round(rep["best_per_layer_us"], 2), "tok_per_s": round(rep["best_tok_per_s"]),
           "bound": rep["bound"], "layer_frac": round(layer_frac(rep), 4),
           "gateup_us": round(ru["us_per_launch"], 2), "gateup_frac": round(ru["frac"], 4)}
    st = rep.get("stages_kernel_us") or rep["stages_us"]
    if "down" in st:
        out["down_us"] = round(st["down"], 2)
    traffic = measured_traffic(name, ru["kernel"])
    if traffic is not None:
        out["gateup_traffic"] = traffic  # HBM bytes per gate/up launch (rocprofv3 counters)
    if "zipf_top4_share" in rep:
        out["zipf_top4_share"] = rep["zipf_top4_share"]
    cb = rep.get("cpu_baseline")
    if cb:
        out["cpu_tok_per_s"] = round(cb["value"], 1)
        out["cpu_threads"] = cb["cores"]
        if "threads_1" in cb:
            out["cpu_tok_per_s_1thread"] = round(cb["threads_1"]["value"], 2)
    elif "cpu_baseline_skipped" in rep:
        out["cpu_tok_per_s"] = None
    return out


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "The design note on sharding describes how the MoE path would split over GPUs.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(1)
    if args.pmc_copy:
        pmc_copy(args.pmc_copy)
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from trifuse_amd import workload as wl

    if args.linear_only:
        print(json.dumps({"dense_linear": measure_dense_linear(dev)}), flush=True)
        return

    log(f"[bench] workload {args.workload}: building resident weights")
    head, report = measure(args.workload, dev, args, args.steps, args.warmup, args.deterministic)
    log(f"[bench] {args.workload}: {report['best_per_layer_us']:.2f} us/layer ({report['step_mode']})")
    roof = dict(report["roofline_gateup"])
    roof["traffic"] = measured_traffic(args.workload, roof["kernel"])
    roof["layer_frac"] = round(layer_frac(report), 4)  # the whole layer at the reported step time

    per = {args.workload: report}
    if not args.no_extra:
        names = [n for n in wl.WORKLOADS if n != args.workload and n != PREFILL_METRIC]
        if PREFILL_METRIC != args.workload:
            names.append(PREFILL_METRIC)  # measured last, printed last
        for name in names:
            log(f"[bench] workload {name}")
            decode = name in DECODE
            steps = args.steps if decode else max(10, args.steps // 2)
            r, rep = measure(name, dev, args, steps, max(3, args.warmup // 2), args.deterministic)
            per[name] = rep
            log(f"[bench] {name}: {rep['best_per_layer_us']:.2f} us/layer")
            if r.wl.zipf:
                top4 = r.route_stats()[1]
                rep["zipf_top4_share"] = {"min": round(min(top4), 4), "mean": round(sum(top4) / len(top4), 4),
                                          "max": round(max(top4), 4), "layers": len(top4)}
            if not args.no_cpu:
                if has_cpu_block(r.wl):
                    log(f"[bench] {name}: CPU block")
                    rep["cpu_baseline"] = workload_cpu_baseline(r)
                else:
                    rep["cpu_baseline_skipped"] = "the oracle's CPU block runs bf16 storage with a dense router only"
            del r
            torch.cuda.empty_cache()

    linear = None
    if not args.no_extra:
        log("[bench] dense affine linear")
        linear = measure_dense_linear(dev)

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline")
        cpu = cpu_baseline(head, args.cpu_seconds, max(1.0, args.cpu_seconds / 2))

    g = head.geom
    line = {
        "metric": METRIC,
        "value": report["best_tok_per_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": report["best_per_layer_us"] * head.nlayers / 1e3,
        "step_mode": report["step_mode"],
        "eager_ms_per_step": report["per_layer_us"] * head.nlayers / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": args.workload, "hidden": g.hidden, "experts": g.experts,
                   "top_k": g.top_k, "intermediate": g.intermediate, "tokens": head.wl.tokens,
                   "layers": head.nlayers, "weights": "4-bit affine g64, bf16 scales/biases",
                   "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "workloads": {n: compact(n, r) for n, r in per.items()
                      if n not in (args.workload, PREFILL_METRIC)},
    }
    if linear is not None:
        line["workloads"]["dense_linear"] = linear
    report["cpu_baseline"] = cpu
    mc = {args.workload: compact(args.workload, report)}
    if PREFILL_METRIC in per:
        mc[PREFILL_METRIC] = compact(PREFILL_METRIC, per[PREFILL_METRIC])
    line["metric_configs"] = mc
    if args.report:
        with open(args.report, "w") as f:
            json.dump({"line": line, "per_workload": per}, f, indent=1)
    for n, c in mc.items():
        log(f"[bench] {n}: " + json.dumps(c))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
