#!/usr/bin/env python3
"""MSDA forward + backward benchmark on one MI355X.

One step = what one training step of a BEVFormer spatial-cross-attention
layer asks of the operator, as the operator's autograd function issues it:
allocate the three gradients (the kernels overwrite them, so nothing is
zero-filled) and the backward scratch, start the backward's binning (it reads
only the geometry) on a second stream, allocate the output and run the
forward, then the rest of the backward -- the timed region of the reference's
benchmark (/root/reference/benchmarks/msda/benchmark_msda.py:85-119), through
the C-ABI entry points the autograd function uses.

Workload: BASELINE config c2 (bs*cams 6, nq 10000, 8 heads x 32 channels,
levels (116,200),(58,100),(29,50),(15,25), 8 points, float32), seeded
synthetic inputs resident in HBM before timing.

value = effective GB/s = algorithmic bytes of fwd+bwd / measured time per step
(byte model: every tensor once at its storage width; see muspace_amd/workloads.py).
The roofline entry prices the dominant kernel, msda_tile_backward (the
backward's second part, ms_deform_attn_backward_rest), on the tensors it reads
or writes once -- value, grad_output and the three float32 gradients -- against
the 8 TB/s HBM peak, from HIP events around its launch on the main stream in
the timed region; `traffic` is its measured HBM bytes per launch (rocprofv3
FETCH_SIZE/WRITE_SIZE, calibrated on a copy kernel) from
profiles/traffic_c2_fp32.json. cpu_baseline times the oracle (a CPU restatement of the reference's
PyTorch path) on a query subset of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

from muspace_amd.workloads import (  # noqa: E402
    CONFIGS,
    HBM_PEAK_GBPS,
    algorithmic_bytes,
    backward_rest_bytes,
    make_inputs,
    make_published_case,
    dfa_algorithmic_bytes,
    make_dfa_inputs,
    make_sca_inputs,
    sca_algorithmic_bytes,
)

METRIC = "MSDA fwd+bwd µs/call + effective GB/s (% HBM peak), BEVFormer SCA shape"
TRAFFIC_FILE = ROOT / "profiles" / "traffic_c2_fp32.json"


class Step:
    """Preallocated inputs of one config and the launches of one step.

    As the operator's autograd function does (binning="fused"): the gradient
    buffers and the backward's workspace are allocated first, one call runs
    the forward together with the backward's binning (the forward kernel stores
    the backward's records), and the rest of the backward follows once
    grad_output is there. binning="side" is the earlier schedule kept for
    comparison: the three binning kernels on a second stream beside the
    forward kernel; "serial" runs them on the main stream before it (for
    per-kernel profiles).
    """

    def __init__(self, lib, cfg, value_dtype, geometry_dtype, device, binning="fused"):
        t = make_inputs(cfg, value_dtype=value_dtype, geometry_dtype=geometry_dtype, device=device)
        self.lib = lib
        self.value = t["value"]
        self.shapes = t["spatial_shapes"]
        self.starts = t["level_start_index"]
        self.loc = t["sampling_locations"]
        self.attn = t["attention_weights"]
        self.grad = t["grad_output"]
        self.out_shape = (cfg.batch, cfg.queries, cfg.heads * cfg.channels)
        self.binning = binning
        # default priority
        self.side = torch.cuda.Stream() if binning == "side" else torch.cuda.current_stream()

    def alloc(self):
        dev = self.value.device
        gv = torch.empty(self.value.shape, dtype=torch.float32, device=dev)
        gl = torch.empty(self.loc.shape, dtype=torch.float32, device=dev)
        ga = torch.empty(self.attn.shape, dtype=torch.float32, device=dev)
        ws = self.lib.backward_workspace(self.value, self.loc)
        return gv, gl, ga, ws

    def bin(self, bufs):
        gv, gl, ga, ws = bufs
        self.lib.ms_deform_attn_backward_bin(self.value, self.shapes, self.starts, self.loc,
                                             self.attn, gv, gl, ga, 64, ws, stream=self.side)

    def forward(self):
        out = torch.empty(self.out_shape, dtype=self.value.dtype, device=self.value.device)
        self.lib.ms_deform_attn_forward(self.value, self.shapes, self.starts, self.loc,
                                        self.attn, out, 64)
        return out

    def forward_bin(self, bufs):
        gv, gl, ga, ws = bufs
        out = torch.empty(self.out_shape, dtype=self.value.dtype, device=self.value.device)
        self.lib.ms_deform_attn_forward_bin(self.value, self.shapes, self.starts, self.loc,
                                            self.attn, out, gv, gl, ga, 64, ws)
        return out

    def rest(self, bufs):
        gv, gl, ga, ws = bufs
        self.lib.ms_deform_attn_backward_rest(self.value, self.shapes, self.starts, self.loc,
                                              self.attn, self.grad, gv, gl, ga, 64, ws)

    def run(self, marks=None):
        """One step; `marks(name)` records a HIP event on the stream that the
        launch named `name` uses, before and after it."""
        main = torch.cuda.current_stream()
        mark = marks or (lambda name, stream: None)
        mark("alloc0", main)
        bufs = self.alloc()
        mark("alloc1", main)
        if self.binning == "fused":
            mark("fwd0", main)
            self.forward_bin(bufs)
            mark("fwd1", main)
            mark("rest0", main)
            self.rest(bufs)
            mark("rest1", main)
            return
        ready = torch.cuda.Event()
        ready.record(main)
        self.side.wait_event(ready)
        mark("bin0", self.side)
        self.bin(bufs)
        mark("bin1", self.side)
        for b in bufs:
            b.record_stream(self.side)
        mark("fwd0", main)
        self.forward()
        mark("fwd1", main)
        done = torch.cuda.Event()
        done.record(self.side)
        main.wait_event(done)
        mark("rest0", main)
        self.rest(bufs)
        mark("rest1", main)


PARITY_QUERIES = 48  # queries per batch entry checked against the oracle


def check_step_parity(step: Step, cfg, value_dtype) -> dict:
    """The timed step's results, from one untimed run of the same launches on
    the same inputs, against the oracle (oracle/msda_torch.py, the CPU
    restatement of the reference's PyTorch path, as the checker only).

    On a seeded subset of PARITY_QUERIES queries (every batch entry) the
    output and the location and weight gradients depend only on those
    queries, so the oracle on the subset gives their exact values. grad_value
    sums over all queries; it is checked at full size through the adjoint
    identities <grad_out, out> = <value, grad_value> = <attn, grad_attn>
    (MSDA is linear in value and in the attention weights), and every
    gradient element must have been written (finite). Tolerances are the
    north star's: float32 output 1e-5 and gradients 1e-4, 16-bit storage
    1e-2 (|a - e| <= tol + tol |e|); adjoint identities 1e-5 (float32) and
    3e-3 (16-bit) of sum |grad_out * out|."""
    from oracle import msda_torch

    bufs = step.alloc()
    if step.binning == "fused":
        out = step.forward_bin(bufs)
    else:
        saved, step.side = step.side, torch.cuda.current_stream()
        step.bin(bufs)
        step.side = saved
        out = step.forward()
    step.rest(bufs)
    torch.cuda.synchronize()
    gv, gl, ga, _ = bufs

    g = torch.Generator().manual_seed(7)
    idx = torch.randperm(cfg.queries, generator=g)[:PARITY_QUERIES].sort().values
    idx_dev = idx.to(out.device)
    value = step.value.float().cpu()
    loc = step.loc[:, idx_dev].float().cpu()
    attn = step.attn[:, idx_dev].float().cpu()
    grad = step.grad[:, idx_dev].float().cpu()
    o_out, _, o_gl, o_ga = msda_torch.msda_forward_backward(value, step.shapes.cpu(), loc, attn,
                                                            grad)
    ftol, btol = (1e-5, 1e-4) if value_dtype == torch.float32 else (1e-2, 1e-2)

    def worst(actual, expected, tol):
        """max of |a - e| / (tol + tol |e|): at most 1 passes"""
        a, e = actual.double().cpu(), expected.double()
        return float(((a - e).abs() / (tol + tol * e.abs())).max())

    ratios = {
        "output": worst(out[:, idx_dev], o_out, ftol),
        "grad_sampling_locations": worst(gl[:, idx_dev], o_gl, btol),
        "grad_attention_weights": worst(ga[:, idx_dev], o_ga, btol),
    }
    written = bool(torch.isfinite(gv).all() and torch.isfinite(gl).all()
                   and torch.isfinite(ga).all())
    lhs = float((out.double() * step.grad.double()).sum())
    scale = float((out.double().abs() * step.grad.double().abs()).sum())
    rel = 1e-5 if value_dtype == torch.float32 else 3e-3
    adj_v = abs(lhs - float((step.value.double() * gv.double()).sum())) / (rel * scale)
    adj_a = abs(lhs - float((step.attn.double() * ga.double()).sum())) / (rel * scale)
    ratios["adjoint_value_grad_value"] = adj_v
    ratios["adjoint_attn_grad_attn"] = adj_a
    ok = written and all(r <= 1.0 for r in ratios.values())
    del bufs, out
    return {
        "ok": ok,
        "checked": f"one run of the timed step's launches, before timing: output, "
                   f"grad_sampling_locations and grad_attention_weights on {PARITY_QUERIES} "
                   f"seeded queries x {cfg.batch} batch entries against oracle/msda_torch.py; "
                   f"grad_value through the adjoint identities at full size",
        "tolerance": {"forward": ftol, "backward": btol, "adjoint_rel": rel},
        "worst_error_over_tolerance": {k: round(v, 4) for k, v in ratios.items()},
        "all_gradients_written": written,
    }


def fused_binning(lib, cfg, value_dtype) -> bool:
    """Whether ms_deform_attn_forward_bin stores the backward's records from
    the forward kernel at this config (else the plain forward and the
    binning kernels run in that call)."""
    value = torch.empty((cfg.batch, cfg.spatial_size, cfg.heads, cfg.channels),
                        dtype=value_dtype, device="meta")
    loc = torch.empty((cfg.batch, cfg.queries, cfg.heads, cfg.num_levels, cfg.points, 2),
                      device="meta")
    return lib.forward_bin_fuses(value, loc)


def time_steps(step: Step, steps: int, warmup: int, per_kernel: bool = True,
               repeats: int = 5) -> dict:
    """Time exactly `steps` steps after `warmup`, as `repeats` back-to-back
    repeats of steps // repeats steps (the remainder goes to the first
    repeats), each bracketed by device synchronisation and HIP events on the
    main stream; ms_per_step is the median of the repeats' per-step means
    (the reference's protocol, /root/reference/benchmarks/_harness.py:226-260),
    with the overall mean beside it. rest_ms is likewise the median over the
    repeats of the repeat's mean rest-of-backward time, so one disturbed
    repeat moves neither figure. Inside the timed region HIP events sit
    only around the rest of the backward (the roofline's kernel) on the main
    stream: each pair of events costs about 10 us a step, and a pair around
    the forward also delays its overlap with the binning. The forward's, the
    binning's and the allocation's durations come from a separate pass of a
    few steps. bwd_ms adds the binning and the rest."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        step.run()
    torch.cuda.synchronize()
    marks = []

    def marker(wanted):
        def mark(name, st):
            if name in wanted:
                e = torch.cuda.Event(enable_timing=True)
                e.record(st)
                marks[-1][name] = e
        return mark

    timed = marker({"rest0", "rest1"})
    repeats = max(1, min(repeats, steps))
    counts = [steps // repeats + (1 if r < steps % repeats else 0) for r in range(repeats)]
    samples, total_ms = [], 0.0
    t0 = time.perf_counter()
    for n in counts:
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(n):
            if per_kernel:
                marks.append({"repeat": len(samples)})
                step.run(timed)
            else:
                step.run()
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end)
        samples.append(ms / n)
        total_ms += ms
    wall = time.perf_counter() - t0
    res = {"ms_per_step": statistics.median(samples), "mean_ms_per_step": total_ms / steps,
           "repeat_ms_per_step": [round(x, 4) for x in samples],
           "wall_ms_per_step": wall * 1e3 / steps}
    if per_kernel:
        def avg(a, b):
            return sum(m[a].elapsed_time(m[b]) for m in marks) / len(marks)
        per_repeat = {}
        for m in marks:
            per_repeat.setdefault(m["repeat"], []).append(m["rest0"].elapsed_time(m["rest1"]))
        res["rest_ms"] = statistics.median(statistics.fmean(v) for v in per_repeat.values())
        res["repeat_rest_ms"] = [round(statistics.fmean(v), 4) for _, v in sorted(per_repeat.items())]
        marks.clear()
        extra = marker({"fwd0", "fwd1", "bin0", "bin1", "alloc0", "alloc1"})
        for _ in range(max(3, min(steps, 10))):
            marks.append({})
            step.run(extra)
        torch.cuda.synchronize()
        res["fwd_ms"] = avg("fwd0", "fwd1")
        # fused: the binning is part of the forward call
        res["bin_ms"] = avg("bin0", "bin1") if step.binning != "fused" else 0.0
        res["zero_ms"] = avg("alloc0", "alloc1")
        res["bwd_ms"] = res["bin_ms"] + res["rest_ms"]
    return res


def harness_ms(fn, warmup: int = 20, iterations: int = 100, repeats: int = 5) -> float:
    """The reference's protocol (/root/reference/benchmarks/_harness.py:226-260):
    `warmup` calls, then `repeats` repeats of `iterations` calls between HIP
    events on the current stream; the median of the repeats' per-call ms."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(repeats):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iterations):
            fn()
        end.record(stream)
        end.synchronize()
        samples.append(start.elapsed_time(end) / iterations)
    return statistics.median(samples)


def _event_ms(fn, steps: int, warmup: int, repeats: int = 3) -> float:
    """ms of fn() per call, HIP events on the current stream: the median over
    `repeats` timed runs of `steps` calls each (one stalled run, such as a
    first allocation inside it, does not set the figure)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    runs = []
    for _ in range(repeats):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        runs.append(start.elapsed_time(end) / steps)
    return statistics.median(runs)


def time_sca(lib, steps: int = 50, warmup: int = 10) -> dict:
    """BEVFormer spatial cross-attention epilogue at c2 (one sample, six cameras,
    200 x 200 BEV grid): the fused scatter-average against the unfused
    composition (dense MSDA output, per-camera ``slots[idx] += out``, then
    ``slots / count``), forward and forward + backward."""
    from muspace_amd import multi_scale_deformable_attn, multi_scale_deformable_attn_scatter_div

    t = make_sca_inputs(device="cuda")
    value, shapes, starts = t["value"], t["spatial_shapes"], t["level_start_index"]
    loc, attn, indexes, count = (t["sampling_locations"], t["attention_weights"], t["indexes"],
                                 t["count"])
    cams, max_len = len(indexes), loc.shape[1]
    row = value.shape[2] * value.shape[3]
    slots = torch.zeros((1, count.shape[1], row), device="cuda")

    index_all = torch.cat(indexes)
    lens = [int(i.numel()) for i in indexes]

    def fused_kernels():  # the all-camera launch alone
        lib.ms_deform_attn_forward_scatter_div_cams(value, shapes, starts, loc, attn, index_all,
                                                    lens, count, slots)

    def per_camera_kernels():  # the reference's interface: one ordered launch per camera
        for cam, index in enumerate(indexes):
            lib.ms_deform_attn_forward_scatter_div(value, shapes, starts, loc, attn, index, count,
                                                   slots, cams, cam)

    def fused():
        return multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                       count)

    def unfused():
        out = multi_scale_deformable_attn(value, shapes, starts, loc, attn).view(
            1, cams, max_len, row)
        acc = torch.zeros((1, count.shape[1], row), device="cuda")
        for cam, index in enumerate(indexes):
            acc[:, index] += out[:, cam, : len(index)]
        return acc / count[..., None]

    grad = torch.randn((1, count.shape[1], row), generator=torch.Generator().manual_seed(1))
    grad = grad.to("cuda")
    leaves = [x.detach().requires_grad_(True) for x in (value, loc, attn)]

    def train(fn):
        def step():
            v, l, a = leaves
            for x in leaves:
                x.grad = None
            if fn is fused:
                y = multi_scale_deformable_attn_scatter_div(v, shapes, starts, l, a, indexes, count)
            else:
                out = multi_scale_deformable_attn(v, shapes, starts, l, a).view(
                    1, cams, max_len, row)
                y = torch.zeros((1, count.shape[1], row), device="cuda")
                for cam, index in enumerate(indexes):
                    y[:, index] += out[:, cam, : len(index)]
                y = y / count[..., None]
            y.backward(grad)
        return step

    kernel_ms = _event_ms(fused_kernels, steps, warmup)
    valid = sum(int(i.numel()) for i in indexes)
    nbytes = sca_algorithmic_bytes(valid, cams, count.shape[1])
    res = {
        "workload": f"c2 as 1 sample x {cams} cameras, BEV 200x200 = {count.shape[1]} queries, "
                    f"{valid} valid camera rows (max_len {max_len})",
        "fused_kernels_us": round(kernel_ms * 1e3, 1),
        "per_camera_kernels_us": round(_event_ms(per_camera_kernels, steps, warmup) * 1e3, 1),
        "fused_fwd_us": round(_event_ms(fused, steps, warmup) * 1e3, 1),
        "unfused_fwd_us": round(_event_ms(unfused, steps, warmup) * 1e3, 1),
        "fused_fwd_bwd_us": round(_event_ms(train(fused), steps // 2, warmup) * 1e3, 1),
        "unfused_fwd_bwd_us": round(_event_ms(train(unfused), steps // 2, warmup) * 1e3, 1),
        "algorithmic_bytes": nbytes,
        "effective_GBps": round(nbytes / (kernel_ms * 1e-3) / 1e9, 1),
    }
    res["pct_hbm_peak"] = round(100 * res["effective_GBps"] / HBM_PEAK_GBPS, 2)
    return res


def time_softmax(lib, steps: int = 50, warmup: int = 10) -> dict:
    """The attention softmax fused into MSDA at c2 (logits in, softmax over
    each query's L*P samples per head) against torch.softmax followed by the
    operator: the kernels alone (native calls, no autograd), the forward
    through the operators, and forward + backward steps."""
    from muspace_amd.ops import (attention_softmax, multi_scale_deformable_attn,
                                 multi_scale_deformable_attn_softmax)

    cfg = CONFIGS["c2"]
    t = make_inputs(cfg, value_dtype=torch.float32, device="cuda")
    value, shapes, starts, loc = (t["value"], t["spatial_shapes"], t["level_start_index"],
                                  t["sampling_locations"])
    g = torch.Generator(device="cpu").manual_seed(5)
    logits = torch.randn(t["attention_weights"].shape, generator=g).to("cuda")
    out = torch.empty((cfg.batch, cfg.queries, cfg.heads * cfg.channels), device="cuda")
    grad = t["grad_output"]

    def fused_kernel():
        lib.ms_deform_attn_forward_softmax(value, shapes, starts, loc, logits, out, 64)

    def unfused_kernels():
        lib.ms_deform_attn_forward(value, shapes, starts, loc, attention_softmax(logits), out, 64)

    def fwd(fused):
        def run():
            with torch.no_grad():
                if fused:
                    multi_scale_deformable_attn_softmax(value, shapes, starts, loc, logits)
                else:
                    multi_scale_deformable_attn(value, shapes, starts, loc,
                                                attention_softmax(logits))
        return run

    leaves = [x.detach().requires_grad_(True) for x in (value, loc, logits)]

    def train(fused):
        def step():
            v, lc, lg = leaves
            for x in leaves:
                x.grad = None
            if fused:
                y = multi_scale_deformable_attn_softmax(v, shapes, starts, lc, lg)
            else:
                y = multi_scale_deformable_attn(v, shapes, starts, lc, attention_softmax(lg))
            y.backward(grad)
        return step

    return {
        "workload": "c2 (BEVFormer SCA, bs*cams 6, 10000 queries, 8 heads x 32, 4 levels x 8 "
                    "points), logits ~ N(0, 1)",
        "fused_kernel_us": round(_event_ms(fused_kernel, steps, warmup) * 1e3, 1),
        "softmax_then_kernel_us": round(_event_ms(unfused_kernels, steps, warmup) * 1e3, 1),
        "fused_fwd_us": round(_event_ms(fwd(True), steps, warmup) * 1e3, 1),
        "unfused_fwd_us": round(_event_ms(fwd(False), steps, warmup) * 1e3, 1),
        "fused_fwd_bwd_us": round(_event_ms(train(True), steps // 2, warmup) * 1e3, 1),
        "unfused_fwd_bwd_us": round(_event_ms(train(False), steps // 2, warmup) * 1e3, 1),
    }


def time_dfa(lib, steps: int = 50, warmup: int = 10) -> dict:
    """Deformable aggregation at SparseDrive's production shape, kernel-only
    scope as the reference's benchmark
    (/root/reference/benchmarks/deformable_aggregation/README.md:31-40): output
    and gradients allocated once before the timed region, one entry-point call
    per launch (the kernels add into those buffers, which changes the values,
    not the work)."""
    t = make_dfa_inputs(device="cuda")
    mc, spatial, start = t["mc_ms_feat"], t["spatial_shape"], t["scale_start_index"]
    loc, weights, grad = t["sampling_location"], t["weights"], t["grad_output"]
    out = torch.zeros((mc.shape[0], loc.shape[1], mc.shape[2]), device="cuda")
    gf, gl, gw = torch.zeros_like(mc), torch.zeros_like(loc), torch.zeros_like(weights)
    fwd_ms = _event_ms(lambda: lib.deformable_aggregation_forward_opt(
        mc, spatial, start, loc, weights, out), steps, warmup)
    bwd_ms = _event_ms(lambda: lib.deformable_aggregation_backward_opt(
        mc, spatial, start, loc, weights, grad, gf, gl, gw), steps, warmup)
    fwd_b, bwd_b = dfa_algorithmic_bytes()
    active = float(((loc > 0) & (loc < 1)).all(-1).float().mean())
    return {
        "workload": "SparseDrive deformable aggregation: mc_ms_feat [8, 89760, 256], 6 cameras x "
                    "4 scales, 900 anchors x 13 points, 8 groups, float32, "
                    f"active fraction {active:.4f}",
        "fwd_us": round(fwd_ms * 1e3, 1),
        "bwd_us": round(bwd_ms * 1e3, 1),
        "fwd_GBps": round(fwd_b / (fwd_ms * 1e-3) / 1e9, 1),
        "bwd_GBps": round(bwd_b / (bwd_ms * 1e-3) / 1e9, 1),
        "algorithmic_bytes": {"fwd": fwd_b, "bwd": bwd_b},
        "published_ms": {"MTT S5000 fwd": 7.7067, "MTT S5000 bwd": 25.1164},
    }


def cpu_threads() -> int:
    """Host cores this process may use: its CPU affinity, bounded by a cgroup
    CPU quota when one is set (a container's share of a larger host)."""
    cores = len(os.sched_getaffinity(0))
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if quota != "max":
            cores = min(cores, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return cores


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


# CPU baseline rows: config -> queries timed (None: all). The oracle's time is
# proportional to the sampled queries (the value is the full tensor), so a
# subset's time is scaled by queries / subset to the full workload.
CPU_ROWS = (("c0", None), ("c1", 2000), ("c2", 1000), ("c3", 8000), ("c4", 500))


def cpu_baseline() -> dict:
    """The oracle (oracle/msda_torch.py, an op-for-op CPU restatement of the
    reference's PyTorch path) on the host CPU with every available core:
    c0 forward only at full size; c1-c3 forward + autograd backward in float32
    and c4 in float32 on value-upcast inputs, each on a query subset scaled to
    the full query count. Protocol: warmup 1, then 3 repeats of 3 iterations,
    median of the repeats' per-call seconds."""
    from oracle import msda_torch

    threads = cpu_threads()
    torch.set_num_threads(threads)
    rows = {}
    for name, subset in CPU_ROWS:
        cfg = CONFIGS[name]
        sample = cfg if subset is None else cfg.with_queries(subset)
        t = make_inputs(sample, device="cpu")
        args = [t[k] for k in ("value", "spatial_shapes", "sampling_locations",
                               "attention_weights")]
        if cfg.backward:
            def run():
                msda_torch.msda_forward_backward(*args, t["grad_output"])
        else:
            def run():
                with torch.no_grad():
                    msda_torch.msda_forward(*args)
        run()
        per_call = []
        for _ in range(3):
            t0 = time.perf_counter()
            for _ in range(3):
                run()
            per_call.append((time.perf_counter() - t0) / 3)
        sec = statistics.median(per_call) * cfg.queries / sample.queries
        fwd_b, bwd_b = algorithmic_bytes(cfg)
        nbytes = fwd_b + (bwd_b if cfg.backward else 0)
        rows[name] = {
            "scope": "fwd+bwd" if cfg.backward else "fwd",
            "ms": round(sec * 1e3, 2),
            "GBps": round(nbytes / sec / 1e9, 3),
            "queries_timed": sample.queries,
            "scale": round(cfg.queries / sample.queries, 3),
        }
        print(f"[bench] cpu {name}: {rows[name]}", file=sys.stderr, flush=True)
    c2 = rows["c2"]
    return {
        "value": c2["GBps"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"oracle/msda_torch.py fwd+autograd bwd, float32, c2 on {c2['queries_timed']} of "
            f"{CONFIGS['c2'].queries} queries per camera (all 6 cameras, full value), median "
            f"of 3 repeats x 3 calls scaled x{c2['scale']:g} to {c2['ms']:.0f} ms per full "
            f"step; {threads} threads on {cpu_model()}"
        ),
        "cpu_model": cpu_model(),
        "rows": rows,
    }


def time_forward_only(lib, name: str) -> dict:
    """A config's forward alone (c0, whose case is forward-only; c2 without a
    gradient graph) through the C-ABI forward, reference protocol."""
    cfg = CONFIGS[name]
    t = make_inputs(cfg, device="cuda", with_grad_output=False)
    out = torch.empty((cfg.batch, cfg.queries, cfg.heads * cfg.channels), device="cuda")
    args = (t["value"], t["spatial_shapes"], t["level_start_index"], t["sampling_locations"],
            t["attention_weights"], out, 64)
    ms = harness_ms(lambda: lib.ms_deform_attn_forward(*args))
    fwd_b, _ = algorithmic_bytes(cfg)
    return {"fwd_us": round(ms * 1e3, 2), "effective_GBps": round(fwd_b / (ms * 1e-3) / 1e9, 1)}


def time_published_case(lib, dtype) -> dict:
    """The reference's published case ``bevformer-1l`` in its own timed region
    (/root/reference/benchmarks/msda/benchmark_msda.py:85-119): allocate the
    output, one forward launch on the forward input set; allocate the three
    float32 gradients (torch.empty: these kernels overwrite them, where the
    reference's accumulate into zero-filled ones), copy the non-contiguous
    grad_output with ``.contiguous()``, one backward launch on the backward
    input set (its workspace allocated inside, as the operator's backward
    does). Every tensor in ``dtype``; warmup 20, 5 repeats x 100, median."""
    case = make_published_case(dtype=dtype, device="cuda")
    names = ("value", "spatial_shapes", "level_start_index", "sampling_locations",
             "attention_weights")
    fwd = tuple(case["forward_inputs"][k] for k in names)
    bwd = tuple(case["backward_inputs"][k] for k in names)
    grad_output = case["backward_inputs"]["grad_output"]
    assert not grad_output.is_contiguous()

    def launch():
        out = fwd[0].new_empty((fwd[0].size(0), fwd[3].size(1), fwd[0].size(2) * fwd[0].size(3)))
        lib.ms_deform_attn_forward(*fwd, out, 64)
        gv = torch.empty(bwd[0].shape, dtype=torch.float32, device="cuda")
        gl = torch.empty(bwd[3].shape, dtype=torch.float32, device="cuda")
        ga = torch.empty(bwd[4].shape, dtype=torch.float32, device="cuda")
        lib.ms_deform_attn_backward(*bwd, grad_output.contiguous(), gv, gl, ga, 64)

    ms = harness_ms(launch)
    published = {torch.float32: {"MTT S5000": 4.2387, "A100 (mmcv CUDA)": 4.0895},
                 torch.bfloat16: {"MTT S5000": 3.9933}}[dtype]
    return {
        "fwd_bwd_us": round(ms * 1e3, 1),
        "published_ms": published,
        "speedup_vs_S5000": round(published["MTT S5000"] / ms, 2),
        "note": "reference inputs and timed region; published rows are other hardware "
                "(benchmarks/msda/README.md:72-73)",
    }


def probe_library():
    import ctypes

    from muspace_amd.build import PROBE_LIBRARY

    if not PROBE_LIBRARY.is_file():
        raise SystemExit(f"{PROBE_LIBRARY} is missing; build with `python -m muspace_amd.build`")
    lib = ctypes.CDLL(str(PROBE_LIBRARY))
    for fn in (lib.muspace_probe_gather, lib.muspace_probe_atomic):
        fn.restype = ctypes.c_int
    lib.muspace_probe_gather.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.muspace_probe_atomic.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_void_p]
    lib.muspace_probe_scatter.restype = ctypes.c_int
    lib.muspace_probe_scatter.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.muspace_probe_lds_atomic.restype = ctypes.c_int
    lib.muspace_probe_lds_atomic.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_void_p]
    return lib


def run_lds_atomic_probe() -> dict:
    """fp32 against u32 and u64 LDS atomic adds (ds_add_f32 / ds_add_u32 /
    ds_add_u64), consecutive (conflict-free for 32-bit) and scattered
    addresses: clocks per wavefront instruction per CU, at the device's
    reported clock."""
    lib = probe_library()
    props = torch.cuda.get_device_properties(0)
    cus = props.multi_processor_count
    clock_hz = getattr(props, "clock_rate", 0) * 1e3 or 2.4e9
    blocks, iters = 2 * cus, 2048
    stream = torch.cuda.current_stream().cuda_stream
    out = torch.empty(blocks * 1024, dtype=torch.int32, device="cuda")
    rows = {}
    for kind, name in ((0, "f32_conflict_free"), (1, "u32_conflict_free"),
                       (2, "f32_scattered"), (3, "u32_scattered"),
                       (5, "u64_consecutive"), (7, "u64_scattered")):
        def launch():
            rc = lib.muspace_probe_lds_atomic(out.data_ptr(), blocks, iters, kind, stream)
            assert rc == 0, rc
        launch()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        launch()
        end.record()
        end.synchronize()
        ms = start.elapsed_time(end)
        wave_instr_per_cu = blocks * 16 * iters / cus
        row = {"ms": round(ms, 3),
               "clk_per_wave_instr_per_cu": round(ms * 1e-3 * clock_hz / wave_instr_per_cu, 2)}
        rows[name] = row
        print(f"[probe] lds atomic {name}: {row}", file=sys.stderr, flush=True)
    return {"lds_atomic_probe": rows}


PROBE_MIB = (1, 2, 4, 8, 16)  # footprint per XCD
SCATTER_PROBE_MIB = (0.25, 0.5, 1, 2, 4, 8, 16)  # records * 12 bytes per XCD


def run_scatter_probe() -> dict:
    """Scattered 12-byte records (a 4-byte and an 8-byte store to random
    records of two arrays, like the tile backward's direct location and weight
    gradient writes), every workgroup in its own XCD's region of 0.25-16 MiB;
    2048 workgroups of 256 threads, 32 records a lane. Reports records per
    second and the time c2's 15.36 M samples' records take at that rate."""
    lib = probe_library()
    blocks, iters = 2048, 32
    stream = torch.cuda.current_stream().cuda_stream
    max_records = int(max(SCATTER_PROBE_MIB) * (1 << 20)) // 12
    ga = torch.zeros(8 * max_records, device="cuda")
    gl = torch.zeros(8 * max_records, 2, device="cuda")
    rows = {}
    for mib in SCATTER_PROBE_MIB:
        records = int(mib * (1 << 20)) // 12

        def launch():
            rc = lib.muspace_probe_scatter(ga.data_ptr(), gl.data_ptr(), records, blocks, iters,
                                           stream)
            assert rc == 0, rc
        launch()
        torch.cuda.synchronize()
        reps = 5
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            launch()
        end.record()
        end.synchronize()
        ms = start.elapsed_time(end) / reps
        per_s = blocks * 256 * iters / (ms * 1e-3)
        row = {"us": round(ms * 1e3, 1), "G_records_per_s": round(per_s / 1e9, 1),
               "us_for_c2_samples": round(15_360_000 / per_s * 1e6, 1)}
        rows[f"{mib}MiB_per_xcd"] = row
        print(f"[probe] scatter {mib} MiB/XCD: {row}", file=sys.stderr, flush=True)
    return {"scatter_probe": rows}


def run_probe(kind: str) -> dict:
    """Random 128-byte line gathers (16 B a lane, 8 independent loads in
    flight per lane) or line-wide fp32 atomic adds, every workgroup in its own
    XCD's region of 1-16 MiB; 2048 workgroups of 256 threads. The atomic sums
    are checked exactly against the number of adds."""
    lib = probe_library()
    blocks, iters = 2048, 512
    stream = torch.cuda.current_stream().cuda_stream
    rows = {}
    max_lines = max(PROBE_MIB) * (1 << 20) // 128
    buf = torch.zeros(8 * max_lines * 32, device="cuda")
    sink = torch.empty(blocks * 256, device="cuda")
    for mib in PROBE_MIB:
        lines = mib * (1 << 20) // 128
        if kind == "gather":
            def launch():
                rc = lib.muspace_probe_gather(buf.data_ptr(), lines, blocks, iters,
                                              sink.data_ptr(), stream)
                assert rc == 0, rc
            lines_moved = blocks * 256 // 8 * iters
        else:
            buf.zero_()

            def launch():
                rc = lib.muspace_probe_atomic(buf.data_ptr(), lines, blocks, iters, stream)
                assert rc == 0, rc
            lines_moved = blocks * 256 // 32 * iters
        launch()
        torch.cuda.synchronize()
        reps = 5
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            launch()
        end.record()
        end.synchronize()
        ms = start.elapsed_time(end) / reps
        row = {"us": round(ms * 1e3, 1),
               "G_lines_per_s": round(lines_moved / (ms * 1e-3) / 1e9, 2),
               "TBps": round(lines_moved * 128 / (ms * 1e-3) / 1e12, 2)}
        if kind == "atomic":
            adds = blocks * 256 * iters * (reps + 1)
            row["sum_exact"] = float(buf.double().sum()) == float(adds)
        rows[f"{mib}MiB_per_xcd"] = row
        print(f"[probe] {kind} {mib} MiB/XCD: {row}", file=sys.stderr, flush=True)
    return {f"{kind}_probe": rows}


def read_traffic():
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (counters cannot be collected
    inside the timed run itself)."""
    if TRAFFIC_FILE.is_file():
        try:
            return json.loads(TRAFFIC_FILE.read_text()).get("rest_traffic_bytes")
        except (ValueError, OSError):
            return None
    return None


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    parser.add_argument("--value-dtype", default="float32",
                        choices=["float32", "bfloat16", "float16"],
                        help="storage type of value and grad_output in the main step "
                             "(locations and weights stay float32); c4 is quoted in the "
                             "16-bit types")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-extra-configs", action="store_true")
    parser.add_argument("--repeats", type=int, default=5,
                        help="the timed steps are split into this many repeats; the median "
                             "repeat is reported")
    parser.add_argument("--gather-probe", action="store_true",
                        help="only the random 128-byte line gather probe (the forward's "
                             "corner-gather ceiling), then exit")
    parser.add_argument("--lds-atomic-probe", action="store_true",
                        help="time fp32 against u32 LDS atomic adds and exit")
    parser.add_argument("--atomic-probe", action="store_true",
                        help="only the line-wide fp32 atomic-add probe, then exit")
    parser.add_argument("--scatter-probe", action="store_true",
                        help="only the scattered 12-byte record store probe (the tile "
                             "backward's direct gradient writes), then exit")
    parser.add_argument("--sca-only", action="store_true",
                        help="only the fused spatial cross-attention scatter-average leg")
    parser.add_argument("--dfa-only", action="store_true",
                        help="only the deformable aggregation leg")
    parser.add_argument("--softmax-only", action="store_true",
                        help="only the fused attention-softmax leg (c2)")
    parser.add_argument("--serial-backward", action="store_true",
                        help="time the earlier schedule with its three binning kernels on "
                             "the main stream before the plain forward kernel, so that "
                             "rocprofv3 sees each kernel alone")
    parser.add_argument("--copy-probe-mib", type=int, default=0,
                        help="only run a device-to-device copy of this many MiB, 5 times "
                             "(calibrates the FETCH_SIZE / WRITE_SIZE counters), then exit")
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MSDA path shards over the batch (cameras) with "
              "no exchange, so a multi-GPU figure adds nothing; run with --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n * 4, "launches": 5}))
        return 0

    if args.gather_probe or args.atomic_probe or args.lds_atomic_probe or args.scatter_probe:
        out = {}
        for kind, wanted in (("gather", args.gather_probe), ("atomic", args.atomic_probe)):
            if wanted:
                out.update(run_probe(kind))
        if args.lds_atomic_probe:
            out.update(run_lds_atomic_probe())
        if args.scatter_probe:
            out.update(run_scatter_probe())
        print(json.dumps(out))
        return 0

    from muspace_amd.runtime.native import load_native_module

    lib = load_native_module()
    if args.sca_only:
        print(json.dumps({"sca-scatter-div-float32": time_sca(lib, args.steps, args.warmup)}))
        return 0
    if args.dfa_only:
        print(json.dumps({"sparsedrive-dfa-float32": time_dfa(lib, args.steps, args.warmup)}))
        return 0
    if args.softmax_only:
        print(json.dumps({"c2-softmax-fused-float32": time_softmax(lib, args.steps,
                                                                     args.warmup)}))
        return 0
    dev = torch.device("cuda:0")
    cfg = CONFIGS[args.config]
    vdt = getattr(torch, args.value_dtype)
    vname = {"float32": "float", "bfloat16": "bf16_t", "float16": "__half"}[args.value_dtype]
    print(f"[bench] inputs for {cfg.name} {args.value_dtype}", file=sys.stderr, flush=True)
    step = Step(lib, cfg, vdt, torch.float32, dev,
                binning="serial" if args.serial_backward else "fused")
    print(f"[bench] parity of the timed step ({cfg.name})", file=sys.stderr, flush=True)
    parity = check_step_parity(step, cfg, vdt)
    print(f"[bench] parity: {parity['ok']} {parity['worst_error_over_tolerance']}",
          file=sys.stderr, flush=True)
    torch.cuda.empty_cache()
    res = time_steps(step, args.steps, args.warmup, repeats=args.repeats)
    fwd_b, bwd_b = algorithmic_bytes(cfg, vdt)
    gbps = (fwd_b + bwd_b) / (res["ms_per_step"] * 1e-3) / 1e9
    print(f"[bench] {cfg.name}: {res}", file=sys.stderr, flush=True)
    del step
    torch.cuda.empty_cache()

    extra = {}
    if not args.no_extra_configs:
        for name, vdt in (("c1", torch.float32), ("c3", torch.float32), ("c4", torch.bfloat16),
                          ("c4", torch.float16), ("bevformer-1l", torch.float32)):
            c = CONFIGS[name]
            print(f"[bench] extra {name} {vdt}", file=sys.stderr, flush=True)
            s = Step(lib, c, vdt, torch.float32, dev)
            r = time_steps(s, 50, 10)
            del s
            # the earlier schedule: three binning kernels on a second stream
            s = Step(lib, c, vdt, torch.float32, dev, binning="side")
            r_side = time_steps(s, 50, 10)
            del s
            f, b = algorithmic_bytes(c, vdt)
            extra[f"{name}-{str(vdt).replace('torch.', '')}"] = {
                "fwd_bwd_us": round(r["ms_per_step"] * 1e3, 1),
                "fwd_us": round(r["fwd_ms"] * 1e3, 1),
                "bwd_us": round(r["bwd_ms"] * 1e3, 1),
                "rest_us": round(r["rest_ms"] * 1e3, 1),
                "alloc_us": round(r["zero_ms"] * 1e3, 1),
                "effective_GBps": round((f + b) / (r["ms_per_step"] * 1e-3) / 1e9, 1),
                "side_stream_binning_fwd_bwd_us": round(r_side["ms_per_step"] * 1e3, 1),
                "forward_kernel_stores_records": fused_binning(lib, c, vdt),
            }
            torch.cuda.empty_cache()
        # the earlier schedule at the headline config: binning kernels on a
        # second stream beside the plain forward kernel
        print(f"[bench] extra {cfg.name} side-stream binning", file=sys.stderr, flush=True)
        s = Step(lib, cfg, torch.float32, torch.float32, dev, binning="side")
        r = time_steps(s, 50, 10)
        extra[f"{cfg.name}-float32-side-stream-binning"] = {
            "fwd_bwd_us": round(r["ms_per_step"] * 1e3, 1),
            "fwd_us": round(r["fwd_ms"] * 1e3, 1),
            "bin_us": round(r["bin_ms"] * 1e3, 1),
            "rest_us": round(r["rest_ms"] * 1e3, 1),
        }
        del s
        torch.cuda.empty_cache()
        print("[bench] extra c0 forward", file=sys.stderr, flush=True)
        extra["c0-float32-forward"] = time_forward_only(lib, "c0")
        torch.cuda.empty_cache()
        # the forward alone (no gradient graph: no binning), beside the main
        # step's forward call, which also bins the samples for the backward
        print("[bench] extra c2 forward only", file=sys.stderr, flush=True)
        extra["c2-float32-forward-only"] = time_forward_only(lib, "c2")
        torch.cuda.empty_cache()
        for dtype in (torch.float32, torch.bfloat16):
            label = str(dtype).replace("torch.", "")
            print(f"[bench] extra published bevformer-1l {label}", file=sys.stderr, flush=True)
            extra[f"bevformer-1l-published-case-{label}"] = time_published_case(lib, dtype)
            torch.cuda.empty_cache()
        print("[bench] extra sca-scatter-div", file=sys.stderr, flush=True)
        extra["sca-scatter-div-float32"] = time_sca(lib)
        torch.cuda.empty_cache()
        print("[bench] extra sparsedrive-dfa", file=sys.stderr, flush=True)
        extra["sparsedrive-dfa-float32"] = time_dfa(lib)
        torch.cuda.empty_cache()
        print("[bench] extra c2-softmax-fused", file=sys.stderr, flush=True)
        extra["c2-softmax-fused-float32"] = time_softmax(lib)
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline()
        if "c0-float32-forward" in extra:
            extra["c0-float32-forward"]["cpu_fwd_us"] = round(cpu["rows"]["c0"]["ms"] * 1e3, 1)

    rest_b = backward_rest_bytes(cfg, vdt)
    # the stored traffic summary is the c2 float32 step's
    headline = cfg.name == "c2" and vdt == torch.float32
    rest_achieved = rest_b / (res["rest_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "timing": {"repeats": len(res["repeat_ms_per_step"]), "statistic": "median of repeats",
                   "repeat_ms_per_step": res["repeat_ms_per_step"],
                   "repeat_rest_ms": res["repeat_rest_ms"],
                   "mean_ms_per_step": round(res["mean_ms_per_step"], 4)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float32": "f32", "bfloat16": "bf16", "float16": "f16"}[args.value_dtype],
        "data": "synthetic (seed 2333; value, grad ~ N(0,1), locations ~ U(0,1), softmax weights)",
        "config": {
            "workload": f"{cfg.name}: {cfg.description}, MSDA fwd+bwd, {args.value_dtype} "
                        f"value, batch {cfg.batch}, "
                        f"nq {cfg.queries}, heads {cfg.heads}, head_dim {cfg.channels}, "
                        f"levels {list(cfg.levels)}, points {cfg.points}",
            "us_per_call": round(res["ms_per_step"] * 1e3, 1),
            "fwd_us": round(res["fwd_ms"] * 1e3, 1),
            "bwd_us": round(res["bwd_ms"] * 1e3, 1),
            "bin_us": round(res["bin_ms"] * 1e3, 1),
            "rest_us": round(res["rest_ms"] * 1e3, 1),
            "alloc_us": round(res["zero_ms"] * 1e3, 1),
            "forward_kernel_stores_records": fused_binning(lib, cfg, vdt),
            "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "algorithmic_bytes": {"fwd": fwd_b, "bwd": bwd_b},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"msda_tile_backward<{vname},32> (ms_deform_attn_backward_rest: "
                      f"{rest_b:,} algorithmic bytes = value, grad_output, grad_value, "
                      "grad_sampling_locations, grad_attention_weights once)",
            "achieved": round(rest_achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(rest_achieved / HBM_PEAK_GBPS, 4),
            "traffic": read_traffic() if headline else None,
            "traffic_source": str(TRAFFIC_FILE.relative_to(ROOT)) if headline else None,
        },
        "parity": parity,
        "cpu_baseline": cpu,
        "other_configs": extra,
    }
    print(json.dumps(line, ensure_ascii=False), flush=True)
    if not parity["ok"]:
        print("[bench] the timed step's results do not match the oracle", file=sys.stderr,
              flush=True)
        return 1
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
