"""Benchmark of the event-sparse path on one MI355X.

One step = one fwd+bwd pass of the whole path over the config's synthetic
batch, inputs resident in HBM:
  forward : extract (count -> fill, the fill deriving the row offsets
            from the count pass's block sums, with x_conv gathered at the
            events and the event index built in the same pass; the host
            reads E while fill runs) -> flat selective scan ->
            zero-order-hold restore
  backward: restore backward -> selective scan backward with the gather
            backward (du at the events, dense dx rows) in the same kernel
All stages run in libbcm_event_scan.so on torch's current stream. Prints one
JSON line (metric / value / roofline / cpu_baseline ...).

Timing: `value` and `ms_per_step` come from the K timed steps, each run cold
(L2 and the MALL flushed by reading 512 MiB first) with HIP events around
the step, as their median; `warm_ms_per_step` is K back-to-back steps with
inputs resident; `api_ms_per_step` times the drop-in Python API (autograd
Functions over the same library) warm.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--cfg 1] [--no-cpu] [--no-api]
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd events/s & achieved HBM GB/s, B32 D256 L2048 N16 at 15% density"
HBM_PEAK_GBS = 8000.0
PROBE_STEPS = 5
CAL_BYTES = 256 << 20  # device-to-device copy that calibrates the PMC byte counters
FLUSH_BYTES = 512 << 20  # read before each timed step: more than the 8 L2s plus the 256 MB MALL

# device kernels behind each stage of FusedStep.KERNELS (symbol substrings)
STAGE_KERNELS = {"count": ["k_count"], "fill": ["k_fill"],
                 "scan_fwd": ["k_scan_fwd"], "restore_fwd": ["k_restore_fwd"],
                 "restore_bwd": ["k_restore_bwd_tiles", "k_restore_bwd_fix", "k_restore_bwd_chain"],
                 "scan_bwd": ["k_scan_bwd", "k_scan_param_reduce", "k_gather_bwd_rows"]}


def algorithmic_bytes(B, D, L, N, E, max_seqlen, s_m, s_u, s_o, expand=1):
    """Compulsory traffic of the path's API contract, each tensor once
    (x_conv read and dx written dense), as the reference's interface moves
    it: extract emits ch, t and k (the indexed path here writes k only and
    reads a 3 MB event index instead of t in restore and gather, so its own
    traffic is below these figures)."""
    M = B * D * L
    NC = B * D
    n_ch = max(1, -(-max_seqlen // 2048))
    st = NC * n_ch * N * 8
    return {
        "fwd_extract_gather": M // expand * s_m + M * s_u + 3 * E * 4 + E * s_u + 4 * (NC + 1),
        "fwd_scan": E * s_u + E * 4 + E * s_u + st,
        "fwd_restore": E * s_u + E * 4 + M * s_o,
        "bwd_restore": M * s_o + E * 4 + E * 4,
        "bwd_scan": E * s_u + E * 4 + E * s_u + st + E * s_u,
        "bwd_gather": E * s_u + 2 * E * 4 + M * s_u,
    }


def own_bytes(B, D, L, N, E, max_seqlen, s_m, s_u, s_o, dy_direct=False, du_stream=True):
    """Compulsory traffic of this build's own kernel interfaces for the same
    step (each tensor once): the fill writes k and u but no ch / t streams;
    restore and the gather backward read the event index (a bitmask of one
    bit per step and a tile table of one int32 per 64 steps) instead of t
    and ch; dy is written in u's dtype by the one-kernel restore backward
    (dy_direct), else as fp32 and, for 16-bit u, copied once to u's dtype
    for the scan backward; the scan backward stores du only with du_stream
    (else dx's rows are its only copy). The reference interface's figure
    (algorithmic_bytes) is the metric's numerator; this one says how close
    the kernels run to their own floor."""
    M, NC = B * D * L, B * D
    n_ch = max(1, -(-max_seqlen // 2048))
    st = NC * n_ch * N * 8
    index = M // 8 + NC * (-(-L // 64) + 1) * 4  # bitmask + tile table
    dy_w = E * s_u if dy_direct else E * 4
    dy_copy = 0 if (s_u == 4 or dy_direct) else E * 4 + E * s_u
    return {
        "count": M * s_m + M // 8 + NC * 4,
        "fill": M // 8 + NC * 4 + M * s_u + E * 4 + E * s_u + index - M // 8 + 4 * (NC + 1),
        "scan_fwd": E * s_u + E * 4 + E * s_u + st,
        "restore_fwd": E * s_u + index + M * s_o,
        "restore_bwd": M * s_o + index + dy_w,
        "scan_bwd": (E * s_u + E * 4 + E * s_u + st + (E * s_u if du_stream else 0) + index + M * s_u
                     + dy_copy),
    }


def calibration_copy(dev):
    """One plain device copy of CAL_BYTES (hipMemcpyAsync's blit kernel)."""
    import torch
    a = torch.empty(CAL_BYTES, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)


def measure_traffic(cfg, stage):
    """HBM bytes per launch of `stage` from two rocprofv3 --pmc child runs
    (FETCH_SIZE, then WRITE_SIZE). Each counter is scaled by what it reads
    for the CAL_BYTES copy in the same child, so the result is in bytes
    whatever the counter's unit. Returns (bytes or None, detail dict)."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, {"skipped": "rocprofv3 not found"}
    if any(k.startswith("ROCPROF") for k in os.environ) or "rocprof" in os.environ.get("LD_PRELOAD", ""):
        # already running under a profiler: its preloaded library has the GPU
        # open, and a nested profiler would re-exec from this process
        return None, {"skipped": "running under a profiler"}
    names = STAGE_KERNELS[stage]
    detail = {"kernels": names, "calibration_bytes": CAL_BYTES}
    total = 0.0
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory(prefix="bcm_pmc_") as d:
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "--", sys.executable,
                   os.path.abspath(__file__), "--pmc-child", "--cfg", str(cfg)]
            try:
                r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=180)
            except subprocess.TimeoutExpired:
                return None, dict(detail, skipped=f"{counter} pass timed out")
            rows = []
            for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
                rows += list(csv.DictReader(open(f)))
            if r.returncode != 0 and not rows:
                return None, dict(detail, skipped=f"{counter} pass failed: {r.stdout.decode()[-300:]}")
        per_disp = {}
        for row in rows:
            if row.get("Counter_Name") != counter:
                continue
            key = (row["Kernel_Name"], row.get("Dispatch_Id", row.get("Correlation_Id", "")))
            per_disp[key] = per_disp.get(key, 0.0) + float(row["Counter_Value"])
        cal = max((v for (k, _), v in per_disp.items() if "copyBuffer" in k), default=0.0)
        if cal <= 0:
            return None, dict(detail, skipped=f"{counter}: calibration copy not found")
        per_launch = 0.0
        for nm in names:
            vals = [v for (k, _), v in per_disp.items() if nm in k]
            if not vals:  # a stage's later kernels run only for some shapes
                if nm == names[0]:
                    return None, dict(detail, skipped=f"{counter}: no dispatch of {nm}")
                continue
            per_launch += sum(vals) / len(vals)
        scale = CAL_BYTES / cal
        detail[counter] = {"raw_per_launch": per_launch, "raw_calibration": cal, "bytes_per_unit": scale}
        total += per_launch * scale
    detail["bytes"] = total
    return total, detail


def cpu_baseline(cfg, batches, reps=3):
    """The torch CPU restatement of the path (oracle/torch_path.py) on a
    bounded sample of the workload: `batches` of the config's B batches."""
    import torch
    from bc_mamba_amd.workloads import CONFIGS, make_workload
    from oracle import torch_path as tp
    # the box's CPU share (OMP_NUM_THREADS there), at most the cores the OS shows
    threads = min(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)), os.cpu_count() or 1)
    torch.set_num_threads(threads)
    w = make_workload(cfg, B=batches)
    args = (w.membrane, w.x_conv.float(), w.dout.float(), w.threshold, w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C,
            w.D_skip)
    tp.path_fwd_bwd(*args)  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        _, _, E = tp.path_fwd_bwd(*args)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": E / med, "unit": "events/s", "cores": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
            "torch_threads": torch.get_num_threads(), "kind": "port",
            "sample": f"config {cfg} with B={batches} of its {CONFIGS[cfg]['B']} batches "
                      f"(E={E} events), torch fp32 restatement (oracle/torch_path.py), median of {reps} "
                      f"fwd+bwd reps, {cpu}", "seconds_per_rep": med}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cfg", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-batches", type=int, default=4)
    ap.add_argument("--no-api", action="store_true", help="skip timing the drop-in Python API path (autograd)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc child runs that measure the dominant kernel's HBM bytes")
    ap.add_argument("--out-proj", choices=["gemm", "mfma", "off"], default="gemm",
                    help="config 4: the blocks' restore -> out_proj op (default gemm; off: restore then linear)")
    ap.add_argument("--restore-bwd", choices=["auto", "chained", "two_pass"], default="auto",
                    help="restore backward form: one kernel with look-back, tile pass + fix-up pass, or the "
                         "first where its tile grid fits one launch")
    ap.add_argument("--du-stream", action="store_true",
                    help="also store the scan backward's du stream (the step's input gradient is dx, whose rows "
                         "the scan backward writes itself; du is the reference's intermediate before its scatter)")
    ap.add_argument("--no-peak", action="store_true",
                    help="config 4: skip the peak-memory steps (fused and reference composition) after timing")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the path shards by batch with no exchange; "
              "multi-GPU runs are not part of it)", file=sys.stderr)
        sys.exit(2)

    import torch
    from bc_mamba_amd import _native
    from bc_mamba_amd.fused_step import FusedStep
    from bc_mamba_amd.workloads import make_workload
    _native.lib()
    dev = torch.device("cuda:0")
    if args.cfg == 4:
        print(json.dumps(model_step_bench(args, dev)), flush=True)
        return
    w = make_workload(args.cfg).to(dev)
    path = FusedStep(w, dev, restore_bwd=args.restore_bwd, keep_du=args.du_stream)

    if args.pmc_child:  # a few steps and the calibration copy, run under rocprofv3 --pmc by the parent
        for _ in range(3):
            path.step()
        calibration_copy(dev)
        torch.cuda.synchronize()
        return

    # untimed warmup (first launches load code objects), then probe steps
    # with events around every kernel pick the dominant kernel
    for _ in range(max(args.warmup, 1)):
        path.step()
    for _ in range(PROBE_STEPS):
        path.step(timed=FusedStep.KERNELS)
    per_kernel = {n: path.kernel_ms(n) for n in FusedStep.KERNELS}
    dominant = max(per_kernel, key=per_kernel.get)
    path.events.clear()

    # timed region: `steps` cold steps (the measurement protocol's headline),
    # each after a 512 MiB read has flushed L2 and the MALL, HIP events
    # around the step alone; value is their median
    cold = cold_steps_ms(path, dev, args.steps)
    ms_per_step = cold["median"]
    # warm figure beside it: back-to-back steps with inputs resident, no
    # events inside (an event record makes the GPU write back its caches,
    # several microseconds of idle device per record), host clock
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        path.step()
    torch.cuda.synchronize()
    warm_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # the dominant kernel's launch duration: HIP events around it, on its
    # stream, over as many steps again right after the timed region
    for _ in range(args.steps):
        path.step(timed=(dominant,))
    torch.cuda.synchronize()
    dom_ms = path.kernel_ms(dominant)

    E, ms = path.E, path.ms
    su = torch.tensor([], dtype=w.dtype).element_size()
    alg = algorithmic_bytes(w.B, w.D, w.L, w.N, E, ms, 4, su, su)
    total_bytes = sum(alg.values())
    own_total = sum(own_bytes(w.B, w.D, w.L, w.N, E, ms, 4, su, su, dy_direct=path.restore_bwd == "chained",
                              du_stream=path.args.du is not None).values())
    # algorithmic bytes of one launch of each kernel (its share of the API-contract traffic)
    kernel_bytes = {"count": w.B * w.D * w.L * 4 + 4 * path.NC,
                    "fill": alg["fwd_extract_gather"] - w.B * w.D * w.L * 4, "scan_fwd": alg["fwd_scan"],
                    "restore_fwd": alg["fwd_restore"], "restore_bwd": alg["bwd_restore"],
                    "scan_bwd": alg["bwd_scan"] + alg["bwd_gather"]}
    dom_gbs = kernel_bytes[dominant] / (dom_ms * 1e-3) / 1e9
    result = {
        # the headline metric is config 1's; the other configs name their own shape
        "metric": METRIC if args.cfg == 1 else
        f"fwd+bwd events/s & achieved HBM GB/s, B{w.B} D{w.D} L{w.L} N{w.N} (config {args.cfg})",
        "value": E / (ms_per_step * 1e-3),
        "unit": "events/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[w.dtype],
        "data": "synthetic",
        "config": {"workload": f"config {args.cfg}: extract+gather -> flat scan -> ZOH restore, fwd+bwd",
                   "B": w.B, "D": w.D, "L": w.L, "N": w.N, "events": E, "density": E / (w.B * w.D * w.L),
                   "max_seqlen": ms},
        "restore_bwd_form": path.restore_bwd,
        # whether the scan backward also stored du (the reference's
        # intermediate before its scatter into dx); dx is written either way
        "du_stream": path.args.du is not None,
        "achieved_gbs": total_bytes / (ms_per_step * 1e-3) / 1e9,
        "algorithmic_bytes": total_bytes,
        # the same time against this build's own compulsory traffic (no ch /
        # t streams, the event index instead): a stricter fraction
        "own_bytes": own_total,
        "path_frac_own_bytes": own_total / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "path_frac_of_hbm_peak": total_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernel_ms": per_kernel,
        # ms_per_step / value: median over the timed steps, each after a
        # 512 MiB read (L2 and the MALL flushed, no dirty lines left), HIP
        # events around the step; warm: back-to-back steps, host clock
        "timing": {"ms_per_step": "median of cold steps (L2 + MALL flushed by a 512 MiB read), HIP events",
                   "reps": len(cold["all"]), "min_ms": min(cold["all"]), "max_ms": max(cold["all"]),
                   "wall_s": cold["wall_s"]},
        "warm_ms_per_step": warm_ms,
        "warm_events_per_s": E / (warm_ms * 1e-3),
        "warm_achieved_gbs": total_bytes / (warm_ms * 1e-3) / 1e9,
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": dom_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom_gbs / HBM_PEAK_GBS, "traffic": None, "launch_ms": dom_ms,
                     "bytes_per_launch": kernel_bytes[dominant]},
    }
    if not args.no_traffic:
        traffic, detail = measure_traffic(args.cfg, dominant)
        result["roofline"]["traffic"] = traffic
        result["roofline"]["traffic_detail"] = detail
    if not args.no_api:
        # the drop-in Python API path (autograd Functions over the same
        # library), warm: what a caller of the reference's interface sees
        result["api_ms_per_step"] = api_path_ms(w, dev, args.steps, args.warmup)
    if args.cfg == 3:
        # the reference encodes config 3's two towers as two B = 32 calls
        # (lra_impl.py:1685-1688): the same inputs as two half-batch steps
        result["towers_2x32"] = towers_bench(w, dev, args)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cfg, args.cpu_batches)
    print(json.dumps(result), flush=True)


class TwoTowers:
    """One step over workload w as two calls of half the batch each (the
    towers of config 3), one FusedStep per half, one after the other on
    the stream."""

    def __init__(self, w, dev, **kw):
        from bc_mamba_amd.fused_step import FusedStep
        from bc_mamba_amd.workloads import Workload
        h = w.B // 2
        self.parts = []
        for sl in (slice(0, h), slice(h, w.B)):
            f = {k: getattr(w, k) for k in w.__dataclass_fields__}
            f["B"] = sl.stop - sl.start
            for k in ("membrane", "x_conv", "dout"):
                f[k] = getattr(w, k)[sl].contiguous()
            self.parts.append(FusedStep(Workload(**f), dev, **kw))

    def step(self):
        for p in self.parts:
            p.step()

    @property
    def E(self):
        return sum(p.E for p in self.parts)


def towers_bench(w, dev, args):
    """Cold and warm step time of the two-call encoding (same protocol as
    the headline figure)."""
    import torch
    two = TwoTowers(w, dev, restore_bwd=args.restore_bwd, keep_du=args.du_stream)
    for _ in range(args.warmup):
        two.step()
    cold = cold_steps_ms(two, dev, args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        two.step()
    torch.cuda.synchronize()
    warm_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    E = two.E
    return {"calls": [p.w.B for p in two.parts], "events": E, "ms_per_step": cold["median"],
            "events_per_s": E / (cold["median"] * 1e-3), "warm_ms_per_step": warm_ms,
            "restore_bwd_form": [p.restore_bwd for p in two.parts]}


def model_step_bench(args, dev):
    """Config 4: one training step (forward, cross-entropy loss, backward) of
    the 6-layer model, B=50 L=1024, random init and byte tokens. events/s
    counts the events every layer's extraction routes (its input spikes,
    times expand) per step."""
    import torch
    from bc_mamba_amd.workloads import make_model_workload
    model, tokens, labels = make_model_workload(device=dev)
    mode = {"gemm": True, "mfma": "mfma", "off": False}[args.out_proj]
    for blk in model.blocks:
        blk.core.fused_out_proj = mode
    events = []
    hooks = [blk.core.register_forward_pre_hook(
        lambda mod, inp: events.append(int((inp[0] > mod.threshold).sum()) * mod.expand)) for blk in model.blocks]

    def step():
        loss = torch.nn.functional.cross_entropy(model(tokens), labels)
        loss.backward()
        for p in model.parameters():
            p.grad = None

    step()
    for h in hooks:
        h.remove()
    per_layer = list(events)
    E = sum(per_layer)
    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    peak = None if args.no_peak else peak_memory(model, step)
    return {
        "metric": "training-step events/s (config 4 model)", "value": E / (ms * 1e-3), "unit": "events/s",
        "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config 4: 6-layer model training step (fwd + CE loss + bwd), d_model 256, "
                               "d_inner 512, N 16, L 1024, B 50, byte tokens, random init",
                   "out_proj": args.out_proj, "events_per_step": E, "events_per_layer": per_layer,
                   "density_per_layer": [e / (50 * 1024 * 512) for e in per_layer]},
        "peak_memory_bytes": peak,
        "roofline": None,
    }


def peak_memory(model, step):
    """torch.cuda.max_memory_allocated over one training step: the fused
    event path (default) and the reference composition (every block with
    fused_event_path=False and the plain STE sampler), same model, inputs
    and parameters. Model state (parameters, and gradients, which step()
    frees) is included in both."""
    import torch
    from bc_mamba_amd.e_model import SpikeSamplerSurrogate
    samplers = [m for m in model.modules() if isinstance(m, SpikeSamplerSurrogate)]
    res = {}
    for name, fused in (("fused", True), ("reference_composition", False)):
        for blk in model.blocks:
            blk.core.fused_event_path = fused
        for sm in samplers:
            sm.fused_bits = fused
        step()  # warm the allocator for this path
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        step()
        torch.cuda.synchronize()
        res[name] = int(torch.cuda.max_memory_allocated())
    for blk in model.blocks:
        blk.core.fused_event_path = True
    for sm in samplers:
        sm.fused_bits = True
    return res


def cold_steps_ms(path, dev, reps):
    """`reps` steps, each after reading a 512 MiB buffer (more than the
    eight L2s and the 256 MB MALL together: the step's inputs are evicted,
    and a read leaves no dirty lines whose write-back the step would pay
    for), HIP events around the step only. Returns the median, every rep
    and the wall time of the whole region (flushes included)."""
    import torch
    scratch = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
    sink = torch.empty((), dtype=torch.float32, device=dev)
    evs = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        torch.sum(scratch, dim=0, out=sink)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        path.step()
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    times = [a.elapsed_time(b) for a, b in evs]
    del scratch
    return {"median": sorted(times)[len(times) // 2], "all": times, "wall_s": wall}


def api_path_ms(w, dev, steps, warmup):
    """ms per fwd+bwd through the drop-in Python modules with autograd."""
    import torch
    from bc_mamba_amd import e_model
    from bc_mamba_amd import extract_events_cuda as ee
    from bc_mamba_amd.selective_scan_interface import selective_scan_flat_ch_fn
    params = [p.detach().requires_grad_(True) for p in (w.dt_idle, w.dt_active, w.A, w.W_B, w.W_C, w.D_skip)]
    x_conv = w.x_conv.detach().requires_grad_(True)

    def one():
        # a training step's zero_grad(set_to_none=True): the backward writes
        # fresh gradients instead of adding into the last step's
        x_conv.grad = None
        for p in params:
            p.grad = None
        ch, t, k, cu, counts, ms = ee.extract_base_events(w.membrane, w.threshold)
        u = e_model.GatherEventsFn.apply(x_conv, ch, t)
        y, _ = selective_scan_flat_ch_fn(u, k, cu, int(ms), *params[:5], D=params[5], is_depthwise_bc=True)
        e_model.restore_dense_fn(y, t, cu, w.D, w.L).backward(w.dout)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


if __name__ == "__main__":
    main()
