"""Benchmark of the MI355X optimizer step (BASELINE config 2 on one GPU).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one optimizer step over the 5B-preset SwiGLU stage window
(W_gate, W_up [6144, 3072] and W_down [3072, 6144]; N = 56,623,104 FP32
masters, held with their moments and export copy in one arena): the
non-finite detector over the FP16 gradients, whose launch also closes the
previous step (skip decision, loss scale, clocks), then the fused unscale +
AdamW + FP16 export kernel -- all on the device, with no host round trip
between steps.  Inputs are synthetic (seeded), resident in HBM before the
timed region.  Other workloads: embedding (config 3), overflow (config 4),
muon (config 5), grads, window, disk, fp8, export, streamed, streamed_muon.

Prints one JSON line.  `value` is whole-step throughput in Gparams/s;
`roofline` is the fused AdamW kernel's algorithmic bandwidth (28 bytes per
parameter) over its average launch time in a sample of the timed steps, from
HIP events that those launches' dispatches stamp on the launch stream;
`cpu_baseline` times torch.optim.AdamW(foreach=False) -- the library the
reference's AdamW group runs -- on this host's cores.
"""
import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
TRAFFIC_PROFILE = ROOT / "profiles" / "adamw_config2_traffic.json"
TRAFFIC_PROFILE_C3 = ROOT / "profiles" / "adamw_config3_traffic.json"
MFMA_PROFILE = ROOT / "profiles" / "muon_config5_mfma.json"
TRAFFIC_PROFILE_MUON = ROOT / "profiles" / "muon_config5_traffic.json"
TRAFFIC_PROFILE_GRADS = ROOT / "profiles" / "grads_config2_traffic.json"
TRAFFIC_PROFILE_WINDOW = ROOT / "profiles" / "window_config2_traffic.json"
# rocprofv3 counters cannot run inside this process: `traffic` is read from the committed
# summary of the FETCH_SIZE / WRITE_SIZE passes over this same workload, not measured here
TRAFFIC_SOURCE = "profiles/%s: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes of this workload (committed, not this run)"
HBM_PEAK_GBS = 8000.0
BYTES_PER_PARAM = 28  # read g16 2 + w 4 + m 4 + v 4; write w 4 + m 4 + v 4 + export 2
CONFIG2_SHAPES = [(6144, 3072), (6144, 3072), (3072, 6144)]  # W_gate, W_up, W_down (nn.Linear storage)
LOSS_SCALE = 65536.0
HYPER = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
CONFIG5_LAYERS = 14        # 5B preset: 14 SwiGLU blocks -> 42 hidden matrices
CONFIG5_ADAM_VECTORS = 326  # x 3072 = 1,001,472 norm/bias parameters


# ------------------------------------------------------------ workloads --
def config2_window(device, seed=0):
    """FP32 masters N(0, .02) for the three SwiGLU matrices of one stage."""
    gen = torch.Generator(device=device).manual_seed(seed)
    return [torch.randn(s, generator=gen, device=device) * 0.02 for s in CONFIG2_SHAPES]


def config2_grads(device, step_seed, shapes=CONFIG2_SHAPES, scale=LOSS_SCALE):
    """FP16 gradients: fp16(N(0, 1e-4) * 2^16), one seeded draw per step."""
    gen = torch.Generator(device=device).manual_seed(step_seed)
    return [(torch.randn(s, generator=gen, device=device) * 1e-4 * scale).half() for s in shapes]


def config3_embedding_grad(step_seed, rows=65536, cols=3072, tokens=4 * 1024, s=1.1,
                           device="cpu"):
    """BF16 tied-embedding gradient: N(0, 1e-3) on Zipf(1.1)-sampled rows, zero elsewhere."""
    gen = torch.Generator().manual_seed(step_seed)
    ranks = torch.arange(1, rows + 1, dtype=torch.float64)
    probs = ranks.pow(-s)
    ids = torch.multinomial(probs / probs.sum(), tokens, replacement=True, generator=gen)
    active = torch.unique(ids)
    g = torch.zeros(rows, cols, dtype=torch.bfloat16)
    g[active] = (torch.randn(active.numel(), cols, generator=gen) * 1e-3).to(torch.bfloat16)
    return g.to(device), active


class Config5(torch.nn.Module):
    """42 hidden Linear weights (Muon) + ~1M norm/bias params (AdamW).

    Per SwiGLU block W_gate, W_up [6144, 3072] and W_down [3072, 6144] in nn.Linear
    storage, so after optimizer.py:15-17's transpose rule every Newton-Schulz
    operand is [3072, 6144].  Weights N(0, .02); norms/biases ones.
    """

    def __init__(self, device):
        super().__init__()
        mk = lambda o, i: torch.nn.Linear(i, o, bias=False, device=device)
        self.blocks = torch.nn.ModuleList(
            torch.nn.ModuleDict(dict(gate=mk(6144, 3072), up=mk(6144, 3072), down=mk(3072, 6144)))
            for _ in range(CONFIG5_LAYERS))
        self.vectors = torch.nn.ParameterList(
            torch.nn.Parameter(torch.ones(3072, device=device)) for _ in range(CONFIG5_ADAM_VECTORS))
        gen = torch.Generator(device=device).manual_seed(5)
        with torch.no_grad():
            for block in self.blocks:
                for lin in block.values():
                    lin.weight.copy_(torch.randn(lin.weight.shape, generator=gen, device=device) * .02)


def host_cpus():
    """Cores for the CPU baselines: every core in this process's affinity mask
    (len(os.sched_getaffinity(0))), bounded by a cgroup CPU quota when the container
    sets one (/sys/fs/cgroup/cpu.max) -- threads beyond the quota only time-slice.
    Sets torch's intra-op thread count and returns the figures the line reports."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        limit, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if limit != "max":
            quota = int(limit) / int(period)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    torch.set_num_threads(threads)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return dict(threads=threads, affinity=affinity, quota=quota, model=model)


def cpu_fields(info):
    """The baseline's core figures: threads used, affinity mask size, cgroup quota, CPU model."""
    return dict(cores=info["threads"], affinity_cores=info["affinity"],
                cgroup_cpu_quota=info["quota"], cpu_model=info["model"])


# --------------------------------------------------------------- timing --
GRAD_SETS = 3  # gradient sets cycled over the steps: 3 x 113 MB exceeds the 256 MB Infinity Cache
STAMP_EVERY = 4  # every 4th AdamW launch of the timed steps stamps its own start/stop events


def time_gpu(steps, warmup):
    """Steps are enqueued back to back (device-resident skip/scale/clock control).

    Each step takes the next of GRAD_SETS gradient sets, so no step finds its
    gradients left in the Infinity Cache by an earlier one (one reused buffer
    would flatter the step without a detector pass by about 10 us).  The AdamW
    launch of every STAMP_EVERY-th timed step (the last of each group) is timed by
    HIP events that its own dispatch stamps (hipExtLaunchKernel's start/stop
    events on the launch stream).  Timing events cost a step about 5 us (255.5
    vs 260.7 us on one box), so only a sample of the timed steps carries them;
    K more steps without any follow (`step_uninstrumented`), then K steps with
    checked=True, the step without the detector pass.
    """
    from morph_amd import DynamicLossScale, FusedAdamW
    from morph_amd.kernels import DispatchTimer

    device = torch.device("cuda", 0)
    masters = config2_window(device)
    sets = [config2_grads(device, 1000 + k) for k in range(GRAD_SETS)]
    n = sum(p.numel() for p in masters)
    scaler = DynamicLossScale(LOSS_SCALE, growth_interval=2000)
    opt = FusedAdamW(masters, **HYPER, loss_scale=scaler, export_dtype=torch.float16, arena=True)
    for t in range(max(warmup, GRAD_SETS)):
        opt.step(sets[t % GRAD_SETS])
    opt.resolve()
    # the sampled steps are the last of each group of STAMP_EVERY (every step when
    # fewer are timed): none is the first step after the idle synchronize
    stamped = {t for t in range(steps) if steps < STAMP_EVERY or t % STAMP_EVERY == STAMP_EVERY - 1}
    timer = DispatchTimer(len(stamped), device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(steps):
        opt.dispatch_timer = timer if t in stamped else None
        opt.step(sets[t % GRAD_SETS])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    opt.dispatch_timer = None
    kernel_ms = timer.elapsed_ms()
    t0 = time.perf_counter()
    for t in range(steps):
        opt.step(sets[t % GRAD_SETS])
    torch.cuda.synchronize()
    elapsed_plain = time.perf_counter() - t0
    # The same step when the gradients' producer has already set the step's
    # non-finite flag (StageGradients.accumulate(..., final=True,
    # found_inf=opt.found_inf)): fused AdamW + step close, no detector pass.
    t0 = time.perf_counter()
    for t in range(steps):
        opt.step(sets[t % GRAD_SETS], checked=True)
    torch.cuda.synchronize()
    elapsed_checked = time.perf_counter() - t0
    opt.resolve()
    if opt.skipped_steps:
        raise RuntimeError(f"{opt.skipped_steps} steps skipped on synthetic finite gradients")
    return dict(n=n, elapsed=elapsed, elapsed_plain=elapsed_plain, elapsed_checked=elapsed_checked,
                avg_kernel_s=sum(kernel_ms) / len(kernel_ms) / 1e3, kernel_ms=kernel_ms,
                scale=scaler.scale, applied=opt.applied_steps,
                copy=copy_ceiling(BYTES_PER_PARAM * n, device))


def copy_ceiling(nbytes, device, reps=10):
    """The HBM rate of a plain FP32 copy moving the bytes of one AdamW launch (half
    read, half written): the library's streaming copy (morph_convert_f32 with FP32
    output), timed by events on its stream after the timed steps, median of `reps`
    launches."""
    from morph_amd import _lib
    n = nbytes // 8
    src = torch.ones(n, device=device)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream(device)
    times = []
    for r in range(reps + 2):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        _lib.check(_lib.lib().morph_convert_f32(
            ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), _lib.DTYPE_F32, n,
            None, _lib.stream_handle(stream)))
        e1.record(stream)
        torch.cuda.synchronize(device)
        if r >= 2:  # the first launches warm the code object and the buffers
            times.append(e0.elapsed_time(e1))
    med = sorted(times)[len(times) // 2]
    gbs = 8 * n / med / 1e6
    return {"achieved": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "copy_kernel (morph_convert_f32 with FP32 output: 64 lanes, one "
                      "non-temporal 16-byte load and store each)",
            "bytes_per_launch": 8 * n, "median_launch_us": round(med * 1e3, 2), "launches": reps}


def cpu_baseline(seconds=10.0):
    """torch.optim.AdamW(foreach=False) on config 2's masters, on this host's cores.

    The oracle's restatement of the reference CPU path: gradients unscaled from
    FP16 (g.float() / scale, streamtrain/disk.py:447) then the library AdamW the
    reference's HybridMuonAdamW runs (streamtrain/optimizer.py:40).  Runs whole
    steps until `seconds` have passed (at least 2) and reports the median.
    """
    from oracle import reference as R
    cpus = host_cpus()
    masters = config2_window("cpu")
    grads16 = config2_grads("cpu", 1000)
    params = [torch.nn.Parameter(m) for m in masters]
    opt = torch.optim.AdamW(params, **HYPER, foreach=False)
    times = []
    start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - start < seconds and len(times) < 20):
        t0 = time.perf_counter()
        for p, g in zip(params, grads16):
            p.grad = g.float() / LOSS_SCALE
        opt.step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    n = sum(p.numel() for p in params)
    cpu = cpus["model"]
    return dict(value=round(n / med / 1e9, 4), unit="Gparams/s", **cpu_fields(cpus), kind="port",
                gbs_28b_equivalent=round(BYTES_PER_PARAM * n / med / 1e9, 2),
                sample=f"config 2 window (N={n}), {len(times)} whole steps, median; "
                       f"torch.optim.AdamW(foreach=False) after FP16 unscale; CPU: {cpu}",
                disk_ops=cpu_baseline_disk(masters, grads16, seconds / 2))


def cpu_baseline_disk(masters, grads16, seconds):
    """The second CPU form: DiskState.update's chunked op sequence (streamtrain/disk.py:207-216,
    1,048,576-element chunks, torch CPU ops, stacked write-back) on the config-2 window's three
    [3, N] states held in RAM (no file I/O, no fsync), gradients unscaled from FP16."""
    import numpy as np
    from oracle import reference as R
    states = [np.stack([m.numpy().reshape(-1), np.zeros(m.numel(), np.float32),
                        np.zeros(m.numel(), np.float32)]) for m in masters]
    grads = [(g.float() / LOSS_SCALE).reshape(-1) for g in grads16]
    times = []
    start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - start < seconds and len(times) < 20):
        t0 = time.perf_counter()
        for st, g in zip(states, grads):
            R.disk_update_torch(st, g, len(times) + 1, HYPER["lr"], 1.0)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    n = sum(m.numel() for m in masters)
    return dict(value=round(n / med / 1e9, 4), unit="Gparams/s",
                sample=f"config 2 window, {len(times)} whole steps, median; DiskState.update's "
                       "chunked torch op sequence on [3, N] states in RAM")


def time_muon(steps, warmup):
    """Config 5 through HybridMuonAdamW: gate, batched Muon (bf16 MFMA NS), AdamW group."""
    from morph_amd.muon import HybridMuonAdamW, ns_flops
    device = torch.device("cuda", 0)
    model = Config5(device)
    gen = torch.Generator(device=device).manual_seed(6)
    for p in model.parameters():
        p.grad = torch.randn(p.shape, generator=gen, device=device) * 1e-3
    opt = HybridMuonAdamW(model, lr=3e-4, muon_lr=0.02)
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    opt.ns_timer = []
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ns_s = sum(a.elapsed_time(b) for a, b, _, _ in opt.ns_timer) / 1e3 / steps
    flops = sum(f for _, _, f, _ in opt.ns_timer) / steps
    executed = sum(x for _, _, _, x in opt.ns_timer) / steps
    n_muon = sum(p.numel() for p in opt.muon)
    n_adam = sum(p.numel() for g in opt.adam.param_groups for p in g["params"])
    return dict(elapsed=elapsed, ns_s=ns_s, flops=flops, executed=executed, n_muon=n_muon,
                n_adam=n_adam, expected_flops=ns_flops(3072, 6144, 42))


def cpu_baseline_muon():
    """The reference's FP32 Muon update (optimizer.py:55-61, torch CPU) on one [6144, 3072]
    matrix of the 42, scaled by 42 to a whole step (the 1M AdamW group is negligible)."""
    from oracle import reference as R
    cpus = host_cpus()
    gen = torch.Generator().manual_seed(7)
    p = torch.randn(6144, 3072, generator=gen) * .02
    g = torch.randn(6144, 3072, generator=gen) * 1e-3
    m = torch.zeros_like(p)
    R.muon_reference_step(p, g, m, .02, .01)  # warm-up
    t0 = time.perf_counter()
    R.muon_reference_step(p, g, m, .02, .01)
    one = time.perf_counter() - t0
    return dict(value=round(42 * one * 1e3, 1), unit="ms/step", **cpu_fields(cpus), kind="port",
                sample=f"one [6144, 3072] Muon matrix (FP32 NS, torch CPU) = {one * 1e3:.1f} ms, "
                       "x42 for the step")


def muon_main(args):
    r = time_muon(args.steps, args.warmup)
    ms = r["elapsed"] / args.steps * 1e3
    achieved = r["executed"] / r["ns_s"] / 1e12  # FLOP the MFMAs execute
    dense = r["flops"] / r["ns_s"] / 1e12       # the dense count (symmetric halves included)
    line = {
        "metric": "Hybrid Muon step, 42 x [3072, 6144] NS bf16 + 1M AdamW, 1 MI355X",
        "value": round(ms, 3), "unit": "ms/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "config 5: 14 x (W_gate, W_up [6144,3072], W_down [3072,6144]) "
                               "Muon (5 NS iterations, bf16 MFMA, lr .02, momentum .95) + "
                               f"{r['n_adam']} AdamW params", "muon_params": r["n_muon"]},
        "ns_ms_per_step": round(r["ns_s"] * 1e3, 3),
        "ns_includes": "the FP32 master update, which the last X' = B' X launch applies in its "
                       "epilogue (morph_muon_newton_schulz_finish); no separate finish pass",
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(TRAFFIC_PROFILE_MUON),
                     "traffic_source": TRAFFIC_SOURCE % TRAFFIC_PROFILE_MUON.name
                     + "; the mean over the three products' launches",
                     "kernel": "gemm_kernel / gemm_apply_kernel (3 launches per Newton-Schulz "
                               "iteration, all 42 matrices batched; the last carries the update)",
                     "flops_per_step": r["executed"],
                     "flops_counted": "executed by the MFMAs: the symmetric products A and B' "
                                      "compute 78 of 144 tiles per matrix",
                     "dense_equivalent_tflops": round(dense, 1),
                     "dense_flops_per_step": r["flops"]},
        "mfma_counters": measured_mfma(),
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_muon(),
    }
    assert r["flops"] == r["expected_flops"]
    print(json.dumps(line), flush=True)


GRADS_MICRO = 4            # micro-batches per stage window in the grads workload
ACCUM_BYTES = 10           # plain pass: read g16 2 + read FP32 window 4 + write 4


def time_grads(steps, warmup):
    """Stage-gradient window (f1): 4 micro-batches of FP16 gradients x 2^16 into the FP32
    config-2 window -- overwrite, 2 plain passes, final pass with flag + FP64 norm."""
    from morph_amd.grads import StageGradients
    device = torch.device("cuda", 0)
    micro = [config2_grads(device, 2000 + k) for k in range(GRADS_MICRO)]
    window = StageGradients(CONFIG2_SHAPES, device)
    n = window.flat.numel()
    stream = torch.cuda.current_stream()

    def one_step(timer=None):
        window.zero_()
        for k, grads in enumerate(micro):
            if timer is not None and 0 < k < GRADS_MICRO - 1:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                window.accumulate(grads, LOSS_SCALE)
                b.record(stream)
                timer.append((a, b))
            else:
                window.accumulate(grads, LOSS_SCALE, final=(k == GRADS_MICRO - 1))

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    timer = []
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step(timer)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    if window.found_inf():
        raise RuntimeError("synthetic finite gradients flagged")
    ms = [a.elapsed_time(b) for a, b in timer]
    return dict(n=n, elapsed=elapsed, avg_pass_s=sum(ms) / len(ms) / 1e3,
                norm_squared=window.norm_squared())


def cpu_baseline_grads():
    """The reference's torch ops on the host (sparse_disk.py:106-107, disk.py:466-468): one
    plain micro-batch pass over the config-2 window plus the chunked FP64 norm pass."""
    from oracle import reference as R
    cpus = host_cpus()
    grads = config2_grads("cpu", 2000)
    window = [torch.zeros(s) for s in CONFIG2_SHAPES]
    n = sum(w.numel() for w in window)
    for d, g in zip(window, grads):  # warm-up (first touch)
        R.accumulate_torch(d, g, LOSS_SCALE)
    t0 = time.perf_counter()
    for d, g in zip(window, grads):
        R.accumulate_torch(d, g, LOSS_SCALE)
    t_acc = time.perf_counter() - t0
    t0 = time.perf_counter()
    R.norm_squared_torch(window)
    t_norm = time.perf_counter() - t0
    return dict(value=round(n / t_acc / 1e9, 4), unit="Gparams/s per micro-batch pass",
                **cpu_fields(cpus), kind="port",
                sample=f"config 2 window (N={n}): one add_(g.float()/scale) pass {t_acc * 1e3:.1f} ms; "
                       f"the FP64 chunked norm pass {t_norm * 1e3:.1f} ms")


def grads_main(args):
    r = time_grads(args.steps, args.warmup)
    n = r["n"]
    ms = r["elapsed"] / args.steps * 1e3
    achieved = ACCUM_BYTES * n / r["avg_pass_s"] / 1e9
    line = {
        "metric": "Stage-gradient accumulate Gparams/s per micro-batch pass, 5B SwiGLU window, 1 MI355X",
        "value": round(n * GRADS_MICRO * args.steps / r["elapsed"] / 1e9, 3),
        "unit": "Gparams/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"config 2 window, {GRADS_MICRO} micro-batches of FP16 gradients x "
                               "2^16: overwrite, plain, plain, final (flag + FP64 norm partials)",
                   "params": n, "shapes": CONFIG2_SHAPES, "grad_dtype": "f16",
                   "loss_scale": LOSS_SCALE},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(TRAFFIC_PROFILE_GRADS),
                     "traffic_source": TRAFFIC_SOURCE % TRAFFIC_PROFILE_GRADS.name,
                     "kernel": "accumulate_kernel<F16,false,false> (plain pass)",
                     "avg_launch_us": round(r["avg_pass_s"] * 1e6, 2),
                     "bytes_per_launch": ACCUM_BYTES * n},
        "norm_squared": r["norm_squared"],
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_grads(),
    }
    print(json.dumps(line), flush=True)


WINDOW_BYTES = 30  # fused update on the resident window: read g32 4 + w,m,v 12; write 12 + f16 copy 2


class _FileStore:
    """[3, N] float32 state files of the reference's DiskState (disk.py:45-70) in a temp dir."""

    def __init__(self, root, names_shapes, seed=0):
        import numpy as np
        self.root = Path(root)
        self.entries = {}
        gen = torch.Generator().manual_seed(seed)
        for i, (name, shape) in enumerate(names_shapes):
            n = int(torch.Size(shape).numel())
            self.entries[name] = dict(shape=list(shape), size=n, file=f"{i:05}.bin")
            state = np.zeros((3, n), np.float32)
            state[0] = (torch.randn(n, generator=gen) * .02).numpy()
            state.tofile(self.root / f"{i:05}.bin")

    def fault(self, point):
        return None


def time_window(steps, warmup, root):
    """Resident window (f2): load the config-2 window's [3, N] files into HBM + FP16 compute
    copy, then per step DiskState.update for the 3 parameters (fused update on the resident
    state + FP16 copy, D2H write-back chunk by chunk, flush, fsync)."""
    from morph_amd.kernels import DispatchTimer
    from morph_amd.window import ResidentWindow
    device = torch.device("cuda", 0)
    names = ["ffn.gate.weight", "ffn.up.weight", "ffn.down.weight"]
    store = _FileStore(root, list(zip(names, CONFIG2_SHAPES)))
    win = ResidentWindow(store, names, torch.float16)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    win.load()
    torch.cuda.synchronize()
    t_load = time.perf_counter() - t0
    gen = torch.Generator(device=device).manual_seed(5)
    grads = {n: torch.randn(s, generator=gen, device=device) * 1e-4 for n, s in zip(names, CONFIG2_SHAPES)}
    step = 0
    for _ in range(warmup):
        step += 1
        for n in names:
            win.update(n, grads[n], step, 3e-4, 1.0)
    # each update launch stamps its own dispatch's start and end: events recorded
    # around it would also count the GPU waking up after the host's file writes
    timer = win.dispatch_timer = DispatchTimer(steps * len(names), device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step += 1
        for n in names:
            win.update(n, grads[n], step, 3e-4, 1.0)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    win.dispatch_timer = None
    kms = timer.elapsed_ms()
    return dict(n=sum(store.entries[n]["size"] for n in names), t_load=t_load, elapsed=elapsed,
                avg_kernel_s=sum(kms) / len(kms) / 1e3, kernels=len(kms) // steps,
                timing={k: round(v, 4) for k, v in win.timing.items()})


def cpu_baseline_window(root):
    """The reference's DiskState.update (disk.py:203-223: memmap, chunked torch ops, np.stack
    write-back, flush, fsync) on one [6144, 3072] parameter file of the window."""
    import numpy as np
    from oracle import reference as R
    cpus = host_cpus()
    store = _FileStore(root, [("w", CONFIG2_SHAPES[0])], seed=1)
    e = store.entries["w"]
    g = torch.randn(e["size"], generator=torch.Generator().manual_seed(2)) * 1e-4
    path = store.root / e["file"]
    t0 = time.perf_counter()
    mapped = np.memmap(path, dtype=np.float32, mode="r+", shape=(3, e["size"]))
    R.disk_update_torch(mapped, g, 1, 3e-4, 1.0)
    mapped.flush()
    del mapped
    fd = os.open(path, os.O_RDWR)
    os.fsync(fd)
    os.close(fd)
    t = time.perf_counter() - t0
    return dict(value=round(e["size"] / t / 1e9, 4), unit="Gparams/s", **cpu_fields(cpus), kind="port",
                sample=f"DiskState.update of one [6144, 3072] state file ({e['size']} params): "
                       f"{t * 1e3:.0f} ms incl. memmap I/O, flush and fsync")


def window_main(args):
    import shutil
    import tempfile
    root = Path(tempfile.mkdtemp(prefix="morph_window_"))
    try:
        (root / "gpu").mkdir()
        r = time_window(args.steps, args.warmup, root / "gpu")
        n = r["n"]
        achieved = WINDOW_BYTES * n / (r["avg_kernel_s"] * r["kernels"]) / 1e9
        line = {
            "metric": "Resident stage-window DiskState.update Gparams/s (fused update, D2H write-back, fsync), 5B SwiGLU window, 1 MI355X",
            "value": round(n * args.steps / r["elapsed"] / 1e9, 3), "unit": "Gparams/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r["elapsed"] / args.steps * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "config 2 window as three [3, N] float32 state files: load into HBM "
                                   "with FP16 compute copy once, then per step update + write-back "
                                   "of every file (chunks of 1M elements, flush, fsync)",
                       "params": n, "shapes": CONFIG2_SHAPES, "compute_dtype": "f16",
                       "state_dir": "tempfile.mkdtemp() on the GPU box"},
            "load_gparams_per_s": round(n / r["t_load"] / 1e9, 3),
            "load_h2d_gbs": round(12 * n / r["t_load"] / 1e9, 2),
            "write_back_gbs": round(12 * n * args.steps / r["elapsed"] / 1e9, 2),
            "host_seconds": r["timing"],
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic(TRAFFIC_PROFILE_WINDOW),
                         "traffic_source": TRAFFIC_SOURCE % TRAFFIC_PROFILE_WINDOW.name,
                         "kernel": "adamw_multi_kernel<F32,F16,host> (resident [3, N] state)",
                         "avg_launch_us": round(r["avg_kernel_s"] * 1e6, 2),
                         "bytes_per_launch": WINDOW_BYTES * n // r["kernels"]},
        }
        if not args.no_cpu_baseline:
            (root / "cpu").mkdir()
            line["cpu_baseline"] = cpu_baseline_window(root / "cpu")
        else:
            line["cpu_baseline"] = None
        print(json.dumps(line), flush=True)
    finally:
        shutil.rmtree(root, ignore_errors=True)


DISK_BYTES = 28  # DiskState.update's chunk pass: read g32 4 + w,m,v 12; write w,m,v 12 (no copy)
DISK_CHUNK = 1 << 20  # DiskState.update's default chunk_elements (disk.py:203)


def time_disk(steps, warmup, root, cached=False):
    """DiskState.update (a1, disk.py:203-223) through GpuDiskUpdate on the config-2 window's
    [3, N] files: per parameter, each 1M-element chunk of the memmapped file is staged through
    pinned memory, updated by one fused launch and written back, then flush and fsync.
    cached=True: CachedDiskState.update (a2, state_cache.py:103-140) with every state in its RAM
    cache, so each update is a hit: the chunks are read from the cache and written to the cache
    and the file."""
    import collections
    import threading
    import numpy as np
    from morph_amd import kernels
    from morph_amd.disk import GpuDiskUpdate

    class Store(GpuDiskUpdate, _FileStore):
        pass

    class CachedStore(Store):
        # the cache attributes of state_cache.py that update() uses (23, 103-140)
        def __init__(self, *a):
            super().__init__(*a)
            self._cache_lock = threading.RLock()
            self._cache = collections.OrderedDict()
            self._cache_stats = dict(hits=0, misses=0, estimated_bytes_avoided=0)
            for name, e in self.entries.items():
                self._cache[name] = np.fromfile(self.root / e["file"], dtype=np.float32).reshape(
                    3, e["size"])

        def _drop(self, name):
            self._cache.pop(name, None)

    device = torch.device("cuda", 0)
    names = ["ffn.gate.weight", "ffn.up.weight", "ffn.down.weight"]
    store = (CachedStore if cached else Store)(root, list(zip(names, CONFIG2_SHAPES)))
    gen = torch.Generator(device=device).manual_seed(5)
    grads = {n: torch.randn(s, generator=gen, device=device) * 1e-4 for n, s in zip(names, CONFIG2_SHAPES)}
    step = 0
    for _ in range(warmup):
        step += 1
        for n in names:
            store.update(n, grads[n], step, 3e-4, 1.0)
    # each chunk's launch stamps its own dispatch's start and end
    launches = steps * sum(-(-store.entries[n]["size"] // DISK_CHUNK) for n in names)
    timer = store.dispatch_timer = kernels.DispatchTimer(launches, device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step += 1
        for n in names:
            store.update(n, grads[n], step, 3e-4, 1.0)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    store.dispatch_timer = None
    kms = timer.elapsed_ms()
    hits = store._cache_stats["hits"] if cached else None
    return dict(n=sum(store.entries[n]["size"] for n in names), elapsed=elapsed,
                launch_s=sum(kms) / len(kms) / 1e3, launches=len(kms), cache_hits=hits)


def disk_main(args):
    import shutil
    import tempfile
    root = Path(tempfile.mkdtemp(prefix="morph_disk_"))
    try:
        (root / "gpu").mkdir()
        r = time_disk(args.steps, args.warmup, root / "gpu", cached=args.cached)
        n = r["n"]
        achieved = DISK_BYTES * DISK_CHUNK / r["launch_s"] / 1e9
        metric = ("CachedDiskState.update Gparams/s on cache hits (chunks from the RAM cache, "
                  "written to the cache and the file, flush, fsync), 5B SwiGLU window, 1 MI355X"
                  if args.cached else
                  "DiskState.update Gparams/s (memmapped [3, N] files: chunked staging, fused "
                  "update, write-back, flush, fsync), 5B SwiGLU window, 1 MI355X")
        line = {
            "metric": metric,
            "value": round(n * args.steps / r["elapsed"] / 1e9, 3), "unit": "Gparams/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r["elapsed"] / args.steps * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "config 2 window as three [3, N] float32 state files; per step "
                                   "GpuDiskUpdate.update of every file (chunks of 1M elements "
                                   "through pinned memory, flush, fsync); FP32 gradients on the GPU",
                       "params": n, "shapes": CONFIG2_SHAPES, "chunk_elements": DISK_CHUNK,
                       "cached": bool(args.cached), "cache_hits": r["cache_hits"],
                       "state_dir": "tempfile.mkdtemp() on the GPU box"},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "adamw_multi_kernel<F32,NoOut,host> (one 1M-element chunk "
                                   "per launch; each timed launch stamps its own dispatch)",
                         "avg_launch_us": round(r["launch_s"] * 1e6, 2),
                         "launches_timed": r["launches"],
                         "bytes_per_launch": DISK_BYTES * DISK_CHUNK},
            "bound_by": "the host: reading and writing the memmapped files and their fsync; a "
                        "chunk's launch is a few microseconds",
        }
        if not args.no_cpu_baseline:
            (root / "cpu").mkdir()
            line["cpu_baseline"] = cpu_baseline_window(root / "cpu")
        else:
            line["cpu_baseline"] = None
        print(json.dumps(line), flush=True)
    finally:
        shutil.rmtree(root, ignore_errors=True)


EXPORT_BYTES = 6  # the export's conversion: read the FP32 master 4, write FP16 2 (+ one flag per chunk)
EXPORT_CHUNK = 1 << 20  # the reference's chunk (export.py:16): one conversion launch and flag each


class _ExportConfig:
    def to_dict(self):
        return dict(preset="5b", d_model=3072, d_ff=6144)


class _ExportModel(torch.nn.Module):
    """The config-2 window's matrices on the meta device, as the export's schema check sees a
    model (export.py:24-25): parameter names, shapes and order, and a config with to_dict()."""

    def __init__(self):
        super().__init__()
        self.config = _ExportConfig()
        mk = lambda o, i: torch.nn.Linear(i, o, bias=False, device="meta")  # noqa: E731
        self.gate, self.up, self.down = mk(6144, 3072), mk(6144, 3072), mk(3072, 6144)


def time_export(steps, warmup, root):
    """FP16 shard export (f3, export.py:16-43) of the config-2 window from its [3, N] state
    files: the rows go through pinned staging, the GPU converts each 1M-element chunk with its
    range flag, the host writes and hashes the shards (SHA-256) and fsyncs them."""
    import shutil
    from morph_amd import _lib
    from morph_amd.export import export_fp16
    device = torch.device("cuda", 0)
    model = _ExportModel()
    state = root / "state"
    state.mkdir()
    store = _FileStore(state, [(n, p.shape) for n, p in model.named_parameters()])
    (state / "manifest.json").write_text(json.dumps(dict(
        entries=store.entries, step=7, dirty=False, config=model.config.to_dict())))
    times = []
    for k in range(warmup + steps):
        out = root / f"out{k}"
        t0 = time.perf_counter()
        export_fp16(state, out, model=model, device=device)
        if k >= warmup:
            times.append(time.perf_counter() - t0)
        shutil.rmtree(out)
    # the export's conversion launch: one 1M-element chunk with its range flag, back to back
    src = torch.randn(EXPORT_CHUNK, device=device) * .02
    dst = torch.empty(EXPORT_CHUNK, dtype=torch.float16, device=device)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    L, sh = _lib.lib(), _lib.stream_handle()
    launch = lambda: _lib.check(L.morph_convert_f32(  # noqa: E731
        ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), _lib.DTYPE_F16,
        EXPORT_CHUNK, ctypes.c_void_p(flag.data_ptr()), sh))
    for _ in range(20):
        launch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(200):
        launch()
    e1.record()
    torch.cuda.synchronize()
    return dict(n=sum(e["size"] for e in store.entries.values()), times=sorted(times),
                launch_s=e0.elapsed_time(e1) / 1e3 / 200, state=state, model=model)


def cpu_baseline_export(state, model, out):
    """The reference's export (export.py:26-36: memmap rows, finite/range check, astype('<f2'),
    write, SHA-256, fsync per shard) restated on the CPU, on the same state files."""
    from oracle import reference as R
    cpus = host_cpus()
    t0 = time.perf_counter()
    R.export_fp16_reference(state, out, model, durable=True)
    t = time.perf_counter() - t0
    n = sum(p.numel() for p in model.parameters())
    return dict(value=round(n / t / 1e9, 4), unit="Gparams/s", **cpu_fields(cpus), kind="port",
                sample=f"one export of the config-2 window's three state files: {t * 1e3:.0f} ms "
                       "(single-threaded numpy, as the reference's loop runs)")


def export_main(args):
    import shutil
    import tempfile
    root = Path(tempfile.mkdtemp(prefix="morph_export_"))
    try:
        r = time_export(args.steps, args.warmup, root)
        n, t = r["n"], r["times"][len(r["times"]) // 2]
        achieved = EXPORT_BYTES * EXPORT_CHUNK / r["launch_s"] / 1e9
        line = {
            "metric": "FP16 shard export Gparams/s (morph-fp16-shards-v1: GPU encode + range check, "
                      "SHA-256, fsync), 5B SwiGLU window, 1 MI355X",
            "value": round(n / t / 1e9, 3), "unit": "Gparams/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t * 1e3, 2),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
            "data": "synthetic",
            "config": {"workload": "config 2 window as three [3, N] float32 state files -> FP16 "
                                   "shards + manifest (one export per step; median)",
                       "params": n, "shapes": CONFIG2_SHAPES, "chunk_elements": EXPORT_CHUNK,
                       "state_dir": "tempfile.mkdtemp() on the GPU box"},
            "shard_write_gbs": round(2 * n / t / 1e9, 3),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "convert_kernel<F16,true> (one 1M-element chunk with its range "
                                   "flag, launches back to back)",
                         "avg_launch_us": round(r["launch_s"] * 1e6, 2),
                         "bytes_per_launch": EXPORT_BYTES * EXPORT_CHUNK},
            "bound_by": "the host: file reads into pinned memory, SHA-256 and fsync of the shards; "
                        "the GPU conversion is a few percent of the export",
        }
        line["cpu_baseline"] = None if args.no_cpu_baseline else cpu_baseline_export(
            r["state"], r["model"], root / "cpu")
        print(json.dumps(line), flush=True)
    finally:
        shutil.rmtree(root, ignore_errors=True)


FP8_PACK_BYTES, FP8_UNPACK_BYTES = 3, 3  # FP16 in 2 + byte out 1 (+ 4 B per 256); byte in 1 + FP16 out 2


def time_fp8(steps, warmup):
    """FP8 transport (precision.py:24-37) of the config-2 window's FP16 compute weights."""
    from morph_amd import fp8
    device = torch.device("cuda", 0)
    gen = torch.Generator(device=device).manual_seed(9)
    w = [(torch.randn(s, generator=gen, device=device) * .02).half() for s in CONFIG2_SHAPES]
    n = sum(t.numel() for t in w)
    stream = torch.cuda.current_stream()

    def one(tp=None, tu=None):
        packed = []
        for t in w:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            packed.append(fp8.pack_fp8(t))
            b.record(stream)
            if tp is not None:
                tp.append((a, b))
        for (enc, sc) in packed:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fp8.unpack_fp8(enc, sc, torch.float16)
            b.record(stream)
            if tu is not None:
                tu.append((a, b))

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    tp, tu = [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        one(tp, tu)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    pack_s = sum(a.elapsed_time(b) for a, b in tp) / 1e3 / steps
    unpack_s = sum(a.elapsed_time(b) for a, b in tu) / 1e3 / steps
    return dict(n=n, elapsed=elapsed, pack_s=pack_s, unpack_s=unpack_s)


def cpu_baseline_fp8():
    """The reference's pack_fp8 / unpack_fp8 (torch CPU ops) on one [6144, 3072] FP16 weight."""
    from oracle import reference as R
    cpus = host_cpus()
    w = (torch.randn(6144, 3072, generator=torch.Generator().manual_seed(9)) * .02).half()
    t0 = time.perf_counter()
    enc, sc = R.pack_fp8_torch(w)
    t_pack = time.perf_counter() - t0
    t0 = time.perf_counter()
    R.unpack_fp8_torch(enc, sc, torch.float16)
    t_unpack = time.perf_counter() - t0
    return dict(value=round(w.numel() / t_pack / 1e9, 4), unit="Gparams/s (pack)", **cpu_fields(cpus),
                kind="port", sample=f"one [6144, 3072] FP16 weight: pack {t_pack * 1e3:.0f} ms, "
                                    f"unpack {t_unpack * 1e3:.0f} ms ({w.numel() / t_unpack / 1e9:.3f} Gparam/s)")


def fp8_main(args):
    r = time_fp8(args.steps, args.warmup)
    n = r["n"]
    achieved = FP8_UNPACK_BYTES * n / r["unpack_s"] / 1e9
    line = {
        "metric": "FP8 E4M3FN block-scaled pack + unpack Gparams/s, 5B SwiGLU window, 1 MI355X",
        "value": round(n * args.steps / r["elapsed"] / 1e9, 3), "unit": "Gparams/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["elapsed"] / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "config 2 window FP16 compute weights: pack to E4M3FN + per-256 FP32 "
                               "scales, unpack back to FP16 (3 tensors)", "params": n,
                   "shapes": CONFIG2_SHAPES},
        "pack_gparams_per_s": round(n / r["pack_s"] / 1e9, 2),
        "unpack_gparams_per_s": round(n / r["unpack_s"] / 1e9, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "unpack_kernel<F16>", "avg_launch_us": round(r["unpack_s"] / 3 * 1e6, 2),
                     "bytes_per_launch": FP8_UNPACK_BYTES * n // 3},
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_fp8(),
    }
    print(json.dumps(line), flush=True)



EMBED_SHAPE = (65536, 3072)
EMBED_GRAD_SETS = 4  # distinct sparse-row gradients, cycled over the steps


def time_embedding(steps, warmup):
    """Config 3: the tied [65536, 3072] embedding, one tensor of 201,326,592 FP32 masters.
    Each step's BF16 gradient is nonzero only on rows drawn Zipf(1.1) from 4 x 1024 token IDs
    (N(0, 1e-3) there); every row still gets the dense update; wd 0, BF16 export.  A step is
    detector (carrying the previous step's close) + fused AdamW, as in the config-2 workload; the AdamW launches of the
    timed steps are timed by dispatch-stamped events."""
    from morph_amd import FusedAdamW
    from morph_amd.kernels import DispatchTimer
    device = torch.device("cuda", 0)
    w = torch.randn(EMBED_SHAPE, generator=torch.Generator(device=device).manual_seed(3),
                    device=device) * .02
    sets, rows = [], []
    for k in range(EMBED_GRAD_SETS):
        g, active = config3_embedding_grad(3000 + k, device=device)
        sets.append([g])
        rows.append(active.numel())
    opt = FusedAdamW([w], lr=3e-4, betas=(.9, .95), eps=1e-8, weight_decay=0.0,
                     export_dtype=torch.bfloat16)
    for t in range(warmup):
        opt.step(sets[t % EMBED_GRAD_SETS])
    opt.resolve()
    timer = opt.dispatch_timer = DispatchTimer(steps, device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(steps):
        opt.step(sets[t % EMBED_GRAD_SETS])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    opt.dispatch_timer = None
    kernel_ms = timer.elapsed_ms()
    opt.resolve()
    if opt.skipped_steps:
        raise RuntimeError(f"{opt.skipped_steps} steps skipped on synthetic finite gradients")
    return dict(n=w.numel(), elapsed=elapsed, avg_kernel_s=sum(kernel_ms) / len(kernel_ms) / 1e3,
                rows=rows)


def cpu_baseline_embedding(seconds=20.0):
    """torch.optim.AdamW(foreach=False) on the [65536, 3072] embedding on the host cores
    (BF16 gradient widened to FP32, wd 0): whole steps until `seconds` have passed (at
    least 2), median."""
    from oracle import reference as R
    cpus = host_cpus()
    w = torch.nn.Parameter(torch.randn(EMBED_SHAPE, generator=torch.Generator().manual_seed(3)) * .02)
    g16, _ = config3_embedding_grad(3000)
    opt = torch.optim.AdamW([w], lr=3e-4, betas=(.9, .95), eps=1e-8, weight_decay=0.0,
                            foreach=False)
    times = []
    start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - start < seconds and len(times) < 10):
        t0 = time.perf_counter()
        w.grad = g16.float()
        opt.step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return dict(value=round(w.numel() / med / 1e9, 4), unit="Gparams/s", **cpu_fields(cpus),
                kind="port", sample=f"[65536, 3072] embedding, {len(times)} whole steps, median; "
                                    "torch.optim.AdamW(foreach=False), BF16 grad widened to FP32")


def embedding_main(args):
    r = time_embedding(args.steps, args.warmup)
    n = r["n"]
    achieved = BYTES_PER_PARAM * n / r["avg_kernel_s"] / 1e9
    line = {
        "metric": "AdamW Gparams/s + achieved HBM GB/s vs peak, tied 65536x3072 embedding, 1 MI355X",
        "value": round(n * args.steps / r["elapsed"] / 1e9, 3), "unit": "Gparams/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["elapsed"] / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config 3: tied [65536, 3072] embedding, FP32 masters, BF16 "
                               "sparse-row grads (Zipf(1.1) rows of 4x1024 tokens, N(0, 1e-3)), "
                               "dense update of every row, wd 0, BF16 export; detector (carrying "
                               "the previous step's close) + fused AdamW",
                   "params": n, "shape": list(EMBED_SHAPE), "grad_dtype": "bf16",
                   "export_dtype": "bf16", "lr": 3e-4, "betas": [0.9, 0.95], "eps": 1e-8,
                   "weight_decay": 0.0, "gradient_rows_per_step": r["rows"]},
        "kernel_gparams_per_s": round(n / r["avg_kernel_s"] / 1e9, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(TRAFFIC_PROFILE_C3),
                     "traffic_source": TRAFFIC_SOURCE % TRAFFIC_PROFILE_C3.name,
                     "kernel": "adamw_multi_kernel<BF16,BF16,dev>",
                     "avg_launch_us": round(r["avg_kernel_s"] * 1e6, 2),
                     "bytes_per_launch": BYTES_PER_PARAM * n},
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_embedding(),
    }
    print(json.dumps(line), flush=True)


def time_streamed(steps, warmup, muon=False, pinned=False, resident=False, device_grads=False,
                  stream_parts=None):
    """The streamed engines' layout (runner.py:41-46, engine.py:75-88): FP32 masters and
    FP32 (already unscaled) gradients in pageable CPU memory, optimizer state resident in
    HBM.  A step uploads every gradient and master through pinned staging, runs the
    device step on the mirrors, and writes the masters back into the CPU tensors before
    step() returns (morph_amd.staging).  muon=False: FusedAdamW over the config-2 window;
    muon=True: HybridMuonAdamW over config 5 (42 matrices + the AdamW vectors).
    pinned=True: the masters are moved into page-locked memory first (pin_host_tensors),
    so they cross PCIe by DMA alone; the gradients stay pageable, as the engine leaves
    them.  resident=True: the optimizers keep the masters' device mirrors between steps
    (resident_masters), so only the gradients go up and the masters come back.
    device_grads=True: the gradients are handed to step() as FP32 tensors on the GPU (the
    engine's device stage buffers, engine.py:67, before Slot.flush copies them to CPU
    p.grad), so no gradient crosses PCIe."""
    from morph_amd import FusedAdamW, pin_host_tensors
    from morph_amd.muon import HybridMuonAdamW
    cpus = host_cpus()  # torch's intra-op threads; the staging copies run on the library's pool
    if muon:
        model = Config5("cpu")
        gen = torch.Generator().manual_seed(6)
        for p in model.parameters():
            p.grad = torch.randn(p.shape, generator=gen) * 1e-3
        if pinned:
            pin_host_tensors(model.parameters())
        opt = HybridMuonAdamW(model, lr=3e-4, muon_lr=0.02, resident_masters=resident)
        if stream_parts is not None:
            opt.stream_parts = stream_parts
        params = list(model.parameters())
        stagings = [opt._muon_masters, opt._muon_grads, opt.adam._staging]
    else:
        params = [torch.nn.Parameter(m) for m in config2_window("cpu")]
        for p, g in zip(params, config2_grads("cpu", 1000)):
            p.grad = g.float() / LOSS_SCALE
        if pinned:
            pin_host_tensors(params)
        opt = FusedAdamW(params, **HYPER, resident_masters=resident)
        stagings = [opt._staging]
    if device_grads:
        device = torch.device("cuda", torch.cuda.current_device())
        dev = [p.grad.to(device) for p in params]
        hand = dict(zip(params, dev)) if muon else dev
        step = lambda: opt.step(hand)  # noqa: E731
    else:
        step = opt.step
    for _ in range(warmup):
        step()
    grad_staging = opt.adam._grad_staging if muon else opt._grad_staging
    if grad_staging is not None:
        stagings.append(grad_staging)
    torch.cuda.synchronize()
    h2d0 = sum(st.bytes_h2d for st in stagings)
    d2h0 = sum(st.bytes_d2h for st in stagings)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()  # returns with the new masters in the CPU tensors
    elapsed = time.perf_counter() - t0
    torch.cuda.synchronize()
    from morph_amd import staging
    return dict(elapsed=elapsed, n=sum(p.numel() for p in params), cpus=cpus,
                h2d=(sum(st.bytes_h2d for st in stagings) - h2d0) / steps,
                d2h=(sum(st.bytes_d2h for st in stagings) - d2h0) / steps,
                copy_threads=staging.COPY_THREADS or staging.default_copy_threads())


def streamed_main(args, muon=False):
    r = time_streamed(args.steps, args.warmup, muon, args.pinned, args.resident_masters,
                      args.device_grads, args.stream_parts)
    n, t = r["n"], r["elapsed"] / args.steps
    line = {
        "metric": ("HybridMuonAdamW step" if muon else "AdamW step") + " with CPU FP32 masters "
                  "(streamed engines), PCIe included, 1 MI355X",
        "value": round(n / t / 1e9, 3), "unit": "Gparams/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(t * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": ("config 5 (42 x [3072, 6144] Muon + 326 AdamW vectors)" if muon
                                else "config-2 window (N = 56,623,104)") +
                               (" with FP32 masters in pinned" if args.pinned else
                                " with FP32 masters in pageable") +
                               (" CPU memory (pin_host_tensors)" if args.pinned else " CPU memory") +
                               (" and FP32 gradients on the GPU (step(grads): the engine's device "
                                "stage buffers); " if args.device_grads else
                                " and FP32 gradients in pageable CPU memory; ") +
                               "state resident in HBM; step = " +
                               ", ".join(
                                   (["upload gradients"] if not args.device_grads else []) +
                                   (["upload masters"] if not args.resident_masters else
                                    ["masters' device mirrors kept between steps "
                                     "(resident_masters)"]) +
                                   ["device step", "masters back into the CPU tensors"]),
                   "params": n, "masters": "pinned" if args.pinned else "pageable",
                   "gradients": "device" if args.device_grads else "pageable",
                   "stream_parts": args.stream_parts,
                   "resident_masters": bool(args.resident_masters)},
        "pcie": {"h2d_bytes_per_step": int(r["h2d"]), "d2h_bytes_per_step": int(r["d2h"]),
                 "h2d_plus_d2h_gb_per_s": round((r["h2d"] + r["d2h"]) / t / 1e9, 2),
                 "host_threads": r["cpus"]["threads"],
                 "staging_copy_threads": r["copy_threads"]},
        "cpu_baseline": None if args.no_cpu_baseline else (
            cpu_baseline_muon() if muon else cpu_baseline()),
    }
    print(json.dumps(line), flush=True)


CONFIG4_STEPS = 16
CONFIG4_OVERFLOW = (3, 7, 12)


def config4_sequence(device, seed=44):
    """Config 4's 16 gradient sets: config-2 FP16 gradients x 2^16, with +inf/-inf/NaN written
    at 1-8 seeded positions in steps 3, 7 and 12 (numpy RandomState(seed) picks the count,
    tensor, position and value, in that order)."""
    import numpy as np
    rng = np.random.RandomState(seed)
    sets = []
    for t in range(1, CONFIG4_STEPS + 1):
        grads = config2_grads(device, 4000 + t)
        if t in CONFIG4_OVERFLOW:
            for _ in range(int(rng.randint(1, 9))):
                k = int(rng.randint(len(grads)))
                flat = grads[k].view(-1)
                flat[int(rng.randint(flat.numel()))] = float(rng.choice([np.inf, -np.inf, np.nan]))
        sets.append(grads)
    return sets


def expected_config4_scales():
    """Loss scale before each of the 16 steps by DynamicLossScale's rule (precision.py:6-17):
    halve on overflow, grow x2 after 2000 good steps (not reached), cap 65536."""
    from morph_amd import DynamicLossScale
    s = DynamicLossScale(LOSS_SCALE, growth_interval=2000)
    out = []
    for t in range(1, CONFIG4_STEPS + 1):
        out.append(s.scale)
        s.overflow() if t in CONFIG4_OVERFLOW else s.success()
    return out, s.state_dict()


def time_overflow(reps):
    """Config 4 on the config-2 window: the 16-step sequence enqueued back to back (skip
    decisions, loss scale and clocks stay on the device).  One optimizer runs it once
    untimed (its launch tables and bias tables are built there), then `reps` more times
    timed; every repetition overflows three more times, so the scale keeps halving
    (2^16 -> 2^4 after four).  Fresh optimizers then give per-launch times and, step by
    step (sync=True), every decision and scale of the config's own 16 steps."""
    from morph_amd import DynamicLossScale, FusedAdamW
    from morph_amd.kernels import DispatchTimer
    device = torch.device("cuda", 0)
    sets = config4_sequence(device)
    masters0 = config2_window(device)
    n = sum(m.numel() for m in masters0)

    def fresh(sync=False):
        scaler = DynamicLossScale(LOSS_SCALE, growth_interval=2000)
        opt = FusedAdamW([m.clone() for m in masters0], **HYPER, loss_scale=scaler,
                         export_dtype=torch.float16, arena=True, sync=sync)
        return opt, scaler

    opt, scaler = fresh()
    for grads in sets:
        opt.step(grads)
    opt.resolve()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        for grads in sets:
            opt.step(grads)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    opt.resolve()
    if opt.skipped_steps != 3 * (reps + 1):
        raise RuntimeError(f"{opt.skipped_steps} skipped steps in {reps + 1} sequences")
    del opt
    # per-launch AdamW times, applied vs skipped steps (dispatch-stamped events)
    opt, _ = fresh()
    timer = opt.dispatch_timer = DispatchTimer(len(sets), device)
    for grads in sets:
        opt.step(grads)
    torch.cuda.synchronize()
    opt.dispatch_timer = None
    kernel_us = [ms * 1e3 for ms in timer.elapsed_ms()]
    opt.resolve()
    # step by step: every decision and the scale before each step
    sopt, sscaler = fresh(sync=True)
    scales, applied = [], []
    for grads in sets:
        scales.append(sscaler.scale)
        applied.append(bool(sopt.step(grads)))
    clocks = [sopt.state[p]["step"] for p in sopt.param_groups[0]["params"]]
    return dict(n=n, elapsed=elapsed, kernel_us=kernel_us, scales=scales, applied=applied,
                scaler_state=sscaler.state_dict(), clocks=clocks,
                async_skipped=opt.skipped_steps, async_applied=opt.applied_steps)


def overflow_main(args):
    reps = min(4, max(1, args.steps // CONFIG4_STEPS))  # 3 halvings per sequence: stay > 1
    r = time_overflow(reps)
    n = r["n"]
    want_scales, want_state = expected_config4_scales()
    skipped = [t for t, a in enumerate(r["applied"], 1) if not a]
    ok = (r["scales"] == want_scales and r["scaler_state"] == want_state
          and skipped == list(CONFIG4_OVERFLOW) and r["async_skipped"] == len(CONFIG4_OVERFLOW)
          and r["clocks"] == [CONFIG4_STEPS - len(CONFIG4_OVERFLOW)] * 3)
    k_app = [u for u, a in zip(r["kernel_us"], r["applied"]) if a]
    k_skip = [u for u, a in zip(r["kernel_us"], r["applied"]) if not a]
    avg_app = sum(k_app) / len(k_app)
    achieved = BYTES_PER_PARAM * n / avg_app / 1e3
    steps_run = reps * CONFIG4_STEPS
    line = {
        "metric": "Conditional-skip AdamW Gparams/s over config 4's 16 steps (3 skipped), 5B SwiGLU window, 1 MI355X",
        "value": round(n * steps_run / r["elapsed"] / 1e9, 3), "unit": "Gparams/s",
        "n_gpus": 1, "steps": steps_run, "warmup": CONFIG4_STEPS,
        "ms_per_step": round(r["elapsed"] / steps_run * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config 4: config-2 window, 16 steps from loss scale 2^16, "
                               "+inf/-inf/NaN at 1-8 seeded positions in steps 3, 7, 12; "
                               "detector (carrying the previous step's close) + fused AdamW, "
                               "enqueued back to back; "
                               "timed: the sequence repeated on one warmed optimizer",
                   "params": n, "shapes": CONFIG2_SHAPES, "overflow_steps": list(CONFIG4_OVERFLOW),
                   "repetitions": reps},
        "sequence_ok": ok,
        "skipped_steps": skipped,
        "scale_before_step": r["scales"],
        "adamw_us_applied": round(avg_app, 2),
        "adamw_us_skipped": round(sum(k_skip) / len(k_skip), 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "adamw_multi_kernel<F16,F16,dev> (applied steps)",
                     "avg_launch_us": round(avg_app, 2), "bytes_per_launch": BYTES_PER_PARAM * n},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    if not ok:
        raise SystemExit("config-4 sequence differs from DynamicLossScale's rule")

def measured_mfma():
    """Per-product MFMA-busy fraction and clock from the committed rocprofv3 counter pass."""
    try:
        d = json.loads(MFMA_PROFILE.read_text())["products"]
    except (OSError, KeyError, ValueError):
        return None
    return {k: {"mfma_busy_pct": v["mfma_busy_pct"], "clock_ghz": v["clock_ghz"]} for k, v in d.items()}


def measured_traffic(path=TRAFFIC_PROFILE):
    """HBM bytes per launch of a workload's dominant kernel, from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE passes."""
    try:
        return json.loads(path.read_text())["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("adamw", "embedding", "overflow", "muon", "grads",
                                           "window", "disk", "fp8", "export", "streamed",
                                           "streamed_muon"),
                    default="adamw",
                    help="adamw: the headline config-2 step (default); embedding: config 3; "
                         "overflow: config 4's skip sequence; muon: config 5; "
                         "grads: the stage-gradient window; window: the HBM-resident [3, N] "
                         "state; disk: DiskState.update on the memmapped [3, N] files; "
                         "fp8: block-scaled FP8 transport encoding; export: FP16 shard "
                         "export of the window's state files; streamed / "
                         "streamed_muon: config 2 / config 5 with CPU FP32 masters, PCIe included")
    ap.add_argument("--pinned", action="store_true",
                    help="streamed / streamed_muon: masters in page-locked host memory "
                         "(pin_host_tensors), moved by DMA alone")
    ap.add_argument("--resident-masters", action="store_true",
                    help="streamed / streamed_muon: keep the masters' device mirrors between "
                         "steps (resident_masters=True), so only gradients cross PCIe upward")
    ap.add_argument("--cached", action="store_true",
                    help="disk: CachedDiskState.update with every state in its RAM cache (hits)")
    ap.add_argument("--device-grads", action="store_true",
                    help="streamed / streamed_muon: hand the gradients to step() as FP32 tensors "
                         "on the GPU (the engine's device stage buffers): no gradient upload")
    ap.add_argument("--stream-parts", type=int, default=None, metavar="K",
                    help="streamed_muon: HybridMuonAdamW.stream_parts (the matrices go through "
                         "the step in K parts; default: the optimizer's choice, 2 with CPU "
                         "gradients, one per 6 matrices with device gradients)")
    ap.add_argument("--copy-calibration", type=int, metavar="MIB", default=0,
                    help="only run 5 plain device copies of MIB MiB (rocprof counter scale)")
    args = ap.parse_args()
    if args.copy_calibration:
        src = torch.ones(args.copy_calibration << 18, device="cuda")  # MiB of float32
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": src.numel() * 4}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported by this "
              "build (the optimizer step shards by contiguous ranges across GPUs, see the "
              "design notes, but no multi-GPU run is part of it)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.workload == "embedding":
        return embedding_main(args)
    if args.workload == "overflow":
        return overflow_main(args)
    if args.workload == "muon":
        return muon_main(args)
    if args.workload == "grads":
        return grads_main(args)
    if args.workload == "window":
        return window_main(args)
    if args.workload in ("streamed", "streamed_muon"):
        return streamed_main(args, muon=args.workload == "streamed_muon")
    if args.workload == "fp8":
        return fp8_main(args)
    if args.workload == "export":
        return export_main(args)
    if args.workload == "disk":
        return disk_main(args)
    r = time_gpu(args.steps, args.warmup)
    n = r["n"]
    ms_per_step = r["elapsed"] / args.steps * 1e3
    achieved = BYTES_PER_PARAM * n / r["avg_kernel_s"] / 1e9
    line = {
        "metric": "AdamW Gparams/s + achieved HBM GB/s vs peak, 5B SwiGLU window, 1 MI355X",
        "value": round(n * args.steps / r["elapsed"] / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config 2: 5B-preset SwiGLU stage window, FP32 masters, "
                               "FP16 grads x 2^16 loss scale, detector + fused AdamW + FP16 export",
                   "params": n, "shapes": CONFIG2_SHAPES, "grad_dtype": "f16",
                   "export_dtype": "f16", **{k: v for k, v in HYPER.items()},
                   "loss_scale": LOSS_SCALE,
                   "state_layout": "one arena: masters, moments, export (FusedAdamW(arena=True))",
                   "gradient_sets": GRAD_SETS},
        "kernel_gparams_per_s": round(n / r["avg_kernel_s"] / 1e9, 3),
        "timing": f"every {STAMP_EVERY}th AdamW launch of the timed steps (steps {STAMP_EVERY - 1}, "
                  f"{2 * STAMP_EVERY - 1}, ...) "
                  "stamps HIP events with its own dispatch (hipExtLaunchKernel, launch stream); "
                  "the two step forms below carry none",
        "kernel_samples": len(r["kernel_ms"]),
        "step_uninstrumented": {
            "gparams_per_s": round(n * args.steps / r["elapsed_plain"] / 1e9, 3),
            "ms_per_step": round(r["elapsed_plain"] / args.steps * 1e3, 4),
            "what": "the same step, K more times, without timing events"},
        "step_checked": {
            "gparams_per_s": round(n * args.steps / r["elapsed_checked"] / 1e9, 3),
            "ms_per_step": round(r["elapsed_checked"] / args.steps * 1e3, 4),
            "what": "fused AdamW + step close with the non-finite flag already set by the "
                    "gradients' producer (step(checked=True)); no detector pass; no timing events"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "traffic_source": TRAFFIC_SOURCE % TRAFFIC_PROFILE.name,
                     "kernel": "adamw_multi_kernel<F16,F16,dev>",
                     "avg_launch_us": round(r["avg_kernel_s"] * 1e6, 2),
                     "bytes_per_launch": BYTES_PER_PARAM * n,
                     "frac_of_copy": round(achieved / r["copy"]["achieved"], 4)},
        "copy_ceiling": r["copy"],
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
