#!/usr/bin/env python3
"""Benchmark of the HeadStartLSTM training hot path on one MI355X.

Workload (the headline): recurrent mode, fp32,
T=256 B=32 D=256 H=512, a=1e-4, x ~ N(0,1), nn.LSTM init, h0=c0=0,
loss = out.sum(); one step = forward + backward (all parameter gradients; x is
data, so no dx, as in the reference's training loop), captured whole in one HIP
graph and replayed.  Synthetic data, seeded.

Prints ONE JSON line:
  value       timesteps*batch/s = T*B / step time
  roofline    the dominant kernel of the step (persistent recurrent kernel),
              algorithmic fp32 MFMA FLOPs per launch / its mean launch time,
              timed with HIP events on its launch stream; the backward kernel's
              FLOPs include the weight-gradient products it accumulates.  traffic:
              HBM bytes per launch from the committed rocprofv3 --pmc summary
              (traffic_source)
  recurrence  per-step latency of the persistent kernels (launch time / T) beside
              the fp32 MFMA floor of one step's recurrent product
  step_tflops FLOPs the step executes (x is data: no dx product) / step time
  cpu_baseline the CPU restatement of the reference torch backend (oracle/),
              same workload, timed on every core of this process's CPU affinity;
              with the parallel-mode restatement (_parallel.py) at configs[1] and
              configs[4] beside it
  scan        configs[4] parallel scan (T=4096 B=16 H=1024) forward and
              backward kernels: algorithmic HBM bytes / launch time
  fused_products  the arithmetic of the products fused into the headline step's
              persistent kernels (split_bf16x6 by default, fp32 with
              hsl_set_split_products(0)); split_products_off: the same step and its
              kernel times with every product on the fp32 instruction
  modes       every configured shape (configs[0..4], configs[1] in both modes, and
              the reference's published T64 B32 (D128 H256) and (D512 H1024) shapes)
              as one graph-replayed fwd+bwd step each; TFLOP/s counts the products
              the step executes: 16*T*B*H*D + 24*T*B*H^2 (recurrent: projection,
              recurrence both ways, dW_ih, dW_hh) or 2*2*T*B*D*4H (parallel:
              projection and dW_ih); x is data, so no dx
"""

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
METRIC = "fwd+bwd ms/step & timesteps·batch/s at T256 B32 D256 H512; scan HBM GB/s"
T, B, D, H = 256, 32, 256, 512
ST, SB, SD, SH = 4096, 16, 256, 1024


def executed_flops(t, b, d, h, parallel):
    """FLOPs of the products one training step executes with x as data (no dx)."""
    if parallel:
        return 2 * (2 * t * b * d * 4 * h)           # projection, dW_ih
    return 16 * t * b * h * d + 24 * t * b * h * h   # projection + dW_ih, 3 recurrent products


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """(HBM bytes per launch of `kernel`, source file) from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a known-size copy), or (None, None)."""
    for f in sorted((ROOT / "profiles").glob("hbm_traffic_*.md")):
        for line in f.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
                return int(float(parts[2])), str(f.relative_to(ROOT))
    return None, None


def make_inputs():
    """configs[2] synthetic inputs: seed 0, the module built on the CPU (a = 1e-4), then
    x ~ N(0, 1) of shape [T, B, D] drawn from the same generator."""
    from prlstm_amd import HeadStartLSTM
    torch.manual_seed(0)
    m = HeadStartLSTM(D, H, a_init=1e-4)
    x = torch.randn(T, B, D)
    return m, x


def _graph_step_ms(m, x, steps, warmup):
    """(ms per step, wall ms per step): `steps` replays of the captured fwd+bwd step after
    `warmup` replays, bracketed by events on the replay stream."""
    from prlstm_amd.graph import GraphedTrainStep
    step = GraphedTrainStep(m, x)
    for _ in range(warmup):
        step.step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step.step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - w0) * 1e3 / steps
    return e0.elapsed_time(e1) / steps, wall_ms


def _kernel_ms(m, x, steps):
    """Mean launch time (ms) of each library kernel kind over `steps` eager steps, from the
    HIP events the library records on the launch stream (hsl_set_timing)."""
    from prlstm_amd import _lib
    kinds = ("rec_fwd", "rec_bwd", "input_proj", "step_fwd", "step_bwd")
    _lib.set_timing(True)
    for k in kinds:
        _lib.timing_collect(k)
    for _ in range(steps):
        m.zero_grad(set_to_none=True)
        out, _ = m(x)
        out.sum().backward()
    torch.cuda.synchronize()
    kern = {}
    for k in kinds:
        tot, n = _lib.timing_collect(k)
        if n:
            kern[k] = tot / n
    _lib.set_timing(False)
    return kern


def bench_gpu(args):
    from prlstm_amd import _lib
    dev = torch.device("cuda", 0)
    m_cpu, x_cpu = make_inputs()
    m = m_cpu.to(dev)
    x = x_cpu.to(dev)
    ms, wall_ms = _graph_step_ms(m, x, args.steps, args.warmup)
    path = _lib.last_recurrent_path()
    kern = _kernel_ms(m, x, args.steps)
    fused = _lib.last_backward_fused()
    log(f"graph step {ms:.4f} ms (wall {wall_ms:.4f} ms), path {path}, fused wgrad {fused}, kernels(ms) {kern}")
    off = None
    if not args.no_split_off:
        # the same step with every fused and separate product on the fp32 instruction
        prev = _lib.set_split_products(0)
        try:
            off_ms, _ = _graph_step_ms(m, x, args.steps, args.warmup)
            off_kern = _kernel_ms(m, x, args.steps)
        finally:
            _lib.set_split_products(prev)
        off = {"arithmetic": "fp32", "ms_per_step": round(off_ms, 5),
               "timesteps_batch_per_s": round(T * B / off_ms * 1e3, 1),
               "kernels_ms": {k: round(v, 5) for k, v in off_kern.items()}}
        log(f"split products off: graph step {off_ms:.4f} ms, kernels(ms) {off_kern}")
    return ms, wall_ms, kern, path, fused, off


def bench_scan(args):
    from prlstm_amd import _lib, HeadStartLSTM
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    m = HeadStartLSTM(SD, SH, a_init=0.0)
    x = torch.randn(ST, SB, SD, device=dev)
    w_ih = m.weight_ih_l0.detach().to(dev)
    b_ih = m.bias_ih_l0.detach().to(dev)
    c0 = torch.zeros(SB, SH, device=dev)
    gates = torch.empty(ST, SB, 4 * SH, device=dev)
    out = torch.empty(ST, SB, SH, device=dev)
    c_ck = torch.empty(_lib.load().hsl_scan_ck_rows(ST), SB, SH, device=dev)
    dout = torch.randn(ST, SB, SH, device=dev)
    dh_n = torch.zeros(SB, SH, device=dev)
    dc_n = torch.zeros(SB, SH, device=dev)
    dgates = torch.empty(ST, SB, 4 * SH, device=dev)
    db_part = torch.empty(SB, 4 * SH, dtype=torch.float64, device=dev)
    P, s = _lib.ptr, _lib.stream_of(dev)
    _lib.call("hsl_par_fwd", P(x), P(c0), P(w_ih), P(b_ih), 1e-6, P(gates), P(out), P(c_ck),
              ST, SB, SD, SH, s)
    reps = max(3, args.steps // 2)
    for warm in (True, False):
        if not warm:
            _lib.set_timing(True)
            _lib.timing_collect("scan_fwd")
            _lib.timing_collect("scan_bwd")
        for _ in range(1 if warm else reps):
            _lib.call("hsl_scan_fwd", P(gates), P(c0), 1e-6, P(out), P(c_ck), ST, SB, SH, s)
            _lib.call("hsl_scan_bwd", P(gates), P(c0), P(c_ck), P(dout), P(dh_n), P(dc_n), 1e-6,
                      P(dgates), P(db_part), None, ST, SB, SH, s)
    torch.cuda.synchronize()
    # known-size elementwise kernel (reads and writes 256 MiB each) for calibrating
    # the FETCH_SIZE / WRITE_SIZE counters of rocprofv3 --pmc runs of this script
    calib = out.view(-1)[: 64 * 2 ** 20]
    torch.mul(dout.view(-1)[: 64 * 2 ** 20], 1.0, out=calib)
    torch.cuda.synchronize()
    tf, nf = _lib.timing_collect("scan_fwd")
    tb, nb = _lib.timing_collect("scan_bwd")
    _lib.set_timing(False)
    fwd_ms, bwd_ms = tf / nf, tb / nb
    n = ST * SB * SH
    # per element: forward reads 4 gates, writes out; backward reads 4 gates and dout, writes
    # 4 dgates; plus the rows of c kept every 8th step (written once, read back once)
    ck = _lib.load().hsl_scan_ck_rows(ST) * SB * SH
    fwd_b, bwd_b = 20 * n + 4 * ck, 36 * n + 4 * (ck - SB * SH)
    res = {
        "config": {"workload": "parallel scan fwd+bwd kernels, configs[4]", "T": ST, "B": SB, "H": SH},
        "fwd_ms": round(fwd_ms, 5), "bwd_ms": round(bwd_ms, 5),
        "fwd_GBps": round(fwd_b / fwd_ms / 1e6, 1), "bwd_GBps": round(bwd_b / bwd_ms / 1e6, 1),
        "GBps": round((fwd_b + bwd_b) / (fwd_ms + bwd_ms) / 1e6, 1),
        "roofline": {"bound": "hbm", "achieved": round((fwd_b + bwd_b) / (fwd_ms + bwd_ms) / 1e6, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round((fwd_b + bwd_b) / (fwd_ms + bwd_ms) / 1e6 / HBM_PEAK_GBS, 4),
                     "traffic": (measured_traffic("scan_fwd_kernel")[0] or 0)
                     + (measured_traffic("scan_bwd_kernel")[0] or 0) or None,
                     "traffic_source": measured_traffic("scan_fwd_kernel")[1],
                     "algorithmic_bytes": fwd_b + bwd_b},
        # the target's own byte count stores c at every step (24 + 40 B per element); these
        # kernels keep c every 8th step, so the same time moves fewer bytes
        "target_bytes_64B": 64 * n,
        "target_ms": round(64 * n / (0.5 * HBM_PEAK_GBS) / 1e6, 4),
    }
    log(f"scan fwd {fwd_ms:.4f} ms ({res['fwd_GBps']} GB/s) bwd {bwd_ms:.4f} ms ({res['bwd_GBps']} GB/s)")
    return res


# configs[0..4] of BASELINE.json (configs[1] in both modes), the two shapes of the
# reference's published table (README.md:73-79) that no config covers, configs[4] with the
# module in bf16 (16-bit input projection), and configs[2] / configs[4] with the module in
# fp64 (the fp64 kernels): (name, T, B, D, H, parallel, a, dtype)
MODE_CONFIGS = [
    ("configs[0]", 32, 16, 64, 128, False, 1e-4, torch.float32),
    ("configs[1]", 128, 32, 256, 256, False, 1e-4, torch.float32),
    ("configs[1]", 128, 32, 256, 256, True, 1e-4, torch.float32),
    ("configs[2] a~U(0,0.5)", 256, 32, 256, 512, False, None, torch.float32),
    ("configs[3]", 64, 32, 1024, 2048, False, 1e-4, torch.float32),
    ("README.md:75 shape", 64, 32, 128, 256, False, 1e-4, torch.float32),
    ("README.md:78 shape", 64, 32, 512, 1024, False, 1e-4, torch.float32),
    ("configs[4]", 4096, 16, 256, 1024, True, 0.0, torch.float32),
    ("configs[4] bf16 module", 4096, 16, 256, 1024, True, 0.0, torch.bfloat16),
    ("configs[2] fp64 module", 256, 32, 256, 512, False, 1e-4, torch.float64),
    ("configs[4] fp64 module", 4096, 16, 256, 1024, True, 0.0, torch.float64),
]


def bench_modes(args):
    """Every configured shape in its mode(s): one graph replay of fwd+bwd per step,
    same recipe as the headline (seed 0, module on CPU, x ~ N(0,1), loss out.sum())."""
    from prlstm_amd import HeadStartLSTM
    from prlstm_amd.graph import GraphedTrainStep
    dev = torch.device("cuda", 0)
    res = []
    for name, t, b, d, h, par, a, dt in MODE_CONFIGS:
        if args.mode_filter and not any(f in name for f in args.mode_filter.split(",")):
            continue
        torch.manual_seed(0)
        m = HeadStartLSTM(d, h, a_init=0.0 if a is None else a, parallel=par)
        if a is None:  # the configs[2] variant: a drawn right after init
            with torch.no_grad():
                m.a.copy_(torch.rand(4) * 0.5)
        x = torch.randn(t, b, d).to(dt)
        m = m.to(dev, dt)
        step = GraphedTrainStep(m, x.to(dev))
        for _ in range(3):
            step.step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = max(5, args.steps // 2)
        e0.record()
        for _ in range(n):
            step.step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        flops = executed_flops(t, b, d, h, par)
        res.append({"config": name, "mode": "parallel" if par else "recurrent", "dtype": str(dt).split(".")[-1],
                    "T": t, "B": b, "D": d, "H": h,
                    "ms_per_step": round(ms, 4), "timesteps_batch_per_s": round(t * b / ms * 1e3, 1),
                    "executed_tflops": round(flops / ms / 1e9, 2)})
        log(f"mode {name} {'parallel' if par else 'recurrent'}: {ms:.4f} ms/step")
        del step, m
        torch.cuda.empty_cache()
    return res


def _split_products_state():
    from prlstm_amd import _lib
    prev = _lib.set_split_products(1)
    _lib.set_split_products(prev)
    return prev


def _host_info():
    """CPU model, cgroup CPU quota and torch's thread settings of this host."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), model)
    except OSError:
        pass
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota = f.read().strip()
    except OSError:
        quota = None
    info = [l.strip() for l in torch.__config__.parallel_info().splitlines() if l.strip() and not l.startswith("-")]
    return model, quota, info[:8]


def _cpu_steps(m, x, budget_s, min_n, max_n):
    """Median seconds of zero_grad + forward + out.sum().backward() over min_n..max_n steps
    after one warm-up, stopping once budget_s seconds are spent (at least min_n steps)."""
    def one():
        m.zero_grad(set_to_none=True)
        t0 = time.perf_counter()
        out, _ = m(x)
        out.sum().backward()
        return time.perf_counter() - t0

    first = one()
    times, spent = [], first
    while len(times) < min_n or (len(times) < max_n and spent + statistics.median(times) <= budget_s):
        times.append(one())
        spent += times[-1]
    return statistics.median(times), len(times), first


def bench_cpu(args):
    """The reference torch backend restated (oracle/), fp32 on every core of this process's
    CPU affinity (configs[2] recurrent), and the parallel-mode restatement (_parallel.py)
    at configs[1] and configs[4] beside it."""
    from oracle.hsl_oracle import RefHeadStartLSTM
    affinity = len(os.sched_getaffinity(0))
    cores = min(affinity, args.cpu_threads) if args.cpu_threads else affinity
    torch.set_num_threads(cores)
    model, quota, pinfo = _host_info()
    torch.manual_seed(0)
    m = RefHeadStartLSTM(D, H, a_init=1e-4)
    x = torch.randn(T, B, D)
    med, n, first = _cpu_steps(m, x, args.cpu_seconds, 1, 15)
    log(f"cpu baseline: {cores} threads ({model}), median {med:.3f} s over {n} steps (warm-up {first:.3f} s)")
    res = {"value": round(T * B / med, 1), "unit": "timesteps·batch/s", "cores": cores,
           "kind": "port", "ms_per_step": round(med * 1e3, 2),
           "sample": f"configs[2] fwd+bwd (out.sum() loss), fp32, torch CPU restatement of "
                     f"_torch.py, median of {n} full steps after 1 warm-up; like _torch.py:162 it "
                     f"always forms dx (a [T*B,4H]x[4H,D] product the GPU step skips, x being data)",
           "affinity_cores": affinity, "cpu_model": model, "cgroup_cpu_max": quota, "torch_parallel_info": pinfo}
    if not args.no_cpu_parallel:
        par = []
        for name, t, b, d, h, nmin in (("configs[1]", 128, 32, 256, 256, 5), ("configs[4]", 4096, 16, 256, 1024, 3)):
            torch.manual_seed(0)
            mp = RefHeadStartLSTM(d, h, a_init=1e-4 if name == "configs[1]" else 0.0, parallel=True)
            xp = torch.randn(t, b, d)
            pmed, pn, pfirst = _cpu_steps(mp, xp, 0.0, nmin, nmin)
            log(f"cpu parallel {name}: median {pmed:.3f} s over {pn} steps (warm-up {pfirst:.3f} s)")
            par.append({"config": name, "mode": "parallel", "T": t, "B": b, "D": d, "H": h,
                        "ms_per_step": round(pmed * 1e3, 2), "timesteps_batch_per_s": round(t * b / pmed, 1),
                        "sample": f"median of {pn} full fwd+bwd steps after 1 warm-up, torch CPU restatement "
                                  f"of _parallel.py:21-74"})
            del mp, xp
        res["parallel_mode"] = par
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="bound on the CPU baseline sample (seconds of CPU work)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the CPU baseline (default 0: every core of the CPU affinity)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-cpu-parallel", action="store_true", help="skip the parallel-mode CPU baseline")
    ap.add_argument("--no-scan", action="store_true")
    ap.add_argument("--no-modes", action="store_true", help="skip the per-config table of both modes")
    ap.add_argument("--mode-filter", default="",
                    help="run only the modes rows whose name contains one of these comma-separated "
                         "strings (e.g. 'configs[3],README.md:78' for a kernel trace of those steps)")
    ap.add_argument("--no-split-off", action="store_true",
                    help="skip the headline step with the split products switched off")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(each box has one MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    ms, wall_ms, kern, path, fused, split_off = bench_gpu(args)
    scan = None if args.no_scan else bench_scan(args)
    modes = None if args.no_modes else bench_modes(args)
    cpu = None if args.no_cpu else bench_cpu(args)

    step_flops = float(executed_flops(T, B, D, H, False))  # fwd+bwd products executed (no dx)
    rec_flops = 2.0 * T * B * H * 4 * H               # recurrent product of one direction
    # per-launch FLOPs: the backward kernel also accumulates dW_hh (and dW_ih) when fused,
    # the forward kernel computes the input projection when no separate launch ran
    proj_flops = 2.0 * T * B * 4 * H * D               # input projection, inside rec_fwd when fused
    kflops = {"rec_fwd": rec_flops + (proj_flops if "input_proj" not in kern else 0.0),
              "step_fwd": rec_flops, "step_bwd": rec_flops,
              "rec_bwd": rec_flops * (1 + (fused >= 1)) + (2.0 * T * B * 4 * H * D if fused == 2 else 0.0)}
    if "rec_fwd" in kern or "rec_bwd" in kern:
        name = max((k for k in ("rec_fwd", "rec_bwd") if k in kern), key=lambda k: kern[k])
        kname = {"rec_fwd": "rec_fwd_persistent", "rec_bwd": "rec_bwd_persistent"}[name]
    else:
        name = max((k for k in ("step_fwd", "step_bwd") if k in kern), key=lambda k: kern[k])
        kname = name + " (per-step launches)"
    kms = kern[name]
    achieved = kflops[name] / (kms * 1e-3) / 1e12
    value = T * B / (ms * 1e-3)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "timesteps·batch/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "HeadStartLSTM recurrent fwd+bwd (configs[2]), one hipGraph replay per step",
                   "T": T, "B": B, "D": D, "H": H, "a": 1e-4, "loss": "out.sum()",
                   "recurrent_path": {1: "per-step", 2: "persistent"}.get(path, path)},
        "roofline": {"bound": "mfma", "kernel": kname, "achieved": round(achieved, 3),
                     "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_F32_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(kname)[0] if kname.endswith("persistent") else None,
                     "traffic_source": measured_traffic(kname)[1] if kname.endswith("persistent") else None,
                     "kernel_ms": round(kms, 5), "flops_per_launch": kflops[name]},
        # per-step latency of the recurrence: launch time / T, beside the time one step's
        # recurrent product (2*B*4H*H FLOPs) takes at the fp32 MFMA peak
        "recurrence": {
            **{f"{k}_us_per_step": round(kern[k] * 1e3 / T, 4) for k in ("rec_fwd", "rec_bwd", "step_fwd", "step_bwd")
               if k in kern},
            "floor_us_per_step": round(rec_flops / T / (MFMA_F32_PEAK_TFLOPS * 1e12) * 1e6, 4),
            "floor_note": "2*B*4H*H FLOPs of one step's recurrent product at the fp32 MFMA peak; "
                          "rec_fwd also runs the input projection (2*B*4H*D per step) and rec_bwd "
                          "the dW_hh and dW_ih products (2*B*4H*(H+D) per step)"},
        "step_tflops": round(step_flops / (ms * 1e-3) / 1e12, 3),
        "step_flops": step_flops,
        "kernels_ms": {k: round(v, 5) for k, v in kern.items()},
        "wall_ms_per_step": round(wall_ms, 5),
        "scan": scan,
        "modes": modes,
        # hsl_set_split_products during the run (the library default is on).  On, the
        # headline step's input projection (inside rec_fwd) and its dW_hh / dW_ih products
        # (inside rec_bwd) run as exact three-piece bf16 splits, six piece products with
        # fp32 accumulation, and so do the modes table's large separate products; the
        # recurrent h W_hh^T and dg W_hh products stay on the fp32 instruction.  The same
        # step with the switch off (every product on the fp32 instruction) is beside it.
        "split_products": bool(_split_products_state()),
        "fused_products": {
            "arithmetic": "split_bf16x6" if _split_products_state() else "fp32",
            "note": "input projection (rec_fwd) and dW_hh/dW_ih (rec_bwd) of the headline step; "
                    "split_bf16x6 = each fp32 operand split exactly into three bf16 pieces, the six "
                    "largest piece products on bf16 MFMA with fp32 accumulation; the recurrent "
                    "products are fp32 MFMA either way"},
        "split_products_off": split_off,
        "cpu_baseline": cpu,
    }
    if cpu:
        line["speedup_vs_cpu"] = round(value / cpu["value"], 1)
        for p in cpu.get("parallel_mode", []):  # GPU step of the same config from the modes table
            g = next((r for r in modes or [] if r["config"] == p["config"] and r["mode"] == "parallel"
                      and r["dtype"] == "float32"), None)
            if g:
                p["gpu_ms_per_step"] = g["ms_per_step"]
                p["speedup_vs_cpu"] = round(p["ms_per_step"] / g["ms_per_step"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
