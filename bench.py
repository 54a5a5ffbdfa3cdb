"""Benchmark of the fused Cheby-RKV forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload W] [--no-others]

Default workload: BASELINE configs[1] ("headline"): B=4, S=16384, D=512
(H=8, hd=64), K=8, fp32, static per-head lambda.  One step = one pass of
the fused operator over one batch held in HBM.  Inputs rotate over 4
buffer sets (>1 GB) so the 256 MB Infinity Cache cannot serve them.
Without --workload the run then times every other workload of
synthetic.CONFIGS the same way (100 warm-up and 100 timed steps each, on
inputs drawn on the device, two buffer sets where x exceeds 256 MB) and
reports them under ``other_workloads``; --workload W times W only.

Prints ONE JSON line (rank 0).  The timed region is exactly K steps
back to back between two HIP events on the stream the kernels run on.
``roofline`` prices the fused operator against HBM: achieved = algorithmic
bytes per launch (every input read once, every output written once) / the
average launch duration over that region (a step is one launch, or one per
chunk for the streaming workload; the TTT step's two small merge kernels,
~2% of it, are counted in).  ``traffic`` is the HBM bytes per launch of the
main kernel measured with rocprofv3's TCC->EA read and write request
counters, by request size (profiles/hbm_traffic.json, written by
``--pmc-summary``).  ``cpu_baseline`` times the CPU restatement of the
reference's PyTorch path (oracle/reference_form.py) on this host's cores:
for the forward workloads BASELINE configs[0] and the workload in full,
otherwise one batch row; median of 3 runs after a warm-up.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from orthossm_amd import cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt  # noqa: E402
from orthossm_amd.ops import v10_chunked_ttt  # noqa: E402
from orthossm_amd.synthetic import CONFIGS, baseline_damping, baseline_lambda, make_config_inputs  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "Clenshaw+EMA tokens/s and HBM GB/s (% of peak) at B=4 S=16K D=512, 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def algorithmic_bytes(cfg) -> int:
    """Compulsory bytes of one pass: x read + out written + coeffs, damping,
    lambda, g (dynamic), EMA state in/out, grad (TTT).  Backward: x, the
    saved output and dL/dout read, dL/dx written, coeffs read, dL/dc
    written, dL/d ema_final read and dL/d ema_init written."""
    esz = 2 if cfg.dtype == torch.bfloat16 else 4
    n = cfg.B * cfg.S * cfg.D
    total = (4 if cfg.bwd else 2) * n * esz
    total += cfg.B * cfg.H * cfg.K * cfg.hd * 4          # coeffs
    total += 2 * cfg.H * 4                               # damping, lambda
    if cfg.dynamic:
        total += cfg.B * cfg.S * cfg.H * 4               # g [B,S,H]
    launches = cfg.S // cfg.chunk if cfg.chunk else 1
    total += 2 * cfg.B * cfg.D * 4 * launches            # ema_init in, ema_final out per launch
    if cfg.ttt or cfg.bwd:
        total += cfg.B * cfg.H * cfg.K * cfg.hd * 4      # grad
    if cfg.v10:
        total += 3 * cfg.B * cfg.H * cfg.K * cfg.hd * 4  # momentum in, coeffs and momentum out
        total -= 2 * cfg.B * cfg.D * 4 * launches        # no EMA state arguments
        total += 8 * 256 * 4                             # LUT
    return total


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (the machine type if absent)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.machine()


def _median_time(run, reps: int = 3) -> float:
    """Median wall time of ``reps`` runs after one untimed warm-up run."""
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline(cfg):
    """The CPU restatement of the reference's PyTorch path on this host's
    cores, median of 3 runs after one warm-up.  Forward workloads: BASELINE
    configs[0] in full and the workload itself in full (the forward
    workloads at most 2^26 elements, a few seconds per run); the other
    workloads: one batch row of at most 16384 tokens."""
    from oracle import reference_form as RF

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    inp = make_config_inputs(cfg)
    forward_only = not (cfg.v10 or cfg.bwd or cfg.ttt)
    full = forward_only and cfg.B * cfg.S * cfg.D <= (1 << 26)
    if full:
        x, c, lam, g = inp["x"].float(), inp["coeffs"], inp["lam"], inp["g"]
        S = cfg.S
    else:
        S = min(cfg.S, 16384)
        x = inp["x"][0:1, :S].float().contiguous()
        c = inp["coeffs"][0:1]
        lam, g = inp["lam"], None if inp["g"] is None else inp["g"][0:1, :S]
    rows = x.shape[0]
    if cfg.v10:
        from oracle import v10_full as V
        xs1, cs1 = x.numpy(), c.double().numpy()
        run = lambda: V.v10_full(xs1, cs1, 0.0 * cs1, n_heads=cfg.H, chunk_size=cfg.v10)   # noqa: E731
        what = "the full path restated in float64 numpy (oracle/v10_full.py), LUT series"
    elif cfg.bwd:
        out, _ = RF.forward(x, c, inp["damping"], lam)
        go = torch.randn(x.shape, generator=torch.Generator().manual_seed(1))
        run = lambda: RF.backward(x, c, inp["damping"], lam, out, go)      # noqa: E731
        what = "masked reverse EMA loop + autograd through basis+einsum+tanh (oracle/reference_form.py)"
    else:
        run = lambda: RF.forward(x, c, inp["damping"], lam)                # noqa: E731
        what = "basis+einsum+tanh and per-head EMA loop (oracle/reference_form.py)"
        if g is not None:
            what += "; static lambda (the loop's cost does not depend on it)"
    t = _median_time(run)
    tokens = rows * S
    res = {
        "value": tokens / t,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{'the whole workload' if full else 'one batch row of the workload'}: B={rows} S={S} "
                   f"D={cfg.D} K={cfg.K} fp32, {what}, median of 3 after a warm-up"),
        "seconds": t,
        "gbs": algorithmic_bytes(cfg) / (cfg.B * cfg.S) * tokens / t / 1e9,
        "cpu": cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }
    if forward_only and cfg.name != "cpu_ref":
        # BASELINE configs[0] (B=1 S=2048 D=512), the reference's CPU-runnable case
        c0 = CONFIGS["cpu_ref"]
        i0 = make_config_inputs(c0)
        t0 = _median_time(lambda: RF.forward(i0["x"], i0["coeffs"], i0["damping"], i0["lam"]))
        res["configs0"] = {"value": c0.B * c0.S / t0, "unit": "tokens/s", "seconds": t0,
                           "sample": "BASELINE configs[0] in full: B=1 S=2048 D=512 K=8 fp32, median of 3 after "
                                     "a warm-up"}
    return res


def measured_traffic(workload: str):
    """HBM bytes per launch (read + write) from profiles/hbm_traffic.json."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f).get(workload)
        return None if entry is None else entry["bytes"]
    except (OSError, ValueError, KeyError):
        return None


# The auxiliary kernels of a step (the TTT's per-launch coefficient table,
# tile merges / reductions).
AUX_KERNELS = ("ttt_mono_prep", "ttt_merge", "ttt_finalize", "bwd_reduce")


def main_kernel(cfg) -> str:
    """Name fragment of the workload's dominant kernel (the backward
    workload also runs forward launches to produce its saved outputs)."""
    if cfg.v10:
        return "v10_chunked_kernel"
    if cfg.bwd:
        return "cheby_ema_bwd_kernel"
    if cfg.ttt:
        return "cheby_ema_ttt_kernel"
    return "cheby_ema_fwd_kernel"
READ_COUNTERS = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_BUBBLE_sum")
WRITE_COUNTERS = ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum")


def _dispatch_counters(path: str):
    """{dispatch id: (kernel name, {counter: value})} from a rocprofv3 --pmc
    output directory (rocpd SQLite databases or counter_collection.csv)."""
    import csv
    import glob
    import sqlite3
    out = {}
    files = [path] if os.path.isfile(path) else glob.glob(os.path.join(path, "**", "*"), recursive=True)
    for fn in files:
        if fn.endswith("_results.db"):
            con = sqlite3.connect(fn)
            rows = con.execute("select dispatch_id, kernel_name, counter_name, value from counters_collection")
            for did, kn, cn, v in rows:
                out.setdefault((fn, did), (kn, {}))[1][cn] = float(v)
            con.close()
        elif fn.endswith("counter_collection.csv"):
            with open(fn) as f:
                for r in csv.DictReader(f):
                    key = (fn, int(r["Dispatch_Id"]))
                    out.setdefault(key, (r["Kernel_Name"], {}))[1][r["Counter_Name"]] = float(r["Counter_Value"])
    return dict(sorted(out.items()))


def read_bytes(c: dict) -> float:
    """HBM read bytes of one dispatch on gfx950: every TCC->EA read request
    that is not a 32-byte one moves one 128-byte line (TCC_BUBBLE, which
    FETCH_SIZE's formula takes as the 128-byte count, stays 0 on this chip,
    so FETCH_SIZE counts such a request as 64 bytes).  Checked on plain
    device copies of known size (copy_read_ratio)."""
    r, r32 = c["TCC_EA0_RDREQ_sum"], c["TCC_EA0_RDREQ_32B_sum"]
    return 128.0 * (r - r32) + 32.0 * r32


def write_bytes(c: dict) -> float:
    """HBM write bytes of one dispatch: 64-byte and 32-byte TCC->EA write
    requests (WRITE_SIZE's formula); checked on the same copies
    (copy_write_ratio)."""
    w, w64 = c["TCC_EA0_WRREQ_sum"], c["TCC_EA0_WRREQ_64B_sum"]
    return 64.0 * w64 + 32.0 * (w - w64)


def pmc_summary(read_path: str, write_path: str, workload: str) -> dict:
    """HBM bytes per launch of the dominant kernel from two rocprofv3 --pmc
    runs of ``bench.py --calibrate-copy --workload W``, one with the read
    request counters (READ_COUNTERS), one with the write ones
    (WRITE_COUNTERS).  The run's last 5 plain device copies (one x buffer,
    size known) validate the byte formulas: their ratios of measured to
    known bytes are stored with the result, nothing is scaled by them.
    Stored under ``workload`` in profiles/hbm_traffic.json."""
    cfg = CONFIGS[workload]
    copy_bytes = cfg.B * cfg.S * cfg.D * (2 if cfg.dtype == torch.bfloat16 else 4)
    launches = cfg.S // cfg.chunk if cfg.chunk else 1
    out = {"method": "TCC->EA request counters: reads 128 B per non-32-byte request, writes 64/32 B per request"}
    for key, path, fn, names in (("read", read_path, read_bytes, READ_COUNTERS),
                                 ("write", write_path, write_bytes, WRITE_COUNTERS)):
        disp = list(_dispatch_counters(path).values())
        main = [fn(c) for k, c in disp if main_kernel(cfg) in k]
        aux = [fn(c) for k, c in disp if any(m in k for m in AUX_KERNELS)]
        copies = [fn(c) for k, c in disp if "copyBuffer" in k][-5:]
        if not main or len(copies) < 5:
            raise SystemExit(f"pmc_summary: {path} lacks {names} for the kernel or the 5 calibration copies")
        per = sum(main) / len(main)
        out[f"{key}_bytes"] = per
        out[f"{key}_dispatches"] = len(main)
        # auxiliary kernels of a step, per launch of the main kernel
        out[f"{key}_aux_bytes"] = sum(aux) / len(main) if aux else 0.0
        out[f"copy_{key}_ratio"] = (sum(copies) / len(copies)) / copy_bytes
        out[f"{key}_counters_mean"] = {n: sum(c.get(n, 0.0) for k, c in disp if main_kernel(cfg) in k) / len(main)
                                       for n in names}
    out["bytes"] = out["read_bytes"] + out["write_bytes"]
    out["step_bytes"] = out["bytes"] + out["read_aux_bytes"] + out["write_aux_bytes"]
    out["algorithmic_bytes"] = algorithmic_bytes(cfg) / launches
    out["ratio"] = out["bytes"] / out["algorithmic_bytes"]
    try:
        with open(TRAFFIC_FILE) as f:
            table = json.load(f)
    except (OSError, ValueError):
        table = {}
    table[workload] = out
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(table, f, indent=1, sort_keys=True)
        f.write("\n")
    return out


def device_inputs(cfg, dev, seed: int = 0):
    """The distributions of synthetic.make_inputs drawn on the device (fast
    for the large configs; values differ from the CPU draw, timings do not
    depend on them)."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    k = torch.arange(cfg.K, dtype=torch.float32, device=dev).view(1, 1, cfg.K, 1)
    return {
        "x": torch.randn(cfg.B, cfg.S, cfg.D, device=dev, generator=gen).to(cfg.dtype),
        "coeffs": torch.randn(cfg.B, cfg.H, cfg.K, cfg.hd, device=dev, generator=gen) / (k + 1.0),
        "damping": baseline_damping(cfg.H).to(dev),
        "lam": baseline_lambda(cfg.H).to(dev),
        "g": (torch.rand(cfg.B, cfg.S, cfg.H, device=dev, generator=gen) * 2.0 - 1.0) if cfg.dynamic else None,
    }


class Workload:
    """Device buffers of one workload (inputs and outputs rotating over
    ``sets`` buffer sets) and its step: one pass of the operator over one
    batch (one launch per chunk for chunked workloads)."""

    def __init__(self, cfg, dev, sets: int, inp: dict):
        self.cfg, self.sets = cfg, sets
        x0 = inp["x"]
        self.c, self.damp, self.lam, self.g = inp["coeffs"], inp["damping"], inp["lam"], inp["g"]
        self.xs = [x0] + [x0.clone() for _ in range(sets - 1)]
        self.outs = [torch.empty_like(x0) for _ in range(sets)]
        # EMA state: every launch reads ema_init and writes ema_final; chunks
        # ping-pong between two state buffers.
        self.state0 = torch.zeros(cfg.B, cfg.D, device=dev)
        self.states = [torch.empty_like(self.state0), torch.empty_like(self.state0)]
        self.grad = torch.empty(cfg.B, cfg.H, cfg.K, cfg.hd, device=dev) if (cfg.ttt or cfg.bwd) else None
        if cfg.bwd:
            # Saved forward outputs and dL/dout per buffer set; dL/dx goes to gxs.
            gen = torch.Generator(device=dev).manual_seed(1)
            for x, out in zip(self.xs, self.outs):
                cheby_ema_forward(x, self.c, self.damp, self.lam, g=self.g, out=out)
            self.gos = [torch.randn(x0.shape, device=dev, generator=gen) for _ in range(sets)]
            self.gxs = [torch.empty_like(x0) for _ in range(sets)]
            torch.cuda.synchronize()
        self.mom = torch.zeros_like(self.c) if cfg.v10 else None

    def step(self, i):
        cfg, c, damp, lam, g = self.cfg, self.c, self.damp, self.lam, self.g
        x, out = self.xs[i % self.sets], self.outs[i % self.sets]
        if cfg.v10:
            v10_chunked_ttt(x, c, self.mom, n_heads=cfg.H, chunk_size=cfg.v10)
        elif cfg.bwd:
            cheby_ema_backward(x, c, damp, lam, out, self.gos[i % self.sets], g=g, grad_state=self.state0,
                               grad_x_out=self.gxs[i % self.sets], grad_coeffs_out=self.grad,
                               grad_init_out=self.states[0])
        elif cfg.ttt:
            cheby_ema_ttt(x, c, damp, lam, g=g, out=out, ema_init=self.state0, state_out=self.states[0],
                          grad_out=self.grad)
        elif cfg.chunk:
            prev = self.state0
            for n, t0 in enumerate(range(0, cfg.S, cfg.chunk)):
                cheby_ema_forward(x[:, t0:t0 + cfg.chunk], c, damp, lam, ema_init=prev,
                                  out=out[:, t0:t0 + cfg.chunk], state_out=self.states[n % 2])
                prev = self.states[n % 2]
        else:
            cheby_ema_forward(x, c, damp, lam, g=g, out=out, ema_init=self.state0, state_out=self.states[0])


def time_steps(step, steps: int, warmup: int, stream) -> float:
    """Milliseconds per step: ``warmup`` untimed steps, then exactly
    ``steps`` steps back to back between two events on the launch stream,
    nothing else enqueued in between."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(steps):
        step(i)
    t_end.record(stream)
    torch.cuda.synchronize()
    return t_start.elapsed_time(t_end) / steps


def launch_figures(cfg, ms_per_step: float) -> dict:
    """Tokens/s and the HBM roofline of the average launch of a step."""
    launches = cfg.S // cfg.chunk if cfg.chunk else 1
    algo_launch = algorithmic_bytes(cfg) / launches
    kernel_ms = ms_per_step / launches
    gbs = algo_launch / (kernel_ms * 1e-3) / 1e9
    return {"value": cfg.B * cfg.S / (ms_per_step * 1e-3), "achieved": gbs, "frac": gbs / HBM_PEAK_GBS,
            "algorithmic_bytes": algo_launch, "launches_per_step": launches, "kernel_ms_mean": kernel_ms}


def other_workloads(skip: str, dev, stream, steps: int, warmup: int) -> dict:
    """The other BASELINE workloads, each timed as the main one is (its own
    warm-up, then ``steps`` steps between two events), on inputs drawn on
    the device, at most two buffer sets above 256 MB of x."""
    res = {}
    for name, cfg in CONFIGS.items():
        if name in (skip, "cpu_ref"):
            continue
        esz = 2 if cfg.dtype == torch.bfloat16 else 4
        sets = 4 if cfg.B * cfg.S * cfg.D * esz <= (256 << 20) else 2
        W = Workload(cfg, dev, sets, device_inputs(cfg, dev))
        ms = time_steps(W.step, steps, warmup, stream)
        f = launch_figures(cfg, ms)
        res[name] = {
            "ms_per_step": ms, "value": f["value"], "unit": "tokens/s",
            "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
            "roofline": {"bound": "hbm", "achieved": f["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": f["frac"], "traffic": measured_traffic(name),
                         "algorithmic_bytes": f["algorithmic_bytes"],
                         "launches_per_step": f["launches_per_step"], "kernel_ms_mean": f["kernel_ms_mean"]},
            "steps": steps, "warmup": warmup, "sets": sets,
            "config": workload_label(cfg),
        }
        del W
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return res


def workload_label(cfg) -> str:
    return (f"BASELINE {cfg.name}: B={cfg.B} S={cfg.S} D={cfg.D} H={cfg.H} hd={cfg.hd} K={cfg.K} "
            f"{'bf16' if cfg.dtype == torch.bfloat16 else 'fp32'}"
            f"{' dynamic-lambda' if cfg.dynamic else ''}{' +TTT-grad' if cfg.ttt else ''}"
            f"{' backward (dL/dx, dL/dc, dL/d ema_init)' if cfg.bwd else ''}"
            f"{f' full path: chunks of {cfg.v10} with Lion, LUT series' if cfg.v10 else ''}"
            f"{f' as {cfg.S // cfg.chunk} chunks with carry' if cfg.chunk else ''}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Defaults: 500 warm-up steps (the GPU reaches steady clocks only after
    # tens of milliseconds of load; with 10 the headline reads ~5% slower)
    # and 500 timed steps (a few seconds at most for any workload).
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--workload", default=None, choices=sorted(CONFIGS),
                    help="time this workload only (default: the headline, then each other workload briefly)")
    ap.add_argument("--no-others", action="store_true",
                    help="without --workload: time the headline only")
    ap.add_argument("--sets", type=int, default=4, help="rotating input/output buffer sets")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the timed steps, run 5 plain device copies of one x buffer (reads and writes "
                         "B*S*D elements each) as the reference kernel for HBM counter scaling")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("READ_RUN", "WRITE_RUN"),
                    help="no GPU work: turn two rocprofv3 --pmc outputs of 'bench.py --calibrate-copy "
                         "--workload W' (read request counters, then write request counters; see "
                         "READ_COUNTERS / WRITE_COUNTERS) into HBM bytes per launch for W, stored in "
                         "profiles/hbm_traffic.json")
    args = ap.parse_args()
    others = args.workload is None and not args.no_others and not args.calibrate_copy
    args.workload = args.workload or "headline"
    if args.pmc_summary:
        print(json.dumps({args.workload: pmc_summary(*args.pmc_summary, args.workload)}, indent=1))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the hot path shards over batch/heads with no "
              "communication (batch rows and heads are independent). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    cfg = CONFIGS[args.workload]
    dev = torch.device("cuda", 0)
    inp = make_config_inputs(cfg)
    W = Workload(cfg, dev, args.sets, {k: (v.to(dev) if v is not None else None) for k, v in inp.items()})
    del inp
    xs, outs, step = W.xs, W.outs, W.step
    stream = torch.cuda.current_stream(dev)
    ms_per_step = time_steps(step, args.steps, args.warmup, stream)
    # Spread of single steps (a second, separately timed pass with an event
    # pair around every step; each pair adds a few microseconds of dispatch
    # overhead, so these read slightly high).
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.steps):
        ev[i][0].record(stream)
        step(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) for a, b in ev)
    # Achievable copy bandwidth on this box, for reference: plain device
    # copies of one x buffer into an output buffer (the same bytes read and
    # written as the forward at this shape), rotating over the buffer sets.
    n_copy = 20
    for i in range(3):
        outs[i % args.sets].copy_(xs[(i + 1) % args.sets])
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    c0.record(stream)
    for i in range(n_copy):
        outs[i % args.sets].copy_(xs[(i + 1) % args.sets])
    c1.record(stream)
    torch.cuda.synchronize()
    copy_ms = c0.elapsed_time(c1) / n_copy
    copy_gbs = 2 * xs[0].numel() * xs[0].element_size() / (copy_ms * 1e-3) / 1e9
    # Chunked workloads launch one kernel per chunk: a copy of one chunk's
    # bytes (consecutive slices of the buffers, as the chunks are) is the
    # like-for-like reference for a launch of that size.
    chunk_copy_gbs = None
    if cfg.chunk:
        n_sl = cfg.S // cfg.chunk

        def copy_chunk(i):
            t0 = (i % n_sl) * cfg.chunk
            outs[i % args.sets][:, t0:t0 + cfg.chunk].copy_(xs[(i + 1) % args.sets][:, t0:t0 + cfg.chunk])

        for i in range(n_sl):
            copy_chunk(i)
        torch.cuda.synchronize()
        c0.record(stream)
        for i in range(10 * n_sl):
            copy_chunk(i)
        c1.record(stream)
        torch.cuda.synchronize()
        chunk_bytes = 2 * cfg.B * cfg.chunk * cfg.D * xs[0].element_size()
        chunk_copy_gbs = chunk_bytes / (c0.elapsed_time(c1) / (10 * n_sl) * 1e-3) / 1e9
    f = launch_figures(cfg, ms_per_step)
    achieved_gbs = f["achieved"]

    res = {
        "metric": METRIC if args.workload == "headline" else
        f"Clenshaw+EMA {'backward ' if cfg.bwd else ''}{'full path (online TTT + Lion) ' if cfg.v10 else ''}"
        f"tokens/s, workload {cfg.name}",
        "value": f["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded N(0,1) inputs, c_k ~ N(0,1/(k+1)^2))",
        "config": {
            "workload": workload_label(cfg),
            "B": cfg.B, "S": cfg.S, "D": cfg.D, "H": cfg.H, "K": cfg.K,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": f["frac"],
            "traffic": measured_traffic(args.workload),
            "algorithmic_bytes": f["algorithmic_bytes"],
            "launches_per_step": f["launches_per_step"],
            "kernel_ms_mean": f["kernel_ms_mean"],
            "step_ms_evented_p10": per[len(per) // 10],
            "step_ms_evented_median": per[len(per) // 2],
            "step_ms_evented_p90": per[(9 * len(per)) // 10],
            "copy_gbs_measured": copy_gbs,
            "frac_of_copy": achieved_gbs / copy_gbs,
        },
    }
    if chunk_copy_gbs is not None:
        res["roofline"]["copy_gbs_one_chunk"] = chunk_copy_gbs
        res["roofline"]["frac_of_chunk_copy"] = achieved_gbs / chunk_copy_gbs
    if args.calibrate_copy:
        for i in range(5):
            outs[i % args.sets].copy_(xs[(i + 1) % args.sets])
        torch.cuda.synchronize()
        res["copy_calibration_bytes_each_way"] = xs[0].numel() * xs[0].element_size()
    if others:
        # Each other BASELINE workload timed in the same run (100 warm-up
        # and 100 timed steps each), so that one run records all of them.
        del W, xs, outs, step
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        res["other_workloads"] = other_workloads(args.workload, dev, stream, steps=100, warmup=100)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
