"""Benchmark for the MI355X quantized decode hot path (one GPU).

Metric: quant GEMV HBM GB/s (% of peak) + decode tok/s, 1.7B-shape
nf4g128.  A "step" here is one pass of the config-4 GEMV sweep: nf4g128 and b6
bit-plane GEMVs on 14336x4096 and 4096x14336 at batch 1, inputs resident in HBM.
Each timed launch reads a different copy of the weights (>256 MB cycled) so the
256 MB Infinity Cache cannot serve them.  Durations come from HIP events recorded on
the stream the kernels run on.

Prints ONE JSON line (see the keys below).  --gpus N > 1 is refused: this build and
its measurements are single-GPU.
"""
import argparse
import json
import os
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kronos-2t_amd"))

HBM_PEAK_GBS = 8000.0
SEED = 20261201


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="", help="comma list of case names to run (profiling)")
    return ap.parse_args()


def gemv_bytes(m_bytes, rows, cols, ntok, bitplane):
    nc = cols // 64
    act = ntok * (cols + 4 * nc + (4 * nc if bitplane else 0))
    return m_bytes + act + ntok * 4 * rows


class GemvCase:
    """One GEMV shape/format with enough weight copies to exceed the Infinity Cache."""

    def __init__(self, ctx, torch, name, fmt, rows, cols, ntok=1):
        import k2t
        self.name, self.fmt, self.rows, self.cols, self.ntok = name, fmt, rows, cols, ntok
        W = k2t.synth_normal(SEED + rows * 3 + cols, rows * cols, 0.02).reshape(rows, cols)
        if fmt == "b6":
            pair, tail = k2t.compile_bipolar(W, 6)
            self.cb = None
        else:
            cb, mu, pair, tail = k2t.compile_nf4(W, 2)
            self.cb = cb
        del W
        self.stream_bytes = pair.size + tail.size + (16 if self.cb is not None else 0)
        ncopy = max(2, int(np.ceil(320e6 / self.stream_bytes)))
        self.mats, self.bufs = [], []
        p0 = torch.from_numpy(pair).cuda()
        t0 = torch.from_numpy(tail if tail.size else np.zeros(16, np.uint8)).cuda()
        for _ in range(ncopy):
            p = p0.clone()
            t = t0.clone()
            self.bufs.append((p, t))
            if fmt == "b6":
                self.mats.append(ctx.wrap_nibble4(rows, cols, 2, p, pair.size, t if tail.size else None, tail.size))
            else:
                self.mats.append(ctx.wrap_nf(rows, cols, 4, 2, self.cb, p, pair.size, t if tail.size else None,
                                             tail.size))
        self.pair_host, self.tail_host = pair, tail
        rng = np.random.default_rng(SEED + cols)
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        for t in range(ntok):
            idx = rng.choice(cols, max(1, cols // 1000), replace=False)
            x[t, idx] *= 30.0
        self.x = torch.from_numpy(x).cuda()
        self.q = torch.empty((ntok, cols), dtype=torch.int8, device="cuda")
        self.s = torch.empty((ntok, cols // 64), dtype=torch.float32, device="cuda")
        self.sm = torch.empty((ntok, cols // 64), dtype=torch.int32, device="cuda")
        ctx.act_quant(self.x, self.q, self.s, self.sm, cols, ntok)
        self.out = torch.empty((ntok, rows), dtype=torch.float32, device="cuda")
        self.bytes = gemv_bytes(self.stream_bytes, rows, cols, ntok, fmt == "b6")
        self.i = 0

    def launch(self, ctx):
        m = self.mats[self.i % len(self.mats)]
        self.i += 1
        ctx.gemv(m, self.q, self.s, self.sm, self.out, ntok=self.ntok, out_stride=self.rows)


def _busy_wait(torch, stream, seconds):
    """Keeps the stream busy while the host enqueues the timed launches, so that the
    events measure device time only (not host launch latency)."""
    try:
        torch.cuda._sleep(int(seconds * 2.0e9))
    except Exception:
        pass


def time_case(ctx, torch, case, steps, warmup):
    """Mean device time per GEMV: `steps` back-to-back launches between two events on
    the kernels' stream, enqueued behind a spin so the host never starves the queue."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        case.launch(ctx)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _busy_wait(torch, stream, 2e-3 + steps * 60e-6)
    a.record(stream)
    for _ in range(steps):
        case.launch(ctx)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / steps


def cpu_baseline(case, seconds=10.0):
    """Reference portable path restated in C (oracle nf_gemv_portable / nibble4 portable):
    dequantize each row, fp32 dot per chunk.  Stripe ranges split over host threads."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    rows, cols = case.rows, case.cols
    q = case.q[0].cpu().numpy()
    s = case.s[0].cpu().numpy()
    stripes = (rows + 15) // 16
    threads = min(16, os.cpu_count() or 1)
    out = np.zeros(rows, np.float32)

    def work(s0, s1):
        o = np.zeros(rows, np.float32)
        if case.fmt == "b6":
            o = O.nibble4_gemv_portable(case.pair_host, case.tail_host, rows, cols, 2, q, s, s0, s1)
        else:
            o = O.nf_gemv_portable(case.pair_host, case.tail_host, rows, cols, 4, 2, case.cb, q, s, s0, s1)
        out[s0 * 16:min(s1 * 16, rows)] = o[s0 * 16:min(s1 * 16, rows)]

    def one_pass():
        per = (stripes + threads - 1) // threads
        per += per & 1
        ths = [threading.Thread(target=work, args=(a, min(stripes, a + per))) for a in range(0, stripes, per)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()

    t0 = time.perf_counter()
    one_pass()
    first = time.perf_counter() - t0
    reps = max(1, int(seconds / max(first, 1e-3)))
    t0 = time.perf_counter()
    for _ in range(reps):
        one_pass()
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(case.bytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{case.name} full matrix x{reps} passes, portable dequantize+fp32-dot path "
                      f"(simd_lut.rs:5719-5748), {threads} host threads over stripe ranges",
            "ms_per_gemv": round(dt * 1e3, 3)}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    import torch
    import k2t
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ctx = k2t.Ctx(0)
    ctx.set_stream(torch.cuda.current_stream())
    if os.environ.get("K2T_SPLITK"):
        ctx.set_splitk(int(os.environ["K2T_SPLITK"]))
    if os.environ.get("K2T_EXACT"):
        ctx.set_exact(int(os.environ["K2T_EXACT"]))

    specs = [("nf4g128_14336x4096", "nf4", 14336, 4096), ("nf4g128_4096x14336", "nf4", 4096, 14336),
             ("b6_14336x4096", "b6", 14336, 4096), ("b6_4096x14336", "b6", 4096, 14336)]
    only = [s for s in args.only.split(",") if s]
    cases = []
    for name, fmt, r, c in specs:
        if only and name not in only:
            continue
        cases.append(GemvCase(ctx, torch, name, fmt, r, c))
        print(f"# built {name}: {cases[-1].stream_bytes} B x {len(cases[-1].mats)} copies", file=sys.stderr,
              flush=True)
    results = {}
    total_t = 0.0
    total_b = 0
    for case in cases:
        mean_s = time_case(ctx, torch, case, args.steps, args.warmup)
        gbs = case.bytes / mean_s / 1e9
        results[case.name] = {"us": round(mean_s * 1e6, 3), "GB_s": round(gbs, 1),
                              "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 2), "bytes": case.bytes}
        total_t += mean_s
        total_b += case.bytes
        print(f"# {case.name}: {mean_s * 1e6:.2f} us  {gbs:.1f} GB/s  {100 * gbs / HBM_PEAK_GBS:.1f}% of peak",
              file=sys.stderr, flush=True)
    dom = max(cases, key=lambda c: results[c.name]["us"])
    dom_r = results[dom.name]
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(next(c for c in cases if c.fmt == "nf4") if any(c.fmt == "nf4" for c in cases)
                           else cases[0])
    value = total_b / total_t / 1e9
    line = {
        "metric": "quant GEMV HBM GB/s (% peak) + decode tok/s, 1.7B-shape nf4g128, 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_t * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xu4/nf4->i32, fp32 epilogue",
        "data": "synthetic: W ~N(0,0.02) seeded, Hadamard RTN-quantized on host; x ~N(0,1) with 0.1% outliers x30",
        "config": {"workload": "config 4 GEMV sweep (nf4g128 + b6, 14336x4096 and 4096x14336, batch 1)",
                   "cases": results},
        "roofline": {"bound": "hbm", "kernel": f"gemv_kernel ({dom.name})", "achieved": dom_r["GB_s"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dom_r["GB_s"] / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
