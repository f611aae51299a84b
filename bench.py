"""Benchmark for the MI355X quantized decode hot path (one GPU).

Metric: quant GEMV HBM GB/s (% of peak) + decode tok/s, 1.7B-shape
nf4g128.  `value` is decode tok/s of the SmolLM2-1.7B-shaped nf4g128 model (config 3:
256-token prefill (NF4 GEMVs on the int8 matrix cores), then greedy decode steps; a "step" is one
decode token).  Also reported: the config-4 GEMV sweep (nf4g128 and b6 GEMVs on
14336x4096 and 4096x14336 at batch 1 and 4, each launch reading a different weight copy
so the 256 MB Infinity Cache cannot serve them; HIP-event burst timing on the kernels'
stream) and the SmolLM2-135M-shaped p55454 decode at context 512 (config 2).

Prints ONE JSON line (see the keys below).  --gpus N > 1 is refused: this build and
its measurements are single-GPU.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kronos-2t_amd"))

HBM_PEAK_GBS = 8000.0
SEED = 20261201


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="", help="comma list of GEMV case names to run (profiling)")
    ap.add_argument("--decode-only", action="store_true", help="skip the GEMV sweep and the 135M run (profiling)")
    ap.add_argument("--moe-only", action="store_true", help="run only the config-5 MoE decode (profiling)")
    ap.add_argument("--no-moe", action="store_true", help="skip the config-5 MoE decode")
    ap.add_argument("--small-only", action="store_true", help="run only the config-2 135M decode (profiling)")
    ap.add_argument("--moe-context", type=int, default=6600)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="also run 3 plain device copies of MB MiB (HBM counter calibration)")
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
        if fmt in ("b4", "b5", "b6"):
            self.planes = int(fmt[1])
            pair, tail = k2t.compile_bipolar(W, self.planes)
            self.cb = None
        else:
            self.bits = 3 if fmt == "nf3" else 4
            cb, mu, pair, tail = k2t.compile_nf4(W, 2, bits=self.bits)
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
            if self.cb is None:
                self.mats.append(ctx.wrap_nibble4(rows, cols, self.planes - 4, p, pair.size, t if tail.size else None,
                                                  tail.size))
            else:
                self.mats.append(ctx.wrap_nf(rows, cols, self.bits, 2, self.cb, p, pair.size,
                                             t if tail.size else None, tail.size))
                # NF3: the device's lane order (what k2t_mat_upload_nf stores), set up once
                self.mats[-1].nf3_lane_order()
        self.pair_host, self.tail_host = pair, tail
        rng = np.random.default_rng(SEED + cols)
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        # config 4: 0.1% outlier channels x30; config 1 (the 576-wide case): 4 channels x20
        n_out, mult = (4, 20.0) if cols == 576 else (max(1, cols // 1000), 30.0)
        for t in range(ntok):
            idx = rng.choice(cols, n_out, replace=False)
            x[t, idx] *= mult
        self.x = torch.from_numpy(x).cuda()
        self.q = torch.empty((ntok, cols), dtype=torch.int8, device="cuda")
        self.s = torch.empty((ntok, cols // 64), dtype=torch.float32, device="cuda")
        self.sm = torch.empty((ntok, cols // 64), dtype=torch.int32, device="cuda")
        ctx.act_quant(self.x, self.q, self.s, self.sm, cols, ntok)
        self.out = torch.empty((ntok, rows), dtype=torch.float32, device="cuda")
        self.bytes = gemv_bytes(self.stream_bytes, rows, cols, ntok, self.cb is None)
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


# Launches averaged per GEMV case (and per ceiling probe), whatever --steps says: each
# timed batch carries a one-off start cost of about 13 us (measured: nf4 4096x14336 b1
# averages 10.1 us over 20 launches, 9.45 us over 128), which must not be spread over
# few launches.
GEMV_LAUNCHES = 200


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


def decode_bench(ctx, torch, name, cfg, fmt, prefill, steps, warmup, log, planes=None):
    """Builds the model, times a `prefill`-token prefill, then `steps` greedy decode steps
    after `warmup` untimed ones.  The decode steps are timed twice: on the host clock
    around generate() (decode_tok_s) and by HIP events recorded on the model's own stream
    around the same steps (kernel_us_per_step: device time of the step's kernels, the
    persistent decode kernel's launch when that path runs)."""
    import k2t
    t0 = time.perf_counter()
    model, mats, host = k2t.build_random_model(ctx, cfg, max_seq=prefill + warmup + steps + 8, fmt=fmt,
                                               planes=planes, seed=7, max_batch=256, keep_host=True, threads=0)
    t_build = time.perf_counter() - t0
    if os.environ.get("K2T_MODEL_EXACT"):
        model.set_exact(int(os.environ["K2T_MODEL_EXACT"]))
    if os.environ.get("K2T_PERSISTENT"):
        model.set_persistent(int(os.environ["K2T_PERSISTENT"]))
    if os.environ.get("K2T_MFMA"):
        ctx.set_mfma(int(os.environ["K2T_MFMA"]))
    wbytes = sum(m.info()[3] for m in mats)
    rng = np.random.default_rng(SEED)
    toks = rng.integers(0, cfg["vocab"], prefill).astype(np.int32)
    # Warm-up: the same prefill once, untimed (the first launch of each kernel variant a
    # batch of this size uses loads its code object), then back to position 0.
    model.prefill(toks, want_logits=True)
    model.reset()
    model.sync()
    t0 = time.perf_counter()
    model.prefill(toks, want_logits=True)
    t_pre = time.perf_counter() - t0
    model.generate(int(toks[-1]), warmup, want_tokens=False)  # graph capture + warm-up
    model.sync()
    persistent = model.persistent_active()
    st = torch.cuda.ExternalStream(model.stream())
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev_a.record(st)
    t0 = time.perf_counter()
    model.generate(int(toks[-1]), steps, want_tokens=False)
    t_dec = time.perf_counter() - t0
    ev_b.record(st)
    ev_b.synchronize()
    kernel_us = ev_a.elapsed_time(ev_b) * 1e3 / steps
    kv_per_tok = cfg["n_layers"] * cfg["n_kv_heads"] * 2 * (cfg["head_dim"] + 4)
    ctx_mid = prefill + warmup + steps / 2
    tok_s = steps / t_dec
    res = {"decode_tok_s": round(tok_s, 1), "ms_per_token": round(t_dec / steps * 1e3, 4),
           "prefill_tok_s": round(prefill / t_pre, 1), "prefill_tokens": prefill, "decode_steps": steps,
           "context_at_decode": [prefill + warmup, prefill + warmup + steps],
           "weight_bytes": int(wbytes), "kv_bytes_per_token": kv_per_tok,
           "decode_GB_s": round((wbytes + kv_per_tok * ctx_mid) * tok_s / 1e9, 1), "build_s": round(t_build, 1),
           "persistent_kernel": bool(persistent), "kernel_us_per_step": round(kernel_us, 2),
           # algorithmic HBM bytes of one decode step: every weight byte once, the K/V read
           # at the mean context of the timed steps, and the new position's K/V written
           "step_bytes": int(wbytes + kv_per_tok * ctx_mid + kv_per_tok)}
    log(f"# {name}: decode {tok_s:.1f} tok/s ({t_dec / steps * 1e3:.3f} ms/token, {kernel_us:.1f} us of device "
        f"time per step), prefill {prefill / t_pre:.0f} tok/s, weights {wbytes / 1e6:.1f} MB")
    return model, mats, host, res


QWEN3_30B_A3B = dict(n_layers=48, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, intermediate=768,
                     vocab=151936, rms_eps=1e-6, rope_theta=1000000.0)
MOE_EXPERTS, MOE_TOPK, MOE_FF, MOE_POOL = 128, 8, 768, 16


def moe_decode_bench(ctx, torch, steps, warmup, context, log):
    """Config 5: Qwen3-30B-A3B-shaped sparse-MoE decode at `context` tokens.  NF4g128
    attention (QK-norm, q_dim 4096 != hidden 2048) and lm_head compiled on the host, an
    untied bf16 embedding, fp32 routers ~N(0, 0.05) from fixed seeds (reproducible
    routing), and a .k2tm bank of 48 x 128 NF3 g128 experts (gate_up 1536x2048, down
    2048x768) in HBM: MOE_POOL experts compiled on the host, their records replicated
    into all 6144 slots (distinct memory, so every routed expert is read from HBM).
    The KV cache is filled with seeded synthetic int8 K/V up to `context`."""
    import k2t
    cfg = dict(QWEN3_30B_A3B, max_seq=context + warmup + steps + 8)
    d, nq, nkv, hd, V, L = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["vocab"], \
        cfg["n_layers"]
    t0 = time.perf_counter()
    lay = k2t.k2tm_expert_layout(d, MOE_FF, 3, 2)
    rec = lay["aligned_expert_bytes"]
    pool = np.zeros((MOE_POOL, rec), np.uint8)
    for j in range(MOE_POOL):
        Wgu = k2t.synth_normal(SEED + 5000 + 2 * j, 2 * MOE_FF * d, 0.02).reshape(2 * MOE_FF, d)
        Wdn = k2t.synth_normal(SEED + 5001 + 2 * j, d * MOE_FF, 0.02).reshape(d, MOE_FF)
        cg, _, pg, _ = k2t.compile_nf4(Wgu, 2, bits=3)
        cd, _, pd, _ = k2t.compile_nf4(Wdn, 2, bits=3)
        pool[j, lay["gu_codebook_off"]:lay["gu_codebook_off"] + 16] = cg.view(np.uint8)
        pool[j, lay["dn_codebook_off"]:lay["dn_codebook_off"] + 16] = cd.view(np.uint8)
        pool[j, lay["gu_pair_off"]:lay["gu_pair_off"] + pg.size] = pg
        pool[j, lay["dn_pair_off"]:lay["dn_pair_off"] + pd.size] = pd
    page = np.zeros(16384, np.uint8)
    page[:12] = np.frombuffer(b"K2TM800B_V1\0", np.uint8)
    page[16:16 + 56] = np.array([L, MOE_EXPERTS, d, MOE_FF, 2, rec, 3], np.uint64).view(np.uint8)
    n_rec = L * MOE_EXPERTS
    bank_t = torch.empty(16384 + n_rec * rec, dtype=torch.uint8, device="cuda")
    bank_t[:16384].copy_(torch.from_numpy(page))
    recs = bank_t[16384:].view(n_rec, rec)
    pool_d = torch.from_numpy(pool).cuda()
    for j in range(MOE_POOL):
        sl = recs[j::MOE_POOL]
        sl.copy_(pool_d[j].unsqueeze(0).expand(sl.shape[0], rec))
    del pool_d
    bank = k2t.ExpertBank.wrap(ctx, bank_t, bank_t.numel(), page)
    bank.nf3_lane_order()  # the device's NF3 lane order (what k2t_experts_upload stores), once
    model = k2t.Model(ctx, cfg, max_batch=1)
    mats = []
    ones_d, ones_hd = np.ones(d, np.float32), np.ones(hd, np.float32)

    def nf4(rows, cols, seed):
        W = k2t.synth_normal(seed, rows * cols, 0.02).reshape(rows, cols)
        cb, _, pair, tail = k2t.compile_nf4(W, 2)
        m = ctx.upload_nf(rows, cols, 4, 2, cb, pair, tail)
        mats.append(m)
        return m

    for li in range(L):
        q = nf4((nq + 2 * nkv) * hd, d, SEED + 100 * li + 1)
        o = nf4(d, nq * hd, SEED + 100 * li + 2)
        model.set_layer(li, q, o, None, None, ones_d, ones_d)
        model.set_qk_norm(li, ones_hd, ones_hd)
        router = k2t.synth_normal(SEED + 100 * li + 3, MOE_EXPERTS * d, 0.05).reshape(MOE_EXPERTS, d)
        model.set_moe(li, bank, li, router, MOE_TOPK, True, k2t.MOE_SOFTMAX)
    head = nf4(V, d, SEED + 99991)
    emb = (k2t.synth_normal(SEED + 99992, V * d, 0.02).view(np.uint32) >> 16).astype(np.uint16)
    model.set_embedding(k2t.EMBED_BF16, emb)
    del emb
    model.set_head(head, ones_d)
    t_build = time.perf_counter() - t0
    model.kv_synthetic(context, seed=SEED)
    model.generate(1, warmup, want_tokens=False)  # graph capture + warm-up
    model.sync()
    t0 = time.perf_counter()
    model.generate(1, steps, want_tokens=False)
    t_dec = time.perf_counter() - t0
    tok_s = steps / t_dec
    attn_bytes = sum(m.info()[3] for m in mats if m is not head)
    expert_bytes = MOE_TOPK * (lay["gu_pair_bytes"] + lay["dn_pair_bytes"] + 32)
    router_bytes = MOE_EXPERTS * d * 4
    wbytes = attn_bytes + head.info()[3] + L * (expert_bytes + router_bytes)
    kv_per_tok = L * nkv * 2 * (hd + 4)
    ctx_mid = context + warmup + steps / 2
    res = {"decode_tok_s": round(tok_s, 1), "ms_per_token": round(t_dec / steps * 1e3, 4), "decode_steps": steps,
           "context_at_decode": [context + warmup, context + warmup + steps],
           "weight_bytes_per_token": int(wbytes), "kv_bytes_per_token_of_context": kv_per_tok,
           "resident_expert_bytes": int(n_rec * rec),
           "decode_GB_s": round((wbytes + kv_per_tok * ctx_mid) * tok_s / 1e9, 1), "build_s": round(t_build, 1)}
    log(f"# 30B-A3B MoE nf3/nf4g128 @ctx {context}: decode {tok_s:.1f} tok/s ({t_dec / steps * 1e3:.3f} ms/token), "
        f"{wbytes / 1e6:.1f} MB weights/token")
    model.close()
    for m in mats:
        m.close()
    bank.close()
    del bank_t
    torch.cuda.empty_cache()
    return res


def load_traffic(name):
    """HBM bytes per launch of a roofline kernel, from the committed rocprofv3 --pmc
    summary profiles/<name>_hbm_traffic.txt (FETCH_SIZE + WRITE_SIZE, each scaled by the
    same counter's reading for a plain copy of known size).  None when none is committed."""
    path = os.path.join(ROOT, "profiles", f"{name}_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for ln in open(path):
        if ln.startswith("traffic_bytes_per_launch:"):
            return int(float(ln.split(":", 1)[1]))
    return None


def copy_probe(torch, mib):
    """Three plain device-to-device copies of `mib` MiB (a kernel of known HBM traffic:
    mib MiB read + mib MiB written) for scaling the PMC byte counters."""
    src = torch.ones(mib << 18, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def read_ceiling(ctx, torch, nbytes, steps=GEMV_LAUNCHES):
    """Practical single-launch HBM read rate at this byte count: k2t_stream_read_probe over
    nbytes, rotated over enough buffers to miss the 256 MB Infinity Cache, timed back to
    back like the GEMV cases.  Returns (GB/s, us)."""
    nb = (nbytes + 15) // 16 * 16
    ncopy = max(2, int(np.ceil(320e6 / nb)))
    bufs = [torch.ones(nb // 4, dtype=torch.float32, device="cuda") for _ in range(ncopy)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for i in range(ncopy):
        ctx.stream_read_probe(bufs[i], nb, sink)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _busy_wait(torch, stream, 2e-3 + steps * 60e-6)
    a.record(stream)
    for i in range(steps):
        ctx.stream_read_probe(bufs[i % ncopy], nb, sink)
    b.record(stream)
    torch.cuda.synchronize()
    t = a.elapsed_time(b) * 1e-3 / steps
    del bufs
    return nb / t / 1e9, t * 1e6


def copy_ceiling(torch, nbytes, steps=GEMV_LAUNCHES):
    """Practical HBM rate of one launch moving this many bytes: device-to-device copies of
    nbytes/2 read + nbytes/2 written, rotated over enough buffers to miss the 256 MB
    Infinity Cache, timed back to back like the GEMV cases.  Returns (GB/s, us)."""
    n = max(1, nbytes // 8)  # float32 elements per source buffer (nbytes/2 bytes)
    ncopy = max(2, int(np.ceil(320e6 / (4 * n))))
    src = [torch.ones(n, dtype=torch.float32, device="cuda") for _ in range(ncopy)]
    dst = [torch.empty_like(src[0]) for _ in range(ncopy)]
    for i in range(ncopy):
        dst[i].copy_(src[i])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _busy_wait(torch, stream, 2e-3 + steps * 60e-6)
    a.record(stream)
    for i in range(steps):
        dst[i % ncopy].copy_(src[i % ncopy])
    b.record(stream)
    torch.cuda.synchronize()
    t = a.elapsed_time(b) * 1e-3 / steps
    del src, dst
    return 8 * n / t / 1e9, t * 1e6


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_decode_baseline(cfg, host, context, seconds=10.0, max_tokens=32, name="1.7B nf4g128"):
    """The reference's portable CPU decode step (dequantize + fp32 dot GEMVs over stripe
    ranges, real_llm.rs:829-836 / simd_lut.rs:5719-5748; scalar q8 attention) restated in
    the oracle's C and driven by a C decode loop over a host thread pool
    (oracle/k2t_cpu_port.c), compiled here with -O3 -march=native: tokens attending
    `context`+ positions (the KV cache is seeded, as the GPU run's cache holds its
    prefill), at all host threads (up to 16, the box's CPU share) for about `seconds`, and
    one token on one thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_port
    path = cpu_port.build()
    threads = min(16, os.cpu_count() or 1)

    def run(nthreads, budget, cap):
        pm = cpu_port.CpuPortModel(cfg, host, nthreads, context + cap + 2, lib_path=path)
        pm.seed_kv(context, seed=1)
        t0 = time.perf_counter()
        ntok = 0
        while ntok < cap and (ntok < 1 or time.perf_counter() - t0 < budget):
            pm.decode(3 + ntok)
            ntok += 1
        dt = (time.perf_counter() - t0) / ntok
        pm.close()
        return ntok, dt

    run(threads, 0.0, 1)  # warm the page cache and thread pool
    ntok, dt = run(threads, seconds, max_tokens)
    _, dt1 = run(1, 0.0, 1)
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "one_thread": {"value": round(1.0 / dt1, 4), "unit": "tok/s", "cores": 1},
            "sample": f"{ntok} decode tokens of the {name} model at context {context}-{context + ntok} (KV "
                      f"cache seeded) on the portable path (dequantize + fp32 dot, simd_lut.rs:5719-5748) restated "
                      f"in C with a C decode loop, gcc -O3 -march=native on this host, {threads} threads; "
                      f"one_thread: 1 token on 1 thread"}


def cpu_gemv_baseline(cases):
    """The portable CPU GEMV (dequantize + fp32 dot, simd_lut.rs:3558-3581 / 5719-5748) on
    the sweep's own matrices and activations, at all host threads (up to 16) and at 1:
    GB/s of the same algorithmic bytes as the GPU line."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from model_oracle import Matrix
    threads = min(16, os.cpu_count() or 1)
    out = {}
    for key, c in cases.items():
        fmt = "n4" if c["fmt"] in ("b4", "b5", "b6") else "nf4"
        hp = int(c["fmt"][1]) - 4 if fmt == "n4" else 0
        m = Matrix(fmt, c["rows"], c["cols"], c["pair"], c["tail"], hp=hp, cb=c["cb"], sgc=2)
        res = {}
        for nt in (threads, 1):
            m.gemv_portable(c["xq"], c["xs"], nt)  # warm
            reps, t0 = 0, time.perf_counter()
            while reps < 3 or (time.perf_counter() - t0 < 0.5 and reps < 200):
                m.gemv_portable(c["xq"], c["xs"], nt)
                reps += 1
            dt = (time.perf_counter() - t0) / reps
            res[f"{nt}t"] = {"us": round(dt * 1e6, 1), "GB_s": round(c["bytes"] / dt / 1e9, 3)}
        out[key] = res
    return {"threads": threads, "cpu_model": cpu_model(), "kind": "port", "cases": out}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    import torch
    import k2t
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    ctx = k2t.Ctx(0)
    ctx.set_stream(torch.cuda.current_stream())
    if os.environ.get("K2T_SPLITK"):
        ctx.set_splitk(int(os.environ["K2T_SPLITK"]))
    if os.environ.get("K2T_EXACT"):
        ctx.set_exact(int(os.environ["K2T_EXACT"]))

    if args.small_only:
        m135, mats135, _, r135 = decode_bench(ctx, torch, "135M p55454", k2t.SMOLLM2_135M, "n4", 512, args.steps,
                                              args.warmup, log)
        print(json.dumps({"metric": "decode tok/s, 135M p55454", "value": r135["decode_tok_s"], "unit": "tok/s",
                          "config": r135}))
        return
    if args.moe_only:
        r30 = moe_decode_bench(ctx, torch, args.steps, args.warmup, args.moe_context, log)
        print(json.dumps({"metric": "decode tok/s, 30B-A3B-shape MoE", "value": r30["decode_tok_s"],
                          "unit": "tok/s", "config": r30}))
        return

    # ---- config 4: GEMV sweep
    specs = [("b4_1536x576", "b4", 1536, 576),  # config 1 (launch-bound: 0.48 MB per call)
             ("nf4g128_14336x4096", "nf4", 14336, 4096), ("nf4g128_4096x14336", "nf4", 4096, 14336),
             ("b6_14336x4096", "b6", 14336, 4096), ("b6_4096x14336", "b6", 4096, 14336),
             ("nf3g128_14336x4096", "nf3", 14336, 4096), ("nf3g128_4096x14336", "nf3", 4096, 14336)]
    only = [s for s in args.only.split(",") if s]
    results = {}
    cpu_cases = {}  # config 1 and config 4 matrices kept on the host for the CPU GEMV leg
    dom = None
    for name, fmt, r, c in specs:
        if (only and name not in only) or args.decode_only:
            continue
        for ntok in (1, 4):
            case = GemvCase(ctx, torch, name, fmt, r, c, ntok=ntok)
            mean_s = time_case(ctx, torch, case, max(args.steps, GEMV_LAUNCHES), args.warmup)
            gbs = case.bytes / mean_s / 1e9
            key = f"{name}_b{ntok}"
            results[key] = {"us": round(mean_s * 1e6, 3), "GB_s": round(gbs, 1),
                            "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 2), "bytes": case.bytes}
            log(f"# {key}: {mean_s * 1e6:.2f} us  {gbs:.1f} GB/s  {100 * gbs / HBM_PEAK_GBS:.1f}% of peak")
            if ntok == 1 and fmt == "nf4" and (dom is None or results[key]["GB_s"] < results[dom]["GB_s"]):
                dom = key
            if ntok == 1 and key in ("b4_1536x576_b1", "nf4g128_4096x14336_b1", "b6_4096x14336_b1"):
                cpu_cases[key] = {"fmt": fmt, "rows": r, "cols": c, "pair": case.pair_host, "tail": case.tail_host,
                                  "cb": case.cb, "xq": case.q[0].cpu().numpy(), "xs": case.s[0].cpu().numpy(),
                                  "bytes": case.bytes}
            del case
    ceiling = rceiling = None
    if dom is not None:
        cg, cu = copy_ceiling(torch, results[dom]["bytes"])
        ceiling = {"GB_s": round(cg, 1), "us": round(cu, 3), "frac": round(cg / HBM_PEAK_GBS, 4)}
        log(f"# copy ceiling at {results[dom]['bytes']} B per launch: {cu:.2f} us  {cg:.1f} GB/s "
            f"{100 * cg / HBM_PEAK_GBS:.1f}% of peak")
        rg, ru = read_ceiling(ctx, torch, results[dom]["bytes"])
        rceiling = {"GB_s": round(rg, 1), "us": round(ru, 3), "frac": round(rg / HBM_PEAK_GBS, 4)}
        log(f"# read ceiling at {results[dom]['bytes']} B per launch: {ru:.2f} us  {rg:.1f} GB/s "
            f"{100 * rg / HBM_PEAK_GBS:.1f}% of peak")
    line = {"metric": "quant GEMV HBM GB/s (% peak) + decode tok/s, 1.7B-shape nf4g128, 1 MI355X"}
    if args.copy_probe:
        copy_probe(torch, args.copy_probe)
    if args.only:
        line.update({"config": {"cases": results, "copy_ceiling": ceiling, "read_ceiling": rceiling}})
        print(json.dumps(line))
        return
    torch.cuda.empty_cache()

    # ---- config 3: 1.7B nf4g128 prefill 256 + greedy decode
    m17, mats17, host17, r17 = decode_bench(ctx, torch, "1.7B nf4g128", k2t.SMOLLM2_1_7B, "nf4", 256, args.steps,
                                            args.warmup, log)
    cpu = None if args.no_cpu_baseline else cpu_decode_baseline(k2t.SMOLLM2_1_7B, host17, 256 + args.warmup)
    if cpu is not None:
        cpu["gemv"] = cpu_gemv_baseline(cpu_cases)
        log(f"# CPU ({cpu['cpu_model']}): decode {cpu['value']} tok/s on {cpu['cores']} threads, "
            f"{cpu['one_thread']['value']} tok/s on 1; GEMV " +
            ", ".join(f"{k} {v[str(cpu['cores']) + 't']['GB_s']} GB/s" for k, v in cpu["gemv"]["cases"].items()))
    m17.close()
    for m in mats17:
        m.close()
    del host17
    # ---- config 2: 135M p55454, decode at context 512
    if args.decode_only:
        print(json.dumps(dict(line, value=r17["decode_tok_s"], unit="tok/s", config=r17)))
        return
    m135, mats135, host135, r135 = decode_bench(ctx, torch, "135M p55454", k2t.SMOLLM2_135M, "n4", 512, 64, 8, log)
    if cpu is not None:
        # the same port on config 2 at the GPU run's context (512 + warmup)
        c2 = cpu_decode_baseline(k2t.SMOLLM2_135M, host135, 512 + 8, seconds=5.0, max_tokens=64,
                                 name="135M p55454")
        cpu["decode_135m_p55454"] = {k: c2[k] for k in ("value", "unit", "cores", "one_thread", "sample")}
        log(f"# CPU 135M p55454: decode {c2['value']} tok/s on {c2['cores']} threads, "
            f"{c2['one_thread']['value']} tok/s on 1")
    del host135
    m135.close()
    for m in mats135:
        m.close()
    torch.cuda.empty_cache()
    # ---- the same 135M shape with 4 bit planes everywhere (the reference's B4 tier)
    mb4, matsb4, hostb4, rb4 = decode_bench(ctx, torch, "135M b4", k2t.SMOLLM2_135M, "n4", 512, 64, 8, log,
                                            planes={k: 4 for k in k2t.P55454})
    del hostb4
    mb4.close()
    for m in matsb4:
        m.close()
    torch.cuda.empty_cache()
    # ---- and with 6 bit planes everywhere (the B6 tier: the 256-thread two-hi-plane kernel)
    mb6, matsb6, hostb6, rb6 = decode_bench(ctx, torch, "135M b6", k2t.SMOLLM2_135M, "n4", 512, 64, 8, log,
                                            planes={k: 6 for k in k2t.P55454})
    del hostb6
    mb6.close()
    for m in matsb6:
        m.close()
    torch.cuda.empty_cache()
    # ---- config 5: 30B-A3B-shaped sparse MoE, decode at context 6600
    r30 = None if args.no_moe else moe_decode_bench(ctx, torch, 32, 4, args.moe_context, log)

    dr = results[dom]
    line.update({
        "value": r17["decode_tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r17["ms_per_token"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 activations x nf4/bit-plane weights -> i32 dots, fp32 epilogue",
        "data": "synthetic: random-init weights ~N(0,0.02) seeded, Hadamard RTN-quantized on the host; seeded "
                "random token ids; greedy decode",
        "config": {"workload": "config 3: SmolLM2-1.7B-shaped nf4g128 (24 layers, d 2048, 32 heads MHA, hd 64, "
                               "ffn 8192, vocab 49152), 256-token prefill (int8-MFMA NF4 GEMVs) then greedy decode",
                   "decode_1_7b_nf4g128": r17, "decode_135m_p55454_ctx512": r135, "decode_135m_b4_ctx512": rb4,
                   "decode_135m_b6_ctx512": rb6,
                   "decode_30b_a3b_moe_nf3_ctx6600": r30, "gemv_sweep": results},
        # the kernel behind `value`: one persistent decode launch per token
        "roofline": {"bound": "hbm",
                     "kernel": "decode_mk_kernel<1,0,512> (one launch per 1.7B nf4g128 decode step)"
                     if r17["persistent_kernel"] else "per-operation decode step (HIP graph)",
                     "achieved": round(r17["step_bytes"] / r17["kernel_us_per_step"] / 1e3, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r17["step_bytes"] / r17["kernel_us_per_step"] / 1e3 / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic("decode_1_7b_nf4g128"),
                     "algorithmic_bytes_per_launch": r17["step_bytes"], "avg_launch_us": r17["kernel_us_per_step"],
                     # the sweep's slowest nf4 batch-1 GEMV (config 4)
                     "gemv": {"kernel": f"gemv_kernel ({dom})", "achieved": dr["GB_s"], "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(dr["GB_s"] / HBM_PEAK_GBS, 4),
                              "traffic": load_traffic(f"gemv_{dom}"), "algorithmic_bytes_per_launch": dr["bytes"],
                              "avg_launch_us": dr["us"], "copy_ceiling_same_bytes": ceiling,
                              "read_ceiling_same_bytes": rceiling}},
        "cpu_baseline": cpu,
    })
    print(json.dumps(line))


if __name__ == "__main__":
    main()
