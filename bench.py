#!/usr/bin/env python3
"""Benchmark of the T2S token-sampling path on one MI355X.

Workload (one bench step): 64 rows x V=8194 fp32 logits x 1000 AR steps, each
row with its own history (50-800 ids, growing by every sampled token) and its
own temperature / top_k / top_p / repetition penalty; the full processor chain
and the xorshift64 draw for every row-step. Inputs (2.1 GB of logits) are
resident in HBM before timing starts. One call of the stream entry point
processes the whole job: the scan kernel reads every (step, row) once and
writes candidate summaries, the per-row chain kernels walk the steps on them
(exact steps where a decision needs the full row), and chunks of steps are
scanned beside the chains of the previous chunk. The calls are issued back to
back on a stream of the bench's own. `value` is sampled rows per second over
that call; --sequential times the single-kernel stream instead.

Also reported: the same chain as one launch per AR step (per_call; with the
history as CSR ids, and kept on the device as a set that each call extends), an HBM
copy probe, bit-exact parity of the first AR steps against the CPU oracle, and
the oracle timed on host cores as the CPU baseline (kind "port").

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "mlx-confucius4-tts_amd"))

METRIC = "sampled rows/sec + achieved HBM GB/s (% peak), V=8194 batch 64"
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def profile_traffic():
    """HBM bytes per stream call (all its kernels) from the committed rocprofv3 PMC summary."""
    path = os.path.join(REPO, "profiles", "stream_batch64_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].split()[0])
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--ar-steps", type=int, default=1000)
    ap.add_argument("--cpu-steps", type=int, default=40,
                    help="AR steps of the 64-row job replayed by the CPU oracle")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sequential", action="store_true",
                    help="time the single-kernel stream (one persistent workgroup per row)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        msg = ("bench.py measures one GPU: rows are independent, a multi-GPU run would shard "
               "rows with no communication (see the sharding paragraph of the design notes); "
               "run with --gpus 1")
        print(msg, file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import c4s
    import c4s_workloads as W

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    ctx = c4s.Context(0)
    R, V, T = 64, W.V_SEMANTIC, args.ar_steps

    # ---- inputs, resident in HBM -------------------------------------------------------
    p = W.batch64_params(seed=2, rows=R, V=V)
    g = torch.Generator(device=dev)
    g.manual_seed(1002)
    logits = torch.randn((T, R, V), generator=g, device=dev, dtype=torch.float32) * 3.0
    spikes = torch.randint(0, V, (T, R, 5), generator=g, device=dev)
    logits.scatter_(2, spikes, 12.0)

    def d(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint64:
            a = a.view(np.int64)
        return torch.from_numpy(a.copy()).to(dev)

    hist_ids, hist_off = d(p["hist_ids"]), d(p["hist_off"])
    temp, top_k, top_p, pen = d(p["temp"]), d(p["top_k"]), d(p["top_p"]), d(p["pen"])
    do_sample = d(p["do_sample"])
    rng0 = d(p["rng"])
    rng = rng0.clone()
    out = torch.empty((T, R), dtype=torch.int32, device=dev)
    stats = torch.zeros((R, 4), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    # The calls go on a stream of their own, as an AR loop would issue them: on
    # the legacy default stream the scan's CU-masked (blocking) stream would
    # add implicit synchronisation to every call.
    work = torch.cuda.Stream()

    def launch(stats_ptr=None):
        ctx.sample_stream(logits, hist_ids, hist_off, temp, top_k, top_p, pen, rng, out,
                          do_sample=do_sample, stop_token=-1, out_stats=stats_ptr,
                          sequential=args.sequential, stream=work)

    # ---- warmup (the first launch starts from the seeded RNG: kept for parity) ------
    log(f"warmup x{args.warmup}")
    launch(stats)
    torch.cuda.synchronize()
    first_tokens = out[: args.cpu_steps].cpu().numpy().copy()
    st = stats.cpu().numpy()
    for _ in range(max(0, args.warmup - 1)):
        launch()
    torch.cuda.synchronize()

    # ---- timed region --------------------------------------------------------------------
    log(f"timed x{args.steps}")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record(work)
    for _ in range(args.steps):
        launch()
    ev1.record(work)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = ev0.elapsed_time(ev1) / args.steps
    rows_per_launch = R * T
    value = rows_per_launch / (ms * 1e-3)

    h0 = np.diff(p["hist_off"]).astype(np.float64)
    alg_bytes = T * R * (4 * V + 4) + 4 * (T * h0.sum() + R * T * (T - 1) / 2)
    design_bytes = T * R * (4 * V + 4) + 4 * h0.sum()
    achieved = alg_bytes / (ms * 1e-3) / 1e9
    log(f"stream: {ms:.3f} ms/call, {value / 1e6:.2f} M rows/s, {achieved:.1f} GB/s "
        f"({100 * achieved / PEAK_HBM_GBS:.1f}% of peak); exact steps {int(st[:, 1].sum())}, "
        f"exact draws {int(st[:, 2].sum())}")

    # ---- per-call: one launch per AR step (64 rows, initial histories) -----------------
    n_calls = 200
    tok1 = torch.empty(R, dtype=torch.int32, device=dev)
    rng1 = rng0.clone()
    for t in range(5):
        ctx.sample_rows(logits[t], hist_ids, hist_off, temp, top_k, top_p, pen, rng1, tok1,
                        do_sample=do_sample)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(n_calls):
        ctx.sample_rows(logits[t % T], hist_ids, hist_off, temp, top_k, top_p, pen, rng1, tok1,
                        do_sample=do_sample)
    e1.record()
    torch.cuda.synchronize()
    call_us = e0.elapsed_time(e1) * 1e3 / n_calls
    call_bytes = R * (4 * V + 4) + 4 * h0.sum()
    # the same loop with the history kept on the device as a set (grows by each token)
    bits = torch.zeros((R, (V + 31) // 32), dtype=torch.int32, device=dev)
    ctx.hist_bits_init(hist_ids, hist_off, R, V, bits)
    rng2 = rng0.clone()
    torch.cuda.synchronize()
    e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e2.record()
    for t in range(n_calls):
        ctx.sample_rows(logits[t % T], None, None, temp, top_k, top_p, pen, rng2, tok1,
                        do_sample=do_sample, hist_bits=bits, stop_token=V - 1)
    e3.record()
    torch.cuda.synchronize()
    bits_us = e2.elapsed_time(e3) * 1e3 / n_calls
    bits_bytes = R * (4 * V + 4 + 4 * ((V + 31) // 32) + 4)
    per_call = {"us_per_call": round(call_us, 3), "rows_per_s": round(R / (call_us * 1e-6), 1),
                "achieved_GBps": round(call_bytes / (call_us * 1e-6) / 1e9, 1),
                "hist_bits_us_per_call": round(bits_us, 3),
                "hist_bits_achieved_GBps": round(bits_bytes / (bits_us * 1e-6) / 1e9, 1)}
    log(f"per-call: {call_us:.2f} us per 64-row step ({bits_us:.2f} us with the history kept as a set)")

    # ---- LM head (LN -> bf16 MFMA GEMM + bias) alone and fused with the chain, 64 rows x D=1280 ----
    D = 1280
    gh = torch.Generator(device=dev)
    gh.manual_seed(77)
    hidden = torch.randn((R, D), generator=gh, device=dev).to(torch.bfloat16)
    weight = (0.02 * torch.randn((V, D), generator=gh, device=dev)).to(torch.bfloat16)
    gamma = 1.0 + 0.02 * torch.randn(D, generator=gh, device=dev)
    beta = 0.02 * torch.randn(D, generator=gh, device=dev)
    bias = 0.02 * torch.randn(V, generator=gh, device=dev)
    head_out = torch.empty((R, V), dtype=torch.float32, device=dev)
    rng3 = rng0.clone()

    def head_only():
        ctx.lmhead(hidden, gamma, beta, weight, bias, head_out)

    def head_sample():
        ctx.lmhead_sample(hidden, gamma, beta, weight, bias, hist_ids, hist_off, temp, top_k, top_p, pen,
                          rng3, tok1, logits=head_out, do_sample=do_sample)

    head_us = {}
    for name, fn in (("lmhead", head_only), ("lmhead_sample", head_sample)):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n_calls):
            fn()
        e1.record()
        torch.cuda.synchronize()
        head_us[name] = e0.elapsed_time(e1) * 1e3 / n_calls
    # weight, hidden, bias, gamma/beta read once; logits written once
    head_bytes = 2 * V * D + 2 * R * D + 4 * V + 8 * D + 4 * R * V
    head_gbs = head_bytes / (head_us["lmhead"] * 1e-6) / 1e9
    per_call.update({"lmhead_us_per_call": round(head_us["lmhead"], 3),
                     "lmhead_achieved_GBps": round(head_gbs, 1),
                     "lmhead_frac_of_hbm_peak": round(head_gbs / PEAK_HBM_GBS, 4),
                     "lmhead_sample_us_per_call": round(head_us["lmhead_sample"], 3)})
    log(f"lm head: {head_us['lmhead']:.2f} us ({head_gbs:.0f} GB/s); with the chain "
        f"{head_us['lmhead_sample']:.2f} us per 64-row step")
    del hidden, weight, head_out

    # ---- HBM probe ------------------------------------------------------------------------
    nb = 1 << 30
    src = torch.empty(nb // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    ctx.hbm_probe(src, dst, nb, 0)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        ctx.hbm_probe(src, dst, nb, 0)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * nb * 5 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    log(f"hbm copy probe: {copy_gbs:.0f} GB/s")

    # ---- parity on the first AR steps + CPU baseline ---------------------------------------
    parity = None
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle
        S = args.cpu_steps
        xs = logits[:S].cpu().numpy()
        log(f"cpu oracle: {S} AR steps x {R} rows, 1 thread")
        c0 = time.perf_counter()
        otoks, _ = oracle.sample_stream(xs, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                        p["top_p"], p["pen"], p["do_sample"], p["rng"],
                                        n_threads=1)
        c1 = time.perf_counter()
        mism = int((otoks != first_tokens).sum())
        parity = {"rows_checked": int(otoks.size), "token_mismatches": mism,
                  "bit_exact": mism == 0}
        cpu = {"value": round(otoks.size / (c1 - c0), 1), "unit": "rows/s", "cores": 1,
               "kind": "port",
               "sample": f"oracle/oracle.cpp (g++ -O3, same STL algorithms as the reference) "
                         f"on the first {S} AR steps x {R} rows of this job ({otoks.size} row-steps), "
                         f"serial row loop as text2semantic.cpp:303"}
        log(f"cpu: {cpu['value']:.0f} rows/s; parity mismatches {mism}")

    traffic = profile_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"batch64 AR stream: {R} rows x V={V} fp32 logits x {T} AR steps, "
                               "per-row history 50-800 ids growing by each sample, per-row "
                               "temperature/top_k/top_p/penalty, full chain + xorshift64 draw, "
                               "one stream call per bench step",
                   "rows": R, "vocab": V, "ar_steps": T,
                   "launch": ("k_stream_lds" if args.sequential else
                              "chunks of 64-256 steps (x6/5), three summary buffers, one call in flight: k_stream_scan of the next chunk on 22 of 32 CUs beside "
                              "k_stream_list + k_stream_chain (4 of 32) | k_stream_rowp + k_stream_segfix (6 of 32)")},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": traffic,
                     "alg_bytes_per_launch": int(alg_bytes),
                     "design_bytes_per_launch": int(design_bytes)},
        "cpu_baseline": cpu,
        "parity": parity,
        "per_call": per_call,
        "hbm_probe_copy_GBps": round(copy_gbs, 1),
        "wall_s_timed": round(wall, 4),
        "exact_steps": int(st[:, 1].sum()),
        "exact_draws": int(st[:, 2].sum()),
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
