"""GPU parity of the multi-step AR stream (one persistent workgroup per row) and
of the per-step batched path driven step by step."""
import numpy as np
import pytest

import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu


def run_stream(ctx, p, x, stop_token=-1, sequential=False, speculate=True):
    import torch
    steps, rows, V = x.shape
    out = torch.full((steps, rows), -9, dtype=torch.int32, device="cuda")
    st = torch.zeros((rows, 4), dtype=torch.int32, device="cuda")
    rng = dev(p["rng"], torch)
    ctx.sample_stream(dev(x, torch), dev(p["hist_ids"], torch), dev(p["hist_off"], torch),
                      dev(p["temp"], torch), dev(p["top_k"], torch), dev(p["top_p"], torch),
                      dev(p["pen"], torch), rng, out, do_sample=dev(p["do_sample"], torch),
                      stop_token=stop_token, out_stats=st, sequential=sequential, speculate=speculate)
    torch.cuda.synchronize()
    return out.cpu().numpy(), rng.cpu().numpy().view(np.uint64), st.cpu().numpy()


def test_stream_10k_rows_bit_exact(orc):
    """64 rows x 157 AR steps = 10,048 sampled rows, tokens bit-exact."""
    import c4s
    ctx = c4s.Context(0)
    steps = 157
    p = W.batch64_params(seed=2)
    x = W.batch64_logits(1002, steps)
    print("stream 10k: gpu", flush=True)
    toks, rng, st = run_stream(ctx, p, x)
    print("stream 10k: oracle", flush=True)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:5].tolist()}"
    assert np.array_equal(rng, orng)
    print("rows", toks.size, "exact steps", int(st[:, 1].sum()), "exact draws", int(st[:, 2].sum()))
    assert int(st[:, 1].sum()) < toks.size // 50      # the candidate summaries decide almost every step
    # Every sampled row advanced its xorshift64 state once per step: the GPU's
    # final states against the shift-matrix construction (text2semantic.cpp:158),
    # independently of the oracle.
    from xorshift_pin import advance
    for r in np.flatnonzero(p["do_sample"]):
        assert int(rng[r]) == advance(int(p["rng"][r]), steps), r
    ctx.close()


def test_stream_bench_workload_bit_exact(orc, gpu_ctx):
    """The whole headline workload: 64 rows x 1000 AR steps at V = 8194 with the
    inputs the bench builds (batch-64 parameters of seed 2, logits drawn on the
    device from seed 1002 with five spikes a row-step), 64,000 sampled rows
    against the oracle, tokens and final RNG states bit for bit."""
    import torch
    T, R, V = 1000, 64, W.V_SEMANTIC
    p = W.batch64_params(seed=2, rows=R, V=V)
    g = torch.Generator(device="cuda")
    g.manual_seed(1002)
    logits = torch.randn((T, R, V), generator=g, device="cuda", dtype=torch.float32) * 3.0
    spikes = torch.randint(0, V, (T, R, 5), generator=g, device="cuda")
    logits.scatter_(2, spikes, 12.0)
    out = torch.full((T, R), -9, dtype=torch.int32, device="cuda")
    rng = dev(p["rng"], torch)
    print("bench workload: gpu", flush=True)
    gpu_ctx.sample_stream(logits, dev(p["hist_ids"], torch), dev(p["hist_off"], torch), dev(p["temp"], torch),
                          dev(p["top_k"], torch), dev(p["top_p"], torch), dev(p["pen"], torch), rng, out,
                          do_sample=dev(p["do_sample"], torch))
    torch.cuda.synchronize()
    toks, grng = out.cpu().numpy(), rng.cpu().numpy().view(np.uint64)
    x = logits.cpu().numpy()
    del logits
    print("bench workload: oracle", flush=True)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"], p["top_p"],
                                    p["pen"], p["do_sample"], p["rng"], n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first (step, row) {bad[:5].tolist()}"
    assert np.array_equal(grng, orng)
    assert toks.size == 64000 and (toks >= 0).all()


def _mixed_params(seed, rows, V):
    """Every row mode of the two-phase stream: greedy, top-k (list), top-k > 64
    and penalty < 1 (exact every step), full vocabulary with p < 1, p = 1, p > 1
    and p <= 0 (chunk masses)."""
    p = W.batch64_params(seed=seed, rows=rows, V=V)
    g = np.random.default_rng(seed)
    kinds = np.resize(np.arange(10), rows)
    g.shuffle(kinds)
    for r, kd in enumerate(kinds):
        if kd == 0:
            p["do_sample"][r] = 0
        elif kd == 1:
            p["top_k"][r] = g.choice([1, 5, 30, 64])
        elif kd == 2:
            p["top_k"][r] = 100
        elif kd == 3:
            p["pen"][r] = 0.7
        elif kd in (4, 5):
            p["top_k"][r] = 0
            p["top_p"][r] = g.choice([0.3, 0.8, 0.95, 0.999])
        elif kd == 6:
            p["top_k"][r], p["top_p"][r] = 0, 1.0
        elif kd == 7:
            p["top_k"][r], p["top_p"][r] = 0, 1.5
        elif kd == 8:
            p["top_k"][r], p["top_p"][r] = 0, 0.0
        else:
            p["top_k"][r], p["temp"][r] = V, 1.0
        if g.random() < 0.5:
            p["pen"][r] = 1.0 if p["pen"][r] != 0.7 else 0.7
    return p


# 8194: the two-phase stream with the pipelined row chain; from 8233 on the
# pipelined chain no longer fits in LDS and the single-kernel stream runs.
@pytest.mark.parametrize("V,rows,steps", [(8194, 40, 60), (1000, 30, 80), (37, 20, 50), (3000, 25, 70),
                                          (8233, 24, 40), (9216, 30, 60), (10092, 20, 40), (10093, 12, 30),
                                          (12288, 20, 40)])
def test_stream_two_phase_all_modes(orc, gpu_ctx, V, rows, steps):
    p = _mixed_params(V + rows, rows, V)
    x = W.batch64_logits(V + 7, steps, rows, V)
    print(f"two-phase V={V} rows={rows} steps={steps}", flush=True)
    toks, rng, st = run_stream(gpu_ctx, p, x, stop_token=V - 1)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], stop_token=V - 1,
                                    n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:5].tolist()}"
    assert np.array_equal(rng, orng)
    stoks, srng, _ = run_stream(gpu_ctx, p, x, stop_token=V - 1, sequential=True)
    assert np.array_equal(stoks, toks) and np.array_equal(srng, rng)
    print("exact steps per row", st[:, 1].tolist())


@pytest.mark.parametrize("V", [8194, 9216, 12288])
def test_stream_overlapped_chunks(orc, gpu_ctx, V):
    """A stream long enough for several chunks whose scans run beside the
    previous chunk's chains on their own CUs: every row mode, stop tokens
    planted in later chunks, against the oracle and the single-kernel stream
    (at 9216 and 12288 the single-kernel stream runs for both calls)."""
    steps, rows = 300, 48
    p = _mixed_params(4242 + V, rows, V)
    x = W.batch64_logits(4243 + V, steps, rows, V)
    stop = V - 1
    for s, r in [(130, 0), (255, 3), (256, 9), (299, 12)]:
        x[s, r, stop] = 80.0
        p["top_k"][r], p["pen"][r], p["do_sample"][r] = 1, 1.0, 1
    # full-vocabulary rows without penalty run in step segments: stops inside
    # a later segment, the first chunk and a segment's first step
    for s, r in [(200, 20), (40, 21), (64, 22), (161, 23)]:
        x[s, r, stop] = 80.0
        p["top_k"][r], p["top_p"][r], p["pen"][r], p["do_sample"][r] = 0, 0.9, 1.0, 1
    print(f"overlapped stream V={V} rows={rows} steps={steps}", flush=True)
    toks, rng, st = run_stream(gpu_ctx, p, x, stop_token=stop)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], stop_token=stop,
                                    n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:5].tolist()}"
    assert np.array_equal(rng, orng)
    assert toks[130, 0] == stop and (toks[131:, 0] == -1).all()
    assert (toks[201:, 20] == -1).all()
    stoks, srng, _ = run_stream(gpu_ctx, p, x, stop_token=stop, sequential=True)
    assert np.array_equal(stoks, toks) and np.array_equal(srng, rng)


@pytest.mark.parametrize("rows,steps", [(64, 260), (65, 260), (80, 260), (1, 300)])
def test_stream_row_counts(orc, gpu_ctx, rows, steps):
    """Row counts around the overlapped stream's limit on a 256-CU device (64
    rows: chains and scans on their CU sets; 65 and more: one chunk on every
    CU) and a single row, every row mode, against the oracle."""
    V = 8194
    p = _mixed_params(5151 + rows, rows, V)
    x = W.batch64_logits(5152 + rows, steps, rows, V)
    stop = V - 1
    for s, r in [(steps - 1, 0), (100, rows - 1), (200, rows // 2)]:
        x[s, r, stop] = 80.0
    print(f"stream V={V} rows={rows} steps={steps}", flush=True)
    toks, rng, st = run_stream(gpu_ctx, p, x, stop_token=stop)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], stop_token=stop,
                                    n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:5].tolist()}"
    assert np.array_equal(rng, orng)


def test_stream_stop_token_and_greedy(orc, gpu_ctx):
    steps, rows, V = 40, 16, 2000
    p = W.batch64_params(seed=9, rows=rows, V=V)
    p["do_sample"][::4] = 0
    x = W.batch64_logits(99, steps, rows, V)
    for s, r in [(3, 1), (10, 2), (20, 5), (0, 7)]:
        x[s, r, 17] = 80.0
        p["top_k"][r] = 1
        p["pen"][r] = 1.0
    toks, rng, st = run_stream(gpu_ctx, p, x, stop_token=17)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], stop_token=17)
    assert np.array_equal(toks, otoks)
    assert np.array_equal(rng, orng)
    assert (toks[1:, 7] == -1).all() and toks[0, 7] == 17


def test_per_step_launches_match_stream(orc, gpu_ctx):
    """Driving c4s_sample_rows step by step with a host-grown history gives the
    stream's tokens (the AR-loop integration of the batched entry point)."""
    import torch
    steps, rows = 6, 64
    p = W.batch64_params(seed=2)
    x = W.batch64_logits(1002, steps)
    hist = [list(p["hist_ids"][p["hist_off"][r]:p["hist_off"][r + 1]]) for r in range(rows)]
    rng = dev(p["rng"], torch)
    got = np.zeros((steps, rows), np.int32)
    for s in range(steps):
        ids, off = W.csr(hist)
        tok = torch.zeros(rows, dtype=torch.int32, device="cuda")
        gpu_ctx.sample_rows(dev(x[s], torch), dev(ids, torch), dev(off, torch), dev(p["temp"], torch),
                            dev(p["top_k"], torch), dev(p["top_p"], torch), dev(p["pen"], torch),
                            rng, tok, do_sample=dev(p["do_sample"], torch))
        got[s] = tok.cpu().numpy()
        for r in range(rows):
            hist[r].append(int(got[s, r]))
    otoks, _ = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                 p["top_p"], p["pen"], p["do_sample"], p["rng"], n_threads=16)
    assert np.array_equal(got, otoks)


@pytest.mark.parametrize("kind", ["nucleus", "dense", "mixed", "list"])
def test_stream_speculative_chain(orc, gpu_ctx, kind):
    """Rows decided several steps ahead and checked in order (the default
    two-phase path) against the oracle and against the chains that decide one
    step after the other: penalised full-vocabulary nucleus rows whose cut
    often moves with the tokens drawn since (many steps decided again, and
    exact-chain steps that stop every wave of the row), dense rows (p = 1 and
    p > 1), rows without penalty, greedy and top-k rows (decided again when a
    token drawn since is one of their survivors), and stop tokens planted
    mid-stream."""
    steps, rows, V = 300, 24, 8194
    p = W.batch64_params(seed=777, rows=rows, V=V)
    g = np.random.default_rng(778)
    p["top_k"][:] = 0
    if kind == "nucleus":
        p["top_p"][:] = g.choice(np.array([0.5, 0.8, 0.9, 0.95], np.float32), rows)
        p["pen"][:] = 10.0
    elif kind == "dense":
        p["top_p"][:] = g.choice(np.array([1.0, 1.2], np.float32), rows)
        p["pen"][:] = g.choice(np.array([1.3, 10.0], np.float32), rows)
    elif kind == "mixed":
        p["top_p"][:] = g.choice(np.array([0.0, 0.3, 0.9, 1.0], np.float32), rows)
        p["pen"][:] = g.choice(np.array([1.0, 1.2, 10.0], np.float32), rows)
    else:
        p["top_k"][:] = g.choice(np.array([1, 2, 5, 20, 50, 64], np.int32), rows)
        p["top_p"][:] = g.choice(np.array([0.5, 0.9, 1.0], np.float32), rows)
        p["pen"][:] = g.choice(np.array([1.0, 1.5, 10.0], np.float32), rows)
        p["do_sample"][::5] = 0   # greedy rows
    x = W.batch64_logits(779, steps, rows, V)
    if kind == "list":   # narrow rows: the penalised ids often come back among the survivors
        x[:, :, :256] += 6.0
    stop = V - 1
    for s, r in [(37, 2), (150, 5), (299, 7), (64, 11)]:
        x[s, r, stop] = 80.0
    print(f"speculative chain {kind}: gpu", flush=True)
    toks, rng, st = run_stream(gpu_ctx, p, x, stop_token=stop)
    ptoks, prng, pst = run_stream(gpu_ctx, p, x, stop_token=stop, speculate=False)
    print(f"speculative chain {kind}: oracle", flush=True)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"], p["top_p"],
                                    p["pen"], p["do_sample"], p["rng"], stop_token=stop, n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first (step, row) {bad[:5].tolist()}"
    assert np.array_equal(rng, orng)
    assert np.array_equal(ptoks, toks) and np.array_equal(prng, rng)
    assert not (st[:, 0].astype(np.uint32) & (1 << 30)).any()   # no row gave up waiting
    print("exact steps", int(st[:, 1].sum()), "per row", st[:, 1].tolist())


@pytest.mark.parametrize("steps", [1024, 1025])
def test_stream_speculation_limit(orc, gpu_ctx, steps):
    """The speculative chains' step limit: 1024 steps is the longest call they
    take (the drawn list and the 16-bit step fields at their largest), 1025 takes
    the one-step-at-a-time chains on the overlapped schedule. Penalised rows of
    every mode against the oracle, no row giving up."""
    rows, V = 8, 8194
    p = W.batch64_params(seed=4242, rows=rows, V=V)
    g = np.random.default_rng(4243)
    p["top_k"][:] = g.choice(np.array([0, 0, 20, 50], np.int32), rows)
    p["top_p"][:] = g.choice(np.array([0.8, 0.9, 1.0], np.float32), rows)
    p["pen"][:] = g.choice(np.array([1.0, 10.0], np.float32), rows)
    p["do_sample"][3] = 0
    x = W.batch64_logits(4244, steps, rows, V)
    print(f"speculation limit {steps}: gpu", flush=True)
    toks, rng, st = run_stream(gpu_ctx, p, x)
    print(f"speculation limit {steps}: oracle", flush=True)
    otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"], p["top_p"],
                                    p["pen"], p["do_sample"], p["rng"], n_threads=16)
    bad = np.argwhere(toks != otoks)
    assert bad.size == 0, f"{len(bad)} mismatches, first (step, row) {bad[:5].tolist()}"
    assert np.array_equal(rng, orng)
    assert not (st[:, 0].astype(np.uint32) & (1 << 30)).any()
    assert gpu_ctx.stream_status() == 0


@pytest.mark.parametrize("steps", [128, 256])
def test_stream_wait_expired_is_an_error(orc, steps):
    """A speculative chain whose bounded wait gives up stops its row; the call
    that follows reports it. The give-up is forced from the host (one poll a
    wait: every checking wave gives up at its first wait and every kernel ends
    normally). 128 steps run on the non-overlapped schedule, 256 on the
    overlapped one. After the report the same context decides bit-exactly again."""
    import torch

    import c4s
    rows, V = 8, 8194
    p = W.batch64_params(seed=2, rows=rows, V=V)
    p["top_k"][::2] = 0          # full-vocabulary rows (k_stream_spec) and top-k rows (k_stream_lspec)
    x = W.batch64_logits(1003, steps, rows, V)
    ctx = c4s.Context(0)
    try:
        ctx.set_wait_limit(1)
        print(f"wait expired {steps}: forced give-up", flush=True)
        toks, rng, st = run_stream(ctx, p, x)
        gave_up = (st[:, 0].astype(np.uint32) >> 30) & 1
        assert gave_up.all(), st[:, 0].tolist()
        assert (toks[-1] == -1).all()              # stopped rows write -1 to the end of the call
        assert ctx.stream_status() == c4s.ETIMEOUT
        assert ctx.stream_status() == c4s.OK       # the report clears the record
        # reported by the next call, which queues nothing
        run_stream(ctx, p, x)
        torch.cuda.synchronize()
        out = torch.full((steps, rows), -9, dtype=torch.int32, device="cuda")
        with pytest.raises(c4s.C4SError, match="code 4"):
            ctx.sample_stream(dev(x, torch), dev(p["hist_ids"], torch), dev(p["hist_off"], torch),
                              dev(p["temp"], torch), dev(p["top_k"], torch), dev(p["top_p"], torch),
                              dev(p["pen"], torch), dev(p["rng"], torch), out,
                              do_sample=dev(p["do_sample"], torch))
        torch.cuda.synchronize()
        assert (out.cpu().numpy() == -9).all()
        # the default limit again: bit-exact, nothing to report
        ctx.set_wait_limit(0)
        print(f"wait expired {steps}: default limit", flush=True)
        toks, rng, st = run_stream(ctx, p, x)
        otoks, orng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"], p["top_p"],
                                        p["pen"], p["do_sample"], p["rng"], n_threads=16)
        assert np.array_equal(toks, otoks) and np.array_equal(rng, orng)
        assert ctx.stream_status() == c4s.OK
    finally:
        ctx.close()
