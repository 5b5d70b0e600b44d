"""GPU parity: the HIP sampling path vs the CPU oracle, bit for bit.

Tokens, RNG states and the masked rows (the row state before argmax/draw) must
be identical. Each workload runs at a size the oracle finishes in seconds.
"""
import numpy as np
import pytest

import c4s
import c4s_workloads as W
from gpu_util import assert_same_rows, compare_with_oracle, dev, gpu_rows

pytestmark = pytest.mark.gpu


def test_single_row_sampled_and_greedy(orc, gpu_ctx):
    samp, greedy = W.single_row(seed=1)
    print("single_row sampled", flush=True)
    compare_with_oracle(orc, gpu_ctx, samp)
    print("single_row greedy", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, greedy)
    assert tok[0] == orc.argmax(orc.repetition_penalty(greedy.logits[0],
                                                       greedy.hist_ids, 10.0))


@pytest.mark.parametrize("masked", [True, False])
@pytest.mark.parametrize("seed", [2, 21, 22])
def test_batch64_one_step(orc, gpu_ctx, seed, masked):
    b = W.batch64(seed=seed, rows=64)
    print(f"batch64 seed={seed} masked={masked}", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=masked)
    print("exact top_p passes", int(st[:, 1].sum()), "exact draws", int(st[:, 2].sum()))
    one_pass = (st[:, 0] & 16) != 0
    print("rows decided in one pass", int(one_pass.sum()), "of", b.n_rows)
    assert one_pass.mean() > 0.9


@pytest.mark.parametrize("masked", [True, False])
def test_long_histories(orc, gpu_ctx, masked):
    """Histories of 1500-3000 ids (more than two per thread of the step's 512):
    every id past the first 1024 of a row joins the penalty set in the
    step's loop after the first two per thread."""
    p = W.batch64_params(seed=61, rows=16, h_lo=1500, h_hi=3000)
    b = W.Batch(logits=W.batch64_logits(1061, 1, 16)[0], **p)
    assert int(np.diff(b.hist_off).min()) > 1024
    print(f"long histories masked={masked}", flush=True)
    compare_with_oracle(orc, gpu_ctx, b, masked=masked)


def test_batch64_general_rows(orc, gpu_ctx):
    """top_k = 0 rows (full-vocabulary nucleus) with assorted p and temperatures."""
    b = W.batch64(seed=31, rows=64)
    b.top_k[:] = 0
    b.top_p[:] = np.resize(np.array([0.5, 0.8, 0.9, 0.95, 0.99, 1.0, 0.2, 0.999], np.float32), 64)
    b.temp[:] = np.resize(np.array([0.6, 1.2, 1.0, 2.0, 0.3], np.float32), 64)
    compare_with_oracle(orc, gpu_ctx, b)


@pytest.mark.parametrize("masked", [True, False])
def test_nucleus_rows_many(orc, gpu_ctx, masked):
    """1024 full-vocabulary nucleus rows (p 0.8-0.99, assorted temperatures and
    penalties): boundaries from a few entries to several hundred (the one-wave
    sort, the rank-counted sorts of up to 128 and 256 entries, the network
    across waves), and cuts close enough to the error bound that the masses are
    taken again in double."""
    b = W.batch64(seed=71, rows=1024)
    b.top_k[:] = 0
    b.top_p[:] = np.resize(np.array([0.8, 0.9, 0.95, 0.99, 0.85], np.float32), 1024)
    print(f"nucleus rows x1024 masked={masked}", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=masked)
    print("exact top_p passes", int(st[:, 1].sum()))
    assert ((st[:, 0] & 16) != 0).mean() > 0.9
    assert st[:, 1].sum() > 0


def test_draw_in_double(orc, gpu_ctx):
    """Draws that the fp32 masses cannot settle go to double: a row of 5 kept
    ids whose r lies 2^-23.7 (relative) from a boundary (one wave, the kept ids
    in id order), and flat rows of thousands of kept ids (the owner's wave)."""
    b = W.batch64(seed=2, rows=64)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=False)
    assert st[0, 3] == 5 and st[0, 2] >= 1, st[0].tolist()
    f = W.batch64(seed=81, rows=1024)
    g = np.random.default_rng(82)
    f.logits[:] = (0.3 * g.standard_normal(f.logits.shape)).astype(np.float32)
    f.top_k[:] = 0
    f.top_p[:] = np.resize(np.array([0.95, 0.99, 1.0, 0.9], np.float32), 1024)
    print("flat rows x1024 for the draw in double", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, f, masked=False)
    wide = (st[:, 2] >= 1) & (st[:, 3] > 64)
    print("draws in double with more than 64 kept ids:", int(wide.sum()))
    assert wide.any()


@pytest.mark.parametrize("masked", [True, False])
@pytest.mark.parametrize("shape,sigma", [("gauss", 0.3), ("gauss", 0.7), ("gauss", 1.5), ("gauss", 1e-4),
                                         ("cluster", 0.02), ("cluster", 0.2)])
def test_flat_rows_refined_boundary(orc, gpu_ctx, shape, sigma, masked):
    """Narrow logit ranges (an LM head's output): hundreds of entries share the
    boundary bucket of the nucleus cut or of the k-th value, so the one-pass
    step refines the boundary buckets in a second histogram. "cluster": a
    tight cluster and a few values 40 below it. sigma 1e-4: every entry in one
    bucket and nearly all in one sub-bucket (more than one sort takes, not one
    value: the multi-pass chain decides)."""
    b = W.batch64(seed=40, rows=64)
    g = np.random.default_rng(41)
    b.logits[:] = (sigma * g.standard_normal(b.logits.shape)).astype(np.float32)
    if shape == "cluster":
        b.logits[:, 1::2000] = -40.0
    b.top_k[:] = np.resize(np.array([0, 0, 0, 50, 200, 0, 400, 0], np.int32), 64)
    b.top_p[:] = np.resize(np.array([0.9, 0.8, 0.95, 1.0, 0.9, 0.5, 1.0, 0.99], np.float32), 64)
    print(f"flat rows {shape} sigma={sigma} masked={masked}", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=masked)
    one_pass = (st[:, 0] & 16) != 0
    print("rows decided in one pass", int(one_pass.sum()), "of", b.n_rows)
    for i in np.flatnonzero(~one_pass):
        print(f"  row {i}: top_k {b.top_k[i]} top_p {b.top_p[i]} temp {b.temp[i]:.3f} pen {b.pen[i]} stats {st[i]}")
    if sigma >= 0.01:
        assert one_pass.mean() > 0.9


@pytest.mark.parametrize("masked", [True, False])
@pytest.mark.parametrize("sweep", ["greedy", "top_k1", "top_p"])
def test_bf16_ties(orc, gpu_ctx, sweep, masked):
    b = W.bf16_ties(seed=3, rows=1024, sweep=sweep)
    print(f"bf16_ties {sweep} masked={masked}", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=masked)
    if sweep == "top_k1":
        assert (st[:, 3] > 1).all()      # the tied maxima all survive top_k=1
    if sweep == "top_p":
        assert st[:, 1].sum() > 0        # rows whose nucleus cut falls in a tie take the exact sort


def _list_decided(st):
    """Rows the candidate-list step decided (statistics word 0, bit 5)."""
    return (st[:, 0] & 32) != 0


@pytest.mark.parametrize("seed", [2, 21])
def test_candidate_list_rows(orc, gpu_ctx, seed):
    """Sampled top-k rows with k <= 64 and no masked-row output are decided on
    a candidate list (every other row takes the one-pass step)."""
    b = W.batch64(seed=seed, rows=64)
    b.top_k[::7] = 64
    b.top_k[3::7] = 1
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=False)
    tk = (b.top_k >= 1) & (b.top_k <= 64) & (b.do_sample != 0)
    used = _list_decided(st)
    print("list rows", int(used.sum()), "of", int(tk.sum()), "top-k rows")
    assert not used[~tk].any()
    assert used[tk].mean() > 0.9


def test_candidate_list_production_defaults(orc, gpu_ctx):
    """The pipeline defaults on every row (pipeline.h:31-35: temperature 0.8,
    top_k 30, top_p 0.8, penalty 10) over ten AR steps, each step's token
    joining the history."""
    b = W.batch64(seed=9, rows=64)
    b.temp[:] = 0.8
    b.top_k[:] = 30
    b.top_p[:] = 0.8
    b.pen[:] = 10.0
    x = W.batch64_logits(77, 10, rows=64)
    hist = [list(b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]]) for r in range(64)]
    for s in range(10):
        b.logits = x[s]
        b.hist_ids, b.hist_off = W.csr([np.asarray(h, np.int32) for h in hist])
        tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=False)
        assert _list_decided(st).mean() > 0.9
        b.rng = gpu_rows(gpu_ctx, b, masked=False)[1]
        for r in range(64):
            hist[r].append(int(tok[r]))


def test_large_vocab(orc, gpu_ctx):
    b = W.large_vocab(seed=4, rows=256)
    print("large_vocab 256 rows", flush=True)
    compare_with_oracle(orc, gpu_ctx, b, masked=True)


def test_large_vocab_general_and_bf16(orc, gpu_ctx):
    b = W.large_vocab(seed=41, rows=8, V=20000, hist_len=300)
    b.top_k[:] = np.array([0, 0, 50, 0, 1, 0, 20000, 19999], np.int32)
    b.top_p[:] = np.array([0.9, 1.0, 0.95, 0.5, 1.0, 0.99, 0.7, 0.8], np.float32)
    b.do_sample[3] = 0
    compare_with_oracle(orc, gpu_ctx, b)
    b.logits = W.f32_to_bf16_bits(b.logits)
    compare_with_oracle(orc, gpu_ctx, b)


def test_large_vocab_one_wave_finish(orc, gpu_ctx):
    """Large-vocabulary top-k rows with at most 64 survivors decide top_p and
    the draw on one wave with parallel sums; a cut within the error margin
    goes to the sequential sums. Rows: two tied maxima at p = 0.5 (the cut
    lies exactly on the boundary: cum = 0.5 <= 1 - p), four tied maxima at
    p = 0.75, min_tokens_to_keep above the survivors' count, k = 64 with
    ties past the k-th value (65 survivors: the sequential path), and plain
    rows; tokens and masked rows bit for bit. Statistics bit 6 (read once) on
    every row."""
    V, n = 20000, 8
    b = W.large_vocab(seed=51, rows=n, V=V, hist_len=300)
    b.pen[:] = 1.0
    b.top_k[:] = np.array([2, 4, 10, 64, 50, 30, 5, 1], np.int32)
    b.top_p[:] = np.array([0.5, 0.75, 0.9, 0.95, 0.5, 0.3, 0.999, 0.8], np.float32)
    x = b.logits
    top = x.max(axis=1) + 3.0
    x[0, [11, 4000]] = top[0]
    x[1, [7, 19, 9000, 15000]] = top[1]
    x[3, 100:165] = top[3]   # 65 equal values at the top: all survive top_k = 64
    mk = np.array([1, 1, 12, 1, 1, 1, 1, 1], np.int32)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, min_keep=mk)
    assert ((st[:, 0] >> 6) & 1).all(), st[:, 0].tolist()


def _rows_from(rows, temp, top_k, top_p, pen, hist, do_sample=None, seed=1234):
    n = len(rows)
    V = max(len(r) for r in rows)
    x = np.full((n, V), -np.inf, np.float32)
    for i, r in enumerate(rows):
        x[i, :len(r)] = r
    ids, off = W.csr(hist)
    return W.Batch(logits=x, hist_ids=ids, hist_off=off, temp=np.asarray(temp, np.float32),
                   top_k=np.asarray(top_k, np.int32), top_p=np.asarray(top_p, np.float32),
                   pen=np.asarray(pen, np.float32),
                   do_sample=np.ones(n, np.uint8) if do_sample is None else np.asarray(do_sample, np.uint8),
                   rng=W.seed_batch(seed, n))


@pytest.mark.parametrize("masked", [True, False])
@pytest.mark.parametrize("V", [1, 2, 3, 63, 64, 65, 1000, 9216, 12288, 12289, 40000])
def test_vocab_sizes(orc, gpu_ctx, V, masked):
    g = np.random.default_rng(V)
    n = 24
    x = (g.standard_normal((n, V)) * 2).astype(np.float32)
    hist = [g.integers(-5, V + 5, size=int(g.integers(0, 50))).astype(np.int32) for _ in range(n)]
    ids, off = W.csr(hist)
    b = W.Batch(logits=x, hist_ids=ids, hist_off=off,
                temp=g.choice(np.array([0.7, 1.0, 1.3, 0.0, -1.0], np.float32), n),
                top_k=g.choice(np.array([0, 1, 2, 5, V - 1, V, V + 1, -3], np.int32), n),
                top_p=g.choice(np.array([0.0, 0.3, 0.8, 1.0, 1.2], np.float32), n),
                pen=g.choice(np.array([1.0, 1.3, 10.0, 0.5], np.float32), n),
                do_sample=(g.random(n) > 0.2).astype(np.uint8), rng=W.seed_batch(V, n))
    mk = g.choice(np.array([1, 1, 1, 0, 2, 7, V + 4], np.int32), n)
    compare_with_oracle(orc, gpu_ctx, b, min_keep=mk, masked=masked)


@pytest.mark.parametrize("masked", [True, False])
def test_edge_rows(orc, gpu_ctx, masked):
    ninf = -np.inf
    rows = [
        [ninf] * 16,                                        # all -inf
        [ninf, 1.0, ninf, 1.0, 0.5] + [ninf] * 11,          # -inf mixed, tie at max
        [0.0] * 16,                                         # all equal
        [-0.0, 0.0, -0.0, 0.0] * 4,                         # signed zeros
        [3.0, 3.0, 3.0, 1.0] * 4,                           # tie groups
        list(np.linspace(-1e30, 1e30, 16)),                 # huge range
        [-1e31] * 16,                                       # below the draw's -1e30 floor
        [5.0] + [-200.0] * 15,                              # underflowing weights
        [-800.0, 0.0, -745.0, -746.0, -744.0] + [-9000.0] * 11,
    ]
    n = len(rows)
    for temp, k, p in [(1.0, 0, 1.0), (0.8, 2, 0.5), (1.0, 1, 0.0), (2.0, 0, 0.3), (0.5, 3, 1.0), (0.8, 16, 0.8),
                       (1.0, 15, 1e-6)]:
        b = _rows_from(rows, [temp] * n, [k] * n, [p] * n, [1.0] * n, [[]] * n)
        compare_with_oracle(orc, gpu_ctx, b, masked=masked)
        for mk in (0, 2, 17):
            compare_with_oracle(orc, gpu_ctx, b, min_keep=np.full(n, mk, np.int32), masked=masked)


@pytest.mark.parametrize("masked", [True, False])
def test_row_active_and_mixed_greedy(orc, gpu_ctx, masked):
    b = W.batch64(seed=5, rows=64)
    b.do_sample[::3] = 0
    active = np.ones(64, np.uint8)
    active[::5] = 0
    tok, st = compare_with_oracle(orc, gpu_ctx, b, row_active=active, masked=masked)
    assert (tok[active == 0] == -1).all()


def test_custom_single_processors(orc, gpu_ctx):
    """The single-processor modes behind the legacy functions, on many rows."""
    import torch
    b = W.batch64(seed=6, rows=16)
    x = b.logits
    cases = [
        (c4s.P_TEMPERATURE, lambda r: orc.temperature(x[r], b.temp[r])),
        (c4s.P_PENALTY, lambda r: orc.repetition_penalty(
            x[r], b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]], b.pen[r])),
        (c4s.P_TOP_K, lambda r: orc.top_k(x[r], int(b.top_k[r]))),
        (c4s.P_TOP_P, lambda r: orc.top_p(x[r], b.top_p[r])),
    ]
    for bit, ref in cases:
        _, rng, m, _ = gpu_rows(gpu_ctx, b, mode=c4s.MODE_CUSTOM | bit)
        want = np.stack([ref(r) for r in range(16)])
        assert_same_rows(m, want)
        assert np.array_equal(rng, b.rng)           # no draw, RNG untouched
    tok, _, _, _ = gpu_rows(gpu_ctx, b, mode=c4s.MODE_CUSTOM | c4s.T_ARGMAX)
    assert list(tok) == [orc.argmax(x[r]) for r in range(16)]
    tok, rng, _, _ = gpu_rows(gpu_ctx, b, mode=c4s.MODE_CUSTOM | c4s.T_DRAW)
    for r in range(16):
        assert (tok[r], rng[r]) == orc.draw(x[r], int(b.rng[r]))


def test_host_helpers_match_oracle(orc, gpu_ctx):
    g = np.random.default_rng(8)
    for n in (1, 5, 64, 8194, 15000):
        x = (g.standard_normal(n) * 3).astype(np.float32)
        ids = g.integers(-2, n + 2, size=40).astype(np.int32)
        assert np.array_equal(gpu_ctx.host_temperature(x, 0.7), orc.temperature(x, 0.7))
        assert np.array_equal(gpu_ctx.host_repetition_penalty(x, ids, 1.3),
                              orc.repetition_penalty(x, ids, 1.3))
        assert np.array_equal(gpu_ctx.host_top_k(x, 10), orc.top_k(x, 10))
        for p, mk in ((0.9, 1), (0.3, 4), (1.0, 1)):
            assert np.array_equal(gpu_ctx.host_top_p(x, p, mk), orc.top_p(x, p, mk))
        assert gpu_ctx.host_argmax(x) == orc.argmax(x)
        y = orc.top_p(orc.top_k(x, 30), 0.8)
        assert gpu_ctx.host_draw(y, 1234) == orc.draw(y, 1234)
    assert gpu_ctx.host_argmax(np.zeros(0, np.float32)) == 0


def test_large_vocab_one_read_and_its_checks(orc, gpu_ctx):
    """Large-vocabulary top-k rows read once (statistics bit 6), all bit for bit
    against the oracle with the masked rows: six of the largest values in one
    thread's stream (its fourth candidate reaches the bound: its wave reads its
    stream again); the 60 largest values penalised below the bound (the bound
    is taken again further down); a value just under a key prefix whose
    quotient by the temperature ties the k-th largest one (0x3fc00200 and the
    float before it, divided by 0.75, both round to 2.0000813); ties at the
    k-th value kept; and a row whose largest values span more binades than the
    candidate bins, which the two passes over the row decide (bit 6 clear).
    V is odd, so the rows start at every 16-byte alignment (the head and tail
    entries a thread holds apart)."""
    rows, V = 6, 100003
    b = W.large_vocab(seed=43, rows=rows, V=V, hist_len=400)
    b.top_p[:] = np.array([0.95, 0.95, 0.9, 1.0, 1.0, 0.8], np.float32)
    head = [((16 - (r * V * 4) % 16) % 16) // 4 for r in range(rows)]
    nt = 1024

    def stream_ids(r, t, n):   # the first n ids of thread t's stream in row r
        return [head[r] + 4 * (t + nt * j) + e for j in range((n + 3) // 4) for e in range(4)][:n]
    # row 1: six of the top values in thread 5's stream
    for i, idx in enumerate(stream_ids(1, 5, 6)):
        b.logits[1, idx] = 30.0 + i
    # row 2: its 60 largest values are in the history, penalty 10
    top = np.argsort(b.logits[2])[::-1][:60]
    hist = [b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]] for r in range(rows)]
    hist[2] = np.concatenate([hist[2], top.astype(np.int32)])
    b.pen[2] = 10.0
    # row 3: 49 large values, then 17 copies of y_k (the smallest value of its
    # key prefix: ranks k to k + 16 at the bound's prefix) and the float below
    # it, whose quotients by T = 0.75 are equal
    g = np.random.default_rng(7)
    b.logits[3] = (0.1 * g.standard_normal(V) - 5.0).astype(np.float32)
    ids3 = g.permutation(V)[:67]
    b.logits[3, ids3[:49]] = (10.0 + 0.25 * np.arange(49)).astype(np.float32)
    b.logits[3, ids3[49:66]] = np.array([0x3FC00200], np.uint32).view(np.float32)[0]
    b.logits[3, ids3[66]] = np.array([0x3FC001FF], np.uint32).view(np.float32)[0]
    b.temp[3], b.pen[3] = 0.75, 1.0
    # row 4: k = 1 with three equal maxima
    b.logits[4, [17, 50001, 99999]] = 40.0
    b.top_k[4], b.pen[4] = 1, 1.0
    # row 5: its 80 largest values from 2^60 down by factors of two
    b.logits[5, g.permutation(V)[:80]] = np.ldexp(1.0, 60 - np.arange(80)).astype(np.float32)
    b.hist_ids, b.hist_off = W.csr(hist)
    print("large vocab one read: checks", flush=True)
    tok, st = compare_with_oracle(orc, gpu_ctx, b, masked=True)
    one = ((st[:, 0] >> 6) & 1).tolist()
    assert one[:3] == [1, 1, 1] and one[4:] == [1, 0], st[:, 0].tolist()
    assert st[4, 3] == 3 and st[3, 3] == 67     # ties kept: three maxima; every tied quotient survives
