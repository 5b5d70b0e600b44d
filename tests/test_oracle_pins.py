"""Pins for the oracle functions that the HF goldens leave open.

Each check comes from mathematics or from an independent computation, chosen
so that a plausible mistake (a wrong shift or direction, an off-by-one rank,
a reversed sort, a dropped min_keep, a draw in the wrong order) fails:

* xorshift64 (text2semantic.cpp:158: x ^= x << 13; x ^= x >> 7; x ^= x << 17):
  the map is linear over GF(2). Its matrix, read off the oracle on the 64
  basis vectors, must equal the product (I + L^17)(I + R^7)(I + L^13) built
  from explicit shift matrices, and must differ from every other order and
  direction of the same three shifts (Marsaglia's eight line variants of a
  full-period triple all have order 2^64-1, so the period alone cannot tell
  them apart). The period check stays as a second, independent property.
* seeds (text2semantic.cpp:109, :292-294): literal constants.
* top_k (sampling.cpp:30-40): threshold by full sort, ties kept.
* top_p (sampling.cpp:42-71): exact rational arithmetic on tiny rows, and the
  nucleus invariants (value suffix, mass >= p, minimality) on full rows.
* argmax (sampling.cpp:73-76): numpy's first-occurrence argmax.
* draw (text2semantic.cpp:150-165): closed form on exactly representable
  weights, and a chi-square test of the draw distribution against softmax.
* chain / stream: composition of the single-processor functions.
* LM head: float64 numpy LayerNorm + GEMV.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from xorshift_pin import REF_STEPS, advance, to_bits, from_bits
from xorshift_pin import xorshift_matrix as _xorshift_matrix

U64 = (1 << 64) - 1


# ---- RNG ---------------------------------------------------------------------------
def _gf2_matrix(orc):
    cols = [orc.xorshift64(1 << i) for i in range(64)]
    M = np.zeros((64, 64), dtype=np.int64)
    for j, c in enumerate(cols):
        for i in range(64):
            M[i, j] = (c >> i) & 1
    return M


def _matpow(M, e):
    R = np.eye(64, dtype=np.int64)
    B = M.copy()
    while e:
        if e & 1:
            R = (R @ B) % 2
        B = (B @ B) % 2
        e >>= 1
    return R


def test_xorshift_shift_order_and_directions(orc):
    import itertools
    M = _gf2_matrix(orc)
    assert (M == _xorshift_matrix(REF_STEPS)).all()
    same = []
    for perm in itertools.permutations([13, 7, 17]):
        for dirs in itertools.product([True, False], repeat=3):
            steps = list(zip(perm, dirs))
            if (_xorshift_matrix(steps) == M).all():
                same.append(steps)
    assert same == [REF_STEPS], same
    # wrong amounts fail as well
    for steps in ([(12, True), (7, False), (17, True)], [(13, True), (8, False), (17, True)]):
        assert not (_xorshift_matrix(steps) == M).all()


def test_xorshift_known_answers(orc):
    """The seeds' streams (text2semantic.cpp:109, :292-294) from the shift-matrix
    construction, 2000 steps each, against the oracle step by step."""
    A = _xorshift_matrix(REF_STEPS)
    for seed in [0x9E3779B97F4A7C15, 1234, (0x9E3779B97F4A7C15 + 63 * 0x100000001B3) & U64, 1]:
        v = to_bits(seed)
        t = seed
        for n in range(2000):
            v = (A @ v) % 2
            t = orc.xorshift64(t)
            if n % 97 == 0 or n == 1999:
                assert from_bits(v) == t
        assert advance(seed, 2000) == t


def test_xorshift_linear(orc):
    rng = np.random.default_rng(7)
    for _ in range(50):
        a, b = (int(x) for x in rng.integers(0, 2**63, size=2, dtype=np.int64))
        a |= 1 << 63
        assert orc.xorshift64(a ^ b) == orc.xorshift64(a) ^ orc.xorshift64(b)


def test_xorshift_full_period(orc):
    M = _gf2_matrix(orc)
    I = np.eye(64, dtype=np.int64)
    assert (_matpow(M, U64) == I).all()
    for q in (3, 5, 17, 257, 641, 65537, 6700417):   # 2^64-1 = 3*5*17*257*641*65537*6700417
        assert not (_matpow(M, U64 // q) == I).all()


def test_xorshift_matches_matrix(orc):
    M = _gf2_matrix(orc)
    s = 0x9E3779B97F4A7C15
    v = np.array([(s >> i) & 1 for i in range(64)], dtype=np.int64)
    t = s
    for _ in range(1000):
        t = orc.xorshift64(t)
    w = (_matpow(M, 1000) @ v) % 2
    assert sum(int(b) << i for i, b in enumerate(w)) == t


def test_seeds(orc):
    assert orc.seed_single(0) == 0x9E3779B97F4A7C15
    assert orc.seed_single(1234) == 1234
    s = orc.seed_batch(1234, 4)
    assert [int(x) for x in s] == [(1234 + b * 0x100000001B3) & U64 for b in range(4)]
    s0 = orc.seed_batch(0, 3)
    assert [int(x) for x in s0] == [(0x9E3779B97F4A7C15 + b * 0x100000001B3) & U64 for b in range(3)]


# ---- processors ------------------------------------------------------------------------
def test_penalty_closed_form(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300) * 3).astype(np.float32)
    x[5] = 0.0
    x[6] = -0.0
    ids = np.array([5, 6, 7, 7, 7, -1, 300, 299, 10, 10, 11], dtype=np.int32)
    got = orc.repetition_penalty(x, ids, 2.5)
    want = x.copy()
    for i in sorted(set(int(t) for t in ids if 0 <= t < 300)):
        want[i] = x[i] * np.float32(2.5) if x[i] < 0 else x[i] / np.float32(2.5)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(orc.repetition_penalty(x, ids, 1.0), x)
    # a history given once or many times penalises once
    u = np.unique(ids)
    assert np.array_equal(orc.repetition_penalty(x, u, 2.5), got)


def test_temperature_noops(orc):
    x = np.linspace(-3, 3, 17, dtype=np.float32)
    for t in (1.0, 0.0, -2.0):
        assert np.array_equal(orc.temperature(x, t), x)
    assert np.array_equal(orc.temperature(x, 0.7), (x / np.float32(0.7)).astype(np.float32))


def test_top_k_by_sort(orc):
    rng = np.random.default_rng(2)
    for trial in range(40):
        n = int(rng.integers(1, 200))
        x = rng.integers(-5, 6, size=n).astype(np.float32)   # many ties
        k = int(rng.integers(-1, n + 2))
        got = orc.top_k(x, k)
        if k <= 0 or k >= n:
            assert np.array_equal(got, x)
            continue
        thresh = np.sort(x)[::-1][k - 1]
        want = np.where(x < thresh, -np.inf, x).astype(np.float32)
        assert np.array_equal(got, want)
        assert np.isfinite(got).sum() >= k


def _exact_top_p_keep(x, p, min_keep):
    """Kept mask via exact rational arithmetic over libm exp values, or None if a
    cumulative sum lies within 1e-12 of the cut (rounding could decide)."""
    n = x.size
    order = sorted(range(n), key=lambda i: (float(x[i]), -i))   # ascending, ties: higher id first
    vmax = np.float32(x.max())
    e = [Fraction(math.exp(float(np.float32(x[i] - vmax)))) for i in order]
    S = sum(e)
    thr = Fraction(1.0 - float(np.float32(p)))
    cum = Fraction(0)
    remove = []
    for j in range(n):
        cum += e[j] / S
        if abs(cum - thr) < Fraction(1, 10**12):
            return None
        remove.append(cum <= thr)
    for j in range(max(0, n - min_keep), n):
        remove[j] = False
    keep = np.ones(n, dtype=bool)
    for j, r in enumerate(remove):
        if r:
            keep[order[j]] = False
    return keep


def test_top_p_exact_rational(orc):
    rng = np.random.default_rng(3)
    checked = 0
    for trial in range(300):
        n = int(rng.integers(1, 12))
        x = (rng.standard_normal(n) * rng.uniform(0.2, 4)).astype(np.float32)
        if trial % 3 == 0:
            x = np.round(x).astype(np.float32)                   # ties
        if trial % 7 == 0 and n > 2:
            x[rng.integers(0, n)] = -np.inf
        p = float(rng.choice([0.0, 0.1, 0.3, 0.5, 0.8, 0.95, 1.0, 1.5]))
        mk = int(rng.choice([0, 1, 1, 1, 2, 3]))
        keep = _exact_top_p_keep(x, p, mk)
        if keep is None:
            continue
        got = orc.top_p(x, p, mk)
        want = np.where(keep, x, -np.inf).astype(np.float32)
        assert np.array_equal(np.isneginf(got), np.isneginf(want)), (x, p, mk)
        assert np.array_equal(got[~np.isneginf(got)], want[~np.isneginf(want)])
        checked += 1
    assert checked > 250


def test_top_p_invariants_full_rows(orc):
    rng = np.random.default_rng(4)
    for trial in range(30):
        n = 8194
        x = (rng.standard_normal(n) * rng.uniform(0.5, 4)).astype(np.float32)
        p = float(rng.uniform(0.05, 0.99))
        got = orc.top_p(x, p)
        kept = ~np.isneginf(got)
        assert kept.sum() >= 1 and kept[np.argmax(x)]
        # value suffix: every kept value >= every removed value
        if (~kept).any():
            assert x[kept].min() >= x[~kept].max()
        e = np.exp((x - x.max()).astype(np.float64))
        S = e.sum()
        mk = e[kept].sum()
        assert mk >= p * S * (1 - 1e-9)
        smallest = np.argmin(np.where(kept, x, np.inf))
        assert mk - e[smallest] < p * S * (1 + 1e-9)
        # monotone in p
        got2 = orc.top_p(x, min(0.999, p + 0.05))
        assert (~np.isneginf(got2))[kept].all()


def test_top_p_ties_lower_id_survives(orc):
    x = np.zeros(10, dtype=np.float32)
    got = orc.top_p(x, 0.35)      # 10 equal weights: 4 survive (cum of 6 removed = 0.6 <= 0.65)
    assert list(np.flatnonzero(~np.isneginf(got))) == [0, 1, 2, 3]


def test_top_p_literal_sort_differs_only_inside_the_cut_tie_group(orc):
    """The reference's value-only std::sort (this host's libstdc++) against the
    declared order (lower id survives) on the tie-heavy bf16 workload: the same
    number of ids survive, and the kept sets differ only among ids whose value
    equals the smallest kept value (the tie group the nucleus cut falls in)."""
    import c4s_workloads as W
    b = W.bf16_ties(seed=3, rows=64, sweep="top_p")
    x = W.bf16_bits_to_f32(b.logits)
    differ = 0
    for r in range(b.n_rows):
        a = orc.top_p(x[r], 0.5)
        lit = orc.top_p(x[r], 0.5, literal=True)
        ka, kl = np.isfinite(a), np.isfinite(lit)
        assert ka.sum() == kl.sum()
        if not np.array_equal(ka, kl):
            differ += 1
            cut = x[r][ka].min()
            assert x[r][ka].min() == x[r][kl].min() == cut
            assert (x[r][ka ^ kl] == cut).all()
    print(f"literal std::sort keeps other ids in {differ}/{b.n_rows} rows")


def test_argmax_first_max(orc):
    rng = np.random.default_rng(5)
    for trial in range(50):
        x = rng.integers(-3, 4, size=int(rng.integers(1, 100))).astype(np.float32)
        assert orc.argmax(x) == int(np.argmax(x))
    assert orc.argmax(np.array([-0.0, 0.0, 0.0], np.float32)) == 0


def _u_after(orc, state):
    s = orc.xorshift64(state)
    return (s >> 11) / float(1 << 53), s


def test_draw_closed_form(orc):
    x = np.array([0.0, -np.inf, 0.0, 0.0], dtype=np.float32)   # weights 1, 0, 1, 1
    for state in [1234, 5, 0x9E3779B97F4A7C15, 77, 123456789, 2**40 + 3]:
        u, s_new = _u_after(orc, state)
        r = u * 3.0
        want = 0 if r <= 1.0 else (2 if r <= 2.0 else 3)
        tok, st = orc.draw(x, state)
        assert (tok, st) == (want, s_new)
    # all weight on one id
    y = np.full(9, -np.inf, np.float32)
    y[6] = 3.5
    for state in range(1, 20):
        assert orc.draw(y, state)[0] == 6


def test_draw_distribution(orc):
    x = np.array([0.0, 1.0, -np.inf, 0.5, -1.0, 2.0], dtype=np.float32)
    pr = np.exp(x - x.max())
    pr = pr / pr.sum()
    counts = np.zeros(x.size)
    state = 1234
    N = 60000
    for _ in range(N):
        tok, state = orc.draw(x, state)
        counts[tok] += 1
    assert counts[2] == 0
    nz = pr > 0
    chi2 = (((counts[nz] - N * pr[nz]) ** 2) / (N * pr[nz])).sum()
    assert chi2 < 30.0, (counts, N * pr)    # 4 dof, p ~ 5e-6


def test_chain_is_composition(orc):
    import c4s_workloads as W
    b = W.batch64(seed=11, rows=12)
    toks, rng2, masked = orc.sample_rows(b.logits, b.hist_ids, b.hist_off, b.temp, b.top_k,
                                         b.top_p, b.pen, b.do_sample, b.rng)
    for r in range(12):
        h = b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]]
        v = orc.repetition_penalty(b.logits[r], h, b.pen[r])
        v = orc.temperature(v, b.temp[r])
        v = orc.top_k(v, int(b.top_k[r]))
        v = orc.top_p(v, b.top_p[r])
        tok, st = orc.draw(v, int(b.rng[r]))
        assert tok == toks[r] and st == int(rng2[r])
        assert np.array_equal(v.view(np.uint32), masked[r].view(np.uint32))


def test_stream_is_repeated_steps(orc):
    import c4s_workloads as W
    rows, steps, V = 6, 5, 300
    p = W.batch64_params(seed=12, rows=rows, V=V, h_lo=0, h_hi=20)
    x = W.batch64_logits(13, steps, rows, V)
    x[2, 1, 7] = 50.0                       # row 1 picks 7 at step 2 (then stops)
    p["top_k"][1] = 1
    p["pen"][1] = 1.0
    toks, rng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"], p["top_p"],
                                  p["pen"], p["do_sample"], p["rng"], stop_token=7)
    hist = [list(p["hist_ids"][p["hist_off"][r]:p["hist_off"][r + 1]]) for r in range(rows)]
    state = p["rng"].copy()
    done = [False] * rows
    for s in range(steps):
        for r in range(rows):
            if done[r]:
                assert toks[s, r] == -1
                continue
            v = orc.repetition_penalty(x[s, r], np.array(hist[r], np.int32), p["pen"][r])
            v = orc.temperature(v, p["temp"][r])
            v = orc.top_k(v, int(p["top_k"][r]))
            v = orc.top_p(v, p["top_p"][r])
            t, st = orc.draw(v, int(state[r]))
            state[r] = st
            assert toks[s, r] == t
            if t == 7:
                done[r] = True
            else:
                hist[r].append(t)
    assert done[1]
    assert np.array_equal(state, rng)


def test_lmhead_vs_numpy(orc):
    """LayerNorm (biased variance, eps) + linear (x @ W^T + b) against numpy in
    float64 (nn.cpp:73-83, :11-16), for each weight kind."""
    import c4s_workloads as W
    head, _ = W.lmhead(seed=3, M=4, D=128, V=50)
    x = W.bf16_bits_to_f32(head.hidden).astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    y = (x - mu) / np.sqrt(var + 1e-5) * head.gamma + head.beta
    logits, h = orc.ln_lmhead(head.hidden, head.gamma, head.beta, head.weight, head.bias, want_h=True)
    assert np.allclose(h, y, rtol=1e-6, atol=1e-7)
    want = y @ W.bf16_bits_to_f32(head.weight).astype(np.float64).T + head.bias
    assert np.allclose(logits, want, rtol=1e-6, atol=1e-6)
    # f32 weights
    g = np.random.default_rng(9)
    wf = (0.02 * g.standard_normal((50, 128))).astype(np.float32)
    got = orc.ln_lmhead(head.hidden, head.gamma, head.beta, wf, head.bias, wkind=orc.W_F32)
    assert np.allclose(got, y @ wf.astype(np.float64).T + head.bias, rtol=1e-6, atol=1e-6)
    # 8-bit affine groups of 64 along D: w = scale * q + bias per group
    q = g.integers(0, 256, size=(50, 128)).astype(np.uint8)
    sc = (0.001 * (1 + g.random((50, 2)))).astype(np.float32)
    bi = (-0.1 * g.random((50, 2))).astype(np.float32)
    wq = q.astype(np.float64) * np.repeat(sc, 64, axis=1) + np.repeat(bi, 64, axis=1)
    got = orc.ln_lmhead(head.hidden, head.gamma, head.beta, q, head.bias, wkind=orc.W_Q8, wscale=sc, wbias=bi,
                        group=64)
    assert np.allclose(got, y @ wq.T + head.bias, rtol=1e-6, atol=1e-6)
