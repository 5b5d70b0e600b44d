"""Seeded synthetic inputs for the T2S token-sampling path.

Five workloads, named by what they are:

* ``single_row``     -- one fp32 row, V=8194, N(0, 3^2) logits with 5 ids set to
  +12, history of 200 uniform ids, penalty 10, temperature 0.8, top_k 30,
  top_p 0.8, one seeded draw; plus a greedy argmax of the same row.
* ``batch64``        -- 64 rows, V=8194 fp32, N(0, 3^2) + 5 per-row spikes at +12
  for every step, per-row history of 50-800 ids and per-row parameters
  (temperature U[0.6, 1.2], top_k in {0, 20, 30, 50}, top_p in {1, 0.9, 0.8},
  penalty in {1, 10}); the AR stream runs many steps, each sampled id joining
  that row's history.
* ``bf16_ties``      -- 1024 rows, V=8194, Student-t(df=3) x 4 logits rounded to
  bf16, 820 ids per row (10%) set to the row maximum, 1000-id history;
  greedy / top_k=1 / top_p=0.5 sweeps.
* ``large_vocab``    -- 256 rows, V=151936, N(0, 2^2) plus a Zipf(1.1) boost
  10 * (rank+1)^-1.1 placed on a seeded permutation of ids; top_k 50,
  top_p 0.95, temperature 0.7, penalty 1.2, 2048-id history.
* ``lmhead``         -- 64 hidden states of dim 1280 (bf16, N(0,1)), LayerNorm
  (gamma ~ N(1, .02), beta ~ N(0, .02)), bf16 LM-head weight (8194 x 1280,
  N(0, .02^2)) and an fp32 bias, then the batch64 processor chain.

Rows are generated with numpy's PCG64 so the CPU oracle and the GPU see the
same bytes. Sizes are parameters so tests can shrink them.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

V_SEMANTIC = 8194          # semantic vocab incl. BOS 8192 / EOS 8193
STOP_TOKEN = 8193
DEFAULT_SEED = 1234        # production default seed (SynthOptions)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x7FFFFF) != 0)
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def seed_batch(seed: int, n: int) -> np.ndarray:
    """Per-row xorshift64 seeds of the batched AR loop: (seed or golden) + b * FNV prime."""
    base = np.uint64(seed if seed else 0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        return base + np.arange(n, dtype=np.uint64) * np.uint64(0x100000001B3)


def csr(histories) -> tuple[np.ndarray, np.ndarray]:
    off = np.zeros(len(histories) + 1, dtype=np.int64)
    off[1:] = np.cumsum([len(h) for h in histories])
    ids = np.concatenate([np.asarray(h, dtype=np.int32) for h in histories]) if len(histories) else \
        np.zeros(0, np.int32)
    return ids.astype(np.int32), off


@dataclass
class Batch:
    """One AR step's worth of rows (or many steps for a stream)."""
    logits: np.ndarray              # [rows, V] f32 or uint16 bf16 bits; or [steps, rows, V]
    hist_ids: np.ndarray            # CSR ids (int32)
    hist_off: np.ndarray            # CSR offsets (int64, rows+1)
    temp: np.ndarray
    top_k: np.ndarray
    top_p: np.ndarray
    pen: np.ndarray
    do_sample: np.ndarray
    rng: np.ndarray                 # uint64 per row
    min_keep: np.ndarray | None = None
    meta: dict = field(default_factory=dict)

    @property
    def n_rows(self):
        return self.temp.shape[0]


def _spiked_normal(g, rows, V, sigma, n_spikes=5, spike=12.0):
    x = (g.standard_normal((rows, V), dtype=np.float32) * np.float32(sigma)).astype(np.float32)
    for r in range(rows):
        ids = g.choice(V, size=n_spikes, replace=False)
        x[r, ids] = np.float32(spike)
    return x


def single_row(seed: int = 1, V: int = V_SEMANTIC) -> tuple[Batch, Batch]:
    """(sampled, greedy) batches of one row each."""
    g = np.random.default_rng(seed)
    x = _spiked_normal(g, 1, V, 3.0)
    hist = g.integers(0, V, size=200, dtype=np.int64).astype(np.int32)
    ids, off = csr([hist])
    common = dict(logits=x, hist_ids=ids, hist_off=off, temp=np.array([0.8], np.float32),
                  top_k=np.array([30], np.int32), top_p=np.array([0.8], np.float32),
                  pen=np.array([10.0], np.float32), rng=np.array([DEFAULT_SEED], np.uint64))
    return (Batch(do_sample=np.ones(1, np.uint8), **common),
            Batch(do_sample=np.zeros(1, np.uint8), **{**common, "logits": x.copy()}))


def batch64_params(seed: int = 2, rows: int = 64, V: int = V_SEMANTIC, h_lo: int = 50,
                   h_hi: int = 800):
    g = np.random.default_rng(seed)
    temp = g.uniform(0.6, 1.2, size=rows).astype(np.float32)
    top_k = g.choice(np.array([0, 20, 30, 50], np.int32), size=rows).astype(np.int32)
    top_p = g.choice(np.array([1.0, 0.9, 0.8], np.float32), size=rows).astype(np.float32)
    pen = g.choice(np.array([1.0, 10.0], np.float32), size=rows).astype(np.float32)
    hist = [g.integers(0, V, size=int(g.integers(h_lo, h_hi + 1)), dtype=np.int64).astype(np.int32)
            for _ in range(rows)]
    ids, off = csr(hist)
    return dict(hist_ids=ids, hist_off=off, temp=temp, top_k=top_k, top_p=top_p, pen=pen,
                do_sample=np.ones(rows, np.uint8), rng=seed_batch(DEFAULT_SEED, rows))


def batch64_logits(seed: int, steps: int, rows: int = 64, V: int = V_SEMANTIC) -> np.ndarray:
    """[steps, rows, V] f32: N(0, 3^2) with 5 spikes at +12 per row and step."""
    g = np.random.default_rng(seed)
    out = np.empty((steps, rows, V), dtype=np.float32)
    for s in range(steps):
        out[s] = _spiked_normal(g, rows, V, 3.0)
    return out


def batch64(seed: int = 2, rows: int = 64, steps: int = 1, V: int = V_SEMANTIC) -> Batch:
    p = batch64_params(seed, rows, V)
    x = batch64_logits(seed + 1000, steps, rows, V)
    return Batch(logits=x[0] if steps == 1 else x, **p)


def bf16_ties(seed: int = 3, rows: int = 1024, V: int = V_SEMANTIC, sweep: str = "top_p",
              hist_len: int = 1000, tie_frac: float = 0.1) -> Batch:
    """sweep: 'greedy', 'top_k1' or 'top_p'."""
    g = np.random.default_rng(seed)
    x = (g.standard_t(3, size=(rows, V)) * 4.0).astype(np.float32)
    bits = f32_to_bf16_bits(x)
    xf = bf16_bits_to_f32(bits)
    n_tie = int(round(tie_frac * V))
    for r in range(rows):
        ids = g.choice(V, size=n_tie, replace=False)
        xf[r, ids] = xf[r].max()
    bits = f32_to_bf16_bits(xf)          # exact: every value is already bf16
    hist = [g.integers(0, V, size=hist_len, dtype=np.int64).astype(np.int32) for _ in range(rows)]
    ids, off = csr(hist)
    k, p, ds = {"greedy": (0, 1.0, 0), "top_k1": (1, 1.0, 1), "top_p": (0, 0.5, 1)}[sweep]
    return Batch(logits=bits, hist_ids=ids, hist_off=off, temp=np.ones(rows, np.float32),
                 top_k=np.full(rows, k, np.int32), top_p=np.full(rows, p, np.float32),
                 pen=np.full(rows, 10.0, np.float32), do_sample=np.full(rows, ds, np.uint8),
                 rng=seed_batch(DEFAULT_SEED, rows), meta={"sweep": sweep})


def large_vocab(seed: int = 4, rows: int = 256, V: int = 151936, hist_len: int = 2048) -> Batch:
    g = np.random.default_rng(seed)
    x = (g.standard_normal((rows, V), dtype=np.float32) * np.float32(2.0)).astype(np.float32)
    boost = (10.0 * (np.arange(V, dtype=np.float64) + 1.0) ** -1.1).astype(np.float32)
    for r in range(rows):
        perm = g.permutation(V)
        x[r, perm] += boost
    hist = [g.integers(0, V, size=hist_len, dtype=np.int64).astype(np.int32) for _ in range(rows)]
    ids, off = csr(hist)
    return Batch(logits=x, hist_ids=ids, hist_off=off, temp=np.full(rows, 0.7, np.float32),
                 top_k=np.full(rows, 50, np.int32), top_p=np.full(rows, 0.95, np.float32),
                 pen=np.full(rows, 1.2, np.float32), do_sample=np.ones(rows, np.uint8),
                 rng=seed_batch(DEFAULT_SEED, rows))


@dataclass
class LMHead:
    hidden: np.ndarray   # [M, D] bf16 bits
    gamma: np.ndarray    # [D] f32
    beta: np.ndarray     # [D] f32
    weight: np.ndarray   # [V, D] bf16 bits
    bias: np.ndarray     # [V] f32
    eps: float = 1e-5


def lmhead(seed: int = 5, M: int = 64, D: int = 1280, V: int = V_SEMANTIC) -> tuple[LMHead, dict]:
    g = np.random.default_rng(seed)
    hidden = f32_to_bf16_bits(g.standard_normal((M, D), dtype=np.float32))
    gamma = (1.0 + 0.02 * g.standard_normal(D)).astype(np.float32)
    beta = (0.02 * g.standard_normal(D)).astype(np.float32)
    weight = f32_to_bf16_bits((0.02 * g.standard_normal((V, D), dtype=np.float32)).astype(np.float32))
    bias = (0.02 * g.standard_normal(V)).astype(np.float32)
    return LMHead(hidden, gamma, beta, weight, bias), batch64_params(seed + 1, M, V)


def head_weight_f32(seed: int, V: int, D: int) -> np.ndarray:
    """semantic_head.weight [V, D] in float32 (the reference's dtype)."""
    return (0.02 * np.random.default_rng(seed).standard_normal((V, D))).astype(np.float32)


def quantize_affine8(w: np.ndarray, group: int = 64) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """8-bit affine groups along the input dimension: codes q in 0..255 with
    w ~ scale * q + bias per group of `group` inputs (bias = the group's
    minimum, scale = its range / 255)."""
    V, D = w.shape
    g = w.astype(np.float64).reshape(V, D // group, group)
    lo, hi = g.min(axis=2), g.max(axis=2)
    scale = np.where(hi > lo, (hi - lo) / 255.0, 1.0)
    q = np.clip(np.rint((g - lo[..., None]) / scale[..., None]), 0, 255).astype(np.uint8).reshape(V, D)
    return q, scale.astype(np.float32), lo.astype(np.float32)

