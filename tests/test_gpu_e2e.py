"""The per-step product chain end to end on the GPU: the LM head's tensors from
a weight store (src/core/weights.cpp:13-58) through c4s_head_weights_load,
then every AR step as one c4s_lmhead_sample call (head(cur) and the sampling
chain, text2semantic.cpp:118-121 and :297-337) with the history kept on the
device as a set that each step's tokens join (:333-334). Each step's tokens
and RNG states are checked bit for bit against the oracle's chain on the
GPU's own logits of that step with the history grown so far; greedy rows are
the first maximum of the penalised row, as tests/test_t2s_kv.cpp:36-60 checks
a greedy generate against the argmax of the full forward."""
import numpy as np
import pytest

import c4s
import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu


def _store(tmp_path, D, V, seed):
    g = np.random.default_rng(seed)
    arrs = {"final_norm.weight": (1 + 0.02 * g.standard_normal(D)).astype(np.float32),
            "final_norm.bias": (0.02 * g.standard_normal(D)).astype(np.float32),
            "semantic_head.weight": (0.05 * g.standard_normal((V, D))).astype(np.float32),
            "semantic_head.bias": (0.5 * g.standard_normal(V)).astype(np.float32)}
    root = tmp_path / "t2s"
    root.mkdir()
    for k, v in arrs.items():
        np.save(root / f"{k}.npy", v)
    return str(root)


def _words(hist, V):
    out = np.zeros((V + 31) // 32, np.uint32)
    for i in hist:
        if 0 <= i < V:
            out[i >> 5] |= np.uint32(1 << (int(i) & 31))
    return out


@pytest.mark.parametrize("kind", ["bf16", "f32", "q8"])
def test_store_head_and_step_loop(tmp_path, orc, gpu_ctx, kind):
    import torch
    D, V, R, T = 1280, 8194, 16, 20
    root = _store(tmp_path, D, V, seed=91)
    wdtype = {"bf16": c4s.W_BF16, "f32": c4s.W_F32, "q8": c4s.W_Q8}[kind]
    hw = c4s.load_head_weights(root, wdtype, 64)
    try:
        p = W.batch64_params(seed=92, rows=R, V=V)
        p["do_sample"][::4] = 0                    # greedy rows
        stop = V - 1
        hist = [list(p["hist_ids"][p["hist_off"][r]:p["hist_off"][r + 1]]) for r in range(R)]
        bits = torch.zeros((R, (V + 31) // 32), dtype=torch.int32, device="cuda")
        gpu_ctx.hist_bits_init(dev(p["hist_ids"], torch), dev(p["hist_off"], torch), R, V, bits)
        temp, top_k, top_p, pen = (dev(p[k], torch) for k in ("temp", "top_k", "top_p", "pen"))
        ds = dev(p["do_sample"], torch)
        rng = dev(p["rng"], torch)
        rng_host = p["rng"].copy()
        logits = torch.empty((R, V), dtype=torch.float32, device="cuda")
        g = np.random.default_rng(93)
        for s in range(T):
            hidden = W.f32_to_bf16_bits((3.0 * g.standard_normal((R, D))).astype(np.float32))
            tok = torch.full((R,), -7, dtype=torch.int32, device="cuda")
            print(f"e2e {kind} step {s}", flush=True)
            gpu_ctx.lmhead_sample_loaded(hw, dev(hidden, torch), temp, top_k, top_p, pen, rng, tok, logits=logits,
                                         hist_bits=bits, do_sample=ds, stop_token=stop)
            torch.cuda.synchronize()
            L = logits.cpu().numpy()
            got, got_rng = tok.cpu().numpy(), rng.cpu().numpy().view(np.uint64)
            ids, off = W.csr([np.array(h, np.int32) for h in hist])
            otok, orng, _ = orc.sample_rows(L, ids, off, p["temp"], p["top_k"], p["top_p"], p["pen"],
                                            p["do_sample"], rng_host, n_threads=16)
            assert np.array_equal(got, otok), (s, np.flatnonzero(got != otok)[:8].tolist())
            assert np.array_equal(got_rng, orng), s
            rng_host = orng.copy()
            for r in range(R):
                if got[r] != stop:
                    hist[r].append(int(got[r]))
        fin = bits.cpu().numpy().view(np.uint32)
        for r in range(R):
            assert np.array_equal(fin[r], _words(hist[r], V)), r
    finally:
        c4s.free_head_weights(hw)
