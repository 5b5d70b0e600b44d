"""GPU parity of the multi-step AR stream (one persistent workgroup per row) and
of the per-step batched path driven step by step."""
import numpy as np
import pytest

import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu


def run_stream(ctx, p, x, stop_token=-1):
    import torch
    steps, rows, V = x.shape
    out = torch.full((steps, rows), -9, dtype=torch.int32, device="cuda")
    st = torch.zeros((rows, 4), dtype=torch.int32, device="cuda")
    rng = dev(p["rng"], torch)
    ctx.sample_stream(dev(x, torch), dev(p["hist_ids"], torch), dev(p["hist_off"], torch),
                      dev(p["temp"], torch), dev(p["top_k"], torch), dev(p["top_p"], torch),
                      dev(p["pen"], torch), rng, out, do_sample=dev(p["do_sample"], torch),
                      stop_token=stop_token, out_stats=st)
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
    print("rows", toks.size, "exact top_p passes", int(st[:, 1].sum()),
          "exact draws", int(st[:, 2].sum()))
    ctx.close()


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
