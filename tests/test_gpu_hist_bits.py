"""GPU parity of the AR loop driven one step per call with the history kept on
the device as a set (c4s_rows.hist_bits, filled by c4s_hist_bits_init): tokens,
RNG states and the final sets match the oracle's multi-step stream
(text2semantic.cpp:296-337, history growth and stop token as :333-334) bit for
bit. The reference applies each distinct history id once (sampling.cpp:22), so
the set is the history."""
import numpy as np
import pytest

import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu


def _words(hist, V):
    out = np.zeros((V + 31) // 32, np.uint32)
    for i in hist:
        if 0 <= i < V:   # sampling.cpp:24
            out[i >> 5] |= np.uint32(1 << (int(i) & 31))
    return out


def test_hist_bits_init(gpu_ctx):
    import torch
    V = 1000
    hists = [[3, 7, 7, 15, 42, 3], [], [-1, 999, 1000, 5000, 0, 31, 32], list(range(0, 1000, 7)), [998]]
    ids, off = W.csr([np.array(h, np.int32) for h in hists])
    R, nw = len(hists), (V + 31) // 32
    bits = torch.full((R, nw), -1, dtype=torch.int32, device="cuda")   # cleared by the call
    print("hist_bits_init", R, "rows V", V, flush=True)
    gpu_ctx.hist_bits_init(dev(ids, torch), dev(off, torch), R, V, bits)
    torch.cuda.synchronize()
    got = bits.cpu().numpy().view(np.uint32)
    for r, h in enumerate(hists):
        assert np.array_equal(got[r], _words(h, V)), r


@pytest.mark.parametrize("V,R,T", [(8194, 64, 40), (20000, 8, 6)])
def test_step_loop_with_hist_bits(orc, gpu_ctx, V, R, T):
    import torch
    p = W.batch64_params(seed=7, rows=R, V=V)
    x = W.batch64_logits(seed=1007, steps=T, rows=R, V=V)
    stop = V - 1
    for s, r in [(3, 1), (10, 5), (T - 2, 0), (1, R - 1)]:   # planted stop tokens
        if s < T and r < R:
            x[s, r, stop] = 40.0
    want, want_rng = orc.sample_stream(x, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"], p["top_p"],
                                       p["pen"], p["do_sample"], p["rng"], stop_token=stop, n_threads=16)
    print(f"step loop with hist_bits V={V} rows={R} steps={T}", flush=True)
    nw = (V + 31) // 32
    bits = torch.zeros((R, nw), dtype=torch.int32, device="cuda")
    gpu_ctx.hist_bits_init(dev(p["hist_ids"], torch), dev(p["hist_off"], torch), R, V, bits)
    rng = dev(p["rng"], torch)
    temp, top_k, top_p, pen = (dev(p[k], torch) for k in ("temp", "top_k", "top_p", "pen"))
    ds = dev(p["do_sample"], torch)
    active = np.ones(R, np.uint8)
    got = np.full((T, R), -7, np.int32)
    for s in range(T):
        tok = torch.full((R,), -7, dtype=torch.int32, device="cuda")
        gpu_ctx.sample_rows(dev(x[s], torch), None, None, temp, top_k, top_p, pen, rng, tok, do_sample=ds,
                            row_active=dev(active, torch), hist_bits=bits, stop_token=stop)
        got[s] = tok.cpu().numpy()
        active &= (got[s] != stop).astype(np.uint8)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} token mismatches, first (step, row) {bad[:5].tolist()}"
    assert np.array_equal(rng.cpu().numpy().view(np.uint64), want_rng)
    fin = bits.cpu().numpy().view(np.uint32)
    for r in range(R):
        h0 = p["hist_ids"][p["hist_off"][r]:p["hist_off"][r + 1]]
        drawn = [t for t in got[:, r] if t >= 0 and t != stop]
        assert np.array_equal(fin[r], _words(list(h0) + drawn, V)), r


def test_hist_bits_bf16_and_lmhead_match_csr(orc, gpu_ctx):
    """The kept set gives the same tokens, masked rows and RNG states as the CSR
    history it was filled from: bf16 logits, and the fused LM head + chain."""
    import torch
    b = W.batch64(seed=23)
    R, V = b.n_rows, b.logits.shape[1]
    bits = torch.zeros((R, (V + 31) // 32), dtype=torch.int32, device="cuda")
    ids, off = dev(b.hist_ids, torch), dev(b.hist_off, torch)
    gpu_ctx.hist_bits_init(ids, off, R, V, bits)
    x16 = dev(W.f32_to_bf16_bits(b.logits), torch)
    args = [dev(getattr(b, k), torch) for k in ("temp", "top_k", "top_p", "pen")]
    outs = []
    for use_bits in (False, True):
        rng = dev(b.rng, torch)
        tok = torch.full((R,), -7, dtype=torch.int32, device="cuda")
        m = torch.zeros((R, V), dtype=torch.float32, device="cuda")
        print("bf16 rows, history", "set" if use_bits else "CSR", flush=True)
        gpu_ctx.sample_rows(x16, None if use_bits else ids, None if use_bits else off, *args, rng, tok,
                            do_sample=dev(b.do_sample, torch), out_masked=m,
                            hist_bits=bits if use_bits else None, stop_token=-1)
        torch.cuda.synchronize()
        outs.append((tok.cpu().numpy(), rng.cpu().numpy(), m.cpu().numpy().view(np.uint32)))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][2], outs[1][2])

    head, p = W.lmhead(seed=5)
    M = head.hidden.shape[0]
    hb = torch.zeros((M, (V + 31) // 32), dtype=torch.int32, device="cuda")
    hids, hoff = dev(p["hist_ids"], torch), dev(p["hist_off"], torch)
    gpu_ctx.hist_bits_init(hids, hoff, M, V, hb)
    res = []
    for use_bits in (False, True):
        rng = dev(p["rng"], torch)
        tok = torch.full((M,), -7, dtype=torch.int32, device="cuda")
        print("lmhead_sample, history", "set" if use_bits else "CSR", flush=True)
        gpu_ctx.lmhead_sample(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch),
                              dev(head.weight, torch), dev(head.bias, torch), None if use_bits else hids,
                              None if use_bits else hoff, dev(p["temp"], torch), dev(p["top_k"], torch),
                              dev(p["top_p"], torch), dev(p["pen"], torch), rng, tok,
                              do_sample=dev(p["do_sample"], torch), hist_bits=hb if use_bits else None)
        torch.cuda.synchronize()
        res.append((tok.cpu().numpy(), rng.cpu().numpy()))
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])
    # the tokens joined the set: it now holds the history and each row's token
    fin = hb.cpu().numpy().view(np.uint32)
    for r in range(M):
        h0 = p["hist_ids"][p["hist_off"][r]:p["hist_off"][r + 1]]
        assert np.array_equal(fin[r], _words(list(h0) + [res[1][0][r]], V)), r
