"""Graph capture: c4s_sample_rows (no workspace at vocab <= 12288) captured
into a HIP graph gives, on every replay, the tokens and RNG states of the same
call made eagerly; a call whose workspace would grow is refused under capture
and captures once an eager call has sized it; c4s_sample_stream refuses
capture with C4S_EINVAL."""
import numpy as np
import pytest

import c4s
import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu


def _args(torch, b):
    return dict(logits=dev(b.logits, torch), hist_ids=dev(b.hist_ids, torch), hist_off=dev(b.hist_off, torch),
                temp=dev(b.temp, torch), top_k=dev(b.top_k, torch), top_p=dev(b.top_p, torch),
                pen=dev(b.pen, torch), do_sample=dev(b.do_sample, torch))


def test_sample_rows_graph_replays_match_eager(gpu_ctx):
    import torch
    b = W.batch64(seed=77, rows=64)
    a = _args(torch, b)
    s = torch.cuda.Stream()
    n_replays = 4
    # eager: the same call n_replays times in a row (the RNG advances each time)
    rng = dev(b.rng, torch)
    tok = torch.zeros(64, dtype=torch.int32, device="cuda")
    want_tok, want_rng = [], []
    with torch.cuda.stream(s):
        for _ in range(n_replays):
            gpu_ctx.sample_rows(a["logits"], a["hist_ids"], a["hist_off"], a["temp"], a["top_k"], a["top_p"],
                                a["pen"], rng, tok, do_sample=a["do_sample"], stream=s)
            s.synchronize()
            want_tok.append(tok.cpu().numpy().copy())
            want_rng.append(rng.cpu().numpy().copy())
    # captured once, replayed n_replays times from the starting RNG state
    rng0 = dev(b.rng, torch)
    rng.copy_(rng0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        gpu_ctx.sample_rows(a["logits"], a["hist_ids"], a["hist_off"], a["temp"], a["top_k"], a["top_p"],
                            a["pen"], rng, tok, do_sample=a["do_sample"], stream=s)
    for k in range(n_replays):
        tok.fill_(-5)
        g.replay()
        torch.cuda.synchronize()
        # eager work between replays
        _ = (a["logits"] * 2).sum().item()
        assert np.array_equal(tok.cpu().numpy(), want_tok[k]), k
        assert np.array_equal(rng.cpu().numpy(), want_rng[k]), k


def test_sample_stream_refuses_capture(gpu_ctx):
    import torch
    p = W.batch64_params(seed=3, rows=4, V=100)
    x = dev(W.batch64_logits(4, 3, 4, 100), torch)
    out = torch.zeros((3, 4), dtype=torch.int32, device="cuda")
    rng = dev(p["rng"], torch)
    d = {k: dev(p[k], torch) for k in ("hist_ids", "hist_off", "temp", "top_k", "top_p", "pen", "do_sample")}
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g, stream=s):
        try:
            gpu_ctx.sample_stream(x, d["hist_ids"], d["hist_off"], d["temp"], d["top_k"], d["top_p"], d["pen"],
                                  rng, out, do_sample=d["do_sample"], stream=s)
        except c4s.C4SError as e:
            err = str(e)
    assert err is not None and "code 1" in err and "captured" in err


def test_large_vocab_workspace_is_sized_outside_capture():
    """A vocabulary above 12288 needs the context's key workspace: the first
    such call under capture is refused (no allocation inside a capture) and
    queues nothing; once an eager call of that shape has sized the workspace,
    the same call captures, and its replays give the eager call's tokens."""
    import torch
    ctx = c4s.Context(0)   # a fresh context: no workspace yet
    try:
        b = W.batch64(seed=91, rows=4, V=20000)
        a = _args(torch, b)
        s = torch.cuda.Stream()
        tok = torch.full((4,), -5, dtype=torch.int32, device="cuda")
        rng = dev(b.rng, torch)
        torch.cuda.synchronize()

        def call():
            ctx.sample_rows(a["logits"], a["hist_ids"], a["hist_off"], a["temp"], a["top_k"], a["top_p"],
                            a["pen"], rng, tok, do_sample=a["do_sample"], stream=s)

        g0 = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(g0, stream=s):
            try:
                call()
            except c4s.C4SError as e:
                err = str(e)
        assert err is not None and "code 1" in err and "graph capture" in err
        assert bool((tok == -5).all()), "the refused call queued work"
        # eager: sizes the workspace and gives the reference tokens
        with torch.cuda.stream(s):
            call()
        s.synchronize()
        want_tok, want_rng = tok.cpu().numpy().copy(), rng.cpu().numpy().copy()
        rng.copy_(dev(b.rng, torch))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            call()
        for k in range(3):
            rng.copy_(dev(b.rng, torch))
            tok.fill_(-5)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            _ = (a["logits"] * 2).sum().item()   # eager work between replays
            assert np.array_equal(tok.cpu().numpy(), want_tok), k
            assert np.array_equal(rng.cpu().numpy(), want_rng), k
    finally:
        ctx.close()
