"""The no-allocation entry point (c4s_lmhead_sample_noalloc) against
c4s_lmhead_sample on the same inputs, through the C ABI: logits within the
LM head's own run-to-run identity (the same kernels), tokens, RNG states and
masked rows bit for bit, on two calls in a row, the second smaller; and the
size limit rejected with C4S_EINVAL."""
import numpy as np
import pytest

import c4s
import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu


def _run(ctx, torch, head, p, noalloc, with_logits):
    M, V = head.hidden.shape[0], head.weight.shape[0]
    rng = dev(p["rng"], torch)
    tok = torch.full((M,), -5, dtype=torch.int32, device="cuda")
    masked = torch.zeros((M, V), dtype=torch.float32, device="cuda")
    logits = torch.zeros((M, V), dtype=torch.float32, device="cuda") if with_logits else None
    fn = ctx.lmhead_sample_noalloc if noalloc else ctx.lmhead_sample
    fn(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch), dev(head.weight, torch),
       dev(head.bias, torch), dev(p["hist_ids"], torch), dev(p["hist_off"], torch), dev(p["temp"], torch),
       dev(p["top_k"], torch), dev(p["top_p"], torch), dev(p["pen"], torch), rng, tok, logits=logits,
       do_sample=dev(p["do_sample"], torch), out_masked=masked)
    torch.cuda.synchronize()
    return (tok.cpu().numpy(), rng.cpu().numpy(), masked.cpu().numpy(),
            None if logits is None else logits.cpu().numpy())


@pytest.mark.parametrize("with_logits", [False, True])
def test_noalloc_matches_lmhead_sample(gpu_ctx, with_logits):
    import torch
    for M, D, V, seed in [(64, 1280, 8194, 5), (20, 640, 3000, 6)]:   # the second call is smaller
        head, p = W.lmhead(seed=seed, M=M, D=D, V=V)
        print(f"noalloc M={M} D={D} V={V} logits={with_logits}", flush=True)
        want = _run(gpu_ctx, torch, head, p, False, True)
        got = _run(gpu_ctx, torch, head, p, True, with_logits)
        assert np.array_equal(got[0], want[0])
        assert np.array_equal(got[1], want[1])
        assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32))
        if with_logits:
            assert np.array_equal(got[3].view(np.uint32), want[3].view(np.uint32))


def test_noalloc_rejects_oversize(gpu_ctx):
    import torch
    head, p = W.lmhead(seed=7, M=300, D=64, V=8194)   # 300 x 8194 x 4 logits > 8 MiB
    with pytest.raises(c4s.C4SError, match="code 1"):
        _run(gpu_ctx, torch, head, p, True, False)


def test_noalloc_under_graph_capture():
    """What the entry point is for: a fresh context (nothing allocated by an
    earlier call) captures it into a HIP graph without a logits buffer (the
    logits live in the static scratch); every replay, with eager work between
    the replays, equals the eager c4s_lmhead_sample (tokens, RNG states, masked
    rows)."""
    import torch
    head, p = W.lmhead(seed=8, M=64, D=1280, V=8194)
    M, V = 64, 8194
    ref_ctx = c4s.Context(0)
    want = _run(ref_ctx, torch, head, p, False, True)
    ref_ctx.close()
    ctx = c4s.Context(0)
    try:
        args = [dev(x, torch) for x in (head.hidden, head.gamma, head.beta, head.weight, head.bias, p["hist_ids"],
                                        p["hist_off"], p["temp"], p["top_k"], p["top_p"], p["pen"])]
        rng0 = dev(p["rng"], torch)
        rng = rng0.clone()
        tok = torch.full((M,), -5, dtype=torch.int32, device="cuda")
        masked = torch.zeros((M, V), dtype=torch.float32, device="cuda")
        ds = dev(p["do_sample"], torch)
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        print("noalloc capture", flush=True)
        with torch.cuda.graph(g, stream=s):
            ctx.lmhead_sample_noalloc(*args, rng, tok, logits=None, do_sample=ds, out_masked=masked)
        for rep in range(3):
            rng.copy_(rng0)                        # eager work between the replays
            tok.fill_(-5)
            masked.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(tok.cpu().numpy(), want[0]), rep
            assert np.array_equal(rng.cpu().numpy(), want[1]), rep
            assert np.array_equal(masked.cpu().numpy().view(np.uint32), want[2].view(np.uint32)), rep
        del g
    finally:
        ctx.close()
