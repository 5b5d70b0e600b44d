"""LM head (LayerNorm folded into one MFMA kernel, + bias) for bf16, fp32 and
8-bit affine weights, and LM head + sampling.

Logits differ from the oracle's float64 LayerNorm + linear by rounding only
(the activations enter the matrix engine as hi + lo bf16 pairs, fp32 weights
too; fp32 accumulation), so they are compared with a tolerance; the tokens
are then checked bit for bit by running the oracle chain on the GPU's own
logits.
"""
import numpy as np
import pytest

import c4s
import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu

# Measured on MI355X: at most 1.5e-5 for rows of mean ~0 and 5.8e-5 for rows of
# mean 4 (the folded LayerNorm's G - mu c cancellation), |logit| <= 4.
ATOL = 2e-4
RTOL = 0.0


def _weights(kind, head, seed, group):
    """(device weight, quant, oracle weight, oracle kwargs) of one kind."""
    import torch
    V, D = head.weight.shape
    if kind == "bf16":
        return dev(head.weight, torch), None, head.weight, {}
    wf = W.head_weight_f32(seed, V, D)
    if kind == "f32":
        return dev(wf, torch), None, wf, {"wkind": 1}
    q, sc, bi = W.quantize_affine8(wf, group)
    quant = (dev(sc, torch), dev(bi, torch), group)
    return dev(q, torch), quant, q, {"wkind": 2, "wscale": sc, "wbias": bi, "group": group}


CASES = [("bf16", 64, 1280, 8194, 64, 0.0), ("bf16", 5, 64, 100, 64, 0.0), ("bf16", 70, 256, 1000, 64, 0.0),
         ("bf16", 3, 2080, 300, 64, 0.0), ("bf16", 9, 4096, 130, 64, 0.0), ("bf16", 16, 1280, 1000, 64, 4.0),
         ("f32", 64, 1280, 8194, 64, 0.0), ("f32", 70, 96, 517, 64, 0.0), ("f32", 16, 1280, 1000, 64, 4.0),
         ("q8", 64, 1280, 8194, 64, 0.0), ("q8", 5, 64, 100, 32, 0.0), ("q8", 70, 256, 1000, 128, 0.0),
         ("q8", 33, 1280, 777, 32, 4.0),
         # column tiles of 64 with the last one wider: 2 and 4 blocks past the fourth, and V below one tile;
         # fp32 weights over two staged K blocks
         ("bf16", 7, 128, 90, 64, 0.0), ("f32", 5, 96, 127, 64, 0.0), ("q8", 9, 256, 37, 32, 0.0),
         ("f32", 3, 2080, 300, 64, 0.0),
         # a last partial tile of exactly 16 columns (its second block skipped) and of 17 (it is not)
         ("bf16", 6, 96, 48, 64, 0.0), ("q8", 6, 128, 49, 32, 0.0)]


@pytest.mark.parametrize("kind,M,D,V,group,shift", CASES)
def test_lmhead_logits(orc, gpu_ctx, kind, M, D, V, group, shift):
    import torch
    head, _ = W.lmhead(seed=M + D, M=M, D=D, V=V)
    if shift:   # hidden rows with mean `shift`: the folded LayerNorm's cancellation case
        head.hidden = W.f32_to_bf16_bits(W.bf16_bits_to_f32(head.hidden) + np.float32(shift))
    wdev, quant, worc, kw = _weights(kind, head, M + D + 1, group)
    print(f"lmhead {kind} M={M} D={D} V={V} group={group} shift={shift}", flush=True)
    logits = torch.zeros((M, V), dtype=torch.float32, device="cuda")
    gpu_ctx.lmhead(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch), wdev,
                   dev(head.bias, torch), logits, quant=quant)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    want = orc.ln_lmhead(head.hidden, head.gamma, head.beta, worc, head.bias, n_threads=16, **kw)
    err = np.abs(got.astype(np.float64) - want)
    print(f"  max abs err {err.max():.3e}  max |logit| {np.abs(want).max():.3f}", flush=True)
    assert np.all(err <= ATOL + RTOL * np.abs(want))


@pytest.mark.parametrize("kind", ["bf16", "f32", "q8"])
def test_lmhead_sample_tokens(orc, gpu_ctx, kind):
    import torch
    head, p = W.lmhead(seed=5)
    M, V = 64, 8194
    wdev, quant, _, _ = _weights(kind, head, 11, 64)
    print(f"lmhead_sample {kind}", flush=True)
    logits = torch.zeros((M, V), dtype=torch.float32, device="cuda")
    rng = dev(p["rng"], torch)
    tok = torch.zeros(M, dtype=torch.int32, device="cuda")
    gpu_ctx.lmhead_sample(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch), wdev,
                          dev(head.bias, torch), dev(p["hist_ids"], torch),
                          dev(p["hist_off"], torch), dev(p["temp"], torch), dev(p["top_k"], torch),
                          dev(p["top_p"], torch), dev(p["pen"], torch), rng, tok, logits=logits,
                          do_sample=dev(p["do_sample"], torch), quant=quant)
    torch.cuda.synchronize()
    L = logits.cpu().numpy()
    otok, orng, _ = orc.sample_rows(L, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], n_threads=16)
    assert np.array_equal(tok.cpu().numpy(), otok)
    assert np.array_equal(rng.cpu().numpy().view(np.uint64), orng)


def test_lmhead_rejects_bad_descriptors(gpu_ctx):
    import torch
    head, _ = W.lmhead(seed=1, M=2, D=64, V=10)
    h, g, b, bias = (dev(x, torch) for x in (head.hidden, head.gamma, head.beta, head.bias))
    out = torch.zeros((2, 10), dtype=torch.float32, device="cuda")
    q = torch.zeros((10, 64), dtype=torch.uint8, device="cuda")
    sc = torch.ones((10, 2), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        gpu_ctx.lmhead(h, g, b, q, bias, out)                          # 8-bit without scales
    with pytest.raises(c4s.C4SError, match="code 1"):
        gpu_ctx.lmhead(h, g, b, q, bias, out, quant=(sc, sc, 48))      # group not 32/64/128
    with pytest.raises(c4s.C4SError, match="code 1"):
        gpu_ctx.lmhead(h, g, b, q, bias, out, quant=(sc, sc, 128))     # group does not divide D


@pytest.mark.parametrize("noalloc", [False, True])
def test_lmhead_sample_bad_rows_queue_nothing(gpu_ctx, noalloc):
    """A rows descriptor that fails validation (no RNG state for sampled rows)
    is reported before anything is queued: the caller's logits keep their
    contents, and so do the token output and the RNG states."""
    import torch
    head, p = W.lmhead(seed=7, M=4, D=64, V=100)
    h, g, b, bias, w = (dev(x, torch) for x in (head.hidden, head.gamma, head.beta, head.bias, head.weight))
    logits = torch.full((4, 100), 7.0, dtype=torch.float32, device="cuda")
    tok = torch.full((4,), -5, dtype=torch.int32, device="cuda")
    fn = gpu_ctx.lmhead_sample_noalloc if noalloc else gpu_ctx.lmhead_sample
    with pytest.raises(c4s.C4SError, match="code 1.*rng_state"):
        fn(h, g, b, w, bias, dev(p["hist_ids"][:0], torch), dev(np.zeros(5, np.int64), torch),
           dev(p["temp"][:4], torch), dev(p["top_k"][:4], torch), dev(p["top_p"][:4], torch),
           dev(p["pen"][:4], torch), None, tok, logits=logits)
    torch.cuda.synchronize()
    assert (logits.cpu().numpy() == 7.0).all()
    assert (tok.cpu().numpy() == -5).all()


@pytest.mark.parametrize("kind", ["bf16", "f32", "q8"])
def test_lmhead_outlier_channels(orc, gpu_ctx, kind):
    """GPT-2-like hidden rows: a few channels with magnitudes of 100-300 in every
    row (the rest N(0, 1)), so that the row's mean and variance are set by
    them. The folded LayerNorm (x - mu) / sigma * gamma . W = (x . gamma W - mu
    gamma . W) / sigma keeps the logits within the same tolerance of the
    float64 LayerNorm + linear."""
    import torch
    M, D, V = 64, 1280, 8194
    head, _ = W.lmhead(seed=17, M=M, D=D, V=V)
    g = np.random.default_rng(18)
    x = g.standard_normal((M, D)).astype(np.float32)
    chans = np.array([37, 138, 447, 1003])
    x[:, chans] = (np.array([150.0, -300.0, 100.0, 220.0]) * (1 + 0.1 * g.standard_normal((M, 4)))).astype(np.float32)
    head.hidden = W.f32_to_bf16_bits(x)
    wdev, quant, worc, kw = _weights(kind, head, 19, 64)
    logits = torch.zeros((M, V), dtype=torch.float32, device="cuda")
    print(f"lmhead outliers {kind}", flush=True)
    gpu_ctx.lmhead(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch), wdev,
                   dev(head.bias, torch), logits, quant=quant)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    want = orc.ln_lmhead(head.hidden, head.gamma, head.beta, worc, head.bias, n_threads=16, **kw)
    err = np.abs(got.astype(np.float64) - want)
    print(f"  max abs err {err.max():.3e}  max |logit| {np.abs(want).max():.3f}", flush=True)
    assert np.all(err <= ATOL + RTOL * np.abs(want))
