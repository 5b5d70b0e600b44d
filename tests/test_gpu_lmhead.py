"""LM head (LayerNorm -> bf16 MFMA GEMM + bias) and LM head + sampling.

Logits differ from the oracle's float64 accumulation by rounding only (fp32
LayerNorm statistics and MFMA accumulation order), so they are compared with a
tolerance; the tokens are then checked bit for bit by running the oracle
chain on the GPU's own logits.
"""
import numpy as np
import pytest

import c4s_workloads as W
from gpu_util import dev

pytestmark = pytest.mark.gpu

# |logit| ~ 1 here; fp32 LN vs double LN can move one bf16 rounding of a
# normalised element (2^-8 relative of that element) -> ~1e-3 absolute at most.
ATOL = 2e-3
RTOL = 1e-3


@pytest.mark.parametrize("M,D,V", [(64, 1280, 8194), (5, 64, 100), (70, 256, 1000), (3, 2080, 300), (9, 4096, 130)])
def test_lmhead_logits(orc, gpu_ctx, M, D, V):
    import torch
    head, _ = W.lmhead(seed=M + D, M=M, D=D, V=V)
    logits = torch.zeros((M, V), dtype=torch.float32, device="cuda")
    gpu_ctx.lmhead(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch),
                   dev(head.weight, torch), dev(head.bias, torch), logits)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    want = orc.ln_lmhead(head.hidden, head.gamma, head.beta, head.weight, head.bias, n_threads=16)
    err = np.abs(got - want)
    print(f"M={M} D={D} V={V} max abs err {err.max():.3e}")
    assert np.all(err <= ATOL + RTOL * np.abs(want))


def test_lmhead_sample_tokens(orc, gpu_ctx):
    import torch
    head, p = W.lmhead(seed=5)
    M, V = 64, 8194
    logits = torch.zeros((M, V), dtype=torch.float32, device="cuda")
    rng = dev(p["rng"], torch)
    tok = torch.zeros(M, dtype=torch.int32, device="cuda")
    gpu_ctx.lmhead_sample(dev(head.hidden, torch), dev(head.gamma, torch), dev(head.beta, torch),
                          dev(head.weight, torch), dev(head.bias, torch), dev(p["hist_ids"], torch),
                          dev(p["hist_off"], torch), dev(p["temp"], torch), dev(p["top_k"], torch),
                          dev(p["top_p"], torch), dev(p["pen"], torch), rng, tok, logits=logits,
                          do_sample=dev(p["do_sample"], torch))
    torch.cuda.synchronize()
    L = logits.cpu().numpy()
    otok, orng, _ = orc.sample_rows(L, p["hist_ids"], p["hist_off"], p["temp"], p["top_k"],
                                    p["top_p"], p["pen"], p["do_sample"], p["rng"], n_threads=16)
    assert np.array_equal(tok.cpu().numpy(), otok)
    assert np.array_equal(rng.cpu().numpy().view(np.uint64), orng)
