"""Writes the HuggingFace logits-processor golden vectors used to pin the oracle.

The reference's only processor parity test (tests/test_sampling.cpp:40-55)
compares its C++ processors against HuggingFace's TemperatureLogitsWarper,
RepetitionPenaltyLogitsProcessor, TopKLogitsWarper and TopPLogitsWarper, on
vectors produced by tools/dump_golden.py:807-825 (torch.manual_seed(51),
randn(1, 64), ids [3,7,7,15,42,3], temperature 0.8, penalty 1.3, top_k 10,
top_p 0.9), with max-abs tolerance 1e-5 and identical -inf masks. That
recipe's outputs are not committed in the reference (its golden/ is
git-ignored), so this script regenerates them with the same third-party
library (transformers, version recorded in the file) and adds more rows of the
same kind (other sizes and parameters, tie-free normal logits).

Run from the repo root:  python tests/golden/make_hf_sampling_golden.py
"""
import os

import numpy as np
import torch
import transformers
from transformers.generation.logits_process import (RepetitionPenaltyLogitsProcessor,
                                                    TemperatureLogitsWarper, TopKLogitsWarper,
                                                    TopPLogitsWarper)

OUT = os.path.dirname(os.path.abspath(__file__))


def recipe_v64():
    torch.manual_seed(51)
    logits = torch.randn(1, 64)
    ids = torch.tensor([[3, 7, 7, 15, 42, 3]])
    return dict(
        logits=logits.numpy()[0].astype(np.float32),
        ids=ids.numpy()[0].astype(np.int64),
        temp=TemperatureLogitsWarper(0.8)(ids, logits.clone()).numpy()[0],
        rep=RepetitionPenaltyLogitsProcessor(1.3)(ids, logits.clone()).numpy()[0],
        topk=TopKLogitsWarper(10)(ids, logits.clone()).numpy()[0],
        topp=TopPLogitsWarper(0.9)(ids, logits.clone()).numpy()[0],
        params=np.array([0.8, 1.3, 10, 0.9], dtype=np.float64),
    )


def extra_rows():
    """Each row goes through all four processors separately, like the recipe."""
    gen = torch.Generator().manual_seed(20260)
    cases = []
    sizes = [64, 257, 1000, 8194, 8194, 8194]
    temps = [0.6, 1.2, 0.8, 0.7, 1.0, 0.95]
    pens = [1.3, 10.0, 1.2, 10.0, 2.0, 1.05]
    ks = [5, 20, 50, 30, 1, 200]
    ps = [0.5, 0.8, 0.95, 0.8, 0.9, 0.3]
    scales = [1.0, 3.0, 2.0, 3.0, 1.0, 4.0]
    for n, t, pen, k, p, sc in zip(sizes, temps, pens, ks, ps, scales):
        logits = torch.randn(1, n, generator=gen) * sc
        ids = torch.randint(-3, n + 3, (1, max(6, n // 10)), generator=gen)
        ids_in = ids.clamp(0, n - 1)  # HF gathers, so it needs in-range ids
        cases.append(dict(
            logits=logits.numpy()[0].astype(np.float32),
            ids=ids_in.numpy()[0].astype(np.int64),
            temp=TemperatureLogitsWarper(t)(ids_in, logits.clone()).numpy()[0],
            rep=RepetitionPenaltyLogitsProcessor(pen)(ids_in, logits.clone()).numpy()[0],
            topk=TopKLogitsWarper(k)(ids_in, logits.clone()).numpy()[0],
            topp=TopPLogitsWarper(p)(ids_in, logits.clone()).numpy()[0],
            params=np.array([t, pen, k, p], dtype=np.float64),
        ))
    return cases


def main():
    meta = np.frombuffer(
        f"transformers {transformers.__version__}; torch {torch.__version__}".encode(), dtype=np.uint8)
    r = recipe_v64()
    np.savez_compressed(os.path.join(OUT, "hf_sampling_v64_seed51.npz"), meta=meta, **r)
    for i, c in enumerate(extra_rows()):
        np.savez_compressed(os.path.join(OUT, f"hf_sampling_extra_{i}.npz"), meta=meta, **c)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
