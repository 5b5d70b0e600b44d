"""Runs the C++ drop-in test (tests/cpp/test_sampling_dropin.cpp): the
c4::t2s::sampling functions with the reference's signatures, on the GPU,
checked like the reference's tests/test_sampling.cpp against the HF golden
fixtures and the oracle's argmax/draw."""
import glob
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "bin", "test_sampling_dropin")


def test_cpp_dropin(orc, tmp_path):
    assert os.path.exists(BIN), "build the package first"
    dirs = []
    for f in sorted(glob.glob(os.path.join(HERE, "golden", "hf_sampling_*.npz"))):
        d = np.load(f, allow_pickle=False)
        temp, pen, k, p = d["params"]
        out = tmp_path / os.path.basename(f)[:-4]
        out.mkdir()
        d["logits"].astype(np.float32).tofile(out / "logits.f32")
        d["ids"].astype(np.int32).tofile(out / "ids.i32")
        for name in ("temp", "rep", "topk", "topp"):
            d[name].astype(np.float32).tofile(out / f"{name}.f32")
        seed = 1234
        (out / "params.txt").write_text(f"{float(temp)!r} {float(pen)!r} {int(k)} {float(p)!r} {seed}\n")
        am = orc.argmax(d["logits"])
        tok, st = orc.draw(orc.top_p(d["logits"], np.float32(p)), orc.seed_single(seed))
        (out / "expect.txt").write_text(f"{am} {tok} {st}\n")
        dirs.append(str(out))
    r = subprocess.run([BIN] + dirs, capture_output=True, text=True, timeout=120)
    print(r.stdout[-4000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert "ALL PASSED" in r.stdout
