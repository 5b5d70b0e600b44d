"""Lane semantics of the DPP wave primitives (scan, max, sum) on the GPU."""
import ctypes as C
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(__file__), "cpp", "bin", "libc4s_selftest.so")


def test_wave_primitives():
    import torch
    L = C.CDLL(LIB)
    rng = np.random.default_rng(0)
    for trial in range(20):
        u = rng.integers(0, 1000, 64).astype(np.uint32)
        d = rng.standard_normal(64) * 10.0 ** rng.integers(-3, 4)
        f = (rng.standard_normal(64) * 5).astype(np.float32)
        if trial % 4 == 1:
            f[:] = -np.inf
            f[rng.integers(0, 64)] = -3.0
        if trial % 4 == 2:
            f = -np.abs(f) - 1.0
        tu, td, tf = (torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a).cuda()
                      for a in (u, d, f))
        ou = torch.zeros(64, dtype=torch.int32, device="cuda")
        od = torch.zeros(64, dtype=torch.float64, device="cuda")
        of = torch.zeros(64, dtype=torch.float32, device="cuda")
        os_ = torch.zeros(64, dtype=torch.float64, device="cuda")
        assert L.c4s_selftest_wave(C.c_void_p(tu.data_ptr()), C.c_void_p(td.data_ptr()),
                                   C.c_void_p(tf.data_ptr()), C.c_void_p(ou.data_ptr()),
                                   C.c_void_p(od.data_ptr()), C.c_void_p(of.data_ptr()),
                                   C.c_void_p(os_.data_ptr())) == 0
        torch.cuda.synchronize()
        assert np.array_equal(ou.cpu().numpy().view(np.uint32), np.cumsum(u).astype(np.uint32))
        assert np.allclose(od.cpu().numpy(), np.cumsum(d), rtol=1e-12, atol=1e-12 * np.abs(d).sum())
        assert (of.cpu().numpy() == f.max()).all()
        assert np.allclose(os_.cpu().numpy(), d.sum(), rtol=1e-12, atol=1e-12 * np.abs(d).sum())


def test_wave_shift_and_integer_max():
    """wave_shl:1 (lane i reads lane i + 1) and DPP maxima of 32/64-bit keys."""
    import torch
    L = C.CDLL(LIB)
    rng = np.random.default_rng(1)
    for trial in range(20):
        u = rng.integers(0, 2**32, 64, dtype=np.uint64).astype(np.uint32)
        q = rng.integers(0, 2**63, 64, dtype=np.uint64)
        if trial % 3 == 1:
            q[:] = q[0]                                # equal keys
            q[rng.integers(0, 64)] ^= 1                # differ in the low word only
        tu = torch.from_numpy(u.view(np.int32)).cuda()
        tq = torch.from_numpy(q.view(np.int64)).cuda()
        on = torch.zeros(64, dtype=torch.int32, device="cuda")
        om = torch.zeros(64, dtype=torch.int32, device="cuda")
        oq = torch.zeros(64, dtype=torch.int64, device="cuda")
        assert L.c4s_selftest_wave2(C.c_void_p(tu.data_ptr()), C.c_void_p(tq.data_ptr()),
                                    C.c_void_p(on.data_ptr()), C.c_void_p(om.data_ptr()),
                                    C.c_void_p(oq.data_ptr())) == 0
        torch.cuda.synchronize()
        nxt = on.cpu().numpy().view(np.uint32)
        assert np.array_equal(nxt[:63], u[1:]) and nxt[63] == 0xdeadbeef
        assert (om.cpu().numpy().view(np.uint32) == u.max()).all()
        assert (oq.cpu().numpy().view(np.uint64) == q.max()).all()
