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


def _draw_reference(ids, e, u, V):
    """text2semantic.cpp:152-164 over ids in ascending order (other ids weigh 0)."""
    order = np.argsort(ids, kind="stable")
    total = 0.0
    for j in order:
        total += float(e[j])
    r = u * total
    if r <= 0.0:
        return 0
    acc = 0.0
    for j in order:
        acc += float(e[j])
        if r <= acc:
            return int(ids[j])
    return V - 1


def test_lane_draw_id_order_and_replay():
    """lane_draw: kept entries scattered over lanes in value order; the token is
    the reference's id-order inverse CDF, including uniforms placed on a
    cumulative boundary (sequential replay), zero masses and r = 0."""
    import torch
    L = C.CDLL(LIB)
    rng = np.random.default_rng(11)
    V, n = 8194, 400
    kept = np.zeros((n, 64), np.uint8)
    ids = np.zeros((n, 64), np.int32)
    slots = np.zeros((n, 64), np.int32)
    es = np.zeros((n, 64), np.float64)
    us = np.zeros(n, np.float64)
    expect = []
    for c in range(n):
        nk = int(rng.integers(1, 65))
        ncand = int(rng.integers(nk, 1025))
        cand = np.sort(rng.choice(V, ncand, replace=False))
        pick = np.sort(rng.choice(ncand, nk, replace=False))
        kind = c % 4
        if kind == 0:
            e = rng.random(nk) * 10.0 ** float(rng.integers(-6, 2))
        elif kind == 1:
            e = rng.integers(0, 4, nk).astype(np.float64)
            e[rng.integers(0, nk)] = 1.0
        elif kind == 2:
            e = rng.random(nk) * 1e-9
            e[rng.integers(0, nk)] = 5.0
        else:
            e = np.exp(-rng.random(nk) * 30.0)
        cum = np.cumsum(e)
        if kind == 1:       # r on a cumulative boundary
            u = float(cum[int(rng.integers(0, nk))]) / float(cum[-1])
        elif c % 40 == 3:
            u = 0.0
        else:
            u = float(rng.random())
        lanes = rng.permutation(64)[:nk]
        kept[c, lanes] = 1
        ids[c, lanes] = cand[pick]
        slots[c, lanes] = pick
        es[c, lanes] = e
        junk = np.setdiff1d(np.arange(64), lanes)
        ids[c, junk] = rng.integers(0, V, junk.size)
        slots[c, junk] = rng.integers(0, 1024, junk.size)
        es[c, junk] = rng.random(junk.size)
        us[c] = u
        expect.append(_draw_reference(cand[pick], e, u, V))
    t = {k: torch.from_numpy(v.reshape(-1)).cuda() for k, v in
         dict(kept=kept, ids=ids, slots=slots, es=es).items()}
    tu = torch.from_numpy(us).cuda()
    out = torch.zeros(2 * n, dtype=torch.int32, device="cuda")
    assert L.c4s_selftest_draw(C.c_void_p(t["kept"].data_ptr()), C.c_void_p(t["ids"].data_ptr()),
                               C.c_void_p(t["slots"].data_ptr()), C.c_void_p(t["es"].data_ptr()),
                               C.c_void_p(tu.data_ptr()), V, n, C.c_void_p(out.data_ptr())) == 0
    torch.cuda.synchronize()
    o = out.cpu().numpy().reshape(n, 2)
    assert o[:, 0].tolist() == expect
    assert o[1::4, 1].sum() > 20      # boundary cases went through the sequential replay


@pytest.mark.parametrize("mode", [0, 1])
def test_hbm_probe(gpu_ctx, mode):
    """The bandwidth probes: copy (mode 0) reproduces the source exactly over
    256 MiB (a size that is not a multiple of the grid's spans); read (mode 1)
    writes nothing for ordinary data. Their runs also calibrate the HBM
    traffic counters (a copy of known size)."""
    import torch
    n = (256 << 20) // 4 + 12
    src = torch.arange(n, dtype=torch.int32, device="cuda").view(torch.float32)
    dst = torch.full((n,), -1, dtype=torch.int32, device="cuda").view(torch.float32)
    gpu_ctx.hbm_probe(src, dst, n * 4, mode)
    torch.cuda.synchronize()
    if mode == 0:
        assert torch.equal(dst.view(torch.int32), src.view(torch.int32))
    else:
        assert bool((dst.view(torch.int32) == -1).all())
