"""Helpers for the GPU parity tests: move a workload to the device, run the C ABI,
bring results back, and compare with the oracle bit for bit."""
import numpy as np


def dev(a, torch):
    """numpy -> cuda tensor (uint64 / uint16 kept as same-width integer views)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint64:
        return torch.from_numpy(a.view(np.int64).copy()).cuda()
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).cuda().view(torch.bfloat16)
    return torch.from_numpy(a.copy()).cuda()


def gpu_rows(ctx, b, mode=0, masked=True, min_keep=None, row_active=None):
    import torch
    n = b.n_rows
    logits = dev(b.logits, torch)
    vocab = b.logits.shape[1]
    rng = dev(b.rng, torch)
    tok = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    out_m = torch.full((n, vocab), 123.0, dtype=torch.float32, device="cuda") if masked else None
    st = torch.zeros((n, 4), dtype=torch.int32, device="cuda")
    ctx.sample_rows(logits, dev(b.hist_ids, torch), dev(b.hist_off, torch), dev(b.temp, torch),
                    dev(b.top_k, torch), dev(b.top_p, torch), dev(b.pen, torch), rng, tok,
                    do_sample=dev(b.do_sample, torch),
                    min_keep=None if min_keep is None else dev(min_keep, torch),
                    row_active=None if row_active is None else dev(row_active, torch),
                    out_masked=out_m, out_stats=st, mode=mode)
    torch.cuda.synchronize()
    return (tok.cpu().numpy(), rng.cpu().numpy().view(np.uint64),
            None if out_m is None else out_m.cpu().numpy(), st.cpu().numpy())


def assert_same_rows(got_masked, want_masked, rows=None):
    """Bit-exact comparison of masked rows (-inf positions and every finite bit)."""
    g = got_masked.view(np.uint32)
    w = want_masked.view(np.uint32)
    if rows is not None:
        g, w = g[rows], w[rows]
    bad = np.argwhere(g != w)
    assert bad.size == 0, f"{len(bad)} differing entries, first at {bad[:5].tolist()}"


def compare_with_oracle(orc, ctx, b, n_threads=16, min_keep=None, row_active=None, masked=True):
    tok, rng, m, st = gpu_rows(ctx, b, masked=masked, min_keep=min_keep, row_active=row_active)
    otok, orng, om = orc.sample_rows(b.logits, b.hist_ids, b.hist_off, b.temp, b.top_k, b.top_p,
                                     b.pen, b.do_sample, b.rng, min_keep=min_keep,
                                     row_active=row_active, want_masked=masked,
                                     n_threads=n_threads)
    bad = np.flatnonzero(tok != otok)
    assert bad.size == 0, f"token mismatch rows {bad[:10].tolist()}: gpu {tok[bad[:10]]} oracle {otok[bad[:10]]}"
    assert np.array_equal(rng, orng)
    if masked:
        active = np.ones(b.n_rows, bool) if row_active is None else row_active.astype(bool)
        assert_same_rows(m, om, rows=active)
    return tok, st
