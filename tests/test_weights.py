"""The LM head's tensors from the reference's weight store (src/core/weights.cpp:
13-58): <root>.safetensors when it exists, else <root>/<name>.npy. The reader
runs on the host; these tests write small synthetic stores with numpy and the
safetensors package and read them back through the C ABI. The device upload
and the head on the loaded tensors are GPU tests at the end."""
import os

import numpy as np
import pytest

import c4s
import c4s_workloads as W

NAMES = ("final_norm.weight", "final_norm.bias", "semantic_head.weight", "semantic_head.bias")


def _head_arrays(seed=3, D=128, V=100):
    g = np.random.default_rng(seed)
    return {"final_norm.weight": (1 + 0.02 * g.standard_normal(D)).astype(np.float32),
            "final_norm.bias": (0.02 * g.standard_normal(D)).astype(np.float32),
            "semantic_head.weight": (0.02 * g.standard_normal((V, D))).astype(np.float32),
            "semantic_head.bias": (0.02 * g.standard_normal(V)).astype(np.float32)}


def _npy_store(tmp_path, arrs, dtype=None):
    root = tmp_path / "t2s"
    root.mkdir()
    for k, v in arrs.items():
        np.save(root / f"{k}.npy", v if dtype is None else v.astype(dtype))
    return str(root)


def _st_store(tmp_path, arrs, name="t2s"):
    from safetensors.numpy import save_file
    save_file({k: np.ascontiguousarray(v) for k, v in arrs.items()}, str(tmp_path / f"{name}.safetensors"))
    return str(tmp_path / name)


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16])
def test_npy_store(tmp_path, dtype):
    arrs = _head_arrays()
    root = _npy_store(tmp_path, arrs, dtype)
    for k in NAMES:
        got = c4s.read_tensor(root, k)
        assert got.shape == arrs[k].shape
        assert np.array_equal(got, arrs[k].astype(dtype).astype(np.float32)), k


def test_safetensors_store_preferred(tmp_path):
    """A <root>.safetensors next to a <root>/ directory wins (weights.cpp:15-22)."""
    arrs = _head_arrays(seed=4)
    root = _st_store(tmp_path, arrs)
    os.makedirs(root)
    np.save(os.path.join(root, "final_norm.weight.npy"), np.zeros(128, np.float32))
    for k in NAMES:
        assert np.array_equal(c4s.read_tensor(root, k), arrs[k]), k


def test_safetensors_dtypes(tmp_path):
    """F16 and BF16 tensors widen exactly; keys that prefix each other stay apart."""
    from safetensors.numpy import save_file
    g = np.random.default_rng(5)
    a = g.standard_normal((7, 33)).astype(np.float16)
    bits = W.f32_to_bf16_bits(g.standard_normal(40).astype(np.float32))
    # BF16 through the raw format: numpy has no bfloat16, so write the file by hand
    import json, struct
    hdr = {"x.bf": {"dtype": "BF16", "shape": [40], "data_offsets": [0, 80]}}
    hb = json.dumps(hdr).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(tmp_path / "b.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + bits.astype("<u2").tobytes())
    assert np.array_equal(c4s.read_tensor(str(tmp_path / "b"), "x.bf"), W.bf16_bits_to_f32(bits))
    save_file({"h": a, "h2": np.ones(3, np.float32)}, str(tmp_path / "h.safetensors"))
    assert np.array_equal(c4s.read_tensor(str(tmp_path / "h"), "h"), a.astype(np.float32))
    assert np.array_equal(c4s.read_tensor(str(tmp_path / "h"), "h2"), np.ones(3, np.float32))


def test_store_errors(tmp_path):
    arrs = _head_arrays()
    root = _npy_store(tmp_path, arrs)
    with pytest.raises(c4s.C4SError, match="code 1.*missing.weight"):
        c4s.read_tensor(root, "missing.weight")
    np.save(os.path.join(root, "f.npy"), np.asfortranarray(np.ones((3, 4), np.float32)))
    with pytest.raises(c4s.C4SError, match="fortran_order"):
        c4s.read_tensor(root, "f")
    with open(os.path.join(root, "bad.npy"), "wb") as f:
        f.write(b"not numpy at all")
    with pytest.raises(c4s.C4SError, match="not a .npy file"):
        c4s.read_tensor(root, "bad")
    np.save(os.path.join(root, "i.npy"), np.ones(4, np.int16))
    with pytest.raises(c4s.C4SError, match="unsupported .npy dtype"):
        c4s.read_tensor(root, "i")
    with pytest.raises(c4s.C4SError, match="no .*safetensors"):
        c4s.read_tensor(str(tmp_path / "nowhere"), "final_norm.weight")


def _raw_safetensors(path, header_bytes, data=b"", length=None):
    import struct
    n = len(header_bytes) if length is None else length
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", n) + header_bytes + data)


def test_corrupt_files_are_errors(tmp_path):
    """Malformed stores come back as C4S_EINVAL with a message, in this process:
    nothing throws through the C ABI and nothing reads past the file."""
    import json
    # a header length whose sum with the 8-byte prefix wraps around 2^64
    _raw_safetensors(tmp_path / "wrap.safetensors", b"{}", length=(1 << 64) - 4)
    with pytest.raises(c4s.C4SError, match="code 1.*truncated .safetensors header"):
        c4s.read_tensor(str(tmp_path / "wrap"), "x")
    # a data offset of 40 digits
    hb = b'{"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 1' + b"0" * 40 + b']}}'
    _raw_safetensors(tmp_path / "big.safetensors", hb, b"\0" * 8)
    with pytest.raises(c4s.C4SError, match="code 1.*data_offsets"):
        c4s.read_tensor(str(tmp_path / "big"), "x")
    # a shape of 30 digits, and a shape with a zero dimension
    for nm, shape in (("huge", [2, 10 ** 30]), ("zero", [4, 0])):
        hb = json.dumps({"x": {"dtype": "F32", "shape": shape, "data_offsets": [0, 0]}}).encode()
        _raw_safetensors(tmp_path / f"{nm}.safetensors", hb)
        with pytest.raises(c4s.C4SError, match="code 1"):
            c4s.read_tensor(str(tmp_path / nm), "x")
    # .npy: a header longer than the file, a shape past the limit, a zero dimension
    root = tmp_path / "npy"
    root.mkdir()
    np.save(root / "ok.npy", np.ones((3, 4), np.float32))
    raw = (root / "ok.npy").read_bytes()
    (root / "trunc.npy").write_bytes(raw[:9])
    with pytest.raises(c4s.C4SError, match="code 1"):
        c4s.read_tensor(str(root), "trunc")
    (root / "longhdr.npy").write_bytes(raw[:8] + b"\xff\xff" + raw[10:40])
    with pytest.raises(c4s.C4SError, match="truncated .npy header"):
        c4s.read_tensor(str(root), "longhdr")
    hdr = raw[10:10 + (raw[8] | raw[9] << 8)]
    for nm, sh in (("npyhuge", b"(3, 99999999999999999999999)"), ("npyzero", b"(0, 4)")):
        h2 = hdr.replace(b"(3, 4)", sh)
        h2 = h2.rstrip(b" \n")
        h2 += b" " * ((64 - (10 + len(h2) + 1) % 64) % 64) + b"\n"
        (root / f"{nm}.npy").write_bytes(raw[:8] + len(h2).to_bytes(2, "little") + h2 + raw[10 + len(hdr):])
        with pytest.raises(c4s.C4SError, match="code 1"):
            c4s.read_tensor(str(root), nm)


def test_packed_head_with_empty_scales_is_an_error(tmp_path):
    """An 8-bit packed head whose scale tensors have zero columns: rejected before
    any division by the group count (and before any device work)."""
    arrs = _head_arrays(D=128, V=10)
    root = _npy_store(tmp_path, {k: v for k, v in arrs.items() if k != "semantic_head.weight"})
    np.save(os.path.join(root, "semantic_head.weight.npy"), np.zeros((10, 32), np.uint32))
    np.save(os.path.join(root, "semantic_head.scales.npy"), np.zeros((10, 0), np.float32))
    np.save(os.path.join(root, "semantic_head.biases.npy"), np.zeros((10, 0), np.float32))
    with pytest.raises(c4s.C4SError, match="code 1"):
        c4s.load_head_weights(root, c4s.W_Q8)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["f32", "bf16", "q8", "q8_packed"])
def test_head_from_store(tmp_path, orc, gpu_ctx, kind):
    """The loaded tensors drive c4s_lmhead; logits against the oracle on the
    same (converted) weights."""
    import torch
    from gpu_util import dev
    D, V, M = 256, 777, 9
    arrs = _head_arrays(seed=6, D=D, V=V)
    hidden = W.f32_to_bf16_bits(np.random.default_rng(7).standard_normal((M, D)).astype(np.float32))
    if kind == "q8_packed":   # an 8-bit head as stored: u32 words of four codes, scales, biases
        q, sc, bi = W.quantize_affine8(arrs["semantic_head.weight"], 64)
        store = dict(arrs)
        store["semantic_head.weight"] = q.reshape(V, D // 4, 4).copy().view(np.uint32).reshape(V, D // 4)
        store["semantic_head.scales"] = sc
        store["semantic_head.biases"] = bi
        root = _st_store(tmp_path, store)
        wdtype = c4s.W_Q8
    else:
        root = _npy_store(tmp_path, arrs)
        wdtype = {"f32": c4s.W_F32, "bf16": c4s.W_BF16, "q8": c4s.W_Q8}[kind]
    hw = c4s.load_head_weights(root, wdtype, 64)
    try:
        assert (hw.D, hw.V, hw.wdtype) == (D, V, wdtype)
        logits = torch.zeros((M, V), dtype=torch.float32, device="cuda")
        gpu_ctx.lmhead_loaded(hw, dev(hidden, torch), logits)
        torch.cuda.synchronize()
        got = logits.cpu().numpy()
    finally:
        c4s.free_head_weights(hw)
    w = arrs["semantic_head.weight"]
    if kind == "f32":
        want = orc.ln_lmhead(hidden, arrs["final_norm.weight"], arrs["final_norm.bias"], w,
                             arrs["semantic_head.bias"], wkind=orc.W_F32)
    elif kind == "bf16":
        want = orc.ln_lmhead(hidden, arrs["final_norm.weight"], arrs["final_norm.bias"], W.f32_to_bf16_bits(w),
                             arrs["semantic_head.bias"])
    else:
        q, sc, bi = W.quantize_affine8(w, 64)
        want = orc.ln_lmhead(hidden, arrs["final_norm.weight"], arrs["final_norm.bias"], q,
                             arrs["semantic_head.bias"], wkind=orc.W_Q8, wscale=sc, wbias=bi, group=64)
    err = np.abs(got.astype(np.float64) - want)
    print(f"{kind}: max abs err {err.max():.3e}", flush=True)
    assert err.max() <= 2e-4
