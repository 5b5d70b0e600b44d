"""C ABI checks that need no GPU: the library loads, exports every function the
public header declares, and fails cleanly (no crash, an error code) when no
device is present or arguments are bad."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import c4s


def test_library_built():
    assert os.path.exists(c4s.LIB_PATH), "run __graft_entry__.build() first"


def test_exports_every_header_symbol():
    names = c4s.header_functions()
    assert len(names) >= 16
    out = subprocess.run(["nm", "-D", "--defined-only", c4s.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    L = c4s.lib()
    for n in names:
        assert hasattr(L, n)


def test_version_string():
    assert b"gfx950" in c4s.lib().c4s_version()


def test_seed_helpers_match_oracle(orc):
    assert c4s.seed_single(0) == orc.seed_single(0)
    assert c4s.seed_single(99) == 99
    assert np.array_equal(c4s.seed_batch(1234, 64), orc.seed_batch(1234, 64))


def test_null_context_is_einval():
    L = c4s.lib()
    assert L.c4s_sample_rows(None, None, None) == c4s.EINVAL
    assert L.c4s_sample_stream(None, None, None) == c4s.EINVAL
    assert L.c4s_lmhead(None, None, None) == c4s.EINVAL
    assert L.c4s_hist_bits_init(None, None, None, 0, 0, None, None) == c4s.EINVAL
    v = np.zeros(4, np.float32)
    assert L.c4s_host_top_k(None, v.ctypes.data, 4, 2) == c4s.EINVAL
    assert L.c4s_create(0, None) == c4s.EINVAL
    assert L.c4s_destroy(None) == c4s.OK


def test_create_without_gpu_reports_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    h = C.c_void_p()
    rc = c4s.lib().c4s_create(0, C.byref(h))
    assert rc in (c4s.EHIP, c4s.EINVAL) and not h.value


def test_cpp_mirror_exports_reference_signatures():
    lib = os.path.join(c4s.HERE, "lib", "libc4tts_sampling.so")
    out = subprocess.run(["nm", "-DC", "--defined-only", lib], capture_output=True, text=True,
                         check=True).stdout
    for sig in ["c4::t2s::sampling::temperature(std::vector<float, std::allocator<float> >&, float)",
                "c4::t2s::sampling::repetition_penalty(std::vector<float, std::allocator<float> >&, "
                "std::vector<int, std::allocator<int> > const&, float)",
                "c4::t2s::sampling::top_k(std::vector<float, std::allocator<float> >&, int)",
                "c4::t2s::sampling::top_p(std::vector<float, std::allocator<float> >&, float, int)",
                "c4::t2s::sampling::argmax(std::vector<float, std::allocator<float> > const&)"]:
        assert sig in out, sig


def test_ctypes_structs_match_the_header(tmp_path):
    """The binding's struct layouts (size, every field's offset) equal what a C
    compiler makes of the public header."""
    structs = {"c4s_rows": c4s.Rows, "c4s_stream": c4s.Stream, "c4s_head": c4s.Head}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{c4s.HEADER}"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, got):
        cname, what, val = line.split()
        py = structs[cname]
        want = C.sizeof(py) if what == "size" else getattr(py, what).offset
        assert int(val) == want, (cname, what, int(val), want)
