"""Python binding of libc4s_sampling.so (C ABI in include/c4s_sampling.h).

ctypes only; torch supplies device memory and streams, nothing else. Loading
fails loudly when the library has not been built or no gfx950 device is
present: there is no CPU fallback in this package.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import re
import weakref

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "lib", "libc4s_sampling.so")
HEADER = os.path.join(REPO, "include", "c4s_sampling.h")

OK, EINVAL, EHIP, ENOMEM, ETIMEOUT = 0, 1, 2, 3, 4
F32, BF16 = 0, 1
MODE_CHAIN = 0
P_PENALTY, P_TEMPERATURE, P_TOP_K, P_TOP_P = 1, 2, 4, 8
T_ARGMAX, T_DRAW = 16, 32
MODE_CUSTOM = 256
STAT_PATH, STAT_TOPP_EXACT, STAT_DRAW_EXACT, STAT_KEPT = 0, 1, 2, 3
STREAM_SEQUENTIAL = 1
STREAM_NO_SPECULATION = 2
W_BF16, W_F32, W_Q8 = 0, 1, 2   # c4s_head.wdtype

_vp = C.c_void_p


class Rows(C.Structure):
    _fields_ = [("logits", _vp), ("ld", C.c_int64), ("dtype", C.c_int32), ("n_rows", C.c_int32),
                ("vocab", C.c_int32), ("hist_ids", _vp), ("hist_offsets", _vp),
                ("temperature", _vp), ("top_k", _vp), ("top_p", _vp), ("rep_penalty", _vp),
                ("min_keep", _vp), ("do_sample", _vp), ("row_active", _vp), ("rng_state", _vp),
                ("out_token", _vp), ("out_masked", _vp), ("out_stats", _vp), ("mode", C.c_uint32),
                ("hist_bits", _vp), ("stop_token", C.c_int32)]


class Stream(C.Structure):
    _fields_ = [("logits", _vp), ("ld", C.c_int64), ("step_stride", C.c_int64),
                ("n_steps", C.c_int32), ("n_rows", C.c_int32), ("vocab", C.c_int32),
                ("stop_token", C.c_int32), ("hist_ids", _vp), ("hist_offsets", _vp),
                ("temperature", _vp), ("top_k", _vp), ("top_p", _vp), ("rep_penalty", _vp),
                ("do_sample", _vp), ("rng_state", _vp), ("out_tokens", _vp), ("out_stats", _vp),
                ("flags", C.c_uint32)]


class Head(C.Structure):
    _fields_ = [("hidden", _vp), ("gamma", _vp), ("beta", _vp), ("eps", C.c_float),
                ("weight", _vp), ("bias", _vp), ("M", C.c_int32), ("D", C.c_int32),
                ("V", C.c_int32), ("logits", _vp), ("ld_out", C.c_int64), ("wdtype", C.c_int32),
                ("group", C.c_int32), ("wscale", _vp), ("wbias", _vp)]


class HeadWeights(C.Structure):
    """c4s_head_weights: the LM head's tensors on the device (c4s_head_weights_load)."""
    _fields_ = [("gamma", _vp), ("beta", _vp), ("weight", _vp), ("bias", _vp), ("wscale", _vp),
                ("wbias", _vp), ("D", C.c_int32), ("V", C.c_int32), ("wdtype", C.c_int32), ("group", C.c_int32)]


def header_functions() -> list[str]:
    """Names of every function the public header declares."""
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(c4s_[a-z0-9_]+)\s*\(", txt)))


_lib = None


def _share_torch_runtime() -> None:
    """torch ships its own HIP runtime library. When torch is present its runtime
    is started before this library loads, so that the library binds to the same
    runtime: a second HIP runtime in the process could not open the device."""
    try:
        import torch
    except ImportError:
        return
    if torch.cuda.device_count() > 0:
        torch.cuda.init()


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    _share_torch_runtime()
    L = C.CDLL(LIB_PATH)
    L.c4s_create.argtypes = [C.c_int, C.POINTER(_vp)]
    L.c4s_destroy.argtypes = [_vp]
    L.c4s_last_error.argtypes = [_vp]
    L.c4s_last_error.restype = C.c_char_p
    L.c4s_version.restype = C.c_char_p
    L.c4s_sample_rows.argtypes = [_vp, C.POINTER(Rows), _vp]
    L.c4s_sample_stream.argtypes = [_vp, C.POINTER(Stream), _vp]
    L.c4s_stream_status.argtypes = [_vp, _vp]
    L.c4s_set_wait_limit.argtypes = [_vp, C.c_int32]
    L.c4s_hist_bits_init.argtypes = [_vp, _vp, _vp, C.c_int32, C.c_int32, _vp, _vp]
    L.c4s_lmhead.argtypes = [_vp, C.POINTER(Head), _vp]
    L.c4s_lmhead_sample.argtypes = [_vp, C.POINTER(Head), C.POINTER(Rows), _vp]
    L.c4s_lmhead_sample_noalloc.argtypes = [_vp, C.POINTER(Head), C.POINTER(Rows), _vp]
    L.c4s_seed_single.argtypes = [C.c_uint64]
    L.c4s_seed_single.restype = C.c_uint64
    L.c4s_seed_batch.argtypes = [C.c_uint64, C.c_int32, _vp]
    L.c4s_host_temperature.argtypes = [_vp, _vp, C.c_int32, C.c_float]
    L.c4s_host_repetition_penalty.argtypes = [_vp, _vp, C.c_int32, _vp, C.c_int64, C.c_float]
    L.c4s_host_top_k.argtypes = [_vp, _vp, C.c_int32, C.c_int32]
    L.c4s_host_top_p.argtypes = [_vp, _vp, C.c_int32, C.c_float, C.c_int32]
    L.c4s_host_argmax.argtypes = [_vp, _vp, C.c_int32, _vp]
    L.c4s_host_draw.argtypes = [_vp, _vp, C.c_int32, _vp, _vp]
    L.c4s_hbm_probe.argtypes = [_vp, _vp, _vp, C.c_int64, C.c_int32, _vp]
    L.c4s_tensor_read_f32.argtypes = [C.c_char_p, C.c_char_p, _vp, C.c_int64, _vp, _vp]
    L.c4s_head_weights_load.argtypes = [C.c_char_p, C.c_int32, C.c_int32, C.POINTER(HeadWeights)]
    L.c4s_head_weights_free.argtypes = [C.POINTER(HeadWeights)]
    L.c4s_weights_last_error.restype = C.c_char_p
    _lib = L
    return L


def _p(t):
    """Device (or host numpy) pointer of a tensor/array, or None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def _stream_handle(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if hasattr(stream, "cuda_stream"):
        return stream.cuda_stream
    return stream


class C4SError(RuntimeError):
    pass


# Contexts still open when the interpreter exits are closed by an atexit hook:
# Python runs atexit hooks before it tears down modules and before the C
# runtime's exit handlers unload the HIP runtime (and, under a profiler, the
# profiler's tool library), so c4s_destroy's stream syncs and frees still find
# a live runtime. Leaving them to __del__ during module teardown would run
# those HIP calls in whatever order the garbage collector picks.
_live_contexts: "weakref.WeakSet[Context]" = weakref.WeakSet()


@atexit.register
def _close_live_contexts() -> None:
    for ctx in list(_live_contexts):
        try:
            ctx.close()
        except Exception:
            pass


def read_tensor(root: str, name: str):
    """One tensor of the reference's weight store (<root>.safetensors, else
    <root>/<name>.npy) as float32 numpy, read by the library on the host."""
    import numpy as np
    shape = np.zeros(8, np.int64)
    nd = C.c_int32(0)
    rc = lib().c4s_tensor_read_f32(root.encode(), name.encode(), None, 0, shape.ctypes.data, C.byref(nd))
    if rc:
        raise C4SError(f"tensor_read: code {rc}: {lib().c4s_weights_last_error().decode()}")
    out = np.empty(tuple(shape[: nd.value]), np.float32)
    rc = lib().c4s_tensor_read_f32(root.encode(), name.encode(), out.ctypes.data, out.size, shape.ctypes.data,
                                   C.byref(nd))
    if rc:
        raise C4SError(f"tensor_read: code {rc}: {lib().c4s_weights_last_error().decode()}")
    return out


def load_head_weights(root: str, wdtype: int = W_BF16, group: int = 64) -> HeadWeights:
    """final_norm.* and semantic_head.* of the store at `root` on the current
    device, in storage `wdtype`; free with free_head_weights."""
    hw = HeadWeights()
    rc = lib().c4s_head_weights_load(root.encode(), wdtype, group, C.byref(hw))
    if rc:
        raise C4SError(f"head_weights_load: code {rc}: {lib().c4s_weights_last_error().decode()}")
    return hw


def free_head_weights(hw: HeadWeights) -> None:
    lib().c4s_head_weights_free(C.byref(hw))


class Context:
    """One library context on one device (not thread-safe)."""

    def __init__(self, device: int = 0):
        self._h = _vp()
        rc = lib().c4s_create(device, C.byref(self._h))
        if rc != OK:
            raise C4SError(f"c4s_create(device={device}) failed with code {rc} "
                           "(no gfx950 device visible?)")
        self.device = device
        _live_contexts.add(self)

    def close(self):
        if self._h:
            h, self._h = self._h, _vp()
            lib().c4s_destroy(h)
        _live_contexts.discard(self)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != OK:
            msg = lib().c4s_last_error(self._h).decode()
            raise C4SError(f"{what}: code {rc}: {msg}")

    # ---- device entry points (torch tensors on the GPU) ------------------------
    def sample_rows(self, logits, hist_ids, hist_off, temp, top_k, top_p, pen, rng, out_token,
                    do_sample=None, min_keep=None, row_active=None, out_masked=None,
                    out_stats=None, mode=MODE_CHAIN, vocab=None, stream=None, hist_bits=None,
                    stop_token=-1):
        import torch
        n_rows, ld = logits.shape
        r = Rows(logits=_p(logits), ld=ld, dtype=BF16 if logits.dtype == torch.bfloat16 else F32,
                 n_rows=n_rows, vocab=vocab or ld, hist_ids=_p(hist_ids), hist_offsets=_p(hist_off),
                 temperature=_p(temp), top_k=_p(top_k), top_p=_p(top_p), rep_penalty=_p(pen),
                 min_keep=_p(min_keep), do_sample=_p(do_sample), row_active=_p(row_active),
                 rng_state=_p(rng), out_token=_p(out_token), out_masked=_p(out_masked),
                 out_stats=_p(out_stats), mode=mode, hist_bits=_p(hist_bits), stop_token=stop_token)
        self._check(lib().c4s_sample_rows(self._h, C.byref(r), _stream_handle(stream)), "sample_rows")

    def hist_bits_init(self, hist_ids, hist_off, n_rows, vocab, hist_bits, stream=None):
        """hist_bits[b] (int32 words, [n_rows][(vocab+31)//32]) = the set of row b's CSR history."""
        self._check(lib().c4s_hist_bits_init(self._h, _p(hist_ids), _p(hist_off), n_rows, vocab, _p(hist_bits),
                                             _stream_handle(stream)), "hist_bits_init")

    def sample_stream(self, logits, hist_ids, hist_off, temp, top_k, top_p, pen, rng, out_tokens,
                      do_sample=None, stop_token=-1, out_stats=None, stream=None, sequential=False,
                      speculate=True):
        n_steps, n_rows, ld = logits.shape
        s = Stream(logits=_p(logits), ld=ld, step_stride=n_rows * ld, n_steps=n_steps,
                   n_rows=n_rows, vocab=ld, stop_token=stop_token, hist_ids=_p(hist_ids),
                   hist_offsets=_p(hist_off), temperature=_p(temp), top_k=_p(top_k),
                   top_p=_p(top_p), rep_penalty=_p(pen), do_sample=_p(do_sample),
                   rng_state=_p(rng), out_tokens=_p(out_tokens), out_stats=_p(out_stats),
                   flags=(STREAM_SEQUENTIAL if sequential else 0) | (0 if speculate else STREAM_NO_SPECULATION))
        self._check(lib().c4s_sample_stream(self._h, C.byref(s), _stream_handle(stream)),
                    "sample_stream")

    def stream_status(self, stream=None):
        """C4S_OK, or C4S_ETIMEOUT when a sample_stream call gave up a row (the
        record is cleared); synchronizes `stream` first."""
        return lib().c4s_stream_status(self._h, _stream_handle(stream))

    def set_wait_limit(self, polls):
        """Polls of the speculative chains' bounded waits before they give up (<= 0: default)."""
        self._check(lib().c4s_set_wait_limit(self._h, int(polls)), "set_wait_limit")

    @staticmethod
    def _head(hidden, gamma, beta, weight, bias, logits, eps, quant=None):
        """quant: None for bf16 or fp32 weights (from weight's dtype), else
        (scales, biases, group) of 8-bit codes (uint8 weight)."""
        M, D = hidden.shape
        V = weight.shape[0]
        kind = {"torch.bfloat16": W_BF16, "torch.int16": W_BF16, "torch.float32": W_F32,
                "torch.uint8": W_Q8}.get(str(weight.dtype))
        if kind is None:
            raise ValueError(f"lmhead: unsupported weight dtype {weight.dtype}")
        if (kind == W_Q8) != (quant is not None):
            raise ValueError("lmhead: 8-bit weights need quant=(scales, biases, group), others none")
        ws, wb, group = quant if quant is not None else (None, None, 0)
        return Head(hidden=_p(hidden), gamma=_p(gamma), beta=_p(beta), eps=eps, weight=_p(weight),
                    bias=_p(bias), M=M, D=D, V=V, logits=_p(logits),
                    ld_out=(logits.shape[1] if logits is not None else V), wdtype=kind, group=group,
                    wscale=_p(ws), wbias=_p(wb))

    def lmhead_loaded(self, hw: HeadWeights, hidden, logits, eps=1e-5, stream=None):
        """c4s_lmhead with the tensors of load_head_weights."""
        M, D = hidden.shape
        if D != hw.D:
            raise ValueError(f"hidden has D={D}, the head D={hw.D}")
        h = Head(hidden=_p(hidden), gamma=hw.gamma, beta=hw.beta, eps=eps, weight=hw.weight, bias=hw.bias,
                 M=M, D=D, V=hw.V, logits=_p(logits), ld_out=logits.shape[1], wdtype=hw.wdtype, group=hw.group,
                 wscale=hw.wscale, wbias=hw.wbias)
        self._check(lib().c4s_lmhead(self._h, C.byref(h), _stream_handle(stream)), "lmhead")

    def lmhead_sample_loaded(self, hw: HeadWeights, hidden, temp, top_k, top_p, pen, rng, out_token, logits=None,
                             hist_ids=None, hist_off=None, hist_bits=None, do_sample=None, stop_token=-1, eps=1e-5,
                             stream=None):
        """c4s_lmhead_sample with the tensors of load_head_weights: one AR step
        from the hidden rows to the tokens (text2semantic.cpp:297-337)."""
        M, D = hidden.shape
        if D != hw.D:
            raise ValueError(f"hidden has D={D}, the head D={hw.D}")
        h = Head(hidden=_p(hidden), gamma=hw.gamma, beta=hw.beta, eps=eps, weight=hw.weight, bias=hw.bias,
                 M=M, D=D, V=hw.V, logits=_p(logits), ld_out=hw.V if logits is None else logits.shape[1],
                 wdtype=hw.wdtype, group=hw.group, wscale=hw.wscale, wbias=hw.wbias)
        r = Rows(hist_ids=_p(hist_ids), hist_offsets=_p(hist_off), temperature=_p(temp), top_k=_p(top_k),
                 top_p=_p(top_p), rep_penalty=_p(pen), do_sample=_p(do_sample), rng_state=_p(rng),
                 out_token=_p(out_token), mode=MODE_CHAIN, hist_bits=_p(hist_bits), stop_token=stop_token)
        self._check(lib().c4s_lmhead_sample(self._h, C.byref(h), C.byref(r), _stream_handle(stream)),
                    "lmhead_sample")

    def lmhead(self, hidden, gamma, beta, weight, bias, logits, eps=1e-5, stream=None, quant=None):
        h = self._head(hidden, gamma, beta, weight, bias, logits, eps, quant)
        self._check(lib().c4s_lmhead(self._h, C.byref(h), _stream_handle(stream)), "lmhead")

    def lmhead_sample(self, hidden, gamma, beta, weight, bias, hist_ids, hist_off, temp, top_k,
                      top_p, pen, rng, out_token, logits=None, do_sample=None, out_masked=None,
                      out_stats=None, eps=1e-5, stream=None, hist_bits=None, stop_token=-1, quant=None):
        h = self._head(hidden, gamma, beta, weight, bias, logits, eps, quant)
        r = Rows(hist_ids=_p(hist_ids), hist_offsets=_p(hist_off), temperature=_p(temp),
                 top_k=_p(top_k), top_p=_p(top_p), rep_penalty=_p(pen), do_sample=_p(do_sample),
                 rng_state=_p(rng), out_token=_p(out_token), out_masked=_p(out_masked),
                 out_stats=_p(out_stats), mode=MODE_CHAIN, hist_bits=_p(hist_bits), stop_token=stop_token)
        self._check(lib().c4s_lmhead_sample(self._h, C.byref(h), C.byref(r), _stream_handle(stream)),
                    "lmhead_sample")

    def lmhead_sample_noalloc(self, hidden, gamma, beta, weight, bias, hist_ids, hist_off, temp, top_k,
                              top_p, pen, rng, out_token, logits=None, do_sample=None, out_masked=None,
                              out_stats=None, eps=1e-5, stream=None, hist_bits=None, stop_token=-1, quant=None):
        """c4s_lmhead_sample with its workspace in the library's static device scratch."""
        h = self._head(hidden, gamma, beta, weight, bias, logits, eps, quant)
        r = Rows(hist_ids=_p(hist_ids), hist_offsets=_p(hist_off), temperature=_p(temp),
                 top_k=_p(top_k), top_p=_p(top_p), rep_penalty=_p(pen), do_sample=_p(do_sample),
                 rng_state=_p(rng), out_token=_p(out_token), out_masked=_p(out_masked),
                 out_stats=_p(out_stats), mode=MODE_CHAIN, hist_bits=_p(hist_bits), stop_token=stop_token)
        self._check(lib().c4s_lmhead_sample_noalloc(self._h, C.byref(h), C.byref(r), _stream_handle(stream)),
                    "lmhead_sample_noalloc")

    def hbm_probe(self, src, dst, nbytes, mode=0, stream=None):
        self._check(lib().c4s_hbm_probe(self._h, _p(src), _p(dst), nbytes, mode,
                                        _stream_handle(stream)), "hbm_probe")

    # ---- host-buffer single-row helpers (numpy, synchronous) ---------------------
    def host_temperature(self, row, temp):
        import numpy as np
        v = np.array(row, dtype=np.float32, copy=True)
        self._check(lib().c4s_host_temperature(self._h, v.ctypes.data, v.size, temp), "temperature")
        return v

    def host_repetition_penalty(self, row, ids, pen):
        import numpy as np
        v = np.array(row, dtype=np.float32, copy=True)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        self._check(lib().c4s_host_repetition_penalty(self._h, v.ctypes.data, v.size,
                                                      ids.ctypes.data if ids.size else None,
                                                      ids.size, pen), "repetition_penalty")
        return v

    def host_top_k(self, row, k):
        import numpy as np
        v = np.array(row, dtype=np.float32, copy=True)
        self._check(lib().c4s_host_top_k(self._h, v.ctypes.data, v.size, k), "top_k")
        return v

    def host_top_p(self, row, p, min_keep=1):
        import numpy as np
        v = np.array(row, dtype=np.float32, copy=True)
        self._check(lib().c4s_host_top_p(self._h, v.ctypes.data, v.size, p, min_keep), "top_p")
        return v

    def host_argmax(self, row):
        import numpy as np
        v = np.ascontiguousarray(row, dtype=np.float32)
        out = C.c_int32(0)
        self._check(lib().c4s_host_argmax(self._h, v.ctypes.data, v.size, C.addressof(out)), "argmax")
        return out.value

    def host_draw(self, row, state):
        import numpy as np
        v = np.ascontiguousarray(row, dtype=np.float32)
        s = C.c_uint64(state)
        out = C.c_int32(0)
        self._check(lib().c4s_host_draw(self._h, v.ctypes.data, v.size, C.addressof(s),
                                        C.addressof(out)), "draw")
        return out.value, s.value


def seed_single(seed: int) -> int:
    return int(lib().c4s_seed_single(seed))


def seed_batch(seed: int, n: int):
    import numpy as np
    out = np.zeros(n, dtype=np.uint64)
    lib().c4s_seed_batch(seed, n, out.ctypes.data)
    return out
