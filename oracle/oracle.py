"""ctypes front end of the CPU oracle (oracle/oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the
CPU-baseline leg of bench.py, always as the checker. The product library never
imports it and has no CPU fallback.

Every function mirrors one piece of the reference's host algorithm; the C++
file header lists the reference file:line each one restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile oracle/oracle.cpp with its Makefile (g++ -O3)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_temperature.argtypes = [_f32p, C.c_int, C.c_float]
        L.orc_repetition_penalty.argtypes = [_f32p, C.c_int, _i32p, C.c_int64, C.c_float]
        L.orc_top_k.argtypes = [_f32p, C.c_int, C.c_int]
        L.orc_top_p.argtypes = [_f32p, C.c_int, C.c_float, C.c_int]
        L.orc_top_p_literal.argtypes = [_f32p, C.c_int, C.c_float, C.c_int]
        L.orc_argmax.argtypes = [_f32p, C.c_int]
        L.orc_argmax.restype = C.c_int
        L.orc_xorshift64.argtypes = [C.c_uint64]
        L.orc_xorshift64.restype = C.c_uint64
        L.orc_seed_single.argtypes = [C.c_uint64]
        L.orc_seed_single.restype = C.c_uint64
        L.orc_seed_batch.argtypes = [C.c_uint64, C.c_int, _u64p]
        L.orc_draw.argtypes = [_f32p, C.c_int, _u64p]
        L.orc_draw.restype = C.c_int
        L.orc_sample_rows.argtypes = [
            C.c_void_p, C.c_int, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p, _f32p, _i32p,
            _f32p, _f32p, C.c_void_p, _u8p, C.c_void_p, _u64p, _i32p, C.c_void_p, C.c_int]
        L.orc_sample_stream.argtypes = [
            _f32p, C.c_int64, C.c_int, C.c_int, C.c_int, _i32p, _i64p, _f32p, _i32p, _f32p, _f32p,
            _u8p, C.c_int, _u64p, _i32p, C.c_int]
        L.orc_ln_lmhead.argtypes = [_u16p, C.c_int, C.c_int, _f32p, _f32p, C.c_float, C.c_void_p, C.c_int,
                                    C.c_void_p, C.c_void_p, C.c_int, _f32p, C.c_int, _f32p, C.c_void_p, C.c_int]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---- single-row processors (return a new array; inputs untouched) ----------
def temperature(row, temp):
    v = np.array(row, dtype=np.float32, copy=True)
    lib().orc_temperature(v, v.size, temp)
    return v


def repetition_penalty(row, ids, pen):
    v = np.array(row, dtype=np.float32, copy=True)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    lib().orc_repetition_penalty(v, v.size, ids, ids.size, pen)
    return v


def top_k(row, k):
    v = np.array(row, dtype=np.float32, copy=True)
    lib().orc_top_k(v, v.size, k)
    return v


def top_p(row, p, min_keep=1, literal=False):
    v = np.array(row, dtype=np.float32, copy=True)
    (lib().orc_top_p_literal if literal else lib().orc_top_p)(v, v.size, p, min_keep)
    return v


def argmax(row):
    v = np.ascontiguousarray(row, dtype=np.float32)
    return lib().orc_argmax(v, v.size)


def xorshift64(state: int) -> int:
    return int(lib().orc_xorshift64(state))


def seed_single(seed: int) -> int:
    return int(lib().orc_seed_single(seed))


def seed_batch(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.uint64)
    lib().orc_seed_batch(seed, n, out)
    return out


def draw(row, state: int):
    """Returns (token, new_state) for the reference's inverse-CDF draw."""
    v = np.ascontiguousarray(row, dtype=np.float32)
    s = np.array([state], dtype=np.uint64)
    tok = lib().orc_draw(v, v.size, s)
    return tok, int(s[0])


def sample_rows(logits, hist_ids, hist_off, temp, top_k, top_p, pen, do_sample, rng,
                min_keep=None, row_active=None, want_masked=True, n_threads=1, vocab=None):
    """One AR step over a batch. `logits` is [n_rows, ld] float32 or uint16 (bf16
    bit patterns). Returns (tokens, new_rng, masked or None)."""
    logits = np.ascontiguousarray(logits)
    n_rows, ld = logits.shape
    vocab = ld if vocab is None else vocab
    dtype = 1 if logits.dtype == np.uint16 else 0
    if dtype == 0:
        assert logits.dtype == np.float32
    rng = np.array(rng, dtype=np.uint64, copy=True)
    out_tok = np.zeros(n_rows, dtype=np.int32)
    masked = np.zeros((n_rows, vocab), dtype=np.float32) if want_masked else None
    hist_ids = np.ascontiguousarray(hist_ids, dtype=np.int32)
    hist_off = np.ascontiguousarray(hist_off, dtype=np.int64)
    mk = None if min_keep is None else np.ascontiguousarray(min_keep, dtype=np.int32)
    ra = None if row_active is None else np.ascontiguousarray(row_active, dtype=np.uint8)
    lib().orc_sample_rows(
        _ptr(logits), dtype, ld, n_rows, vocab, _ptr(hist_ids), _ptr(hist_off),
        np.ascontiguousarray(temp, dtype=np.float32), np.ascontiguousarray(top_k, dtype=np.int32),
        np.ascontiguousarray(top_p, dtype=np.float32), np.ascontiguousarray(pen, dtype=np.float32),
        _ptr(mk), np.ascontiguousarray(do_sample, dtype=np.uint8), _ptr(ra), rng, out_tok,
        _ptr(masked), n_threads)
    return out_tok, rng, masked


def sample_stream(logits, hist_ids, hist_off, temp, top_k, top_p, pen, do_sample, rng,
                  stop_token=-1, n_threads=1, vocab=None):
    """Multi-step stream; logits [n_steps, n_rows, ld] float32. Returns (tokens[n_steps, n_rows], rng)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    n_steps, n_rows, ld = logits.shape
    vocab = ld if vocab is None else vocab
    rng = np.array(rng, dtype=np.uint64, copy=True)
    out = np.zeros((n_steps, n_rows), dtype=np.int32)
    lib().orc_sample_stream(
        logits, ld, n_steps, n_rows, vocab, np.ascontiguousarray(hist_ids, dtype=np.int32),
        np.ascontiguousarray(hist_off, dtype=np.int64), np.ascontiguousarray(temp, dtype=np.float32),
        np.ascontiguousarray(top_k, dtype=np.int32), np.ascontiguousarray(top_p, dtype=np.float32),
        np.ascontiguousarray(pen, dtype=np.float32), np.ascontiguousarray(do_sample, dtype=np.uint8),
        stop_token, rng, out, n_threads)
    return out, rng


W_BF16, W_F32, W_Q8 = 0, 1, 2


def ln_lmhead(hidden_bf16, gamma, beta, W, bias, eps=1e-5, n_threads=1, want_h=False, wkind=W_BF16,
              wscale=None, wbias=None, group=64):
    """LayerNorm + linear in double. W: [V][D] bf16 bits (uint16), f32, or
    8-bit affine groups (uint8 codes with f32 scales/biases [V][D/group])."""
    hidden_bf16 = np.ascontiguousarray(hidden_bf16, dtype=np.uint16)
    dt = {W_BF16: np.uint16, W_F32: np.float32, W_Q8: np.uint8}[wkind]
    W = np.ascontiguousarray(W, dtype=dt)
    M, D = hidden_bf16.shape
    V = W.shape[0]
    out = np.zeros((M, V), dtype=np.float32)
    h = np.zeros((M, D), dtype=np.float32) if want_h else None
    ws = None if wscale is None else np.ascontiguousarray(wscale, dtype=np.float32)
    wb = None if wbias is None else np.ascontiguousarray(wbias, dtype=np.float32)
    lib().orc_ln_lmhead(hidden_bf16, M, D, np.ascontiguousarray(gamma, dtype=np.float32),
                        np.ascontiguousarray(beta, dtype=np.float32), eps, W.ctypes.data_as(C.c_void_p), wkind,
                        _ptr(ws), _ptr(wb), group, np.ascontiguousarray(bias, dtype=np.float32), V, out, _ptr(h),
                        n_threads)
    return (out, h) if want_h else out
