"""xorshift64 of text2semantic.cpp:158 (x ^= x << 13; x ^= x >> 7; x ^= x << 17)
built as a GF(2) matrix from explicit shift matrices, independently of any
implementation of the step: used to pin the oracle's step and the GPU's RNG
states."""
import numpy as np

U64 = (1 << 64) - 1
REF_STEPS = [(13, True), (7, False), (17, True)]   # (amount, left shift) in order


def shift_matrix(k, left):
    """GF(2) matrix of x -> x << k (left) or x >> k on 64-bit words; bit i of a
    word is coordinate i."""
    S = np.zeros((64, 64), dtype=np.int64)
    for j in range(64):
        i = j + k if left else j - k
        if 0 <= i < 64:
            S[i, j] = 1
    return S


def xorshift_matrix(steps=REF_STEPS):
    """Matrix of x ^= shift(x) applied for each (amount, left) in order."""
    I = np.eye(64, dtype=np.int64)
    M = I
    for k, left in steps:
        M = ((I + shift_matrix(k, left)) @ M) % 2
    return M


def matpow(M, e):
    R = np.eye(64, dtype=np.int64)
    B = M.copy()
    while e:
        if e & 1:
            R = (R @ B) % 2
        B = (B @ B) % 2
        e >>= 1
    return R


def to_bits(x):
    return np.array([(int(x) >> i) & 1 for i in range(64)], dtype=np.int64)


def from_bits(v):
    return sum(int(b) << i for i, b in enumerate(v))


def advance(state, n, steps=REF_STEPS):
    """The state after n xorshift64 steps, from the matrix construction."""
    return from_bits((matpow(xorshift_matrix(steps), n) @ to_bits(state)) % 2)
