"""Shared helpers of the test suite."""
import hashlib

import numpy as np


def xorshift_uniform(n, state=0x9E3779B9):
    """The reference tests' deterministic generator (tests/check.h:37-44):
    [-1, 1) floats from a 32-bit xorshift."""
    out = np.zeros(n, dtype=np.float32)
    g = state
    for i in range(n):
        g ^= (g << 13) & 0xFFFFFFFF
        g ^= g >> 17
        g ^= (g << 5) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(g & 0xFFFFFF) / np.float32(0x1000000) * np.float32(2.0)
                            - np.float32(1.0))
    return out


def sha_bytes(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
