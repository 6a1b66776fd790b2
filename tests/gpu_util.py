"""Shared helpers of the GPU parity tests."""
import numpy as np

import oracle as O

# Tolerance of every floating-point parity check:
REL_L2 = 1e-3
COS = 0.9999


def assert_close(got, ref, rel=REL_L2, cos=COS, what=""):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    r = O.rel_l2(got, ref)
    c = O.cosine(got, ref)
    assert r <= rel and c >= cos, f"{what}: rel_l2={r:.3e} cos={c:.8f}"
    return r, c


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.float32:
        nan_a, nan_b = np.isnan(a), np.isnan(b)
        return np.array_equal(nan_a, nan_b) and np.array_equal(a[~nan_a].view(np.uint32), b[~nan_b].view(np.uint32))
    return np.array_equal(a, b)



def assert_f16_row_close(got_bits, want_f32, what=""):
    """A row stored as f16 (the KV cache's type) against the oracle's f32 row
    before rounding, at the floating-point bar: the f16 rounding itself is at
    most 2^-11 relative per element."""
    g = np.asarray(got_bits, np.uint16).view(np.float16).astype(np.float32)
    return assert_close(g, want_f32, what=what)
