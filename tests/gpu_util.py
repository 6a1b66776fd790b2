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


def assert_f16_rows_close(got_bits, want_bits, what=""):
    """Rows stored as f16 (the KV cache's type) against the oracle's own f16
    rows: every element within one f16 ulp (two roundings of f32 values that
    agree to f32 accuracy can land on adjacent f16 values; a rel-L2 bar on
    the rounded rows would measure the rounding, not the kernel)."""
    g = np.asarray(got_bits, np.uint16).view(np.float16).astype(np.float32)
    w = np.asarray(want_bits, np.uint16).view(np.float16).astype(np.float32)
    assert np.all(np.isfinite(g)), f"{what}: non-finite"
    bad = np.abs(g - w) > 2.0 ** -10 * np.maximum(np.abs(w), 2.0 ** -14)
    assert not np.any(bad), f"{what}: {np.count_nonzero(bad)} elements more than one f16 ulp apart"
