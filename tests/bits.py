"""Comparison helpers shared by the tests: ulp distance on bf16/f16/f32 bit
patterns and the stated tolerances (bf16: within 1 ulp, i.e. rtol 1e-2 /
atol 1e-3; f32: rtol 1e-5)."""
from __future__ import annotations

import numpy as np

BF16_RTOL, BF16_ATOL = 1e-2, 1e-3
F32_RTOL = 1e-5


def _ordered(bits: np.ndarray, width: int) -> np.ndarray:
    """Map IEEE bit patterns to integers ordered like the values (-0 == +0)."""
    b = bits.astype(np.int64)
    sign = 1 << (width - 1)
    return np.where(b & sign, -(b & (sign - 1)), b)


def ulp_dist(a: np.ndarray, b: np.ndarray, dt: int) -> np.ndarray:
    """Elementwise distance in units in the last place between two arrays of
    storage bits (uint16 for bf16/f16, float32 for f32)."""
    if dt == 0:
        ai = np.ascontiguousarray(a, np.float32).view(np.uint32)
        bi = np.ascontiguousarray(b, np.float32).view(np.uint32)
        return np.abs(_ordered(ai, 32) - _ordered(bi, 32))
    return np.abs(_ordered(a.astype(np.uint16), 16) - _ordered(b.astype(np.uint16), 16))


def nan_mask(a: np.ndarray, dt: int) -> np.ndarray:
    if dt == 0:
        return np.isnan(a)
    a = a.astype(np.uint16)
    if dt == 1:
        return ((a & 0x7F80) == 0x7F80) & ((a & 0x7F) != 0)
    return ((a & 0x7C00) == 0x7C00) & ((a & 0x3FF) != 0)


def assert_close(got, ref, dt, *, max_ulp=1, what="", rtol=None, atol=None, max_bad_frac=0.0):
    """bf16/f16: |ulp distance| <= max_ulp everywhere and allclose at the stated
    tolerance; f32: allclose at rtol (1e-5 by default) plus atol."""
    import oracle

    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    gn, rn = nan_mask(got, dt), nan_mask(ref, dt)
    assert np.array_equal(gn, rn), f"{what}: NaN positions differ"
    g = oracle.to_f32(got, dt)[~gn]
    r = oracle.to_f32(ref, dt)[~rn]
    if dt == 0:
        rt = F32_RTOL if rtol is None else rtol
        at = 0.0 if atol is None else atol
    else:
        rt = BF16_RTOL if rtol is None else rtol
        at = BF16_ATOL if atol is None else atol
        d = ulp_dist(got[~gn], ref[~rn], dt)
        # ulp distance is meaningless next to zero: |diff| <= atol also passes
        far = (d > max_ulp) & (np.abs(g - r) > at)
        n_bad = int(far.sum())
        assert n_bad <= max_bad_frac * d.size, (
            f"{what}: {n_bad} of {d.size} elements differ by more than {max_ulp} ulp "
            f"and atol {at} (max {int(d[far].max()) if n_bad else 0} ulp)")
    bad = ~np.isclose(g, r, rtol=rt, atol=at)
    n_bad = int(bad.sum())
    if n_bad > max_bad_frac * g.size:
        i = int(np.argmax(bad))
        raise AssertionError(
            f"{what}: {n_bad} of {g.size} elements outside rtol={rt} atol={at}; "
            f"first at {i}: got {g[i]!r} ref {r[i]!r}")


def exact_frac(got, ref, dt) -> float:
    return float((ulp_dist(np.asarray(got), np.asarray(ref), dt) == 0).mean())
