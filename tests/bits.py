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


def check_rope_parity(got, ref_libm, ref_dev, dt, what=""):
    """The RoPE bar, with no allowance for stray elements.

    ref_dev is the oracle with the device's cos/sin evaluation (f32 of f64
    cos/sin); ref_libm the oracle with libm's f32 cosf/sinf, as MLX's CPU rope.
    Against ref_dev every element must be within 1 ulp (or atol 1e-3) for
    16-bit outputs, within rtol 1e-5 for f32. Against ref_libm every element
    outside that bar must sit where the two oracles themselves differ, i.e.
    where a cos/sin value rounds differently. Returns a one-line summary."""
    got, ref_libm, ref_dev = np.asarray(got), np.asarray(ref_libm), np.asarray(ref_dev)
    if dt == 0:
        assert_close(got, ref_dev, dt, rtol=F32_RTOL, atol=0.0, what=what)
        g = got.astype(np.float64)
        r = ref_libm.astype(np.float64)
        beyond = ~np.isclose(g, r, rtol=F32_RTOL, atol=0.0)
        differ = ref_libm.view(np.uint32) != ref_dev.view(np.uint32)
    else:
        assert_close(got, ref_dev, dt, max_ulp=1, what=what)
        import oracle

        d = ulp_dist(got, ref_libm, dt)
        diff = np.abs(oracle.to_f32(got, dt) - oracle.to_f32(ref_libm, dt))
        beyond = (d > 1) & (diff > BF16_ATOL)
        differ = ref_libm != ref_dev
    unexplained = beyond & ~differ
    worst = int(ulp_dist(got, ref_libm, dt)[beyond].max()) if beyond.any() else 0
    assert not unexplained.any(), (
        f"{what}: {int(unexplained.sum())} elements outside the bar against the libm oracle where "
        f"the two oracles agree (first at {np.argwhere(unexplained)[0]})")
    return (f"exact vs device-trig oracle {exact_frac(got, ref_dev, dt):.6f}, max ulp "
            f"{int(ulp_dist(got, ref_dev, dt).max()) if got.size else 0}; vs libm oracle "
            f"{int(beyond.sum())} of {got.size} beyond the bar (worst {worst} ulp), all where "
            f"the oracles' cos/sin differ ({int(differ.sum())} such elements)")


def check_geglu_f32(got, ref, g, u, what="", chunk=1 << 22):
    """The f32 GeGLU bar. The reference composes 0.5 g (1 + tanh(k0 (g + k1
    g^3))) u in f32; for negative g the sum 1 + tanh(.) cancels, and tanhf's
    error (at most 2 ulp, 2^-23 near -1) comes through it as an absolute error
    of up to 2^-24 |g u| in the reference's own value. The device evaluates g /
    (1 + e^(-2x)), which does not cancel. Bar: every element within
    rtol 1e-5 plus 2^-23 |g u| (twice that bound), and within rtol 1e-5 alone
    wherever g >= -2 (where 1 + tanh >= 0.045, so the cancellation moves the
    reference by less than 3e-6 relative). g and u are the f32 inputs.
    Returns a one-line summary with the worst ratio to the bar."""
    got, ref = np.asarray(got).reshape(-1), np.asarray(ref).reshape(-1)
    g, u = np.asarray(g).reshape(-1), np.asarray(u).reshape(-1)
    worst, worst_at, worst_mild, worst_neg, n_neg = 0.0, -1, 0.0, 0.0, 0
    for lo in range(0, got.size, chunk):
        sl = slice(lo, lo + chunk)
        gg, uu = g[sl].astype(np.float64), u[sl].astype(np.float64)
        r = ref[sl].astype(np.float64)
        err = np.abs(got[sl].astype(np.float64) - r)
        tol = F32_RTOL * np.abs(r) + 2.0 ** -23 * np.abs(gg * uu)
        over = err > tol
        assert not over.any(), (
            f"{what}: {int(over.sum())} elements outside rtol 1e-5 + 2^-23|g u|, first at "
            f"{lo + int(np.argmax(over))}: got {got[lo + int(np.argmax(over))]!r} "
            f"ref {ref[lo + int(np.argmax(over))]!r}")
        ratio = np.where(tol > 0, err / np.where(tol > 0, tol, 1.0), 0.0)
        if ratio.max() > worst:
            worst, worst_at = float(ratio.max()), lo + int(np.argmax(ratio))
        # relative errors are reported where the reference is not zero (for
        # g < -2 the reference's 1 + tanh may round to exactly 0)
        rel = np.where(r != 0, err / np.where(r != 0, np.abs(r), 1.0), 0.0)
        mild = gg >= -2.0
        bad = mild & (err > F32_RTOL * np.abs(r))
        assert not bad.any(), (
            f"{what}: {int(bad.sum())} elements with g >= -2 outside rtol 1e-5, first at "
            f"{lo + int(np.argmax(bad))}")
        if mild.any():
            worst_mild = max(worst_mild, float(rel[mild].max()))
        if (~mild).any():
            worst_neg = max(worst_neg, float(rel[~mild].max()))
            n_neg += int((~mild).sum())
    return (f"worst ratio to the bar {worst:.3f} (element {worst_at}); g >= -2: worst "
            f"relative error {worst_mild:.3g}; g < -2: {n_neg} elements, worst relative error "
            f"{worst_neg:.3g} where the reference is not 0")
