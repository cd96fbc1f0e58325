"""Parity bars shared by the GPU tests, with the achieved errors recorded.

bf16 outputs: |got - ref| <= rtol * |ref| + atol with rtol = 2e-2 and
atol = min(1e-2, 2e-2 * RMS(ref)): the reference's device tolerance is
rtol = atol = 1e-2 on the output (tests/utils.py:19-25), the bf16 bar of the
workloads is rtol 2e-2, and outputs whose RMS is below 0.5 get a floor
proportional to their scale instead of the fixed 1e-2 (a fixed floor would
be loose for them).  With ``axis`` the RMS is taken per slice along that
axis (attention rows attend over different numbers of keys, so their
scales differ).  Every check records its worst errors; the session summary
prints them.
"""

from __future__ import annotations

import numpy as np

RECORDS = []


def ulp_bf16(v):
    """Spacing of bf16 values at |v| (8 significant bits)."""
    v = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_close(got, ref, name: str, rtol: float = 2e-2, atol: float = 1e-2, floor: float = 2e-2,
                 axis=None, rounded=None, max_flip_frac: float = 0.01):
    """``rounded``: an intermediate the computation rounds to bf16 before a
    later add (e.g. p in bf16(z + bf16(p))).  Its fp32 value depends on the
    accumulation order, so its rounding may land one bf16 step away from the
    reference's; up to ``max_flip_frac`` of the elements may then be off by
    one ulp of that intermediate beyond the bar."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{name}: non-finite output"
    if axis is None:
        rms = np.sqrt(np.mean(ref ** 2))
    else:
        rms = np.sqrt(np.mean(ref ** 2, axis=axis, keepdims=True))
    a = np.minimum(atol, floor * rms)
    err = np.abs(got - ref)
    bound = rtol * np.abs(ref) + a
    over = err > bound
    flips = 0
    if rounded is not None:
        step = ulp_bf16(rounded) * 1.0001 + ulp_bf16(ref)
        flips = int(over.sum())
        assert np.all(err[over] <= (bound + step)[over]), \
            f"{name}: errors beyond one rounding step of the bf16 intermediate"
        assert flips <= max_flip_frac * err.size, f"{name}: {flips} of {err.size} elements off by a rounding step"
        ratio = float(np.max(np.where(over, 0.0, err / bound))) if err.size else 0.0
    else:
        ratio = float(np.max(err / bound)) if err.size else 0.0
    rec = {"check": name, "n": int(err.size), "max_abs": float(err.max()) if err.size else 0.0,
           "max_rel": float(np.max(err / np.maximum(np.abs(ref), 1e-30))) if err.size else 0.0,
           "worst_of_bar": ratio, "flips": flips}
    RECORDS.append(rec)
    assert ratio <= 1.0, (f"{name}: {int(over.sum())} of {err.size} elements out of tolerance; "
                          f"max abs {rec['max_abs']:.3e}, worst {ratio:.3f} of the bar")
    return rec


def record_close(got, ref, name: str, **kw) -> float:
    """``assert_close``'s measurement without its assertion: records the
    check and returns its worst error as a fraction of the bar."""
    try:
        assert_close(got, ref, name, **kw)
    except AssertionError:
        pass
    return RECORDS[-1]["worst_of_bar"]


def assert_rel(got, ref, name: str, tol: float):
    """fp32 bar: max |got - ref| / |ref| <= tol."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    rel = float(np.max(err / np.abs(ref)))
    RECORDS.append({"check": name, "n": int(err.size), "max_abs": float(err.max()), "max_rel": rel,
                    "worst_of_bar": rel / tol})
    assert rel <= tol, f"{name}: max rel err {rel:.3e} > {tol:.1e}"


def assert_matches_numpy(got, ref, what: str):
    """A kernel run against the same function run by NumPy (tuples item by
    item).  fp32: |got - ref| <= 1e-4 |ref| + 1e-4 max(1, RMS(ref)); fp16:
    1e-2 on both parts; integers and booleans exactly."""
    if isinstance(ref, (tuple, list)):
        assert isinstance(got, (tuple, list)) and len(got) == len(ref), what
        for i, (g, r) in enumerate(zip(got, ref)):
            assert_matches_numpy(g, r, f"{what}[{i}]")
        return
    ref = np.asarray(ref)
    got = np.asarray(got)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    if not np.issubdtype(ref.dtype, np.floating):
        np.testing.assert_array_equal(got.astype(np.int64), ref.astype(np.int64), err_msg=what)
        return
    tol = 1e-2 if ref.dtype == np.float16 else 1e-4
    r = ref.astype(np.float64)
    g = got.astype(np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(r)), f"{what}: NaN positions differ"
    fin = ~np.isnan(r)
    r, g = r[fin], g[fin]
    scale = max(1.0, float(np.sqrt(np.mean(r * r)))) if r.size else 1.0
    err = np.abs(g - r)
    bound = tol * np.abs(r) + tol * scale
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} of {r.size} out of tolerance, max abs {err.max():.3e}"


def launch_symbols(plan):
    """Kernel symbols of a plan's launches in order, for a freshly lowered
    plan or for one loaded from the artefact cache (a kernel compiled
    earlier in the same process with the same graph)."""
    if hasattr(plan, "records"):
        return [r.symbol for r in plan.records]
    return [l.symbol for st in plan.steps for l in st.launches(lambda v: 1 << 40)]
