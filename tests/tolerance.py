"""Tolerance helpers shared by the GPU parity tests.

``close`` asserts the norm-relative bound the parity contract states
(max|got - ref| / max|ref| <= rel) and also reports the elementwise relative
error |got - ref| / |ref| over the elements whose magnitude is at least
``floor`` times max|ref| (smaller elements have no meaningful relative error
at bf16 precision), so that a test log shows both figures.
"""

from __future__ import annotations

import torch


def errors(got, ref, floor: float = 1e-2):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    scale = ref.abs().max().clamp_min(1e-30)
    diff = (got - ref).abs()
    big = ref.abs() >= floor * scale
    elem = diff[big] / ref.abs()[big]
    n = elem.numel()
    return {
        "max_norm_rel": (diff.max() / scale).item() if diff.numel() else 0.0,
        "elem_rel_max": elem.max().item() if n else 0.0,
        "elem_rel_p99": elem.kthvalue(max(1, min(n, round(0.99 * n)))).values.item() if n else 0.0,
        "elem_rel_median": elem.median().item() if n else 0.0,
    }


def scalar_close(got: float, want: float, rel: float, floor: float, name: str = "") -> None:
    """|got - want| <= rel * max(|want|, floor): relative, except for values below
    ``floor``, whose relative error is rounding noise (e.g. a gate of 1e-7)."""
    assert abs(got - want) <= rel * max(abs(want), floor), f"{name}: {got} vs {want}"


def close(got, ref, rel: float, name: str = "", elem_p99: float = None, floor: float = 1e-2) -> dict:
    """Assert max|got - ref| <= rel * max|ref| (and, if given, the 99th
    percentile of the elementwise relative error <= elem_p99); print both."""
    g = got.detach().float().cpu()
    assert torch.isfinite(g).all(), f"{name}: non-finite"
    e = errors(got, ref, floor)
    print(f"{name}: max-norm rel {e['max_norm_rel']:.3e}; elementwise rel (|ref| >= {floor:g} max) "
          f"median {e['elem_rel_median']:.3e} p99 {e['elem_rel_p99']:.3e} max {e['elem_rel_max']:.3e}")
    assert e["max_norm_rel"] <= rel, f"{name}: max error {e['max_norm_rel']:.3e} of max|ref| exceeds {rel:.1e}"
    if elem_p99 is not None:
        assert e["elem_rel_p99"] <= elem_p99, \
            f"{name}: 99th percentile elementwise relative error {e['elem_rel_p99']:.3e} exceeds {elem_p99:.1e}"
    return e
