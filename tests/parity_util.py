"""Shared checks: device record / meta against the CPU oracle."""

from __future__ import annotations

import math

from golden_io import same_value
from oracle import torch_verdict as tv

# fp64 sums are accumulated in a different order on the device; the contract is 1e-6 relative
SUM_RTOL = 1e-6
# near_zero_mean_abs: torch sums float32 in its own cascade order; the device sums in fp64
MEAN_RTOL = 1e-5

EXACT_FIELDS = ("ulp_hist", "nan_pairs", "equal_count", "max_abs_index", "max_rel_index", "finite_violations",
                "first_finite_violation", "nan_gen", "nan_ref", "posinf_gen", "posinf_ref", "neginf_gen",
                "neginf_ref")


def close(a: float, b: float, rtol: float) -> bool:
    if a is None or b is None:
        return a is b
    if math.isnan(a) or math.isnan(b):
        return math.isnan(a) and math.isnan(b)
    if math.isinf(a) or math.isinf(b):
        return a == b
    return abs(a - b) <= rtol * max(abs(a), abs(b)) or abs(a - b) <= 1e-300


def record_vs_oracle(rec: dict, gen_cpu, ref_cpu, tolerance_policy=None):
    """Problems between a device record and the oracle's extension record (empty list = parity)."""
    exp = tv.extension_record(gen_cpu, ref_cpu, tolerance_policy)
    got = dict(rec)
    got["equal_count"] = got["ulp_hist"][0]
    bad = []
    for k in EXACT_FIELDS:
        if not same_value(got[k], exp[k]):
            bad.append(f"{k}: device {got[k]!r} != oracle {exp[k]!r}")
    for k in ("max_abs", "max_rel"):
        if exp[k] is None:
            continue
        if not same_value(float(got[k]), float(exp[k])):
            bad.append(f"{k}: device {got[k]!r} != oracle {exp[k]!r}")
    for k in ("sum_gg", "sum_rr", "sum_gr", "sum_dd", "rel_l2", "cosine"):
        if not close(got[k], exp[k], SUM_RTOL):
            bad.append(f"{k}: device {got[k]!r} vs oracle {exp[k]!r}")
    return bad


# sampled cosine / norm ratio: fp64 sums in another order, then round(., 4).  The
# unrounded values agree to SUM_RTOL; rounding hides that unless the value is
# large (no digits dropped) or sits on a rounding boundary (one step apart).
SAMPLED_SUM_KEYS = ("cosine_similarity", "norm_ratio")


def sampled_sum_close(a, b) -> bool:
    if same_value(a, b):
        return True
    if not isinstance(a, float) or not isinstance(b, float):
        return False
    return close(a, b, SUM_RTOL) or abs(a - b) <= 1e-4 + 1e-12


def meta_problems(got: dict, want: dict):
    """Exact meta comparison (key order included) except the near-zero mean (float32
    summation order) and the sampled cosine / norm ratio (fp64 summation order)."""
    out = []
    if list(got.keys()) != list(want.keys()):
        out.append(f"key order {list(got.keys())} != {list(want.keys())}")
    for k in want:
        if k not in got:
            continue
        if k in SAMPLED_SUM_KEYS:
            if not sampled_sum_close(got[k], want[k]):
                out.append(f"{k}: device {got[k]!r} vs oracle {want[k]!r}")
        elif k == "near_zero_mean_abs" and got[k] is not None and want[k] is not None:
            if not close(got[k], want[k], MEAN_RTOL):
                out.append(f"{k}: {got[k]!r} vs {want[k]!r}")
        elif not same_value(got[k], want[k]):
            out.append(f"{k}: device {got[k]!r} != oracle {want[k]!r}")
    return out


def details_match(got, want) -> bool:
    return list(got) == list(want)
