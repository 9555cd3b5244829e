"""Shared checks: device record / meta against the CPU oracle."""

from __future__ import annotations

import math

import torch

from golden_io import same_value
from oracle import torch_verdict as tv

# fp64 sums are accumulated in a different order on the device; the contract is 1e-6 relative
SUM_RTOL = 1e-6
# near_zero_mean_abs: torch sums float32 in its own cascade order; the device sums in fp64 and
# rounds once.  Over 3,000 seeded near-zero samples (1 to 10^6 values: 1-ULP bf16 steps with
# exact zeros, fp16 diffs, 30 binades of range, tiny values with rare large ones) the largest
# relative gap between the two was 5.5e-7.
MEAN_RTOL = 1e-6

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


def record_vs_oracle(rec: dict, gen_cpu, ref_cpu, tolerance_policy=None, max_samples=tv.MAX_SAMPLES):
    """Problems between a device record and the oracle's extension record, the sampled
    cosine and norm ratio included (empty list = parity)."""
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
    bad += sampled_record_problems(rec, gen_cpu, ref_cpu, max_samples)
    return bad


# Sampled cosine and norm ratio (GCR:351-393).  Device and torch both sum fp64
# products and differ only in summation order, so the unrounded values agree to
# about 1e-15; the check is 1e-12 relative (with a 1e-15 floor for cosines near
# zero), far inside the declared 1e-6.  After round(., 4) the metas must then be
# identical, except where the oracle's unrounded value lies within 1e-9 of a
# rounding boundary (x.xxxx5), where either neighbour is accepted, and where the
# magnitude is so large (>= 1e11, fp64 spacing above 1e-5) that round(., 4)
# keeps every digit, so the meta shows the unrounded value (1e-12 relative).
UNROUNDED_RTOL = 1e-12
UNROUNDED_FLOOR = 1e-15
BOUNDARY_EPS = 1e-9
ROUNDING_IDENTITY = 1e11
SAMPLED_SUM_KEYS = ("cosine_similarity", "norm_ratio")


def unrounded_close(a, b) -> bool:
    if a is None or b is None:
        return a is b
    a, b = float(a), float(b)
    if math.isnan(a) or math.isnan(b):
        return math.isnan(a) and math.isnan(b)
    if math.isinf(a) or math.isinf(b):
        return a == b
    return abs(a - b) <= max(UNROUNDED_RTOL * max(abs(a), abs(b)), UNROUNDED_FLOOR)


def near_rounding_boundary(x, places: int = 4, eps: float = BOUNDARY_EPS) -> bool:
    """True when x is within eps of a value halfway between two 4-place neighbours."""
    if x is None or not math.isfinite(x):
        return False
    scaled = abs(x) * 10 ** places
    return abs(scaled - math.floor(scaled) - 0.5) <= eps * 10 ** places


def sampled_unrounded(gen_cpu, ref_cpu, max_samples=tv.MAX_SAMPLES) -> dict:
    """The oracle's cosine similarity and norm ratio before rounding."""
    return {"cosine_similarity": tv.cosine_similarity_value(gen_cpu, ref_cpu, max_samples),
            "norm_ratio": tv.norm_ratio_value(gen_cpu, ref_cpu, max_samples)}


def rounded_sampled_ok(got, want, unrounded) -> bool:
    """A device meta value against the reference's: equal, or one step apart at a rounding boundary."""
    if same_value(got, want):
        return True
    if not isinstance(got, float) or not isinstance(want, float):
        return False
    if math.isfinite(want) and abs(want) >= ROUNDING_IDENTITY and unrounded_close(got, want):
        return True
    if unrounded is None:
        return False
    return near_rounding_boundary(unrounded) and abs(got - want) <= 1e-4 + 1e-12


def meta_problems(got: dict, want: dict, gen_cpu=None, ref_cpu=None, max_samples=tv.MAX_SAMPLES):
    """Exact meta comparison (key order included).  Two exceptions: the near-zero mean (the
    reference sums float32 in torch's cascade order, the device fp64; 1e-5 relative) and the
    sampled cosine / norm ratio at a rounding boundary of the oracle's unrounded value, which
    needs the pair (gen_cpu, ref_cpu) to be recomputed."""
    out = []
    if list(got.keys()) != list(want.keys()):
        out.append(f"key order {list(got.keys())} != {list(want.keys())}")
    unrounded = None
    for k in want:
        if k not in got:
            continue
        if k in SAMPLED_SUM_KEYS:
            if same_value(got[k], want[k]):
                continue
            if unrounded is None and gen_cpu is not None:
                unrounded = sampled_unrounded(gen_cpu, ref_cpu, max_samples)
            if not rounded_sampled_ok(got[k], want[k], unrounded[k] if unrounded else None):
                out.append(f"{k}: device {got[k]!r} vs reference {want[k]!r} (oracle unrounded "
                           f"{unrounded[k] if unrounded else 'not computed'!r})")
        elif k == "near_zero_mean_abs" and got[k] is not None and want[k] is not None:
            if not close(got[k], want[k], MEAN_RTOL):
                out.append(f"{k}: {got[k]!r} vs {want[k]!r}")
        elif not same_value(got[k], want[k]):
            out.append(f"{k}: device {got[k]!r} != oracle {want[k]!r}")
    return out


def sampled_record_problems(rec: dict, gen_cpu, ref_cpu, max_samples=tv.MAX_SAMPLES):
    """The record's unrounded sample_cosine / sample_norm_ratio against the oracle's (float inputs)."""
    if not torch.is_floating_point(ref_cpu) or ref_cpu.numel() == 0:
        return []
    want = sampled_unrounded(gen_cpu, ref_cpu, max_samples)
    bad = []
    for rk, k in (("sample_cosine", "cosine_similarity"), ("sample_norm_ratio", "norm_ratio")):
        if not unrounded_close(rec[rk], want[k]):
            bad.append(f"{rk}: device {rec[rk]!r} vs oracle {want[k]!r} (unrounded, rtol {UNROUNDED_RTOL})")
    return bad


def details_match(got, want) -> bool:
    return list(got) == list(want)
