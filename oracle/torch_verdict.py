"""CPU oracle for the numerical-agreement verdict -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``kernelverse_amd.verdict``) never calls it and
fails loudly when the HIP library is missing.

It restates, with the same torch-CPU operations in the same order, the
verdict of KernelVerse ``runner/generated_correctness_runner.py`` (GCR):

* ``dtype_name``              GCR:212-223
* ``dtype_policy``            GCR:305-328 (+ ``TOLERANCE_POLICY`` GCR:39-44)
* ``format_number``           GCR:331-335
* ``sample_flat_values``      GCR:338-348
* ``cosine_similarity_meta``  GCR:351-372 (``cosine_similarity_value``: the same
  before its final rounding)
* ``norm_ratio_meta``         GCR:375-393 (``norm_ratio_value`` likewise)
* ``p99_meta``                GCR:396-402
* ``mean_meta``               GCR:405-411
* ``finite_pattern_pass``     GCR:414-437
* ``threshold_pass`` / ``cosine_pass`` / ``range_pass``  GCR:440-478
* ``near_zero_abs_policy_pass``  GCR:481-548
* ``evaluate_tensor_policy``  GCR:551-606
* ``compare_tensors``         GCR:672-786
* ``compare_outputs``         GCR:789-833

* ``mismatch_parts`` / ``mismatch_stats``  GCR:712-771 (the abs/rel diff,
  mismatch mask, count, maxima over the mismatches and first index, factored
  out of ``compare_tensors`` so tests can merge them over chunks)

and the policy helpers of ``runner/correctness_policy.py`` (CP:146-179) that
those functions call.  The arithmetic is torch's own (torch 2.10 CPU), which
is what the reference runs (``torch.isclose``, ``torch.quantile``,
``Tensor.max``, ``torch.argmax``; torch is the reference's unpinned
third-party dependency, requirements.txt:1-2).

How each part is pinned:

* every function restating GCR/CP: against fixtures that the reference itself
  wrote in this container (``tests/golden/make_golden.py``; 51 verdict cases
  covering every dtype family, strided and 0-d inputs, empty tensors, shape and
  dtype mismatches, NaN/Inf tables, sampling above 1,000,000 elements, all
  three policies, nested outputs, and the float8 error), compared key by key
  in ``tests/test_oracle_golden.py``; ``mismatch_stats`` and the finite-pattern
  count against the same fixtures in ``tests/test_oracle_properties.py``;
* ``extension_record`` (the builder-defined fields that the reference does
  not have: max abs/rel error over all elements with argmax, a 16-bucket
  ULP-distance histogram, fp64 sums for relative-L2 and full-tensor cosine,
  NaN/Inf class counts and finite-pattern violation counts): the argmax is
  ``torch.argmax`` itself; the ULP distance against an independent method
  (rank distance in the sorted list of all finite values, over every code of
  fp16, bf16 and both fp8 formats; nextafter stepping for fp32); the sums and
  derived ratios against closed forms (identical inputs, g = -r, g = 2r, zero
  vectors) -- all in ``tests/test_oracle_properties.py``.
"""

from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Tuple

import torch

MAX_SAMPLES = 1_000_000

# GCR:39-44
TOLERANCE_POLICY = {
    "fp32": {"rtol": 1.3e-6, "atol": 1e-5},
    "fp16": {"rtol": 0.001, "atol": 0.0001},
    "bf16": {"rtol": 0.016, "atol": 1e-3},
    "int8": {"max_abs_diff": 1},
}

_FP8_DTYPES = tuple(
    getattr(torch, name) for name in ("float8_e4m3fn", "float8_e5m2") if hasattr(torch, name)
)


# ---------------------------------------------------------------- CP:146-179
def policy_name(correctness_policy: Optional[Dict[str, Any]]) -> str:
    if not correctness_policy:
        return "strict"
    return str(correctness_policy.get("policy") or "strict")


def thresholds_for_dtype(correctness_policy, dtype_name_: str) -> Dict[str, float]:
    if not correctness_policy:
        return {}
    thresholds = correctness_policy.get("thresholds") or {}
    upper = str(dtype_name_).upper()
    row = thresholds.get(upper) or thresholds.get(upper.lower()) or thresholds.get(upper.capitalize())
    if row is not None:
        return dict(row)
    return dict(thresholds.get("FP32") or {})


# ---------------------------------------------------------------- GCR helpers
def dtype_name(tensor: torch.Tensor) -> str:
    """GCR:212-223."""
    if tensor.dtype == torch.float32:
        return "FP32"
    if tensor.dtype == torch.float16:
        return "FP16"
    if tensor.dtype == torch.bfloat16:
        return "BF16"
    if tensor.dtype in (torch.int8, torch.uint8):
        return "INT8"
    return str(tensor.dtype).replace("torch.", "").upper()


def dtype_policy(tensor: torch.Tensor, tolerance_policy: Optional[Dict[str, Any]] = None):
    """GCR:305-328."""
    name = dtype_name(tensor)
    if tolerance_policy:
        configured = tolerance_policy.get(name) or tolerance_policy.get(name.lower()) or tolerance_policy.get(name.upper())
        if configured is not None:
            return configured
    if tensor.dtype in (torch.int8, torch.uint8):
        return TOLERANCE_POLICY["int8"]
    if tensor.dtype == torch.float32:
        return TOLERANCE_POLICY["fp32"]
    if tensor.dtype == torch.float16:
        return TOLERANCE_POLICY["fp16"]
    if tensor.dtype == torch.bfloat16:
        return TOLERANCE_POLICY["bf16"]
    if torch.is_floating_point(tensor):
        return TOLERANCE_POLICY["fp32"]
    return {"max_abs_diff": 0}


def format_number(value: Any) -> str:
    """GCR:331-335."""
    try:
        return f"{float(value):.6g}"
    except (TypeError, ValueError):
        return str(value)


def sample_flat_values(values: torch.Tensor, max_samples: int = MAX_SAMPLES) -> torch.Tensor:
    """GCR:338-348: all elements, or the strided gather idx_i = i*(n-1)//(m-1)."""
    values = values.reshape(-1)
    numel = values.numel()
    if numel <= max_samples:
        return values
    idx = torch.arange(max_samples, dtype=torch.int64) * (numel - 1) // (max_samples - 1)
    return values[idx]


def cosine_similarity_value(generated, reference, max_samples: int = MAX_SAMPLES) -> Optional[float]:
    """GCR:351-371 before the final ``round(., 4)``: the clamped fp64 cosine of the
    strided samples, or the exact 1.0 / 0.0 of the zero-norm conventions."""
    if generated.numel() == 0 or not torch.is_floating_point(reference):
        return None
    g = sample_flat_values(generated, max_samples).to(torch.float64)
    r = sample_flat_values(reference, max_samples).to(torch.float64)
    gn = torch.linalg.vector_norm(g)
    rn = torch.linalg.vector_norm(r)
    g_zero = bool(gn.item() == 0.0)
    r_zero = bool(rn.item() == 0.0)
    if g_zero and r_zero:
        return 1.0
    if g_zero or r_zero:
        return 0.0
    cos = torch.clamp(torch.dot(g, r) / (gn * rn), -1.0, 1.0)
    return float(cos.item())


def cosine_similarity_meta(generated, reference, max_samples: int = MAX_SAMPLES) -> Optional[float]:
    """GCR:351-372 (the conventions' exact 1.0 / 0.0 are unchanged by the rounding)."""
    v = cosine_similarity_value(generated, reference, max_samples)
    return None if v is None else round(v, 4)


def norm_ratio_value(generated, reference, max_samples: int = MAX_SAMPLES) -> Optional[float]:
    """GCR:375-392 before the final ``round(., 4)``: ||g|| / ||r|| of the strided
    samples in fp64, or the exact 1.0 / 0.0 / inf of the zero-norm conventions."""
    if generated.numel() == 0 or not torch.is_floating_point(reference):
        return None
    g = sample_flat_values(generated, max_samples).to(torch.float64)
    r = sample_flat_values(reference, max_samples).to(torch.float64)
    gn = torch.linalg.vector_norm(g)
    rn = torch.linalg.vector_norm(r)
    g_zero = bool(gn.item() == 0.0)
    r_zero = bool(rn.item() == 0.0)
    if g_zero and r_zero:
        return 1.0
    if g_zero:
        return 0.0
    if r_zero:
        return float("inf")
    return float((gn / rn).item())


def norm_ratio_meta(generated, reference, max_samples: int = MAX_SAMPLES) -> Optional[float]:
    """GCR:375-393."""
    v = norm_ratio_value(generated, reference, max_samples)
    return None if v is None else round(v, 4)


def p99_meta(values, max_samples: int = MAX_SAMPLES) -> Optional[float]:
    """GCR:396-402."""
    if values.numel() == 0:
        return None
    values = sample_flat_values(values, max_samples).to(torch.float32)
    return float(torch.quantile(values, 0.99).item())


def mean_meta(values, max_samples: int = MAX_SAMPLES) -> Optional[float]:
    """GCR:405-411."""
    if values.numel() == 0:
        return None
    values = sample_flat_values(values, max_samples).to(torch.float32)
    return float(values.mean().item())


def finite_pattern_pass(generated, reference, fp8_decode: bool = False) -> bool:
    """GCR:414-437.

    torch-CPU has no ``isfinite`` for float8 tensors, so the reference raises
    NotImplementedError there; ``fp8_decode=True`` is the declared extension
    that evaluates the same rule on the float32-decoded values instead.
    """
    if not torch.is_floating_point(reference):
        return True
    if fp8_decode and reference.dtype in _FP8_DTYPES:
        generated = generated.to(torch.float32)
        reference = reference.to(torch.float32)
    gf = torch.isfinite(generated)
    rf = torch.isfinite(reference)
    if not torch.equal(gf, rf):
        return False
    nonfinite = ~rf
    if not bool(nonfinite.any().item()):
        return True
    g = generated[nonfinite]
    r = reference[nonfinite]
    same_nan = torch.isnan(g) & torch.isnan(r)
    same_inf = torch.isinf(g) & torch.isinf(r) & (g == r)
    return bool((same_nan | same_inf).all().item())


def threshold_pass(value, threshold) -> bool:
    """GCR:440-449."""
    if value is None or threshold is None:
        return False
    v, t = float(value), float(threshold)
    if not math.isfinite(v) or not math.isfinite(t):
        return False
    return v <= t


def cosine_pass(value, threshold) -> bool:
    """GCR:452-461."""
    if value is None or threshold is None:
        return False
    v, t = float(value), float(threshold)
    if not math.isfinite(v) or not math.isfinite(t):
        return False
    return v >= t


def range_pass(value, lo, hi) -> bool:
    """GCR:464-478."""
    if value is None or lo is None or hi is None:
        return False
    v, a, b = float(value), float(lo), float(hi)
    if not (math.isfinite(v) and math.isfinite(a) and math.isfinite(b)):
        return False
    return a <= v <= b


def near_zero_abs_policy_pass(reference, abs_diff, mismatch_mask, meta, correctness_policy,
                              max_samples: int = MAX_SAMPLES) -> bool:
    """GCR:481-548 (diagnostic: the verdict never reads the result)."""
    meta["near_zero_abs_pass"] = False
    if not torch.is_floating_point(reference):
        return False
    if reference.dtype not in (torch.float16, torch.bfloat16):
        return False
    if policy_name(correctness_policy) != "tolerant":
        return False
    thresholds = thresholds_for_dtype(correctness_policy, dtype_name(reference))
    near_zero_abs = thresholds.get("near_zero_abs")
    max_bad_abs = thresholds.get("max_near_zero_bad_abs")
    if near_zero_abs is None or max_bad_abs is None:
        return False
    ref_abs = reference.to(torch.float32).abs()
    near = ref_abs <= float(near_zero_abs)
    far = ~near
    near_count = int(near.sum().item())
    far_count = int(far.sum().item())
    numel = int(reference.numel())
    far_mismatch = int((mismatch_mask & far).sum().item())
    meta["near_zero_abs"] = float(near_zero_abs)
    meta["near_zero_rate"] = round((near_count / numel) if numel else 0.0, 4)
    meta["far_mismatch_rate"] = round((far_mismatch / far_count) if far_count else 0.0, 4)
    if near_count == 0:
        meta["near_zero_p99_abs"] = None
        meta["near_zero_mean_abs"] = None
        meta["near_zero_bad_rate"] = 0.0
        return False
    near_abs = abs_diff[near]
    bad = int((near_abs > float(max_bad_abs)).sum().item())
    meta["near_zero_p99_abs"] = p99_meta(near_abs, max_samples)
    meta["near_zero_mean_abs"] = mean_meta(near_abs, max_samples)
    meta["near_zero_bad_rate"] = round(bad / near_count, 4)
    meta["near_zero_abs_pass"] = bool(
        meta.get("finite_pass")
        and far_mismatch == 0
        and threshold_pass(meta.get("near_zero_p99_abs"), thresholds.get("max_near_zero_p99_abs"))
        and threshold_pass(meta.get("near_zero_mean_abs"), thresholds.get("max_near_zero_mean_abs"))
        and threshold_pass(meta.get("near_zero_bad_rate"), thresholds.get("max_near_zero_bad_rate"))
    )
    return bool(meta["near_zero_abs_pass"])


def evaluate_tensor_policy(reference, meta, correctness_policy) -> bool:
    """GCR:551-606."""
    if meta.get("allclose_pass"):
        return True
    if not torch.is_floating_point(reference):
        return False
    name = policy_name(correctness_policy)
    if name not in ("cosine", "tolerant"):
        return False
    th = thresholds_for_dtype(correctness_policy, dtype_name(reference))
    cosine_ok = cosine_pass(meta.get("cosine_similarity"), th.get("min_cosine"))
    mismatch_ok = threshold_pass(meta.get("mismatch_rate"), th.get("max_mismatch_rate"))
    p99_abs_ok = threshold_pass(meta.get("p99_abs"), th.get("max_p99_abs"))
    p99_rel_ok = threshold_pass(meta.get("p99_rel"), th.get("max_p99_rel"))
    finite_ok = bool(meta.get("finite_pass"))
    normal = bool(finite_ok and cosine_ok and mismatch_ok and (p99_abs_ok or p99_rel_ok))
    if name == "cosine":
        ratio_ok = range_pass(meta.get("norm_ratio"), th.get("min_norm_ratio"), th.get("max_norm_ratio"))
        cos_metric = bool(finite_ok and cosine_ok and ratio_ok)
        meta["normal_metric_pass"] = normal
        meta["norm_ratio_pass"] = ratio_ok
        meta["cosine_metric_pass"] = cos_metric
        return bool(normal or cos_metric)
    meta["normal_metric_pass"] = normal
    return normal


def mismatch_parts(generated: torch.Tensor, reference: torch.Tensor, tolerance_policy=None):
    """GCR:712-730: (abs_diff, rel_diff, mismatch mask, tolerance dict) under the dtype policy of GCR:305-328.
    Integer mode: int32 casts (int64 wraps) and |g - r| > max_abs_diff; float mode: float32 casts and
    ~torch.isclose(r, g, rtol, atol); rel_diff = abs_diff / (|r| + 1e-12) in float32."""
    policy = dtype_policy(reference, tolerance_policy)
    if "max_abs_diff" in policy:
        g = generated.to(torch.int32)
        r = reference.to(torch.int32)
        abs_diff = (g - r).abs()
        mismatch = abs_diff > int(policy["max_abs_diff"])
        tolerance = {"max_abs_diff": int(policy["max_abs_diff"])}
    else:
        g = generated.to(torch.float32)
        r = reference.to(torch.float32)
        abs_diff = (g - r).abs()
        rtol = float(policy["rtol"])
        atol = float(policy["atol"])
        mismatch = ~torch.isclose(r, g, rtol=rtol, atol=atol)
        tolerance = {"rtol": rtol, "atol": atol}
    rel_diff = abs_diff.to(torch.float32) / (reference.to(torch.float32).abs() + 1e-12)
    return abs_diff, rel_diff, mismatch, tolerance


def mismatch_stats(generated: torch.Tensor, reference: torch.Tensor, tolerance_policy=None) -> Dict[str, Any]:
    """GCR:731-771 without the sampling: the mismatch count, the row-major flat index of the first mismatch
    (-1 if none), and the NaN-propagating max of abs_diff / rel_diff over the mismatches (None if none)."""
    g = generated.detach().cpu().reshape(-1)
    r = reference.detach().cpu().reshape(-1)
    abs_diff, rel_diff, mismatch, _ = mismatch_parts(g, r, tolerance_policy)
    count = int(mismatch.sum().item())
    out = {"mismatch_count": count, "first_mismatch_index": _first_true(mismatch),
           "mismatch_max_abs": None, "mismatch_max_rel": None}
    if count:
        out["mismatch_max_abs"] = float(abs_diff[mismatch].max().item())
        out["mismatch_max_rel"] = float(rel_diff[mismatch].max().item())
    return out


def compare_tensors(
    generated: torch.Tensor,
    reference: torch.Tensor,
    path: str,
    tolerance_policy: Optional[Dict[str, Any]] = None,
    correctness_policy: Optional[Dict[str, Any]] = None,
    fp8_decode: bool = False,
    max_samples: int = MAX_SAMPLES,
) -> Tuple[bool, List[str], Dict[str, Any]]:
    """GCR:672-786, on CPU tensors (``max_samples`` is the reference's fixed 1,000,000 by default)."""
    generated = generated.detach().cpu()
    reference = reference.detach().cpu()
    active = policy_name(correctness_policy)
    meta: Dict[str, Any] = {"path": path, "correctness_policy": active}
    for label, bad, text in (
        ("shape", generated.shape != reference.shape,
         f"{path}.shape mismatch: expected {tuple(reference.shape)}, got {tuple(generated.shape)}"),
        ("dtype", generated.dtype != reference.dtype,
         f"{path}.dtype mismatch: expected {reference.dtype}, got {generated.dtype}"),
    ):
        if bad:
            meta["allclose_pass"] = False
            meta["metric_pass"] = False
            meta["policy_pass"] = False
            meta["mismatch_rate"] = 1.0
            meta["p99_abs"] = None
            meta["p99_rel"] = None
            return False, [text], meta
    meta["cosine_similarity"] = cosine_similarity_meta(generated, reference, max_samples)
    meta["norm_ratio"] = norm_ratio_meta(generated, reference, max_samples)

    abs_diff, rel_diff, mismatch, tolerance = mismatch_parts(generated, reference, tolerance_policy)
    count = int(mismatch.sum().item())
    numel = int(reference.numel())
    allclose = bool(count == 0)
    meta["mismatch_rate"] = round((count / numel) if numel else 0.0, 4)
    meta["p99_abs"] = p99_meta(abs_diff, max_samples)
    meta["p99_rel"] = p99_meta(rel_diff, max_samples)
    meta["allclose_pass"] = allclose
    meta["normal_metric_pass"] = False
    meta["cosine_metric_pass"] = False
    meta["norm_ratio_pass"] = False
    if torch.is_floating_point(reference):
        meta["finite_pass"] = finite_pattern_pass(generated, reference, fp8_decode=fp8_decode)
        near_zero_abs_policy_pass(reference, abs_diff, mismatch, meta, correctness_policy, max_samples)
    meta["metric_pass"] = False if allclose else evaluate_tensor_policy(reference, meta, correctness_policy)
    meta["policy_pass"] = bool(allclose or meta["metric_pass"])
    if generated.numel() == 0 or count == 0:
        return True, [], meta

    max_abs = abs_diff[mismatch].max().item()
    max_rel = rel_diff[mismatch].max().item()
    meta["max_abs"] = float(max_abs)
    meta["max_rel"] = float(max_rel)
    if mismatch.dim() == 0:
        first = "()"
    else:
        nz = torch.nonzero(mismatch, as_tuple=False)
        first = tuple(int(v) for v in nz[0].tolist()) if nz.numel() > 0 else None
    meta["first_mismatch_index"] = first
    detail = (
        f"{path}: policy={active}, policy_pass={meta['policy_pass']}, "
        f"allclose_pass={meta['allclose_pass']}, metric_pass={meta['metric_pass']}, "
        f"normal_metric_pass={meta.get('normal_metric_pass')}, "
        f"cosine_metric_pass={meta.get('cosine_metric_pass')}, "
        f"near_zero_abs_pass={meta.get('near_zero_abs_pass')}, "
        f"{count}/{numel} elements mismatched, "
        f"max_abs={format_number(max_abs)}, max_rel={format_number(max_rel)}, "
        f"p99_abs={format_number(meta['p99_abs'])}, p99_rel={format_number(meta['p99_rel'])}, "
        f"cosine_similarity={format_number(meta.get('cosine_similarity'))}, "
        f"norm_ratio={format_number(meta.get('norm_ratio'))}, "
        f"first_mismatch_index={first}, tolerance={tolerance}"
    )
    ok = bool(meta["policy_pass"])
    return ok, ([] if ok else [detail]), meta


def compare_outputs(generated, reference, path="output", tolerance_policy=None, correctness_policy=None,
                    fp8_decode: bool = False, max_samples: int = MAX_SAMPLES):
    """GCR:789-833."""
    if isinstance(generated, torch.Tensor) and isinstance(reference, torch.Tensor):
        ok, details, meta = compare_tensors(generated, reference, path, tolerance_policy, correctness_policy,
                                            fp8_decode=fp8_decode, max_samples=max_samples)
        return ok, details, [meta]
    if isinstance(generated, (list, tuple)) and isinstance(reference, (list, tuple)):
        if len(generated) != len(reference):
            return False, [f"{path} length mismatch: expected {len(reference)}, got {len(generated)}"], []
        all_ok, details, metas = True, [], []
        for i, (g, r) in enumerate(zip(generated, reference)):
            ok, d, m = compare_outputs(g, r, f"{path}[{i}]", tolerance_policy, correctness_policy,
                                       fp8_decode=fp8_decode, max_samples=max_samples)
            all_ok = all_ok and ok
            details.extend(d)
            metas.extend(m)
        return all_ok, details, metas
    if generated == reference:
        return True, [], []
    return False, [f"{path} type/value mismatch: expected {type(reference).__name__}, got {type(generated).__name__}"], []


# ------------------------------------------------------- builder extensions
HIST_BUCKETS = 16

_CODE_VIEW = {
    torch.float32: (torch.int32, 32),
    torch.float16: (torch.int16, 16),
    torch.bfloat16: (torch.int16, 16),
    torch.float64: (torch.int64, 64),
}
for _d in _FP8_DTYPES:
    _CODE_VIEW[_d] = (torch.int8, 8)


def _ordered_magnitudes(t: torch.Tensor):
    """(sign, magnitude) of the raw sign-magnitude code of each float element, as int64."""
    view_dtype, width = _CODE_VIEW[t.dtype]
    raw = t.contiguous().view(view_dtype).to(torch.int64)
    if width < 64:
        raw = raw & ((1 << width) - 1)            # unsigned code
        sign = (raw >> (width - 1)) & 1
        mag = raw & ((1 << (width - 1)) - 1)
    else:
        sign = (raw < 0).to(torch.int64)
        mag = raw & 0x7FFFFFFFFFFFFFFF
    return sign, mag


def ulp_bucket(d: torch.Tensor) -> torch.Tensor:
    """Bucket of a non-negative int64 distance: 0 for d == 0, else min(bit_length(d), 15)."""
    b = torch.zeros_like(d)
    for k in range(1, HIST_BUCKETS):
        b = torch.where(d >= (1 << (k - 1)), torch.full_like(d, k), b)
    return b


def ulp_distance_buckets(generated: torch.Tensor, reference: torch.Tensor):
    """Per-element ULP bucket and NaN-pair mask (declared extension).

    Float dtypes: codes are mapped to o(u) = sign ? -mag : mag (so +0 and -0
    coincide), d = |o(g) - o(r)|; a pair with a NaN on either side is a NaN
    pair and gets no bucket.  Integer and bool dtypes: d = |g - r| on the
    integer values.  Distances of 2**14 or more all land in bucket 15, so the
    overflow of d itself never matters.
    """
    g = generated.reshape(-1)
    r = reference.reshape(-1)
    if torch.is_floating_point(reference):
        gs, gm = _ordered_magnitudes(g)
        rs, rm = _ordered_magnitudes(r)
        same = gs == rs
        big = (gm >= (1 << 14)) | (rm >= (1 << 14))
        d_same = (gm - rm).abs()
        d_diff = torch.where(big, torch.full_like(gm, 1 << 14), gm + rm)
        d = torch.where(same, d_same, d_diff)
        nan_pair = torch.isnan(g.to(torch.float32) if g.dtype in _FP8_DTYPES else g) | torch.isnan(
            r.to(torch.float32) if r.dtype in _FP8_DTYPES else r)
    else:
        gi = g.to(torch.int64)
        ri = r.to(torch.int64)
        big = (gi.abs() >= (1 << 14)) | (ri.abs() >= (1 << 14))
        d = torch.where(big & ((gi < 0) != (ri < 0)), torch.full_like(gi, 1 << 14), (gi - ri).abs())
        # same-sign int64 differences cannot overflow; a wrapped value is still >= 2**14 when big
        d = torch.where(d < 0, torch.full_like(d, 1 << 14), d)
        nan_pair = torch.zeros_like(gi, dtype=torch.bool)
    return ulp_bucket(d), nan_pair


def _first_true(mask: torch.Tensor) -> int:
    nz = torch.nonzero(mask.reshape(-1), as_tuple=False)
    return int(nz[0, 0]) if nz.numel() else -1


def extension_record(generated: torch.Tensor, reference: torch.Tensor,
                     tolerance_policy: Optional[Dict[str, Any]] = None) -> Dict[str, Any]:
    """Builder-defined verdict fields over ALL elements (no sampling).

    * ``max_abs``/``max_abs_index``: the reference's abs_diff tensor (GCR:716-724)
      reduced with ``torch.argmax`` over the row-major flattening: NaN counts as
      the maximum and ties go to the lowest index.  Likewise ``max_rel`` over
      rel_diff (GCR:730).  Integer mode keeps torch's int32 abs_diff (which
      wraps: |INT_MIN| stays negative).
    * ``ulp_hist``/``nan_pairs``: see ``ulp_distance_buckets``;
      ``sum(ulp_hist) + nan_pairs == numel``; ``equal_count == ulp_hist[0]``.
    * ``sum_gg``, ``sum_rr``, ``sum_gr``, ``sum_dd``: fp64 sums of g*g, r*r, g*r
      and (g-r)^2 with g, r the original values converted to float64.
      ``rel_l2 = sqrt(sum_dd)/sqrt(sum_rr)`` and ``cosine = sum_gr/(sqrt(sum_gg)
      sqrt(sum_rr))`` clamped to [-1, 1] with the zero conventions of GCR:364-369.
    * NaN/+Inf/-Inf counts of each side, and the count and first index of the
      positions that break the finite-pattern rule of GCR:414-437.
    """
    g = generated.detach().cpu().reshape(-1)
    r = reference.detach().cpu().reshape(-1)
    n = int(r.numel())
    policy = dtype_policy(reference, tolerance_policy)
    if "max_abs_diff" in policy:
        abs_diff = (g.to(torch.int32) - r.to(torch.int32)).abs()
    else:
        abs_diff = (g.to(torch.float32) - r.to(torch.float32)).abs()
    rel_diff = abs_diff.to(torch.float32) / (r.to(torch.float32).abs() + 1e-12)
    rec: Dict[str, Any] = {"numel": n}
    if n:
        ia = int(torch.argmax(abs_diff))
        ir = int(torch.argmax(rel_diff))
        rec["max_abs"] = float(abs_diff[ia].item())
        rec["max_abs_index"] = ia
        rec["max_rel"] = float(rel_diff[ir].item())
        rec["max_rel_index"] = ir
    else:
        rec.update(max_abs=None, max_abs_index=-1, max_rel=None, max_rel_index=-1)
    buckets, nan_pair = ulp_distance_buckets(g, r)
    hist = torch.bincount(buckets[~nan_pair], minlength=HIST_BUCKETS)
    rec["ulp_hist"] = [int(v) for v in hist.tolist()]
    rec["nan_pairs"] = int(nan_pair.sum().item())
    rec["equal_count"] = rec["ulp_hist"][0]
    g64 = g.to(torch.float64)
    r64 = r.to(torch.float64)
    d64 = g64 - r64
    sums = {
        "sum_gg": float((g64 * g64).sum().item()),
        "sum_rr": float((r64 * r64).sum().item()),
        "sum_gr": float((g64 * r64).sum().item()),
        "sum_dd": float((d64 * d64).sum().item()),
    }
    rec.update(sums)
    rec["rel_l2"] = rel_l2_from_sums(sums["sum_dd"], sums["sum_rr"])
    rec["cosine"] = cosine_from_sums(sums["sum_gr"], sums["sum_gg"], sums["sum_rr"])
    if torch.is_floating_point(reference):
        gf = g.to(torch.float32) if g.dtype in _FP8_DTYPES else g
        rf = r.to(torch.float32) if r.dtype in _FP8_DTYPES else r
        for side, t in (("gen", gf), ("ref", rf)):
            rec[f"nan_{side}"] = int(torch.isnan(t).sum().item())
            rec[f"posinf_{side}"] = int((t == float("inf")).sum().item())
            rec[f"neginf_{side}"] = int((t == float("-inf")).sum().item())
        fin_g = torch.isfinite(gf)
        fin_r = torch.isfinite(rf)
        ok = (fin_g & fin_r) | (torch.isnan(gf) & torch.isnan(rf)) | (torch.isinf(gf) & torch.isinf(rf) & (gf == rf))
        viol = ~ok
        rec["finite_violations"] = int(viol.sum().item())
        rec["first_finite_violation"] = _first_true(viol)
    else:
        for side in ("gen", "ref"):
            rec[f"nan_{side}"] = rec[f"posinf_{side}"] = rec[f"neginf_{side}"] = 0
        rec["finite_violations"] = 0
        rec["first_finite_violation"] = -1
    return rec


def rel_l2_from_sums(sum_dd: float, sum_rr: float) -> float:
    """||g-r|| / ||r||; 0 when both are zero, inf when only ||r|| is zero."""
    dn, rn = math.sqrt(sum_dd), math.sqrt(sum_rr)
    if rn == 0.0:
        return 0.0 if dn == 0.0 else float("inf")
    return dn / rn


def cosine_from_sums(sum_gr: float, sum_gg: float, sum_rr: float) -> float:
    """Cosine from fp64 sums with the zero conventions of GCR:364-371 (no rounding)."""
    gn, rn = math.sqrt(sum_gg), math.sqrt(sum_rr)
    if gn == 0.0 and rn == 0.0:
        return 1.0
    if gn == 0.0 or rn == 0.0:
        return 0.0
    c = sum_gr / (gn * rn)
    if math.isnan(c):
        return c
    return max(-1.0, min(1.0, c))
