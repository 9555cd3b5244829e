"""Per-operator correctness policy: which fallback rule applies when allclose fails.

Mirrors the public surface of KernelVerse ``runner/correctness_policy.py``
(CP:1-179) so that callers that import these names keep working unchanged:
the three policy names, the category defaults, the per-dtype threshold tables
and the helper predicates.  Everything here is host-side dictionary logic; the
data-parallel part of the verdict lives in ``kernelverse_amd.verdict`` and the
HIP library.
"""

from __future__ import annotations

from copy import deepcopy
from typing import Any, Dict, Optional

POLICY_STRICT = "strict"
POLICY_TOLERANT = "tolerant"
POLICY_COSINE = "cosine"

# Category -> default policy (CP:14-28).
CATEGORY_DEFAULT_POLICIES: Dict[str, str] = {
    "activation": POLICY_STRICT,
    "attention": POLICY_COSINE,
    "convolution": POLICY_TOLERANT,
    "gemm": POLICY_TOLERANT,
    "kv_cache": POLICY_STRICT,
    "logits_sampling": POLICY_TOLERANT,
    "moe": POLICY_TOLERANT,
    "normalization": POLICY_TOLERANT,
    "positional_embedding": POLICY_COSINE,
    "quantization": POLICY_STRICT,
    "reduction": POLICY_TOLERANT,
    "state_space": POLICY_COSINE,
    "tensor_ops": POLICY_STRICT,
}

# Metric thresholds of the tolerant policy, per dtype name (CP:31-60).
_NEAR_ZERO_16BIT = {
    "near_zero_abs": 0.25,
    "max_near_zero_p99_abs": 1.0,
    "max_near_zero_mean_abs": 0.05,
    "max_near_zero_bad_abs": 2.0,
    "max_near_zero_bad_rate": 0.01,
}
TOLERANT_THRESHOLDS: Dict[str, Dict[str, float]] = {
    "FP32": {"min_cosine": 0.9990, "max_mismatch_rate": 0.01, "max_p99_abs": 1e-4, "max_p99_rel": 1e-4},
    "FP16": {"min_cosine": 0.9900, "max_mismatch_rate": 0.02, "max_p99_abs": 0.25, "max_p99_rel": 0.03,
             **_NEAR_ZERO_16BIT},
    "BF16": {"min_cosine": 0.9900, "max_mismatch_rate": 0.03, "max_p99_abs": 0.5, "max_p99_rel": 0.05,
             **_NEAR_ZERO_16BIT},
}


def _cosine_row(dtype_name: str, min_cosine: float, min_ratio: float, max_ratio: float) -> Dict[str, float]:
    tolerant = TOLERANT_THRESHOLDS[dtype_name]
    row = {"min_cosine": min_cosine}
    for key in ("max_mismatch_rate", "max_p99_abs", "max_p99_rel"):
        row[key] = tolerant[key]
    row["min_norm_ratio"] = min_ratio
    row["max_norm_ratio"] = max_ratio
    return row


# Metric thresholds of the cosine policy (CP:63-88): the tolerant rate/p99
# limits plus a cosine floor and a norm-ratio window.
COSINE_THRESHOLDS: Dict[str, Dict[str, float]] = {
    "FP32": _cosine_row("FP32", 0.995, 0.98, 1.02),
    "FP16": _cosine_row("FP16", 0.99, 0.80, 1.25),
    "BF16": _cosine_row("BF16", 0.99, 0.75, 1.35),
}

DEFAULT_THRESHOLDS_BY_POLICY = {
    POLICY_TOLERANT: TOLERANT_THRESHOLDS,
    POLICY_COSINE: COSINE_THRESHOLDS,
}


def _default_policy_name(category: str, op_name: str) -> str:
    """Category default with the reduction-family exceptions (CP:97-103)."""
    if category == "reduction":
        if op_name in ("argmax", "max", "max_reduce"):
            return POLICY_STRICT
        if op_name in ("cumsum", "sum_reduce"):
            return POLICY_COSINE
    return CATEGORY_DEFAULT_POLICIES.get(category, POLICY_STRICT)


def _merge_thresholds(base_thresholds: Dict[str, Dict[str, float]], override_thresholds: Any) -> Dict[str, Dict[str, float]]:
    """Per-dtype shallow merge of config ``thresholds`` over a copy of the defaults (CP:106-122).

    Dtype keys of the override are upper-cased; entries that are not dicts are skipped.
    """
    merged = deepcopy(base_thresholds)
    if not isinstance(override_thresholds, dict):
        return merged
    for raw_name, overrides in override_thresholds.items():
        if not isinstance(overrides, dict):
            continue
        name = str(raw_name).upper()
        row = dict(merged.get(name, {}))
        row.update(overrides)
        merged[name] = row
    return merged


def resolve_correctness_policy(operator_spec: Dict[str, Any]) -> Dict[str, Any]:
    """Effective policy of one operator spec (CP:125-143).

    ``config.policy`` wins over the category default; the threshold table of
    the chosen policy is merged with ``config.thresholds``.
    """
    config = operator_spec.get("config") or {}
    category = str(operator_spec.get("category") or "")
    op_name = str(operator_spec.get("op_name") or "")
    configured = config.get("policy")
    name = str(configured or _default_policy_name(category, op_name))
    thresholds = _merge_thresholds(DEFAULT_THRESHOLDS_BY_POLICY.get(name, {}), config.get("thresholds"))
    return {
        "policy": name,
        "category": category,
        "source": "config" if configured is not None else "category_default",
        "thresholds": thresholds,
    }


def policy_name(correctness_policy: Optional[Dict[str, Any]]) -> str:
    """Policy name, ``strict`` when absent or empty (CP:146-149)."""
    if not correctness_policy:
        return POLICY_STRICT
    return str(correctness_policy.get("policy") or POLICY_STRICT)


def is_tolerant_policy(correctness_policy: Optional[Dict[str, Any]]) -> bool:
    return policy_name(correctness_policy) == POLICY_TOLERANT


def is_cosine_policy(correctness_policy: Optional[Dict[str, Any]]) -> bool:
    return policy_name(correctness_policy) == POLICY_COSINE


def is_metric_policy(correctness_policy: Optional[Dict[str, Any]]) -> bool:
    return policy_name(correctness_policy) in (POLICY_TOLERANT, POLICY_COSINE)


def thresholds_for_dtype(correctness_policy: Optional[Dict[str, Any]], dtype_name: str) -> Dict[str, float]:
    """Threshold row for a dtype name; upper, lower, then capitalised key, else the FP32 row (CP:164-179)."""
    if not correctness_policy:
        return {}
    table = correctness_policy.get("thresholds") or {}
    upper = str(dtype_name).upper()
    row = table.get(upper) or table.get(upper.lower()) or table.get(upper.capitalize())
    if row is not None:
        return dict(row)
    return dict(table.get("FP32") or {})
