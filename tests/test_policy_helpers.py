"""The drop-in's policy helpers against the reference's own answers (CPU).

``tests/golden/policy_resolution.json`` was written by the reference itself
(``tests/golden/make_golden.py``): ``resolve_correctness_policy`` (CP:125-143)
and ``_operator_tolerance_policy`` (GCR:886-888) for every operator
``config.json`` it ships plus seven edge specs, ``thresholds_for_dtype`` /
``policy_name`` / ``is_metric_policy`` (CP:146-179) lookups, and
``_correctness_criteria`` (GCR:609-669) for each policy kind.  Threshold
tables keep the reference's key order, which downstream ``evaluation.json``
readers see; the comparisons here are ordered (``same_value`` compares dict
key order).
"""

import json

import pytest

from golden_io import load_policy_fixture, same_value
from kernelverse_amd import correctness_policy as cp
from kernelverse_amd import verdict

FX = load_policy_fixture()


def _spec(entry):
    """The operator spec the reference resolved: the trimmed config plus its tolerances."""
    cfg = entry["config"]
    if isinstance(cfg, dict):
        cfg = dict(cfg)
        if entry.get("has_tolerances"):
            cfg["tolerances"] = entry["tolerance_policy"]
    return {"category": entry["category"], "op_name": entry["op_name"], "config": cfg}


def _ordered(a, b) -> bool:
    return same_value(json.loads(json.dumps(a)), json.loads(json.dumps(b)))


def test_fixture_covers_every_shipped_config():
    assert len(FX["policies"]) == 207
    assert len(FX["criteria"]) == 6
    assert len(FX["thresholds_for_dtype"]) == 42


@pytest.mark.parametrize("entry", FX["policies"], ids=[f"{e['category']}/{e['op_name']}" for e in FX["policies"]])
def test_resolve_correctness_policy(entry):
    got = cp.resolve_correctness_policy(_spec(entry))
    assert _ordered(got, entry["resolved"]), (got, entry["resolved"])


@pytest.mark.parametrize("entry", FX["policies"], ids=[f"{e['category']}/{e['op_name']}" for e in FX["policies"]])
def test_operator_tolerance_policy(entry):
    got = verdict._operator_tolerance_policy(_spec(entry))
    assert _ordered(got, entry["tolerance_policy"]), (got, entry["tolerance_policy"])


def test_threshold_lookups():
    for entry in FX["thresholds_for_dtype"]:
        pol = entry["policy"]
        assert _ordered(cp.thresholds_for_dtype(pol, entry["dtype"]), entry["thresholds"]), entry
        assert cp.policy_name(pol) == entry["name"]
        assert cp.is_metric_policy(pol) == entry["is_metric"]


@pytest.mark.parametrize("entry", FX["criteria"], ids=[f"{e['policy']['policy']}-{e['baseline_compute_mode']}"
                                                        for e in FX["criteria"]])
def test_correctness_criteria(entry):
    got = verdict._correctness_criteria(entry["tolerance_policy"], entry["policy"], entry["baseline_compute_mode"],
                                        entry["random_correctness"], entry["shape_mode"])
    assert _ordered(got, entry["criteria"]), (got, entry["criteria"])


def test_key_order_is_checked():
    """The comparison sees a reordered threshold table (what a sort_keys round trip did)."""
    entry = next(e for e in FX["policies"] if e["resolved"]["policy"] == "tolerant")
    got = cp.resolve_correctness_policy(_spec(entry))
    row = got["thresholds"]["FP16"]
    got["thresholds"]["FP16"] = dict(sorted(row.items()))
    assert list(got["thresholds"]["FP16"]) != list(row)
    assert not _ordered(got, entry["resolved"])
