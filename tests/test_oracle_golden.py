"""The CPU oracle reproduces, case by case, what the reference's own verdict returned."""

import pytest
import torch

from golden_io import diff_meta, load_cases, load_policy_fixture, same_value
from oracle import torch_verdict as tv

CASES = load_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_reference_fixture(case):
    exp = case["expected"]
    kwargs = dict(tolerance_policy=case["tolerance_policy"], correctness_policy=case["correctness_policy"])
    if "raises" in exp:
        with pytest.raises(Exception) as info:
            tv.compare_outputs(case["generated"], case["reference"], **kwargs)
        assert type(info.value).__name__ == exp["raises"]
        assert str(info.value) == exp["message"]
        return
    ok, details, metas = tv.compare_outputs(case["generated"], case["reference"], **kwargs)
    assert ok == exp["ok"]
    assert details == exp["details"]
    assert len(metas) == len(exp["metas"])
    for got, want in zip(metas, exp["metas"]):
        assert not diff_meta(got, want), diff_meta(got, want)


def test_policy_fixture_round_trip():
    fx = load_policy_fixture()
    for entry in fx["thresholds_for_dtype"]:
        assert tv.thresholds_for_dtype(entry["policy"], entry["dtype"]) == entry["thresholds"]
        assert tv.policy_name(entry["policy"]) == entry["name"]
