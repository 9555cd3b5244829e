"""Pins the oracle's own functions where the reference fixtures do not reach.

* ULP distance (declared extension): checked against an independent method,
  the distance between the two values' ranks in the sorted list of all
  finite values of the format (+0 and -0 share a rank), over every code of
  fp16, bf16 and both fp8 formats, and against nextafter stepping for fp32.
* Extension record closed forms: identical inputs, g = -r, g = 2r, NaN-pair
  accounting, integer distances.
* mismatch_stats: against the mismatch rate, maxima and first index that the
  reference itself returned for every fixture case with mismatches.
* finite-pattern counts: zero exactly when the reference said finite_pass.
"""

import math

import numpy as np
import pytest
import torch

from golden_io import load_cases
from oracle import torch_verdict as tv

FLOAT_FORMATS = [torch.float16, torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2]
CODE_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float8_e4m3fn: torch.uint8,
             torch.float8_e5m2: torch.uint8}


def _bucket(d: np.ndarray) -> np.ndarray:
    """0 for 0, else min(bit_length(d), 15), by repeated halving (no shifts shared with the oracle)."""
    out = np.zeros_like(d)
    v = d.copy()
    k = np.zeros_like(d)
    while (v > 0).any():
        k += (v > 0)
        v //= 2
    out[:] = np.minimum(k, 15)
    return out


def _all_codes(dtype):
    bits = 16 if CODE_VIEW[dtype] == torch.int16 else 8
    codes = torch.arange(0, 1 << bits, dtype=torch.int64)
    if bits == 16:
        codes = torch.where(codes >= 1 << 15, codes - (1 << 16), codes).to(torch.int16)
    else:
        codes = codes.to(torch.uint8)
    return codes.view(dtype)


@pytest.mark.parametrize("dtype", FLOAT_FORMATS, ids=str)
def test_ulp_distance_is_rank_distance(dtype):
    vals = _all_codes(dtype)
    v32 = vals.to(torch.float32).numpy()
    finite = np.isfinite(v32)
    order = np.unique(v32[finite])          # sorted distinct finite values; +0 and -0 are one value
    rank = np.full(v32.shape, -1, dtype=np.int64)
    rank[finite] = np.searchsorted(order, v32[finite])
    rng = np.random.default_rng(7)
    fin_idx = np.nonzero(finite)[0]
    a = rng.choice(fin_idx, size=200_000)
    # near partners (small distances) and far partners (any finite code)
    near = np.clip(a + rng.integers(-40, 41, size=a.size), 0, vals.numel() - 1)
    near = np.where(finite[near], near, a)
    b = np.concatenate([near, rng.choice(fin_idx, size=a.size)])
    a = np.concatenate([a, a])
    g, r = vals[torch.from_numpy(a)], vals[torch.from_numpy(b)]
    got, nan_pair = tv.ulp_distance_buckets(g, r)
    assert not nan_pair.any()
    want = _bucket(np.abs(rank[a] - rank[b]))
    assert np.array_equal(got.numpy(), want)


@pytest.mark.parametrize("dtype", FLOAT_FORMATS, ids=str)
def test_nan_pairs_get_no_bucket(dtype):
    vals = _all_codes(dtype)
    nan = torch.isnan(vals.to(torch.float32))
    g = vals
    r = vals[torch.arange(vals.numel() - 1, -1, -1)]
    _, nan_pair = tv.ulp_distance_buckets(g, r)
    want = nan | nan.flip(0)
    assert torch.equal(nan_pair, want)
    rec = tv.extension_record(g, r)
    assert sum(rec["ulp_hist"]) + rec["nan_pairs"] == vals.numel()


def test_fp32_ulp_distance_by_nextafter_steps():
    rng = np.random.default_rng(11)
    start = torch.from_numpy(rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-40, 39, 4096))
    start[:64] = torch.tensor([0.0, -0.0] * 32)
    steps = torch.from_numpy(rng.integers(0, 20_000, 4096))
    steps[::7] = torch.from_numpy(rng.integers(0, 4, steps[::7].numel()))
    direction = torch.where(torch.from_numpy(rng.random(4096) < 0.5), float("inf"), float("-inf"))
    x = start.clone()
    for k in range(int(steps.max()) + 1):
        move = steps > k
        x = torch.where(move, torch.nextafter(x, direction.to(torch.float32)), x)
    ok = torch.isfinite(x)
    got, nan_pair = tv.ulp_distance_buckets(start[ok], x[ok])
    assert not nan_pair.any()
    # nextafter treats -0 and +0 as one point when stepping through zero, as the distance does
    assert np.array_equal(got.numpy(), _bucket(steps[ok].numpy()))


def test_integer_distances():
    a = torch.tensor([-128, -128, 127, 0, 5], dtype=torch.int8)
    b = torch.tensor([127, -128, -128, 1, 5], dtype=torch.int8)
    got, nan_pair = tv.ulp_distance_buckets(a, b)
    assert not nan_pair.any()
    assert got.tolist() == _bucket(np.array([255, 0, 255, 1, 0])).tolist()


def test_extension_closed_forms():
    rng = np.random.default_rng(3)
    r = torch.from_numpy(rng.standard_normal(10_000))
    same = tv.extension_record(r.clone(), r)
    assert same["ulp_hist"][0] == r.numel() and same["nan_pairs"] == 0
    assert same["sum_gg"] == same["sum_rr"] == same["sum_gr"] and same["sum_dd"] == 0.0
    assert same["rel_l2"] == 0.0 and same["cosine"] == 1.0
    assert same["max_abs"] == 0.0 and same["max_abs_index"] == 0
    neg = tv.extension_record(-r, r)
    assert neg["cosine"] == -1.0 and math.isclose(neg["rel_l2"], 2.0, rel_tol=1e-12)
    dbl = tv.extension_record(2 * r, r)
    assert math.isclose(dbl["rel_l2"], 1.0, rel_tol=1e-12) and math.isclose(dbl["cosine"], 1.0, rel_tol=1e-12)
    assert dbl["max_abs_index"] == int(torch.argmax(r.abs()))
    zero = tv.extension_record(torch.zeros(5), torch.zeros(5))
    assert zero["cosine"] == 1.0 and zero["rel_l2"] == 0.0
    only_r0 = tv.extension_record(torch.ones(5), torch.zeros(5))
    assert only_r0["cosine"] == 0.0 and only_r0["rel_l2"] == float("inf")


def _single_tensor_cases():
    out = []
    for c in load_cases():
        exp = c["expected"]
        if "raises" in exp or not isinstance(c["generated"], torch.Tensor) or len(exp["metas"]) != 1:
            continue
        meta = exp["metas"][0]
        if "mismatch_rate" not in meta or meta.get("p99_abs", 0) is None and meta["mismatch_rate"] == 1.0:
            continue
        if c["generated"].shape != c["reference"].shape or c["generated"].dtype != c["reference"].dtype:
            continue
        out.append(c)
    return out


SINGLE = _single_tensor_cases()


@pytest.mark.parametrize("case", SINGLE, ids=[c["name"] for c in SINGLE])
def test_mismatch_stats_match_reference(case):
    meta = case["expected"]["metas"][0]
    g, r = case["generated"], case["reference"]
    st = tv.mismatch_stats(g, r, case["tolerance_policy"])
    n = r.numel()
    assert (round(st["mismatch_count"] / n, 4) if n else 0.0) == meta["mismatch_rate"]
    assert (st["mismatch_count"] == 0) == meta["allclose_pass"]
    if st["mismatch_count"]:
        for k, mk in (("mismatch_max_abs", "max_abs"), ("mismatch_max_rel", "max_rel")):
            a, b = st[k], meta[mk]
            assert (math.isnan(a) and math.isnan(b)) or a == b, (k, a, b)
        first = meta["first_mismatch_index"]
        flat = 0 if first == "()" else int(np.ravel_multi_index(first, tuple(r.shape)))
        assert st["first_mismatch_index"] == flat


@pytest.mark.parametrize("case", [c for c in SINGLE if "finite_pass" in c["expected"]["metas"][0]],
                         ids=[c["name"] for c in SINGLE if "finite_pass" in c["expected"]["metas"][0]])
def test_finite_pattern_count_matches_reference(case):
    meta = case["expected"]["metas"][0]
    rec = tv.extension_record(case["generated"], case["reference"], case["tolerance_policy"])
    assert (rec["finite_violations"] == 0) == meta["finite_pass"]
