"""fp32 pairs that differ at (nearly) every element, against the CPU oracle (needs an MI355X).

Such items take the scan's in-place dense path: each lane finishes its pairs
of one sign with a finite, nonzero difference itself (mismatches and rel-argmax
candidates through the exact tests, the others through one-compare bounds),
and queues the rest (NaN/Inf, sign changes, +0 against -0) for the full
per-element treatment.  Every case here mixes the kinds inside items, in
single calls and in batches, and checks every exact field (ULP histogram,
argmax indices, counts), the sums and the metas; the tolerance-boundary cases
put abs_diff within a few ULPs of the allowed bound.
"""

import sys

import numpy as np
import pytest
import torch

from parity_util import meta_problems, record_vs_oracle
from oracle import torch_verdict as tv

pytestmark = pytest.mark.gpu

DEV = "cuda"
N = (1 << 20) + 37  # whole items and a partial last vector


def _problems(rec, g, r, tol):
    probs = record_vs_oracle(rec, g, r, tol)
    mm = tv.mismatch_stats(g, r, tol)
    for k in ("mismatch_count", "first_mismatch_index"):
        if rec[k] != mm[k]:
            probs.append(f"{k}: device {rec[k]} != oracle {mm[k]}")
    return probs


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def kv():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    from kernelverse_amd import _lib, verdict
    _lib.load()
    return verdict


def _noise(rng, n, scale=1e-6):
    r = rng.standard_normal(n).astype(np.float32)
    g = (r + rng.standard_normal(n).astype(np.float32) * np.float32(scale)).astype(np.float32)
    same = g == r
    g[same] = np.nextafter(r[same], np.float32(np.inf))  # every pair differs
    return g, r


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    g, r = _noise(rng, N)
    out.append(("noise", g, r, None))
    # references near zero: many pairs change sign (queued), the rest stay lean
    g, r = _noise(rng, N)
    r[: N // 3] *= np.float32(1e-7)
    g[: N // 3] = r[: N // 3] + rng.standard_normal(N // 3).astype(np.float32) * np.float32(1e-7)
    out.append(("sign_changes", g, r, None))
    # NaN / Inf on either side and on both, scattered through noise
    g, r = _noise(rng, N)
    spots = rng.choice(N, 3000, replace=False)
    kinds = spots % 6
    r[spots[kinds == 0]] = np.nan
    g[spots[kinds == 1]] = np.nan
    g[spots[kinds == 2]] = np.inf
    r[spots[kinds == 3]] = -np.inf
    both = spots[kinds == 4]
    g[both] = np.inf
    r[both] = np.inf
    g[spots[kinds == 5]] = np.float32(3e38)
    r[spots[kinds == 5]] = np.float32(-3e38)  # finite values, infinite abs_diff
    out.append(("nonfinite", g, r, None))
    # relative noise up to 1e-2: ULP distances across every bucket, mismatches under the default tolerance
    r = rng.standard_normal(N).astype(np.float32)
    g = (r * (1 + rng.uniform(-1e-2, 1e-2, N))).astype(np.float32)
    g[g == r] = np.nextafter(r[g == r], np.float32(np.inf))
    out.append(("wide_ulp", g, r, None))
    # a zero tolerance: every pair a mismatch
    g, r = _noise(rng, N)
    out.append(("zero_tolerance", g, r, {"FP32": {"atol": 0.0, "rtol": 0.0}}))
    # about half the pairs beyond a tight tolerance, at random positions
    g, r = _noise(rng, N)
    far = rng.random(N) < 0.5
    g[far] = r[far] + np.float32(1e-3)
    out.append(("half_mismatch", g, r, {"FP32": {"atol": 1e-5, "rtol": 1e-5}}))
    # ties: one abs_diff everywhere (exact), its argmax the first element; two
    # larger equal ones far apart (different waves), the lower index wins
    r = (np.arange(N) % 1000).astype(np.float32) * np.float32(0.5) + np.float32(1.0)
    g = r + np.float32(0.25)
    g[700_001] += np.float32(0.5)
    g[300_003] += np.float32(0.5)
    out.append(("abs_ties", g, r, {"FP32": {"atol": 1.0, "rtol": 0.0}}))
    # abs_diff right at the allowed bound fl(atol + fl(rtol * |g|)) and a few ULPs either side: g on a
    # grid of 2^-13 in [1, 2) (either sign) makes that bound exact, r = g - bound, then r moves by k ULPs.
    # Pairs between the lowered in-place bound and the exact one take the exact test.
    for nm, atol, rtol in (("tol_boundary", 2.0 ** -10, 2.0 ** -10), ("tol_boundary_rtol_only", 0.0, 2.0 ** -7)):
        mag = (np.float32(1.0) + rng.integers(0, 1 << 13, N).astype(np.float32) * np.float32(2.0 ** -13))
        bound = (np.float32(atol) + mag * np.float32(rtol)).astype(np.float32)
        rm = (mag - bound).astype(np.float32)
        k = rng.integers(-3, 4, N).astype(np.float32)
        rm = (rm + k * np.float32(2.0 ** -23)).astype(np.float32)
        sign = np.where(rng.random(N) < 0.5, np.float32(1), np.float32(-1))
        g, r = (sign * mag).astype(np.float32), (sign * rm).astype(np.float32)
        allowed = (np.float32(atol) + np.abs(np.float32(rtol) * g)).astype(np.float32)
        ad = np.abs(g - r)
        assert (ad == allowed).sum() > 100_000 and (ad > allowed).sum() > 100_000
        out.append((nm, g, r, {"FP32": {"atol": atol, "rtol": rtol}}))
    # an atol below the in-place test's range (every pair takes the exact test)
    g, r = _noise(rng, N)
    out.append(("tiny_atol", g, r, {"FP32": {"atol": 1e-35, "rtol": 1e-5}}))
    # rel_diff ties: the largest rel_diff first appears halfway and then every 1000 elements; the lowest
    # index wins (lanes, waves and items apart)
    i = np.arange(N)
    r = (np.float32(2.5) + (i % 1000).astype(np.float32) * np.float32(0.5)).astype(np.float32)
    r[(i >= N // 2) & (i % 1000 == 0)] = np.float32(2.0)
    g = (r + np.float32(0.5)).astype(np.float32)
    out.append(("rel_ties", g, r, {"FP32": {"atol": 1.0, "rtol": 0.0}}))
    return [(nm, torch.from_numpy(np.ascontiguousarray(a)), torch.from_numpy(np.ascontiguousarray(b)), tol)
            for nm, a, b, tol in out]


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_dense_record_matches_oracle(kv, case):
    name, g, r, tol = case
    _say("dense record", name, g.numel())
    rec = kv.verdict_record(g.to(DEV), r.to(DEV), tolerance_policy=tol)
    probs = _problems(rec, g, r, tol)
    assert not probs, probs


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_dense_meta_matches_oracle(kv, case):
    name, g, r, tol = case
    _say("dense meta", name)
    want = tv.compare_tensors(g, r, "output", tol, None)
    got = kv._compare_tensors(g.to(DEV), r.to(DEV), "output", tol, None)
    probs = meta_problems(got[2], want[2], g, r)
    assert not probs, probs
    assert got[0] == want[0]
    assert got[1] == want[1]


def test_dense_batch_matches_oracle(kv):
    """The same pairs in one batched call (the batch kernels, per-pair tolerances), in pieces of
    several sizes so that waves cross segment boundaries inside their item ranges."""
    pairs = []
    for name, g, r, tol in CASES:
        for lo, hi in ((0, 4096), (4096, 70_001), (70_001, N)):
            pairs.append((name, g[lo:hi].clone(), r[lo:hi].clone(), tol))
    _say("dense batch", len(pairs))
    recs = kv.verdict_records([(g.to(DEV), r.to(DEV), tol) for _, g, r, tol in pairs])
    for (name, g, r, tol), rec in zip(pairs, recs):
        probs = _problems(rec, g, r, tol)
        assert not probs, (name, g.numel(), probs)
