"""p99 of large sample groups through the digit levels (needs an MI355X).

A group of more than 8192 samples in a single pair, or in a batch with fewer
such groups than the device has CUs, is selected in digit levels: level 0
histograms the top 8 key bits, level 1 histograms bits 23..12 under the
ranks' prefixes and keeps those values as candidates, and the final read-off
counts the last 12 bits of the target group's candidates.  Level 1 counts
exact zeros (the abs/rel diffs of identical pairs) instead of keeping them,
and a NaN among the samples ends the search early.  Each case below must give
the oracle's torch.quantile over the sampled abs_diff / rel_diff
(GCR:338-348, 396-402): order statistics inside the zeros, in a target group
that holds the zeros and subnormal diffs together, straddling the last zero and
the first subnormal, with NaN, and at strided sample positions.
"""

import math
import sys

import numpy as np
import pytest
import torch

from golden_io import same_value
from oracle import torch_verdict as tv
from parity_util import record_vs_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
SUB = 1.401298464324817e-45  # the smallest float32 subnormal


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


def _q99_ranks(n):
    rk = np.float32(0.99) * np.float32(n - 1)
    return int(rk), int(math.ceil(rk))


def _mostly_identical(n, frac, rng, step=0.5):
    r = torch.from_numpy(rng.standard_normal(n).astype(np.float32))
    g = r.clone()
    idx = torch.from_numpy(rng.choice(n, size=int(n * frac), replace=False))
    g[idx] += step
    return g, r


def _subnormal_diffs(n, frac, rng):
    """abs_diff = k * 2^-149 (k < 4096: digit 0 of the +0 prefix) on `frac` of the
    positions, exact zeros elsewhere: the target group holds zeros and candidates."""
    r = torch.zeros(n, dtype=torch.float32)
    g = r.clone()
    idx = torch.from_numpy(rng.choice(n, size=int(n * frac), replace=False))
    k = rng.integers(1, 4096, size=idx.numel()).astype(np.float64)
    g[idx] = torch.from_numpy((k * SUB).astype(np.float32))
    return g, r


def _straddle(n, rng):
    """The lower order statistic is the last exact zero, the upper the first subnormal diff."""
    while True:
        lo, hi = _q99_ranks(n)
        if hi > lo:
            break
        n += 1
    r = torch.zeros(n, dtype=torch.float32)
    g = r.clone()
    nz = n - hi
    idx = torch.from_numpy(rng.choice(n, size=nz, replace=False))
    g[idx] = torch.from_numpy((rng.integers(1, 4096, size=nz) * SUB).astype(np.float32))
    return g, r


def _cases():
    rng = np.random.default_rng(2024)
    bf = _mostly_identical(3_000_000, 0.004, rng)
    cases = [
        ("fp32 2M 0.5% differ (p99 in the zeros)", *_mostly_identical(2_000_000, 0.005, rng), None),
        ("fp32 1.5M zeros + 2% subnormal diffs", *_subnormal_diffs(1_500_000, 0.02, rng), None),
        ("fp32 straddle zero / subnormal", *_straddle(1_000_003, rng), None),
        ("bf16 3M 0.4% differ", bf[0].to(torch.bfloat16), bf[1].to(torch.bfloat16), None),
        ("fp32 5M 0.5% differ, strided samples", *_mostly_identical(5_000_000, 0.005, rng), None),
        ("fp32 1.2M zeros + 1.5% subnormal, cap 300k", *_subnormal_diffs(1_200_000, 0.015, rng), 300_000),
    ]
    i8r = torch.from_numpy(rng.integers(-100, 100, size=4_000_000).astype(np.int8))
    i8g = i8r.clone()
    i8g[torch.from_numpy(rng.choice(i8r.numel(), size=1000, replace=False))] += 3
    cases.append(("int8 4M 1000 changed", i8g, i8r, None))
    g, r = _mostly_identical(1_000_000, 0.003, rng)
    g[::4099] = float("nan")
    cases.append(("fp32 1M zeros with NaN", g, r, None))
    return cases


CASES = _cases()


def _check(rec, g, r, ms):
    probs = record_vs_oracle(rec, g, r, None, ms)
    abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, None)
    for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
        want = tv.p99_meta(vals, ms)
        if not same_value(float(rec[k]), float(want)):
            probs.append(f"{k}: device {rec[k]!r} != oracle {want!r}")
    return probs


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_single_pair_levels(kv, case):
    name, g, r, ms = case
    ms = ms or tv.MAX_SAMPLES
    _say("select levels, single pair:", name)
    rec = kv.verdict_record(g.to(DEV), r.to(DEV), max_samples=ms)
    probs = _check(rec, g, r, ms)
    assert not probs, (name, probs)


def test_batch_levels(kv):
    """A batch with a few large groups (fewer than the CUs): the level launches
    after the main pass, with the zero counts kept per group."""
    rng = np.random.default_rng(7)
    pairs = [_mostly_identical(400_000, 0.005, rng), _subnormal_diffs(300_000, 0.02, rng),
             _straddle(250_001, rng), _mostly_identical(9_000, 0.2, rng), _subnormal_diffs(120_000, 0.5, rng)]
    _say("select levels, batch of", len(pairs))
    recs = kv.verdict_records([(g.to(DEV), r.to(DEV)) for g, r in pairs])
    for i, ((g, r), rec) in enumerate(zip(pairs, recs)):
        probs = _check(rec, g, r, tv.MAX_SAMPLES)
        assert not probs, (i, probs)
