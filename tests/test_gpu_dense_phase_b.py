"""Items whose pairs are mostly slow, finished in place (needs an MI355X).

When every lane of a wave has at least 3/4 of its element slots slow (pairs
that differ), items of 32- and 64-bit elements skip the phase-B queue: each
lane finishes its own slots in order, with the slots that are not slow masked
off.  These pairs put every wave on that path (all elements differ), on it with
masked slots (1 % identical pairs), and across the threshold (30 % identical:
the queue); integer pairs take the max-abs-diff branch (GCR:716-719), float
pairs the isclose branch (GCR:722-727).  Each record must match the oracle:
counts, ULP histogram, argmaxima, first mismatch, fp64 sums and the p99s
(GCR:338-348, 396-402).
"""

import sys

import numpy as np
import pytest
import torch

from golden_io import same_value
from oracle import torch_verdict as tv
from parity_util import record_vs_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"


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


def _ints(rng, dtype, n, same_frac):
    r = torch.from_numpy(rng.integers(-1_000_000, 1_000_000, size=n)).to(dtype)
    step = rng.integers(1, 6, size=n) * rng.choice([-1, 1], size=n)
    g = r + torch.from_numpy(step).to(dtype)
    if same_frac:
        idx = torch.from_numpy(rng.choice(n, size=int(n * same_frac), replace=False))
        g[idx] = r[idx]
    return g, r


def _floats(rng, dtype, n, same_frac):
    r = torch.from_numpy(rng.standard_normal(n)).to(dtype)
    g = (r.double() * (1.0 + 1e-5 * torch.from_numpy(rng.standard_normal(n)))).to(dtype)
    g[g == r] = (r[g == r].double() * 1.001 + 1e-3).to(dtype)  # every pair differs
    if same_frac:
        idx = torch.from_numpy(rng.choice(n, size=int(n * same_frac), replace=False))
        g[idx] = r[idx]
    return g, r


def _cases():
    rng = np.random.default_rng(77)
    return [
        ("fp32 1M all differ", *_floats(rng, torch.float32, 1_000_003, 0.0)),
        ("fp32 700k 1% identical", *_floats(rng, torch.float32, 700_001, 0.01)),
        ("fp32 400k 30% identical", *_floats(rng, torch.float32, 400_000, 0.30)),
        ("fp64 300k all differ", *_floats(rng, torch.float64, 300_007, 0.0)),
        ("int32 500k all differ", *_ints(rng, torch.int32, 500_003, 0.0)),
        ("int32 500k 1% identical", *_ints(rng, torch.int32, 500_000, 0.01)),
        ("int64 250k all differ", *_ints(rng, torch.int64, 250_001, 0.0)),
    ]


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_mostly_slow_items(kv, case):
    name, g, r = case
    _say("dense phase B:", name)
    rec = kv.verdict_record(g.to(DEV), r.to(DEV))
    probs = record_vs_oracle(rec, g, r)
    st = tv.mismatch_stats(g, r)
    if rec["mismatch_count"] != st["mismatch_count"]:
        probs.append(f"mismatch_count: device {rec['mismatch_count']} != oracle {st['mismatch_count']}")
    if rec["first_mismatch_index"] != st["first_mismatch_index"]:
        probs.append(f"first_mismatch_index: device {rec['first_mismatch_index']} != oracle {st['first_mismatch_index']}")
    abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, None)
    for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
        want = tv.p99_meta(vals, tv.MAX_SAMPLES)
        if not same_value(float(rec[k]), float(want)):
            probs.append(f"{k}: device {rec[k]!r} != oracle {want!r}")
    assert not probs, (name, probs)
