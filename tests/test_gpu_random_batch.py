"""Seeded random batches of the device verdict against the CPU oracle (needs an MI355X).

Each batch mixes element types, shapes, layouts (contiguous, transposed,
strided, misaligned), perturbations and special values in one
``kvv_verdict_batch`` call, under one tolerance policy and sample cap:

* small batches (most pairs far below 8192 samples): the batch path with its
  per-group select levels;
* many-group batches (more pairs of over 8192 samples than the device has CUs):
  p99 of contiguous pairs from the inputs, other layouts from sample arrays.

Every record must match the oracle's (``parity_util``: exact integers,
indices, maxima and p99; fp64 sums within 1e-6), and the metas and details of
``_compare_outputs`` over the whole nested output must match the oracle's
``compare_outputs`` (float8 pairs, whose metas the reference refuses, are left
out of that part).
"""

import sys

import numpy as np
import pytest
import torch

import test_gpu_random_sweep as sweep
from golden_io import same_value
from oracle import torch_verdict as tv
from parity_util import meta_problems, record_vs_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


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


def _large_case(rng):
    """A pair of 8.2 K - 60 K elements: random dtype, perturbation and layout."""
    pool = sweep.FLOATS * 3 + list(FP8) + sweep.INTS
    dtype = pool[int(rng.integers(0, len(pool)))]
    n = int(rng.integers(8_200, 60_000))
    shape = (n,) if rng.integers(0, 3) else (int(rng.integers(91, 180)), n // 180 + 1)
    ref = sweep._values(rng, dtype, int(np.prod(shape))).view(shape)
    gen = sweep._perturb(rng, dtype, ref)
    return dtype, gen, ref, sweep._layout(rng, gen)


def _tolerance(rng):
    if rng.integers(0, 2):
        return None
    return {"FP32": {"rtol": float(10.0 ** rng.integers(-6, -2)), "atol": float(10.0 ** rng.integers(-6, -2))},
            "BF16": {"rtol": 1.6e-2, "atol": 1e-2}, "INT32": {"max_abs_diff": int(rng.integers(0, 3))}}


def _check_batch(kv, cases, tol, max_samples, tag):
    cpu = [(layout(g), layout(r)) for _, g, r, layout in cases]
    dev = [(layout(g.to(DEV)), layout(r.to(DEV))) for _, g, r, layout in cases]
    _say("batch", tag, len(cases), "pairs", "max_samples", max_samples, "tol", tol)
    recs = kv.verdict_records(dev, tolerance_policy=tol, max_samples=max_samples)
    for i, ((g, r), rec) in enumerate(zip(cpu, recs)):
        probs = record_vs_oracle(rec, g, r, tol, max_samples)
        if g.numel():
            abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, tol)
            for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
                want = tv.p99_meta(vals, max_samples)
                if not same_value(float(rec[k]), float(want)):
                    probs.append(f"{k}: device {rec[k]!r} != oracle {want!r}")
        assert not probs, (tag, i, g.dtype, tuple(g.shape), tuple(g.stride()), probs)
    keep = [i for i, (dt, *_rest) in enumerate(cases) if dt not in FP8]
    pol = {"name": "strict", **__import__("kernelverse_amd.correctness_policy", fromlist=["x"]).resolve_correctness_policy(
        {"category": "gemm", "op_name": "matmul"})}
    got = kv._compare_outputs(tuple(dev[i][0] for i in keep), tuple(dev[i][1] for i in keep), tolerance_policy=tol,
                              correctness_policy=pol, max_samples=max_samples)
    want = tv.compare_outputs(tuple(cpu[i][0] for i in keep), tuple(cpu[i][1] for i in keep), tolerance_policy=tol,
                              correctness_policy=pol, max_samples=max_samples)
    assert got[0] == want[0] and got[1] == want[1], tag
    assert len(got[2]) == len(want[2])
    for i, a, b in zip(keep, got[2], want[2]):
        probs = meta_problems(a, b, cpu[i][0], cpu[i][1], max_samples)
        assert not probs, (tag, probs)


@pytest.mark.parametrize("seed", range(16))
def test_random_small_batch(kv, seed):
    rng = np.random.default_rng(500 + seed)
    cases = []
    for k in range(int(rng.integers(5, 60))):
        dtype, g, r, layout, _, _ = sweep._case(2000 + 100 * seed + k)
        cases.append((dtype, g, r, layout))
    _check_batch(kv, cases, _tolerance(rng), [1_000_000, 997, 37][seed % 3], f"small{seed}")


@pytest.mark.parametrize("seed", range(6))
def test_random_many_group_batch(kv, seed):
    rng = np.random.default_rng(900 + seed)
    cases = [_large_case(rng) for _ in range(300)]
    # a few small pairs ride along (selected at the first tail level)
    for k in range(10):
        dtype, g, r, layout, _, _ = sweep._case(3000 + 100 * seed + k)
        cases.append((dtype, g, r, layout))
    _check_batch(kv, cases, _tolerance(rng), [1_000_000, 20_011, 9_001][seed % 3], f"many{seed}")
