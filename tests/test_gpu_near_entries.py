"""Near-zero diagnostics of single fp16/bf16 pairs taken as entries in the main pass (needs an MI355X).

Under the tolerant policy the reference compacts abs_diff over |ref| <= near_zero_abs
in row-major order and samples the compacted array (GCR:481-548, 525-529).  A
single vector-kind fp16/bf16 pair records, in its one pass, the near-zero
elements with a nonzero abs_diff ("entries": rank and value); the first tail
launch ranks them globally and builds the near-zero sample.  These tests check
that record against the two-pass path (KVV_FLAG_NEAR_EXACT: a second pass over
the inputs) field by field, the drop-in's meta against the oracle, and the
overflow path: a pair whose entries do not fit the pool comes back with
KVV_STATUS_NEAR_RETRY and the drop-in reruns it exactly.
"""

import ctypes
import math
import sys

import numpy as np
import pytest
import torch

from parity_util import meta_problems
from oracle import torch_verdict as tv

pytestmark = pytest.mark.gpu

DEV = "cuda"
NEAR_FIELDS = ("near_zero_count", "far_count", "far_mismatch_count", "near_zero_bad_count", "near_zero_sample_count",
               "near_zero_p99_abs")


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


def _tolerant():
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    return resolve_correctness_policy({"category": "gemm", "op_name": "x"})


def _record(kv, g, r, tol, pol, extra_flags=0, max_samples=1_000_000):
    """One kvv_verdict record through the C ABI (no retry)."""
    from kernelverse_amd import _lib
    lib = _lib.load()
    job = kv._Job(g, r, "output", tol, pol, max_samples)
    job.kpolicy.flags |= extra_flags
    gt, rt, held = kv._device_views(g, r)
    size = ctypes.c_size_t()
    _lib.check(lib.kvv_workspace_size(gt, rt, job.kpolicy, ctypes.byref(size)), "kvv_workspace_size")
    ws = torch.empty(size.value, dtype=torch.uint8, device=DEV)
    out = torch.empty(ctypes.sizeof(_lib.KvvResult), dtype=torch.uint8, pin_memory=True)
    _lib.check(lib.kvv_verdict(gt, rt, job.kpolicy, out.data_ptr(), ws.data_ptr(), size.value,
                               torch.cuda.current_stream().cuda_stream), "kvv_verdict")
    torch.cuda.current_stream().synchronize()
    del held
    return _lib.KvvResult.from_buffer_copy(out.numpy().tobytes()).to_dict()


def _flipped_rows(rows, cols, pitch, seed, dtype):
    from kernelverse_amd import synth
    g, r = synth.code_flip_pair(rows * cols, seed=seed, dtype=dtype, std=0.4, p1=0.2, p3=0.02)
    out = []
    for t in (g, r):
        base = torch.zeros(rows, pitch, dtype=dtype)
        base[:, :cols] = t.reshape(rows, cols)
        out.append(base[:, :cols])
    return out[0], out[1]


def _cases():
    from kernelverse_amd import synth
    bf, hf = torch.bfloat16, torch.float16
    cases = [
        # every near-zero rank is a sample (c <= 10^6)
        ("bf16 c1 model 4M", *synth.code_flip_pair(4_194_304, seed=71), {"BF16": {"rtol": 1e-3, "atol": 1e-4}}, 1_000_000),
        # c > 10^6: the rank-strided sample of the compacted array
        ("bf16 c1 model 24M", *synth.code_flip_pair(24_000_000, seed=72), {"BF16": {"rtol": 1e-3, "atol": 1e-4}},
         1_000_000),
        ("fp16 small values 3M", *synth.code_flip_pair(3_000_000, seed=73, dtype=hf, std=0.5, p1=0.3, p3=0.01),
         {"FP16": {"rtol": 1e-4, "atol": 1e-5}}, 1_000_000),
        # strided rows (the row kernel), partial vectors, a small cap on the samples
        ("fp16 rows 2048x1000 pitch 1024", *_flipped_rows(2048, 1000, 1024, 74, hf), None, 1_000_000),
        ("bf16 odd size 100003", *synth.code_flip_pair(100_003, seed=75, std=0.3, p1=0.3), None, 1_000_000),
        ("bf16 2M cap 997", *synth.code_flip_pair(2_000_000, seed=76, std=0.3, p1=0.2), None, 997),
        ("fp16 5000 (small near sample)", *synth.code_flip_pair(5_000, seed=77, dtype=hf, std=0.3, p1=0.3), None,
         1_000_000),
    ]
    # NaN and infinities among the near-zero references' candidates
    g, r = synth.code_flip_pair(1_500_000, seed=78, std=0.3, p1=0.1)
    g[::1009] = float("nan")
    g[5::2003] = float("inf")
    cases.append(("bf16 with NaN/Inf candidates", g, r, None, 1_000_000))
    return cases


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_entries_match_exact_path_and_oracle(kv, case):
    from kernelverse_amd import _lib
    name, g, r, tol, ms = case
    _say("near entries", name)
    pol = _tolerant()
    gd, rd = g.to(DEV), r.to(DEV)
    ent = _record(kv, gd, rd, tol, pol, 0, ms)
    exact = _record(kv, gd, rd, tol, pol, _lib.FLAG_NEAR_EXACT, ms)
    assert ent["status"] == 0 and exact["status"] == 0, (ent["status"], exact["status"])
    bad = []
    for k in ent:
        if k == "near_zero_mean_abs":
            a, b = ent[k], exact[k]
            if not (a == b or (math.isnan(a) and math.isnan(b)) or abs(a - b) <= 1e-6 * abs(b)):
                bad.append(f"{k}: entries {a!r} vs exact {b!r}")
        elif k in ("sample_sum_gg", "sample_sum_rr", "sample_sum_gr", "sample_cosine", "sample_norm_ratio", "sum_gg",
                   "sum_rr", "sum_gr", "sum_dd", "rel_l2", "cosine"):
            continue  # the same main pass computes these either way
        else:
            a, b = ent[k], exact[k]
            same = a == b or (isinstance(a, float) and math.isnan(a) and math.isnan(b))
            if not same:
                bad.append(f"{k}: entries {a!r} vs exact {b!r}")
    assert not bad, (name, bad)
    assert ent["near_zero_count"] > 0
    got = kv._compare_tensors(gd, rd, "output", tol, pol, max_samples=ms)
    want = tv.compare_tensors(g, r, "output", tol, pol, max_samples=ms)
    probs = meta_problems(got[2], want[2], g, r, ms)
    assert not probs, (name, probs)
    assert got[0] == want[0] and got[1] == want[1]


def test_pool_overflow_is_retried_exactly(kv):
    """Every element near zero and different: the entries outgrow the pool (each wave's share),
    the record says KVV_STATUS_NEAR_RETRY, and the drop-in's rerun with the exact path gives the
    oracle's meta."""
    from kernelverse_amd import _lib, synth
    rng = np.random.default_rng(79)
    r = torch.from_numpy(rng.uniform(-0.2, 0.2, 4_194_304).astype(np.float32)).to(torch.float16)
    steps = np.ones(r.numel(), dtype=np.int64)
    g = synth.step_codes(r, np.arange(r.numel()), steps, rng)
    pol = _tolerant()
    gd, rd = g.to(DEV), r.to(DEV)
    _say("near entries: pool overflow")
    rec = _record(kv, gd, rd, None, pol)
    assert rec["status"] == _lib.STATUS_NEAR_RETRY
    exact = _record(kv, gd, rd, None, pol, _lib.FLAG_NEAR_EXACT)
    assert exact["status"] == 0
    # the fields outside the near-zero sample are valid in the retried record too
    for k in ("mismatch_count", "first_mismatch_index", "ulp_hist", "near_zero_count", "near_zero_bad_count"):
        assert rec[k] == exact[k], k
    got = kv._compare_tensors(gd, rd, "output", None, pol)
    want = tv.compare_tensors(g, r, "output", None, pol)
    probs = meta_problems(got[2], want[2], g, r)
    assert not probs, probs
    assert got[0] == want[0] and got[1] == want[1]
