"""Near-zero diagnostics of single fp16/bf16 pairs taken as entries in the main pass (needs an MI355X).

Under the tolerant policy the reference compacts abs_diff over |ref| <= near_zero_abs
in row-major order and samples the compacted array (GCR:481-548, 525-529).  A
single vector-kind fp16/bf16 pair records, in its one pass, the near-zero
elements with a nonzero abs_diff ("entries": rank and value); the first tail
launch ranks them globally and builds the near-zero sample.  These tests check
that record against the two-pass path (KVV_FLAG_NEAR_EXACT: a second pass over
the inputs) field by field, the drop-in's meta against the oracle, and the
overflow path: the waves whose entries do not fit their share of the pool are
read again by the first tail launch of the same call.
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


def _exact_fields_match(ent, exact):
    """Entry-path record against the exact path's: everything equal except the near-zero mean,
    whose fp64 sum runs in another order (1e-12 relative)."""
    bad = []
    for k in ent:
        a, b = ent[k], exact[k]
        if k == "near_zero_mean_abs":
            if not (a == b or (math.isnan(a) and math.isnan(b)) or abs(a - b) <= 1e-12 * abs(b)):
                bad.append(f"{k}: entries {a!r} vs exact {b!r}")
        elif k in ("sample_sum_gg", "sample_sum_rr", "sample_sum_gr", "sample_cosine", "sample_norm_ratio", "sum_gg",
                   "sum_rr", "sum_gr", "sum_dd", "rel_l2", "cosine"):
            continue
        elif not (a == b or (isinstance(a, float) and math.isnan(a) and math.isnan(b))):
            bad.append(f"{k}: entries {a!r} vs exact {b!r}")
    return bad


def _all_near_stepped(n, seed, dtype):
    """Every reference value near zero and every candidate one code away: each wave's entries
    outgrow its share of the pool."""
    from kernelverse_amd import synth
    rng = np.random.default_rng(seed)
    r = torch.from_numpy(rng.uniform(-0.2, 0.2, n).astype(np.float32)).to(dtype)
    g = synth.step_codes(r, np.arange(n), np.ones(n, dtype=np.int64), rng)
    return g, r


def test_pool_overflow_is_read_again_in_the_same_call(kv):
    """Every element near zero and different: every wave's entries overflow its share, the first
    tail launch reads those waves again, and the record comes back complete (status 0) with the
    exact path's near-zero fields and the oracle's meta."""
    from kernelverse_amd import _lib
    g, r = _all_near_stepped(4_194_304, 79, torch.float16)
    pol = _tolerant()
    gd, rd = g.to(DEV), r.to(DEV)
    _say("near entries: every wave overflows")
    rec = _record(kv, gd, rd, None, pol)
    exact = _record(kv, gd, rd, None, pol, _lib.FLAG_NEAR_EXACT)
    assert rec["status"] == 0 and exact["status"] == 0
    assert rec["near_zero_count"] == r.numel()
    bad = _exact_fields_match(rec, exact)
    assert not bad, bad
    got = kv._compare_tensors(gd, rd, "output", None, pol)
    want = tv.compare_tensors(g, r, "output", None, pol)
    probs = meta_problems(got[2], want[2], g, r)
    assert not probs, probs
    assert got[0] == want[0] and got[1] == want[1]


def test_some_waves_overflow(kv):
    """A pair whose first 3 M elements are all near zero and stepped (their waves overflow) and
    whose other 9 M follow the C1 model (their waves keep their entries): both kinds of wave in one
    call, against the exact path and the oracle."""
    from kernelverse_amd import _lib, synth
    g1, r1 = _all_near_stepped(3_000_000, 80, torch.bfloat16)
    g2, r2 = synth.code_flip_pair(9_000_000, seed=81)
    g, r = torch.cat([g1, g2]), torch.cat([r1, r2])
    pol = _tolerant()
    gd, rd = g.to(DEV), r.to(DEV)
    _say("near entries: some waves overflow")
    rec = _record(kv, gd, rd, None, pol)
    exact = _record(kv, gd, rd, None, pol, _lib.FLAG_NEAR_EXACT)
    assert rec["status"] == 0
    bad = _exact_fields_match(rec, exact)
    assert not bad, bad
    got = kv._compare_tensors(gd, rd, "output", None, pol)
    want = tv.compare_tensors(g, r, "output", None, pol)
    probs = meta_problems(got[2], want[2], g, r)
    assert not probs, probs


def test_least_pool_of_the_noalloc_entry(kv):
    """A tolerant pair whose full entry pool would not fit the no-alloc scratch (64 MiB): the
    no-alloc entry runs with the least pool (waves beyond it read again) and gives kvv_verdict's
    record (fresh workspace, full pool)."""
    from kernelverse_amd import _lib, synth
    lib = _lib.load()
    g, r = synth.code_flip_pair_device(50_000_000, seed=82, device=DEV, std=0.3, p1=0.5)
    pol = _tolerant()
    job = kv._Job(g, r, "output", None, pol, kv.MAX_SAMPLES)
    gt, rt, held = kv._device_views(g, r)
    size = ctypes.c_size_t()
    _lib.check(lib.kvv_workspace_size(gt, rt, job.kpolicy, ctypes.byref(size)), "kvv_workspace_size")
    assert size.value > _lib.NOALLOC_SCRATCH_BYTES  # the full pool does not fit the scratch
    _say("near entries: no-alloc with the least pool")
    full = _record(kv, g, r, None, pol)
    out = torch.empty(ctypes.sizeof(_lib.KvvResult), dtype=torch.uint8, pin_memory=True)
    _lib.check(lib.kvv_verdict_noalloc(gt, rt, job.kpolicy, out.data_ptr(), torch.cuda.current_stream().cuda_stream),
               "kvv_verdict_noalloc")
    torch.cuda.current_stream().synchronize()
    least = _lib.KvvResult.from_buffer_copy(out.numpy().tobytes()).to_dict()
    assert least["status"] == 0 and full["status"] == 0
    bad = _exact_fields_match(least, full)
    assert not bad, bad
