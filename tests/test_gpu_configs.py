"""The benchmark configurations at full size (C1-C4) on the device.

Every record field that decomposes over elements is checked against the CPU
oracle chunk by chunk (16 Mi elements at a time, merged in order): mismatch
count and first index, maxima over the mismatches, global argmax of abs and
rel diff, ULP histogram, NaN/Inf counts, finite-pattern violations, fp64
sums.  The sampled fields (p99, sampled cosine and norm ratio) are checked
against the oracle run on the strided sample itself, gathered on the device.
Where the generator fixes a count (17 finite-pattern breaks, 1000 changed
int8 positions), that count is asserted too.
"""

import math
import sys

import pytest
import torch

from golden_io import same_value
from parity_util import SUM_RTOL, close, unrounded_close
from oracle import torch_verdict as tv

pytestmark = pytest.mark.gpu

DEV = "cuda"
CHUNK = 1 << 24
COUNT_FIELDS = ("mismatch_count", "nan_pairs", "finite_violations", "nan_gen", "nan_ref", "posinf_gen", "posinf_ref",
                "neginf_gen", "neginf_ref")


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


def _nan_max(a, b):
    """torch's max over a concatenation: NaN if either part has one."""
    if a is None:
        return b
    if b is None:
        return a
    if math.isnan(a) or math.isnan(b):
        return float("nan")
    return max(a, b)


def _argmax_merge(best, cand):
    """(value, index) pairs in index order: NaN is maximal, ties keep the earlier index."""
    if best is None:
        return cand
    bv, cv = best[0], cand[0]
    if math.isnan(bv):
        return best
    if math.isnan(cv) or cv > bv:
        return cand
    return best


def chunked_oracle(g_dev, r_dev, tol):
    """Oracle fields over all elements of a (possibly strided) device pair, 16 Mi elements at a time."""
    gf, rf = g_dev.reshape(-1), r_dev.reshape(-1)
    n = rf.numel()
    out = {k: 0 for k in COUNT_FIELDS}
    out.update(ulp_hist=[0] * tv.HIST_BUCKETS, first_mismatch_index=-1, first_finite_violation=-1,
               mismatch_max_abs=None, mismatch_max_rel=None, sum_gg=0.0, sum_rr=0.0, sum_gr=0.0, sum_dd=0.0)
    best_abs = best_rel = None
    for s in range(0, n, CHUNK):
        gc, rc = gf[s:s + CHUNK].cpu(), rf[s:s + CHUNK].cpu()
        ext = tv.extension_record(gc, rc, tol)
        mm = tv.mismatch_stats(gc, rc, tol)
        for k in COUNT_FIELDS:
            out[k] += (mm if k == "mismatch_count" else ext)[k]
        out["ulp_hist"] = [a + b for a, b in zip(out["ulp_hist"], ext["ulp_hist"])]
        if out["first_mismatch_index"] < 0 and mm["first_mismatch_index"] >= 0:
            out["first_mismatch_index"] = s + mm["first_mismatch_index"]
        if out["first_finite_violation"] < 0 and ext["first_finite_violation"] >= 0:
            out["first_finite_violation"] = s + ext["first_finite_violation"]
        out["mismatch_max_abs"] = _nan_max(out["mismatch_max_abs"], mm["mismatch_max_abs"])
        out["mismatch_max_rel"] = _nan_max(out["mismatch_max_rel"], mm["mismatch_max_rel"])
        best_abs = _argmax_merge(best_abs, (ext["max_abs"], s + ext["max_abs_index"]))
        best_rel = _argmax_merge(best_rel, (ext["max_rel"], s + ext["max_rel_index"]))
        for k in ("sum_gg", "sum_rr", "sum_gr", "sum_dd"):
            out[k] += ext[k]
    out["max_abs"], out["max_abs_index"] = best_abs
    out["max_rel"], out["max_rel_index"] = best_rel
    out["rel_l2"] = tv.rel_l2_from_sums(out["sum_dd"], out["sum_rr"])
    out["cosine"] = tv.cosine_from_sums(out["sum_gr"], out["sum_gg"], out["sum_rr"])
    return out


def sampled_oracle(g_dev, r_dev, tol, m=tv.MAX_SAMPLES):
    """p99 of abs/rel diff, sampled cosine and norm ratio: the oracle on the strided sample of GCR:338-348."""
    gf, rf = g_dev.reshape(-1), r_dev.reshape(-1)
    n = rf.numel()
    if n > m:
        idx = torch.arange(m, device=rf.device, dtype=torch.int64) * (n - 1) // (m - 1)
        gf, rf = gf[idx], rf[idx]
    gs, rs = gf.cpu(), rf.cpu()
    abs_d, rel_d, _, _ = tv.mismatch_parts(gs, rs, tol)
    return {"p99_abs": tv.p99_meta(abs_d), "p99_rel": tv.p99_meta(rel_d),
            "sample_cosine": tv.cosine_similarity_value(gs, rs), "sample_norm_ratio": tv.norm_ratio_value(gs, rs)}


def check_record(rec, g_dev, r_dev, tol):
    exp = chunked_oracle(g_dev, r_dev, tol)
    bad = []
    exact = COUNT_FIELDS + ("ulp_hist", "first_mismatch_index", "first_finite_violation", "max_abs_index",
                            "max_rel_index")
    for k in exact:
        if not same_value(rec[k], exp[k]):
            bad.append(f"{k}: device {rec[k]!r} != oracle {exp[k]!r}")
    for k in ("max_abs", "max_rel"):
        if not same_value(float(rec[k]), float(exp[k])):
            bad.append(f"{k}: device {rec[k]!r} != oracle {exp[k]!r}")
    if exp["mismatch_count"]:
        for k in ("mismatch_max_abs", "mismatch_max_rel"):
            if not same_value(float(rec[k]), float(exp[k])):
                bad.append(f"{k}: device {rec[k]!r} != oracle {exp[k]!r}")
    for k in ("sum_gg", "sum_rr", "sum_gr", "sum_dd", "rel_l2", "cosine"):
        if not close(rec[k], exp[k], SUM_RTOL):
            bad.append(f"{k}: device {rec[k]!r} vs oracle {exp[k]!r}")
    smp = sampled_oracle(g_dev, r_dev, tol)
    for k in ("p99_abs", "p99_rel"):
        if not same_value(float(rec[k]), float(smp[k])):
            bad.append(f"{k}: device {rec[k]!r} != oracle {smp[k]!r}")
    # before the meta's round(., 4): fp64 sums in another order, 1e-12 relative
    for k in ("sample_cosine", "sample_norm_ratio"):
        if smp[k] is not None and not unrounded_close(rec[k], smp[k]):
            bad.append(f"{k}: device {rec[k]!r} vs oracle {smp[k]!r} (unrounded)")
    n = r_dev.numel()
    if sum(rec["ulp_hist"]) + rec["nan_pairs"] != n:
        bad.append("ulp_hist + nan_pairs != numel")
    return bad, exp


def test_c1_bf16_256mi(kv):
    from kernelverse_amd import synth
    _say("C1 bf16 268,435,456")
    g, r = synth.c1_pair(DEV)
    tol = {"BF16": {"rtol": 1.6e-2, "atol": 1e-2}}
    rec = kv.verdict_record(g, r, tolerance_policy=tol)
    bad, exp = check_record(rec, g, r, tol)
    assert not bad, bad
    # by construction: only 1-ULP and 3-ULP steps, no non-finite values
    assert rec["ulp_hist"][3:] == [0] * 13 and rec["nan_pairs"] == 0 and rec["finite_violations"] == 0
    assert 0.049 < rec["ulp_hist"][1] / rec["numel"] < 0.051
    assert 0.8e-4 < rec["ulp_hist"][2] / rec["numel"] < 1.2e-4


@pytest.mark.parametrize("p1", [0.05, 0.5])
def test_c1_bf16_tolerant_full_size(kv, p1):
    """C1 under the tolerant policy (the category default of gemm): the near-zero diagnostics come
    from entries the main pass records (one pass over 268 M elements, ~27 M of them near zero; with
    p1 = 0.5 half of all elements moved, so ~13 M near-zero elements carry entries).
    Against the oracle (GCR:481-548): near/far counts, far mismatches and bad counts exact, chunk by
    chunk; near_zero_p99_abs exact and near_zero_mean_abs within 1e-6 on the strided sample of the
    compacted near-zero abs_diff array, gathered on the device; every other field as for strict C1."""
    from kernelverse_amd import synth
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    from parity_util import MEAN_RTOL
    _say("C1 bf16 268,435,456 tolerant, moved fraction", p1)
    g, r = synth.c1_pair(DEV, p1=p1)
    tol = {"BF16": {"rtol": 1.6e-2, "atol": 1e-2}}
    pol = resolve_correctness_policy({"category": "gemm", "op_name": "x"})
    nz_abs, nz_bad = 0.25, 2.0
    assert tv.thresholds_for_dtype(pol, "BF16")["near_zero_abs"] == nz_abs
    assert tv.thresholds_for_dtype(pol, "BF16")["max_near_zero_bad_abs"] == nz_bad
    rec = kv.verdict_record(g, r, tolerance_policy=tol, correctness_policy=pol)
    assert rec["status"] == 0
    gf, rf = g.reshape(-1), r.reshape(-1)
    near = far_mm = bad = 0
    for s in range(0, rf.numel(), CHUNK):
        gc, rc = gf[s:s + CHUNK].cpu(), rf[s:s + CHUNK].cpu()
        abs_d, _, mism, _ = tv.mismatch_parts(gc, rc, tol)
        nm = rc.to(torch.float32).abs() <= nz_abs
        near += int(nm.sum())
        far_mm += int((mism & ~nm).sum())
        bad += int((abs_d[nm] > nz_bad).sum())
    _say("C1 tolerant: counts", near, far_mm, bad)
    assert (rec["near_zero_count"], rec["far_count"], rec["far_mismatch_count"], rec["near_zero_bad_count"]) == (
        near, rf.numel() - near, far_mm, bad)
    # GCR:525-529: abs_diff over the near-zero positions in row-major order, then its strided sample
    comp = (gf.to(torch.float32) - rf.to(torch.float32)).abs()[rf.to(torch.float32).abs() <= nz_abs]
    c = comp.numel()
    m = min(c, tv.MAX_SAMPLES)
    idx = torch.arange(m, device=comp.device, dtype=torch.int64) * (c - 1) // (m - 1)
    sample = comp[idx].cpu()
    del comp
    assert rec["near_zero_sample_count"] == m
    p99, mean = tv.p99_meta(sample), tv.mean_meta(sample)
    assert same_value(float(rec["near_zero_p99_abs"]), p99), (rec["near_zero_p99_abs"], p99)
    assert close(rec["near_zero_mean_abs"], mean, MEAN_RTOL), (rec["near_zero_mean_abs"], mean)
    bad_fields, _ = check_record(rec, g, r, tol)
    assert not bad_fields, bad_fields


def test_c2_fp16_strided(kv):
    from kernelverse_amd import synth
    _say("C2 fp16 4096x32768 stride 32896")
    g, r = synth.c2_pair(DEV)
    assert not g.is_contiguous() and g.stride() == (32896, 1)
    tol = {"FP16": {"rtol": 1e-3, "atol": 1e-3}}
    rec = kv.verdict_record(g, r, tolerance_policy=tol)
    bad, _ = check_record(rec, g, r, tol)
    assert not bad, bad
    assert rec["finite_violations"] == 17
    # both infinities occur, and the breaks mix kinds (see synth.C2_BREAKS): NaN -> 1.0 four times,
    # NaN -> +-Inf three times, finite -> NaN three times
    assert rec["posinf_ref"] > 0 and rec["neginf_ref"] > 0
    assert rec["nan_ref"] - rec["nan_gen"] == 4
    assert rec["posinf_gen"] + rec["neginf_gen"] == rec["posinf_ref"] + rec["neginf_ref"]


@pytest.mark.parametrize("policy", [None, "gemm", "attention"])
def test_c0_fp32_1m(kv, policy):
    """C0 at its own size (1,048,576 elements: every element a sample, n just above the 10^6 cap
    of the sampled metas): the full record against the oracle, and the drop-in meta under each policy
    kind against the oracle's (the reference's own answers are the c0_* fixtures)."""
    from kernelverse_amd import synth
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    from parity_util import meta_problems
    _say("C0 fp32 1,048,576", policy)
    g, r = synth.fp32_noise_pair(1 << 20, seed=0)
    tol = {"FP32": {"rtol": 1e-5, "atol": 1e-5}}
    gd, rd = g.to(DEV), r.to(DEV)
    rec = kv.verdict_record(gd, rd, tolerance_policy=tol)
    bad, exp = check_record(rec, gd, rd, tol)
    assert not bad, bad
    assert rec["mismatch_count"] == exp["mismatch_count"] > 0
    pol = resolve_correctness_policy({"category": policy, "op_name": "x"}) if policy else None
    want = tv.compare_tensors(g, r, "output", tol, pol)
    got = kv._compare_tensors(gd, rd, "output", tol, pol)
    probs = meta_problems(got[2], want[2], g, r)
    assert not probs, probs
    assert got[0] == want[0] and got[1] == want[1]


def test_c3_fp8_codes(kv):
    from kernelverse_amd import synth
    _say("C3 fp8 e4m3fn 134,217,728")
    g, r = synth.c3_fp8_pair(DEV)
    rec = kv.verdict_record(g, r)
    bad, _ = check_record(rec, g, r, None)
    assert not bad, bad
    changed = int((g.view(torch.uint8) != r.view(torch.uint8)).sum().item())
    assert rec["ulp_hist"][1] == changed and sum(rec["ulp_hist"][2:]) == 0


def test_c3_int8_equality(kv):
    from kernelverse_amd import synth
    _say("C3 int8 134,217,728")
    g, r = synth.c3_int8_pair(DEV)
    rec = kv.verdict_record(g, r)
    bad, _ = check_record(rec, g, r, None)
    assert not bad, bad
    assert rec["mismatch_count"] == 1000
    assert rec["ulp_hist"][0] == r.numel() - 1000


C4_PARTS = 8


@pytest.fixture(scope="module")
def c4(kv):
    """C4 as the bench runs it: 4096 pairs with their own tolerances (synth.c4_tolerance) in one
    kvv_verdict_batch call; the records are kept for the parts below."""
    from kernelverse_amd import synth
    _say("C4 4096 ragged pairs, per-pair tolerances, one batched call")
    pairs = synth.c4_batch(DEV)
    recs = kv.verdict_records(pairs)
    assert len(recs) == len(pairs)
    return pairs, recs


def test_c4_tolerances_are_per_pair(c4):
    """Neighbouring pairs of one dtype carry different tolerances, and for a pair whose mismatch
    count depends on them the device count follows the pair's own (checked against the oracle
    under both the pair's and its neighbour's tolerance)."""
    pairs, recs = c4
    seen = {}
    for i, (g, r, tol) in enumerate(pairs):
        (name, t), = tol.items()
        seen.setdefault(name, set()).add((t["rtol"], t["atol"]))
    assert {k: len(v) for k, v in seen.items()} == {"FP32": 4, "BF16": 4}
    distinguished = 0
    for i in range(0, 400):
        g, r, tol = pairs[i]
        other = pairs[i + 2][2]  # the next pair of the same dtype
        own = tv.mismatch_stats(g.cpu(), r.cpu(), tol)["mismatch_count"]
        alt = tv.mismatch_stats(g.cpu(), r.cpu(), other)["mismatch_count"]
        assert recs[i]["mismatch_count"] == own, (i, tol, recs[i]["mismatch_count"], own)
        distinguished += own != alt
        if distinguished >= 40:
            break
    assert distinguished >= 40


@pytest.mark.parametrize("part", range(C4_PARTS))
def test_c4_every_pair_vs_oracle(kv, c4, part):
    """Every C4 pair (pairs part, part + 8, ...) against the oracle under its own tolerance:
    counts, first indices, argmaxes, ULP histogram and p99 exact; fp64 sums within 1e-6."""
    pairs, recs = c4
    idx = list(range(part, len(pairs), C4_PARTS))
    for k, i in enumerate(idx):
        if k % 128 == 0:
            _say(f"C4 part {part}: pair {i} ({k}/{len(idx)})")
        g, r, tol = pairs[i]
        bad, _ = check_record(recs[i], g, r, tol)
        assert not bad, (i, g.numel(), g.dtype, tol, bad)


def test_c4_batch_matches_single_calls(kv, c4):
    """Every 16th C4 pair as a single-pair call: the same record (the fp64 sums depend on how the
    launch cut the pair into runs, 1e-6; all else exact)."""
    pairs, recs = c4
    summed = ("sample_sum_gg", "sample_sum_rr", "sample_sum_gr", "sample_cosine", "sample_norm_ratio",
              "sum_gg", "sum_rr", "sum_gr", "sum_dd", "rel_l2", "cosine")
    for i in range(0, len(pairs), 16):
        g, r, tol = pairs[i]
        single = kv.verdict_record(g, r, tolerance_policy=tol)
        diff = [k for k in single if k not in summed and not same_value(single[k], recs[i][k])]
        diff += [k for k in summed if not close(single[k], recs[i][k], SUM_RTOL)]
        assert not diff, (i, diff)
