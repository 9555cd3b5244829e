"""p99 selected from the inputs in many-group batches (needs an MI355X).

A batch with at least as many groups of more than 8192 samples as the device
has CUs selects the p99 of each contiguous pair straight from its two inputs
(two passes over the samples, the target bins' values compacted, zeros only
counted).  Every p99 here must equal the oracle's torch.quantile over the
sampled abs_diff / rel_diff, across twelve element types and the cases the compaction
distinguishes: the order statistics inside the zeros, straddling the last zero
and the first non-zero value, in two adjacent bins, with more than 8192 values
in the target bin (streamed, not in LDS), negative int32 abs_diff (|INT_MIN|
wraps), NaN, and sizes that end in a partial 16-byte vector.
"""

import math
import sys

import numpy as np
import pytest
import torch

from golden_io import same_value
from oracle import torch_verdict as tv
from parity_util import SUM_RTOL, close, record_vs_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {"FP32": {"rtol": 1e-5, "atol": 1e-5}, "BF16": {"rtol": 1.6e-2, "atol": 1e-2},
       "FP16": {"rtol": 1e-3, "atol": 1e-3}, "INT32": {"max_abs_diff": 1}, "INT64": {"max_abs_diff": 2}}


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


def _pair(i, rng):
    """One pair of the batch: (generated, reference) on the CPU."""
    kind = i % 12
    n = int(rng.integers(8_200, 30_000))
    if kind == 0:       # 99.5 % identical: both order statistics are zeros
        r = torch.from_numpy(rng.standard_normal(n).astype(np.float32))
        g = r.clone()
        idx = torch.from_numpy(rng.choice(n, size=n // 200, replace=False))
        g[idx] += 0.5
        return g, r
    if kind == 1:       # the lower order statistic is the last zero, the upper the first non-zero value
        while True:
            lo, hi = _q99_ranks(n)
            if hi > lo:
                break
            n += 1
        r = torch.from_numpy(rng.standard_normal(n).astype(np.float32))
        g = r.clone()
        nz = n - hi  # zeros at ranks 0..hi-1
        idx = torch.from_numpy(rng.choice(n, size=nz, replace=False))
        g[idx] += torch.from_numpy(rng.uniform(1.0, 2.0, size=nz).astype(np.float32))
        return g, r
    if kind == 2:       # int32 with |INT_MIN| differences (negative abs_diff after the int32 wrap)
        r = torch.from_numpy(rng.integers(-1000, 1000, size=n).astype(np.int32))
        g = r.clone()
        idx = torch.from_numpy(rng.choice(n, size=n // 50, replace=False))
        g[idx] = g[idx] ^ torch.tensor(-2**31, dtype=torch.int32)
        g[: n // 40] += 3
        return g, r
    if kind == 3:       # fp16 noise
        r = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(torch.float16)
        g = (r.float() * (1 + 1e-3 * torch.from_numpy(rng.standard_normal(n).astype(np.float32)))).to(torch.float16)
        return g, r
    if kind == 4:       # every abs_diff in [1, 1.25): one target bin of n > 8192 values (streamed)
        r = torch.zeros(n, dtype=torch.float32)
        g = torch.from_numpy(rng.uniform(1.0, 1.25, size=n).astype(np.float32))
        return g, r
    if kind == 5:       # bf16 code steps on 3 % of positions, the rest identical
        r = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(torch.bfloat16)
        g = r.clone()
        idx = torch.from_numpy(rng.choice(n, size=n * 3 // 100, replace=False))
        codes = g.view(torch.int16)
        codes[idx] += 1
        return g, r
    if kind == 6:       # float64 noise
        r = torch.from_numpy(rng.standard_normal(n))
        return r + 1e-9 * torch.from_numpy(rng.standard_normal(n)), r
    if kind == 7:       # uint8 / int8 off by a few at 5 % of positions
        dt = torch.uint8 if i % 24 == 7 else torch.int8
        r = torch.from_numpy(rng.integers(0, 100, size=n)).to(dt)
        g = r.clone()
        idx = torch.from_numpy(rng.choice(n, size=n // 20, replace=False))
        g[idx] += 2
        return g, r
    if kind == 8:       # NaN in the generated output: both p99 are NaN
        g, r = _fp32_noise(n, rng)
        g[:: 1000] = float("nan")
        return g, r
    if kind == 9:       # values spread over two adjacent bins at the order statistics
        r = torch.ones(n, dtype=torch.float32)
        g = r.clone()
        lo, hi = _q99_ranks(n)
        d = torch.full((n,), 0.1, dtype=torch.float32)
        d[hi:] = 0.2                      # ranks >= hi fall in a higher bin
        g = r + d[torch.from_numpy(rng.permutation(n))]
        return g, r
    if kind == 10:      # fp8 code flips (e4m3fn, or e5m2 every other time)
        dt = torch.float8_e5m2 if i % 24 == 10 else torch.float8_e4m3fn
        r = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(dt)
        g = r.clone()
        codes = g.view(torch.int8)
        idx = torch.from_numpy(rng.choice(n, size=n // 30, replace=False))
        codes[idx] ^= 1
        return g, r
    if kind == 11 and i % 36 == 11:  # int64 beyond int32 (the int32 casts wrap)
        r = torch.from_numpy(rng.integers(-2**40, 2**40, size=n))
        g = r.clone()
        idx = torch.from_numpy(rng.choice(n, size=n // 25, replace=False))
        g[idx] += torch.from_numpy(rng.integers(-5, 6, size=idx.numel()))
        return g, r
    if kind == 11 and i % 36 == 23:  # int16 and bool
        r = torch.from_numpy(rng.integers(-300, 300, size=n).astype(np.int16))
        g = r.clone()
        g[:: 7] += 1
        return g, r
    if kind == 11 and i % 36 == 35:
        r = torch.from_numpy(rng.integers(0, 2, size=n).astype(np.bool_))
        g = r.clone()
        g[:: 13] = ~g[:: 13]
        return g, r
    return _fp32_noise(n, rng)


def _fp32_noise(n, rng):
    r = torch.from_numpy(rng.standard_normal(n).astype(np.float32))
    return r + torch.from_numpy((1e-6 * rng.standard_normal(n)).astype(np.float32)), r


def test_input_select_matches_oracle(kv):
    rng = np.random.default_rng(77)
    pairs = [_pair(i, rng) for i in range(300)]
    # a few strided members take the sample-array path in the same batch
    for k in range(4):
        a = torch.from_numpy(rng.standard_normal((130, 90)).astype(np.float32))
        pairs.append(((a + 1e-4).t(), a.t()))
    dev_pairs = [(g.to(DEV), r.to(DEV)) for g, r in pairs[:300]]
    dev_pairs += [(g.t().to(DEV).t(), r.t().to(DEV).t()) for g, r in pairs[300:]]
    _say("input-select batch", len(pairs))
    recs = kv.verdict_records(dev_pairs, tolerance_policy=TOL)
    for i, ((g, r), rec) in enumerate(zip(pairs, recs)):
        probs = record_vs_oracle(rec, g, r, TOL)
        abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, TOL)
        for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
            want = tv.p99_meta(vals)
            if not same_value(float(rec[k]), float(want)):
                probs.append(f"{k}: device {rec[k]!r} != oracle {want!r}")
        assert not probs, (i, i % 12, tuple(g.shape), g.dtype, probs)


def test_input_select_repeat_and_sizes(kv):
    """Two batches in a row on the same workspace sizes (the compaction counters
    start at zero each call), the second with every pair one element shorter."""
    rng = np.random.default_rng(5)
    base = [_fp32_noise(int(rng.integers(8_300, 20_000)), rng) for _ in range(280)]
    for cut in (0, 1):
        pairs = [(g[: g.numel() - cut], r[: r.numel() - cut]) for g, r in base]
        recs = kv.verdict_records([(g.to(DEV), r.to(DEV)) for g, r in pairs])
        for (g, r), rec in zip(pairs, recs):
            abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, None)
            assert same_value(float(rec["p99_abs"]), float(tv.p99_meta(abs_d))), cut
            assert same_value(float(rec["p99_rel"]), float(tv.p99_meta(rel_d))), cut


def test_input_select_strided_samples(kv):
    """max_samples below n: the chunks walk the strided sample positions
    (idx_i = i*(n-1)//(m-1)) and also carry the sampled fp64 sums."""
    rng = np.random.default_rng(91)
    ms = 9_001
    pairs = [_pair(i, rng) for i in range(280)]
    recs = kv.verdict_records([(g.to(DEV), r.to(DEV)) for g, r in pairs], tolerance_policy=TOL, max_samples=ms)
    for i, ((g, r), rec) in enumerate(zip(pairs, recs)):
        abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, TOL)
        probs = []
        for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
            want = tv.p99_meta(vals, ms)
            if not same_value(float(rec[k]), float(want)):
                probs.append(f"{k}: device {rec[k]!r} != oracle {want!r}")
        gs = tv.sample_flat_values(g.reshape(-1).double(), ms)
        rs = tv.sample_flat_values(r.reshape(-1).double(), ms)
        for k, want in (("sample_sum_gg", float((gs * gs).sum())), ("sample_sum_rr", float((rs * rs).sum())),
                        ("sample_sum_gr", float((gs * rs).sum()))):
            got = float(rec[k])
            # fp64 sums in another order; the dense members' sums come from the main pass,
            # whose 16-bit dot forms are within the declared 1e-6
            if not close(got, want, SUM_RTOL):
                probs.append(f"{k}: device {got!r} vs {want!r}")
        assert not probs, (i, i % 12, tuple(g.shape), g.dtype, probs)


def test_input_select_long_strided_pair(kv):
    """One pair of 50 M elements (10^6 strided samples, stride ~50) among 260
    smaller ones: the chunks step far-apart sample indices, and the sampled
    sums of its 31 chunks are folded in order."""
    rng = np.random.default_rng(13)
    big = _fp32_noise(50_000_000, rng)
    big[0][:: 77_777] += 0.25
    pairs = [big] + [_fp32_noise(int(rng.integers(9_000, 20_000)), rng) for _ in range(260)]
    recs = kv.verdict_records([(g.to(DEV), r.to(DEV)) for g, r in pairs], tolerance_policy=TOL)
    g, r = big
    rec = recs[0]
    abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, TOL)
    for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
        want = tv.p99_meta(vals)
        assert same_value(float(rec[k]), float(want)), (k, rec[k], want)
    gs = tv.sample_flat_values(g.double(), 1_000_000)
    rs = tv.sample_flat_values(r.double(), 1_000_000)
    for k, want in (("sample_sum_gg", float((gs * gs).sum())), ("sample_sum_rr", float((rs * rs).sum())),
                    ("sample_sum_gr", float((gs * rs).sum()))):
        assert close(float(rec[k]), want, SUM_RTOL), (k, rec[k], want)
    for (g2, r2), rec2 in zip(pairs[1:40], recs[1:40]):
        a2, _, _, _ = tv.mismatch_parts(g2, r2, TOL)
        assert same_value(float(rec2["p99_abs"]), float(tv.p99_meta(a2)))


def _pivot_positions(m):
    """The elements the capture pivot reads: 64 runs of 64, run j from (j * (m - 64)) // 63."""
    return np.concatenate([np.arange(s, s + 64) for s in ((j * (m - 64)) // 63 for j in range(64))])


def test_capture_thresholds_miss_and_edges(kv):
    """Dense members (every element a sample) have their values at or above pivot
    thresholds captured by the main pass.  Here the pivot runs misrepresent some
    pairs on purpose: thresholds above the p99 (the pair falls back to the
    input-select passes), thresholds far below it (most values captured, more
    than 8192: streamed); plus NaN and Inf away from the pivot runs, in fp32 and
    bf16, and captured values in a segment's partial last vector, between 270
    ordinary members."""
    rng = np.random.default_rng(404)
    pairs = [_fp32_noise(int(rng.integers(8_300, 20_000)), rng) for _ in range(270)]
    special = []
    for n, dt in ((200_000, torch.float32), (120_001, torch.bfloat16)):
        pos = _pivot_positions(n)
        r = rng.standard_normal(n).astype(np.float32)
        # the pivot sees only large differences: thresholds above the p99
        g = r + (1e-4 * rng.standard_normal(n)).astype(np.float32)
        g[pos] = r[pos] + np.float32(1.0) + rng.uniform(0, 1, pos.size).astype(np.float32)
        special.append((torch.from_numpy(g).to(dt), torch.from_numpy(r).to(dt)))
        # the pivot sees only tiny differences: nearly every value captured
        g = r + (1e-1 * rng.standard_normal(n)).astype(np.float32)
        g[pos] = r[pos]
        special.append((torch.from_numpy(g).to(dt), torch.from_numpy(r).to(dt)))
        # NaN and a few Inf away from the pivot runs
        away = np.setdiff1d(np.arange(n), pos)
        g = r + (1e-2 * rng.standard_normal(n)).astype(np.float32)
        g[rng.choice(away, 3, replace=False)] = np.nan
        special.append((torch.from_numpy(g).to(dt), torch.from_numpy(r).to(dt)))
        g = r + (1e-2 * rng.standard_normal(n)).astype(np.float32)
        rr = r.copy()
        inf_at = rng.choice(away, 40, replace=False)
        rr[inf_at[:20]] = np.inf            # abs_diff inf, rel_diff NaN
        g[inf_at[20:]] = -np.inf            # abs_diff inf, rel_diff inf
        special.append((torch.from_numpy(g).to(dt), torch.from_numpy(rr).to(dt)))
    # the segment ends in a partial vector whose values are all captured, in the last of a
    # lane's four vectors of an fp32 item (n % 1024 > 4 * 193): that vector is finished
    # while the wave's lane 0, whose vectors are all whole, is idle
    for n in (100 * 1024 + 907, 99 * 1024 + 1023):
        r = rng.standard_normal(n).astype(np.float32)
        g = r + (1e-3 * rng.standard_normal(n)).astype(np.float32)
        g[-3:] = r[-3:] + np.float32(10.0)
        special.append((torch.from_numpy(g), torch.from_numpy(r)))
    pairs = special + pairs
    _say("capture batch", len(pairs))
    recs = kv.verdict_records([(g.to(DEV), r.to(DEV)) for g, r in pairs], tolerance_policy=TOL)
    for i, ((g, r), rec) in enumerate(zip(pairs, recs)):
        probs = record_vs_oracle(rec, g, r, TOL) if i < len(special) else []
        abs_d, rel_d, _, _ = tv.mismatch_parts(g, r, TOL)
        for k, vals in (("p99_abs", abs_d), ("p99_rel", rel_d)):
            want = tv.p99_meta(vals)
            if not same_value(float(rec[k]), float(want)):
                probs.append(f"{k}: device {rec[k]!r} != oracle {want!r}")
        assert not probs, (i, tuple(g.shape), g.dtype, probs)
