"""KVV_FLAG_WS_KEPT: consecutive verdicts on one workspace (needs an MI355X).

Every single-pair verdict leaves its select slots clear (the final read-off
zeroes what it read); with KVV_FLAG_WS_KEPT the next verdict on the same
workspace skips the clearing launch when its slots lie where the previous
call's did, and clears them otherwise (a different layout, a batch call in
between, the first call).  Each record of a sequence on one shared workspace
must equal, field by field, the record of the same verdict on a fresh workspace
without the flag: sizes that move the slots, NaN groups (level 1 returns
early), the tolerant policy's near-zero sample (the third slot), int8 with its
p99 in the zeros, strided samples and a batch call in between.
"""

import ctypes
import math
import sys

import numpy as np
import pytest
import torch

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


def _pairs():
    from kernelverse_amd import synth
    rng = np.random.default_rng(404)
    out = []
    g, r = synth.code_flip_pair(3_000_000, seed=41)
    out.append(("bf16 3M", g, r, "strict"))
    r32 = torch.from_numpy(rng.standard_normal(2_000_000).astype(np.float32))
    g32 = r32 + torch.from_numpy((1e-3 * rng.standard_normal(2_000_000)).astype(np.float32))
    out.append(("fp32 2M", g32, r32, "strict"))
    g2 = g32.clone()
    g2[::777] = float("nan")
    out.append(("fp32 2M NaN", g2, r32, "strict"))
    g, r = synth.code_flip_pair(1_500_000, seed=42, std=0.3, p1=0.2)
    out.append(("bf16 1.5M tolerant", g, r, "tolerant"))
    i8 = torch.from_numpy(rng.integers(-100, 100, size=5_000_000).astype(np.int8))
    j8 = i8.clone()
    j8[torch.from_numpy(rng.choice(i8.numel(), size=500, replace=False))] += 2
    out.append(("int8 5M", j8, i8, "strict"))
    g, r = synth.code_flip_pair(9_000_000, seed=43)
    out.append(("bf16 9M strided samples", g, r, "strict"))
    out.append(("bf16 3M again", *out[0][1:3], "strict"))
    return out


def _policy(name):
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    cat = {"strict": "activation", "tolerant": "gemm"}[name]
    return resolve_correctness_policy({"category": cat, "op_name": "x"})


def _call(kv, g, r, pol, ws, flags):
    from kernelverse_amd import _lib
    lib = _lib.load()
    job = kv._Job(g, r, "output", None, pol, kv.MAX_SAMPLES)
    job.kpolicy.flags |= flags
    gt, rt, held = kv._device_views(g, r)
    size = ctypes.c_size_t()
    _lib.check(lib.kvv_workspace_size(gt, rt, job.kpolicy, ctypes.byref(size)), "kvv_workspace_size")
    if ws is None:
        ws = torch.empty(size.value, dtype=torch.uint8, device=DEV)
    assert ws.numel() >= size.value
    out = torch.empty(ctypes.sizeof(_lib.KvvResult), dtype=torch.uint8, pin_memory=True)
    _lib.check(lib.kvv_verdict(gt, rt, job.kpolicy, out.data_ptr(), ws.data_ptr(), size.value,
                               torch.cuda.current_stream().cuda_stream), "kvv_verdict")
    torch.cuda.current_stream().synchronize()
    del held
    return _lib.KvvResult.from_buffer_copy(out.numpy().tobytes()).to_dict()


def _same(a, b):
    bad = []
    for k in a:
        x, y = a[k], b[k]
        if isinstance(x, float) and math.isnan(x) and isinstance(y, float) and math.isnan(y):
            continue
        if x != y:
            bad.append(f"{k}: {x!r} vs {y!r}")
    return bad


def test_sequence_on_one_workspace(kv):
    from kernelverse_amd import _lib
    pairs = [(n, g.to(DEV), r.to(DEV), p) for n, g, r, p in _pairs()]
    shared = torch.empty(256 << 20, dtype=torch.uint8, device=DEV)
    fresh = {}
    for n, g, r, p in pairs:
        fresh[n] = _call(kv, g, r, _policy(p), None, 0)
    # the shared workspace in order, then again (each layout follows a different one)
    for rnd in range(2):
        for n, g, r, p in pairs:
            _say("kept workspace:", rnd, n)
            got = _call(kv, g, r, _policy(p), shared, _lib.FLAG_WS_KEPT)
            assert got["status"] == 0
            bad = _same(got, fresh[n])
            assert not bad, (rnd, n, bad)
    # a batch call on the same workspace voids the record; the next single call clears again
    recs = kv.verdict_records([(pairs[0][1], pairs[0][2]), (pairs[1][1], pairs[1][2])])
    assert recs[0]["mismatch_count"] == fresh[pairs[0][0]]["mismatch_count"]
    from kernelverse_amd import _lib as L
    lib = L.load()
    gts = [kv._kvv_tensor(pairs[k][1]) for k in (0, 1)]
    rts = [kv._kvv_tensor(pairs[k][2]) for k in (0, 1)]
    pols = [kv._Job(pairs[k][1], pairs[k][2], "o", None, None, kv.MAX_SAMPLES).kpolicy for k in (0, 1)]
    GA, PA = L.KvvTensor * 2, L.KvvPolicy * 2
    size = ctypes.c_size_t()
    L.check(lib.kvv_batch_workspace_size(2, GA(*gts), GA(*rts), PA(*pols), ctypes.byref(size)), "ws")
    assert size.value <= shared.numel()
    out = torch.empty(2 * ctypes.sizeof(L.KvvResult), dtype=torch.uint8, pin_memory=True)
    L.check(lib.kvv_verdict_batch(2, GA(*gts), GA(*rts), PA(*pols), out.data_ptr(), shared.data_ptr(), size.value,
                                  torch.cuda.current_stream().cuda_stream), "batch")
    torch.cuda.current_stream().synchronize()
    for n, g, r, p in pairs[:2]:
        _say("kept workspace after a batch:", n)
        got = _call(kv, g, r, _policy(p), shared, L.FLAG_WS_KEPT)
        bad = _same(got, fresh[n])
        assert not bad, ("after batch", n, bad)


def test_dropin_repeats_match_oracle(kv):
    """The drop-in reuses its workspace and passes the flag from the second call on."""
    from oracle import torch_verdict as tv
    from parity_util import meta_problems
    from kernelverse_amd import synth
    g, r = synth.code_flip_pair(2_500_000, seed=44)
    want = tv.compare_tensors(g, r, "output", None, None)
    gd, rd = g.to(DEV), r.to(DEV)
    for k in range(3):
        got = kv._compare_tensors(gd, rd, "output", None, None)
        probs = meta_problems(got[2], want[2], g, r)
        assert not probs, (k, probs)
        assert got[0] == want[0]


def _near_pair(n, near_frac, seed):
    """bf16 pair whose reference has about near_frac of its values at |x| <= 0.25 (the
    tolerant policy's near-zero band) and the rest at 1 <= |x| <= 4; 30% of all
    positions are moved by one code, so near-zero elements carry nonzero abs_diffs."""
    from kernelverse_amd import synth
    rng = np.random.default_rng(seed)
    big = rng.uniform(1.0, 4.0, size=n) * rng.choice([-1.0, 1.0], size=n)
    small = rng.uniform(-0.25, 0.25, size=n)
    ref = torch.from_numpy(np.where(rng.random(n) < near_frac, small, big).astype(np.float32)).to(torch.bfloat16)
    pos = np.sort(rng.choice(n, size=int(0.3 * n), replace=False))
    gen = synth.step_codes(ref, pos, np.ones(pos.size, dtype=np.int64), rng)
    return gen, ref


def test_tolerant_small_then_large_near_zero_sample(kv):
    """A tolerant verdict whose abs/rel sample is a large group but whose near-zero
    sample is small (selected in one block, its select slot never used), then one of
    the same shape whose near-zero sample is large, on one kept workspace: the second
    must not read anything the first left in the near-zero slot."""
    from kernelverse_amd import _lib
    from oracle import torch_verdict as tv
    from parity_util import meta_problems
    pol = _policy("tolerant")
    small = _near_pair(100_000, 0.05, 901)    # ~5k near-zero refs: <= 8192 samples
    large = _near_pair(100_000, 0.40, 902)    # ~40k near-zero refs
    seq = [("small", *small), ("large", *large), ("small again", *small), ("large again", *large)]
    dev = {n: (g.to(DEV), r.to(DEV)) for n, g, r in seq}
    near_counts = {}
    shared = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    flags = 0
    for n, g, r in seq:
        _say("tolerant near-zero sample on a kept workspace:", n)
        gd, rd = dev[n]
        fresh = _call(kv, gd, rd, pol, None, 0)
        got = _call(kv, gd, rd, pol, shared, flags)
        flags = _lib.FLAG_WS_KEPT
        assert got["status"] == 0 and fresh["status"] == 0
        bad = _same(got, fresh)
        assert not bad, (n, bad)
        near_counts[n] = got["near_zero_count"]
    assert near_counts["small"] <= 8192 < near_counts["large"], near_counts
    # the drop-in keeps its workspace and passes the flag from its second call on
    for n, g, r in seq:
        _say("drop-in tolerant near-zero sample:", n)
        gd, rd = dev[n]
        want = tv.compare_tensors(g, r, "output", None, pol)
        got = kv._compare_tensors(gd, rd, "output", None, pol)
        probs = meta_problems(got[2], want[2], g, r)
        assert not probs, (n, probs)
