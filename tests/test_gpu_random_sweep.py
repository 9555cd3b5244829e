"""Seeded random sweep of the device verdict against the CPU oracle (needs an MI355X).

Each case draws a dtype, a shape (numel from 0 up to ~400 K, often not a
multiple of any vector width), a layout (contiguous, transposed, strided slice,
misaligned start), a perturbation (identical, noise, code steps, NaN/Inf
injection, sign flips) and a tolerance policy and sample cap; the device
record and meta must match the oracle's (``parity_util``: exact integers,
indices, maxima and p99; fp64 sums within 1e-6).
"""

import sys

import numpy as np
import pytest
import torch

from parity_util import meta_problems, record_vs_oracle
from oracle import torch_verdict as tv

pytestmark = pytest.mark.gpu

DEV = "cuda"
N_CASES = 240

FLOATS = [torch.float32, torch.bfloat16, torch.float16, torch.float64]
FP8 = [torch.float8_e4m3fn, torch.float8_e5m2]
INTS = [torch.int8, torch.uint8, torch.int16, torch.int32, torch.int64, torch.bool]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _shape(rng):
    kind = rng.integers(0, 6)
    if kind == 0:
        return (int(rng.integers(0, 5)),)                       # tiny, possibly empty
    if kind == 1:
        return (int(rng.integers(1, 400_000)),)
    if kind == 2:
        return (int(rng.integers(1, 700)), int(rng.integers(1, 700)))
    if kind == 3:
        return tuple(int(x) for x in rng.integers(1, 40, size=3))
    if kind == 4:
        return (int(rng.integers(1, 9)), int(rng.integers(1, 200)), int(rng.integers(1, 300)))
    return (int(rng.integers(1, 3000)), 64)


def _values(rng, dtype, n):
    if dtype == torch.bool:
        return torch.from_numpy(rng.integers(0, 2, size=n).astype(np.bool_))
    if dtype in INTS:
        info = torch.iinfo(dtype)
        lo, hi = max(info.min, -2**40), min(info.max, 2**40)
        return torch.from_numpy(rng.integers(lo, hi, size=n, endpoint=True)).to(dtype)
    scale = float(10.0 ** rng.integers(-3, 4))
    x = torch.from_numpy(rng.standard_normal(n).astype(np.float64) * scale)
    if dtype == torch.float8_e4m3fn:
        x = x.clamp(-448, 448)
    if dtype == torch.float8_e5m2:
        x = x.clamp(-57344, 57344)
    return x.to(dtype)


def _perturb(rng, dtype, ref):
    g = ref.clone()
    n = g.numel()
    if n == 0:
        return g
    how = rng.integers(0, 5)
    flat = g.view(-1)
    if how == 0:
        return g                                                # identical
    if dtype == torch.bool:
        idx = torch.from_numpy(rng.choice(n, size=max(1, n // 50), replace=True))
        flat[idx] = ~flat[idx]
        return g
    if dtype in INTS:
        idx = torch.from_numpy(rng.choice(n, size=max(1, n // 20), replace=True))
        flat[idx] = flat[idx] + torch.from_numpy(rng.integers(-3, 4, size=idx.numel())).to(dtype)
        return g
    if how == 1:                                                # relative noise
        noise = torch.from_numpy(rng.standard_normal(n)) * float(10.0 ** rng.integers(-7, -1))
        return (ref.double().view(-1) * (1 + noise)).to(dtype).view(ref.shape)
    if how == 2:                                                # code steps
        bits = {torch.float32: torch.int32, torch.float64: torch.int64, torch.bfloat16: torch.int16,
                torch.float16: torch.int16, torch.float8_e4m3fn: torch.int8, torch.float8_e5m2: torch.int8}[dtype]
        codes = g.view(bits).view(-1)
        idx = torch.from_numpy(rng.choice(n, size=max(1, n // 10), replace=True))
        step = torch.from_numpy(rng.integers(-3, 4, size=idx.numel())).to(bits)
        codes[idx] = codes[idx] + step
        return g
    if how == 3:                                                # NaN / Inf injections (both sides sometimes)
        k = max(1, n // 100)
        idx = torch.from_numpy(rng.choice(n, size=k, replace=True))
        vals = [float("nan"), float("inf"), float("-inf")]
        if dtype == torch.float8_e4m3fn:
            vals = [float("nan")]
        flat[idx] = torch.tensor([vals[i % len(vals)] for i in range(k)], dtype=torch.float64).to(dtype)
        if rng.integers(0, 2):
            ref.view(-1)[idx[: k // 2]] = flat[idx[: k // 2]]
        return g
    return (-g.double()).to(dtype).view(ref.shape)             # sign flip everywhere


def _layout(rng, g):
    """A layout to apply to both tensors where they live (the device copy of a
    view would be contiguous and aligned): transposed, strided or misaligned."""
    how = int(rng.integers(0, 4))
    step = int(rng.integers(2, 4))
    if how == 1 and g.dim() >= 2:
        return lambda t: t.transpose(0, 1)
    if how == 2 and g.numel() > 8:
        return lambda t: t.view(-1)[::step]
    if how == 3 and g.numel() > 2:
        return lambda t: t.view(-1)[1:]
    return lambda t: t


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    pool = FLOATS * 3 + FP8 + INTS
    dtype = pool[int(rng.integers(0, len(pool)))]
    shape = _shape(rng)
    n = int(np.prod(shape)) if shape else 1
    ref = _values(rng, dtype, n).view(shape)
    gen = _perturb(rng, dtype, ref)
    layout = _layout(rng, gen)
    tol = None
    if dtype in FLOATS and rng.integers(0, 3) == 0:
        name = {torch.float32: "FP32", torch.bfloat16: "BF16", torch.float16: "FP16", torch.float64: "FLOAT64"}[dtype]
        tol = {name: {"rtol": float(10.0 ** rng.integers(-6, -1)), "atol": float(10.0 ** rng.integers(-6, -1))}}
    max_samples = [1_000_000, 1_000_000, 997, 37][int(rng.integers(0, 4))]
    return dtype, gen, ref, layout, tol, max_samples


@pytest.fixture(scope="module")
def kv():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    from kernelverse_amd import _lib, verdict
    _lib.load()
    return verdict


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_case_matches_oracle(kv, seed):
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    dtype, g0, r0, layout, tol, max_samples = _case(seed)
    g, r = layout(g0), layout(r0)
    gd, rd = layout(g0.to(DEV)), layout(r0.to(DEV))
    _say("sweep", seed, dtype, tuple(gd.shape), tuple(gd.stride()), gd.storage_offset(), tol, max_samples)
    if g.numel() > 0:
        rec = kv.verdict_record(gd, rd, tolerance_policy=tol, max_samples=max_samples)
        probs = record_vs_oracle(rec, g, r, tol, max_samples)
        assert not probs, probs
    if dtype in FP8:
        return  # the reference raises on float8 metas (pinned by the fixtures)
    pol = resolve_correctness_policy({"category": ["gemm", "attention", "activation"][seed % 3], "op_name": "x"})
    want = tv.compare_tensors(g, r, "output", tol, pol, max_samples=max_samples)
    got = kv._compare_tensors(gd, rd, "output", tol, pol, max_samples=max_samples)
    probs = meta_problems(got[2], want[2], g, r, max_samples)
    assert not probs, probs
    assert got[0] == want[0]
    assert got[1] == want[1]
