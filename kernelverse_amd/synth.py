"""Seeded synthetic tensor pairs for the verdict workloads.

Every generator draws from numpy's PCG64 (bit-identical across machines for a
given numpy version) and casts with torch on the CPU, so a (seed, size) pair
always yields the same bytes here and on the GPU box.  ``*_device`` variants
build the same *kind* of pair directly on a GPU with torch's device generator
(fast, for benchmarking; not byte-identical to the CPU variants).

Workload shapes follow the five benchmark configurations of the verdict:

* ``fp32_noise_pair``   fp32, ref ~ N(0,1), cand = ref + N(0,1e-6), 0.1% of
  positions pushed by +U(1e-3, 1e-1).
* ``code_flip_pair``    bf16 / fp16 / fp8: cand = ref with same-sign +-k code
  steps at seeded positions (so the ULP distance of each step is exactly k).
* ``fp16_nonfinite_pair``  fp16 U(-60000, 60000) with seeded NaN/+-Inf and a
  given number of finite-pattern breaks, as a strided (row-pitched) view.
* ``int8_pair``         int8 U[-128,127], cand differs at exactly k positions.
* ``ragged_batch``      list of fp32/bf16 pairs with log-uniform sizes.
"""

from __future__ import annotations

import math
from typing import List, Tuple

import numpy as np
import torch

_CODE_INFO = {
    # dtype: (int view dtype, numpy unsigned dtype, magnitude mask, first non-finite magnitude)
    torch.bfloat16: (torch.int16, np.uint16, 0x7FFF, 0x7F80),
    torch.float16: (torch.int16, np.uint16, 0x7FFF, 0x7C00),
    torch.float8_e4m3fn: (torch.int8, np.uint8, 0x7F, 0x7F),
    torch.float8_e5m2: (torch.int8, np.uint8, 0x7F, 0x7C),
}


def _rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def _distinct_positions(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """k distinct positions in [0, n), sorted."""
    k = min(k, n)
    if k == 0:
        return np.zeros(0, dtype=np.int64)
    if k * 4 >= n:
        return np.sort(rng.permutation(n)[:k]).astype(np.int64)
    pos = np.unique(rng.integers(0, n, size=int(k * 1.3) + 16))
    while pos.size < k:
        pos = np.unique(np.concatenate([pos, rng.integers(0, n, size=k)]))
    return np.sort(rng.permutation(pos)[:k]).astype(np.int64)


def fp32_noise_pair(n: int, seed: int, noise: float = 1e-6, frac: float = 1e-3,
                    lo: float = 1e-3, hi: float = 1e-1) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cand, ref) fp32: ref ~ N(0,1); cand = ref + N(0,noise); frac of positions get +U(lo,hi)."""
    rng = _rng(seed)
    ref = rng.standard_normal(n, dtype=np.float32)
    cand = ref + (rng.standard_normal(n, dtype=np.float32) * np.float32(noise))
    pos = _distinct_positions(rng, n, int(round(n * frac)))
    cand[pos] += rng.uniform(lo, hi, size=pos.size).astype(np.float32)
    return torch.from_numpy(cand), torch.from_numpy(ref)


def step_codes(ref: torch.Tensor, positions: np.ndarray, steps: np.ndarray, rng: np.random.Generator) -> torch.Tensor:
    """Copy of ``ref`` whose codes at ``positions`` move by ``steps`` code units of magnitude.

    The sign bit is kept and the direction is random but chosen so that the
    new magnitude stays finite and non-negative: the ULP distance of every
    moved element to its original is exactly its step.
    """
    view, npu, mag_mask, nonfinite = _CODE_INFO[ref.dtype]
    codes = ref.contiguous().view(view).numpy().view(npu).copy()
    c = codes[positions].astype(np.int64)
    sign = c & ~mag_mask
    mag = c & mag_mask
    up = rng.integers(0, 2, size=positions.size).astype(bool)
    new_up = mag + steps
    new_dn = mag - steps
    go_up = np.where(up, new_up < nonfinite, new_dn < 0)
    go_up &= new_up < nonfinite
    new = np.where(go_up, new_up, new_dn)
    codes[positions] = (sign | new).astype(npu)
    out = torch.from_numpy(codes.view(np.int16 if npu == np.uint16 else np.int8).copy()).view(ref.dtype)
    return out.reshape(ref.shape)


def code_flip_pair(n: int, seed: int, dtype: torch.dtype = torch.bfloat16, std: float = 2.0,
                   p1: float = 0.05, p3: float = 1e-4, clamp: float = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cand, ref): ref = dtype(N(0,std)); cand moves disjoint positions by 1 code (fraction p1) or 3 codes (p3)."""
    rng = _rng(seed)
    x = rng.standard_normal(n, dtype=np.float32) * np.float32(std)
    if clamp is not None:
        np.clip(x, -clamp, clamp, out=x)
    ref = torch.from_numpy(x).to(dtype)
    k1 = int(round(n * p1))
    k3 = int(round(n * p3))
    pos = _distinct_positions(rng, n, k1 + k3)
    perm = rng.permutation(pos.size)
    steps = np.ones(pos.size, dtype=np.int64)
    steps[perm[:k3]] = 3
    cand = step_codes(ref, pos, steps, rng)
    return cand, ref


def fp16_nonfinite_pair(rows: int, cols: int, row_stride: int, seed: int, p_nan: float = 5e-4,
                        p_inf: float = 5e-4, breaks: int = 17) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cand, ref) fp16 views of shape (rows, cols) with strides (row_stride, 1).

    ref ~ U(-60000, 60000) with seeded NaN and +-Inf; cand copies ref (pattern
    included) except at ``breaks`` seeded positions whose finite/NaN/Inf class
    is changed.  The padding columns hold values that must never be read.
    """
    rng = _rng(seed)
    n = rows * cols
    vals = rng.uniform(-60000.0, 60000.0, size=n).astype(np.float32)
    k_nan = int(round(n * p_nan))
    k_inf = int(round(n * p_inf))
    pos = _distinct_positions(rng, n, k_nan + k_inf)
    perm = rng.permutation(pos.size)
    nan_pos = pos[perm[:k_nan]]
    inf_pos = pos[perm[k_nan:]]
    vals[nan_pos] = np.nan
    vals[inf_pos] = np.where(rng.integers(0, 2, size=inf_pos.size) == 1, np.inf, -np.inf)
    ref_logical = vals.astype(np.float16)
    cand_logical = ref_logical.copy()
    bpos = _distinct_positions(rng, n, breaks)
    for j, p in enumerate(bpos):
        v = ref_logical[p]
        if np.isnan(v):
            cand_logical[p] = np.float16(1.0) if j % 2 else np.float16(np.inf)
        elif np.isinf(v):
            cand_logical[p] = np.float16(np.nan) if j % 2 else -v
        else:
            cand_logical[p] = np.float16(np.nan) if j % 2 else np.float16(np.inf)
    out = []
    for logical, pad_val in ((cand_logical, 7.0), (ref_logical, -7.0)):
        base = np.full((rows, row_stride), pad_val, dtype=np.float16)
        base[:, :cols] = logical.reshape(rows, cols)
        t = torch.from_numpy(base.reshape(-1).copy())
        out.append(t.as_strided((rows, cols), (row_stride, 1)))
    return out[0], out[1]


def int8_pair(n: int, seed: int, changed: int = 1000) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cand, ref) int8: ref ~ U[-128,127]; cand differs from ref at exactly ``changed`` positions."""
    rng = _rng(seed)
    ref = rng.integers(-128, 128, size=n, dtype=np.int16).astype(np.int8)
    cand = ref.copy()
    pos = _distinct_positions(rng, n, changed)
    delta = rng.integers(1, 256, size=pos.size)
    cand[pos] = ((ref[pos].astype(np.int16) + 128 + delta) % 256 - 128).astype(np.int8)
    return torch.from_numpy(cand), torch.from_numpy(ref)


def fp8_pair(n: int, seed: int, p: float = 0.02, std: float = 4.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cand, ref) float8_e4m3fn: ref = e4m3(clamp(N(0,std), +-448)); cand moves a fraction p by one code."""
    return code_flip_pair(n, seed, dtype=torch.float8_e4m3fn, std=std, p1=p, p3=0.0, clamp=448.0)


def ragged_sizes(count: int, seed: int, lo: int = 1024, hi: int = 1 << 20) -> List[int]:
    """Log-uniform integer sizes in [lo, hi]."""
    rng = _rng(seed)
    u = rng.uniform(math.log(lo), math.log(hi), size=count)
    return [int(min(hi, max(lo, round(math.exp(v))))) for v in u]


RAGGED_TOLERANCES = ({"rtol": 1e-5, "atol": 1e-5}, {"rtol": 1.6e-2, "atol": 1e-2},
                     {"rtol": 1e-3, "atol": 1e-4}, {"rtol": 5e-4, "atol": 5e-4})


def ragged_batch(count: int, seed: int, lo: int = 1024, hi: int = 1 << 20):
    """List of (cand, ref, tolerance) with dtype alternating fp32 / bf16 and the fp32 noise model; pair i takes
    RAGGED_TOLERANCES[(i // 2) % 4], so each dtype cycles through all four."""
    sizes = ragged_sizes(count, seed, lo, hi)
    out = []
    for i, n in enumerate(sizes):
        cand, ref = fp32_noise_pair(n, seed * 100003 + i)
        if i % 2:
            cand, ref = cand.to(torch.bfloat16), ref.to(torch.bfloat16)
        out.append((cand, ref, dict(RAGGED_TOLERANCES[(i // 2) % len(RAGGED_TOLERANCES)])))
    return out


# ------------------------------------------------------------ device variants
def code_flip_pair_device(n: int, seed: int, device, dtype=torch.bfloat16, std: float = 2.0,
                          p1: float = 0.05, p3: float = 1e-4, clamp: float = None):
    """Device-side analogue of ``code_flip_pair`` (same statistics, different bytes)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(n, generator=gen, device=device, dtype=torch.float32) * std
    if clamp is not None:
        x.clamp_(-clamp, clamp)
    ref = x.to(dtype)
    del x
    view, _, mag_mask, nonfinite = _CODE_INFO[dtype]
    u = torch.rand(n, generator=gen, device=device)
    steps = torch.where(u < p3, 3, torch.where(u < p3 + p1, 1, 0)).to(torch.int32)
    del u
    codes = ref.view(view).to(torch.int32) & ((mag_mask << 1) | 1)
    sign = codes & ~mag_mask
    mag = codes & mag_mask
    up = mag + steps
    new = torch.where(up < nonfinite, up, mag - steps)
    cand_codes = (sign | new)
    cand_codes = torch.where(cand_codes > mag_mask, cand_codes - (2 * (mag_mask + 1)), cand_codes)
    cand = cand_codes.to(view).view(dtype)
    return cand, ref


# ------------------------------------------------------------ benchmark configurations
# The five workloads of the verdict benchmark, generated on the device from fixed seeds.

def c1_pair(device, p1: float = 0.05):
    """C1: bf16, 268,435,456 elements; ref = bf16(N(0,2)); cand = ref with 1-ULP steps at 5% (or `p1`) and 3-ULP
    at 0.01%.  p1 = 0.5 is the C1 shape with half of all elements moved (outputs of GEMM-like operators differ
    almost everywhere, so under the tolerant policy most near-zero elements carry a nonzero abs_diff)."""
    return code_flip_pair_device(268_435_456, seed=1, device=device, dtype=torch.bfloat16, std=2.0, p1=p1, p3=1e-4)


# The 17 finite-pattern breaks of C2, by kind: (reference class, candidate value).
C2_BREAKS = (("nan", 1.0), ("nan", 1.0), ("nan", 1.0), ("nan", 1.0),
             ("inf", 1.0), ("inf", 1.0), ("inf", 1.0),
             ("inf", "negated"), ("inf", "negated"), ("inf", "negated"), ("inf", "negated"),
             ("finite", float("nan")), ("finite", float("nan")), ("finite", float("nan")),
             ("nan", float("inf")), ("nan", float("inf")), ("nan", float("-inf")))


def c2_pair(device, rows: int = 4096, cols: int = 32768, stride: int = 32896, seed: int = 2):
    """C2: fp16 (rows, cols) views with row stride `stride`; ref ~ U(-60000, 60000) with 0.05% NaN and 0.05% +-Inf
    (either sign); the candidate copies the reference except at 17 seeded positions whose class it breaks
    (``C2_BREAKS``): NaN or +-Inf replaced by 1.0, +-Inf negated, a finite value replaced by NaN, NaN replaced by
    +-Inf.  Every break is one finite-pattern violation."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    base_r = (torch.rand(rows, stride, generator=gen, device=device) * 120000.0 - 60000.0).to(torch.float16)
    u = torch.rand(rows, stride, generator=gen, device=device)
    sign = torch.rand(rows, stride, generator=gen, device=device) < 0.5
    base_r[u < 5e-4] = float("nan")
    inf = (u >= 5e-4) & (u < 1e-3)
    base_r[inf & sign] = float("inf")
    base_r[inf & ~sign] = float("-inf")
    del u, sign, inf
    base_g = base_r.clone()
    flat = base_r[:, :cols].reshape(-1)
    pools = {"nan": torch.nonzero(torch.isnan(flat)).reshape(-1), "inf": torch.nonzero(torch.isinf(flat)).reshape(-1)}
    cand = torch.randint(0, rows * cols, (4096,), generator=gen, device=device)
    pools["finite"] = cand[torch.isfinite(flat[cand])].unique()
    for kind in pools:
        pools[kind] = pools[kind][torch.randperm(pools[kind].numel(), generator=gen, device=device)]
    taken = {k: 0 for k in pools}
    for kind, value in C2_BREAKS:
        p = pools[kind][taken[kind]]
        taken[kind] += 1
        row, col = p // cols, p % cols
        base_g[row, col] = -base_r[row, col] if value == "negated" else value
    return base_g[:, :cols], base_r[:, :cols]


def c3_fp8_pair(device):
    """C3 fp8: e4m3fn, 134,217,728 elements; ref from N(0,4) clamped to +-448; cand = ref +- 1 code at 2%."""
    return code_flip_pair_device(134_217_728, seed=3, device=device, dtype=torch.float8_e4m3fn, std=4.0,
                                 p1=0.02, p3=0.0, clamp=448.0)


def c3_int8_pair(device, n: int = 134_217_728, changed: int = 1000, seed: int = 4):
    """C3 int8: ref ~ U[-128, 127]; cand equal except `changed` distinct seeded positions (each moved by 77)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    r = torch.randint(-128, 128, (n,), generator=gen, device=device, dtype=torch.int8)
    g = r.clone()
    pos = torch.randperm(n, generator=gen, device=device)[:changed]
    g[pos] = (g[pos].to(torch.int16) + 77).to(torch.int8)
    return g, r


# C4's per-pair tolerances: pair i takes entry (i // 2) % 4 of its dtype's list (fp32 pairs are the even
# ones), so neighbouring pairs of one dtype in a batch never share a tolerance.
C4_TOLERANCES = {
    "FP32": ({"rtol": 1e-5, "atol": 1e-5}, {"rtol": 1.3e-6, "atol": 1e-5}, {"rtol": 5e-4, "atol": 5e-4},
             {"rtol": 1e-4, "atol": 1e-6}),
    "BF16": ({"rtol": 1.6e-2, "atol": 1e-2}, {"rtol": 1.6e-2, "atol": 1e-3}, {"rtol": 1e-2, "atol": 1e-2},
             {"rtol": 5e-3, "atol": 1e-3}),
}


def c4_tolerance(i: int) -> dict:
    """The tolerance table of C4's pair i: its dtype's entry (i // 2) % 4."""
    name = "BF16" if i % 2 else "FP32"
    return {name: dict(C4_TOLERANCES[name][(i // 2) % 4])}


def c4_batch(device, count: int = 4096, seed: int = 5, gen_device=None):
    """C4: `count` pairs, dtype alternating fp32 / bf16, sizes log-uniform in [1024, 2^20], the C0 noise model
    (ref ~ N(0,1); cand = ref + N(0,1e-6); 0.1% of positions + U(1e-3, 1e-1)); each pair is its own allocation
    with its own tolerances (``c4_tolerance``).  `gen_device` (default `device`) draws the values there and
    moves them to `device` (same model, other bytes: the host draw runs no generator kernels on the GPU).
    Returns [(cand, ref, tolerance)]."""
    sizes = ragged_sizes(count, seed)
    gdev = device if gen_device is None else gen_device
    gen = torch.Generator(device=gdev)
    gen.manual_seed(seed)
    out = []
    for i, n in enumerate(sizes):
        ref = torch.randn(n, generator=gen, device=gdev)
        cand = ref + 1e-6 * torch.randn(n, generator=gen, device=gdev)
        hit = torch.rand(n, generator=gen, device=gdev) < 1e-3
        cand = torch.where(hit, cand + (1e-3 + (1e-1 - 1e-3) * torch.rand(n, generator=gen, device=gdev)), cand)
        if i % 2:
            cand, ref = cand.to(torch.bfloat16), ref.to(torch.bfloat16)
        out.append((cand.to(device), ref.to(device), c4_tolerance(i)))
    return out
