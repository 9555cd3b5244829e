"""The drop-in keeps one workspace and pinned record buffer per (device, stream) between calls
(needs an MI355X).  Calls of different sizes, policies and streams in a row give the same metas
as calls on freshly allocated buffers, and the same as the oracle."""

import sys

import pytest
import torch

from oracle import torch_verdict as tv
from parity_util import meta_problems

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _pairs():
    from kernelverse_amd import synth
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    tolerant = resolve_correctness_policy({"category": "gemm", "op_name": "x"})
    strict = resolve_correctness_policy({"category": "activation", "op_name": "x"})
    g0, r0 = synth.fp32_noise_pair(1 << 20, seed=11)
    g1, r1 = synth.code_flip_pair(1000, seed=12)
    g2, r2 = synth.code_flip_pair(3_000_000, seed=13, std=0.4, p1=0.1)
    g3, r3 = synth.code_flip_pair(10, seed=14, dtype=torch.float16)
    return [("fp32 1Mi strict", g0, r0, strict), ("bf16 1000 strict", g1, r1, strict),
            ("bf16 3M tolerant", g2, r2, tolerant), ("fp16 10 tolerant", g3, r3, tolerant),
            ("fp32 1Mi again", g0, r0, strict)]


def test_reused_buffers_match_fresh_ones_and_the_oracle():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    from kernelverse_amd import _lib, verdict
    _lib.load()
    pairs = _pairs()
    side = torch.cuda.Stream()
    for name, g, r, pol in pairs:
        _say("drop-in buffers:", name)
        gd, rd = g.to(DEV), r.to(DEV)
        torch.cuda.synchronize()
        reused = verdict._compare_tensors(gd, rd, "output", None, pol)
        with torch.cuda.stream(side):
            other = verdict._compare_tensors(gd, rd, "output", None, pol)
        verdict.release_buffers()
        fresh = verdict._compare_tensors(gd, rd, "output", None, pol)
        assert reused == fresh, name
        assert other == fresh, name
        want = tv.compare_tensors(g, r, "output", None, pol)
        assert reused[0] == want[0] and reused[1] == want[1], name
        probs = meta_problems(reused[2], want[2], g, r)
        assert not probs, (name, probs)
    assert len(verdict._BUFFERS) >= 1
    verdict.release_buffers()
    assert not verdict._BUFFERS
