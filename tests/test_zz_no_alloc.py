"""kvv_verdict_noalloc against kvv_verdict, through the C ABI (needs an MI355X).

The no-alloc entry point runs the same plan and kernels as kvv_verdict on the
library's fixed per-device scratch array instead of a caller workspace, so
its record must equal kvv_verdict's bit for bit.  Calls follow each other on
one GPU and share that array: the second call has a smaller input and must
not see the first call's leftovers (select histograms, counters, samples).
"""

import ctypes
import math
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    from kernelverse_amd import _lib
    return _lib.load()


def _records(lib, g, r, tol, policy=None, max_samples=1_000_000):
    """(kvv_verdict record with a torch workspace, kvv_verdict_noalloc record) of one pair."""
    from kernelverse_amd import _lib, verdict
    job = verdict._Job(g, r, "output", tol, policy, max_samples, fp8_errors=False)
    gt, rt, held = verdict._device_views(g, r)
    size = ctypes.c_size_t()
    _lib.check(lib.kvv_workspace_size(gt, rt, job.kpolicy, ctypes.byref(size)), "kvv_workspace_size")
    assert size.value <= _lib.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(size.value, dtype=torch.uint8, device=DEV)
    rec_size = ctypes.sizeof(_lib.KvvResult)
    out = torch.empty(2 * rec_size, dtype=torch.uint8, pin_memory=True)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.kvv_verdict(gt, rt, job.kpolicy, out.data_ptr(), ws.data_ptr(), size.value, stream), "kvv_verdict")
    _lib.check(lib.kvv_verdict_noalloc(gt, rt, job.kpolicy, out.data_ptr() + rec_size, stream), "kvv_verdict_noalloc")
    torch.cuda.current_stream().synchronize()
    host = out.numpy().tobytes()
    del held
    return (_lib.KvvResult.from_buffer_copy(host, 0).to_dict(), _lib.KvvResult.from_buffer_copy(host, rec_size).to_dict())


def _same(a, b):
    bad = []
    for k in a:
        x, y = a[k], b[k]
        if isinstance(x, float) and math.isnan(x) and isinstance(y, float) and math.isnan(y):
            continue
        if x != y:
            bad.append(f"{k}: kvv_verdict {x!r} != kvv_verdict_noalloc {y!r}")
    return bad


def test_noalloc_matches_workspace_entry_on_consecutive_calls(lib):
    from kernelverse_amd import synth
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    tolerant = resolve_correctness_policy({"category": "gemm", "op_name": "x"})
    calls = [
        # large: strided sample walk, three select levels, the near-zero sample of the tolerant policy
        ("bf16 4M tolerant", *synth.code_flip_pair(4_194_304, seed=61), {"BF16": {"rtol": 1e-3, "atol": 1e-4}},
         tolerant),
        # smaller, on the scratch the first call left behind: dense samples, fp32
        ("fp32 300k strict", *synth.fp32_noise_pair(300_000, seed=62), {"FP32": {"rtol": 1e-5, "atol": 1e-5}},
         None),
        # smaller still, under the select-in-one-block size
        ("fp32 5000 strict", *synth.fp32_noise_pair(5_000, seed=63), None, None),
    ]
    for name, g, r, tol, pol in calls:
        _say("noalloc", name)
        a, b = _records(lib, g.to(DEV), r.to(DEV), tol, pol)
        bad = _same(a, b)
        assert not bad, (name, bad)
        assert a["numel"] == g.numel() and a["mismatch_count"] > 0


def test_noalloc_rejects_a_verdict_beyond_its_scratch(lib):
    from kernelverse_amd import _lib, verdict
    n = 10_000_000  # 10 M samples of abs and rel: 80 MB of sample arrays alone
    g = torch.zeros(n, dtype=torch.bfloat16, device=DEV)
    job = verdict._Job(g, g, "output", None, None, n)
    gt, rt, _ = verdict._device_views(g, g)
    out = torch.empty(ctypes.sizeof(_lib.KvvResult), dtype=torch.uint8, pin_memory=True)
    rc = lib.kvv_verdict_noalloc(gt, rt, job.kpolicy, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == -2
    assert f"no-alloc entry point holds {_lib.NOALLOC_SCRATCH_BYTES}".encode() in lib.kvv_last_error()


def test_noalloc_captured_graphs_alternate_with_eager_calls(lib):
    """kvv_verdict_noalloc captured into HIP graphs (torch.cuda.graph) for two layouts;
    the graphs are replayed alternately, with eager no-alloc calls of the other layout
    and synchronisations in between, and every replay's record must equal kvv_verdict's
    on a fresh workspace.  The eager calls and the other graph write the shared scratch
    between replays, so a graph that skipped its slot clearing would read their leftovers."""
    from kernelverse_amd import _lib, synth, verdict
    from kernelverse_amd.correctness_policy import resolve_correctness_policy
    tolerant = resolve_correctness_policy({"category": "gemm", "op_name": "x"})
    cases = {
        "A bf16 3M tolerant": (*synth.code_flip_pair(3_000_000, seed=71), {"BF16": {"rtol": 1e-3, "atol": 1e-4}},
                               tolerant),
        "B fp32 600k strict": (*synth.fp32_noise_pair(600_000, seed=72), {"FP32": {"rtol": 1e-5, "atol": 1e-5}},
                               None),
    }
    rec_size = ctypes.sizeof(_lib.KvvResult)
    views, want = {}, {}
    for name, (g, r, tol, pol) in cases.items():
        gd, rd = g.to(DEV), r.to(DEV)
        job = verdict._Job(gd, rd, "output", tol, pol, verdict.MAX_SAMPLES, fp8_errors=False)
        gt, rt, held = verdict._device_views(gd, rd)
        views[name] = (gt, rt, job.kpolicy, held)
        _say("noalloc graph: expected record of", name)
        want[name], eager = _records(lib, gd, rd, tol, pol)
        assert not _same(want[name], eager), name

    def eager_noalloc(name):
        gt, rt, pol, _ = views[name]
        out = torch.zeros(rec_size, dtype=torch.uint8, pin_memory=True)
        _lib.check(lib.kvv_verdict_noalloc(gt, rt, pol, out.data_ptr(), torch.cuda.current_stream().cuda_stream),
                   "kvv_verdict_noalloc")
        torch.cuda.current_stream().synchronize()
        return _lib.KvvResult.from_buffer_copy(out.numpy().tobytes()).to_dict()

    graphs, outs = {}, {}
    for name in cases:
        gt, rt, pol, _ = views[name]
        outs[name] = torch.zeros(rec_size, dtype=torch.uint8, device=DEV)
        graphs[name] = torch.cuda.CUDAGraph()
        _say("noalloc graph: capture", name)
        with torch.cuda.graph(graphs[name]):
            rc = lib.kvv_verdict_noalloc(gt, rt, pol, outs[name].data_ptr(), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "kvv_verdict_noalloc under capture")
    torch.cuda.synchronize()
    order = ["replay A", "eager B", "replay B", "eager A", "replay A", "replay B", "eager B", "replay A", "eager A",
             "replay B"]
    for step in order:
        kind, key = step.split()
        name = next(n for n in cases if n.startswith(key + " "))
        _say("noalloc graph:", step)
        if kind == "replay":
            outs[name].zero_()
            graphs[name].replay()
            torch.cuda.synchronize()
            got = _lib.KvvResult.from_buffer_copy(outs[name].cpu().numpy().tobytes()).to_dict()
        else:
            got = eager_noalloc(name)
        bad = _same(want[name], got)
        assert not bad, (step, bad)
        assert got["status"] == 0 and got["numel"] == cases[name][0].numel()
