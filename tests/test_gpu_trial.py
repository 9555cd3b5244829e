"""Trial driver and timing harness on the device (needs an MI355X).

The trial fixtures hold what the reference's own ``_run_correctness_trial_once``
(GCR:1281-1322) returned on the CPU for the operator pairs of
``trial_models``; those pairs compute bit-identically on the GPU, so the
device trial must return the same ``(ok, details, metas)``.
"""

import os
import sys

import pytest
import torch

import trial_models
from golden_io import load_trial_cases
from parity_util import meta_problems

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    from kernelverse_amd import _lib
    _lib.load()
    return torch.device("cuda", 0)


class _Backend:
    def __init__(self):
        self.calls = 0

    def synchronize(self, device=None):
        self.calls += 1
        torch.cuda.synchronize(device=device)


TRIALS = load_trial_cases()


@pytest.mark.parametrize("case", TRIALS, ids=[c["name"] for c in TRIALS])
def test_device_trial_matches_reference_trial(dev, case):
    from kernelverse_amd import trial

    _say("trial", case["name"], case["n"])
    backend = _Backend()
    got = trial._run_correctness_trial_once(
        language="hip", correctness_shape={"n": case["n"]},
        generated_model_class=trial_models.MODELS[case["generated"]],
        reference_model_class=trial_models.MODELS[case["reference"]],
        generate_inputs_fn=trial_models.generate_inputs, backend=backend, device=dev,
        input_seed=trial_models.INPUT_SEED, param_seed=trial_models.PARAM_SEED,
        tolerance_policy=case["tolerance_policy"], correctness_policy=case["correctness_policy"])
    assert backend.calls == 2
    ok, details, metas = case["expected"]["value"]
    assert len(got[2]) == len(metas)
    for g, w in zip(got[2], metas):
        probs = meta_problems(g, w)
        assert not probs, probs
    assert got[0] == ok
    assert got[1] == details


def test_trial_outputs_stay_on_device(dev, monkeypatch):
    """The verdict gets the models' device tensors: nothing is copied to the host first."""
    from kernelverse_amd import trial, verdict

    seen = []
    real = verdict._run_jobs

    def spy(jobs):
        seen.extend((j.gen.device.type, j.ref.device.type) for j in jobs)
        return real(jobs)

    monkeypatch.setattr(verdict, "_run_jobs", spy)
    trial._run_correctness_trial_once(
        language="hip", correctness_shape={"n": 4096}, generated_model_class=trial_models.PairOut,
        reference_model_class=trial_models.PairOut, generate_inputs_fn=trial_models.generate_inputs,
        backend=None, device=dev, input_seed=5, param_seed=6, tolerance_policy=None, correctness_policy=None)
    assert seen == [("cuda", "cuda"), ("cuda", "cuda")]


# ------------------------------------------------------------ timing harness
def test_time_execution_protocol(dev, monkeypatch):
    from kernelverse_amd import timing

    monkeypatch.setenv("OP_EVAL_CUDA_NUM_WARMUP", "2")
    monkeypatch.setenv("OP_EVAL_CUDA_NUM_TRIALS", "4")
    monkeypatch.setenv("OP_EVAL_CUDA_DISCARD_FIRST", "1")
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    runs = []

    def run_once():
        runs.append(1)
        dst.copy_(src)

    _say("timing 256 MiB copies")
    times = timing._time_execution_cuda_event(run_once, device=dev)
    assert len(runs) == 2 + 1 + 4 and len(times) == 4
    # 512 MiB of HBM traffic per copy: at most 8 TB/s, so at least 67 us; well under 100 ms
    assert all(0.067 < t < 100.0 for t in times), times
    assert torch.equal(dst[:16], src[:16])
    buf = timing._FLUSH[dev.index]
    assert buf.numel() == timing.FLUSH_BYTES
    timing._flush_caches(dev)
    assert timing._FLUSH[dev.index].data_ptr() == buf.data_ptr()  # allocated once per device


def test_time_execution_without_flush(dev, monkeypatch):
    from kernelverse_amd import timing

    monkeypatch.setenv("OP_EVAL_CUDA_NUM_WARMUP", "0")
    monkeypatch.setenv("OP_EVAL_CUDA_NUM_TRIALS", "3")
    monkeypatch.setenv("OP_EVAL_CUDA_DISCARD_FIRST", "0")
    monkeypatch.setenv("OP_EVAL_CUDA_CLEAR_L2_CACHE", "0")
    x = torch.ones(1 << 20, device=dev)
    times = timing._time_execution_cuda_event(lambda: x.mul_(1.0), device=dev)
    assert len(times) == 3 and all(t > 0 for t in times)


class _Scale(torch.nn.Module):
    def __init__(self, shape):
        super().__init__()
        self.k = float(shape["k"])

    def forward(self, x):
        return x * self.k


def test_profile_case_payload(dev, monkeypatch):
    from kernelverse_amd import timing

    monkeypatch.delenv("OP_EVAL_CUDA_NUM_TRIALS", raising=False)
    out = timing.profile_case(language="hip", device_id=0, op_name="scale", case_name="case_0",
                              shape={"k": 2.0, "n": 1 << 20}, model_class=_Scale,
                              generate_inputs_fn=lambda s: torch.randn(s["n"]), perf_trials=3)
    perf = out["performance"]
    assert out["profiling"] is None
    assert list(perf) == ["mean", "std", "min", "max", "num_trials"] and perf["num_trials"] == 3
    assert perf["min"] <= perf["mean"] <= perf["max"]
    assert "OP_EVAL_CUDA_NUM_TRIALS" not in os.environ  # restored after the call
