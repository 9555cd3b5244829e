"""Case finalisation, random-mode summary, timing payload and trial helpers against reference-written fixtures."""

import copy
import os

import pytest
import torch

from golden_io import load_finalize_cases, load_host_logic, same_value
from kernelverse_amd import timing, trial

HOST = load_host_logic()


def _check(outcome, fn, *args, **kwargs):
    if "raises" in outcome:
        with pytest.raises(Exception) as info:
            fn(*args, **kwargs)
        assert type(info.value).__name__ == outcome["raises"]
        assert str(info.value) == outcome["message"]
        return None
    got = fn(*args, **kwargs)
    assert same_value(got, outcome["value"]), (got, outcome["value"])
    return got


@pytest.mark.parametrize("case", HOST["resolve_random_correctness"], ids=lambda c: str(c["spec"])[:60])
def test_resolve_random_correctness_config(case):
    _check(case["expected"], trial._resolve_random_correctness_config, case["spec"])


def test_random_case_summary():
    for case in HOST["random_case_summary"]:
        _check(case["expected"], trial._random_case_summary, **case["kwargs"])


FINAL = load_finalize_cases()


@pytest.mark.parametrize("case", FINAL, ids=[f"{i}-{c['result']['language']}-{c['kwargs']['shape_mode']}"
                                             for i, c in enumerate(FINAL)])
def test_finalize_generated_operator_result(case):
    result = copy.deepcopy(case["result"])
    got = _check(case["expected"], trial.finalize_generated_operator_result, result=result, **case["kwargs"])
    if got is not None:
        assert got is result  # updated in place and returned, as the reference does


def test_build_cuda_perf_result():
    for case in HOST["perf_result"]:
        assert same_value(timing._build_cuda_perf_result(case["times"]), case["expected"])


def test_perf_seed_for_op(monkeypatch):
    monkeypatch.delenv("OP_EVAL_PERF_SEED_SALT", raising=False)
    monkeypatch.delenv("OP_EVAL_PERF_SEED_BASE", raising=False)
    for case in HOST["perf_seed"]:
        assert timing.perf_seed_for_op(case["op_name"]) == case["seed"]


def test_bool_env(monkeypatch):
    monkeypatch.delenv("KVV_TEST_FLAG", raising=False)
    assert timing._bool_env("KVV_TEST_FLAG", True) is True
    for raw, want in (("1", True), (" Yes ", True), ("on", True), ("0", False), ("no", False), ("", False)):
        monkeypatch.setenv("KVV_TEST_FLAG", raw)
        assert timing._bool_env("KVV_TEST_FLAG", True) is want


def test_normalize_device():
    assert timing._normalize_device(1) == torch.device("cuda:1")
    assert timing._normalize_device("cuda:0") == torch.device("cuda:0")
    assert timing._normalize_device(torch.device("cpu")) == torch.device("cpu")
    with pytest.raises(TypeError):
        timing._normalize_device(1.5)


def test_profile_case_rejects_other_runtimes():
    with pytest.raises(ValueError):
        timing.profile_case(language="ascendc", device_id=0, op_name="x", case_name="c", shape={},
                            model_class=object, generate_inputs_fn=lambda s: ())
    with pytest.raises(NotImplementedError):
        timing.profile_case(language="hip", device_id=0, op_name="x", case_name="c", shape={},
                            model_class=object, generate_inputs_fn=lambda s: (), use_torch_compile=True)


# ------------------------------------------------------------ trial helpers (GCR:78-163)
def test_containers_keep_their_types():
    a, b = torch.arange(3.0), torch.ones(2)
    nest = (a, [b, {"k": a, "n": 3}], "s")
    cl = trial._clone_input(nest)
    assert type(cl) is tuple and type(cl[1]) is list and type(cl[1][1]) is dict and cl[2] == "s"
    assert cl[1][1]["n"] == 3 and torch.equal(cl[0], a) and cl[0].data_ptr() != a.data_ptr()
    moved = trial._to_device(nest, "cpu")
    assert moved[0] is a  # .to() of a tensor already there is the tensor itself
    assert trial._as_list((1, 2)) == [1, 2] and trial._as_list(5) == [5]
    lst = [1]
    assert trial._as_list(lst) is lst


def test_seed_all_reproduces_inputs():
    trial._seed_all(7, "hip")
    x = torch.randn(4)
    trial._seed_all(7, "biren")
    assert torch.equal(x, torch.randn(4))


def test_tf32_switches_are_restored():
    before = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32,
              torch.get_float32_matmul_precision())
    with trial._disable_tf32_for_correctness():
        assert not torch.backends.cuda.matmul.allow_tf32 and not torch.backends.cudnn.allow_tf32
        assert torch.get_float32_matmul_precision() == "highest"
    assert (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32,
            torch.get_float32_matmul_precision()) == before


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_trial_without_gpu_raises():
    import trial_models
    from kernelverse_amd import _lib

    with pytest.raises(_lib.KvvLibraryError):
        trial._run_correctness_trial_once(
            language="hip", correctness_shape={"n": 16}, generated_model_class=trial_models.ScaleAdd,
            reference_model_class=trial_models.ScaleAdd, generate_inputs_fn=trial_models.generate_inputs,
            backend=None, device="cpu", input_seed=1, param_seed=2, tolerance_policy=None, correctness_policy=None)


def test_round4_matches_builtin_round():
    """verdict._round4 is round(x, 4) bit for bit (signed zeros, NaN and infinities included), on random
    values of every magnitude and on values a few ulps either side of the ties k / 10^4 + 5e-5."""
    import math
    import random
    from kernelverse_amd.verdict import _round4
    rng = random.Random(20261202)
    vals = [0.0, -0.0, 1.0, -1.0, 0.99995, 0.00005, -0.00005, 1e-300, -1e-300, 5e-5, 1.5e-4, 2.5e-4,
            math.inf, -math.inf, math.nan, 1e15, -1e15, 4e11, 4.1e11, 1e300]
    for _ in range(20000):
        e = rng.uniform(-12, 12)
        vals.append(rng.choice((1, -1)) * 10 ** e)
        vals.append(rng.random())
    for _ in range(20000):
        k = rng.randint(-10**7, 10**7)
        t = (k + 0.5) / 10000.0
        for steps in range(-3, 4):
            x = t
            for _ in range(abs(steps)):
                x = math.nextafter(x, math.inf if steps > 0 else -math.inf)
            vals.append(x)
    for x in vals:
        a, b = _round4(x), round(x, 4)
        assert (a != a and b != b) or (a == b and math.copysign(1.0, a) == math.copysign(1.0, b)), (x, a, b)
