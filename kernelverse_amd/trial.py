"""Correctness trial driver and case finalisation, with the verdict on the device.

Same call surface as KernelVerse ``runner/generated_correctness_runner.py``
(GCR) for the code around the verdict:

* ``_run_correctness_trial_once`` (GCR:1281-1322) builds the inputs and both
  models from the same seeds, runs them, and judges the outputs.  The
  reference copies both outputs to the host (``_to_cpu``, GCR:1315-1316) and
  compares them there.  Here the outputs stay where the models wrote them:
  ``verdict._compare_outputs`` reads them once in HBM (one batched launch
  sequence for nested outputs) and only the per-pair records cross PCIe.
* ``finalize_generated_operator_result`` (GCR:1760-1810),
  ``_random_case_summary`` (GCR:279-302) and
  ``_resolve_random_correctness_config`` (GCR:250-276) turn per-case results
  into the operator's correctness summary.  They are host logic over plain
  dicts and keep the reference's keys, rounding and error texts.

The helpers ``_as_list``, ``_to_device``, ``_to_cpu``, ``_clone_input``,
``_seed_all`` and ``_disable_tf32_for_correctness`` (GCR:78-163) follow the
reference so that a trial sees the same inputs and parameters.
"""

from __future__ import annotations

import contextlib
from typing import Any, Dict, List, Optional, Tuple

import torch

from .verdict import _compare_outputs

RANDOM_CORRECTNESS_CONFIG_KEY = "random_correctness"
DEFAULT_RANDOM_CORRECTNESS = {"max_failed_case_rate": 0.03}


# ------------------------------------------------------------ containers
def _map_nested(value: Any, leaf) -> Any:
    """Applies ``leaf`` to every tensor of a tuple/list/dict nest, keeping the containers' types."""
    if isinstance(value, torch.Tensor):
        return leaf(value)
    if isinstance(value, tuple):
        return tuple(_map_nested(v, leaf) for v in value)
    if isinstance(value, list):
        return [_map_nested(v, leaf) for v in value]
    if isinstance(value, dict):
        return {k: _map_nested(v, leaf) for k, v in value.items()}
    return value


def _as_list(value: Any) -> List[Any]:
    """GCR:96-101: a tuple becomes a list, a list stays itself, anything else is wrapped."""
    if isinstance(value, list):
        return value
    if isinstance(value, tuple):
        return list(value)
    return [value]


def _to_device(value: Any, device: Any) -> Any:
    """GCR:104-115."""
    return _map_nested(value, lambda t: t.to(device))


def _to_cpu(value: Any) -> Any:
    """GCR:118-129 (kept for callers that want host copies; the trial below does not use it)."""
    return _map_nested(value, lambda t: t.detach().cpu())


def _clone_input(value: Any) -> Any:
    """GCR:132-143."""
    return _map_nested(value, lambda t: t.detach().clone())


def _seed_all(seed: int, language: str) -> None:
    """GCR:146-163 for the ROCm backends: the CPU generator and every GPU generator.

    The reference's extra branches seed vendor runtimes ("biren", "ascendc")
    that do not exist on a ROCm system; ``language`` is accepted for the same
    signature.
    """
    del language
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


@contextlib.contextmanager
def _disable_tf32_for_correctness():
    """GCR:78-93: full fp32 matmul precision while the trial's models run."""
    saved = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32,
             torch.get_float32_matmul_precision())
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    try:
        yield
    finally:
        torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = saved[0], saved[1]
        torch.set_float32_matmul_precision(saved[2])


# ------------------------------------------------------------ one trial
def _run_correctness_trial_once(
    *,
    language: str,
    correctness_shape: Dict[str, Any],
    generated_model_class: type,
    reference_model_class: type,
    generate_inputs_fn,
    backend: Any,
    device: Any,
    input_seed: int,
    param_seed: int,
    tolerance_policy: Dict[str, Any],
    correctness_policy: Dict[str, Any],
) -> Tuple[bool, List[str], List[Dict[str, Any]]]:
    """GCR:1281-1322: one seeded trial of a generated operator against its reference.

    The inputs come from ``generate_inputs_fn`` under ``input_seed`` and are
    moved to ``device``; each model gets its own clone of them, and both
    models are built under ``param_seed``.  The outputs are judged where they
    are, on the device, by the HIP verdict; the reference instead copies both
    to the host first.  Returns ``(ok, details, metas)`` exactly as the
    reference's ``_compare_outputs`` would on host copies of the same outputs.
    """
    _seed_all(input_seed, language)
    device_inputs = [_to_device(item, device) for item in _as_list(generate_inputs_fn(correctness_shape))]
    generated_inputs = [_clone_input(item) for item in device_inputs]
    reference_inputs = [_clone_input(item) for item in device_inputs]
    sync = getattr(backend, "synchronize", None)

    with torch.no_grad(), _disable_tf32_for_correctness():
        _seed_all(param_seed, language)
        generated_model = generated_model_class(correctness_shape).to(device).eval()
        _seed_all(param_seed, language)
        reference_model = reference_model_class(correctness_shape).to(device).eval()
        generated_output = generated_model(*generated_inputs)
        if sync is not None:
            sync(device=device)
        reference_output = reference_model(*reference_inputs)
        if sync is not None:
            sync(device=device)

    return _compare_outputs(generated_output, reference_output, tolerance_policy=tolerance_policy,
                            correctness_policy=correctness_policy)


# ------------------------------------------------------------ case finalisation
def _resolve_random_correctness_config(operator_spec: Dict[str, Any]) -> Dict[str, float]:
    """GCR:250-276: the operator's ``random_correctness.max_failed_case_rate`` (default 0.03), checked."""
    op_name = operator_spec.get("op_name", "<unknown>")
    section = (operator_spec.get("config") or {}).get(RANDOM_CORRECTNESS_CONFIG_KEY) or {}
    if not isinstance(section, dict):
        raise ValueError(f"{op_name} has invalid {RANDOM_CORRECTNESS_CONFIG_KEY}: expected object.")
    raw = section.get("max_failed_case_rate", DEFAULT_RANDOM_CORRECTNESS["max_failed_case_rate"])
    try:
        rate = float(raw)
    except (TypeError, ValueError) as exc:
        raise ValueError(f"{op_name} has invalid random_correctness.max_failed_case_rate: {raw!r}.") from exc
    if not 0.0 <= rate <= 1.0:
        raise ValueError(f"{op_name} has invalid random_correctness.max_failed_case_rate: "
                         f"{rate}. Expected a value in [0.0, 1.0].")
    return {"max_failed_case_rate": rate}


def _random_case_summary(*, shape_mode: str, total_cases: int, failed_cases: int,
                         random_correctness_config: Dict[str, float]) -> Dict[str, Any]:
    """GCR:279-302: failed-case rate (1.0 with no cases) against the allowed rate, random mode only."""
    allowed = float(random_correctness_config["max_failed_case_rate"])
    rate = failed_cases / total_cases if total_cases > 0 else 1.0
    return {
        "total_cases": total_cases,
        "failed_cases": failed_cases,
        "failed_case_rate": round(rate, 4),
        "max_failed_case_rate": allowed,
        "within_tolerance": shape_mode == "random" and total_cases > 0 and rate <= allowed,
    }


def _case_error_text(case_result: Dict[str, Any]) -> str:
    """GCR:999-1014: every diagnostic string of a case, newline-joined and lower-cased."""
    parts = [str(case_result.get("error_type") or ""), str(case_result.get("error_message") or "")]
    for failure in case_result.get("failed_trials") or []:
        if isinstance(failure, dict):
            parts += [str(d) for d in failure.get("details") or []]
    perf = case_result.get("performance_error_message")
    if isinstance(perf, dict):
        parts += [str(v) for v in perf.values() if v]
    elif perf:
        parts.append(str(perf))
    return "\n".join(parts).lower()


# Diagnostics the reference reads as a failed extension build of a "biren" case
# (GCR:1017-1040): any of the first group, or a compiler "fatal error:" that
# names one of the second.
_BUILD_FAILURE_MARKERS = ("casecompilefailed", "error building extension", "build command failed",
                          "generated code compilation failed", "ninja: build stopped", "compilation terminated")
_FATAL_ERROR_CONTEXT = ("brcc", "kernel.su", "main.cpp", "file not found", "no such file or directory",
                        "compiling for device")


def _is_biren_case_compile_failure(case_result: Dict[str, Any]) -> bool:
    """GCR:1017-1040."""
    text = _case_error_text(case_result)
    if any(m in text for m in _BUILD_FAILURE_MARKERS):
        return True
    return "fatal error:" in text and any(m in text for m in _FATAL_ERROR_CONTEXT)


def finalize_generated_operator_result(*, result: Dict[str, Any], shape_mode: str,
                                       random_correctness_config: Dict[str, float],
                                       total_cases: Optional[int] = None) -> Dict[str, Any]:
    """GCR:1760-1810: the operator's correctness summary from its completed cases (updates ``result``).

    Cases are ordered by ``case_index``; their failed trials are concatenated.
    Random shape mode passes when the failed-case rate is within the allowed
    rate; every other mode needs every expected case present and passing.  A
    "biren" result whose case diagnostics show a failed extension build is
    marked as not compiled.
    """
    cases = sorted(result.get("cases") or [], key=lambda c: int(c.get("case_index", 0)))
    result["cases"] = cases
    failed_trials: List[Dict[str, Any]] = []
    failed = 0
    for case in cases:
        if not bool(case.get("success")):
            failed += 1
        failed_trials.extend(case.get("failed_trials") or [])
    expected = len(cases) if total_cases is None else int(total_cases)
    summary = _random_case_summary(shape_mode=shape_mode, total_cases=expected, failed_cases=failed,
                                   random_correctness_config=random_correctness_config)
    build_failed = str(result.get("language", "")).lower() == "biren" and any(
        isinstance(c, dict) and _is_biren_case_compile_failure(c) for c in cases)
    if build_failed:
        message = "Biren case worker reported an extension compilation failure."
        result["compiled"] = False
        result["compile_info"] = message
        result["error_type"] = "CaseCompileFailed"
        result["error_message"] = message
    correctness = result["correctness"]
    if shape_mode == "random":
        correctness["random_case_summary"] = summary
        passed = summary["within_tolerance"]
    else:
        passed = failed == 0 and len(cases) == expected
    correctness["success"] = passed and not build_failed
    correctness["failed_trials"] = failed_trials
    return result
