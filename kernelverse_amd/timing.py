"""Operator timing on MI355X with HIP events.

Same call surface as KernelVerse ``utils/performance.py`` (PERF) and
``runner/profiler_runner.py`` ``profile_case`` (PR:84-143):

* ``_time_execution_cuda_event(run_once, device=...)`` (PERF:102-148) runs
  the callable ``OP_EVAL_CUDA_NUM_WARMUP`` times, then times
  ``OP_EVAL_CUDA_DISCARD_FIRST`` + ``OP_EVAL_CUDA_NUM_TRIALS`` runs, each
  bracketed by a pair of HIP events on the current stream after a device
  synchronisation and a cache flush.  The first discarded runs are dropped.
  The environment variables, their defaults and the result payload
  (``_build_cuda_perf_result``, PERF:151-162) are the reference's.
* ``time_execution_event_template`` / ``_time_execution_cuda_event_template``
  (PERF:165-230) build the model from a backend context and time it.
* ``profile_case`` (PR:84-143) times one benchmark case on a ROCm device.

What is sized for MI355X is the flush.  The reference writes a fresh
256 MiB tensor before each timed run (PERF:75-79), which does not reliably
evict MI355X's 256 MB last-level cache (MALL), nor the eight XCDs' 4 MB L2s
behind it.  Here a 512 MiB buffer, allocated once per device, is rewritten
before each timed run.  Because the flush buffer is never re-allocated, the
timed region sees no allocator work.
"""

from __future__ import annotations

import hashlib
import os
import random
from typing import Any, Callable, Dict, List, Optional, Tuple

import numpy as np
import torch

from .trial import _as_list

NUM_PERF_TRIALS = int(os.environ.get("OP_EVAL_CUDA_NUM_TRIALS", "5"))
NUM_WARMUP = int(os.environ.get("OP_EVAL_CUDA_NUM_WARMUP", "3"))
SEED_NUM = int(os.environ.get("OP_EVAL_PERF_SEED_BASE", "1024"))

FLUSH_BYTES = 512 << 20  # two MALL capacities

_PREHEATED: set = set()
_FLUSH: Dict[int, torch.Tensor] = {}


def _bool_env(name: str, default: bool = False) -> bool:
    """PERF:17-21."""
    raw = os.environ.get(name)
    return default if raw is None else raw.strip().lower() in ("1", "true", "yes", "on")


def _round3(value: Optional[float]) -> Optional[float]:
    return None if value is None else round(float(value), 3)


def _normalize_device(device) -> torch.device:
    """PERF:30-37: a ``torch.device``, a device index or a device string."""
    if isinstance(device, torch.device):
        return device
    if isinstance(device, int):
        return torch.device(f"cuda:{device}")
    if isinstance(device, str):
        return torch.device(device)
    raise TypeError(f"Unsupported device type: {type(device)}")


def perf_seed_for_op(op_name: str) -> int:
    """PERF:40-45: a per-operator seed from SHA-256 of ``salt:op_name``, offset by the seed base."""
    salt = os.environ.get("OP_EVAL_PERF_SEED_SALT", "op_benchmark_perf_seed")
    base = int(os.environ.get("OP_EVAL_PERF_SEED_BASE", str(SEED_NUM)))
    h = int.from_bytes(hashlib.sha256(f"{salt}:{op_name}".encode("utf-8")).digest()[:8], "little")
    return (base + h) % (2**31 - 1)


def set_perf_seed(op_name: Optional[str]) -> None:
    """PERF:48-57: seeds Python, NumPy, the CPU and every GPU generator for the operator's inputs."""
    if not op_name:
        return
    seed = perf_seed_for_op(op_name)
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def _flush_caches(device: torch.device) -> None:
    """Rewrites the device's flush buffer (512 MiB), evicting the MALL and the L2s before a timed run."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    buf = _FLUSH.get(index)
    if buf is None:
        buf = _FLUSH[index] = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=device)
    buf.fill_(42)


def _preheat_cuda_device(device) -> None:
    """PERF:82-99: one 8192^3 fp16 matmul per process and device before the first timing (clock ramp)."""
    device = _normalize_device(device)
    with torch.cuda.device(device):
        index = device.index if device.index is not None else torch.cuda.current_device()
        if index in _PREHEATED:
            return
        a = torch.randn((8192, 8192), dtype=torch.float16, device=device)
        b = torch.randn((8192, 8192), dtype=torch.float16, device=device)
        c = torch.empty((8192, 8192), dtype=torch.float16, device=device)
        torch.mm(a, b, out=c)
        torch.cuda.synchronize(device=device)
        del a, b, c
        _PREHEATED.add(index)


def _time_execution_cuda_event(run_once: Callable[[], None], *, device) -> List[float]:
    """PERF:102-148: per-run milliseconds from HIP events (see the module docstring for the protocol)."""
    warmup = max(0, int(os.environ.get("OP_EVAL_CUDA_NUM_WARMUP", str(NUM_WARMUP))))
    trials = max(1, int(os.environ.get("OP_EVAL_CUDA_NUM_TRIALS", str(NUM_PERF_TRIALS))))
    discard = max(0, int(os.environ.get("OP_EVAL_CUDA_DISCARD_FIRST", "1")))
    flush = _bool_env("OP_EVAL_CUDA_CLEAR_L2_CACHE", True)
    device = _normalize_device(device)
    times: List[float] = []
    with torch.cuda.device(device):
        _preheat_cuda_device(device)
        for _ in range(warmup):
            run_once()
            torch.cuda.synchronize(device=device)
        torch.cuda.empty_cache()
        stream = torch.cuda.current_stream(device)
        for trial in range(trials + discard):
            torch.cuda.synchronize(device=device)
            if flush:
                try:
                    _flush_caches(device)
                except Exception:  # noqa: BLE001 - the reference times without the flush once it fails
                    flush = False
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            run_once()
            end.record(stream)
            torch.cuda.synchronize(device=device)
            if trial >= discard:
                times.append(float(start.elapsed_time(end)))
    return times


def _build_cuda_perf_result(elapsed_times_ms: List[float]) -> Dict[str, Any]:
    """PERF:151-162: mean, population std, min, max (rounded to 3 places) and the trial count."""
    if not elapsed_times_ms:
        return {"performance": None, "profiling": None}
    x = np.asarray(elapsed_times_ms, dtype=np.float64)
    return {"performance": {"mean": _round3(float(x.mean())), "std": _round3(float(x.std())),
                            "min": _round3(float(x.min())), "max": _round3(float(x.max())),
                            "num_trials": len(elapsed_times_ms)},
            "profiling": None}


def _time_execution_cuda_event_template(context, device, eval_target) -> Tuple[List[float], Optional[Dict[str, Any]]]:
    """PERF:165-199: builds ``context[eval_target]`` from the context's init inputs and times its forward."""
    if not torch.cuda.is_available():
        raise RuntimeError("CUDA timing requested but torch.cuda.is_available() is False.")
    device = _normalize_device(device)
    if device.type != "cuda":
        raise ValueError(f"Expected CUDA device, got {device}.")
    set_perf_seed(context.get("_op_eval_op_name"))
    move = lambda xs: [x.to(device) if isinstance(x, torch.Tensor) else x for x in xs]  # noqa: E731
    inputs = move(context["get_inputs"]())
    init_inputs = move(context["get_init_inputs"]())
    with torch.no_grad():
        model = context[eval_target](*init_inputs).to(device).eval()
        times = _time_execution_cuda_event(lambda: model(*inputs), device=device)
    return times, _build_cuda_perf_result(times)


def time_execution_event_template(context, device, synchronize, event_class,
                                  eval_target) -> Tuple[List[float], Optional[Dict[str, Any]]]:
    """PERF:202-217: the backend-facing entry point (``synchronize`` and ``event_class`` are unused)."""
    del synchronize, event_class
    dev = _normalize_device(device)
    if dev.type != "cuda":
        raise ValueError(f"Only CUDA timing is supported by standalone op_benchmark, got {dev}.")
    return _time_execution_cuda_event_template(context=context, device=dev, eval_target=eval_target)


_ROCM_LANGUAGES = ("cuda", "hip", "rocm", "triton")


def profile_case(*, language: str, device_id: int, op_name: str, case_name: str, shape: Dict[str, Any],
                 model_class: type, generate_inputs_fn: Callable[..., Any], perf_trials: Optional[int] = None,
                 use_torch_compile: bool = False) -> Dict[str, Any]:
    """PR:84-143 on a ROCm device: ``{"performance": {...}, "profiling": None}`` for one case.

    The case's model is built from ``shape`` and timed on ``cuda:device_id``
    with inputs from ``generate_inputs_fn(shape)``, seeded per operator tag
    ``op_benchmark/<op>/<case>/operator_defined``.  ``perf_trials``
    overrides ``OP_EVAL_CUDA_NUM_TRIALS`` for this call only.  The compiled
    mode of the reference (``torch.compile``) has no counterpart here.
    """
    if str(language).lower() not in _ROCM_LANGUAGES:
        raise ValueError(f"profile_case times ROCm devices only (languages {_ROCM_LANGUAGES}), got {language!r}")
    if use_torch_compile:
        raise NotImplementedError("use_torch_compile: no tracing compiler on this path")
    torch.cuda.set_device(device_id)
    device = torch.device(f"cuda:{device_id}")

    def get_inputs():
        return _as_list(generate_inputs_fn(shape))

    context = {"Model": model_class, "get_inputs": get_inputs, "get_init_inputs": lambda: [shape],
               "_op_eval_op_name": f"op_benchmark/{op_name}/{case_name}/operator_defined"}
    previous = os.environ.get("OP_EVAL_CUDA_NUM_TRIALS")
    if perf_trials is not None:
        os.environ["OP_EVAL_CUDA_NUM_TRIALS"] = str(perf_trials)
    try:
        _, result = time_execution_event_template(context, device, torch.cuda.synchronize, torch.cuda.Event,
                                                  eval_target="Model")
        return result if result is not None else {"performance": None, "profiling": None}
    finally:
        if previous is None:
            os.environ.pop("OP_EVAL_CUDA_NUM_TRIALS", None)
        else:
            os.environ["OP_EVAL_CUDA_NUM_TRIALS"] = previous

