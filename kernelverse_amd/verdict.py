"""Drop-in numerical-agreement verdict backed by the MI355X HIP library.

Same call surface as KernelVerse ``runner/generated_correctness_runner.py``
(GCR): ``_compare_tensors`` (GCR:672-786) and ``_compare_outputs``
(GCR:789-833) take the same arguments and return the same
``(ok, details, meta)`` structures -- key order, rounding, ``None``/NaN
conventions and detail strings included -- together with the policy helpers
they use (``TOLERANCE_POLICY`` GCR:39-44, ``_dtype_name`` GCR:212-223,
``_dtype_policy`` GCR:305-328, ``_evaluate_tensor_policy`` GCR:551-606,
``_correctness_criteria`` GCR:609-669, ``_operator_tolerance_policy``
GCR:886-888).

What changed is where the data-parallel work runs: every tensor pair is read
once in HBM by ``libkvv.so`` (one launch sequence per call; a batch launch for
nested outputs) and only a ~600-byte record per pair comes back to the host.
Tensors already on a ROCm device are used in place; CPU tensors (what the
reference's trial driver hands over, GCR:1315-1316) are copied to the current
device first.  There is no CPU fallback: without the library or a GPU these
functions raise.

Extensions (``verdict_record``) expose the full device record: max abs/rel
error over all elements with argmax, the 16-bucket ULP histogram, fp64
relative-L2 and cosine, NaN/Inf counts and finite-pattern violations.
"""

from __future__ import annotations

import ctypes
import math
import threading
from collections import OrderedDict
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib
from .correctness_policy import (
    is_cosine_policy,
    is_metric_policy,
    is_tolerant_policy,
    policy_name,
    thresholds_for_dtype,
)

TOLERANCE_POLICY = {
    "fp32": {"rtol": 1.3e-6, "atol": 1e-5},
    "fp16": {"rtol": 0.001, "atol": 0.0001},
    "bf16": {"rtol": 0.016, "atol": 1e-3},
    "int8": {"max_abs_diff": 1},
}

MAX_SAMPLES = 1_000_000

# The reference's finite-pattern check (GCR:420) calls torch.isfinite, which
# torch-CPU implements for float8_e5m2 but not for float8_e4m3fn or the fnuz
# formats: the reference verdict raises NotImplementedError for those.  True
# keeps that behaviour; False evaluates the finite-pattern rule on the decoded
# values instead (the kernels decode e4m3fn and e5m2).
FP8_REFERENCE_ERRORS = True


def _isfinite_errors() -> Dict[Any, str]:
    """The float8 dtypes whose torch-CPU isfinite raises, with torch's own message (probed once)."""
    out = {}
    for name in ("float8_e4m3fn", "float8_e5m2", "float8_e4m3fnuz", "float8_e5m2fnuz"):
        dt = getattr(torch, name, None)
        if dt is None:
            continue
        try:
            torch.isfinite(torch.zeros(1, dtype=dt))
        except NotImplementedError as exc:
            out[dt] = str(exc)
    return out


_ISFINITE_ERRORS = _isfinite_errors()

# complex inputs take the integer branch (not floating point) and torch's casts
# to int32 and float32 keep only the real part: the kernels read that part
_COMPLEX_REAL = {torch.complex64: torch.float32, torch.complex128: torch.float64}

_DTYPE_CODES = {
    torch.float32: _lib.F32,
    torch.float16: _lib.F16,
    torch.bfloat16: _lib.BF16,
    torch.float64: _lib.F64,
    torch.float8_e4m3fn: _lib.F8E4M3FN,
    torch.float8_e5m2: _lib.F8E5M2,
    torch.int8: _lib.I8,
    torch.uint8: _lib.U8,
    torch.int16: _lib.I16,
    torch.int32: _lib.I32,
    torch.int64: _lib.I64,
    torch.bool: _lib.BOOL,
    torch.uint16: _lib.U16,
    torch.uint32: _lib.U32,
    torch.uint64: _lib.U64,
}


# ------------------------------------------------------------ policy helpers
def _dtype_name(tensor) -> str:
    """GCR:212-223: FP32/FP16/BF16, INT8 for int8 and uint8, else the upper-cased torch name."""
    dt = tensor.dtype
    if dt == torch.float32:
        return "FP32"
    if dt == torch.float16:
        return "FP16"
    if dt == torch.bfloat16:
        return "BF16"
    if dt in (torch.int8, torch.uint8):
        return "INT8"
    return str(dt).replace("torch.", "").upper()


def _dtype_policy(tensor, tolerance_policy: Optional[Dict[str, Any]] = None):
    """GCR:305-328: configured entry (exact, lower or upper name), else the built-in default."""
    name = _dtype_name(tensor)
    if tolerance_policy:
        configured = tolerance_policy.get(name) or tolerance_policy.get(name.lower()) or tolerance_policy.get(name.upper())
        if configured is not None:
            return configured
    dt = tensor.dtype
    if dt in (torch.int8, torch.uint8):
        return TOLERANCE_POLICY["int8"]
    if dt == torch.float32:
        return TOLERANCE_POLICY["fp32"]
    if dt == torch.float16:
        return TOLERANCE_POLICY["fp16"]
    if dt == torch.bfloat16:
        return TOLERANCE_POLICY["bf16"]
    if torch.is_floating_point(tensor):
        return TOLERANCE_POLICY["fp32"]
    return {"max_abs_diff": 0}


def _format_number(value: Any) -> str:
    """GCR:331-335."""
    if type(value) is float:
        return format(value, ".6g")
    try:
        return f"{float(value):.6g}"
    except (TypeError, ValueError):
        return str(value)


def _threshold_pass(value: Any, threshold: Any) -> bool:
    """GCR:440-449: finite value <= finite threshold."""
    if value is None or threshold is None:
        return False
    v, t = float(value), float(threshold)
    return math.isfinite(v) and math.isfinite(t) and v <= t


def _cosine_pass(value: Any, threshold: Any) -> bool:
    """GCR:452-461: finite value >= finite threshold."""
    if value is None or threshold is None:
        return False
    v, t = float(value), float(threshold)
    return math.isfinite(v) and math.isfinite(t) and v >= t


def _range_pass(value: Any, min_value: Any, max_value: Any) -> bool:
    """GCR:464-478: finite value inside the closed finite range."""
    if value is None or min_value is None or max_value is None:
        return False
    v, lo, hi = float(value), float(min_value), float(max_value)
    if not (math.isfinite(v) and math.isfinite(lo) and math.isfinite(hi)):
        return False
    return lo <= v <= hi


def _evaluate_tensor_policy(reference, meta: Dict[str, Any], correctness_policy: Optional[Dict[str, Any]]) -> bool:
    """GCR:551-606: the metric fallback of the tolerant and cosine policies."""
    if meta.get("allclose_pass"):
        return True
    if not torch.is_floating_point(reference):
        return False
    cosine = is_cosine_policy(correctness_policy)
    if not cosine and not is_tolerant_policy(correctness_policy):
        return False
    th = thresholds_for_dtype(correctness_policy, _dtype_name(reference))
    finite_ok = bool(meta.get("finite_pass"))
    cosine_ok = _cosine_pass(meta.get("cosine_similarity"), th.get("min_cosine"))
    rate_ok = _threshold_pass(meta.get("mismatch_rate"), th.get("max_mismatch_rate"))
    p99_ok = _threshold_pass(meta.get("p99_abs"), th.get("max_p99_abs")) or _threshold_pass(
        meta.get("p99_rel"), th.get("max_p99_rel"))
    normal = bool(finite_ok and cosine_ok and rate_ok and p99_ok)
    meta["normal_metric_pass"] = normal
    if not cosine:
        return normal
    ratio_ok = _range_pass(meta.get("norm_ratio"), th.get("min_norm_ratio"), th.get("max_norm_ratio"))
    cos_metric = bool(finite_ok and cosine_ok and ratio_ok)
    meta["norm_ratio_pass"] = ratio_ok
    meta["cosine_metric_pass"] = cos_metric
    return bool(normal or cos_metric)


_METRIC_RULE = ("finite_pass AND cosine_similarity >= min_cosine AND mismatch_rate <= max_mismatch_rate AND "
                "(p99_abs <= max_p99_abs OR p99_rel <= max_p99_rel)")


def _correctness_criteria(tolerance_policy, correctness_policy, baseline_compute_mode, random_correctness_config,
                          shape_mode) -> Dict[str, Any]:
    """GCR:609-669: the criteria block stored next to each result."""
    metric = is_metric_policy(correctness_policy)
    fallback: Dict[str, Any] = {"enabled": metric}
    if metric and is_cosine_policy(correctness_policy):
        fallback["pass_rule"] = "allclose_pass OR normal_metric_pass OR cosine_metric_pass"
        fallback["tolerant_metric_pass_rule"] = _METRIC_RULE
        fallback["cosine_metric_pass_rule"] = (
            "finite_pass AND cosine_similarity >= min_cosine AND min_norm_ratio <= norm_ratio <= max_norm_ratio")
        fallback["thresholds"] = correctness_policy.get("thresholds") or {}
    elif metric:
        fallback["pass_rule"] = "allclose_pass OR normal_metric_pass"
        fallback["metric_pass_rule"] = _METRIC_RULE
        fallback["thresholds"] = correctness_policy.get("thresholds") or {}
    return {
        "baseline_compute_mode": baseline_compute_mode,
        "policy": {
            "name": policy_name(correctness_policy),
            "category": correctness_policy.get("category"),
            "source": correctness_policy.get("source"),
        },
        "allclose": {"enabled": True, "tolerances": tolerance_policy},
        "metric_fallback": fallback,
        "random_correctness": {
            "enabled": shape_mode == "random",
            "max_failed_case_rate": random_correctness_config["max_failed_case_rate"],
        },
    }


def _operator_tolerance_policy(operator_spec: Dict[str, Any]) -> Dict[str, Any]:
    """GCR:886-888."""
    config = operator_spec.get("config") or {}
    return config.get("tolerances") or TOLERANCE_POLICY


# ------------------------------------------------------------ device plumbing
class _Job:
    """One tensor pair on its way to the device, with what the meta builder needs."""

    __slots__ = ("gen", "ref", "path", "policy", "tolerance", "near_thresholds", "correctness_policy", "kpolicy",
                 "record", "is_float", "active", "tol_text", "pkey")

    def __init__(self, gen, ref, path, tolerance_policy, correctness_policy, max_samples, fp8_errors=None):
        self.gen, self.ref, self.path = gen, ref, path
        self.correctness_policy = correctness_policy
        dt = ref.dtype
        self.policy = pol = _dtype_policy(ref, tolerance_policy)
        ms = int(max_samples)
        mad = rtol = atol = 0
        if "max_abs_diff" in pol:
            mode = _lib.MODE_MAX_ABS_DIFF
            mad = int(pol["max_abs_diff"])
            if not -2**31 <= mad < 2**31:
                raise RuntimeError(f"value cannot be converted to type int32_t without overflow")
            self.tolerance = {"max_abs_diff": mad}
        else:
            rtol = float(pol["rtol"])
            atol = float(pol["atol"])
            mode = _lib.MODE_ISCLOSE
            self.tolerance = {"rtol": rtol, "atol": atol}
        self.near_thresholds = None
        nz = None
        if dt in _HALF_DTYPES and is_tolerant_policy(correctness_policy):
            th = thresholds_for_dtype(correctness_policy, _dtype_name(ref))
            if th.get("near_zero_abs") is not None and th.get("max_near_zero_bad_abs") is not None:
                self.near_thresholds = th
                nz = (float(th["near_zero_abs"]), float(th["max_near_zero_bad_abs"]))
        # the policy's part of the single-pair plan key (the values kpolicy is built from)
        self.pkey = pkey = (mode, rtol, atol, mad, nz, ms)
        info = _DTYPE_INFO.get(dt)
        if info is None:
            info = _dtype_info(dt)
        if info[0] is not None and (FP8_REFERENCE_ERRORS if fp8_errors is None else fp8_errors):
            raise NotImplementedError(info[0])
        if not info[1]:
            raise TypeError(f"verdict does not support dtype {dt}")
        tmpl = _KP_TEMPLATES.get(pkey)
        if tmpl is None:
            tmpl = _kp_template(pkey)
        self.kpolicy = _lib.KvvPolicy.from_buffer_copy(tmpl)
        self.record = None
        self.tol_text = None
        self.is_float = info[2]
        self.active = policy_name(correctness_policy)


_HALF_DTYPES = (torch.float16, torch.bfloat16)
_DTYPE_INFO: Dict[Any, Tuple[Optional[str], bool, bool]] = {}
_KP_TEMPLATES: Dict[tuple, bytes] = {}


def _dtype_info(dt) -> Tuple[Optional[str], bool, bool]:
    """Per dtype: the isfinite error the reference raises for it (or None), whether the library
    supports it, whether it is a floating type."""
    info = (_ISFINITE_ERRORS.get(dt), _COMPLEX_REAL.get(dt, dt) in _DTYPE_CODES, dt.is_floating_point)
    _DTYPE_INFO[dt] = info
    return info


def _kp_template(pkey: tuple) -> bytes:
    """The C-ABI policy of a job's policy key, as bytes (a fresh KvvPolicy is copied from them per job)."""
    mode, rtol, atol, mad, nz, ms = pkey
    kp = _lib.KvvPolicy()
    kp.max_samples = ms
    kp.mode = mode
    if mode == _lib.MODE_MAX_ABS_DIFF:
        kp.max_abs_diff = mad
    else:
        kp.rtol, kp.atol = rtol, atol
    if nz is not None:
        kp.flags |= _lib.FLAG_NEAR_ZERO
        kp.near_zero_abs, kp.near_zero_bad_abs = nz
    tmpl = bytes(kp)
    if len(_KP_TEMPLATES) >= 256:
        _KP_TEMPLATES.clear()
    _KP_TEMPLATES[pkey] = tmpl
    return tmpl


def _device_for(*tensors) -> torch.device:
    for t in tensors:
        if t.device.type == "cuda":
            return t.device
    if not torch.cuda.is_available():
        raise _lib.KvvLibraryError("the verdict runs on a ROCm GPU and none is visible (no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


def _kvv_tensor(t: torch.Tensor, sizes=None, strides=None) -> _lib.KvvTensor:
    """The C-ABI view of ``t`` (its own shape and strides unless given)."""
    sizes = list(t.shape) if sizes is None else sizes
    strides = list(t.stride()) if strides is None else strides
    if len(sizes) > _lib.MAX_DIMS:
        raise _lib.KvvLibraryError(f"tensors of more than {_lib.MAX_DIMS} dims must be coalesced first")
    kt = _lib.KvvTensor()
    kt.data = t.data_ptr() if t.numel() else 0
    kt.dtype = _DTYPE_CODES[t.dtype]
    kt.ndim = len(sizes)
    for i, (s, st) in enumerate(zip(sizes, strides)):
        kt.sizes[i] = s
        kt.strides[i] = st
    return kt


def _device_views(g: torch.Tensor, r: torch.Tensor):
    """C-ABI views of a same-shape pair on the device.

    Complex tensors are read through their real part (see ``_COMPLEX_REAL``).
    A pair of more than eight dims is coalesced jointly: size-1 dims dropped,
    a dim merged into its outer neighbour where both tensors' strides chain.
    The row-major logical order, and so every reported index, is unchanged.
    Only when that still leaves more than eight dims are both tensors copied
    to contiguous memory on the device.  Returns (gen view, ref view, tensors
    to keep alive until the call has been issued).
    """
    if g.dtype in _COMPLEX_REAL:
        g, r = torch.view_as_real(g.resolve_conj())[..., 0], torch.view_as_real(r.resolve_conj())[..., 0]
    if g.dim() <= _lib.MAX_DIMS:
        return _kvv_tensor(g), _kvv_tensor(r), (g, r)
    sz, gs, rs = [], [], []
    for s, a, b in zip(g.shape, g.stride(), r.stride()):
        if s == 1:
            continue
        if sz and gs[-1] == a * s and rs[-1] == b * s:
            sz[-1] *= s
            gs[-1], rs[-1] = a, b
        else:
            sz.append(s)
            gs.append(a)
            rs.append(b)
    if g.numel() == 0:
        sz, gs, rs = [0], [1], [1]
    if len(sz) > _lib.MAX_DIMS:
        g, r = g.contiguous(), r.contiguous()
        sz, gs, rs = [g.numel()], [1], [1]
    return _kvv_tensor(g, sz, gs), _kvv_tensor(r, sz, rs), (g, r)


def _run_jobs(jobs: List[_Job]) -> None:
    """Runs every job's pair through libkvv (one call for one pair, a batch call otherwise).

    A single fp16/bf16 pair under the tolerant policy takes its near-zero
    diagnostics from entries recorded in the main pass; a part of the pair whose
    entries outgrow the workspace's pool is read again inside the same call, so
    every record comes back complete (status 0)."""
    if not jobs:
        return
    _launch(jobs)
    for j in jobs:
        if j.record.status != 0:
            raise _lib.KvvLibraryError(f"the device verdict of {j.path} reported status {j.record.status}")


class _Buffers:
    """The workspace and the pinned record buffer of one (device, stream), kept between calls.

    Every call synchronises its stream before it returns, so consecutive calls
    on one stream can reuse both; the lock serialises threads that share the
    stream.  Each grows to the largest call seen.  At most ``_MAX_STREAMS``
    (device, stream) entries are kept: a new stream evicts the least recently
    used idle one, and ``release_buffers`` frees them all.
    ``kept``: the workspace went through a previous call and nothing else writes
    it, so single-pair calls pass KVV_FLAG_WS_KEPT (the library then skips
    clearing the select slots that call left clear).
    ``plans``: per single-pair layout and policy, the C-ABI views (their data
    pointers set per call) and the workspace size, so a repeated call plans nothing
    on the host."""

    __slots__ = ("lock", "ws", "out", "kept", "stream", "handle", "plans", "ws_bytes", "ws_ptr", "out_ptr", "out_rec")

    def __init__(self, stream):
        self.lock = threading.Lock()
        self.ws = None
        self.out = None
        self.kept = False
        self.stream = stream
        self.handle = stream.cuda_stream
        self.plans: "OrderedDict[tuple, tuple]" = OrderedDict()
        self.ws_bytes = self.ws_ptr = self.out_ptr = 0
        self.out_rec = None  # the first record's bytes in `out`, as a ctypes view


_MAX_STREAMS = 8
_MAX_PLANS = 64
_BUFFERS: "OrderedDict[Tuple[int, int], _Buffers]" = OrderedDict()
_BUFFERS_LOCK = threading.Lock()
_LAST = [None]  # the most recently used entry (its LRU position needs no update)
# the current stream's raw handle without building a torch Stream object (falls back to the public call)
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_buffers(dev: torch.device) -> _Buffers:
    """The buffers of dev's current stream (created, and the LRU bound kept, on first use)."""
    idx = dev.index
    handle = _RAW_STREAM(idx) if _RAW_STREAM is not None else torch.cuda.current_stream(dev).cuda_stream
    key = (idx, handle)
    b = _BUFFERS.get(key)
    if b is not None:
        if b is not _LAST[0]:
            with _BUFFERS_LOCK:
                if key in _BUFFERS:
                    _BUFFERS.move_to_end(key)
                    _LAST[0] = b
        return b
    cur = torch.cuda.current_stream(dev)
    with _BUFFERS_LOCK:
        b = _BUFFERS.get(key)
        if b is None:
            b = _BUFFERS[key] = _Buffers(cur)
            _LAST[0] = b
            # evict the least recently used idle entries beyond the bound (their memory goes back to torch)
            for old in list(_BUFFERS.keys())[:-1]:
                if len(_BUFFERS) <= _MAX_STREAMS:
                    break
                ob = _BUFFERS[old]
                if ob.lock.acquire(blocking=False):
                    try:
                        ob.ws = ob.out = ob.out_rec = None
                        ob.plans.clear()
                        del _BUFFERS[old]
                    finally:
                        ob.lock.release()
    return b


def release_buffers() -> None:
    """Frees the workspaces and record buffers the drop-in keeps between calls."""
    with _BUFFERS_LOCK:
        for b in _BUFFERS.values():
            with b.lock:
                b.ws = b.out = b.out_rec = None
                b.plans.clear()
        _BUFFERS.clear()
        _LAST[0] = None


def _ensure(buf: _Buffers, dev: torch.device, ws_bytes: int, records: int) -> None:
    """Grows buf's workspace and pinned record buffer to this call's needs (under buf.lock)."""
    rec_size = ctypes.sizeof(_lib.KvvResult)
    if buf.ws is None or buf.ws.numel() < ws_bytes:
        buf.ws = None
        buf.kept = False
        buf.ws = torch.empty(max(ws_bytes, 1 << 20), dtype=torch.uint8, device=dev)
        buf.ws_bytes, buf.ws_ptr = buf.ws.numel(), buf.ws.data_ptr()
    if buf.out is None or buf.out.numel() < rec_size * records:
        # the records are written by the kernels straight into pinned host memory
        buf.out = torch.empty(max(rec_size * records, 64 * rec_size), dtype=torch.uint8, pin_memory=True)
        buf.out_ptr = buf.out.data_ptr()
        buf.out_rec = (ctypes.c_char * rec_size).from_address(buf.out_ptr)


def _device_of(job: _Job) -> torch.device:
    g, r = job.gen, job.ref
    if r.device.type == "cuda":
        return r.device
    if g.device.type == "cuda":
        return g.device
    return _device_for(r, g)


_REC_SIZE = ctypes.sizeof(_lib.KvvResult)
_GET_DEVICE = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device
_DEVICES: Dict[int, torch.device] = {}


def _cuda_device(index: int) -> torch.device:
    d = _DEVICES.get(index)
    if d is None:
        d = _DEVICES[index] = torch.device("cuda", index)
    return d


def _launch_single(job: _Job) -> None:
    """One pair through kvv_verdict, with the views and workspace size cached per layout and policy."""
    lib = _lib.load()
    g, r = job.gen, job.ref
    gi, ri = g.get_device(), r.get_device()
    if ri < 0 or gi != ri:
        dev = _device_of(job)
        g = g if g.device == dev else g.to(dev)
        r = r if r.device == dev else r.to(dev)
        ri = dev.index
    ctx = torch.cuda.device(ri) if ri != _GET_DEVICE() else None
    if ctx is not None:
        ctx.__enter__()
    try:
        buf = _stream_buffers(_cuda_device(ri))
        kp = job.kpolicy
        gp, rp = g.data_ptr(), r.data_ptr()
        key = (job.pkey, g.dtype, g.shape, g.stride(), r.stride(), (gp & 15) == 0, (rp & 15) == 0)
        with buf.lock:
            plan = buf.plans.get(key)
            if plan is None:
                gt, rt, _ = _device_views(g, r)
                size = ctypes.c_size_t()
                _lib.check(lib.kvv_workspace_size(gt, rt, kp, ctypes.byref(size)), "kvv_workspace_size")
                plan = (gt, rt, size.value)
                buf.plans[key] = plan
                if len(buf.plans) > _MAX_PLANS:
                    buf.plans.popitem(last=False)
            elif gp:
                plan[0].data = gp
                plan[1].data = rp
            gt, rt, size = plan
            if buf.ws is None or buf.ws_bytes < size or buf.out is None:
                _ensure(buf, torch.device("cuda", ri), size, 1)
            flags = kp.flags
            if buf.kept:
                kp.flags = flags | _lib.FLAG_WS_KEPT
            buf.kept = False  # (until this call has gone through)
            try:
                rc = lib.kvv_verdict(gt, rt, kp, buf.out_ptr, buf.ws_ptr, size, buf.handle)
            finally:
                kp.flags = flags
            _lib.check(rc, "kvv_verdict")
            # host work that needs no record, done while the device runs
            job.tol_text = f"{job.tolerance}"
            buf.stream.synchronize()
            buf.kept = True
            job.record = _lib.KvvResult.from_buffer_copy(buf.out_rec)
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)


def _launch(jobs: List[_Job]) -> None:
    if len(jobs) == 1 and jobs[0].gen.dtype not in _COMPLEX_REAL and jobs[0].gen.dim() <= _lib.MAX_DIMS:
        _launch_single(jobs[0])
        return
    lib = _lib.load()
    dev = _device_for(*[j.ref for j in jobs], *[j.gen for j in jobs])
    keep = []
    gts, rts = [], []
    for j in jobs:
        g = j.gen if j.gen.device == dev else j.gen.to(dev)
        r = j.ref if j.ref.device == dev else j.ref.to(dev)
        gt, rt, held = _device_views(g, r)
        keep += [g, r, *held]
        gts.append(gt)
        rts.append(rt)
    n = len(jobs)
    rec_size = ctypes.sizeof(_lib.KvvResult)
    switch = dev.index != torch.cuda.current_device()
    ctx = torch.cuda.device(dev) if switch else None
    if ctx is not None:
        ctx.__enter__()
    try:
        buf = _stream_buffers(dev)
        stream = buf.stream.cuda_stream
        size = ctypes.c_size_t()
        if n == 1:
            _lib.check(lib.kvv_workspace_size(gts[0], rts[0], jobs[0].kpolicy, ctypes.byref(size)), "kvv_workspace_size")
        else:
            GA, PA = _lib.KvvTensor * n, _lib.KvvPolicy * n
            garr, rarr, parr = GA(*gts), GA(*rts), PA(*[j.kpolicy for j in jobs])
            _lib.check(lib.kvv_batch_workspace_size(n, garr, rarr, parr, ctypes.byref(size)), "kvv_batch_workspace_size")
        with buf.lock:
            _ensure(buf, dev, size.value, n)
            ws, out = buf.ws, buf.out
            if n == 1:
                pol = _lib.KvvPolicy.from_buffer_copy(jobs[0].kpolicy)
                if buf.kept:
                    pol.flags |= _lib.FLAG_WS_KEPT
                buf.kept = False  # (until this call has gone through)
                rc = lib.kvv_verdict(gts[0], rts[0], pol, out.data_ptr(), ws.data_ptr(), size.value, stream)
                _lib.check(rc, "kvv_verdict")
            else:
                buf.kept = False
                rc = lib.kvv_verdict_batch(n, garr, rarr, parr, out.data_ptr(), ws.data_ptr(), size.value, stream)
                _lib.check(rc, "kvv_verdict_batch")
            buf.stream.synchronize()
            buf.kept = True
            host = ctypes.string_at(out.data_ptr(), rec_size * n)
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    del keep
    for i, j in enumerate(jobs):
        j.record = _lib.KvvResult.from_buffer_copy(host, i * rec_size)


# ------------------------------------------------------------ meta assembly
def _mismatch_meta(path: str, correctness_policy, text: str) -> Tuple[bool, List[str], Dict[str, Any]]:
    meta = {"path": path, "correctness_policy": policy_name(correctness_policy), "allclose_pass": False,
            "metric_pass": False, "policy_pass": False, "mismatch_rate": 1.0, "p99_abs": None, "p99_rel": None}
    return False, [text], meta


def _precheck(generated, reference, path, correctness_policy):
    """Shape and dtype guards of GCR:687-710; returns the early result or None."""
    if generated.shape != reference.shape:
        return _mismatch_meta(path, correctness_policy,
                              f"{path}.shape mismatch: expected {tuple(reference.shape)}, got {tuple(generated.shape)}")
    if generated.dtype != reference.dtype:
        return _mismatch_meta(path, correctness_policy,
                              f"{path}.dtype mismatch: expected {reference.dtype}, got {generated.dtype}")
    return None


def _unravel(index: int, shape: Sequence[int]) -> Tuple[int, ...]:
    out = []
    for s in reversed(list(shape)):
        out.append(index % s)
        index //= s
    return tuple(reversed(out))


def _meta_from_record(job: _Job) -> Tuple[bool, List[str], Dict[str, Any]]:
    """Builds GCR:681-786's (ok, details, meta) from the device record."""
    rec = job.record
    path = job.path
    numel = rec.numel
    is_float = job.is_float
    active = job.active
    meta: Dict[str, Any] = {"path": path, "correctness_policy": active}
    if numel == 0 or not is_float:
        meta["cosine_similarity"] = None
        meta["norm_ratio"] = None
    else:
        meta["cosine_similarity"] = _rounded_or_convention(rec.sample_cosine, rec.sample_sum_gg, rec.sample_sum_rr)
        meta["norm_ratio"] = _norm_ratio_value(rec)
    count = rec.mismatch_count
    allclose = count == 0
    meta["mismatch_rate"] = _round4(count / numel) if count else 0.0
    p99_abs = None if numel == 0 else rec.p99_abs
    p99_rel = None if numel == 0 else rec.p99_rel
    meta["p99_abs"] = p99_abs
    meta["p99_rel"] = p99_rel
    meta["allclose_pass"] = allclose
    meta["normal_metric_pass"] = False
    meta["cosine_metric_pass"] = False
    meta["norm_ratio_pass"] = False
    if is_float:
        meta["finite_pass"] = rec.finite_violations == 0
        _near_zero_meta(job, meta, numel)
    metric = False if allclose else _evaluate_tensor_policy(job.ref, meta, job.correctness_policy)
    meta["metric_pass"] = metric
    ok = bool(allclose or metric)
    meta["policy_pass"] = ok
    if numel == 0 or count == 0:
        return True, [], meta
    if job.kpolicy.mode == _lib.MODE_MAX_ABS_DIFF:
        max_abs: Any = int(rec.mismatch_max_abs)
    else:
        max_abs = rec.mismatch_max_abs
    max_rel = rec.mismatch_max_rel
    meta["max_abs"] = float(max_abs)
    meta["max_rel"] = max_rel
    ref = job.ref
    first = "()" if ref.dim() == 0 else _unravel(rec.first_mismatch_index, ref.shape)
    meta["first_mismatch_index"] = first
    if ok:
        return True, [], meta
    # (the policy failed, so policy_pass and metric_pass are False)
    fmt = _format_number
    detail = (
        f"{path}: policy={active}, policy_pass=False, allclose_pass=False, metric_pass=False, "
        f"normal_metric_pass={meta['normal_metric_pass']}, cosine_metric_pass={meta['cosine_metric_pass']}, "
        f"near_zero_abs_pass={meta.get('near_zero_abs_pass')}, {count}/{numel} elements mismatched, "
        f"max_abs={fmt(max_abs)}, max_rel={fmt(max_rel)}, p99_abs={fmt(p99_abs)}, p99_rel={fmt(p99_rel)}, "
        f"cosine_similarity={fmt(meta['cosine_similarity'])}, norm_ratio={fmt(meta['norm_ratio'])}, "
        f"first_mismatch_index={first}, tolerance={job.tol_text if job.tol_text is not None else job.tolerance}"
    )
    return False, [detail], meta


def _round4(x: float) -> float:
    """round(x, 4), exactly, without its decimal conversion where it is not needed.

    round(x, 4) is the double nearest to k / 10^4, k the integer nearest to x * 10^4
    (exactly).  fl(x * 10^4) is within half an ulp of the exact product, so where it
    lies clearly away from a half-integer, floor(fl + 0.5) is that k, and k / 10000.0
    (both exact doubles, k < 2^53) is the nearest double to k / 10^4.  Near a
    half-integer, and for non-finite or huge x, the built-in takes over."""
    y = x * 10000.0
    if -4.0e15 < y < 4.0e15:
        k = math.floor(y + 0.5)
        t = y - k
        if -0.4999 < t < 0.4999:
            return k / 10000.0 if k else math.copysign(0.0, x)
    return round(x, 4)


def _rounded_or_convention(cos: float, gg: float, rr: float) -> float:
    """GCR:364-372: exact 1.0 / 0.0 for zero norms, else round(cosine, 4).  (A norm is the square root of
    a sum of squares, which is >= 0, -0.0 or NaN: the norm is zero exactly when the sum is.)"""
    g_zero = gg == 0.0
    r_zero = rr == 0.0
    if g_zero and r_zero:
        return 1.0
    if g_zero or r_zero:
        return 0.0
    return _round4(float(cos))


def _norm_ratio_value(rec) -> float:
    """GCR:383-393."""
    g_zero = rec.sample_sum_gg == 0.0
    r_zero = rec.sample_sum_rr == 0.0
    if g_zero and r_zero:
        return 1.0
    if g_zero:
        return 0.0
    if r_zero:
        return float("inf")
    return _round4(float(rec.sample_norm_ratio))


def _near_zero_meta(job: _Job, meta: Dict[str, Any], numel: int) -> None:
    """GCR:481-548 from the device counts (diagnostic: the verdict never reads it)."""
    meta["near_zero_abs_pass"] = False
    th = job.near_thresholds
    if th is None:
        return
    rec = job.record
    near = rec.near_zero_count
    far = rec.far_count
    far_mm = rec.far_mismatch_count
    meta["near_zero_abs"] = float(th["near_zero_abs"])
    meta["near_zero_rate"] = _round4(near / numel) if near else 0.0
    meta["far_mismatch_rate"] = _round4(far_mm / far) if far_mm else 0.0
    if near == 0:
        meta["near_zero_p99_abs"] = None
        meta["near_zero_mean_abs"] = None
        meta["near_zero_bad_rate"] = 0.0
        return
    meta["near_zero_p99_abs"] = rec.near_zero_p99_abs
    meta["near_zero_mean_abs"] = rec.near_zero_mean_abs
    meta["near_zero_bad_rate"] = _round4(rec.near_zero_bad_count / near)
    meta["near_zero_abs_pass"] = bool(
        meta.get("finite_pass")
        and far_mm == 0
        and _threshold_pass(meta.get("near_zero_p99_abs"), th.get("max_near_zero_p99_abs"))
        and _threshold_pass(meta.get("near_zero_mean_abs"), th.get("max_near_zero_mean_abs"))
        and _threshold_pass(meta.get("near_zero_bad_rate"), th.get("max_near_zero_bad_rate"))
    )


# ------------------------------------------------------------ public surface
def _compare_tensors(
    generated,
    reference,
    path: str,
    tolerance_policy: Optional[Dict[str, Any]] = None,
    correctness_policy: Optional[Dict[str, Any]] = None,
    max_samples: int = MAX_SAMPLES,
) -> Tuple[bool, List[str], Dict[str, Any]]:
    """GCR:672-786 on the GPU: (policy_pass, [detail] if failing, meta)."""
    early = _precheck(generated, reference, path, correctness_policy)
    if early is not None:
        return early
    job = _Job(generated, reference, path, tolerance_policy, correctness_policy, max_samples)
    _run_jobs([job])
    return _meta_from_record(job)


def _walk(generated, reference, path, tolerance_policy, correctness_policy, max_samples, plan: list) -> None:
    """GCR:789-833's recursion, recording tensor jobs and structural results in visiting order."""
    if isinstance(generated, torch.Tensor) and isinstance(reference, torch.Tensor):
        early = _precheck(generated, reference, path, correctness_policy)
        if early is not None:
            plan.append(("done", early[0], early[1], [early[2]]))
        else:
            plan.append(("job", _Job(generated, reference, path, tolerance_policy, correctness_policy, max_samples)))
        return
    if isinstance(generated, (list, tuple)) and isinstance(reference, (list, tuple)):
        if len(generated) != len(reference):
            plan.append(("done", False,
                         [f"{path} length mismatch: expected {len(reference)}, got {len(generated)}"], []))
            return
        for index, (g, r) in enumerate(zip(generated, reference)):
            _walk(g, r, f"{path}[{index}]", tolerance_policy, correctness_policy, max_samples, plan)
        return
    if generated == reference:
        plan.append(("done", True, [], []))
        return
    plan.append(("done", False,
                 [f"{path} type/value mismatch: expected {type(reference).__name__}, got {type(generated).__name__}"],
                 []))


def _compare_outputs(
    generated: Any,
    reference: Any,
    path: str = "output",
    tolerance_policy: Optional[Dict[str, Any]] = None,
    correctness_policy: Optional[Dict[str, Any]] = None,
    max_samples: int = MAX_SAMPLES,
) -> Tuple[bool, List[str], List[Dict[str, Any]]]:
    """GCR:789-833: every tensor pair of a nested output in one batched device call."""
    plan: list = []
    _walk(generated, reference, path, tolerance_policy, correctness_policy, max_samples, plan)
    _run_jobs([p[1] for p in plan if p[0] == "job"])
    all_ok, details, metas = True, [], []
    for p in plan:
        if p[0] == "job":
            ok, d, m = _meta_from_record(p[1])
            m = [m]
        else:
            _, ok, d, m = p
        all_ok = all_ok and ok
        details.extend(d)
        metas.extend(m)
    return all_ok, details, metas


def verdict_record(generated: torch.Tensor, reference: torch.Tensor, tolerance_policy=None, correctness_policy=None,
                   max_samples: int = MAX_SAMPLES) -> Dict[str, Any]:
    """The full device record of one pair (reference fields and extensions) as a dict."""
    if generated.shape != reference.shape or generated.dtype != reference.dtype:
        raise ValueError("verdict_record needs tensors of equal shape and dtype")
    job = _Job(generated, reference, "output", tolerance_policy, correctness_policy, max_samples, fp8_errors=False)
    _run_jobs([job])
    return job.record.to_dict()


def verdict_records(pairs, tolerance_policy=None, correctness_policy=None, max_samples: int = MAX_SAMPLES):
    """Records of many pairs from one batched device call.  A pair is (generated, reference) or
    (generated, reference, tolerance_policy): the third item, when given, is that pair's own
    tolerance table in place of ``tolerance_policy``."""
    jobs = []
    for i, p in enumerate(pairs):
        g, r = p[0], p[1]
        tol = p[2] if len(p) > 2 and p[2] is not None else tolerance_policy
        jobs.append(_Job(g, r, f"output[{i}]", tol, correctness_policy, max_samples, fp8_errors=False))
    _run_jobs(jobs)
    return [j.record.to_dict() for j in jobs]
