"""ctypes binding of libkvv.so (declared in include/kvv.h).

The library must have been built (``python -m kernelverse_amd.build`` or
``__graft_entry__.build()``); there is no fallback: every verdict entry point
raises ``KvvLibraryError`` when the shared object cannot be loaded.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_int32, c_int64, c_uint32, c_uint64, c_void_p, c_size_t, c_char_p, POINTER
from pathlib import Path

LIB_PATH = Path(os.environ.get("KVV_LIB", Path(__file__).resolve().parent / "libkvv.so"))

MAX_DIMS = 8
HIST_BUCKETS = 16

# enum kvv_dtype
F32, F16, BF16, F64, F8E4M3FN, F8E5M2, I8, U8, I16, I32, I64, BOOL, U16, U32, U64 = range(15)
# enum kvv_mode
MODE_ISCLOSE, MODE_MAX_ABS_DIFF = 0, 1
FLAG_NEAR_ZERO = 0x1
FLAG_NEAR_EXACT = 0x2
FLAG_WS_KEPT = 0x4
# kvv_result.status value of ABI version 1 that kvv_verdict no longer returns (KVV_STATUS_NEAR_RETRY)
STATUS_NEAR_RETRY = 1

STATUS_NAMES = {0: "OK", -1: "INVALID", -2: "WORKSPACE", -3: "HIP", -4: "UNSUPPORTED"}


class KvvLibraryError(RuntimeError):
    """libkvv.so is missing or a call into it failed."""


class KvvTensor(ctypes.Structure):
    _fields_ = [
        ("data", c_void_p),
        ("dtype", c_int32),
        ("ndim", c_int32),
        ("sizes", c_int64 * MAX_DIMS),
        ("strides", c_int64 * MAX_DIMS),
    ]


class KvvPolicy(ctypes.Structure):
    _fields_ = [
        ("mode", c_int32),
        ("flags", c_uint32),
        ("rtol", c_double),
        ("atol", c_double),
        ("max_abs_diff", c_int64),
        ("near_zero_abs", c_double),
        ("near_zero_bad_abs", c_double),
        ("max_samples", c_int64),
    ]


class KvvResult(ctypes.Structure):
    _fields_ = [
        ("numel", c_int64),
        ("mismatch_count", c_int64),
        ("first_mismatch_index", c_int64),
        ("mismatch_max_abs", c_double),
        ("mismatch_max_rel", c_double),
        ("sample_count", c_int64),
        ("p99_abs", c_double),
        ("p99_rel", c_double),
        ("sample_sum_gg", c_double),
        ("sample_sum_rr", c_double),
        ("sample_sum_gr", c_double),
        ("sample_cosine", c_double),
        ("sample_norm_ratio", c_double),
        ("finite_violations", c_int64),
        ("first_finite_violation", c_int64),
        ("nan_gen", c_int64),
        ("nan_ref", c_int64),
        ("posinf_gen", c_int64),
        ("posinf_ref", c_int64),
        ("neginf_gen", c_int64),
        ("neginf_ref", c_int64),
        ("near_zero_count", c_int64),
        ("far_count", c_int64),
        ("far_mismatch_count", c_int64),
        ("near_zero_bad_count", c_int64),
        ("near_zero_sample_count", c_int64),
        ("near_zero_p99_abs", c_double),
        ("near_zero_mean_abs", c_double),
        ("max_abs", c_double),
        ("max_abs_index", c_int64),
        ("max_rel", c_double),
        ("max_rel_index", c_int64),
        ("ulp_hist", c_uint64 * HIST_BUCKETS),
        ("nan_pairs", c_int64),
        ("sum_gg", c_double),
        ("sum_rr", c_double),
        ("sum_gr", c_double),
        ("sum_dd", c_double),
        ("rel_l2", c_double),
        ("cosine", c_double),
        ("status", c_int32),
        ("reserved", c_int32),
    ]

    def to_dict(self):
        out = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            out[name] = list(v) if name == "ulp_hist" else v
        return out


EXPORTED = ("kvv_abi_version", "kvv_last_error", "kvv_workspace_size", "kvv_verdict", "kvv_verdict_timed",
            "kvv_verdict_noalloc", "kvv_batch_workspace_size", "kvv_verdict_batch")

# the fixed workspace of kvv_verdict_noalloc (bytes)
NOALLOC_SCRATCH_BYTES = 64 << 20

_lib = None


def load() -> ctypes.CDLL:
    """Load libkvv.so once; raise KvvLibraryError if it is absent or incompatible."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise KvvLibraryError(
            f"{LIB_PATH} is not built: run `python -m kernelverse_amd.build` (the verdict has no CPU fallback)")
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise KvvLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
    lib.kvv_abi_version.restype = c_int32
    lib.kvv_abi_version.argtypes = []
    lib.kvv_last_error.restype = c_char_p
    lib.kvv_last_error.argtypes = []
    lib.kvv_workspace_size.restype = c_int32
    lib.kvv_workspace_size.argtypes = [POINTER(KvvTensor), POINTER(KvvTensor), POINTER(KvvPolicy), POINTER(c_size_t)]
    lib.kvv_verdict.restype = c_int32
    lib.kvv_verdict.argtypes = [POINTER(KvvTensor), POINTER(KvvTensor), POINTER(KvvPolicy), c_void_p, c_void_p,
                                c_size_t, c_void_p]
    lib.kvv_verdict_timed.restype = c_int32
    lib.kvv_verdict_timed.argtypes = [POINTER(KvvTensor), POINTER(KvvTensor), POINTER(KvvPolicy), c_void_p, c_void_p,
                                      c_size_t, c_void_p, c_void_p, c_void_p]
    lib.kvv_verdict_noalloc.restype = c_int32
    lib.kvv_verdict_noalloc.argtypes = [POINTER(KvvTensor), POINTER(KvvTensor), POINTER(KvvPolicy), c_void_p,
                                        c_void_p]
    lib.kvv_batch_workspace_size.restype = c_int32
    lib.kvv_batch_workspace_size.argtypes = [c_int32, POINTER(KvvTensor), POINTER(KvvTensor), POINTER(KvvPolicy),
                                             POINTER(c_size_t)]
    lib.kvv_verdict_batch.restype = c_int32
    lib.kvv_verdict_batch.argtypes = [c_int32, POINTER(KvvTensor), POINTER(KvvTensor), POINTER(KvvPolicy), c_void_p,
                                      c_void_p, c_size_t, c_void_p]
    if lib.kvv_abi_version() != 1:
        raise KvvLibraryError(f"{LIB_PATH} has ABI version {lib.kvv_abi_version()}, expected 1")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().kvv_last_error().decode("utf-8", "replace")
        raise KvvLibraryError(f"{what} failed ({STATUS_NAMES.get(rc, rc)}): {msg}")
