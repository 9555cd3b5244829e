"""Load the golden verdict fixtures written by ``tests/golden/make_golden.py``."""

from __future__ import annotations

import base64
import hashlib
import json
import math
from pathlib import Path
from typing import Any, Dict, List

import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

_DTYPES = {str(d).replace("torch.", ""): d for d in (
    torch.float32, torch.float16, torch.bfloat16, torch.float64, torch.int8, torch.uint8, torch.int16,
    torch.int32, torch.int64, torch.bool, torch.float8_e4m3fn, torch.float8_e5m2, torch.float8_e4m3fnuz,
    torch.float8_e5m2fnuz, torch.uint16, torch.uint32, torch.uint64, torch.complex64)}


def _storages() -> Dict[str, bytes]:
    out: Dict[str, bytes] = {}
    for p in sorted(GOLDEN.glob("tensors_*.json")):
        for k, v in json.loads(p.read_text()).items():
            out[k] = base64.b64decode(v)
    return out


def decode_tensor(spec: Dict[str, Any], storages: Dict[str, bytes]) -> torch.Tensor:
    dtype = _DTYPES[spec["dtype"]]
    raw = bytearray(storages[spec["storage"]])
    base = torch.frombuffer(raw, dtype=torch.uint8) if raw else torch.zeros(0, dtype=torch.uint8)
    base = base.view(dtype) if dtype != torch.bool else base.view(torch.bool)
    return base.as_strided(spec["size"], spec["stride"], spec["offset"])


def decode_value(v, storages):
    if isinstance(v, dict):
        if "__tensor__" in v:
            return decode_tensor(v["__tensor__"], storages)
        if "__tuple__" in v:
            return tuple(decode_value(x, storages) for x in v["__tuple__"])
        return {k: decode_value(x, storages) for k, x in v.items()}
    if isinstance(v, list):
        return [decode_value(x, storages) for x in v]
    return v


def tensor_sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b"").hexdigest()


def load_cases(include_recipes: bool = True) -> List[Dict[str, Any]]:
    """All verdict cases with ``generated``/``reference`` decoded to CPU tensors (recipes regenerated)."""
    from kernelverse_amd import synth

    storages = _storages()
    cases = []
    for p in sorted(GOLDEN.glob("verdict_cases_*.json")):
        for c in json.loads(p.read_text()):
            if "recipe" in c:
                if not include_recipes:
                    continue
                g, r = getattr(synth, c["recipe"]["fn"])(**c["recipe"]["kwargs"])
                if [tensor_sha256(g), tensor_sha256(r)] != c["sha256"]:
                    raise AssertionError(f"recipe {c['name']} no longer reproduces its recorded bytes")
                c["generated"], c["reference"] = g, r
            else:
                c["generated"] = decode_value(c["generated"], storages)
                c["reference"] = decode_value(c["reference"], storages)
            c["expected"] = decode_value(c["expected"], storages)
            cases.append(c)
    return cases


def load_policy_fixture() -> Dict[str, Any]:
    d = json.loads((GOLDEN / "policy_resolution.json").read_text())
    tables = d["tables"]

    def expand(v):
        if isinstance(v, dict):
            if set(v) == {"__table__"}:
                return tables[v["__table__"]]
            return {k: expand(x) for k, x in v.items()}
        if isinstance(v, list):
            return [expand(x) for x in v]
        return v

    return {k: expand(v) for k, v in d.items() if k != "tables"}


def same_value(a, b) -> bool:
    """Equality that treats NaN == NaN and compares tuples/lists elementwise."""
    if isinstance(a, float) and isinstance(b, float) and math.isnan(a) and math.isnan(b):
        return True
    if isinstance(a, (list, tuple)) and isinstance(b, (list, tuple)):
        return type(a) is type(b) and len(a) == len(b) and all(same_value(x, y) for x, y in zip(a, b))
    if isinstance(a, dict) and isinstance(b, dict):
        return list(a.keys()) == list(b.keys()) and all(same_value(a[k], b[k]) for k in a)
    if type(a) is not type(b) and not (isinstance(a, (int, float)) and isinstance(b, (int, float))
                                       and not isinstance(a, bool) and not isinstance(b, bool)):
        return False
    return a == b


def diff_meta(a: Dict[str, Any], b: Dict[str, Any]) -> List[str]:
    out = []
    if list(a.keys()) != list(b.keys()):
        out.append(f"key order {list(a.keys())} != {list(b.keys())}")
    for k in a:
        if k in b and not same_value(a[k], b[k]):
            out.append(f"{k}: {a[k]!r} != {b[k]!r}")
    return out


def load_host_logic() -> Dict[str, Any]:
    """Random-mode configuration and summary, timing payload and perf-seed fixtures."""
    return json.loads((GOLDEN / "host_logic.json").read_text())


def load_finalize_cases() -> List[Dict[str, Any]]:
    out: List[Dict[str, Any]] = []
    for p in sorted(GOLDEN.glob("finalize_cases_*.json")):
        out += json.loads(p.read_text())
    return out


def load_trial_cases() -> List[Dict[str, Any]]:
    """Reference trial results (GCR:1281-1322 run on the CPU) for the pairs of ``trial_models``."""
    cases = json.loads((GOLDEN / "trial_cases.json").read_text())
    for c in cases:
        c["expected"] = decode_value(c["expected"], {})
    return cases
