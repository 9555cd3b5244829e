"""Write golden verdict fixtures by running the reference's own verdict code.

Run in the build container only (the GPU box has no reference):

    python tests/golden/make_golden.py /root/reference

It imports KernelVerse ``runner.generated_correctness_runner`` (GCR) and
``runner.correctness_policy`` (CP) read-only, with bytecode writing disabled,
and records for each case the inputs (raw storage bytes plus the view, or a
seeded recipe with the SHA-256 of the bytes it makes) and what the reference
returns: ``_compare_outputs`` -> (ok, details, metas), or the exception it
raises.  It also records ``resolve_correctness_policy`` and
``_operator_tolerance_policy`` for every operator ``config.json`` the
reference ships, and ``_correctness_criteria`` for each policy kind.

The fixtures pin the branching and reporting logic (key order, rounding,
policy rules, detail strings) that no library routine or closed form pins.

``--part host`` writes only the fixtures of the code around the verdict:
``host_logic.json`` (random-mode configuration and summary GCR:250-302; the
timing payload and per-operator perf seed of ``utils/performance.py``),
``finalize_cases_*.json`` (case finalisation GCR:999-1040, 1760-1810) and
``trial_cases.json`` (``_run_correctness_trial_once`` GCR:1281-1322 run on the
CPU with the operator pairs of ``tests/trial_models.py``).
"""

from __future__ import annotations

import base64
import hashlib
import json
import math
import os
import sys
import traceback
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from kernelverse_amd import synth  # noqa: E402

MAX_FIXTURE_BYTES = 64 * 1024


# ------------------------------------------------------------- encoding
STORAGES = {}


def encode_tensor(t: torch.Tensor) -> dict:
    """View parameters plus the SHA-256 key of the raw storage bytes (kept once in ``tensors_*.json``)."""
    raw = bytes(t.untyped_storage())
    key = hashlib.sha256(raw).hexdigest()[:24]
    STORAGES[key] = base64.b64encode(raw).decode("ascii")
    return {
        "dtype": str(t.dtype).replace("torch.", ""),
        "size": list(t.shape),
        "stride": list(t.stride()),
        "offset": int(t.storage_offset()),
        "storage": key,
    }


def tensor_sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b"").hexdigest()


def encode_value(v):
    if isinstance(v, torch.Tensor):
        return {"__tensor__": encode_tensor(v)}
    if isinstance(v, tuple):
        return {"__tuple__": [encode_value(x) for x in v]}
    if isinstance(v, list):
        return [encode_value(x) for x in v]
    if isinstance(v, dict):
        return {k: encode_value(x) for k, x in v.items()}
    return v


# ------------------------------------------------------------- cases
def _t(x, dtype):
    return torch.tensor(x, dtype=dtype)


def tensor_cases():
    """(name, generated, reference, tolerance_policy, correctness_policy_spec) with small inputs."""
    cases = []
    g, r = synth.fp32_noise_pair(2048, seed=11)
    cases.append(("fp32_noise_default_tol", g, r, None, None))
    cases.append(("fp32_noise_c0_tol_strict", g, r, {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, None))
    cases.append(("fp32_noise_c0_tol_tolerant", g, r, {"FP32": {"rtol": 1e-5, "atol": 1e-5}},
                  {"category": "gemm", "op_name": "matmul"}))
    cases.append(("fp32_noise_c0_tol_cosine", g, r, {"FP32": {"rtol": 1e-5, "atol": 1e-5}},
                  {"category": "attention", "op_name": "sdpa"}))
    g2, r2 = synth.fp32_noise_pair(3000, seed=12, noise=1e-3, frac=0.2, lo=0.1, hi=2.0)
    cases.append(("fp32_heavy_noise_tolerant", g2, r2, None, {"category": "gemm", "op_name": "matmul"}))
    cases.append(("fp32_heavy_noise_cosine", g2, r2, None, {"category": "attention", "op_name": "sdpa"}))
    cases.append(("fp32_scaled_cosine_ratio", g2 * 1.01, r2, None, {"category": "attention", "op_name": "sdpa"}))
    cases.append(("fp32_transposed", g2[:2000].reshape(40, 50).t(), r2[:2000].reshape(40, 50).t(),
                  {"FP32": {"rtol": 1e-4, "atol": 1e-4}}, None))
    gb, rb = synth.code_flip_pair(4096, seed=13, dtype=torch.bfloat16, p1=0.05, p3=0.01)
    cases.append(("bf16_flips_default", gb, rb, None, None))
    cases.append(("bf16_flips_c1_tol_strict", gb, rb, {"BF16": {"rtol": 1.6e-2, "atol": 1e-2}}, None))
    cases.append(("bf16_flips_tight_tolerant", gb, rb, {"BF16": {"rtol": 1e-3, "atol": 1e-4}},
                  {"category": "normalization", "op_name": "layernorm"}))
    cases.append(("bf16_flips_tight_cosine", gb, rb, {"BF16": {"rtol": 1e-3, "atol": 1e-4}},
                  {"category": "attention", "op_name": "sdpa"}))
    gb2, rb2 = synth.code_flip_pair(4096, seed=14, dtype=torch.bfloat16, std=0.1, p1=0.3, p3=0.05)
    cases.append(("bf16_small_values_tolerant", gb2, rb2, {"BF16": {"rtol": 1e-3, "atol": 1e-4}},
                  {"category": "moe", "op_name": "router", "config": {"thresholds": {"bf16": {"max_p99_rel": 0.5}}}}))
    gh, rh = synth.code_flip_pair(4096, seed=15, dtype=torch.float16, std=1.0, p1=0.1, p3=0.01)
    cases.append(("fp16_flips_tolerant", gh, rh, {"FP16": {"rtol": 1e-4, "atol": 1e-5}},
                  {"category": "gemm", "op_name": "matmul"}))
    gn, rn = synth.fp16_nonfinite_pair(16, 64, 72, seed=16, p_nan=0.02, p_inf=0.02, breaks=3)
    cases.append(("fp16_nonfinite_strided_strict", gn, rn, {"FP16": {"rtol": 1e-3, "atol": 1e-3}}, None))
    cases.append(("fp16_nonfinite_strided_tolerant", gn, rn, {"FP16": {"rtol": 1e-3, "atol": 1e-3}},
                  {"category": "gemm", "op_name": "matmul"}))
    gn2, rn2 = synth.fp16_nonfinite_pair(8, 32, 40, seed=17, p_nan=0.03, p_inf=0.03, breaks=0)
    cases.append(("fp16_nonfinite_pattern_ok_cosine", gn2, rn2, None, {"category": "attention", "op_name": "sdpa"}))
    gi, ri = synth.int8_pair(4096, seed=18, changed=40)
    cases.append(("int8_default", gi, ri, None, None))
    cases.append(("int8_zero_tol_tolerant", gi, ri, {"INT8": {"max_abs_diff": 0}}, {"category": "gemm", "op_name": "x"}))
    cases.append(("uint8_default", gi.view(torch.uint8), ri.view(torch.uint8), None, None))
    i32r = torch.arange(-300, 300, dtype=torch.int32) * 7919
    i32g = i32r.clone()
    i32g[::37] += 3
    i32g[5] = 2**31 - 1
    i32r[5] = -2**31
    cases.append(("int32_wrap", i32g, i32r, None, None))
    i64r = torch.arange(0, 512, dtype=torch.int64) * (2**33 + 5)
    i64g = i64r.clone()
    i64g[3::50] += 2**32
    i64g[7] += 1
    cases.append(("int64_low32_compare", i64g, i64r, {"INT64": {"max_abs_diff": 0}}, None))
    cases.append(("int16_default", (i32g % 30000).to(torch.int16), (i32r % 30000).to(torch.int16), None, None))
    bg = torch.arange(100) % 3 == 0
    br = torch.arange(100) % 4 == 0
    cases.append(("bool_default", bg, br, None, None))
    cases.append(("int32_with_float_tolerance", i32g[:64], i32r[:64], {"INT32": {"rtol": 1e-3, "atol": 2.0}}, None))
    cases.append(("fp16_with_int_tolerance", gh[:512] * 300, rh[:512] * 300, {"FP16": {"max_abs_diff": 1}}, None))
    cases.append(("shape_mismatch", torch.zeros(3, 4), torch.zeros(4, 3), None, None))
    cases.append(("dtype_mismatch", torch.zeros(4, dtype=torch.float16), torch.zeros(4), None, None))
    cases.append(("empty_fp32", torch.zeros(0, 5), torch.zeros(0, 5), None, None))
    cases.append(("empty_int32", torch.zeros(0, dtype=torch.int32), torch.zeros(0, dtype=torch.int32), None, None))
    cases.append(("scalar_equal", torch.tensor(1.5), torch.tensor(1.5), None, None))
    cases.append(("scalar_mismatch", torch.tensor(2.5), torch.tensor(1.5), None, {"category": "gemm", "op_name": "x"}))
    cases.append(("all_equal", r2.clone(), r2, None, None))
    cases.append(("all_zero", torch.zeros(300), torch.zeros(300), None, {"category": "attention", "op_name": "x"}))
    cases.append(("negated", -r2, r2, None, {"category": "attention", "op_name": "x"}))
    cases.append(("zero_reference", r2, torch.zeros_like(r2), None, {"category": "attention", "op_name": "x"}))
    cases.append(("zero_generated", torch.zeros_like(r2), r2, None, {"category": "attention", "op_name": "x"}))
    specials = [0.0, -0.0, 1e-45, -1e-45, 1e-38, 3.4e38, -3.4e38, float("inf"), float("-inf"), float("nan"), 1.0, -1.0]
    sg, sr = [], []
    for a in specials:
        for b in specials:
            sg.append(a)
            sr.append(b)
    cases.append(("fp32_special_table", _t(sg, torch.float32), _t(sr, torch.float32),
                  {"FP32": {"rtol": 1e-3, "atol": 1e-3}}, {"category": "gemm", "op_name": "x"}))
    cases.append(("fp32_special_table_zero_tol", _t(sg, torch.float32), _t(sr, torch.float32),
                  {"FP32": {"rtol": 0.0, "atol": 0.0}}, None))
    cases.append(("bf16_special_table", _t(sg, torch.float32).to(torch.bfloat16), _t(sr, torch.float32).to(torch.bfloat16),
                  None, {"category": "gemm", "op_name": "x"}))
    nan_g = r2[:256].clone()
    nan_g[17] = float("nan")
    cases.append(("fp32_one_nan_in_gen", nan_g, r2[:256], None, {"category": "gemm", "op_name": "x"}))
    both_nan = r2[:256].clone()
    both_nan[[3, 9]] = float("nan")
    cases.append(("fp32_matching_nans", both_nan, both_nan.clone(), None, {"category": "gemm", "op_name": "x"}))
    f8g, f8r = synth.fp8_pair(1024, seed=19, p=0.05)
    cases.append(("fp8_e4m3fn_reference_raises", f8g, f8r, None, None))
    # float8_e5m2 has a torch-CPU isfinite, so the reference returns a verdict for it
    e5g, e5r = synth.code_flip_pair(2048, seed=41, dtype=torch.float8_e5m2, std=4.0, p1=0.05, p3=0.01)
    cases.append(("fp8_e5m2_flips_default", e5g, e5r, None, None))
    cases.append(("fp8_e5m2_flips_cosine", e5g, e5r, None, {"category": "attention", "op_name": "x"}))
    cases.append(("fp8_e5m2_flips_tolerant", e5g, e5r, {"FLOAT8_E5M2": {"rtol": 0.25, "atol": 0.1}},
                  {"category": "gemm", "op_name": "x"}))
    e5codes = torch.arange(256, dtype=torch.int16).to(torch.uint8)
    e5gc = e5codes.clone()
    e5gc[0x7C] = 0xFC      # +inf -> -inf
    e5gc[0x7E] = 0x3C      # NaN -> 1.0
    e5gc[0x3C] = 0x7D      # 1.0 -> NaN
    e5gc[0xFC] = 0xFE      # -inf -> NaN
    e5gc[0x10:0x18] += 1   # finite one-code steps
    cases.append(("fp8_e5m2_nonfinite_codes", e5gc.view(torch.float8_e5m2), e5codes.view(torch.float8_e5m2),
                  None, {"category": "gemm", "op_name": "x"}))
    fz = torch.tensor([0.5, 1.0, -2.0, 3.0])
    cases.append(("fp8_e4m3fnuz_reference_raises", fz.to(torch.float8_e4m3fnuz), (fz * 1.5).to(torch.float8_e4m3fnuz),
                  None, None))
    cases.append(("fp8_e5m2fnuz_reference_raises", fz.to(torch.float8_e5m2fnuz), (fz * 1.5).to(torch.float8_e5m2fnuz),
                  None, None))
    # unsigned and complex integer-branch inputs: int32 casts wrap, rel_diff divides by the float32 value
    # (unsigned tensors built in numpy: torch-CPU has no arithmetic kernels for them)
    u16 = (np.arange(0, 1024, dtype=np.int64) * 64 + 3).astype(np.uint16)
    u16g = u16.copy()
    u16g[::29] += 2
    cases.append(("uint16_default", torch.from_numpy(u16g), torch.from_numpy(u16), None, None))
    cases.append(("uint16_max_abs_diff", torch.from_numpy(u16g), torch.from_numpy(u16), {"UINT16": {"max_abs_diff": 1}},
                  None))
    u32 = (np.arange(0, 1024, dtype=np.int64) * 4194301 + 17).astype(np.uint32)
    u32g = u32.copy()
    u32g[::31] += 5
    u32g[7] = 0
    u32[7] = 2**31 + 9
    cases.append(("uint32_wrap", torch.from_numpy(u32g), torch.from_numpy(u32), None, None))
    u64 = np.arange(0, 512, dtype=np.uint64) * np.uint64(2**54 + 77)
    u64g = u64.copy()
    u64g[3::50] += np.uint64(2**32)
    u64g[11] += np.uint64(9)
    cases.append(("uint64_low32_compare", torch.from_numpy(u64g), torch.from_numpy(u64), {"UINT64": {"max_abs_diff": 2}},
                  None))
    cre = torch.from_numpy(np.linspace(-300.0, 300.0, 600).astype(np.float32))
    cplx_r = torch.complex(cre, cre * 0.5)
    cplx_g = torch.complex(cre + (torch.arange(600) % 7 == 0).float() * 2.5, cre * -0.25)
    cases.append(("complex64_real_part", cplx_g, cplx_r, None, None))
    # more than eight dimensions: one contiguous, one permuted view
    hg, hr = synth.fp32_noise_pair(2048, seed=42, noise=1e-4, frac=0.05)
    cases.append(("fp32_nine_dims", hg[:512].reshape((2,) * 9), hr[:512].reshape((2,) * 9),
                  {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, {"category": "gemm", "op_name": "x"}))
    perm = (9, 0, 8, 1, 7, 2, 6, 3, 5, 4)
    cases.append(("fp32_ten_dims_permuted", hg[:1024].reshape((2,) * 10).permute(perm),
                  hr[:1024].reshape((2,) * 10).permute(perm), {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, None))
    return cases


def structure_cases():
    """``_compare_outputs`` over tuples, lists and non-tensor leaves."""
    g, r = synth.fp32_noise_pair(512, seed=21)
    gi, ri = synth.int8_pair(256, seed=22, changed=3)
    return [
        ("tuple_two_tensors", (g, gi), (r, ri), None, None),
        ("list_nested", [g, [gi, g[:10]]], [r, [ri, r[:10]]], None, {"category": "gemm", "op_name": "x"}),
        ("length_mismatch", (g, gi), (r,), None, None),
        ("non_tensor_equal", (g, 3), (r, 3), None, None),
        ("non_tensor_unequal", (g, 3), (r, 4), None, None),
        ("tensor_vs_int", g, 3, None, None),
    ]


def recipe_cases():
    """Cases too large to store: seeded recipes (+ SHA-256 of the bytes they make)."""
    return [
        ("fp32_sampled_1p5m", {"fn": "fp32_noise_pair", "kwargs": {"n": 1_500_000, "seed": 31}},
         {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, {"category": "gemm", "op_name": "x"}),
        ("bf16_sampled_near_zero_3m", {"fn": "code_flip_pair", "kwargs": {"n": 3_000_000, "seed": 32, "std": 0.5,
                                                                          "p1": 0.05, "p3": 0.01}},
         {"BF16": {"rtol": 1e-3, "atol": 1e-4}}, {"category": "gemm", "op_name": "x"}),
        # the C0 benchmark configuration at its own size, under each policy kind
        ("c0_fp32_1m_strict", {"fn": "fp32_noise_pair", "kwargs": {"n": 1_048_576, "seed": 0}},
         {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, None),
        ("c0_fp32_1m_tolerant", {"fn": "fp32_noise_pair", "kwargs": {"n": 1_048_576, "seed": 0}},
         {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, {"category": "gemm", "op_name": "x"}),
        ("c0_fp32_1m_cosine", {"fn": "fp32_noise_pair", "kwargs": {"n": 1_048_576, "seed": 0}},
         {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, {"category": "attention", "op_name": "x"}),
        # a C1-like bf16 pair under the tolerant policy (near-zero diagnostics over a sampled compaction)
        ("bf16_c1_model_tolerant_4m", {"fn": "code_flip_pair", "kwargs": {"n": 4_194_304, "seed": 33}},
         {"BF16": {"rtol": 1.6e-2, "atol": 1e-2}}, {"category": "gemm", "op_name": "x"}),
    ]


def run_recipe(recipe):
    fn = getattr(synth, recipe["fn"])
    kwargs = dict(recipe["kwargs"])
    return fn(**kwargs)


# ------------------------------------------------------------- driver
def main(reference_root: str) -> None:
    sys.dont_write_bytecode = True
    sys.path.insert(0, reference_root)
    import runner.correctness_policy as cp  # noqa: E402
    import runner.generated_correctness_runner as gcr  # noqa: E402

    def policy_for(spec):
        if spec is None:
            return None
        full = {"category": spec.get("category"), "op_name": spec.get("op_name"), "config": spec.get("config") or {}}
        return cp.resolve_correctness_policy(full)

    def run(gen, ref, tol, spec):
        pol = policy_for(spec)
        try:
            ok, details, metas = gcr._compare_outputs(gen, ref, tolerance_policy=tol, correctness_policy=pol)
            return {"ok": ok, "details": details, "metas": encode_value(metas)}, pol
        except Exception as exc:  # the reference raising is itself the expected result
            return {"raises": type(exc).__name__, "message": str(exc)}, pol

    out_cases = []
    for name, g, r, tol, spec in tensor_cases() + structure_cases():
        result, pol = run(g, r, tol, spec)
        out_cases.append({"name": name, "generated": encode_value(g), "reference": encode_value(r),
                          "tolerance_policy": tol, "correctness_policy": pol, "expected": result})
    for name, recipe, tol, spec in recipe_cases():
        g, r = run_recipe(recipe)
        result, pol = run(g, r, tol, spec)
        out_cases.append({"name": name, "recipe": recipe, "sha256": [tensor_sha256(g), tensor_sha256(r)],
                          "tolerance_policy": tol, "correctness_policy": pol, "expected": result})

    def shard(items, size_of):
        chunks, cur, cur_bytes = [], [], 0
        for it in items:
            size = size_of(it)
            if cur and cur_bytes + size > MAX_FIXTURE_BYTES:
                chunks.append(cur)
                cur, cur_bytes = [], 0
            cur.append(it)
            cur_bytes += size
        if cur:
            chunks.append(cur)
        return chunks

    for pattern in ("verdict_cases_*.json", "tensors_*.json"):
        for old in HERE.glob(pattern):
            old.unlink()
    chunks = shard(out_cases, lambda c: len(json.dumps(c)))
    for i, chunk in enumerate(chunks):
        (HERE / f"verdict_cases_{i:02d}.json").write_text(json.dumps(chunk, indent=0, allow_nan=True))
    tchunks = shard(sorted(STORAGES.items()), lambda kv: len(kv[1]) + 40)
    for i, chunk in enumerate(tchunks):
        (HERE / f"tensors_{i:02d}.json").write_text(json.dumps(dict(chunk), indent=0))

    # policy resolution for every operator config shipped with the reference
    ops_root = Path(reference_root) / "operators"
    policies = []
    for cfg_path in sorted(ops_root.glob("*/*/config.json")):
        category, op = cfg_path.parts[-3], cfg_path.parts[-2]
        config = json.loads(cfg_path.read_text())
        spec = {"category": category, "op_name": op, "config": config}
        policies.append({"category": category, "op_name": op, "config": config,
                         "resolved": cp.resolve_correctness_policy(spec),
                         "tolerance_policy": gcr._operator_tolerance_policy(spec)})
    extra_specs = [
        {"category": "reduction", "op_name": "argmax", "config": {}},
        {"category": "reduction", "op_name": "cumsum", "config": {}},
        {"category": "reduction", "op_name": "mean", "config": {}},
        {"category": "unknown_cat", "op_name": "x", "config": {}},
        {"category": "gemm", "op_name": "x", "config": {"policy": "cosine",
                                                       "thresholds": {"fp32": {"min_cosine": 0.5}, "int8": {"a": 1},
                                                                      "BF16": "skip"}}},
        {"category": "gemm", "op_name": "x", "config": {"policy": ""}},
        {"category": None, "op_name": None, "config": None},
    ]
    for spec in extra_specs:
        policies.append({"category": spec["category"], "op_name": spec["op_name"], "config": spec["config"],
                         "resolved": cp.resolve_correctness_policy(spec),
                         "tolerance_policy": gcr._operator_tolerance_policy(spec)})
    lookups = []
    for spec in extra_specs[:5] + [{"category": "gemm", "op_name": "x", "config": {}}]:
        pol = cp.resolve_correctness_policy(spec)
        for dt in ("FP32", "FP16", "BF16", "INT8", "fp32", "Float64", "FLOAT8_E4M3FN"):
            lookups.append({"policy": pol, "dtype": dt, "thresholds": cp.thresholds_for_dtype(pol, dt),
                            "is_metric": cp.is_metric_policy(pol), "name": cp.policy_name(pol)})
    criteria = []
    for spec in ({"category": "gemm", "op_name": "x", "config": {}},
                 {"category": "attention", "op_name": "x", "config": {}},
                 {"category": "activation", "op_name": "x", "config": {}}):
        pol = cp.resolve_correctness_policy(spec)
        for mode, shape_mode in (("correctness", "single"), ("performance", "random")):
            criteria.append({"policy": pol, "baseline_compute_mode": mode, "shape_mode": shape_mode,
                             "tolerance_policy": gcr.TOLERANCE_POLICY,
                             "random_correctness": {"max_failed_case_rate": 0.03},
                             "criteria": gcr._correctness_criteria(gcr.TOLERANCE_POLICY, pol, mode,
                                                                   {"max_failed_case_rate": 0.03}, shape_mode)})
    # intern the (large, highly repeated) resolved threshold tables and trim configs to the keys the verdict reads;
    # a table's key is its JSON text in the reference's own key order, so the order survives the round trip
    tables = {}

    def intern(pol):
        key = json.dumps(pol["thresholds"])
        tables.setdefault(key, len(tables))
        out = dict(pol)
        out["thresholds"] = {"__table__": tables[key]}
        return out

    for entry in policies:
        cfg = entry["config"]
        if isinstance(cfg, dict):
            # "tolerances" is what _operator_tolerance_policy returns, kept once under "tolerance_policy"
            entry["config"] = {k: v for k, v in cfg.items() if k in ("policy", "thresholds")}
            entry["has_tolerances"] = "tolerances" in cfg
        entry["resolved"] = intern(entry["resolved"])
    for entry in lookups:
        entry["policy"] = intern(entry["policy"])
    for entry in criteria:
        entry["policy"] = intern(entry["policy"])
        entry["criteria"]["metric_fallback"] = dict(entry["criteria"]["metric_fallback"])
        if "thresholds" in entry["criteria"]["metric_fallback"]:
            th = entry["criteria"]["metric_fallback"]["thresholds"]
            key = json.dumps(th)
            tables.setdefault(key, len(tables))
            entry["criteria"]["metric_fallback"]["thresholds"] = {"__table__": tables[key]}
    table_list = [json.loads(k) for k, _ in sorted(tables.items(), key=lambda kv: kv[1])]
    (HERE / "policy_resolution.json").write_text(json.dumps(
        {"tables": table_list, "policies": policies, "thresholds_for_dtype": lookups, "criteria": criteria},
        separators=(",", ":")))
    print(f"wrote {len(out_cases)} verdict cases in {len(chunks)} files, {len(policies)} policy resolutions")


# ------------------------------------------------------------- code around the verdict
def _outcome(fn, *args, **kwargs):
    """What a reference call returns, or the exception it raises."""
    try:
        return {"value": encode_value(fn(*args, **kwargs))}
    except Exception as exc:  # the reference raising is itself the expected result
        return {"raises": type(exc).__name__, "message": str(exc)}


def host_fixtures(reference_root: str) -> None:
    sys.dont_write_bytecode = True
    sys.path.insert(0, reference_root)
    import copy

    import runner.correctness_policy as cp  # noqa: E402
    import runner.generated_correctness_runner as gcr  # noqa: E402
    import utils.performance as perf  # noqa: E402

    sys.path.insert(0, str(HERE.parent))
    import trial_models  # noqa: E402

    # random-mode configuration and summary
    specs = [{"op_name": "a", "config": {}}, {"op_name": "b", "config": None}, {"config": {"random_correctness": {}}},
             {"op_name": "c", "config": {"random_correctness": {"max_failed_case_rate": 0.1}}},
             {"op_name": "d", "config": {"random_correctness": {"max_failed_case_rate": "0.25"}}},
             {"op_name": "e", "config": {"random_correctness": {"max_failed_case_rate": "x"}}},
             {"op_name": "f", "config": {"random_correctness": {"max_failed_case_rate": None}}},
             {"op_name": "g", "config": {"random_correctness": {"max_failed_case_rate": 1.5}}},
             {"op_name": "h", "config": {"random_correctness": {"max_failed_case_rate": -0.01}}},
             {"op_name": "i", "config": {"random_correctness": [0.1]}},
             {"op_name": "j", "config": {"random_correctness": {"max_failed_case_rate": 0}}},
             {"op_name": "k", "config": {"random_correctness": {"max_failed_case_rate": 1}}}]
    resolve = [{"spec": sp, "expected": _outcome(gcr._resolve_random_correctness_config, sp)} for sp in specs]
    summaries = []
    for mode in ("random", "single", "fixed"):
        for total, failed in ((0, 0), (1, 0), (1, 1), (3, 1), (33, 1), (100, 3), (100, 4), (7, 7), (10, 0)):
            for rate in (0.0, 0.03, 0.5, 1.0):
                kw = dict(shape_mode=mode, total_cases=total, failed_cases=failed,
                          random_correctness_config={"max_failed_case_rate": rate})
                summaries.append({"kwargs": kw, "expected": _outcome(gcr._random_case_summary, **kw)})

    def case(i, ok, details=None, **extra):
        c = {"case_index": i, "success": ok, "failed_trials": [{"case_index": i, "trial": 0, "details": d}
                                                               for d in (details or [])]}
        c.update(extra)
        return c

    results = [
        {"language": "cuda", "cases": [case(2, True), case(0, True), case(1, True)]},
        {"language": "cuda", "cases": [case(1, False, [["output mismatch"]]), case(0, True)]},
        {"language": "cuda", "cases": []},
        {"language": "hip", "cases": [case(i, i % 40 != 5, [["x"]] if i % 40 == 5 else None) for i in range(40)]},
        {"language": "biren", "cases": [case(0, False, error_type="CaseCompileFailed")]},
        {"language": "BIREN", "cases": [case(0, False, [["fatal error: main.cpp: No such file or directory"]])]},
        {"language": "biren", "cases": [case(0, False, [["fatal error: something else"]])]},
        {"language": "biren", "cases": [case(0, True, performance_error_message={"generated": "ninja: build stopped"})]},
        {"language": "biren", "cases": [case(0, True, performance_error_message="Error building extension 'x'")]},
        {"language": "cuda", "cases": [case(0, False, error_type="CaseCompileFailed")]},
        {"language": "cuda", "cases": [{"case_index": 0}, case(1, True)]},
    ]
    finals = []
    for res in results:
        for mode in ("random", "single"):
            for total in (None, len(res["cases"]), len(res["cases"]) + 1):
                r = copy.deepcopy(res)
                r["correctness"] = {"existing": 1}
                kw = dict(shape_mode=mode, random_correctness_config={"max_failed_case_rate": 0.03},
                          total_cases=total)
                finals.append({"result": copy.deepcopy(r), "kwargs": kw,
                               "expected": _outcome(gcr.finalize_generated_operator_result, result=r, **kw)})
    perf_results = [{"times": t, "expected": perf._build_cuda_perf_result(t)}
                    for t in ([], [1.0], [0.5, 0.25], [1.23456, 1.23449, 2.0004999, 0.0001], list(np.linspace(0.1, 3, 17)))]
    seeds = [{"op_name": n, "seed": perf.perf_seed_for_op(n)}
             for n in ("op_benchmark/gelu/case_0/operator_defined", "matmul", "", "ünïcode")]
    (HERE / "host_logic.json").write_text(json.dumps(
        {"resolve_random_correctness": resolve, "random_case_summary": summaries,
         "perf_result": perf_results, "perf_seed": seeds}, separators=(",", ":")))
    half = (len(finals) + 1) // 2
    for i, part in enumerate((finals[:half], finals[half:])):
        (HERE / f"finalize_cases_{i:02d}.json").write_text(json.dumps(part, separators=(",", ":")))

    # trials on the CPU: the reference's own driver, with host outputs
    trials = []
    for name, gen, ref, n, spec, tol in trial_models.TRIAL_CASES:
        pol = cp.resolve_correctness_policy({"category": spec.get("category"), "op_name": spec.get("op_name"),
                                             "config": spec.get("config") or {}}) if spec else None
        tol = tol if tol is not None else gcr.TOLERANCE_POLICY
        out = _outcome(gcr._run_correctness_trial_once, language="cuda", correctness_shape={"n": n},
                       generated_model_class=trial_models.MODELS[gen], reference_model_class=trial_models.MODELS[ref],
                       generate_inputs_fn=trial_models.generate_inputs, backend=None, device="cpu",
                       input_seed=trial_models.INPUT_SEED, param_seed=trial_models.PARAM_SEED,
                       tolerance_policy=tol, correctness_policy=pol)
        trials.append({"name": name, "generated": gen, "reference": ref, "n": n, "tolerance_policy": tol,
                       "correctness_policy": pol, "expected": out})
    (HERE / "trial_cases.json").write_text(json.dumps(trials, indent=0, allow_nan=True))
    print(f"wrote {len(resolve) + len(summaries) + len(finals) + len(perf_results) + len(seeds)} host-logic "
          f"fixtures, {len(trials)} trial fixtures")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--part")]
    part = next((a.split("=", 1)[1] for a in sys.argv[1:] if a.startswith("--part=")), "all")
    root = args[0] if args else "/root/reference"
    if part in ("all", "verdict"):
        main(root)
    if part in ("all", "host"):
        host_fixtures(root)
