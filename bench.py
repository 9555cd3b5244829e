#!/usr/bin/env python3
"""Verdict throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1]

A step is one complete verdict of one tensor pair that is already resident in
HBM: every kernel of libkvv's launch sequence plus the copy of the result
record to the host and the stream synchronisation.  ``value`` is algorithmic
input bytes (both tensors read once) per second of step time.

The ``roofline`` object covers the dominant kernel (the main pass): its
duration is measured live with HIP events recorded by the library around
that launch on the bench's stream (kvv_verdict_timed), averaged over the timed
steps.  ``cpu_baseline`` times the torch-CPU oracle (a restatement of the
reference's own torch-CPU verdict) on a bounded slice of the same workload.

Configurations (BASELINE.json ``configs``): c0 fp32 1 Mi, c1 bf16 256 Mi
(default, the headline), c2 fp16 4096x32768 strided, c3fp8 / c3int8 128 Mi.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "verdict throughput GB/s (both tensors read) and % HBM peak; µs/verdict"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_workload(name: str, dev):
    """(gen, ref, tolerance, description, dtype label) on the device."""
    from kernelverse_amd import synth
    if name == "c1":
        n = 268_435_456
        g, r = synth.code_flip_pair_device(n, seed=1, device=dev, dtype=torch.bfloat16, std=2.0, p1=0.05, p3=1e-4)
        return g, r, {"BF16": {"rtol": 1.6e-2, "atol": 1e-2}}, (
            "bf16 pair, 268,435,456 elements (1 GiB read); ref=bf16(N(0,2)); cand = ref with 1-ULP steps at 5% "
            "and 3-ULP steps at 0.01%; atol=1e-2 rtol=1.6e-2; full verdict + 16-bucket ULP histogram"), "bf16"
    if name == "c0":
        g, r = synth.fp32_noise_pair(1 << 20, seed=0)
        return g.to(dev), r.to(dev), {"FP32": {"rtol": 1e-5, "atol": 1e-5}}, (
            "fp32 pair, 1,048,576 elements, contiguous; C0 noise model; atol=rtol=1e-5"), "f32"
    if name == "c2":
        rows, cols, stride = 4096, 32768, 32896
        gen = torch.Generator(device=dev)
        gen.manual_seed(2)
        base_r = (torch.rand(rows, stride, generator=gen, device=dev) * 120000.0 - 60000.0).to(torch.float16)
        u = torch.rand(rows, stride, generator=gen, device=dev)
        base_r[u < 5e-4] = float("nan")
        base_r[(u >= 5e-4) & (u < 1e-3)] = float("inf")
        base_g = base_r.clone()
        flat = base_g.view(-1)
        pos = torch.randint(0, rows * cols, (17,), generator=gen, device=dev)
        flat[(pos // cols) * stride + pos % cols] = 1.0
        return base_g[:, :cols], base_r[:, :cols], {"FP16": {"rtol": 1e-3, "atol": 1e-3}}, (
            "fp16 pair, 4096x32768 row-major, row stride 32896; U(-60000,60000) with 0.05% NaN and 0.05% Inf; "
            "17 finite-pattern breaks; atol=rtol=1e-3"), "f16"
    if name == "c3fp8":
        g, r = synth.code_flip_pair_device(134_217_728, seed=3, device=dev, dtype=torch.float8_e4m3fn, std=4.0,
                                           p1=0.02, p3=0.0, clamp=448.0)
        return g, r, None, "fp8 e4m3fn pair, 134,217,728 elements; +-1 code at 2%; ULP histogram over codes", "fp8"
    if name == "c3int8":
        gen = torch.Generator(device=dev)
        gen.manual_seed(4)
        r = torch.randint(-128, 128, (134_217_728,), generator=gen, device=dev, dtype=torch.int8)
        g = r.clone()
        pos = torch.randint(0, r.numel(), (1000,), generator=gen, device=dev)
        g[pos] = (g[pos].to(torch.int16) + 77).to(torch.int8)
        return g, r, None, "int8 pair, 134,217,728 elements; 1000 changed positions; exact-equality count", "i8"
    raise SystemExit(f"unknown config {name}")


def cpu_baseline(g_dev, r_dev, tol, budget_s: float = 20.0):
    """Torch-CPU oracle verdict on a bounded leading slice of the workload."""
    from oracle import torch_verdict as tv
    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    n = g_dev.numel()
    sample = min(n, 1 << 24)
    g = g_dev.reshape(-1)[:sample].cpu() if g_dev.is_contiguous() else g_dev.flatten()[:sample].cpu()
    r = r_dev.reshape(-1)[:sample].cpu() if r_dev.is_contiguous() else r_dev.flatten()[:sample].cpu()
    tv.compare_tensors(g, r, "output", tol)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        tv.compare_tensors(g, r, "output", tol)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    t = statistics.median(times)
    bytes_read = 2 * sample * g.element_size()
    return {
        "value": round(bytes_read / t / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"torch-CPU oracle compare_tensors (restatement of GCR:672-786) on the first {sample:,} elements "
                   f"of the same pair, median of {len(times)} runs, {t * 1e3:.1f} ms each; D2H copy excluded"),
    }


def copy_calibration(steps: int):
    """A plain device copy of known size: 512 MiB read + 512 MiB written per launch."""
    dev = torch.device("cuda", 0)
    src = torch.empty(512 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"copy_bytes_read": src.numel(), "copy_bytes_written": dst.numel(),
                      "us_per_copy": round(dt * 1e6, 1), "GBps_read_plus_write": round(2 * src.numel() / dt / 1e9, 1)}),
          flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c1")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="time a plain 512 MiB device copy instead (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counts to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; the verdict path has no multi-GPU mode "
                                   "(see DESIGN.md for how it would shard)"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    if args.copy_calibration:
        copy_calibration(args.steps)
        return
    from kernelverse_amd import _lib, verdict

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"[bench] building workload {args.config}")
    g, r, tol, desc, dlabel = make_workload(args.config, dev)
    torch.cuda.synchronize()
    job = verdict._Job(g, r, "output", tol, None, verdict.MAX_SAMPLES, fp8_errors=False)
    gt, rt = verdict._kvv_tensor(g), verdict._kvv_tensor(r)
    size = ctypes.c_size_t()
    _lib.check(lib.kvv_workspace_size(gt, rt, job.kpolicy, ctypes.byref(size)), "kvv_workspace_size")
    ws = torch.empty(size.value, dtype=torch.uint8, device=dev)
    out = torch.empty(ctypes.sizeof(_lib.KvvResult), dtype=torch.uint8, device=dev)
    host = torch.empty_like(out, device="cpu").pin_memory()
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    n = g.numel()
    bytes_read = 2 * n * g.element_size()

    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev) if bytes_read < (512 << 20) else None

    def step(ev0=None, ev1=None):
        if ev0 is None:
            rc = lib.kvv_verdict(gt, rt, job.kpolicy, out.data_ptr(), ws.data_ptr(), size.value, sh)
        else:
            rc = lib.kvv_verdict_timed(gt, rt, job.kpolicy, out.data_ptr(), ws.data_ptr(), size.value, sh,
                                       ev0.cuda_event, ev1.cuda_event)
        if rc:
            _lib.check(rc, "kvv_verdict")
        host.copy_(out, non_blocking=True)
        stream.synchronize()

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    evs = []
    for _ in range(args.steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)  # materialise the events before handing their handles over
        e1.record(stream)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} steps")
    step_times = []
    for i in range(args.steps):
        if flush is not None:
            flush.fill_(i & 255)  # evict the 256 MB MALL so small inputs come from HBM
            stream.synchronize()
        t0 = time.perf_counter()
        step(*evs[i])
        step_times.append(time.perf_counter() - t0)
    torch.cuda.synchronize()
    ms_per_step = 1e3 * sum(step_times) / len(step_times)
    main_ms = [a.elapsed_time(b) for a, b in evs]
    main_avg = sum(main_ms) / len(main_ms)
    rec = _lib.KvvResult.from_buffer_copy(host.numpy().tobytes())
    value = bytes_read / (ms_per_step * 1e-3) / 1e9
    achieved = bytes_read / (main_avg * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "us_per_verdict": round(ms_per_step * 1e3, 1),
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dlabel,
        "data": "synthetic (seeded, generated on the device)",
        "config": {"workload": desc, "config_id": args.config, "numel": n, "bytes_read": bytes_read,
                   "tolerance": tol, "correctness_policy": "strict"},
        "roofline": {
            "bound": "hbm",
            "kernel": "kvv::scan_kernel (main pass)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel_avg_us": round(main_avg * 1e3, 2),
        },
        "verdict_check": {"mismatch_count": rec.mismatch_count, "ulp_hist_b0_b1_b2": list(rec.ulp_hist)[:3],
                          "finite_violations": rec.finite_violations, "p99_abs": rec.p99_abs},
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(g, r, tol)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
