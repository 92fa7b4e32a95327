#!/usr/bin/env python3
"""Benchmark of the MI355X-native Vedic GEMM hot path.

Default workload (the headline): FFN up-projection,
X[8192x1024] fp16 . W[1024x4096] fp16 + bias[4096], fused tanh-GELU epilogue,
fp32 accumulate and fp32 output, on one GPU.  One "step" is one launch of the
fused GEMM over the whole problem, inputs already resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints one JSON line (rank 0) with the metric named in BASELINE.json plus:
  roofline      the dominant kernel against MI355X's published dense fp16
                MFMA peak (2.5 PFLOP/s), its average launch duration taken
                with HIP events on the launch stream over the timed region;
  cpu_baseline  the reference CPU path (the reference's own vedic_gemm_bias +
                gelu built from its sources into oracle/_ref when that was
                built, else the bitwise restatement in oracle/) on a bounded
                row sample of the same workload, single-threaded as the
                reference is.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOP/s + % of MFMA peak, FFN-up 8192x1024x4096 fp16->fp32, 1 GPU"
PEAK_TFLOPS = {"fp16": 2500.0, "fp32": 157.3}  # MI355X dense MFMA, published

# name: (M, K, N, op, dtype, epilogue)
WORKLOADS = {
    "ffn_up_fp16_bias_gelu": (8192, 1024, 4096, "NN", "fp16", "bias_gelu"),
    "ffn_down_dx_nt_fp16": (8192, 1024, 4096, "NT", "fp16", "none"),
    "ffn_down_dw_tn_fp16": (4096, 8192, 1024, "TN", "fp16", "none"),
    "lm_head_fp16": (8192, 1024, 8192, "NN", "fp16", "none"),
    "lm_head_fp32": (8192, 1024, 8192, "NN", "fp32", "none"),
    "fp32_nn_512": (512, 1024, 1024, "NN", "fp32", "none"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="ffn_up_fp16_bias_gelu", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-rows", type=int, default=None,
                    help="rows of the workload timed on the CPU baseline (default: ~10-30 s of work)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    return ap.parse_args()


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by the rocprofv3 --pmc runs whose summary
    is committed under profiles/ (FETCH_SIZE + WRITE_SIZE, scaled by the copy
    kernel calibration); None if that summary is absent."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return int(json.load(f)["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def cpu_baseline(M, K, N, op, dtype, epi, rows):
    """Times the reference CPU path on `rows` rows of the workload (1 thread)."""
    from oracle import oracle as o

    rng = np.random.default_rng(7)
    kind = "reference" if o.ref_available() else "port"
    A = rng.standard_normal((rows, K), dtype=np.float32)
    B = (rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
    bias = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.01))
    if dtype == "fp16":
        A, B = o.f16_round(A), o.f16_round(B)
    if op == "NT":
        Bt = np.ascontiguousarray(B.T)
    t0 = time.perf_counter()
    if kind == "reference":
        if op == "NN":
            C = o.ref_vedic_gemm_bias(A, B, bias) if epi != "none" else o.ref_vedic_gemm(A, B)
        elif op == "NT":
            C = o.ref_gemm_nt(A, Bt)
        else:  # TN: output rows are columns of X[K x M]
            C = o.ref_gemm_tn(np.ascontiguousarray(A.T), B)
        if epi == "bias_gelu":
            C = o.ref_gelu(C)
    else:
        if op == "NN":
            C = o.vedic_gemm_bias(A, B, bias, nthreads=1) if epi != "none" else o.vedic_gemm(A, B, nthreads=1)
        elif op == "NT":
            C = o.gemm_nt(A, Bt, nthreads=1)
        else:
            C = o.gemm_tn(np.ascontiguousarray(A.T), B, nthreads=1)
        if epi == "bias_gelu":
            C = o.gelu(C)
    dt = time.perf_counter() - t0
    flops = 2.0 * rows * K * N
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{rows} of {M} rows ({rows * K * N * 2 / 1e9:.1f} GFLOP), {dt:.1f} s, "
                  f"single thread, reference flags -O3 -march=x86-64",
        "threads_available": os.cpu_count(),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    from logos_amd import _lib, vedic

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    M, K, N, op, dtype, epi = WORKLOADS[args.workload]
    lib = _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0x4C4F474F)
    op_code = {"NN": vedic.OP_NN, "NT": vedic.OP_NT, "TN": vedic.OP_TN}[op]
    a_shape = (K, M) if op == "TN" else (M, K)
    b_shape = (N, K) if op == "NT" else (K, N)
    A32 = torch.randn(a_shape, generator=g, device=dev)
    B32 = torch.randn(b_shape, generator=g, device=dev) * 0.02
    bias = torch.randn((N,), generator=g, device=dev) * 0.01
    if dtype == "fp16":
        A = vedic.cast_fp32_to_fp16(A32)
        B = vedic.cast_fp32_to_fp16(B32)
        del A32, B32
    else:
        A, B = A32, B32
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()
    desc = _lib.GemmDesc(
        op=op_code, in_dtype=_lib.DT_F16 if dtype == "fp16" else _lib.DT_F32, out_dtype=_lib.DT_F32,
        M=M, N=N, K=K, A=A.data_ptr(), lda=A.shape[1], B=B.data_ptr(), ldb=B.shape[1],
        C=C.data_ptr(), ldc=N, alpha=1.0, beta=0.0,
        bias=bias.data_ptr() if epi != "none" else None,
        epilogue=_lib.EPI_BIAS_GELU if epi == "bias_gelu" else _lib.EPI_NONE,
        preact=None, ld_preact=0, stream=stream.cuda_stream)
    pdesc = ctypes.byref(desc)
    gemm = lib.vedic_gemm

    def step():
        rc = gemm(pdesc)
        if rc:
            raise RuntimeError(f"vedic_gemm failed: {_lib.status_string(rc)}")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / args.steps
    flops = 2.0 * M * N * K
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_TFLOPS[dtype]

    cpu = None
    if not args.no_cpu:
        rows = args.cpu_rows
        if rows is None:
            # ~10-30 s of single-thread work at ~8-10 GFLOP/s
            rows = max(64, min(M, int(1.6e11 / (2.0 * K * N))))
            rows -= rows % 64
        cpu = cpu_baseline(M, K, N, op, dtype, epi, rows)

    out = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded torch.randn: X~N(0,1), W~N(0,0.02), bias~N(0,0.01); "
                "fp16 by the library's clamp+RNE cast)",
        "config": {"workload": args.workload, "M": M, "K": K, "N": N, "op": op,
                   "accumulate": "fp32", "output": "fp32", "epilogue": epi},
        "pct_of_peak": round(100.0 * tflops / peak, 2),
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(tflops / peak, 4),
            "traffic": traffic_from_profiles(args.workload),
            "kernel_avg_us": round(ms_per_step * 1e3, 3),
            "algorithmic_flops_per_launch": flops,
        },
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
