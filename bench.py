#!/usr/bin/env python3
"""Benchmark of the MI355X-native Vedic GEMM hot path.

Default workload (the headline): FFN up-projection,
X[8192x1024] fp16 . W[1024x4096] fp16 + bias[4096], fused tanh-GELU epilogue,
fp32 accumulate and fp32 output, on one GPU.  One "step" is one launch of the
fused GEMM over the whole problem, inputs already resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
    python bench.py --all            # every BASELINE configuration, one JSON line each
    python bench.py --summarize-traffic FETCH_DIR WRITE_DIR COPY_FETCH_DIR COPY_WRITE_DIR
                                     # rocprofv3 --pmc CSVs -> profiles/traffic_<workload>.txt

The default run prints one JSON line with the metric named in BASELINE.json plus:
  roofline      the GEMM kernel against MI355X's published dense MFMA peak
                (fp16 2.5 PFLOP/s, fp32 157.3 TFLOP/s) or, for the skinny
                decode shapes, against 8 TB/s of HBM; its average launch time is
                taken with HIP events on the launch stream over the timed region.
                `traffic` is the HBM bytes per launch from the committed
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary, scaled by a copy
                kernel of known size (None when no summary is committed);
  cpu_baseline  the reference CPU path on a bounded sample of the same workload:
                all host cores (at most 16) as `value` and one thread beside it
                in `single_thread`, with the CPU model.  Both run the
                reference's own vedic_gemm built from its sources into
                oracle/_ref where that exists (kind "reference"; the threads
                take blocks of output rows), else the bitwise restatement in
                oracle/ (kind "port", 64-row blocks).
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOP/s + % of MFMA peak, FFN-up 8192x1024x4096 fp16->fp32, 1 GPU"
PEAK = {"fp16": 2500.0, "fp32": 157.3}  # MI355X dense MFMA, TFLOP/s (published)
HBM_PEAK_GBS = 8000.0                   # MI355X HBM3E, GB/s (published)

# One GEMM: (M, K, N, op, dtype, epilogue, beta).  op as stored:
#   NN A[MxK] B[KxN]; NT A[MxK] B[NxK]; TN A[KxM] B[KxN].
#   dtype "amp": A fp32, converted to binary16 inside the GEMM (the AMP path from
#   an fp32 activation); cast_a: an fp32 A cast into a binary16 buffer by a
#   separate launch before the fp16 GEMM, every step (the reference's amp_gemm).
#   gather: A read from that many [M x K / gather] head matrices, accumulated
#   head by head (vedic_gemm_gather).
def _g(M, K, N, op="NN", dtype="fp16", epi="none", beta=0.0, checked=False, heads=0, alpha=1.0, cast_a=False,
       gather=0):
    return dict(M=M, K=K, N=N, op=op, dtype=dtype, epi=epi, beta=beta, checked=checked, heads=heads, alpha=alpha,
                cast_a=cast_a, gather=gather)


# BASELINE.json configs; each workload is a list of GEMMs run back to back per step.
WORKLOADS = {
    "fp32_nn_512x1024x1024": dict(cfg=1, gemms=[_g(512, 1024, 1024, dtype="fp32")]),
    "ffn_up_fp16_bias_gelu": dict(cfg=2, gemms=[_g(8192, 1024, 4096, epi="bias_gelu")]),
    # the FFN-up from the fp32 activation: converted inside the GEMM, against the
    # reference's per-call cast into a binary16 buffer followed by the fp16 GEMM
    # (cuda/ModelGPU.cu:840-856)
    "ffn_up_amp_fp32_act": dict(cfg=2, gemms=[_g(8192, 1024, 4096, dtype="amp", epi="bias_gelu")]),
    "ffn_up_cast_then_fp16": dict(cfg=2, gemms=[_g(8192, 1024, 4096, epi="bias_gelu", cast_a=True)]),
    "ffn_down_dx_nt_fp16": dict(cfg=3, gemms=[_g(8192, 1024, 4096, op="NT")]),
    "ffn_down_dw_tn_fp16": dict(cfg=3, gemms=[_g(4096, 8192, 1024, op="TN", beta=1.0)]),
    # FFN backward through the activation, fused: dH = (dY . W2^T) * gelu'(H)
    # with db1 += colsum(dH), at config 3's NT shape and config 2's activation
    "ffn_bwd_dh_gelu_nt_fp16": dict(cfg=3, gemms=[_g(8192, 1024, 4096, op="NT", epi="gelu_bwd")]),
    # the Q/K/V projection of one layer: the reference's 48 per-head GEMMs
    # (cuda/ModelGPU.cu:894-906) against one packed GEMM scattered into the same 48 head buffers
    # the reference's per-head projections (cuda/ModelGPU.cu:900-906): 48 calls on
    # the same activation X with each head's own [1024 x 64] weight
    "qkv_per_head_fp16": dict(cfg=5, share_a=True, gemms=[_g(8192, 1024, 64) for _ in range(48)]),
    "qkv_packed_scatter_fp16": dict(cfg=5, gemms=[_g(8192, 1024, 3072, heads=48)]),
    # the attention-output projection of one layer: the reference's 16 per-head
    # amp_gemm(hc.head_out, W_O[h]) calls, each added into the zeroed concat by
    # residual_add_kernel (cuda/ModelGPU.cu:976-986; here beta = 1 into the one
    # shared concat, no temporary), against one launch that gathers the 16 fp32
    # head outputs and multiplies the row-stacked W_O, added head by head (the
    # same bits)
    "attn_out_per_head_amp": dict(cfg=5, share_c=True,
                                  gemms=[_g(8192, 64, 1024, dtype="amp", beta=1.0) for _ in range(16)]),
    "attn_out_stacked_amp": dict(cfg=5, gemms=[_g(8192, 1024, 1024, dtype="amp", gather=16)]),
    # the FFN-down with its bias and the residual add in the epilogue: the
    # reference's amp_gemm_bias into a temporary, then residual_add_kernel
    # (cuda/ModelGPU.cu:1044-1048); C holds the residual stream X
    "ffn_down_bias_residual_fp16": dict(cfg=5, gemms=[_g(8192, 4096, 1024, epi="bias_residual")]),
    # one attention head's GEMMs at seq = 8192, DH = 64, strict fp32 as in the reference
    # (cuda/train_gpu.cu:422-479, 672-692): scores = Q K^T / sqrt(DH) (NT, alpha),
    # out = P V (NN), dP = dO V^T (NT), dV += P^T dO (TN, beta = 1), dQ = dS K (NN), dK = dS^T Q (TN);
    # the softmax and its backward stay with the caller
    "attn_head_fwd_bwd_fp32": dict(cfg=5, gemms=[
        _g(8192, 64, 8192, op="NT", dtype="fp32", alpha=0.125), _g(8192, 8192, 64, dtype="fp32"),
        _g(8192, 64, 8192, op="NT", dtype="fp32"), _g(8192, 8192, 64, op="TN", dtype="fp32", beta=1.0),
        _g(8192, 8192, 64, dtype="fp32"), _g(8192, 8192, 64, op="TN", dtype="fp32"),
    ]),
    "lm_head_fp16": dict(cfg=4, gemms=[_g(8192, 1024, 8192)]),
    "lm_head_fp32": dict(cfg=4, gemms=[_g(8192, 1024, 8192, dtype="fp32")]),
    # the LM-head GEMM with its Gunitasamuchayah check computed on the way;
    # synchronous per step, like the reference's verify
    "lm_head_fp16_checked": dict(cfg=4, gemms=[_g(8192, 1024, 8192, checked=True)]),
    **{f"decode_fp16_m{m}": dict(cfg=4, hbm=True, gemms=[_g(m, 1024, 8192)]) for m in (1, 2, 4, 8, 16, 32)},
    **{f"decode_fp32_m{m}": dict(cfg=4, hbm=True, gemms=[_g(m, 1024, 8192, dtype="fp32")]) for m in (1, 32)},
    # one 219M-model block at d=1024, seq=8192: 4 forward GEMMs + their dX (NT) and dW (TN, beta=1)
    "block_fwd_bwd_fp16": dict(cfg=5, gemms=[
        _g(8192, 1024, 3072), _g(8192, 1024, 1024), _g(8192, 1024, 4096, epi="bias_gelu"),
        _g(8192, 4096, 1024, epi="bias"),
        _g(8192, 3072, 1024, op="NT"), _g(8192, 1024, 1024, op="NT"), _g(8192, 4096, 1024, op="NT"),
        _g(8192, 1024, 4096, op="NT"),
        _g(1024, 8192, 3072, op="TN", beta=1.0), _g(1024, 8192, 1024, op="TN", beta=1.0),
        _g(1024, 8192, 4096, op="TN", beta=1.0), _g(4096, 8192, 1024, op="TN", beta=1.0),
    ]),
}
# Fused attention forward (cuda_flash_attention_fwd, cuda/VedicGEMM.cu:1065-1104) at the
# reference's call: seq 8192, DH 64, 16 heads, causal, scale 1/sqrt(DH), fp32.  "per_head"
# makes the reference's 16 one-head calls (cuda/ModelGPU.cu:959); "16heads" one launch.
# The backward workloads time the fused backward (dQ, dK, dV from Q, K, V, O, dO and
# the forward's lse; the reference's cuda/train_gpu.cu:672-740) with the forward done once
# outside the timed region.
def _fa(seq=8192, dh=64, heads=16, batched=True, causal=1, shunyam=0, window=0, stride=1, bwd=False):
    return dict(seq=seq, dh=dh, heads=heads, batched=batched, causal=causal, shunyam=shunyam, window=window,
                stride=stride, dtype="fp32", bwd=bwd)


WORKLOADS.update({
    "flash_attn_fwd_fp32_16heads": dict(cfg=5, attn=_fa()),
    "flash_attn_fwd_fp32_per_head": dict(cfg=5, attn=_fa(batched=False)),
    "flash_attn_bwd_fp32_16heads": dict(cfg=5, attn=_fa(bwd=True)),
    # the same layer width split into 8 heads of DH 128 (the kernels' other width)
    "flash_attn_fwd_fp32_8heads_dh128": dict(cfg=5, attn=_fa(dh=128, heads=8)),
    "flash_attn_bwd_fp32_8heads_dh128": dict(cfg=5, attn=_fa(dh=128, heads=8, bwd=True)),
})
COPY_WORKLOAD = "copy_256mib"  # calibration for the FETCH_SIZE / WRITE_SIZE counters
# The library's own widening copy (vedic_cast_f16_to_f32 of 64 Mi values: 128 MiB
# read, 256 MiB written) as a second calibration: its loads take the same path
# as the GEMM kernels' operand loads.
CAST_WORKLOAD = "cast_f16_f32_64mi"
# The activation producer: layer normalisation of the 8192 x 1024 residual
# stream (cuda_layernorm, cuda/ModelGPU.cu:772) writing the fp32 rows and their
# binary16 copy in one pass, timed beside the two passes it replaces (the fp32
# normalisation, then the cast the reference's amp_gemm runs per call,
# cuda/ModelGPU.cu:825-827).  HBM-bound: 4 + 4 + 2 bytes per element.
LN_WORKLOAD = "layernorm_fp16_copy_8192x1024"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The GPU's shader clock ramps over the first ~10 ms of sustained work
    # (a 20-step warmup of the headline measured 86 us per step, 200 or more
    # 75-77 us): the default warmup runs the kernel for ~40 ms first.
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--workload", default="ffn_up_fp16_bias_gelu", choices=sorted(WORKLOADS) + [COPY_WORKLOAD, CAST_WORKLOAD, LN_WORKLOAD])
    ap.add_argument("--all", action="store_true", help="every workload, one JSON line each")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target CPU time of the cpu_baseline sample (default run)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--profiled-steps", type=int, default=25,
                    help="steps (--steps + --warmup) of the counter runs --summarize-traffic reads")
    ap.add_argument("--summarize-traffic", nargs=4, metavar="DIR",
                    help="FETCH, WRITE, copy FETCH, copy WRITE rocprofv3 output directories")
    return ap.parse_args()


# ------------------------------------------------------------- traffic summary

def _pmc_kib(dirpath: str, counter: str, kernel_substr: str):
    """Mean per-dispatch value of `counter` (KiB) over dispatches of kernels
    whose name contains kernel_substr, from a rocprofv3 --pmc -f csv run."""
    vals = []
    for root, _, files in os.walk(dirpath):
        for fn in files:
            if not fn.endswith("counter_collection.csv"):
                continue
            with open(os.path.join(root, fn)) as f:
                for r in csv.DictReader(f):
                    if r["Counter_Name"] == counter and kernel_substr in r["Kernel_Name"]:
                        vals.append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit(f"no {counter} rows for '{kernel_substr}' under {dirpath}")
    return sum(vals) / len(vals), len(vals)


# Kernels of the profiled process that are not the library's: torch's own
# (input set-up) and the runtime's blits.
_NOT_LIBRARY = ("at::native", "copyBuffer", "fillBuffer", "elementwise_kernel")
# Kernels whose global reads are 64-byte requests (FETCH_SIZE counts them at
# their size); every other kernel's reads are 128-byte requests, which
# FETCH_SIZE counts as 64 bytes on gfx950 (hence the copy calibration).
_FETCH_64B = ("gemm_skinny_kernel<vedic::SkinnyF16",)


def _pmc_library_total(dirpath: str, counter: str, only_64b=None):
    """Sum of `counter` over every dispatch of this library's kernels (only_64b:
    True for the 64-byte-request kernels only, False for the others)."""
    total, n = 0.0, 0
    for root, _, files in os.walk(dirpath):
        for fn in files:
            if fn.endswith("counter_collection.csv"):
                with open(os.path.join(root, fn)) as f:
                    for r in csv.DictReader(f):
                        name = r["Kernel_Name"]
                        if r["Counter_Name"] != counter or any(x in name for x in _NOT_LIBRARY):
                            continue
                        if only_64b is not None and any(x in name for x in _FETCH_64B) != only_64b:
                            continue
                        total += float(r["Counter_Value"])
                        n += 1
    if not n and only_64b is None:
        raise SystemExit(f"no {counter} rows of the library's kernels under {dirpath}")
    return total, n


def summarize_traffic(args):
    """HBM bytes per step of a workload: FETCH_SIZE and WRITE_SIZE summed over
    the library's dispatches of the profiled run, divided by its steps
    (--steps + --warmup of that run), each scaled by what the same counter
    reads for torch's copy of 256 MiB (bench.py --workload copy_256mib)."""
    fetch_dir, write_dir, cfetch_dir, cwrite_dir = args.summarize_traffic
    steps = args.profiled_steps
    fetch, _ = _pmc_library_total(fetch_dir, "FETCH_SIZE", only_64b=False)
    fetch64, _ = _pmc_library_total(fetch_dir, "FETCH_SIZE", only_64b=True)
    write, _ = _pmc_library_total(write_dir, "WRITE_SIZE")
    fetch, fetch64, write = fetch / steps, fetch64 / steps, write / steps
    cfetch, _ = _pmc_kib(cfetch_dir, "FETCH_SIZE", "copyBuffer")
    cwrite, _ = _pmc_kib(cwrite_dir, "WRITE_SIZE", "copyBuffer")
    ref_kib = 256.0 * 1024
    f_fetch, f_write = ref_kib / cfetch, ref_kib / cwrite
    hbm = (fetch * f_fetch + fetch64 + write * f_write) * 1024.0
    out = os.path.join(ROOT, "profiles", f"traffic_{args.workload}.txt")
    with open(out, "w") as f:
        f.write(f"# HBM traffic per step of bench.py --workload {args.workload} (the library's dispatches)\n")
        f.write(f"# python3 bench.py --workload {args.workload} --profiled-steps {steps} --summarize-traffic "
                f"{fetch_dir} {write_dir} {cfetch_dir} {cwrite_dir}\n")
        f.write("# over rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE runs of bench.py --workload "
                f"{args.workload} (KiB per dispatch),\n")
        f.write("# each scaled by the same counter on torch's copy of 256 MiB (bench.py --workload copy_256mib).\n")
        f.write("# FETCH_SIZE counts L2-to-fabric reads: repeated fetches by different XCDs' L2s\n")
        f.write("# are all counted, whether the Infinity Cache or HBM serves them.  The decode\n")
        f.write("# kernel's fp16 reads are 64-byte requests, counted at their size: their FETCH is not scaled.\n")
        f.write(f"fetch_kib_per_step: {fetch:.1f}\nfetch_64b_kib_per_step: {fetch64:.1f}\n"
                f"write_kib_per_step: {write:.1f}\n")
        f.write(f"copy_fetch_kib: {cfetch:.1f}\ncopy_write_kib: {cwrite:.1f}\n")
        f.write(f"fetch_scale: {f_fetch:.4f}\nwrite_scale: {f_write:.4f}\n")
        f.write(f"hbm_bytes_per_launch: {int(hbm)}\n")
    print(open(out).read())


def traffic_from_profiles(workload: str):
    """HBM bytes per launch from the committed summary, or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(line.split(":")[1].split()[0])
    return None


# ------------------------------------------------------------------ CPU leg

def attn_pairs(a: dict, q_begin: int = 0, q_end: int | None = None) -> int:
    """(query, key) pairs the mask allows, summed over query rows [q_begin, q_end)."""
    from oracle import oracle as o

    seq = a["seq"]
    q_end = seq if q_end is None else q_end
    if not a["shunyam"] or seq <= a["window"]:
        if a["causal"]:
            return sum(q + 1 for q in range(q_begin, q_end))
        return (q_end - q_begin) * seq
    return int(o.attention_mask(seq, a["causal"], a["shunyam"], a["window"], a["stride"])[q_begin:q_end].sum())


def cpu_baseline_attn(w: dict, seconds: float, seed: int = 7):
    """The reference's flash_attention_kernel restated on the CPU (oracle/, one
    thread, as one CUDA thread computes one query row there), on the last
    query rows of one head: the rows with the most keys; flops are counted over
    the allowed (query, key) pairs, 4 DH per pair, as on the GPU."""
    from oracle import oracle as o

    a = w["attn"]
    seq, dh = a["seq"], a["dh"]
    rng = np.random.default_rng(seed)
    if a["bwd"]:
        # the reference's backward keeps two seq x seq matrices: time it on one head at seq 2048
        s2 = 2048
        Q, K, V, dO = (rng.standard_normal((s2, dh), dtype=np.float32) for _ in range(4))
        t0 = time.perf_counter()
        reps = 0
        while True:
            o.attention_backward_reference(Q, K, V, dO, 1.0 / np.sqrt(dh))
            reps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        dt = time.perf_counter() - t0
        flops = reps * 10.0 * dh * s2 * (s2 + 1) / 2
        return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
                "sample": f"one head at seq {s2} x{reps} ({flops / 1e9:.1f} GFLOP counted as 10 DH per causal "
                          f"pair in {dt:.1f} s), single thread, -O3 -march=x86-64",
                "threads_available": os.cpu_count()}
    Q, K, V = (rng.standard_normal((seq, dh), dtype=np.float32) for _ in range(3))
    rows = max(1, min(seq, int(2.0e9 * seconds / (4.0 * dh * seq))))  # ~2 GFLOP/s single thread
    q0 = seq - rows
    t0 = time.perf_counter()
    reps = 0
    while True:
        o.flash_attention_rows(Q, K, V, 1.0 / np.sqrt(dh), q0, seq, a["causal"], a["shunyam"], a["window"],
                               a["stride"])
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    flops = reps * 4.0 * dh * attn_pairs(a, q0, seq)
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": f"query rows {q0}..{seq - 1} of one head x{reps} ({flops / 1e9:.1f} GFLOP in {dt:.1f} s), "
                  f"single thread, -O3 -march=x86-64",
        "threads_available": os.cpu_count(),
    }


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def baseline_threads() -> int:
    """Host threads for the all-cores CPU baseline: the cores this process may
    use, at most 16 (the host share of one GPU on the GPU boxes)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _ref_rows(o, g, B, bias):
    """The reference's own path for one GEMM of the workload on a block of
    output rows: its GEMM (vedic_gemm / vedic_gemm_bias, or the transpose +
    vedic_gemm of gemm_backward) and the element-wise work that follows it
    in the reference (gelu; gelu_backward + bias_backward; the residual add)."""
    op, epi = g["op"], g["epi"]

    def run(a, h=None, x=None):
        if op == "NN":
            C = o.ref_vedic_gemm_bias(a, B, bias) if epi in ("bias", "bias_gelu", "bias_residual") else o.ref_vedic_gemm(a, B)
        elif op == "NT":
            C = o.ref_gemm_nt(a, B)
        else:
            C = o.ref_gemm_tn(a, B)
        if epi == "bias_gelu":
            C = o.ref_gelu(C)
        if epi == "gelu_bwd":  # ffn_backward's gelu_backward + bias_backward
            C = o.ref_gelu_backward(h, C)
            o.ref_bias_backward(C)
        if epi == "bias_residual":  # the residual add after the FFN-down
            C = x + C
        return C

    return run


def _cpu_gemm_sample(w: dict, seconds: float, nthreads: int, seed: int):
    """(flops, seconds, kind, parts): the reference CPU path on row samples of
    the workload's GEMMs, repeated until about `seconds`.  Where the
    reference's own CPU GEMM is built in place (oracle/_ref, kind
    "reference") it runs on `nthreads` host threads, each taking one block of
    output rows (the reference functions are called through ctypes, which
    releases the interpreter lock; rows of a product are independent and each
    element is summed in the same order whichever rows share a call, so the
    GEMM's bits are the one-call result); else the bitwise restatement runs
    (kind "port"), sharded by 64-row blocks on `nthreads` threads."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import oracle as o

    kind = "reference" if o.ref_available() else "port"
    pool = ThreadPoolExecutor(nthreads) if kind == "reference" and nthreads > 1 else None
    rng = np.random.default_rng(seed)
    per_gemm = max(seconds / len(w["gemms"]), 0.5)
    total_flops = 0.0
    total_t = 0.0
    parts = []
    for g in w["gemms"]:
        M, K, N, op = g["M"], g["K"], g["N"], g["op"]
        # ~20 GFLOP/s per thread: rows for about per_gemm seconds, 1..M
        rows = int(max(1, min(M, 2.0e10 * nthreads * per_gemm / (2.0 * K * N))))
        if nthreads > 1:
            rows = max(64, rows // 64 * 64) if M >= 64 else rows
            rows = min(rows, M)
        A = rng.standard_normal((rows, K), dtype=np.float32)
        B = (rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
        bias = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.01))
        if g["dtype"] in ("fp16", "amp"):
            A, B = o.f16_round(A), o.f16_round(B)
        Hs = (rng.standard_normal((rows, N), dtype=np.float32) * np.float32(2.0)) if g["epi"] == "gelu_bwd" else None
        Xs = rng.standard_normal((rows, N), dtype=np.float32) if g["epi"] == "bias_residual" else None
        if op == "NT":
            B = np.ascontiguousarray(B.T)
        if op == "TN":
            A = np.ascontiguousarray(A.T)
        t0 = time.perf_counter()
        reps = 0
        while True:
            if kind == "reference":
                run = _ref_rows(o, g, B, bias)
                if pool is None:
                    C = run(A, Hs, Xs)
                else:
                    # output rows are A's rows (NN, NT) or A's columns (TN: A is K x rows)
                    cuts = np.linspace(0, rows, nthreads + 1).astype(int)
                    jobs = []
                    for r0, r1 in zip(cuts[:-1], cuts[1:]):
                        if r1 > r0:
                            a = A[:, r0:r1] if op == "TN" else A[r0:r1]
                            jobs.append(pool.submit(run, np.ascontiguousarray(a),
                                                    None if Hs is None else Hs[r0:r1],
                                                    None if Xs is None else Xs[r0:r1]))
                    C = [j.result() for j in jobs]
            else:
                if op == "NN":
                    C = (o.vedic_gemm_bias(A, B, bias, nthreads=nthreads)
                         if g["epi"] in ("bias", "bias_gelu", "bias_residual")
                         else o.vedic_gemm(A, B, nthreads=nthreads))
                elif op == "NT":
                    C = o.gemm_nt(A, B, nthreads=nthreads)
                else:
                    C = o.gemm_tn(A, B, nthreads=nthreads)
                if g["epi"] == "bias_gelu":
                    C = o.gelu(C)
                if g["epi"] == "gelu_bwd":
                    C = o.gelu_bwd_reference_f32(C, Hs)
                    C.sum(axis=0)
                if g["epi"] == "bias_residual":
                    C = Xs + C
            reps += 1
            if time.perf_counter() - t0 >= per_gemm:
                break
        dt = time.perf_counter() - t0
        total_flops += reps * 2.0 * rows * K * N
        total_t += dt
        parts.append(f"{op} {rows}/{M} rows x{reps}")
    if pool is not None:
        pool.shutdown()
    return total_flops, total_t, kind, parts


def cpu_baseline(w: dict, seconds: float, seed: int = 7):
    """The reference CPU path on row samples of the workload's GEMMs: all host
    cores (the reference build on blocks of rows where it is built, else the
    restatement sharded by 64-row blocks) as `value`, and one thread beside
    it, each for about half of `seconds`.  Rows of every GEMM are independent and cost the same,
    so TFLOP/s over a row sample is the rate of the whole GEMM."""
    n = baseline_threads()
    f1, t1, k1, p1 = _cpu_gemm_sample(w, seconds / 2, 1, seed)
    fn, tn, kn, pn = _cpu_gemm_sample(w, seconds / 2, n, seed)
    flags = "-O3 -march=x86-64 -ffp-contract=off"
    return {
        "value": fn / tn / 1e12,
        "unit": "TFLOP/s",
        "cores": n,
        "kind": kn,
        "sample": (f"{'; '.join(pn)} ({fn / 1e9:.1f} GFLOP in {tn:.1f} s), {n} threads"
                   f"{' by row blocks of the reference build' if kn == 'reference' else ' by 64-row blocks'}, {flags}"),
        "single_thread": {"value": f1 / t1 / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": k1,
                          "sample": f"{'; '.join(p1)} ({f1 / 1e9:.1f} GFLOP in {t1:.1f} s), {flags}"},
        "cpu_model": cpu_model(),
        "threads_available": os.cpu_count(),
    }


# ------------------------------------------------------------------ GPU leg

def make_step(w: dict, dev, torch):
    """Allocates seeded inputs for every GEMM of the workload and returns
    (step function, list of (desc, flops, algorithmic HBM bytes))."""
    from logos_amd import _lib

    lib = _lib.load()
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x4C4F474F ^ (w["cfg"] << 8))
    stream = torch.cuda.current_stream()
    keep = []
    items = []
    shared_a = None  # share_a: every GEMM reads the first one's A (one activation, several weights)
    shared_c = None  # share_c: every GEMM accumulates into the first one's C
    for g in w["gemms"]:
        M, K, N, op = g["M"], g["K"], g["N"], g["op"]
        a_shape = (K, M) if op == "TN" else (M, K)
        b_shape = (N, K) if op == "NT" else (K, N)
        A = torch.randn(a_shape, generator=gen, device=dev)
        B = torch.randn(b_shape, generator=gen, device=dev) * 0.02
        bias = torch.randn((N,), generator=gen, device=dev) * 0.01
        A32 = None
        if g["dtype"] == "fp16":
            if g["cast_a"]:
                A32 = A
            A, B = A.half(), B.half()
        elif g["dtype"] == "amp":
            B = B.half()
        a_again = False
        if w.get("share_a"):
            if shared_a is None:
                shared_a = A
            else:
                A, a_again = shared_a, True
        g["_cast"] = (A32, A) if A32 is not None else None
        keep.append(A32)
        resid = g["epi"] == "bias_residual"
        C = (torch.randn((M, N), generator=gen, device=dev) * (1.0 if resid else 1e-3) if g["beta"] or resid
             else torch.empty((M, N), device=dev))
        if w.get("share_c"):
            if shared_c is None:
                shared_c = C
            else:
                C = shared_c
        aheads = None
        if g["gather"]:
            hc = K // g["gather"]
            hts = [torch.randn((M, hc), generator=gen, device=dev) for _ in range(g["gather"])]
            if g["dtype"] == "fp16":
                hts = [t.half() for t in hts]
            keep += hts
            A = hts[0]
            aheads = (ctypes.c_void_p * g["gather"])(*[t.data_ptr() for t in hts])
            keep.append(aheads)
        g["_aheads"] = aheads
        keep += [A, B, bias, C]
        epi = {"none": _lib.EPI_NONE, "bias": _lib.EPI_BIAS, "bias_gelu": _lib.EPI_BIAS_GELU,
               "gelu_bwd": _lib.EPI_GELU_BWD, "bias_residual": _lib.EPI_BIAS_RESIDUAL}[g["epi"]]
        gbwd = g["epi"] == "gelu_bwd"
        H = torch.randn((M, N), generator=gen, device=dev) * 2.0 if gbwd else None
        db = torch.zeros((N,), device=dev) if gbwd else None
        keep += [H, db]
        d = _lib.GemmDesc(
            op={"NN": _lib.OP_NN, "NT": _lib.OP_NT, "TN": _lib.OP_TN}[op],
            in_dtype={"fp16": _lib.DT_F16, "fp32": _lib.DT_F32, "amp": _lib.DT_F32_F16}[g["dtype"]],
            out_dtype=_lib.DT_F32,
            M=M, N=N, K=K, A=A.data_ptr(), lda=A.shape[1], B=B.data_ptr(), ldb=B.shape[1],
            C=C.data_ptr(), ldc=N, alpha=g["alpha"], beta=g["beta"],
            bias=bias.data_ptr() if g["epi"] in ("bias", "bias_gelu", "bias_residual") else None, epilogue=epi,
            preact=H.data_ptr() if gbwd else None, ld_preact=N if gbwd else 0, stream=stream.cuda_stream,
            colsum=db.data_ptr() if gbwd else None, colsum_beta=1.0)
        es = 2 if g["dtype"] == "fp16" else 4
        es_b = 4 if g["dtype"] == "fp32" else 2
        # algorithmic HBM bytes of this launch: its operands once, C (read
        # too when accumulated), bias, pre-activation, cast and check passes
        hbm_launch = M * K * es + K * N * es_b + M * N * 4 * (2 if g["beta"] or resid else 1) + \
            (N * 4 if g["epi"] != "none" else 0)
        if g["cast_a"]:
            hbm_launch += M * K * 6  # the cast pass: fp32 read, binary16 written
        if gbwd:
            hbm_launch += M * N * 4 + N * 4  # H read, db read and written
        if g["checked"]:
            hbm_launch += (M * K + K * N) * es  # one more pass over A and B for the prediction
        # the step's bytes count an activation that several launches share once
        hbm = hbm_launch - (M * K * es if a_again else 0)
        heads = None
        if g["heads"]:
            hc = N // g["heads"]
            hts = [torch.empty((M, hc), device=dev) for _ in range(g["heads"])]
            keep += hts
            heads = (ctypes.c_void_p * g["heads"])(*[t.data_ptr() for t in hts])
            keep.append(heads)
        items.append((d, 2.0 * M * N * K, hbm, hbm_launch))
        g["_heads"] = heads
    ptrs = [(ctypes.byref(d), g) for (d, _, _, _), g in zip(items, w["gemms"])]
    gemm = lib.vedic_gemm
    vres = _lib.VerifyResult()

    cast = lib.vedic_cast_f32_to_f16
    sp = stream.cuda_stream

    def step():
        for p, g in ptrs:
            checked = g["checked"]
            if g["_cast"] is not None:
                src, dst = g["_cast"]
                rc = cast(src.data_ptr(), dst.data_ptr(), src.numel(), sp)
                if rc:
                    raise RuntimeError(f"vedic_cast_f32_to_f16 failed: {_lib.status_string(rc)}")
            if g["heads"]:
                rc = lib.vedic_gemm_scatter(p, g["_heads"], g["heads"], g["N"] // g["heads"])
            elif g["gather"]:
                rc = lib.vedic_gemm_gather(p, g["_aheads"], g["gather"], g["K"] // g["gather"])
            else:
                rc = lib.vedic_gemm_checked(p, 0.05, ctypes.byref(vres)) if checked else gemm(p)
            if rc:
                raise RuntimeError(f"vedic_gemm failed: {_lib.status_string(rc)}")
            if checked and not vres.pass_:
                raise RuntimeError(f"checksum failed: rel err {vres.relative_error}")

    step.keep = keep  # inputs stay alive with the closure
    return step, items


def time_steps(step, steps, warmup, torch):
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / steps, wall


def make_attn_step(w: dict, dev, torch):
    """Seeded Q/K/V for every head and the step: one multi-head launch, or one
    launch per head as the reference calls it."""
    from logos_amd import _lib

    lib = _lib.load()
    a = w["attn"]
    seq, dh, H = a["seq"], a["dh"], a["heads"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x4C4F474F ^ (w["cfg"] << 8))
    stream = torch.cuda.current_stream().cuda_stream
    qs, ks, vs, outs = [], [], [], []
    for _ in range(H):
        qs.append(torch.randn((seq, dh), generator=gen, device=dev))
        ks.append(torch.randn((seq, dh), generator=gen, device=dev))
        vs.append(torch.randn((seq, dh), generator=gen, device=dev))
        outs.append(torch.empty((seq, dh), device=dev))
    arr = lambda ts: (ctypes.c_void_p * H)(*[t.data_ptr() for t in ts])
    pq, pk, pv, po = arr(qs), arr(ks), arr(vs), arr(outs)
    scale = 1.0 / float(dh) ** 0.5
    flags = (a["causal"], a["shunyam"], a["window"], a["stride"])
    if a["bwd"]:
        lses = [torch.empty((seq,), device=dev) for _ in range(H)]
        douts = [torch.randn((seq, dh), generator=gen, device=dev) for _ in range(H)]
        grads = [[torch.empty((seq, dh), device=dev) for _ in range(H)] for _ in range(3)]
        pl, pdo = arr(lses), arr(douts)
        pg = [arr(g) for g in grads]
        rc = lib.vedic_flash_attention_fwd_heads(pq, pk, pv, po, pl, H, seq, dh, scale, *flags, stream)
        if rc:
            raise RuntimeError(f"flash attention failed: {_lib.status_string(rc)}")

        def bstep():
            rc = lib.vedic_flash_attention_bwd_heads(pq, pk, pv, po, pdo, pl, pg[0], pg[1], pg[2], H, seq, dh, scale,
                                                     *flags, stream)
            if rc:
                raise RuntimeError(f"flash attention backward failed: {_lib.status_string(rc)}")

        bstep.keep = (qs, ks, vs, outs, lses, douts, grads, pq, pk, pv, po, pl, pdo, pg)
        flops = 10.0 * dh * attn_pairs(a) * H  # S, dP, dV, dQ, dK once each
        return bstep, flops, 9 * seq * dh * 4 * H, 2

    def step():
        if a["batched"]:
            rc = lib.vedic_flash_attention_fwd_heads(pq, pk, pv, po, None, H, seq, dh, scale, *flags, stream)
            if rc:
                raise RuntimeError(f"flash attention failed: {_lib.status_string(rc)}")
            return
        for h in range(H):
            rc = lib.vedic_flash_attention_fwd(qs[h].data_ptr(), ks[h].data_ptr(), vs[h].data_ptr(),
                                               outs[h].data_ptr(), None, seq, dh, scale, *flags, stream)
            if rc:
                raise RuntimeError(f"flash attention failed: {_lib.status_string(rc)}")

    step.keep = (qs, ks, vs, outs, pq, pk, pv, po)
    flops = 4.0 * dh * attn_pairs(a) * H
    hbm = 4 * seq * dh * 4 * H  # Q, K, V read once, out written
    launches = 1 if a["batched"] else H
    return step, flops, hbm, launches


def run_attn_workload(name, args, torch, dev, with_cpu):
    w = WORKLOADS[name]
    a = w["attn"]
    step, flops, hbm, launches = make_attn_step(w, dev, torch)
    ms, wall = time_steps(step, args.steps, args.warmup, torch)
    tflops = flops / (ms * 1e-3) / 1e12
    roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK["fp32"], "unit": "TFLOP/s",
            "frac": round(tflops / PEAK["fp32"], 4), "traffic": traffic_from_profiles(name),
            "algorithmic_flops_per_launch": flops / launches, "algorithmic_bytes_per_launch": hbm / launches,
            "kernel_avg_us": round(ms * 1e3 / launches, 3)}
    cpu = cpu_baseline_attn(w, args.cpu_seconds) if with_cpu else None
    return {
        "metric": f"attention {'backward' if a['bwd'] else 'forward'} TFLOP/s, {name}, 1 GPU",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded torch.randn Q, K, V ~ N(0,1))",
        "config": {"workload": name, "baseline_config": w["cfg"], "seq": a["seq"], "dh": a["dh"],
                   "heads": a["heads"], "launches": launches, "causal": a["causal"], "shunyam": a["shunyam"],
                   "scale": "1/sqrt(dh)",
                   "flops": f"{10 if a['bwd'] else 4} dh per allowed (query, key) pair"},
        "pct_of_peak": round(100.0 * tflops / PEAK["fp32"], 2),
        "roofline": roof,
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }


def run_workload(name, args, torch, dev, with_cpu):
    w = WORKLOADS[name]
    if "attn" in w:
        return run_attn_workload(name, args, torch, dev, with_cpu)
    step, items = make_step(w, dev, torch)
    ms, wall = time_steps(step, args.steps, args.warmup, torch)
    flops = sum(f for _, f, _, _ in items)
    hbm = sum(b for _, _, b, _ in items)
    hbm_launches = sum(b for _, _, _, b in items)
    dtype = w["gemms"][0]["dtype"]
    peak_key = "fp32" if dtype == "fp32" else "fp16"  # the AMP path multiplies binary16 values
    tflops = flops / (ms * 1e-3) / 1e12
    # The bound is the larger of the two floors over the step's launches: the
    # flops at the MFMA peak, or each launch's algorithmic bytes at the HBM
    # peak (a launch re-reads what an earlier one read: the reference's
    # per-head call patterns)
    t_mfma = flops / (PEAK[peak_key] * 1e12)
    t_hbm = hbm_launches / (HBM_PEAK_GBS * 1e9)
    if w.get("hbm") or t_hbm > t_mfma:
        gbs = hbm_launches / (ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(name),
                "algorithmic_bytes_per_launch": hbm_launches / len(items),
                "floors_us": {"mfma": round(t_mfma * 1e6, 2), "hbm": round(t_hbm * 1e6, 2)}}
    else:
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK[peak_key], "unit": "TFLOP/s",
                "frac": round(tflops / PEAK[peak_key], 4), "traffic": traffic_from_profiles(name),
                "algorithmic_flops_per_launch": flops, "algorithmic_bytes_per_launch": hbm,
                "floors_us": {"mfma": round(t_mfma * 1e6, 2), "hbm": round(t_hbm * 1e6, 2)}}
    roof["kernel_avg_us"] = round(ms * 1e3 / len(items), 3)
    cpu = cpu_baseline(w, args.cpu_seconds) if with_cpu else None
    g0 = w["gemms"][0]
    config = {"workload": name, "baseline_config": w["cfg"], "gemms": len(items),
              "accumulate": "fp32", "output": "fp32"}
    if len(items) == 1:
        config.update({k: g0[k] for k in ("M", "K", "N", "op", "epi", "beta")})
    return {
        "metric": METRIC if name == "ffn_up_fp16_bias_gelu" else f"GEMM TFLOP/s, {name}, 1 GPU",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded torch.randn: activations N(0,1), weights N(0,0.02), bias N(0,0.01); "
                "fp16 operands rounded by torch's half() cast)",
        "config": config,
        "pct_of_peak": round(100.0 * tflops / PEAK[peak_key], 2),
        "roofline": roof,
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }


def run_copy(args, torch, dev):
    n = 256 * 1024 * 1024 // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    ms, _ = time_steps(lambda: dst.copy_(src), args.steps, args.warmup, torch)
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    return {"workload": COPY_WORKLOAD, "ms_per_copy": round(ms, 5), "GB/s": round(gbs, 1)}


def run_cast(args, torch, dev):
    from logos_amd import _lib

    lib = _lib.load()
    n = 64 * 1024 * 1024
    src = torch.randn(n, device=dev).half()
    dst = torch.empty(n, device=dev)
    s = torch.cuda.current_stream().cuda_stream

    def step():
        rc = lib.vedic_cast_f16_to_f32(src.data_ptr(), dst.data_ptr(), n, s)
        if rc:
            raise RuntimeError(_lib.status_string(rc))

    ms, _ = time_steps(step, args.steps, args.warmup, torch)
    gbs = 6 * n / (ms * 1e-3) / 1e9
    return {"workload": CAST_WORKLOAD, "ms_per_cast": round(ms, 5), "GB/s": round(gbs, 1),
            "bytes_read": 2 * n, "bytes_written": 4 * n}


def run_layernorm(args, torch, dev):
    from logos_amd import _lib

    lib = _lib.load()
    seq, d = 8192, 1024
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x4C4E)
    X = torch.randn((seq, d), generator=gen, device=dev)
    g = 1.0 + 0.1 * torch.randn(d, generator=gen, device=dev)
    b = 0.1 * torch.randn(d, generator=gen, device=dev)
    Y = torch.empty_like(X)
    Y16 = torch.empty((seq, d), dtype=torch.float16, device=dev)
    s = torch.cuda.current_stream().cuda_stream

    def ok(rc):
        if rc:
            raise RuntimeError(_lib.status_string(rc))

    def fused():
        ok(lib.vedic_layernorm(X.data_ptr(), g.data_ptr(), b.data_ptr(), Y.data_ptr(), Y16.data_ptr(), seq, d,
                               1e-5, s))

    def two_pass():
        ok(lib.vedic_layernorm(X.data_ptr(), g.data_ptr(), b.data_ptr(), Y.data_ptr(), None, seq, d, 1e-5, s))
        ok(lib.vedic_cast_f32_to_f16(Y.data_ptr(), Y16.data_ptr(), seq * d, s))

    ms, _ = time_steps(fused, args.steps, args.warmup, torch)
    ms2, _ = time_steps(two_pass, args.steps, args.warmup, torch)
    nbytes = seq * d * (4 + 4 + 2)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": LN_WORKLOAD, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
            "value": round(gbs, 1), "unit": "GB/s", "GB/s": round(gbs, 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s",
                         "frac": round(gbs / 8000.0, 4)},
            "two_pass_ms": round(ms2, 5), "bytes_per_step": nbytes}


def main():
    args = parse()
    if args.summarize_traffic:
        summarize_traffic(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == COPY_WORKLOAD:
        print(json.dumps(run_copy(args, torch, dev)), flush=True)
        return
    if args.workload == LN_WORKLOAD:
        print(json.dumps(run_layernorm(args, torch, dev)), flush=True)
        return
    if args.workload == CAST_WORKLOAD:
        print(json.dumps(run_cast(args, torch, dev)), flush=True)
        return
    if args.all:
        for name in WORKLOADS:
            out = run_workload(name, args, torch, dev, with_cpu=not args.no_cpu)
            print(json.dumps(out), flush=True)
            torch.cuda.empty_cache()
        return
    print(json.dumps(run_workload(args.workload, args, torch, dev, with_cpu=not args.no_cpu)), flush=True)


if __name__ == "__main__":
    main()
