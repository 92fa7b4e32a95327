"""Build recipe for liblogos_vedic.so (the gfx950 HIP library) and the CPU oracle.

Usage:  python -m logos_amd.build [--jobs N]

The library is compiled in-tree with hipcc for gfx950 only.  Every HIP
translation unit is compiled with packed-fp32 instruction selection disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``); the host pass prints a
harmless "not a recognized feature" warning for it.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "logos_amd")
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblogos_vedic.so")
SOURCES = [
    "vedic_gemm_f16_nn.hip",
    "vedic_gemm_f16_nt.hip",
    "vedic_gemm_f16_tn.hip",
    "vedic_gemm_f16_amp.hip",
    "vedic_gemm_f16_gather.hip",
    "vedic_gemm_f32_nn.hip",
    "vedic_gemm_f32_nt.hip",
    "vedic_gemm_f32_tn.hip",
    "vedic_gemm_mfma.hip",
    "vedic_gemm_skinny.hip",
    "vedic_flash_attn.hip",
    "vedic_flash_attn_bwd.hip",
    "vedic_flash_probs.hip",
    "vedic_layernorm.hip",
    "vedic_capi.hip",
]

ARCH = "gfx950"
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _run(cmd: list[str], cwd: str | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build_library(jobs: int = 6) -> str:
    os.makedirs(OBJ, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()
    tmp = LIB + ".tmp"
    _run([cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs])
    check_wide_stores(tmp)
    os.replace(tmp, LIB)
    return LIB


def check_wide_stores(lib: str) -> None:
    """Fails the build if a 12- or 16-byte store's data registers are
    rewritten within isa_check.WINDOW wait states on any path (isa_check)."""
    from logos_amd import isa_check

    total, found = isa_check.scan(lib)
    if found:
        lines = [f"{f}: {st} ; {u} after {ws} wait states" for f, st, u, ws in found[:20]]
        raise RuntimeError(f"{len(found)} of {total} wide stores have a data register rewritten within "
                           f"{isa_check.WINDOW} wait states:\n" + "\n".join(lines))


CPP_DIR = os.path.join(ROOT, "tests", "cpp")
CPP_TEST_SRC = os.path.join(CPP_DIR, "vedic_hip_test.cpp")
CPP_TEST_BIN = os.path.join(CPP_DIR, "vedic_hip_test")
CPP_TENSOR_SRC = os.path.join(CPP_DIR, "vedic_tensor_test.cpp")
CPP_TENSOR_BIN = os.path.join(CPP_DIR, "vedic_tensor_test")


def build_cpp_test() -> str:
    """The C++ test programs of the drop-in headers: vedic_hip_test over
    include/VedicGEMM_hip.hpp (its raw-launch kernels are device code, hence
    gfx950) and vedic_tensor_test over include/VedicGEMM.hpp with the test
    Tensor of tests/cpp/tensor_stub; each linked against the library with an
    rpath relative to itself (so it runs wherever the tree is)."""
    inc = f"-I{os.path.join(ROOT, 'include')}"
    common = ["-O2", "-std=c++17", "-Wall", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
              "-packed-fp32-ops", inc]
    link = [f"-L{PKG}", "-llogos_vedic", "-Wl,-rpath,$ORIGIN/../../logos_amd"]
    for src, out, extra in ((CPP_TEST_SRC, CPP_TEST_BIN, []),
                            (CPP_TENSOR_SRC, CPP_TENSOR_BIN, [f"-I{os.path.join(CPP_DIR, 'tensor_stub')}"])):
        tmp = out + ".tmp"
        _run([hipcc(), *common, *extra, src, *link, "-o", tmp])
        os.replace(tmp, out)
    return CPP_TEST_BIN


def build_oracle(with_reference: bool = True) -> None:
    odir = os.path.join(ROOT, "oracle")
    _run(["make", "-s", "-B", "liblogos_oracle.so"], cwd=odir)
    if with_reference and os.path.isdir("/root/reference/include"):
        _run(["make", "-s", "-B", "ref"], cwd=odir)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=6)
    ap.add_argument("--no-oracle", action="store_true")
    args = ap.parse_args()
    print(build_library(args.jobs))
    print(build_cpp_test())
    if not args.no_oracle:
        build_oracle()


if __name__ == "__main__":
    main()
