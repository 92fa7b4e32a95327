"""The C++ drop-in headers: include/VedicGEMM_hip.hpp (the reference's GPUTensor /
cuda_vedic_gemm / cuda_gemm_fp16_fp32out surface over the C ABI, and the
kernels its callers launch raw), driven by tests/cpp/vedic_hip_test.cpp, and
include/VedicGEMM.hpp (reference_gemm / vedic_gemm / vedic_gemm_bias on
Tensor), driven by tests/cpp/vedic_tensor_test.cpp; logos_amd/build.py
compiles both.

CPU: the program was built and links liblogos_vedic.so and the HIP runtime.
GPU: the program runs its known-answer, layout, fp16 and error-path checks.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "vedic_hip_test")
TENSOR_BIN = os.path.join(ROOT, "tests", "cpp", "vedic_tensor_test")


def test_cpp_program_links_the_library():
    assert os.path.exists(BIN), "tests/cpp/vedic_hip_test missing: run `python -m logos_amd.build`"
    out = subprocess.run(["ldd", BIN], capture_output=True, text=True, check=True).stdout
    assert "liblogos_vedic.so" in out and "amdhip64" in out


def test_header_declares_reference_names():
    text = open(os.path.join(ROOT, "include", "VedicGEMM_hip.hpp")).read()
    for name in ["struct GPUTensor", "struct HalfTensor", "gpu_alloc(", "half_alloc(", "h2d(", "d2h(",
                 "cuda_vedic_gemm(", "cuda_vedic_gemm_bias(", "cuda_vedic_gemm_uses_cublas(",
                 "cuda_gelu(", "cuda_vedic_verify(", "cuda_gemm_fp16_fp32out(", "cuda_gemm_fp16_fp16out(",
                 "cuda_cast_fp32_to_fp16(", "cuda_cast_fp16_to_fp32(", "cuda_vedic_gemm_nt(",
                 "cuda_vedic_gemm_tn(", "cuda_gemm_fp16_bias_gelu("]:
        assert name in text, name


def test_tensor_header_declares_reference_names():
    text = open(os.path.join(ROOT, "include", "VedicGEMM.hpp")).read()
    for name in ["VEDIC_BLOCK = 64", "inline Tensor reference_gemm(const Tensor& A, const Tensor& B)",
                 "inline Tensor vedic_gemm(const Tensor& A, const Tensor& B)",
                 "inline Tensor vedic_gemm_bias(const Tensor& A, const Tensor& W, const Tensor& bias)",
                 "std::invalid_argument", '#include "Tensor.hpp"']:
        assert name in text, name
    assert os.path.exists(TENSOR_BIN), "tests/cpp/vedic_tensor_test missing: run `python -m logos_amd.build`"


@pytest.mark.gpu
@pytest.mark.parametrize("binary", [BIN, TENSOR_BIN])
def test_cpp_program_on_gpu(binary):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print("running", binary, flush=True)
    proc = subprocess.run([binary], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ALL PASSED" in proc.stdout
