"""The workspace block kept per (device, stream) for the temporaries of
library calls (split-K slabs, column partials, the AMP cast buffer):

  - calls on two streams, queued back to back without synchronising, give
    the single-stream results bit for bit;
  - a call that needs more than the block holds (the block grows at the next
    call) and calls after vedic_workspace_release give the same bits;
  - host threads sharing one stream (ctypes releases the GIL, so the calls
    really overlap on the host) give the same bits: a call holds the block
    until its last kernel is queued.
Results are the single-stream results of the same calls (themselves checked
against the oracle in test_gpu_parity.py)."""
import ctypes
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from logos_amd import _lib  # noqa: E402
from tests._gpu_helpers import dev, normal  # noqa: E402

pytestmark = pytest.mark.gpu


def V():
    from logos_amd import vedic

    return vedic


def split_case(rng, M, N, K):
    """fp16 NN product small enough in M x N and long enough in K to be split
    over K (a workspace slab per slice)."""
    a = dev(normal(rng, (M, K))).half()
    b = dev(normal(rng, (K, N), std=0.05)).half()
    return a, b


def colsum_case(rng, M, N, K):
    a = dev(normal(rng, (M, K))).half()
    b = dev(normal(rng, (K, N), std=0.05)).half()
    return a, b


def run_split(vedic, a, b):
    return vedic.gemm(vedic.OP_NN, a, b)


def run_colsum(vedic, a, b):
    cs = torch.zeros(b.shape[1], device="cuda")
    C = vedic.gemm(vedic.OP_NN, a, b, colsum=cs)
    return C, cs


def test_two_streams_match_one():
    vedic = V()
    rng = np.random.default_rng(1)
    cases = [split_case(rng, 256, 256, 4096), split_case(rng, 128, 384, 8192), colsum_case(rng, 1000, 264, 512)]
    ref = [run_split(vedic, *cases[0]), run_split(vedic, *cases[1]), run_colsum(vedic, *cases[2])]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(3):
        for i, s in enumerate((s1, s2)):
            with torch.cuda.stream(s):
                outs.append((run_split(vedic, *cases[(i + rep) % 2]), (i + rep) % 2))
                outs.append((run_colsum(vedic, *cases[2]), 2))
    torch.cuda.synchronize()
    for got, k in outs:
        if k == 2:
            assert torch.equal(got[0], ref[2][0]) and torch.equal(got[1], ref[2][1])
        else:
            assert torch.equal(got, ref[k])


def test_growth_and_release():
    vedic = V()
    lib = _lib.load()
    rng = np.random.default_rng(2)
    small = split_case(rng, 128, 128, 2048)
    big = split_case(rng, 1024, 1024, 8192)
    r_small, r_big = run_split(vedic, *small), run_split(vedic, *big)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert lib.vedic_workspace_release(s.cuda_stream) == 0
        got = [run_split(vedic, *small), run_split(vedic, *big), run_split(vedic, *big), run_split(vedic, *small)]
        assert lib.vedic_workspace_release(s.cuda_stream) == 0
        got.append(run_split(vedic, *big))
    torch.cuda.synchronize()
    for g, r in zip(got, [r_small, r_big, r_big, r_small, r_big]):
        assert torch.equal(g, r)


def test_threads_sharing_a_stream():
    vedic = V()
    lib = _lib.load()
    rng = np.random.default_rng(3)
    M, N, K = 256, 256, 4096
    cases = [split_case(rng, M, N, K) for _ in range(4)]
    refs = [run_split(vedic, *c) for c in cases]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    outs = [[torch.empty((M, N), device="cuda") for _ in range(8)] for _ in cases]
    torch.cuda.synchronize()
    errors = []

    def work(t):
        a, b = cases[t]
        for rep in range(8):
            d = _lib.GemmDesc(op=0, in_dtype=1, out_dtype=0, M=M, N=N, K=K, A=a.data_ptr(), lda=K, B=b.data_ptr(),
                              ldb=N, C=outs[t][rep].data_ptr(), ldc=N, alpha=1.0, beta=0.0, stream=s.cuda_stream)
            st = lib.vedic_gemm(ctypes.byref(d))
            if st != 0:
                errors.append(st)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(cases))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors
    for t, r in enumerate(refs):
        for g in outs[t]:
            assert torch.equal(g, r)


HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread ((hipStream_t)2, hip_runtime_api.h)


def test_threads_on_their_per_thread_streams():
    """Host threads passing the hipStreamPerThread handle each run on their
    own stream; the library keeps their workspace blocks apart (one handle
    value, several streams), so the split products, whose slices live in
    the block, match the single-stream results bit for bit.  Each thread
    releases its block before it ends."""
    vedic = V()
    lib = _lib.load()
    rng = np.random.default_rng(4)
    M, N, K = 256, 256, 4096
    cases = [split_case(rng, M, N, K) for _ in range(4)]
    refs = [run_split(vedic, *c) for c in cases]
    outs = [[torch.empty((M, N), device="cuda") for _ in range(8)] for _ in cases]
    torch.cuda.synchronize()
    errors = []
    barrier = threading.Barrier(len(cases))

    def work(t):
        a, b = cases[t]
        barrier.wait()
        for rep in range(8):
            d = _lib.GemmDesc(op=0, in_dtype=1, out_dtype=0, M=M, N=N, K=K, A=a.data_ptr(), lda=K, B=b.data_ptr(),
                              ldb=N, C=outs[t][rep].data_ptr(), ldc=N, alpha=1.0, beta=0.0,
                              stream=HIP_STREAM_PER_THREAD)
            st = lib.vedic_gemm(ctypes.byref(d))
            if st != 0:
                errors.append(st)
        torch.cuda.synchronize()
        st = lib.vedic_workspace_release(HIP_STREAM_PER_THREAD)
        if st != 0:
            errors.append(st)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(cases))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, [_lib.status_string(e) for e in errors]
    for t, r in enumerate(refs):
        for g in outs[t]:
            assert torch.equal(g, r)


def test_checked_gemm_with_work_queued_ahead_and_threads():
    """vedic_gemm_checked returns once its last kernel has published the
    result in host memory (polled, with a stream synchronisation as the
    fallback).  With a long product queued ahead on the same stream, and with
    four host threads each on its own stream, every call returns the values
    of a quiet single-thread call, bit for bit."""
    vedic = V()
    rng = np.random.default_rng(4)
    M, N, K = 1024, 2048, 1024
    cases = [(dev(normal(rng, (M, K))).half(), dev(normal(rng, (K, N), std=0.02)).half()) for _ in range(4)]
    refs = []
    for a, b in cases:
        C, r = vedic.gemm_checked(vedic.OP_NN, a, b)
        refs.append((C.clone(), r.checksum_C, r.checksum_vedic))
    big_a = dev(normal(rng, (8192, 4096))).half()
    big_b = dev(normal(rng, (4096, 4096), std=0.02)).half()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for _ in range(3):
            vedic.gemm(vedic.OP_NN, big_a, big_b)  # about a millisecond of queued work
        C, r = vedic.gemm_checked(vedic.OP_NN, *cases[0])
        assert torch.equal(C, refs[0][0]) and (r.checksum_C, r.checksum_vedic) == refs[0][1:]
    torch.cuda.synchronize()
    errors = []

    def work(t):
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            for _ in range(20):
                C, r = vedic.gemm_checked(vedic.OP_NN, *cases[t])
                if not (torch.equal(C, refs[t][0]) and (r.checksum_C, r.checksum_vedic) == refs[t][1:]):
                    errors.append(t)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors


def test_attention_queue_counter_between_calls():
    """The one-head attention forward takes its split key ranges from a
    work-queue counter kept per (device, stream) and put back to zero by the
    merge kernel: calls interleaved with split-K GEMMs (which reuse the
    workspace block), on a second stream, and after vedic_workspace_release
    (which frees the counter) all give the first call's bits."""
    vedic = V()
    lib = _lib.load()
    rng = np.random.default_rng(4)
    seq, dh = 4096, 64
    Q, K, Vv = (dev(normal(rng, (seq, dh))) for _ in range(3))
    ref = vedic.flash_attention_fwd(Q, K, Vv)
    split = split_case(rng, 1024, 1024, 8192)
    r_split = run_split(vedic, *split)
    torch.cuda.synchronize()
    got, splits = [], []
    for s in (torch.cuda.current_stream(), torch.cuda.Stream()):
        with torch.cuda.stream(s):
            for rep in range(3):
                got.append(vedic.flash_attention_fwd(Q, K, Vv))
                splits.append(run_split(vedic, *split))
                got.append(vedic.flash_attention_fwd(Q, K, Vv))
            assert lib.vedic_workspace_release(s.cuda_stream) == 0
            got.append(vedic.flash_attention_fwd(Q, K, Vv))
    torch.cuda.synchronize()
    for g in got:
        assert torch.equal(g, ref)
    for g in splits:
        assert torch.equal(g, r_split)
