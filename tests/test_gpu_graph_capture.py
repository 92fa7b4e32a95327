"""vedic_gemm_noalloc under HIP graph capture, the callers it is meant for.

Each case records one vedic_gemm_noalloc call into a graph
(torch.cuda.graph, global capture mode, so any allocating or synchronising
HIP call inside would end the capture with an error), then replays the graph
four times.  Between replays the program does its own eager work: another
vedic_gemm_noalloc call of a different shape, which overwrites the shared
scratch region, a vedic_gemm call, and the reset of C (and of the column
sums) to their starting values, then a device synchronisation.  Every replay
must reproduce the eager call's C (and column sums) bit for bit: a replay
that read scratch contents left by an earlier call, or a captured node that
behaved differently on later replays, shows up here.

The cases use each kind of temporary the entry point carves from its region:
split-K partial slabs (a TN product with beta = 1), the column partials of the
GELU backward, the binary16 copy of an fp32 activation (AMP product wider
than the in-kernel conversion serves), and none (bias + GELU on the 256 x 256
tiles)."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

from logos_amd import _lib  # noqa: E402

pytestmark = pytest.mark.gpu

CASES = ["splitk_tn_f16", "gelu_bwd_colsum", "amp_cast", "bias_gelu_f16"]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield _lib.load()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _desc(op, in_dtype, M, N, K, A, B, C, *, beta=0.0, epilogue=_lib.EPI_NONE, bias=None, preact=None,
          colsum=None, colsum_beta=0.0):
    return _lib.GemmDesc(op=op, in_dtype=in_dtype, out_dtype=_lib.DT_F32, M=M, N=N, K=K,
                         A=A.data_ptr(), lda=A.shape[1], B=B.data_ptr(), ldb=B.shape[1], C=C.data_ptr(), ldc=N,
                         alpha=1.0, beta=beta, bias=bias.data_ptr() if bias is not None else None,
                         epilogue=epilogue, preact=preact.data_ptr() if preact is not None else None,
                         ld_preact=N if preact is not None else 0,
                         stream=torch.cuda.current_stream().cuda_stream,
                         colsum=colsum.data_ptr() if colsum is not None else None, colsum_beta=colsum_beta)


def _case(case, g):
    r = lambda *s, std=1.0: torch.randn(*s, generator=g, device="cuda") * std  # noqa: E731
    if case == "splitk_tn_f16":  # 1024 x 1024 over K = 8192: four slices into the region
        M, N, K = 1024, 1024, 8192
        A, B = r(K, M).half(), r(K, N, std=1e-2).half()
        return M, N, K, A, B, r(M, N, std=1e-3), dict(op=_lib.OP_TN, in_dtype=_lib.DT_F16, beta=1.0), False
    if case == "gelu_bwd_colsum":  # column partials of every 32-row block in the region
        M, N, K = 2048, 1024, 512
        A, B = r(M, K, std=1e-3).half(), r(N, K, std=0.02).half()
        args = dict(op=_lib.OP_NT, in_dtype=_lib.DT_F16, epilogue=_lib.EPI_GELU_BWD, preact=r(M, N, std=2.0))
        return M, N, K, A, B, torch.zeros(M, N, device="cuda"), args, True
    if case == "amp_cast":  # fp32 activation, N = 2048: cast into the region, then the fp16 product
        M, N, K = 1024, 2048, 1024
        A, B = r(M, K), r(K, N, std=0.02).half()
        args = dict(op=_lib.OP_NN, in_dtype=_lib.DT_F32_F16, epilogue=_lib.EPI_BIAS_GELU, bias=r(N, std=0.01))
        return M, N, K, A, B, torch.zeros(M, N, device="cuda"), args, False
    if case == "bias_gelu_f16":  # no temporaries
        M, N, K = 2048, 2048, 1024
        A, B = r(M, K).half(), r(K, N, std=0.02).half()
        args = dict(op=_lib.OP_NN, in_dtype=_lib.DT_F16, epilogue=_lib.EPI_BIAS_GELU, bias=r(N, std=0.01))
        return M, N, K, A, B, torch.zeros(M, N, device="cuda"), args, False
    raise ValueError(case)


def _bits(t):
    return t.contiguous().view(torch.int32)


@pytest.mark.parametrize("case", CASES)
def test_noalloc_graph_replays(lib, case):
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    M, N, K, A, B, C0, args, want_cs = _case(case, g)
    # the eager work between replays: a split-K product through the same
    # region (other contents), and an ordinary vedic_gemm
    oA, oB = torch.randn(4096, 512, generator=g, device="cuda").half(), \
        torch.randn(4096, 768, generator=g, device="cuda").half()
    oC = torch.zeros(512, 768, device="cuda")
    xA, xB = torch.randn(512, 256, generator=g, device="cuda").half(), \
        torch.randn(256, 384, generator=g, device="cuda").half()
    xC = torch.empty(512, 384, device="cuda")

    C = C0.clone()
    cs = torch.full((N,), 0.5, device="cuda") if want_cs else None
    d = _desc(M=M, N=N, K=K, A=A, B=B, C=C, colsum=cs, colsum_beta=1.0 if want_cs else 0.0, **args)
    assert lib.vedic_gemm_noalloc(ctypes.byref(d)) == _lib.STATUS_OK, case  # eager, and the region's lookup
    torch.cuda.synchronize()
    want, want_sums = C.clone(), cs.clone() if want_cs else None

    graph = torch.cuda.CUDAGraph()
    C.copy_(C0)
    if want_cs:
        cs.fill_(0.5)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        dg = _desc(M=M, N=N, K=K, A=A, B=B, C=C, colsum=cs, colsum_beta=1.0 if want_cs else 0.0, **args)
        status = lib.vedic_gemm_noalloc(ctypes.byref(dg))
    assert status == _lib.STATUS_OK, f"{case}: status {status} under capture"

    for rep in range(4):
        od = _desc(op=_lib.OP_TN, in_dtype=_lib.DT_F16, M=512, N=768, K=4096, A=oA, B=oB, C=oC)
        assert lib.vedic_gemm_noalloc(ctypes.byref(od)) == _lib.STATUS_OK
        xd = _desc(op=_lib.OP_NN, in_dtype=_lib.DT_F16, M=512, N=384, K=256, A=xA, B=xB, C=xC)
        assert lib.vedic_gemm(ctypes.byref(xd)) == _lib.STATUS_OK
        C.copy_(C0)
        if want_cs:
            cs.fill_(0.5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(C), _bits(want)), \
            f"{case}: replay {rep}: {int((C != want).sum())} outputs differ from the eager call"
        if want_cs:
            assert torch.equal(_bits(cs), _bits(want_sums)), f"{case}: replay {rep}: column sums differ"
    del graph
