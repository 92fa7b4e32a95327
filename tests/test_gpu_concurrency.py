"""GEMMs from several host threads, each on its own stream, interleaved with
torch kernels on those streams: every result must equal, bit for bit, the
result of the same product computed alone.

Regression test for the stage pipelines' barrier: a wave's last LDS reads of
a stage could still be in flight at the stage barrier (the compiler places
the stage's last MFMAs, and the waits for their fragments, after it), and
another wave's direct loads into that buffer -- the zero loads past a work
item's range arrive within a few hundred cycles -- could overtake them when
a workgroup of another kernel on the same CU held up the LDS.  About 1 % of
such calls came out wrong before the barrier waited for the wave's reads."""
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests._gpu_helpers import dev, normal  # noqa: E402

pytestmark = pytest.mark.gpu


def V():
    from logos_amd import vedic

    return vedic


@pytest.mark.parametrize("shape,dtype", [((1024, 2048, 1024), "fp16"),   # 128 x 128 tiles
                                         ((2048, 2048, 1024), "fp16"),   # 256 x 128 / 256 x 256 tiles
                                         ((512, 1024, 1024), "fp32")])   # wave-split fp32 tiles
def test_threads_on_own_streams_match_alone(shape, dtype):
    vedic = V()
    M, N, K = shape
    rng = np.random.default_rng(M + N + K)
    cases = []
    for _ in range(4):
        a = dev(normal(rng, (M, K)))
        b = dev(normal(rng, (K, N), std=0.02))
        cases.append((a.half(), b.half()) if dtype == "fp16" else (a, b))
    refs = [vedic.gemm(vedic.OP_NN, a, b).clone() for a, b in cases]
    torch.cuda.synchronize()
    errors = []
    iters = 100

    def work(t, st):
        with torch.cuda.stream(st):
            for i in range(iters):
                C = vedic.gemm(vedic.OP_NN, *cases[t])
                if not torch.equal(C, refs[t]):  # a torch kernel on this stream, beside other threads' GEMMs
                    errors.append((t, i, float((C - refs[t]).abs().max())))

    threads = [threading.Thread(target=work, args=(t, torch.cuda.Stream())) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors[:5]


def test_mixed_kernel_families_on_threads_match_alone():
    """Four host threads on their own streams, each drawing calls at random
    from every kernel family (256 x 256, NT, TN and split-K fp16 GEMMs, the
    fp32 tiled and row-block GEMMs, fp16 and fp32 decode, both AMP paths,
    the fused GELU backward with its bias gradient, gathered and scattered
    products, attention forward + backward, layer normalisation): every
    result equals, bit for bit, the same call made alone."""
    vedic = V()
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    r = lambda *s, std=1.0: torch.randn(*s, generator=g, device="cuda") * std  # noqa: E731
    A, B, Bt, bias = r(1024, 512).half(), r(512, 1024, std=0.02).half(), r(1024, 512, std=0.02).half(), r(1024)
    X, dY = r(4096, 512).half(), r(4096, 384, std=1e-2).half()
    X2, dY2 = r(8192, 256).half(), r(8192, 256, std=1e-2).half()
    F, G, F2, G2 = r(512, 1024), r(1024, 1024, std=0.02), r(1024, 512), r(512, 1536, std=0.02)
    a16, w16, a32, w32 = r(8, 1024).half(), r(1024, 2048, std=0.02).half(), r(1, 1024), r(1024, 2048, std=0.02)
    Aa, W16 = r(512, 1024), r(1024, 2048, std=0.02).half()
    dYg, Wg, Hg = r(1024, 512, std=1e-2).half(), r(1024, 512, std=0.02).half(), r(1024, 1024, std=2.0)
    heads, Wo = [r(512, 64).half() for _ in range(8)], r(512, 512, std=0.02).half()
    Q, K, Vv = r(256, 64), r(256, 64), r(256, 64)
    Xl, gam, bet = r(1024, 1024), 1 + 0.1 * r(1024), 0.1 * r(1024)

    def gbwd():
        db = torch.zeros(1024, device="cuda")
        return torch.cat([vedic.gemm_nt_gelu_bwd(dYg, Wg, Hg, db=db).flatten(), db])

    def scat():
        hs = [torch.empty(512, 64, device="cuda") for _ in range(8)]
        vedic.gemm_scatter(A[:512], Bt[:512].t().contiguous(), hs)
        return torch.cat([h.flatten() for h in hs])

    def attn():
        lse = torch.empty(256, device="cuda")
        o = vedic.flash_attention_fwd(Q, K, Vv, lse=lse, causal=True)
        dq, dk, dv = vedic.flash_attention_bwd(Q, K, Vv, o, torch.full_like(o, 0.01), lse, causal=True)
        return torch.cat([o.flatten(), lse, dq.flatten(), dk.flatten(), dv.flatten()])

    calls = [lambda: vedic.gemm_bias_gelu(A, B, bias), lambda: vedic.gemm(vedic.OP_NT, A, Bt),
             lambda: vedic.gemm(vedic.OP_TN, X, dY), lambda: vedic.gemm(vedic.OP_TN, X2, dY2),
             lambda: vedic.gemm(vedic.OP_NN, F, G), lambda: vedic.gemm(vedic.OP_NN, F2, G2),
             lambda: vedic.gemm(vedic.OP_NN, a16, w16), lambda: vedic.gemm(vedic.OP_NN, a32, w32),
             lambda: vedic.gemm(vedic.OP_NN, Aa, W16), lambda: vedic.gemm(vedic.OP_NN, Aa[:, :512], W16[:512, :1024]),
             gbwd, lambda: vedic.gemm_gather(heads, Wo), scat, attn,
             lambda: vedic.layernorm(Xl, gam, bet)[0]]
    refs = []
    for fn in calls:
        refs.append(fn().clone())
        torch.cuda.synchronize()
    errors, iters = [], 120

    def work(t, st):
        rng = np.random.default_rng(t)
        with torch.cuda.stream(st):
            for i in range(iters):
                k = int(rng.integers(len(calls)))
                out = calls[k]()
                st.synchronize()
                if not torch.equal(out.view(torch.int32), refs[k].view(torch.int32)):
                    errors.append((t, i, k, float((out - refs[k]).abs().max())))

    threads = [threading.Thread(target=work, args=(t, torch.cuda.Stream())) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors[:5]
