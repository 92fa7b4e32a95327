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
