"""The allocation-free GEMM entry point (qmatmul_gemm_noalloc) against qmatmul_gemm, through the C ABI: two calls in a
row on the static scratch array, the second with a smaller input, each bit-identical to qmatmul_gemm's result (the
same kernels run on the same inputs; only where the workspace lives differs). Also: a shape beyond the scratch's
capacity is refused with QM_ERR_WORKSPACE, and a shape on the int8 path (no scratch) matches too."""
import numpy as np
import pytest

from arcinfer_amd import formats as F

pytestmark = pytest.mark.gpu


def _case(qm, dev, qtype, M, N, K, seed):
    import torch
    W = F.synth_weight(qtype, N, K, seed=seed)
    x = F.synth_activations(M, K, seed=seed + 1, outlier_frac=0.01)
    aq, asc, absum = qm.quantize_act(torch.from_numpy(x).to(dev))
    w = qm.QWeight(qtype, torch.from_numpy(W).to(dev), N, K)
    return w, aq, asc, absum


def test_noalloc_matches_gemm_twice(qm, dev):
    import torch
    for (M, N, K, seed) in [(512, 384, 2048, 1), (200, 256, 1024, 2)]:  # second call smaller than the first
        w, aq, asc, absum = _case(qm, dev, F.Q4_K, M, N, K, seed)
        ref = qm.gemm(w, aq, asc, absum)
        got = qm.gemm(w, aq, asc, absum, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, N, K)
        # accumulate into an offset window, as qmatmul_gemm does
        C0 = torch.randn(M, N + 8, device=dev)
        C1 = C0.clone()
        qm.gemm(w, aq, asc, absum, C=C0, ldc=N + 8, c_off=3, accumulate=1)
        qm.gemm(w, aq, asc, absum, C=C1, ldc=N + 8, c_off=3, accumulate=1, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(C0, C1)
        w.release()


def test_noalloc_int8_path_and_capacity(qm, dev):
    import torch
    w, aq, asc, absum = _case(qm, dev, F.IQ4_XS, 64, 256, 1024, 5)
    ref = qm.gemm(w, aq, asc, absum)
    got = qm.gemm(w, aq, asc, absum, noalloc=True)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    w.release()
    # 4096 x 5120 needs 2 * 4096 * 5120 + 4 * 4096 * 160 bytes = 44.6 MB > 32 MiB: refused, nothing written
    M, N, K = 4096, 128, 5120
    w, aq, asc, absum = _case(qm, dev, F.Q4_K, M, N, K, 7)
    C = torch.full((M, N), 3.0, device=dev)
    with pytest.raises(qm.QMatmulError) as ei:
        qm.gemm(w, aq, asc, absum, C=C, ldc=N, noalloc=True)
    assert ei.value.status == 6  # QM_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert bool(torch.all(C == 3.0))
    w.release()
