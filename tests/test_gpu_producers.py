"""GPU parity of the activation producers (rmsnorm_quant, swiglu_quant, add_norm_quant; zero/kernels/ops.cl:82-128,
2025-2075) against the oracle. The f32 values entering the quantizer come from f32 sums of squares and expf in
another order than the CPU's, so they are compared with a tolerance (max |err| / max |ref| < 2e-6), and where the
kernel exposes them (h, the updated x) the int8 outputs must be the quantizer's exact result on those values. Where it
does not, int8 values may differ by one step only next to a rounding tie (at most 0.1 % of them)."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def near_int8(a, b):
    d = np.abs(a.astype(np.int32) - b.astype(np.int32))
    return d.max() <= 1 and np.mean(d > 0) <= 1e-3


@pytest.mark.parametrize("M,Ms,K", [(1, 16, 5120), (7, 8, 2048), (3, 3, 17408), (2, 4, 96), (300, 304, 2048)])
def test_rmsnorm_quant(qm, dev, M, Ms, K):
    import torch
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10)).astype(np.float32)
    w = rng.uniform(0.2, 2.0, K).astype(np.float32)
    aq, asc, absum, h = qm.rmsnorm_quant(to_dev(x, dev), to_dev(w, dev), 1e-6, M_stride=Ms, want_h=True)
    torch.cuda.synchronize()
    raq, rasc, rabs, rh = oracle.rmsnorm_quant(x, w, 1e-6, M_stride=Ms)
    hg = h.cpu().numpy()
    assert rel(hg, rh) < 2e-6
    assert np.all(hg[M:] == 0)
    q2, s2, a2 = oracle.quantize_act(hg[:M], M_stride=Ms)  # the quantizer's exact result on the kernel's own y
    assert np.array_equal(aq.cpu().numpy(), q2) and np.array_equal(absum.cpu().numpy(), a2)
    assert np.array_equal(asc.cpu().numpy().view(np.uint32), s2.view(np.uint32))
    assert near_int8(aq.cpu().numpy(), raq) and rel(asc.cpu().numpy(), rasc) < 2e-6


@pytest.mark.parametrize("gelu", [False, True])
@pytest.mark.parametrize("M,Ms,F", [(1, 16, 17408), (5, 8, 512), (2, 2, 96), (260, 260, 1024)])
def test_swiglu_quant(qm, dev, gelu, M, Ms, F):
    import torch
    rng = np.random.default_rng(F + M)
    gu = (rng.standard_normal((M, 2 * F)) * 3).astype(np.float32)
    aq, asc, absum = qm.swiglu_quant(to_dev(gu, dev), F, gelu=gelu, M_stride=Ms)
    torch.cuda.synchronize()
    raq, rasc, rabs, rh = oracle.swiglu_quant(gu, F, gelu=gelu, M_stride=Ms)
    assert near_int8(aq.cpu().numpy(), raq) and rel(asc.cpu().numpy(), rasc) < 2e-6
    assert np.all(aq.cpu().numpy()[M:] == 0)


def test_swiglu_quant_fused_is_the_quantizer(qm, dev):
    import torch
    rng = np.random.default_rng(9)
    rows = rng.standard_normal((5, 1024)).astype(np.float32)
    aq, asc, absum = qm.swiglu_quant(to_dev(rows, dev), 1024, fused=True, M_stride=8)
    torch.cuda.synchronize()
    q2, s2, a2 = oracle.quantize_act(rows, M_stride=8)
    assert np.array_equal(aq.cpu().numpy(), q2) and np.array_equal(absum.cpu().numpy(), a2)
    assert np.array_equal(asc.cpu().numpy().view(np.uint32), s2.view(np.uint32))


@pytest.mark.parametrize("with_w2", [False, True])
@pytest.mark.parametrize("M,Ms,K", [(1, 16, 5120), (4, 4, 2048), (2, 8, 16384)])
def test_add_norm_quant(qm, dev, with_w2, M, Ms, K):
    import torch
    rng = np.random.default_rng(K + M + with_w2)
    x = rng.standard_normal((M, K)).astype(np.float32)
    t = (rng.standard_normal((M, K)) * 4).astype(np.float32)
    w = rng.uniform(0.2, 2.0, K).astype(np.float32)
    w2 = rng.uniform(0.2, 2.0, K).astype(np.float32) if with_w2 else None
    xd = to_dev(x, dev)
    aq, asc, absum = qm.add_norm_quant(xd, to_dev(t, dev), to_dev(w, dev), 1e-6, 0.8,
                                       w2=None if w2 is None else to_dev(w2, dev), M_stride=Ms)
    torch.cuda.synchronize()
    rx, raq, rasc, rabs, rh = oracle.add_norm_quant(x, t, w, 1e-6, 0.8, w2=w2, M_stride=Ms)
    xg = xd.cpu().numpy()
    assert rel(xg, rx) < 2e-6
    if w2 is None:  # y is the updated x: the int8 outputs are the quantizer's exact result on it
        q2, s2, a2 = oracle.quantize_act(xg, M_stride=Ms)
        assert np.array_equal(aq.cpu().numpy(), q2) and np.array_equal(absum.cpu().numpy(), a2)
        assert np.array_equal(asc.cpu().numpy().view(np.uint32), s2.view(np.uint32))
    assert near_int8(aq.cpu().numpy(), raq) and rel(asc.cpu().numpy(), rasc) < 2e-6
    assert np.all(aq.cpu().numpy()[M:] == 0)


def test_producer_feeds_the_gemv(qm, dev):
    """rmsnorm_quant -> IQ4_XS GEMV, end to end against the oracle's rmsnorm_quant -> blockdot."""
    import torch
    from arcinfer_amd import formats as F
    rng = np.random.default_rng(21)
    N, K = 512, 2048
    W = F.synth_weight(F.IQ4_XS, N, K, seed=21)
    x = rng.standard_normal((1, K)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    qw = qm.QWeight(F.IQ4_XS, to_dev(W, dev), N, K)
    aq, asc, absum, _ = qm.rmsnorm_quant(to_dev(x, dev), to_dev(w, dev), 1e-6, M_stride=16)
    y = qm.gemv(qw, aq, asc, absum)
    torch.cuda.synchronize()
    raq, rasc, rabs, _ = oracle.rmsnorm_quant(x, w, 1e-6, M_stride=16)
    ref = oracle.blockdot(F.IQ4_XS, W, K, raq, rasc, rabs, M=1)
    assert rel(y.cpu().numpy(), ref) < 1e-3
    qw.release()
