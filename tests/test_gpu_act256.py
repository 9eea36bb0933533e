"""GPU parity of the per-256 activation layout (the reference's act32 = false: quantize_act_cpu with B = 256,
src/quants.h:559-576; the gemm.cl build without -DACT32, zero/kernels/gemm.cl:413-447; Engine::matmul's act32 flag,
zero/engine.h:3151, 3300): the quantizer and the producers bit-exact against the oracle (on the kernel's own f32
values where they are exposed), and qmatmul_gemm_ex(act32 = 0) against the oracle's per-256 product to the f32
bars of test_gpu_parity.py."""
import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F

from tests.test_gpu_parity import TOL_INT8_PATH, TOL_F32_REF, assert_elementwise, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _same_acts(got, ref):
    aq, asc, absum = (t.cpu().numpy() for t in got)
    raq, rasc, rabs = ref
    assert np.array_equal(aq, raq)
    assert np.array_equal(asc.view(np.uint32), rasc.view(np.uint32))
    assert np.array_equal(absum, rabs)


@pytest.mark.parametrize("M,Ms,K", [(1, 16, 5120), (7, 8, 2048), (300, 304, 4096), (2, 2, 17408)])
def test_quantizer_per256_bit_exact(qm, dev, M, Ms, K):
    import torch
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * rng.choice([1.0, 30.0, 1e-3], size=(M, K))).astype(np.float32)
    x[0, :256] = 0.0  # a zero superblock
    x[0, 256:512] = np.float32(0.5) * (np.arange(256, dtype=np.float32) - 128)  # ties: amax 64 -> step 127/64
    got = qm.quantize_act(to_dev(x, dev), M_stride=Ms, act32=False)
    torch.cuda.synchronize()
    assert got[1].shape == (K // 256, Ms)
    _same_acts(got, oracle.quantize_act(x, M_stride=Ms, act32=False))


@pytest.mark.parametrize("M,Ms,K", [(1, 16, 5120), (5, 8, 2048), (260, 260, 4096)])
def test_producers_per256(qm, dev, M, Ms, K):
    import torch
    rng = np.random.default_rng(7 * M + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10)).astype(np.float32)
    w = rng.uniform(0.2, 2.0, K).astype(np.float32)
    # rmsnorm_quant: the int8 output is the quantizer's exact result on the kernel's own y (h)
    aq, asc, absum, h = qm.rmsnorm_quant(to_dev(x, dev), to_dev(w, dev), 1e-6, M_stride=Ms, want_h=True, act32=False)
    torch.cuda.synchronize()
    hg = h.cpu().numpy()
    assert rel_err(hg, oracle.rmsnorm_quant(x, w, 1e-6, M_stride=Ms)[3]) < 2e-6
    _same_acts((aq, asc, absum), oracle.quantize_act(hg[:M], M_stride=Ms, act32=False))
    # swiglu_quant(fused) is the quantizer itself
    got = qm.swiglu_quant(to_dev(x, dev), K, fused=True, M_stride=Ms, act32=False)
    torch.cuda.synchronize()
    _same_acts(got, oracle.quantize_act(x, M_stride=Ms, act32=False))
    # swiglu_quant: y = silu(g) * u in f32 (expf order differs): scales within 2e-6, int8 within one step
    gu = (rng.standard_normal((M, 2 * K)) * 3).astype(np.float32)
    saq, sasc, _ = qm.swiglu_quant(to_dev(gu, dev), K, M_stride=Ms, act32=False)
    torch.cuda.synchronize()
    _, _, _, rh = oracle.swiglu_quant(gu, K, M_stride=Ms)
    raq, rasc, _ = oracle.quantize_act(rh[:M], M_stride=Ms, act32=False)
    d = np.abs(saq.cpu().numpy().astype(np.int32) - raq.astype(np.int32))
    assert d.max() <= 1 and np.mean(d > 0) <= 1e-3
    assert rel_err(sasc.cpu().numpy(), rasc) < 2e-6
    # add_norm_quant without w2: y is the updated x, which the kernel writes back
    t = rng.standard_normal((M, K)).astype(np.float32)
    xd = to_dev(x, dev)
    got = qm.add_norm_quant(xd, to_dev(t, dev), to_dev(w, dev), 1e-6, 0.5, M_stride=Ms, act32=False)
    torch.cuda.synchronize()
    xn = xd.cpu().numpy()
    assert rel_err(xn, oracle.add_norm_quant(x, t, w, 1e-6, 0.5, M_stride=Ms)[0]) < 2e-6
    _same_acts(got, oracle.quantize_act(xn, M_stride=Ms, act32=False))


@pytest.mark.parametrize("qtype", [F.Q4_K, F.Q8_0, F.IQ4_XS, F.Q6_K, F.IQ3_S, F.Q5_K, F.Q3_K, F.Q2_0, F.Q2_K, F.IQ1_S,
                                   F.IQ1_M])
@pytest.mark.parametrize("M,Ms,N,K", [(40, 48, 256, 2048), (256, 256, 384, 5120), (130, 130, 128, 1024)])
def test_gemm_per256_parity(qm, dev, qtype, M, Ms, N, K):
    """Q4_K at M >= 128 runs the f16 kernel, everything else the int8 kernels: both read scale b >> 3."""
    import torch
    W = F.synth_weight(qtype, N, K, seed=qtype + 2 * M + N)
    x = F.synth_activations(M, K, seed=M + K, outlier_frac=0.01)
    aq, asc, absum = qm.quantize_act(to_dev(x, dev), M_stride=Ms, act32=False)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    C = qm.gemm(w, aq, asc, absum, M=M, act32=False)
    torch.cuda.synchronize()
    naq, nasc, nabs = aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy()
    ref = oracle.blockdot256(qtype, W, K, naq, nasc, nabs, M=M)
    assert rel_err(C.cpu().numpy(), ref) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy(), ref)
    xq = naq[:M].astype(np.float32) * np.repeat(nasc[:, :M].T, 256, axis=1)
    assert rel_err(C.cpu().numpy(), oracle.matmul_f32(qtype, W, K, xq)) < TOL_F32_REF


def test_gemm_per256_accumulate_and_refusals(qm, dev):
    import torch
    M, N, K = 128, 256, 1024
    W = F.synth_weight(F.Q4_K, N, K, seed=9)
    x = F.synth_activations(M, K, seed=9)
    aq, asc, absum = qm.quantize_act(to_dev(x, dev), act32=False)
    w = qm.QWeight(F.Q4_K, to_dev(W, dev), N, K)
    base = qm.gemm(w, aq, asc, absum, act32=False)
    C = torch.randn(M, N, device=dev)
    C0 = C.clone()
    qm.gemm(w, aq, asc, absum, C=C, ldc=N, accumulate=1, act32=False)
    torch.cuda.synchronize()
    assert torch.equal(C, C0 + base)
    # K not a multiple of 256 cannot carry per-256 scales
    xs = torch.randn(4, 96, device=dev)
    with pytest.raises(qm.QMatmulError):
        qm.quantize_act(xs, act32=False)
