"""Known-answer vectors (tests/golden/known_answers.npz, written by tests/golden/make_golden.py from block fields,
independently of the oracle and the product): the oracle on the CPU, and the HIP path through the C ABI on the GPU.
Edge cases: d = 0, d = +-65504, subnormal d, all-15 nibbles, IQ3_S grid bit 8 and all sign bits, the IQ2 / IQ3_XXS
last grid index with every stored sign set, quantizer ties,
zero blocks, +-amax and subnormal inputs."""
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "known_answers.npz")
TYPES = [(8, "q8_0"), (12, "q4_k"), (23, "iq4_xs"), (21, "iq3_s"), (14, "q6_k"), (13, "q5_k"), (2, "q4_0"),
         (20, "iq4_nl"), (16, "iq2_xxs"), (17, "iq2_xs"), (22, "iq2_s"), (18, "iq3_xxs")]
K = 512


@pytest.fixture(scope="module")
def g():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_quantizer_known_answers(g):
    aq, asc, absum = oracle.quantize_act(g["quant_x"])
    assert np.array_equal(aq, g["quant_aq"])
    assert np.array_equal(asc.view(np.uint32), g["quant_asc"].view(np.uint32))
    assert np.array_equal(absum, g["quant_absum"])


@pytest.mark.parametrize("qtype,name", TYPES)
def test_oracle_dequant_known_answers(g, qtype, name):
    dq = oracle.dequant_rows(qtype, g[f"{name}_raw"], K)
    assert np.array_equal(dq.view(np.uint32), g[f"{name}_dq"].view(np.uint32))


@pytest.mark.parametrize("qtype,name", TYPES)
def test_oracle_blockdot_known_answers(g, qtype, name):
    aq, asc, absum = oracle.quantize_act(g[f"{name}_x"])
    C, isum, msum = oracle.blockdot(qtype, g[f"{name}_raw"], K, aq, asc, absum, blocksums=True)
    assert np.array_equal(isum[0].astype(np.int64), g[f"{name}_isum"])
    if qtype in (12, 13):
        assert np.array_equal(msum[0].astype(np.int64), g[f"{name}_msum"])
    y = g[f"{name}_y"]
    assert np.max(np.abs(C[0] - y)) <= 1e-6 * np.max(np.abs(y))


@pytest.mark.gpu
def test_gpu_quantizer_known_answers(g, qm, dev):
    import torch
    aq, asc, absum = qm.quantize_act(torch.from_numpy(g["quant_x"]).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(aq.cpu().numpy(), g["quant_aq"])
    assert np.array_equal(asc.cpu().numpy().view(np.uint32), g["quant_asc"].view(np.uint32))
    assert np.array_equal(absum.cpu().numpy(), g["quant_absum"])


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,name", TYPES)
def test_gpu_gemv_known_answers(g, qm, dev, qtype, name):
    import torch
    raw = g[f"{name}_raw"]
    w = qm.QWeight(qtype, torch.from_numpy(raw).to(dev), raw.shape[0], K)
    aq, asc, absum = qm.quantize_act(torch.from_numpy(g[f"{name}_x"]).to(dev), M_stride=16)
    isum, msum = qm.gemv_blocksums(w, aq, absum)
    y = qm.gemv(w, aq, asc, absum)
    # the prompt GEMM on the same row (M = 16 padded rows; row 0 is the token)
    ygemm = qm.gemm(w, aq, asc, absum, M=16)
    torch.cuda.synchronize()
    assert np.array_equal(isum.cpu().numpy()[0].astype(np.int64), g[f"{name}_isum"])
    if qtype in (12, 13):
        assert np.array_equal(msum.cpu().numpy()[0].astype(np.int64), g[f"{name}_msum"])
    ref = g[f"{name}_y"]
    scale = np.max(np.abs(ref))
    assert np.max(np.abs(y.cpu().numpy()[0] - ref)) <= 1e-4 * scale
    assert np.max(np.abs(ygemm.cpu().numpy()[0] - ref)) <= 1e-4 * scale
    w.release()
