"""Rows that are not whole superblocks, and the prompt GEMM with a caller-owned workspace.

Q8_0, Q4_0 and IQ4_NL rows of K % 32 == 0 (Q2_0: K % 64 == 0) are padded at preparation with zero blocks to K rounded up to 256, as the
reference's load_w_pad / pad_small_block_rows (zero/engine.h:2102-2116; src/quants.h:581-595). The oracle computes on
the explicitly padded GGUF rows (F.pad_small_rows) and activations of the padded length whose tail is zero -- the
reference's own arithmetic on its padded weights. The MoE case is Flash Next's expert width 640 (down projection read
as 768, zero/engine_moe.h:12, 318-326); its oracle pads the gate / up experts with zero rows, which give h = 0 exactly.
"""
import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F
from tests.test_gpu_moe import moe_check
from tests.test_gpu_parity import TOL_INT8_PATH, acts, assert_elementwise, rel_err, to_dev

pytestmark = pytest.mark.gpu

SMALL = [F.Q8_0, F.Q4_0, F.IQ4_NL, F.Q2_0]


def padded_acts(M, K, seed):
    Kp = F.padded_k(K)
    x = np.zeros((M, Kp), dtype=np.float32)
    x[:, :K] = F.synth_activations(M, K, seed=seed)
    return x


@pytest.mark.parametrize("qtype", SMALL)
@pytest.mark.parametrize("N,K,M", [(64, 640, 1), (48, 640, 3), (32, 96, 8), (144, 640, 40), (128, 1312, 130)])
def test_padded_rows_gemv_and_gemm(qm, dev, qtype, N, K, M):
    import torch
    if K % F.small_block(qtype):
        pytest.skip("Q2_0 rows are whole 64-element blocks")
    Kp = F.padded_k(K)
    W = F.synth_weight(qtype, N, K, seed=qtype * 7 + K + M)
    assert W.shape[1] == F.row_bytes(qtype, K)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    assert w.K == Kp and w.K_raw == K
    x = padded_acts(M, K, seed=M + K)
    aq, asc, absum = acts(qm, x, dev, M_stride=max(M, 16))
    C = qm.gemv(w, aq, asc, absum, T=M) if M <= 8 else qm.gemm(w, aq, asc, absum, M=M)
    torch.cuda.synchronize()
    ref = oracle.blockdot(qtype, F.pad_small_rows(qtype, W, K), Kp, aq.cpu().numpy(), asc.cpu().numpy(),
                          absum.cpu().numpy(), M=M)
    got = C.cpu().numpy()[:M]
    assert rel_err(got, ref) < TOL_INT8_PATH
    assert_elementwise(got, ref)
    # the padded blocks are zero: the products equal the oracle on the unpadded row with the activations cut to K
    xq = aq.cpu().numpy()[:M, :K].astype(np.float32) * np.repeat(asc.cpu().numpy()[:K // 32, :M].T, 32, axis=1)
    assert rel_err(got, oracle.matmul_f32(qtype, F.pad_small_rows(qtype, W, K)[:, :], Kp,
                                          np.pad(xq, ((0, 0), (0, Kp - K))))) < 1e-3
    w.release()


@pytest.mark.parametrize("T,NU", [(2, 4), (40, 4)])  # decode-size experts, and the slot-tile path
@pytest.mark.parametrize("td", [F.Q8_0, F.IQ4_NL, F.Q2_0])
def test_moe_padded_expert_width(qm, dev, T, NU, td):
    """Experts of width Fv = 640: gate / up IQ4_XS with 640 rows per expert, down of 640-long rows padded to 768."""
    import torch
    NE, E, Fv = 8, 256, 640
    Fp = F.padded_k(Fv)
    tg = tu = F.IQ4_XS
    Wg = F.synth_weight(tg, NE * Fv, E, seed=5, sigma=0.05)
    Wu = F.synth_weight(tu, NE * Fv, E, seed=6, sigma=0.05)
    Wd = F.synth_weight(td, NE * E, Fv, seed=7, sigma=0.05)
    x = F.synth_activations(T, E, seed=8)
    lg = F.zipf_router_logits(T, NE, seed=9)
    aq, asc, _ = qm.quantize_act(to_dev(x, dev))
    g, u, d = qm.QWeight(tg, to_dev(Wg, dev), NE * Fv, E), qm.QWeight(tu, to_dev(Wu, dev), NE * Fv, E), \
        qm.QWeight(td, to_dev(Wd, dev), NE * E, Fv)
    assert d.K == Fp
    ws = qm.moe_workspace(T, NE, NU, E, Fp, device=dev)
    ws.fill_(0x7F)  # (stale workspace bytes: the padded h columns are never written, their products must still be 0)
    out = torch.zeros((T, E), dtype=torch.float32, device=dev)
    qm.moe_grouped(g, u, d, NE, to_dev(lg, dev), NU, aq, asc, out, ws)
    torch.cuda.synchronize()

    def pad_rows(W):  # each expert's 640 rows followed by 128 zero rows (all-zero IQ4_XS superblocks: d = 0)
        P = np.zeros((NE, Fp, W.shape[1]), dtype=np.uint8)
        P[:, :Fv] = W.reshape(NE, Fv, -1)
        return P.reshape(NE * Fp, -1)

    s = dict(Wg=pad_rows(Wg), Wu=pad_rows(Wu), Wd=F.pad_small_rows(td, Wd, Fv), lg=lg, aq=aq, asc=asc, ws=ws, out=out)
    if T * NU > 64:
        # the two-stage check reads the GPU's quantized h: its padded columns, never written, are set to the zeros
        # the oracle's zero rows give (the output above was computed with the stale bytes in place)
        L = qm.moe_ws_layout(T, NE, NU, E, Fp)
        hq = ws[L.hq:L.hq + L.slots * Fp].view(L.slots, Fp)
        hq[:, Fv:] = 0
        torch.cuda.synchronize()
    moe_check(qm, s, (tg, tu, td), NE, E, Fp, T, NU)
    for wt in (g, u, d):
        wt.release()


@pytest.mark.parametrize("qtype,M,act32", [(F.Q4_K, 256, 1), (F.Q4_K, 300, 0), (F.IQ4_XS, 64, 1), (F.Q4_K, 64, 1)])
def test_gemm_caller_workspace(qm, dev, qtype, M, act32):
    """qmatmul_gemm_ws equals qmatmul_gemm(_ex) bit for bit; a short or missing workspace is refused."""
    import torch
    N, K = 256, 1024
    W = F.synth_weight(qtype, N, K, seed=21)
    x = F.synth_activations(M, K, seed=22, outlier_frac=0.01)
    aq, asc, absum = qm.quantize_act(to_dev(x, dev), act32=bool(act32))
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    need = qm.gemm_workspace_size(w, M)
    assert (need > 0) == (qtype == F.Q4_K and M >= 128)
    ref = qm.gemm(w, aq, asc, absum, act32=bool(act32))
    ws = torch.empty((need,), dtype=torch.uint8, device=dev) if need else None
    got = qm.gemm_ws(w, aq, asc, absum, ws, act32=bool(act32))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    if need:
        short = torch.empty((need - 256,), dtype=torch.uint8, device=dev)
        with pytest.raises(qm.QMatmulError) as ei:
            qm.gemm_ws(w, aq, asc, absum, short, act32=bool(act32))
        assert ei.value.status == 6
        with pytest.raises(qm.QMatmulError):
            qm.gemm_ws(w, aq, asc, absum, None, act32=bool(act32))
    w.release()
