"""GPU parity of the HIP path (through the C ABI) against the CPU oracle on the same seeded inputs.

Bars: quantized activations and int32 block sums bit-exact, taken from the same kernel
instantiation (route, token chunking, row tiles) that computes the product; f32 outputs within 1e-4 of the oracle's
int8 path and within 1e-3 of the f32 dequantized reference as max |err| / max |ref| over the output, and element by
element |err| <= 1e-4 |ref| + 1e-5 max |ref| against the int8 path (the absolute term covers outputs that cancel to
near zero, whose relative error the f32 summation order alone can make large).
"""
import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F

pytestmark = pytest.mark.gpu

TOL_INT8_PATH = 1e-4
TOL_F32_REF = 1e-3
TYPES = [F.Q8_0, F.Q4_K, F.IQ4_XS, F.IQ3_S]
GEMV_TYPES = TYPES + [F.Q6_K, F.Q5_K, F.Q4_0, F.IQ4_NL, F.IQ2_XXS, F.IQ2_XS, F.IQ2_S, F.IQ3_XXS, F.Q3_K, F.Q2_0, F.Q2_K,
                      F.IQ1_S, F.IQ1_M]


def rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def assert_elementwise(got, ref, rel=1e-4, floor=1e-5):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = rel * np.abs(ref) + floor * max(np.max(np.abs(ref)), 1e-30)
    worst = float(np.max(np.abs(got - ref) / bound))
    assert worst <= 1.0, f"element-wise error {worst:.3f} x the bound"


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def acts(qm, x, dev, M_stride=None):
    import torch
    xt = to_dev(x.astype(np.float32), dev)
    aq, asc, absum = qm.quantize_act(xt, M_stride=M_stride)
    torch.cuda.synchronize()
    return aq, asc, absum


# ---- (a) activation quantizer
@pytest.mark.parametrize("M,Ms,K", [(1, 16, 4096), (7, 16, 512), (64, 64, 5120), (3, 3, 17408)])
def test_quantizer_bit_exact(qm, dev, M, Ms, K):
    rng = np.random.default_rng(M * 1000 + K)
    x = rng.standard_normal((M, K)).astype(np.float32) * rng.choice([1.0, 30.0, 1e-3], size=(M, K)).astype(np.float32)
    x[0, :32] = 0.0  # a zero block
    x[0, 32:64] = np.float32(0.5) * np.arange(32, dtype=np.float32)  # ties at amax 15.5? (q = 127 * v / 15.5)
    if K >= 128:
        x[0, 64:96] = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5] + [3.5] * 26, dtype=np.float32)  # exact ties
    aq, asc, absum = acts(qm, x, dev, Ms)
    raq, rasc, rabs = oracle.quantize_act(x, M_stride=Ms)
    assert np.array_equal(aq.cpu().numpy(), raq)
    assert np.array_equal(asc.cpu().numpy().view(np.uint32), rasc.view(np.uint32))
    assert np.array_equal(absum.cpu().numpy(), rabs)


def test_quantizer_strided_input(qm, dev):
    import torch
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 1024)).astype(np.float32)
    xt = to_dev(x, dev)[:, :512]  # ldx 1024, K 512
    aq, asc, absum = qm.quantize_act(xt, M_stride=8)
    torch.cuda.synchronize()
    raq, rasc, rabs = oracle.quantize_act(np.ascontiguousarray(x[:, :512]), M_stride=8)
    assert np.array_equal(aq.cpu().numpy(), raq) and np.array_equal(absum.cpu().numpy(), rabs)
    assert np.array_equal(asc.cpu().numpy(), rasc)


# ---- (b) decode GEMV
@pytest.mark.parametrize("qtype", GEMV_TYPES)
@pytest.mark.parametrize("N,K,T", [(64, 1024, 1), (48, 768, 3), (40, 8192, 1), (16, 256, 8),
                                   (24, 17408, 1), (20, 17408, 2),   # 128 lanes per row (two waves combined)
                                   (32, 6144, 8), (40, 4096, 6),     # tokens chunked per launch
                                   (16, 34816, 1), (12, 33024, 3),   # K > 32768: the generic kernel
                                   (6160, 5120, 1)])  # 32 lanes per row, 5 blocks per lane (batch-1 per-type routes)
def test_gemv_blocksums_bit_exact(qm, dev, qtype, N, K, T):
    rng = np.random.default_rng(qtype + N + K)
    W = F.synth_weight(qtype, N, K, seed=qtype * 7 + K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    aq, asc, absum = acts(qm, x, dev, M_stride=max(T, 16))
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    isum, msum = qm.gemv_blocksums(w, aq, absum, T=T)
    _, risum, rmsum = oracle.blockdot(qtype, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=T,
                                      blocksums=True)
    assert np.array_equal(isum.cpu().numpy(), risum)
    if msum is not None:  # (Q4_K, Q5_K, Q2_K)
        assert np.array_equal(msum.cpu().numpy(), rmsum)


@pytest.mark.parametrize("qtype", GEMV_TYPES)
@pytest.mark.parametrize("N,K,T", [(64, 1024, 1), (200, 2048, 1), (72, 17408, 1), (96, 5120, 2), (64, 1536, 5),
                                   (64, 34816, 1), (24, 33024, 3),  # (K > 32768: the generic kernel)
                                   # tokens per launch capped at 4 (6 blocks per lane; Q6_K beyond 4, the IQ2 grids
                                   # beyond 3): 8 tokens as two launches, 6 as 4 + 2
                                   (48, 6144, 8), (32, 5120, 8), (40, 4096, 6),
                                   (6160, 5120, 1)])  # (more than 6144 rows: the 32-lane batch-1 route)
def test_gemv_f32_parity(qm, dev, qtype, N, K, T):
    import torch
    rng = np.random.default_rng(qtype * 3 + N)
    W = F.synth_weight(qtype, N, K, seed=qtype + 11 * N)
    x = F.synth_activations(T, K, seed=N + K, outlier_frac=0.01)
    aq, asc, absum = acts(qm, x, dev, M_stride=16)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    C = qm.gemv(w, aq, asc, absum, T=T)
    torch.cuda.synchronize()
    naq, nasc, nabs = aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy()
    ref = oracle.blockdot(qtype, W, K, naq, nasc, nabs, M=T)
    assert rel_err(C.cpu().numpy(), ref) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy(), ref)
    xq = naq[:T].astype(np.float32) * np.repeat(nasc[:, :T].T, 32, axis=1)
    ref32 = oracle.matmul_f32(qtype, W, K, xq)
    assert rel_err(C.cpu().numpy(), ref32) < TOL_F32_REF


@pytest.mark.parametrize("qtype", [F.Q8_0, F.IQ4_XS])
def test_gemv_accumulate_offset_and_tokens(qm, dev, qtype):
    import torch
    N, K = 128, 2048
    W = F.synth_weight(qtype, N, K, seed=9)
    x = F.synth_activations(4, K, seed=10)
    aq, asc, absum = acts(qm, x, dev, M_stride=16)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    one = [qm.gemv(w, aq[t:t + 1].contiguous(), asc[:, t:t + 1].contiguous(), absum[:, t:t + 1].contiguous(), T=1)
           for t in range(4)]
    multi = qm.gemv(w, aq, asc, absum, T=4)
    torch.cuda.synchronize()
    for t in range(4):  # (4 tokens per launch against 1: the f32 sums may run in another order)
        assert rel_err(multi[t].cpu().numpy(), one[t][0].cpu().numpy()) < 1e-5
    C = torch.full((4, 3 * N), 2.0, device=dev)
    qm.gemv(w, aq, asc, absum, T=4, C=C, ldc=3 * N, c_off=N, accumulate=1)
    torch.cuda.synchronize()
    assert torch.equal(C[:, N:2 * N], multi + 2.0)
    assert torch.all(C[:, :N] == 2.0) and torch.all(C[:, 2 * N:] == 2.0)


def test_gemv_baseline_q8_0_4096(qm, dev):
    """Q8_0 4096 x 4096, seed 0."""
    import torch
    N = K = 4096
    W = F.synth_weight(F.Q8_0, N, K, seed=0)
    x = F.synth_activations(1, K, seed=0)
    aq, asc, absum = acts(qm, x, dev, M_stride=16)
    w = qm.QWeight(F.Q8_0, to_dev(W, dev), N, K)
    C = qm.gemv(w, aq, asc, absum)
    torch.cuda.synchronize()
    ref = oracle.blockdot(F.Q8_0, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=1)
    assert rel_err(C.cpu().numpy(), ref) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy(), ref)


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408)])
def test_gemv_baseline_iq4_xs(qm, dev, N, K):
    """BASELINE config 1 (north star shapes), full size."""
    import torch
    W = F.synth_weight(F.IQ4_XS, N, K, seed=1)
    x = F.synth_activations(1, K, seed=1)
    aq, asc, absum = acts(qm, x, dev, M_stride=16)
    w = qm.QWeight(F.IQ4_XS, to_dev(W, dev), N, K)
    C = qm.gemv(w, aq, asc, absum)
    torch.cuda.synchronize()
    ref = oracle.blockdot(F.IQ4_XS, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=1)
    assert rel_err(C.cpu().numpy(), ref) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy(), ref)


@pytest.mark.parametrize("qtype", [F.IQ4_XS, F.Q4_K, F.Q8_0, F.IQ3_S])
@pytest.mark.parametrize("N", [2049, 3000, 5136])
def test_gemv_long_rows_first_round_split(qm, dev, qtype, N):
    """Batch-1 rows of 544 blocks (K = 17408) take the route whose first-dispatch-round work-groups also take the rows
    past the lockstep sweep; row counts that leave a ragged remainder (and 2049: the split just engaged) against the
    oracle, block sums bit-exact."""
    import torch
    K = 17408
    W = F.synth_weight(qtype, N, K, seed=N + qtype)
    x = F.synth_activations(1, K, seed=N)
    aq, asc, absum = acts(qm, x, dev, M_stride=16)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    C = qm.gemv(w, aq, asc, absum)
    isum, msum = qm.gemv_blocksums(w, aq, absum, T=1)
    torch.cuda.synchronize()
    ref, risum, rmsum = oracle.blockdot(qtype, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=1,
                                        blocksums=True)
    assert rel_err(C.cpu().numpy(), ref) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy(), ref)
    assert np.array_equal(isum.cpu().numpy(), risum)
    if msum is not None:
        assert np.array_equal(msum.cpu().numpy(), rmsum)
    w.release()


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408)])
def test_gemv_baseline_iq4_xs_blocksums(qm, dev, N, K):
    """North-star shapes at full size: the int32 block sums of the shipped batch-1 GEMV, bit-exact."""
    W = F.synth_weight(F.IQ4_XS, N, K, seed=1)
    x = F.synth_activations(1, K, seed=1)
    aq, asc, absum = acts(qm, x, dev, M_stride=16)
    w = qm.QWeight(F.IQ4_XS, to_dev(W, dev), N, K)
    isum, _ = qm.gemv_blocksums(w, aq, absum, T=1)
    _, risum, _ = oracle.blockdot(F.IQ4_XS, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=1,
                                  blocksums=True)
    assert np.array_equal(isum.cpu().numpy(), risum)


# ---- (c) prompt GEMM (int8 MFMA; Q4_K with M >= 128 on the f16 matrix pipe)
@pytest.mark.parametrize("qtype", GEMV_TYPES)
@pytest.mark.parametrize("M,N,K", [(32, 128, 512), (37, 144, 768),  # one / two 32-row tiles per work-group
                                   (130, 144, 1024)])  # (Q4_K: the f16 kernel)
def test_gemm_blocksums_bit_exact(qm, dev, qtype, M, N, K):
    rng = np.random.default_rng(M + N + qtype)
    W = F.synth_weight(qtype, N, K, seed=qtype * 5 + M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    aq, asc, absum = acts(qm, x, dev, M_stride=M)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    isum = qm.gemm_blocksums(w, aq)
    _, risum, _ = oracle.blockdot(qtype, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(),
                                  blocksums=True)
    assert np.array_equal(isum.cpu().numpy(), risum)


@pytest.mark.parametrize("qtype", GEMV_TYPES)
@pytest.mark.parametrize("M,Ms,N,K", [(64, 64, 256, 1024), (100, 128, 384, 2048), (16, 16, 128, 256),
                                      (130, 130, 512, 5120), (96, 96, 128, 17408)])
def test_gemm_f32_parity(qm, dev, qtype, M, Ms, N, K):
    import torch
    W = F.synth_weight(qtype, N, K, seed=qtype + M + N)
    x = F.synth_activations(M, K, seed=M * 3 + K, outlier_frac=0.01)
    aq, asc, absum = acts(qm, x, dev, M_stride=Ms)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    C = qm.gemm(w, aq, asc, absum, M=M)
    torch.cuda.synchronize()
    naq, nasc, nabs = aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy()
    ref = oracle.blockdot(qtype, W, K, naq, nasc, nabs, M=M)
    assert rel_err(C.cpu().numpy(), ref) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy(), ref)
    xq = naq[:M].astype(np.float32) * np.repeat(nasc[:, :M].T, 32, axis=1)
    assert rel_err(C.cpu().numpy(), oracle.matmul_f32(qtype, W, K, xq)) < TOL_F32_REF


@pytest.mark.parametrize("qtype", [F.IQ4_XS, F.Q4_K])
def test_gemm_accumulate_modes(qm, dev, qtype):
    import torch
    M, N, K = 64, 256, 1024
    W = F.synth_weight(qtype, N, K, seed=3)
    x = F.synth_activations(M, K, seed=4)
    aq, asc, absum = acts(qm, x, dev)
    w = qm.QWeight(qtype, to_dev(W, dev), N, K)
    base = qm.gemm(w, aq, asc, absum)
    C = torch.randn(M, 2 * N + 16, device=dev)
    C0 = C.clone()
    qm.gemm(w, aq, asc, absum, C=C, ldc=2 * N + 16, c_off=N, accumulate=1)
    torch.cuda.synchronize()
    assert torch.equal(C[:, N:2 * N], C0[:, N:2 * N] + base)
    assert torch.equal(C[:, :N], C0[:, :N]) and torch.equal(C[:, 2 * N:], C0[:, 2 * N:])
    G = torch.randn(M, N, device=dev)
    S = G.clone()
    qm.gemm(w, aq, asc, absum, C=S, ldc=N, accumulate=2)
    torch.cuda.synchronize()
    ref = (G.double() / (1 + torch.exp(-G.double()))) * base.double()
    assert torch.max(torch.abs(S.double() - ref)) / torch.max(torch.abs(ref)) < 1e-6


def test_gemm_baseline_q4_k_2k_sampled(qm, dev):
    """BASELINE config 2 at full size: M 2048, K 5120, N 17408. Every 67th output column against the oracle (67 is
    coprime with the 128-row weight tile, so the 260 sampled columns cover every row position of the tile: every
    wave, lane half and result register of the f16 epilogue), plus the whole last 128-row tile (rows 17280-17407)."""
    import torch
    M, N, K = 2048, 17408, 5120
    W = F.synth_weight(F.Q4_K, N, K, seed=2)
    x = F.synth_activations(M, K, seed=2, outlier_frac=0.01, outlier_scale=20.0)
    aq, asc, absum = acts(qm, x, dev)
    w = qm.QWeight(F.Q4_K, to_dev(W, dev), N, K)
    C = qm.gemm(w, aq, asc, absum)
    torch.cuda.synchronize()
    Cn = C.cpu().numpy()
    naq, nasc, nabs = aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy()
    ref = oracle.blockdot(F.Q4_K, W, K, naq, nasc, nabs, col_stride=67)
    assert len(set(np.arange(0, N, 67) % 128)) == 128
    assert rel_err(Cn[:, ::67], ref[:, ::67]) < TOL_INT8_PATH
    assert_elementwise(Cn[:, ::67], ref[:, ::67])
    last = oracle.blockdot(F.Q4_K, W[N - 128:], K, naq, nasc, nabs)
    assert rel_err(Cn[:, N - 128:], last) < TOL_INT8_PATH
    assert_elementwise(Cn[:, N - 128:], last)
    assert np.all(np.isfinite(Cn))


def test_gemm_baseline_q4_k_2k_blocksums(qm, dev):
    """BASELINE config 2's kernel at M = 2048, K = 5120: the exact block sums sc * isum of the shipped f16 GEMM for
    the weight's first 256 rows (the full 17408 rows would be 22.8 GB of sums; every row tile runs the same code)."""
    M, N, K = 2048, 256, 5120
    W = F.synth_weight(F.Q4_K, 17408, K, seed=2)[:N].copy()
    x = F.synth_activations(M, K, seed=2, outlier_frac=0.01, outlier_scale=20.0)
    aq, asc, absum = acts(qm, x, dev)
    w = qm.QWeight(F.Q4_K, to_dev(W, dev), N, K)
    isum = qm.gemm_blocksums(w, aq)
    _, risum, _ = oracle.blockdot(F.Q4_K, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(),
                                  blocksums=True)
    assert np.array_equal(isum.cpu().numpy(), risum)


@pytest.mark.parametrize("M", [1, 512])
def test_iq3_s_baseline_5120(qm, dev, M):
    """IQ3_S 5120 x 5120 at M = 1 (GEMV) and M = 512 (GEMM, every 16th column checked)."""
    import torch
    N = K = 5120
    W = F.synth_weight(F.IQ3_S, N, K, seed=3)
    x = F.synth_activations(M, K, seed=3)
    aq, asc, absum = acts(qm, x, dev, M_stride=max(M, 16))
    w = qm.QWeight(F.IQ3_S, to_dev(W, dev), N, K)
    C = qm.gemv(w, aq, asc, absum) if M == 1 else qm.gemm(w, aq, asc, absum, M=M)
    torch.cuda.synchronize()
    stride = 1 if M == 1 else 16
    ref = oracle.blockdot(F.IQ3_S, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=M,
                          col_stride=stride)
    assert rel_err(C.cpu().numpy()[:, ::stride], ref[:, ::stride]) < TOL_INT8_PATH
    assert_elementwise(C.cpu().numpy()[:M, ::stride], ref[:, ::stride])


@pytest.mark.parametrize("M,N,K,c_off,extra", [(300, 144, 1024, 3, 5), (64, 128, 256, 0, 0), (257, 272, 2048, 1, 2)])
def test_gemm_q4_k_edges(qm, dev, M, N, K, c_off, extra):
    """Q4_K prompt GEMM at ragged shapes (token and row tiles partly filled, unaligned output columns) with
    superblocks whose d or dmin is zero (the carried-scale path treats d = 0 specially)."""
    import torch
    W = F.synth_weight(F.Q4_K, N, K, seed=M + N).copy()
    nsb = K // 256
    sbv = W.reshape(N, nsb, 144)
    sbv[::3, 0, 0:2] = 0      # d = 0 in the first superblock of every third row
    sbv[1::5, -1, 2:4] = 0    # dmin = 0 in the last superblock of every fifth row
    sbv[2, :, 0:4] = 0        # row 2: d = dmin = 0 everywhere
    x = F.synth_activations(M, K, seed=M, outlier_frac=0.01, outlier_scale=20.0)
    aq, asc, absum = acts(qm, x, dev)
    w = qm.QWeight(F.Q4_K, to_dev(W, dev), N, K)
    ldc = c_off + N + extra
    C = torch.full((M, ldc), 7.0, device=dev)
    qm.gemm(w, aq, asc, absum, C=C, ldc=ldc, c_off=c_off)
    torch.cuda.synchronize()
    Cn = C.cpu().numpy()
    ref = oracle.blockdot(F.Q4_K, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=M)
    assert rel_err(Cn[:, c_off:c_off + N], ref) < TOL_INT8_PATH
    assert np.all(Cn[:, :c_off] == 7.0) and np.all(Cn[:, c_off + N:] == 7.0)
    assert np.all(Cn[:, c_off + 2] == 0.0)  # row 2 of the weight is all zero


def test_gemm_k_split_is_deterministic_and_stays_in_its_columns(qm, dev):
    """A dense product with few tiles splits K in two (the halves are added into C after it is zeroed): the result is
    the same bits on every call, the columns outside [c_off, c_off + N) are untouched, and it meets the f32 bars."""
    import torch
    M, N, K = 100, 384, 2048
    W = F.synth_weight(F.IQ3_S, N, K, seed=17)
    x = F.synth_activations(M, K, seed=18)
    aq, asc, absum = acts(qm, x, dev)
    w = qm.QWeight(F.IQ3_S, to_dev(W, dev), N, K)
    ldc = N + 40
    C = torch.full((M, ldc), float("nan"), device=dev)
    qm.gemm(w, aq, asc, absum, C=C, ldc=ldc, c_off=24)
    first = C.clone()
    for _ in range(3):
        C.fill_(float("nan"))
        qm.gemm(w, aq, asc, absum, C=C, ldc=ldc, c_off=24)
        torch.cuda.synchronize()
        assert torch.equal(C[:, 24:24 + N], first[:, 24:24 + N])
    assert torch.all(torch.isnan(C[:, :24])) and torch.all(torch.isnan(C[:, 24 + N:]))
    ref = oracle.blockdot(F.IQ3_S, W, K, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy())
    got = first[:, 24:24 + N].cpu().numpy()
    assert rel_err(got, ref) < TOL_INT8_PATH
    assert_elementwise(got, ref)
