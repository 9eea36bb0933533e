"""Pins the oracle's arithmetic: the activation quantizer, the int8 block-dot products, the f32 reference, routing
and the MoE pipeline, each against something computed another way (brute-force integer sums, float64 products of
dequantized values, textbook stable-sort routing)."""
import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F


# ---- activation quantizer (src/quants.h:559-576)
def test_quantize_ties_round_half_even_and_special_blocks():
    K = 32 * 6
    x = np.zeros((1, K), dtype=np.float32)
    # block 0: amax 127 -> inv 1.0: values k + 0.5 must round to even
    x[0, 0:32] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 127.0] + [3.5] * 24, dtype=np.float32)
    # block 1: all zeros -> scale 0, q 0
    # block 2: +-amax -> +-127
    x[0, 64:96] = np.linspace(-7.0, 7.0, 32, dtype=np.float32)
    # block 3: negative zero and subnormals with a normal amax
    x[0, 96:128] = np.float32(1e-40)
    x[0, 96] = np.float32(-0.0)
    x[0, 97] = np.float32(3.0)
    # block 4: a single non-zero value
    x[0, 130] = np.float32(-2.75)
    aq, asc, absum = oracle.quantize_act(x)
    assert list(aq[0, :8]) == [0, 2, 2, 0, -2, -2, 126, 127]
    assert np.all(aq[0, 32:64] == 0) and asc[1, 0] == 0.0
    assert aq[0, 64] == -127 and aq[0, 95] == 127
    assert aq[0, 97] == 127 and np.all(aq[0, 98:128] == 0)
    assert aq[0, 130] == -127 and np.sum(np.abs(aq[0, 128:160])) == 127
    assert asc[0, 0] == np.float32(127.0) / np.float32(127.0)


def test_quantize_uses_multiply_by_127_over_amax():
    """q = rint(v * (127/amax)), not rint(v / (amax/127)): find values where the two differ and check the former."""
    rng = np.random.default_rng(7)
    found = 0
    for _ in range(2000):
        v = rng.standard_normal(32).astype(np.float32)
        amax = np.max(np.abs(v))
        a = np.rint(v * (np.float32(127.0) / amax)).astype(np.int64)
        b = np.rint(v / (amax / np.float32(127.0))).astype(np.int64)
        if np.any(a != b):
            aq, _, _ = oracle.quantize_act(v[None])
            assert np.array_equal(aq[0].astype(np.int64), a)
            found += 1
            if found > 5:
                break
    assert found > 0


def test_quantize_layout_padding_and_absum():
    rng = np.random.default_rng(8)
    M, Ms, K = 5, 8, 256
    x = rng.standard_normal((M, K)).astype(np.float32) * 3
    aq, asc, absum = oracle.quantize_act(x, M_stride=Ms)
    assert aq.shape == (Ms, K) and asc.shape == (K // 32, Ms) and absum.shape == (K // 16, Ms)
    assert np.all(aq[M:] == 0) and np.all(asc[:, M:] == 0) and np.all(absum[:, M:] == 0)
    for m in range(M):
        for b in range(K // 32):
            blk = x[m, 32 * b:32 * b + 32]
            assert asc[b, m] == np.float32(np.max(np.abs(blk))) / np.float32(127.0)
        for b in range(K // 16):
            assert absum[b, m] == int(aq[m, 16 * b:16 * b + 16].astype(np.int64).sum())
    # dequantized values are within half a step of the inputs
    deq = aq[:M].astype(np.float32) * np.repeat(asc[:, :M].T, 32, axis=1)
    assert np.all(np.abs(deq - x) <= 0.5 * np.repeat(asc[:, :M].T, 32, axis=1) * 1.0001)


# ---- int8 block-dot products
@pytest.mark.parametrize("qtype", [F.Q4_0, F.Q8_0, F.Q4_K, F.Q5_K, F.Q6_K, F.IQ4_NL, F.IQ4_XS, F.IQ3_S, F.IQ2_XXS,
                                   F.IQ2_XS, F.IQ2_S, F.IQ3_XXS])
def test_blockdot_int_sums_brute_force(qtype):
    rng = np.random.default_rng(10 + qtype)
    N, K, M = 12, 512, 3
    W = F.synth_weight(qtype, N, K, seed=qtype)
    x = rng.standard_normal((M, K)).astype(np.float32)
    aq, asc, absum = oracle.quantize_act(x)
    C, isum, msum = oracle.blockdot(qtype, W, K, aq, asc, absum, blocksums=True)
    nb = K // 32
    for n in range(N):
        sbs = [oracle.decode_sb(qtype, W[n, s * F.SB_BYTES[qtype]:(s + 1) * F.SB_BYTES[qtype]]) for s in range(K // 256)]
        q = np.concatenate([s["q"] for s in sbs])
        sc16 = np.concatenate([s["sc16"] for s in sbs])
        mn = np.concatenate([s["mn"] for s in sbs])
        for m in range(M):
            # per 16-element half: sc0 * lo + sc1 * hi (decode.cl:695-706)
            prod16 = (q * aq[m].astype(np.int64)).reshape(2 * nb, 16).sum(axis=1)
            assert np.array_equal(isum[m, n], (sc16 * prod16).reshape(nb, 2).sum(axis=1))
            if qtype in (F.Q4_K, F.Q5_K):
                bs = aq[m].astype(np.int64).reshape(nb, 32).sum(axis=1)
                assert np.array_equal(msum[m, n], mn * bs)


@pytest.mark.parametrize("qtype", [F.Q4_0, F.Q8_0, F.Q4_K, F.Q5_K, F.Q6_K, F.IQ4_NL, F.IQ4_XS, F.IQ3_S, F.IQ2_XXS,
                                   F.IQ2_XS, F.IQ2_S, F.IQ3_XXS])
def test_blockdot_f32_vs_dequantized_double(qtype):
    rng = np.random.default_rng(20 + qtype)
    N, K, M = 40, 1024, 4
    W = F.synth_weight(qtype, N, K, seed=100 + qtype)
    x = rng.standard_normal((M, K)).astype(np.float32)
    aq, asc, absum = oracle.quantize_act(x)
    C = oracle.blockdot(qtype, W, K, aq, asc, absum)
    w = oracle.dequant_rows(qtype, W, K).astype(np.float64)
    xq = aq.astype(np.float64) * np.repeat(asc.T.astype(np.float64), 32, axis=1)
    ref = xq @ w.T
    err = np.max(np.abs(C - ref)) / np.max(np.abs(ref))
    assert err < 1e-5, err
    # the f32 reference (ref_forward matmul) on the dequantized activations agrees as well
    Y = oracle.matmul_f32(qtype, W, K, xq.astype(np.float32))
    assert np.max(np.abs(Y - ref)) / np.max(np.abs(ref)) < 1e-6


def test_quantize_per256_scales():
    """act32 = false (quantize_act_cpu with B = 256): one amax per 256 values. Where every 32-block of a superblock
    has the superblock's amax, the result is the per-32 one with each scale repeated; the element at amax maps to
    +-127; rows past M are zero; absum stays per 16."""
    rng = np.random.default_rng(5)
    M, Ms, K = 3, 4, 1024
    x = rng.standard_normal((M, K)).astype(np.float32)
    for m in range(M):
        for s_ in range(K // 256):
            a = np.float32(rng.uniform(0.5, 40))
            x[m, 256 * s_: 256 * s_ + 256] = np.clip(x[m, 256 * s_: 256 * s_ + 256], -a, a)
            x[m, 256 * s_: 256 * s_ + 256: 32] = a  # every 32-block holds the superblock's amax
    q256, s256, a256 = oracle.quantize_act(x, M_stride=Ms, act32=False)
    q32, s32, a32 = oracle.quantize_act(x, M_stride=Ms)
    assert s256.shape == (K // 256, Ms) and a256.shape == (K // 16, Ms)
    assert np.array_equal(q256, q32) and np.array_equal(a256, a32)
    assert np.array_equal(np.repeat(s256, 8, axis=0), s32)
    # general rows: the scale is max |x| over the 256 values / 127, and that element maps to +-127
    y = rng.standard_normal((2, 512)).astype(np.float32) * np.float32(3)
    y[1, 256:512] = 0
    q, sc, ab = oracle.quantize_act(y, act32=False)
    for m in range(2):
        for s_ in range(2):
            seg = y[m, 256 * s_: 256 * s_ + 256]
            amax = np.max(np.abs(seg))
            assert sc[s_, m] == np.float32(amax) / np.float32(127)
            if amax > 0:
                i = int(np.argmax(np.abs(seg)))
                assert abs(int(q[m, 256 * s_ + i])) == 127
                inv = np.float32(127) / np.float32(amax)
                assert np.array_equal(q[m, 256 * s_: 256 * s_ + 256], np.rint(seg * inv).astype(np.int8))
            else:
                assert np.all(q[m, 256 * s_: 256 * s_ + 256] == 0)
    assert np.array_equal(ab, q.reshape(2, -1, 16).astype(np.int32).sum(axis=2).T.astype(np.int16))


@pytest.mark.parametrize("qtype", [F.Q8_0, F.Q4_K, F.Q6_K, F.IQ4_XS, F.IQ3_S])
def test_blockdot_per256_vs_dequantized_double(qtype):
    """blockdot256 (the act32 = false product) against float64 products of the dequantized weights and the
    activations dequantized with their superblock scale."""
    rng = np.random.default_rng(30 + qtype)
    N, K, M = 40, 1024, 4
    W = F.synth_weight(qtype, N, K, seed=200 + qtype)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    aq, asc, absum = oracle.quantize_act(x, act32=False)
    C = oracle.blockdot256(qtype, W, K, aq, asc, absum)
    w = oracle.dequant_rows(qtype, W, K).astype(np.float64)
    xq = aq.astype(np.float64) * np.repeat(asc.T.astype(np.float64), 256, axis=1)
    ref = xq @ w.T
    assert np.max(np.abs(C - ref)) / np.max(np.abs(ref)) < 1e-5


def test_blockdot_column_sampling():
    W = F.synth_weight(F.IQ4_XS, 64, 512, seed=1)
    aq, asc, absum = oracle.quantize_act(np.random.default_rng(0).standard_normal((2, 512)).astype(np.float32))
    full = oracle.blockdot(F.IQ4_XS, W, 512, aq, asc, absum)
    samp = oracle.blockdot(F.IQ4_XS, W, 512, aq, asc, absum, col_stride=16)
    assert np.array_equal(samp[:, ::16], full[:, ::16])


# ---- routing (tests/test_route.cpp recipe: stable sort, softmax over the selection)
def _route_textbook(lg, NU):
    T, NE = lg.shape
    ids = np.zeros((T, NU), np.int64)
    w = np.zeros((T, NU))
    for t in range(T):
        order = sorted(range(NE), key=lambda e: -float(lg[t, e]))  # Python's sort is stable: ties keep lower ids
        sel = order[:NU]
        p = np.exp(lg[t, sel].astype(np.float64) - float(lg[t, order[0]]))
        ids[t], w[t] = sel, p / p.sum()
    return ids, w


def test_route_matches_textbook():
    rng = np.random.default_rng(11)
    for NE, NU, T in [(256, 6, 7), (256, 8, 33), (64, 4, 5)]:
        lg = (rng.standard_normal((T, NE)) * 2).astype(np.float32)
        ids, w, counts = oracle.moe_route(lg, NU)
        rid, rw = _route_textbook(lg, NU)
        assert np.array_equal(ids, rid)
        assert np.max(np.abs(w - rw)) < 1e-6
        assert np.array_equal(counts, np.bincount(rid.ravel(), minlength=NE))


def test_route_ties_go_to_the_lower_expert():
    lg = np.zeros((2, 16), dtype=np.float32)
    lg[1, [3, 9, 12]] = 1.0
    ids, w, _ = oracle.moe_route(lg, 4)
    assert list(ids[0]) == [0, 1, 2, 3] and np.allclose(w[0], 0.25)
    assert list(ids[1]) == [3, 9, 12, 0]


def test_route_expert_scales():
    """moe.cl:75-77 (-DESCALE): the normalized weight times the chosen expert's scale; the selection is unchanged."""
    rng = np.random.default_rng(13)
    lg = rng.standard_normal((9, 32)).astype(np.float32)
    esc = rng.uniform(0.25, 4.0, 32).astype(np.float32)
    ids, w, _ = oracle.moe_route(lg, 4)
    ids2, w2, _ = oracle.moe_route(lg, 4, escale=esc)
    assert np.array_equal(ids, ids2)
    assert np.array_equal(w2, (w * esc[ids]).astype(np.float32))


@pytest.mark.parametrize("tg,tu,td,escale,shared", [
    (F.IQ4_XS, F.IQ4_XS, F.IQ4_XS, False, None),
    (F.IQ3_S, F.IQ4_XS, F.Q6_K, True, "gated"),     # gate, up and down of three types (a GGUF mix)
    (F.IQ2_XS, F.IQ2_S, F.Q8_0, False, "plain"),    # per-16 integer scales; shared expert without a gate
])
def test_moe_forward_vs_numpy_pipeline(tg, tu, td, escale, shared):
    rng = np.random.default_rng(12)
    NE, E, Fd, NU, T = 8, 256, 256, 2, 6
    Wg = F.synth_weight(tg, NE * Fd, E, seed=1, sigma=0.05)
    Wu = F.synth_weight(tu, NE * Fd, E, seed=2, sigma=0.05)
    Wd = F.synth_weight(td, NE * E, Fd, seed=3, sigma=0.05)
    x = rng.standard_normal((T, E)).astype(np.float32)
    aq, asc, _ = oracle.quantize_act(x)
    lg = rng.standard_normal((T, NE + 1)).astype(np.float32)  # (column NE: the shared expert's gate logit)
    esc = rng.uniform(0.5, 2.0, NE).astype(np.float32) if escale else None
    sh = rng.standard_normal((T, E)).astype(np.float32) if shared else None
    out = oracle.moe_forward(tg, Wg, tu, Wu, td, Wd, NE, E, Fd, lg, NU, aq, asc, escale=esc, sh=sh,
                             sh_gated=shared == "gated")
    # numpy pipeline from the pinned pieces: textbook routing, dequantized products in float64, h quantized by the
    # (pinned) quantizer
    rid, rw = _route_textbook(lg[:, :NE], NU)
    if escale:
        rw = rw * esc[rid]
    wg = oracle.dequant_rows(tg, Wg, E).astype(np.float64).reshape(NE, Fd, E)
    wu = oracle.dequant_rows(tu, Wu, E).astype(np.float64).reshape(NE, Fd, E)
    wd = oracle.dequant_rows(td, Wd, Fd).astype(np.float64).reshape(NE, E, Fd)
    xq = aq.astype(np.float64) * np.repeat(asc.T.astype(np.float64), 32, axis=1)
    ref = np.zeros((T, E))
    for ti in range(T):
        for k in range(NU):
            e = rid[ti, k]
            g = wg[e] @ xq[ti]
            u = wu[e] @ xq[ti]
            h = (u * (g / (1 + np.exp(-g)))).astype(np.float32)
            hq, hs, _ = oracle.quantize_act(h[None])
            hd = hq[0].astype(np.float64) * np.repeat(hs[:, 0].astype(np.float64), 32)
            ref[ti] += rw[ti, k] * (wd[e] @ hd)
        if shared:
            g = 1.0 / (1.0 + np.exp(-float(lg[ti, NE]))) if shared == "gated" else 1.0
            ref[ti] += g * sh[ti]
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert err < 2e-3, err  # (h's int8 requantization may flip a value where float64 and the f32 path differ)
