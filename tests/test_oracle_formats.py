"""Pins the oracle's format code (oracle/qref.c) without retyping it:
  - fp16 conversions against numpy's IEEE half (exhaustive for half -> float);
  - the codebooks against published ggml values and structural invariants;
  - each block decoder against an independent encoder (tests/encoders.py, written from the GGML block structs):
    chosen fields must come back exactly, and the dequantized values must equal the field formula;
  - closed forms: a block whose nibbles are all i dequantizes to d * sc * kvalues[i], zero scales give zeros.
"""
import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F
from tests import encoders as enc

KV_PUBLISHED = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def test_fp16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = oracle.fp16_to_f32(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_fp16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 4000),
        # exact half-way cases between adjacent halves (ties go to even), normal and subnormal
        ((np.arange(1, 400, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)),
        ((np.arange(1, 400, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)),
        np.array([0.0, -0.0, 65504.0, 65519.0, 6e-8, 3e-8, 2.98e-8], dtype=np.float32),
    ]).astype(np.float32)
    ref = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_fp16(x)
    assert np.array_equal(got, ref)


def test_codebooks_match_published_and_invariants():
    import re
    txt = open(oracle.HERE + "/iq_tables.inc").read()
    kv = [int(v) for v in re.search(r"QM_IQ4NL_VALUES_INIT \{([^}]*)\}", txt).group(1).split(",")]
    assert kv == KV_PUBLISHED
    grid = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", re.search(r"QM_IQ3S_GRID_INIT \{(.*?)\}", txt, re.S).group(1))]
    assert len(grid) == 512
    assert grid[0] == 0x01010101 and grid[1] == 0x01010103 and grid[-1] == 0x0F0F0101  # published end entries
    assert grid == sorted(grid) and len(set(grid)) == 512  # ggml's IQ3_S grid is sorted and distinct
    for g in grid:
        for j in range(4):
            b = (g >> (8 * j)) & 0xFF
            assert b % 2 == 1 and 1 <= b <= 15  # IQ3_S grid values are odd magnitudes 1..15
    # the product's copy is the same data
    prod = open(oracle.HERE + "/../arcinfer_amd/csrc/iq_tables.inc").read()
    assert prod == txt


def _kv():
    return np.array(KV_PUBLISHED, dtype=np.int64)


def test_q8_0_decoder_round_trip():
    rng = np.random.default_rng(1)
    for _ in range(20):
        d8 = rng.standard_normal(8).astype(np.float16).astype(np.float32)
        q = rng.integers(-128, 128, 256)
        o = oracle.decode_sb(F.Q8_0, enc.enc_q8_0(d8, q))
        assert np.array_equal(o["q"], q) and np.array_equal(o["d8"], d8)
        w = oracle.dequant_rows(F.Q8_0, enc.enc_q8_0(d8, q)[None], 256)[0]
        assert np.array_equal(w, (np.repeat(d8, 32) * q.astype(np.float32)).astype(np.float32))


def test_q4_k_decoder_round_trip():
    rng = np.random.default_rng(2)
    for _ in range(50):
        d, dmin = np.float16(rng.random()), np.float16(rng.random())
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        raw = enc.enc_q4_k(d, dmin, sc, mn, q)
        o = oracle.decode_sb(F.Q4_K, raw)
        assert np.array_equal(o["sc"], sc) and np.array_equal(o["mn"], mn) and np.array_equal(o["q"], q)
        assert o["d"] == np.float32(d) and o["dmin"] == np.float32(dmin)
        w = oracle.dequant_rows(F.Q4_K, raw[None], 256)[0]
        e = np.arange(256) // 32
        ref = (np.float32(d) * sc[e].astype(np.float32) * q.astype(np.float32)
               - np.float32(dmin) * mn[e].astype(np.float32)).astype(np.float32)
        assert np.array_equal(w, ref)


def test_iq4_xs_decoder_round_trip_and_closed_form():
    rng = np.random.default_rng(3)
    kv = _kv()
    for _ in range(50):
        d = np.float16(rng.standard_normal())
        ls, idx = rng.integers(0, 64, 8), rng.integers(0, 16, 256)
        raw = enc.enc_iq4_xs(d, ls, idx)
        o = oracle.decode_sb(F.IQ4_XS, raw)
        assert np.array_equal(o["sc"], ls - 32) and np.array_equal(o["q"], kv[idx])
    # closed form: every nibble i, every scale 33 (sc 1), d 1 -> the codebook itself
    for i in range(16):
        raw = enc.enc_iq4_xs(np.float16(1.0), [33] * 8, [i] * 256)
        assert np.all(oracle.dequant_rows(F.IQ4_XS, raw[None], 256)[0] == KV_PUBLISHED[i])
    # ls = 32 -> scale 0 -> all zeros
    raw = enc.enc_iq4_xs(np.float16(3.0), [32] * 8, rng.integers(0, 16, 256))
    assert np.all(oracle.dequant_rows(F.IQ4_XS, raw[None], 256)[0] == 0)


def test_iq3_s_decoder_round_trip():
    import re
    txt = open(oracle.HERE + "/iq_tables.inc").read()
    body = re.search(r"QM_IQ3S_GRID_INIT \{(.*?)\}", txt, re.S).group(1)
    grid = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", body)], dtype=np.int64)
    rng = np.random.default_rng(4)
    for it in range(50):
        d = np.float16(rng.random())
        nib = rng.integers(0, 16, 8)
        gidx = rng.integers(0, 512, 64)
        if it == 0:
            gidx[:] = 256 + np.arange(64)  # the 9th index bit set everywhere
        sign = rng.random(256) < 0.5
        if it == 1:
            sign[:] = True
        raw = enc.enc_iq3_s(d, nib, gidx, sign)
        o = oracle.decode_sb(F.IQ3_S, raw)
        mag = np.array([(grid[gidx[e // 4]] >> (8 * (e % 4))) & 0xFF for e in range(256)])
        assert np.array_equal(o["q"], np.where(sign, -mag, mag))
        assert np.array_equal(o["sc"], 1 + 2 * nib)
        w = oracle.dequant_rows(F.IQ3_S, raw[None], 256)[0]
        ref = (np.float32(d) * (1 + 2 * nib[np.arange(256) // 32]).astype(np.float32)
               * np.where(sign, -mag, mag).astype(np.float32)).astype(np.float32)
        assert np.array_equal(w, ref)


@pytest.mark.parametrize("qtype", [F.Q4_0, F.Q8_0, F.Q4_K, F.Q5_K, F.Q6_K, F.IQ4_NL, F.IQ4_XS, F.IQ3_S, F.IQ2_XXS,
                                   F.IQ2_XS, F.IQ2_S, F.IQ3_XXS, F.Q3_K, F.Q2_0, F.Q2_K,
                                   F.IQ1_S, F.IQ1_M])
def test_synth_weights_have_the_requested_statistics(qtype):
    W = F.synth_weight(qtype, 64, 512, seed=5)
    assert W.shape == (64, F.row_bytes(qtype, 512))
    w = oracle.dequant_rows(qtype, W, 512)
    assert np.all(np.isfinite(w))
    if qtype == F.Q8_0:
        q = W.reshape(-1, 34)[:, 2:].view(np.int8)
        assert q.min() >= -127 and q.max() <= 127


def test_q6_k_decoder_round_trip():
    rng = np.random.default_rng(5)
    for it in range(40):
        d = np.float16(rng.standard_normal())
        sc16 = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, 256)
        if it == 0:
            q[:] = 63
            sc16[:] = -128
        raw = enc.enc_q6_k(d, sc16, q)
        o = oracle.decode_sb(F.Q6_K, raw)
        assert np.array_equal(o["q"], q - 32) and np.array_equal(o["sc16"], sc16) and o["d"] == np.float32(d)
        w = oracle.dequant_rows(F.Q6_K, raw[None], 256)[0]
        ref = (np.float32(d) * sc16[np.arange(256) // 16].astype(np.float32) * (q - 32).astype(np.float32))
        assert np.array_equal(w, ref.astype(np.float32))


def test_q5_k_decoder_round_trip():
    rng = np.random.default_rng(6)
    for it in range(40):
        d, dmin = np.float16(rng.random()), np.float16(rng.random())
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 32, 256)
        if it == 0:
            q[:] = 31
        raw = enc.enc_q5_k(d, dmin, sc, mn, q)
        o = oracle.decode_sb(F.Q5_K, raw)
        assert np.array_equal(o["q"], q) and np.array_equal(o["sc"], sc) and np.array_equal(o["mn"], mn)
        w = oracle.dequant_rows(F.Q5_K, raw[None], 256)[0]
        e = np.arange(256) // 32
        ref = (np.float32(d) * sc[e].astype(np.float32) * q.astype(np.float32)
               - np.float32(dmin) * mn[e].astype(np.float32)).astype(np.float32)
        assert np.array_equal(w, ref)


@pytest.mark.parametrize("qtype", [F.Q4_0, F.IQ4_NL])
def test_q4_0_and_iq4_nl_decoders(qtype):
    rng = np.random.default_rng(qtype)
    kv = _kv()
    for _ in range(30):
        d8 = (rng.standard_normal(8) * 0.1).astype(np.float16).astype(np.float32)
        nib = rng.integers(0, 16, 256)
        raw = enc.enc_q4_0(d8, nib)
        o = oracle.decode_sb(qtype, raw)
        q = nib - 8 if qtype == F.Q4_0 else kv[nib]
        assert np.array_equal(o["q"], q) and np.array_equal(o["d8"], d8)
        w = oracle.dequant_rows(qtype, raw[None], 256)[0]
        assert np.array_equal(w, (np.repeat(d8, 32) * q.astype(np.float32)).astype(np.float32))


# ---- IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS
def _grid(name, width):
    import re
    txt = open(oracle.HERE + "/iq_tables.inc").read()
    body = re.search(name + r"_INIT \{(.*?)\}", txt, re.S).group(1)
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]+)u", body)]
    return np.array(vals, dtype=np.uint64), width


def _signs8(sgn7):
    """the 8 sign bits of a 7-bit sign word: the 7 bits, then their parity (an even number of negatives)"""
    s = np.asarray(sgn7, dtype=np.int64)
    par = np.array([bin(int(v)).count("1") & 1 for v in s])
    return s | (par << 7)


def test_iq2_iq3xxs_codebooks_published_and_invariants():
    g2xxs, _ = _grid("QM_IQ2XXS_GRID", 8)
    g2xs, _ = _grid("QM_IQ2XS_GRID", 8)
    g2s, _ = _grid("QM_IQ2S_GRID", 8)
    g3xxs, _ = _grid("QM_IQ3XXS_GRID", 4)
    assert (len(g2xxs), len(g2xs), len(g2s), len(g3xxs)) == (256, 512, 1024, 256)
    # published first entries (ggml-common.h)
    assert int(g2xxs[0]) == 0x0808080808080808 and int(g2xxs[1]) == 0x080808080808082b
    assert int(g3xxs[0]) == 0x04040404 and int(g3xxs[1]) == 0x04040414
    for g, w, allowed in ((g2xxs, 8, {8, 25, 43}), (g2xs, 8, {8, 25, 43}), (g2s, 8, {8, 25, 43}),
                          (g3xxs, 4, {4, 12, 20, 28, 36, 44, 52, 62})):
        assert len(set(g.tolist())) == len(g)  # distinct
        vals = {(int(v) >> (8 * j)) & 0xFF for v in g for j in range(w)}
        assert vals <= allowed
    # the sign table is the 7 bits plus their parity (the table is data; this is the rule it follows)
    import re
    txt = open(oracle.HERE + "/iq_tables.inc").read()
    ks = [int(v) for v in re.search(r"QM_KSIGNS_IQ2XS_INIT \{([^}]*)\}", txt).group(1).split(",")]
    assert ks == _signs8(np.arange(128)).tolist()


def _expect(grid, idx, width, signs8):
    """elements of groups of `width` grid bytes with sign bytes signs8 (one per 8 elements)"""
    mag = np.array([(int(grid[idx[e // width]]) >> (8 * (e % width))) & 0xFF for e in range(256)], dtype=np.int64)
    neg = np.array([(int(signs8[e // 8]) >> (e % 8)) & 1 for e in range(256)], dtype=bool)
    return np.where(neg, -mag, mag)


@pytest.mark.parametrize("qtype", [F.IQ2_XXS, F.IQ2_XS, F.IQ2_S, F.IQ3_XXS])
def test_iq2_iq3xxs_decoder_round_trip(qtype):
    rng = np.random.default_rng(qtype * 11)
    for it in range(30):
        d = np.float16(rng.random() + 0.1)
        if qtype == F.IQ2_XXS:
            grid, _ = _grid("QM_IQ2XXS_GRID", 8)
            nib = rng.integers(0, 16, 8)
            gidx, sgn7 = rng.integers(0, 256, 32), rng.integers(0, 128, 32)
            raw = enc.enc_iq2_xxs(d, nib, gidx, sgn7)
            q, sc16, dd = _expect(grid, gidx, 8, _signs8(sgn7)), np.repeat(1 + 2 * nib, 2), np.float32(d) / 8
        elif qtype == F.IQ2_XS:
            grid, _ = _grid("QM_IQ2XS_GRID", 8)
            nib16 = rng.integers(0, 16, 16)
            gidx, sgn7 = rng.integers(0, 512, 32), rng.integers(0, 128, 32)
            if it == 0:
                gidx[:] = 256 + np.arange(32)  # the 9th index bit everywhere
            raw = enc.enc_iq2_xs(d, nib16, gidx, sgn7)
            q, sc16, dd = _expect(grid, gidx, 8, _signs8(sgn7)), 1 + 2 * nib16, np.float32(d) / 8
        elif qtype == F.IQ2_S:
            grid, _ = _grid("QM_IQ2S_GRID", 8)
            nib16 = rng.integers(0, 16, 16)
            gidx, signs8 = rng.integers(0, 1024, 32), rng.integers(0, 256, 32)
            if it == 0:
                gidx[:] = 768 + np.arange(32)  # both high index bits everywhere
                signs8[:] = 255
            raw = enc.enc_iq2_s(d, nib16, gidx, signs8)
            q, sc16, dd = _expect(grid, gidx, 8, signs8), 1 + 2 * nib16, np.float32(d) / 8
        else:
            grid, _ = _grid("QM_IQ3XXS_GRID", 4)
            nib = rng.integers(0, 16, 8)
            gidx, sgn7 = rng.integers(0, 256, 64), rng.integers(0, 128, 32)
            raw = enc.enc_iq3_xxs(d, nib, gidx, sgn7)
            q, sc16, dd = _expect(grid, gidx, 4, _signs8(sgn7)), np.repeat(1 + 2 * nib, 2), np.float32(d) / 4
        assert raw.size == F.SB_BYTES[qtype]
        o = oracle.decode_sb(qtype, raw)
        assert np.array_equal(o["q"], q) and np.array_equal(o["sc16"], sc16) and o["d"] == dd
        w = oracle.dequant_rows(qtype, raw[None], 256)[0]
        ref = (dd * sc16[np.arange(256) // 16].astype(np.float32) * q.astype(np.float32)).astype(np.float32)
        assert np.array_equal(w, ref)


def test_q3_k_decoder_round_trip_and_closed_form():
    """The oracle's Q3_K decode (src/quants.h:465-494, the 12 scale bytes unpacked through the kmask shuffle) against
    ggml's packing (tests/encoders.py), plus a closed form: block ib's values all ib - 4 with scales 32 + 2i + 1."""
    rng = np.random.default_rng(11)
    for it in range(40):
        d = np.float16(rng.standard_normal())
        sc6 = rng.integers(0, 64, 16)
        q = rng.integers(-4, 4, 256)
        if it == 0:
            q = np.repeat(np.arange(8) - 4, 32)
            sc6 = 32 + 2 * np.arange(16) + 1
        if it == 1:
            q[:] = -4
            sc6[:] = 0
        raw = enc.enc_q3_k(d, sc6, q)
        assert raw.size == 110
        o = oracle.decode_sb(F.Q3_K, raw)
        assert np.array_equal(o["q"], q) and np.array_equal(o["sc16"], sc6 - 32) and o["d"] == np.float32(d)
        w = oracle.dequant_rows(F.Q3_K, raw[None], 256)[0]
        ref = np.float32(d) * (sc6 - 32)[np.arange(256) // 16].astype(np.float32) * q.astype(np.float32)
        assert np.array_equal(w, ref.astype(np.float32))
        if it == 0:  # element 32 ib + e: d * (33 + 2 (2 ib + e // 16) - 32) * (ib - 4)
            e = np.arange(256)
            assert np.array_equal(w, (np.float32(d) * (1 + 2 * (e // 16)).astype(np.float32)
                                      * (e // 32 - 4).astype(np.float32)).astype(np.float32))


def test_q2_0_decoder_round_trip_and_closed_form():
    """Q2_0 (the reference's 64-element blocks, value (code - 1) d, src/quants.h:540-548): random codes round trip,
    and the byte 0xE4 (codes 0, 1, 2, 3 from bit 0 up) decodes to -1, 0, 1, 2 for every four elements."""
    rng = np.random.default_rng(12)
    for it in range(30):
        d4 = (rng.standard_normal(4) * 0.1).astype(np.float16).astype(np.float32)
        codes = rng.integers(0, 4, 256)
        if it == 0:
            codes = np.tile(np.arange(4), 64)
        raw = enc.enc_q2_0(d4, codes)
        if it == 0:
            assert np.all(raw.reshape(4, 18)[:, 2:] == 0xE4)
        o = oracle.decode_sb(F.Q2_0, raw)
        assert np.array_equal(o["q"], codes - 1) and np.array_equal(o["d8"], np.repeat(d4, 2))
        w = oracle.dequant_rows(F.Q2_0, raw[None], 256)[0]
        assert np.array_equal(w, (np.repeat(d4, 64) * (codes - 1).astype(np.float32)).astype(np.float32))
    assert F.row_bytes(F.Q2_0, 640) == 10 * 18 and F.row_bytes(F.Q3_K, 512) == 220


def test_q2_k_decoder_round_trip():
    """Q2_K (src/quants.h:159-169: scale and min per 16 elements) against ggml's block struct (tests/encoders.py)."""
    rng = np.random.default_rng(13)
    for it in range(40):
        d, dmin = np.float16(rng.random()), np.float16(rng.random())
        sc4, mn4 = rng.integers(0, 16, 16), rng.integers(0, 16, 16)
        q = rng.integers(0, 4, 256)
        if it == 0:
            q[:] = 3
            sc4[:], mn4[:] = 15, 15
        raw = enc.enc_q2_k(d, dmin, sc4, mn4, q)
        assert raw.size == 84
        o = oracle.decode_sb(F.Q2_K, raw)
        assert np.array_equal(o["q"], q) and np.array_equal(o["sc16"], sc4) and np.array_equal(o["mn16"], mn4)
        assert o["d"] == np.float32(d) and o["dmin"] == np.float32(dmin)
        w = oracle.dequant_rows(F.Q2_K, raw[None], 256)[0]
        e16 = np.arange(256) // 16
        ref = (np.float32(d) * sc4[e16].astype(np.float32) * q.astype(np.float32)
               - np.float32(dmin) * mn4[e16].astype(np.float32)).astype(np.float32)
        assert np.array_equal(w, ref)


def test_per16_mins_enter_the_block_dot():
    """The block-dot oracle's Q2_K min term is mn0 * bs0 + mn1 * bs1 (decode.cl:703-706): with all values 0 the
    block sums vanish and the product is -sa * dmin * (mn0 * bs0 + mn1 * bs1) per block, brute-forced here."""
    rng = np.random.default_rng(14)
    d, dmin = np.float16(0.5), np.float16(0.25)
    mn4 = rng.integers(0, 16, 16)
    raw = enc.enc_q2_k(d, dmin, rng.integers(0, 16, 16), mn4, np.zeros(256, np.int64))
    x = rng.standard_normal((1, 256)).astype(np.float32)
    aq, asc, absum = oracle.quantize_act(x)
    C, isum, msum = oracle.blockdot(F.Q2_K, raw[None], 256, aq, asc, absum, blocksums=True)
    assert np.all(isum == 0)
    bs = absum[:, 0].astype(np.int64)
    want_m = np.array([mn4[2 * b] * bs[2 * b] + mn4[2 * b + 1] * bs[2 * b + 1] for b in range(8)])
    assert np.array_equal(msum.reshape(-1), want_m)
    want = sum(float(np.float32(asc[b, 0]) * (np.float32(d) * np.float32(0) - np.float32(dmin) * np.float32(want_m[b])))
               for b in range(8))
    assert abs(float(C[0, 0]) - want) <= 1e-6 * max(1.0, abs(want))


def _iq1_grid():
    import re
    txt = open(oracle.HERE + "/iq_tables.inc").read()
    body = re.search(r"QM_IQ1S_GRID_INIT \{(.*?)\}", txt, re.S).group(1)
    g = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", body)], dtype=np.uint64)
    return g.view(np.int8).reshape(2048, 8).astype(np.int64)


def test_iq1_codebook_published_and_invariants():
    g = _iq1_grid()
    assert g.shape == (2048, 8)
    assert set(np.unique(g)) <= {-1, 0, 1}
    assert np.all(g[0] == -1) and list(g[1]) == [1, -1, -1, -1, -1, -1, -1, -1]  # published first entries
    assert len({tuple(r) for r in g}) == 2048  # distinct


@pytest.mark.parametrize("qtype", [F.IQ1_S, F.IQ1_M])
def test_iq1_decoders_round_trip(qtype):
    """IQ1_S / IQ1_M (src/quants.h:263-296) against ggml's block structs: q = 8 * grid + delta, sc = 2 s + 1 (per 32
    for IQ1_S, per 16 for IQ1_M), d / 8; grid entry 0 (all -1) with delta +1 gives -7 throughout."""
    g = _iq1_grid()
    rng = np.random.default_rng(qtype)
    for it in range(25):
        d = np.float16(abs(rng.standard_normal()) + 0.01)
        gidx = rng.integers(0, 2048, 32)
        if qtype == F.IQ1_S:
            s3, neg = rng.integers(0, 8, 8), rng.integers(0, 2, 8)
            if it == 0:
                gidx[:], neg[:], s3[:] = 0, 0, 7
            raw = enc.enc_iq1_s(d, s3, neg, gidx)
            dl = np.repeat(np.where(neg == 1, -1, 1), 32)
            sc16 = np.repeat(2 * s3 + 1, 2)
        else:
            s3, neg = rng.integers(0, 8, 16), rng.integers(0, 2, 32)
            if it == 0:
                gidx[:], neg[:], s3[:] = 0, 0, 7
            raw = enc.enc_iq1_m(d, s3, neg, gidx)
            dl = np.repeat(np.where(neg == 1, -1, 1), 8)
            sc16 = 2 * s3 + 1
        assert raw.size == F.SB_BYTES[qtype]
        o = oracle.decode_sb(qtype, raw)
        q = 8 * g[gidx].reshape(-1) + dl
        assert np.array_equal(o["q"], q) and np.array_equal(o["sc16"], sc16)
        assert o["d"] == np.float32(np.float32(d) / 8)
        if it == 0:
            assert np.all(o["q"] == -7)
        w = oracle.dequant_rows(qtype, raw[None], 256)[0]
        ref = (np.float32(np.float32(d) / 8) * sc16[np.arange(256) // 16].astype(np.float32) * q.astype(np.float32))
        assert np.array_equal(w, ref.astype(np.float32))
