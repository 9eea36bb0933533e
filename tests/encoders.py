"""Independent numpy encoders of the GGUF block structs, written from the GGML block definitions
(ggml-common.h: block_q8_0 {d; qs[32]}, block_q4_K {d; dmin; scales[12]; qs[128]}, block_iq4_xs {d; scales_h;
scales_l[4]; qs[128]}, block_iq3_s {d; qs[64]; qh[8]; signs[32]; scales[4]}, block_q6_k {ql[128]; qh[64];
scales[16]; d}, and the IQ2 / IQ3_XXS structs listed below), NOT from the oracle's decoders: they
pack chosen integer fields into bytes, so decoding them back pins the decoders' bit positions."""
import numpy as np


def _h(d):
    return np.array([d], dtype=np.float16).view(np.uint8)


def enc_q8_0(d8, q):
    """d8: 8 floats (one per 32-block), q: 256 ints in [-128, 127] -> 272 bytes"""
    out = bytearray()
    for b in range(8):
        out += _h(d8[b]).tobytes()
        out += np.asarray(q[32 * b:32 * b + 32], dtype=np.int8).tobytes()
    return np.frombuffer(bytes(out), dtype=np.uint8)


def enc_q4_k(d, dmin, sc, mn, q):
    """sc, mn: 8 six-bit ints; q: 256 ints 0..15 -> 144 bytes (6-bit scale packing of ggml's K-quants)"""
    s = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    qs = np.zeros(128, dtype=np.uint8)
    for j in range(4):  # 64-element chunk j: low nibbles elements 64j..64j+31, high nibbles 64j+32..64j+63
        for l in range(32):
            qs[32 * j + l] = (q[64 * j + l] & 0xF) | ((q[64 * j + 32 + l] & 0xF) << 4)
    return np.concatenate([_h(d), _h(dmin), s, qs])


def enc_iq4_xs(d, ls, idx):
    """ls: 8 six-bit scales (the value is ls - 32), idx: 256 codebook indices 0..15 -> 136 bytes"""
    sh = 0
    sl = np.zeros(4, dtype=np.uint8)
    for ib in range(8):
        sl[ib // 2] |= (ls[ib] & 0xF) << (4 * (ib % 2))
        sh |= ((ls[ib] >> 4) & 3) << (2 * ib)
    qs = np.zeros(128, dtype=np.uint8)
    for ib in range(8):
        for j in range(16):
            qs[16 * ib + j] = (idx[32 * ib + j] & 0xF) | ((idx[32 * ib + 16 + j] & 0xF) << 4)
    return np.concatenate([_h(d), np.array([sh], dtype=np.uint16).view(np.uint8), sl, qs])


def enc_iq3_s(d, scale_nib, gidx, sign):
    """scale_nib: 8 four-bit scales (value 1 + 2 * nib); gidx: 64 nine-bit grid indices (one per 4 elements, in
    element order); sign: 256 bools -> 110 bytes"""
    qs = np.zeros(64, dtype=np.uint8)
    qh = np.zeros(8, dtype=np.uint8)
    signs = np.zeros(32, dtype=np.uint8)
    sc = np.zeros(4, dtype=np.uint8)
    for g in range(64):
        ib, r = divmod(g, 8)
        qs[8 * ib + r] = gidx[g] & 0xFF
        qh[ib] |= ((gidx[g] >> 8) & 1) << r
    for e in range(256):
        if sign[e]:
            signs[e // 8] |= 1 << (e % 8)
    for ib in range(8):
        sc[ib // 2] |= (scale_nib[ib] & 0xF) << (4 * (ib % 2))
    return np.concatenate([_h(d), qs, qh, signs, sc])


def enc_q6_k(d, sc16, q):
    """sc16: 16 int8 scales (one per 16 elements), q: 256 ints 0..63 (the stored 6-bit values) -> 210 bytes.
    Element 128n + 32c + l (c = 0..3): low 4 bits in ql[64n + l + 32 (c & 1)], nibble c >> 1; high 2 bits in
    qh[32n + l], bits 2c..2c+1."""
    ql = np.zeros(128, dtype=np.uint8)
    qh = np.zeros(64, dtype=np.uint8)
    for n in range(2):
        for c in range(4):
            for l in range(32):
                v = int(q[128 * n + 32 * c + l])
                ql[64 * n + l + 32 * (c & 1)] |= (v & 0xF) << (4 * (c >> 1))
                qh[32 * n + l] |= ((v >> 4) & 3) << (2 * c)
    return np.concatenate([ql, qh, np.asarray(sc16, dtype=np.int8).view(np.uint8), _h(d)])


def enc_q5_k(d, dmin, sc, mn, q):
    """q: 256 ints 0..31 -> 176 bytes: d, dmin, scales[12] (as Q4_K), qh[32] (bit 2j / 2j+1 of qh[l]: fifth bit of
    elements 64j + l / 64j + 32 + l), qs[128] (low nibbles as Q4_K)."""
    base = enc_q4_k(d, dmin, sc, mn, np.asarray(q) & 0xF)
    qh = np.zeros(32, dtype=np.uint8)
    for j in range(4):
        for l in range(32):
            qh[l] |= ((int(q[64 * j + l]) >> 4) & 1) << (2 * j)
            qh[l] |= ((int(q[64 * j + 32 + l]) >> 4) & 1) << (2 * j + 1)
    return np.concatenate([base[:16], qh, base[16:]])


def enc_q4_0(d8, nib):
    """d8: 8 floats (one per 32), nib: 256 nibbles 0..15 (element order) -> 8 blocks of (f16 d, 16 bytes)."""
    out = bytearray()
    for b in range(8):
        out += _h(d8[b]).tobytes()
        out += bytes(int(nib[32 * b + i]) | (int(nib[32 * b + 16 + i]) << 4) for i in range(16))
    return np.frombuffer(bytes(out), dtype=np.uint8)


enc_iq4_nl = enc_q4_0  # (the same block struct: f16 d + 32 nibbles; the nibbles index the IQ4_NL codebook)


# ---- the IQ2 / IQ3_XXS codebook types (ggml-common.h: block_iq2_xxs {d; qs[32] as u16}, block_iq2_xs {d; qs[32] as
# u16; scales[8]}, block_iq2_s {d; qs[64]; qh[8]; scales[8]}, block_iq3_xxs {d; qs[96]}). Sign groups of 8 elements
# carry an even number of negatives in these formats: the stored 7 bits are the first 7 signs and the 8th is their
# parity, so the encoders take 7-bit sign words.

def _u32(v):
    return np.array([v], dtype=np.uint32).view(np.uint8)


def enc_iq2_xxs(d, scale_nib, gidx, sgn7):
    """scale_nib: 8 four-bit scales (value 1 + 2 nib, per 32); gidx: 32 eight-bit grid indices (one per 8 elements,
    in element order); sgn7: 32 seven-bit sign words -> 66 bytes"""
    out = [_h(d)]
    for ib in range(8):
        a0 = sum(int(gidx[4 * ib + l]) << (8 * l) for l in range(4))
        a1 = sum(int(sgn7[4 * ib + l]) << (7 * l) for l in range(4)) | (int(scale_nib[ib]) << 28)
        out += [_u32(a0), _u32(a1)]
    return np.concatenate(out)


def enc_iq2_xs(d, scale_nib16, gidx, sgn7):
    """scale_nib16: 16 four-bit scales (per 16 elements); gidx: 32 nine-bit grid indices; sgn7: 32 seven-bit sign
    words -> 74 bytes"""
    qs = np.array([(int(gidx[g]) & 511) | (int(sgn7[g]) << 9) for g in range(32)], dtype=np.uint16).view(np.uint8)
    sc = np.array([(int(scale_nib16[2 * ib]) & 0xF) | ((int(scale_nib16[2 * ib + 1]) & 0xF) << 4) for ib in range(8)],
                  dtype=np.uint8)
    return np.concatenate([_h(d), qs, sc])


def enc_iq2_s(d, scale_nib16, gidx, signs8):
    """scale_nib16: 16 four-bit scales; gidx: 32 ten-bit grid indices; signs8: 32 sign bytes (bit j: element j of
    the group negative; all 8 bits stored) -> 82 bytes"""
    qs = np.array([int(g) & 0xFF for g in gidx], dtype=np.uint8)
    qh = np.zeros(8, dtype=np.uint8)
    for g in range(32):
        ib, l = divmod(g, 4)
        qh[ib] |= ((int(gidx[g]) >> 8) & 3) << (2 * l)
    sc = np.array([(int(scale_nib16[2 * ib]) & 0xF) | ((int(scale_nib16[2 * ib + 1]) & 0xF) << 4) for ib in range(8)],
                  dtype=np.uint8)
    return np.concatenate([_h(d), qs, np.asarray(signs8, dtype=np.uint8), qh, sc])


def enc_iq3_xxs(d, scale_nib, gidx, sgn7):
    """scale_nib: 8 four-bit scales (per 32); gidx: 64 eight-bit grid indices (one per 4 elements); sgn7: 32 seven-bit
    sign words (one per 8 elements) -> 98 bytes"""
    qs = np.asarray(gidx, dtype=np.uint8)
    ss = [_u32(sum(int(sgn7[4 * ib + l]) << (7 * l) for l in range(4)) | (int(scale_nib[ib]) << 28)) for ib in range(8)]
    return np.concatenate([_h(d), qs] + ss)


# ---- Q3_K (ggml-common.h block_q3_K {hmask[32]; qs[64]; scales[12]; d}) and the reference's Q2_0 (src/gguf.h:26:
# blocks of 64, f16 d then 16 bytes of 2-bit codes)
def enc_q3_k(d, sc6, q):
    """sc6: 16 scales 0..63 (stored; the value is sc6 - 32), q: 256 values -4..3 -> 110 bytes. Packed as ggml's
    quantizer writes them: L = q + 4; element j's high bit (L > 3) in hmask[j % 32] bit j / 32 and its low 2 bits in
    qs[32 (j / 128) + j % 32], bits 2 ((j % 128) / 32); scale j: low nibble in scales[j % 8] (nibble j / 8), top 2
    bits in scales[8 + j % 4] (bits 2 (j / 4))."""
    L = np.asarray(q, dtype=np.int64) + 4
    hmask = np.zeros(32, dtype=np.uint8)
    qs = np.zeros(64, dtype=np.uint8)
    for j in range(256):
        if L[j] > 3:
            hmask[j % 32] |= 1 << (j // 32)
        qs[32 * (j // 128) + j % 32] |= (int(L[j]) & 3) << (2 * ((j % 128) // 32))
    scales = np.zeros(12, dtype=np.uint8)
    for j in range(16):
        ls = int(sc6[j])
        if j < 8:
            scales[j] = ls & 0xF
        else:
            scales[j - 8] |= (ls & 0xF) << 4
        scales[8 + j % 4] |= (ls >> 4) << (2 * (j // 4))
    return np.concatenate([hmask, qs, scales, _h(d)])


def enc_q2_0(d4, codes):
    """d4: 4 floats (one per 64), codes: 256 ints 0..3 -> 4 blocks of (f16 d, 16 bytes: element j in bits 2 (j % 4) of
    byte j / 4)."""
    out = bytearray()
    for g in range(4):
        out += _h(d4[g]).tobytes()
        c = [int(v) for v in codes[64 * g:64 * g + 64]]
        out += bytes(c[4 * t] | (c[4 * t + 1] << 2) | (c[4 * t + 2] << 4) | (c[4 * t + 3] << 6) for t in range(16))
    return np.frombuffer(bytes(out), dtype=np.uint8)


def enc_q2_k(d, dmin, sc4, mn4, q):
    """ggml block_q2_K {scales[16]; qs[64]; d; dmin}: sc4 / mn4 16 scales and mins 0..15 (per 16 elements, scale in
    the low nibble), q 256 values 0..3: element 128n + 32j + l in qs[32n + l], bits 2j -> 84 bytes."""
    scales = (np.asarray(sc4, dtype=np.int64) | (np.asarray(mn4, dtype=np.int64) << 4)).astype(np.uint8)
    qs = np.zeros(64, dtype=np.uint8)
    for e in range(256):
        n, j, l = e // 128, (e % 128) // 32, e % 32
        qs[32 * n + l] |= int(q[e]) << (2 * j)
    return np.concatenate([scales, qs, _h(d), _h(dmin)])


# ---- IQ1_S / IQ1_M (ggml-common.h block_iq1_s {d; qs[32]; qh[8] as u16}, block_iq1_m {qs[32]; qh[16]; scales[8]})
def enc_iq1_s(d, s3, neg, gidx):
    """s3: 8 scales 0..7 (sc = 2 s + 1), neg: 8 delta signs (per 32), gidx: 32 grid indices 0..2047 (4 per block, one
    per 8 elements) -> 50 bytes: qh[ib] = 3 high index bits per group (bits 3l..3l+2) | s << 12 | neg << 15."""
    qs = np.array([g & 0xFF for g in gidx], dtype=np.uint8)
    qh = np.zeros(8, dtype=np.uint16)
    for ib in range(8):
        v = (int(s3[ib]) << 12) | (int(neg[ib]) << 15)
        for l in range(4):
            v |= ((int(gidx[4 * ib + l]) >> 8) & 7) << (3 * l)
        qh[ib] = v
    return np.concatenate([_h(d), qs, qh.view(np.uint8)])


def enc_iq1_m(d, s3, neg, gidx):
    """s3: 16 scales 0..7 (per 16), neg: 32 delta signs (per 8), gidx: 32 grid indices -> 56 bytes: qh per 8-group a
    nibble (3 high index bits, sign bit 3), scales as 4 u16 of four 3-bit fields (bits 0-11) with d's 16 bits in their
    top nibbles (word i holds d's bits 4i..4i+3)."""
    qs = np.array([g & 0xFF for g in gidx], dtype=np.uint8)
    qh = np.zeros(16, dtype=np.uint8)
    for g in range(32):
        qh[g // 2] |= ((((int(gidx[g]) >> 8) & 7) | (int(neg[g]) << 3)) << (4 * (g % 2)))
    dbits = int(_h(d).view(np.uint16)[0])
    sw = np.zeros(4, dtype=np.uint16)
    for i in range(4):
        v = 0
        for f in range(4):
            v |= int(s3[4 * i + f]) << (3 * f)
        sw[i] = v | (((dbits >> (4 * i)) & 0xF) << 12)
    return np.concatenate([qs, qh, sw.view(np.uint8)])
