"""GGUF block geometry of the weight types of the path, and seeded synthetic weights in GGUF block form.

Geometry: src/gguf.h:43-72 of the reference (Q8_0 32 elements / 34 bytes, Q4_0 and IQ4_NL 32 / 18, Q4_K 256 / 144,
Q5_K 256 / 176, Q6_K 256 / 210, IQ2_XXS 256 / 66, IQ2_XS 256 / 74, IQ2_S 256 / 82, IQ3_XXS 256 / 98, IQ3_S 256 / 110,
IQ4_XS 256 / 136, Q2_K 256 / 84, IQ1_S 256 / 50, IQ1_M 256 / 56, Q3_K 256 / 110, and the reference's own Q2_0 64 / 18, src/gguf.h:26, 69). The synthetic generators produce the BASELINE configurations' distributions directly as block
bytes: every quant / index / sign / sub-scale bit uniform, the f16 super-scales |N(0, sigma)|.
"""
import numpy as np

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS = 2, 8, 12, 13, 14, 20, 21, 23
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ2_S = 16, 17, 18, 22
Q2_K, Q3_K, Q2_0 = 10, 11, 42
IQ1_S, IQ1_M = 19, 29
TYPE_NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ4_NL: "IQ4_NL", IQ3_S: "IQ3_S",
              IQ4_XS: "IQ4_XS", IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS", IQ3_XXS: "IQ3_XXS", IQ2_S: "IQ2_S", Q3_K: "Q3_K",
              Q2_0: "Q2_0", Q2_K: "Q2_K", IQ1_S: "IQ1_S", IQ1_M: "IQ1_M"}
TYPES_BY_NAME = {v: k for k, v in TYPE_NAMES.items()}

# bytes of one 256-element superblock (Q8_0: 8 blocks of 34)
SB_BYTES = {Q4_0: 144, Q8_0: 272, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_NL: 144, IQ3_S: 110, IQ4_XS: 136, IQ2_XXS: 66,
            IQ2_XS: 74, IQ3_XXS: 98, IQ2_S: 82, Q3_K: 110, Q2_0: 72, Q2_K: 84, IQ1_S: 50, IQ1_M: 56}


SMALL_BLOCK_TYPES = (Q8_0, Q4_0, IQ4_NL, Q2_0)  # 32- (Q2_0: 64-) element blocks: rows may end inside a superblock


def small_block(qtype):
    """Elements per GGUF block of a small-block type."""
    return 64 if qtype == Q2_0 else 32


def row_bytes(qtype, K):
    if qtype in SMALL_BLOCK_TYPES and K % small_block(qtype) == 0:
        return K // 32 * (SB_BYTES[qtype] // 8)
    if K % 256:
        raise ValueError(f"K = {K} is not a multiple of 256")
    return K // 256 * SB_BYTES[qtype]


def padded_k(K):
    return (K + 255) // 256 * 256


def pad_small_rows(qtype, W, K):
    """Rows of K elements of a small-block type -> rows of padded_k(K) elements, the added blocks all zero (an f16
    zero scale: they decode to 0), as the reference's pad_small_block_rows (src/quants.h:581-595)."""
    assert qtype in SMALL_BLOCK_TYPES and K % small_block(qtype) == 0
    out = np.zeros((W.shape[0], row_bytes(qtype, padded_k(K))), dtype=np.uint8)
    out[:, :row_bytes(qtype, K)] = W
    return out


def weight_bytes(qtype, N, K):
    """Algorithmic weight bytes of an N x K matrix: N * (K/256) * superblock bytes."""
    return N * row_bytes(qtype, K)


def f16_bits(x):
    """float array -> IEEE half bit patterns (round to nearest even), as uint16."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def synth_weight(qtype, N, K, seed, sigma=None):
    """N rows of K elements in GGUF block form (uint8 [N, row_bytes]).

    Q8_0:   q uniform in [-127, 127], d = f16(|N(0, 0.02)| / 127) per 32 (sigma: the normal's sigma)
    Q4_K:   quants, 6-bit scales and mins uniform (all bits random), d and dmin = f16(|N(0, 0.01)|)
    IQ4_XS: nibbles and 6-bit sub-scales uniform, d = f16(|N(0, 0.01)|)
    IQ3_S:  9-bit grid indices, signs and 4-bit sub-scales uniform, d = f16(|N(0, 0.01)|)
    Q6_K:   6-bit quants and int8 per-16 scales uniform, d = f16(|N(0, 0.01)|) (d is the last field)
    Q5_K:   as Q4_K (the fifth bits uniform too)
    Q4_0 / IQ4_NL: nibbles uniform, d = f16(|N(0, 0.02)| / 8) per 32
    IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS: grid indices, sign indices or bits and 4-bit sub-scales uniform,
            d = f16(|N(0, 0.01)|)
    Q3_K:   2-bit values, high bits and 6-bit scales uniform, d = f16(|N(0, 0.01)|) (d is the last field)
    Q2_0:   2-bit codes uniform, d = f16(|N(0, 0.02)|) per 64
    Q2_K:   2-bit values, 4-bit scales and mins uniform, d and dmin = f16(|N(0, 0.01)|) (the last two fields)
    IQ1_S / IQ1_M: 11-bit grid indices, delta signs and 3-bit scales uniform, d = f16(|N(0, 0.01)|) (IQ1_M: its
            bits in the top nibbles of the four scale words)
    """
    rng = np.random.default_rng(seed)
    nsb = K // 256
    if qtype == Q8_0:
        sig = 0.02 if sigma is None else sigma
        nblk = N * K // 32
        blk = np.empty((nblk, 34), dtype=np.uint8)
        d = f16_bits(np.abs(rng.normal(0.0, sig, nblk)) / 127.0)
        blk[:, 0] = d & 0xFF
        blk[:, 1] = d >> 8
        blk[:, 2:] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
        return blk.reshape(N, K // 32 * 34)
    if qtype in (Q4_0, IQ4_NL):
        sig = 0.02 if sigma is None else sigma
        nblk = N * K // 32
        blk = rng.integers(0, 256, size=(nblk, 18), dtype=np.uint8)
        d = f16_bits(np.abs(rng.normal(0.0, sig, nblk)) / 8.0)
        blk[:, 0] = d & 0xFF
        blk[:, 1] = d >> 8
        return blk.reshape(N, K // 32 * 18)
    if qtype == Q2_0:
        sig = 0.02 if sigma is None else sigma
        nblk = N * K // 64
        blk = rng.integers(0, 256, size=(nblk, 18), dtype=np.uint8)
        d = f16_bits(np.abs(rng.normal(0.0, sig, nblk)))
        blk[:, 0] = d & 0xFF
        blk[:, 1] = d >> 8
        return blk.reshape(N, K // 64 * 18)
    sig = 0.01 if sigma is None else sigma
    sb = SB_BYTES[qtype]
    raw = rng.integers(0, 256, size=(N * nsb, sb), dtype=np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, sig, N * nsb)))
    at = {Q6_K: 208, Q3_K: 108, Q2_K: 80}.get(qtype, 0)
    raw[:, at] = d & 0xFF
    raw[:, at + 1] = d >> 8
    if qtype == IQ1_M:  # (d's 16 bits go to the top nibbles of the scale words at bytes 48..55)
        sw = raw[:, 48:56].copy().view(np.uint16).reshape(-1, 4) & np.uint16(0x0FFF)
        for i in range(4):
            sw[:, i] |= ((d >> (4 * i)) & 0xF).astype(np.uint16) << 12
        raw[:, 48:56] = sw.reshape(-1, 4).view(np.uint8).reshape(-1, 8)
        raw[:, 0] = rng.integers(0, 256, N * nsb, dtype=np.uint8)  # (byte 0 is a grid index, not d)
        raw[:, 1] = rng.integers(0, 256, N * nsb, dtype=np.uint8)
    if qtype in (Q4_K, Q5_K, Q2_K):
        dm = f16_bits(np.abs(rng.normal(0.0, sig, N * nsb)))
        am = 82 if qtype == Q2_K else 2
        raw[:, am] = dm & 0xFF
        raw[:, am + 1] = dm >> 8
    return raw.reshape(N, nsb * sb)


def synth_activations(M, K, seed, outlier_frac=0.0, outlier_scale=20.0):
    """f32 [M, K] N(0, 1); with outlier_frac > 0 a fixed seeded set of that fraction of the channels x outlier_scale."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    if outlier_frac > 0:
        n_out = max(1, int(round(K * outlier_frac)))
        ch = rng.choice(K, size=n_out, replace=False)
        x[:, ch] *= np.float32(outlier_scale)
    return x


def zipf_router_logits(T, NE, seed, s=1.1):
    """Router logits whose top-8 is Zipf(s)-distributed over the experts: logit_e = -s * ln(rank_e) + Gumbel(0, 1),
    with a seeded random rank permutation (top-k of Gumbel-perturbed log-weights samples k distinct experts with
    probability proportional to rank^-s)."""
    rng = np.random.default_rng(seed)
    rank = rng.permutation(NE) + 1
    g = rng.gumbel(0.0, 1.0, size=(T, NE))
    return (-s * np.log(rank)[None, :] + g).astype(np.float32)
