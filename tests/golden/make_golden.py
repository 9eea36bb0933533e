"""Writes tests/golden/known_answers.npz: known-answer vectors for the quantized matmul path.

Every expected value here is computed from the chosen integer FIELDS of each block (scales, nibbles, grid indices,
sign bits) with numpy, following the GGML block definitions and the reference's per-element formulas
(src/quants.h:149-158 Q8_0, 91-114 Q4_K / Q5_K, 115-135 Q6_K, 136-148 Q4_0 / IQ4_NL, 297-312 IQ4_XS, 240-262 IQ3_S,
170-239 IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS;
quantizer 559-576; GEMV per-block expression zero/kernels/decode.cl:695-706). Nothing here calls the oracle or the product, so the fixture pins both.
The block bytes come from tests/encoders.py (packing written from the GGML structs).

Edge cases: d = 0, d = +-65504 (largest half), d = 2^-24 (smallest subnormal half), all-15 nibbles, IQ3_S grid
indices with bit 8 set, all sign bits set, Q5_K with only the fifth bits set, all-0 and all-15 Q4_0 / IQ4_NL
nibbles, the IQ2 / IQ3_XXS types' last grid index with every stored sign set; quantizer rows with exact ties, zero
blocks, +-amax, subnormals.

Run: python tests/golden/make_golden.py   (deterministic; rewrites the .npz)
"""
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from tests import encoders as enc  # noqa: E402

KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int64)
F32 = np.float32
D_EDGE = [0.0, 65504.0, -65504.0, 2.0 ** -24]


def _table(name):
    """the integers of one #define'd initializer of oracle/iq_tables.inc (the codebooks are data, not arithmetic)"""
    txt = open(os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle", "iq_tables.inc")).read()
    body = re.search(r"#define " + name + r" \{(.*?)\}", txt, re.S).group(1)
    return np.array([int(v, 0) for v in re.findall(r"0x[0-9a-f]+|\d+", body)], dtype=np.uint64)


def iq3s_grid():
    return _table("QM_IQ3S_GRID_INIT").astype(np.int64)


def _bytes_of(v, n):
    return np.array([(int(v) >> (8 * j)) & 0xFF for j in range(n)], dtype=np.int64)


def _sign8(s7):
    """the 8 signs of a 7-bit sign word: bits 0-6 stored, bit 7 their parity (an even count of negatives)"""
    bits = [(int(s7) >> j) & 1 for j in range(7)]
    return np.array(bits + [sum(bits) & 1], dtype=bool)


def iq2_superblocks(qtype, rng):
    """IQ2_XXS (16), IQ2_XS (17), IQ2_S (22), IQ3_XXS (18) superblocks from chosen fields (src/quants.h:170-239):
    value = (d / 8 or d / 4) * (1 + 2 * nibble) * (+-grid byte)"""
    grid = {16: _table("QM_IQ2XXS_GRID_INIT"), 17: _table("QM_IQ2XS_GRID_INIT"), 22: _table("QM_IQ2S_GRID_INIT"),
            18: _table("QM_IQ3XXS_GRID_INIT")}[qtype]
    out = []
    for i in range(len(D_EDGE) + 28):
        d = np.float16(D_EDGE[i]) if i < len(D_EDGE) else np.float16(abs(rng.standard_normal()) * 0.01)
        per16 = qtype in (17, 22)
        nib = rng.integers(0, 16, 16 if per16 else 8)
        if qtype == 18:
            gidx = rng.integers(0, 256, 64)
        else:
            gidx = rng.integers(0, len(grid), 32)
        sg = rng.integers(0, 256 if qtype == 22 else 128, 32)
        if i == 1:  # largest index, all stored signs set, largest scale
            gidx[:] = len(grid) - 1
            sg[:] = 255 if qtype == 22 else 127
            nib[:] = 15
        if qtype == 18:
            mag = np.concatenate([_bytes_of(grid[g], 4) for g in gidx])
        else:
            mag = np.concatenate([_bytes_of(grid[g], 8) for g in gidx])
        neg = np.concatenate([np.array([(int(v) >> j) & 1 for j in range(8)], dtype=bool) if qtype == 22 else _sign8(v)
                              for v in sg])
        q = np.where(neg, -mag, mag)
        if qtype == 16:
            raw = enc.enc_iq2_xxs(d, nib, gidx, sg)
        elif qtype == 17:
            raw = enc.enc_iq2_xs(d, nib, gidx, sg)
        elif qtype == 22:
            raw = enc.enc_iq2_s(d, nib, gidx, sg)
        else:
            raw = enc.enc_iq3_xxs(d, nib, gidx, sg)
        sc = 1 + 2 * nib  # per 16 (IQ2_XS, IQ2_S) or per 32
        wd = F32(d) / F32(4.0 if qtype == 18 else 8.0)
        e = np.arange(256) // (16 if per16 else 32)
        dq = ((wd * sc[e].astype(F32)) * q.astype(F32)).astype(F32)
        out.append((raw, q, sc, np.zeros(8, np.int64), wd, F32(0), dq))
    return out


def superblocks(qtype, rng, grid):
    """(raw bytes [n][sb], int quants [n][256], int scales [n][8], int mins [n][8], d [n], dmin [n], dq f32 [n][256])"""
    if qtype in (16, 17, 18, 22):
        return iq2_superblocks(qtype, rng)
    out = []
    n_rand = 28
    for i in range(len(D_EDGE) + n_rand):
        d = np.float16(D_EDGE[i]) if i < len(D_EDGE) else np.float16(abs(rng.standard_normal()) * 0.01)
        e = np.arange(256) // 32
        if qtype == 8:  # Q8_0: per-32 half scales
            d8 = np.full(8, d, dtype=np.float16) if i < len(D_EDGE) else \
                (np.abs(rng.standard_normal(8)) * 0.02 / 127).astype(np.float16)
            q = rng.integers(-127, 128, 256)
            if i == 1:
                q[:] = 127
            raw = enc.enc_q8_0(d8.astype(np.float32), q)
            sc, mn = np.ones(8, np.int64), np.zeros(8, np.int64)
            dq = (d8.astype(F32)[e] * q.astype(F32)).astype(F32)
            out.append((raw, q, sc, mn, d8.astype(F32), F32(0), dq))
            continue
        if qtype == 14:  # Q6_K: per-16 int8 scales, 6-bit q stored with an offset of 32
            sc16 = rng.integers(-128, 128, 16)
            q6 = rng.integers(0, 64, 256)
            if i == 1:
                q6[:] = 63
                sc16[:] = -128
            raw = enc.enc_q6_k(d, sc16, q6)
            e16 = np.arange(256) // 16
            dq = ((F32(d) * sc16[e16].astype(F32)) * (q6 - 32).astype(F32)).astype(F32)
            out.append((raw, q6 - 32, sc16, np.zeros(8, np.int64), F32(d), F32(0), dq))
            continue
        if qtype in (2, 20):  # Q4_0 / IQ4_NL: per-32 half scales, nibbles (q - 8 / the IQ4_NL codebook)
            d8 = np.full(8, d, dtype=np.float16) if i < len(D_EDGE) else \
                (np.abs(rng.standard_normal(8)) * 0.02 / 8).astype(np.float16)
            nib = rng.integers(0, 16, 256)
            if i == 1:
                nib[:] = 15
            if i == 2:
                nib[:] = 0
            raw = enc.enc_q4_0(d8.astype(np.float32), nib)
            q = nib - 8 if qtype == 2 else KV[nib]
            dq = (d8.astype(F32)[e] * q.astype(F32)).astype(F32)
            out.append((raw, q, np.ones(8, np.int64), np.zeros(8, np.int64), d8.astype(F32), F32(0), dq))
            continue
        if qtype == 13:  # Q5_K: Q4_K's scales and mins, 5-bit q
            dmin = np.float16(D_EDGE[(i + 1) % len(D_EDGE)]) if i < len(D_EDGE) else np.float16(abs(rng.standard_normal()) * 0.01)
            sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
            q = rng.integers(0, 32, 256)
            if i == 1:
                q[:] = 31
                sc[:] = 63
            if i == 2:
                q[:] = 16  # only the fifth bits set
            raw = enc.enc_q5_k(d, dmin, sc, mn, q)
            dq = ((F32(d) * sc[e].astype(F32)) * q.astype(F32) - F32(dmin) * mn[e].astype(F32)).astype(F32)
            out.append((raw, q, sc, mn, F32(d), F32(dmin), dq))
            continue
        if qtype == 12:  # Q4_K
            dmin = np.float16(D_EDGE[(i + 1) % len(D_EDGE)]) if i < len(D_EDGE) else np.float16(abs(rng.standard_normal()) * 0.01)
            sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
            q = rng.integers(0, 16, 256)
            if i == 1:
                q[:] = 15
                sc[:] = 63
            raw = enc.enc_q4_k(d, dmin, sc, mn, q)
            dq = ((F32(d) * sc[e].astype(F32)) * q.astype(F32) - F32(dmin) * mn[e].astype(F32)).astype(F32)
            out.append((raw, q, sc, mn, F32(d), F32(dmin), dq))
        elif qtype == 23:  # IQ4_XS
            ls, idx = rng.integers(0, 64, 8), rng.integers(0, 16, 256)
            if i == 1:
                idx[:] = 15
                ls[:] = 63
            raw = enc.enc_iq4_xs(d, ls, idx)
            sc = ls - 32
            dq = ((F32(d) * sc[e].astype(F32)) * KV[idx].astype(F32)).astype(F32)
            out.append((raw, KV[idx], sc, np.zeros(8, np.int64), F32(d), F32(0), dq))
        else:  # IQ3_S
            nib = rng.integers(0, 16, 8)
            gidx = rng.integers(0, 512, 64)
            sign = rng.random(256) < 0.5
            if i == 1:
                gidx[:] = 256 + np.arange(64)
                sign[:] = True
                nib[:] = 15
            mag = np.array([(grid[gidx[k // 4]] >> (8 * (k % 4))) & 0xFF for k in range(256)])
            q = np.where(sign, -mag, mag)
            raw = enc.enc_iq3_s(d, nib, gidx, sign)
            sc = 1 + 2 * nib
            dq = ((F32(d) * sc[e].astype(F32)) * q.astype(F32)).astype(F32)
            out.append((raw, q, sc, np.zeros(8, np.int64), F32(d), F32(0), dq))
    return out


def quantize(x):
    """aq [M][K] int8, asc [K/32][M] f32, absum [K/16][M] int16 (src/quants.h:559-576: q = rint(v * (127/amax)))"""
    M, K = x.shape
    aq = np.zeros((M, K), np.int8)
    asc = np.zeros((K // 32, M), F32)
    absum = np.zeros((K // 16, M), np.int16)
    for m in range(M):
        for b in range(K // 32):
            v = x[m, 32 * b:32 * b + 32]
            amax = F32(np.max(np.abs(v)))
            if amax > 0:
                q = np.rint(v * (F32(127.0) / amax)).astype(np.int64)
                asc[b, m] = amax / F32(127.0)
            else:
                q = np.zeros(32, np.int64)
            aq[m, 32 * b:32 * b + 32] = q
            absum[2 * b, m] = q[:16].sum()
            absum[2 * b + 1, m] = q[16:].sum()
    return aq, asc, absum


def main():
    rng = np.random.default_rng(20240611)
    grid = iq3s_grid()
    data = {}
    # quantizer rows (K = 256): ties, zero block, +-amax, negative zero and subnormals, one large outlier
    x = rng.standard_normal((3, 256)).astype(F32)
    x[0, 0:32] = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5] + [3.5] * 24, dtype=F32)
    x[0, 32:64] = 0.0
    x[0, 64:96] = np.linspace(-7.0, 7.0, 32, dtype=F32)
    x[1, 96:128] = F32(1e-40)
    x[1, 96] = F32(-0.0)
    x[1, 97] = F32(3.0)
    x[2, 128:160] *= F32(1000.0)
    aq, asc, absum = quantize(x)
    data.update(quant_x=x, quant_aq=aq, quant_asc=asc, quant_absum=absum)
    # per type: edge + random superblocks as an N x K matrix (N = 16 rows of K = 512), its dequantized values,
    # the int32 block sums against the first quantizer row pattern, and the GEMV output
    for qtype, name in ((8, "q8_0"), (12, "q4_k"), (23, "iq4_xs"), (21, "iq3_s"), (14, "q6_k"), (13, "q5_k"),
                        (2, "q4_0"), (20, "iq4_nl"), (16, "iq2_xxs"), (17, "iq2_xs"), (22, "iq2_s"),
                        (18, "iq3_xxs")):
        sbs = superblocks(qtype, rng, grid)
        N, K = 16, 512
        nsb = K // 256
        assert len(sbs) == N * nsb
        raw = np.stack([s[0] for s in sbs]).reshape(N, -1)
        dq = np.stack([s[6] for s in sbs]).reshape(N, K)
        xa = rng.standard_normal((1, K)).astype(F32)
        aq1, asc1, absum1 = quantize(xa)
        isum = np.zeros((N, K // 32), np.int64)   # sc * sum(q * a) per 32-block
        msum = np.zeros((N, K // 32), np.int64)   # Q4_K: mn * sum(a) per 32-block
        y = np.zeros(N, np.float64)
        for n in range(N):
            for s in range(nsb):
                raw_, q, sc, mn, d, dmin, _ = sbs[n * nsb + s]
                for j in range(8):
                    b = 8 * s + j
                    a = aq1[0, 32 * b:32 * b + 32].astype(np.int64)
                    qq = q[32 * j:32 * j + 32].astype(np.int64)
                    if qtype in (14, 17, 22):  # sc0 * lo + sc1 * hi
                        iv = int(sc[2 * j]) * int(np.dot(qq[:16], a[:16])) + int(sc[2 * j + 1]) * int(np.dot(qq[16:], a[16:]))
                    else:
                        iv = int(sc[j]) * int(np.dot(qq, a))
                    isum[n, b] = iv
                    sa = asc1[b, 0]
                    if qtype in (8, 2, 20):
                        y[n] += float(sa * d[j] * F32(iv))
                    elif qtype in (12, 13):
                        mv = int(mn[j]) * int(a.sum())
                        msum[n, b] = mv
                        y[n] += float(sa * (d * F32(iv) - dmin * F32(mv)))
                    else:
                        y[n] += float(sa * d * F32(iv))
        data.update({f"{name}_raw": raw, f"{name}_dq": dq, f"{name}_x": xa, f"{name}_isum": isum,
                     f"{name}_msum": msum, f"{name}_y": y})
    path = os.path.join(HERE, "known_answers.npz")
    np.savez_compressed(path, **data)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
