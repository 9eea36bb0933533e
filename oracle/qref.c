/* CPU oracle for the quantized matrix-product path -- TEST INFRASTRUCTURE ONLY (see qref.h).
 *
 * Compiled with -ffp-contract=off and without fast-math, so float expressions round exactly as written.
 * Reference citations are rizagp/arcinfer paths relative to its root.
 */
#include "qref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static const uint32_t k_iq3s_grid[512] = QM_IQ3S_GRID_INIT;
static const int8_t k_iq4nl[16] = QM_IQ4NL_VALUES_INIT;
static const uint64_t k_iq2xxs_grid[256] = QM_IQ2XXS_GRID_INIT;
static const uint64_t k_iq2xs_grid[512] = QM_IQ2XS_GRID_INIT;
static const uint64_t k_iq2s_grid[1024] = QM_IQ2S_GRID_INIT;
static const uint32_t k_iq3xxs_grid[256] = QM_IQ3XXS_GRID_INIT;
static const uint8_t k_ksigns[128] = QM_KSIGNS_IQ2XS_INIT;
static const uint64_t k_iq1s_grid[2048] = QM_IQ1S_GRID_INIT;

/* src/quants.h:17-31 -- IEEE half to float, subnormals normalised by shifting */
float qref_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, f;
  if (e == 0) {
    if (m == 0) {
      f = sign;
    } else {
      e = 127 - 15 + 1;
      while (!(m & 0x400u)) {
        m <<= 1;
        --e;
      }
      f = sign | (e << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    f = sign | 0x7F800000u | (m << 13);
  } else {
    f = sign | ((e + 127 - 15) << 23) | (m << 13);
  }
  float r;
  memcpy(&r, &f, 4);
  return r;
}

/* src/quants.h:33-52 -- float to half, round to nearest even, NaN kept quiet, overflow to infinity */
uint16_t qref_f32_to_fp16(float x) {
  uint32_t f;
  memcpy(&f, &x, 4);
  const uint32_t sign = (f >> 16) & 0x8000u;
  const int32_t e = (int32_t)((f >> 23) & 0xFFu) - 127 + 15;
  uint32_t m = f & 0x7FFFFFu;
  if (((f >> 23) & 0xFFu) == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)h;
}

/* src/gguf.h:43-72 (the block geometry of the path's types) */
int qref_block_info(int type, int* blk, int* bytes) {
  switch (type) {
    case QREF_Q8_0: *blk = 32; *bytes = 34; return 0;
    case QREF_Q4_K: *blk = 256; *bytes = 144; return 0;
    case QREF_Q5_K: *blk = 256; *bytes = 176; return 0;
    case QREF_Q6_K: *blk = 256; *bytes = 210; return 0;
    case QREF_Q4_0: *blk = 32; *bytes = 18; return 0;
    case QREF_IQ4_NL: *blk = 32; *bytes = 18; return 0;
    case QREF_IQ3_S: *blk = 256; *bytes = 110; return 0;
    case QREF_IQ4_XS: *blk = 256; *bytes = 136; return 0;
    case QREF_IQ2_XXS: *blk = 256; *bytes = 66; return 0;
    case QREF_IQ2_XS: *blk = 256; *bytes = 74; return 0;
    case QREF_IQ2_S: *blk = 256; *bytes = 82; return 0;
    case QREF_IQ3_XXS: *blk = 256; *bytes = 98; return 0;
    case QREF_Q3_K: *blk = 256; *bytes = 110; return 0;
    case QREF_Q2_K: *blk = 256; *bytes = 84; return 0;
    case QREF_IQ1_S: *blk = 256; *bytes = 50; return 0;
    case QREF_IQ1_M: *blk = 256; *bytes = 56; return 0;
    case QREF_Q2_0: *blk = 64; *bytes = 18; return 0;  /* (the reference's own type, src/gguf.h:26, 69) */
    default: return -1;
  }
}

int qref_sb_bytes(int type) {
  int blk, bytes;
  if (qref_block_info(type, &blk, &bytes)) return -1;
  return bytes * (256 / blk);
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

/* 8 elements from an 8-byte grid entry and a sign byte (bit j set: element j negative) (src/quants.h:178-180) */
static void grid8_signs(uint64_t g, unsigned sg, int16_t* q) {
  for (int j = 0; j < 8; ++j) {
    const int v = (int)((g >> (8 * j)) & 0xFF);
    q[j] = (int16_t)((sg & (1u << j)) ? -v : v);
  }
}

/* src/quants.h:61-69 */
static void scale_min_k4(int j, const uint8_t* q, int* d, int* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
  }
}

/* src/quants.h:89-315 (cases Q4_K / Q5_K 91-114, Q6_K 115-135, Q4_0 136-148, Q8_0 149-158, IQ2_XXS 170-184,
 * IQ2_XS 185-201, IQ2_S 202-219, IQ3_XXS 220-239, IQ3_S 240-262, IQ4_XS 297-312; IQ4_NL from dequant_row
 * 527-538) */
static int decode_sb_raw(int type, const uint8_t* p, qref_sb* o) {
  memset(o, 0, sizeof(*o));
  switch (type) {
    case QREF_Q4_K:
    case QREF_Q5_K: {
      /* src/quants.h:91-114: d, dmin, 12 bytes of 6-bit scales/mins; Q5_K then qh[32] (bit 2j / 2j+1 of qh[l]: the
       * fifth bit of elements 64j + l / 64j + 32 + l), then qs[128] */
      o->d = qref_fp16_to_f32(rd16(p));
      o->dmin = qref_fp16_to_f32(rd16(p + 2));
      for (int b = 0; b < 8; ++b) scale_min_k4(b, p + 4, &o->sc[b], &o->mn[b]);
      const uint8_t* qh = type == QREF_Q5_K ? p + 16 : NULL;
      const uint8_t* qs = type == QREF_Q5_K ? p + 48 : p + 16;
      for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
          int lo = qs[32 * j + l] & 0xF, hi = qs[32 * j + l] >> 4;
          if (qh) {
            lo |= ((qh[l] >> (2 * j)) & 1) << 4;
            hi |= ((qh[l] >> (2 * j + 1)) & 1) << 4;
          }
          o->q[64 * j + l] = (int16_t)lo;
          o->q[64 * j + 32 + l] = (int16_t)hi;
        }
      return 0;
    }
    case QREF_Q4_0:
    case QREF_IQ4_NL: {
      /* src/quants.h:136-148 (Q4_0: q = nibble - 8) and 527-538 (IQ4_NL: q = kvalues_iq4nl[nibble]): 8 blocks of
       * (f16 d, 16 bytes: low nibbles = elements 0..15, high = 16..31) */
      for (int b = 0; b < 8; ++b) {
        const uint8_t* blk = p + 18 * b;
        o->d8[b] = qref_fp16_to_f32(rd16(blk));
        o->sc[b] = 1;
        for (int i = 0; i < 16; ++i) {
          const int lo = blk[2 + i] & 0xF, hi = blk[2 + i] >> 4;
          o->q[32 * b + i] = (int16_t)(type == QREF_Q4_0 ? lo - 8 : k_iq4nl[lo]);
          o->q[32 * b + 16 + i] = (int16_t)(type == QREF_Q4_0 ? hi - 8 : k_iq4nl[hi]);
        }
      }
      return 0;
    }
    case QREF_Q2_0: {
      /* src/quants.h:540-548 (dequant_row): 4 blocks of 64 (f16 d, 16 bytes: element j = bits 2 (j % 4) of byte j / 4),
       * value (q - 1) * d */
      for (int g = 0; g < 4; ++g) {
        const uint8_t* blk = p + 18 * g;
        o->d8[2 * g] = o->d8[2 * g + 1] = qref_fp16_to_f32(rd16(blk));
        o->sc[2 * g] = o->sc[2 * g + 1] = 1;
        for (int j = 0; j < 64; ++j) o->q[64 * g + j] = (int16_t)(((blk[2 + j / 4] >> (2 * (j % 4))) & 3) - 1);
      }
      return 0;
    }
    case QREF_IQ1_S: {
      /* src/quants.h:263-276: d | qs[32] | qh[8] (u16 per 32: 3 high grid-index bits per 8 elements, bits 12-14 the
       * scale, bit 15 the delta sign); wd = d / 8, sc = 2 s + 1, q = 8 * grid byte + delta */
      const uint8_t* qs = p + 2;
      o->d = qref_fp16_to_f32(rd16(p)) / 8;
      for (int ib = 0; ib < 8; ++ib) {
        const unsigned qh = rd16(p + 34 + 2 * ib);
        o->sc[ib] = (int)(2 * ((qh >> 12) & 7) + 1);
        const int dl = (qh & 0x8000) ? -1 : 1;
        for (int l = 0; l < 4; ++l) {
          const uint64_t g = k_iq1s_grid[qs[4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)];
          for (int j = 0; j < 8; ++j) o->q[32 * ib + 8 * l + j] = (int16_t)(8 * (int)(int8_t)(g >> (8 * j)) + dl);
        }
      }
      return 0;
    }
    case QREF_IQ1_M: {
      /* src/quants.h:277-296: qs[32] | qh[16] | scales (4 u16: two 3-bit scales per 32-block, the f16 d in their top
       * nibbles); per 8 elements 3 high grid-index bits and a delta sign in a nibble of qh */
      const uint8_t *qs = p, *qh = p + 32;
      const unsigned sc[4] = {rd16(p + 48), rd16(p + 50), rd16(p + 52), rd16(p + 54)};
      const unsigned su = (sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000);
      o->d = qref_fp16_to_f32((uint16_t)su) / 8;
      for (int ib = 0; ib < 8; ++ib) {
        o->sc16[2 * ib] = (int)(2 * ((sc[ib / 2] >> (6 * (ib % 2))) & 7) + 1);
        o->sc16[2 * ib + 1] = (int)(2 * ((sc[ib / 2] >> (6 * (ib % 2) + 3)) & 7) + 1);
        o->sc[ib] = o->sc16[2 * ib];
        const unsigned h0 = qh[2 * ib], h1 = qh[2 * ib + 1];
        const unsigned idx[4] = {qs[4 * ib] | ((h0 << 8) & 0x700), qs[4 * ib + 1] | ((h0 << 4) & 0x700),
                                 qs[4 * ib + 2] | ((h1 << 8) & 0x700), qs[4 * ib + 3] | ((h1 << 4) & 0x700)};
        const int dl[4] = {(h0 & 0x08) ? -1 : 1, (h0 & 0x80) ? -1 : 1, (h1 & 0x08) ? -1 : 1, (h1 & 0x80) ? -1 : 1};
        for (int l = 0; l < 4; ++l) {
          const uint64_t g = k_iq1s_grid[idx[l]];
          for (int j = 0; j < 8; ++j) o->q[32 * ib + 8 * l + j] = (int16_t)(8 * (int)(int8_t)(g >> (8 * j)) + dl[l]);
        }
      }
      return 0;
    }
    case QREF_Q2_K: {
      /* src/quants.h:159-169: scales[16] (per 16 elements: scale = low nibble, min = high nibble) | qs[64] | d | dmin;
       * element e (n = e / 128, j = (e % 128) / 32): q = (qs[32 n + e % 32] >> 2 j) & 3 */
      const uint8_t *sc = p, *qs = p + 16;
      o->d = qref_fp16_to_f32(rd16(p + 80));
      o->dmin = qref_fp16_to_f32(rd16(p + 82));
      for (int i = 0; i < 16; ++i) {
        o->sc16[i] = sc[i] & 0xF;
        o->mn16[i] = sc[i] >> 4;
      }
      for (int e = 0; e < 256; ++e) {
        const int n = e / 128, r = e % 128, j = r / 32;
        o->q[e] = (int16_t)((qs[32 * n + r % 32] >> (2 * j)) & 3);
      }
      for (int b = 0; b < 8; ++b) {
        o->sc[b] = o->sc16[2 * b];  /* (per-32 view: the first half's scale and min) */
        o->mn[b] = o->mn16[2 * b];
      }
      return 0;
    }
    case QREF_Q3_K: {
      /* src/quants.h:465-494 (dequant_q3_k, llama.cpp's order): hmask[32] | qs[64] | scales[12] | d. The 12 scale bytes
       * unpack to 16 6-bit scales through the kmask shuffle; per 128 elements n and 2-bit shift j: 16 elements from
       * q[l] and 16 from q[l + 16] (l < 16), value ((q >> shift) & 3) - (hmask & m ? 0 : 4), m = 1 << (4 n + j), the
       * scales taken in order */
      const uint8_t *hm = p, *q = p + 32;
      o->d = qref_fp16_to_f32(rd16(p + 108));
      uint32_t aux[4];
      memcpy(aux, p + 96, 12);
      const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu, tmp = aux[2];
      aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
      aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
      aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
      aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
      const int8_t* scales = (const int8_t*)aux;
      int is = 0, e = 0;
      unsigned m = 1;
      for (int n = 0; n < 256; n += 128) {
        int shift = 0;
        for (int j = 0; j < 4; ++j) {
          o->sc16[is] = scales[is] - 32;
          ++is;
          for (int l = 0; l < 16; ++l) o->q[e++] = (int16_t)(((q[l] >> shift) & 3) - ((hm[l] & m) ? 0 : 4));
          o->sc16[is] = scales[is] - 32;
          ++is;
          for (int l = 0; l < 16; ++l) o->q[e++] = (int16_t)(((q[l + 16] >> shift) & 3) - ((hm[l + 16] & m) ? 0 : 4));
          shift += 2;
          m <<= 1;
        }
        q += 32;
      }
      for (int b = 0; b < 8; ++b) o->sc[b] = o->sc16[2 * b];  /* (per-32 view: the first half's scale) */
      return 0;
    }
    case QREF_Q8_0: {
      for (int b = 0; b < 8; ++b) {
        const uint8_t* blk = p + 34 * b;
        o->d8[b] = qref_fp16_to_f32(rd16(blk));
        o->sc[b] = 1;
        for (int i = 0; i < 32; ++i) o->q[32 * b + i] = (int16_t)(int8_t)blk[2 + i];
      }
      return 0;
    }
    case QREF_IQ3_S: {
      o->d = qref_fp16_to_f32(rd16(p));
      const uint8_t *qs = p + 2, *qh = p + 66, *signs = p + 74, *scales = p + 106;
      for (int ib = 0; ib < 8; ++ib) {
        o->sc[ib] = 1 + 2 * ((scales[ib / 2] >> (4 * (ib % 2))) & 0xF);
        const unsigned h = qh[ib];
        for (int l = 0; l < 4; ++l) {
          const uint32_t g1 = k_iq3s_grid[qs[8 * ib + 2 * l] | ((h << (8 - 2 * l)) & 256)];
          const uint32_t g2 = k_iq3s_grid[qs[8 * ib + 2 * l + 1] | ((h << (7 - 2 * l)) & 256)];
          const unsigned sg = signs[4 * ib + l];
          for (int j = 0; j < 4; ++j) {
            const int v1 = (int)((g1 >> (8 * j)) & 0xFF), v2 = (int)((g2 >> (8 * j)) & 0xFF);
            o->q[32 * ib + 8 * l + j] = (int16_t)((sg & (1u << j)) ? -v1 : v1);
            o->q[32 * ib + 8 * l + j + 4] = (int16_t)((sg & (1u << (j + 4))) ? -v2 : v2);
          }
        }
      }
      return 0;
    }
    case QREF_IQ2_XXS: {
      /* src/quants.h:170-184: d (f16) then 8 blocks of (a0: 4 grid indices, a1: 4 x 7-bit sign indices + 4-bit
       * scale); wd = d / 8 */
      o->d = qref_fp16_to_f32(rd16(p)) / 8;
      for (int ib = 0; ib < 8; ++ib) {
        const uint32_t a0 = rd32(p + 2 + 8 * ib), a1 = rd32(p + 2 + 8 * ib + 4);
        o->sc[ib] = 1 + 2 * (int)(a1 >> 28);
        for (int l = 0; l < 4; ++l)
          grid8_signs(k_iq2xxs_grid[(a0 >> (8 * l)) & 0xFF], k_ksigns[(a1 >> (7 * l)) & 127], o->q + 32 * ib + 8 * l);
      }
      return 0;
    }
    case QREF_IQ2_XS: {
      /* src/quants.h:185-201: d, qs[32] (u16: 9-bit grid index, 7-bit sign index), scales[8] (4 bits per 16) */
      o->d = qref_fp16_to_f32(rd16(p)) / 8;
      const uint8_t* scales = p + 66;
      for (int ib = 0; ib < 8; ++ib) {
        o->sc16[2 * ib] = 1 + 2 * (scales[ib] & 0xF);
        o->sc16[2 * ib + 1] = 1 + 2 * (scales[ib] >> 4);
        o->sc[ib] = o->sc16[2 * ib];
        for (int l = 0; l < 4; ++l) {
          const unsigned q16 = rd16(p + 2 + 2 * (4 * ib + l));
          grid8_signs(k_iq2xs_grid[q16 & 511], k_ksigns[q16 >> 9], o->q + 32 * ib + 8 * l);
        }
      }
      return 0;
    }
    case QREF_IQ2_S: {
      /* src/quants.h:202-219: d, qs[32] (grid index low 8 bits), signs[32], qh[8] (2 high bits per 8 elements),
       * scales[8] (4 bits per 16) */
      o->d = qref_fp16_to_f32(rd16(p)) / 8;
      const uint8_t *qs = p + 2, *signs = p + 34, *qh = p + 66, *scales = p + 74;
      for (int ib = 0; ib < 8; ++ib) {
        o->sc16[2 * ib] = 1 + 2 * (scales[ib] & 0xF);
        o->sc16[2 * ib + 1] = 1 + 2 * (scales[ib] >> 4);
        o->sc[ib] = o->sc16[2 * ib];
        for (int l = 0; l < 4; ++l)
          grid8_signs(k_iq2s_grid[qs[4 * ib + l] | ((qh[ib] << (8 - 2 * l)) & 0x300)], signs[4 * ib + l],
                      o->q + 32 * ib + 8 * l);
      }
      return 0;
    }
    case QREF_IQ3_XXS: {
      /* src/quants.h:220-239: d, qs[64] (grid indices), then per block a word of 4 x 7-bit sign indices + 4-bit
       * scale; wd = d / 4 */
      o->d = qref_fp16_to_f32(rd16(p)) / 4;
      const uint8_t *qs = p + 2, *ss = p + 66;
      for (int ib = 0; ib < 8; ++ib) {
        const uint32_t a = rd32(ss + 4 * ib);
        o->sc[ib] = 1 + 2 * (int)(a >> 28);
        for (int l = 0; l < 4; ++l) {
          const unsigned sg = k_ksigns[(a >> (7 * l)) & 127];
          const uint32_t g1 = k_iq3xxs_grid[qs[8 * ib + 2 * l]], g2 = k_iq3xxs_grid[qs[8 * ib + 2 * l + 1]];
          for (int j = 0; j < 4; ++j) {
            const int v1 = (int)((g1 >> (8 * j)) & 0xFF), v2 = (int)((g2 >> (8 * j)) & 0xFF);
            o->q[32 * ib + 8 * l + j] = (int16_t)((sg & (1u << j)) ? -v1 : v1);
            o->q[32 * ib + 8 * l + j + 4] = (int16_t)((sg & (1u << (j + 4))) ? -v2 : v2);
          }
        }
      }
      return 0;
    }
    case QREF_IQ4_XS: {
      o->d = qref_fp16_to_f32(rd16(p));
      const unsigned sh = rd16(p + 2);
      const uint8_t *sl = p + 4, *qs = p + 8;
      for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xF) | (int)(((sh >> (2 * ib)) & 3) << 4);
        o->sc[ib] = ls - 32;
        for (int j = 0; j < 16; ++j) {
          o->q[32 * ib + j] = k_iq4nl[qs[16 * ib + j] & 0xF];
          o->q[32 * ib + 16 + j] = k_iq4nl[qs[16 * ib + j] >> 4];
        }
      }
      return 0;
    }
    case QREF_Q6_K: {
      /* src/quants.h:115-135: ql[128] | qh[64] | scales[16] (int8, per 16) | d; q = (4 low bits | 2 high bits << 4)
       * - 32, kept signed here (the reference keeps q and subtracts 32 in dequant_value, :320) */
      const uint8_t *ql = p, *qh = p + 128;
      o->d = qref_fp16_to_f32(rd16(p + 208));
      for (int i = 0; i < 16; ++i) o->sc16[i] = (int8_t)p[192 + i];
      for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
          const uint8_t *L = ql + 64 * n, *H = qh + 32 * n;
          o->q[128 * n + l] = (int16_t)(((L[l] & 0xF) | (((H[l] >> 0) & 3) << 4)) - 32);
          o->q[128 * n + l + 32] = (int16_t)(((L[l + 32] & 0xF) | (((H[l] >> 2) & 3) << 4)) - 32);
          o->q[128 * n + l + 64] = (int16_t)(((L[l] >> 4) | (((H[l] >> 4) & 3) << 4)) - 32);
          o->q[128 * n + l + 96] = (int16_t)(((L[l + 32] >> 4) | (((H[l] >> 6) & 3) << 4)) - 32);
        }
      for (int b = 0; b < 8; ++b) o->sc[b] = o->sc16[2 * b];  /* (per-32 view: the first half's scale) */
      return 0;
    }
    default: return -1;
  }
}

int qref_decode_sb(int type, const uint8_t* p, qref_sb* o) {
  const int r = decode_sb_raw(type, p, o);
  if (r == 0 && type != QREF_Q6_K && type != QREF_Q3_K && type != QREF_Q2_K && type != QREF_IQ2_XS && type != QREF_IQ2_S &&
      type != QREF_IQ1_M)
    for (int i = 0; i < 16; ++i) o->sc16[i] = o->sc[i / 2];
  if (r == 0 && type != QREF_Q2_K)
    for (int i = 0; i < 16; ++i) o->mn16[i] = o->mn[i / 2];
  return r;
}

/* src/quants.h:317-324 (dequant_value) via :496-555 (dequant_row): float expressions as written there */
static float dequant_value(int type, const qref_sb* o, int e) {
  switch (type) {
    case QREF_Q4_K:
    case QREF_Q5_K: return o->d * (float)o->sc[e / 32] * (float)o->q[e] - o->dmin * (float)o->mn[e / 32];
    case QREF_Q8_0:
    case QREF_Q4_0:
    case QREF_IQ4_NL: return o->d8[e / 32] * (float)o->q[e];
    case QREF_Q2_0: return o->d8[e / 32] * (float)o->q[e];  /* (d * (float)(q - 1), src/quants.h:546) */
    case QREF_Q6_K: return o->d * (float)o->sc16[e / 16] * (float)o->q[e];
    /* (Q3_K: dl * q with dl = d_all * (scale - 32), src/quants.h:486-489) */
    case QREF_Q3_K: return o->d * (float)o->sc16[e / 16] * (float)o->q[e];
    /* (Q2_K: wd * wsc * q - wdmin * wmn per 16, src/quants.h:322) */
    case QREF_Q2_K: return o->d * (float)o->sc16[e / 16] * (float)o->q[e] - o->dmin * (float)o->mn16[e / 16];
    /* (the IQ types: o.wd * o.wsc[e / 16] * (o.q[e] - o.qoff) - 0 with qoff = 0, src/quants.h:322) */
    default: return o->d * (float)o->sc16[e / 16] * (float)o->q[e] - 0.0f;
  }
}

int qref_dequant_row(int type, const uint8_t* row, int K, float* out) {
  const int sb = qref_sb_bytes(type);
  if (sb < 0 || K % 256) return -1;
  qref_sb o;
  for (int s = 0; s < K / 256; ++s) {
    qref_decode_sb(type, row + (size_t)s * sb, &o);
    for (int e = 0; e < 256; ++e) out[s * 256 + e] = dequant_value(type, &o, e);
  }
  return 0;
}

/* src/quants.h:559-576 (quantize_act_cpu); zero rows past M as rmsnorm_quant writes them (ops.cl:82-104) */
void qref_quantize_act(const float* x, int M, int K, int M_stride, int act32, int8_t* aq, float* asc, int16_t* absum) {
  const int B = act32 ? 32 : 256;
  for (int m = 0; m < M_stride; ++m)
    for (int b0 = 0; b0 < K; b0 += B) {
      float amax = 0.0f;
      if (m < M)
        for (int i = 0; i < B; ++i) amax = fmaxf(amax, fabsf(x[(size_t)m * K + b0 + i]));
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      asc[(size_t)(b0 / B) * M_stride + m] = amax / 127.0f;
      for (int i = 0; i < B; ++i)
        aq[(size_t)m * K + b0 + i] = m < M ? (int8_t)lrintf(x[(size_t)m * K + b0 + i] * inv) : 0;
    }
  for (int m = 0; m < M_stride; ++m)
    for (int b = 0; b < K / 16; ++b) {
      int sum = 0;
      for (int i = 0; i < 16; ++i) sum += aq[(size_t)m * K + b * 16 + i];
      absum[(size_t)b * M_stride + m] = (int16_t)sum;
    }
}

/* One row's superblocks decoded once: int8 quants and per-32 integer scales / float superblock scales. */
typedef struct {
  int8_t* q;   /* [K] */
  int* sc;     /* [K/16]: integer scale of each 16-element half-block */
  int* mn;     /* [K/16]: min of each 16-element half-block */
  float* d;    /* [K/32]: d of the block's superblock (Q8_0: the block's own scale) */
  float* dmin; /* [K/32] */
} row_dec;

static void decode_row(int type, const uint8_t* row, int K, row_dec* r) {
  const int sb = qref_sb_bytes(type);
  qref_sb o;
  for (int s = 0; s < K / 256; ++s) {
    qref_decode_sb(type, row + (size_t)s * sb, &o);
    for (int e = 0; e < 256; ++e) r->q[s * 256 + e] = (int8_t)o.q[e];
    for (int i = 0; i < 16; ++i) r->sc[s * 16 + i] = o.sc16[i];
    for (int b = 0; b < 8; ++b) {
      r->mn[s * 16 + 2 * b] = o.mn16[2 * b];
      r->mn[s * 16 + 2 * b + 1] = o.mn16[2 * b + 1];
      r->d[s * 8 + b] = (type == QREF_Q8_0 || type == QREF_Q4_0 || type == QREF_IQ4_NL || type == QREF_Q2_0) ? o.d8[b] : o.d;
      r->dmin[s * 8 + b] = o.dmin;
    }
  }
}

/* decode.cl:695-706 (gemv) and 1107-1115 (gemv_v): per 32-block, int sums of int8 products over its two 16-element
 * halves; the block's value sa * d * (float)(sc0 * lo + sc1 * hi) [- sa * dmin * (float)(mn0 * bs0 + mn1 * bs1) for
 * Q4_K]; sc0 != sc1 only for Q6_K (scales per 16), mn0 = mn1 (mins per 32). */
static double row_dot(int type, const row_dec* r, int K, const int8_t* a, const float* asc, const int16_t* absum,
                      int m, int M_stride, int32_t* bsums, int32_t* msums) {
  double acc = 0.0;
  for (int b = 0; b < K / 32; ++b) {
    int lo = 0, hi = 0;
    for (int i = 0; i < 16; ++i) lo += (int)a[32 * b + i] * (int)r->q[32 * b + i];
    for (int i = 16; i < 32; ++i) hi += (int)a[32 * b + i] * (int)r->q[32 * b + i];
    const int iv = r->sc[2 * b] * lo + r->sc[2 * b + 1] * hi;
    const float sa = asc[(size_t)b * M_stride + m];
    float v;
    if (type == QREF_Q4_K || type == QREF_Q5_K || type == QREF_Q2_K) {
      /* (mn0 * bs0 + mn1 * bs1, decode.cl:703-706; one min per 32 for Q4_K / Q5_K) */
      const int bs0 = absum[(size_t)(2 * b) * M_stride + m], bs1 = absum[(size_t)(2 * b + 1) * M_stride + m];
      const int mv = r->mn[2 * b] * bs0 + r->mn[2 * b + 1] * bs1;
      v = sa * (r->d[b] * (float)iv - r->dmin[b] * (float)mv);
      if (msums) msums[b] = mv;
    } else {
      v = sa * r->d[b] * (float)iv;
    }
    if (bsums) bsums[b] = iv;
    acc += (double)v;
  }
  return acc;
}

int qref_blockdot(int type, const uint8_t* W, int N, int K, const int8_t* aq, const float* asc, const int16_t* absum,
                  int M, int M_stride, float* C, int ldc, int32_t* blocksums, int32_t* minsums, int n_col_stride,
                  int nthreads) {
  const int sb = qref_sb_bytes(type);
  if (sb < 0 || K % 256 || M > M_stride || n_col_stride < 1) return -1;
  const size_t rb = (size_t)(K / 256) * sb;
  const int nb = K / 32;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    row_dec r;
    r.q = (int8_t*)malloc((size_t)K);
    r.sc = (int*)malloc(sizeof(int) * 2 * nb);
    r.mn = (int*)malloc(sizeof(int) * 2 * nb);
    r.d = (float*)malloc(sizeof(float) * nb);
    r.dmin = (float*)malloc(sizeof(float) * nb);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
    for (int n = 0; n < N; n += n_col_stride) {
      decode_row(type, W + (size_t)n * rb, K, &r);
      for (int m = 0; m < M; ++m) {
        int32_t* bs = blocksums ? blocksums + ((size_t)m * N + n) * nb : NULL;
        int32_t* ms = minsums ? minsums + ((size_t)m * N + n) * nb : NULL;
        C[(size_t)m * ldc + n] = (float)row_dot(type, &r, K, aq + (size_t)m * K, asc, absum, m, M_stride, bs, ms);
      }
    }
    free(r.q);
    free(r.sc);
    free(r.mn);
    free(r.d);
    free(r.dmin);
  }
  return 0;
}

/* tools/ref_forward.cpp:137-159 -- dequant_row, then double dot products */
int qref_matmul_f32(int type, const uint8_t* W, int N, int K, const float* X, int M, float* Y, int nthreads) {
  const int sb = qref_sb_bytes(type);
  if (sb < 0 || K % 256) return -1;
  const size_t rb = (size_t)(K / 256) * sb;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
    for (int n = 0; n < N; ++n) {
      qref_dequant_row(type, W + (size_t)n * rb, K, w);
      for (int m = 0; m < M; ++m) {
        double acc = 0.0;
        const float* x = X + (size_t)m * K;
        for (int k = 0; k < K; ++k) acc += (double)w[k] * (double)x[k];
        Y[(size_t)m * N + n] = (float)acc;
      }
    }
    free(w);
  }
  return 0;
}

/* zero/kernels/moe.cl:42-81 (moe_route): repeated arg-max over the logits (ties: the lower expert), p = exp(l - max)
 * in float, weights p / sum over the selection (sum in selection order) */
void qref_moe_route_ex(const float* logits, int ldl, int T, int NE, int NU, const float* escale, int* ids, float* wts,
                       int* counts) {
  if (counts)
    for (int e = 0; e < NE; ++e) counts[e] = 0;
  char* taken = (char*)malloc((size_t)NE);
  for (int t = 0; t < T; ++t) {
    const float* l = logits + (size_t)t * ldl;
    float mx = -INFINITY;
    for (int e = 0; e < NE; ++e) mx = fmaxf(mx, l[e]);
    memset(taken, 0, (size_t)NE);
    float p[64], sum = 0.0f;
    for (int k = 0; k < NU; ++k) {
      int bi = -1;
      for (int e = 0; e < NE; ++e)
        if (!taken[e] && (bi < 0 || l[e] > l[bi])) bi = e;
      taken[bi] = 1;
      ids[(size_t)t * NU + k] = bi;
      /* (a row whose logits are all -inf: every weight 0, the token takes no expert output) */
      p[k] = l[bi] > -INFINITY ? expf(l[bi] - mx) : 0.0f;
      sum += p[k];
      if (counts) ++counts[bi];
    }
    /* moe.cl:75-77: the normalized weight, times the expert's scale when the model has one (-DESCALE) */
    for (int k = 0; k < NU; ++k) {
      const float w = sum > 0.0f ? p[k] / sum : 0.0f;
      wts[(size_t)t * NU + k] = escale ? w * escale[ids[(size_t)t * NU + k]] : w;
    }
  }
  free(taken);
}

void qref_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts) {
  qref_moe_route_ex(logits, ldl, T, NE, NU, NULL, ids, wts, counts);
}

int qref_moe_forward_ex(int type_gate, const uint8_t* Wg, int type_up, const uint8_t* Wu, int type_down,
                        const uint8_t* Wd, int NE, int E, int F, const float* logits, int ldl, int T, int NU,
                        const int8_t* aq, const float* asc, int M_stride, const float* escale, const float* sh,
                        int ldsh, int sh_gated, float* x, int accumulate, int nthreads) {
  const int sbg = qref_sb_bytes(type_gate), sbu = qref_sb_bytes(type_up), sbd = qref_sb_bytes(type_down);
  if (sbg < 0 || sbu < 0 || sbd < 0 || E % 256 || F % 256 || NU > 64 || T > M_stride) return -1;
  /* (types with per-block mins need the activation sums, which the expert path does not carry: the reference's
   *  expert GEMMs take no min types either, zero/engine_moe.h:284-301) */
  if (type_gate == QREF_Q4_K || type_up == QREF_Q4_K || type_down == QREF_Q4_K || type_gate == QREF_Q5_K ||
      type_up == QREF_Q5_K || type_down == QREF_Q5_K || type_gate == QREF_Q2_K || type_up == QREF_Q2_K ||
      type_down == QREF_Q2_K)
    return -1;
  if (sh && sh_gated && ldl < NE + 1) return -1;
  int* ids = (int*)malloc(sizeof(int) * (size_t)T * NU);
  float* wts = (float*)malloc(sizeof(float) * (size_t)T * NU);
  qref_moe_route_ex(logits, ldl, T, NE, NU, escale, ids, wts, NULL);
  const size_t rbg = (size_t)(E / 256) * sbg, rbu = (size_t)(E / 256) * sbu, rbd = (size_t)(F / 256) * sbd;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    row_dec r;
    const int KM = E > F ? E : F;
    r.q = (int8_t*)malloc((size_t)KM);
    r.sc = (int*)malloc(sizeof(int) * KM / 16);
    r.mn = (int*)malloc(sizeof(int) * KM / 16);
    r.d = (float*)malloc(sizeof(float) * KM / 32);
    r.dmin = (float*)malloc(sizeof(float) * KM / 32);
    float* h = (float*)malloc(sizeof(float) * F);
    int8_t* hq = (int8_t*)malloc((size_t)F);
    float* hsc = (float*)malloc(sizeof(float) * F / 32);
    int16_t* hab = (int16_t*)malloc(sizeof(int16_t) * F / 16);
    float* y = (float*)malloc(sizeof(float) * (size_t)NU * E);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int t = 0; t < T; ++t) {
      for (int k = 0; k < NU; ++k) {
        const int e = ids[(size_t)t * NU + k];
        /* gate / up: h = up * silu(gate) as gemm.cl:464-471 (accumulate 2) */
        for (int f = 0; f < F; ++f) {
          decode_row(type_gate, Wg + ((size_t)e * F + f) * rbg, E, &r);
          const float g = (float)row_dot(type_gate, &r, E, aq + (size_t)t * E, asc, NULL, t, M_stride, NULL, NULL);
          decode_row(type_up, Wu + ((size_t)e * F + f) * rbu, E, &r);
          const float u = (float)row_dot(type_up, &r, E, aq + (size_t)t * E, asc, NULL, t, M_stride, NULL, NULL);
          h[f] = u * (g / (1.0f + expf(-g)));
        }
        /* moe.cl:251-282: h quantized per 32 */
        qref_quantize_act(h, 1, F, 1, 1, hq, hsc, hab);
        /* down, times the routing weight (moe.cl:327) */
        const float w = wts[(size_t)t * NU + k];
        for (int c = 0; c < E; ++c) {
          decode_row(type_down, Wd + ((size_t)e * E + c) * rbd, F, &r);
          const float v = (float)row_dot(type_down, &r, F, hq, hsc, hab, 0, 1, NULL, NULL);
          y[(size_t)k * E + c] = w * v;
        }
      }
      /* moe.cl:332-340: the token's NU outputs summed in selection order, plus the shared expert's output times
       * its gate sigmoid(logits[t][NE]) (moe.cl:37-41; without a gate: times 1) */
      const float sg = sh ? (sh_gated ? 1.0f / (1.0f + expf(-logits[(size_t)t * ldl + NE])) : 1.0f) : 0.0f;
      for (int c = 0; c < E; ++c) {
        float v = 0.0f;
        for (int k = 0; k < NU; ++k) v += y[(size_t)k * E + c];
        if (sh) {
          const float gs = sg * sh[(size_t)t * ldsh + c];
          v = v + gs;
        }
        x[(size_t)t * E + c] = accumulate ? x[(size_t)t * E + c] + v : v;
      }
    }
    free(r.q);
    free(r.sc);
    free(r.mn);
    free(r.d);
    free(r.dmin);
    free(h);
    free(hq);
    free(hsc);
    free(hab);
    free(y);
  }
  free(ids);
  free(wts);
  return 0;
}

int qref_moe_forward(int type_gate, const uint8_t* Wg, int type_up, const uint8_t* Wu, int type_down,
                     const uint8_t* Wd, int NE, int E, int F, const float* logits, int ldl, int T, int NU,
                     const int8_t* aq, const float* asc, int M_stride, float* x, int accumulate, int nthreads) {
  return qref_moe_forward_ex(type_gate, Wg, type_up, Wu, type_down, Wd, NE, E, F, logits, ldl, T, NU, aq, asc,
                             M_stride, NULL, NULL, 0, 0, x, accumulate, nthreads);
}

/* ---- activation producers: the kernels that write the path's int8 activations --------------------------------- */

static double sumsq_f64(const float* v, int K) {
  double ss = 0.0;
  for (int i = 0; i < K; ++i) ss += (double)v[i] * (double)v[i];
  return ss;
}

/* zero/kernels/ops.cl:82-104 (rmsnorm_quant, act32): y = x * r * w with r = 1 / sqrt(ss / K + eps), ss = sum of x^2
 * (accumulated in double here; the GPU kernels sum in f32, in their own order), then quantized per 32 as
 * quant_store16 (ops.cl:18-77). Rows M..M_stride-1 are zero rows (the reference's `valid` flag). h (optional, row
 * stride K) receives y, zero rows included. */
void qref_rmsnorm_quant(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps, int8_t* aq,
                        float* asc, int16_t* absum, float* h) {
  float* y = (float*)calloc((size_t)M_stride * K, sizeof(float));
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (size_t)m * ldx;
    const float ss = (float)sumsq_f64(xr, K);
    const float r = 1.0f / sqrtf(ss / (float)K + eps);
    for (int i = 0; i < K; ++i) y[(size_t)m * K + i] = xr[i] * r * w[i];
  }
  qref_quantize_act(y, M, K, M_stride, 1, aq, asc, absum);
  if (h) memcpy(h, y, sizeof(float) * (size_t)M_stride * K);
  free(y);
}

/* ops.cl:13 (silu) and 107 (gelu_tanh) */
static float silu_f(float x) { return x / (1.0f + expf(-x)); }
static float gelu_tanh_f(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

/* ops.cl:110-128 (swiglu_quant, act32): y = silu(gate) * up (gelu_tanh with `gelu`) from rows [gate(F) | up(F)], or
 * with `fused` the row itself (the GEMM already applied the activation: the engine's quant_rows, engine.h:3451-3456),
 * quantized per 32. Row stride ldg. */
void qref_swiglu_quant(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int8_t* aq,
                       float* asc, int16_t* absum, float* h) {
  float* y = (float*)calloc((size_t)M_stride * F, sizeof(float));
  for (int m = 0; m < M; ++m) {
    const float* g = gu + (size_t)m * ldg;
    for (int i = 0; i < F; ++i)
      y[(size_t)m * F + i] = fused ? g[i] : (gelu ? gelu_tanh_f(g[i]) : silu_f(g[i])) * g[F + i];
  }
  qref_quantize_act(y, M, F, M_stride, 1, aq, asc, absum);
  if (h) memcpy(h, y, sizeof(float) * (size_t)M_stride * F);
  free(y);
}

/* ops.cl:2025-2075 (add_norm_quant, act32): per row, x = (x + t * r * w) * s with r from t's mean square, written
 * back to x; then y = x * r2 * w2 (r2 from the new x's mean square) or, with w2 == NULL, y = x; y quantized per 32.
 * x and t rows have stride K. */
void qref_add_norm_quant(float* x, const float* t, const float* w, int K, float eps, float s, const float* w2, int M,
                         int M_stride, int8_t* aq, float* asc, int16_t* absum, float* h) {
  float* y = (float*)calloc((size_t)M_stride * K, sizeof(float));
  for (int m = 0; m < M; ++m) {
    float* xr = x + (size_t)m * K;
    const float* tr = t + (size_t)m * K;
    const float r = 1.0f / sqrtf((float)sumsq_f64(tr, K) / (float)K + eps);
    for (int i = 0; i < K; ++i) xr[i] = (xr[i] + tr[i] * r * w[i]) * s;
    const float r2 = w2 ? 1.0f / sqrtf((float)sumsq_f64(xr, K) / (float)K + eps) : 1.0f;
    for (int i = 0; i < K; ++i) y[(size_t)m * K + i] = w2 ? xr[i] * r2 * w2[i] : xr[i];
  }
  qref_quantize_act(y, M, K, M_stride, 1, aq, asc, absum);
  if (h) memcpy(h, y, sizeof(float) * (size_t)M_stride * K);
  free(y);
}
