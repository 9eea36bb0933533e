// Weight preparation (GGUF -> prepared planes) and the per-32 activation quantizer.
#include "qm_launch.h"

namespace qm {

// ---------------------------------------------------------------------------------------------------------------
// One thread per (row, superblock): reads the GGUF superblock bytewise (any alignment) and writes its payload and
// header into the two planes (layout in qm_device.h). Follows the field offsets of src/quants.h:89-315.
// kraw: 32-blocks per raw row. It is K / 32 except for the types of 32-element blocks (Q8_0, Q4_0, IQ4_NL) whose rows
// are not whole superblocks: those are padded to K = the next multiple of 256 with zero blocks (scale 0, so every
// padded element decodes to 0), as the reference's pad_small_block_rows / load_w_pad do (src/quants.h:581-595;
// zero/engine.h:2102-2116).
template <int TYPE>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ raw, int rows, int K, int kraw,
                                                     uint8_t* __restrict__ qs, uint8_t* __restrict__ hdr) {
  using Tr = Traits<TYPE>;
  const int nsb = K / 256;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * nsb) return;
  const long n = i / nsb;
  const int s = (int)(i % nsb);
  // (the small-block types: raw rows of kraw blocks of Tr::GGUF_SB / 8 bytes; the others: rows of nsb superblocks)
  constexpr bool small = TYPE == T_Q8_0 || TYPE == T_Q4_0 || TYPE == T_IQ4_NL || TYPE == T_Q2_0;
  const size_t row_bytes = small ? (size_t)kraw * (Tr::GGUF_SB / 8) : (size_t)nsb * Tr::GGUF_SB;
  const uint8_t* p = raw + (size_t)n * row_bytes + (size_t)s * Tr::GGUF_SB;
  const int nblk = min(8, kraw - 8 * s);  // blocks of this superblock present in the raw row
  (void)nblk;
  uint8_t* q = qs + ((size_t)n * (K / 32) + (size_t)s * 8) * Tr::QB;
  uint8_t* h = hdr + ((size_t)n * nsb + s) * Tr::HB;
  if constexpr (TYPE == T_Q8_0) {
    // 8 GGUF blocks of (f16 d, int8 q[32])
    for (int b = 0; b < 8; ++b) {
      const bool in = b < nblk;
      h[2 * b] = in ? p[34 * b] : 0;
      h[2 * b + 1] = in ? p[34 * b + 1] : 0;
      for (int e = 0; e < 32; ++e) q[32 * b + e] = in ? p[34 * b + 2 + e] : 0;
    }
  } else if constexpr (TYPE == T_Q4_K) {
    // d, dmin, scales[12] | qs[128]: chunk j (64 elements) = qs[32j..32j+31], low nibbles elements 0..31 of the
    // chunk, high nibbles 32..63. Block 2j takes the low nibbles, 2j+1 the high ones; within a block byte t holds
    // elements t (low nibble) and 16 + t (high nibble).
    for (int e = 0; e < 16; ++e) h[e] = p[e];
    const uint8_t* src = p + 16;
    for (int j = 0; j < 4; ++j)
      for (int t = 0; t < 16; ++t) {
        const uint8_t a = src[32 * j + t], c = src[32 * j + 16 + t];
        q[16 * (2 * j) + t] = (uint8_t)((a & 0xF) | ((c & 0xF) << 4));
        q[16 * (2 * j + 1) + t] = (uint8_t)((a >> 4) | ((c >> 4) << 4));
      }
  } else if constexpr (TYPE == T_IQ4_XS) {
    // d, scales_h, scales_l[4] | qs[128] (block ib = qs[16 ib .. 16 ib + 15], already per-32); scales_h is stored
    // with bit 1 of each 2-bit field flipped (0xAAAA), which makes the field a signed (high bits - 2)
    for (int e = 0; e < 8; ++e) h[e] = p[e];
    h[2] ^= 0xAA;
    h[3] ^= 0xAA;
    for (int e = 0; e < 128; ++e) q[e] = p[8 + e];
  } else if constexpr (TYPE == T_Q5_K) {
    // d, dmin, scales[12] | qh[32] | qs[128] (src/quants.h:91-114): chunk j's low / high nibbles are blocks 2j / 2j+1,
    // their fifth bits bit 2j / 2j+1 of qh[l]
    for (int e = 0; e < 16; ++e) h[e] = p[e];
    const uint8_t *qh = p + 16, *src = p + 48;
    for (int j = 0; j < 4; ++j)
      for (int half = 0; half < 2; ++half) {
        const int b = 2 * j + half;
        uint8_t* dst = q + 20 * b;
        uint8_t n[32], hb[32];
        for (int l = 0; l < 32; ++l) {
          n[l] = half ? (uint8_t)(src[32 * j + l] >> 4) : (uint8_t)(src[32 * j + l] & 0xF);
          hb[l] = (uint8_t)((qh[l] >> b) & 1);
        }
        for (int hh = 0; hh < 2; ++hh)
          for (int t = 0; t < 8; ++t) dst[8 * hh + t] = (uint8_t)(n[16 * hh + t] | (n[16 * hh + 8 + t] << 4));
        for (int i = 0; i < 4; ++i) {
          uint8_t v = 0;
          for (int k = 0; k < 4; ++k) v |= (uint8_t)((hb[4 * k + i] << k) | (hb[16 + 4 * k + i] << (4 + k)));
          dst[16 + i] = v;
        }
      }
  } else if constexpr (TYPE == T_Q4_0 || TYPE == T_IQ4_NL) {
    // 8 GGUF blocks of (f16 d, 16 nibble bytes)
    for (int b = 0; b < 8; ++b) {
      const bool in = b < nblk;
      h[2 * b] = in ? p[18 * b] : 0;
      h[2 * b + 1] = in ? p[18 * b + 1] : 0;
      for (int t = 0; t < 16; ++t) q[16 * b + t] = in ? p[18 * b + 2 + t] : 0;
    }
  } else if constexpr (TYPE == T_Q2_0) {
    // 4 GGUF blocks of (f16 d, 16 code bytes: element e of the 64 in bits 2 (e % 4) of byte e / 4), value (code - 1) d
    // (src/quants.h:540-548; decode.cl:248-256); 32-block b is half b % 2 of block b / 2. Blocks past the raw row
    // stay all zero (scale 0), as pad_small_block_rows writes them.
    for (int t = 0; t < 8 * Tr::QB; ++t) q[t] = 0;
    for (int g = 0; g < 4; ++g) {
      const bool in = 2 * g < nblk;
      h[2 * g] = in ? p[18 * g] : 0;
      h[2 * g + 1] = in ? p[18 * g + 1] : 0;
      if (!in) continue;
      for (int hb = 0; hb < 2; ++hb) {
        uint8_t* dst = q + Tr::QB * (2 * g + hb);
        for (int e = 0; e < 32; ++e) {
          const int E = 32 * hb + e, k = e >> 2, i = e & 3;
          const int c = (p[18 * g + 2 + E / 4] >> (2 * (E % 4))) & 3;
          dst[4 * (k >> 2) + i] |= (uint8_t)(c << (2 * (k & 3)));
        }
      }
    }
  } else if constexpr (TYPE == T_IQ1_S) {
    // d | qs[32] | qh[8] (u16 per 32-block) (src/quants.h:263-276; decode.cl:326-345): block ib's payload = its 4 grid
    // index low bytes and its qh
    for (int ib = 0; ib < 8; ++ib) {
      for (int e = 0; e < 4; ++e) q[8 * ib + e] = p[2 + 4 * ib + e];
      q[8 * ib + 4] = p[34 + 2 * ib];
      q[8 * ib + 5] = p[34 + 2 * ib + 1];
      q[8 * ib + 6] = 0;
      q[8 * ib + 7] = 0;
    }
    h[0] = p[0];
    h[1] = p[1];
    h[2] = 0;
    h[3] = 0;
  } else if constexpr (TYPE == T_IQ1_M) {
    // qs[32] | qh[16] | scales (4 u16) (src/quants.h:277-296; decode.cl:346-366): block ib's payload = its 4 grid index
    // low bytes, qh[2 ib], qh[2 ib + 1] and its two 3-bit scales (bits 6 (ib % 2) .. + 5 of scale word ib / 2); the
    // f16 d is the top nibbles of the four scale words
    const uint8_t *qs = p, *qh = p + 32, *sw = p + 48;
    uint32_t w4[4];
    for (int i = 0; i < 4; ++i) w4[i] = (uint32_t)sw[2 * i] | ((uint32_t)sw[2 * i + 1] << 8);
    for (int ib = 0; ib < 8; ++ib) {
      for (int e = 0; e < 4; ++e) q[8 * ib + e] = qs[4 * ib + e];
      q[8 * ib + 4] = qh[2 * ib];
      q[8 * ib + 5] = qh[2 * ib + 1];
      q[8 * ib + 6] = (uint8_t)((w4[ib >> 1] >> (6 * (ib & 1))) & 0x3Fu);
      q[8 * ib + 7] = 0;
    }
    const uint32_t su = (w4[0] >> 12) | ((w4[1] >> 8) & 0x00F0u) | ((w4[2] >> 4) & 0x0F00u) | (w4[3] & 0xF000u);
    h[0] = (uint8_t)(su & 0xFF);
    h[1] = (uint8_t)(su >> 8);
    h[2] = 0;
    h[3] = 0;
  } else if constexpr (TYPE == T_Q2_K) {
    // scales[16] (scale low nibble, min high nibble, per 16) | qs[64] | d | dmin (src/quants.h:159-169; decode.cl:151-160):
    // element e of 32-block ib has the value (qs[32 (ib / 4) + e] >> 2 (ib % 4)) & 3
    const uint8_t* qs = p + 16;
    for (int t = 0; t < 8 * Tr::QB; ++t) q[t] = 0;
    for (int ib = 0; ib < 8; ++ib) {
      uint8_t* dst = q + Tr::QB * ib;
      for (int e = 0; e < 32; ++e) {
        const int v = (qs[32 * (ib >> 2) + e] >> (2 * (ib & 3))) & 3, k = e >> 2, i = e & 3;
        dst[4 * (k >> 2) + i] |= (uint8_t)(v << (2 * (k & 3)));
      }
    }
    h[0] = p[80];
    h[1] = p[81];
    h[2] = p[82];
    h[3] = p[83];
    for (int i = 0; i < 16; ++i) h[4 + i] = p[i];
  } else if constexpr (TYPE == T_Q3_K) {
    // hmask[32] | qs[64] | scales[12] | d (src/quants.h:465-494; decode.cl:162-176): element e of 32-block ib has the
    // low 2 bits (qs[32 (ib / 4) + e] >> 2 (ib % 4)) & 3 and the high bit (hmask[e] >> ib) & 1, value (low | high << 2)
    // - 4; scale i of 16 elements: low 4 bits from scales[i % 8] (nibble i / 8), top 2 bits from scales[8 + i % 4]
    // (bits 2 (i / 4)), minus 32
    const uint8_t *hm = p, *qs = p + 32, *sc = p + 96;
    for (int t = 0; t < 8 * Tr::QB; ++t) q[t] = 0;
    for (int ib = 0; ib < 8; ++ib) {
      uint8_t* dst = q + Tr::QB * ib;
      for (int e = 0; e < 32; ++e) {
        const int lo = (qs[32 * (ib >> 2) + e] >> (2 * (ib & 3))) & 3, hi = (hm[e] >> ib) & 1;
        const int k = e >> 2, i = e & 3;
        dst[4 * (k >> 2) + i] |= (uint8_t)(lo << (2 * (k & 3)));
        dst[8 + i] |= (uint8_t)(hi << k);
      }
    }
    for (int i = 0; i < 16; ++i) {
      const int v = ((sc[i & 7] >> (4 * (i >> 3))) & 0xF) | (((sc[8 + (i & 3)] >> (2 * (i >> 2))) & 3) << 4);
      h[i] = (uint8_t)(v - 32);
    }
    h[16] = p[108];
    h[17] = p[109];
    h[18] = 0;
    h[19] = 0;
  } else if constexpr (TYPE == T_Q6_K) {
    // ql[128] | qh[64] | scales[16] | d (src/quants.h:115-135): element 128n + 32c + l has its low 4 bits in
    // ql[64n + l + 32 (c & 1)] (nibble c >> 1) and its high 2 bits in qh[32n + l] (bits 2c..2c+1); block b = 4n + c
    const uint8_t *ql = p, *qh = p + 128;
    for (int b = 0; b < 8; ++b) {
      const int n2 = b >> 2, c = b & 3;
      uint8_t lo4[32], hi2[32];
      for (int l = 0; l < 32; ++l) {
        lo4[l] = (uint8_t)((ql[64 * n2 + l + 32 * (c & 1)] >> (4 * (c >> 1))) & 0xF);
        hi2[l] = (uint8_t)((qh[32 * n2 + l] >> (2 * c)) & 3);
      }
      uint8_t* dst = q + 24 * b;
      for (int t = 0; t < 16; ++t) dst[t] = (uint8_t)(lo4[t] | (lo4[16 + t] << 4));
      for (int hw = 0; hw < 2; ++hw)
        for (int i = 0; i < 4; ++i) {
          uint8_t v = 0;
          for (int k = 0; k < 4; ++k) v |= (uint8_t)(hi2[16 * hw + 4 * k + i] << (2 * k));
          dst[16 + 4 * hw + i] = v;
        }
    }
    for (int e = 0; e < 16; ++e) h[e] = p[192 + e];
    h[16] = p[208];
    h[17] = p[209];
    h[18] = 0;
    h[19] = 0;
  } else if constexpr (TYPE == T_IQ2_XXS || TYPE == T_IQ2_XS) {
    // d | 8 blocks of 8 bytes (IQ2_XXS: a0, a1; IQ2_XS: four u16) [| IQ2_XS scales[8]]
    for (int e = 0; e < 64; ++e) q[e] = p[2 + e];
    if constexpr (TYPE == T_IQ2_XS) {
      for (int e = 0; e < 8; ++e) h[e] = p[66 + e];
      h[8] = p[0];
      h[9] = p[1];
      h[10] = 0;
      h[11] = 0;
    } else {
      h[0] = p[0];
      h[1] = p[1];
      h[2] = 0;
      h[3] = 0;
    }
  } else if constexpr (TYPE == T_IQ2_S) {
    // d | qs[32] | signs[32] | qh[8] | scales[8]
    for (int b = 0; b < 8; ++b)
      for (int e = 0; e < 4; ++e) {
        q[8 * b + e] = p[2 + 4 * b + e];
        q[8 * b + 4 + e] = p[34 + 4 * b + e];
      }
    for (int e = 0; e < 16; ++e) h[e] = p[66 + e];
    h[16] = p[0];
    h[17] = p[1];
    h[18] = 0;
    h[19] = 0;
  } else if constexpr (TYPE == T_IQ3_XXS) {
    // d | qs[64] | 8 sign/scale words
    for (int b = 0; b < 8; ++b) {
      for (int e = 0; e < 8; ++e) q[12 * b + e] = p[2 + 8 * b + e];
      for (int e = 0; e < 4; ++e) q[12 * b + 8 + e] = p[66 + 4 * b + e];
    }
    h[0] = p[0];
    h[1] = p[1];
    h[2] = 0;
    h[3] = 0;
  } else {  // IQ3_S: d | qs[64] | qh[8] | signs[32] | scales[4]
    for (int b = 0; b < 8; ++b) {
      for (int e = 0; e < 8; ++e) q[12 * b + e] = p[2 + 8 * b + e];
      for (int e = 0; e < 4; ++e) q[12 * b + 8 + e] = p[74 + 4 * b + e];
    }
    for (int e = 0; e < 8; ++e) h[e] = p[66 + e];
    for (int e = 0; e < 4; ++e) h[8 + e] = p[106 + e];
    h[12] = p[0];
    h[13] = p[1];
    h[14] = 0;
    h[15] = 0;
  }
}

hipError_t launch_repack(int type, const uint8_t* raw, int rows, int K, int kraw, uint8_t* qs, uint8_t* hdr,
                         hipStream_t s) {
  const long n = (long)rows * (K / 256);
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  switch (type) {
    case T_Q8_0: repack_kernel<T_Q8_0><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q4_K: repack_kernel<T_Q4_K><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ4_XS: repack_kernel<T_IQ4_XS><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ3_S: repack_kernel<T_IQ3_S><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q6_K: repack_kernel<T_Q6_K><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q3_K: repack_kernel<T_Q3_K><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q2_K: repack_kernel<T_Q2_K><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ1_S: repack_kernel<T_IQ1_S><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ1_M: repack_kernel<T_IQ1_M><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q2_0: repack_kernel<T_Q2_0><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q5_K: repack_kernel<T_Q5_K><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_Q4_0: repack_kernel<T_Q4_0><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ4_NL: repack_kernel<T_IQ4_NL><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ2_XXS: repack_kernel<T_IQ2_XXS><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ2_XS: repack_kernel<T_IQ2_XS><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ2_S: repack_kernel<T_IQ2_S><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    case T_IQ3_XXS: repack_kernel<T_IQ3_XXS><<<grid, block, 0, s>>>(raw, rows, K, kraw, qs, hdr); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Activation quantizer: 8 lanes per 32-block, 4 values per lane. amax is combined over the 8 lanes (max is
// order-free), then each value is rounded on its own: q = rint(v * (127 / amax)) with IEEE division and
// round-half-even, the expression of quantize_act_cpu (src/quants.h:559-576) -- bit-exact. Rows m >= M (up to
// M_stride) are written as zero rows with scale 0. A32 = false: one scale per 256 values (quantize_act_cpu with
// act32 = false, asc [K/256][M_stride]); a superblock's 64 lanes are one whole wave (K % 256 == 0), so amax is the
// wave maximum.
template <bool A32>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ x, int ldx, int M, int M_stride,
                                                       int K, int8_t* __restrict__ aq, float* __restrict__ asc,
                                                       int16_t* __restrict__ absum) {
  const int nb = K / 32;
  const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;  // one lane = 4 values
  const long blk = g >> 3;
  const int sub = (int)(g & 7);
  const bool live = blk < (long)M_stride * nb;
  const int m = live ? (int)(blk / nb) : 0;
  const int b = live ? (int)(blk % nb) : 0;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (live && m < M) {
    const float* src = x + (size_t)m * ldx + 32 * b + 4 * sub;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = src[i];
  }
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = A32 ? max8(amax) : wave_max(amax);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int sum = 0;
  uint32_t pk = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = (int)__builtin_rintf(v[i] * inv);
    sum += q;
    pk |= (uint32_t)(q & 0xFF) << (8 * i);
  }
  sum = sum4_i(sum);
  if (!live) return;
  *(uint32_t*)(aq + (size_t)m * K + 32 * b + 4 * sub) = pk;
  if (A32 ? sub == 0 : (sub == 0 && (b & 7) == 0)) asc[(size_t)(A32 ? b : b >> 3) * M_stride + m] = amax / 127.0f;
  if ((sub & 3) == 0) absum[(size_t)(2 * b + (sub >> 2)) * M_stride + m] = (int16_t)sum;
}

hipError_t launch_quantize(const float* x, int ldx, int M, int M_stride, int K, bool act32, int8_t* aq, float* asc,
                           int16_t* absum, hipStream_t s) {
  const long lanes = (long)M_stride * (K / 32) * 8;
  const dim3 grid((unsigned)((lanes + 255) / 256)), block(256);
  if (act32) quantize_kernel<true><<<grid, block, 0, s>>>(x, ldx, M, M_stride, K, aq, asc, absum);
  else quantize_kernel<false><<<grid, block, 0, s>>>(x, ldx, M, M_stride, K, aq, asc, absum);
  return hipGetLastError();
}

}  // namespace qm
