// Per-lane decode of one 32-block of a prepared weight row into int8 words, shared by the decode GEMVs and the
// MoE decode kernels.
#pragma once
#include "qm_launch.h"

namespace qm {

template <int TYPE> struct LdsFor { struct type { int unused; }; };
template <> struct LdsFor<T_IQ3_S> { using type = Iq3Lds; };
template <> struct LdsFor<T_IQ2_XXS> { using type = IqLds<T_IQ2_XXS>; };
template <> struct LdsFor<T_IQ2_XS> { using type = IqLds<T_IQ2_XS>; };
template <> struct LdsFor<T_IQ2_S> { using type = IqLds<T_IQ2_S>; };
template <> struct LdsFor<T_IQ3_XXS> { using type = IqLds<T_IQ3_XXS>; };
template <> struct LdsFor<T_IQ1_S> { using type = Iq1Lds; };
template <> struct LdsFor<T_IQ1_M> { using type = Iq1Lds; };

// Fills a work-group's LDS tables for TYPE (nothing for the types without codebooks in LDS); the caller
// synchronizes before use.
template <int TYPE>
__device__ __forceinline__ void lds_fill(typename LdsFor<TYPE>::type* t) {
  if constexpr (TYPE == T_IQ3_S) iq3_lds_fill(t);
  else if constexpr (kIq2<TYPE>) iq_lds_fill<TYPE>(t);
  else if constexpr (kIq1<TYPE>) iq1_lds_fill(t);
}

// The raw bytes a lane needs for 32-block b of row n: payload (q0; Q8_0, Q5_K and Q6_K also q1) and header (h).
// (native vector members: arrays of structs holding HIP's uint4 are kept in scratch memory)
struct RawBlk {
  u32x4_t q0, q1, h;
};

// qrow / hrow: the row's payload and header planes; b: the block
template <int TYPE>
__device__ __forceinline__ RawBlk load_block_at(const uint8_t* qrow, const uint8_t* hrow, int b) {
  using Tr = Traits<TYPE>;
  const uint8_t* qp = qrow + (uint32_t)(b * Tr::QB);
  const uint8_t* hp = hrow + (uint32_t)((b >> 3) * Tr::HB);
  RawBlk r;
  r.q1 = u32x4_t{0u, 0u, 0u, 0u};
  r.h = u32x4_t{0u, 0u, 0u, 0u};
  if constexpr (TYPE == T_Q8_0) {
    r.q0 = ld_stream16(qp);
    r.q1 = ld_stream16(qp + 16);
    r.h.x = ((const uint16_t*)hp)[b & 7];
  } else if constexpr (TYPE == T_Q4_0 || TYPE == T_IQ4_NL) {
    r.q0 = ld_stream16(qp);
    r.h.x = ((const uint16_t*)hp)[b & 7];
  } else if constexpr (kIq1<TYPE>) {
    const uint32_t* q = (const uint32_t*)qp;
    r.q0 = u32x4_t{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1), 0u, 0u};
    r.h.x = *(const uint32_t*)hp;  // f16 d
  } else if constexpr (TYPE == T_Q2_0 || TYPE == T_Q2_K) {
    const uint32_t* q = (const uint32_t*)qp;
    r.q0 = u32x4_t{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1), 0u, 0u};
    if constexpr (TYPE == T_Q2_0) {
      r.h.x = ((const uint16_t*)hp)[block_scale_slot<TYPE>(b & 7)];
    } else {
      r.h.x = *(const uint32_t*)hp;                  // d, dmin
      r.h.y = ((const uint16_t*)(hp + 4))[b & 7];   // the block's two scale / min bytes
    }
  } else if constexpr (TYPE == T_Q3_K) {
    const uint32_t* q = (const uint32_t*)qp;
    r.q0 = u32x4_t{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1), __builtin_nontemporal_load(q + 2),
                   0u};
    r.h.x = ((const uint16_t*)hp)[b & 7];  // the block's two int8 scales
    r.h.y = ((const uint16_t*)hp)[8];      // f16 d
  } else if constexpr (TYPE == T_Q5_K) {
    r.q0 = ld_stream16(qp);
    r.q1.x = __builtin_nontemporal_load((const uint32_t*)(qp + 16));
    r.h = *(const u32x4_t*)hp;
  } else if constexpr (TYPE == T_Q6_K) {
    r.q0 = ld_stream16(qp);
    const uint32_t* q = (const uint32_t*)(qp + 16);
    r.q1.x = __builtin_nontemporal_load(q);
    r.q1.y = __builtin_nontemporal_load(q + 1);
    r.h.x = ((const uint16_t*)hp)[b & 7];  // the block's two int8 scales
    r.h.y = ((const uint16_t*)hp)[8];      // f16 d
  } else if constexpr (kIq2<TYPE>) {
    // (payload words q0.x..z; header: IQ2_XS scales in h.x, h.y and d in h.z, IQ2_S qh in h.x, h.y, scales in
    //  h.z, h.w and d in q1.x, the others d in h.x)
    const uint32_t* q = (const uint32_t*)qp;
    r.q0 = u32x4_t{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1),
                   TYPE == T_IQ3_XXS ? __builtin_nontemporal_load(q + 2) : 0u, 0u};
    const uint32_t* hw = (const uint32_t*)hp;
    if constexpr (TYPE == T_IQ2_XS) {
      r.h.x = hw[0];
      r.h.y = hw[1];
      r.h.z = hw[2];
    } else if constexpr (TYPE == T_IQ2_S) {
      r.h = *(const u32x4_t*)hp;
      r.q1.x = hw[4];
    } else {
      r.h.x = hw[0];
    }
  } else if constexpr (TYPE == T_IQ3_S) {
    const uint32_t* q = (const uint32_t*)qp;
    r.q0 = u32x4_t{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1), __builtin_nontemporal_load(q + 2),
                   0u};
    r.h = *(const u32x4_t*)hp;
  } else {
    r.q0 = ld_stream16(qp);
    if constexpr (TYPE == T_IQ4_XS) {
      const uint2 h = *(const uint2*)hp;
      r.h.x = h.x;
      r.h.y = h.y;
    } else {
      r.h = *(const u32x4_t*)hp;
    }
  }
  return r;
}

template <int TYPE>
__device__ __forceinline__ RawBlk load_block(const WView& w, int n, int b) {
  using Tr = Traits<TYPE>;
  return load_block_at<TYPE>(w.qs + (size_t)n * (w.K / 32) * Tr::QB, w.hdr + (size_t)n * (w.K / 256) * Tr::HB, b);
}

// x >> 4 as one 64-bit shift (the compiler would split it into two 32-bit shifts where only masked bits differ)
__device__ __forceinline__ uint64_t shr64_4(uint64_t x) {
  uint64_t r;
  asm("v_lshrrev_b64 %0, 4, %1" : "=v"(r) : "v"(x));
  return r;
}

// Decodes a loaded 32-block (index ib = b % 8 in its superblock): w[k] = elements 4k..4k+3 (int8x4), the integer
// scales sc (elements 0-15) and sc1 (16-31; = sc except Q6_K, Q3_K, Q2_K, IQ2_XS and IQ2_S), the min mn (Q2_K: the
// first half's min | the second's << 16), the float scales d (and dmin). Q6_K's values come out as the stored 6-bit
// numbers 0..63 (the offset of 32 is removed by block_product).
template <int TYPE>
__device__ __forceinline__ void decode_block32(const RawBlk& r, const typename LdsFor<TYPE>::type* lds, int ib,
                                               const KvTab& kv, uint32_t wd[8], int& sc, int& sc1, int& mn,
                                               float& d, float& dmin) {
  mn = 0;
  dmin = 0.0f;
  if constexpr (TYPE == T_Q6_K) {
    const uint32_t qq[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
    const uint32_t A = r.q1.x, B = r.q1.y;  // high 2 bits of elements 0-15 / 16-31: byte i, bits 2k = element 4k+i
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t ha = k < 2 ? A << (4 - 2 * k) : A >> (2 * k - 4);
      const uint32_t hb = k < 2 ? B << (4 - 2 * k) : B >> (2 * k - 4);
      wd[k] = (qq[k] & 0x0F0F0F0Fu) | (ha & 0x30303030u);
      wd[4 + k] = ((qq[k] >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u);
    }
    sc = (int)(int8_t)(r.h.x & 0xFFu);
    sc1 = (int)(int8_t)((r.h.x >> 8) & 0xFFu);
    d = h2f(r.h.y);
    return;
  }
  if constexpr (TYPE == T_Q3_K) {
#pragma unroll
    for (int k = 0; k < 8; ++k) wd[k] = q3_word(r.q0.x, r.q0.y, r.q0.z, k);
    sc = (int)(int8_t)(r.h.x & 0xFFu);
    sc1 = (int)(int8_t)((r.h.x >> 8) & 0xFFu);
    d = h2f(r.h.y);
    return;
  }
  if constexpr (kIq1<TYPE>) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint32_t idx;
      bool neg;
      iq1_index<TYPE>(r.q0.x, r.q0.y, l, idx, neg);
      iq1_group(lds, idx, neg, wd[2 * l], wd[2 * l + 1]);
    }
    if constexpr (TYPE == T_IQ1_S) {
      sc = sc1 = 2 * (int)((r.q0.y >> 12) & 7u) + 1;
    } else {
      sc = 2 * (int)((r.q0.y >> 16) & 7u) + 1;
      sc1 = 2 * (int)((r.q0.y >> 19) & 7u) + 1;
    }
    d = h2f(r.h.x) * 0.125f;
    return;
  }
  if constexpr (TYPE == T_Q2_K) {
    // values 0..3 as stored; per 16: scale (low nibble) and min (high nibble); mn holds both halves' mins
#pragma unroll
    for (int k = 0; k < 8; ++k) wd[k] = ((k < 4 ? r.q0.x : r.q0.y) >> (2 * (k & 3))) & 0x03030303u;
    sc = (int)(r.h.y & 0xFu);
    sc1 = (int)((r.h.y >> 8) & 0xFu);
    mn = (int)((r.h.y >> 4) & 0xFu) | (int)(((r.h.y >> 12) & 0xFu) << 16);
    d = h2f(r.h.x);
    dmin = h2f(r.h.x >> 16);
    return;
  }
  if constexpr (TYPE == T_Q2_0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) wd[k] = q2_word(r.q0.x, r.q0.y, k);
    d = h2f(r.h.x);
    sc = 1;
  } else if constexpr (TYPE == T_Q8_0) {
    wd[0] = r.q0.x; wd[1] = r.q0.y; wd[2] = r.q0.z; wd[3] = r.q0.w;
    wd[4] = r.q1.x; wd[5] = r.q1.y; wd[6] = r.q1.z; wd[7] = r.q1.w;
    d = h2f(r.h.x);
    sc = 1;
  } else if constexpr (TYPE == T_Q4_0 || TYPE == T_IQ4_NL) {
    const uint32_t qq[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (TYPE == T_Q4_0) {
        wd[k] = sub8_bytes(qq[k] & 0x0F0F0F0Fu);
        wd[4 + k] = sub8_bytes((qq[k] >> 4) & 0x0F0F0F0Fu);
      } else {
        wd[k] = kv_lookup4(kv, qq[k] & 0x0F0F0F0Fu);
        wd[4 + k] = kv_lookup4(kv, (qq[k] >> 4) & 0x0F0F0F0Fu);
      }
    }
    d = h2f(r.h.x);
    sc = 1;
  } else if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
    const uint32_t qq[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
    if constexpr (TYPE == T_Q4_K) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wd[k] = qq[k] & 0x0F0F0F0Fu;
        wd[4 + k] = (qq[k] >> 4) & 0x0F0F0F0Fu;
      }
    } else {
      // half h's 16 nibbles in words 2h, 2h+1 (low nibbles: its elements 0-7, high: 8-15), fifth bits in q1.x
      wd[0] = r.q0.x & 0x0F0F0F0Fu;
      wd[1] = r.q0.y & 0x0F0F0F0Fu;
      wd[2] = (r.q0.x >> 4) & 0x0F0F0F0Fu;
      wd[3] = (r.q0.y >> 4) & 0x0F0F0F0Fu;
      wd[4] = r.q0.z & 0x0F0F0F0Fu;
      wd[5] = r.q0.w & 0x0F0F0F0Fu;
      wd[6] = (r.q0.z >> 4) & 0x0F0F0F0Fu;
      wd[7] = (r.q0.w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wd[k] |= ((r.q1.x >> k) & 0x01010101u) << 4;
        wd[4 + k] |= ((r.q1.x >> (4 + k)) & 0x01010101u) << 4;
      }
    }
    d = h2f(r.h.x);
    dmin = h2f(r.h.x >> 16);
    q4k_scale_min(r.h.y, r.h.z, r.h.w, ib, sc, mn);
  } else if constexpr (TYPE == T_IQ4_XS) {
    const uint32_t qq[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
    // high nibbles: one 64-bit shift serves two words (the bits shifted in from the upper word land in the masked-out
    // top nibble)
    const uint64_t s01 = shr64_4((uint64_t)r.q0.y << 32 | r.q0.x), s23 = shr64_4((uint64_t)r.q0.w << 32 | r.q0.z);
    const uint32_t qh[4] = {(uint32_t)s01, (uint32_t)(s01 >> 32), (uint32_t)s23, (uint32_t)(s23 >> 32)};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wd[k] = kv_lookup4(kv, qq[k] & 0x0F0F0F0Fu);
      wd[4 + k] = kv_lookup4(kv, qh[k] & 0x0F0F0F0Fu);
    }
    d = h2f(r.h.x);
    sc = iq4xs_scale(r.h.x, r.h.y, ib);
  } else if constexpr (TYPE == T_IQ3_S) {
    const uint32_t qh = ((ib < 4 ? r.h.x : r.h.y) >> (8 * (ib & 3))) & 0xFFu;
    iq3s_pair<0>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[0], wd[1]);
    iq3s_pair<1>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[2], wd[3]);
    iq3s_pair<2>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[4], wd[5]);
    iq3s_pair<3>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[6], wd[7]);
    sc = 1 + 2 * (int)((r.h.z >> (4 * ib)) & 0xFu);
    d = h2f(r.h.w);
  } else if constexpr (kIq2<TYPE>) {
    const uint32_t qh = TYPE == T_IQ2_S ? ((ib < 4 ? r.h.x : r.h.y) >> (8 * (ib & 3))) & 0xFFu : 0u;
#pragma unroll
    for (int l = 0; l < 4; ++l) iq_group<TYPE>(lds, r.q0.x, r.q0.y, r.q0.z, qh, l, wd[2 * l], wd[2 * l + 1]);
    if constexpr (Traits<TYPE>::SPLIT) {
      const uint32_t sb = TYPE == T_IQ2_XS ? (((ib < 4 ? r.h.x : r.h.y) >> (8 * (ib & 3))) & 0xFFu)
                                           : (((ib < 4 ? r.h.z : r.h.w) >> (8 * (ib & 3))) & 0xFFu);
      sc = 1 + 2 * (int)(sb & 0xFu);
      sc1 = 1 + 2 * (int)(sb >> 4);
      d = h2f(TYPE == T_IQ2_XS ? r.h.z : r.q1.x) * kIqDScale<TYPE>;
      return;
    }
    sc = 1 + 2 * (int)((TYPE == T_IQ2_XXS ? r.q0.y : r.q0.z) >> 28);
    d = h2f(r.h.x) * kIqDScale<TYPE>;
  }
  sc1 = sc;
}

// One 32-block's integer products with one token's int8 activations (x0: elements 0-15, x1: 16-31; bs0 / bs1 their
// per-16 sums, used by Q4_K, Q5_K and Q6_K): iv = sc0 * lo + sc1 * hi over the signed quants and, for Q4_K / Q5_K,
// the min term
// mv = mn * (bs0 + bs1) -- the reference's per-block integers (zero/kernels/decode.cl:695-706). Q6_K's stored
// values q carry an offset of 32: sum a * (q - 32) = lo - 32 * bs.
struct BlockInts {
  int iv, mv;
  float d, dmin;
};

// iv / mv of decoded words wd with one token (see BlockInts); d / dmin are left to the caller
template <int TYPE>
__device__ __forceinline__ void block_dot(const uint32_t wd[8], int sc, int sc1, int mn, const uint4& x0,
                                          const uint4& x1, int bs0, int bs1, int& iv, int& mv) {
  if constexpr (kMin16<TYPE>) mv = __mul24(mn & 0xFFFF, bs0) + __mul24(mn >> 16, bs1);
  else mv = Traits<TYPE>::MINS ? __mul24(mn, bs0 + bs1) : 0;
  if constexpr (!Traits<TYPE>::SC16 && !Traits<TYPE>::SPLIT) {
    // one integer scale per 32-block: a single chain of 8 dot products
    int sum = dot4(x0.x, wd[0], 0);
    sum = dot4(x0.y, wd[1], sum);
    sum = dot4(x0.z, wd[2], sum);
    sum = dot4(x0.w, wd[3], sum);
    sum = dot4(x1.x, wd[4], sum);
    sum = dot4(x1.y, wd[5], sum);
    sum = dot4(x1.z, wd[6], sum);
    sum = dot4(x1.w, wd[7], sum);
    iv = kBlockScales<TYPE> ? sum : __mul24(sc, sum);
    return;
  }
  int lo = dot4(x0.x, wd[0], 0);
  lo = dot4(x0.y, wd[1], lo);
  lo = dot4(x0.z, wd[2], lo);
  lo = dot4(x0.w, wd[3], lo);
  int hi = dot4(x1.x, wd[4], 0);
  hi = dot4(x1.y, wd[5], hi);
  hi = dot4(x1.z, wd[6], hi);
  hi = dot4(x1.w, wd[7], hi);
  if constexpr (Traits<TYPE>::SC16) {
    // (|lo - 32 bs| < 2^17 and |sc| < 2^7: the 24-bit multiplies are exact)
    iv = __mul24(sc, lo - 32 * bs0) + __mul24(sc1, hi - 32 * bs1);
  } else if constexpr (Traits<TYPE>::SPLIT) {
    iv = __mul24(sc, lo) + __mul24(sc1, hi);
  }
}

template <int TYPE>
__device__ __forceinline__ BlockInts block_product(const RawBlk& r, const typename LdsFor<TYPE>::type* lds, int ib,
                                                   const KvTab& kv, const uint4& x0, const uint4& x1, int bs0,
                                                   int bs1) {
  uint32_t wd[8];
  int sc, sc1, mn;
  BlockInts o;
  decode_block32<TYPE>(r, lds, ib, kv, wd, sc, sc1, mn, o.d, o.dmin);
  block_dot<TYPE>(wd, sc, sc1, mn, x0, x1, bs0, bs1, o.iv, o.mv);
  return o;
}

// the reference's per-block float term: sa * d * (float)iv [ - sa * dmin * (float)mv ] (decode.cl:702-706)
template <int TYPE>
__device__ __forceinline__ float block_value(float sa, const BlockInts& b) {
  if constexpr (Traits<TYPE>::MINS) return sa * (b.d * (float)b.iv - b.dmin * (float)b.mv);
  else return sa * b.d * (float)b.iv;
}

}  // namespace qm
