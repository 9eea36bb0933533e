// Per-lane decode of one 32-block of a prepared weight row into int8 words, shared by the decode GEMVs and the
// MoE decode kernels.
#pragma once
#include "qm_launch.h"

namespace qm {

template <int TYPE> struct LdsFor { struct type { int unused; }; };
template <> struct LdsFor<T_IQ3_S> { using type = Iq3Lds; };

// The raw bytes a lane needs for 32-block b of row n: payload (q0; Q8_0 also q1) and header (h).
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

// Decodes a loaded 32-block (index ib = b % 8 in its superblock): w[k] = elements 4k..4k+3 (int8x4), the integer
// scale sc (and min mn), the float scale d (and dmin).
template <int TYPE>
__device__ __forceinline__ void decode_block32(const RawBlk& r, const typename LdsFor<TYPE>::type* lds, int ib,
                                               const KvTab& kv, uint32_t wd[8], int& sc, int& mn, float& d,
                                               float& dmin) {
  mn = 0;
  dmin = 0.0f;
  if constexpr (TYPE == T_Q8_0) {
    wd[0] = r.q0.x; wd[1] = r.q0.y; wd[2] = r.q0.z; wd[3] = r.q0.w;
    wd[4] = r.q1.x; wd[5] = r.q1.y; wd[6] = r.q1.z; wd[7] = r.q1.w;
    d = h2f(r.h.x);
    sc = 1;
  } else if constexpr (TYPE == T_Q4_K) {
    const uint32_t qq[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wd[k] = qq[k] & 0x0F0F0F0Fu;
      wd[4 + k] = (qq[k] >> 4) & 0x0F0F0F0Fu;
    }
    d = h2f(r.h.x);
    dmin = h2f(r.h.x >> 16);
    q4k_scale_min(r.h.y, r.h.z, r.h.w, ib, sc, mn);
  } else if constexpr (TYPE == T_IQ4_XS) {
    const uint32_t qq[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wd[k] = kv_lookup4(kv, qq[k] & 0x0F0F0F0Fu);
      wd[4 + k] = kv_lookup4(kv, (qq[k] >> 4) & 0x0F0F0F0Fu);
    }
    d = h2f(r.h.x);
    sc = iq4xs_scale(r.h.x, r.h.y, ib);
  } else {  // IQ3_S
    const uint32_t qh = ((ib < 4 ? r.h.x : r.h.y) >> (8 * (ib & 3))) & 0xFFu;
    iq3s_pair<0>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[0], wd[1]);
    iq3s_pair<1>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[2], wd[3]);
    iq3s_pair<2>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[4], wd[5]);
    iq3s_pair<3>(lds, r.q0.x, r.q0.y, qh, r.q0.z, wd[6], wd[7]);
    sc = 1 + 2 * (int)((r.h.z >> (4 * ib)) & 0xFu);
    d = h2f(r.h.w);
  }
}

}  // namespace qm
