// Device-side building blocks shared by the qmatmul kernels (gfx950 / CDNA4, wave64).
//
// Prepared weight layout (written by qm_repack_kernel, read by every product). Per weight: two planes,
//   payload plane  [rows][K/32][QB]  bytes: the quants of each 32-element block, 16-byte aligned rows
//   header plane   [rows][K/256][HB] bytes: the scales of each 256-element superblock
// so a lane that owns 32-block b of row n reads QB contiguous bytes, and consecutive lanes read consecutive blocks
// (coalesced). The bytes are the GGUF bytes regrouped (IQ3_S: +2 bytes of padding per superblock):
//   Q8_0   QB 32: int8 q[32]                         HB 16: the 8 blocks' f16 scales
//   Q4_K   QB 16: byte t = q[t] | q[16+t] << 4       HB 16: f16 d, f16 dmin, 12 bytes of 6-bit scales/mins (GGUF)
//   IQ4_XS QB 16: byte t = i[t] | i[16+t] << 4       HB  8: f16 d, u16 scales_h, u8 scales_l[4] (GGUF)
//   IQ3_S  QB 12: 8 index low bytes, 4 sign bytes    HB 16: qh[8], scales[4], f16 d, 2 bytes zero
// (Q4_K's GGUF nibble order -- 64-element chunks, low nibbles first -- is regrouped to IQ4_XS's per-32 order, so
// the 4-bit types share one unpacking path.)
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "iq_tables.inc"

namespace qm {

enum : int { T_Q8_0 = 8, T_Q4_K = 12, T_IQ3_S = 21, T_IQ4_XS = 23 };

template <int TYPE> struct Traits;
template <> struct Traits<T_Q8_0> { static constexpr int QB = 32, HB = 16, GGUF_SB = 272; static constexpr bool MINS = false; };
template <> struct Traits<T_Q4_K> { static constexpr int QB = 16, HB = 16, GGUF_SB = 144; static constexpr bool MINS = true; };
template <> struct Traits<T_IQ4_XS> { static constexpr int QB = 16, HB = 8, GGUF_SB = 136; static constexpr bool MINS = false; };
template <> struct Traits<T_IQ3_S> { static constexpr int QB = 12, HB = 16, GGUF_SB = 110; static constexpr bool MINS = false; };

// A prepared weight as the kernels see it.
struct WView {
  const uint8_t* qs;   // payload plane
  const uint8_t* hdr;  // header plane
  int rows, K;
};

__device__ __forceinline__ float h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFFu))); }

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value {hi:lo} (sel 0..3 -> lo, 4..7 -> hi).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// IQ4_NL codebook as four packed words (bytes kv[4i..4i+3]); values: ggml's kvalues_iq4nl.
struct KvTab { uint32_t t0, t1, t2, t3; };
__device__ __forceinline__ KvTab kv_tab() {
  constexpr int8_t kv[16] = QM_IQ4NL_VALUES_INIT;
  KvTab t;
  t.t0 = (uint8_t)kv[0] | ((uint8_t)kv[1] << 8) | ((uint8_t)kv[2] << 16) | ((uint32_t)(uint8_t)kv[3] << 24);
  t.t1 = (uint8_t)kv[4] | ((uint8_t)kv[5] << 8) | ((uint8_t)kv[6] << 16) | ((uint32_t)(uint8_t)kv[7] << 24);
  t.t2 = (uint8_t)kv[8] | ((uint8_t)kv[9] << 8) | ((uint8_t)kv[10] << 16) | ((uint32_t)(uint8_t)kv[11] << 24);
  t.t3 = (uint8_t)kv[12] | ((uint8_t)kv[13] << 8) | ((uint8_t)kv[14] << 16) | ((uint32_t)(uint8_t)kv[15] << 24);
  return t;
}

// Four 4-bit codebook indices (bits 0..3 of each byte of n; bits 4..7 ignored) -> four int8 codebook values.
// Two byte permutes read the 8-entry halves, a third picks per byte by the index's bit 3.
__device__ __forceinline__ uint32_t kv_lookup4(const KvTab& t, uint32_t n) {
  const uint32_t sel = n & 0x07070707u;
  const uint32_t lo = perm(t.t1, t.t0, sel);
  const uint32_t hi = perm(t.t3, t.t2, sel);
  const uint32_t pick = ((n >> 1) & 0x04040404u) | 0x03020100u;
  return perm(hi, lo, pick);
}

// ---- per-block scale decoding from the header plane

// Q4_K: the 6-bit scale and min of 32-block j (0..7) from the 12 packed bytes s[0..11] held as three words
// (src/quants.h:61-69, get_scale_min_k4).
__device__ __forceinline__ void q4k_scale_min(uint32_t s03, uint32_t s47, uint32_t s811, int j, int& sc, int& mn) {
  const int jj = j & 3, sh = 8 * jj;
  const int sc_lo = (int)((s03 >> sh) & 63u), mn_lo = (int)((s47 >> sh) & 63u);
  const uint32_t b8 = (s811 >> sh) & 0xFFu;
  const int sc_hi = (int)((b8 & 0xFu) | (((s03 >> sh) >> 6 & 3u) << 4));
  const int mn_hi = (int)((b8 >> 4) | (((s47 >> sh) >> 6 & 3u) << 4));
  sc = j < 4 ? sc_lo : sc_hi;
  mn = j < 4 ? mn_lo : mn_hi;
}

// IQ4_XS: the signed scale (ls - 32) of 32-block ib from the header's first two words (src/quants.h:297-312).
__device__ __forceinline__ int iq4xs_scale(uint32_t h0, uint32_t h1, int ib) {
  const int ls = (int)(((h1 >> (4 * ib)) & 0xFu) | (((h0 >> (16 + 2 * ib)) & 3u) << 4));
  return ls - 32;
}

// IQ3_S sign masks: for a sign byte s, m[0]/m[1] = 0xFF in each byte whose sign bit (bits 0..3 / 4..7) is set, and
// x[0]/x[1] = 0x01 there; a grid word g becomes the signed word (g ^ m) + x (grid bytes are odd, >= 1: no carries).
struct SgnMask { uint32_t m0, m1, x0, x1; };
__device__ __forceinline__ SgnMask sign_mask_of(uint32_t s) {
  SgnMask r;
  const uint32_t a = ((s & 0xFu) * 0x00204081u) & 0x01010101u, b = (((s >> 4) & 0xFu) * 0x00204081u) & 0x01010101u;
  r.x0 = a;
  r.x1 = b;
  r.m0 = a * 0xFFu;
  r.m1 = b * 0xFFu;
  return r;
}

// Device-resident IQ3_S codebook (ggml's, see iq_tables.inc): one copy per code object (no relocatable device code).
static __device__ const uint32_t g_iq3s_grid[512] = QM_IQ3S_GRID_INIT;

// LDS copies of the IQ3_S grid and the 256 sign masks: 2 KB + 4 KB per work-group.
struct Iq3Lds {
  uint32_t grid[512];
  uint4 sgn[256];
};
__device__ __forceinline__ void iq3_lds_fill(Iq3Lds* t) {
  for (int i = threadIdx.x; i < 512; i += blockDim.x) t->grid[i] = g_iq3s_grid[i];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) {
    const SgnMask m = sign_mask_of((uint32_t)i);
    t->sgn[i] = make_uint4(m.m0, m.m1, m.x0, m.x1);
  }
}

// IQ3_S: 8 elements 8l..8l+7 of a 32-block -> two signed int8x4 words (src/quants.h:240-262).
//   q01: the block's 8 index low bytes (two words), h: its qh byte, s: the sign byte of elements 8l..8l+7
template <int L>
__device__ __forceinline__ void iq3s_pair(const Iq3Lds* t, uint32_t q0, uint32_t q1, uint32_t h, uint32_t sgw,
                                          uint32_t& w0, uint32_t& w1) {
  const uint32_t qw = L < 2 ? q0 : q1;
  const uint32_t i1 = ((qw >> (16 * (L & 1))) & 0xFFu) | ((h << (8 - 2 * L)) & 256u);
  const uint32_t i2 = ((qw >> (16 * (L & 1) + 8)) & 0xFFu) | ((h << (7 - 2 * L)) & 256u);
  const uint4 m = t->sgn[(sgw >> (8 * L)) & 0xFFu];
  w0 = (t->grid[i1] ^ m.x) + m.z;
  w1 = (t->grid[i2] ^ m.y) + m.w;
}

// ---- wave-level reductions (wave64)
__device__ __forceinline__ float wave_sum_width(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace qm
