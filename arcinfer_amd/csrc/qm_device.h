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
//   Q5_K   QB 20: per 16-element half h, 8 bytes: byte t = low4[16h+t] | low4[16h+8+t] << 4 (a prompt-GEMM lane
//                 loads only its half), then a word of fifth bits: byte i, bit k = bit4[4k+i], bit 4+k = bit4[16+4k+i]
//                 HB 16: as Q4_K
//   Q4_0, IQ4_NL QB 16: byte t = n[t] | n[16+t] << 4 (GGUF order)       HB 16: the 8 blocks' f16 scales (as Q8_0)
//   Q6_K   QB 24: byte t = low4[t] | low4[16+t] << 4, then two words of 2-bit high parts: word h (h = 0, 1),
//                 byte i, bits 2k..2k+1 = high2[16h + 4k + i]          HB 20: int8 scales[16] (per 16), f16 d, 2 zero
//   IQ2_XXS QB 8: GGUF a0 (4 grid indices), a1 (4 x 7-bit sign indices, 4-bit scale)   HB 4: f16 d, 2 zero
//   IQ2_XS  QB 8: GGUF qs[4] (u16: 9-bit grid index | 7-bit sign index << 9)  HB 12: scales[8], f16 d, 2 zero
//   IQ2_S   QB 8: 4 grid index low bytes, 4 sign bytes          HB 20: qh[8], scales[8], f16 d, 2 zero
//   IQ3_XXS QB 12: 8 grid index bytes, GGUF sign/scale word (4 x 7-bit sign indices, 4-bit scale)  HB 4: f16 d, 2 zero
//   Q3_K   QB 12: two words of 2-bit fields, then a word of high bits: word h (h = 0, 1), byte i, bits 2j..2j+1 = the
//                 low 2 bits of element 4 (4h + j) + i; word 2, byte i, bit k = the high bit (GGUF hmask) of element
//                 4k + i. Value = (low | high << 2) - 4            HB 20: int8 scales[16] (6-bit - 32), f16 d, 2 zero
//   Q2_K   QB 8: two words of 2-bit values laid out as Q3_K's first two (values 0..3)
//                 HB 20: f16 d, f16 dmin, GGUF scales[16] (per 16 elements: scale low nibble, min high nibble)
//   IQ1_S  QB 8: the block's 4 grid index low bytes, then GGUF qh (u16: 3 high index bits per 8 elements, bits 12-14
//                 the scale s, bit 15 the delta sign), 2 zero      HB 4: f16 d, 2 zero
//   IQ1_M  QB 8: the block's 4 grid index low bytes, GGUF qh[2] (per 8 elements: 3 high index bits, delta sign), then
//                 the block's two 3-bit scales (bits 0-2, 3-5)     HB 4: f16 d (assembled from the GGUF scale words), 2 zero
//                 value = 8 * grid + delta (delta = -1 where the sign bit is set, else 1), w = d / 8 * (2 s + 1) * value
//   Q2_0   QB 8: two words of 2-bit codes laid out as Q3_K's first two; value = code - 1
//                 HB 8: the four 64-blocks' f16 d (a 32-block uses its 64-block's: half-block b -> scale b / 2)
// (the GGUF fields of Q6_K are ql[128] | qh[64] | scales[16] | d, 210 bytes per superblock; prepared: 212)
// (Q4_K's GGUF nibble order -- 64-element chunks, low nibbles first -- is regrouped to IQ4_XS's per-32 order, so
// the 4-bit types share one unpacking path.)
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "iq_tables.inc"

namespace qm {

enum : int {
  T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ2_XXS = 16, T_IQ2_XS = 17, T_IQ3_XXS = 18,
  T_IQ4_NL = 20, T_IQ3_S = 21, T_IQ2_S = 22, T_IQ4_XS = 23, T_Q2_K = 10, T_Q3_K = 11, T_Q2_0 = 42,
  T_IQ1_S = 19, T_IQ1_M = 29
};

template <int TYPE> struct Traits;
// MINS: per-block mins (the activation block sums enter the result); SC16: two integer scales per 32-block (one per
// 16) and quants stored with an offset of 32 (removed with the per-16 activation sums); SPLIT: two integer scales per
// 32-block, signed quants (no offset)
template <> struct Traits<T_Q8_0> { static constexpr int QB = 32, HB = 16, GGUF_SB = 272; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_Q4_K> { static constexpr int QB = 16, HB = 16, GGUF_SB = 144; static constexpr bool MINS = true, SC16 = false, SPLIT = false; };
template <> struct Traits<T_Q5_K> { static constexpr int QB = 20, HB = 16, GGUF_SB = 176; static constexpr bool MINS = true, SC16 = false, SPLIT = false; };
template <> struct Traits<T_Q4_0> { static constexpr int QB = 16, HB = 16, GGUF_SB = 144; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_IQ4_NL> { static constexpr int QB = 16, HB = 16, GGUF_SB = 144; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_Q6_K> { static constexpr int QB = 24, HB = 20, GGUF_SB = 210; static constexpr bool MINS = false, SC16 = true, SPLIT = false; };
template <> struct Traits<T_IQ4_XS> { static constexpr int QB = 16, HB = 8, GGUF_SB = 136; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_IQ3_S> { static constexpr int QB = 12, HB = 16, GGUF_SB = 110; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_IQ2_XXS> { static constexpr int QB = 8, HB = 4, GGUF_SB = 66; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_IQ2_XS> { static constexpr int QB = 8, HB = 12, GGUF_SB = 74; static constexpr bool MINS = false, SC16 = false, SPLIT = true; };
template <> struct Traits<T_IQ2_S> { static constexpr int QB = 8, HB = 20, GGUF_SB = 82; static constexpr bool MINS = false, SC16 = false, SPLIT = true; };
template <> struct Traits<T_IQ3_XXS> { static constexpr int QB = 12, HB = 4, GGUF_SB = 98; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_Q2_K> { static constexpr int QB = 8, HB = 20, GGUF_SB = 84; static constexpr bool MINS = true, SC16 = false, SPLIT = true; };
template <> struct Traits<T_Q3_K> { static constexpr int QB = 12, HB = 20, GGUF_SB = 110; static constexpr bool MINS = false, SC16 = false, SPLIT = true; };
template <> struct Traits<T_IQ1_S> { static constexpr int QB = 8, HB = 4, GGUF_SB = 50; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
template <> struct Traits<T_IQ1_M> { static constexpr int QB = 8, HB = 4, GGUF_SB = 56; static constexpr bool MINS = false, SC16 = false, SPLIT = true; };
template <> struct Traits<T_Q2_0> { static constexpr int QB = 8, HB = 8, GGUF_SB = 72; static constexpr bool MINS = false, SC16 = false, SPLIT = false; };
// f16 scales per 32-block in the header (Q8_0's layout; Q2_0: one per 64-block), no integer sub-scales
template <int TYPE> constexpr bool kBlockScales = TYPE == T_Q8_0 || TYPE == T_Q4_0 || TYPE == T_IQ4_NL || TYPE == T_Q2_0;
// the header's f16 scale of 32-block b (0..7) for kBlockScales types: its index among the header's halfwords
template <int TYPE> __host__ __device__ constexpr int block_scale_slot(int b) { return TYPE == T_Q2_0 ? b >> 1 : b; }
// mins per 16 elements (two per 32-block; the other MINS types have one per 32-block)
template <int TYPE> constexpr bool kMin16 = TYPE == T_Q2_K;
// whether the kernels need the per-16 activation sums (absum)
template <int TYPE> constexpr bool kNeedsBsum = Traits<TYPE>::MINS || Traits<TYPE>::SC16;
// the codebook types whose tables live in LDS
template <int TYPE> constexpr bool kIq2 = TYPE == T_IQ2_XXS || TYPE == T_IQ2_XS || TYPE == T_IQ2_S || TYPE == T_IQ3_XXS;
template <int TYPE> constexpr bool kIq1 = TYPE == T_IQ1_S || TYPE == T_IQ1_M;

// A prepared weight as the kernels see it.
struct WView {
  const uint8_t* qs;   // payload plane
  const uint8_t* hdr;  // header plane
  int rows, K;
};

__device__ __forceinline__ float h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFFu))); }

// 16-byte streaming load (non-temporal: weights are read once per product and should not displace cached data)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4_t ld_stream16(const void* p) {
  return __builtin_nontemporal_load((const u32x4_t*)p);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value {hi:lo} (sel 0..3 -> lo, 4..7 -> hi).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// IQ4_NL / IQ4_XS codebook lookup with two byte permutes and an XOR.
// v_perm_b32 picks byte `sel` (0..7) of an 8-byte table; for sel 8..11 it returns 0xFF or 0x00 by the sign of table
// byte 1, 3, 5 or 7, for 12 it returns 0x00 and for 13..15 0xFF. A raw 4-bit code n (0..15) is therefore a valid
// selector: table A answers codes 0..7 and returns 0x00/0xFF for 8..15, table B (selector n ^ 8) answers codes 8..15
// and returns 0x00/0xFF for 0..7. Storing each entry pre-XORed with what the other table returns for the same code
// makes pA ^ pB the codebook value for every code. The junk depends on the tables' own sign bits, so the tables are
// the fixed point of that rule, computed here at compile time from the codebook.
struct KvTab { uint32_t a0, a1, b0, b1; };
namespace detail {
constexpr uint8_t perm_byte(const uint8_t* in, int sel) {
  return sel >= 13 ? 0xFF : sel == 12 ? 0x00 : sel >= 8 ? ((in[2 * (sel - 8) + 1] & 0x80) ? 0xFF : 0x00) : in[sel];
}
constexpr KvTab make_kv_tab() {
  constexpr int8_t kv[16] = QM_IQ4NL_VALUES_INIT;
  uint8_t ta[8] = {}, tb[8] = {};
  for (int i = 0; i < 8; ++i) {
    ta[i] = (uint8_t)kv[i];
    tb[i] = (uint8_t)kv[8 + i];
  }
  for (int it = 0; it < 8; ++it) {
    for (int n = 8; n < 16; ++n) tb[n - 8] = (uint8_t)((uint8_t)kv[n] ^ perm_byte(ta, n));
    for (int n = 0; n < 8; ++n) ta[n] = (uint8_t)((uint8_t)kv[n] ^ perm_byte(tb, n ^ 8));
  }
  KvTab t{};
  t.a0 = ta[0] | (ta[1] << 8) | (ta[2] << 16) | ((uint32_t)ta[3] << 24);
  t.a1 = ta[4] | (ta[5] << 8) | (ta[6] << 16) | ((uint32_t)ta[7] << 24);
  t.b0 = tb[0] | (tb[1] << 8) | (tb[2] << 16) | ((uint32_t)tb[3] << 24);
  t.b1 = tb[4] | (tb[5] << 8) | (tb[6] << 16) | ((uint32_t)tb[7] << 24);
  return t;
}
constexpr bool kv_tab_ok() {
  constexpr int8_t kv[16] = QM_IQ4NL_VALUES_INIT;
  const KvTab t = make_kv_tab();
  const uint8_t ta[8] = {(uint8_t)t.a0, (uint8_t)(t.a0 >> 8), (uint8_t)(t.a0 >> 16), (uint8_t)(t.a0 >> 24),
                         (uint8_t)t.a1, (uint8_t)(t.a1 >> 8), (uint8_t)(t.a1 >> 16), (uint8_t)(t.a1 >> 24)};
  const uint8_t tb[8] = {(uint8_t)t.b0, (uint8_t)(t.b0 >> 8), (uint8_t)(t.b0 >> 16), (uint8_t)(t.b0 >> 24),
                         (uint8_t)t.b1, (uint8_t)(t.b1 >> 8), (uint8_t)(t.b1 >> 16), (uint8_t)(t.b1 >> 24)};
  for (int n = 0; n < 16; ++n)
    if ((uint8_t)(perm_byte(ta, n) ^ perm_byte(tb, n ^ 8)) != (uint8_t)kv[n]) return false;
  return true;
}
}  // namespace detail
static_assert(detail::kv_tab_ok(), "IQ4_NL permute tables do not reproduce the codebook");
__device__ __forceinline__ KvTab kv_tab() { return detail::make_kv_tab(); }

// Four 4-bit codes (bits 0..3 of each byte of n, bits 4..7 zero) -> four int8 codebook values.
__device__ __forceinline__ uint32_t kv_lookup4(const KvTab& t, uint32_t n) {
  return perm(t.a1, t.a0, n) ^ perm(t.b1, t.b0, n ^ 0x08080808u);
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

// IQ4_XS: the signed scale ls - 32 of 32-block ib from the prepared header's first two words (src/quants.h:297-312).
// The prepared header stores scales_h with bit 1 of every 2-bit field flipped, so each field read as a signed 2-bit
// number is (high bits of ls) - 2, and (field << 4) | (low 4 bits) is ls - 32 in one sign-extending extract.
__device__ __forceinline__ int iq4xs_scale(uint32_t h0, uint32_t h1, int ib) {
  const int hi = __builtin_amdgcn_sbfe((int)h0, 16 + 2 * ib, 2);  // (one signed bit-field extract)
  return hi * 16 + (int)__builtin_amdgcn_ubfe(h1, 4 * ib, 4);
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

// ---- the 2-bit / IQ3_XXS codebook types (src/quants.h:170-239)
// Device-resident codebooks (ggml's, see iq_tables.inc) and the 7-bit sign index -> sign byte table (the 8th sign is
// the parity of the 7 stored ones).
static __device__ const uint64_t g_iq2xxs_grid[256] = QM_IQ2XXS_GRID_INIT;
static __device__ const uint64_t g_iq2xs_grid[512] = QM_IQ2XS_GRID_INIT;
static __device__ const uint64_t g_iq2s_grid[1024] = QM_IQ2S_GRID_INIT;
static __device__ const uint32_t g_iq3xxs_grid[256] = QM_IQ3XXS_GRID_INIT;

template <int TYPE> struct IqGrid;
template <> struct IqGrid<T_IQ2_XXS> { using G = uint2; static constexpr int NG = 256, NS = 128; };
template <> struct IqGrid<T_IQ2_XS> { using G = uint2; static constexpr int NG = 512, NS = 128; };
template <> struct IqGrid<T_IQ2_S> { using G = uint2; static constexpr int NG = 1024, NS = 256; };
template <> struct IqGrid<T_IQ3_XXS> { using G = uint32_t; static constexpr int NG = 256, NS = 128; };

// LDS copies of a type's grid and its sign masks (indexed by the stored sign field: 7 bits, IQ2_S 8 bits):
// IQ2_XXS 4 KB, IQ2_XS 6 KB, IQ2_S 12 KB, IQ3_XXS 3 KB per work-group.
template <int TYPE> struct IqLds {
  typename IqGrid<TYPE>::G grid[IqGrid<TYPE>::NG];
  uint4 sgn[IqGrid<TYPE>::NS];
};
template <int TYPE>
__device__ __forceinline__ void iq_lds_fill(IqLds<TYPE>* t) {
  using I = IqGrid<TYPE>;
  for (int i = threadIdx.x; i < I::NG; i += blockDim.x) {
    if constexpr (TYPE == T_IQ3_XXS) {
      t->grid[i] = g_iq3xxs_grid[i];
    } else {
      const uint64_t g = TYPE == T_IQ2_XXS ? g_iq2xxs_grid[i] : TYPE == T_IQ2_XS ? g_iq2xs_grid[i] : g_iq2s_grid[i];
      t->grid[i] = make_uint2((uint32_t)g, (uint32_t)(g >> 32));
    }
  }
  for (int i = threadIdx.x; i < I::NS; i += blockDim.x) {
    const uint32_t sb = I::NS == 128 ? (uint32_t)i | ((__builtin_popcount(i) & 1u) << 7) : (uint32_t)i;
    const SgnMask m = sign_mask_of(sb);
    t->sgn[i] = make_uint4(m.m0, m.m1, m.x0, m.x1);
  }
}

// Group l (elements 8l..8l+7, l = 0..3) of a 32-block -> two signed int8x4 words, from the block's payload words
// p0, p1, p2 (prepared layout above) and, for IQ2_S, its qh byte. Grid bytes are >= 4, so (g ^ m) + x negates the
// masked bytes without carries.
template <int TYPE>
__device__ __forceinline__ void iq_group(const IqLds<TYPE>* t, uint32_t p0, uint32_t p1, uint32_t p2, uint32_t qh,
                                         int l, uint32_t& w0, uint32_t& w1) {
  if constexpr (TYPE == T_IQ3_XXS) {
    const uint32_t qw = l < 2 ? p0 : p1;
    const int sh = 16 * (l & 1);
    const uint4 m = t->sgn[(p2 >> (7 * l)) & 127u];
    w0 = (t->grid[(qw >> sh) & 0xFFu] ^ m.x) + m.z;
    w1 = (t->grid[(qw >> (sh + 8)) & 0xFFu] ^ m.y) + m.w;
  } else {
    uint32_t gi, si;
    if constexpr (TYPE == T_IQ2_XXS) {
      gi = (p0 >> (8 * l)) & 0xFFu;
      si = (p1 >> (7 * l)) & 127u;
    } else if constexpr (TYPE == T_IQ2_XS) {
      const uint32_t q16 = ((l < 2 ? p0 : p1) >> (16 * (l & 1))) & 0xFFFFu;
      gi = q16 & 511u;
      si = q16 >> 9;
    } else {
      gi = ((p0 >> (8 * l)) & 0xFFu) | ((qh << (8 - 2 * l)) & 0x300u);
      si = (p1 >> (8 * l)) & 0xFFu;
    }
    const uint2 g = t->grid[gi];
    const uint4 m = t->sgn[si];
    w0 = (g.x ^ m.x) + m.z;
    w1 = (g.y ^ m.y) + m.w;
  }
}

// ---- IQ1_S / IQ1_M (src/quants.h:263-296): the grid (ggml's iq1s_grid, every byte -1, 0 or 1) and, in LDS, one
// word per entry: byte i holds (grid byte i) + 1 in bits 0-1 and (grid byte 4 + i) + 1 in bits 2-3, so an entry's
// two int8x4 words of 8 * grid + delta are two byte permutes of a 3-value table.
static __device__ const uint64_t g_iq1s_grid[2048] = QM_IQ1S_GRID_INIT;
struct Iq1Lds {
  uint32_t grid[2048];
};
__device__ __forceinline__ void iq1_lds_fill(Iq1Lds* t) {
  for (int i = threadIdx.x; i < 2048; i += blockDim.x) {
    const uint64_t g = g_iq1s_grid[i];
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t c0 = (uint32_t)((int)(int8_t)(g >> (8 * b)) + 1), c1 = (uint32_t)((int)(int8_t)(g >> (8 * b + 32)) + 1);
      w |= (c0 | (c1 << 2)) << (8 * b);
    }
    t->grid[i] = w;
  }
}
// elements 8l..8l+7 of a 32-block (grid entry idx, delta sign neg) -> two int8x4 words
__device__ __forceinline__ void iq1_group(const Iq1Lds* t, uint32_t idx, bool neg, uint32_t& w0, uint32_t& w1) {
  const uint32_t e = t->grid[idx];
  const uint32_t tab = neg ? 0x0007FFF7u : 0x000901F9u;  // {8 (g) + delta} for g + 1 = 0, 1, 2: {-9, -1, 7} / {-7, 1, 9}
  w0 = __builtin_amdgcn_perm(0u, tab, e & 0x03030303u);
  w1 = __builtin_amdgcn_perm(0u, tab, (e >> 2) & 0x03030303u);
}
// group l's grid index and delta sign from a prepared IQ1 payload word pair (q0: index low bytes, q1: qh and scales)
template <int TYPE>
__device__ __forceinline__ void iq1_index(uint32_t q0, uint32_t q1, int l, uint32_t& idx, bool& neg) {
  const uint32_t lo = (q0 >> (8 * l)) & 0xFFu;
  if constexpr (TYPE == T_IQ1_S) {
    idx = lo | (((q1 >> (3 * l)) & 7u) << 8);
    neg = (q1 & 0x8000u) != 0;
  } else {  // IQ1_M: byte l / 2 of q1, nibble l % 2: 3 index bits, then the sign bit
    const uint32_t nib = (q1 >> (4 * l)) & 0xFu;
    idx = lo | ((nib & 7u) << 8);
    neg = (nib & 8u) != 0;
  }
}

// Per-type scale unit: IQ2 d / 8, IQ3_XXS d / 4 (src/quants.h:172, 222) -- exact powers of two
template <int TYPE> constexpr float kIqDScale = TYPE == T_IQ3_XXS ? 0.25f : 0.125f;

// ---- cross-lane operations (wave64). Lane moves within a 16-lane row are DPP operands of the VALU op itself; the
// four rows are combined through v_readlane. (__shfl_xor would be an LDS round trip, ds_bpermute, per step.) Every
// lane of the wave must be active.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane 7 - i of its 8-lane half-row: the other quad of the 8 lanes
constexpr int kDppMirror = 0x140;      // lane 15 - i of its row: the other 8 lanes of the row

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// max over the 8-lane group holding the lane (every lane of the group receives it)
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}
// sum over the 4-lane quad holding the lane (exact for ints)
__device__ __forceinline__ int sum4_i(int v) {
  v += dpp_i<kDppXor1>(v);
  return v + dpp_i<kDppXor2>(v);
}

// Sum over the aligned group of `width` lanes (2..64, a power of two, known at compile time at every call site).
// Lane 0 of each group receives the sum; the other lanes of a group of <= 16 receive the same value summed in another
// order, and every lane of a 32- or 64-lane group receives lane 0's value.
__device__ __forceinline__ float wave_sum_width(float v, int width) {
  v += dpp_f<kDppXor1>(v);
  if (width == 2) return v;
  v += dpp_f<kDppXor2>(v);
  if (width == 4) return v;
  v += dpp_f<kDppHalfMirror>(v);
  if (width == 8) return v;
  v += dpp_f<kDppMirror>(v);
  if (width == 16) return v;
  const float r0 = readlane_f(v, 0), r1 = readlane_f(v, 16), r2 = readlane_f(v, 32), r3 = readlane_f(v, 48);
  if (width == 32) return (threadIdx.x & 32) ? r2 + r3 : r0 + r1;
  return (r0 + r1) + (r2 + r3);
}

// max over the 32-lane half of the wave holding the lane; every lane receives it
__device__ __forceinline__ float max32(float v) {
  v = max8(v);
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  const float r0 = readlane_f(v, 0), r1 = readlane_f(v, 16), r2 = readlane_f(v, 32), r3 = readlane_f(v, 48);
  return (threadIdx.x & 32) ? fmaxf(r2, r3) : fmaxf(r0, r1);
}

// max over the wave; every lane receives it
__device__ __forceinline__ float wave_max(float v) {
  v = max8(v);
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

}  // namespace qm

namespace qm {
// n - 8 for four nibble values 0..15 held one per byte: a byte-wise subtract without borrows
__device__ __forceinline__ uint32_t sub8_bytes(uint32_t n) { return ((n | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }

// Q2_0 / Q3_K (prepared layout above): word k (elements 4k..4k+3) of a 32-block as four signed bytes.
//   Q2_0: code - 1 by a byte permute of the table {-1, 0, 1, 2}; Q3_K: (low | high << 2) - 4 by a permute of
//   {-4, ..., 3}. d01: the payload's two words of 2-bit fields, hw: Q3_K's word of high bits.
__device__ __forceinline__ uint32_t q2_word(uint32_t d0, uint32_t d1, int k) {
  const uint32_t c = ((k < 4 ? d0 : d1) >> (2 * (k & 3))) & 0x03030303u;
  return __builtin_amdgcn_perm(0u, 0x020100FFu, c);
}
__device__ __forceinline__ uint32_t q3_word(uint32_t d0, uint32_t d1, uint32_t hw, int k) {
  const uint32_t c = (((k < 4 ? d0 : d1) >> (2 * (k & 3))) & 0x03030303u) | (((hw >> k) & 0x01010101u) << 2);
  return __builtin_amdgcn_perm(0x03020100u, 0xFFFEFDFCu, c);
}
}  // namespace qm
