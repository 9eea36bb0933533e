// Prompt GEMM on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8), dense and MoE-tile modes.
//
// Work-group: 256 threads = 4 waves, a tile of BM = 32*MT activation rows x BN = 128 weight rows; wave w owns
// weight rows n0 + 32w .. +31 (one MFMA column tile) and all MT row tiles. K advances one 256-element superblock
// at a time:
//   - the activation rows of the superblock (int8, 256 B per row) are staged in LDS with 16-byte loads, rows
//     padded to 272 B so the MFMA operand reads (lane = row, 16 B at the lane's k-half) spread over the banks;
//     their per-32 scales (and, for Q4_K, scale x per-32 sum) go to LDS as well;
//   - each lane decodes its weight row's 32-block straight into the MFMA B operand: the 16 int8 of its k-half
//     (lanes 0-31: elements 0..15, lanes 32-63: 16..31), from one 16-byte payload load (IQ3_S: grid + sign masks
//     in LDS), so weights go from their 4.25-bit form to int8 in registers, never through an int8 copy in memory;
//   - one MFMA per 32-block and row tile gives the exact int32 block sums sum_k a*q (the reference's int32
//     accumulators); the f32 epilogue applies activation scale x weight scale per block
//     (zero/kernels/gemm.cl:367-412 applies the same per-32 scales), and Q4_K's min term from the per-32 sums.
// The 32x32 MFMA result layout: lane l holds column j = l % 32 and rows 8*(r/4) + 4*(l/32) + r%4, r = 0..15.
#include <stdlib.h>

#include "qm_decode.h"

namespace qm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int A_STRIDE = 272;  // LDS bytes per staged activation row

template <int TYPE, int MT> struct GemmLds {
  // (two buffers: superblock s is read from one while superblock s + 1 is written into the other)
  alignas(16) uint8_t a[2][32 * MT * A_STRIDE];
  alignas(16) float asc[2][8 * 32 * MT];
  float u[2][Traits<TYPE>::MINS ? 8 * 32 * MT : 1];
  int arow[32 * MT];
  typename LdsFor<TYPE>::type tab;  // (IQ3_S and the IQ2 / IQ3_XXS types: codebook and sign tables)
};

// IQ3_S, pair L (elements 8L..8L+7) with L known only at run time.
__device__ __forceinline__ void iq3s_pair_rt(const Iq3Lds* t, uint32_t q0, uint32_t q1, uint32_t h, uint32_t sgw,
                                             int L, uint32_t& w0, uint32_t& w1) {
  const uint32_t qw = L < 2 ? q0 : q1;
  const int sh = 16 * (L & 1);
  const uint32_t i1 = ((qw >> sh) & 0xFFu) | ((h << (8 - 2 * L)) & 256u);
  const uint32_t i2 = ((qw >> (sh + 8)) & 0xFFu) | ((h << (7 - 2 * L)) & 256u);
  const uint4 m = t->sgn[(sgw >> (8 * L)) & 0xFFu];
  w0 = (t->grid[i1] ^ m.x) + m.z;
  w1 = (t->grid[i2] ^ m.y) + m.w;
}

// A lane's payload of one 32-block (the bytes its k-half needs): 16 B for Q8_0 (its half of the 32 int8), the block's
// 16 nibble bytes for the other 4-bit types, Q5_K's 8 nibble bytes of its half and the word of fifth bits (.x .y
// nibbles, .z fifth bits, .w unused), the 8 index bytes + 4 sign bytes for IQ3_S (.w unused).
template <int TYPE>
__device__ __forceinline__ uint4 load_payload(const WView& w, int n, int blk, int hf) {
  using Tr = Traits<TYPE>;
  const uint8_t* qp = w.qs + ((size_t)n * (w.K / 32) + blk) * Tr::QB;
  if constexpr (TYPE == T_Q8_0) {
    return *(const uint4*)(qp + 16 * hf);
  } else if constexpr (TYPE == T_Q5_K) {
    const uint2 nib = *(const uint2*)(qp + 8 * hf);
    return make_uint4(nib.x, nib.y, *(const uint32_t*)(qp + 16), 0u);
  } else if constexpr (TYPE == T_IQ3_S || TYPE == T_IQ3_XXS) {
    const uint32_t* q = (const uint32_t*)qp;
    return make_uint4(q[0], q[1], q[2], 0u);
  } else if constexpr (Traits<TYPE>::QB == 8) {
    const uint2 q = *(const uint2*)qp;
    return make_uint4(q.x, q.y, 0u, 0u);
  } else {
    return *(const uint4*)qp;
  }
}

template <int TYPE>
__device__ __forceinline__ uint4 load_header(const WView& w, int n, int s) {
  const uint8_t* hp = w.hdr + ((size_t)n * (w.K / 256) + s) * Traits<TYPE>::HB;
  if constexpr (Traits<TYPE>::HB == 8) {
    const uint2 h = *(const uint2*)hp;
    return make_uint4(h.x, h.y, 0u, 0u);
  } else if constexpr (Traits<TYPE>::HB == 4) {
    return make_uint4(*(const uint32_t*)hp, 0u, 0u, 0u);
  } else {
    return *(const uint4*)hp;
  }
}

// The MFMA B operand (16 int8 weights of k-half hf) from a lane's payload of 32-block b of its superblock.
template <int TYPE>
__device__ __forceinline__ v4i b_operand(uint4 q, uint4 hdr, int b, int hf, const KvTab& kv,
                                         const typename LdsFor<TYPE>::type* tab) {
  v4i r;
  if constexpr (TYPE == T_Q8_0) {
    r[0] = (int)q.x; r[1] = (int)q.y; r[2] = (int)q.z; r[3] = (int)q.w;
  } else if constexpr (TYPE == T_Q2_0) {
    // (k-half hf: words 4 hf .. 4 hf + 3, all four from payload word hf)
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = (int)q2_word(q.x, q.y, 4 * hf + k);
  } else if constexpr (TYPE == T_Q5_K) {
    // (fifth bits: byte i, bit k = element 4k+i of the first half, bit 4+k = of the second)
    r[0] = (int)(q.x & 0x0F0F0F0Fu); r[1] = (int)(q.y & 0x0F0F0F0Fu);
    r[2] = (int)((q.x >> 4) & 0x0F0F0F0Fu); r[3] = (int)((q.y >> 4) & 0x0F0F0F0Fu);
    const uint32_t hb = q.z >> (4 * hf);
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] |= (int)(((hb >> k) & 0x01010101u) << 4);
  } else if constexpr (kIq1<TYPE>) {
    // (k-half hf: groups 2 hf and 2 hf + 1 of the block)
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      uint32_t idx, w0, w1;
      bool neg;
      iq1_index<TYPE>(q.x, q.y, 2 * hf + g, idx, neg);
      iq1_group(tab, idx, neg, w0, w1);
      r[2 * g] = (int)w0;
      r[2 * g + 1] = (int)w1;
    }
  } else if constexpr (kIq2<TYPE>) {
    uint32_t w0, w1, w2, w3;
    iq_group<TYPE>(tab, q.x, q.y, q.z, 0u, 2 * hf, w0, w1);
    iq_group<TYPE>(tab, q.x, q.y, q.z, 0u, 2 * hf + 1, w2, w3);
    r[0] = (int)w0; r[1] = (int)w1; r[2] = (int)w2; r[3] = (int)w3;
  } else if constexpr (TYPE != T_IQ3_S) {
    const int sh = 4 * hf;
    const uint32_t x0 = q.x >> sh, x1 = q.y >> sh, x2 = q.z >> sh, x3 = q.w >> sh;
    if constexpr (TYPE == T_Q4_K) {
      r[0] = (int)(x0 & 0x0F0F0F0Fu); r[1] = (int)(x1 & 0x0F0F0F0Fu);
      r[2] = (int)(x2 & 0x0F0F0F0Fu); r[3] = (int)(x3 & 0x0F0F0F0Fu);
    } else if constexpr (TYPE == T_Q4_0) {
      r[0] = (int)sub8_bytes(x0 & 0x0F0F0F0Fu); r[1] = (int)sub8_bytes(x1 & 0x0F0F0F0Fu);
      r[2] = (int)sub8_bytes(x2 & 0x0F0F0F0Fu); r[3] = (int)sub8_bytes(x3 & 0x0F0F0F0Fu);
    } else {
      r[0] = (int)kv_lookup4(kv, x0 & 0x0F0F0F0Fu); r[1] = (int)kv_lookup4(kv, x1 & 0x0F0F0F0Fu);
      r[2] = (int)kv_lookup4(kv, x2 & 0x0F0F0F0Fu); r[3] = (int)kv_lookup4(kv, x3 & 0x0F0F0F0Fu);
    }
  } else {
    const uint32_t qh = ((b < 4 ? hdr.x : hdr.y) >> (8 * (b & 3))) & 0xFFu;
    uint32_t w0, w1, w2, w3;
    iq3s_pair_rt(tab, q.x, q.y, qh, q.z, 2 * hf, w0, w1);
    iq3s_pair_rt(tab, q.x, q.y, qh, q.z, 2 * hf + 1, w2, w3);
    r[0] = (int)w0; r[1] = (int)w1; r[2] = (int)w2; r[3] = (int)w3;
  }
  return r;
}

// Per-block weight scales of one superblock from its header (IQ2_XXS, IQ3_XXS, IQ1_S: and its blocks' payloads pay,
// which hold the integer scale): dsc[b] = d * sc_b (Q8_0: the block's f16 scale), dmn[b] = dmin * mn_b (Q4_K),
// isc[b] = the integer scale.
template <int TYPE>
__device__ __forceinline__ void sb_scales(uint4 h, const uint4* pay, float dsc[8], float dmn[8], int isc[8]) {
  if constexpr (TYPE == T_IQ1_S) {  // (the scale in bits 12-14 of the payload's qh)
    const float d = h2f(h.x) * 0.125f;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      isc[b] = 2 * (int)((pay[b].y >> 12) & 7u) + 1;
      dsc[b] = d * (float)isc[b];
      dmn[b] = 0.0f;
    }
  } else if constexpr (TYPE == T_IQ2_XXS || TYPE == T_IQ3_XXS) {
    const float d = h2f(h.x) * kIqDScale<TYPE>;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      isc[b] = 1 + 2 * (int)((TYPE == T_IQ2_XXS ? pay[b].y : pay[b].z) >> 28);
      dsc[b] = d * (float)isc[b];
      dmn[b] = 0.0f;
    }
  } else if constexpr (kBlockScales<TYPE>) {
    const uint32_t hh[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int j = block_scale_slot<TYPE>(b);
      dsc[b] = h2f(hh[j >> 1] >> (16 * (j & 1)));
      dmn[b] = 0.0f;
      isc[b] = 1;
    }
  } else if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      int sc, mn;
      q4k_scale_min(h.y, h.z, h.w, b, sc, mn);
      dsc[b] = d * (float)sc;
      dmn[b] = dmin * (float)mn;
      isc[b] = sc;
    }
  } else if constexpr (TYPE == T_IQ4_XS) {
    const float d = h2f(h.x);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      isc[b] = iq4xs_scale(h.x, h.y, b);
      dsc[b] = d * (float)isc[b];
      dmn[b] = 0.0f;
    }
  } else {
    const float d = h2f(h.w);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      isc[b] = 1 + 2 * (int)((h.z >> (4 * b)) & 0xFu);
      dsc[b] = d * (float)isc[b];
      dmn[b] = 0.0f;
    }
  }
}

// Work-group -> (column tile, row tile). Dense launches are remapped so that each of the 8 XCDs (work-groups are
// dealt to XCDs round-robin) sweeps a contiguous range of column tiles, row tiles fastest: concurrent work-groups
// of an XCD share weight tiles in its L2.
__device__ __forceinline__ void dense_tile(int& nt, int& mtile) {
  const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
  int lin = blockIdx.y * gx + blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  nt = lin / gy;
  mtile = lin % gy;
}

// lo in lanes where m is 0, hi where m is all ones
__device__ __forceinline__ float lane_pick(uint32_t m, float lo, float hi) {
  return __uint_as_float((__float_as_uint(lo) & ~m) | (__float_as_uint(hi) & m));
}

// Result of an MoE tile mode for slot row `slot` and expert column n of this lane (ok: both in range). Every lane of
// the wave must call it (the h quantization takes the maximum over the 32 columns of a half-wave):
//   GEMM_MOE_DOWN: y[slot][n] = routing weight * v
//   GEMM_MOE_G:    g[slot][n] = v (the gate projection, f32, into C)
//   GEMM_MOE_GATEUP / GEMM_MOE_UH: h = u * silu(g) (zero/kernels/gemm.cl:464-471) with g = v, u = v2 (one launch) or
//     g from C, u = v (after a GEMM_MOE_G launch), then quantized per 32 columns -- the wave's 32 columns (lanes of one
//     half) are one 32-block of the h row -- as moe_quant (zero/kernels/moe.cl:251-282)
template <int MODE>
__device__ __forceinline__ void moe_store(const GemmArgs& a, int slot, int n, bool ok, float v, float v2, int lc) {
  if constexpr (MODE == GEMM_MOE_DOWN) {
    if (ok) a.C[(size_t)slot * a.ldc + n] = a.rowscale[slot] * v;
  } else if constexpr (MODE == GEMM_MOE_G) {
    if (ok) a.C[(size_t)slot * a.ldc + n] = v;
  } else {
    float g, u;
    if constexpr (MODE == GEMM_MOE_GATEUP) {
      g = v;
      u = v2;
    } else {
      g = ok ? a.C[(size_t)slot * a.ldc + n] : 0.0f;
      u = v;
    }
    const float h = u * (g / (1.0f + expf(-g)));
    const float amax = max32(fabsf(h));
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    const int q = (int)__builtin_rintf(h * inv);
    if (ok) {
      a.hq[(size_t)slot * a.ldc + n] = (int8_t)q;
      if (lc == 0) a.hsc[(size_t)(n / 32) * a.slots + slot] = amax / 127.0f;
    }
  }
}

// The work-group's rows: a dense M tile, or (MoE modes) one sub-tile of BM slots of an expert's tile of up to
// kMoeTileRows slots (returns false for work-groups past the tile count or past the tile's rows). wrow0: the
// expert's first weight row.
template <int MODE, int BM>
__device__ __forceinline__ bool tile_rows(const GemmArgs& a, int& m0, int& nvalid, int& wrow0, int& nt) {
  if constexpr (MODE == GEMM_DENSE) {
    int mtile;
    dense_tile(nt, mtile);
    m0 = mtile * BM;
    nvalid = min(BM, a.M - m0);
    wrow0 = 0;
    return true;
  } else if constexpr (BM > kMoeTileRows) {
    // two consecutive tiles of one expert (the tile list starts every expert's tiles at an even index, the second
    // of a pair possibly empty)
    const int t = 2 * (int)blockIdx.y;
    if (t >= a.tiles[0]) return false;
    const int e = a.tiles[1 + 3 * t];
    m0 = a.tiles[2 + 3 * t];
    nvalid = a.tiles[3 + 3 * t] + (t + 1 < a.tiles[0] ? a.tiles[3 + 3 * (t + 1)] : 0);
    if (nvalid <= 0) return false;
    wrow0 = e * a.expert_rows;
    nt = blockIdx.x;
    return true;
  } else {
    constexpr int SUB = kMoeTileRows / BM;
    const int t = blockIdx.y / SUB, sub = blockIdx.y % SUB;
    if (t >= a.tiles[0]) return false;
    const int e = a.tiles[1 + 3 * t];
    m0 = a.tiles[2 + 3 * t] + sub * BM;
    nvalid = min(BM, a.tiles[3 + 3 * t] - sub * BM);
    if (nvalid <= 0) return false;
    wrow0 = e * a.expert_rows;
    nt = blockIdx.x;
    return true;
  }
}

template <int TYPE, int MT, int MODE, bool DUMP>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
  constexpr int BM = 32 * MT;
  constexpr bool MINS = Traits<TYPE>::MINS;
  constexpr bool GU = MODE == GEMM_MOE_GATEUP;
  constexpr int ACH = BM * 16 / 256;        // 16-byte activation chunks per thread per superblock
  constexpr int SCH = (8 * BM + 255) / 256;  // scale values per thread per superblock
  __shared__ GemmLds<TYPE, MT> L;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, lc = lane & 31;
  const int K = a.w.K, nb = K / 32, nsb = K / 256;
  // K split (dense, gridDim.z = 2): this work-group's superblocks [sb0, sb1); the two halves are added into a zeroed C
  const int sb0 = (int)blockIdx.z * nsb / (int)gridDim.z, sb1 = ((int)blockIdx.z + 1) * nsb / (int)gridDim.z;

  // ---- which rows: dense (M tile), or one MoE tile (expert e, slots r0 .. r0 + nr - 1)
  int m0, nvalid, wrow0, nt;
  if (!tile_rows<MODE, BM>(a, m0, nvalid, wrow0, nt)) return;
  const int n_loc = nt * 128 + wave * 32 + lc;  // this lane's weight row (within the expert)
  const int n_rows = MODE == GEMM_DENSE ? a.w.rows : a.expert_rows;
  const int n = wrow0 + min(n_loc, n_rows - 1);

  if (tid < BM) {
    const int i = min(tid, nvalid - 1);
    int src;
    if constexpr (MODE == GEMM_MOE_GATEUP || MODE == GEMM_MOE_G || MODE == GEMM_MOE_UH) src = a.rowmap[m0 + i];
    else src = m0 + i;
    L.arow[tid] = src;
  }
  lds_fill<TYPE>(&L.tab);
  const KvTab kv = kv_tab();
  const uint32_t hfm = 0u - (uint32_t)hf;  // all ones in the upper half-wave
  __syncthreads();

  // ---- global -> register staging of one superblock's activation rows and scales (issued one superblock ahead)
  u32x4_t st_a[ACH];  // (a native vector type: an array of HIP's uint4 structs is kept in scratch memory)
  float st_sc[SCH], st_u[SCH];
#define QM_FETCH_ACTS(SB)                                                                                  \
  {                                                                                                        \
    _Pragma("unroll") for (int c = 0; c < ACH; ++c) {                                                      \
      const int ch = tid + 256 * c, row = ch >> 4, col = ch & 15;                                          \
      st_a[c] = *(const u32x4_t*)(a.aq + (size_t)L.arow[row] * K + (SB) * 256 + col * 16);                   \
    }                                                                                                      \
    if constexpr (!DUMP) {                                                                                 \
      _Pragma("unroll") for (int c = 0; c < SCH; ++c) {                                                    \
        const int idx = min(tid + 256 * c, 8 * BM - 1), blk = idx / BM, src = L.arow[idx % BM];            \
        st_sc[c] = a.asc[(size_t)(((SB) * 8 + blk) >> a.ash) * a.M_stride + src];                                \
        if constexpr (MINS) {                                                                              \
          const int bs = (int)a.absum[(size_t)(2 * ((SB) * 8 + blk)) * a.M_stride + src] +                 \
                         (int)a.absum[(size_t)(2 * ((SB) * 8 + blk) + 1) * a.M_stride + src];              \
          st_u[c] = st_sc[c] * (float)bs;                                                                  \
        }                                                                                                  \
      }                                                                                                    \
    }                                                                                                      \
  }
#define QM_STORE_ACTS(BUF)                                                                                 \
  {                                                                                                        \
    _Pragma("unroll") for (int c = 0; c < ACH; ++c) {                                                      \
      const int ch = tid + 256 * c, row = ch >> 4, col = ch & 15;                                          \
      *(u32x4_t*)(L.a[BUF] + row * A_STRIDE + col * 16) = st_a[c];                                        \
    }                                                                                                      \
    if constexpr (!DUMP) {                                                                                 \
      _Pragma("unroll") for (int c = 0; c < SCH; ++c) {                                                    \
        const int idx = tid + 256 * c;                                                                     \
        if (idx < 8 * BM) {                                                                                \
          L.asc[BUF][idx] = st_sc[c];                                                                      \
          if constexpr (MINS) L.u[BUF][idx] = st_u[c];                                                     \
        }                                                                                                  \
      }                                                                                                    \
    }                                                                                                      \
  }
  // ---- this lane's weight row: payloads and header, one superblock ahead (rolling: a block's registers are
  // reloaded with the next superblock's block as soon as they are consumed)
  // (gate and up over two slot tiles: a ring of four blocks, two block pairs ahead, for the registers; the types whose
  //  block scales sit in the payloads need the whole superblock at its start)
  constexpr int NP = GU && MT == 2 ? 4 : 8;
  static_assert(NP == 8 || (TYPE != T_IQ2_XXS && TYPE != T_IQ3_XXS && TYPE != T_IQ1_S),
                "payload-held scales need the whole superblock");
  uint4 pay[NP], pay2[GU ? NP : 1];
  uint4 hdr, hdr2 = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int b = 0; b < NP; ++b) pay[b] = load_payload<TYPE>(a.w, n, sb0 * 8 + b, hf);
  hdr = load_header<TYPE>(a.w, n, sb0);
  if constexpr (GU) {
#pragma unroll
    for (int b = 0; b < NP; ++b) pay2[b] = load_payload<TYPE>(a.w2, n, sb0 * 8 + b, hf);
    hdr2 = load_header<TYPE>(a.w2, n, sb0);
  }

  v16f acc[MT], acc2[GU ? MT : 1];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
    if constexpr (GU) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc2[mt][r] = 0.0f;
    }
  }
  const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  v32f zero32;
#pragma unroll
  for (int r = 0; r < 32; ++r) zero32[r] = 0.0f;

  QM_FETCH_ACTS(sb0)
  QM_STORE_ACTS(0)
  __syncthreads();

  for (int s = sb0; s < sb1; ++s) {
    const int cur = (s - sb0) & 1;
    const int sn = s + 1 < sb1 ? s + 1 : s;  // (the last superblock reloads itself: no conditional register state)
    QM_FETCH_ACTS(sn)

    float dsc[8], dmn[8], dsc2[8], dmn2[8];
    int isc[8], isc2[8];
    sb_scales<TYPE>(hdr, pay, dsc, dmn, isc);
    if constexpr (GU) sb_scales<TYPE>(hdr2, pay2, dsc2, dmn2, isc2);
    // each lane carries block 2p + hf's scales into pair p's f32 outer products: picked once per superblock, so only
    // the lane's four blocks stay live (a bit select, not hf ? x[2p+1] : x[2p]: the compiler turns that into a
    // lane-dependent index into the array, which it then keeps in scratch memory)
    float my_dsc4[4], my_dmn4[4], my_dsc24[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      my_dsc4[p] = lane_pick(hfm, dsc[2 * p], dsc[2 * p + 1]);
      my_dmn4[p] = -lane_pick(hfm, dmn[2 * p], dmn[2 * p + 1]);
      my_dsc24[p] = GU ? lane_pick(hfm, dsc2[2 * p], dsc2[2 * p + 1]) : 0.0f;
    }
    const uint4 hcur = hdr, hcur2 = hdr2;
    hdr = load_header<TYPE>(a.w, n, sn);
    if constexpr (GU) hdr2 = load_header<TYPE>(a.w2, n, sn);

#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // superblock sn's activations into the other buffer, halfway through (its loads have had two pairs' time;
      // that buffer's last readers passed the barrier that ended the previous superblock)
      if (p == 2) QM_STORE_ACTS(cur ^ 1)
      // blocks 2p and 2p+1: lanes of k-half hf carry block 2p+hf's scales into the f32 outer-product MFMAs
      const float my_dsc = my_dsc4[p], my_dmn = my_dmn4[p], my_dsc2 = my_dsc24[p];
      v4i bop[2], bop2[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int b = 2 * p + q, sl = b % NP;
        // the block that takes this slot: the next superblock's block b, or (ring of four) block b + 4 of this one
        // for the first two pairs and block b - 4 of the next for the last two
        const int bn = NP == 8 ? sn * 8 + b : (p < 2 ? s * 8 + b + 4 : sn * 8 + b - 4);
        bop[q] = b_operand<TYPE>(pay[sl], hcur, b, hf, kv, &L.tab);
        pay[sl] = load_payload<TYPE>(a.w, n, bn, hf);
        if constexpr (GU) {
          bop2[q] = b_operand<TYPE>(pay2[sl], hcur2, b, hf, kv, &L.tab);
          pay2[sl] = load_payload<TYPE>(a.w2, n, bn, hf);
        }
      }
      if constexpr (MODE == GEMM_DENSE && MT == 2) {
        // both row tiles' MFMAs first, then the epilogues: row tile 0's VALU epilogue runs while row tile 1's
        // MFMAs execute, and row tile 1's epilogue while row tile 0's mins MFMA does
        v16i dv[2][2];
        v32f sc[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const uint4 av = *(const uint4*)(L.a[cur] + (mt * 32 + lc) * A_STRIDE + 32 * (2 * p + q) + 16 * hf);
            const v4i aop = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
            dv[mt][q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[q], zero16, 0, 0, 0);
          }
          if constexpr (!DUMP) {
            const float my_asc = L.asc[cur][(2 * p + hf) * BM + mt * 32 + lc];
            sc[mt] = __builtin_amdgcn_mfma_f32_32x32x1f32(my_asc, my_dsc, zero32, 0, 0, 0);
          }
        }
        if constexpr (DUMP) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int i = mt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3), blk = s * 8 + 2 * p + q;
                if (i < nvalid && n_loc < n_rows)
                  a.dbg_isum[((size_t)(m0 + i) * n_rows + n_loc) * nb + blk] = isc[2 * p + q] * dv[mt][q][r];
              }
        } else {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc[mt][r] = fmaf(sc[mt][r], (float)dv[mt][0][r], acc[mt][r]);
            acc[mt][r] = fmaf(sc[mt][16 + r], (float)dv[mt][1][r], acc[mt][r]);
          }
          if constexpr (MINS) {
            const float my_u = L.u[cur][(2 * p + hf) * BM + mt * 32 + lc];
            acc[mt] = __builtin_amdgcn_mfma_f32_32x32x2f32(my_u, my_dmn, acc[mt], 0, 0, 0);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(acc[mt][r]));
          }
        }
        }
      } else if constexpr (GU && MT == 2 && !DUMP) {
        // two slot tiles share each decoded weight operand; per tile the gate part, then the up part (one pair of
        // MFMA results and one outer product live at a time); a tile with no slots (a half-empty pair) is skipped
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          if (mt > 0 && nvalid <= 32) break;
          __builtin_amdgcn_sched_barrier(0);
          v4i aop[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const uint4 av = *(const uint4*)(L.a[cur] + (mt * 32 + lc) * A_STRIDE + 32 * (2 * p + q) + 16 * hf);
            aop[q] = v4i{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
          }
          const float my_asc = L.asc[cur][(2 * p + hf) * BM + mt * 32 + lc];
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            v16i dv[2];
#pragma unroll
            for (int q = 0; q < 2; ++q)
              dv[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[q], g ? bop2[q] : bop[q], zero16, 0, 0, 0);
            const v32f sc = __builtin_amdgcn_mfma_f32_32x32x1f32(my_asc, g ? my_dsc2 : my_dsc, zero32, 0, 0, 0);
            v16f& ac = g ? acc2[mt] : acc[mt];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              ac[r] = fmaf(sc[r], (float)dv[0][r], ac[r]);
              ac[r] = fmaf(sc[16 + r], (float)dv[1][r], ac[r]);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(ac[r]));
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      } else
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (MODE != GEMM_DENSE && mt > 0 && nvalid <= 32 * mt) break;  // (a pair's empty second tile)
        v16i dv[2], dv2[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint4 av = *(const uint4*)(L.a[cur] + (mt * 32 + lc) * A_STRIDE + 32 * (2 * p + q) + 16 * hf);
          const v4i aop = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
          dv[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[q], zero16, 0, 0, 0);
          if constexpr (GU) dv2[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop2[q], zero16, 0, 0, 0);
        }
        if constexpr (DUMP) {
#pragma unroll
          for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int i = mt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3), blk = s * 8 + 2 * p + q;
              if (i < nvalid && n_loc < n_rows)
                a.dbg_isum[((size_t)(m0 + i) * n_rows + n_loc) * nb + blk] = isc[2 * p + q] * dv[q][r];
            }
        } else {
          // s[i][j] = asc[i][b] * dsc[j][b] for both blocks of the pair: one 2-block f32 outer product (lanes
          // 0-31 carry block 2p, lanes 32-63 block 2p+1; result registers 0-15 / 16-31)
          const float my_asc = L.asc[cur][(2 * p + hf) * BM + mt * 32 + lc];
          const v32f sc = __builtin_amdgcn_mfma_f32_32x32x1f32(my_asc, my_dsc, zero32, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc[mt][r] = fmaf(sc[r], (float)dv[0][r], acc[mt][r]);
            acc[mt][r] = fmaf(sc[16 + r], (float)dv[1][r], acc[mt][r]);
          }
          if constexpr (!MINS) {
            // (pins the accumulator between block pairs: without it the scheduler overlaps every pair's MFMA
            //  results and runs out of registers)
#pragma unroll
            for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(acc[mt][r]));
          }
          if constexpr (MINS) {
            // - sum over the pair of (asc * bsum)[i][b] * (dmin * mn)[j][b]: one K=2 f32 MFMA into the accumulator
            const float my_u = L.u[cur][(2 * p + hf) * BM + mt * 32 + lc];
            acc[mt] = __builtin_amdgcn_mfma_f32_32x32x2f32(my_u, my_dmn, acc[mt], 0, 0, 0);
          }
          if constexpr (GU) {
#pragma unroll
            for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(acc2[mt][r]));
            const v32f sc2 = __builtin_amdgcn_mfma_f32_32x32x1f32(my_asc, my_dsc2, zero32, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              acc2[mt][r] = fmaf(sc2[r], (float)dv2[0][r], acc2[mt][r]);
              acc2[mt][r] = fmaf(sc2[16 + r], (float)dv2[1][r], acc2[mt][r]);
            }
          }
        }
      }
      // (keeps the scheduler from hoisting every pair's MFMAs together, which needs more than 512 registers)
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // superblock s's buffer is free, superblock sn's is complete
  }
#undef QM_FETCH_ACTS
#undef QM_STORE_ACTS
  if constexpr (DUMP) return;

  // ---- epilogue
  const bool col_ok = n_loc < n_rows;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = mt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
      const bool row_ok = i < nvalid;
      if constexpr (MODE == GEMM_DENSE) {
        if (row_ok && col_ok) {
          float* cp = a.C + (size_t)(m0 + i) * a.ldc + a.c_off + n_loc;
          float v = acc[mt][r];
          if (gridDim.z > 1) {  // (K split: C was zeroed; 0 + x + y is the same float in either order)
            unsafeAtomicAdd(cp, v);
            continue;
          }
          if (a.accumulate == 1) {
            v += *cp;
          } else if (a.accumulate == 2) {
            const float g = *cp;
            v *= g / (1.0f + expf(-g));
          }
          *cp = v;
        }
      } else {
        moe_store<MODE>(a, m0 + i, n_loc, row_ok && col_ok, acc[mt][r], GU ? acc2[mt][r] : 0.0f, lc);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Prompt GEMM of the types with an integer scale per 16 elements (Q6_K, IQ2_XS, IQ2_S): each 32-block needs its two
// halves' int32 sums separately (the reference's sc0 * lo + sc1 * hi): two v_mfma_i32_32x32x16_i8 per block and row
// tile, lane half h holding elements 8h..8h+7 of each 16-element half. The B operand is decoded in registers to
// signed int8 (Q6_K: the 6-bit value minus 32, a byte-wise subtract without borrows; IQ2: grid words with their
// signs, groups h and 2 + h of the block); one 2-block f32 outer product gives asc * d * sc for both halves (lanes
// 0-31: the first half's scale, lanes 32-63: the second's). Tiles, staging and epilogue as gemm_kernel's dense mode.
template <int TYPE, int MT, int MODE, bool DUMP>
__global__ __launch_bounds__(256, 2) void gemm_s16_kernel(GemmArgs a) {
  constexpr int BM = 32 * MT;
  constexpr int ACH = BM * 16 / 256;
  constexpr int SCH = (8 * BM + 255) / 256;
  using Tr = Traits<TYPE>;
  __shared__ GemmLds<TYPE, MT> L;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, lc = lane & 31;
  const int K = a.w.K, nb = K / 32, nsb = K / 256;
  int m0, nvalid, wrow0, nt;
  if (!tile_rows<MODE, BM>(a, m0, nvalid, wrow0, nt)) return;
  const int n_loc = nt * 128 + wave * 32 + lc;
  const int n_rows = MODE == GEMM_DENSE ? a.w.rows : a.expert_rows;
  const int n = wrow0 + min(n_loc, n_rows - 1);
  if (tid < BM) {
    const int i = min(tid, nvalid - 1);
    L.arow[tid] = (MODE == GEMM_MOE_G || MODE == GEMM_MOE_UH) ? a.rowmap[m0 + i] : m0 + i;
  }
  lds_fill<TYPE>(&L.tab);
  __syncthreads();

  u32x4_t st_a[ACH];
  float st_sc[SCH];
  auto fetch = [&](int sb) {
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const int ch = tid + 256 * c, row = ch >> 4, col = ch & 15;
      st_a[c] = *(const u32x4_t*)(a.aq + (size_t)L.arow[row] * K + sb * 256 + col * 16);
    }
    if constexpr (!DUMP) {
#pragma unroll
      for (int c = 0; c < SCH; ++c) {
        const int idx = min(tid + 256 * c, 8 * BM - 1), blk = idx / BM, src = L.arow[idx % BM];
        st_sc[c] = a.asc[(size_t)((sb * 8 + blk) >> a.ash) * a.M_stride + src];
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const int ch = tid + 256 * c, row = ch >> 4, col = ch & 15;
      *(u32x4_t*)(L.a[buf] + row * A_STRIDE + col * 16) = st_a[c];
    }
    if constexpr (!DUMP) {
#pragma unroll
      for (int c = 0; c < SCH; ++c) {
        const int idx = tid + 256 * c;
        if (idx < 8 * BM) L.asc[buf][idx] = st_sc[c];
      }
    }
  };
  // this lane's share of a block: Q6_K nibble bytes 8h..8h+7 and both 2-bit words (record: 16 nibble bytes, 2
  // words); Q3_K its whole record (nib: the 2-bit words, hw.x: the high bits); IQ2_XS / IQ2_S the block's whole
  // 8-byte record (nib)
  const uint8_t* qrow = a.w.qs + (size_t)n * nb * Tr::QB;
  const uint8_t* hrow = a.w.hdr + (size_t)n * nsb * Tr::HB;
  auto load_blk = [&](int blk, uint2& nib, uint2& hw) {
    const uint8_t* r = qrow + (size_t)blk * Tr::QB;
    if constexpr (TYPE == T_Q6_K) {
      nib = *(const uint2*)(r + 8 * hf);
      hw = *(const uint2*)(r + 16);
    } else if constexpr (TYPE == T_Q3_K) {  // (the block's two words of 2-bit fields and its word of high bits)
      nib = *(const uint2*)r;
      hw = make_uint2(*(const uint32_t*)(r + 8), 0u);
    } else if constexpr (TYPE == T_Q2_K) {
      nib = *(const uint2*)r;
      hw = make_uint2(0u, 0u);
    } else {
      nib = *(const uint2*)r;
      hw = make_uint2(0u, 0u);
    }
  };
  uint2 nib[8], hw[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) load_blk(b, nib[b], hw[b]);
  // (header records are 20 or 12 bytes: 4-byte aligned, so read as dwords) sc: Q6_K / Q3_K int8 scales[16], IQ2_XS
  // scales[8] (.x .y), IQ2_S qh[8] (.x .y) and scales[8] (.z .w); dd: f16 d
  auto load_hdr = [&](int sb, uint4& sc, uint32_t& dd) {
    const uint32_t* h = (const uint32_t*)(hrow + (size_t)sb * Tr::HB);
    if constexpr (TYPE == T_IQ2_XS) {
      sc = make_uint4(h[0], h[1], 0u, 0u);
      dd = h[2];
    } else if constexpr (TYPE == T_Q2_K) {  // (d and dmin first, then the 16 scale / min bytes)
      sc = make_uint4(h[1], h[2], h[3], h[4]);
      dd = h[0];
    } else if constexpr (TYPE == T_IQ1_M) {  // (d alone: the scales are in the payloads)
      sc = make_uint4(0u, 0u, 0u, 0u);
      dd = h[0];
    } else {
      sc = make_uint4(h[0], h[1], h[2], h[3]);
      dd = h[4];
    }
  };
  uint4 hsc;
  uint32_t hd;
  load_hdr(0, hsc, hd);
  v16f acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
  const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  v32f zero32;
#pragma unroll
  for (int r = 0; r < 32; ++r) zero32[r] = 0.0f;
  fetch(0);
  store(0);
  __syncthreads();

  for (int s = 0; s < nsb; ++s) {
    const int cur = s & 1;
    const int sn = s + 1 < nsb ? s + 1 : s;
    fetch(sn);
    const uint32_t scw[4] = {hsc.x, hsc.y, hsc.z, hsc.w};
    const float d = (TYPE == T_Q6_K || TYPE == T_Q3_K || TYPE == T_Q2_K) ? h2f(hd) : h2f(hd) * kIqDScale<TYPE>;
    const float dmin = TYPE == T_Q2_K ? h2f(hd >> 16) : 0.0f;
    load_hdr(sn, hsc, hd);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      if (b == 4) store(cur ^ 1);
      // B operands: elements 8hf..8hf+7 of the block's first half (o0) and of its second half (o1), signed
      uint32_t w[4];
      int sc0, sc1, mn0 = 0, mn1 = 0;
      if constexpr (TYPE == T_Q2_K) {
        const uint32_t wd[4] = {2u * hf, 2u * hf + 1, 4u + 2 * hf, 5u + 2 * hf};
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = ((wd[k] < 4 ? nib[b].x : nib[b].y) >> (2 * (wd[k] & 3))) & 0x03030303u;
        const uint32_t sm = (scw[b >> 1] >> (16 * (b & 1))) & 0xFFFFu;
        sc0 = (int)(sm & 0xFu);
        mn0 = (int)((sm >> 4) & 0xFu);
        sc1 = (int)((sm >> 8) & 0xFu);
        mn1 = (int)(sm >> 12);
      } else if constexpr (TYPE == T_Q6_K) {
        const uint32_t A2 = hf ? hw[b].x : hw[b].x << 4, B2 = hf ? hw[b].y : hw[b].y << 4;
        w[0] = (nib[b].x & 0x0F0F0F0Fu) | (A2 & 0x30303030u);
        w[1] = (nib[b].y & 0x0F0F0F0Fu) | ((A2 >> 2) & 0x30303030u);
        w[2] = ((nib[b].x >> 4) & 0x0F0F0F0Fu) | (B2 & 0x30303030u);
        w[3] = ((nib[b].y >> 4) & 0x0F0F0F0Fu) | ((B2 >> 2) & 0x30303030u);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = ((w[k] | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
        sc0 = (int)(int8_t)((scw[b >> 1] >> (16 * (b & 1))) & 0xFFu);
        sc1 = (int)(int8_t)((scw[b >> 1] >> (16 * (b & 1) + 8)) & 0xFFu);
      } else if constexpr (TYPE == T_IQ1_M) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {  // (groups hf and 2 + hf: elements 8 hf .. 8 hf + 7 of each 16-element half)
          uint32_t idx;
          bool neg;
          iq1_index<TYPE>(nib[b].x, nib[b].y, hf + 2 * g, idx, neg);
          iq1_group(&L.tab, idx, neg, w[2 * g], w[2 * g + 1]);
        }
        sc0 = 2 * (int)((nib[b].y >> 16) & 7u) + 1;
        sc1 = 2 * (int)((nib[b].y >> 19) & 7u) + 1;
      } else if constexpr (TYPE == T_Q3_K) {
        w[0] = q3_word(nib[b].x, nib[b].y, hw[b].x, 2 * hf);
        w[1] = q3_word(nib[b].x, nib[b].y, hw[b].x, 2 * hf + 1);
        w[2] = q3_word(nib[b].x, nib[b].y, hw[b].x, 4 + 2 * hf);
        w[3] = q3_word(nib[b].x, nib[b].y, hw[b].x, 5 + 2 * hf);
        sc0 = (int)(int8_t)((scw[b >> 1] >> (16 * (b & 1))) & 0xFFu);
        sc1 = (int)(int8_t)((scw[b >> 1] >> (16 * (b & 1) + 8)) & 0xFFu);
      } else {
        const uint32_t qh = TYPE == T_IQ2_S ? (scw[b >> 2] >> (8 * (b & 3))) & 0xFFu : 0u;
        iq_group<TYPE>(&L.tab, nib[b].x, nib[b].y, 0u, qh, hf, w[0], w[1]);
        iq_group<TYPE>(&L.tab, nib[b].x, nib[b].y, 0u, qh, 2 + hf, w[2], w[3]);
        const uint32_t sb = (scw[(TYPE == T_IQ2_S ? 2 : 0) + (b >> 2)] >> (8 * (b & 3))) & 0xFFu;
        sc0 = 1 + 2 * (int)(sb & 0xFu);
        sc1 = 1 + 2 * (int)(sb >> 4);
      }
      const long o0 = (long)(((uint64_t)w[1] << 32) | w[0]), o1 = (long)(((uint64_t)w[3] << 32) | w[2]);
      load_blk(sn * 8 + b, nib[b], hw[b]);
      const float my_dsc = d * (float)(hf ? sc1 : sc0);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (MODE != GEMM_DENSE && mt > 0 && nvalid <= 32 * mt) break;  // (a pair's empty second tile)
        const uint8_t* ar = L.a[cur] + (mt * 32 + lc) * A_STRIDE + 32 * b + 8 * hf;
        const long a0 = *(const long*)ar, a1 = *(const long*)(ar + 16);
        const v16i d0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, o0, zero16, 0, 0, 0);
        const v16i d1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1, o1, zero16, 0, 0, 0);
        if constexpr (DUMP) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int i = mt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (i < nvalid && n_loc < n_rows)
              a.dbg_isum[((size_t)(m0 + i) * n_rows + n_loc) * nb + s * 8 + b] = sc0 * d0[r] + sc1 * d1[r];
          }
        } else {
          const float my_asc = L.asc[cur][b * BM + mt * 32 + lc];
          const v32f sc = __builtin_amdgcn_mfma_f32_32x32x1f32(my_asc, my_dsc, zero32, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc[mt][r] = fmaf(sc[r], (float)d0[r], acc[mt][r]);
            acc[mt][r] = fmaf(sc[16 + r], (float)d1[r], acc[mt][r]);
          }
          if constexpr (kMin16<TYPE>) {
            // the mins per 16: acc -= sum over the halves h of (asc * bsum_h)[token] * (dmin * mn_h)[row], one K = 2 f32
            // outer product (lane half hf: half hf); bsum_h of the token row from its staged int8 values
            const uint4 av = *(const uint4*)(L.a[cur] + (mt * 32 + lc) * A_STRIDE + 32 * b + 16 * hf);
            int bs = dot4(av.x, 0x01010101u, 0);
            bs = dot4(av.y, 0x01010101u, bs);
            bs = dot4(av.z, 0x01010101u, bs);
            bs = dot4(av.w, 0x01010101u, bs);
            const float my_u = my_asc * (float)bs, my_t = -dmin * (float)(hf ? mn1 : mn0);
            acc[mt] = __builtin_amdgcn_mfma_f32_32x32x2f32(my_u, my_t, acc[mt], 0, 0, 0);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(acc[mt][r]));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
  }
  if constexpr (DUMP) return;
  const bool col_ok = n_loc < n_rows;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = mt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
      if constexpr (MODE == GEMM_DENSE) {
        if (i < nvalid && col_ok) {
          float* cp = a.C + (size_t)(m0 + i) * a.ldc + a.c_off + n_loc;
          float v = acc[mt][r];
          if (a.accumulate == 1) {
            v += *cp;
          } else if (a.accumulate == 2) {
            const float g = *cp;
            v *= g / (1.0f + expf(-g));
          }
          *cp = v;
        }
      } else {
        moe_store<MODE>(a, m0 + i, n_loc, i < nvalid && col_ok, acc[mt][r], 0.0f, lc);
      }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// MoE down projection, weight-stationary: a work-group owns 128 output columns (weight rows n of one expert, one
// 32-row MFMA tile per wave) and walks `group` consecutive slot tiles of the tile list. Each lane decodes its row's
// whole K = F (KB superblocks, 8 * KB 32-blocks of its k-half) into int8 MFMA B operands once per expert and keeps
// them in registers (64 registers at F = 512), so an expert's weights are decoded once per work-group instead of once
// per slot tile. Per slot tile: the 32 quantized h rows (int8, F bytes each), their per-32 scales and routing weights
// are staged in LDS (the next tile's loads are issued before the current tile's MFMAs); per block pair two
// v_mfma_i32_32x32x32_i8 give the exact int32 block sums, one 2-block f32 outer product asc * d * sc, and 32 VALU
// scale-accumulate in f32 -- the arithmetic of gemm_kernel's MOE_DOWN mode, so the results are the same bits.
// (Measured: double-buffered LDS with the y stores issued before the next tile's staging ran slower.)
constexpr int RW_STRIDE = 16;  // LDS padding per staged row (bytes): rows of F + 16 bytes spread the operand reads

template <int TYPE, int KB>
__global__ __launch_bounds__(256, 2) void moe_down_rw_kernel(GemmArgs a, int group) {
  constexpr int NB = 8 * KB, F = 256 * KB, RS = F + RW_STRIDE;
  constexpr int ACH = 32 * F / 16 / 256;   // 16-byte chunks of the A tile per thread
  constexpr int SCH = (NB * 32 + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint8_t sa[32 * RS];
  __shared__ float ssc[NB * 32];
  __shared__ float srs[32];
  __shared__ typename LdsFor<TYPE>::type tab;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, lc = lane & 31;
  const int ntile = a.tiles[0];
  const int t0 = blockIdx.y * group;
  if (t0 >= ntile) return;
  const int t1 = min(t0 + group, ntile);
  const int n_loc = blockIdx.x * 128 + wave * 32 + lc;  // output column = weight row within the expert
  const bool col_ok = n_loc < a.expert_rows;
  const uint32_t hfm = 0u - (uint32_t)hf;
  lds_fill<TYPE>(&tab);
  const KvTab kv = kv_tab();
  const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  v32f zero32;
#pragma unroll
  for (int r = 0; r < 32; ++r) zero32[r] = 0.0f;

  u32x4_t st_a[ACH];
  float st_sc[SCH], st_rs = 0.0f;
  auto fetch = [&](int t) {
    const int m0 = a.tiles[2 + 3 * t], nr = a.tiles[3 + 3 * t];
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const int ch = tid + 256 * c, row = ch / (F / 16), col = ch % (F / 16);
      st_a[c] = *(const u32x4_t*)(a.aq + (size_t)(m0 + min(row, max(nr, 1) - 1)) * F + col * 16);
    }
#pragma unroll
    for (int c = 0; c < SCH; ++c) {
      const int idx = min(tid + 256 * c, NB * 32 - 1), blk = idx >> 5, row = idx & 31;
      st_sc[c] = a.asc[(size_t)blk * a.M_stride + m0 + min(row, max(nr, 1) - 1)];
    }
    if (tid < 32) st_rs = a.rowscale[m0 + min(tid, max(nr, 1) - 1)];
  };

  v4i bop[NB];
  float my_dsc[NB / 2];
  int cur_e = -1;
  fetch(t0);
  for (int t = t0; t < t1; ++t) {
    const int e = a.tiles[1 + 3 * t], m0 = a.tiles[2 + 3 * t], nr = a.tiles[3 + 3 * t];
    __syncthreads();  // (the previous tile's operand reads are done)
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const int ch = tid + 256 * c, row = ch / (F / 16), col = ch % (F / 16);
      *(u32x4_t*)(sa + row * RS + col * 16) = st_a[c];
    }
#pragma unroll
    for (int c = 0; c < SCH; ++c) {
      const int idx = tid + 256 * c;
      if (idx < NB * 32) ssc[idx] = st_sc[c];
    }
    if (tid < 32) srs[tid] = st_rs;
    if (e != cur_e) {  // (uniform: one tile, one expert) this lane's row of expert e, decoded
      cur_e = e;
      const int n = e * a.expert_rows + min(n_loc, a.expert_rows - 1);
#pragma unroll
      for (int sb = 0; sb < KB; ++sb) {
        uint4 pay[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) pay[b] = load_payload<TYPE>(a.w, n, sb * 8 + b, hf);
        const uint4 hdr = load_header<TYPE>(a.w, n, sb);
        float dsc[8], dmn[8];
        int isc[8];
        sb_scales<TYPE>(hdr, pay, dsc, dmn, isc);
#pragma unroll
        for (int b = 0; b < 8; ++b) bop[sb * 8 + b] = b_operand<TYPE>(pay[b], hdr, b, hf, kv, &tab);
#pragma unroll
        for (int p = 0; p < 4; ++p) my_dsc[sb * 4 + p] = lane_pick(hfm, dsc[2 * p], dsc[2 * p + 1]);
      }
    }
    __syncthreads();
    if (t + 1 < t1) fetch(t + 1);  // (the next tile's loads fly during this tile's MFMAs)
    if (nr == 0) continue;  // (an empty tile: the second of an expert's last pair)
    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int p = 0; p < NB / 2; ++p) {
      v16i dv[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint4 av = *(const uint4*)(sa + lc * RS + 32 * (2 * p + q) + 16 * hf);
        const v4i aop = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
        dv[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop[2 * p + q], zero16, 0, 0, 0);
      }
      const float my_asc = ssc[(2 * p + hf) * 32 + lc];
      const v32f sc = __builtin_amdgcn_mfma_f32_32x32x1f32(my_asc, my_dsc[p], zero32, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[r] = fmaf(sc[r], (float)dv[0][r], acc[r]);
        acc[r] = fmaf(sc[16 + r], (float)dv[1][r], acc[r]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(acc[r]));
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r >> 2) + 4 * hf + (r & 3);
      if (i < nr && col_ok) a.C[(size_t)(m0 + i) * a.ldc + n_loc] = srs[i] * acc[r];
    }
  }
}

// Slot tiles per work-group of moe_down_rw_kernel
// (measured at the BASELINE MoE shape: 2 tiles 257 us, 4 217, 8 207, 16 221)
constexpr int kDownRwGroup = 8;

template <int TYPE, int KB>
static hipError_t go_down_rw(const GemmArgs& a, hipStream_t s) {
  const unsigned gx = (unsigned)((a.expert_rows + 127) / 128);
  const unsigned gy = (unsigned)((a.max_tiles + kDownRwGroup - 1) / kDownRwGroup);
  moe_down_rw_kernel<TYPE, KB><<<dim3(gx, gy), dim3(256), 0, s>>>(a, kDownRwGroup);
  return hipGetLastError();
}

template <int TYPE, int MT, int MODE, bool DUMP>
static hipError_t go_s16(const GemmArgs& a, hipStream_t s) {
  const int n_rows = MODE == GEMM_DENSE ? a.w.rows : a.expert_rows;
  const unsigned gx = (unsigned)((n_rows + 127) / 128);
  const unsigned gy = MODE == GEMM_DENSE      ? (unsigned)((a.M + 32 * MT - 1) / (32 * MT))
                     : 32 * MT > kMoeTileRows ? (unsigned)((a.max_tiles + 1) / 2)
                                              : (unsigned)(a.max_tiles * (kMoeTileRows / (32 * MT)));
  gemm_s16_kernel<TYPE, MT, MODE, DUMP><<<dim3(gx, gy), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

// zeroes C[m][c_off .. c_off + n) for m < M (a kernel, not a memset, so the call stays capturable in a HIP graph)
__global__ void zero_rows_kernel(float* C, int ldc, int c_off, int n, int M) {
  const int m = blockIdx.y;
  for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) C[(size_t)m * ldc + c_off + j] = 0.0f;
}

template <int TYPE, int MT, int MODE, bool DUMP>
static hipError_t go(const GemmArgs& a, hipStream_t s) {
  const int n_rows = MODE == GEMM_DENSE ? a.w.rows : a.expert_rows;
  const unsigned gx = (unsigned)((n_rows + 127) / 128);
  const unsigned gy = MODE == GEMM_DENSE      ? (unsigned)((a.M + 32 * MT - 1) / (32 * MT))
                     : 32 * MT > kMoeTileRows ? (unsigned)((a.max_tiles + 1) / 2)
                                              : (unsigned)(a.max_tiles * (kMoeTileRows / (32 * MT)));
  // A dense product with too few tiles to give every CU two work-groups (M = 512, N = 5120: 320 tiles) splits K in two:
  // each half adds its partial sums into a zeroed C, so the grid doubles. Two partials keep the result deterministic
  // (0 + x + y rounds the same in either order); only with accumulate = 0 (C + x + y would not).
  unsigned gz = 1;
  if (MODE == GEMM_DENSE && !DUMP && a.accumulate == 0 && gx * gy < 512 && a.w.K / 256 >= 8) {
    gz = 2;
    zero_rows_kernel<<<dim3((unsigned)((n_rows + 255) / 256), (unsigned)a.M), dim3(256), 0, s>>>(a.C, a.ldc, a.c_off,
                                                                                                   n_rows, a.M);
  }
  gemm_kernel<TYPE, MT, MODE, DUMP><<<dim3(gx, gy, gz), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t dispatch(int mode, const GemmArgs& a, hipStream_t s) {
  // (the block-sum mode takes the product's row-tile count, so the sums checked are those of the kernel that runs)
  if (a.dbg_isum) return a.M <= 32 ? go<TYPE, 1, GEMM_DENSE, true>(a, s) : go<TYPE, 2, GEMM_DENSE, true>(a, s);
  switch (mode) {
    case GEMM_DENSE:
      return a.M <= 32 ? go<TYPE, 1, GEMM_DENSE, false>(a, s) : go<TYPE, 2, GEMM_DENSE, false>(a, s);
    case GEMM_MOE_GATEUP:
      // (two slot tiles per work-group, each decoded weight operand feeding both; IQ2_XXS / IQ3_XXS keep their block
      //  scales in the payloads, which the two-tile kernel's payload ring does not hold whole)
      if constexpr (TYPE != T_IQ2_XXS && TYPE != T_IQ3_XXS && TYPE != T_IQ1_S)
        return go<TYPE, 2, GEMM_MOE_GATEUP, false>(a, s);
      return go<TYPE, 1, GEMM_MOE_GATEUP, false>(a, s);
    case GEMM_MOE_DOWN:
      // (expert width F <= 512: the whole row's operands fit in registers; types with mins are not MoE types)
      if constexpr (!Traits<TYPE>::MINS) {
        if (a.w.K == 256) return go_down_rw<TYPE, 1>(a, s);
        if (a.w.K == 512) return go_down_rw<TYPE, 2>(a, s);
        // (F = 768, e.g. Qwen3-30B-A3B: 96 operand registers, a few spilled; measured 0.88 -> 0.77 ms for the layer
        //  against two slot tiles per work-group in the tile kernel)
        if (a.w.K == 768) return go_down_rw<TYPE, 3>(a, s);
      }
      // wider experts (and the payload-scale types IQ2_XXS / IQ3_XXS): two slot tiles per work-group (0.88 -> 0.85 ms
      // at F = 768)
      return go<TYPE, 2, GEMM_MOE_DOWN, false>(a, s);
    // (gate and up of different types: each launch over slot-tile pairs as well; measured 227 -> 181 us for the gate
    //  launch at the BASELINE MoE shape)
    case GEMM_MOE_G: return go<TYPE, 2, GEMM_MOE_G, false>(a, s);
    case GEMM_MOE_UH: return go<TYPE, 2, GEMM_MOE_UH, false>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE>
static hipError_t dispatch_s16(int mode, const GemmArgs& a, hipStream_t s) {
  if (a.dbg_isum) return a.M <= 32 ? go_s16<TYPE, 1, GEMM_DENSE, true>(a, s) : go_s16<TYPE, 2, GEMM_DENSE, true>(a, s);
  switch (mode) {
    case GEMM_DENSE:
      return a.M <= 32 ? go_s16<TYPE, 1, GEMM_DENSE, false>(a, s) : go_s16<TYPE, 2, GEMM_DENSE, false>(a, s);
    // (MoE modes over slot-tile pairs: at the BASELINE MoE shape Q6_K down 0.94 -> 0.82 ms for the layer, all-Q6_K
    //  1.50 -> 1.16, IQ2_XS unchanged)
    case GEMM_MOE_G: return go_s16<TYPE, 2, GEMM_MOE_G, false>(a, s);
    case GEMM_MOE_UH: return go_s16<TYPE, 2, GEMM_MOE_UH, false>(a, s);
    case GEMM_MOE_DOWN: return go_s16<TYPE, 2, GEMM_MOE_DOWN, false>(a, s);
    default: return hipErrorInvalidValue;  // (gate and up in one launch: the int8 kernel's GATEUP mode only)
  }
}

hipError_t launch_gemm(int type, int mode, const GemmArgs& a, hipStream_t s) {
  switch (type) {
    case T_Q6_K: return dispatch_s16<T_Q6_K>(mode, a, s);
    case T_Q3_K: return dispatch_s16<T_Q3_K>(mode, a, s);
    case T_Q2_K: return mode == GEMM_DENSE ? dispatch_s16<T_Q2_K>(mode, a, s) : hipErrorInvalidValue;
    case T_IQ1_M: return mode == GEMM_DENSE ? dispatch_s16<T_IQ1_M>(mode, a, s) : hipErrorInvalidValue;
    case T_IQ2_XS: return dispatch_s16<T_IQ2_XS>(mode, a, s);
    case T_IQ2_S: return dispatch_s16<T_IQ2_S>(mode, a, s);
    default: break;
  }
  switch (type) {
    case T_Q8_0: return dispatch<T_Q8_0>(mode, a, s);
    case T_Q4_K: return dispatch<T_Q4_K>(mode, a, s);
    case T_IQ4_XS: return dispatch<T_IQ4_XS>(mode, a, s);
    case T_IQ3_S: return dispatch<T_IQ3_S>(mode, a, s);
    case T_Q4_0: return dispatch<T_Q4_0>(mode, a, s);
    case T_Q2_0: return dispatch<T_Q2_0>(mode, a, s);
    case T_IQ4_NL: return dispatch<T_IQ4_NL>(mode, a, s);
    case T_Q5_K: return mode == GEMM_DENSE ? dispatch<T_Q5_K>(mode, a, s) : hipErrorInvalidValue;
    case T_IQ2_XXS: return dispatch<T_IQ2_XXS>(mode, a, s);
    case T_IQ3_XXS: return dispatch<T_IQ3_XXS>(mode, a, s);
    case T_IQ1_S: return mode == GEMM_DENSE ? dispatch<T_IQ1_S>(mode, a, s) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm
