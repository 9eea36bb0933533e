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
#include "qm_launch.h"

namespace qm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int A_STRIDE = 272;  // LDS bytes per staged activation row

template <int TYPE, int MT> struct GemmLds {
  uint8_t a[32 * MT * A_STRIDE];
  float asc[8 * 32 * MT];
  float u[Traits<TYPE>::MINS ? 8 * 32 * MT : 1];
  int arow[32 * MT];
  typename std::conditional<TYPE == T_IQ3_S, Iq3Lds, int>::type iq3;
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

// Per-superblock weight scales of row n: dsc[b] = d * sc_b (Q8_0: the block's f16 scale), dmn[b] = dmin * mn_b;
// isc[b] = the integer scale (for the block-sum hook).
template <int TYPE>
__device__ __forceinline__ void sb_scales(const WView& w, int n, int s, float dsc[8], float dmn[8], int isc[8]) {
  using Tr = Traits<TYPE>;
  const uint8_t* hp = w.hdr + ((size_t)n * (w.K / 256) + s) * Tr::HB;
  if constexpr (TYPE == T_Q8_0) {
    const uint4 h = *(const uint4*)hp;
    const uint32_t hh[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      dsc[b] = h2f(hh[b >> 1] >> (16 * (b & 1)));
      dmn[b] = 0.0f;
      isc[b] = 1;
    }
  } else if constexpr (TYPE == T_Q4_K) {
    const uint4 h = *(const uint4*)hp;
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
    const uint2 h = *(const uint2*)hp;
    const float d = h2f(h.x);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      isc[b] = iq4xs_scale(h.x, h.y, b);
      dsc[b] = d * (float)isc[b];
      dmn[b] = 0.0f;
    }
  } else {
    const uint4 h = *(const uint4*)hp;
    const float d = h2f(h.w);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      isc[b] = 1 + 2 * (int)((h.z >> (4 * b)) & 0xFu);
      dsc[b] = d * (float)isc[b];
      dmn[b] = 0.0f;
    }
  }
}

// The MFMA B operand of row n, 32-block blk, k-half hf: 16 int8 weights.
template <int TYPE>
__device__ __forceinline__ v4i b_operand(const WView& w, const Iq3Lds* iq3, const KvTab& kv, int n, int blk, int hf,
                                         int s) {
  using Tr = Traits<TYPE>;
  const int nb = w.K / 32;
  const uint8_t* qp = w.qs + ((size_t)n * nb + blk) * Tr::QB;
  v4i r;
  if constexpr (TYPE == T_Q8_0) {
    const uint4 q = *(const uint4*)(qp + 16 * hf);
    r[0] = (int)q.x; r[1] = (int)q.y; r[2] = (int)q.z; r[3] = (int)q.w;
  } else if constexpr (TYPE == T_Q4_K || TYPE == T_IQ4_XS) {
    const uint4 q = *(const uint4*)qp;
    const int sh = 4 * hf;
    uint32_t x0 = q.x >> sh, x1 = q.y >> sh, x2 = q.z >> sh, x3 = q.w >> sh;
    if constexpr (TYPE == T_Q4_K) {
      r[0] = (int)(x0 & 0x0F0F0F0Fu); r[1] = (int)(x1 & 0x0F0F0F0Fu);
      r[2] = (int)(x2 & 0x0F0F0F0Fu); r[3] = (int)(x3 & 0x0F0F0F0Fu);
    } else {
      r[0] = (int)kv_lookup4(kv, x0); r[1] = (int)kv_lookup4(kv, x1);
      r[2] = (int)kv_lookup4(kv, x2); r[3] = (int)kv_lookup4(kv, x3);
    }
  } else {
    const uint32_t* qw = (const uint32_t*)qp;
    const uint32_t q0 = qw[0], q1 = qw[1], sg = qw[2];
    const uint8_t* hp = w.hdr + ((size_t)n * (w.K / 256) + s) * Tr::HB;
    const uint32_t qh = hp[blk & 7];
    uint32_t w0, w1, w2, w3;
    iq3s_pair_rt(iq3, q0, q1, qh, sg, 2 * hf, w0, w1);
    iq3s_pair_rt(iq3, q0, q1, qh, sg, 2 * hf + 1, w2, w3);
    r[0] = (int)w0; r[1] = (int)w1; r[2] = (int)w2; r[3] = (int)w3;
  }
  return r;
}

template <int TYPE, int MT, int MODE, bool DUMP>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
  constexpr int BM = 32 * MT;
  constexpr bool MINS = Traits<TYPE>::MINS;
  __shared__ GemmLds<TYPE, MT> L;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, lc = lane & 31;
  const int K = a.w.K, nb = K / 32, nsb = K / 256;

  // ---- which rows: dense (M tile), or one MoE tile (expert e, slots r0 .. r0 + nr - 1)
  int m0, nvalid, wrow0;
  if constexpr (MODE == GEMM_DENSE) {
    m0 = blockIdx.y * BM;
    nvalid = min(BM, a.M - m0);
    wrow0 = 0;
  } else {
    const int t = blockIdx.y;
    if (t >= a.tiles[0]) return;
    const int e = a.tiles[1 + 3 * t];
    m0 = a.tiles[2 + 3 * t];
    nvalid = a.tiles[3 + 3 * t];
    wrow0 = e * a.expert_rows;
  }
  const int n_loc = blockIdx.x * 128 + wave * 32 + lc;  // this lane's weight row (within the expert)
  const int n_rows = MODE == GEMM_DENSE ? a.w.rows : a.expert_rows;
  const int n = wrow0 + min(n_loc, n_rows - 1);

  if (tid < BM) {
    const int i = min(tid, nvalid - 1);
    int src;
    if constexpr (MODE == GEMM_DENSE) src = m0 + i;
    else if constexpr (MODE == GEMM_MOE_GATEUP) src = a.rowmap[m0 + i];
    else src = m0 + i;
    L.arow[tid] = src;
  }
  if constexpr (TYPE == T_IQ3_S) iq3_lds_fill(&L.iq3);
  const KvTab kv = kv_tab();

  float acc[MT][16], acc2[MODE == GEMM_MOE_GATEUP ? MT : 1][16];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
  if constexpr (MODE == GEMM_MOE_GATEUP) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc2[mt][r] = 0.0f;
  }

  const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int s = 0; s < nsb; ++s) {
    __syncthreads();
    // stage the activation rows of superblock s
#pragma unroll
    for (int c = tid; c < BM * 16; c += 256) {
      const int row = c >> 4, col = c & 15;
      const uint4 v = *(const uint4*)(a.aq + (size_t)L.arow[row] * K + s * 256 + col * 16);
      *(uint4*)(L.a + row * A_STRIDE + col * 16) = v;
    }
    for (int c = tid; c < 8 * BM && !DUMP; c += 256) {
      const int blk = c / BM, i = c % BM, src = L.arow[i];
      const float sc = a.asc[(size_t)(s * 8 + blk) * a.M_stride + src];
      L.asc[c] = sc;
      if constexpr (MINS) {
        const int bs = (int)a.absum[(size_t)(2 * (s * 8 + blk)) * a.M_stride + src] +
                       (int)a.absum[(size_t)(2 * (s * 8 + blk) + 1) * a.M_stride + src];
        L.u[c] = sc * (float)bs;
      }
    }
    __syncthreads();

    float dsc[8], dmn[8], dsc2[8], dmn2[8];
    int isc[8], isc2[8];
    sb_scales<TYPE>(a.w, n, s, dsc, dmn, isc);
    if constexpr (MODE == GEMM_MOE_GATEUP) sb_scales<TYPE>(a.w2, n, s, dsc2, dmn2, isc2);

#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int blk = s * 8 + b;
      const v4i bop = b_operand<TYPE>(a.w, (const Iq3Lds*)&L.iq3, kv, n, blk, hf, s);
      v4i bop2;
      if constexpr (MODE == GEMM_MOE_GATEUP) bop2 = b_operand<TYPE>(a.w2, (const Iq3Lds*)&L.iq3, kv, n, blk, hf, s);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 av = *(const uint4*)(L.a + (mt * 32 + lc) * A_STRIDE + 32 * b + 16 * hf);
        const v4i aop = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
        const v16i dv = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, zero16, 0, 0, 0);
        v16i dv2;
        if constexpr (MODE == GEMM_MOE_GATEUP) dv2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop2, zero16, 0, 0, 0);
        if constexpr (DUMP) {
          // block sums of rows m0 + i(r), weight row n_loc: isum[(m*rows + n)*nb + blk] = sc * sum
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int i = mt * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (i < nvalid && n_loc < n_rows)
              a.dbg_isum[((size_t)(m0 + i) * n_rows + n_loc) * nb + blk] = isc[b] * dv[r];
          }
        } else {
          float sr[16], ur[16];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 v = *(const float4*)(L.asc + b * BM + mt * 32 + 8 * q + 4 * hf);
            sr[4 * q] = v.x; sr[4 * q + 1] = v.y; sr[4 * q + 2] = v.z; sr[4 * q + 3] = v.w;
            if constexpr (MINS) {
              const float4 uv = *(const float4*)(L.u + b * BM + mt * 32 + 8 * q + 4 * hf);
              ur[4 * q] = uv.x; ur[4 * q + 1] = uv.y; ur[4 * q + 2] = uv.z; ur[4 * q + 3] = uv.w;
            }
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc[mt][r] = fmaf(sr[r] * dsc[b], (float)dv[r], acc[mt][r]);
            if constexpr (MINS) acc[mt][r] = fmaf(ur[r], -dmn[b], acc[mt][r]);
            if constexpr (MODE == GEMM_MOE_GATEUP) acc2[mt][r] = fmaf(sr[r] * dsc2[b], (float)dv2[r], acc2[mt][r]);
          }
        }
      }
    }
  }
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
          if (a.accumulate == 1) {
            v += *cp;
          } else if (a.accumulate == 2) {
            const float g = *cp;
            v *= g / (1.0f + expf(-g));
          }
          *cp = v;
        }
      } else if constexpr (MODE == GEMM_MOE_DOWN) {
        if (row_ok && col_ok) {
          const int slot = m0 + i;
          a.C[(size_t)slot * a.ldc + n_loc] = a.rowscale[slot] * acc[mt][r];
        }
      } else {
        // h = up * silu(gate) (zero/kernels/gemm.cl:464-471), then quantized per 32 columns: the wave's 32 columns
        // (lanes of one half) are one 32-block of the h row, as moe_quant (zero/kernels/moe.cl:251-282)
        const float g = acc[mt][r];
        const float h = acc2[mt][r] * (g / (1.0f + expf(-g)));
        float amax = fabsf(h);
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        const int q = (int)__builtin_rintf(h * inv);
        if (row_ok && col_ok) {
          const int slot = m0 + i;
          a.hq[(size_t)slot * a.expert_rows + n_loc] = (int8_t)q;
          if (lc == 0) a.hsc[(size_t)(n_loc / 32) * a.slots + slot] = amax / 127.0f;
        }
      }
    }
  }
}

template <int TYPE, int MT, int MODE, bool DUMP>
static hipError_t go(const GemmArgs& a, hipStream_t s) {
  const int n_rows = MODE == GEMM_DENSE ? a.w.rows : a.expert_rows;
  const unsigned gx = (unsigned)((n_rows + 127) / 128);
  const unsigned gy = MODE == GEMM_DENSE ? (unsigned)((a.M + 32 * MT - 1) / (32 * MT)) : (unsigned)a.max_tiles;
  gemm_kernel<TYPE, MT, MODE, DUMP><<<dim3(gx, gy), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t dispatch(int mode, const GemmArgs& a, hipStream_t s) {
  if (a.dbg_isum) return go<TYPE, 1, GEMM_DENSE, true>(a, s);
  switch (mode) {
    case GEMM_DENSE: return a.M <= 32 ? go<TYPE, 1, GEMM_DENSE, false>(a, s) : go<TYPE, 2, GEMM_DENSE, false>(a, s);
    case GEMM_MOE_GATEUP: return go<TYPE, 1, GEMM_MOE_GATEUP, false>(a, s);
    case GEMM_MOE_DOWN: return go<TYPE, 1, GEMM_MOE_DOWN, false>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm(int type, int mode, const GemmArgs& a, hipStream_t s) {
  switch (type) {
    case T_Q8_0: return dispatch<T_Q8_0>(mode, a, s);
    case T_Q4_K: return dispatch<T_Q4_K>(mode, a, s);
    case T_IQ4_XS: return dispatch<T_IQ4_XS>(mode, a, s);
    case T_IQ3_S: return dispatch<T_IQ3_S>(mode, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm
