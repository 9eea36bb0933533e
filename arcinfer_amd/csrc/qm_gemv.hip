// Decode GEMV on the prepared planes: C[t][n] (+)= sum_k W[n][k] * a_t[k] for T <= 8 tokens per weight read.
//
// Mapping: a wave is split into 64/LPR lane groups; each group owns R consecutive rows and walks the row's 32-blocks
// with its LPR lanes (lane j: blocks j, j + LPR, ...). Per block a lane loads the token activations once (32 int8 +
// the f32 scale per token) and, per row, the block's payload (one 16-byte load for the 4-bit types) and header,
// decodes 32 int8 weights in registers (IQ4_XS: byte permutes over the 16-value codebook; IQ3_S: grid and sign
// masks from LDS), takes 8 v_dot4_i32_i8 per token and scales the int32 block sum in f32 -- per block exactly
// the reference's expression `sa * d * (float)(sc0 * lo + sc1 * hi)` (zero/kernels/decode.cl:695-706, 1107-1115),
// with the min term for Q4_K. A cross-lane butterfly then sums the group's partial results.
#include "qm_launch.h"

namespace qm {

template <int TYPE> struct LdsFor { struct type { int unused; }; };
template <> struct LdsFor<T_IQ3_S> { using type = Iq3Lds; };

// Decodes 32-block b of row n: w[k] = elements 4k..4k+3 (int8x4), integer scale sc (and min mn), float d (dmin).
template <int TYPE>
__device__ __forceinline__ void decode_block32(const WView& w, const typename LdsFor<TYPE>::type* lds, int n, int b,
                                               const KvTab& kv, uint32_t wd[8], int& sc, int& mn, float& d,
                                               float& dmin) {
  using Tr = Traits<TYPE>;
  const int nb = w.K / 32, nsb = w.K / 256, ib = b & 7;
  const uint8_t* qp = w.qs + ((size_t)n * nb + b) * Tr::QB;
  const uint8_t* hp = w.hdr + ((size_t)n * nsb + (b >> 3)) * Tr::HB;
  mn = 0;
  dmin = 0.0f;
  if constexpr (TYPE == T_Q8_0) {
    const uint4 q0 = *(const uint4*)qp, q1 = *(const uint4*)(qp + 16);
    wd[0] = q0.x; wd[1] = q0.y; wd[2] = q0.z; wd[3] = q0.w;
    wd[4] = q1.x; wd[5] = q1.y; wd[6] = q1.z; wd[7] = q1.w;
    d = h2f(((const uint16_t*)hp)[ib]);
    sc = 1;
  } else if constexpr (TYPE == T_Q4_K) {
    const uint4 q = *(const uint4*)qp;
    const uint4 h = *(const uint4*)hp;
    const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wd[k] = qq[k] & 0x0F0F0F0Fu;
      wd[4 + k] = (qq[k] >> 4) & 0x0F0F0F0Fu;
    }
    d = h2f(h.x);
    dmin = h2f(h.x >> 16);
    q4k_scale_min(h.y, h.z, h.w, ib, sc, mn);
  } else if constexpr (TYPE == T_IQ4_XS) {
    const uint4 q = *(const uint4*)qp;
    const uint2 h = *(const uint2*)hp;
    const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wd[k] = kv_lookup4(kv, qq[k]);
      wd[4 + k] = kv_lookup4(kv, qq[k] >> 4);
    }
    d = h2f(h.x);
    sc = iq4xs_scale(h.x, h.y, ib);
  } else {  // IQ3_S
    const uint32_t* qw = (const uint32_t*)qp;
    const uint32_t q0 = qw[0], q1 = qw[1], sg = qw[2];
    const uint4 h = *(const uint4*)hp;
    const uint32_t qh = ((ib < 4 ? h.x : h.y) >> (8 * (ib & 3))) & 0xFFu;
    iq3s_pair<0>(lds, q0, q1, qh, sg, wd[0], wd[1]);
    iq3s_pair<1>(lds, q0, q1, qh, sg, wd[2], wd[3]);
    iq3s_pair<2>(lds, q0, q1, qh, sg, wd[4], wd[5]);
    iq3s_pair<3>(lds, q0, q1, qh, sg, wd[6], wd[7]);
    sc = 1 + 2 * (int)((h.z >> (4 * ib)) & 0xFu);
    d = h2f(h.w);
  }
}

template <int TYPE, int LPR, int R, int TB, bool DUMP>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  __shared__ typename LdsFor<TYPE>::type lds;
  if constexpr (TYPE == T_IQ3_S) {
    iq3_lds_fill(&lds);
    __syncthreads();
  }
  constexpr int G = 64 / LPR;
  const int K = a.w.K, nb = K / 32, rows = a.w.rows;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane / LPR, gl = lane % LPR;
  const int row0 = ((blockIdx.x * 4 + wave) * G + grp) * R;
  const int T = a.T;
  const KvTab kv = kv_tab();

  float acc[R][TB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[r][t] = 0.0f;

  for (int b = gl; b < nb; b += LPR) {
    uint32_t av[TB][8];
    float sa[TB];
    int bs[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      if (t < T) {
        const uint4* ap = (const uint4*)(a.aq + (size_t)t * K + 32 * b);
        const uint4 x0 = ap[0], x1 = ap[1];
        av[t][0] = x0.x; av[t][1] = x0.y; av[t][2] = x0.z; av[t][3] = x0.w;
        av[t][4] = x1.x; av[t][5] = x1.y; av[t][6] = x1.z; av[t][7] = x1.w;
        sa[t] = DUMP ? 0.0f : a.asc[(size_t)b * a.M_stride + t];
        if constexpr (Traits<TYPE>::MINS)
          bs[t] = (int)a.absum[(size_t)(2 * b) * a.M_stride + t] + (int)a.absum[(size_t)(2 * b + 1) * a.M_stride + t];
        else
          bs[t] = 0;
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) av[t][k] = 0u;
        sa[t] = 0.0f;
        bs[t] = 0;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = min(row0 + r, rows - 1);
      uint32_t wd[8];
      int sc, mn;
      float d, dmin;
      decode_block32<TYPE>(a.w, &lds, n, b, kv, wd, sc, mn, d, dmin);
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        int isum = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) isum = dot4(av[t][k], wd[k], isum);
        const int iv = sc * isum;
        if constexpr (DUMP) {
          if (t < T && row0 + r < rows) {
            const size_t o = ((size_t)t * rows + (row0 + r)) * nb + b;
            a.dbg_isum[o] = iv;
            if constexpr (Traits<TYPE>::MINS) a.dbg_msum[o] = mn * bs[t];
          }
        } else if constexpr (Traits<TYPE>::MINS) {
          acc[r][t] += sa[t] * (d * (float)iv - dmin * (float)(mn * bs[t]));
        } else {
          acc[r][t] += sa[t] * d * (float)iv;
        }
      }
    }
  }
  if constexpr (!DUMP) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        const float v = wave_sum_width(acc[r][t], LPR);
        const int n = row0 + r;
        if (gl == 0 && n < rows && t < T) {
          float* cp = a.C + (size_t)t * a.ldc + a.c_off + n;
          *cp = a.accumulate ? *cp + v : v;
        }
      }
  }
}

template <int TYPE, int LPR, int R, int TB, bool DUMP>
static hipError_t go(const GemvArgs& a, hipStream_t s) {
  constexpr int rows_per_wg = 4 * (64 / LPR) * R;
  const dim3 grid((unsigned)((a.w.rows + rows_per_wg - 1) / rows_per_wg)), block(256);
  gemv_kernel<TYPE, LPR, R, TB, DUMP><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t dispatch(const GemvArgs& a, hipStream_t s) {
  const int nb = a.w.K / 32;
  if (a.dbg_isum) {
    switch (a.T <= 1 ? 1 : a.T <= 2 ? 2 : a.T <= 4 ? 4 : 8) {
      case 1: return go<TYPE, 8, 1, 1, true>(a, s);
      case 2: return go<TYPE, 8, 1, 2, true>(a, s);
      case 4: return go<TYPE, 8, 1, 4, true>(a, s);
      default: return go<TYPE, 8, 1, 8, true>(a, s);
    }
  }
  const bool l32 = nb % 32 == 0;
  if (a.T <= 1) {
    // short rows (many rows): 2 rows per lane group; long rows (few rows, K >= 8192): 1, for more waves in flight
    if (l32) return a.w.K >= 8192 ? go<TYPE, 32, 1, 1, false>(a, s) : go<TYPE, 32, 2, 1, false>(a, s);
    return go<TYPE, 8, 2, 1, false>(a, s);
  }
  if (a.T <= 2) return l32 ? go<TYPE, 32, 1, 2, false>(a, s) : go<TYPE, 8, 1, 2, false>(a, s);
  if (a.T <= 4) return l32 ? go<TYPE, 32, 1, 4, false>(a, s) : go<TYPE, 8, 1, 4, false>(a, s);
  return l32 ? go<TYPE, 32, 1, 8, false>(a, s) : go<TYPE, 8, 1, 8, false>(a, s);
}

hipError_t launch_gemv(int type, const GemvArgs& a, hipStream_t s) {
  switch (type) {
    case T_Q8_0: return dispatch<T_Q8_0>(a, s);
    case T_Q4_K: return dispatch<T_Q4_K>(a, s);
    case T_IQ4_XS: return dispatch<T_IQ4_XS>(a, s);
    case T_IQ3_S: return dispatch<T_IQ3_S>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm
