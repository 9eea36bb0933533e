// MoE FFN at decode sizes (a few tokens): GEMV-shaped kernels instead of expert-grouped GEMM tiles, the role of the
// reference's per-tile moe_gateup_q / moe_down_q (zero/kernels/decode.cl:1500-1847). Same arithmetic as the tile
// path: h = up * silu(gate) per expert row, h quantized per 32 (moe.cl:251-282), down times the routing weight, and
// the token's NU expert outputs summed in selection order (moe.cl:332-340).
#include "qm_decode.h"
#include "qm_route.h"

namespace qm {

namespace {

template <int TYPE>
__device__ __forceinline__ int block_isum(const RawBlk& r, const typename LdsFor<TYPE>::type* lds, int b,
                                          const KvTab& kv, const uint8_t* sq, int nb, float& d) {
  const uint4 x0 = *(const uint4*)(sq + b * 16), x1 = *(const uint4*)(sq + (size_t)nb * 16 + b * 16);
  const BlockInts bi = block_product<TYPE>(r, lds, b & 7, kv, x0, x1, 0, 0);  // (types without per-16 sums)
  d = bi.d;
  return bi.iv;
}

}  // namespace

// Gate/up: grid (slots, F / (256 / LPR)), routing included (logits non-null; else ids holds the routing). Wave 0
// of every work-group routes the slot's token (route_token:
// the route kernel's arithmetic, so every work-group of a token selects the same experts) while the work-group stages
// the token's int8 row in LDS (two 16-byte planes per 32-block, as the decode GEMV); the work-groups with
// blockIdx.y == 0 of the token's first slot publish ids / wts for the down kernel. Then its lane groups of LPR take
// one expert row j each: g = gate_e[j] . a_t, u = up_e[j] . a_t, h[slot][j] = u * silu(g). CH >= E / (32 LPR) blocks
// per lane.
template <int TYPE, int CH, int PER_LANE, int LPR = 32>
__global__ __launch_bounds__(256) void moe_gateup_dec_kernel(WView gate, WView up, const float* __restrict__ logits,
                                                             int ldl, int NE, int* __restrict__ ids,
                                                             float* __restrict__ wts, int NU, int F,
                                                             const int8_t* __restrict__ aq,
                                                             const float* __restrict__ asc, int M_stride,
                                                             float* __restrict__ h) {
  extern __shared__ uint4 smem[];
  __shared__ typename LdsFor<TYPE>::type lds;
  __shared__ int sel[64];
  using Tr = Traits<TYPE>;
  const int E = gate.K, nb = E / 32;
  uint8_t* sq = (uint8_t*)smem;
  float* ssc = (float*)(sq + (size_t)E);
  const int slot = blockIdx.x, t = slot / NU, k = slot % NU;
  if (threadIdx.x < 64 && !logits) {
    if (threadIdx.x < NU) sel[threadIdx.x] = ids[(size_t)t * NU + threadIdx.x];  // (routed by a separate launch)
  } else if (threadIdx.x < 64) {
    int my_e;
    float my_w;
    route_token<PER_LANE>(logits + (size_t)t * ldl, NE, NU, threadIdx.x, my_e, my_w);
    if (threadIdx.x < NU) {
      sel[threadIdx.x] = my_e;
      if (blockIdx.y == 0 && k == 0) {
        ids[(size_t)t * NU + threadIdx.x] = my_e;
        wts[(size_t)t * NU + threadIdx.x] = my_w;
      }
    }
  }
  lds_fill<TYPE>(&lds);
  for (int i = threadIdx.x; i < 2 * nb; i += 256) {
    const int b = i >> 1, hh = i & 1;
    *(uint4*)(sq + (size_t)hh * nb * 16 + b * 16) = *(const uint4*)(aq + (size_t)t * E + 32 * b + 16 * hh);
  }
  for (int b = threadIdx.x; b < nb; b += 256) ssc[b] = asc[(size_t)b * M_stride + t];
  __syncthreads();
  const int e = sel[k];
  constexpr int RPW = 256 / LPR;  // expert rows per work-group
  const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
  const int j = min((int)blockIdx.y * RPW + grp, F - 1);
  const size_t row = (size_t)e * F + j;
  RawBlk rg[CH], ru[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int b = min(gl + LPR * u, nb - 1);
    rg[u] = load_block_at<TYPE>(gate.qs + row * nb * Tr::QB, gate.hdr + row * (nb / 8) * Tr::HB, b);
    ru[u] = load_block_at<TYPE>(up.qs + row * nb * Tr::QB, up.hdr + row * (nb / 8) * Tr::HB, b);
  }
  const KvTab kv = kv_tab();
  float g = 0.0f, uu = 0.0f;
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int b = gl + LPR * u;
    if (b < nb) {
      float d;
      const int ig = block_isum<TYPE>(rg[u], &lds, b, kv, sq, nb, d);
      g += ssc[b] * d * (float)ig;
      const int iu = block_isum<TYPE>(ru[u], &lds, b, kv, sq, nb, d);
      uu += ssc[b] * d * (float)iu;
    }
  }
  g = wave_sum_width(g, LPR);
  uu = wave_sum_width(uu, LPR);
  if (gl == 0 && (int)blockIdx.y * RPW + grp < F) h[(size_t)slot * F + j] = uu * (g / (1.0f + expf(-g)));
}

// Down + combine: grid (T, ceil(E / GPW)). The work-group quantizes its token's NU rows of h per 32 into LDS (two
// planes per row, as the activations of the decode GEMV), then each lane group of LPR lanes takes one output column c:
// for k = 0..NU-1, y_k = w_k * (down_{e_k}[c] . q(h_k)), summed in k order; x[t][c] (+)= the sum. The NU expert rows
// of a column are loaded before any is decoded. F / 32 <= LPR * CH, NU <= 8.
template <int TYPE, int LPR, int CH>
__global__ __launch_bounds__(256) void moe_down_dec_kernel(WView down, int E, const int* __restrict__ ids,
                                                           const float* __restrict__ wts, int NU,
                                                           const float* __restrict__ h, float* __restrict__ x,
                                                           int accumulate) {
  extern __shared__ uint4 smem[];
  __shared__ typename LdsFor<TYPE>::type lds;
  using Tr = Traits<TYPE>;
  constexpr int GPW = 256 / LPR, NUMAX = 8;
  const int F = down.K, nb = F / 32;
  uint8_t* sq = (uint8_t*)smem;               // [NU][2][nb][16]
  float* ssc = (float*)(sq + (size_t)NU * F);  // [NU][nb]
  const int t = blockIdx.x, grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
  const int c_raw = blockIdx.y * GPW + grp, c = min(c_raw, E - 1);
  RawBlk r[NUMAX][CH];
#pragma unroll
  for (int k = 0; k < NUMAX; ++k)
    if (k < NU) {
      const size_t row = (size_t)ids[(size_t)t * NU + k] * E + c;
#pragma unroll
      for (int u = 0; u < CH; ++u)
        r[k][u] = load_block_at<TYPE>(down.qs + row * nb * Tr::QB, down.hdr + row * (nb / 8) * Tr::HB,
                                      min(gl + LPR * u, nb - 1));
    }
  lds_fill<TYPE>(&lds);
  // h rows of the token's NU slots, quantized per 32 (8 lanes per block: the quantizer's arithmetic); the loads of
  // four passes are issued before any is quantized (each is an L2 round trip)
  constexpr int QB = 4;
  for (int b00 = 0; b00 < NU * nb; b00 += 32 * QB) {
    float4 hv[QB];
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int bi = b00 + 32 * q + (threadIdx.x >> 3), sub = threadIdx.x & 7;
      hv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (bi < NU * nb) hv[q] = *(const float4*)(h + ((size_t)t * NU + bi / nb) * F + 32 * (bi % nb) + 4 * sub);
    }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int bi = b00 + 32 * q + (threadIdx.x >> 3), sub = threadIdx.x & 7;
      const bool live = bi < NU * nb;
      const int k = live ? bi / nb : 0, b = live ? bi % nb : 0;
      const float v[4] = {hv[q].x, hv[q].y, hv[q].z, hv[q].w};
      float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
      amax = max8(amax);
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      uint32_t pk = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) pk |= (uint32_t)((int)__builtin_rintf(v[i] * inv) & 0xFF) << (8 * i);
      if (live) {
        *(uint32_t*)(sq + (size_t)k * F + (size_t)(sub >> 2) * nb * 16 + b * 16 + 4 * (sub & 3)) = pk;
        if (sub == 0) ssc[k * nb + b] = amax / 127.0f;
      }
    }
  }
  __syncthreads();
  const KvTab kv = kv_tab();
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < NUMAX; ++k)
    if (k < NU) {
      float acc = 0.0f;
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int b = gl + LPR * u;
        if (b < nb) {
          float d;
          const int iv = block_isum<TYPE>(r[k][u], &lds, b, kv, sq + (size_t)k * F, nb, d);
          acc += ssc[k * nb + b] * d * (float)iv;
        }
      }
      acc = wave_sum_width(acc, LPR);
      const float y = wts[(size_t)t * NU + k] * acc;
      v += y;
    }
  if (gl == 0 && c_raw < E) {
    float* xp = x + (size_t)t * E + c;
    *xp = accumulate ? *xp + v : v;
  }
}

template <int TYPE, int PL>
static void gateup_dec(int slots, size_t shg, int nbE, const WView& gate, const WView& up, const float* logits,
                       int ldl, int NE, int* ids, float* wts, int NU, int F, const int8_t* aq, const float* asc,
                       int M_stride, float* h, hipStream_t s) {
  // 16 lanes per expert row up to 64 blocks per row (16 rows per work-group: half the work-groups, each routing and
  // staging the token once; measured faster at 4 and 8 tokens, equal at 1), 32 lanes beyond
#define QM_GUD(CH, LPR)                                                                                       \
  moe_gateup_dec_kernel<TYPE, CH, PL, LPR><<<dim3((unsigned)slots, (unsigned)((F + 256 / LPR - 1) / (256 / LPR))), \
                                              256, shg, s>>>(gate, up, logits, ldl, NE, ids, wts, NU, F, aq, asc,   \
                                                             M_stride, h)
  if (nbE <= 16) QM_GUD(1, 16);
  else if (nbE <= 32) QM_GUD(2, 16);
  else if (nbE <= 64) QM_GUD(4, 16);
  else if (nbE <= 128) QM_GUD(4, 32);
  else QM_GUD(8, 32);
#undef QM_GUD
}

template <int TYPE>
static hipError_t moe_dec_typed(const WView& gate, const WView& up, const WView& down, int T, int NU, int E, int F,
                                const float* logits, int ldl, int NE, int* ids, float* wts, const int8_t* aq,
                                const float* asc, int M_stride, float* h, float* x, int accumulate, hipStream_t s) {
  const int slots = T * NU, nbE = E / 32, nbF = F / 32;
  const size_t shg = (size_t)E + sizeof(float) * nbE;
  if (T > 4) {
    // (more tokens: every gate/up work-group routing its token in front of its weight loads costs more than a
    //  separate route launch; measured at T = 8)
    const hipError_t e = launch_moe_route(logits, ldl, T, NE, NU, ids, wts, nullptr, s);
    if (e != hipSuccess) return e;
    logits = nullptr;
  }
  if (NE <= 256) gateup_dec<TYPE, 4>(slots, shg, nbE, gate, up, logits, ldl, NE, ids, wts, NU, F, aq, asc, M_stride, h, s);
  else gateup_dec<TYPE, 16>(slots, shg, nbE, gate, up, logits, ldl, NE, ids, wts, NU, F, aq, asc, M_stride, h, s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t shd = (size_t)NU * F + sizeof(float) * NU * nbF;
  if (nbF <= 16) {
    const dim3 gd((unsigned)T, (unsigned)((E + 15) / 16));
    moe_down_dec_kernel<TYPE, 16, 1><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate);
  } else {
    const dim3 gd((unsigned)T, (unsigned)((E + 7) / 8));
    if (nbF <= 32) moe_down_dec_kernel<TYPE, 32, 1><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate);
    else if (nbF <= 64) moe_down_dec_kernel<TYPE, 32, 2><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate);
    else moe_down_dec_kernel<TYPE, 32, 4><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate);
  }
  return hipGetLastError();
}

hipError_t launch_moe_decode(int type, const WView& gate, const WView& up, const WView& down, int T, int NU, int E,
                             int F, const float* logits, int ldl, int NE, int* ids, float* wts, const int8_t* aq,
                             const float* asc, int M_stride, float* h, float* x, int accumulate, hipStream_t s) {
  switch (type) {
    case T_Q8_0: return moe_dec_typed<T_Q8_0>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    case T_IQ4_XS: return moe_dec_typed<T_IQ4_XS>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    case T_IQ3_S: return moe_dec_typed<T_IQ3_S>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    case T_Q4_0: return moe_dec_typed<T_Q4_0>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    case T_IQ4_NL: return moe_dec_typed<T_IQ4_NL>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    case T_IQ2_XXS: return moe_dec_typed<T_IQ2_XXS>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    case T_IQ3_XXS: return moe_dec_typed<T_IQ3_XXS>(gate, up, down, T, NU, E, F, logits, ldl, NE, ids, wts, aq, asc, M_stride, h, x, accumulate, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm
