// MoE FFN at decode sizes (a few tokens): GEMV-shaped kernels instead of expert-grouped GEMM tiles, the role of the
// reference's per-tile moe_gateup_q / moe_down_q (zero/kernels/decode.cl:1500-1847). Same arithmetic as the tile
// path: h = up * silu(gate) per expert row, h quantized per 32 (moe.cl:251-282), down times the routing weight, and
// the token's NU expert outputs summed in selection order, plus the shared expert's gated output (moe.cl:332-340).
// Gate, up and down may each have their own type (zero/engine_moe.h:297-306): with gate and up of one type one
// launch computes both; otherwise a gate launch stores g and an up launch forms h from it.
#include "qm_decode.h"
#include "qm_launch.h"
#include "qm_route.h"

namespace qm {

// gate/up launch roles
enum : int { GU_BOTH = 0, GU_GATE = 1, GU_UP = 2 };

namespace {

// One 32-block's contribution sa * (weights . activations) from the staged planes (sq: [2][nb][16] int8 planes,
// bs: the block's two per-16 activation sums, needed by Q6_K's offset-32 values).
template <int TYPE>
__device__ __forceinline__ float block_term(const RawBlk& r, const typename LdsFor<TYPE>::type* lds, int b,
                                            const KvTab& kv, const uint8_t* sq, int nb, float sa, int bs) {
  const uint4 x0 = *(const uint4*)(sq + b * 16), x1 = *(const uint4*)(sq + (size_t)nb * 16 + b * 16);
  const BlockInts bi = block_product<TYPE>(r, lds, b & 7, kv, x0, x1, (int)(int16_t)(bs & 0xFFFF), bs >> 16);
  return block_value<TYPE>(sa, bi);
}

// the sum of 16 int8 values held in a 16-byte word (v_dot4 against ones)
__device__ __forceinline__ int sum16(uint4 v) {
  int s = dot4(v.x, 0x01010101u, 0);
  s = dot4(v.y, 0x01010101u, s);
  s = dot4(v.z, 0x01010101u, s);
  return dot4(v.w, 0x01010101u, s);
}

}  // namespace

// Gate/up: grid (T * NU slots, ceil(F / rows per work-group)); h rows of F values, of which the first Fv are the
// experts' rows (Fv < F: the down projection's rows were padded with zero blocks to F = Fv rounded up to 256, and
// h[Fv..F) is written as 0). The work-group stages its token's int8 row in LDS as two
// 16-byte planes, with the per-32 scales and per-16 sums; with routing inside (logits non-null, T <= 4) wave 0 routes
// the token while the others stage. Each LPR-lane group computes one expert row j: GU_BOTH h = u * silu(g) from gate
// and up, GU_GATE stores g into h, GU_UP reads g from h and stores u * silu(g).
template <int TYPE, int MODE, int CH, int PER_LANE, int LPR = 32>
__global__ __launch_bounds__(256) void moe_gateup_dec_kernel(WView gate, WView up, const float* __restrict__ logits,
                                                             int ldl, int NE, int* __restrict__ ids,
                                                             float* __restrict__ wts, const float* __restrict__ escale,
                                                             int NU, int F, int Fv, const int8_t* __restrict__ aq,
                                                             const float* __restrict__ asc, int M_stride,
                                                             float* __restrict__ h) {
  extern __shared__ uint4 smem[];
  __shared__ typename LdsFor<TYPE>::type lds;
  __shared__ int sel[64];
  using Tr = Traits<TYPE>;
  const WView& W0 = MODE == GU_UP ? up : gate;
  const int E = W0.K, nb = E / 32;
  uint8_t* sq = (uint8_t*)smem;
  float* ssc = (float*)(sq + (size_t)E);
  int* sbs = (int*)(ssc + nb);  // per block: the two per-16 sums, packed int16 pairs
  const int slot = blockIdx.x, t = slot / NU, k = slot % NU;
  if (threadIdx.x < 64 && !logits) {
    if (threadIdx.x < NU) sel[threadIdx.x] = ids[(size_t)t * NU + threadIdx.x];  // (routed by a separate launch)
  } else if (threadIdx.x < 64) {
    int my_e;
    float my_w;
    route_token<PER_LANE>(logits + (size_t)t * ldl, NE, NU, threadIdx.x, my_e, my_w, escale);
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
    const uint4 v = *(const uint4*)(aq + (size_t)t * E + 32 * b + 16 * hh);
    *(uint4*)(sq + (size_t)hh * nb * 16 + b * 16) = v;
    if constexpr (kNeedsBsum<TYPE>) ((int16_t*)sbs)[i] = (int16_t)sum16(v);
  }
  for (int b = threadIdx.x; b < nb; b += 256) ssc[b] = asc[(size_t)b * M_stride + t];
  __syncthreads();
  const int e = sel[k];
  constexpr int RPW = 256 / LPR;  // expert rows per work-group
  const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
  const int jj = (int)blockIdx.y * RPW + grp, j = min(jj, Fv - 1);
  const size_t row = (size_t)e * Fv + j;
  RawBlk r0[CH], r1[MODE == GU_BOTH ? CH : 1];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int b = min(gl + LPR * u, nb - 1);
    r0[u] = load_block_at<TYPE>(W0.qs + row * nb * Tr::QB, W0.hdr + row * (nb / 8) * Tr::HB, b);
    if constexpr (MODE == GU_BOTH)
      r1[u] = load_block_at<TYPE>(up.qs + row * nb * Tr::QB, up.hdr + row * (nb / 8) * Tr::HB, b);
  }
  const KvTab kv = kv_tab();
  float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int b = gl + LPR * u;
    if (b < nb) {
      const int bs = kNeedsBsum<TYPE> ? sbs[b] : 0;
      v0 += block_term<TYPE>(r0[u], &lds, b, kv, sq, nb, ssc[b], bs);
      if constexpr (MODE == GU_BOTH) v1 += block_term<TYPE>(r1[u], &lds, b, kv, sq, nb, ssc[b], bs);
    }
  }
  v0 = wave_sum_width(v0, LPR);
  if constexpr (MODE == GU_BOTH) v1 = wave_sum_width(v1, LPR);
  if (gl == 0 && jj < F) {
    float* hp = h + (size_t)slot * F + jj;
    if (jj >= Fv) {
      *hp = 0.0f;
    } else if constexpr (MODE == GU_BOTH) {
      *hp = v1 * (v0 / (1.0f + expf(-v0)));
    } else if constexpr (MODE == GU_GATE) {
      *hp = v0;
    } else {
      const float g = *hp;
      *hp = v0 * (g / (1.0f + expf(-g)));
    }
  }
}

// Down + combine: grid (T, ceil(E / GPW)). The work-group quantizes its token's NU rows of h per 32 into LDS (two
// planes per row, as the activations of the decode GEMV; with their per-16 sums), then each lane group of LPR lanes
// takes one output column c: for k = 0..NU-1, y_k = w_k * (down_{e_k}[c] . q(h_k)), summed in k order, plus the shared
// expert's g_t * sh[t][c]; x[t][c] (+)= the sum. The NU expert rows of a column are loaded before any is decoded.
// F / 32 <= LPR * CH, NU <= 8.
template <int TYPE, int LPR, int CH>
__global__ __launch_bounds__(256) void moe_down_dec_kernel(WView down, int E, const int* __restrict__ ids,
                                                           const float* __restrict__ wts, int NU,
                                                           const float* __restrict__ h, float* __restrict__ x,
                                                           int accumulate, MoeShared sh) {
  extern __shared__ uint4 smem[];
  __shared__ typename LdsFor<TYPE>::type lds;
  using Tr = Traits<TYPE>;
  constexpr int GPW = 256 / LPR, NUMAX = 8;
  const int F = down.K, nb = F / 32;
  uint8_t* sq = (uint8_t*)smem;                  // [NU][2][nb][16]
  float* ssc = (float*)(sq + (size_t)NU * F);     // [NU][nb]
  int16_t* sbs = (int16_t*)(ssc + (size_t)NU * nb);  // [NU][nb][2] per-16 sums
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
      int qs = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qv = (int)__builtin_rintf(v[i] * inv);
        pk |= (uint32_t)(qv & 0xFF) << (8 * i);
        qs += qv;
      }
      if constexpr (kNeedsBsum<TYPE>) qs = sum4_i(qs);  // (lanes sub 0-3: elements 0-15, 4-7: 16-31)
      if (live) {
        *(uint32_t*)(sq + (size_t)k * F + (size_t)(sub >> 2) * nb * 16 + b * 16 + 4 * (sub & 3)) = pk;
        if (sub == 0) ssc[k * nb + b] = amax / 127.0f;
        if (kNeedsBsum<TYPE> && (sub & 3) == 0) sbs[(k * nb + b) * 2 + (sub >> 2)] = (int16_t)qs;
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
          const int bs = kNeedsBsum<TYPE> ? (int)(uint16_t)sbs[(k * nb + b) * 2] | ((int)sbs[(k * nb + b) * 2 + 1] << 16)
                                          : 0;
          acc += block_term<TYPE>(r[k][u], &lds, b, kv, sq + (size_t)k * F, nb, ssc[k * nb + b], bs);
        }
      }
      acc = wave_sum_width(acc, LPR);
      const float y = wts[(size_t)t * NU + k] * acc;
      v += y;
    }
  if (sh.sh) {
    const float g = sh.gl ? 1.0f / (1.0f + expf(-sh.gl[(size_t)t * sh.ldl])) : 1.0f;
    v = v + g * sh.sh[(size_t)t * sh.ldsh + c];
  }
  if (gl == 0 && c_raw < E) {
    float* xp = x + (size_t)t * E + c;
    *xp = accumulate ? *xp + v : v;
  }
}

template <int TYPE, int MODE, int PL>
static void gateup_dec(int slots, size_t shg, int nbE, const WView& gate, const WView& up, const float* logits,
                       int ldl, int NE, int* ids, float* wts, const float* escale, int NU, int F, int Fv,
                       const int8_t* aq, const float* asc, int M_stride, float* h, hipStream_t s) {
  // 16 lanes per expert row up to 64 blocks per row (16 rows per work-group: half the work-groups, each routing and
  // staging the token once; measured faster at 4 and 8 tokens, equal at 1), 32 lanes beyond
#define QM_GUD(CH, LPR)                                                                                       \
  moe_gateup_dec_kernel<TYPE, MODE, CH, PL, LPR>                                                              \
      <<<dim3((unsigned)slots, (unsigned)((F + 256 / LPR - 1) / (256 / LPR))), 256, shg, s>>>(                \
          gate, up, logits, ldl, NE, ids, wts, escale, NU, F, Fv, aq, asc, M_stride, h)
  if (nbE <= 16) QM_GUD(1, 16);
  else if (nbE <= 32) QM_GUD(2, 16);
  else if (nbE <= 64) QM_GUD(4, 16);
  else if (nbE <= 128) QM_GUD(4, 32);
  else QM_GUD(8, 32);
#undef QM_GUD
}

template <int TYPE, int MODE>
static hipError_t gateup_typed(int T, int NU, int E, int F, int Fv, const WView& gate, const WView& up, const float* logits,
                               int ldl, int NE, int* ids, float* wts, const float* escale, const int8_t* aq,
                               const float* asc, int M_stride, float* h, hipStream_t s) {
  const int slots = T * NU, nbE = E / 32;
  const size_t shg = (size_t)E + sizeof(float) * nbE + sizeof(int) * nbE;
  if (NE <= 256) gateup_dec<TYPE, MODE, 4>(slots, shg, nbE, gate, up, logits, ldl, NE, ids, wts, escale, NU, F, Fv, aq, asc, M_stride, h, s);
  else gateup_dec<TYPE, MODE, 16>(slots, shg, nbE, gate, up, logits, ldl, NE, ids, wts, escale, NU, F, Fv, aq, asc, M_stride, h, s);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t down_typed(int T, int NU, int E, int F, const WView& down, const int* ids, const float* wts,
                             const float* h, float* x, int accumulate, const MoeShared& sh, hipStream_t s) {
  const int nbF = F / 32;
  const size_t shd = (size_t)NU * F + sizeof(float) * NU * nbF + sizeof(int) * NU * nbF;
  if (nbF <= 16) {
    const dim3 gd((unsigned)T, (unsigned)((E + 15) / 16));
    moe_down_dec_kernel<TYPE, 16, 1><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate, sh);
  } else {
    const dim3 gd((unsigned)T, (unsigned)((E + 7) / 8));
    if (nbF <= 32) moe_down_dec_kernel<TYPE, 32, 1><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate, sh);
    else if (nbF <= 64) moe_down_dec_kernel<TYPE, 32, 2><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate, sh);
    else moe_down_dec_kernel<TYPE, 32, 4><<<gd, 256, shd, s>>>(down, E, ids, wts, NU, h, x, accumulate, sh);
  }
  return hipGetLastError();
}

// the expert types of the MoE paths: one integer (or f16) scale per 16 or 32 and no per-block mins, as the
// reference's moe_rg (zero/engine_moe.h:297-301)
#define QM_MOE_TYPES(X) X(T_Q8_0) X(T_Q4_0) X(T_IQ4_NL) X(T_IQ4_XS) X(T_IQ3_S) X(T_IQ2_XXS) X(T_IQ2_XS) X(T_IQ2_S) \
  X(T_Q3_K) X(T_Q2_0) \
  X(T_IQ3_XXS) X(T_Q6_K)

template <int MODE>
static hipError_t gateup_any(int type, int T, int NU, int E, int F, int Fv, const WView& gate, const WView& up,
                             const float* logits, int ldl, int NE, int* ids, float* wts, const float* escale,
                             const int8_t* aq, const float* asc, int M_stride, float* h, hipStream_t s) {
  switch (type) {
#define QM_CASE(TY) \
  case TY: return gateup_typed<TY, MODE>(T, NU, E, F, Fv, gate, up, logits, ldl, NE, ids, wts, escale, aq, asc, M_stride, h, s);
    QM_MOE_TYPES(QM_CASE)
#undef QM_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_moe_decode(int tg, int tu, int td, const WView& gate, const WView& up, const WView& down, int T,
                             int NU, int E, int F, int Fv, const float* logits, int ldl, int NE, const float* escale, int* ids,
                             float* wts, const int8_t* aq, const float* asc, int M_stride, float* h, float* x,
                             int accumulate, const MoeShared& sh, hipStream_t s) {
  if (T > 4 || tg != tu) {
    // (more tokens: every gate/up work-group routing its token in front of its weight loads costs more than a
    //  separate route launch, measured at T = 8; two gate/up launches route once, here)
    const hipError_t e = launch_moe_route(logits, ldl, T, NE, NU, ids, wts, nullptr, escale, nullptr, s);
    if (e != hipSuccess) return e;
    logits = nullptr;
  }
  hipError_t e;
  if (tg == tu) {
    e = gateup_any<GU_BOTH>(tg, T, NU, E, F, Fv, gate, up, logits, ldl, NE, ids, wts, escale, aq, asc, M_stride, h, s);
  } else {
    e = gateup_any<GU_GATE>(tg, T, NU, E, F, Fv, gate, up, logits, ldl, NE, ids, wts, escale, aq, asc, M_stride, h, s);
    if (e == hipSuccess)
      e = gateup_any<GU_UP>(tu, T, NU, E, F, Fv, gate, up, logits, ldl, NE, ids, wts, escale, aq, asc, M_stride, h, s);
  }
  if (e != hipSuccess) return e;
  switch (td) {
#define QM_CASE(TY) case TY: return down_typed<TY>(T, NU, E, F, down, ids, wts, h, x, accumulate, sh, s);
    QM_MOE_TYPES(QM_CASE)
#undef QM_CASE
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm
