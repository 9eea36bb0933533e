// Decode GEMV on the prepared planes: C[t][n] (+)= sum_k W[n][k] * a_t[k] for T <= 8 tokens per weight read.
//
// Mapping: a wave is split into 64/LPR lane groups; each group owns R consecutive rows and walks the row's 32-blocks
// with its LPR lanes (lane j: blocks j, j + LPR, ...). Per block a lane loads the token activations once (32 int8 +
// the f32 scale per token) and, per row, the block's payload (one 16-byte load for the 4-bit types) and header,
// decodes 32 int8 weights in registers (IQ4_XS: byte permutes over the 16-value codebook; IQ3_S: grid and sign
// masks from LDS), takes 8 v_dot4_i32_i8 per token and scales the int32 block sum in f32 -- per block exactly
// the reference's expression `sa * d * (float)(sc0 * lo + sc1 * hi)` (zero/kernels/decode.cl:695-706, 1107-1115),
// with the min term for Q4_K. A cross-lane butterfly then sums the group's partial results.
#pragma once

#include "qm_decode.h"

namespace qm {

// U consecutive iterations of the block loop are loaded before any is decoded, so each lane keeps U*R weight loads
// in flight (the loop is bandwidth-bound: bytes in flight, not instructions, set its speed).
template <int TYPE, int LPR, int R, int TB, int U, bool DUMP>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  __shared__ typename LdsFor<TYPE>::type lds;
  if constexpr (TYPE == T_IQ3_S || kIq2<TYPE> || kIq1<TYPE>) {
    lds_fill<TYPE>(&lds);
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

  for (int b0 = gl; b0 < nb; b0 += LPR * U) {
    RawBlk raw[U][R];
    uint32_t av[U][TB][8];
    float sa[U][TB];
    int bs0[U][TB], bs1[U][TB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = min(b0 + LPR * u, nb - 1);  // (past the row's end: reload its last block, masked below)
#pragma unroll
      for (int r = 0; r < R; ++r) raw[u][r] = load_block<TYPE>(a.w, min(row0 + r, rows - 1), b);
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        const int tt = min(t, T - 1);
        const uint4* ap = (const uint4*)(a.aq + (size_t)tt * K + 32 * b);
        const uint4 x0 = ap[0], x1 = ap[1];
        av[u][t][0] = x0.x; av[u][t][1] = x0.y; av[u][t][2] = x0.z; av[u][t][3] = x0.w;
        av[u][t][4] = x1.x; av[u][t][5] = x1.y; av[u][t][6] = x1.z; av[u][t][7] = x1.w;
        sa[u][t] = DUMP ? 0.0f : a.asc[(size_t)b * a.M_stride + tt];
        if constexpr (kNeedsBsum<TYPE>) {
          bs0[u][t] = a.absum[(size_t)(2 * b) * a.M_stride + tt];
          bs1[u][t] = a.absum[(size_t)(2 * b + 1) * a.M_stride + tt];
        } else {
          bs0[u][t] = bs1[u][t] = 0;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + LPR * u;
      const bool live = b < nb;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint32_t wd[8];
        int sc, sc1, mn;
        BlockInts bi;
        decode_block32<TYPE>(raw[u][r], &lds, b & 7, kv, wd, sc, sc1, mn, bi.d, bi.dmin);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
          const uint4 x0 = make_uint4(av[u][t][0], av[u][t][1], av[u][t][2], av[u][t][3]);
          const uint4 x1 = make_uint4(av[u][t][4], av[u][t][5], av[u][t][6], av[u][t][7]);
          block_dot<TYPE>(wd, sc, sc1, mn, x0, x1, bs0[u][t], bs1[u][t], bi.iv, bi.mv);
          if constexpr (DUMP) {
            if (live && t < T && row0 + r < rows) {
              const size_t o = ((size_t)t * rows + (row0 + r)) * nb + b;
              a.dbg_isum[o] = bi.iv;
              if constexpr (Traits<TYPE>::MINS) a.dbg_msum[o] = bi.mv;
            }
          } else if (live) {
            acc[r][t] += block_value<TYPE>(sa[u][t], bi);
          }
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

// ---------------------------------------------------------------------------------------------------------------
// Batch-1 decode GEMV, persistent sweep. LPR lanes share a row (32, or 128 = two waves with an LDS combine); lane j
// takes blocks j, j + LPR, ... (CH of them). The grid is a few work-groups per CU and lane group g walks rows
// g, g + G, g + 2G, ... (G = lane groups in the grid), so the whole grid moves through the weight matrix together
// and every group has at most two rows in flight (one or two tokens; one row with more): row i + 1's loads are
// issued before row i is decoded. Measured on MI355X this beats issuing every row's loads up front (the decode then
// piles up behind the stream) and a third row in flight. The token's int8 row, its per-32 scales (and Q4_K / Q5_K /
// Q6_K per-16 sums) are staged in LDS once per work-group; the int8 row is split into two planes (bytes 0-15 and 16-31 of each 32-block) so lanes reading
// consecutive blocks read consecutive 16-byte words. DUMP: the same kernel writes each block's int32 sums
// (dbg_isum, and Q4_K / Q5_K min sums to dbg_msum) instead of the output.
//
// AREG (batch 1 only): lane j reads the same blocks of the token row for every weight row, so it loads them once into
// registers (two 16-byte words, the scale and the Q4_K / Q5_K / Q6_K sums per block) and nothing is staged in LDS.
template <int TYPE, int LPR, int CH, bool EXACT, int TB, int PF, bool DUMP, bool AREG = false, int NT = 256,
          bool SPLIT = false>
__global__ __launch_bounds__(NT) void gemvs_kernel(GemvArgs a) {
  static_assert(!AREG || TB == 1, "token blocks in registers: batch 1 only");
  extern __shared__ uint4 smem[];
  using Tr = Traits<TYPE>;
  constexpr int GPW = NT / LPR;                  // lane groups per work-group
  constexpr int WPR = LPR > 64 ? LPR / 64 : 1;   // waves per row
  const int K = a.w.K, nb = K / 32, rows = a.w.rows, T = a.T;
  // LDS: per token t < TB: int8 planes [2][nb][16] at t*K, then scales [TB][nb], then Q4_K block sums [TB][nb]
  uint8_t* sq = (uint8_t*)smem;
  float* ssc = (float*)(sq + (size_t)TB * K);
  int* sbs = (int*)(ssc + (size_t)TB * nb);
  __shared__ typename LdsFor<TYPE>::type lds;
  constexpr int RC = WPR > 1 ? 8 : 1;  // rows per cross-wave combine (several waves per row)
  __shared__ float part[2][RC][GPW][WPR][TB];
  const int grp = threadIdx.x / LPR, gl = threadIdx.x % LPR;
  const int G = gridDim.x * GPW;
  const int g0 = blockIdx.x * GPW + grp;
  // Rows: steps i < s2 sweep all groups in lockstep (row g0 + G i). With a split (a.split > 0: the work-groups of the
  // first dispatch round, one per CU), s2 is two steps short of the sweep and the first-round groups then take the
  // remaining rows: the second work-group on a CU issues its loads behind the first one's, so its rows arrive about
  // two row steps later; on the 17408-wide down projection the two rounds then end together (12.4 vs 13.0 us in a
  // launch loop on one box).
  // (a compile-time switch: the split's row mapping costs registers that the multi-token instantiations need)
  const int split = SPLIT ? a.split : 0, G1 = split * GPW;
  const int s2 = split > 0 ? max(1, (rows + G - 1) / G - 2) : (rows + G - 1) / G;
  auto row_of = [&](int i) { return i < s2 ? g0 + G * i : G * s2 + g0 + G1 * (i - s2); };
  auto steps_of = [&](int g) {
    if (split > 0 && g < G1 && G * s2 + g < rows) return s2 + (rows - 1 - G * s2 - g) / G1 + 1;
    return g < rows ? min(s2, (rows - 1 - g) / G + 1) : 0;
  };
  // (with several waves per row every group of the work-group runs its first group's step count, for the combine's
  // barrier; the extra steps of its other groups recompute a row past the end without storing it)
  // (two rows in flight, no split: the first group of a wave has the most rows, and every group of the wave runs its
  //  step count -- a group's extra step reads a clamped row and stores nothing. A wave-uniform trip count keeps the
  //  loop off the exec mask; with a per-group count the compiler must assume the loads of a step that some lanes
  //  skipped are still pending at the next fetch, and waits there for nearly every load in flight. Measured on the
  //  IQ4_XS gate/up shape: 10.86 -> 10.53 us; the one-row-in-flight launches keep the per-group count)
  const int steps = WPR > 1 ? steps_of((int)blockIdx.x * GPW)
                    : (SPLIT || PF != 2) ? steps_of(g0)
                            : __builtin_amdgcn_readfirstlane(steps_of((int)blockIdx.x * GPW + (int)(threadIdx.x / 64) * (64 / LPR)));
  RawBlk cur[CH];
  auto fetch = [&](int i, RawBlk* dst) {
    const int n = min(row_of(i), rows - 1);
    const uint8_t* qrow = a.w.qs + (size_t)n * nb * Tr::QB;
    const uint8_t* hrow = a.w.hdr + (size_t)n * (nb / 8) * Tr::HB;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int b = gl + LPR * u;
      dst[u] = load_block_at<TYPE>(qrow, hrow, EXACT ? b : min(b, nb - 1));
    }
  };
  fetch(0, cur);
  lds_fill<TYPE>(&lds);
  u32x4_t xr[AREG ? CH : 1][2];
  float xs[AREG ? CH : 1];
  int xb[AREG ? CH : 1];
  if constexpr (AREG) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int b = EXACT ? gl + LPR * u : min(gl + LPR * u, nb - 1);
      xr[u][0] = *(const u32x4_t*)(a.aq + 32 * b);
      xr[u][1] = *(const u32x4_t*)(a.aq + 32 * b + 16);
      if constexpr (!DUMP) xs[u] = a.asc[(size_t)b * a.M_stride];
      if constexpr (kNeedsBsum<TYPE>)
        xb[u] = (int)(uint16_t)a.absum[(size_t)(2 * b) * a.M_stride] | ((int)a.absum[(size_t)(2 * b + 1) * a.M_stride] << 16);
    }
  }
  // staging: every thread issues all of its loads (at most SB 16-byte chunks, predicated) before its first LDS store
  // (a loop of load -> store pairs waits out one L2 round trip per chunk)
  constexpr int SB = 8;
  if constexpr (!AREG)
  for (int i0 = threadIdx.x; i0 < 2 * nb * TB; i0 += NT * SB) {
    u32x4_t v[SB];  // (a native vector type: an array of uint4 structs would live in scratch memory)
#pragma unroll
    for (int k = 0; k < SB; ++k) {
      const int i = i0 + NT * k;
      if (i < 2 * nb * TB) {
        const int t = i / (2 * nb), r = i % (2 * nb), b = r >> 1, h = r & 1;
        const int tt = min(t, T - 1);  // (tokens past T: a copy of the last, never stored)
        v[k] = *(const u32x4_t*)(a.aq + (size_t)tt * K + 32 * b + 16 * h);
      }
    }
#pragma unroll
    for (int k = 0; k < SB; ++k) {
      const int i = i0 + NT * k;
      if (i < 2 * nb * TB) {
        const int t = i / (2 * nb), r = i % (2 * nb), b = r >> 1, h = r & 1;
        *(u32x4_t*)(sq + (size_t)t * K + (size_t)h * nb * 16 + b * 16) = v[k];
      }
    }
  }
  if constexpr (!AREG)
  for (int i0 = threadIdx.x; i0 < nb * TB; i0 += NT * SB) {
    float sv[SB];
    int bv[SB];
#pragma unroll
    for (int k = 0; k < SB; ++k) {
      const int i = i0 + NT * k;
      if (i < nb * TB) {
        const int t = i / nb, b = i % nb, tt = min(t, T - 1);
        if constexpr (!DUMP) sv[k] = a.asc[(size_t)b * a.M_stride + tt];  // (the block-sum mode has no scales)
        if constexpr (kNeedsBsum<TYPE>)
          bv[k] = (int)(uint16_t)a.absum[(size_t)(2 * b) * a.M_stride + tt] |
                  ((int)a.absum[(size_t)(2 * b + 1) * a.M_stride + tt] << 16);
      }
    }
#pragma unroll
    for (int k = 0; k < SB; ++k) {
      const int i = i0 + NT * k;
      if (i < nb * TB) {
        if constexpr (!DUMP) ssc[i] = sv[k];
        if constexpr (kNeedsBsum<TYPE>) sbs[i] = bv[k];
      }
    }
  }
  __syncthreads();
  const KvTab kv = kv_tab();
  // one row step: decode the group's row i from cur, reduce across the row's lanes, store
  auto row_step = [&](int i, const RawBlk* cur) {
    float acc[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int b = gl + LPR * u;
      if (EXACT || b < nb) {
        uint32_t wd[8];
        int sc, sc1, mn;
        BlockInts bi;
        decode_block32<TYPE>(cur[u], &lds, b & 7, kv, wd, sc, sc1, mn, bi.d, bi.dmin);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
          uint4 x0, x1;
          int bp;
          if constexpr (AREG) {
            x0 = uint4{xr[u][0][0], xr[u][0][1], xr[u][0][2], xr[u][0][3]};
            x1 = uint4{xr[u][1][0], xr[u][1][1], xr[u][1][2], xr[u][1][3]};
            bp = kNeedsBsum<TYPE> ? xb[u] : 0;
          } else {
            const uint8_t* st = sq + (size_t)t * K;
            x0 = *(const uint4*)(st + b * 16);
            x1 = *(const uint4*)(st + (size_t)nb * 16 + b * 16);
            bp = kNeedsBsum<TYPE> ? sbs[t * nb + b] : 0;
          }
          block_dot<TYPE>(wd, sc, sc1, mn, x0, x1, (int)(int16_t)(bp & 0xFFFF), bp >> 16, bi.iv, bi.mv);
          if constexpr (DUMP) {
            const int n = row_of(i);
            if (n < rows && t < T) {
              const size_t o = ((size_t)t * rows + n) * nb + b;
              a.dbg_isum[o] = bi.iv;
              if constexpr (Traits<TYPE>::MINS) a.dbg_msum[o] = bi.mv;
            }
          } else {
            acc[t] += block_value<TYPE>(AREG ? xs[u] : ssc[t * nb + b], bi);
          }
        }
      }
      // (eight tokens: one block's token rows at a time -- left free, the compiler reads every block's rows for
      // every token from LDS up front and runs out of registers)
      if constexpr (TB >= 8) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (PF == 2 && !EXACT) {
      // (the last chunk is decoded under a branch that whole waves skip; a use of its registers on every path marks
      //  its loads complete here -- otherwise the compiler assumes them pending at the next fetch and waits there for
      //  nearly every load in flight, the other row's included)
#pragma unroll
      for (int u = 0; u < CH; ++u) asm volatile("" ::"v"(cur[u].q0), "v"(cur[u].h));
    }
    if constexpr (WPR > 1) {
      // each wave's row sum goes to LDS; every RC rows one barrier, then lane j of the group adds the WPR partials of
      // the chunk's row j (in wave order) and stores it. Two chunk buffers: a chunk's partials are read after the
      // barrier that ends it and overwritten only after the next one.
      const int hb = (i / RC) & 1, slot = i % RC;
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        const float w = wave_sum_width(acc[t], 64);
        if ((threadIdx.x & 63) == 0) part[hb][slot][grp][gl >> 6][t] = w;
      }
      if (slot == RC - 1 || i == steps - 1) {
        __syncthreads();
        const int nj = slot + 1, j = gl;
        const int nr = row_of(i - slot + j);
        if (!DUMP && j < nj && nr < rows) {
#pragma unroll
          for (int t = 0; t < TB; ++t) {
            float v = part[hb][j][grp][0][t];
#pragma unroll
            for (int k = 1; k < WPR; ++k) v += part[hb][j][grp][k][t];
            if (t < T) {
              float* cp = a.C + (size_t)t * a.ldc + a.c_off + nr;
              *cp = a.accumulate ? *cp + v : v;
            }
          }
        }
      }
      return;
    }
    const int n = row_of(i);
    float v[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) v[t] = wave_sum_width(acc[t], LPR);
    if (!DUMP && gl == 0 && n < rows) {
#pragma unroll
      for (int t = 0; t < TB; ++t)
        if (t < T) {
          float* cp = a.C + (size_t)t * a.ldc + a.c_off + n;
          *cp = a.accumulate ? *cp + v[t] : v[t];
        }
    }
  };
  if constexpr (PF == 2) {
    // two rows in flight per group: row i + 1's loads are issued before row i is decoded (two register sets that
    // alternate, so no copy waits for a load)
    // (no exit between the two halves: with one, the compiler merges the path that leaves after the first half into
    //  the loop head, takes that half's loads as pending there and waits for nearly every load in flight before the
    //  next fetch)
    RawBlk nxt[CH];
    int i = 0;
    for (; i + 1 < steps; i += 2) {
      fetch(i + 1, nxt);  // (clamped to the last row: loads past the group's rows are harmless)
      row_step(i, cur);
      fetch(i + 2, cur);
      row_step(i + 1, nxt);
    }
    if (i < steps) row_step(i, cur);
  } else {
    for (int i = 0; i < steps; ++i) {
      row_step(i, cur);
      fetch(i + 1, cur);  // (unconditional and clamped to the last row: no branch between the decode and the loads)
    }
  }
}

// Most tokens per gemvs_kernel launch: 8, or 4 where eight tokens' registers would spill (more than 5 blocks per lane,
// more than 4 for Q6_K) or where two 4-token launches measured faster (IQ2_XXS at 4+ blocks per lane, applied to the
// grid-decoded types alike); more tokens run as chunks.
template <int TYPE>
constexpr int gemvs_max_tb(int ch) { return ch <= (TYPE == T_Q6_K ? 4 : (kIq2<TYPE> || kIq1<TYPE>) ? 3 : 5) ? 8 : 4; }

// LDS bytes of gemvs_kernel for TB tokens (the per-16 sums for the types that read them: kNeedsBsum)
template <int TYPE>
static size_t gemvs_lds(int K, int TB) {
  const int nb = K / 32;
  return (size_t)TB * ((size_t)K + sizeof(float) * nb + (kNeedsBsum<TYPE> ? sizeof(int) * nb : 0));
}

template <int TYPE, int LPR, int CH, bool EXACT, int TB, bool DUMP, bool AREG = false, int PC = (LPR == 256 ? 3 : 2),
          bool SPLIT = false>
static hipError_t gos(const GemvArgs& a0, hipStream_t s) {
  constexpr int GPW = 256 / LPR;
  // batch 1: two rows in flight per lane group (three measured slower: 11.4 -> 13.0 us on the down projection,
  // 10.5 -> 11.8 on gate/up, also with one work-group per CU); two tokens: two rows as well where the registers
  // allow (IQ4_XS 5120 -> 17408 at T 2: 13.7 -> 12.6 us); more tokens: registers to tokens (at T 4 two rows spill:
  // 17.7 -> 21.6 us)
  constexpr int PF = TB == 1 || (TB == 2 && CH <= 5) ? 2 : 1;
  // Persistent grid: PC work-groups per CU (two; three with four waves per row or where measured faster), or as many
  // as the kernel's registers and LDS let reside (the 8-token instantiation needs more than 256 registers: one wave per
  // SIMD), so the whole grid is resident at once; fewer when the matrix has fewer rows than lane groups. Occupancy is
  // queried once, for this instantiation's largest K.
  static const int per_cu = [] {
    int n = 0;
    const size_t lds_max = AREG ? 0 : gemvs_lds<TYPE>(32 * LPR * CH, TB);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemvs_kernel<TYPE, LPR, CH, EXACT, TB, PF, false, AREG, 256, SPLIT>, 256, lds_max) !=
            hipSuccess || n < 1)
      n = 1;
    return min(PC, n);
  }();
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1)
      n = 256;
    return n;
  }();
  const int wgs = min(per_cu * cus, (a0.w.rows + GPW - 1) / GPW);
  GemvArgs a = a0;
  a.split = SPLIT && wgs > cus && a.w.rows > 2 * wgs * GPW ? cus : 0;
  gemvs_kernel<TYPE, LPR, CH, EXACT, TB, PF, DUMP, AREG, 256, SPLIT><<<wgs, 256, AREG ? 0 : gemvs_lds<TYPE>(a.w.K, TB), s>>>(a);
  return hipGetLastError();
}

template <int TYPE, int LPR, int CH, bool EXACT, bool DUMP>
static hipError_t gos_tb(const GemvArgs& a, hipStream_t s) {
  switch (a.T <= 1 ? 1 : a.T <= 2 ? 2 : a.T <= 4 ? 4 : 8) {
    case 1:
      // batch 1, 32 lanes per row (K 5120 -> N 17408, A/B in one process): IQ3_S and IQ3_XXS with the token blocks in
      // registers and three work-groups per CU 14.0 -> 13.1 and 12.5 -> 12.0 us (less LDS traffic beside their
      // codebook lookups); Q3_K with three work-groups per CU 10.8 -> 10.5 us; the other types measured no faster
      if constexpr (LPR == 32 && (TYPE == T_IQ3_S || TYPE == T_IQ3_XXS)) return gos<TYPE, LPR, CH, EXACT, 1, DUMP, true, 3>(a, s);
      if constexpr (LPR == 32 && TYPE == T_Q3_K) return gos<TYPE, LPR, CH, EXACT, 1, DUMP, false, 3>(a, s);
      return gos<TYPE, LPR, CH, EXACT, 1, DUMP>(a, s);
    case 2: return gos<TYPE, LPR, CH, EXACT, 2, DUMP>(a, s);
    case 4: return gos<TYPE, LPR, CH, EXACT, 4, DUMP>(a, s);
    default:
      if constexpr (gemvs_max_tb<TYPE>(CH) >= 8) return gos<TYPE, LPR, CH, EXACT, 8, DUMP>(a, s);
      else return hipErrorInvalidValue;  // (the dispatcher never asks: it chunks by gemvs_max_tb)
  }
}

template <int TYPE, int LPR, int R, int TB, bool DUMP, int U = (TYPE == T_IQ3_S || kIq2<TYPE> || kIq1<TYPE> ? 1 : TB == 1 ? 4 : TB <= 2 ? 2 : 1)>
static hipError_t go(const GemvArgs& a, hipStream_t s) {
  constexpr int rows_per_wg = 4 * (64 / LPR) * R;
  const dim3 grid((unsigned)((a.w.rows + rows_per_wg - 1) / rows_per_wg)), block(256);
  gemv_kernel<TYPE, LPR, R, TB, U, DUMP><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

// The route of one call: the sweep kernel for rows of up to 1024 blocks (K <= 32768), in token chunks; the generic
// kernel beyond. The block-sum mode (DUMP) takes exactly the route, instantiation and token chunking of the
// product, so the sums checked are those of the kernels that run.
template <int TYPE, bool DUMP>
static hipError_t gemv_route(const GemvArgs& a, hipStream_t s) {
  const int nb = a.w.K / 32;
  const bool l32 = nb % 32 == 0;
  if (nb <= 1024) {
    // tokens per launch: as many as fit in 80 KB of LDS (two work-groups per CU), up to 8; more tokens -> chunks
    // of tokens, each launch reading the weights once
    int tb = gemvs_max_tb<TYPE>(nb <= 256 ? (nb + 31) / 32 : (nb + 127) / 128);
    const size_t cap = 80 * 1024 - sizeof(typename LdsFor<TYPE>::type);  // (the codebook tables' static LDS)
    while (tb > 1 && gemvs_lds<TYPE>(a.w.K, tb) > cap) tb >>= 1;
    for (int t0 = 0; t0 < a.T; t0 += tb) {
      GemvArgs c = a;
      c.T = min(tb, a.T - t0);
      c.aq = a.aq + (size_t)t0 * a.w.K;
      if (!DUMP) {
        c.asc = a.asc + t0;
        if (a.absum) c.absum = a.absum + t0;
        c.C = a.C + (size_t)t0 * a.ldc;
      } else {
        if (a.absum) c.absum = a.absum + t0;
        c.dbg_isum = a.dbg_isum + (size_t)t0 * a.w.rows * nb;
        if (a.dbg_msum) c.dbg_msum = a.dbg_msum + (size_t)t0 * a.w.rows * nb;
      }
      hipError_t e;
      if (a.T == 1 && nb > 64 && nb <= 256 && a.w.rows <= 6144) {
        // batch 1, a small matrix (the grid has about one row per 32-lane group) with rows of more than 64 blocks (so
        // at least half of the 128 lanes have a block): 128 lanes per row, token blocks in registers, three
        // work-groups per CU. Measured against 32 lanes per row: Q8_0 4096 x 4096 6.8 -> 6.4 us,
        // IQ3_S 5120 x 5120 7.7 -> 6.8 us, IQ4_XS 5120 x 5120 6.7 -> 6.2 us. Q8_0 (32 payload bytes per block, twice the
        // 4-bit types') with two work-groups per CU instead: 4096 x 4096 6.2 -> 5.8 us, 5120 x 5120 8.6 -> 7.9 us (A/B
        // in one process; every 4-bit and grid type measured faster with three)
        constexpr int PCS = TYPE == T_Q8_0 ? 2 : 3;
        e = nb <= 128 ? gos<TYPE, 128, 1, false, 1, DUMP, true, PCS>(c, s)
                      : gos<TYPE, 128, 2, false, 1, DUMP, true, PCS>(c, s);
      } else if (a.T == 1 && nb > 512 && nb <= 768) {
        // batch 1, long rows: 128 lanes (two waves) per row, token blocks in registers: the 17408-wide down projection
        // (544 blocks) at 11.9 us against 12.3 us with four waves per row and the token row in LDS
        e = nb <= 640 ? gos<TYPE, 128, 5, false, 1, DUMP, true, 2, true>(c, s)
                      : gos<TYPE, 128, 6, false, 1, DUMP, true, 2, true>(c, s);
      } else if (nb <= 256) {  // 32 lanes per row, up to 8 blocks per lane
        switch ((nb + 31) / 32) {
          case 1: e = nb == 32 ? gos_tb<TYPE, 32, 1, true, DUMP>(c, s) : gos_tb<TYPE, 32, 1, false, DUMP>(c, s); break;
          case 2: e = nb == 64 ? gos_tb<TYPE, 32, 2, true, DUMP>(c, s) : gos_tb<TYPE, 32, 2, false, DUMP>(c, s); break;
          case 3: e = nb == 96 ? gos_tb<TYPE, 32, 3, true, DUMP>(c, s) : gos_tb<TYPE, 32, 3, false, DUMP>(c, s); break;
          case 4: e = nb == 128 ? gos_tb<TYPE, 32, 4, true, DUMP>(c, s) : gos_tb<TYPE, 32, 4, false, DUMP>(c, s); break;
          case 5: e = nb == 160 ? gos_tb<TYPE, 32, 5, true, DUMP>(c, s) : gos_tb<TYPE, 32, 5, false, DUMP>(c, s); break;
          case 6: e = nb == 192 ? gos_tb<TYPE, 32, 6, true, DUMP>(c, s) : gos_tb<TYPE, 32, 6, false, DUMP>(c, s); break;
          case 7: e = nb == 224 ? gos_tb<TYPE, 32, 7, true, DUMP>(c, s) : gos_tb<TYPE, 32, 7, false, DUMP>(c, s); break;
          default: e = nb == 256 ? gos_tb<TYPE, 32, 8, true, DUMP>(c, s) : gos_tb<TYPE, 32, 8, false, DUMP>(c, s); break;
        }
      } else if (nb > 512 && nb <= 768) {
        // several tokens: 256 lanes (the work-group's four waves) per row, 3 blocks per lane, three work-groups per CU
        e = nb == 768 ? gos_tb<TYPE, 256, 3, true, DUMP>(c, s) : gos_tb<TYPE, 256, 3, false, DUMP>(c, s);
      } else {  // long rows: 128 lanes (two waves) per row, up to 8 blocks per lane
        switch ((nb + 127) / 128) {
          case 3: e = nb == 384 ? gos_tb<TYPE, 128, 3, true, DUMP>(c, s) : gos_tb<TYPE, 128, 3, false, DUMP>(c, s); break;
          case 4: e = nb == 512 ? gos_tb<TYPE, 128, 4, true, DUMP>(c, s) : gos_tb<TYPE, 128, 4, false, DUMP>(c, s); break;
          case 5: e = nb == 640 ? gos_tb<TYPE, 128, 5, true, DUMP>(c, s) : gos_tb<TYPE, 128, 5, false, DUMP>(c, s); break;
          case 6: e = nb == 768 ? gos_tb<TYPE, 128, 6, true, DUMP>(c, s) : gos_tb<TYPE, 128, 6, false, DUMP>(c, s); break;
          case 7: e = nb == 896 ? gos_tb<TYPE, 128, 7, true, DUMP>(c, s) : gos_tb<TYPE, 128, 7, false, DUMP>(c, s); break;
          default: e = nb == 1024 ? gos_tb<TYPE, 128, 8, true, DUMP>(c, s) : gos_tb<TYPE, 128, 8, false, DUMP>(c, s); break;
        }
      }
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  if (a.T <= 1) {
    // long rows (K > 32768: few rows): one row per lane group, for more waves in flight
    return l32 ? go<TYPE, 32, 1, 1, DUMP>(a, s) : go<TYPE, 8, 2, 1, DUMP>(a, s);
  }
  if (a.T <= 2) return l32 ? go<TYPE, 32, 1, 2, DUMP>(a, s) : go<TYPE, 8, 1, 2, DUMP>(a, s);
  if (a.T <= 4) return l32 ? go<TYPE, 32, 1, 4, DUMP>(a, s) : go<TYPE, 8, 1, 4, DUMP>(a, s);
  return l32 ? go<TYPE, 32, 1, 8, DUMP>(a, s) : go<TYPE, 8, 1, 8, DUMP>(a, s);
}

template <int TYPE>
hipError_t gemv_dispatch(const GemvArgs& a, hipStream_t s) {
  return a.dbg_isum ? gemv_route<TYPE, true>(a, s) : gemv_route<TYPE, false>(a, s);
}

}  // namespace qm
