// Prompt GEMM on the f16 matrix pipe for the types whose per-block weight scale is an integer and whose block values
// times that scale fit an f16 exactly (Q4_K: sc * q <= 63 * 15 = 945 < 2048).
//
// The reference's product (zero/kernels/gemm.cl:367-398) is, per token m, weight row n, 32-block b and superblock s,
//   I[m,n,b] = sc[n,b] * sum_k a[m,k] q[n,k]                  (the int32 block sum times the integer block scale)
//   tq  = sum_b fma(asc[m,b], I, .)        tmn = sum_b fma(asc[m,b], mn[n,b] * bsum[m,b], .)     (Q4_K mins)
//   res = fma(d[n,s], tq, fma(-dmin[n,s], tmn, res))
// Here I comes from two v_mfma_f32_32x32x16_f16 per block and 32 x 32 tile: the weights are decoded to sc * q in f16
// and the activations are their int8 values in f16, so every product is exact and the f32 sum of 32 of them
// (|I| <= 32 * 127 * 945 < 2^24) is the exact integer. The per-block activation scale is then applied with one f32 fma
// per element, as the reference does; with tokens on the MFMA's columns, asc is one value per lane. tmn is one bf16
// MFMA per superblock (asc * bsum split into two bf16 parts, 16 bits; mn exact), and d, dmin are applied once per
// superblock in the reference's order.
//
// Work-group: 4 waves, a tile of 128 weight rows x 128 tokens; wave w owns weight rows 32w..32w+31 (one MFMA row
// tile, decoded once per block in registers) for all 128 tokens (four 32-token column tiles). Two work-groups per CU,
// so one wave's scaling and decoding overlaps the other wave's MFMAs. The activations (f16, written by a prepass in
// MFMA operand order) are staged in LDS a block pair at a time, one pair ahead.
// MFMA orientation: A = weights (rows: weight rows n), B = activations (columns: tokens m).
// 32x32 result layout: lane l holds column l % 32 and rows 8 * (r / 4) + 4 * (l / 32) + r % 4, r = 0..15.
#include <stdlib.h>

#include <mutex>

#include "qm_decode.h"
#include "qm_launch.h"

namespace qm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kF16BM = 128;                        // tokens per work-group tile
constexpr int kF16BN = 128;                        // weight rows per work-group tile
constexpr int kF16Piece = 1024;                    // one MFMA operand piece of a 32-token tile: 64 lanes x 16 bytes
constexpr int kF16PairTile = 4 * kF16Piece;        // per 32-token tile and block pair: (block, chunk) pieces
constexpr int kF16PairBytes = 4 * kF16PairTile;    // per 128-token tile and block pair (16 KB)

// Element order inside a lane's 8-value f16 operand: the weight decode turns a word of nibble bytes t0..t3 into the
// f16 pairs (t0, t2), (t1, t3), so operand position i holds element 8h + f16_perm8(i) of its 16-element chunk.
__host__ __device__ constexpr int f16_perm8(int i) { return (i & 4) | ((i & 1) << 1) | ((i >> 1) & 1); }

static size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Workspace of one call (device bytes), for M tokens and K columns: the f16 activations, then the mins operand.
size_t f16_workspace_bytes(int M, int K) {
  const size_t Mp = round_up((size_t)M, kF16BM);
  return round_up(Mp * (size_t)K * 2, 256) + Mp * (size_t)(K / 32) * 4;
}

// ---- prepass: the int8 activations as f16 in MFMA operand order, and (MINS) the mins operand u = asc * bsum split
// into two bf16 parts (one 32-bit word per token and block: bf16 hi | lo << 16; per superblock the 8 words are the
// bf16 MFMA's B operand, slot 8h + i = block 4h + i / 2, part i % 2).
// One thread per (token, 32-block, k-half h); consecutive threads take consecutive lanes of one operand piece
// (token % 32, then h), so each wave writes whole 1 KB pieces. A thread writes lane (token % 32, h)'s 16 bytes of the
// block's two pieces: chunk c = 0 holds elements 8h + perm8(i), chunk 1 elements 16 + 8h + perm8(i).
template <bool MINS>
__global__ __launch_bounds__(256) void f16_act_kernel(const int8_t* aq, const float* asc, const int16_t* absum, int M,
                                                      int M_stride, int ash, int Mp, int K, uint8_t* af, uint32_t* u) {
  const int nb = K / 32;
  const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int lanei = (int)(gid & 63), h = lanei >> 5;
  const int b = (int)((gid >> 6) % nb), mtile = (int)((gid >> 6) / nb);
  const int m = mtile * 32 + (lanei & 31);
  if (m >= Mp) return;
  uint32_t hw[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (m < M) {
    const int8_t* src = aq + (size_t)m * K + 32 * b;
    const uint2 q0 = *(const uint2*)(src + 8 * h), q1 = *(const uint2*)(src + 16 + 8 * h);
    const uint32_t qw[4] = {q0.x, q0.y, q1.x, q1.y};
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        uint32_t pr = 0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int e = f16_perm8(i + t);  // element 16c + 8h + e
          const int8_t qv = (int8_t)(qw[2 * c + (e >> 2)] >> (8 * (e & 3)));
          pr |= (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)qv) << (16 * t);
        }
        hw[4 * c + i / 2] = pr;
      }
  }
  // destination: [m / 128][pair b / 2][token tile (m % 128) / 32][piece 2 * (b % 2) + c][lane][16 B]
  uint8_t* base = af + ((size_t)(m / kF16BM) * (K / 64) + b / 2) * kF16PairBytes + ((m % kF16BM) / 32) * kF16PairTile +
                  (2 * (b & 1)) * kF16Piece + lanei * 16;
  *(uint4*)(base) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  *(uint4*)(base + kF16Piece) = make_uint4(hw[4], hw[5], hw[6], hw[7]);
  if constexpr (MINS) {
    if (h == 0) {
      float uv = 0.0f;
      if (m < M) {
        const int bs = (int)absum[(size_t)(2 * b) * M_stride + m] + (int)absum[(size_t)(2 * b + 1) * M_stride + m];
        uv = asc[(size_t)(b >> ash) * M_stride + m] * (float)bs;
      }
      const __bf16 uh = (__bf16)uv;
      const __bf16 ul = (__bf16)(uv - (float)uh);
      u[(size_t)m * nb + b] =
          (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, ul) << 16);
    }
  }
}

// ---- the GEMM

struct F16Args {
  WView w;
  const uint8_t* af;   // prepass output
  const uint32_t* u;   // mins operand
  const float* asc;
  int M, M_stride;
  int ash;             // asc row of 32-block b: b >> ash (per-32 scales: 0; per-256: 3)
  float* C;
  int ldc, c_off, accumulate;
  int32_t* dbg_isum;   // non-null: write the exact block sums sc * isum [M][rows][K/32] instead of C
};

// one VALU op: (x & mask) | c
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(c));
  return r;
}

// Q4_K: the lane's 16 values of one 32-block (payload bytes 8h..8h+7: x, y) times the integer block scale, as two
// f16 operands: chunk 0 the low nibbles (elements 8h + perm8(i)), chunk 1 the high nibbles (16 + 8h + perm8(i)).
// (1024 + q) as f16 is the bit pattern 0x6400 | q; one packed fma makes (1024 + q) sc - 1024 sc = sc q exactly. The
// high nibbles are not shifted down: left in mantissa bits 4-7 under the exponent of 16384 (0x7400 | q << 4) they
// read as 16384 + 256 q, and (16384 + 256 q) (sc / 256) - 64 sc = sc q exactly too (sc / 256 and 64 sc are exact in
// f16, and the fused multiply-add rounds only its exact integer result).
__device__ __forceinline__ void q4k_f16_decode(uint32_t x, uint32_t y, int sc, uint32_t c64, f16x8& b0, f16x8& b1) {
  const _Float16 s = (_Float16)sc;
  const f16x2 sc2 = {s, s}, off2 = {(_Float16)(-1024.0f) * s, (_Float16)(-1024.0f) * s};
  const _Float16 sh = s * (_Float16)0.00390625f;  // sc / 256
  const f16x2 sch2 = {sh, sh}, offh2 = {(_Float16)(-64.0f) * s, (_Float16)(-64.0f) * s};
  const uint32_t m = 0x000F000Fu, mh = 0x00F000F0u, c74 = 0x74007400u;
  const uint32_t x8 = x >> 8, y8 = y >> 8;
  const uint32_t w[8] = {and_or(x, m, c64), and_or(x8, m, c64), and_or(y, m, c64), and_or(y8, m, c64),
                         and_or(x, mh, c74), and_or(x8, mh, c74), and_or(y, mh, c74), and_or(y8, mh, c74)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 v0 = __builtin_bit_cast(f16x2, w[i]) * sc2 + off2;
    const f16x2 v1 = __builtin_bit_cast(f16x2, w[4 + i]) * sch2 + offh2;
    b0[2 * i] = v0[0];
    b0[2 * i + 1] = v0[1];
    b1[2 * i] = v1[0];
    b1[2 * i + 1] = v1[1];
  }
}

// Work-group -> (128-row weight tile, 128-token tile); consecutive work-groups of one XCD (work-groups are dealt to
// the 8 XCDs round-robin) take neighbouring weight tiles of one token tile, so the token tile stays in that XCD's L2.
__device__ __forceinline__ void f16_tile(int& nt, int& mt) {
  const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
  int lin = blockIdx.y * gx + blockIdx.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  mt = lin / gx;
  nt = lin % gx;
}

// S256: per-256 activation scales (the reference's act32 = false, gemm.cl:413-447): one scale per token and superblock,
// so the f16 MFMAs accumulate the whole superblock's products (sum_b sc * isum, in f32: exact while the partial sums
// stay below 2^24, i.e. for all but extreme rows, and within f32 rounding otherwise) and the scale is applied once per
// superblock, res = fma(d * asc, I, fma(-dmin, tmn, res)) -- no per-block VALU work.
template <int TYPE, bool DUMP, bool S256 = false>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(F16Args a) {
  // two activation stages of 16 KB, reused at the end to transpose the result tiles (4 waves x 32 x 33 floats)
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kF16PairBytes];
  __shared__ float dtab[4][2][32];  // per wave: d and dmin of its 32 rows (current superblock)
  __shared__ float sasc[2][2][kF16BM];  // per stage: the activation scales of the pair's two blocks, [block][token]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, lc = lane & 31;
  const int K = a.w.K, nb = K / 32, nsb = K / 256, npair = K / 64;
  int nt, mt;
  f16_tile(nt, mt);
  const int m0 = mt * kF16BM;
  const int n_rows = a.w.rows;
  const int nbase = nt * kF16BN + wave * 32;
  const int nrow = min(nbase + lc, n_rows - 1);  // this lane's A-operand row
  const uint8_t* qrow = a.w.qs + (size_t)nrow * nb * 16 + 8 * h;
  const uint8_t* hrow = a.w.hdr + (size_t)nrow * nsb * 16;
  const uint8_t* abase = a.af + (size_t)mt * npair * kF16PairBytes;
  const uint32_t c64 = 0x64006400u;

  // activation staging: 16 KB per block pair, 4 x 16 bytes per thread
  u32x4_t st[4];
  auto fetch = [&](int g) {
#pragma unroll
    for (int c = 0; c < 4; ++c) st[c] = *(const u32x4_t*)(abase + (size_t)g * kF16PairBytes + (tid + 256 * c) * 16);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) *(u32x4_t*)(lds + buf * kF16PairBytes + (tid + 256 * c) * 16) = st[c];
  };
  // activation scales of a block pair, staged with its activations: thread tid takes block tid / 128, token tid % 128
  float st_sc;
  const int sc_row = min(m0 + (tid & (kF16BM - 1)), a.M - 1);
  // (the block-sum mode has no activation scales: a.asc is null there and is never read)
  auto fetch_sa = [&](int g) {
    if constexpr (!DUMP) st_sc = a.asc[(size_t)((2 * g + (tid >> 7)) >> a.ash) * a.M_stride + sc_row];
  };
  auto store_sa = [&](int buf) {
    if constexpr (!DUMP) sasc[buf][tid >> 7][tid & (kF16BM - 1)] = st_sc;
  };

  f32x16 tq[4], res[4];
  float sv256[4];  // S256: the superblock's activation scale of each token tile
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) res[t][r] = 0.0f;
  const f32x16 zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  uint4 hdr = *(const uint4*)hrow, hdr_n;
  uint2 pay[2], pay_n[2];
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) pay[bb] = *(const uint2*)(qrow + bb * 16);
  fetch_sa(0);
  fetch(0);
  store(0);
  store_sa(0);
  __syncthreads();

  for (int s = 0; s < nsb; ++s) {
    const int sn = s + 1 < nsb ? s + 1 : s;
    hdr_n = *(const uint4*)(hrow + (size_t)sn * 16);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int g = 4 * s + p, cur = g & 1;
      const int gn = g + 1 < npair ? g + 1 : g;
      fetch(gn);
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) pay_n[bb] = *(const uint2*)(qrow + (size_t)(2 * gn + bb) * 16);
      fetch_sa(gn);
      // (keeps the loads here: issued a whole pair of MFMA work before their data is needed)
      __builtin_amdgcn_sched_barrier(0);
      f16x8 aw[2][2];
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        int sc, mn;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * p + bb, sc, mn);
        (void)mn;
        q4k_f16_decode(pay[bb].x, pay[bb].y, sc, c64, aw[bb][0], aw[bb][1]);
      }
      const uint8_t* L = lds + cur * kF16PairBytes + lane * 16;
      if constexpr (S256) {
        // items block-major (k = 4 bb + t): consecutive MFMAs feed different token tiles' accumulators
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int t = k & 3, bb = k >> 2;
          const uint8_t* Lt = L + t * kF16PairTile;
          const f16x8 b0 = *(const f16x8*)(Lt + (2 * bb) * kF16Piece);
          const f16x8 b1 = *(const f16x8*)(Lt + (2 * bb + 1) * kF16Piece);
          const f32x16 c = (p == 0 && bb == 0) ? zero16 : tq[t];
          tq[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aw[bb][0], b0, c, 0, 0, 0);
          tq[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aw[bb][1], b1, tq[t], 0, 0, 0);
        }
      } else {
        // items k = (token tile t, block bb), t = k / 2, bb = k % 2. Stage k: item k's first MFMA, item k + 1's
        // operands read from LDS, half of item k - 1's scaling fmas, item k's second MFMA (it accumulates onto the
        // first, so it waits for it: the eight fmas fill that wait), the other half of the fmas. One MFMA result is in
        // flight while the previous one is consumed, and the next item's LDS round trip runs under both (605 -> 579 ->
        // 561 us on the 2048 x 5120 x 17408 shape for the operand prefetch and then the split fmas, A/B in one process).
        f32x16 Iprev;
        f16x8 nb0 = *(const f16x8*)(L), nb1 = *(const f16x8*)(L + kF16Piece);  // (item 0)
        float nsv = DUMP ? 0.0f : sasc[cur][0][lc], svprev = 0.0f;
#pragma unroll
        for (int k = 0; k <= 8; ++k) {
          f32x16 Icur;
          float svcur = 0.0f;
          const int bb = k & 1;
          const f16x8 b1 = nb1;
          if (k < 8) {
            const f16x8 b0 = nb0;
            svcur = nsv;
            Icur = __builtin_amdgcn_mfma_f32_32x32x16_f16(aw[bb][0], b0, zero16, 0, 0, 0);
            if (k + 1 < 8) {
              const int t1 = (k + 1) >> 1, bb1 = (k + 1) & 1;
              const uint8_t* Lt = L + t1 * kF16PairTile;
              nb0 = *(const f16x8*)(Lt + (2 * bb1) * kF16Piece);
              nb1 = *(const f16x8*)(Lt + (2 * bb1 + 1) * kF16Piece);
              if constexpr (!DUMP) nsv = sasc[cur][bb1][32 * t1 + lc];
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          const int tp = (k - 1) >> 1, bbp = (k - 1) & 1;
          if constexpr (!DUMP) {
            if (k > 0) {
#pragma unroll
              for (int r = 0; r < 8; ++r)
                tq[tp][r] = (p == 0 && bbp == 0) ? svprev * Iprev[r] : fmaf(svprev, Iprev[r], tq[tp][r]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          if (k < 8) Icur = __builtin_amdgcn_mfma_f32_32x32x16_f16(aw[bb][1], b1, Icur, 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
          if (k > 0) {
            if constexpr (DUMP) {
              const int m = m0 + 32 * tp + lc, blk = 8 * s + 2 * p + bbp;
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int n = nbase + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < a.M && n < n_rows) a.dbg_isum[((size_t)m * n_rows + n) * nb + blk] = (int)Iprev[r];
              }
            } else {
#pragma unroll
              for (int r = 8; r < 16; ++r)
                tq[tp][r] = (p == 0 && bbp == 0) ? svprev * Iprev[r] : fmaf(svprev, Iprev[r], tq[tp][r]);
              // (pins the scaled sums here: otherwise the compiler defers every fma to the superblock end and keeps
              // each block's MFMA result alive meanwhile, in scratch memory)
#pragma unroll
              for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(tq[tp][r]));
            }
          }
          if (k < 8) {
            Iprev = Icur;
            svprev = svcur;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (S256 && !DUMP) {
        // the superblock's scale (its last pair's stage) is read before this pair's barrier: the next superblock's
        // first pair overwrites that stage after the barrier, possibly while a slower wave is still in this epilogue
        if (p == 3)
#pragma unroll
          for (int t = 0; t < 4; ++t) sv256[t] = sasc[cur][0][32 * t + lc];
      }
      store(cur ^ 1);
      store_sa(cur ^ 1);
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) pay[bb] = pay_n[bb];
      __syncthreads();
    }
    if constexpr (!DUMP) {
      // superblock epilogue: res = fma(d, tq, fma(-dmin, tmn, res)) (gemm.cl:395-398). d and dmin are per weight row,
      // i.e. per result register: each lane publishes its row's pair in LDS and reads those of its 16 rows.
      if (h == 0) {
        dtab[wave][0][lc] = h2f(hdr.x);
        dtab[wave][1][lc] = h2f(hdr.x >> 16);
      }
      int mn[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        int scv;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, b, scv, mn[b]);
      }
      // mins operand (A: weight rows): slot 8h + i = mn of block 4h + i / 2 (a bit select on the two candidates: a
      // lane-dependent array index would put mn in scratch memory)
      bf16x8 mnop;
      const int hm = -h;
#pragma unroll
      for (int i = 0; i < 8; ++i) mnop[i] = (__bf16)(float)((mn[i / 2] & ~hm) | (mn[4 + i / 2] & hm));
      float dr[16], dmr[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 dv = *(const float4*)&dtab[wave][0][8 * q + 4 * h];
        const float4 mv = *(const float4*)&dtab[wave][1][8 * q + 4 * h];
        dr[4 * q] = dv.x; dr[4 * q + 1] = dv.y; dr[4 * q + 2] = dv.z; dr[4 * q + 3] = dv.w;
        dmr[4 * q] = -mv.x; dmr[4 * q + 1] = -mv.y; dmr[4 * q + 2] = -mv.z; dmr[4 * q + 3] = -mv.w;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint4 uv = *(const uint4*)(a.u + (size_t)(m0 + 32 * t + lc) * nb + 8 * s + 4 * h);
        const f32x16 tmn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mnop, __builtin_bit_cast(bf16x8, uv), zero16, 0, 0, 0);
        if constexpr (S256) {
          const float sv = sv256[t];
#pragma unroll
          for (int r = 0; r < 16; ++r) res[t][r] = fmaf(dr[r] * sv, tq[t][r], fmaf(dmr[r], tmn[r], res[t][r]));
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) res[t][r] = fmaf(dr[r], tq[t][r], fmaf(dmr[r], tmn[r], res[t][r]));
        }
      }
    }
    hdr = hdr_n;
  }
  if constexpr (DUMP) return;

  // ---- store through LDS: each wave writes a 32 x 32 result tile as [row n][token m], then lanes 0-31 / 32-63 store
  // tokens 2k / 2k + 1 with 32 consecutive weight rows each (128-byte rows of C)
  float* T = (float*)lds + wave * 32 * 33;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) T[(8 * (r >> 2) + 4 * h + (r & 3)) * 33 + lc] = res[t][r];
    __builtin_amdgcn_wave_barrier();
    const int n = nbase + lc;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int ml = 2 * k + h, m = m0 + 32 * t + ml;
      const float v0 = T[lc * 33 + ml];
      if (m < a.M && n < n_rows) {
        float* cp = a.C + (size_t)m * a.ldc + a.c_off + n;
        float v = v0;
        if (a.accumulate == 1) {
          v += *cp;
        } else if (a.accumulate == 2) {
          const float gv = *cp;
          v *= gv / (1.0f + expf(-gv));
        }
        *cp = v;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---- host side

bool f16_gemm_supported(int type, int M, int K) {
  if (type != T_Q4_K) return false;
  return M >= 128 && K % 256 == 0;
}

// One memory pool per device for the per-call workspace (stream-ordered: concurrent calls on different streams get
// different buffers; the pool keeps freed memory for the next call).
static hipError_t f16_pool(hipMemPool_t* out) {
  static std::mutex mu;
  static hipMemPool_t pools[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!pools[dev]) {
    hipMemPoolProps props{};
    props.allocType = hipMemAllocationTypePinned;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t p;
    e = hipMemPoolCreate(&p, &props);
    if (e != hipSuccess) return e;
    uint64_t thr = ~0ull;
    e = hipMemPoolSetAttribute(p, hipMemPoolAttrReleaseThreshold, &thr);
    if (e != hipSuccess) return e;
    pools[dev] = p;
  }
  *out = pools[dev];
  return hipSuccess;
}

// Allocation-free workspace for qmatmul_gemm_noalloc: a file-scope device array (each GPU holds its own copy until
// the process ends). Host code never passes the array's name to a kernel or a copy -- in host code it is only a
// stand-in for the symbol -- but the device address that hipGetSymbolAddress returns for the current device, looked
// up once per device (under a lock) and kept.
constexpr size_t kF16ScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kF16ScratchBytes];

hipError_t f16_scratch(void** out, size_t* bytes) {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  *bytes = kF16ScratchBytes;
  return hipSuccess;
}

hipError_t launch_gemm_f16(int type, const GemmArgs& g, void* ws, hipStream_t s) {
  if (type != T_Q4_K) return hipErrorInvalidValue;
  const int M = g.M, K = g.w.K;
  const int Mp = (int)round_up((size_t)M, kF16BM);
  void* buf = ws;
  hipError_t e = hipSuccess;
  if (!buf) {
    hipMemPool_t pool = nullptr;
    e = f16_pool(&pool);
    if (e == hipSuccess) e = hipMallocFromPoolAsync(&buf, f16_workspace_bytes(M, K), pool, s);
    if (e != hipSuccess) return e;
  }
  uint8_t* af = (uint8_t*)buf;
  uint32_t* u = (uint32_t*)(af + round_up((size_t)Mp * K * 2, 256));
  const size_t threads = (size_t)Mp * (K / 32) * 2;
  // (the block-sum mode reads no activation scales: no mins operand)
  if (g.dbg_isum)
    f16_act_kernel<false><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s>>>(g.aq, nullptr, nullptr, M,
                                                                                       g.M_stride, 0, Mp, K, af, u);
  else
    f16_act_kernel<true><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s>>>(g.aq, g.asc, g.absum, M,
                                                                                      g.M_stride, g.ash, Mp, K, af, u);
  e = hipGetLastError();
  if (e == hipSuccess) {
    F16Args a{};
    a.w = g.w;
    a.af = af;
    a.u = u;
    a.asc = g.asc;
    a.M = M;
    a.M_stride = g.M_stride;
    a.ash = g.ash;
    a.C = g.C;
    a.ldc = g.ldc;
    a.c_off = g.c_off;
    a.accumulate = g.accumulate;
    a.dbg_isum = g.dbg_isum;
    const dim3 grid((unsigned)((g.w.rows + kF16BN - 1) / kF16BN), (unsigned)(Mp / kF16BM));
    if (g.dbg_isum) gemm_f16_kernel<T_Q4_K, true><<<grid, dim3(256), 0, s>>>(a);
    else if (g.ash == 3) gemm_f16_kernel<T_Q4_K, false, true><<<grid, dim3(256), 0, s>>>(a);
    else gemm_f16_kernel<T_Q4_K, false><<<grid, dim3(256), 0, s>>>(a);
    e = hipGetLastError();
  }
  if (!ws) {
    const hipError_t e2 = hipFreeAsync(buf, s);
    if (e == hipSuccess) e = e2;
  }
  return e;
}

}  // namespace qm
