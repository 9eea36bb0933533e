// Mixture-of-experts routing and data movement: route (top-k of the router logits), scan (slot ranges and tiles
// per expert), scatter (device-side token -> slot permutation) and combine (each token's expert outputs summed in
// selection order). The expert matrices themselves run in qm_gemm.hip's tile modes.
#include "qm_launch.h"
#include "qm_route.h"

namespace qm {

// One wave per token (each wave walks tpw tokens): the top NU of the NE logits by repeated arg-max (ties: the lower
// expert), weights exp(l - max) / sum over the selection (summed in selection order; route_token). Per-expert counts
// go through a work-group histogram in LDS, then either one global atomic per (work-group, expert) (counts) or a
// plain store of the histogram row (part; the tile path, whose scan sums the rows): the router's skew (Zipf) would
// otherwise serialise thousands of atomics on the popular experts' counters.
// zero/kernels/moe.cl:42-81 (moe_route), with 64-lane waves instead of 16-lane sub-groups.
template <int PER_LANE>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int ldl, int T, int NE, int NU,
                                                   int tpw, int* __restrict__ ids, float* __restrict__ wts,
                                                   int* __restrict__ counts, const float* __restrict__ escale,
                                                   int* __restrict__ part) {
  __shared__ int hist[64 * PER_LANE];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool hst = counts || part;
  if (hst)
    for (int e = threadIdx.x; e < NE; e += 256) hist[e] = 0;
  __syncthreads();
  // the next token's logits are loaded while the current one is selected
  const int t0 = (blockIdx.x * 4 + wave) * tpw;
  float nv[PER_LANE];
  if (t0 < T) route_load<PER_LANE>(logits + (size_t)t0 * ldl, NE, lane, nv);
  for (int j = 0; j < tpw; ++j) {
    const int t = t0 + j;
    if (t >= T) break;
    float v[PER_LANE];
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) v[i] = nv[i];
    if (j + 1 < tpw && t + 1 < T) route_load<PER_LANE>(logits + (size_t)(t + 1) * ldl, NE, lane, nv);
    int my_e;
    float my_w;
    route_select<PER_LANE>(v, NE, NU, lane, my_e, my_w, escale);
    if (lane < NU) {
      ids[(size_t)t * NU + lane] = my_e;
      wts[(size_t)t * NU + lane] = my_w;
      if (hst) atomicAdd(&hist[my_e], 1);
    }
  }
  if (!hst) return;
  __syncthreads();
  if (part) {
    for (int e = threadIdx.x; e < NE; e += 256) part[(size_t)blockIdx.x * NE + e] = hist[e];
  } else {
    for (int e = threadIdx.x; e < NE; e += 256)
      if (hist[e]) atomicAdd(&counts[e], hist[e]);
  }
}

hipError_t launch_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts,
                            const float* escale, int* part, hipStream_t s) {
  // tokens per wave: moe_route_tpw (about 2048 waves; more tokens each for large T)
  const int tpw = moe_route_tpw(T);
  const dim3 grid((unsigned)moe_route_groups(T)), block(256);
  if (NE <= 64) route_kernel<1><<<grid, block, 0, s>>>(logits, ldl, T, NE, NU, tpw, ids, wts, counts, escale, part);
  else if (NE <= 256) route_kernel<4><<<grid, block, 0, s>>>(logits, ldl, T, NE, NU, tpw, ids, wts, counts, escale, part);
  else route_kernel<16><<<grid, block, 0, s>>>(logits, ldl, T, NE, NU, tpw, ids, wts, counts, escale, part);
  return hipGetLastError();
}

// Work-group e (256 threads) sums expert e's column of the routing histograms part [G][NE] and rewrites it as
// running sums (row g: how many of expert e's slots routing work-groups 0 .. g-1 took), then writes counts[e].
__global__ __launch_bounds__(256) void scan_cols_kernel(int* __restrict__ part, int G, int* __restrict__ counts,
                                                        int NE) {
  __shared__ int red[256];
  const int tid = threadIdx.x, e = blockIdx.x;
  // this thread's rows [r0, r1): loaded at once (unconditional loads of clamped rows, zeroed past the range)
  constexpr int RB = 8;
  const int r0 = (int)((long long)tid * G / 256), r1 = (int)((long long)(tid + 1) * G / 256), nr = r1 - r0;
  int v[RB], sum = 0;
  const int rl = max(r1 - 1, 0);
#pragma unroll
  for (int k = 0; k < RB; ++k) v[k] = part[(size_t)min(r0 + k, rl) * NE + e];
#pragma unroll
  for (int k = 0; k < RB; ++k) {
    v[k] = k < nr ? v[k] : 0;
    sum += v[k];
  }
  for (int r = r0 + RB; r < r1; ++r) sum += part[(size_t)r * NE + e];  // (G > 2048 only)
  red[tid] = sum;
  __syncthreads();
  for (int d = 1; d < 256; d <<= 1) {
    const int x = tid >= d ? red[tid - d] : 0;
    __syncthreads();
    red[tid] += x;
    __syncthreads();
  }
  int base = red[tid] - sum;  // the expert's slots taken by the rows before r0
#pragma unroll
  for (int k = 0; k < RB; ++k)
    if (k < nr) {
      part[(size_t)(r0 + k) * NE + e] = base;
      base += v[k];
    }
  for (int r = r0 + RB; r < r1; ++r) {
    int* q = part + (size_t)r * NE + e;
    const int x = *q;
    *q = base;
    base += x;
  }
  if (tid == 255) counts[e] = red[255];
}

hipError_t launch_moe_scan(int* part, int groups, int* counts, int NE, hipStream_t s) {
  if (NE > 1024) return hipErrorInvalidValue;
  scan_cols_kernel<<<NE, 256, 0, s>>>(part, groups, counts, NE);
  return hipGetLastError();
}

// Every (token, k) pair takes the next slot of its expert: slot order within an expert is arbitrary, so every
// consumer works per slot and the combine reads the slots back through inv in k order. Each work-group first scans
// the counts in LDS (exclusive scans of the counts: first slots; of the tile counts ceil(count / tile_rows), rounded
// up to even so every expert's tiles start at an even index and pair up: tile starts); work-group 0 writes those
// (cursor, tstart) and every work-group a share of the tile list tiles[0] = #entries, (expert, first slot, rows) per
// entry (an odd count's extra entry: 0 rows, at the expert's last slot), entry i found by a binary search
// (zero/kernels/moe.cl:133-160, moe_scan). Then work-group g takes the pairs of routing work-group g's tokens, ranks
// them per expert in LDS and adds the ranks to the expert's first slot and the slots the routing work-groups before g
// took (row g of part, as scan_cols_kernel left it): no global atomics. zero/kernels/moe.cl:163-171 (moe_scatter).
__global__ __launch_bounds__(256) void scatter_kernel(const int* __restrict__ ids, const float* __restrict__ wts,
                                                      int n, int per_group, int NU, int NE,
                                                      const int* __restrict__ part, const int* __restrict__ counts,
                                                      int* __restrict__ cursor, int* __restrict__ tstart,
                                                      int* __restrict__ tiles, int tile_rows, int* __restrict__ stok,
                                                      float* __restrict__ swt, int* __restrict__ inv) {
  __shared__ int ra[256], rb[256], sa[1024], sb[1024], cnt[1024];
  const int tid = threadIdx.x;
  for (int e = tid; e < NE; e += 256) cnt[e] = 0;
  const int per = (NE + 255) / 256;  // experts per thread, consecutive (NE <= 1024)
  int c4[4], n4[4], cs = 0, ns = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int x = tid * per + k;
    c4[k] = k < per && x < NE ? counts[x] : 0;
    n4[k] = (c4[k] + tile_rows - 1) / tile_rows;
    n4[k] += n4[k] & 1;  // (an even number of tile entries per expert: the gate/up kernel takes tiles in pairs)
    cs += c4[k];
    ns += n4[k];
  }
  ra[tid] = cs;
  rb[tid] = ns;
  __syncthreads();
  for (int d = 1; d < 256; d <<= 1) {
    const int x = tid >= d ? ra[tid - d] : 0, y = tid >= d ? rb[tid - d] : 0;
    __syncthreads();
    ra[tid] += x;
    rb[tid] += y;
    __syncthreads();
  }
  int co = ra[tid] - cs, no = rb[tid] - ns;  // exclusive prefixes at this thread's first expert
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int x = tid * per + k;
    if (k < per && x < NE) {
      if (blockIdx.x == 0) {
        cursor[x] = co;
        tstart[x] = no;
      }
      co += c4[k];
      no += n4[k];
      sa[x] = co;  // inclusive prefixes over experts
      sb[x] = no;
    }
  }
  __syncthreads();
  const int ntot = sb[NE - 1];
  if (blockIdx.x == 0 && tid == 0) {
    tiles[0] = ntot;
    tstart[NE] = ntot;
  }
  // this work-group's share of the tile list: tile i belongs to the first expert whose inclusive tile prefix exceeds i
  for (int i = blockIdx.x * 256 + tid; i < ntot; i += gridDim.x * 256) {
    int lo = 0, hi = NE;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sb[mid] > i) hi = mid;
      else lo = mid + 1;
    }
    const int x = lo, first = x == 0 ? 0 : sa[x - 1], cx = sa[x] - first, k = i - (x == 0 ? 0 : sb[x - 1]);
    int* tp = tiles + 1 + 3 * i;
    const bool pad = k * tile_rows >= cx;  // (the empty entry that evens an odd tile count: at the last slot)
    tp[0] = x;
    tp[1] = pad ? first + cx - 1 : first + k * tile_rows;
    tp[2] = pad ? 0 : min(tile_rows, cx - k * tile_rows);
  }
  // the slots
  const int i0 = blockIdx.x * per_group, i1 = min(n, i0 + per_group);
  const int* base = part + (size_t)blockIdx.x * NE;
  for (int i = i0 + tid; i < i1; i += 256) {
    const int e = ids[i];
    const int slot = (e == 0 ? 0 : sa[e - 1]) + base[e] + atomicAdd(&cnt[e], 1);
    stok[slot] = i / NU;
    swt[slot] = wts[i];
    inv[i] = slot;
  }
}

hipError_t launch_moe_scatter(const int* ids, const float* wts, int T, int NU, int NE, const int* part,
                              const int* counts, int* cursor, int* tstart, int* tiles, int tile_rows, int* stok,
                              float* swt, int* inv, hipStream_t s) {
  if (NE > 1024) return hipErrorInvalidValue;
  const int per_group = 4 * moe_route_tpw(T) * NU;
  scatter_kernel<<<moe_route_groups(T), 256, 0, s>>>(ids, wts, T * NU, per_group, NU, NE, part, counts, cursor, tstart,
                                                     tiles, tile_rows, stok, swt, inv);
  return hipGetLastError();
}

// x[t][c] (+)= sum_k y[inv[t*NU + k]][c] (k in selection order) + g_t * sh[t][c] (zero/kernels/moe.cl:332-340):
// the shared expert's output sh, when given, with its gate g_t = sigmoid(gl[t * ldl]) (gl = the logits' column NE) or
// 1 without a gate logit. 4 columns per thread.
__global__ __launch_bounds__(256) void combine_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                      const int* __restrict__ inv, int T, int NU, int E,
                                                      int accumulate, MoeShared sh) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int cq = E / 4;
  if (i >= (long)T * cq) return;
  const int t = (int)(i / cq), c = (int)(i % cq) * 4;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k = 0; k < NU; ++k) {
    const float4 u = *(const float4*)(y + (size_t)inv[(size_t)t * NU + k] * E + c);
    v.x += u.x;
    v.y += u.y;
    v.z += u.z;
    v.w += u.w;
  }
  if (sh.sh) {
    const float g = sh.gl ? 1.0f / (1.0f + expf(-sh.gl[(size_t)t * sh.ldl])) : 1.0f;
    const float4 o = *(const float4*)(sh.sh + (size_t)t * sh.ldsh + c);
    v.x = v.x + g * o.x;
    v.y = v.y + g * o.y;
    v.z = v.z + g * o.z;
    v.w = v.w + g * o.w;
  }
  float4* xp = (float4*)(x + (size_t)t * E + c);
  if (accumulate) {
    const float4 o = *xp;
    v.x = o.x + v.x;
    v.y = o.y + v.y;
    v.z = o.z + v.z;
    v.w = o.w + v.w;
  }
  *xp = v;
}

hipError_t launch_moe_combine(float* x, const float* y, const int* inv, int T, int NU, int E, int accumulate,
                              const MoeShared& sh, hipStream_t s) {
  const long n = (long)T * (E / 4);
  combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, y, inv, T, NU, E, accumulate, sh);
  return hipGetLastError();
}

// A fill kernel (not hipMemsetAsync, so the calls stay capturable in HIP graphs).
__global__ void fill_i32_kernel(int* p, int value, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = value;
}

hipError_t launch_fill_i32(int* p, int value, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  fill_i32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, value, n);
  return hipGetLastError();
}

}  // namespace qm
