// Mixture-of-experts routing and data movement: route (top-k of the router logits), scan (slot ranges and tiles
// per expert), scatter (device-side token -> slot permutation) and combine (each token's expert outputs summed in
// selection order). The expert matrices themselves run in qm_gemm.hip's tile modes.
#include "qm_launch.h"
#include "qm_route.h"

namespace qm {

// One wave per token (each wave walks tpw tokens): the top NU of the NE logits by repeated arg-max (ties: the lower
// expert), weights exp(l - max) / sum over the selection (summed in selection order; route_token). Per-expert counts go through
// a work-group histogram in LDS and one global atomic per (work-group, expert), not one per (token, k): the router's
// skew (Zipf) would otherwise serialise thousands of atomics on the popular experts' counters.
// zero/kernels/moe.cl:42-81 (moe_route), with 64-lane waves instead of 16-lane sub-groups.
template <int PER_LANE>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int ldl, int T, int NE, int NU,
                                                    int tpw, int* __restrict__ ids, float* __restrict__ wts,
                                                    int* __restrict__ counts, const float* __restrict__ escale) {
  __shared__ int hist[64 * PER_LANE];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (counts)
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
      if (counts) atomicAdd(&hist[my_e], 1);
    }
  }
  if (counts) {
    __syncthreads();
    for (int e = threadIdx.x; e < NE; e += 256)
      if (hist[e]) atomicAdd(&counts[e], hist[e]);
  }
}

hipError_t launch_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts,
                            const float* escale, hipStream_t s) {
  // tokens per wave: enough work-groups to cover the CUs (about 1024 waves), more tokens each for large T
  const int tpw = T >= 2048 ? min(16, T / 1024) : 1;
  const dim3 grid((unsigned)((T + 4 * tpw - 1) / (4 * tpw))), block(256);
  if (NE <= 64) route_kernel<1><<<grid, block, 0, s>>>(logits, ldl, T, NE, NU, tpw, ids, wts, counts, escale);
  else if (NE <= 256) route_kernel<4><<<grid, block, 0, s>>>(logits, ldl, T, NE, NU, tpw, ids, wts, counts, escale);
  else route_kernel<16><<<grid, block, 0, s>>>(logits, ldl, T, NE, NU, tpw, ids, wts, counts, escale);
  return hipGetLastError();
}

// One work-group of NE threads: exclusive scans of the counts (slot offsets) and of the tile counts
// (ceil(count / tile_rows)), then the tile list tiles[0] = #tiles, (expert, first slot, rows) per tile.
// zero/kernels/moe.cl:133-160 (moe_scan).
__global__ __launch_bounds__(1024) void scan_kernel(const int* __restrict__ counts, int* __restrict__ cursor,
                                                    int* __restrict__ tstart, int* __restrict__ tiles, int NE,
                                                    int tile_rows) {
  __shared__ int sa[1024], sb[1024];
  const int e = threadIdx.x;
  const int c = e < NE ? counts[e] : 0, nt = (c + tile_rows - 1) / tile_rows;
  sa[e] = c;
  sb[e] = nt;
  __syncthreads();
  for (int d = 1; d < (int)blockDim.x; d <<= 1) {
    const int x = e >= d ? sa[e - d] : 0, y = e >= d ? sb[e - d] : 0;
    __syncthreads();
    sa[e] += x;
    sb[e] += y;
    __syncthreads();
  }
  if (e >= NE) return;
  const int off = sa[e] - c, toff = sb[e] - nt;
  cursor[e] = off;
  tstart[e] = toff;
  if (e == NE - 1) {
    tiles[0] = sb[e];
    tstart[NE] = sb[e];
  }
  for (int i = 0; i < nt; ++i) {
    int* tp = tiles + 1 + 3 * (toff + i);
    tp[0] = e;
    tp[1] = off + i * tile_rows;
    tp[2] = min(tile_rows, c - i * tile_rows);
  }
}

hipError_t launch_moe_scan(int* counts, int* cursor, int* tstart, int* tiles, int NE, int tile_rows, hipStream_t s) {
  int threads = 64;
  while (threads < NE) threads <<= 1;
  scan_kernel<<<1, threads, 0, s>>>(counts, cursor, tstart, tiles, NE, tile_rows);
  return hipGetLastError();
}

// Every (token, k) pair takes the next slot of its expert: slot order within an expert is arbitrary, so every
// consumer works per slot and the combine reads the slots back through inv in k order. A work-group ranks its 256
// pairs per expert in LDS, reserves each expert's range with one global atomic, then writes the slots.
// zero/kernels/moe.cl:163-171 (moe_scatter).
__global__ __launch_bounds__(256) void scatter_kernel(const int* __restrict__ ids, const float* __restrict__ wts, int n,
                                                      int NU, int NE, int* __restrict__ cursor, int* __restrict__ stok,
                                                      float* __restrict__ swt, int* __restrict__ inv) {
  extern __shared__ int sh[];
  int* cnt = sh;        // [NE] pairs of this work-group per expert
  int* base = sh + NE;  // [NE] first slot reserved for them
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  for (int e = threadIdx.x; e < NE; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  const int e = i < n ? ids[i] : 0;
  const int r = i < n ? atomicAdd(&cnt[e], 1) : 0;
  __syncthreads();
  for (int x = threadIdx.x; x < NE; x += blockDim.x)
    if (cnt[x]) base[x] = atomicAdd(&cursor[x], cnt[x]);
  __syncthreads();
  if (i >= n) return;
  const int slot = base[e] + r;
  stok[slot] = i / NU;
  swt[slot] = wts[i];
  inv[i] = slot;
}

hipError_t launch_moe_scatter(const int* ids, const float* wts, int n, int NU, int NE, int* cursor, int* stok,
                              float* swt, int* inv, hipStream_t s) {
  scatter_kernel<<<(n + 255) / 256, 256, 2 * sizeof(int) * NE, s>>>(ids, wts, n, NU, NE, cursor, stok, swt, inv);
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
