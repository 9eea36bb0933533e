// Activation producers: the kernels that write the path's int8 activations from f32 rows -- RMS norm, SwiGLU /
// GELU gating and the residual add + norm -- fused with the per-32 quantizer (zero/kernels/ops.cl:82-128,
// 2025-2075). One work-group of 256 threads per row. The quantization step is the same arithmetic as
// quantize_kernel: 8 lanes per 32-block, 4 values per lane, amax over the 8 lanes, q = rint(v * (127 / amax)).
#include "qm_launch.h"

namespace qm {

namespace {

// Quantizes one 32-block held by 8 consecutive lanes (lane `sub` holds elements 4*sub .. 4*sub+3). Every lane of the
// wave calls it (the shuffles); `store` masks the writes. a32 = 0: one scale per 256 values (asc [K/256][M_stride]);
// every caller gives wave w the blocks 8w .. 8w+7 of a 32-block-aligned pass, i.e. one whole superblock, so its amax
// is the wave maximum.
__device__ __forceinline__ void quant8(const float v[4], int sub, bool store, int m, int b, int M_stride, int K,
                                       int8_t* __restrict__ aq, float* __restrict__ asc,
                                       int16_t* __restrict__ absum, int a32) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = a32 ? max8(amax) : wave_max(amax);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int sum = 0;
  uint32_t pk = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = (int)__builtin_rintf(v[i] * inv);
    sum += q;
    pk |= (uint32_t)(q & 0xFF) << (8 * i);
  }
  sum = sum4_i(sum);
  if (!store) return;
  *(uint32_t*)(aq + (size_t)m * K + 32 * b + 4 * sub) = pk;
  if (sub == 0 && (a32 || (b & 7) == 0)) asc[(size_t)(a32 ? b : b >> 3) * M_stride + m] = amax / 127.0f;
  if ((sub & 3) == 0) absum[(size_t)(2 * b + (sub >> 2)) * M_stride + m] = (int16_t)sum;
}

// Sum over the work-group's 256 threads, in a fixed order (wave sums, then the 4 wave sums in order).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum_width(v, 64);
  __syncthreads();  // (red may still be read from a previous call)
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

__device__ __forceinline__ float sumsq_row(const float* __restrict__ r, int K, float* red) {
  float ss = 0.0f;
  for (int i = 4 * threadIdx.x; i < K; i += 1024) {
    const float4 v = *(const float4*)(r + i);
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  return block_sum(ss, red);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float gelu_tanh(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

}  // namespace

// y = x * r * w, r = 1 / sqrt(mean(x^2) + eps) (ops.cl:82-104); rows M..M_stride-1 zero. h: optional f32 copy.
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const float* __restrict__ x, int ldx,
                                                            const float* __restrict__ w, int K, int M, int M_stride,
                                                            float eps, int8_t* __restrict__ aq,
                                                            float* __restrict__ asc, int16_t* __restrict__ absum,
                                                            float* __restrict__ h, int ldh, int a32) {
  __shared__ float red[4];
  const int m = blockIdx.x, nb = K / 32, sub = threadIdx.x & 7;
  const bool valid = m < M;
  const float* xr = x + (size_t)m * ldx;
  const float r = valid ? 1.0f / sqrtf(sumsq_row(xr, K, red) / (float)K + eps) : 0.0f;
  for (int b0 = 0; b0 < nb; b0 += 32) {
    const int b = b0 + (threadIdx.x >> 3);
    const bool live = b < nb;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && valid) {
      const float4 xv = *(const float4*)(xr + 32 * b + 4 * sub), wv = *(const float4*)(w + 32 * b + 4 * sub);
      v[0] = xv.x * r * wv.x;
      v[1] = xv.y * r * wv.y;
      v[2] = xv.z * r * wv.z;
      v[3] = xv.w * r * wv.w;
    }
    if (h && live) *(float4*)(h + (size_t)m * ldh + 32 * b + 4 * sub) = make_float4(v[0], v[1], v[2], v[3]);
    quant8(v, sub, live, m, b, M_stride, K, aq, asc, absum, a32);
  }
}

// y = act(gate) * up from rows [gate(F) | up(F)] (act = silu, or gelu_tanh), or the row itself with `fused`
// (ops.cl:110-128).
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float* __restrict__ gu, int ldg, int F, int M,
                                                           int M_stride, int fused, int gelu,
                                                           int8_t* __restrict__ aq, float* __restrict__ asc,
                                                           int16_t* __restrict__ absum, int a32) {
  const int m = blockIdx.x, nb = F / 32, sub = threadIdx.x & 7;
  const bool valid = m < M;
  const float* g = gu + (size_t)m * ldg;
  // (grid.y splits the row: no step crosses a 32-block, so chunks of 32 blocks are independent)
  for (int b0 = 32 * blockIdx.y; b0 < nb; b0 += 32 * gridDim.y) {
    const int b = b0 + (threadIdx.x >> 3);
    const bool live = b < nb;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && valid) {
      const float4 gv = *(const float4*)(g + 32 * b + 4 * sub);
      const float ga[4] = {gv.x, gv.y, gv.z, gv.w};
      if (fused) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = ga[i];
      } else {
        const float4 uv = *(const float4*)(g + F + 32 * b + 4 * sub);
        const float ua[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (gelu ? gelu_tanh(ga[i]) : silu(ga[i])) * ua[i];
      }
    }
    quant8(v, sub, live, m, b, M_stride, F, aq, asc, absum, a32);
  }
}

// rmsnorm_quant_kernel for K <= 16384 with the row held in registers: work-group (m, c) reads the whole row x once
// (every load issued up front) for the mean square, then scales and quantizes its passes c, c + gridDim.y, ... of 32
// blocks (1024 values) each. With few rows the launch splits each row over work-groups (gridDim.y > 1: every one
// re-reads the row, cheap at decode sizes); with many rows one work-group takes the whole row. Thread t holds elements 1024 p + 4 t .. + 3 of pass p, the elements and order of sumsq_row's loop,
// so every work-group of a row computes the same, bit-identical r as rmsnorm_quant_kernel.
template <int PASSES>
__global__ __launch_bounds__(256) void rmsnorm_quant_reg_kernel(const float* __restrict__ x, int ldx,
                                                                const float* __restrict__ w, int K, int M,
                                                                int M_stride, float eps, int8_t* __restrict__ aq,
                                                                float* __restrict__ asc, int16_t* __restrict__ absum,
                                                                float* __restrict__ h, int ldh, int a32) {
  __shared__ float red[4];
  const int m = blockIdx.x, c = blockIdx.y, nb = K / 32, sub = threadIdx.x & 7;
  const bool valid = m < M;
  const float* xr = x + (size_t)m * ldx;
  float4 xv[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int b = 32 * p + (threadIdx.x >> 3);
    xv[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (b < nb && valid) xv[p] = *(const float4*)(xr + 32 * b + 4 * sub);
  }
  float ss = 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    ss = fmaf(xv[p].x, xv[p].x, ss);
    ss = fmaf(xv[p].y, xv[p].y, ss);
    ss = fmaf(xv[p].z, xv[p].z, ss);
    ss = fmaf(xv[p].w, xv[p].w, ss);
  }
  ss = block_sum(ss, red);
  const float r = valid ? 1.0f / sqrtf(ss / (float)K + eps) : 0.0f;
  // this work-group's passes: c, c + gridDim.y, ... (all of them when the grid does not split rows)
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    if (p % gridDim.y != (unsigned)c) continue;
    const int b = 32 * p + (threadIdx.x >> 3);
    const bool live = b < nb;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && valid) {
      const float4 wv = *(const float4*)(w + 32 * b + 4 * sub);
      v[0] = xv[p].x * r * wv.x;
      v[1] = xv[p].y * r * wv.y;
      v[2] = xv[p].z * r * wv.z;
      v[3] = xv[p].w * r * wv.w;
    }
    if (h && live) *(float4*)(h + (size_t)m * ldh + 32 * b + 4 * sub) = make_float4(v[0], v[1], v[2], v[3]);
    quant8(v, sub, live, m, b, M_stride, K, aq, asc, absum, a32);
  }
}

// x = (x + t * r * w) * s (r from t's mean square), stored back; y = x * r2 * w2 (r2 from the new x) or, without
// w2, y = x; y quantized (ops.cl:2025-2075). The new x stays in registers between the two steps (PASSES = K / 1024
// rounded up, at most 16: K <= 16384).
template <int PASSES>
__global__ __launch_bounds__(256) void add_norm_quant_kernel(float* __restrict__ x, const float* __restrict__ t,
                                                             const float* __restrict__ w, int K, float eps, float s,
                                                             const float* __restrict__ w2, int M, int M_stride,
                                                             int8_t* __restrict__ aq, float* __restrict__ asc,
                                                             int16_t* __restrict__ absum, int a32) {
  __shared__ float red[4];
  const int m = blockIdx.x, nb = K / 32, sub = threadIdx.x & 7;
  const bool valid = m < M;
  float* xr = x + (size_t)m * K;
  const float* tr = t + (size_t)m * K;
  // every load of x, t and w issued up front; thread t holds elements 1024 p + 4 t .. + 3, the order of sumsq_row's
  // loop, so the mean square of t is bit-identical to a separate pass over t
  float4 x4s[PASSES], t4s[PASSES], w4s[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int b = 32 * p + (threadIdx.x >> 3);
    x4s[p] = t4s[p] = w4s[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (b < nb && valid) {
      const int o = 32 * b + 4 * sub;
      x4s[p] = *(const float4*)(xr + o);
      t4s[p] = *(const float4*)(tr + o);
      w4s[p] = *(const float4*)(w + o);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    ss = fmaf(t4s[p].x, t4s[p].x, ss);
    ss = fmaf(t4s[p].y, t4s[p].y, ss);
    ss = fmaf(t4s[p].z, t4s[p].z, ss);
    ss = fmaf(t4s[p].w, t4s[p].w, ss);
  }
  ss = block_sum(ss, red);
  const float r = valid ? 1.0f / sqrtf(ss / (float)K + eps) : 0.0f;
  float xv[PASSES][4];
  float s2 = 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int b = 32 * p + (threadIdx.x >> 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[p][i] = 0.0f;
    if (b < nb && valid) {
      const int o = 32 * b + 4 * sub;
      const float4 x4 = x4s[p], t4 = t4s[p], w4 = w4s[p];
      xv[p][0] = (x4.x + t4.x * r * w4.x) * s;
      xv[p][1] = (x4.y + t4.y * r * w4.y) * s;
      xv[p][2] = (x4.z + t4.z * r * w4.z) * s;
      xv[p][3] = (x4.w + t4.w * r * w4.w) * s;
      *(float4*)(xr + o) = make_float4(xv[p][0], xv[p][1], xv[p][2], xv[p][3]);
#pragma unroll
      for (int i = 0; i < 4; ++i) s2 = fmaf(xv[p][i], xv[p][i], s2);
    }
  }
  const float tot = block_sum(s2, red);
  const float r2 = w2 && valid ? 1.0f / sqrtf(tot / (float)K + eps) : 1.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int b = 32 * p + (threadIdx.x >> 3);
    const bool live = b < nb;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = xv[p][i];
    if (w2 && live && valid) {
      const float4 w4 = *(const float4*)(w2 + 32 * b + 4 * sub);
      v[0] = xv[p][0] * r2 * w4.x;
      v[1] = xv[p][1] * r2 * w4.y;
      v[2] = xv[p][2] * r2 * w4.z;
      v[3] = xv[p][3] * r2 * w4.w;
    }
    quant8(v, sub, live, m, b, M_stride, K, aq, asc, absum, a32);
  }
}

hipError_t launch_rmsnorm_quant(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps,
                                int8_t* aq, float* asc, int16_t* absum, float* h, int ldh, bool act32, hipStream_t s) {
  const int a32 = act32 ? 1 : 0;
  const int passes = (K / 32 + 31) / 32;
  const unsigned split = M_stride < 256 ? (unsigned)passes : 1u;  // (few rows: the GPU would be nearly idle)
#define QM_RNQ(P) rmsnorm_quant_reg_kernel<P><<<dim3(M_stride, split), 256, 0, s>>>(x, ldx, w, K, M, M_stride, eps, aq, asc, absum, h, ldh, a32)
  if (passes <= 1) QM_RNQ(1);
  else if (passes <= 2) QM_RNQ(2);
  else if (passes <= 4) QM_RNQ(4);
  else if (passes <= 8) QM_RNQ(8);
  else if (passes <= 16) QM_RNQ(16);
  else rmsnorm_quant_kernel<<<M_stride, 256, 0, s>>>(x, ldx, w, K, M, M_stride, eps, aq, asc, absum, h, ldh, a32);
#undef QM_RNQ
  return hipGetLastError();
}

hipError_t launch_swiglu_quant(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int8_t* aq,
                               float* asc, int16_t* absum, bool act32, hipStream_t s) {
  const int a32 = act32 ? 1 : 0;
  // one work-group per row and chunk of 32 blocks (1024 values): a decode row of F = 17408 spreads over 17
  const unsigned chunks = (unsigned)((F / 32 + 31) / 32);
  swiglu_quant_kernel<<<dim3(M_stride, chunks), 256, 0, s>>>(gu, ldg, F, M, M_stride, fused, gelu, aq, asc, absum, a32);
  return hipGetLastError();
}

hipError_t launch_add_norm_quant(float* x, const float* t, const float* w, int K, float eps, float scale,
                                 const float* w2, int M, int M_stride, int8_t* aq, float* asc, int16_t* absum,
                                 bool act32, hipStream_t s) {
  const int a32 = act32 ? 1 : 0;
  const int passes = (K / 32 + 31) / 32;
#define QM_ANQ(P) add_norm_quant_kernel<P><<<M_stride, 256, 0, s>>>(x, t, w, K, eps, scale, w2, M, M_stride, aq, asc, absum, a32)
  if (passes <= 1) QM_ANQ(1);
  else if (passes <= 2) QM_ANQ(2);
  else if (passes <= 4) QM_ANQ(4);
  else if (passes <= 8) QM_ANQ(8);
  else if (passes <= 16) QM_ANQ(16);
  else return hipErrorInvalidValue;
#undef QM_ANQ
  return hipGetLastError();
}

}  // namespace qm
