// Top-k routing of one token by one 64-lane wave: softmax over the selected experts of a row of router logits.
// Selection takes the largest logit NU times (ties to the lower expert; -inf logits in expert order), the weights
// are exp(l - max) / sum over the selection (summed in selection order). zero/kernels/moe.cl:42-81 (moe_route), with
// 64-lane waves instead of 16-lane sub-groups: the wave maximum on DPP / v_readlane, the arg-max by ballot. Used by
// route_kernel (qm_moe.hip) and, at decode sizes, inside the expert gate/up kernel.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include "qm_device.h"

namespace qm {

// v[i] = logit i * 64 + lane of the token's NE logits lg (-inf past NE)
template <int PER_LANE>
__device__ __forceinline__ void route_load(const float* __restrict__ lg, int NE, int lane, float (&v)[PER_LANE]) {
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int e = i * 64 + lane;
    v[i] = e < NE ? lg[e] : -INFINITY;
  }
}

// the selection from the loaded logits (route_load); lane < NU receives the k = lane-th selected expert and its weight
// (times escale[expert] when escale is non-null: moe.cl:22-28, 75-77, -DESCALE)
template <int PER_LANE>
__device__ __forceinline__ void route_select(float (&v)[PER_LANE], int NE, int NU, int lane, int& my_e, float& my_w,
                                             const float* __restrict__ escale = nullptr) {
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) mx = fmaxf(mx, v[i]);
  mx = wave_max(mx);
  float sum = 0.0f, my_p = 0.0f;
  unsigned taken = 0;  // bit i: expert i * 64 + lane selected
  my_e = 0;
  for (int k = 0; k < NU; ++k) {
    float bv = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) bv = fmaxf(bv, v[i]);
    const float gv = wave_max(bv);
    // the lowest expert index holding the maximum: the first slice i (experts 64 i .. 64 i + 63) with a match, its
    // lowest lane. With no finite logit left, the lowest expert not yet selected (a stable sort's order, as the
    // reference's route test; its OpenCL kernel would yield the out-of-range index NE there). NU <= NE.
    int gi = NE;
#pragma unroll
    for (int i = PER_LANE - 1; i >= 0; --i) {
      const bool cand = gv > -INFINITY ? v[i] == gv : !((taken >> i) & 1u) && i * 64 + lane < NE;
      const unsigned long long m = __ballot(cand);
      if (m) gi = i * 64 + __builtin_ctzll(m);
    }
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i)
      if (i * 64 + lane == gi) {
        v[i] = -INFINITY;
        taken |= 1u << i;
      }
    const float p = gv > -INFINITY ? expf(gv - mx) : 0.0f;  // (a row of only -inf logits: every weight 0)
    sum += p;
    if (lane == k) {
      my_p = p;
      my_e = gi;
    }
  }
  my_w = sum > 0.0f ? my_p / sum : 0.0f;
  if (escale && lane < NU) my_w *= escale[my_e];
}

// lg: the token's NE logits; lane < NU receives the k = lane-th selected expert and its weight
template <int PER_LANE>
__device__ __forceinline__ void route_token(const float* __restrict__ lg, int NE, int NU, int lane, int& my_e,
                                            float& my_w, const float* __restrict__ escale = nullptr) {
  float v[PER_LANE];
  route_load<PER_LANE>(lg, NE, lane, v);
  route_select<PER_LANE>(v, NE, NU, lane, my_e, my_w, escale);
}

}  // namespace qm
