// Host-side launchers of the qmatmul kernels (one per kernel family, defined next to the kernels).
// All return hipSuccess or the launch error; shapes are validated by the C-ABI layer (qm_api.hip) beforehand.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qm_device.h"

namespace qm {

// GGUF rows -> prepared planes (qm_prep.hip)
// K: the prepared row length (a multiple of 256); kraw: 32-blocks per raw row (K / 32, or fewer for a padded
// Q8_0 / Q4_0 / IQ4_NL row)
hipError_t launch_repack(int type, const uint8_t* raw, int rows, int K, int kraw, uint8_t* qs, uint8_t* hdr,
                         hipStream_t s);
// f32 rows -> int8 + per-32 scales + per-16 sums (qm_prep.hip)
hipError_t launch_quantize(const float* x, int ldx, int M, int M_stride, int K, bool act32, int8_t* aq, float* asc,
                           int16_t* absum, hipStream_t s);

struct GemvArgs {
  WView w;
  const int8_t* aq;
  const float* asc;
  const int16_t* absum;
  int M_stride, T;
  float* C;
  int ldc, c_off, accumulate;
  int32_t* dbg_isum;  // non-null: write the block sums instead of C
  int32_t* dbg_msum;
  int split = 0;      // batch-1 sweep: work-groups of the first dispatch round (0: every group takes the same rows)
};
hipError_t launch_gemv(int type, const GemvArgs& a, hipStream_t s);

// Row source of a GEMM's activation tile: dense (row m = token m), gathered (row r = token rowmap[r]) or slots.
struct GemmArgs {
  WView w;       // weight (MoE: gate or down, stacked experts)
  WView w2;      // MoE gate/up: the up projection
  const int8_t* aq;
  const float* asc;
  const int16_t* absum;
  int M, M_stride;
  float* C;
  int ldc, c_off, accumulate;
  int32_t* dbg_isum;
  int ash = 0;  // activation scales per 32 << ash values: asc row of 32-block b is b >> ash (0, or 3 = per 256)
  // MoE tile mode
  const int* tiles;    // [0] = count, then (expert, first slot, rows) per tile
  const int* rowmap;   // slot -> token (gate/up), or null (down: slot rows)
  const float* rowscale;  // slot -> routing weight (down), or null
  int8_t* hq;          // gate/up: quantized h rows [slots][ldc] (ldc = F, the down projection's K)
  float* hsc;          // gate/up: h scales [F/32][slots]
  int slots;           // row stride of hsc
  int max_tiles;
  int expert_rows;     // rows per expert in w (Fv <= F for gate/up, E for down)
};
// MoE tile modes: GATEUP (gate and up of one type in one launch: h quantized), G (gate alone: f32 g into C),
// UH (up alone after G: h from u and g, quantized), DOWN (routing-weighted y)
enum GemmMode : int { GEMM_DENSE = 0, GEMM_MOE_GATEUP = 1, GEMM_MOE_DOWN = 2, GEMM_MOE_G = 3, GEMM_MOE_UH = 4 };
hipError_t launch_gemm(int type, int mode, const GemmArgs& a, hipStream_t s);
// Prompt GEMM on the f16 matrix pipe (qm_gemm_f16.hip): the types and shapes it takes, its per-call workspace, and
// the launcher (ws = null: the workspace comes from a per-device stream-ordered pool). dbg_isum: block-sum mode.
bool f16_gemm_supported(int type, int M, int K);
size_t f16_workspace_bytes(int M, int K);
hipError_t launch_gemm_f16(int type, const GemmArgs& a, void* ws, hipStream_t s);
// The current device's copy of the static scratch array (device address and size) for the allocation-free entry
hipError_t f16_scratch(void** ptr, size_t* bytes);
// slots per MoE tile (one expert each); a 64-row tile (fewer, larger tiles) measured slower under the Zipf skew
constexpr int kMoeTileRows = 32;

// Activation producers (qm_producers.hip)
hipError_t launch_rmsnorm_quant(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps,
                                int8_t* aq, float* asc, int16_t* absum, float* h, int ldh, bool act32, hipStream_t s);
hipError_t launch_swiglu_quant(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int8_t* aq,
                               float* asc, int16_t* absum, bool act32, hipStream_t s);
hipError_t launch_add_norm_quant(float* x, const float* t, const float* w, int K, float eps, float scale,
                                 const float* w2, int M, int M_stride, int8_t* aq, float* asc, int16_t* absum,
                                 bool act32, hipStream_t s);

// The shared expert of an MoE layer: sh [T][ldsh] (null: none), added times g_t = sigmoid(gl[t * ldl]) (gl null:
// g_t = 1). zero/kernels/moe.cl:332-340, 37-41.
struct MoeShared {
  const float* sh;
  int ldsh;
  const float* gl;
  int ldl;
};

// MoE routing (qm_moe.hip); escale [NE] (or null): each chosen expert's weight times its scale
// Tokens per wave of the routing kernel, and its work-groups (four waves each) for T tokens.
// (about 2048 waves, two per SIMD: the selection is latency-bound, T = 4096 measured 20 us for the route + scan +
// scatter chain at 2 tokens per wave, 23 at 4, 22 at 1)
inline int moe_route_tpw(int T) { return T >= 4096 ? (T / 2048 < 16 ? T / 2048 : 16) : 1; }
inline int moe_route_groups(int T) { return (T + 4 * moe_route_tpw(T) - 1) / (4 * moe_route_tpw(T)); }
// counts (or null): per-expert counts by global atomics (counts zeroed first); part (or null): each work-group's
// expert histogram as row blockIdx.x of part [moe_route_groups(T)][NE], plain stores
hipError_t launch_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts,
                            const float* escale, int* part, hipStream_t s);
// From the routing histograms: counts; part's columns become running sums over the routing work-groups
hipError_t launch_moe_scan(int* part, int groups, int* counts, int NE, hipStream_t s);
// The slot permutation (stok, swt, inv) and the scan's outputs: first slots (cursor), tile starts, the tile list
hipError_t launch_moe_scatter(const int* ids, const float* wts, int T, int NU, int NE, const int* part,
                              const int* counts, int* cursor, int* tstart, int* tiles, int tile_rows, int* stok,
                              float* swt, int* inv, hipStream_t s);
hipError_t launch_moe_combine(float* x, const float* y, const int* inv, int T, int NU, int E, int accumulate,
                              const MoeShared& sh, hipStream_t s);
hipError_t launch_fill_i32(int* p, int value, size_t n, hipStream_t s);
// MoE at decode sizes (qm_moe_dec.hip): routing + gate/up -> ids, wts, h (f32 [T*NU][F]), then down + combine into x
// (gate, up, down of types tg, tu, td; escale: routing expert scales or null; sh: the shared expert or sh.sh null)
hipError_t launch_moe_decode(int tg, int tu, int td, const WView& gate, const WView& up, const WView& down, int T,
                             int NU, int E, int F, int Fv, const float* logits, int ldl, int NE, const float* escale,
                             int* ids, float* wts, const int8_t* aq, const float* asc, int M_stride, float* h, float* x,
                             int accumulate, const MoeShared& sh, hipStream_t s);

}  // namespace qm
