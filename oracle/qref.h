/* CPU oracle for the quantized matrix-product path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU semantics (rizagp/arcinfer, src/quants.h and tools/ref_forward.cpp)
 * and of the integer arithmetic of its GPU kernels (zero/kernels/decode.cl, gemm.cl, moe.cl). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the checker or the timed CPU
 * baseline: the product (arcinfer_amd/) never calls it.
 *
 * Every function names the reference lines it follows. The checks that pin each function (tests/test_oracle_*.py)
 * are listed in the header of tests/test_oracle_formats.py.
 */
#ifndef QREF_H
#define QREF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (src/gguf.h:20-27) */
enum { QREF_Q4_0 = 2, QREF_Q8_0 = 8, QREF_Q4_K = 12, QREF_Q5_K = 13, QREF_Q6_K = 14, QREF_IQ2_XXS = 16,
       QREF_IQ2_XS = 17, QREF_IQ3_XXS = 18, QREF_IQ4_NL = 20, QREF_IQ3_S = 21, QREF_IQ2_S = 22, QREF_IQ4_XS = 23,
       QREF_Q2_K = 10, QREF_Q3_K = 11, QREF_IQ1_S = 19, QREF_IQ1_M = 29, QREF_Q2_0 = 42 };

/* A decoded 256-element superblock: integer quants plus the per-type scales.
 *   Q8_0:   w[e] = d8[e/32] * q[e]
 *   Q4_K:   w[e] = d * sc[e/32] * q[e] - dmin * mn[e/32]
 *   IQ4_XS: w[e] = d * sc[e/32] * q[e]   (sc = ls - 32, q = kvalues_iq4nl[nibble])
 *   IQ3_S:  w[e] = d * sc[e/32] * q[e]   (sc = 1 + 2 * nibble, q = +-grid byte)
 *   Q6_K:   w[e] = d * sc16[e/16] * q[e]  (q = 6-bit value - 32; sc16 signed int8 per 16)
 *   Q5_K:   as Q4_K with q = 0..31
 *   Q4_0:   w[e] = d8[e/32] * q[e]        (q = nibble - 8)
 *   IQ4_NL: w[e] = d8[e/32] * q[e]        (q = kvalues_iq4nl[nibble])
 *   IQ2_XXS, IQ2_XS, IQ2_S: w[e] = d * sc16[e/16] * q[e]  (d = f16 d / 8, sc = 1 + 2 * 4-bit scale per 32 (XXS) or
 *           per 16 (XS, S), q = +-grid byte)
 *   IQ3_XXS: w[e] = d * sc[e/32] * q[e]   (d = f16 d / 4, sc = 1 + 2 * 4-bit scale, q = +-grid byte)
 *   Q3_K:   w[e] = d * sc16[e/16] * q[e]  (sc16 = 6-bit scale - 32 per 16, q = 2-bit value - (hmask bit ? 0 : 4))
 *   Q2_0:   w[e] = d8[e/32] * q[e]        (blocks of 64: one f16 d, q = 2-bit code - 1; d8 of both halves = d)
 *   Q2_K:   w[e] = d * sc16[e/16] * q[e] - dmin * mn16[e/16]   (q = 2-bit value, 4-bit scale and min per 16)
 *   IQ1_S, IQ1_M: w[e] = d * sc16[e/16] * q[e]  (d = f16 d / 8, sc = 2 s + 1 per 32 (S) or per 16 (M), q = 8 * grid
 *           byte + delta, delta = -1 / +1 per 32 (S) or per 8 (M))
 * sc16[i] is the integer scale of elements 16i..16i+15 for every type (sc16[2b] = sc16[2b+1] = sc[b] except Q6_K,
 * Q3_K, Q2_K, IQ2_XS, IQ2_S and IQ1_M, whose scales are per 16); mn16[i] likewise the min of elements 16i..16i+15
 * (= mn[i/2] but for Q2_K, whose mins are per 16). */
typedef struct {
  float d, dmin;
  float d8[8];
  int sc[8];
  int mn[8];
  int16_t q[256];
  int sc16[16];
  int mn16[16];
} qref_sb;

float qref_fp16_to_f32(uint16_t h);
uint16_t qref_f32_to_fp16(float x);
/* elements and bytes of one GGML block (src/gguf.h:43-72); returns 0, or -1 for an unknown type */
int qref_block_info(int type, int* blk, int* bytes);
/* bytes of one 256-element superblock (8 blocks for Q8_0) */
int qref_sb_bytes(int type);
int qref_decode_sb(int type, const uint8_t* p, qref_sb* o);
int qref_dequant_row(int type, const uint8_t* row, int K, float* out);

/* activation quantizer (quantize_act_cpu, src/quants.h:559-576): aq [M_stride][K], asc [K/B][M_stride],
 * absum [K/16][M_stride]; rows M..M_stride-1 are written as zeros (scale 0) */
void qref_quantize_act(const float* x, int M, int K, int M_stride, int act32, int8_t* aq, float* asc, int16_t* absum);

/* int8 block-dot product C[m*ldc + n] = sum over 32-blocks of the reference's per-block expression
 * (decode.cl:695-706): sa * d * (float)(sc * isum) for Q8_0/IQ4_XS/IQ3_S, and
 * sa * (d * (float)(sc * isum) - dmin * (float)(mn * bsum)) for Q4_K, accumulated in double.
 * W: N rows of K elements in GGUF block form. blocksums (nullable) [M][N][K/32]: sc * isum (Q8_0: isum);
 * minsums (nullable, Q4_K) [M][N][K/32]: mn * bsum. nthreads: OpenMP threads (0 = default). */
int qref_blockdot(int type, const uint8_t* W, int N, int K, const int8_t* aq, const float* asc, const int16_t* absum,
                  int M, int M_stride, float* C, int ldc, int32_t* blocksums, int32_t* minsums, int n_col_stride,
                  int nthreads);

/* f32 reference (tools/ref_forward.cpp:137-159): Y[m][n] = sum_k dequant(W)[n][k] * X[m][k] in double */
int qref_matmul_f32(int type, const uint8_t* W, int N, int K, const float* X, int M, float* Y, int nthreads);

/* routing (moe.cl:42-81): top NU of the logits (ties: lower expert), w = exp(l - max) / sum over the selection */
/* Activation producers (zero/kernels/ops.cl:82-128, 2025-2075), act32 layout; h (optional) receives the f32 values
 * that were quantized, [M_stride][K]. */
void qref_rmsnorm_quant(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps, int8_t* aq,
                        float* asc, int16_t* absum, float* h);
void qref_swiglu_quant(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int8_t* aq,
                       float* asc, int16_t* absum, float* h);
void qref_add_norm_quant(float* x, const float* t, const float* w, int K, float eps, float s, const float* w2, int M,
                         int M_stride, int8_t* aq, float* asc, int16_t* absum, float* h);

void qref_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts);
/* the same, each weight then times escale[expert] when escale is non-null (moe.cl:22-28, 75-77: -DESCALE) */
void qref_moe_route_ex(const float* logits, int ldl, int T, int NE, int NU, const float* escale, int* ids, float* wts,
                       int* counts);

/* full MoE FFN on the int8 path (engine_moe.h:8-282, moe.cl:251-340):
 * x[t][E] (+)= sum_k w_k * down_e( quant( silu(gate_e(xq_t)) * up_e(xq_t) ) )
 * gate/up: NE x F rows of E (GGUF), down: NE x E rows of F. aq/asc: x quantized (act32, row stride M_stride).
 * If ids/wts are non-null they are used instead of routing from logits. accumulate: 0 store, 1 add. */
int qref_moe_forward(int type_gate, const uint8_t* Wg, int type_up, const uint8_t* Wu, int type_down,
                     const uint8_t* Wd, int NE, int E, int F, const float* logits, int ldl, int T, int NU,
                     const int8_t* aq, const float* asc, int M_stride, float* x, int accumulate, int nthreads);
/* the same with the expert scales of the routing (escale [NE] or NULL) and a shared expert: sh [T][ldsh] (or NULL)
 * is added as x[t] += sum_k y_k + g_t * sh[t], g_t = sigmoid(logits[t][NE]) if sh_gated (ldl > NE), else 1
 * (moe.cl:332-340, 37-41) */
int qref_moe_forward_ex(int type_gate, const uint8_t* Wg, int type_up, const uint8_t* Wu, int type_down,
                        const uint8_t* Wd, int NE, int E, int F, const float* logits, int ldl, int T, int NU,
                        const int8_t* aq, const float* asc, int M_stride, const float* escale, const float* sh,
                        int ldsh, int sh_gated, float* x, int accumulate, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
