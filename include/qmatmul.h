/* qmatmul -- MI355X (gfx950) quantized matrix products for GGUF weights: the C ABI.
 *
 * The drop-in boundary for arcinferzero's quantized matmul path (rizagp/arcinfer). Plain C: device pointers,
 * sizes and status codes; no C++ or HIP types. `stream` is a hipStream_t passed as void* (NULL = the null stream).
 * Every call is stream-ordered and asynchronous (no host synchronisation inside), except qmatmul_prepare_weight with
 * a host source, which copies synchronously. Calls never throw or exit: they return a qm_status and leave a message
 * for qmatmul_last_error() (thread-local).
 *
 * Activation layout (the reference's quant_store16 layout, zero/kernels/ops.cl:18-77, act32):
 *   aq    int8  [M_stride][K]   row-major, one row per token
 *   asc   float [K/32][M_stride] scale of each 32-block, token fastest
 *   absum int16 [K/16][M_stride] sum of each 16-block's int8 values, token fastest (needed by Q4_K only)
 * Rows M..M_stride-1 of a padded batch are zero rows.
 * The per-256 layout (act32 = 0 in the reference: Engine::matmul's act32 flag, zero/engine.h:3151, 3300, and
 * quantize_act_cpu with B = 256, src/quants.h:559-576) has asc float [K/256][M_stride], one scale per 256 values;
 * it is written by the *_ex producers and the quantizer with act32 = 0 and read by qmatmul_gemm_ex with act32 = 0
 * (the reference uses it only for prompt GEMMs: every GEMV and MoE input is per-32, zero/engine.h:3300).
 *
 * Weights: GGUF blocks, rows of K elements, K a multiple of 256 (Q8_0: 8 blocks of 32 per 256). A weight is
 * prepared once (qmatmul_prepare_weight) into this library's own device layout and then read by every product.
 * Rows of the 32-element block types (Q8_0, Q4_0, IQ4_NL) may have any K % 32 == 0, rows of Q2_0 (the reference's
 * own 64-element blocks, src/gguf.h:26) any K % 64 == 0: they are padded at preparation
 * with zero blocks to the next multiple of 256, which is then the weight's K (qmatmul_weight_info); the activations
 * of such a weight are K values long, the padding zeros.
 *
 * Output buffers (C, x) must be ordinary device memory (hipMalloc, a torch tensor): when a prompt GEMM has few output
 * tiles, its two K halves are added into C with hardware float atomics, which fine-grained or host-coherent memory
 * does not guarantee.
 *
 * accumulate (all products): 0 = store, 1 = C += result, 2 = C = silu(C) * result (GEMM only, fused SwiGLU:
 * C holds the gate projection), as zero/kernels/gemm.cl:464-471.
 */
#ifndef QMATMUL_H
#define QMATMUL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (src/gguf.h:20-27) of the weight types this path decodes */
typedef enum {
  QM_Q4_0 = 2, QM_Q8_0 = 8, QM_Q4_K = 12, QM_Q5_K = 13, QM_Q6_K = 14, QM_IQ2_XXS = 16, QM_IQ2_XS = 17,
  QM_IQ3_XXS = 18, QM_IQ4_NL = 20, QM_IQ3_S = 21, QM_IQ2_S = 22, QM_IQ4_XS = 23, QM_Q2_K = 10, QM_Q3_K = 11,
  QM_IQ1_S = 19, QM_IQ1_M = 29, QM_Q2_0 = 42
} qm_type;

typedef enum {
  QM_OK = 0,
  QM_ERR_ARG = 1,       /* null pointer or invalid argument */
  QM_ERR_SHAPE = 2,     /* a shape the kernels do not cover (the reference throws runtime_error here,
                           zero/engine.h:3255-3257) */
  QM_ERR_TYPE = 3,      /* weight type not supported by this entry point */
  QM_ERR_HIP = 4,       /* a HIP runtime call failed (message holds hipGetErrorString) */
  QM_ERR_NOMEM = 5,     /* device allocation failed */
  QM_ERR_WORKSPACE = 6  /* workspace too small */
} qm_status;

typedef struct qm_weight qm_weight; /* opaque: a prepared (device-resident) weight matrix */

/* Per-device one-time set-up (codebooks to the device). Optional: every entry point calls it on first use.
 * Replaces the table upload of Engine::build_kernels (zero/engine.h:1921-1922, src/quants.h:622-634). */
int qmatmul_init(void);

/* Message of the last failed call on this thread ("" if none). */
const char* qmatmul_last_error(void);

/* Bytes of one 256-element superblock in GGUF (0 for an unsupported type); src/gguf.h:43-72. */
size_t qmatmul_sb_bytes(int type);

/* Device bytes a prepared weight of `rows` x K takes (the GGUF bytes, plus 2 bytes of padding per IQ3_S, Q6_K,
 * IQ2_XXS, IQ2_XS, IQ2_S or IQ3_XXS superblock, 6 per Q3_K, 18 per IQ1_S and 12 per IQ1_M superblock; a padded
 * Q8_0 / Q4_0 / IQ4_NL / Q2_0
 * row counts its zero blocks). */
size_t qmatmul_weight_bytes(int type, int rows, int K);

/* Prepares a weight from its GGUF bytes: rows x (K/256) superblocks, row-major, as stored in a GGUF tensor (a
 * stacked expert tensor [NE][N][K] is NE*N rows). raw is a device pointer if raw_on_device, else a host pointer.
 * Allocates the prepared copy and returns it in *out. Replaces Engine::make_weight / upload_padded
 * (zero/engine.h:1936-2014; src/quants.h:643-681). Q8_0, Q4_0 and IQ4_NL rows may be K % 32 == 0 long (rows of
 * K/32 GGUF blocks), Q2_0 rows K % 64 == 0 long: they are padded with zero blocks to K rounded up to 256, as the
 * reference's load_w_pad /
 * pad_small_block_rows (zero/engine.h:2102-2116; src/quants.h:581-595); every other type needs K % 256 == 0. */
int qmatmul_prepare_weight(int type, const void* raw, int raw_on_device, int rows, int K, void* stream,
                           qm_weight** out);

/* Frees a prepared weight (waits for the device). */
int qmatmul_release_weight(qm_weight* w);

/* Type, rows and K of a prepared weight (any output pointer may be NULL); K is the prepared (padded) row length. */
int qmatmul_weight_info(const qm_weight* w, int* type, int* rows, int* K);

/* Activation quantizer: x f32 [M][ldx] -> aq, asc, absum (layout above; rows M..M_stride-1 zeroed).
 * Per 32 values: amax = max |v|; asc = amax / 127; q = round-half-even(v * (127 / amax)), 0 if amax == 0;
 * absum = sum of q per 16. Bit-exact with quantize_act_cpu(act32 = true), src/quants.h:559-576, which is the CPU
 * twin of quant_store16 (zero/kernels/ops.cl:18-77) as rmsnorm_quant / swiglu_quant(fused=1) use it
 * (zero/engine.h:3302-3308, 3451-3456). K % 32 == 0. */
int qmatmul_quantize_act(const float* x, int ldx, int M, int M_stride, int K, int8_t* aq, float* asc, int16_t* absum,
                         void* stream);
/* The same with the reference's act32 flag: act32 = 1 is qmatmul_quantize_act; act32 = 0 takes amax over each 256
 * values and writes asc [K/256][M_stride] (K % 256 == 0), bit-exact with quantize_act_cpu(act32 = false). */
int qmatmul_quantize_act_ex(const float* x, int ldx, int M, int M_stride, int K, int act32, int8_t* aq, float* asc,
                            int16_t* absum, void* stream);

/* Producers of the activations (the step before every product), fused with the quantizer above (act32 layout):
 *
 * qmatmul_rmsnorm_quant: y[m] = x[m] * r * w, r = 1 / sqrt(mean(x[m]^2) + eps), quantized; rows M..M_stride-1 zero.
 *   h (optional, row stride ldh) receives y. Replaces the rmsnorm_quant kernel (zero/kernels/ops.cl:82-104, launched
 *   by Engine::rmsnorm_quant, zero/engine.h:3302-3308); its row_off is a pointer offset on x here.
 * qmatmul_swiglu_quant: y[m] = silu(gate) * up (gelu_tanh(gate) * up with gelu) from rows [gate(F) | up(F)] of stride
 *   ldg, or y[m] = the row itself with fused (the engine's quant_rows), quantized. Replaces swiglu_quant
 *   (ops.cl:110-128; zero/engine.h:3451-3456).
 * qmatmul_add_norm_quant: x[m] = (x[m] + t[m] * r * w) * s (r from t[m]'s mean square; x updated in place), then
 *   y[m] = x[m] * r2 * w2 (r2 from the new x[m]) or, with w2 == NULL, y[m] = x[m]; y quantized. Rows of stride K,
 *   K <= 16384. Replaces add_norm_quant (ops.cl:2025-2075; zero/engine.h:3415).
 * Sums of squares are f32, so y matches a CPU evaluation to float tolerance, not bit for bit; the quantization of y
 * is the quantizer's exact arithmetic. Pointers to f32 rows must be 16-byte aligned with row strides % 4 == 0. */
int qmatmul_rmsnorm_quant(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps, int8_t* aq,
                          float* asc, int16_t* absum, float* h, int ldh, void* stream);
int qmatmul_swiglu_quant(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int8_t* aq,
                         float* asc, int16_t* absum, void* stream);
int qmatmul_add_norm_quant(float* x, const float* t, const float* w, int K, float eps, float s, const float* w2, int M,
                           int M_stride, int8_t* aq, float* asc, int16_t* absum, void* stream);
/* The three producers with the reference's act32 argument (Engine::rmsnorm_quant / add_norm_quant / quant_rows,
 * zero/engine.h:3302, 3415, 3451): act32 = 1 is the functions above; act32 = 0 writes per-256 scales
 * (asc [K/256][M_stride], K % 256 == 0). */
int qmatmul_rmsnorm_quant_ex(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps, int act32,
                             int8_t* aq, float* asc, int16_t* absum, float* h, int ldh, void* stream);
int qmatmul_swiglu_quant_ex(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int act32,
                            int8_t* aq, float* asc, int16_t* absum, void* stream);
int qmatmul_add_norm_quant_ex(float* x, const float* t, const float* w, int K, float eps, float s, const float* w2,
                              int M, int M_stride, int act32, int8_t* aq, float* asc, int16_t* absum, void* stream);

/* Decode GEMV, T tokens (1..8) against one read of the weight:
 *   C[t*ldc + c_off + n] (+)= sum_k W[n][k] * a_t[k],  t < T, n < rows(w)
 * a_t = token t's int8 row of aq with its per-32 scales. accumulate 0 or 1. absum is required for Q4_K, Q5_K, Q6_K and Q2_K.
 * Replaces the gemv / gemv_v / gemv_mt / gemv_mt_v launches of Engine::matmul1 (zero/engine.h:3184-3232;
 * zero/kernels/decode.cl:636-737, 1074-1141, 1145-1411). */
int qmatmul_gemv(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M_stride, int T,
                 float* C, int ldc, int c_off, int accumulate, void* stream);

/* Prompt GEMM: C[m*ldc + c_off + n] (op)= sum_k W[n][k] * a_m[k] for m < M.
 * M <= M_stride; any M >= 1 and rows(w) % 16 == 0. Replaces decode_w8 + gemm of Engine::matmul1 for T > 8 and
 * gemm_ext (zero/engine.h:3234-3297; zero/kernels/gemm.cl:132-475). Q4_K is computed exactly (scales and mins),
 * not requantized as the reference's W8 path does (zero/kernels/decode.cl:455-507). Q4_K with M >= 128 runs on the
 * f16 matrix pipe (exact integer block sums from f16 products) and takes a per-call workspace of about 2*M*K bytes
 * from a per-device stream-ordered memory pool; every other case runs on int8 MFMA and allocates nothing. A caller
 * that owns all memory passes the workspace itself (qmatmul_gemm_ws). */
int qmatmul_gemm(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M, int M_stride,
                 float* C, int ldc, int c_off, int accumulate, void* stream);
/* qmatmul_gemm with the act32 argument of Engine::matmul / matmul1 (zero/engine.h:3151, 3184, 3247; gemm.cl built
 * with or without -DACT32): act32 = 1 is qmatmul_gemm; act32 = 0 reads per-256 activation scales (asc [K/256][M_stride],
 * K % 256 == 0) -- the same kernels, which then take the scale of 32-block b from row b / 8. The per-256 result
 * equals the reference's superblock form asc * (d * sum_b sc*isum - dmin * sum_b mn*bsum) (gemm.cl:413-447) up to
 * f32 rounding order. */
int qmatmul_gemm_ex(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M, int M_stride,
                    int act32, float* C, int ldc, int c_off, int accumulate, void* stream);

/* The prompt GEMM with a caller-owned workspace, as the reference's engine owns its W8 staging buffers
 * (zero/engine.h:3238-3246): qmatmul_gemm_ex's arguments plus ws (device, 256-byte aligned) of at least
 * qmatmul_gemm_workspace_size(w, M) bytes. That size is 0 for every call but Q4_K with M >= 128 (then
 * 2*Mp*K + 4*Mp*K/32 bytes, Mp = M rounded up to 128); ws may be NULL when it is 0. No allocation, no host
 * synchronisation; calls on different streams need different workspaces. QM_ERR_WORKSPACE if ws is too small. */
size_t qmatmul_gemm_workspace_size(const qm_weight* w, int M);
int qmatmul_gemm_ws(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M, int M_stride,
                    int act32, float* C, int ldc, int c_off, int accumulate, void* ws, size_t ws_bytes, void* stream);

/* qmatmul_gemm without any device allocation. No counterpart in the reference: for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). Same arguments, results and kernels
 * as qmatmul_gemm; where qmatmul_gemm would take its pool workspace, this entry uses a static 32 MiB device array
 * (one per GPU, held until the process ends) and returns QM_ERR_WORKSPACE when the call needs more
 * (f16 path: 2*Mp*K + 4*Mp*K/32 bytes, Mp = M rounded up to 128; e.g. M 2048 x K 5120 needs 22.3 MB).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (different streams, or threads) race
 * and must be ordered by the caller. Each call writes every scratch byte it reads before reading it. It takes per-32
 * activation scales only (qmatmul_gemm's act32 = 1); a caller with per-256 scales that cannot allocate passes its
 * own workspace to qmatmul_gemm_ws. */
int qmatmul_gemm_noalloc(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M,
                         int M_stride, float* C, int ldc, int c_off, int accumulate, void* stream);

/* Workspace bytes of qmatmul_moe_grouped for T tokens, NE experts, NU experts per token, hidden E, expert width F
 * (the down projection's K). */
size_t qmatmul_moe_workspace_size(int T, int NE, int NU, int E, int F);

/* Routing alone (test and reuse): top NU of each token's NE logits (row stride ldl; ties go to the lower expert),
 * weights exp(l - max) / sum over the selection, per-expert counts (counts is overwritten).
 * zero/kernels/moe.cl:42-81 (moe_route). */
int qmatmul_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts,
                      void* stream);

/* Mixture-of-experts FFN over T tokens (Qwen3.5-MoE style), the expert part of Engine::layer_moe
 * (zero/engine_moe.h:8-282):
 *   x[t][:E] (op)= sum_k w_tk * down_e( q( silu(gate_e(a_t)) * up_e(a_t) ) ),  e = k-th expert of token t
 * gate, up: NE*Fv rows of E; down: NE*E rows of F (stacked experts), F = Fv, or F = Fv rounded up to 256 for a down
 * projection prepared from Fv-long Q8_0 / Q4_0 / IQ4_NL / Q2_0 rows (zero-padded; the h rows then have F values, the last
 * F - Fv zero: Flash Next's 640-wide experts as 768, zero/engine_moe.h:12, 318-326). a_t: token t of aq/asc (E values). q(): the h
 * rows quantized per 32 as moe_quant (moe.cl:251-282). Route, exclusive scan into tiles, device-side scatter of
 * (token, expert) pairs to slots, expert-grouped int8 MFMA GEMMs over the slot tiles, and the combine in fixed
 * order (moe.cl:332-340); at decode sizes (T * NU <= 64) GEMV-shaped expert kernels instead. Gate, up and down each
 * have their own type, any of Q8_0, Q4_0, IQ4_NL, IQ4_XS, IQ3_S, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, Q6_K, Q3_K, Q2_0 --
 * the types of the reference's expert GEMM moe_rg (zero/engine_moe.h:297-306); types with per-block mins (Q4_K, Q5_K, Q2_K) return
 * QM_ERR_TYPE, as there. accumulate 0 or 1.
 * ws: device workspace of at least qmatmul_moe_workspace_size bytes (layout: qmatmul_moe_ws_layout). */
int qmatmul_moe_grouped(const qm_weight* gate, const qm_weight* up, const qm_weight* down, int NE, const float* logits,
                        int ldl, int T, int NU, const int8_t* aq, const float* asc, int M_stride, float* x,
                        int accumulate, void* ws, size_t ws_bytes, void* stream);

/* qmatmul_moe_grouped with the routing and combine options of the reference's moe.cl:
 *   escale [NE] (or NULL): each selected expert's weight, after the normalization over the selection, times
 *     escale[e] (moe.cl:22-28, 75-77, -DESCALE);
 *   sh [T][ldsh] (or NULL): the shared expert's output for each token (computed by the caller), added to x as
 *     x[t] (op)= sum_k w_tk * y_tk + g_t * sh[t], with g_t = sigmoid(logits[t][NE]) when sh_gated (the router's
 *     extra column: ldl > NE) and g_t = 1 otherwise (moe.cl:37-41, 332-340; -DSH_NOGATE). ldsh >= E, a multiple of 4.
 * qmatmul_moe_grouped is this call with escale = sh = NULL. */
int qmatmul_moe_grouped_ex(const qm_weight* gate, const qm_weight* up, const qm_weight* down, int NE,
                           const float* logits, int ldl, int T, int NU, const int8_t* aq, const float* asc,
                           int M_stride, const float* escale, const float* sh, int ldsh, int sh_gated, float* x,
                           int accumulate, void* ws, size_t ws_bytes, void* stream);

/* Byte offsets of the MoE workspace's arrays (for tests and tools reading the routing state). After a tile-path call
 * (T * NU > 64): ids / wts the routing; counts[e] the slots of expert e; cursor[e] its first slot; tstart[e] its first
 * tile (tstart[NE] = the tile count); tiles[0] = the tile count, then (expert, first slot, rows) per tile, every
 * expert's tiles starting at an even index (an odd count gets one more entry of 0 rows at its last slot); stok / swt
 * each slot's token and routing weight; inv[t * NU + k] the slot of (token t, pick k). The workspace also holds
 * internal routing histograms after hf (inside total). */
typedef struct {
  size_t ids, wts, counts, cursor, tstart, tiles, stok, swt, inv, hq, hsc, y, hf, total;
  int slots, max_tiles, tile_rows;
} qm_moe_ws_layout;
int qmatmul_moe_ws_layout(int T, int NE, int NU, int E, int F, qm_moe_ws_layout* out);

/* Verification hooks: the integer block sums of the GEMV / GEMM kernels, from the same decode and dot-product
 * code as the products. For each token m < M, row n and 32-block b (index (m*rows + n)*(K/32) + b):
 *   isum[...] = sc_b * sum_{k in b} q[n][k] * a_m[k]   (Q8_0: sc_b = 1)
 *   msum[...] = mn_b * (absum of the block's two 16-halves)   (Q4_K, Q5_K; Q2_K: mn0 * bs0 + mn1 * bs1 with its
 *               mins per 16; NULL otherwise)
 * These are the reference's `sc0 * lo + sc1 * hi` and `mn0 * bs0 + mn1 * bs1` (zero/kernels/decode.cl:695-706). */
int qmatmul_gemv_blocksums(const qm_weight* w, const int8_t* aq, const int16_t* absum, int M_stride, int T,
                           int32_t* isum, int32_t* msum, void* stream);
int qmatmul_gemm_blocksums(const qm_weight* w, const int8_t* aq, int M, int M_stride, int32_t* isum, void* stream);

/* GGUF files (host side). Maps a GGUF v2/v3 file read-only and indexes its metadata and tensors, so a weight can
 * go to qmatmul_prepare_weight straight from the mapping (raw_on_device = 0; rows = dims[1] * dims[2] * ..., K =
 * dims[0]). Replaces the reference's GgufFile (src/gguf.h:85-305; Win32 mapping there, POSIX here). A split model
 * (name-00001-of-0000N.gguf, "split.count" metadata) is opened from part 1: the other parts are mapped from the same
 * directory and their tensors appended (src/gguf.h:170-187); a missing part fails the open. Pointers returned by
 * the accessors live until qmatmul_gguf_close. Reading is bounds-checked: truncated or malformed files fail with
 * QM_ERR_ARG and a message. Metadata: numbers of any GGUF numeric type read
 * through get_int / get_float; strings through get_str; arrays are indexed but not exposed. */
typedef struct qm_gguf qm_gguf;
int qmatmul_gguf_open(const char* path, qm_gguf** out);
int qmatmul_gguf_close(qm_gguf* g);
int qmatmul_gguf_tensor_count(const qm_gguf* g, int* n);
int qmatmul_gguf_find_tensor(const qm_gguf* g, const char* name, int* index);
int qmatmul_gguf_tensor_info(const qm_gguf* g, int i, const char** name, int* type, int* n_dims, uint64_t* dims,
                             const void** data, uint64_t* nbytes);
int qmatmul_gguf_get_int(const qm_gguf* g, const char* key, int64_t* out);
int qmatmul_gguf_get_float(const qm_gguf* g, const char* key, double* out);
int qmatmul_gguf_get_str(const qm_gguf* g, const char* key, const char** out);

#ifdef __cplusplus
}
#endif
#endif /* QMATMUL_H */
