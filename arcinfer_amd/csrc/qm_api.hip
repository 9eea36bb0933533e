// The C ABI of include/qmatmul.h: argument and shape checks, weight preparation, workspace layout, launches.
// Never throws or exits; errors come back as qm_status with a message in qmatmul_last_error().
#include <stdlib.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/qmatmul.h"
#include "qm_gguf.h"
#include "qm_launch.h"

struct qm_weight {
  int type, rows, K, device;
  uint8_t* base;
  size_t bytes;
  qm::WView view;
};

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(QM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool known_type(int t) {
  return t == QM_Q4_0 || t == QM_Q8_0 || t == QM_Q4_K || t == QM_Q5_K || t == QM_Q6_K || t == QM_IQ4_NL || t == QM_IQ3_S ||
         t == QM_IQ4_XS || t == QM_IQ2_XXS || t == QM_IQ2_XS || t == QM_IQ2_S || t == QM_IQ3_XXS || t == QM_Q3_K ||
         t == QM_Q2_0 || t == QM_Q2_K || t == QM_IQ1_S || t == QM_IQ1_M;
}

int payload_bytes(int t) {
  switch (t) {
    case QM_Q8_0: return 32;
    case QM_Q6_K: return 24;
    case QM_Q5_K: return 20;
    case QM_IQ3_S: case QM_IQ3_XXS: case QM_Q3_K: return 12;
    case QM_IQ2_XXS: case QM_IQ2_XS: case QM_IQ2_S: case QM_Q2_0: case QM_Q2_K: case QM_IQ1_S: case QM_IQ1_M: return 8;
    default: return 16;
  }
}
int header_bytes(int t) {
  switch (t) {
    case QM_IQ4_XS: case QM_Q2_0: return 8;
    case QM_Q6_K: case QM_IQ2_S: case QM_Q3_K: case QM_Q2_K: return 20;
    case QM_IQ2_XS: return 12;
    case QM_IQ2_XXS: case QM_IQ3_XXS: case QM_IQ1_S: case QM_IQ1_M: return 4;
    default: return 16;
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// the types of 32- (Q2_0: 64-) element blocks, whose rows may end inside a superblock (padded with zero blocks when
// prepared)
bool small_block_type(int t) { return t == QM_Q8_0 || t == QM_Q4_0 || t == QM_IQ4_NL || t == QM_Q2_0; }
bool row_length_ok(int t, int K) {
  return K > 0 && (K % 256 == 0 || (small_block_type(t) && K % (t == QM_Q2_0 ? 64 : 32) == 0));
}
int padded_k(int K) { return (K + 255) / 256 * 256; }


size_t plane_qs_bytes(int t, int rows, int K) { return (size_t)rows * (K / 32) * payload_bytes(t); }
size_t plane_hdr_bytes(int t, int rows, int K) { return (size_t)rows * (K / 256) * header_bytes(t); }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

std::once_flag g_init_once;
int g_init_status = QM_OK;
char g_init_err[512] = "";

int ensure_init() {
  std::call_once(g_init_once, [] {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    hipDeviceProp_t p;
    if (e == hipSuccess) e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) {
      g_init_status = QM_ERR_HIP;
      snprintf(g_init_err, sizeof(g_init_err), "qmatmul_init: %s", hipGetErrorString(e));
      return;
    }
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
      g_init_status = QM_ERR_HIP;
      snprintf(g_init_err, sizeof(g_init_err), "qmatmul_init: device is %s, the kernels are built for gfx950",
               p.gcnArchName);
    }
  });
  if (g_init_status != QM_OK) return fail(g_init_status, "%s", g_init_err);
  return QM_OK;
}

#define QM_CHECK_INIT()            \
  do {                             \
    const int st_ = ensure_init(); \
    if (st_) return st_;           \
  } while (0)

struct MoeLayout {
  size_t ids, wts, counts, cursor, tstart, tiles, stok, swt, inv, hq, hsc, y, hf, part, total;
  int slots, max_tiles, tile_rows;
};


MoeLayout moe_layout(int T, int NE, int NU, int E, int F) {
  MoeLayout L;
  L.slots = T * NU;
  L.tile_rows = qm::kMoeTileRows;
  L.max_tiles = (L.slots + qm::kMoeTileRows - 1) / qm::kMoeTileRows + 2 * NE;  // (+ one even-ing entry per expert)
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  L.ids = take(sizeof(int) * (size_t)L.slots);
  L.wts = take(sizeof(float) * (size_t)L.slots);
  L.counts = take(sizeof(int) * (size_t)NE);
  L.cursor = take(sizeof(int) * (size_t)NE);
  L.tstart = take(sizeof(int) * (size_t)(NE + 1));
  L.tiles = take(sizeof(int) * (size_t)(1 + 3 * L.max_tiles));
  L.stok = take(sizeof(int) * (size_t)L.slots);
  L.swt = take(sizeof(float) * (size_t)L.slots);
  L.inv = take(sizeof(int) * (size_t)L.slots);
  L.hq = take((size_t)L.slots * F);
  L.hsc = take(sizeof(float) * (size_t)(F / 32) * L.slots);
  L.y = take(sizeof(float) * (size_t)L.slots * E);
  L.hf = take(sizeof(float) * (size_t)L.slots * F);
  L.part = take(sizeof(int) * (size_t)qm::moe_route_groups(T) * NE);  // routing histograms, then running sums
  L.total = o;
  return L;
}

}  // namespace

extern "C" {

int qmatmul_init(void) {
  QM_CHECK_INIT();
  return QM_OK;
}

const char* qmatmul_last_error(void) { return g_err; }

size_t qmatmul_sb_bytes(int type) {
  switch (type) {
    case QM_Q8_0: return 272;
    case QM_Q4_K: return 144;
    case QM_Q6_K: return 210;
    case QM_Q5_K: return 176;
    case QM_Q4_0: return 144;
    case QM_IQ4_NL: return 144;
    case QM_IQ3_S: return 110;
    case QM_IQ4_XS: return 136;
    case QM_IQ2_XXS: return 66;
    case QM_IQ2_XS: return 74;
    case QM_IQ2_S: return 82;
    case QM_IQ3_XXS: return 98;
    case QM_Q3_K: return 110;
    case QM_Q2_0: return 72;
    case QM_Q2_K: return 84;
    case QM_IQ1_S: return 50;
    case QM_IQ1_M: return 56;
    default: return 0;
  }
}

size_t qmatmul_weight_bytes(int type, int rows, int K) {
  if (!known_type(type) || rows <= 0 || !row_length_ok(type, K)) return 0;
  K = padded_k(K);
  return align256(plane_qs_bytes(type, rows, K)) + plane_hdr_bytes(type, rows, K);
}

int qmatmul_prepare_weight(int type, const void* raw, int raw_on_device, int rows, int K, void* stream,
                           qm_weight** out) {
  if (!out || !raw) return fail(QM_ERR_ARG, "qmatmul_prepare_weight: null pointer");
  *out = nullptr;
  if (!known_type(type)) return fail(QM_ERR_TYPE, "qmatmul_prepare_weight: unsupported type %d", type);
  if (rows <= 0 || !row_length_ok(type, K))
    return fail(QM_ERR_SHAPE,
                "qmatmul_prepare_weight: rows %d, K %d (K must be a positive multiple of 256, or of 32 for Q8_0, "
                "Q4_0 and IQ4_NL, of 64 for Q2_0)", rows, K);
  QM_CHECK_INIT();
  hipStream_t s = (hipStream_t)stream;
  const int kraw = K / 32;  // 32-blocks per raw row
  const size_t rawb = small_block_type(type) ? (size_t)rows * kraw * (qmatmul_sb_bytes(type) / 8)
                                             : (size_t)rows * (K / 256) * qmatmul_sb_bytes(type);
  K = padded_k(K);  // (the prepared row: zero blocks up to whole superblocks)
  const size_t qsb = plane_qs_bytes(type, rows, K), total = qmatmul_weight_bytes(type, rows, K);
  qm_weight* w = new (std::nothrow) qm_weight();
  if (!w) return fail(QM_ERR_NOMEM, "qmatmul_prepare_weight: host allocation");
  hipError_t e = hipGetDevice(&w->device);
  if (e != hipSuccess) {
    delete w;
    return hip_fail(e, "qmatmul_prepare_weight: hipGetDevice");
  }
  e = hipMalloc((void**)&w->base, total);
  if (e != hipSuccess) {
    delete w;
    return fail(QM_ERR_NOMEM, "qmatmul_prepare_weight: hipMalloc(%zu): %s", total, hipGetErrorString(e));
  }
  const uint8_t* src = (const uint8_t*)raw;
  uint8_t* staged = nullptr;
  if (!raw_on_device) {
    e = hipMalloc((void**)&staged, rawb);
    if (e == hipSuccess) e = hipMemcpyAsync(staged, raw, rawb, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) {
      if (staged) (void)hipFree(staged);
      (void)hipFree(w->base);
      delete w;
      return hip_fail(e, "qmatmul_prepare_weight: staging the host bytes");
    }
    src = staged;
  }
  w->type = type;
  w->rows = rows;
  w->K = K;
  w->bytes = total;
  w->view.qs = w->base;
  w->view.hdr = w->base + align256(qsb);
  w->view.rows = rows;
  w->view.K = K;
  e = qm::launch_repack(type, src, rows, K, kraw, w->base, w->base + align256(qsb), s);
  if (e == hipSuccess && staged) e = hipStreamSynchronize(s);
  if (staged) (void)hipFree(staged);
  if (e != hipSuccess) {
    (void)hipFree(w->base);
    delete w;
    return hip_fail(e, "qmatmul_prepare_weight: repack");
  }
  *out = w;
  return QM_OK;
}

int qmatmul_release_weight(qm_weight* w) {
  if (!w) return fail(QM_ERR_ARG, "qmatmul_release_weight: null weight");
  hipError_t e = hipFree(w->base);
  delete w;
  if (e != hipSuccess) return hip_fail(e, "qmatmul_release_weight: hipFree");
  return QM_OK;
}

int qmatmul_weight_info(const qm_weight* w, int* type, int* rows, int* K) {
  if (!w) return fail(QM_ERR_ARG, "qmatmul_weight_info: null weight");
  if (type) *type = w->type;
  if (rows) *rows = w->rows;
  if (K) *K = w->K;
  return QM_OK;
}

int qmatmul_quantize_act_ex(const float* x, int ldx, int M, int M_stride, int K, int act32, int8_t* aq, float* asc,
                            int16_t* absum, void* stream) {
  if (!x || !aq || !asc || !absum) return fail(QM_ERR_ARG, "qmatmul_quantize_act: null pointer");
  if (act32 != 0 && act32 != 1) return fail(QM_ERR_ARG, "qmatmul_quantize_act: act32 %d (0 or 1)", act32);
  if (K <= 0 || K % (act32 ? 32 : 256) || M < 0 || M_stride < 1 || M > M_stride || ldx < K)
    return fail(QM_ERR_SHAPE, "qmatmul_quantize_act: M %d, M_stride %d, K %d, ldx %d, act32 %d", M, M_stride, K, ldx,
                act32);
  if (!aligned(aq, 4)) return fail(QM_ERR_ARG, "qmatmul_quantize_act: aq must be 4-byte aligned");
  QM_CHECK_INIT();
  const hipError_t e = qm::launch_quantize(x, ldx, M, M_stride, K, act32 != 0, aq, asc, absum, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_quantize_act");
}

int qmatmul_quantize_act(const float* x, int ldx, int M, int M_stride, int K, int8_t* aq, float* asc, int16_t* absum,
                         void* stream) {
  return qmatmul_quantize_act_ex(x, ldx, M, M_stride, K, 1, aq, asc, absum, stream);
}

static int check_out_acts(const char* fn, int M, int M_stride, int K, int act32, const int8_t* aq, const float* asc,
                          const int16_t* absum) {
  if (!aq || !asc || !absum) return fail(QM_ERR_ARG, "%s: null output pointer", fn);
  if (act32 != 0 && act32 != 1) return fail(QM_ERR_ARG, "%s: act32 %d (0 or 1)", fn, act32);
  if (K <= 0 || K % (act32 ? 32 : 256) || M < 0 || M_stride < 1 || M > M_stride)
    return fail(QM_ERR_SHAPE, "%s: M %d, M_stride %d, K %d, act32 %d", fn, M, M_stride, K, act32);
  if (!aligned(aq, 4)) return fail(QM_ERR_ARG, "%s: aq must be 4-byte aligned", fn);
  return QM_OK;
}

int qmatmul_rmsnorm_quant_ex(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps, int act32,
                             int8_t* aq, float* asc, int16_t* absum, float* h, int ldh, void* stream) {
  if (int st = check_out_acts("qmatmul_rmsnorm_quant", M, M_stride, K, act32, aq, asc, absum)) return st;
  if (!x || !w) return fail(QM_ERR_ARG, "qmatmul_rmsnorm_quant: null input");
  if (ldx < K || ldx % 4 || !aligned(x, 16) || !aligned(w, 16) || (h && (ldh < K || ldh % 4 || !aligned(h, 16))))
    return fail(QM_ERR_ARG, "qmatmul_rmsnorm_quant: x, w, h need 16-byte aligned rows (ldx %d, ldh %d, K %d)", ldx,
                ldh, K);
  QM_CHECK_INIT();
  const hipError_t e = qm::launch_rmsnorm_quant(x, ldx, w, K, M, M_stride, eps, aq, asc, absum, h, ldh,
                                                act32 != 0, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_rmsnorm_quant");
}

int qmatmul_rmsnorm_quant(const float* x, int ldx, const float* w, int K, int M, int M_stride, float eps, int8_t* aq,
                          float* asc, int16_t* absum, float* h, int ldh, void* stream) {
  return qmatmul_rmsnorm_quant_ex(x, ldx, w, K, M, M_stride, eps, 1, aq, asc, absum, h, ldh, stream);
}

int qmatmul_swiglu_quant_ex(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int act32,
                            int8_t* aq, float* asc, int16_t* absum, void* stream) {
  if (int st = check_out_acts("qmatmul_swiglu_quant", M, M_stride, F, act32, aq, asc, absum)) return st;
  if (!gu) return fail(QM_ERR_ARG, "qmatmul_swiglu_quant: null input");
  if (ldg < (fused ? F : 2 * F) || ldg % 4 || !aligned(gu, 16))
    return fail(QM_ERR_ARG, "qmatmul_swiglu_quant: ldg %d for F %d (fused %d), 16-byte aligned rows", ldg, F, fused);
  QM_CHECK_INIT();
  const hipError_t e = qm::launch_swiglu_quant(gu, ldg, F, M, M_stride, fused ? 1 : 0, gelu ? 1 : 0, aq, asc, absum,
                                               act32 != 0, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_swiglu_quant");
}

int qmatmul_swiglu_quant(const float* gu, int ldg, int F, int M, int M_stride, int fused, int gelu, int8_t* aq,
                         float* asc, int16_t* absum, void* stream) {
  return qmatmul_swiglu_quant_ex(gu, ldg, F, M, M_stride, fused, gelu, 1, aq, asc, absum, stream);
}

int qmatmul_add_norm_quant_ex(float* x, const float* t, const float* w, int K, float eps, float s, const float* w2,
                              int M, int M_stride, int act32, int8_t* aq, float* asc, int16_t* absum, void* stream) {
  if (int st = check_out_acts("qmatmul_add_norm_quant", M, M_stride, K, act32, aq, asc, absum)) return st;
  if (!x || !t || !w) return fail(QM_ERR_ARG, "qmatmul_add_norm_quant: null input");
  if (K > 16384) return fail(QM_ERR_SHAPE, "qmatmul_add_norm_quant: K %d (at most 16384)", K);
  if (!aligned(x, 16) || !aligned(t, 16) || !aligned(w, 16) || (w2 && !aligned(w2, 16)))
    return fail(QM_ERR_ARG, "qmatmul_add_norm_quant: x, t, w, w2 must be 16-byte aligned");
  QM_CHECK_INIT();
  const hipError_t e = qm::launch_add_norm_quant(x, t, w, K, eps, s, w2, M, M_stride, aq, asc, absum,
                                                 act32 != 0, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_add_norm_quant");
}

int qmatmul_add_norm_quant(float* x, const float* t, const float* w, int K, float eps, float s, const float* w2, int M,
                           int M_stride, int8_t* aq, float* asc, int16_t* absum, void* stream) {
  return qmatmul_add_norm_quant_ex(x, t, w, K, eps, s, w2, M, M_stride, 1, aq, asc, absum, stream);
}

static int check_acts(const char* fn, const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum,
                      int rows_needed, int M_stride) {
  if (!w || !aq || !asc) return fail(QM_ERR_ARG, "%s: null pointer", fn);
  if ((w->type == QM_Q4_K || w->type == QM_Q5_K || w->type == QM_Q6_K || w->type == QM_Q2_K) && !absum)
    return fail(QM_ERR_ARG, "%s: Q4_K, Q5_K, Q6_K and Q2_K need the per-16 activation sums", fn);
  if (rows_needed < 1 || M_stride < rows_needed)
    return fail(QM_ERR_SHAPE, "%s: %d activation rows with M_stride %d", fn, rows_needed, M_stride);
  if (!aligned(aq, 16)) return fail(QM_ERR_ARG, "%s: aq must be 16-byte aligned", fn);
  return QM_OK;
}

int qmatmul_gemv(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M_stride, int T,
                 float* C, int ldc, int c_off, int accumulate, void* stream) {
  if (int st = check_acts("qmatmul_gemv", w, aq, asc, absum, T, M_stride)) return st;
  if (!C) return fail(QM_ERR_ARG, "qmatmul_gemv: null output");
  if (T < 1 || T > 8) return fail(QM_ERR_SHAPE, "qmatmul_gemv: T = %d (1..8 tokens per call)", T);
  if (accumulate != 0 && accumulate != 1) return fail(QM_ERR_ARG, "qmatmul_gemv: accumulate %d (0 or 1)", accumulate);
  if (c_off < 0 || (T > 1 && ldc < c_off + w->rows))
    return fail(QM_ERR_SHAPE, "qmatmul_gemv: ldc %d, c_off %d, rows %d", ldc, c_off, w->rows);
  QM_CHECK_INIT();
  qm::GemvArgs a{};
  a.w = w->view;
  a.aq = aq;
  a.asc = asc;
  a.absum = absum;
  a.M_stride = M_stride;
  a.T = T;
  a.C = C;
  a.ldc = ldc;
  a.c_off = c_off;
  a.accumulate = accumulate;
  const hipError_t e = qm::launch_gemv(w->type, a, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_gemv");
}

int qmatmul_gemv_blocksums(const qm_weight* w, const int8_t* aq, const int16_t* absum, int M_stride, int T,
                           int32_t* isum, int32_t* msum, void* stream) {
  static const float unused = 0.0f;  // (the block-sum mode reads no scales)
  if (int st = check_acts("qmatmul_gemv_blocksums", w, aq, &unused, absum, T, M_stride)) return st;
  if (!isum || ((w->type == QM_Q4_K || w->type == QM_Q5_K || w->type == QM_Q2_K) && !msum))
    return fail(QM_ERR_ARG, "qmatmul_gemv_blocksums: null output");
  if (T < 1 || T > 8) return fail(QM_ERR_SHAPE, "qmatmul_gemv_blocksums: T = %d", T);
  QM_CHECK_INIT();
  qm::GemvArgs a{};
  a.w = w->view;
  a.aq = aq;
  a.absum = absum;
  a.M_stride = M_stride;
  a.T = T;
  a.dbg_isum = isum;
  a.dbg_msum = msum;
  const hipError_t e = qm::launch_gemv(w->type, a, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_gemv_blocksums");
}

// qmatmul_gemm, qmatmul_gemm_ex, qmatmul_gemm_ws and qmatmul_gemm_noalloc: one argument check and dispatch. act32 = 0
// takes per-256 activation scales (asc [K/256][M_stride]); the kernels then read the scale of 32-block b at row b >> 3.
// The workspace of the f16 path comes from the per-device pool (WS_POOL), the caller (WS_CALLER: ws, ws_bytes) or the
// static scratch array (WS_STATIC); every other case needs none.
enum WsMode { WS_POOL, WS_CALLER, WS_STATIC };

static int gemm_impl(const char* fn, const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum,
                     int M, int M_stride, int act32, float* C, int ldc, int c_off, int accumulate, WsMode wm,
                     void* ws, size_t ws_bytes, void* stream) {
  if (int st = check_acts(fn, w, aq, asc, absum, M, M_stride)) return st;
  if (!C) return fail(QM_ERR_ARG, "%s: null output", fn);
  if (w->rows % 16) return fail(QM_ERR_SHAPE, "%s: rows %d not a multiple of 16", fn, w->rows);
  if (accumulate < 0 || accumulate > 2) return fail(QM_ERR_ARG, "%s: accumulate %d (0..2)", fn, accumulate);
  if (c_off < 0 || ldc < c_off + w->rows)
    return fail(QM_ERR_SHAPE, "%s: ldc %d, c_off %d, rows %d", fn, ldc, c_off, w->rows);
  if (act32 != 0 && act32 != 1) return fail(QM_ERR_ARG, "%s: act32 %d (0 or 1)", fn, act32);
  if (!act32 && w->view.K % 256)
    return fail(QM_ERR_SHAPE, "%s: per-256 activation scales need K %% 256 == 0 (K %d)", fn, w->view.K);
  QM_CHECK_INIT();
  qm::GemmArgs a{};
  a.w = w->view;
  a.aq = aq;
  a.asc = asc;
  a.absum = absum;
  a.M = M;
  a.M_stride = M_stride;
  a.C = C;
  a.ldc = ldc;
  a.c_off = c_off;
  a.accumulate = accumulate;
  a.ash = act32 ? 0 : 3;
  hipError_t e;
  if (qm::f16_gemm_supported(w->type, M, w->view.K)) {
    void* scr = nullptr;  // null: the f16 path takes its workspace from the per-device pool
    const size_t need = qm::f16_workspace_bytes(M, w->view.K);
    if (wm == WS_STATIC) {
      size_t cap = 0;
      e = qm::f16_scratch(&scr, &cap);
      if (e != hipSuccess) return hip_fail(e, "qmatmul_gemm_noalloc: scratch lookup");
      if (need > cap)
        return fail(QM_ERR_WORKSPACE, "%s: M %d x K %d needs %zu bytes of scratch, the static scratch holds %zu "
                    "(use qmatmul_gemm or qmatmul_gemm_ws)", fn, M, w->view.K, need, cap);
    } else if (wm == WS_CALLER) {
      if (!ws || ws_bytes < need)
        return fail(QM_ERR_WORKSPACE, "%s: M %d x K %d needs a workspace of %zu bytes (given %zu%s)", fn, M,
                    w->view.K, need, ws_bytes, ws ? "" : ", null");
      if (!aligned(ws, 256)) return fail(QM_ERR_ARG, "%s: the workspace must be 256-byte aligned", fn);
      scr = ws;
    }
    e = qm::launch_gemm_f16(w->type, a, scr, (hipStream_t)stream);
  } else {
    e = qm::launch_gemm(w->type, qm::GEMM_DENSE, a, (hipStream_t)stream);  // (this kernel uses no workspace)
  }
  return e == hipSuccess ? QM_OK : hip_fail(e, fn);
}

int qmatmul_gemm(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M, int M_stride,
                 float* C, int ldc, int c_off, int accumulate, void* stream) {
  return gemm_impl("qmatmul_gemm", w, aq, asc, absum, M, M_stride, 1, C, ldc, c_off, accumulate, WS_POOL, nullptr, 0,
                   stream);
}

int qmatmul_gemm_ex(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M, int M_stride,
                    int act32, float* C, int ldc, int c_off, int accumulate, void* stream) {
  return gemm_impl("qmatmul_gemm_ex", w, aq, asc, absum, M, M_stride, act32, C, ldc, c_off, accumulate, WS_POOL,
                   nullptr, 0, stream);
}

size_t qmatmul_gemm_workspace_size(const qm_weight* w, int M) {
  if (!w || M < 1) return 0;
  return qm::f16_gemm_supported(w->type, M, w->view.K) ? qm::f16_workspace_bytes(M, w->view.K) : 0;
}

int qmatmul_gemm_ws(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M, int M_stride,
                    int act32, float* C, int ldc, int c_off, int accumulate, void* ws, size_t ws_bytes, void* stream) {
  return gemm_impl("qmatmul_gemm_ws", w, aq, asc, absum, M, M_stride, act32, C, ldc, c_off, accumulate, WS_CALLER, ws,
                   ws_bytes, stream);
}

int qmatmul_gemm_noalloc(const qm_weight* w, const int8_t* aq, const float* asc, const int16_t* absum, int M,
                         int M_stride, float* C, int ldc, int c_off, int accumulate, void* stream) {
  return gemm_impl("qmatmul_gemm_noalloc", w, aq, asc, absum, M, M_stride, 1, C, ldc, c_off, accumulate, WS_STATIC,
                   nullptr, 0, stream);
}

int qmatmul_gemm_blocksums(const qm_weight* w, const int8_t* aq, int M, int M_stride, int32_t* isum, void* stream) {
  static const float unused = 0.0f;  // (the block-sum mode reads no scales or sums)
  if (int st = check_acts("qmatmul_gemm_blocksums", w, aq, &unused, (const int16_t*)&unused, M, M_stride)) return st;
  if (!isum) return fail(QM_ERR_ARG, "qmatmul_gemm_blocksums: null output");
  if (w->rows % 16) return fail(QM_ERR_SHAPE, "qmatmul_gemm_blocksums: rows %d not a multiple of 16", w->rows);
  QM_CHECK_INIT();
  qm::GemmArgs a{};
  a.w = w->view;
  a.aq = aq;
  a.M = M;
  a.M_stride = M_stride;
  a.dbg_isum = isum;
  // (the same kernel choice as qmatmul_gemm makes for this type and shape)
  const hipError_t e = qm::f16_gemm_supported(w->type, M, w->view.K)
                           ? qm::launch_gemm_f16(w->type, a, nullptr, (hipStream_t)stream)
                           : qm::launch_gemm(w->type, qm::GEMM_DENSE, a, (hipStream_t)stream);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_gemm_blocksums");
}

size_t qmatmul_moe_workspace_size(int T, int NE, int NU, int E, int F) {
  if (T < 1 || NE < 1 || NU < 1 || E < 1 || F < 1) return 0;
  return moe_layout(T, NE, NU, E, F).total;
}

int qmatmul_moe_ws_layout(int T, int NE, int NU, int E, int F, qm_moe_ws_layout* out) {
  if (!out) return fail(QM_ERR_ARG, "qmatmul_moe_ws_layout: null output");
  if (T < 1 || NE < 1 || NU < 1 || E < 1 || F < 1) return fail(QM_ERR_SHAPE, "qmatmul_moe_ws_layout: bad sizes");
  const MoeLayout L = moe_layout(T, NE, NU, E, F);
  out->ids = L.ids;
  out->wts = L.wts;
  out->counts = L.counts;
  out->cursor = L.cursor;
  out->tstart = L.tstart;
  out->tiles = L.tiles;
  out->stok = L.stok;
  out->swt = L.swt;
  out->inv = L.inv;
  out->hq = L.hq;
  out->hsc = L.hsc;
  out->y = L.y;
  out->hf = L.hf;
  out->total = L.total;
  out->slots = L.slots;
  out->max_tiles = L.max_tiles;
  out->tile_rows = L.tile_rows;
  return QM_OK;
}

int qmatmul_moe_route(const float* logits, int ldl, int T, int NE, int NU, int* ids, float* wts, int* counts,
                      void* stream) {
  if (!logits || !ids || !wts) return fail(QM_ERR_ARG, "qmatmul_moe_route: null pointer");
  if (T < 1 || NE < 1 || NE > 1024 || NU < 1 || NU > NE || NU > 64 || ldl < NE)
    return fail(QM_ERR_SHAPE, "qmatmul_moe_route: T %d, NE %d (<= 1024), NU %d (<= 64), ldl %d", T, NE, NU, ldl);
  QM_CHECK_INIT();
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  if (counts) e = qm::launch_fill_i32(counts, 0, (size_t)NE, s);
  if (e == hipSuccess) e = qm::launch_moe_route(logits, ldl, T, NE, NU, ids, wts, counts, nullptr, nullptr, s);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_moe_route");
}

int qmatmul_moe_grouped_ex(const qm_weight* gate, const qm_weight* up, const qm_weight* down, int NE,
                           const float* logits, int ldl, int T, int NU, const int8_t* aq, const float* asc,
                           int M_stride, const float* escale, const float* sh, int ldsh, int sh_gated, float* x,
                           int accumulate, void* ws, size_t ws_bytes, void* stream) {
  if (!gate || !up || !down || !logits || !aq || !asc || !x || !ws)
    return fail(QM_ERR_ARG, "qmatmul_moe_grouped: null pointer");
  for (const qm_weight* w : {gate, up, down})
    if (w->type == QM_IQ1_S || w->type == QM_IQ1_M)
      return fail(QM_ERR_TYPE, "qmatmul_moe_grouped: IQ1_S / IQ1_M are not expert types of the reference's moe_rg "
                               "(zero/engine_moe.h:296-301)");
  for (const qm_weight* w : {gate, up, down})
    if (w->type == QM_Q4_K || w->type == QM_Q5_K || w->type == QM_Q2_K)
      return fail(QM_ERR_TYPE,
                  "qmatmul_moe_grouped: Q4_K, Q5_K and Q2_K expert weights (per-block mins) are not supported, as in the "
                  "reference's expert GEMMs (zero/engine_moe.h:284-301)");
  if (NE < 1 || NE > 1024 || NU < 1 || NU > NE || NU > 64 || T < 1 || M_stride < T || ldl < NE)
    return fail(QM_ERR_SHAPE, "qmatmul_moe_grouped: NE %d, NU %d, T %d, M_stride %d, ldl %d", NE, NU, T, M_stride, ldl);
  // F: the down projection's K (the h row length); Fv: the experts' gate/up rows. Fv < F when the down projection's
  // rows were padded with zero blocks at preparation (Q8_0 / Q4_0 / IQ4_NL experts of a width that is not whole
  // superblocks: Flash Next's 640 as 768, zero/engine_moe.h:12, 318-326); h[Fv..F) is then zero.
  const int E = gate->K, F = down->K, Fv = gate->rows / NE;
  if (gate->rows != NE * Fv || up->rows != NE * Fv || up->K != E || down->rows != NE * E || Fv % 32 || E % 4 ||
      !(Fv == F || (F % 256 == 0 && padded_k(Fv) == F)))
    return fail(QM_ERR_SHAPE,
                "qmatmul_moe_grouped: gate %dx%d, up %dx%d, down %dx%d do not fit NE %d experts of F x E / E x F",
                gate->rows, gate->K, up->rows, up->K, down->rows, down->K, NE);
  if (accumulate != 0 && accumulate != 1)
    return fail(QM_ERR_ARG, "qmatmul_moe_grouped: accumulate %d (0 or 1)", accumulate);
  if (sh && (ldsh < E || ldsh % 4 || !aligned(sh, 16)))
    return fail(QM_ERR_ARG, "qmatmul_moe_grouped: sh needs ldsh >= E (%d), a multiple of 4, 16-byte alignment", E);
  if (sh && sh_gated && ldl < NE + 1)
    return fail(QM_ERR_SHAPE, "qmatmul_moe_grouped: a gated shared expert reads logits[t][NE]: ldl %d <= NE %d", ldl, NE);
  if (!aligned(aq, 16) || !aligned(x, 16) || !aligned(ws, 256))
    return fail(QM_ERR_ARG, "qmatmul_moe_grouped: aq/x need 16-byte, ws 256-byte alignment");
  const MoeLayout L = moe_layout(T, NE, NU, E, F);
  if (ws_bytes < L.total)
    return fail(QM_ERR_WORKSPACE, "qmatmul_moe_grouped: workspace %zu < %zu bytes", ws_bytes, L.total);
  QM_CHECK_INIT();
  hipStream_t s = (hipStream_t)stream;
  uint8_t* b = (uint8_t*)ws;
  int* ids = (int*)(b + L.ids);
  float* wts = (float*)(b + L.wts);
  int* counts = (int*)(b + L.counts);
  int* cursor = (int*)(b + L.cursor);
  int* tstart = (int*)(b + L.tstart);
  int* tiles = (int*)(b + L.tiles);
  int* stok = (int*)(b + L.stok);
  float* swt = (float*)(b + L.swt);
  int* inv = (int*)(b + L.inv);
  int8_t* hq = (int8_t*)(b + L.hq);
  float* hsc = (float*)(b + L.hsc);
  float* y = (float*)(b + L.y);
  float* hf = (float*)(b + L.hf);
  const qm::MoeShared shd{sh, ldsh, sh && sh_gated ? logits + NE : nullptr, ldl};
  // decode sizes: GEMV-shaped expert kernels (no tiles, no scatter): routing with gate/up, then down + combine
  if (T * NU <= 64 && NU <= 8 && F <= 4096 && E <= 8192) {
    const hipError_t e = qm::launch_moe_decode(gate->type, up->type, down->type, gate->view, up->view, down->view, T,
                                               NU, E, F, Fv, logits, ldl, NE, escale, ids, wts, aq, asc, M_stride, hf, x,
                                               accumulate, shd, s);
    return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_moe_grouped");
  }
  int* part = (int*)(b + L.part);
  hipError_t e = qm::launch_moe_route(logits, ldl, T, NE, NU, ids, wts, nullptr, escale, part, s);
  if (e == hipSuccess) e = qm::launch_moe_scan(part, qm::moe_route_groups(T), counts, NE, s);
  if (e == hipSuccess)
    e = qm::launch_moe_scatter(ids, wts, T, NU, NE, part, counts, cursor, tstart, tiles, L.tile_rows, stok, swt, inv, s);
  // gate and up: one launch when they share a type the int8 kernel takes in one pass; otherwise the gate projection
  // into hf, then the up projection forming h from it
  const bool s16 = [](int t) { return t == QM_Q6_K || t == QM_IQ2_XS || t == QM_IQ2_S || t == QM_Q3_K; }(gate->type);
  const bool fused = gate->type == up->type && !s16;
  if (e == hipSuccess) {
    qm::GemmArgs a{};
    a.w = gate->view;
    a.w2 = up->view;
    a.aq = aq;
    a.asc = asc;
    a.M = L.slots;
    a.M_stride = M_stride;
    a.tiles = tiles;
    a.rowmap = stok;
    a.hq = hq;
    a.hsc = hsc;
    a.slots = L.slots;
    a.max_tiles = L.max_tiles;
    a.expert_rows = Fv;
    a.C = hf;
    a.ldc = F;
    if (fused) {
      e = qm::launch_gemm(gate->type, qm::GEMM_MOE_GATEUP, a, s);
    } else {
      e = qm::launch_gemm(gate->type, qm::GEMM_MOE_G, a, s);
      a.w = up->view;
      if (e == hipSuccess) e = qm::launch_gemm(up->type, qm::GEMM_MOE_UH, a, s);
    }
  }
  // (padded h columns: scale 0 -- their weight blocks are zero, so the products are 0 whatever the int8 values)
  if (e == hipSuccess && Fv < F) e = qm::launch_fill_i32((int*)(hsc + (size_t)(Fv / 32) * L.slots), 0,
                                                         (size_t)((F - Fv) / 32) * L.slots, s);
  if (e == hipSuccess) {
    qm::GemmArgs a{};
    a.w = down->view;
    a.aq = hq;
    a.asc = hsc;
    a.M = L.slots;
    a.M_stride = L.slots;
    a.C = y;
    a.ldc = E;
    a.tiles = tiles;
    a.rowscale = swt;
    a.slots = L.slots;
    a.max_tiles = L.max_tiles;
    a.expert_rows = E;
    e = qm::launch_gemm(down->type, qm::GEMM_MOE_DOWN, a, s);
  }
  if (e == hipSuccess) e = qm::launch_moe_combine(x, y, inv, T, NU, E, accumulate, shd, s);
  return e == hipSuccess ? QM_OK : hip_fail(e, "qmatmul_moe_grouped");
}

int qmatmul_moe_grouped(const qm_weight* gate, const qm_weight* up, const qm_weight* down, int NE, const float* logits,
                        int ldl, int T, int NU, const int8_t* aq, const float* asc, int M_stride, float* x,
                        int accumulate, void* ws, size_t ws_bytes, void* stream) {
  return qmatmul_moe_grouped_ex(gate, up, down, NE, logits, ldl, T, NU, aq, asc, M_stride, nullptr, nullptr, 0, 0, x,
                                accumulate, ws, ws_bytes, stream);
}


// ---- GGUF files ----------------------------------------------------------------------------------------------------
struct qm_gguf {
  std::unique_ptr<qm::Gguf> g;
};

int qmatmul_gguf_open(const char* path, qm_gguf** out) {
  if (!path || !out) return fail(QM_ERR_ARG, "qmatmul_gguf_open: null pointer");
  *out = nullptr;
  std::string err;
  std::unique_ptr<qm::Gguf> g = qm::Gguf::open(path, err);
  if (!g) return fail(QM_ERR_ARG, "qmatmul_gguf_open: %s: %s", path, err.c_str());
  *out = new qm_gguf{std::move(g)};
  return QM_OK;
}

int qmatmul_gguf_close(qm_gguf* g) {
  delete g;
  return QM_OK;
}

int qmatmul_gguf_tensor_count(const qm_gguf* g, int* n) {
  if (!g || !n) return fail(QM_ERR_ARG, "qmatmul_gguf_tensor_count: null pointer");
  *n = (int)g->g->tensors.size();
  return QM_OK;
}

int qmatmul_gguf_find_tensor(const qm_gguf* g, const char* name, int* index) {
  if (!g || !name || !index) return fail(QM_ERR_ARG, "qmatmul_gguf_find_tensor: null pointer");
  auto it = g->g->index.find(name);
  if (it == g->g->index.end()) return fail(QM_ERR_ARG, "qmatmul_gguf_find_tensor: no tensor %s", name);
  *index = (int)it->second;
  return QM_OK;
}

int qmatmul_gguf_tensor_info(const qm_gguf* g, int i, const char** name, int* type, int* n_dims, uint64_t* dims,
                             const void** data, uint64_t* nbytes) {
  if (!g) return fail(QM_ERR_ARG, "qmatmul_gguf_tensor_info: null handle");
  if (i < 0 || i >= (int)g->g->tensors.size()) return fail(QM_ERR_ARG, "qmatmul_gguf_tensor_info: index %d", i);
  const qm::GgufTensorInfo& t = g->g->tensors[i];
  if (name) *name = t.name.c_str();
  if (type) *type = (int)t.type;
  if (n_dims) *n_dims = (int)t.n_dims;
  if (dims)
    for (int d = 0; d < 8; ++d) dims[d] = d < (int)t.n_dims ? t.dims[d] : 0;
  if (data) *data = t.data;
  if (nbytes) *nbytes = t.nbytes;
  return QM_OK;
}

static const qm::GgufValue* gguf_value(const qm_gguf* g, const char* key, const char* fn) {
  if (!g || !key) {
    fail(QM_ERR_ARG, "%s: null pointer", fn);
    return nullptr;
  }
  auto it = g->g->kv.find(key);
  if (it == g->g->kv.end()) {
    fail(QM_ERR_ARG, "%s: no key %s", fn, key);
    return nullptr;
  }
  return &it->second;
}

int qmatmul_gguf_get_int(const qm_gguf* g, const char* key, int64_t* out) {
  const qm::GgufValue* v = gguf_value(g, key, "qmatmul_gguf_get_int");
  if (!v) return QM_ERR_ARG;
  if (v->type == qm::GV_STR || v->type == qm::GV_ARR)
    return fail(QM_ERR_TYPE, "qmatmul_gguf_get_int: %s is not a number", key);
  if (out) *out = v->i;
  return QM_OK;
}

int qmatmul_gguf_get_float(const qm_gguf* g, const char* key, double* out) {
  const qm::GgufValue* v = gguf_value(g, key, "qmatmul_gguf_get_float");
  if (!v) return QM_ERR_ARG;
  if (v->type == qm::GV_STR || v->type == qm::GV_ARR)
    return fail(QM_ERR_TYPE, "qmatmul_gguf_get_float: %s is not a number", key);
  if (out) *out = v->f;
  return QM_OK;
}

int qmatmul_gguf_get_str(const qm_gguf* g, const char* key, const char** out) {
  const qm::GgufValue* v = gguf_value(g, key, "qmatmul_gguf_get_str");
  if (!v) return QM_ERR_ARG;
  if (v->type != qm::GV_STR) return fail(QM_ERR_TYPE, "qmatmul_gguf_get_str: %s is not a string", key);
  if (out) *out = v->s.c_str();
  return QM_OK;
}

}  // extern "C"
