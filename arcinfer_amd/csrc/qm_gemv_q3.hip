// Decode GEMV instantiations for Q3_K, Q2_0, Q2_K; the kernels are in qm_gemv_impl.h (one translation unit per pair of
// weight types, so the instantiations compile in parallel).
#include "qm_gemv_impl.h"

namespace qm {
template hipError_t gemv_dispatch<T_Q3_K>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_Q2_0>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_Q2_K>(const GemvArgs&, hipStream_t);
}  // namespace qm
