// Decode GEMV instantiations for Q4_K, Q5_K; the kernels are in qm_gemv_impl.h (one translation unit per pair of
// weight types, so the instantiations compile in parallel).
#include "qm_gemv_impl.h"

namespace qm {
template hipError_t gemv_dispatch<T_Q4_K>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_Q5_K>(const GemvArgs&, hipStream_t);
}  // namespace qm
