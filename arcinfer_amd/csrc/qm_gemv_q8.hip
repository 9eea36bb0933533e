// Decode GEMV instantiations for Q8_0, Q4_0; the kernels are in qm_gemv_impl.h (one translation unit per pair of
// weight types, so the instantiations compile in parallel).
#include "qm_gemv_impl.h"

namespace qm {
template hipError_t gemv_dispatch<T_Q8_0>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_Q4_0>(const GemvArgs&, hipStream_t);
}  // namespace qm
