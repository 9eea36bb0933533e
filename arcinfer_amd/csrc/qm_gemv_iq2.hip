// Decode GEMV instantiations for IQ2_XXS, IQ2_XS; the kernels are in qm_gemv_impl.h (one translation unit per pair of
// weight types, so the instantiations compile in parallel).
#include "qm_gemv_impl.h"

namespace qm {
template hipError_t gemv_dispatch<T_IQ2_XXS>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_IQ2_XS>(const GemvArgs&, hipStream_t);
}  // namespace qm
