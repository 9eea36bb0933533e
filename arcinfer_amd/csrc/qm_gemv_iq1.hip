// Decode GEMV instantiations for IQ1_S, IQ1_M; the kernels are in qm_gemv_impl.h (one translation unit per pair of
// weight types, so the instantiations compile in parallel).
#include "qm_gemv_impl.h"

namespace qm {
template hipError_t gemv_dispatch<T_IQ1_S>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_IQ1_M>(const GemvArgs&, hipStream_t);
}  // namespace qm
