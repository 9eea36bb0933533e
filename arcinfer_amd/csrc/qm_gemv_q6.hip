// Decode GEMV instantiations for Q6_K, IQ4_NL; the kernels are in qm_gemv_impl.h (one translation unit per pair of
// weight types, so the instantiations compile in parallel).
#include "qm_gemv_impl.h"

namespace qm {
template hipError_t gemv_dispatch<T_Q6_K>(const GemvArgs&, hipStream_t);
template hipError_t gemv_dispatch<T_IQ4_NL>(const GemvArgs&, hipStream_t);
}  // namespace qm
