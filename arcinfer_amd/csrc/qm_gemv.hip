// Decode GEMV entry: routes a weight type to its instantiation (qm_gemv_*.hip; kernels in qm_gemv_impl.h).
#include "qm_launch.h"

namespace qm {

template <int TYPE> hipError_t gemv_dispatch(const GemvArgs& a, hipStream_t s);

hipError_t launch_gemv(int type, const GemvArgs& a, hipStream_t s) {
  switch (type) {
    case T_Q8_0: return gemv_dispatch<T_Q8_0>(a, s);
    case T_Q4_K: return gemv_dispatch<T_Q4_K>(a, s);
    case T_IQ4_XS: return gemv_dispatch<T_IQ4_XS>(a, s);
    case T_IQ3_S: return gemv_dispatch<T_IQ3_S>(a, s);
    case T_Q6_K: return gemv_dispatch<T_Q6_K>(a, s);
    case T_Q5_K: return gemv_dispatch<T_Q5_K>(a, s);
    case T_Q4_0: return gemv_dispatch<T_Q4_0>(a, s);
    case T_IQ4_NL: return gemv_dispatch<T_IQ4_NL>(a, s);
    case T_IQ2_XXS: return gemv_dispatch<T_IQ2_XXS>(a, s);
    case T_IQ2_XS: return gemv_dispatch<T_IQ2_XS>(a, s);
    case T_IQ2_S: return gemv_dispatch<T_IQ2_S>(a, s);
    case T_IQ3_XXS: return gemv_dispatch<T_IQ3_XXS>(a, s);
    case T_Q3_K: return gemv_dispatch<T_Q3_K>(a, s);
    case T_Q2_0: return gemv_dispatch<T_Q2_0>(a, s);
    case T_Q2_K: return gemv_dispatch<T_Q2_K>(a, s);
    case T_IQ1_S: return gemv_dispatch<T_IQ1_S>(a, s);
    case T_IQ1_M: return gemv_dispatch<T_IQ1_M>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm
