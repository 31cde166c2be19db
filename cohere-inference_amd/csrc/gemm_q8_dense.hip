// Instantiations of the int8 GEMM kernel template (gemm_q8.h) for the dense weights.
#include "gemm_q8.h"

namespace cohere_gemm {

template <>
bool launch_gemm<false>(int tile, int epi, bool grouped, const GemmArgs& p, hipStream_t s) {
  if (grouped) {
    switch (epi) {
      case EPI_BIAS: return launch_tiles<false, EPI_BIAS, true>(tile, p, s);
      case EPI_RESID: return launch_tiles<false, EPI_RESID, true>(tile, p, s);
      case EPI_GLU: return launch_tiles<false, EPI_GLU, true>(tile, p, s);
      case EPI_SILU_Q8: return launch_tiles<false, EPI_SILU_Q8, true>(tile, p, s);
      default: return false;
    }
  }
  switch (epi) {
    case EPI_BIAS: return launch_tiles<false, EPI_BIAS, false>(tile, p, s);
    case EPI_RESID: return launch_tiles<false, EPI_RESID, false>(tile, p, s);
    case EPI_GLU: return launch_tiles<false, EPI_GLU, false>(tile, p, s);
    case EPI_SILU_Q8: return launch_tiles<false, EPI_SILU_Q8, false>(tile, p, s);
    case EPI_I32: return launch_tiles<false, EPI_I32, false>(tile, p, s);
    default: return false;
  }
}

}  // namespace cohere_gemm
