// Instantiations of the GEMM kernel template (gemm_q8.h) for bf16 operands: the reference's bf16 GEMM with fused
// epilogues (kernels/csrc/gemm.cu), used by the encoder's subsampling convolutions and projections.
#include "gemm_q8.h"

namespace cohere_gemm {

namespace {

template <int EPI>
bool tiles_bf16(int tile, const GemmArgs& p, hipStream_t s) {
  switch (tile) {
    case 0: launch_tile<128, 128, 2, 2, 4, 16, EPI, false, false, true>(p, s); return true;
    case 1: launch_tile<128, 256, 2, 2, 3, 16, EPI, false, false, true>(p, s); return true;
    case 3: launch_tile<64, 128, 2, 2, 4, 16, EPI, false, false, true>(p, s); return true;
    case 6: launch_tile<256, 256, 2, 4, 2, 16, EPI, false, false, true>(p, s); return true;
    case 7: launch_tile<64, 64, 2, 2, 4, 16, EPI, false, false, true>(p, s); return true;
    case 9: launch_tile<128, 256, 2, 4, 3, 16, EPI, false, false, true>(p, s); return true;
    default: return false;
  }
}

}  // namespace

bool launch_gemm_bf16(int tile, int epi, const GemmArgs& p, hipStream_t s) {
  switch (epi) {
    case EPI_BIAS: return tiles_bf16<EPI_BIAS>(tile, p, s);
    case EPI_SILU: return tiles_bf16<EPI_SILU>(tile, p, s);
    case EPI_RELU: return tiles_bf16<EPI_RELU>(tile, p, s);
    case EPI_RESID: return tiles_bf16<EPI_RESID>(tile, p, s);
    case EPI_GLU: return tiles_bf16<EPI_GLU>(tile, p, s);
    case EPI_CONV_RELU: return tiles_bf16<EPI_CONV_RELU>(tile, p, s);
    default: return false;
  }
}

}  // namespace cohere_gemm
