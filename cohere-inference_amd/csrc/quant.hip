// Producers of the int8 GEMM inputs: per-row activation quantization (reference kernels/csrc/encoder_ops.cu:18-54
// store_q8 / quantize_rows) and LayerNorm(s) with int8 or bf16 output (encoder_ops.cu:57-79, 501-543;
// layernorm.cuh:6-43).
//
// One wave per row; each lane holds up to VEC 8-element chunks of the row in registers (16-byte loads), so a row is
// read once and written once. The quantization arithmetic is the reference's: mx = max|bf16 x|, s = mx > 0 ?
// mx / 127 : 1, inv = 1 / s (both correctly rounded fp32 divisions), q = rint_half_even(clamp(x * inv, +-127)).
#include "cohere_hip.h"
#include "common.h"
#include "rows.h"

#include <string>

namespace {

using namespace cohere_rows;

template <int VEC>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                            int8_t* __restrict__ q, int64_t ldq, float* __restrict__ s,
                                                            int rows, int cols) {
  const int row = blockIdx.x * 4 + wave_id(), lane = lane_id();
  if (row >= rows) return;
  Row<VEC> r;
  load_row<VEC>(x + (int64_t)row * ldx, cols, lane, r);
  store_q8<VEC>(r, cols, lane, q + (int64_t)row * ldq, s + row);
}

// h = LN(x); with TWO, x = LN1(x) in place and h = LN2(x). Q8: h as int8 hq with one scale per row in hs;
// otherwise h bf16 (h may be x itself: the row is in registers before anything is stored)
template <int VEC, bool TWO, bool Q8>
__global__ void __launch_bounds__(256) layernorm_kernel(uint16_t* x, int64_t ldx, const uint16_t* w1,
                                                        const uint16_t* b1, float eps1, const uint16_t* w2,
                                                        const uint16_t* b2, float eps2, int8_t* hq, int64_t ldq,
                                                        float* hs, uint16_t* h, int64_t ldh, int rows, int cols) {
  const int row = blockIdx.x * 4 + wave_id(), lane = lane_id();
  if (row >= rows) return;
  const LnParams<VEC> p1 = load_ln<VEC>(w1, b1, cols, lane);
  LnParams<VEC> p2;
  if constexpr (TWO) p2 = load_ln<VEC>(w2, b2, cols, lane);
  Row<VEC> r;
  uint16_t* xr = x + (int64_t)row * ldx;
  load_row<VEC>(xr, cols, lane, r);
  ln_row<VEC>(r, cols, lane, p1, eps1);
  if constexpr (TWO) {
    store_row<VEC>(r, cols, lane, xr);
    ln_row<VEC>(r, cols, lane, p2, eps2);
  }
  if constexpr (Q8)
    store_q8<VEC>(r, cols, lane, hq + (int64_t)row * ldq, hs + row);
  else
    store_row<VEC>(r, cols, lane, h + (int64_t)row * ldh);
}

template <bool Q8>
void launch_layernorm(int vec, bool two, int grid, hipStream_t st, uint16_t* x, int64_t ldx, const uint16_t* w1,
                      const uint16_t* b1, float eps1, const uint16_t* w2, const uint16_t* b2, float eps2, int8_t* hq,
                      int64_t ldq, float* hs, uint16_t* h, int64_t ldh, int rows, int cols) {
#define LNK(V, T) \
  layernorm_kernel<V, T, Q8><<<grid, 256, 0, st>>>(x, ldx, w1, b1, eps1, w2, b2, eps2, hq, ldq, hs, h, ldh, rows, cols)
  switch (vec) {
    case 1: if (two) LNK(1, true); else LNK(1, false); break;
    case 2: if (two) LNK(2, true); else LNK(2, false); break;
    case 3: if (two) LNK(3, true); else LNK(3, false); break;
    default: if (two) LNK(4, true); else LNK(4, false); break;
  }
#undef LNK
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

extern "C" int cohere_quantize_rows(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* s, int64_t rows,
                                    int64_t cols, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 8192,
                 "quantize_rows: cols must be a multiple of 8, at most 8192");
  COHERE_REQUIRE(x && q && s && al16(x) && ldx % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0 && ldq % 8 == 0,
                 "quantize_rows: rows must be aligned");
  if (rows == 0) return 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int grid = (int)((rows + 3) / 4), vec = (int)((cols + 511) / 512);
#define QR(V) quantize_rows_kernel<V><<<grid, 256, 0, st>>>(x, ldx, q, ldq, s, (int)rows, (int)cols)
  if (vec <= 1) QR(1);
  else if (vec <= 2) QR(2);
  else if (vec <= 3) QR(3);
  else if (vec <= 4) QR(4);
  else if (vec <= 8) QR(8);
  else if (vec <= 10) QR(10);
  else QR(16);
#undef QR
  return cohere::check_launch("quantize_rows");
}

extern "C" int cohere_layernorm_q8(uint16_t* x, int64_t ldx, const uint16_t* w1, const uint16_t* b1, float eps1,
                                   const uint16_t* w2, const uint16_t* b2, float eps2, int8_t* hq, int64_t ldq,
                                   float* hs, int64_t rows, int64_t cols, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 2048,
                 "layernorm_q8: cols must be a multiple of 8, at most 2048");
  COHERE_REQUIRE(x && w1 && b1 && hq && hs && al16(x) && ldx % 8 == 0 && al16(w1) && al16(b1) &&
                     (reinterpret_cast<uintptr_t>(hq) & 7) == 0 && ldq % 8 == 0,
                 "layernorm_q8: rows must be aligned");
  COHERE_REQUIRE(!w2 || (b2 && al16(w2) && al16(b2)), "layernorm_q8: second LayerNorm needs aligned w2 and b2");
  if (rows == 0) return 0;
  launch_layernorm<true>((int)((cols + 511) / 512), w2 != nullptr, (int)((rows + 3) / 4),
                         reinterpret_cast<hipStream_t>(stream), x, ldx, w1, b1, eps1, w2, b2, eps2, hq, ldq, hs,
                         nullptr, 0, (int)rows, (int)cols);
  return cohere::check_launch("layernorm_q8");
}

extern "C" int cohere_layernorm(uint16_t* x, int64_t ldx, const uint16_t* w1, const uint16_t* b1, float eps1,
                                const uint16_t* w2, const uint16_t* b2, float eps2, uint16_t* h, int64_t ldh,
                                int64_t rows, int64_t cols, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 2048,
                 "layernorm: cols must be a multiple of 8, at most 2048");
  COHERE_REQUIRE(x && w1 && b1 && h && al16(x) && ldx % 8 == 0 && al16(w1) && al16(b1) && al16(h) && ldh % 8 == 0,
                 "layernorm: rows must be aligned");
  COHERE_REQUIRE(!w2 || (b2 && al16(w2) && al16(b2)), "layernorm: second LayerNorm needs aligned w2 and b2");
  if (rows == 0) return 0;
  launch_layernorm<false>((int)((cols + 511) / 512), w2 != nullptr, (int)((rows + 3) / 4),
                          reinterpret_cast<hipStream_t>(stream), x, ldx, w1, b1, eps1, w2, b2, eps2, nullptr, 0,
                          nullptr, h, ldh, (int)rows, (int)cols);
  return cohere::check_launch("layernorm");
}
