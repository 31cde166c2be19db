// Device and host helpers shared by the gfx950 kernels of the quantized-GEMM path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#define DEVI __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define LDS_AS __attribute__((address_space(3)))

// ---- bf16 (stored as uint16 bit patterns) ----------------------------------------------------------------------------

DEVI float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16, round to nearest even (NaN kept quiet)
DEVI uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

DEVI float round_bf(float f) { return bf2f(f2bf(f)); }

DEVI uint32_t pack_bf2(float lo, float hi) { return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16); }

// logistic for the activation epilogues; their results are rounded to bf16 or int8 right after
DEVI float sigmoid_fast(float x) { return 1.f / (1.f + __expf(-x)); }

// ---- wave helpers ----------------------------------------------------------------------------------------------------

DEVI int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
DEVI int lane_id() { return threadIdx.x & 63; }

DEVI float wave_max_xor(float v, int width) {
  for (int o = 1; o < width; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// wait for this wave's outstanding vector-memory operations (incl. global -> LDS transfers)
DEVI void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- C-ABI error reporting -------------------------------------------------------------------------------------------

namespace cohere {
void set_error(const std::string& msg);
void clear_error();
// after a launch: records hipGetLastError(); returns 0 or -1
int check_launch(const char* what);
}  // namespace cohere

#define COHERE_REQUIRE(cond, msg)                \
  do {                                           \
    if (!(cond)) {                               \
      ::cohere::set_error(std::string(msg));     \
      return 1;                                  \
    }                                            \
  } while (0)
