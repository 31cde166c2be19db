// Device and host helpers shared by the gfx950 kernels of the quantized-GEMM path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#define DEVI __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define LDS_AS __attribute__((address_space(3)))

// ---- bf16 (stored as uint16 bit patterns) ----------------------------------------------------------------------------

DEVI float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16, round to nearest even: gfx950's v_cvt_pk_bf16_f32
DEVI uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

DEVI float round_bf(float f) { return bf2f(f2bf(f)); }

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
DEVI uint32_t pack_bf2(float lo, float hi) {
  const v2bf v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// logistic for the activation epilogues (hardware exp and reciprocal); their results are rounded to bf16 or int8
// right after, far coarser than these approximations
DEVI float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// ---- wave helpers ----------------------------------------------------------------------------------------------------

DEVI int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
DEVI int lane_id() { return threadIdx.x & 63; }

DEVI float wave_max_xor(float v, int width) {
  for (int o = 1; o < width; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// wait for this wave's outstanding vector-memory operations (incl. global -> LDS transfers)
DEVI void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// workgroup barrier for LDS pipelines: this wave's LDS operations complete, then s_barrier. Unlike __syncthreads()
// it carries no memory fence, so the compiler does not drain the global -> LDS transfers still in flight for later
// stages (the caller waits for the ones it needs with an explicit vmcnt first).
DEVI void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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
