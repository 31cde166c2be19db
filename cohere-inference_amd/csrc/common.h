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

// round_bf in one instruction: the conversion packs bf16(0) below bf16(f), which is bf16(f)'s fp32 bit pattern (the
// same packing written in C becomes the conversion plus a byte permute). Only for an f that an ordinary VALU
// instruction wrote: the compiler puts no wait states before inline assembly, and reading a matrix instruction's
// result (or a transcendental's) that early gives stale values.
DEVI float round_bf_valu(float f) {
  float r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(f));
  return r;
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
DEVI uint32_t pack_bf2(float lo, float hi) {
  const v2bf v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// four values as int8, rint(clamp(f * inv, -127, 127)) each, packed low byte first, for inv = 1 / (m / 127) where m
// is at least the largest |f| of the values quantized with it: then |f * inv| <= 127 (1 + 4 ulp) < 127.5 and the
// clamp never acts. Adding 1.5 * 2^23 to the rounded product rounds it to an integer, half to even like rintf, and
// leaves that integer k in the low mantissa bits (0x4B400000 + k), so the sum's low byte is k's two's-complement
// byte; two byte permutes pack the four (selector byte 0x0c gives a zero byte).
DEVI uint32_t q8x4(float a, float b, float c, float d, float inv) {
  const uint32_t ba = __float_as_uint(a * inv + 12582912.f), bb = __float_as_uint(b * inv + 12582912.f),
                 bc = __float_as_uint(c * inv + 12582912.f), bd = __float_as_uint(d * inv + 12582912.f);
  return __builtin_amdgcn_perm(__builtin_amdgcn_perm(bd, bc, 0x0c0c0400u), __builtin_amdgcn_perm(bb, ba, 0x0c0c0400u),
                               0x05040100u);
}

// logistic for the activation epilogues (hardware exp and reciprocal); their results are rounded to bf16 or int8
// right after, far coarser than these approximations
DEVI float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// ---- wave helpers ----------------------------------------------------------------------------------------------------

DEVI int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
DEVI int lane_id() { return threadIdx.x & 63; }

// ---- cross-lane reductions on DPP lane moves (within rows of 16 lanes) and v_readlane, without the LDS round trip
// of a bpermute shuffle. Each gives the xor-butterfly reduction's result (v op= shfl_xor(v, 1), 2, 4, ...) bit for
// bit: every level combines the same two partial results, at most in commuted order.
constexpr int DPP_XOR1 = 0xB1;         // quad_perm(1, 0, 3, 2): lane ^ 1
constexpr int DPP_XOR2 = 0x4E;         // quad_perm(2, 3, 0, 1): lane ^ 2
constexpr int DPP_HALF_MIRROR = 0x141; // lane i of each 8 <- lane 7 - i (lane ^ 4 once quads are uniform)
constexpr int DPP_ROR4 = 0x124;        // row_ror:4, lane i of each 16 <- lane i - 4
constexpr int DPP_ROR8 = 0x128;        // row_ror:8
template <int CTRL>
DEVI float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
DEVI float lane_value(float v, int lane) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane)); }

// lane I of each aligned group of 8 lanes, in every lane of the group: a quad broadcast of lane I % 4, then the
// group's other quad takes it across the half mirror (bank mask: only that quad's lanes are written)
template <int I>
DEVI float group8_bcast_c(float v) {
  constexpr int k = I & 3;
  const int x = __builtin_amdgcn_update_dpp(0, __float_as_int(v), k | k << 2 | k << 4 | k << 6, 0xF, 0xF, false);
  return __int_as_float(__builtin_amdgcn_update_dpp(x, x, DPP_HALF_MIRROR, 0xF, I < 4 ? 0xA : 0x5, false));
}
// the same for an index that is a constant after unrolling
DEVI float group8_bcast(float v, int i) {
  switch (i) {
    case 0: return group8_bcast_c<0>(v);
    case 1: return group8_bcast_c<1>(v);
    case 2: return group8_bcast_c<2>(v);
    case 3: return group8_bcast_c<3>(v);
    case 4: return group8_bcast_c<4>(v);
    case 5: return group8_bcast_c<5>(v);
    case 6: return group8_bcast_c<6>(v);
    default: return group8_bcast_c<7>(v);
  }
}
// over each aligned group of 8 lanes, in every lane of the group
DEVI float group8_sum(float v) {
  v += dpp_mov<DPP_XOR1>(v);
  v += dpp_mov<DPP_XOR2>(v);
  return v + dpp_mov<DPP_HALF_MIRROR>(v);
}
DEVI float group8_max(float v) {
  v = fmaxf(v, dpp_mov<DPP_XOR1>(v));
  v = fmaxf(v, dpp_mov<DPP_XOR2>(v));
  return fmaxf(v, dpp_mov<DPP_HALF_MIRROR>(v));
}
// over each row of 16 lanes, in every lane of the row (the row's total in lane 15 is the butterfly's order)
DEVI float row16_sum(float v) {
  v += dpp_mov<DPP_XOR1>(v);
  v += dpp_mov<DPP_XOR2>(v);
  v += dpp_mov<DPP_ROR4>(v);
  return v + dpp_mov<DPP_ROR8>(v);
}
DEVI float row16_max(float v) {
  v = fmaxf(v, dpp_mov<DPP_XOR1>(v));
  v = fmaxf(v, dpp_mov<DPP_XOR2>(v));
  v = fmaxf(v, dpp_mov<DPP_ROR4>(v));
  return fmaxf(v, dpp_mov<DPP_ROR8>(v));
}
// over the 64 lanes (all active), the same value in every lane
DEVI float wave_sum64(float v) {
  v = row16_sum(v);
  return (lane_value(v, 15) + lane_value(v, 31)) + (lane_value(v, 47) + lane_value(v, 63));
}
DEVI float wave_max64(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 15), lane_value(v, 31)), fmaxf(lane_value(v, 47), lane_value(v, 63)));
}

// v combined with lane ^ 16's / lane ^ 32's value (gfx950 v_permlane16_swap / v_permlane32_swap: with both operands
// v, the two results hold, in every lane, its own and its partner's value), as v op shfl_xor(v, 16 / 32)
DEVI float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
DEVI float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
DEVI float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
DEVI float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// the same two maxima for non-negative values (not NaN): compared as unsigned bit patterns, whose order is theirs,
// which takes one integer maximum where fmaxf first quiets both operands
DEVI float xor16_max_pos(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0] > r[1] ? r[0] : r[1]);
}
DEVI float xor32_max_pos(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0] > r[1] ? r[0] : r[1]);
}

DEVI float wave_max_xor(float v, int width) {
  if (width == 64) return wave_max64(v);
  for (int o = 1; o < width; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// wait for this wave's outstanding vector-memory operations (incl. global -> LDS transfers)
DEVI void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// wait until at most n (0..15, a constant after unrolling) of the wave's vector memory operations are in flight
DEVI void wait_vm_upto(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
  }
}

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
