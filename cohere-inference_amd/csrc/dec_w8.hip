// Skinny decoder projections (M <= 64 rows) for gfx950: W8A16 (int8 weights widened to bf16 in registers, the
// reference's dec_w8_linear, kernels/csrc/dec_w8.cu) and plain bf16 weights (the reference's Triton/cuBLAS `linear`,
// kernels/decoder_kernels.py), both on v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
//
// These GEMMs read each weight byte once and do little arithmetic per byte: they are bound by HBM. The design keeps
// as many weight bytes in flight as the register file allows and streams them straight into registers (no LDS):
//  * A workgroup owns 64 output channels (4 strips of 16) and a K slice; its 4 waves take interleaved 64-wide K
//    blocks of the slice. Every lane issues all its weight loads (16 bytes each) before the first MFMA.
//  * The MFMA A operand is the weight strip (16 channels), B the activations (16 rows): a lane holds 4 consecutive
//    channels of one row in the result. One activation fragment serves the 4 strips.
//  * int8 weights arrive in prepare_w8's layout (uint8 = int8 + 128, bytes of every 16 K permuted so that physical
//    bytes 0-7 hold logical K {0,1,8,9,2,3,10,11} and 8-15 hold {4,5,12,13,6,7,14,15}). A lane's 16 weight bytes feed
//    two MFMAs; the activation pairs for the same logical K are picked from the 32 contiguous bytes the lane loads,
//    so the layout is consumed as the reference stores it. Widening: (float)u8 - 128 is exact, and so is its bf16
//    (an integer of at most 8 significant bits).
//  * The 4 waves' partial tiles are summed through LDS in wave order; with several K slices (gridDim.y) each
//    workgroup writes its partial to the caller's workspace and the last one to finish (an atomic counter per
//    channel tile) adds the slices in slice order and resets the counter, so the kernel replays in HIP graphs and the
//    result does not depend on timing.
#include "common.h"
#include "cohere_hip.h"

#include <string>

namespace {

struct SkinnyArgs {
  const uint16_t* X;  // [M, K] bf16
  const void* W;      // uint8 [N, K] (prepare_w8) or bf16 [N, K]
  const float* sw;    // [N] (int8 weights only)
  const uint16_t* bias;
  uint16_t* Y;        // [M, N]
  float* ws;          // [N/64, S, 64 rows, 64 cols] partials
  int32_t* counters;  // [N/64]
  int64_t ldx, ldy;
  int M, N, K;
  int ks;             // K per slice (multiple of 256)
  int relu;
};

constexpr int BNC = 64;        // channels per workgroup
constexpr int STRIPS = 4;      // 16-channel strips per wave
constexpr int KB = 64;         // K per block

// 8 weight bytes (offset uint8) -> 8 bf16
DEVI v8bf widen8(uint32_t lo, uint32_t hi) {
  v8bf r;
  const uint32_t w[2] = {lo, hi};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float f = (float)((w[d] >> (8 * b)) & 0xffu) - 128.f;
      r[d * 4 + b] = __builtin_bit_cast(__bf16, (uint16_t)(__float_as_uint(f) >> 16));
    }
  }
  return r;
}

DEVI v8bf as_bf8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const v4i v = v4i{(int)a, (int)b, (int)c, (int)d};
  return __builtin_bit_cast(v8bf, v);
}

template <int MB, bool W8, bool RELU>
__global__ void __launch_bounds__(256) skinny_kernel(const SkinnyArgs p) {
  constexpr int MAXB = W8 ? 4 : 2;  // K blocks per wave held in registers at once (64 VGPRs of weights)
  __shared__ __attribute__((aligned(16))) float red[4][MB * 16][BNC + 4];
  const int tile = blockIdx.x, split = blockIdx.y, nsplit = gridDim.y;
  const int n0 = tile * BNC;
  const int lane = threadIdx.x & 63, wave = wave_id(), h = lane >> 4, c16 = lane & 15;
  const int64_t kbase = (int64_t)split * p.ks;
  const int nkb = p.ks / KB;  // blocks in the slice; wave w takes w, w+4, ...

  v4f acc[STRIPS][MB];
#pragma unroll
  for (int s = 0; s < STRIPS; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[s][mb] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int b0 = wave; b0 < nkb; b0 += 4 * MAXB) {
    // all of this round's weight loads first
    uint4 wreg[MAXB][STRIPS][W8 ? 1 : 2];
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      const int kb = b0 + 4 * b;
      if (kb < nkb) {
        const int64_t k = kbase + (int64_t)kb * KB;
#pragma unroll
        for (int s = 0; s < STRIPS; ++s) {
          const int64_t n = n0 + s * 16 + c16;
          if constexpr (W8) {
            wreg[b][s][0] = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.W) + n * p.K + k + 16 * h);
          } else {
            const uint16_t* wr = static_cast<const uint16_t*>(p.W) + n * p.K + k;
            wreg[b][s][0] = *reinterpret_cast<const uint4*>(wr + 8 * h);
            wreg[b][s][1] = *reinterpret_cast<const uint4*>(wr + 32 + 8 * h);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      const int kb = b0 + 4 * b;
      if (kb >= nkb) break;
      const int64_t k = kbase + (int64_t)kb * KB;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = min(mb * 16 + c16, p.M - 1);
        const uint16_t* xr = p.X + (int64_t)m * p.ldx + k;
        v8bf x0, x1;
        if constexpr (W8) {
          const uint4 lo = *reinterpret_cast<const uint4*>(xr + 16 * h);      // logical 0..7 of this 16-block
          const uint4 hi = *reinterpret_cast<const uint4*>(xr + 16 * h + 8);  // logical 8..15
          x0 = as_bf8(lo.x, hi.x, lo.y, hi.y);  // pairs (0,1) (8,9) (2,3) (10,11)
          x1 = as_bf8(lo.z, hi.z, lo.w, hi.w);  // pairs (4,5) (12,13) (6,7) (14,15)
        } else {
          const uint4 a = *reinterpret_cast<const uint4*>(xr + 8 * h);
          const uint4 c = *reinterpret_cast<const uint4*>(xr + 32 + 8 * h);
          x0 = as_bf8(a.x, a.y, a.z, a.w);
          x1 = as_bf8(c.x, c.y, c.z, c.w);
        }
#pragma unroll
        for (int s = 0; s < STRIPS; ++s) {
          v8bf w0, w1;
          if constexpr (W8) {
            w0 = widen8(wreg[b][s][0].x, wreg[b][s][0].y);
            w1 = widen8(wreg[b][s][0].z, wreg[b][s][0].w);
          } else {
            const uint4 a = wreg[b][s][0], c = wreg[b][s][1];
            w0 = as_bf8(a.x, a.y, a.z, a.w);
            w1 = as_bf8(c.x, c.y, c.z, c.w);
          }
          acc[s][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, x0, acc[s][mb], 0, 0, 0);
          acc[s][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, x1, acc[s][mb], 0, 0, 0);
        }
      }
    }
  }

  // the waves' partial tiles, summed in wave order
#pragma unroll
  for (int s = 0; s < STRIPS; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][mb * 16 + c16][s * 16 + h * 4 + r] = acc[s][mb][r];
  __syncthreads();
  constexpr int ROWS = MB * 16;
  const int tid = threadIdx.x;
  auto finish = [&](int m, int c, float v) {
    const int n = n0 + c;
    if constexpr (W8) v = __builtin_fmaf(v, p.sw[n], p.bias ? bf2f(p.bias[n]) : 0.f);
    else if (p.bias) v = v + bf2f(p.bias[n]);
    if (RELU) v = fmaxf(v, 0.f);
    p.Y[(int64_t)m * p.ldy + n] = f2bf(v);
  };
  if (nsplit == 1) {
    for (int i = tid; i < p.M * BNC; i += 256) {
      const int m = i / BNC, c = i % BNC;
      finish(m, c, ((red[0][m][c] + red[1][m][c]) + red[2][m][c]) + red[3][m][c]);
    }
    return;
  }
  float* part = p.ws + ((int64_t)tile * nsplit + split) * (64 * BNC);
  for (int i = tid; i < ROWS * BNC; i += 256) {
    const int m = i / BNC, c = i % BNC;
    part[i] = ((red[0][m][c] + red[1][m][c]) + red[2][m][c]) + red[3][m][c];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  __shared__ int last;
  if (tid == 0) last = atomicAdd(p.counters + tile, 1) == nsplit - 1;
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const float* base = p.ws + (int64_t)tile * nsplit * (64 * BNC);
  for (int i = tid; i < p.M * BNC; i += 256) {
    float v = 0.f;
    for (int s = 0; s < nsplit; ++s) v += base[(int64_t)s * 64 * BNC + i];
    finish(i / BNC, i % BNC, v);
  }
  if (tid == 0) atomicExch(p.counters + tile, 0);
}

template <bool W8, bool RELU>
void launch_rows(const SkinnyArgs& p, int splits, hipStream_t s) {
  const dim3 grid(p.N / BNC, splits);
  switch ((p.M + 15) / 16) {
    case 1: skinny_kernel<1, W8, RELU><<<grid, 256, 0, s>>>(p); break;
    case 2: skinny_kernel<2, W8, RELU><<<grid, 256, 0, s>>>(p); break;
    case 3: skinny_kernel<3, W8, RELU><<<grid, 256, 0, s>>>(p); break;
    default: skinny_kernel<4, W8, RELU><<<grid, 256, 0, s>>>(p); break;
  }
}

// K slices: enough workgroups to cover the CUs, each slice at least 256 K (one block per wave)
int choose_splits(int N, int K, int64_t ws_len, int64_t counters_len) {
  const int tiles = N / BNC;
  int s = 1;
  while (tiles * s < 256 && K % (256 * s * 2) == 0 && s < 16) s *= 2;
  while (s > 1 && ((int64_t)tiles * s * 64 * BNC > ws_len || counters_len < tiles)) s /= 2;
  return s;
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

int skinny_entry(SkinnyArgs& p, bool w8, int64_t ws_len, int64_t counters_len, hipStream_t s, const char* name) {
  const std::string nm(name);
  COHERE_REQUIRE(p.M >= 0 && p.M <= 64, nm + ": at most 64 rows per call (got " + std::to_string(p.M) + ")");
  COHERE_REQUIRE(p.N > 0 && p.N % BNC == 0, nm + ": N must be a multiple of 64");
  COHERE_REQUIRE(p.K > 0 && p.K % 256 == 0, nm + ": K must be a multiple of 256");
  COHERE_REQUIRE(p.X && p.W && p.Y && (!w8 || p.sw), nm + ": null pointer");
  COHERE_REQUIRE(al16(p.X) && p.ldx % 8 == 0 && al16(p.W), nm + ": x rows and weights must be 16-byte aligned");
  if (p.M == 0) return 0;
  const int splits = choose_splits(p.N, p.K, p.ws ? ws_len : 0, p.counters ? counters_len : 0);
  p.ks = p.K / splits;
  if (w8) p.relu ? launch_rows<true, true>(p, splits, s) : launch_rows<true, false>(p, splits, s);
  else p.relu ? launch_rows<false, true>(p, splits, s) : launch_rows<false, false>(p, splits, s);
  return cohere::check_launch(name);
}

}  // namespace

extern "C" int cohere_dec_w8_linear(const uint16_t* x, int64_t ldx, const uint8_t* w, const float* sw,
                                    const uint16_t* bias, uint16_t* y, int64_t ldy, int32_t relu, int64_t bn,
                                    int64_t splits, float* ws, int64_t ws_len, int32_t* counters, int64_t counters_len,
                                    int64_t M, int64_t N, int64_t K, void* stream) {
  cohere::clear_error();
  // the reference's knobs, checked as it checks them (dec_w8.cu:210-213); the gfx950 kernel picks its own tiling
  COHERE_REQUIRE((bn == 16 || bn == 32 || bn == 64) && N % bn == 0 && splits >= 1 && splits <= 16 &&
                     K % (128 * splits) == 0,
                 "dec_w8_linear: shape (" + std::to_string(N) + ", " + std::to_string(K) + "), bn " +
                     std::to_string(bn) + ", splits " + std::to_string(splits));
  COHERE_REQUIRE(splits == 1 || (ws && ws_len >= (N / bn) * splits * 64 * bn && counters && counters_len >= N / bn),
                 "dec_w8_linear: workspace or counters too small");
  SkinnyArgs p{};
  p.X = x; p.W = w; p.sw = sw; p.bias = bias; p.Y = y; p.ws = ws; p.counters = counters;
  p.ldx = ldx; p.ldy = ldy; p.M = (int)M; p.N = (int)N; p.K = (int)K; p.relu = relu;
  return skinny_entry(p, true, ws_len, counters_len, reinterpret_cast<hipStream_t>(stream), "dec_w8_linear");
}

extern "C" int cohere_linear_bf16(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* bias,
                                  uint16_t* y, int64_t ldy, int32_t relu, int64_t M, int64_t N, int64_t K,
                                  void* stream) {
  cohere::clear_error();
  SkinnyArgs p{};
  p.X = x; p.W = w; p.sw = nullptr; p.bias = bias; p.Y = y; p.ws = nullptr; p.counters = nullptr;
  p.ldx = ldx; p.ldy = ldy; p.M = (int)M; p.N = (int)N; p.K = (int)K; p.relu = relu;
  return skinny_entry(p, false, 0, 0, reinterpret_cast<hipStream_t>(stream), "linear_bf16");
}
