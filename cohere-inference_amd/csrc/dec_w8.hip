// Skinny decoder projections (M <= 64 rows) for gfx950: W8A16 (int8 weights widened to bf16 in registers, the
// reference's dec_w8_linear, kernels/csrc/dec_w8.cu) and plain bf16 weights (the reference's Triton/cuBLAS `linear`,
// kernels/decoder_kernels.py), both on v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
//
// These GEMMs read each weight byte once and do little arithmetic per byte: they are bound by HBM. The design keeps
// as many weight bytes in flight as the register file allows and streams them straight into registers (no LDS):
//  * A workgroup owns NS strips of 16 output channels and the whole K range; its NW waves (4-16) take interleaved
//    64-wide K blocks. Every lane issues its weight loads (16 bytes each, up to 64 VGPRs' worth) before the first
//    MFMA, so a 1024-thread workgroup keeps up to 256 KB of weights in flight.
//  * The MFMA A operand is the weight strip (16 channels), B the activations (16 rows): a lane holds 4 consecutive
//    channels of one row in the result. One activation fragment serves the NS strips.
//  * int8 weights arrive in prepare_w8's layout (uint8 = int8 + 128, bytes of every 16 K permuted so that physical
//    bytes 0-7 hold logical K {0,1,8,9,2,3,10,11} and 8-15 hold {4,5,12,13,6,7,14,15}). A lane's 16 weight bytes feed
//    two MFMAs; the activation pairs for the same logical K are picked from the 32 contiguous bytes the lane loads,
//    so the layout is consumed as the reference stores it. Widening: (float)u8 - 128 is exact, and so is its bf16
//    (an integer of at most 8 significant bits).
//  * K is reduced inside the workgroup: the waves' partial tiles go to LDS and are summed in wave order. There is no
//    cross-workgroup split-K: on MI355X each XCD has its own L2, so publishing partial sums across workgroups needs an
//    agent-scope release/acquire that writes back and invalidates L2 -- far costlier than these GEMMs. The result is
//    deterministic and the kernel is graph-replayable with no state; the reference's workspace and counters are
//    accepted (and checked as it checks them) but not needed.
//  * Fused forms for the decoder step (cohere_dec_linear_fused): a LayerNorm prologue (each wave normalises rows of
//    the workgroup's block with dec_add_ln's arithmetic into LDS, and the K loop reads the activations there) and a
//    residual epilogue (y = bf16(y + bf16(result)), dec_add_ln's sum, in place). Folding the step's residual
//    LayerNorms into the projections this way gives the same bits as the separate launches.
#include "common.h"
#include "cohere_hip.h"
#include "rows.h"

#include <string>

namespace {

struct SkinnyArgs {
  const uint16_t* X;  // [M, K] bf16 (with a LayerNorm prologue: the residual stream before the norm)
  const void* W;      // uint8 [N, K] (prepare_w8) or bf16 [N, K]
  const float* sw;    // [N] (int8 weights only)
  const uint16_t* bias;
  uint16_t* Y;        // [M, N] (residual epilogue: read and updated in place)
  const uint16_t* lnw;  // LayerNorm prologue weight and bias [K] (null: X is the GEMM input as it is)
  const uint16_t* lnb;
  float eps;
  int64_t ldx, ldy;
  int M, N, K;
};

// epilogues
enum { EP_NONE = 0, EP_RELU = 1, EP_RESID = 2 };
constexpr int LN_K = 1024;           // widest LayerNorm prologue (the rows are held in LDS)
constexpr int LN_ROW = LN_K * 2 + 16;  // LDS bytes per normalised row (16 bytes of padding: conflict-free reads)


constexpr int KB = 64;  // K per block

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

// MB row blocks of 16, NS strips of 16 channels, NW waves; EP the epilogue; LN: the rows are LayerNormed first (one
// wave per row, the same arithmetic as dec_add_ln) into LDS, and the K loop reads its activations from there.
// RB < 16 (with MB == 1): the workgroup takes RB rows only; the matrix instruction's 16 activation columns repeat
// them (lanes 16 apart load the same addresses, so no extra bytes are fetched) and the repeats are not written.
// BPW > 0: K holds exactly NW * BPW blocks, so every wave's loads are unconditional: without a LayerNorm the
// activations (L2 hits, written by the previous launch) are issued first, then the weights (from HBM), so that waiting
// for a block's activations never waits for weights (loads complete in order), and each matrix instruction waits for
// its own block's weights only. (Conditional loads made the compiler wait for all weights at the branches' join and
// then fetch each block's activations as a round trip of its own.)
template <int MB, int NS, int NW, bool W8, int EP, bool LN, int RB = 16, int BPW = 0>
__global__ void __launch_bounds__(NW * 64) skinny_kernel(const SkinnyArgs p) {
  static_assert(RB == 16 || (MB == 1 && (RB == 8 || RB == 4)), "row block");
  constexpr int ROWS = RB == 16 ? MB * 16 : RB;  // rows per workgroup
  constexpr int MAXB = BPW > 0 ? BPW : (W8 ? 16 : 8) / NS;  // K blocks per wave in registers at once (<= 64 VGPRs)
  static_assert(BPW == 0 || BPW * NS * (W8 ? 1 : 2) <= 16, "weight registers");
  constexpr bool XPRE = BPW > 0 && !LN;  // the activations loaded ahead of the weights
  constexpr bool FULLROW = LN && BPW * NW * KB == LN_K;  // K is the LayerNorm's full 1024: unguarded row loads
  constexpr int COLS = NS * 16, LDR = COLS + 4;
  constexpr int RED = NW * MB * 16 * LDR * 4, XS = LN ? ROWS * LN_ROW : 0;
  // the waves' partial tiles (after the K loop) share LDS with the normalised rows (during it)
  __shared__ __attribute__((aligned(16))) char smem[RED > XS ? RED : XS];
  auto red = reinterpret_cast<float (*)[MB * 16][LDR]>(smem);
  const int n0 = blockIdx.x * COLS, m_base = blockIdx.y * ROWS;  // grid.y > 1: the rows split over workgroups
  const int lane = threadIdx.x & 63, wave = wave_id(), h = lane >> 4, c16 = lane & 15;
  const int xrow = c16 & (RB - 1);  // the activation row of this lane's matrix column
  const int nkb = p.K / KB;  // wave w takes blocks w, w + NW, ...

  v4f acc[NS][MB];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[s][mb] = v4f{0.f, 0.f, 0.f, 0.f};
  // the epilogue's channel scale and bias: a thread always writes channel n0 + tid % COLS (COLS divides the thread
  // count), so both are loaded now, with the weights, not after the reduction (the bias load is unconditional -- from
  // the weights when there is no bias, the value then unused: a load under a branch is waited for at the join)
  static_assert((NW * 64) % COLS == 0, "epilogue channel per thread");
  const int n_ep = n0 + (int)(threadIdx.x % COLS);
  const float sw_ep = W8 ? p.sw[n_ep] : 1.f;
  const uint16_t* bsrc = p.bias ? p.bias : static_cast<const uint16_t*>(p.W);
  const uint16_t b_ep = bsrc[n_ep];

  // LayerNorm prologue: each wave's rows (two loaded before the weights, so that only they are waited for ahead of
  // the weights; the rest, with MB > 1, after)
  constexpr int RPW = LN ? ROWS / NW : 1, PRE = RPW < 2 ? RPW : 2;
  static_assert(!LN || (ROWS % NW == 0 && RPW >= 1), "rows per wave");
  cohere_rows::Row<2> rows_pre[PRE];
  cohere_rows::LnParams<2> lnp;
  if constexpr (LN) {
    lnp = cohere_rows::load_ln<2, FULLROW>(p.lnw, p.lnb, p.K, lane);
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
      const int m = min(m_base + wave * RPW + j, p.M - 1);
      cohere_rows::load_row<2, FULLROW>(p.X + (int64_t)m * p.ldx, p.K, lane, rows_pre[j]);
    }
  }

  bool first = true;
  for (int b0 = wave; b0 < nkb; b0 += NW * MAXB) {
    uint4 wreg[MAXB][NS][W8 ? 1 : 2];
    uint4 xreg[XPRE ? MAXB : 1][XPRE ? MB : 1][2];
    if constexpr (XPRE) {
#pragma unroll
      for (int b = 0; b < MAXB; ++b) {
        const int64_t k = (int64_t)(b0 + NW * b) * KB;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const uint16_t* xr = p.X + (int64_t)min(m_base + mb * 16 + xrow, p.M - 1) * p.ldx + k;
          xreg[b][mb][0] = *reinterpret_cast<const uint4*>(xr + (W8 ? 16 * h : 8 * h));
          xreg[b][mb][1] = *reinterpret_cast<const uint4*>(xr + (W8 ? 16 * h + 8 : 32 + 8 * h));
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // the activations' loads stay ahead of the weights'
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      const int kb = b0 + NW * b;
      if (BPW > 0 || kb < nkb) {
        const int64_t k = (int64_t)kb * KB;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
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
    if constexpr (BPW > 0) __builtin_amdgcn_sched_barrier(0);  // every load issued before the first product
    if constexpr (LN) {
      if (first) {
        // every wave reaches this (the caller guarantees at least NW blocks of K)
        // rows_pre is a ring of PRE rows in flight: row j + PRE is issued before row j is normalised, so with more
        // rows than PRE per wave their loads overlap the LayerNorms instead of each waiting a round trip of its own
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
          cohere_rows::Row<2> r = rows_pre[j % PRE];
          if (j + PRE < RPW) {
            const int m = min(m_base + wave * RPW + j + PRE, p.M - 1);
            cohere_rows::load_row<2, FULLROW>(p.X + (int64_t)m * p.ldx, p.K, lane, rows_pre[j % PRE]);
          }
          cohere_rows::ln_row<2>(r, p.K, lane, lnp, p.eps);
          cohere_rows::store_row<2>(r, p.K, lane, reinterpret_cast<uint16_t*>(smem + (wave * RPW + j) * LN_ROW));
        }
        __syncthreads();
        first = false;
      }
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      const int kb = b0 + NW * b;
      if (BPW == 0 && kb >= nkb) break;
      const int64_t k = (int64_t)kb * KB;
      v8bf w0[NS], w1[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if constexpr (W8) {
          w0[s] = widen8(wreg[b][s][0].x, wreg[b][s][0].y);
          w1[s] = widen8(wreg[b][s][0].z, wreg[b][s][0].w);
        } else {
          const uint4 a = wreg[b][s][0], c = wreg[b][s][1];
          w0[s] = as_bf8(a.x, a.y, a.z, a.w);
          w1[s] = as_bf8(c.x, c.y, c.z, c.w);
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint16_t* xr;
        if constexpr (LN) {
          xr = reinterpret_cast<const uint16_t*>(smem + (mb * 16 + xrow) * LN_ROW) + k;
        } else {
          const int m = min(m_base + mb * 16 + xrow, p.M - 1);
          xr = p.X + (int64_t)m * p.ldx + k;
        }
        v8bf x0, x1;
        if constexpr (W8) {
          const uint4 lo = XPRE ? xreg[XPRE ? b : 0][XPRE ? mb : 0][0]
                                : *reinterpret_cast<const uint4*>(xr + 16 * h);  // logical 0..7 of this 16-block
          const uint4 hi = XPRE ? xreg[XPRE ? b : 0][XPRE ? mb : 0][1]
                                : *reinterpret_cast<const uint4*>(xr + 16 * h + 8);  // logical 8..15
          x0 = as_bf8(lo.x, hi.x, lo.y, hi.y);  // pairs (0,1) (8,9) (2,3) (10,11)
          x1 = as_bf8(lo.z, hi.z, lo.w, hi.w);  // pairs (4,5) (12,13) (6,7) (14,15)
        } else {
          const uint4 a = XPRE ? xreg[XPRE ? b : 0][XPRE ? mb : 0][0] : *reinterpret_cast<const uint4*>(xr + 8 * h);
          const uint4 c = XPRE ? xreg[XPRE ? b : 0][XPRE ? mb : 0][1]
                               : *reinterpret_cast<const uint4*>(xr + 32 + 8 * h);
          x0 = as_bf8(a.x, a.y, a.z, a.w);
          x1 = as_bf8(c.x, c.y, c.z, c.w);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          acc[s][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0[s], x0, acc[s][mb], 0, 0, 0);
          acc[s][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1[s], x1, acc[s][mb], 0, 0, 0);
        }
      }
    }
  }

  // the waves' partial tiles, summed in wave order
  if constexpr (LN) __syncthreads();  // every wave is done reading the normalised rows
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      *reinterpret_cast<v4f*>(&red[wave][mb * 16 + c16][s * 16 + h * 4]) = acc[s][mb];
  __syncthreads();
  const int rows = min(p.M - m_base, ROWS);
  for (int i = threadIdx.x; i < rows * COLS; i += NW * 64) {
    const int r = i / COLS, c = i % COLS, m = m_base + r;
    float v = red[0][r][c];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][r][c];
    if constexpr (W8) v = __builtin_fmaf(v, sw_ep, p.bias ? bf2f(b_ep) : 0.f);
    else if (p.bias) v = v + bf2f(b_ep);
    if constexpr (EP == EP_RELU) v = fmaxf(v, 0.f);
    uint16_t* y = p.Y + (int64_t)m * p.ldy + n0 + c;
    // residual: y = bf16(y + bf16(v)), dec_add_ln's sum
    if constexpr (EP == EP_RESID) v = bf2f(*y) + round_bf(v);
    *y = f2bf(v);
  }
}

int g_skinny_override = -1;  // (NS << 8) | NW, tuning hook

int device_cus() {
  static const int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess || v <= 0)
      v = 256;
    return v;
  }();
  return n;
}

// the kernel with every wave's loads unconditional when K splits into exactly 2 or 8 blocks per wave (the decoder's
// 1024 and 4096) and the registers fit; otherwise the general loop
template <int MB, int NS, int NW, bool W8, int EP, bool LN, int RB = 16>
void launch_k(dim3 grid, const SkinnyArgs& p, hipStream_t s) {
  constexpr int WR = NS * (W8 ? 1 : 2);  // weight registers (x4) per block
  const int nkb = p.K / KB;
  if (nkb == 2 * NW && (LN || MB <= 4)) {
    skinny_kernel<MB, NS, NW, W8, EP, LN, RB, 2><<<grid, NW * 64, 0, s>>>(p);
    return;
  }
  if constexpr (8 * WR <= 16 && MB == 1) {
    if (nkb == 8 * NW) {
      skinny_kernel<MB, NS, NW, W8, EP, LN, RB, 8><<<grid, NW * 64, 0, s>>>(p);
      return;
    }
  }
  skinny_kernel<MB, NS, NW, W8, EP, LN, RB><<<grid, NW * 64, 0, s>>>(p);
}

template <int NS, int NW, bool W8, int EP, bool LN>
void launch_rows(const SkinnyArgs& p, hipStream_t s) {
  const int grid = p.N / (NS * 16), mblocks = (p.M + 15) / 16, mblocks8 = (p.M + 7) / 8;
  if (grid * mblocks < grid * mblocks8 && grid * mblocks8 <= device_cus()) {
    // fewer (strip, 16 rows) workgroups than CUs: one workgroup per (strip, 8 rows) instead -- twice the CUs stream
    // the weights, and each fetches half the activations (9-32 rows of the 1024 x 1024 and 1024 x 4096 projections)
    launch_k<1, NS, NW, W8, EP, LN, 8>(dim3(grid, mblocks8), p, s);
    return;
  }
  if (grid * mblocks <= 512 && mblocks > 1) {
    // few channel strips: one workgroup per (strip, 16 rows), so that every CU streams (the strip is read once per
    // 16 rows, the repeats mostly from L2 / MALL)
    launch_k<1, NS, NW, W8, EP, LN>(dim3(grid, mblocks), p, s);
    return;
  }
  switch (mblocks) {
    case 1: launch_k<1, NS, NW, W8, EP, LN>(dim3(grid), p, s); break;
    case 2: launch_k<2, NS, NW, W8, EP, LN>(dim3(grid), p, s); break;
    case 3: launch_k<3, NS, NW, W8, EP, LN>(dim3(grid), p, s); break;
    default: launch_k<4, NS, NW, W8, EP, LN>(dim3(grid), p, s); break;
  }
}

template <bool W8, int EP, bool LN>
int launch_shape(int ns, int nw, const SkinnyArgs& p, hipStream_t s) {
  const int key = (ns << 8) | nw;
  if constexpr (LN || EP == EP_RESID) {
    // the fused forms: eight waves
    switch (key) {
      case (1 << 8) | 8: launch_rows<1, 8, W8, EP, LN>(p, s); return 0;
      case (2 << 8) | 8: launch_rows<2, 8, W8, EP, LN>(p, s); return 0;
      case (4 << 8) | 8: launch_rows<4, 8, W8, EP, LN>(p, s); return 0;
      default: break;
    }
  } else {
    switch (key) {
      case (1 << 8) | 16: launch_rows<1, 16, W8, EP, LN>(p, s); return 0;
      case (1 << 8) | 8: launch_rows<1, 8, W8, EP, LN>(p, s); return 0;
      case (1 << 8) | 4: launch_rows<1, 4, W8, EP, LN>(p, s); return 0;
      case (2 << 8) | 8: launch_rows<2, 8, W8, EP, LN>(p, s); return 0;
      case (2 << 8) | 4: launch_rows<2, 4, W8, EP, LN>(p, s); return 0;
      case (4 << 8) | 8: launch_rows<4, 8, W8, EP, LN>(p, s); return 0;
      case (4 << 8) | 4: launch_rows<4, 4, W8, EP, LN>(p, s); return 0;
      default: break;
    }
  }
  cohere::set_error("skinny: no kernel for ns=" + std::to_string(ns) + " nw=" + std::to_string(nw));
  return 1;
}

// channels per workgroup (strips of 16) and waves per workgroup, measured on MI355X for the decoder's shapes (graph
// replays, 1-64 rows): 8 waves; one strip while the workgroups of one strip per 16 rows stay at or below ~256, more
// strips per workgroup beyond that (2 for 17-32 rows, 4 above, for N of 2048-8192; the head, N >= 8192, 2 strips
// up to 16 rows and 4 above: at 32 rows one workgroup per (4 strips, 16 rows) normalises half the rows that one per
// (2 strips, 32 rows) did, config 4 end to end +0.3 %). Long K (the feed-forward's second projection) keeps one strip.
void choose_shape(int N, int K, int M, int& ns, int& nw) {
  if (g_skinny_override > 0) {
    ns = g_skinny_override >> 8;
    nw = g_skinny_override & 255;
    if (N % (ns * 16) == 0) return;
  }
  nw = 8;
  if (K >= 2048 || N < 2048) ns = 1;
  else if (N >= 8192) ns = M > 16 ? 4 : 2;
  else ns = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  while (ns > 1 && N % (ns * 16) != 0) ns >>= 1;
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

int skinny_entry(SkinnyArgs& p, bool w8, int ep, hipStream_t s, const char* name) {
  const std::string nm(name);
  COHERE_REQUIRE(p.M >= 0 && p.M <= 64, nm + ": at most 64 rows per call (got " + std::to_string(p.M) + ")");
  COHERE_REQUIRE(p.N > 0 && p.N % 16 == 0, nm + ": N must be a multiple of 16");
  COHERE_REQUIRE(p.K > 0 && p.K % KB == 0, nm + ": K must be a multiple of 64");
  COHERE_REQUIRE(p.X && p.W && p.Y && (!w8 || p.sw), nm + ": null pointer");
  COHERE_REQUIRE(al16(p.X) && p.ldx % 8 == 0 && al16(p.W), nm + ": x rows and weights must be 16-byte aligned");
  COHERE_REQUIRE(ep >= EP_NONE && ep <= EP_RESID, nm + ": unknown epilogue " + std::to_string(ep));
  const bool ln = p.lnw != nullptr;
  COHERE_REQUIRE(!ln || (p.lnb && p.K >= 8 * KB && p.K <= LN_K && al16(p.lnw) && al16(p.lnb)),
                 nm + ": a LayerNorm prologue takes 512 <= K <= 1024 (got " + std::to_string(p.K) +
                     ") and 16-byte aligned weight and bias");
  if (p.M == 0) return 0;
  int ns, nw;
  choose_shape(p.N, p.K, p.M, ns, nw);
  if (ln || ep == EP_RESID) nw = 8;
  int rc;
  if (ln) {
    if (ep == EP_RESID) rc = 1, cohere::set_error(nm + ": no residual epilogue after a LayerNorm prologue");
    else if (w8) rc = ep == EP_RELU ? launch_shape<true, EP_RELU, true>(ns, nw, p, s)
                                    : launch_shape<true, EP_NONE, true>(ns, nw, p, s);
    else rc = ep == EP_RELU ? launch_shape<false, EP_RELU, true>(ns, nw, p, s)
                            : launch_shape<false, EP_NONE, true>(ns, nw, p, s);
  } else if (ep == EP_RESID) {
    rc = w8 ? launch_shape<true, EP_RESID, false>(ns, nw, p, s) : launch_shape<false, EP_RESID, false>(ns, nw, p, s);
  } else if (w8) {
    rc = ep == EP_RELU ? launch_shape<true, EP_RELU, false>(ns, nw, p, s)
                       : launch_shape<true, EP_NONE, false>(ns, nw, p, s);
  } else {
    rc = ep == EP_RELU ? launch_shape<false, EP_RELU, false>(ns, nw, p, s)
                       : launch_shape<false, EP_NONE, false>(ns, nw, p, s);
  }
  if (rc) return rc;
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
  p.X = x; p.W = w; p.sw = sw; p.bias = bias; p.Y = y;
  p.ldx = ldx; p.ldy = ldy; p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return skinny_entry(p, true, relu ? EP_RELU : EP_NONE, reinterpret_cast<hipStream_t>(stream), "dec_w8_linear");
}

extern "C" int cohere_linear_bf16(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* bias,
                                  uint16_t* y, int64_t ldy, int32_t relu, int64_t M, int64_t N, int64_t K,
                                  void* stream) {
  cohere::clear_error();
  SkinnyArgs p{};
  p.X = x; p.W = w; p.sw = nullptr; p.bias = bias; p.Y = y;
  p.ldx = ldx; p.ldy = ldy; p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return skinny_entry(p, false, relu ? EP_RELU : EP_NONE, reinterpret_cast<hipStream_t>(stream), "linear_bf16");
}

extern "C" int cohere_dec_linear_fused(const uint16_t* x, int64_t ldx, const uint16_t* ln_w, const uint16_t* ln_b,
                                       float eps, const void* w, const float* sw, const uint16_t* bias, uint16_t* y,
                                       int64_t ldy, int32_t epilogue, int64_t M, int64_t N, int64_t K, void* stream) {
  cohere::clear_error();
  SkinnyArgs p{};
  p.X = x; p.W = w; p.sw = sw; p.bias = bias; p.Y = y; p.lnw = ln_w; p.lnb = ln_b; p.eps = eps;
  p.ldx = ldx; p.ldy = ldy; p.M = (int)M; p.N = (int)N; p.K = (int)K;
  return skinny_entry(p, sw != nullptr, epilogue, reinterpret_cast<hipStream_t>(stream), "dec_linear_fused");
}

extern "C" int cohere_set_skinny_shape(int32_t strips, int32_t waves) {
  g_skinny_override = strips > 0 ? (strips << 8) | waves : -1;
  return 0;
}
