// W8A8 int8 GEMM kernel template for gfx950: dense (v_mfma_i32_16x16x64_i8) and 2:4 sparse
// (v_smfmac_i32_16x16x128_i8), with the reference's fused epilogues. Instantiated by gemm_q8_dense.hip and
// gemm_q8_sparse.hip; the C ABI entry points are in gemm_q8.hip.
//
// Semantics follow kernels/csrc/gemm_int8.cu (dense) and kernels/csrc/gemm_sparse.cu (sparse) of the reference:
//   acc = sum_k X[m,k] W[n,k]                  int32, exact
//   per-row scales:   x = fmul((float)acc, sx[m])
//   grouped scales:   x = fmaf((float)acc_g, sx[m,g], x) over the K-groups g in order (gemm_int8.cu:146-163)
//   v = bias ? fmaf(x, sw[n], bias[n]) : fmul(x, sw[n])
//   epilogues BIAS / RESID / GLU / SILU_Q8 as gemm_int8.cu:201-288; I32 writes acc (parity hook).
// The integer sums do not depend on the order of K, so any tile shape gives the same bits, and the sparse kernel
// equals the dense one on the decompressed weights.
//
// gfx950 design:
//  * The matrix cores compute the transposed tile D = W X^T: the MFMA/SMFMAC A operand is the weight (for the sparse
//    kernel the instruction requires the sparse operand there), B the tokens. A lane then holds 4 consecutive output
//    channels of one token: one token scale, a float4 of channel scales, and 8-byte (bf16) output stores.
//  * K tiles of 128 bytes are copied global -> LDS by the load unit itself (global_load_lds_dwordx4: 1 KB per wave
//    instruction, no staging registers) through a ST-stage ring: the next ST-1 tiles stream in while the matrix
//    cores run on the current one. Each wave waits only for its own transfers of the tile it needs (vmcnt), then one
//    plain s_barrier per tile (no memory fence, which would drain every transfer in flight).
//  * LDS rows are 128 bytes (64 for compressed weights) with 16-byte chunks XOR-swizzled by row, so both the DMA
//    writes (8 lanes per row) and the fragment reads (16 rows, one chunk) are bank-conflict free. The swizzle is
//    applied on the global side: lane i of a DMA instruction lands in LDS slot i, so it fetches the chunk that
//    belongs there.
//  * Operand layouts (measured on gfx950): mfma_i32_16x16x64_i8 lane l holds row l%16, K bytes 16(l/16)..+15 of both
//    A and B, and D rows 4(l/16)..+3 of column l%16. smfmac_i32_16x16x128_i8: A (compressed) lane l holds row l%16,
//    the 16 kept bytes of K 32(l/16)..+31 with their selector word; B lane l holds column l%16, K 16(l/16)..+15 in
//    bytes 0-15 and K 64+16(l/16)..+15 in bytes 16-31. kernels/sparse.py's compress_24 rows are therefore the A
//    operand as stored, with no repacking.
//  * The epilogue is a template parameter and runs from registers: the tile's token scales, channel scales and bias
//    are copied to LDS when the kernel starts (no dependent global loads after the main loop), results are stored
//    straight from the accumulators, and SILU_Q8 reduces each row's column group with lane shuffles and a small LDS
//    table.
//  * Workgroups are remapped so that consecutive tiles land on the same XCD (workgroups are dealt round-robin over
//    the 8 XCDs, each with its own L2), then rastered in groups of 8 token tiles sharing a weight tile.
#pragma once
#include <type_traits>

#include "common.h"

namespace cohere_gemm {

// the reference's epilogue ids (kernels/cuda_ext.py:28); SILU, RELU and CONV_RELU are bf16-operand only, I32 is ours
enum { EPI_BIAS = 0, EPI_SILU = 1, EPI_RELU = 2, EPI_RESID = 3, EPI_GLU = 4, EPI_SILU_Q8 = 5, EPI_CONV_RELU = 6,
       EPI_I32 = 7 };

struct GemmArgs {
  const int8_t* X;       // tokens [M, K], row stride ldx
  const float* sx;       // [M, ldsx] per-row (and K-group) scales
  const int8_t* W;       // dense [N, K] or 2:4 kept values [N, K/2]
  const int32_t* E;      // 2:4 selectors [N, K/32]
  const float* sw;       // [N]
  const uint16_t* bias;  // [N] bf16 or null
  void* C;
  const uint16_t* R;     // residual, bf16
  float* qs;             // SILU_Q8 scales
  int64_t ldx, ldsx, ldc, ldr, ldqs;
  int M, N, K;
  int group;             // K per token-scale group (group == K: one scale per row)
  int qgroup;            // SILU_Q8 columns per scale
  int epi;               // host-side dispatch only: the kernels take the epilogue as a template parameter
  float alpha;
  int xcd_rows;          // > 0: the token tiles split into xcd_rows parts and the channel tiles into 8 / xcd_rows,
                         // one part each per XCD (set by launch_tile); 0: contiguous tile ranges per XCD
  int tiled;             // 2:4 only: W holds the stage-tiled layout of the kept values and selectors (E unused)
};

// The stage-tiled 2:4 weight layout (cohere_pack_24_tiled): for each block of 16 output channels rb and each
// 128-wide K stage kt, one contiguous record of TILED_REC bytes at (rb * K/128 + kt) * TILED_REC: 1024 bytes of kept
// values, 16-byte chunk i holding row i / 4's logical chunk (i % 4) ^ ((i / 8) % 4) of its 64 kept bytes of the stage
// (the LDS swizzle, so a DMA lane's 16 bytes land where the fragment reads expect them), then 256 bytes of
// selectors, row r's four words of the stage at 16 r, with words 0-1 and 2-3 swapped in rows 8-15 (a selector read
// of 32 lanes -- rows 0-15, two words each -- then touches 32 distinct banks: unswizzled, rows r and r + 8 share
// banks). Every 1 KB DMA instruction then reads one contiguous kilobyte
// (row-major weights give 16 rows x 64 bytes: half of each 128-byte line), and a stage's selectors of 16 rows one
// 256-byte run (row-major: 16 bytes of each of 16 lines).
constexpr int TILED_REC = 1280;

constexpr int LDS_BYTES = 160 * 1024;
inline bool g_xcd_split = true;  // tuning hook (cohere_set_gemm_tile with tile -2 / -3 switches it)

template <int BM, int BN, int WM, int WN, int ST, int MS, bool GROUPED, bool SPARSE>
struct Tile {
  static constexpr int NW = WM * WN, NT = NW * 64;
  static constexpr int TM = BM / WM, TN = BN / WN, MI = TM / MS, NI = TN / MS;
  // K per matrix instruction, instructions per 128-byte K tile, values per lane per instruction
  static constexpr int KSTEP = MS == 16 ? (SPARSE ? 128 : 64) : (SPARSE ? 64 : 32);
  static constexpr int SPS = 128 / KSTEP;
  static constexpr int RPL = MS == 16 ? 4 : 16;
  static constexpr bool PF = NW <= 4 && MI * NI <= 32;  // fragment double-buffering (register budget)
  static constexpr int X_STAGE = BM * 128;
  static constexpr int W_STAGE = SPARSE ? BN * 64 : BN * 128;
  static constexpr int E_STAGE = SPARSE ? BN * 16 : 0;
  static constexpr int STAGE = X_STAGE + W_STAGE + E_STAGE;
  static constexpr int PIPE = ST * STAGE;
  static constexpr int PARAMS = (BM + 2 * BN) * 4;  // token scales, channel scales, bias (fp32)
  static constexpr int GFIT = (LDS_BYTES - PIPE - PARAMS) / (BM * 4);
  static constexpr int GMAX = GROUPED ? (GFIT < 32 ? GFIT : 32) : 0;  // K-groups whose token scales live in LDS
  static constexpr int SMEM = PIPE + PARAMS + GMAX * BM * 4;
  // 1 KB DMA instructions per stage: tokens (8 rows each), weights (8 dense rows / 16 compressed rows), selectors
  // (one per wave, BN/NW rows)
  static constexpr int X_SLOTS = BM / 8, W_SLOTS = SPARSE ? BN / 16 : BN / 8;
  static constexpr int LPS = X_SLOTS / NW + W_SLOTS / NW + (SPARSE ? 1 : 0);  // per wave per stage
  static_assert(MS == 16 || MS == 32, "matrix instruction size");
  static_assert(TM % MS == 0 && TN % MS == 0 && MI >= 1 && NI >= 1, "tile shape");
  static_assert(X_SLOTS % NW == 0 && W_SLOTS % NW == 0 && BN / NW <= 64, "DMA slots must split evenly over waves");
  static_assert(LPS * (ST - 1) <= 63 && ST >= 2 && ST <= 4, "vmcnt range");
  static_assert(SMEM <= LDS_BYTES, "LDS");
  static_assert(BM * (BN / MS + 2 * BN / 64) * 4 <= PIPE, "SILU_Q8 tables reuse the pipeline buffers");
  static_assert(!GROUPED || GMAX >= 1, "grouped tile needs room for scales");
};

DEVI void dma16(const void* g, char* lds_slot) {
  __builtin_amdgcn_global_load_lds(g, (LDS_AS void*)lds_slot, 16, 0, 0);
}

template <int N>
DEVI void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait until at most `after` stages of this wave's DMA (LPS instructions each) are still in flight
template <int LPS, int ST>
DEVI void wait_stages(int after) {
  if constexpr (ST >= 4) {
    if (after >= 3) {
      wait_vm<3 * LPS>();
      return;
    }
  }
  if constexpr (ST >= 3) {
    if (after >= 2) {
      wait_vm<2 * LPS>();
      return;
    }
  }
  if constexpr (ST >= 2) {
    if (after >= 1) {
      wait_vm<LPS>();
      return;
    }
  }
  wait_vm<0>();
}

// 16-byte chunk `c` (0..7) of row `r` of a 128-byte-row tile
// The XOR key of row r: its low three bits for the 16-row reads of the 16x16 instructions; for the 32-row reads of the
// 32x32 instructions (32 rows at chunk c, 32 at c ^ 1), rows 8-15, 16-23 and 24-31 take it XORed with 1, 2 and 3,
// which measured free of bank conflicts on gfx950 where the plain key is not (rocprofv3 SQ_LDS_BANK_CONFLICT)
template <int MS>
DEVI int row_key(int r) { return MS == 32 ? (r ^ (r >> 3)) & 7 : r & 7; }
template <int MS>
DEVI int sw128(int r, int c) { return r * 128 + ((c ^ row_key<MS>(r)) << 4); }
// chunk `c` (0..3) of row `r` of a 64-byte-row tile
DEVI int sw64(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 3)) << 4); }

// GS > 0 (grouped only): the K steps per scale group, fixed at compile time -- the main loop then runs whole groups
// with the fold at a static place; GS == 0 reads it from p.group
//
// BF (bf16 operands, kernels/csrc/gemm.cu of the reference): X and W hold bf16 values and K, ldx count bytes (two per
// value). v_mfma_f32_16x16x32_bf16 / 32x32x16_bf16 take 16 bytes per lane in exactly the lane layout of the int8
// instructions of the same shape, so the DMA ring, swizzle and fragment reads are shared; accumulation is fp32 and
// the epilogue adds the bias in fp32 before its first rounding (CONV_RELU rounds the sum first, as a convolution
// whose bias is added after).
template <int BM, int BN, int WM, int WN, int ST, int MS, int EPI, bool GROUPED, bool SPARSE, int GS = 0,
          bool BF = false>
__global__ void __launch_bounds__(WM* WN * 64) gemm_q8_kernel(const GemmArgs p) {
  static_assert(!BF || (!SPARSE && !GROUPED && EPI != EPI_SILU_Q8 && EPI != EPI_I32), "bf16 operands");
  static_assert(BF || (EPI != EPI_SILU && EPI != EPI_RELU && EPI != EPI_CONV_RELU), "bf16-only epilogue");
  using T = Tile<BM, BN, WM, WN, ST, MS, GROUPED, SPARSE>;
  constexpr int NW = T::NW, NT = T::NT, TM = T::TM, TN = T::TN, MI = T::MI, NI = T::NI, LPS = T::LPS;
  constexpr int KSTEP = T::KSTEP, SPS = T::SPS, RPL = T::RPL;
  using AccI = typename std::conditional<MS == 16, v4i, v16i>::type;
  using AccF = typename std::conditional<MS == 16, v4f, v16f>::type;
  using Acc = typename std::conditional<BF, AccF, AccI>::type;
  __shared__ __attribute__((aligned(16))) char smem[T::SMEM];

  const int M = p.M, N = p.N, K = p.K;
  const int ntm = (M + BM - 1) / BM, ntn = N / BN, ntiles = ntm * ntn;
  int m0, n0;
  if (p.xcd_rows > 0) {
    // workgroup b runs on XCD b % 8: XCD x takes token part x / (8 / xcd_rows) and channel part x % (8 / xcd_rows)
    // of the tile grid, so each XCD's L2 fetches only its part's tokens and weights (the grid divides evenly)
    const int parts_n = 8 / p.xcd_rows, rm = ntm / p.xcd_rows, rn = ntn / parts_n;
    const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
    m0 = ((xcd / parts_n) * rm + idx % rm) * BM;
    n0 = ((xcd % parts_n) * rn + idx / rm) * BN;
  } else {
    int t;
    {  // XCD-aware remap: workgroup b runs on XCD b % 8; give each XCD a contiguous range of logical tiles
      const int b = blockIdx.x, xcd = b & 7, idx = b >> 3, per = ntiles >> 3, rem = ntiles & 7;
      t = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    }
    constexpr int GM = 8;
    const int gw = GM * ntn, first = (t / gw) * GM, gs = min(ntm - first, GM);
    m0 = (first + (t % gw) % gs) * BM;
    n0 = ((t % gw) / gs) * BN;
  }

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / WN, wn = wave % WN;

  const int KT = (K + 127) / 128;
  const bool half_last = (K & 127) != 0;  // dense only: the last tile holds 64 K
  const int NSTEPS = K / KSTEP;

  // the epilogue's per-row / per-channel values and (grouped) every group's token scales live in LDS past the
  // pipeline buffers; the first barrier publishes them
  float* pS = reinterpret_cast<float*>(smem + T::PIPE);
  float* pW = pS + BM;
  float* pB = pW + BN;
  float* sS = pB + BN;
  static_assert(GS == 0 || (GROUPED && GS % SPS == 0 && (GS % 2 == 0 || !T::PF)), "static group steps");
  const int group_steps = GS > 0 ? GS : (GROUPED ? p.group / KSTEP : 1);
  const int G = GROUPED ? K / p.group : 1;
  const bool scales_in_lds = GROUPED && G <= T::GMAX;
  // the epilogue's per-row / per-channel values and (grouped) every group's token scales: copied into LDS by the
  // load unit itself (global_load_lds, 4 bytes a lane), issued between the first stage's transfers and the others.
  // They hold no registers and need no wait of their own: the first stage's wait covers them (they are older than
  // the later stages' transfers), and a value loaded into a register and used before that wait would make the compiler
  // wait for the first stage's transfers too. The bias stays bf16 in LDS (pairs of values per lane).
  uint16_t* pBh = reinterpret_cast<uint16_t*>(pB);
  auto dma4 = [&](const void* g, void* lds) { __builtin_amdgcn_global_load_lds(g, (LDS_AS void*)lds, 4, 0, 0); };
  auto issue_params = [&]() {
    if constexpr (EPI != EPI_I32) {
      int k = 0;  // instruction index across the kinds, dealt round-robin to the waves
      if constexpr (!GROUPED && !BF) {
#pragma unroll
        for (int b = 0; b < BM; b += 64, ++k)
          if (k % NW == wave && b + lane < BM) dma4(p.sx + (int64_t)min(m0 + b + lane, M - 1) * p.ldsx, pS + b);
      }
      if constexpr (!BF) {
#pragma unroll
        for (int b = 0; b < BN; b += 64, ++k)
          if (k % NW == wave) dma4(p.sw + n0 + b + lane, pW + b);
      }
      if (p.bias) {
#pragma unroll
        for (int b = 0; b < BN / 2; b += 64, ++k)
          if (k % NW == wave && b + lane < BN / 2)
            dma4(reinterpret_cast<const uint32_t*>(p.bias + n0) + b + lane, pBh + 2 * b);
      }
      if constexpr (GROUPED) {
        // group g's scales of rows r0 .. r0 + 63 to sS[g][r0 ..]
        if (scales_in_lds)
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int b = 0; b < BM; b += 64, ++k)
              if (k % NW == wave && b + lane < BM)
                dma4(p.sx + (int64_t)min(m0 + b + lane, M - 1) * p.ldsx + g, sS + g * BM + b);
      }
    }
  };

  auto issue = [&](int buf, int kt) {
    char* base = smem + buf * T::STAGE;
    const bool half = half_last && kt == KT - 1;
    const int64_t k0 = (int64_t)kt * 128;
#pragma unroll
    for (int j = 0; j < T::X_SLOTS / NW; ++j) {  // tokens: 8 rows of 128 B per instruction
      const int s = wave + j * NW;
      const int r = s * 8 + (lane >> 3);
      int lc = (lane & 7) ^ row_key<MS>(r);
      if (half) lc &= 3;
      dma16(p.X + (int64_t)min(m0 + r, M - 1) * p.ldx + k0 + lc * 16, base + s * 1024);
    }
    char* wbase = base + T::X_STAGE;
    if constexpr (!SPARSE) {
#pragma unroll
      for (int j = 0; j < T::W_SLOTS / NW; ++j) {
        const int s = wave + j * NW;
        const int r = s * 8 + (lane >> 3);
        int lc = (lane & 7) ^ row_key<MS>(r);
        if (half) lc &= 3;
        dma16(p.W + (int64_t)(n0 + r) * K + k0 + lc * 16, wbase + s * 1024);
      }
    } else if (p.tiled) {
      // stage-tiled weights: instruction s takes the kept values of channel block (n0 / 16 + s), stage kt
      const int8_t* rec = p.W + ((int64_t)(n0 >> 4) * KT + kt) * TILED_REC;
#pragma unroll
      for (int j = 0; j < T::W_SLOTS / NW; ++j) {
        const int s = wave + j * NW;
        dma16(rec + (int64_t)s * KT * TILED_REC + lane * 16, wbase + s * 1024);
      }
      constexpr int ER = BN / NW;
      char* ebase = wbase + T::W_STAGE + wave * ER * 16;
      const int r = wave * ER + lane;
      if (lane < ER) dma16(rec + (int64_t)(r >> 4) * KT * TILED_REC + 1024 + (r & 15) * 16, ebase);
    } else {
#pragma unroll
      for (int j = 0; j < T::W_SLOTS / NW; ++j) {  // kept values: 16 rows of 64 B per instruction
        const int s = wave + j * NW;
        const int r = s * 16 + (lane >> 2), lc = (lane & 3) ^ ((r >> 1) & 3);
        dma16(p.W + (int64_t)(n0 + r) * (K / 2) + k0 / 2 + lc * 16, wbase + s * 1024);
      }
      // selectors: 16 B (4 words) a row; wave w brings rows [w BN/NW, (w+1) BN/NW)
      constexpr int ER = BN / NW;
      char* ebase = wbase + T::W_STAGE + wave * ER * 16;
      const int r = wave * ER + lane;
      if (lane < ER) dma16(p.E + (int64_t)(n0 + r) * (K / 32) + k0 / 32, ebase);
    }
  };

  Acc acc[NI][MI];
  AccF accf[GROUPED ? NI : 1][GROUPED ? MI : 1];
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      acc[j][i] = Acc{};
      if constexpr (GROUPED) accf[j][i] = AccF{};
    }

  // a lane's token row within the tile for instruction-block row i, and its first channel for block column j and
  // group q of 4 consecutive channels (16x16: one group of 4; 32x32: four groups, 8 channels apart)
  const int lrow = MS == 16 ? (lane & 15) : (lane & 31);
  const int lhi = MS == 16 ? (lane >> 4) : (lane >> 5);
  auto tok = [&](int i) { return wm * TM + i * MS + lrow; };
  auto chan = [&](int j, int q) { return wn * TN + j * MS + (MS == 16 ? lhi * 4 : 8 * q + 4 * lhi); };

  // grouped scales: at the first K step of each group, just before that step's matrix instruction for a block, the
  // block's finished group sums are folded into fp32 with each token's scale of that group and reset. Interleaved
  // with the next group's instructions, the fold reads results finished long before, so the matrix cores keep going.
  auto group_scale = [&](int g, int i) {
    const int r = tok(i);
    // GS > 0 is launched only when every group's scales are in LDS: a plain LDS read (a select between the two
    // pointers makes the compiler read through a flat pointer)
    if constexpr (GS > 0) return sS[g * BM + r];
    else return scales_in_lds ? sS[g * BM + r] : p.sx[(int64_t)min(m0 + r, M - 1) * p.ldsx + g];
  };
  // the finished group of block (j, i) into fp32; the next group's first matrix instruction then takes a zero
  // accumulator (mma_block's `fresh`), so the int32 accumulators are not cleared with register moves
  auto fold_block = [&](int j, int i, float sc) {
    if constexpr (GROUPED) {
#pragma unroll
      for (int q = 0; q < RPL; ++q) accf[j][i][q] = __builtin_fmaf((float)acc[j][i][q], sc, accf[j][i][q]);
    }
  };

  // ---- main loop: ST-stage DMA ring; matrix-core fragments of K step u read from stage u / SPS ------------------
  struct Frags {
    typename std::conditional<SPARSE, v8i, v4i>::type bx[MI];
    v4i aw[NI];
    int ix[SPARSE ? NI : 1];
  };
  auto load_frags = [&](Frags& F, int u) {
    const int st = u / SPS, s = u % SPS;
    const char* xs = smem + (st % ST) * T::STAGE;
    const char* ws = xs + T::X_STAGE;
    if constexpr (!SPARSE) {
      // 16x16x64: chunk 4s + lane/16 of rows lane%16; 32x32x32: chunk 2s + lane/32 of rows lane%32
      const int lc = MS == 16 ? s * 4 + lhi : s * 2 + lhi;
#pragma unroll
      for (int i = 0; i < MI; ++i) F.bx[i] = *reinterpret_cast<const v4i*>(xs + sw128<MS>(wm * TM + i * MS + lrow, lc));
#pragma unroll
      for (int j = 0; j < NI; ++j) F.aw[j] = *reinterpret_cast<const v4i*>(ws + sw128<MS>(wn * TN + j * MS + lrow, lc));
    } else {
      const char* es = ws + T::W_STAGE;
      // B (tokens): 16x16x128 reads chunks h and 4 + h (h = lane/16); 32x32x64 step s reads 4s + h and 4s + 2 + h
      // (h = lane/32). A (kept weights): compressed chunk h / 2s + h, and the selector word of the same 32 K.
      const int c0 = MS == 16 ? lhi : 4 * s + lhi, c1 = MS == 16 ? 4 + lhi : 4 * s + 2 + lhi;
      const int ca = MS == 16 ? lhi : 2 * s + lhi;
      // the stage-tiled layout stores rows 8-15 of each 16-row block with selector words 0-1 and 2-3 swapped
      const int cs = ca ^ (p.tiled ? (lrow & 8) >> 2 : 0);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = wm * TM + i * MS + lrow;
        const v4i lo = *reinterpret_cast<const v4i*>(xs + sw128<MS>(r, c0));
        const v4i hi = *reinterpret_cast<const v4i*>(xs + sw128<MS>(r, c1));
        F.bx[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int r = wn * TN + j * MS + lrow;
        F.aw[j] = *reinterpret_cast<const v4i*>(ws + sw64(r, ca));
        F.ix[j] = *reinterpret_cast<const int*>(es + r * 16 + cs * 4);
      }
    }
  };
  int kstep = 0;
  auto mma_block = [&](const Frags& F, int j, int i, bool fresh = false) {
    const Acc c = fresh ? Acc{} : acc[j][i];
    if constexpr (BF && MS == 16)
      acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, F.aw[j]),
                                                         __builtin_bit_cast(v8bf, F.bx[i]), c, 0, 0, 0);
    else if constexpr (BF)
      acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, F.aw[j]),
                                                         __builtin_bit_cast(v8bf, F.bx[i]), c, 0, 0, 0);
    else if constexpr (SPARSE && MS == 16)
      acc[j][i] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(F.aw[j], F.bx[i], c, F.ix[j], 0, 0);
    else if constexpr (SPARSE)
      acc[j][i] = __builtin_amdgcn_smfmac_i32_32x32x64_i8(F.aw[j], F.bx[i], c, F.ix[j], 0, 0);
    else if constexpr (MS == 16)
      acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(F.aw[j], F.bx[i], c, 0, 0, 0);
    else
      acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(F.aw[j], F.bx[i], c, 0, 0, 0);
  };
  // one K step; with fold, the finished group gprev is folded block by block just before the block's instruction
  auto mma_step = [&](const Frags& F, bool fold, int gprev) {
    if (fold) {
      float gsc[MI];
#pragma unroll
      for (int i = 0; i < MI; ++i) gsc[i] = group_scale(gprev, i);
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          fold_block(j, i, gsc[i]);
          mma_block(F, j, i, true);
        }
      return;
    }
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int i = 0; i < MI; ++i) mma_block(F, j, i);
  };
  auto mma = [&](const Frags& F) {
    if constexpr (GROUPED) {
      const bool fold = kstep > 0 && kstep % group_steps == 0;  // uniform: this step also folds the last group
      const int gprev = kstep / group_steps - 1;
      ++kstep;
      if (fold) {
        mma_step(F, true, gprev);
        return;
      }
    }
    mma_step(F, false, 0);
  };
  // before reading step u, the first of stage t = u / SPS: stage t landed everywhere and stage t - 1 is free, so
  // stage t - 1 + ST can stream into its buffer
  // Dense: the freed buffer's next transfer is issued after the step's matrix instructions (flush_issue), so that a
  // busy load unit never holds up the matrix cores at the start of a step (measured: 5 % faster dense loops; the
  // sparse tiles, with one step per stage, are faster issuing at once).
  // LAG2 (double-buffered fragments and at least 4 stages): entering stage t frees stage t - 2, not t - 1. A wave
  // then still has the previous step's fragment reads (from stage t - 1) in flight at the barrier, and the barrier
  // does not wait for them (lgkmcnt), so those reads overlap the matrix instructions; the DMA runs ST - 2 stages
  // ahead instead of ST - 1.
  constexpr bool LAG2 = T::PF && ST >= 4;
  constexpr int AHEAD = LAG2 ? ST - 2 : ST - 1;  // stages in flight beyond the one being waited for, at most
  int pending = -1;
  auto enter_stage = [&](int t) {
    wait_stages<LPS, ST>(min(KT - 1 - t, AHEAD - 1));
    if constexpr (LAG2) asm volatile("s_barrier" ::: "memory");
    else lds_barrier();
    const int next = t + AHEAD;
    if (next < KT) {
      if constexpr (SPARSE) issue(next % ST, next);
      else pending = next;
    }
  };
  // the step's matrix instructions interleaved with the next step's fragment reads (scheduling hints only)
  auto interleave = [&]() {
    constexpr int NMFMA = MI * NI;
    constexpr int NREAD = SPARSE ? 2 * MI + 2 * NI : MI + NI;
    constexpr int PER = (NREAD + NMFMA - 1) / NMFMA;
#pragma unroll
    for (int k = 0; k < NMFMA; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one matrix instruction
      __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);  // then up to PER LDS reads
    }
  };
  auto flush_issue = [&]() {
    if (pending >= 0) {
      issue(pending % ST, pending);
      pending = -1;
    }
  };

  issue(0, 0);
  issue_params();
  if constexpr (EPI != EPI_I32) {
    // no bias: -0.0 in its place, so the epilogue's one fma (x * w + b, or x + b) equals the plain product (sum)
    // bit for bit, the sign of a zero included
    if (!p.bias)
      for (int c = tid; c < BN / 2; c += NT) reinterpret_cast<uint32_t*>(pBh)[c] = 0x80008000u;
  }
#pragma unroll
  for (int s = 1; s <= AHEAD; ++s)
    if (s < KT) issue(s, s);
  wait_stages<LPS, ST>(min(KT - 1, AHEAD));
  lds_barrier();
  if constexpr (GS > 0) {
    // whole groups of GS steps, unrolled: the fold sits at each group's first step (not the first group's), so the
    // accumulators keep one register assignment through the loop
    Frags F[T::PF ? 2 : 1];
    if constexpr (T::PF) load_frags(F[0], 0);
    auto group = [&](int g, auto fold_tag) {
#pragma unroll
      for (int s = 0; s < GS; ++s) {
        const int u = g * GS + s;
        if constexpr (T::PF) {
          if (u + 1 < NSTEPS) {
            if ((s + 1) % SPS == 0) enter_stage((u + 1) / SPS);
            load_frags(F[(s + 1) & 1], u + 1);
          }
          mma_step(F[s & 1], decltype(fold_tag)::value && s == 0, g - 1);
          flush_issue();
        } else {
          if (u > 0 && s % SPS == 0) enter_stage(u / SPS);
          load_frags(F[0], u);
          mma_step(F[0], decltype(fold_tag)::value && s == 0, g - 1);
          flush_issue();
        }
      }
    };
    group(0, std::false_type{});
    for (int g = 1; g < G; ++g) group(g, std::true_type{});
  } else if constexpr (T::PF) {
    // fragments of step u + 1 are read while the matrix cores work on step u
    // the steady state has no conditional fragment loads (they made the compiler copy fragment registers at every
    // join); the last one or two steps are peeled
    Frags F0, F1;
    load_frags(F0, 0);
    int u = 0;
    for (; u + 2 < NSTEPS; u += 2) {
      if ((u + 1) % SPS == 0) enter_stage((u + 1) / SPS);
      load_frags(F1, u + 1);
      mma(F0);
      if constexpr (!GROUPED) interleave();
      flush_issue();
      if ((u + 2) % SPS == 0) enter_stage((u + 2) / SPS);
      load_frags(F0, u + 2);
      mma(F1);
      if constexpr (!GROUPED) interleave();
      flush_issue();
    }
    if (u + 1 < NSTEPS) {
      if ((u + 1) % SPS == 0) enter_stage((u + 1) / SPS);
      load_frags(F1, u + 1);
      mma(F0);
      flush_issue();
      mma(F1);
      flush_issue();
    } else {
      mma(F0);
      flush_issue();
    }
  } else {
    // two waves per SIMD hide each other's LDS latency
    Frags F0;
    for (int u = 0; u < NSTEPS; ++u) {
      if (u > 0 && u % SPS == 0) enter_stage(u / SPS);
      load_frags(F0, u);
      mma(F0);
      flush_issue();
    }
  }

  if constexpr (GROUPED) {  // the last group
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const float sc = group_scale(G - 1, i);
#pragma unroll
      for (int j = 0; j < NI; ++j) fold_block(j, i, sc);
    }
  }

  // ---- epilogue, from registers --------------------------------------------------------------------------------
  constexpr int NQ = RPL / 4;  // groups of 4 consecutive channels per lane per block
  if constexpr (EPI == EPI_I32) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = m0 + tok(i);
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          *reinterpret_cast<v4i*>(reinterpret_cast<int32_t*>(p.C) + (int64_t)m * p.ldc + n0 + chan(j, q)) =
              v4i{acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
    }
    return;
  } else {
    // dequantized value (+ bias) of block (j, i), values 4q..4q+3: computed where it is stored, so no second copy
    // of the accumulators is held
    float srow[MI];
#pragma unroll
    for (int i = 0; i < MI; ++i) srow[i] = pS[tok(i)];
    auto dequant = [&](int j, int i, int q, float (&v)[4]) {
      const v4f w4 = *reinterpret_cast<const v4f*>(pW + chan(j, q));
      const uint2 braw = *reinterpret_cast<const uint2*>(pBh + chan(j, q));
      const float b4[4] = {__uint_as_float(braw.x << 16), __uint_as_float(braw.x & 0xffff0000u),
                           __uint_as_float(braw.y << 16), __uint_as_float(braw.y & 0xffff0000u)};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (BF) {
          const float x = EPI == EPI_CONV_RELU ? round_bf(acc[j][i][4 * q + r]) : acc[j][i][4 * q + r];
          v[r] = x + b4[r];
        } else {
          const float x = GROUPED ? accf[j][i][4 * q + r] : (float)acc[j][i][4 * q + r] * srow[i];
          v[r] = __builtin_fmaf(x, w4[r], b4[r]);
        }
      }
    };
    if constexpr (EPI == EPI_BIAS || EPI == EPI_RESID || EPI == EPI_GLU || EPI == EPI_SILU || EPI == EPI_RELU ||
                  EPI == EPI_CONV_RELU) {
      // the tile's bf16 results are staged in LDS (over the pipeline buffers, free now) and written out as whole
      // rows: each 16-byte store then covers 8 consecutive channels of one row, where the lanes' own results would
      // give 16 rows x 8 bytes per instruction. A row's 8-byte units (4 channels) are XOR-swizzled by the row's low
      // four bits, so the stage writes (16 rows, one unit: 16 distinct bank pairs) are free of bank conflicts; a
      // 16-byte row read then finds its chunk at cc ^ (g >> 1), its two halves swapped when g is odd.
      constexpr int OC = EPI == EPI_GLU ? BN / 2 : BN;  // output channels per tile row
      constexpr int CPR = OC / 8;                       // 16-byte chunks per row
      constexpr int GM = (OC / 4 < 16 ? OC / 4 : 16) - 1;
      static_assert(BM * OC * 2 <= T::PIPE && (CPR & (CPR - 1)) == 0, "epilogue staging");
      char* so = smem;
      auto slot = [&](int row, int col) {  // byte offset of output column col (bf16) of tile row row
        return row * (OC * 2) + (((col >> 2) ^ (row & GM)) << 3) + (col & 3) * 2;
      };
      lds_barrier();  // every wave is done reading the pipeline buffers
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int rl = tok(i);
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const int c = chan(j, q);
            float v[4];
            dequant(j, i, q, v);
            if constexpr (EPI == EPI_GLU) {
              // interleaved (a, gate) channel pairs are adjacent in a lane: output column c / 2
              *reinterpret_cast<uint32_t*>(so + slot(rl, c / 2)) =
                  pack_bf2(round_bf(v[0]) * sigmoid_fast(round_bf(v[1])), round_bf(v[2]) * sigmoid_fast(round_bf(v[3])));
            } else {
              if constexpr (EPI == EPI_SILU) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const float t = round_bf(v[r]);
                  v[r] = t * sigmoid_fast(t);
                }
              } else if constexpr (EPI == EPI_RELU || EPI == EPI_CONV_RELU) {
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = fmaxf(v[r], 0.f);
              }
              *reinterpret_cast<uint2*>(so + slot(rl, c)) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
            }
          }
      }
      lds_barrier();
      const int oc0 = EPI == EPI_GLU ? n0 / 2 : n0;
      for (int idx = tid; idx < BM * CPR; idx += NT) {
        const int rl = idx / CPR, cc = idx % CPR, m = m0 + rl, g = rl & GM;
        if (m >= M) continue;
        uint4 o = *reinterpret_cast<const uint4*>(so + rl * (OC * 2) + ((cc ^ (g >> 1)) << 4));
        if (g & 1) o = make_uint4(o.z, o.w, o.x, o.y);
        if constexpr (EPI == EPI_RESID) {
          // out = bf16(alpha * bf16(v) + r); out may be r itself (this thread reads the chunk before writing it)
          const uint4 rv = *reinterpret_cast<const uint4*>(p.R + (int64_t)m * p.ldr + oc0 + cc * 8);
          const uint32_t ov[4] = {o.x, o.y, o.z, o.w}, rr[4] = {rv.x, rv.y, rv.z, rv.w};
          uint32_t res[4];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            res[k] = pack_bf2(__builtin_fmaf(p.alpha, __uint_as_float(ov[k] << 16), __uint_as_float(rr[k] << 16)),
                              __builtin_fmaf(p.alpha, __uint_as_float(ov[k] & 0xffff0000u),
                                             __uint_as_float(rr[k] & 0xffff0000u)));
          o = make_uint4(res[0], res[1], res[2], res[3]);
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p.C) + (int64_t)m * p.ldc + oc0 + cc * 8) = o;
      }
    } else if constexpr (EPI == EPI_SILU_Q8) {
      // u = bf16(silu(bf16(v))), kept (as float bits) in the accumulator registers; the max |u| of each (row,
      // MS-column block) across the lanes holding it goes to an LDS table [BN/MS][BM] (over the pipeline buffers,
      // free now); then each lane reads its group's blocks and quantizes
      constexpr int CB = BN / MS;
      float* red = reinterpret_cast<float*>(smem);
      lds_barrier();  // every wave is done reading the pipeline buffers
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          // u = bf16(silu(bf16(v))) as fp32 bits in the accumulator; the maximum of |u| over the lane's block
          float mx = 0.f;
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            float v[4];
            dequant(j, i, q, v);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float t = round_bf_valu(v[r]);  // v: an fma's result
              const float u = round_bf_valu(t * sigmoid_fast(t));
              mx = fmaxf(mx, fabsf(u));
              acc[j][i][4 * q + r] = __float_as_int(u);
            }
          }
          if constexpr (MS == 16) mx = xor32_max_pos(xor16_max_pos(mx));
          else mx = xor32_max_pos(mx);
          if (lhi == 0) red[(wn * TN + j * MS) / MS * BM + tok(i)] = mx;  // column-block major: 16 rows, 16 banks
        }
      __syncthreads();
      // each (row, column group) maximum once, from the block table (consecutive threads take consecutive rows, so
      // each read touches consecutive words), and from it the group's scale and its reciprocal into gsc / ginv
      // [BM][BN / qgroup]; the maximum of non-negative values does not depend on the order
      const int blocks = p.qgroup / MS, ngroups = BN / p.qgroup;
      float* gsc = red + BM * CB;
      float* ginv = gsc + BM * (BN / 64);
      for (int id = tid; id < BM * ngroups; id += NT) {
        const int row = id % BM, g = id / BM;
        const float* src = red + g * blocks * BM + row;
        float mx = 0.f;
        for (int b = 0; b < blocks; ++b) mx = fmaxf(mx, src[b * BM]);
        const float sc = mx > 0.f ? mx / 127.f : 1.f;
        gsc[row * ngroups + g] = sc;
        ginv[row * ngroups + g] = 1.f / sc;
      }
      __syncthreads();
      // the int8 tile is staged in LDS past the tables and written out as whole rows (16-byte stores of 16
      // consecutive channels, where the lanes' own values would be 4-byte stores, 16 rows per instruction). A row's
      // 4-byte units are XOR-swizzled by twice the row's low four bits, so the stage writes (16 rows at one unit,
      // 16 rows at the next: 32 distinct banks) are free of bank conflicts; a 16-byte row read then finds its chunk
      // at cc ^ (g >> 2), its two halves swapped when g & 2.
      constexpr int CPR = BN / 16;  // 16-byte chunks per tile row
      constexpr int TABLES = BM * (CB + 2 * BN / 64) * 4;
      static_assert(TABLES + BM * BN <= T::PIPE && (CPR & (CPR - 1)) == 0, "int8 staging");
      char* so = smem + TABLES;
      auto swz = [&](int row) { return ((row & 15) << 1) & (BN / 4 - 1); };
      auto slot = [&](int row, int col) { return row * BN + (((col >> 2) ^ swz(row)) << 2) + (col & 3); };
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int rl = tok(i), m = m0 + rl;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int cb = (wn * TN + j * MS) / MS, g0 = cb - cb % blocks;
          const int gi = rl * ngroups + cb / blocks;
          const float inv = ginv[gi];
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const uint32_t o = q8x4(__int_as_float(acc[j][i][4 * q]), __int_as_float(acc[j][i][4 * q + 1]),
                                    __int_as_float(acc[j][i][4 * q + 2]), __int_as_float(acc[j][i][4 * q + 3]), inv);
            *reinterpret_cast<uint32_t*>(so + slot(rl, chan(j, q))) = o;
          }
          if (lhi == 0 && cb == g0 && m < M) p.qs[(int64_t)m * p.ldqs + (n0 + cb * MS) / p.qgroup] = gsc[gi];
        }
      }
      lds_barrier();
      for (int idx = tid; idx < BM * CPR; idx += NT) {
        const int rl = idx / CPR, cc = idx % CPR, m = m0 + rl, g = swz(rl);
        if (m >= M) continue;
        uint4 o = *reinterpret_cast<const uint4*>(so + rl * BN + ((cc ^ (g >> 2)) << 4));
        if (g & 2) o = make_uint4(o.z, o.w, o.x, o.y);
        *reinterpret_cast<uint4*>(reinterpret_cast<int8_t*>(p.C) + (int64_t)m * p.ldc + n0 + cc * 16) = o;
      }
    }
  }
}

// the XCD split of launch_tile: among the splits of the tile grid into xcd_rows x (8 / xcd_rows) equal parts, the one
// whose L2 fetches are fewest (tokens fetched once per channel part, weights once per token part); 0 when the grid
// does not split evenly
inline int xcd_split(int ntm, int ntn, double x_bytes, double w_bytes) {
  int best = 0;
  double cost = 0.0;
  for (int a = 1; a <= 8; a *= 2) {
    if (ntm % a != 0 || ntn % (8 / a) != 0) continue;
    const double c = (8 / a) * x_bytes + a * w_bytes;
    if (best == 0 || c < cost) best = a, cost = c;
  }
  return best;
}

template <int BM, int BN, int WM, int WN, int ST, int MS, int EPI, bool GROUPED, bool SPARSE, bool BF = false>
void launch_tile(const GemmArgs& args, hipStream_t s) {
  const int ntm = (args.M + BM - 1) / BM, ntn = args.N / BN, grid = ntm * ntn;
  GemmArgs p = args;
  p.xcd_rows = g_xcd_split ? xcd_split(ntm, ntn, (double)p.M * p.K,
                                       SPARSE ? (double)p.N * p.K * 0.625 : (double)p.N * p.K) : 0;
  // the feed-forward W2's grouping (256 K per scale) runs the static-group loop (tiles of one wave per SIMD: with
  // two, its unrolled groups do not fit the registers)
  constexpr int GS = 256 / Tile<BM, BN, WM, WN, ST, MS, GROUPED, SPARSE>::KSTEP;
  if constexpr (GROUPED && EPI == EPI_RESID &&
                (WM * WN <= 4 || Tile<BM, BN, WM, WN, ST, MS, GROUPED, SPARSE>::MI * Tile<BM, BN, WM, WN, ST, MS,
                                                                                       GROUPED, SPARSE>::NI <= 8)) {
    if (p.group == 256 && p.K / 256 <= Tile<BM, BN, WM, WN, ST, MS, GROUPED, SPARSE>::GMAX) {  // scales all in LDS
      gemm_q8_kernel<BM, BN, WM, WN, ST, MS, EPI, GROUPED, SPARSE, GS><<<grid, WM * WN * 64, 0, s>>>(p);
      return;
    }
  }
  gemm_q8_kernel<BM, BN, WM, WN, ST, MS, EPI, GROUPED, SPARSE, 0, BF><<<grid, WM * WN * 64, 0, s>>>(p);
}

// tile ids (tokens x channels, waves M x N, pipeline stages):
//   0 128x128 (2x2, 4)   1 128x256 (2x2, 3)   2 256x128 (2x2, 3)   3 64x128 (2x2, 4)   4 64x256 (1x4, 3)
//   5 32x128 (1x4, 4)    6 256x256 (2x4, 2 dense / 3 sparse)        7 64x64 (2x2, 4)    8 256x128 (4x2, 3)
//   9 128x256 (2x4, 3)   10 256x256 (4x2, 2 dense / 3 sparse)   11 256x128 (2x2, 3)   12 128x128 (2x2, 4)
//   13 128x256 (2x2, 3)   14 256x256 (2x2, 2 dense / 3 sparse)   15 256x256 (4x4: 16 waves, 2 dense / 3 sparse)
//   16 128x128 (4x2: 8 waves of 32 tokens x 64 channels, 4)   17 128x128 (2x4: 8 waves of 64 tokens x 32 channels, 4);
//   tiles 11-13 use the 32x32 matrix instructions, the others 16x16
struct TileInfo {
  int bm, bn;
  bool grouped_ok;
};
constexpr TileInfo TILES[] = {{128, 128, true}, {128, 256, false}, {256, 128, false}, {64, 128, true},
                              {64, 256, true},  {32, 128, true},   {256, 256, false}, {64, 64, true},
                              {256, 128, true}, {128, 256, true},  {256, 256, false}, {256, 128, false},
                              {128, 128, true}, {128, 256, false}, {256, 256, false}, {256, 256, false},
                              {128, 128, true}, {128, 128, true}};
constexpr int N_TILES = sizeof(TILES) / sizeof(TILES[0]);

// launches tile `tile` for one (SPARSE, EPI, GROUPED); false when the tile has no such instantiation
template <bool SPARSE, int EPI, bool GROUPED>
bool launch_tiles(int tile, const GemmArgs& p, hipStream_t s) {
  switch (tile) {
    case 0: launch_tile<128, 128, 2, 2, 4, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 3: launch_tile<64, 128, 2, 2, 4, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 4: launch_tile<64, 256, 1, 4, 3, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 5: launch_tile<32, 128, 1, 4, 4, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 7: launch_tile<64, 64, 2, 2, 4, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 8: launch_tile<256, 128, 4, 2, 3, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 9: launch_tile<128, 256, 2, 4, 3, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 12: launch_tile<128, 128, 2, 2, 4, 32, EPI, GROUPED, SPARSE>(p, s); return true;
    case 16: launch_tile<128, 128, 4, 2, 4, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    case 17: launch_tile<128, 128, 2, 4, 4, 16, EPI, GROUPED, SPARSE>(p, s); return true;
    default: break;
  }
  if constexpr (!GROUPED) {
    switch (tile) {
      case 1: launch_tile<128, 256, 2, 2, 3, 16, EPI, false, SPARSE>(p, s); return true;
      case 2: launch_tile<256, 128, 2, 2, 3, 16, EPI, false, SPARSE>(p, s); return true;
      case 6: launch_tile<256, 256, 2, 4, SPARSE ? 3 : 2, 16, EPI, false, SPARSE>(p, s); return true;
      case 10: launch_tile<256, 256, 4, 2, SPARSE ? 3 : 2, 16, EPI, false, SPARSE>(p, s); return true;
      case 11: launch_tile<256, 128, 2, 2, 3, 32, EPI, false, SPARSE>(p, s); return true;
      case 13: launch_tile<128, 256, 2, 2, 3, 32, EPI, false, SPARSE>(p, s); return true;
      case 14: launch_tile<256, 256, 2, 2, SPARSE ? 3 : 2, 16, EPI, false, SPARSE>(p, s); return true;
      case 15: launch_tile<256, 256, 4, 4, SPARSE ? 3 : 2, 16, EPI, false, SPARSE>(p, s); return true;
      default: break;
    }
  }
  return false;
}

// instantiated in gemm_q8_dense.hip / gemm_q8_sparse.hip
template <bool SPARSE>
bool launch_gemm(int tile, int epi, bool grouped, const GemmArgs& p, hipStream_t s);

// bf16 operands (instantiated in gemm_bf16.hip): the tiles with a bf16 instantiation, and the launch
constexpr bool bf16_tile(int tile) { return tile == 0 || tile == 1 || tile == 3 || tile == 6 || tile == 7 || tile == 9; }
bool launch_gemm_bf16(int tile, int epi, const GemmArgs& p, hipStream_t s);

}  // namespace cohere_gemm
