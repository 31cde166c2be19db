// W8A8 int8 GEMMs for gfx950: dense (v_mfma_i32_16x16x64_i8) and 2:4 sparse (v_smfmac_i32_16x16x128_i8), one kernel
// template for both, with the reference's fused epilogues.
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
//    channels of one token, so the per-token scale is one value and the per-channel scale/bias a float4.
//  * K tiles of 128 bytes are copied global -> LDS by the load unit itself (global_load_lds_dwordx4: 1 KB per wave
//    instruction, no staging registers), double-buffered: the next tile streams in while the matrix cores run on
//    the current one, one barrier per tile.
//  * LDS rows are 128 bytes (64 for compressed weights) with 16-byte chunks XOR-swizzled by row, so both the DMA
//    writes (8 lanes per row) and the fragment reads (16 rows, one chunk) are bank-conflict free. The swizzle is
//    applied on the global side: lane i of a DMA instruction lands in LDS slot i, so it fetches the chunk that
//    belongs there.
//  * Operand layouts (measured on gfx950): mfma_i32_16x16x64_i8 lane l holds row l%16, K bytes 16(l/16)..+15 of both
//    A and B, and D rows 4(l/16)..+3 of column l%16. smfmac_i32_16x16x128_i8: A (compressed) lane l holds row l%16,
//    the 16 kept bytes of K 32(l/16)..+31 with their selector word; B lane l holds column l%16, K 16(l/16)..+15 in
//    bytes 0-15 and K 64+16(l/16)..+15 in bytes 16-31. kernels/sparse.py's compress_24 rows are therefore the A
//    operand as stored, with no repacking.
//  * The output tile is staged through LDS as bf16 and written in 16-byte row chunks (residual read the same way);
//    SILU_Q8 reduces each row's column group in registers across the lanes that hold it.
//  * Workgroups are remapped so that consecutive tiles land on the same XCD (workgroups are dealt round-robin over
//    the 8 XCDs, each with its own L2), then rastered in groups of 8 token tiles sharing a weight tile.
#include "common.h"
#include "cohere_hip.h"

#include <algorithm>
#include <cstdio>
#include <string>

namespace {

enum { EPI_BIAS = 0, EPI_RESID = 3, EPI_GLU = 4, EPI_SILU_Q8 = 5, EPI_I32 = 7 };

struct GemmArgs {
  const int8_t* X;     // tokens [M, K], row stride ldx
  const float* sx;     // [M, ldsx] per-row (and K-group) scales
  const int8_t* W;     // dense [N, K] or 2:4 kept values [N, K/2]
  const int32_t* E;    // 2:4 selectors [N, K/32]
  const float* sw;     // [N]
  const uint16_t* bias;  // [N] bf16 or null
  void* C;
  const uint16_t* R;   // residual, bf16
  float* qs;           // SILU_Q8 scales
  int64_t ldx, ldsx, ldc, ldr, ldqs;
  int M, N, K;
  int group_steps;     // K steps per scale group (grouped only)
  int qgroup;          // SILU_Q8 columns per scale
  int epi;
  float alpha;
};

template <int BM, int BN, int WM, int WN, int ST, bool GROUPED, bool SPARSE>
struct Tile {
  static constexpr int NW = WM * WN, NT = NW * 64;
  static constexpr int TM = BM / WM, TN = BN / WN, MI = TM / 16, NI = TN / 16;
  static constexpr int X_STAGE = BM * 128;
  static constexpr int W_STAGE = SPARSE ? BN * 64 : BN * 128;
  static constexpr int E_STAGE = SPARSE ? BN * 16 : 0;
  static constexpr int STAGE = X_STAGE + W_STAGE + E_STAGE;
  static constexpr int PIPE = ST * STAGE;
  static constexpr int GFIT = (160 * 1024 - PIPE) / (BM * 4);
  static constexpr int GMAX = GFIT < 32 ? GFIT : 32;  // K-groups whose token scales are kept in LDS
  static constexpr int SCALES = GROUPED ? GMAX * BM * 4 : 0;
  static constexpr int LDC = BN + 8;  // staged output row (bf16 elements)
  static constexpr int OUTB = BM * LDC * 2;
  static constexpr int SMEM = (PIPE + SCALES) > OUTB ? (PIPE + SCALES) : OUTB;
  // 1 KB DMA instructions per stage: tokens (8 rows each), weights (8 dense rows / 16 compressed rows), selectors
  // (one per wave, BN/NW rows)
  static constexpr int X_SLOTS = BM / 8, W_SLOTS = SPARSE ? BN / 16 : BN / 8;
  static constexpr int LPS = X_SLOTS / NW + W_SLOTS / NW + (SPARSE ? 1 : 0);  // per wave per stage
  static_assert(TM % 16 == 0 && TN % 16 == 0, "tile shape");
  static_assert(X_SLOTS % NW == 0 && W_SLOTS % NW == 0 && BN / NW <= 64, "DMA slots must split evenly over waves");
  static_assert(LPS * (ST - 2 > 0 ? ST - 2 : 0) <= 63, "vmcnt range");
  static_assert(PIPE + SCALES <= 160 * 1024, "LDS");
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
    if (after >= 2) { wait_vm<2 * LPS>(); return; }
  }
  if constexpr (ST >= 3) {
    if (after >= 1) { wait_vm<LPS>(); return; }
  }
  wait_vm<0>();
}

// 16-byte chunk `c` (0..7) of row `r` of a 128-byte-row tile
DEVI int sw128(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }
// chunk `c` (0..3) of row `r` of a 64-byte-row tile
DEVI int sw64(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 3)) << 4); }

template <int BM, int BN, int WM, int WN, int ST, bool GROUPED, bool SPARSE>
__global__ void __launch_bounds__(WM* WN * 64) gemm_q8_kernel(const GemmArgs p) {
  using T = Tile<BM, BN, WM, WN, ST, GROUPED, SPARSE>;
  constexpr int NW = T::NW, NT = T::NT, TM = T::TM, TN = T::TN, MI = T::MI, NI = T::NI, LPS = T::LPS;
  __shared__ __attribute__((aligned(16))) char smem[T::SMEM];

  const int M = p.M, N = p.N, K = p.K;
  const int ntm = (M + BM - 1) / BM, ntn = N / BN, ntiles = ntm * ntn;
  int t;
  {  // XCD-aware remap: workgroup b runs on XCD b % 8; give each XCD a contiguous range of logical tiles
    const int b = blockIdx.x, xcd = b & 7, idx = b >> 3, per = ntiles >> 3, rem = ntiles & 7;
    t = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  }
  constexpr int GM = 8;
  const int gw = GM * ntn, first = (t / gw) * GM, gs = min(ntm - first, GM);
  const int m0 = (first + (t % gw) % gs) * BM, n0 = ((t % gw) / gs) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / WN, wn = wave % WN;

  const int KT = (K + 127) / 128;
  const bool half_last = (K & 127) != 0;  // dense only: the last tile holds 64 K

  // grouped: every group's token scales of this tile in LDS, loaded before the first DMA (read after a barrier)
  float* sS = reinterpret_cast<float*>(smem + T::PIPE);
  const int G = GROUPED ? K / (p.group_steps * (SPARSE ? 128 : 64)) : 1;
  const bool scales_in_lds = GROUPED && G <= T::GMAX;
  if (scales_in_lds) {
    for (int i = tid; i < G * BM; i += NT) {
      const int g = i / BM, r = i % BM;
      sS[i] = p.sx[(int64_t)min(m0 + r, M - 1) * p.ldsx + g];
    }
  }

  auto issue = [&](int buf, int kt) {
    char* base = smem + buf * T::STAGE;
    const bool half = half_last && kt == KT - 1;
    const int64_t k0 = (int64_t)kt * 128;
#pragma unroll
    for (int j = 0; j < T::X_SLOTS / NW; ++j) {  // tokens: 8 rows of 128 B per instruction
      const int s = wave + j * NW;
      const int r = s * 8 + (lane >> 3);
      int lc = (lane & 7) ^ (r & 7);
      if (half) lc &= 3;
      dma16(p.X + (int64_t)min(m0 + r, M - 1) * p.ldx + k0 + lc * 16, base + s * 1024);
    }
    char* wbase = base + T::X_STAGE;
    if constexpr (!SPARSE) {
#pragma unroll
      for (int j = 0; j < T::W_SLOTS / NW; ++j) {
        const int s = wave + j * NW;
        const int r = s * 8 + (lane >> 3);
        int lc = (lane & 7) ^ (r & 7);
        if (half) lc &= 3;
        dma16(p.W + (int64_t)(n0 + r) * K + k0 + lc * 16, wbase + s * 1024);
      }
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

  v4i acc[NI][MI];
  v4f accf[GROUPED ? NI : 1][GROUPED ? MI : 1];
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[j][i] = v4i{0, 0, 0, 0};
  if constexpr (GROUPED) {
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int i = 0; i < MI; ++i) accf[j][i] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  // fold the finished K-group's int32 sums into fp32 with each token's scale of that group
  auto fold = [&](int g) {
    if constexpr (GROUPED) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = wm * TM + i * 16 + (lane & 15);
        const float s = scales_in_lds ? sS[g * BM + r] : p.sx[(int64_t)min(m0 + r, M - 1) * p.ldsx + g];
#pragma unroll
        for (int j = 0; j < NI; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q) accf[j][i][q] = __builtin_fmaf((float)acc[j][i][q], s, accf[j][i][q]);
          acc[j][i] = v4i{0, 0, 0, 0};
        }
      }
    }
  };

#pragma unroll
  for (int s = 0; s < ST - 1; ++s)
    if (s < KT) issue(s, s);
  int kstep = 0;
  for (int kt = 0; kt < KT; ++kt) {
    wait_stages<LPS, ST>(min(KT - 1 - kt, ST - 2));
    __syncthreads();
    if (kt + ST - 1 < KT) issue((kt + ST - 1) % ST, kt + ST - 1);
    const char* xs = smem + (kt % ST) * T::STAGE;
    const char* ws = xs + T::X_STAGE;
    if constexpr (!SPARSE) {
      const bool two = !(half_last && kt == KT - 1);
      v4i bx[2][MI], aw[2][NI];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 1 && !two) break;
        const int lc = s * 4 + (lane >> 4);
#pragma unroll
        for (int i = 0; i < MI; ++i)
          bx[s][i] = *reinterpret_cast<const v4i*>(xs + sw128(wm * TM + i * 16 + (lane & 15), lc));
#pragma unroll
        for (int j = 0; j < NI; ++j)
          aw[s][j] = *reinterpret_cast<const v4i*>(ws + sw128(wn * TN + j * 16 + (lane & 15), lc));
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 1 && !two) break;
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int i = 0; i < MI; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aw[s][j], bx[s][i], acc[j][i], 0, 0, 0);
        if constexpr (GROUPED) {
          ++kstep;
          if (kstep % p.group_steps == 0) fold(kstep / p.group_steps - 1);
        }
      }
    } else {
      const char* es = ws + T::W_STAGE;
      v8i bx[MI];
      v4i aw[NI];
      int ix[NI];
      const int h = lane >> 4;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = wm * TM + i * 16 + (lane & 15);
        const v4i lo = *reinterpret_cast<const v4i*>(xs + sw128(r, h));
        const v4i hi = *reinterpret_cast<const v4i*>(xs + sw128(r, 4 + h));
        bx[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int r = wn * TN + j * 16 + (lane & 15);
        aw[j] = *reinterpret_cast<const v4i*>(ws + sw64(r, h));
        ix[j] = *reinterpret_cast<const int*>(es + r * 16 + h * 4);
      }
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i)
          acc[j][i] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(aw[j], bx[i], acc[j][i], ix[j], 0, 0);
      if constexpr (GROUPED) {
        ++kstep;
        if (kstep % p.group_steps == 0) fold(kstep / p.group_steps - 1);
      }
    }
  }
  wait_vm<0>();
  __syncthreads();

  // ---- epilogue ----------------------------------------------------------------------------------------------------
  const int epi = p.epi;
  const int ml0 = wm * TM + (lane & 15);          // + i * 16
  const int nl0 = wn * TN + (lane >> 4) * 4;      // + j * 16
  if (!GROUPED && epi == EPI_I32) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = m0 + ml0 + i * 16;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < NI; ++j)
        *reinterpret_cast<v4i*>(reinterpret_cast<int32_t*>(p.C) + (int64_t)m * p.ldc + n0 + nl0 + j * 16) = acc[j][i];
    }
    return;
  }

  float srow[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) srow[i] = GROUPED ? 1.f : p.sx[(int64_t)min(m0 + ml0 + i * 16, M - 1) * p.ldsx];
  uint16_t* sC = reinterpret_cast<uint16_t*>(smem);
  const int ldc_s = epi == EPI_GLU ? BN / 2 + 8 : T::LDC;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int n = n0 + nl0 + j * 16;
    const float4 w4 = *reinterpret_cast<const float4*>(p.sw + n);
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
      const uint2 b2 = *reinterpret_cast<const uint2*>(p.bias + n);
      bv[0] = __uint_as_float(b2.x << 16);
      bv[1] = __uint_as_float(b2.x & 0xffff0000u);
      bv[2] = __uint_as_float(b2.y << 16);
      bv[3] = __uint_as_float(b2.y & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = GROUPED ? accf[j][i][r] : (float)acc[j][i][r] * srow[i];
        v[r] = p.bias ? __builtin_fmaf(x, wv[r], bv[r]) : x * wv[r];
      }
      const int ml = ml0 + i * 16, nl = nl0 + j * 16;
      if (epi == EPI_GLU) {
        const uint32_t o = pack_bf2(round_bf(v[0]) * sigmoid_fast(round_bf(v[1])),
                                    round_bf(v[2]) * sigmoid_fast(round_bf(v[3])));
        *reinterpret_cast<uint32_t*>(sC + ml * ldc_s + nl / 2) = o;
      } else {
        if (epi == EPI_SILU_Q8) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float tv = round_bf(v[r]);
            v[r] = tv * sigmoid_fast(tv);
          }
        }
        *reinterpret_cast<uint2*>(sC + ml * ldc_s + nl) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
      }
    }
  }
  __syncthreads();

  if (epi == EPI_SILU_Q8) {
    // rows of BN bf16 as BN/8 chunks; a wave holds 64 / (BN/8) rows; qgroup/8 lanes share a scale
    constexpr int CH = BN / 8;
    static_assert(64 % CH == 0 || CH % 64 == 0, "row chunks per wave");
    const int lanes_q = p.qgroup / 8;
    for (int id0 = 0; id0 < BM * CH; id0 += NT) {
      const int id = id0 + tid;
      const int r = id / CH, c = (id % CH) * 8, row = m0 + r;
      const bool ok = id < BM * CH && row < M;
      uint4 u = make_uint4(0, 0, 0, 0);
      if (id < BM * CH) u = *reinterpret_cast<const uint4*>(sC + r * T::LDC + c);
      const uint32_t wds[4] = {u.x, u.y, u.z, u.w};
      float e[8];
      float mx = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        e[2 * k] = __uint_as_float(wds[k] << 16);
        e[2 * k + 1] = __uint_as_float(wds[k] & 0xffff0000u);
        mx = fmaxf(mx, fmaxf(fabsf(e[2 * k]), fabsf(e[2 * k + 1])));
      }
      for (int o = 1; o < lanes_q; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
      uint32_t q[2] = {0, 0};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int qi = (int)rintf(fminf(fmaxf(e[k] * inv, -127.f), 127.f));
        q[k >> 2] |= (uint32_t)(qi & 0xff) << ((k & 3) * 8);
      }
      if (ok) {
        *reinterpret_cast<uint2*>(reinterpret_cast<int8_t*>(p.C) + (int64_t)row * p.ldc + n0 + c) = make_uint2(q[0], q[1]);
        if ((c % p.qgroup) == 0) p.qs[(int64_t)row * p.ldqs + (n0 + c) / p.qgroup] = sc;
      }
    }
    return;
  }

  const int out_n = epi == EPI_GLU ? BN / 2 : BN;
  const int ch = out_n / 8;
  const int col0 = epi == EPI_GLU ? n0 / 2 : n0;
  for (int id = tid; id < BM * ch; id += NT) {
    const int r = id / ch, c = (id % ch) * 8, row = m0 + r;
    if (row >= M) continue;
    uint4 v = *reinterpret_cast<const uint4*>(sC + r * ldc_s + c);
    uint16_t* dst = reinterpret_cast<uint16_t*>(p.C) + (int64_t)row * p.ldc + col0 + c;
    if (epi == EPI_RESID) {
      const uint4 rv = *reinterpret_cast<const uint4*>(p.R + (int64_t)row * p.ldr + col0 + c);
      const uint32_t y[4] = {v.x, v.y, v.z, v.w}, rr[4] = {rv.x, rv.y, rv.z, rv.w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = __builtin_fmaf(p.alpha, __uint_as_float(y[k] << 16), __uint_as_float(rr[k] << 16));
        const float hi =
            __builtin_fmaf(p.alpha, __uint_as_float(y[k] & 0xffff0000u), __uint_as_float(rr[k] & 0xffff0000u));
        o[k] = pack_bf2(lo, hi);
      }
      v = make_uint4(o[0], o[1], o[2], o[3]);
    }
    *reinterpret_cast<uint4*>(dst) = v;
  }
}

// ---- tile table --------------------------------------------------------------------------------------------------

struct TileInfo {
  int bm, bn;
  bool grouped_ok;
};

// tile id: tokens x channels (waves M x N, pipeline stages)
//   0 128x128 (2x2, 4)   1 128x256 (2x2, 3)   2 256x128 (2x2, 3)   3 64x128 (2x2, 4)   4 64x256 (1x4, 3)
//   5 32x128 (1x4, 4)    6 256x256 (2x4, 2)   7 64x64 (2x2, 4)     8 256x128 (4x2, 3)  9 128x256 (2x4, 3)
constexpr TileInfo TILES[] = {{128, 128, true}, {128, 256, false}, {256, 128, false}, {64, 128, true},
                              {64, 256, true},  {32, 128, true},   {256, 256, false}, {64, 64, true},
                              {256, 128, true}, {128, 256, true}};
constexpr int N_TILES = sizeof(TILES) / sizeof(TILES[0]);

int g_tile_override = -1;

template <int BM, int BN, int WM, int WN, int ST, bool GROUPED, bool SPARSE>
void launch_tile(const GemmArgs& p, hipStream_t s) {
  const int grid = ((p.M + BM - 1) / BM) * (p.N / BN);
  gemm_q8_kernel<BM, BN, WM, WN, ST, GROUPED, SPARSE><<<grid, WM * WN * 64, 0, s>>>(p);
}

template <bool GROUPED, bool SPARSE>
int launch(int tile, const GemmArgs& p, hipStream_t s) {
  switch (tile) {
    case 0: launch_tile<128, 128, 2, 2, 4, GROUPED, SPARSE>(p, s); break;
    case 3: launch_tile<64, 128, 2, 2, 4, GROUPED, SPARSE>(p, s); break;
    case 4: launch_tile<64, 256, 1, 4, 3, GROUPED, SPARSE>(p, s); break;
    case 5: launch_tile<32, 128, 1, 4, 4, GROUPED, SPARSE>(p, s); break;
    case 7: launch_tile<64, 64, 2, 2, 4, GROUPED, SPARSE>(p, s); break;
    case 8: launch_tile<256, 128, 4, 2, 3, GROUPED, SPARSE>(p, s); break;
    case 9: launch_tile<128, 256, 2, 4, 3, GROUPED, SPARSE>(p, s); break;
    default:
      if constexpr (!GROUPED) {
        switch (tile) {
          case 1: launch_tile<128, 256, 2, 2, 3, false, SPARSE>(p, s); break;
          case 2: launch_tile<256, 128, 2, 2, 3, false, SPARSE>(p, s); break;
          case 6: launch_tile<256, 256, 2, 4, 2, false, SPARSE>(p, s); break;
          default: cohere::set_error("gemm: bad tile"); return 1;
        }
      } else {
        cohere::set_error("gemm: tile cannot take grouped scales");
        return 1;
      }
  }
  return cohere::check_launch("gemm_q8_kernel");
}

// gfx950 tile choice: the largest tile that still gives every CU work; SILU_Q8 needs the scale group inside a tile
int choose_tile(const GemmArgs& p, bool grouped) {
  auto fits = [&](int id) {
    const TileInfo& t = TILES[id];
    if (p.N % t.bn) return false;
    if (grouped && !t.grouped_ok) return false;
    if (p.epi == EPI_SILU_Q8 && (t.bn % p.qgroup || t.bn > 512)) return false;
    return true;
  };
  if (g_tile_override >= 0 && g_tile_override < N_TILES && fits(g_tile_override)) return g_tile_override;
  auto tiles_of = [&](int id) { return (int64_t)((p.M + TILES[id].bm - 1) / TILES[id].bm) * (p.N / TILES[id].bn); };
  static const int order[] = {9, 1, 8, 2, 0, 4, 3, 5};  // preferred first
  for (int id : order)
    if (fits(id) && tiles_of(id) >= 400) return id;
  for (int id : {0, 4, 3, 5})
    if (fits(id) && tiles_of(id) >= 200) return id;
  for (int id : {5, 3, 4, 0, 7})
    if (fits(id)) return id;
  return -1;
}

// the SILU_Q8 output group of each of the reference's int8 configs (its BN, gemm_int8.cu:321-345); -2 = unknown id
int ref_cfg_group(int cfg) {
  switch (cfg) {
    case -1: return 256;
    case 0: case 1: case 3: case 7: case 10: return 128;
    case 4: case 6: case 8: return 256;
    case 5: case 9: return 64;
    default: return -2;
  }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

template <bool SPARSE>
int gemm_entry(GemmArgs& p, int64_t group, int64_t lda_k_req, hipStream_t s, const char* name) {
  const std::string nm(name);
  COHERE_REQUIRE(p.M >= 0 && p.N > 0 && p.K > 0, nm + ": bad sizes");
  COHERE_REQUIRE(p.X && p.sx && p.W && p.sw && p.C, nm + ": null pointer");
  COHERE_REQUIRE(!SPARSE || p.E, nm + ": null selectors");
  COHERE_REQUIRE(p.K % lda_k_req == 0, nm + ": K=" + std::to_string(p.K) + " not a multiple of " +
                                           std::to_string(lda_k_req));
  COHERE_REQUIRE(group > 0 && group % lda_k_req == 0 && p.K % group == 0,
                 nm + ": group must divide K and be a multiple of " + std::to_string(lda_k_req));
  COHERE_REQUIRE(p.N % 64 == 0, nm + ": N must be a multiple of 64");
  COHERE_REQUIRE(p.epi == EPI_BIAS || p.epi == EPI_RESID || p.epi == EPI_GLU || p.epi == EPI_SILU_Q8 ||
                     p.epi == EPI_I32,
                 nm + ": unsupported epilogue " + std::to_string(p.epi));
  COHERE_REQUIRE(p.epi != EPI_RESID || p.R, nm + ": residual epilogue needs resid");
  COHERE_REQUIRE(p.epi != EPI_SILU_Q8 || p.qs, nm + ": SILU_Q8 needs qs");
  const bool grouped = group < p.K;
  COHERE_REQUIRE(!(grouped && p.epi == EPI_I32), nm + ": the int32 hook takes per-row scales only");
  COHERE_REQUIRE(p.ldx % 16 == 0 && aligned16(p.X), nm + ": tokens rows must be 16-byte aligned");
  COHERE_REQUIRE(aligned16(p.W) && aligned16(p.sw), nm + ": weights must be 16-byte aligned");
  COHERE_REQUIRE(!SPARSE || aligned16(p.E), nm + ": selectors must be 16-byte aligned");
  COHERE_REQUIRE(!p.bias || (reinterpret_cast<uintptr_t>(p.bias) & 7) == 0, nm + ": bias must be 8-byte aligned");
  const int out_align = p.epi == EPI_SILU_Q8 ? 8 : 16;
  const int esize = p.epi == EPI_SILU_Q8 ? 1 : (p.epi == EPI_I32 ? 4 : 2);
  COHERE_REQUIRE((reinterpret_cast<uintptr_t>(p.C) % out_align) == 0 && (p.ldc * esize) % out_align == 0,
                 nm + ": output rows must be aligned");
  COHERE_REQUIRE(p.epi != EPI_RESID || (aligned16(p.R) && p.ldr % 8 == 0), nm + ": residual rows must be aligned");
  if (p.M == 0) return 0;
  p.group_steps = (int)(group / (SPARSE ? 128 : 64));
  const int tile = choose_tile(p, grouped);
  COHERE_REQUIRE(tile >= 0, nm + ": no gfx950 tile fits N=" + std::to_string(p.N));
  return grouped ? launch<true, SPARSE>(tile, p, s) : launch<false, SPARSE>(tile, p, s);
}

}  // namespace

extern "C" int cohere_set_gemm_tile(int32_t tile) {
  g_tile_override = tile;
  return N_TILES;
}

extern "C" int cohere_gemm_i8(const int8_t* a, int64_t lda, const float* sa, int64_t ldsa, int64_t group,
                              const int8_t* w, const float* sw, const uint16_t* bias, void* out, int64_t ldc,
                              int32_t epi, const uint16_t* resid, int64_t ldr, float alpha, float* qs, int64_t ldqs,
                              int64_t M, int64_t N, int64_t K, int32_t cfg, void* stream) {
  cohere::clear_error();
  const int qg = ref_cfg_group(cfg);
  COHERE_REQUIRE(qg != -2, "gemm_i8: unknown config " + std::to_string(cfg));
  GemmArgs p{};
  p.X = a; p.sx = sa; p.W = w; p.E = nullptr; p.sw = sw; p.bias = bias; p.C = out; p.R = resid; p.qs = qs;
  p.ldx = lda; p.ldsx = ldsa; p.ldc = ldc; p.ldr = ldr; p.ldqs = ldqs;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.qgroup = qg; p.epi = epi; p.alpha = alpha;
  return gemm_entry<false>(p, group, 64, reinterpret_cast<hipStream_t>(stream), "gemm_i8");
}

extern "C" int cohere_gemm_sp(const int8_t* x, int64_t ldx, const float* sx, int64_t ldsx, int64_t group,
                              const int8_t* wc, const int32_t* e, const float* sw, const uint16_t* bias, void* out,
                              int64_t ldc, int32_t epi, const uint16_t* resid, int64_t ldr, float alpha, float* qs,
                              int64_t ldqs, int64_t M, int64_t N, int64_t K, int32_t cfg, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(cfg >= -1 && cfg <= 4, "gemm_sp: unknown config " + std::to_string(cfg));
  GemmArgs p{};
  p.X = x; p.sx = sx; p.W = wc; p.E = e; p.sw = sw; p.bias = bias; p.C = out; p.R = resid; p.qs = qs;
  p.ldx = ldx; p.ldsx = ldsx; p.ldc = ldc; p.ldr = ldr; p.ldqs = ldqs;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.qgroup = 256; p.epi = epi; p.alpha = alpha;
  return gemm_entry<true>(p, group, 128, reinterpret_cast<hipStream_t>(stream), "gemm_sp");
}
