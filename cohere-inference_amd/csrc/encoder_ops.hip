// The FastConformer layer's non-GEMM producers on packed variable-length batches (every sequence's frames
// concatenated, no padding), for gfx950:
//   * the convolution module's depthwise convolution (kernel 9) + BatchNorm + SiLU, with bf16 output (reference
//     kernels/csrc/encoder_ops.cu:455-498 dwconv_tile_kernel, 643-656) or quantized per row for the next int8 GEMM
//     (encoder_ops.cu:559-641 dwconv_q8_kernel, 658-674);
//   * relative-position self-attention (Transformer-XL / ParakeetEncoderAttention, encoder_ops.cu:82-337, 676-707):
//       score[i, j] = ((q_i + u) . k_j) * scale + bf16(bf16((q_i + v) . R[i - j]) * scale)
//     with R[d] row d + rel_off of a per-layer table of projected sinusoids, softmax over the sequence's keys, and
//     the probabilities rounded to bf16 for the value product.
#include "cohere_hip.h"
#include "common.h"

#include <string>

namespace {

// ---- depthwise convolution + BatchNorm + SiLU --------------------------------------------------------------------------
// One workgroup holds DW_ROWS consecutive packed rows; each thread owns DW_CH = 4 channels, with their 9 taps, bias
// and BatchNorm affine in registers and the DW_ROWS + 8 input rows it needs loaded once (8-byte loads). Small
// per-thread state keeps four waves per SIMD and many workgroups in flight: the kernel is latency-bound, its bytes
// are few. A tap reads frame row + k - 4 only inside the row's own sequence [lo, hi) (zero padding at both ends of
// every sequence). Per channel: acc = fmaf chain over the taps from the conv bias; a = bf16(acc);
// a = bf16(fmaf(a, bn_scale, bn_shift)); y = bf16(a * sigmoid(a)). Q8 quantizes each output row with one scale
// (absmax / 127) instead of storing bf16.
constexpr int DW_K = 9, DW_PAD = 4, DW_ROWS = 4, DW_CH = 4, DW_MAXW = 8;

DEVI float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
DEVI float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <bool Q8>
__global__ void __launch_bounds__(64 * DW_MAXW) dwconv_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ w, const float* __restrict__ cb,
    const float* __restrict__ bn_scale, const float* __restrict__ bn_shift, const int32_t* __restrict__ seq_lo,
    const int32_t* __restrict__ seq_hi, uint16_t* __restrict__ y, int8_t* __restrict__ q, float* __restrict__ qs,
    int rows, int C) {
  __shared__ float red[DW_MAXW][DW_ROWS];
  // XCD-aware order: workgroup b runs on XCD b % 8, so each XCD takes one contiguous run of row blocks and the 8
  // halo rows a block shares with its neighbours are fetched into that XCD's L2 once
  const int nb = (int)gridDim.x, xcd = (int)blockIdx.x % 8;
  const int blk = xcd * (nb / 8) + min(xcd, nb % 8) + (int)blockIdx.x / 8;
  const int tid = threadIdx.x, c = tid * DW_CH, r0 = blk * DW_ROWS;
  const bool active = c < C;
  uint2 in[DW_ROWS + DW_K - 1];
  // a thread's 4 channels x 9 taps are 36 consecutive floats of the (C, 9) layout: 9 16-byte loads
  float wk[DW_CH][DW_K], bias[DW_CH], sc[DW_CH], sh[DW_CH];
  if (active) {
#pragma unroll
    for (int i = 0; i < DW_ROWS + DW_K - 1; ++i) {
      const int gr = r0 - DW_PAD + i;
      in[i] = gr >= 0 && gr < rows ? *reinterpret_cast<const uint2*>(x + (int64_t)gr * C + c) : make_uint2(0, 0);
    }
    float* wf = &wk[0][0];
#pragma unroll
    for (int v = 0; v < DW_CH * DW_K / 4; ++v)
      *reinterpret_cast<float4*>(wf + 4 * v) = *reinterpret_cast<const float4*>(w + (int64_t)c * DW_K + 4 * v);
    *reinterpret_cast<float4*>(bias) = *reinterpret_cast<const float4*>(cb + c);
    *reinterpret_cast<float4*>(sc) = *reinterpret_cast<const float4*>(bn_scale + c);
    *reinterpret_cast<float4*>(sh) = *reinterpret_cast<const float4*>(bn_shift + c);
  }
  float out[DW_ROWS][DW_CH];
  float mx[DW_ROWS];
#pragma unroll
  for (int r = 0; r < DW_ROWS; ++r) {
    const int row = r0 + r;
    mx[r] = 0.f;
#pragma unroll
    for (int j = 0; j < DW_CH; ++j) out[r][j] = 0.f;
    if (!active || row >= rows) continue;
    const int lo = seq_lo[row], hi = seq_hi[row];
    float acc[DW_CH];
#pragma unroll
    for (int j = 0; j < DW_CH; ++j) acc[j] = bias[j];
#pragma unroll
    for (int k = 0; k < DW_K; ++k) {
      const int src = row + k - DW_PAD;
      if (src < lo || src >= hi) continue;
      const uint32_t e[2] = {in[r + k].x, in[r + k].y};
#pragma unroll
      for (int j = 0; j < DW_CH; ++j) {
        const float xv = j & 1 ? bf_hi(e[j >> 1]) : bf_lo(e[j >> 1]);
        acc[j] = __builtin_fmaf(xv, wk[j][k], acc[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < DW_CH; ++j) {
      float a = round_bf(acc[j]);
      a = round_bf(__builtin_fmaf(a, sc[j], sh[j]));
      out[r][j] = round_bf(a * sigmoid_fast(a));
      mx[r] = fmaxf(mx[r], fabsf(out[r][j]));
    }
  }
  if constexpr (!Q8) {
    if (!active) return;
#pragma unroll
    for (int r = 0; r < DW_ROWS; ++r) {
      const int row = r0 + r;
      if (row >= rows) break;
      *reinterpret_cast<uint2*>(y + (int64_t)row * C + c) =
          make_uint2(pack_bf2(out[r][0], out[r][1]), pack_bf2(out[r][2], out[r][3]));
    }
  } else {
    const int wv = tid >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int r = 0; r < DW_ROWS; ++r) {
      const float m = wave_max_xor(mx[r], 64);
      if ((tid & 63) == 0) red[wv][r] = m;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < DW_ROWS; ++r) {
      const int row = r0 + r;
      if (row >= rows) break;
      float m = red[0][r];
      for (int k = 1; k < nw; ++k) m = fmaxf(m, red[k][r]);
      const float s = m > 0.f ? m / 127.f : 1.f, inv = 1.f / s;
      if (active) {
        static_assert(DW_CH == 4, "one q8x4 per row");
        *reinterpret_cast<uint32_t*>(q + (int64_t)row * C + c) = q8x4(out[r][0], out[r][1], out[r][2], out[r][3], inv);
      }
      if (tid == 0) qs[row] = s;
    }
  }
}

// ---- relative-position self-attention ----------------------------------------------------------------------------------
// One workgroup = one (64-query tile of one sequence, head): 4 waves of 16 queries. The matrix cores compute the
// transposed products, so every lane owns one query (lane % 16) throughout and no probability ever moves between
// lanes:
//   S^T[key, q]   = K_tile (A, 16 keys x 32 dims per instruction, from LDS) . (q + u)^T (B, registers)
//   P^T[dist, q]  = R_ring (A, 16 distances, from LDS) . (q + v)^T (B, registers)
//   O^T[dim, q]  += V^T (A, 16 dims x 32 keys, from a transposed LDS copy of the value tile) . p^T (B, the lane's
//                   own 8 probabilities: the 32 keys are ordered so that k slot b of lane group g is key 4g + b for
//                   b < 4 and 16 + 4g + b - 4 after -- the same key order on both operands)
// with v_mfma_f32_16x16x32_bf16 (lane l: row/col l % 16, k = 8 (l / 16) + b; result element e of lane l: row
// 4 (l / 16) + e, col l % 16); a head size that is an odd multiple of 16 ends with one v_mfma_f32_16x16x16_bf16 step
// (k = 4 (l / 16) + b). Keys stream in tiles of 32 with an online softmax in fp32. The position term a key tile
// needs spans 95 distances; each wave computes its own 48 (3 blocks of 16) from a ring of 128 table rows in LDS, of
// which each key tile adds 32, rounds them as the module does and gathers its scores from them through a small
// per-wave LDS buffer.
constexpr int AT_Q = 64, AT_KEYS = 32, AT_RING = 128, AT_PW = 52;  // per-wave position buffer row (48 + pad)

template <int D>
struct AttnShape {
  static constexpr bool TAIL = D % 32 != 0;   // one last k step of 16
  static constexpr int KS = D / 32;           // k steps of 32
  static constexpr int DP = D + 8;            // LDS row of K / R tiles (elements; 16-byte aligned, off bank stride)
  static constexpr int OB = D / 16;           // 16-dim blocks of the output
  static constexpr int VT = AT_KEYS + 4;      // LDS row of the transposed value tile
  // key and value tiles double-buffered where three workgroups still fit a CU's 160 KB (one barrier per key tile)
  static constexpr int NBUF = D <= 96 ? 2 : 1;
  static constexpr int K_ELEMS = AT_KEYS * DP, V_ELEMS = D * VT, R_ELEMS = AT_RING * DP, P_ELEMS = 4 * 16 * AT_PW;
  static constexpr int LDS_BYTES = 2 * (NBUF * (K_ELEMS + V_ELEMS) + R_ELEMS + P_ELEMS);
  static_assert(D % 16 == 0, "head size");
};

struct AttnArgs {
  const uint16_t* qkv;  // (rows, 3 H D): q | k | v, head-major within each
  const uint16_t* rk;   // (rel_rows, H D)
  const uint16_t* bu;   // (H, D)
  const uint16_t* bv;   // (H, D)
  uint16_t* out;        // (rows, H D)
  const int32_t* tiles; // (n, 4): sequence start, sequence length, first query row, unused
  int H, rel_off, rel_rows, n_tiles;
  float scale;
};

typedef short v4s __attribute__((ext_vector_type(4)));

// 16 bytes at element offset off of a uniform base: a 32-bit byte offset from the base in scalar registers
DEVI uint4 ld16(const uint16_t* base, uint32_t off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + (off << 1));
}

// bf16(q + bias) for dims col .. col + N - 1 of one query row (zero for rows past the sequence), N = 8 or 4
template <int N>
DEVI void q_plus(const uint16_t* qrow, const uint16_t* bias, int col, bool valid, uint16_t* __restrict__ r) {
  uint32_t qa[N / 2], ba[N / 2];
  if constexpr (N == 8) {
    const uint4 qv = *reinterpret_cast<const uint4*>(qrow + col), bv = *reinterpret_cast<const uint4*>(bias + col);
    qa[0] = qv.x, qa[1] = qv.y, qa[2] = qv.z, qa[3] = qv.w, ba[0] = bv.x, ba[1] = bv.y, ba[2] = bv.z, ba[3] = bv.w;
  } else {
    const uint2 qv = *reinterpret_cast<const uint2*>(qrow + col), bv = *reinterpret_cast<const uint2*>(bias + col);
    qa[0] = qv.x, qa[1] = qv.y, ba[0] = bv.x, ba[1] = bv.y;
  }
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const uint32_t v = pack_bf2(bf_lo(qa[k]) + bf_lo(ba[k]), bf_hi(qa[k]) + bf_hi(ba[k]));
    reinterpret_cast<uint32_t*>(r)[k] = valid ? v : 0u;
  }
}

// one 16-row block of a product over the head size: acc += A rows (LDS, row pointer per lane) . B (registers)
template <int D>
struct HeadDot {
  using S = AttnShape<D>;
  v8bf b[S::KS];
  v4s bt;  // the last 16 dims when the head size is an odd multiple of 16
  DEVI void load(const uint16_t* qrow, const uint16_t* bias, int g, bool valid) {
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      uint16_t r[8];
      q_plus<8>(qrow, bias, ks * 32 + g * 8, valid, r);
      b[ks] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(r));
    }
    if constexpr (S::TAIL) {
      uint16_t r[4];
      q_plus<4>(qrow, bias, S::KS * 32 + g * 4, valid, r);
      bt = __builtin_bit_cast(v4s, *reinterpret_cast<const uint2*>(r));
    }
  }
  DEVI v4f step(const uint16_t* row, int g, int ks, v4f acc) const {
    if (ks < S::KS)
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const v8bf*>(row + ks * 32 + g * 8), b[ks], acc,
                                                     0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(*reinterpret_cast<const v4s*>(row + S::KS * 32 + g * 4), bt, acc,
                                                      0, 0, 0);
  }
  static constexpr int steps = S::KS + (S::TAIL ? 1 : 0);
};

// Head size 80 keeps the register budget of four waves per SIMD (128 VGPRs) although its LDS admits three
// workgroups per CU: the compiler's schedule within 168 registers ran slower.
template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 96 ? 4 : 1, D <= 96 ? 4 : 8)))
relpos_attention_kernel(const AttnArgs p) {
  using S = AttnShape<D>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[S::LDS_BYTES / 2];
  uint16_t* sK0 = lds;                             // [NBUF][32 keys][DP]
  uint16_t* sV0 = sK0 + S::NBUF * S::K_ELEMS;      // [NBUF][D dims][VT]
  uint16_t* sR = sV0 + S::NBUF * S::V_ELEMS;       // [128 ring slots][DP], slot = table row & 127
  uint16_t* sP = sR + S::R_ELEMS;                  // [4 waves][16 queries][AT_PW]

  // XCD-aware order: workgroup b runs on XCD b % 8, so each XCD takes a contiguous run of (head, tile) items, tiles
  // innermost: the query tiles of one sequence and head share their keys, values and table rows in that XCD's L2
  const int total = p.n_tiles * p.H, per = total / 8, rem = total % 8;
  const int xcd = (int)blockIdx.x % 8, item = xcd * per + min(xcd, rem) + (int)blockIdx.x / 8;
  const int4 tile = reinterpret_cast<const int4*>(p.tiles)[item % p.n_tiles];
  const int start = tile.x, len = tile.y, q0 = tile.z, h = item / p.n_tiles;
  const int tid = threadIdx.x, w = wave_id(), lane = lane_id(), iq = lane & 15, g = lane >> 4;
  const int HD = p.H * D, ld = 3 * HD;
  uint16_t* sPw = sP + w * 16 * AT_PW;

  // this lane's query plus either bias, as the B operand of both products
  const int qrow = q0 + 16 * w + iq;
  const bool qvalid = qrow < len;
  const uint16_t* qptr = p.qkv + (int64_t)(start + (qvalid ? qrow : 0)) * ld + h * D;
  HeadDot<D> qu, qv;
  qu.load(qptr, p.bu + h * D, g, qvalid);
  qv.load(qptr, p.bv + h * D, g, qvalid);

  v4f o[S::OB];
#pragma unroll
  for (int i = 0; i < S::OB; ++i) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;  // running maximum (natural units) and sum of this lane's query

  const uint16_t* kbase = p.qkv + (int64_t)start * ld + HD + h * D;
  const uint16_t* vbase = kbase + HD;
  const uint16_t* rbase = p.rk + h * D;
  constexpr int CH = D / 8;  // 16-byte chunks per row
  // a key tile's global data: keys j0 .. j0 + 31, their values, and the 32 table rows of distances
  // q0 - j0 - 31 .. q0 - j0 (the tile reads distances up to q0 - j0 + 63; the previous tiles brought those). Loaded
  // into registers one tile ahead, so the loads of tile j0 + 32 fly while tile j0 computes. Chunk item x of a thread
  // is (row id / CH, chunk id % CH) for keys and table rows; for values it is (key pair item % 16, chunk item / 16),
  // so that the pair's 8 dims go to LDS as 8 dwords of the transposed tile with the lanes of a wave on distinct
  // banks. 32-bit element offsets from uniform bases (a layer's qkv and table stay below 2^31 elements); keys past
  // the sequence load its last key (their scores are masked and their probabilities exactly 0, the values finite, so
  // no register is zeroed) and table rows are clamped to the table.
  constexpr int NC = (AT_KEYS * CH + 255) / 256;      // key / table chunks per thread
  constexpr int NV = (AT_KEYS / 2 * CH + 255) / 256;  // value chunk pairs per thread
  uint4 pk[NC], pr[NC], pw[NV][2];
#pragma unroll
  for (int x = 0; x < NC; ++x) pk[x] = pr[x] = make_uint4(0, 0, 0, 0);  // once: the chunks past 32 rows
#pragma unroll
  for (int x = 0; x < NV; ++x) pw[x][0] = pw[x][1] = make_uint4(0, 0, 0, 0);
  auto fetch = [&](int j0) {
    const int d0 = q0 - j0 - (AT_KEYS - 1) + p.rel_off;  // table row of the tile's first new distance
#pragma unroll
    for (int x = 0; x < NC; ++x) {
      const int id = tid + x * 256;
      if (id < AT_KEYS * CH) {
        const int r = id / CH, c = (id % CH) * 8, key = min(j0 + r, len - 1);
        pk[x] = ld16(kbase, (uint32_t)key * (uint32_t)ld + (uint32_t)c);
        const int trow = min(max(d0 + r, 0), p.rel_rows - 1);
        pr[x] = ld16(rbase, (uint32_t)trow * (uint32_t)HD + (uint32_t)c);
      }
    }
#pragma unroll
    for (int x = 0; x < NV; ++x) {
      const int item = tid + x * 256;
      if (item < AT_KEYS / 2 * CH) {
        const int rp = item % 16, c = (item / 16) * 8;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int key = min(j0 + 2 * rp + k, len - 1);
          pw[x][k] = ld16(vbase, (uint32_t)key * (uint32_t)ld + (uint32_t)c);
        }
      }
    }
  };
  auto stash = [&](int j0, uint16_t* sK, uint16_t* sVt) {
#pragma unroll
    for (int x = 0; x < NC; ++x) {
      const int id = tid + x * 256;
      if (id < AT_KEYS * CH) {
        const int r = id / CH, c = (id % CH) * 8;
        *reinterpret_cast<uint4*>(sK + r * S::DP + c) = pk[x];
        const int d = q0 - j0 - (AT_KEYS - 1) + r;
        *reinterpret_cast<uint4*>(sR + ((d + p.rel_off) & (AT_RING - 1)) * S::DP + c) = pr[x];
      }
    }
#pragma unroll
    for (int x = 0; x < NV; ++x) {
      const int item = tid + x * 256;
      if (item < AT_KEYS / 2 * CH) {
        const int rp = item % 16, c = (item / 16) * 8;
        const uint32_t a[4] = {pw[x][0].x, pw[x][0].y, pw[x][0].z, pw[x][0].w};
        const uint32_t b[4] = {pw[x][1].x, pw[x][1].y, pw[x][1].z, pw[x][1].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          *reinterpret_cast<uint32_t*>(sVt + (c + 2 * k) * S::VT + 2 * rp) = (a[k] & 0xffffu) | (b[k] << 16);
          *reinterpret_cast<uint32_t*>(sVt + (c + 2 * k + 1) * S::VT + 2 * rp) = (a[k] >> 16) | (b[k] & 0xffff0000u);
        }
      }
    }
  };
  // the first tile also reads distances q0 + 1 .. q0 + 63, straight into the ring
  for (int id = tid; id < (AT_Q - 1) * CH; id += 256) {
    const int d = q0 + 1 + id / CH, c = (id % CH) * 8;
    const int trow = min(max(d + p.rel_off, 0), p.rel_rows - 1);
    *reinterpret_cast<uint4*>(sR + ((d + p.rel_off) & (AT_RING - 1)) * S::DP + c) =
        *reinterpret_cast<const uint4*>(p.rk + (int64_t)trow * HD + h * D + c);
  }

  // one key tile from the given key and value buffers: scores, the online softmax and the value product
  constexpr float L2E = 1.4426950408889634f;
  auto key_tile = [&](int j0, const uint16_t* sK, const uint16_t* sVt) {
    // position term of this wave's queries: distances dw0 + db, db < 48 (3 blocks of 16), its three products
    // interleaved per k step; then the content scores of keys kb * 16 + 4 g + e while those finish
    const int dw0 = q0 + 16 * w - j0 - (AT_KEYS - 1);
    const uint16_t* rrow[3];
#pragma unroll
    for (int pb = 0; pb < 3; ++pb) rrow[pb] = sR + ((dw0 + pb * 16 + iq + p.rel_off) & (AT_RING - 1)) * S::DP;
    v4f acc[3], s[2];
#pragma unroll
    for (int pb = 0; pb < 3; ++pb) acc[pb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < HeadDot<D>::steps; ++ks)
#pragma unroll
      for (int pb = 0; pb < 3; ++pb) acc[pb] = qv.step(rrow[pb], g, ks, acc[pb]);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[kb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < HeadDot<D>::steps; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) s[kb] = qu.step(sK + (kb * 16 + iq) * S::DP, g, ks, s[kb]);
    // the position scores rounded as the module rounds them, to the wave's buffer
#pragma unroll
    for (int pb = 0; pb < 3; ++pb) {
      uint2 u;
      u.x = pack_bf2(round_bf(acc[pb][0]) * p.scale, round_bf(acc[pb][1]) * p.scale);
      u.y = pack_bf2(round_bf(acc[pb][2]) * p.scale, round_bf(acc[pb][3]) * p.scale);
      *reinterpret_cast<uint2*>(sPw + iq * AT_PW + pb * 16 + g * 4) = u;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's position rows, written by other lanes
    // the 8 position scores of this lane, read together: key k = kb·16 + 4g + e sits at element
    // iq·(AT_PW + 1) + 31 - k of the wave's buffer, inside it for every key, so no read waits under the key mask.
    // Eight half-word reads from one base, written out so that the compiler neither fuses neighbours into misaligned
    // wider reads nor moves each read under the mask, one after another.
    float pos[8];
    {
      const uint32_t a = (uint32_t)reinterpret_cast<uintptr_t>(sPw + iq * AT_PW + iq + AT_KEYS - 1 - g * 4 - 19);
      uint32_t r[8];
      asm volatile(
          "ds_read_u16 %0, %8 offset:38\n\tds_read_u16 %1, %8 offset:36\n\tds_read_u16 %2, %8 offset:34\n\t"
          "ds_read_u16 %3, %8 offset:32\n\tds_read_u16 %4, %8 offset:6\n\tds_read_u16 %5, %8 offset:4\n\t"
          "ds_read_u16 %6, %8 offset:2\n\tds_read_u16 %7, %8\n\ts_waitcnt lgkmcnt(0)"
          : "=v"(r[0]), "=v"(r[1]), "=v"(r[2]), "=v"(r[3]), "=v"(r[4]), "=v"(r[5]), "=v"(r[6]), "=v"(r[7])
          : "v"(a)
          : "memory");
#pragma unroll
      for (int k = 0; k < 8; ++k) pos[k] = __uint_as_float(r[k] << 16);
    }

    // scores (masked past the sequence in the last tile); online softmax per query (the 4 lane groups hold its
    // 32 keys). exp(v - mx) is taken as exp2(v log2 e - mx log2 e).
    float sv[8], mx = m;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[kb * 4 + e] = __builtin_fmaf(s[kb][e], p.scale, pos[kb * 4 + e]);
    if (j0 + AT_KEYS > len) {
#pragma unroll
      for (int k = 0; k < 8; ++k) sv[k] = j0 + (k >> 2) * 16 + g * 4 + (k & 3) < len ? sv[k] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) mx = fmaxf(mx, sv[k]);
    mx = xor32_max(xor16_max(mx));
    const float alpha = __builtin_amdgcn_exp2f((m - mx) * L2E), nb = -mx * L2E;
    m = mx;
    float rs = 0.f;
    v8bf pb;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[k], L2E, nb));
      rs += e;
      pb[k] = (__bf16)e;
    }
    rs = xor32_sum(xor16_sum(rs));
    l = l * alpha + rs;
    // the rescale only when some query of the wave has a new maximum (alpha == 1 elsewhere: o * 1 is o, bit for bit)
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int ob = 0; ob < S::OB; ++ob) o[ob] *= alpha;
    }
#pragma unroll
    for (int ob = 0; ob < S::OB; ++ob) {
      const uint16_t* vrow = sVt + (ob * 16 + iq) * S::VT;
      const uint2 lo = *reinterpret_cast<const uint2*>(vrow + g * 4);
      const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 + g * 4);
      const v8bf va = __builtin_bit_cast(v8bf, make_uint4(lo.x, lo.y, hi.x, hi.y));
      o[ob] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, o[ob], 0, 0, 0);
    }
  };

  fetch(0);
  if constexpr (S::NBUF == 2) {
    // tile t computes from buffer t & 1 while tile t + 1's data goes to the other one; the barrier after each tile
    // publishes the next tile and retires the reads of this one. The table rows tile t + 1 adds to the ring
    // (distances q0 - j0 - 63 .. q0 - j0 - 32) are not among the 96 that tile t reads (q0 - j0 - 31 .. q0 - j0 + 64),
    // modulo the ring's 128, so they are written while tile t computes
    stash(0, sK0, sV0);
    __syncthreads();
    for (int j0 = 0, t = 0; j0 < len; j0 += AT_KEYS, ++t) {
      const bool more = j0 + AT_KEYS < len;
      if (more) fetch(j0 + AT_KEYS);
      key_tile(j0, sK0 + (t & 1) * S::K_ELEMS, sV0 + (t & 1) * S::V_ELEMS);
      if (more) stash(j0 + AT_KEYS, sK0 + ((t + 1) & 1) * S::K_ELEMS, sV0 + ((t + 1) & 1) * S::V_ELEMS);
      __syncthreads();
    }
  } else {
    for (int j0 = 0; j0 < len; j0 += AT_KEYS) {
      stash(j0, sK0, sV0);
      __syncthreads();
      if (j0 + AT_KEYS < len) fetch(j0 + AT_KEYS);
      key_tile(j0, sK0, sV0);
      __syncthreads();  // every wave is done with the key and value tiles
    }
  }

  if (!qvalid) return;
  const float inv = 1.f / l;
  uint16_t* dst = p.out + (int64_t)(start + qrow) * HD + h * D;
#pragma unroll
  for (int ob = 0; ob < S::OB; ++ob) {
    uint2 u;
    u.x = pack_bf2(o[ob][0] * inv, o[ob][1] * inv);
    u.y = pack_bf2(o[ob][2] * inv, o[ob][3] * inv);
    *reinterpret_cast<uint2*>(dst + ob * 16 + g * 4) = u;
  }
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

template <bool Q8>
int dwconv_entry(const uint16_t* x, const float* w, const float* cb, const float* bn_scale, const float* bn_shift,
                 const int32_t* seq_lo, const int32_t* seq_hi, uint16_t* y, int8_t* q, float* qs, int64_t rows,
                 int64_t C, int64_t K, void* stream, const char* name) {
  const std::string nm(name);
  COHERE_REQUIRE(rows >= 0 && C > 0 && C % 8 == 0 && C <= 2048, nm + ": channels must be a multiple of 8, at most 2048");
  COHERE_REQUIRE(K == DW_K, nm + ": kernel size must be 9");
  COHERE_REQUIRE(x && w && cb && bn_scale && bn_shift && seq_lo && seq_hi && al16(x) && al16(w) && al16(cb) &&
                     al16(bn_scale) && al16(bn_shift),
                 nm + ": bad pointer (x, the taps and the per-channel vectors 16-byte aligned)");
  COHERE_REQUIRE(Q8 ? (q && qs && (reinterpret_cast<uintptr_t>(q) & 7) == 0) : (y && al16(y)),
                 nm + ": bad output pointer");
  if (rows == 0) return 0;
  const int threads = (int)((C / DW_CH + 63) / 64 * 64);
  const int grid = (int)((rows + DW_ROWS - 1) / DW_ROWS);
  dwconv_kernel<Q8><<<grid, threads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi, y, q, qs, (int)rows, (int)C);
  return cohere::check_launch(name);
}

}  // namespace

extern "C" int cohere_dwconv_bn_silu(const uint16_t* x, const float* w, const float* cb, const float* bn_scale,
                                     const float* bn_shift, const int32_t* seq_lo, const int32_t* seq_hi, uint16_t* y,
                                     int64_t rows, int64_t channels, int64_t ksize, void* stream) {
  cohere::clear_error();
  return dwconv_entry<false>(x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi, y, nullptr, nullptr, rows, channels, ksize,
                             stream, "dwconv_bn_silu");
}

extern "C" int cohere_dwconv_bn_silu_q8(const uint16_t* x, const float* w, const float* cb, const float* bn_scale,
                                        const float* bn_shift, const int32_t* seq_lo, const int32_t* seq_hi,
                                        int8_t* hq, float* hs, int64_t rows, int64_t channels, int64_t ksize,
                                        void* stream) {
  cohere::clear_error();
  return dwconv_entry<true>(x, w, cb, bn_scale, bn_shift, seq_lo, seq_hi, nullptr, hq, hs, rows, channels, ksize,
                            stream, "dwconv_bn_silu_q8");
}

extern "C" int cohere_relpos_attention(const uint16_t* qkv, const uint16_t* rk, int64_t rel_rows, const uint16_t* bu,
                                       const uint16_t* bv, const int32_t* tiles, int64_t n_tiles, int64_t heads,
                                       int64_t head_dim, int64_t rel_off, int64_t max_len, float scale, uint16_t* out,
                                       void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(head_dim == 80 || head_dim == 160, "relpos_attention: head size must be 80 or 160");
  COHERE_REQUIRE(heads > 0 && heads <= 65535 && n_tiles >= 0, "relpos_attention: bad sizes");
  COHERE_REQUIRE(qkv && rk && bu && bv && tiles && out && al16(qkv) && al16(rk) && al16(bu) && al16(bv) && al16(out) &&
                     al16(tiles),
                 "relpos_attention: pointers must be 16-byte aligned");
  COHERE_REQUIRE(max_len - 1 <= rel_off && rel_off + max_len + AT_Q - 2 < rel_rows,
                 "relpos_attention: sequence too long for the distance table (" + std::to_string(max_len) + ")");
  if (n_tiles == 0) return 0;
  AttnArgs p;
  p.qkv = qkv; p.rk = rk; p.bu = bu; p.bv = bv; p.out = out; p.tiles = tiles;
  COHERE_REQUIRE(n_tiles * heads < (1LL << 31), "relpos_attention: too many tiles");
  p.H = (int)heads; p.rel_off = (int)rel_off; p.rel_rows = (int)rel_rows; p.n_tiles = (int)n_tiles; p.scale = scale;
  const dim3 grid((unsigned)(n_tiles * heads));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 160)
    relpos_attention_kernel<160><<<grid, 256, 0, s>>>(p);
  else
    relpos_attention_kernel<80><<<grid, 256, 0, s>>>(p);
  return cohere::check_launch("relpos_attention");
}
