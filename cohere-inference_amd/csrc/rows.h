// Row helpers of the one-wave-per-row kernels (quantizers, LayerNorms, the decoder's embedding and residual
// LayerNorms): a row of up to VEC x 512 bf16 values held by one wave, 8 consecutive values per lane per chunk.
#pragma once
#include "common.h"

namespace cohere_rows {

template <int VEC>
struct Row {
  float v[VEC][8];
};

// FULL: cols == VEC * 512, so every lane's chunks are in the row and the loads need no guard (a guarded load is a
// branch, and the compiler waits for every load in flight where the branches join)
template <int VEC, bool FULL = false>
DEVI void load_row(const uint16_t* x, int cols, int lane, Row<VEC>& r) {
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int c = (i * 64 + lane) * 8;
    uint4 u = make_uint4(0, 0, 0, 0);
    if (FULL || c < cols) u = *reinterpret_cast<const uint4*>(x + c);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r.v[i][2 * k] = __uint_as_float(w[k] << 16);
      r.v[i][2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
}

// the row (already bf16 values) as int8 with one scale per row
template <int VEC>
DEVI void store_q8(const Row<VEC>& r, int cols, int lane, int8_t* q, float* scale) {
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(r.v[i][k]));
  mx = wave_max_xor(mx, 64);
  const float s = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / s;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c >= cols) continue;
    const float* f = r.v[i];
    *reinterpret_cast<uint2*>(q + c) = make_uint2(q8x4(f[0], f[1], f[2], f[3], inv), q8x4(f[4], f[5], f[6], f[7], inv));
  }
  if (lane == 0) *scale = s;
}

DEVI float wave_sum(float v) { return wave_sum64(v); }

// a LayerNorm's weight and bias as this lane's 16-byte chunks (bf16), loaded before the row's statistics so that no
// load waits behind them
template <int VEC>
struct LnParams {
  uint4 w[VEC], b[VEC];
};

template <int VEC, bool FULL = false>
DEVI LnParams<VEC> load_ln(const uint16_t* w, const uint16_t* b, int cols, int lane) {
  LnParams<VEC> p;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int c = (i * 64 + lane) * 8;
    p.w[i] = FULL || c < cols ? *reinterpret_cast<const uint4*>(w + c) : make_uint4(0, 0, 0, 0);
    p.b[i] = FULL || c < cols ? *reinterpret_cast<const uint4*>(b + c) : make_uint4(0, 0, 0, 0);
  }
  return p;
}

// LayerNorm of the row in place (fp32 statistics over the bf16 inputs), the result rounded to bf16
template <int VEC>
DEVI void ln_row(Row<VEC>& r, int cols, int lane, const LnParams<VEC>& p, float eps) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) s += r.v[i][k];
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    if ((i * 64 + lane) * 8 >= cols) continue;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float d = r.v[i][k] - mean;
      q += d * d;
    }
  }
  const float rstd = 1.f / sqrtf(wave_sum(q) / (float)cols + eps);
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c >= cols) continue;
    const uint32_t ww[4] = {p.w[i].x, p.w[i].y, p.w[i].z, p.w[i].w}, bb[4] = {p.b[i].x, p.b[i].y, p.b[i].z, p.b[i].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float wk = __uint_as_float(k & 1 ? ww[k >> 1] & 0xffff0000u : ww[k >> 1] << 16);
      const float bk = __uint_as_float(k & 1 ? bb[k >> 1] & 0xffff0000u : bb[k >> 1] << 16);
      r.v[i][k] = round_bf(__builtin_fmaf((r.v[i][k] - mean) * rstd, wk, bk));
    }
  }
}

template <int VEC>
DEVI void store_row(const Row<VEC>& r, int cols, int lane, uint16_t* x) {
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c >= cols) continue;
    uint4 u;
    u.x = pack_bf2(r.v[i][0], r.v[i][1]);
    u.y = pack_bf2(r.v[i][2], r.v[i][3]);
    u.z = pack_bf2(r.v[i][4], r.v[i][5]);
    u.w = pack_bf2(r.v[i][6], r.v[i][7]);
    *reinterpret_cast<uint4*>(x + c) = u;
  }
}

}  // namespace cohere_rows
