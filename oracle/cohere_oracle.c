/* CPU restatement of cohere-inference's quantized-GEMM arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests, smoke() and bench.py's cpu_baseline leg
 * compare the HIP kernels against; the product path never calls it.
 *
 * Every function follows a cited reference location (paths relative to the reference repository root) and keeps its
 * roundings: fp32 divides and multiplies are single IEEE operations, fmaf() is the correctly rounded fused multiply-add
 * (built with -ffp-contract=off so the compiler adds no others), bf16 conversions round to nearest even, and
 * rintf() rounds half to even under the default rounding mode.
 *
 * Pinning (what checks each function against something other than itself) is listed in oracle/__init__.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { EPI_BIAS = 0, EPI_SILU = 1, EPI_RELU = 2, EPI_RESID = 3, EPI_GLU = 4, EPI_SILU_Q8 = 5, EPI_I32 = 7 };

static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float round_bf(float f) { return bf2f(f2bf(f)); }

/* the textbook logistic in fp32 (the reference's kernels use a fast exp; the tests allow for the difference) */
static inline float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

static void set_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
}

/* a1: kernels/fast_encoder.py:60-63 quantize_rows (weights, per output channel):
 * s = max(amax|w|, 1e-12) / 127; q = clamp(round_half_even(w / s), -127, 127). w holds the bf16 weights as fp32.
 * The reference quantizes the weights where the model lives, on the GPU, and PyTorch's GPU division of a tensor by a
 * Python scalar is a multiplication by the scalar's fp32 reciprocal (ATen div_true on a CPU scalar: a * (1 / b)), so
 * the scale is max(amax, 1e-12) * fp32(1 / 127); the division w / s is tensor by tensor, a true division. */
void orc_quantize_weight_rows(const float* w, int64_t n, int64_t k, int8_t* q, float* s) {
  for (int64_t r = 0; r < n; ++r) {
    const float* row = w + r * k;
    float mx = 0.f;
    for (int64_t c = 0; c < k; ++c) mx = fmaxf(mx, fabsf(row[c]));
    const float sc = fmaxf(mx, 1e-12f) * (1.f / 127.f);
    s[r] = sc;
    for (int64_t c = 0; c < k; ++c) {
      float v = rintf(row[c] / sc);
      v = fminf(fmaxf(v, -127.f), 127.f);
      q[r * k + c] = (int8_t)v;
    }
  }
}

/* a2: kernels/csrc/encoder_ops.cu:18-42 store_q8 (used by quantize_rows 45-54, layernorm_q8 57-79):
 * mx = max|x| over the bf16 row; s = mx > 0 ? mx / 127 : 1; inv = 1 / s; q = rint_half_even(clamp(x * inv, +-127)). */
void orc_q8_rows(const uint16_t* x, int64_t ldx, int64_t rows, int64_t cols, int8_t* q, int64_t ldq, float* s) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* row = x + r * ldx;
    float mx = 0.f;
    for (int64_t c = 0; c < cols; ++c) mx = fmaxf(mx, fabsf(bf2f(row[c])));
    const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
    s[r] = sc;
    for (int64_t c = 0; c < cols; ++c) {
      const float v = fminf(fmaxf(bf2f(row[c]) * inv, -127.f), 127.f);
      q[r * ldq + c] = (int8_t)rintf(v);
    }
  }
}

/* int32 dot product of two int8 rows (exact) */
static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int64_t k) {
  int32_t acc = 0;
  for (int64_t i = 0; i < k; ++i) acc += (int32_t)a[i] * (int32_t)b[i];
  return acc;
}

/* a3, a4, a5: kernels/csrc/gemm_int8.cu:146-163 (grouped fold), 201-288 (epilogues).
 *   acc_g = sum over K-group g of A[m,k] W[n,k] (int32, exact)
 *   per-row scales (group == K):  x = fmul((float)acc, sa[m])
 *   grouped (group < K):          x = fmaf((float)acc_g, sa[m,g], x) over g in order, from 0
 *   v = bias ? fmaf(x, sw[n], bias[n]) : fmul(x, sw[n])
 *   EPI_BIAS     out = bf16(v)
 *   EPI_RESID    out = bf16(fmaf(alpha, bf16(v), resid))            (out may alias resid)
 *   EPI_GLU      out[:, j] = bf16(bf16(v[2j]) * sigmoid(bf16(v[2j+1])))
 *   EPI_SILU_Q8  u = bf16(t * sigmoid(t)), t = bf16(v); int8 per (row, qgroup columns) as store_q8, scale to qs
 *   EPI_I32      out = acc (int32; per-row scales only; a parity hook with no counterpart in the reference)
 * acc_out (optional, M x N int32, per-row scales only) receives the raw accumulators. */
int orc_gemm_i8(const int8_t* a, int64_t lda, const float* sa, int64_t ldsa, int64_t group, const int8_t* w,
                int64_t ldw, const float* sw, const uint16_t* bias, void* out, int64_t ldc, int epi,
                const uint16_t* resid, int64_t ldr, float alpha, float* qs, int64_t ldqs, int64_t qgroup, int64_t M,
                int64_t N, int64_t K, int32_t* acc_out, int nthreads) {
  if (group <= 0 || K % group != 0) return -1;
  if (epi == EPI_SILU_Q8 && (qgroup <= 0 || N % qgroup != 0)) return -2;
  if (epi == EPI_GLU && N % 2 != 0) return -3;
  const int grouped = group < K;
  if (grouped && (epi == EPI_I32 || acc_out)) return -4;
  const int64_t G = K / group;
  set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t m = 0; m < M; ++m) {
    float* v = (float*)malloc(sizeof(float) * (size_t)N);
    const int8_t* arow = a + m * lda;
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* wrow = w + n * ldw;
      float x;
      if (!grouped) {
        const int32_t acc = dot_i8(arow, wrow, K);
        if (acc_out) acc_out[m * N + n] = acc;
        if (epi == EPI_I32) {
          ((int32_t*)out)[m * ldc + n] = acc;
          continue;
        }
        x = (float)acc * sa[m * ldsa];
      } else {
        x = 0.f;
        for (int64_t g = 0; g < G; ++g) {
          const int32_t acc = dot_i8(arow + g * group, wrow + g * group, group);
          x = fmaf((float)acc, sa[m * ldsa + g], x);
        }
      }
      v[n] = bias ? fmaf(x, sw[n], bf2f(bias[n])) : x * sw[n];
    }
    if (epi == EPI_BIAS) {
      uint16_t* o = (uint16_t*)out + m * ldc;
      for (int64_t n = 0; n < N; ++n) o[n] = f2bf(v[n]);
    } else if (epi == EPI_RESID) {
      uint16_t* o = (uint16_t*)out + m * ldc;
      const uint16_t* r = resid + m * ldr;
      for (int64_t n = 0; n < N; ++n) o[n] = f2bf(fmaf(alpha, round_bf(v[n]), bf2f(r[n])));
    } else if (epi == EPI_GLU) {
      uint16_t* o = (uint16_t*)out + m * ldc;
      for (int64_t j = 0; j < N / 2; ++j) o[j] = f2bf(round_bf(v[2 * j]) * sigmoid(round_bf(v[2 * j + 1])));
    } else if (epi == EPI_SILU_Q8) {
      int8_t* o = (int8_t*)out + m * ldc;
      for (int64_t n = 0; n < N; ++n) {
        const float t = round_bf(v[n]);
        v[n] = round_bf(t * sigmoid(t));
      }
      for (int64_t g0 = 0; g0 < N; g0 += qgroup) {
        float mx = 0.f;
        for (int64_t n = g0; n < g0 + qgroup; ++n) mx = fmaxf(mx, fabsf(v[n]));
        const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
        qs[m * ldqs + g0 / qgroup] = sc;
        for (int64_t n = g0; n < g0 + qgroup; ++n) o[n] = (int8_t)rintf(fminf(fmaxf(v[n] * inv, -127.f), 127.f));
      }
    }
    free(v);
  }
  return 0;
}

/* a6: kernels/sparse.py:26-39 compress_24. Per group of 4 along K: the positions to keep are the nonzero ones in
 * increasing order, then zero ones in increasing order, the first two of that list, sorted; kept values in that order;
 * selector nibble = i0 | i1 << 2, eight nibbles per int32 word, the lowest group in the lowest nibble.
 * Returns -1 when K % 32 != 0, -2 when a group has more than two nonzero values. */
int orc_compress_24(const int8_t* w, int64_t n, int64_t k, int8_t* kept, int32_t* words) {
  if (k % 32 != 0) return -1;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t wd = 0; wd < k / 32; ++wd) {
      uint32_t word = 0;
      for (int gi = 0; gi < 8; ++gi) {
        const int8_t* g = w + r * k + wd * 32 + gi * 4;
        int order[4], cnt = 0, nnz = 0;
        for (int p = 0; p < 4; ++p)
          if (g[p] != 0) order[cnt++] = p, ++nnz;
        if (nnz > 2) return -2;
        for (int p = 0; p < 4; ++p)
          if (g[p] == 0) order[cnt++] = p;
        int i0 = order[0], i1 = order[1];
        if (i0 > i1) {
          const int t = i0;
          i0 = i1;
          i1 = t;
        }
        const int64_t kp = r * (k / 2) + wd * 16 + gi * 2;
        kept[kp] = g[i0];
        kept[kp + 1] = g[i1];
        word |= (uint32_t)(i0 | (i1 << 2)) << (4 * gi);
      }
      words[r * (k / 32) + wd] = (int32_t)word;
    }
  }
  return 0;
}

/* inverse of compress_24: the dense (n, k) int8 matrix the compressed form stands for */
void orc_decompress_24(const int8_t* kept, const int32_t* words, int64_t n, int64_t k, int8_t* w) {
  memset(w, 0, (size_t)(n * k));
  for (int64_t r = 0; r < n; ++r)
    for (int64_t g = 0; g < k / 4; ++g) {
      const uint32_t word = (uint32_t)words[r * (k / 32) + g / 8];
      const int nib = (word >> (4 * (g % 8))) & 15;
      const int i0 = nib & 3, i1 = nib >> 2;
      w[r * k + 4 * g + i0] += kept[r * (k / 2) + 2 * g];
      w[r * k + 4 * g + i1] += kept[r * (k / 2) + 2 * g + 1];
    }
}

/* a7: kernels/sparse.py:42-46 prune_24_magnitude: the two smallest |w| of every group of four along K set to zero.
 * torch.topk leaves the order of equal magnitudes unspecified; here, of equal magnitudes, the higher index is zeroed
 * first (the lowest index is kept). */
void orc_prune_24(const float* w, int64_t n, int64_t k, float* out) {
  for (int64_t i = 0; i < n * k; i += 4) {
    int idx[4] = {0, 1, 2, 3};
    for (int a = 0; a < 4; ++a)
      for (int b = a + 1; b < 4; ++b) {
        const float fa = fabsf(w[i + idx[a]]), fb = fabsf(w[i + idx[b]]);
        /* ascending magnitude; of equal magnitudes the higher index first */
        if (fb < fa || (fb == fa && idx[b] > idx[a])) {
          const int t = idx[a];
          idx[a] = idx[b];
          idx[b] = t;
        }
      }
    for (int p = 0; p < 4; ++p) out[i + p] = w[i + p];
    out[i + idx[0]] = 0.f;
    out[i + idx[1]] = 0.f;
  }
}

/* a10: kernels/stream_decoder.py:38-48 prepare_w8: per output channel s = max(amax|w|, 1e-12) / 127 (on the GPU:
 * max(amax, 1e-12) * fp32(1 / 127), as orc_quantize_weight_rows),
 * u8 = clamp(round_half_even(w / s), +-127) + 128, the bytes of every 16 along K permuted by W8_PERM (physical
 * position j holds logical k = PERM[j]). */
static const int W8_PERM[16] = {0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15};

void orc_prepare_w8(const float* w, int64_t n, int64_t k, uint8_t* q, float* s) {
  for (int64_t r = 0; r < n; ++r) {
    const float* row = w + r * k;
    float mx = 0.f;
    for (int64_t c = 0; c < k; ++c) mx = fmaxf(mx, fabsf(row[c]));
    const float sc = fmaxf(mx, 1e-12f) * (1.f / 127.f);
    s[r] = sc;
    for (int64_t b = 0; b < k; b += 16)
      for (int j = 0; j < 16; ++j) {
        float v = rintf(row[b + W8_PERM[j]] / sc);
        v = fminf(fmaxf(v, -127.f), 127.f) + 128.f;
        q[r * k + b + j] = (uint8_t)v;
      }
  }
}

/* a11: kernels/csrc/dec_w8.cu:46-180 dec_w8_linear: y = bf16(acc * sw[n] + bias[n]) (ReLU), acc the sum of the exact
 * products bf16(x) * (u8 - 128). The kernel sums in fp32 in its own order; here in fp64, rounded to fp32 once. */
void orc_dec_w8_linear(const uint16_t* x, int64_t ldx, const uint8_t* w, const float* sw, const uint16_t* bias,
                       uint16_t* y, int64_t ldy, int relu, int64_t M, int64_t N, int64_t K, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int64_t b = 0; b < K; b += 16)
        for (int j = 0; j < 16; ++j)
          acc += (double)bf2f(x[m * ldx + b + W8_PERM[j]]) * (double)((int)w[n * K + b + j] - 128);
      float v = fmaf((float)acc, sw[n], bias ? bf2f(bias[n]) : 0.f);
      if (relu) v = fmaxf(v, 0.f);
      y[m * ldy + n] = f2bf(v);
    }
  }
}

/* a12: kernels/decoder_kernels.py:19-34 (and F.linear above 32 rows): y = bf16(x W^T + bias) (ReLU), fp32
 * accumulation of bf16 products (here fp64, rounded to fp32 once), the bias added before the single rounding. */
void orc_linear_bf16(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* bias, uint16_t* y,
                     int64_t ldy, int relu, int64_t M, int64_t N, int64_t K, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += (double)bf2f(x[m * ldx + k]) * (double)bf2f(w[n * K + k]);
      float v = (float)(acc + (bias ? (double)bf2f(bias[n]) : 0.0));
      if (relu) v = fmaxf(v, 0.f);
      y[m * ldy + n] = f2bf(v);
    }
}

/* ---- the encoder layer's other producers (row a9's launch loop) ---------------------------------------------- */

/* kernels/csrc/layernorm.cuh:6-43 + encoder_ops.cu:57-79: h = bf16(fmaf((x - mean) * rstd, w, b)) with fp32
 * statistics over the bf16 row (here accumulated in fp64 and rounded to fp32 once; the kernel's warp tree sums in
 * fp32), rstd = 1 / sqrt(var + eps). With w2: x = LN1(x) in place, then h = LN2(x). h may alias x. */
static void ln_row(const float* v, int64_t cols, const uint16_t* w, const uint16_t* b, float eps, float* out) {
  double s = 0.0;
  for (int64_t k = 0; k < cols; ++k) s += v[k];
  const float mean = (float)(s / (double)cols);
  double q = 0.0;
  for (int64_t k = 0; k < cols; ++k) {
    const float d = v[k] - mean;
    q += (double)d * (double)d;
  }
  const float rstd = 1.f / sqrtf((float)(q / (double)cols) + eps);
  for (int64_t k = 0; k < cols; ++k) out[k] = round_bf(fmaf((v[k] - mean) * rstd, bf2f(w[k]), bf2f(b[k])));
}

void orc_layernorm(uint16_t* x, int64_t ldx, const uint16_t* w1, const uint16_t* b1, float eps1, const uint16_t* w2,
                   const uint16_t* b2, float eps2, uint16_t* h, int64_t ldh, int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float* v = (float*)malloc(sizeof(float) * cols * 2);
    float* o = v + cols;
    for (int64_t k = 0; k < cols; ++k) v[k] = bf2f(x[r * ldx + k]);
    ln_row(v, cols, w1, b1, eps1, o);
    if (w2) {
      for (int64_t k = 0; k < cols; ++k) x[r * ldx + k] = f2bf(o[k]);
      memcpy(v, o, sizeof(float) * cols);
      ln_row(v, cols, w2, b2, eps2, o);
    }
    for (int64_t k = 0; k < cols; ++k) h[r * ldh + k] = f2bf(o[k]);
    free(v);
  }
}

/* kernels/csrc/encoder_ops.cu:455-498 (dwconv_tile_kernel) and 559-641 (dwconv_q8_kernel, whose int8 rows are
 * q8_rows of this output): per channel c of row r, acc = cb[c], then for taps k = 0..8 in order, for source row
 * src = r + k - 4 inside [lo[r], hi[r]): acc = fmaf(x[src, c], w[c, k], acc); a = bf16(acc);
 * a = bf16(fmaf(a, bn_scale[c], bn_shift[c])); y = bf16(a * sigmoid(a)). */
void orc_dwconv_bn_silu(const uint16_t* x, const float* w, const float* cb, const float* bn_scale,
                        const float* bn_shift, const int32_t* lo, const int32_t* hi, uint16_t* y, int64_t rows,
                        int64_t C) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < C; ++c) {
      float acc = cb[c];
      for (int k = 0; k < 9; ++k) {
        const int64_t src = r + k - 4;
        if (src < lo[r] || src >= hi[r]) continue;
        acc = fmaf(bf2f(x[src * C + c]), w[c * 9 + k], acc);
      }
      float a = round_bf(acc);
      a = round_bf(fmaf(a, bn_scale[c], bn_shift[c]));
      y[r * C + c] = f2bf(a * sigmoid(a));
    }
}

/* kernels/csrc/encoder_ops.cu:82-337 relpos_attention_kernel, for each (sequence, head, query i):
 *   qu = bf16(q_i + u), qv = bf16(q_i + v) (fp32 adds);
 *   s_j = fmaf(qu . k_j, scale, bf16(bf16(qv . R[clamp(i - j + rel_off)]) * scale)) for keys j of the sequence;
 *   keys in tiles of 32 with the online softmax of the kernel: m' = max(m, max_j s_j), alpha = exp(m - m'),
 *   p_j = exp(s_j - m'), l = l * alpha + sum p_j, o = o * alpha + sum bf16(p_j) v_j; out = bf16(o * (1 / l)).
 * Dot products in fp64, rounded to fp32 once (the kernel accumulates fp32 on the tensor cores). */
void orc_relpos_attention(const uint16_t* qkv, const uint16_t* rk, int64_t rel_rows, const uint16_t* bu,
                          const uint16_t* bv, const int32_t* seq_start, const int32_t* seq_len, int64_t n_seq,
                          int64_t H, int64_t D, int64_t rel_off, float scale, uint16_t* out) {
  const int64_t HD = H * D, ld = 3 * HD;
  for (int64_t sq = 0; sq < n_seq; ++sq) {
    const int64_t start = seq_start[sq], len = seq_len[sq];
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t i = 0; i < len; ++i) {
        float* buf = (float*)malloc(sizeof(float) * (3 * D + 32));
        float *qu = buf, *qv = buf + D, *o = buf + 2 * D, *sv = buf + 3 * D;
        const uint16_t* q = qkv + (start + i) * ld + h * D;
        for (int64_t d = 0; d < D; ++d) {
          qu[d] = round_bf(bf2f(q[d]) + bf2f(bu[h * D + d]));
          qv[d] = round_bf(bf2f(q[d]) + bf2f(bv[h * D + d]));
          o[d] = 0.f;
        }
        float m = -INFINITY, l = 0.f;
        for (int64_t j0 = 0; j0 < len; j0 += 32) {
          const int64_t jn = len - j0 < 32 ? len - j0 : 32;
          float mx = m;
          for (int64_t jj = 0; jj < jn; ++jj) {
            const int64_t j = j0 + jj;
            const uint16_t* k = qkv + (start + j) * ld + HD + h * D;
            int64_t row = i - j + rel_off;
            row = row < 0 ? 0 : (row >= rel_rows ? rel_rows - 1 : row);
            const uint16_t* r = rk + row * HD + h * D;
            double ac = 0.0, bd = 0.0;
            for (int64_t d = 0; d < D; ++d) {
              ac += (double)qu[d] * (double)bf2f(k[d]);
              bd += (double)qv[d] * (double)bf2f(r[d]);
            }
            const float pos = round_bf(round_bf((float)bd) * scale);
            sv[jj] = fmaf((float)ac, scale, pos);
            if (sv[jj] > mx) mx = sv[jj];
          }
          const float alpha = expf(m - mx);
          m = mx;
          float rs = 0.f;
          for (int64_t d = 0; d < D; ++d) o[d] *= alpha;
          for (int64_t jj = 0; jj < jn; ++jj) {
            const float p = expf(sv[jj] - mx);
            rs += p;
            const float pr = round_bf(p);
            const uint16_t* v = qkv + (start + j0 + jj) * ld + 2 * HD + h * D;
            for (int64_t d = 0; d < D; ++d) o[d] = fmaf(pr, bf2f(v[d]), o[d]);
          }
          l = l * alpha + rs;
        }
        const float inv = 1.f / l;
        for (int64_t d = 0; d < D; ++d) out[(start + i) * HD + h * D + d] = f2bf(o[d] * inv);
        free(buf);
      }
  }
}

/* ---- the decoder step's other kernels (row a13) ------------------------------------------------------------------ */

/* kernels/csrc/decoder_ops.cu:24-54: x = LN0(bf16(emb[tok[s]] + ptab[pos[s]])), h = LN1(x) for s = active[r] */
void orc_dec_embed(const int32_t* active, int64_t rows, const int64_t* tok, const int32_t* pos, const uint16_t* emb,
                   const uint16_t* ptab, const uint16_t* w0, const uint16_t* b0, float eps0, const uint16_t* w1,
                   const uint16_t* b1, float eps1, uint16_t* x, uint16_t* h, int64_t width) {
  float* v = (float*)malloc(sizeof(float) * width * 2);
  float* o = v + width;
  for (int64_t r = 0; r < rows; ++r) {
    const int s = active[r];
    for (int64_t c = 0; c < width; ++c) v[c] = round_bf(bf2f(emb[tok[s] * width + c]) + bf2f(ptab[(int64_t)pos[s] * width + c]));
    ln_row(v, width, w0, b0, eps0, o);
    for (int64_t c = 0; c < width; ++c) x[r * width + c] = f2bf(o[c]);
    memcpy(v, o, sizeof(float) * width);
    ln_row(v, width, w1, b1, eps1, o);
    for (int64_t c = 0; c < width; ++c) h[r * width + c] = f2bf(o[c]);
  }
  free(v);
}

/* kernels/csrc/decoder_ops.cu:56-83: x = bf16(x + y), h = LN(x) */
void orc_dec_add_ln(uint16_t* x, const uint16_t* y, int64_t ldy, const uint16_t* w, const uint16_t* b, float eps,
                    uint16_t* h, int64_t rows, int64_t width) {
  float* v = (float*)malloc(sizeof(float) * width * 2);
  float* o = v + width;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < width; ++c) {
      v[c] = round_bf(bf2f(x[r * width + c]) + bf2f(y[r * ldy + c]));
      x[r * width + c] = f2bf(v[c]);
    }
    ln_row(v, width, w, b, eps, o);
    for (int64_t c = 0; c < width; ++c) h[r * width + c] = f2bf(o[c]);
  }
  free(v);
}

/* kernels/csrc/dec_attn.cuh:38-58 store16_q8: a 128-vector as int8 with scale absmax / 127 (1 for a zero vector) */
static void q8_vec(const float* f, int8_t* q, float* scale) {
  float mx = 0.f;
  for (int k = 0; k < 128; ++k) mx = fmaxf(mx, fabsf(f[k]));
  const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
  for (int k = 0; k < 128; ++k) q[k] = (int8_t)rintf(fminf(fmaxf(f[k] * inv, -127.f), 127.f));
  *scale = sc;
}

/* kernels/csrc/dec_attn.cuh:84-188 (attend_item) for every row and head: softmax(q k^T * scale) v over the slot's
 * keys. self: the new key and value (columns H*128 and 2*H*128 of q's row) are written at position n[s] (int8: by
 * q8_vec) and attended unquantized, keys 0 .. n[s]-1 come from the cache; cross: keys 0 .. n[s]-1. Cached values are
 * dequantized as the kernel does (fp32 int8 * scale). Scores: s_j = fp32(q . k_j) * scale; the softmax in fp64 in one
 * pass (the kernel runs it online in fp32 per key group; the order of the sums is not restated). q8 == 0: bf16
 * caches k, v. */
void orc_dec_attention(int self, int q8, const int32_t* active, int64_t rows, const uint16_t* q, int64_t ldq,
                       uint16_t* k, uint16_t* v, int8_t* k8, int8_t* v8, float* ks, float* vs, const int32_t* n,
                       int64_t H, int64_t T, float scale, uint16_t* out) {
  const int64_t HD = 128;
  for (int64_t r = 0; r < rows; ++r) {
    const int s = active[r];
    for (int64_t h = 0; h < H; ++h) {
      const int64_t vec0 = ((int64_t)s * H + h) * T;
      const int nk = n[s];
      float qf[128], kn[128], vn[128], kk[128];
      double acc[128];
      for (int d = 0; d < HD; ++d) qf[d] = bf2f(q[r * ldq + h * HD + d]);
      const int total = nk + (self ? 1 : 0);
      double* sc = (double*)malloc(sizeof(double) * (total > 0 ? total : 1));
      if (self) {
        for (int d = 0; d < HD; ++d) {
          kn[d] = bf2f(q[r * ldq + H * HD + h * HD + d]);
          vn[d] = bf2f(q[r * ldq + 2 * H * HD + h * HD + d]);
        }
      }
      double mx = -INFINITY;
      for (int j = 0; j < total; ++j) {
        const int is_new = self && j == nk;
        if (is_new) {
          memcpy(kk, kn, sizeof kk);
        } else if (q8) {
          for (int d = 0; d < HD; ++d) kk[d] = (float)k8[(vec0 + j) * HD + d] * ks[vec0 + j];
        } else {
          for (int d = 0; d < HD; ++d) kk[d] = bf2f(k[(vec0 + j) * HD + d]);
        }
        double dot = 0.0;
        for (int d = 0; d < HD; ++d) dot += (double)qf[d] * (double)kk[d];
        sc[j] = (double)((float)dot * scale);
        if (sc[j] > mx) mx = sc[j];
      }
      double l = 0.0;
      for (int d = 0; d < HD; ++d) acc[d] = 0.0;
      for (int j = 0; j < total; ++j) {
        const double e = exp(sc[j] - mx);
        l += e;
        const int is_new = self && j == nk;
        for (int d = 0; d < HD; ++d) {
          const float vv = is_new ? vn[d] : (q8 ? (float)v8[(vec0 + j) * HD + d] * vs[vec0 + j] : bf2f(v[(vec0 + j) * HD + d]));
          acc[d] += e * (double)vv;
        }
      }
      for (int d = 0; d < HD; ++d) out[r * H * HD + h * HD + d] = f2bf((float)(acc[d] / l));
      free(sc);
      if (self) {  /* the cache write (after the attention reads: the new position is not read from the cache) */
        if (q8) {
          q8_vec(kn, k8 + (vec0 + nk) * HD, ks + vec0 + nk);
          q8_vec(vn, v8 + (vec0 + nk) * HD, vs + vec0 + nk);
        } else {
          for (int d = 0; d < HD; ++d) {
            k[(vec0 + nk) * HD + d] = f2bf(kn[d]);
            v[(vec0 + nk) * HD + d] = f2bf(vn[d]);
          }
        }
      }
    }
  }
}

/* kernels/csrc/decoder_ops.cu:106-159 dec_pick */
void orc_dec_pick(const uint16_t* logits, int64_t rows, int64_t V, const int32_t* active, int64_t dummy, int64_t* tok,
                  int32_t* pos, uint8_t* finished, const int64_t* forced, int64_t FP, const int32_t* plen,
                  const int32_t* limit, int64_t* out, int64_t OUT, int64_t eos) {
  for (int64_t r = 0; r < rows; ++r) {
    const int s = active[r];
    if (s == dummy || finished[s]) continue;
    float best = -INFINITY;
    int64_t arg = 0;
    for (int64_t i = 0; i < V; ++i) {
      const float v = bf2f(logits[r * V + i]);
      if (v > best) {
        best = v;
        arg = i;
      }
    }
    const int at = pos[s] + 1;
    const int in_prompt = at < plen[s];
    const int64_t nt = in_prompt ? forced[(int64_t)s * FP + at] : arg;
    out[(int64_t)s * OUT + at] = nt;
    tok[s] = nt;
    pos[s] = at;
    finished[s] = (!in_prompt && (nt == eos || at >= limit[s])) ? 1 : 0;
  }
}

/* kernels/csrc/decoder_ops.cu:163-204 dec_scatter_kv(_q8): row i of kv (L x 2 x H x 128 per row) into slot
 * slot_of[i], frame frame_of[i] of the caches (L, S, H, T, 128); q8 by q8_vec per 128-vector */
void orc_dec_scatter_kv(int q8, const uint16_t* kv, int64_t rows, const int32_t* slot_of, const int32_t* frame_of,
                        uint16_t* ck, uint16_t* cv, int8_t* ck8, int8_t* cv8, float* cks, float* cvs, int64_t L,
                        int64_t S, int64_t H, int64_t T) {
  const int64_t HD = 128;
  float f[128];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t l = 0; l < L; ++l)
      for (int kvi = 0; kvi < 2; ++kvi)
        for (int64_t h = 0; h < H; ++h) {
          const uint16_t* src = kv + r * L * 2 * H * HD + ((l * 2 + kvi) * H + h) * HD;
          const int64_t vec = ((l * S + slot_of[r]) * H + h) * T + frame_of[r];
          if (q8) {
            for (int d = 0; d < HD; ++d) f[d] = bf2f(src[d]);
            q8_vec(f, (kvi ? cv8 : ck8) + vec * HD, (kvi ? cvs : cks) + vec);
          } else {
            memcpy((kvi ? cv : ck) + vec * HD, src, HD * 2);
          }
        }
}

/* ---- bf16 GEMM and the encoder's front end (config 4) ----------------------------------------------------------- */

/* kernels/csrc/gemm.cu:150-212: out = epi(a W^T + bias) on bf16 operands. The accumulator (fp32 in the kernel, here
 * fp64 rounded to fp32 once), then in fp32: CONV_RELU rounds it to bf16 first; + bias; BIAS -> bf16; SILU t = bf16(v),
 * t * sigmoid(t); RELU / CONV_RELU max(v, 0); GLU bf16(bf16(v[2j]) * sigmoid(bf16(v[2j+1]))); RESID
 * bf16(fmaf(alpha, bf16(v), r)) (r may be out). */
void orc_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* w, const uint16_t* bias, uint16_t* out,
                   int64_t ldc, int epi, const uint16_t* resid, int64_t ldr, float alpha, int64_t M, int64_t N,
                   int64_t K, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float* v = (float*)malloc(sizeof(float) * N);
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += (double)bf2f(a[m * lda + k]) * (double)bf2f(w[n * K + k]);
      float x = (float)acc;
      if (epi == 6) x = round_bf(x);
      if (bias) x = x + bf2f(bias[n]);
      v[n] = x;
    }
    uint16_t* o = out + m * ldc;
    if (epi == 4) {
      for (int64_t j = 0; j < N / 2; ++j) o[j] = f2bf(round_bf(v[2 * j]) * sigmoid(round_bf(v[2 * j + 1])));
    } else {
      for (int64_t n = 0; n < N; ++n) {
        float x = v[n];
        if (epi == 1) {
          const float t = round_bf(x);
          x = t * sigmoid(t);
        } else if (epi == 2 || epi == 6) {
          x = fmaxf(x, 0.f);
        } else if (epi == 3) {
          x = fmaf(alpha, round_bf(x), bf2f(resid[m * ldr + n]));
        }
        o[n] = f2bf(x);
      }
    }
    free(v);
  }
}

/* in-place radix-2 FFT of n (a power of two) complex doubles, forward (e^{-2 pi i k n / N}) */
static void fft_double(double* re, double* im, int n) {
  for (int i = 1, j = 0; i < n; ++i) {
    int bit = n >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) {
      double t = re[i]; re[i] = re[j]; re[j] = t;
      t = im[i]; im[i] = im[j]; im[j] = t;
    }
  }
  for (int len = 2; len <= n; len <<= 1) {
    for (int i = 0; i < n; i += len)
      for (int k = 0; k < len / 2; ++k) {
        const double ang = -2.0 * 3.14159265358979323846 * k / len, c = cos(ang), s = sin(ang);
        const double xr = re[i + k + len / 2], xi = im[i + k + len / 2];
        const double tr = xr * c - xi * s, ti = xr * s + xi * c;
        re[i + k + len / 2] = re[i + k] - tr;
        im[i + k + len / 2] = im[i + k] - ti;
        re[i + k] += tr;
        im[i + k] += ti;
      }
  }
}

/* kernels/csrc/features.cu:34-102 (and kernels/features.py:90-108, transformers' CohereAsrFeatureExtractor): for each
 * valid frame t < n / 160 of each piece, the 512 samples centred at 160 t, pre-emphasised (x[s] - fp32(p x[s-1])),
 * zero outside the piece, times the window (fp32); the real DFT (here in fp64, rounded to fp32); power
 * fp32(sqrt(re^2 + im^2))^2; mel bands as fp32 fma over their nonzero bins in order; log(mel + 2^-24); then per piece
 * and band (v - mean) / (std + 1e-5) with fp64 mean and unbiased variance, bf16 into out [pieces, T, 128] (other
 * frames untouched). meta as cohere_logmel_features: first sample, length, cumulative valid frames. */
void orc_logmel(const float* x, const int64_t* meta, int64_t pieces, const float* window, const float* mel,
                const int32_t* band, float preemph, uint16_t* out, int64_t T, int nthreads) {
  enum { NF = 512, NB = 257, NM = 128 };
  set_threads(nthreads);
  const int64_t* frame_start = meta + 2 * pieces;
  const int64_t total = frame_start[pieces];
  float* lm = (float*)malloc(sizeof(float) * (total > 0 ? total : 1) * NM);
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t f = 0; f < total; ++f) {
    int64_t p = 0;
    while (p + 1 < pieces && frame_start[p + 1] <= f) ++p;
    const int64_t t = f - frame_start[p], n = meta[pieces + p];
    const float* xp = x + meta[p];
    double re[NF], im[NF];
    for (int j = 0; j < NF; ++j) {
      const int64_t s = t * 160 - NF / 2 + j;
      float e = 0.f;
      if (s >= 0 && s < n) e = s == 0 ? xp[0] : xp[s] - preemph * xp[s - 1];
      re[j] = (double)(e * window[j]);
      im[j] = 0.0;
    }
    fft_double(re, im, NF);
    float pw[NB];
    for (int k = 0; k < NB; ++k) {
      const float r = (float)re[k], i = (float)im[k];
      const float a = sqrtf(r * r + i * i);
      pw[k] = a * a;
    }
    for (int m = 0; m < NM; ++m) {
      float acc = 0.f;
      for (int k = band[2 * m]; k < band[2 * m + 1]; ++k) acc = fmaf(mel[m * NB + k], pw[k], acc);
      lm[f * NM + m] = logf(acc + 5.9604644775390625e-8f);
    }
  }
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < pieces; ++p) {
    const int64_t f0 = frame_start[p], nv = frame_start[p + 1] - f0;
    if (nv == 0) continue;
    for (int m = 0; m < NM; ++m) {
      double s = 0.0;
      for (int64_t t = 0; t < nv; ++t) s += lm[(f0 + t) * NM + m];
      const float mean = (float)(s / (double)nv);
      double q = 0.0;
      for (int64_t t = 0; t < nv; ++t) {
        const double d = (double)lm[(f0 + t) * NM + m] - (double)mean;
        q += d * d;
      }
      const float den = (float)sqrt(q / (double)(nv - 1)) + 1e-5f;
      for (int64_t t = 0; t < nv; ++t) out[(p * T + t) * NM + m] = f2bf((lm[(f0 + t) * NM + m] - mean) / den);
    }
  }
  free(lm);
}

/* kernels/csrc/encoder_ops.cu:339-413 (transformers' ParakeetEncoderSubsamplingConv2D layers 0-2 per sequence):
 * conv0 (1 -> C, 3x3, stride 2, padding 1) as an fp32 fma chain over its taps row by row from 0, rounded to bf16, +
 * bias, rounded again, ReLU; then the depthwise 3x3 stride-2 convolution from its bias, an fp32 fma per tap row by
 * row, one rounding. Rows of conv0 / the mel input outside the sequence are zeros. out [n_rows, 32, C]. */
void orc_sub_conv0_dw(const uint16_t* feats, int64_t ld_seq, const int32_t* mel_len, const int32_t* rows,
                      int64_t n_rows, const float* w0, const float* b0, const float* w2, const float* b2, uint16_t* out,
                      int64_t C, int nthreads) {
  enum { NM = 128, F1 = 64, F2 = 32 };
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n_rows; ++i) {
    const int seq = rows[2 * i], t2 = rows[2 * i + 1], L = mel_len[seq], T1 = (L - 1) / 2 + 1;
    const uint16_t* xs = feats + seq * ld_seq;
    for (int64_t c = 0; c < C; ++c) {
      float c0[3][F1];  /* conv0 rows 2 t2 - 1 .. 2 t2 + 1, after ReLU; zero outside */
      for (int r = 0; r < 3; ++r) {
        const int t1 = 2 * t2 - 1 + r;
        for (int f1 = 0; f1 < F1; ++f1) {
          if (t1 < 0 || t1 >= T1) { c0[r][f1] = 0.f; continue; }
          float s = 0.f;
          for (int di = 0; di < 3; ++di)
            for (int dj = 0; dj < 3; ++dj) {
              const int mr = 2 * t1 - 1 + di, mc = 2 * f1 - 1 + dj;
              const float v = (mr >= 0 && mr < L && mc >= 0 && mc < NM) ? bf2f(xs[(int64_t)mr * NM + mc]) : 0.f;
              s = fmaf(w0[c * 9 + di * 3 + dj], v, s);
            }
          c0[r][f1] = fmaxf(round_bf(round_bf(s) + b0[c]), 0.f);
        }
      }
      for (int f2 = 0; f2 < F2; ++f2) {
        float acc = b2[c];
        for (int r = 0; r < 3; ++r) {
          if (2 * t2 - 1 + r < 0 || 2 * t2 - 1 + r >= T1) continue;
          for (int dj = 0; dj < 3; ++dj) {
            const int f1 = 2 * f2 - 1 + dj;
            if (f1 < 0 || f1 >= F1) continue;
            acc = fmaf(w2[c * 9 + r * 3 + dj], c0[r][f1], acc);
          }
        }
        out[(i * F2 + f2) * C + c] = f2bf(acc);
      }
    }
  }
}

/* kernels/csrc/encoder_ops.cu:415-448: depthwise 3x3 stride-2 convolution + bias on channels-last sequences x
 * [sum T_in, F_in, C] (in_start / in_len per sequence), from the bias, an fp32 fma per tap row by row, one rounding:
 * out [n_rows, F_in / 2, C] for rows (sequence, t). */
void orc_sub_dw(const uint16_t* x, const int32_t* in_start, const int32_t* in_len, const int32_t* rows, int64_t n_rows,
                const float* w, const float* b, uint16_t* out, int64_t F_in, int64_t C, int nthreads) {
  set_threads(nthreads);
  const int64_t F_out = F_in / 2;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n_rows; ++i) {
    const int seq = rows[2 * i], t = rows[2 * i + 1], start = in_start[seq], len = in_len[seq];
    for (int64_t f = 0; f < F_out; ++f)
      for (int64_t c = 0; c < C; ++c) {
        float acc = b[c];
        for (int di = 0; di < 3; ++di) {
          const int ti = 2 * t - 1 + di;
          if (ti < 0 || ti >= len) continue;
          for (int dj = 0; dj < 3; ++dj) {
            const int64_t fi = 2 * f - 1 + dj;
            if (fi < 0 || fi >= F_in) continue;
            acc = fmaf(w[c * 9 + di * 3 + dj], bf2f(x[(((int64_t)start + ti) * F_in + fi) * C + c]), acc);
          }
        }
        out[(i * F_out + f) * C + c] = f2bf(acc);
      }
  }
}

/* bf16 <-> fp32 helpers exported for the Python side of the checker */
void orc_f32_to_bf16(const float* f, uint16_t* h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) h[i] = f2bf(f[i]);
}
void orc_bf16_to_f32(const uint16_t* h, float* f, int64_t n) {
  for (int64_t i = 0; i < n; ++i) f[i] = bf2f(h[i]);
}
