// The encoder's front end on gfx950: normalized log-mel features of packed audio pieces and the subsampling stem's
// convolutions (the stem's pointwise convolutions and final projection are bf16 GEMMs, gemm_bf16.hip).
//
// Reference: kernels/features.py + kernels/csrc/features.cu (log-mel), kernels/csrc/encoder_ops.cu:339-448 and
// kernels/fast_encoder.py:185-202 (subsampling), whose semantics follow transformers' CohereAsrFeatureExtractor and
// ParakeetEncoderSubsamplingConv2D.
//
// logmel_kernel: one wavefront per frame, four frames per workgroup, everything between the samples and the log-mel
// values in registers and LDS -- no frame buffer and no spectrum in HBM. The 512-sample real frame is transformed as a
// 256-point complex FFT of (even, odd) sample pairs: four radix-4 Stockham passes (one butterfly per lane per pass,
// natural order out, no bit reversal) through a per-wave LDS ping-pong buffer, twiddles from a 512-entry table
// computed once per workgroup in double precision; then the usual split into the 257 bins of the real transform,
// |X|^2, the mel bands over their nonzero bins, and log.
#include "cohere_hip.h"
#include "common.h"

namespace {

constexpr int NFFT = 512, HOP = 160, BINS = NFFT / 2 + 1, MELS = 128, NZ = NFFT / 2;
constexpr int FPW = 4;  // frames (waves) per workgroup

struct Cx {
  float re, im;
};
DEVI Cx cadd(Cx a, Cx b) { return {a.re + b.re, a.im + b.im}; }
DEVI Cx csub(Cx a, Cx b) { return {a.re - b.re, a.im - b.im}; }
DEVI Cx cmul(Cx a, Cx b) { return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re}; }
DEVI Cx mul_mi(Cx a) { return {a.im, -a.re}; }  // a * (-i)

// the piece holding flat frame f: the last p with frame_start[p] <= f
DEVI int piece_of(const int64_t* frame_start, int pieces, int64_t f) {
  int lo = 0, hi = pieces - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (frame_start[mid] <= f) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__global__ void __launch_bounds__(FPW * 64) logmel_kernel(const float* __restrict__ x, const int64_t* __restrict__ meta,
                                                          int pieces, int64_t total_frames,
                                                          const float* __restrict__ window,
                                                          const float* __restrict__ mel, const int* __restrict__ band,
                                                          float preemph, float* __restrict__ logmel) {
  __shared__ Cx tw[NFFT];            // e^{-2 pi i k / 512}
  __shared__ Cx buf[FPW][2][NZ];     // Stockham ping-pong, per wave
  __shared__ float power[FPW][BINS + 3];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int k = threadIdx.x; k < NFFT; k += FPW * 64) {
    double s, c;
    sincospi(-(double)k / 256.0, &s, &c);
    tw[k] = {(float)c, (float)s};
  }
  const int64_t f = (int64_t)blockIdx.x * FPW + w;
  const bool live = f < total_frames;
  const int64_t* sample_start = meta;
  const int64_t* lens = meta + pieces;
  const int64_t* frame_start = meta + 2 * pieces;

  // lane j holds z[j + 64 r] = frame[2 (j + 64 r)] + i frame[2 (j + 64 r) + 1], r = 0..3; frame[j] is sample
  // 160 t - 256 + j of the piece, pre-emphasised (x[s] - p x[s-1], the product rounded first), zero outside it, times
  // the centred window
  Cx v[4];
  if (live) {
    const int p = piece_of(frame_start, pieces, f);
    const int64_t t = f - frame_start[p];
    const float* xp = x + sample_start[p];
    const int64_t n = lens[p];
    auto sample = [&](int j) {
      const int64_t s = t * HOP - NFFT / 2 + j;
      float e = 0.f;
      if (s >= 0 && s < n) e = s == 0 ? xp[0] : __fsub_rn(xp[s], __fmul_rn(preemph, xp[s - 1]));
      return __fmul_rn(e, window[j]);
    };
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 2 * (lane + 64 * r);
      v[r] = {sample(j), sample(j + 1)};
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = {0.f, 0.f};
  }
  __syncthreads();  // twiddle table

  // radix-4 Stockham passes, Ns = 1, 4, 16, 64: lane j combines in[j + 64 r] (twiddled by W_{4 Ns}^{r (j % Ns)}) and
  // writes out[(j / Ns) 4 Ns + j % Ns + r Ns]
  int cur = 0;
#pragma unroll
  for (int Ns = 1; Ns < NZ; Ns *= 4) {
    const int jm = lane % Ns;
    if (Ns > 1) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = buf[w][cur][lane + 64 * r];
#pragma unroll
      for (int r = 1; r < 4; ++r) v[r] = cmul(v[r], tw[(r * jm * (128 / Ns)) & (NFFT - 1)]);
      cur ^= 1;
    }
    const Cx a0 = cadd(v[0], v[2]), a1 = csub(v[0], v[2]), a2 = cadd(v[1], v[3]), a3 = mul_mi(csub(v[1], v[3]));
    const int o = (lane / Ns) * 4 * Ns + jm;
    buf[w][cur][o] = cadd(a0, a2);
    buf[w][cur][o + Ns] = cadd(a1, a3);
    buf[w][cur][o + 2 * Ns] = csub(a0, a2);
    buf[w][cur][o + 3 * Ns] = csub(a1, a3);
    __syncthreads();
  }
  // Z = buf[w][cur] in natural order. Bins of the real transform: X[k] = E[k] + W_512^k O[k] with
  // E = (Z[k] + conj Z[256-k]) / 2, O = (Z[k] - conj Z[256-k]) / 2i; X[256] = E[0] - O[0]. Power as the extractor:
  // |X| then squared.
  const Cx* Z = buf[w][cur];
  float* pw = power[w];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k = lane + 64 * q;
    const Cx zk = Z[k], zc0 = Z[(NZ - k) & (NZ - 1)];
    const Cx zc = {zc0.re, -zc0.im};
    const Cx e = {0.5f * (zk.re + zc.re), 0.5f * (zk.im + zc.im)};
    const Cx d = csub(zk, zc);
    const Cx o = {0.5f * d.im, -0.5f * d.re};  // d / 2i
    const Cx X = cadd(e, cmul(tw[k], o));
    const float a = __fsqrt_rn(__fadd_rn(__fmul_rn(X.re, X.re), __fmul_rn(X.im, X.im)));
    pw[k] = __fmul_rn(a, a);
    if (k == 0) {
      const float x256 = e.re - o.re;  // E[0] and O[0] are real
      const float a2 = __fsqrt_rn(__fmul_rn(x256, x256));
      pw[NZ] = __fmul_rn(a2, a2);
    }
  }
  __syncthreads();
  // mel bands m = lane and lane + 64 (a narrow low band with a wide high one), fp32 over the band's nonzero bins in
  // order; log(mel + 2^-24)
  if (live) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = lane + 64 * h;
      const float* wm = mel + (int64_t)m * BINS;
      const int k0 = band[2 * m], k1 = band[2 * m + 1];
      float acc = 0.f;
      for (int k = k0; k < k1; ++k) acc = __builtin_fmaf(wm[k], pw[k], acc);
      logmel[f * MELS + m] = logf(__fadd_rn(acc, 5.9604644775390625e-8f));
    }
  }
}

// per piece and mel band: mean and unbiased variance over the piece's valid frames (fp64 sums, 16 frame groups added
// in a fixed order), then (v - mean) / (std + 1e-5) as bf16 into out (pieces, T, 128) at the piece's first frames.
// Workgroup (piece, 16 bands): thread (g, m) = frames g, g + 16, ... of band 16 blockIdx.y + m.
constexpr int NG = 16, MB = 16;
__global__ void __launch_bounds__(NG* MB) normalize_kernel(const float* __restrict__ logmel,
                                                           const int64_t* __restrict__ frame_start, int64_t T,
                                                           uint16_t* __restrict__ out) {
  __shared__ double part[NG][MB];
  const int p = blockIdx.x, m = threadIdx.x % MB, g = threadIdx.x / MB, band = blockIdx.y * MB + m;
  const int64_t f0 = frame_start[p], nv = frame_start[p + 1] - f0;
  if (nv == 0) return;
  const float* v = logmel + f0 * MELS + band;
  uint16_t* o = out + (int64_t)p * T * MELS + band;
  auto total = [&](double s) {
    part[g][m] = s;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < NG; ++k) t += part[k][m];
    __syncthreads();
    return t;
  };
  double s = 0.0;
  for (int64_t t = g; t < nv; t += NG) s += v[t * MELS];
  const float mean = (float)(total(s) / (double)nv);
  double q = 0.0;
  for (int64_t t = g; t < nv; t += NG) {
    const double d = (double)v[t * MELS] - (double)mean;
    q += d * d;
  }
  const float den = __fadd_rn((float)sqrt(total(q) / (double)(nv - 1)), 1e-5f);
  for (int64_t t = g; t < nv; t += NG) o[t * MELS] = f2bf(__fdiv_rn(__fsub_rn(v[t * MELS], mean), den));
}

// ---- subsampling convolutions ------------------------------------------------------------------------------------
// ParakeetEncoderSubsamplingConv2D on one sequence at a time (its masking of padded frames after every convolution
// is zero padding at the sequence's ends), channels-last. Roundings as PyTorch's bf16 convolutions: conv0's sum is
// rounded, its bias added and rounded again (cuDNN adds the bias after), ReLU; the depthwise convolutions add the bias
// in fp32 and round once.

// conv0 (1 -> C, 3x3, stride 2, padding 1) + bias + ReLU, then the first depthwise 3x3 stride-2 convolution + bias,
// for one output row (sequence, t2) per workgroup and one channel per thread: out [rows, 32, C] bf16. The 7 mel rows
// the row needs (4 t2 - 3 .. 4 t2 + 3) are staged in LDS as fp32 with a zero column on the left (mel column c at index
// c + 1), so conv0 column f1 reads the float2 at index 2 f1 and the first value of the next.
constexpr int SUB_F1 = 64, SUB_F2 = 32, SUB_LD = MELS + 4;
__global__ void __launch_bounds__(1024) sub_conv0_dw_kernel(const uint16_t* __restrict__ feats, int64_t ld_seq,
                                                            const int* __restrict__ mel_len,
                                                            const int* __restrict__ rows, const float* __restrict__ w0,
                                                            const float* __restrict__ b0, const float* __restrict__ w2,
                                                            const float* __restrict__ b2, uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float mrow[7][SUB_LD];
  const int seq = rows[2 * blockIdx.x], t2 = rows[2 * blockIdx.x + 1];
  const int c = threadIdx.x, C = blockDim.x;
  const int L = mel_len[seq], T1 = (L - 1) / 2 + 1;
  const uint16_t* xs = feats + (int64_t)seq * ld_seq;
  for (int i = threadIdx.x; i < 7 * SUB_LD; i += C) {
    const int r = 4 * t2 - 3 + i / SUB_LD, col = i % SUB_LD - 1;
    mrow[i / SUB_LD][i % SUB_LD] = (r >= 0 && r < L && col >= 0 && col < MELS) ? bf2f(xs[(int64_t)r * MELS + col]) : 0.f;
  }
  float k0[9], kd[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    k0[i] = w0[c * 9 + i];
    kd[i] = w2[c * 9 + i];
  }
  const float bias0 = b0[c];
  float acc[SUB_F2];
#pragma unroll
  for (int i = 0; i < SUB_F2; ++i) acc[i] = b2[c];
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 3; ++r) {  // conv0 row t1 = 2 t2 - 1 + r is the depthwise tap row r
    const int t1 = 2 * t2 - 1 + r;
    if (t1 < 0 || t1 >= T1) continue;
    const float* m0 = mrow[2 * r];
    const float* m1 = mrow[2 * r + 1];
    const float* m2 = mrow[2 * r + 2];
    float2 p0 = *reinterpret_cast<const float2*>(m0), p1 = *reinterpret_cast<const float2*>(m1),
           p2 = *reinterpret_cast<const float2*>(m2);
#pragma unroll
    for (int f1 = 0; f1 < SUB_F1; ++f1) {
      // mel columns 2 f1 - 1, 2 f1, 2 f1 + 1
      const float2 n0 = *reinterpret_cast<const float2*>(m0 + 2 * f1 + 2);
      const float2 n1 = *reinterpret_cast<const float2*>(m1 + 2 * f1 + 2);
      const float2 n2 = *reinterpret_cast<const float2*>(m2 + 2 * f1 + 2);
      float s = 0.f;
      s = __builtin_fmaf(k0[0], p0.x, s);
      s = __builtin_fmaf(k0[1], p0.y, s);
      s = __builtin_fmaf(k0[2], n0.x, s);
      s = __builtin_fmaf(k0[3], p1.x, s);
      s = __builtin_fmaf(k0[4], p1.y, s);
      s = __builtin_fmaf(k0[5], n1.x, s);
      s = __builtin_fmaf(k0[6], p2.x, s);
      s = __builtin_fmaf(k0[7], p2.y, s);
      s = __builtin_fmaf(k0[8], n2.x, s);
      const float a = fmaxf(round_bf(round_bf(s) + bias0), 0.f);
      // depthwise output f2 reads conv0 columns 2 f2 - 1, 2 f2, 2 f2 + 1 (taps 0, 1, 2): f1 ascending adds each
      // output's taps in order
      if (f1 & 1) {
        if ((f1 + 1) / 2 < SUB_F2) acc[(f1 + 1) / 2] = __builtin_fmaf(kd[3 * r], a, acc[(f1 + 1) / 2]);
        acc[(f1 - 1) / 2] = __builtin_fmaf(kd[3 * r + 2], a, acc[(f1 - 1) / 2]);
      } else {
        acc[f1 / 2] = __builtin_fmaf(kd[3 * r + 1], a, acc[f1 / 2]);
      }
      p0 = n0;
      p1 = n1;
      p2 = n2;
    }
  }
  uint16_t* o = out + (int64_t)blockIdx.x * SUB_F2 * C + c;
#pragma unroll
  for (int i = 0; i < SUB_F2; ++i) o[(int64_t)i * C] = f2bf(acc[i]);
}

// depthwise 3x3 stride-2 convolution + bias on channels-last sequences x [sum T_in, F_in, C]: output row
// (sequence, t) = rows[i] into out [n, F_in / 2, C]; a thread per (row, frequency, 8 channels)
__global__ void __launch_bounds__(256) sub_dw_kernel(const uint16_t* __restrict__ x, const int* __restrict__ in_start,
                                                     const int* __restrict__ in_len, const int* __restrict__ rows,
                                                     const float* __restrict__ w, const float* __restrict__ b,
                                                     uint16_t* __restrict__ out, int64_t n, int F_in, int C) {
  const int F_out = F_in / 2, chunks = C / 8;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n * F_out * chunks) return;
  const int c = (int)(id % chunks) * 8, fo = (int)((id / chunks) % F_out);
  const int64_t i = id / chunks / F_out;
  const int seq = rows[2 * i], t = rows[2 * i + 1];
  // this thread's 8 channels x 9 taps are 72 consecutive floats of the (C, 9) layout: 18 16-byte loads, issued
  // with the bias before the row's own loads (not one 4-byte load per tap inside the guarded loops)
  float wk[8 * 9], acc[8];
#pragma unroll
  for (int v = 0; v < 18; ++v)
    *reinterpret_cast<float4*>(wk + 4 * v) = *reinterpret_cast<const float4*>(w + (int64_t)c * 9 + 4 * v);
  *reinterpret_cast<float4*>(acc) = *reinterpret_cast<const float4*>(b + c);
  *reinterpret_cast<float4*>(acc + 4) = *reinterpret_cast<const float4*>(b + c + 4);
  const int start = in_start[seq], len = in_len[seq];
  // the 3 x 3 input chunks (zero outside the sequence or the frequency range), all loaded before the first use
  uint4 u[9];
#pragma unroll
  for (int di = 0; di < 3; ++di)
#pragma unroll
    for (int dj = 0; dj < 3; ++dj) {
      const int ti = 2 * t - 1 + di, fi = 2 * fo - 1 + dj;
      const bool in = ti >= 0 && ti < len && fi >= 0 && fi < F_in;
      const int64_t off = in ? (((int64_t)start + ti) * F_in + fi) * C + c : 0;
      u[di * 3 + dj] = *reinterpret_cast<const uint4*>(x + off);
      if (!in) u[di * 3 + dj] = make_uint4(0, 0, 0, 0);
    }
  // the taps in the same order as before (missing taps skipped, not added as zeros: the fma chain is unchanged)
#pragma unroll
  for (int di = 0; di < 3; ++di) {
    const int ti = 2 * t - 1 + di;
    if (ti < 0 || ti >= len) continue;
#pragma unroll
    for (int dj = 0; dj < 3; ++dj) {
      const int fi = 2 * fo - 1 + dj;
      if (fi < 0 || fi >= F_in) continue;
      const uint4 v = u[di * 3 + dj];
      const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float xv = __uint_as_float(k & 1 ? e[k / 2] & 0xffff0000u : e[k / 2] << 16);
        acc[k] = __builtin_fmaf(wk[k * 9 + di * 3 + dj], xv, acc[k]);
      }
    }
  }
  uint4 o;
  o.x = pack_bf2(acc[0], acc[1]);
  o.y = pack_bf2(acc[2], acc[3]);
  o.z = pack_bf2(acc[4], acc[5]);
  o.w = pack_bf2(acc[6], acc[7]);
  *reinterpret_cast<uint4*>(out + ((int64_t)i * F_out + fo) * C + c) = o;
}

bool aligned(const void* q, int a) { return (reinterpret_cast<uintptr_t>(q) % a) == 0; }

}  // namespace

extern "C" int64_t cohere_logmel_workspace_bytes(int64_t total_frames) {
  return total_frames < 0 ? -1 : total_frames * MELS * (int64_t)sizeof(float);
}

extern "C" int cohere_logmel_features(const float* x, const int64_t* meta, int64_t pieces, int64_t total_frames,
                                      const float* window, const float* mel, const int32_t* band, float preemph,
                                      uint16_t* out, int64_t T, float* work, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(pieces >= 0 && total_frames >= 0 && T >= 0 && pieces < (1 << 30), "logmel_features: bad sizes");
  if (total_frames == 0 || pieces == 0) return 0;
  COHERE_REQUIRE(x && meta && window && mel && band && out && work, "logmel_features: null pointer");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t blocks = (total_frames + FPW - 1) / FPW;
  COHERE_REQUIRE(blocks < (1LL << 31), "logmel_features: too many frames");
  logmel_kernel<<<(unsigned)blocks, FPW * 64, 0, s>>>(x, meta, (int)pieces, total_frames, window, mel, band, preemph,
                                                       work);
  normalize_kernel<<<dim3((unsigned)pieces, MELS / MB), NG * MB, 0, s>>>(work, meta + 2 * pieces, T, out);
  return cohere::check_launch("logmel_features");
}

extern "C" int cohere_sub_conv0_dw(const uint16_t* feats, int64_t ld_seq, const int32_t* mel_len, const int32_t* rows,
                                   int64_t n_rows, const float* w0, const float* b0, const float* w2, const float* b2,
                                   uint16_t* out, int64_t C, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(n_rows >= 0 && n_rows < (1LL << 31), "sub_conv0_dw: bad row count");
  COHERE_REQUIRE(C >= 64 && C <= 1024 && C % 64 == 0, "sub_conv0_dw: channels must be a multiple of 64, at most 1024");
  if (n_rows == 0) return 0;
  COHERE_REQUIRE(feats && mel_len && rows && w0 && b0 && w2 && b2 && out, "sub_conv0_dw: null pointer");
  sub_conv0_dw_kernel<<<(unsigned)n_rows, (unsigned)C, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      feats, ld_seq, mel_len, rows, w0, b0, w2, b2, out);
  return cohere::check_launch("sub_conv0_dw");
}

extern "C" int cohere_sub_dw(const uint16_t* x, const int32_t* in_start, const int32_t* in_len, const int32_t* rows,
                             int64_t n_rows, const float* w, const float* b, uint16_t* out, int64_t F_in, int64_t C,
                             void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(n_rows >= 0 && F_in >= 2 && F_in <= 4096 && C > 0 && C % 8 == 0 && C <= 65536,
                 "sub_dw: bad sizes (C % 8 == 0)");
  if (n_rows == 0) return 0;
  COHERE_REQUIRE(x && in_start && in_len && rows && w && b && out, "sub_dw: null pointer");
  COHERE_REQUIRE(aligned(x, 16) && aligned(out, 16) && aligned(w, 16) && aligned(b, 16),
                 "sub_dw: x, out, the taps and the bias must be 16-byte aligned");
  const int64_t total = n_rows * (F_in / 2) * (C / 8);
  COHERE_REQUIRE((total + 255) / 256 < (1LL << 31), "sub_dw: too many rows");
  sub_dw_kernel<<<(unsigned)((total + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      x, in_start, in_len, rows, w, b, out, n_rows, (int)F_in, (int)C);
  return cohere::check_launch("sub_dw");
}
