// The FastConformer layers' int8 forward as one host call (reference kernels/csrc/encoder_loop.cpp:50-99, the
// int8 branch): per layer 14-15 launches in the reference's order, each through this library's own C entry points,
// on one stream, with no host synchronisation. From Python the ~700 launches of 48 layers would each pay the
// interpreter and argument parsing; here the loop is native.
//
// Per layer (x (rows, 1280) bf16 in place; hq/hs the int8 rows and scales feeding the next GEMM):
//   FF1:  tq, ts = SILU_Q8(hq W1);  x = x + 0.5 (tq W2)          (W1 / W2 2:4 sparse when their compressed weights
//                                                                  are given)
//   ATT:  hq = LN_att(x);  qkv = hq Wqkv + b;  a = relpos_attention(qkv);  hq = q8(a);  x = x + (hq Wo + bo)
//   CONV: hq = LN_conv(x); a = GLU(hq Wpw1 + b);  hq = q8(silu(bn(dwconv(a))));  x = x + (hq Wpw2 + b)
//   FF2:  hq = LN_ff2(x);  as FF1
//   OUT:  x = LN_out(x) and, fused, hq = LN_ff1 of the next layer (the last layer: x = LN_out(x) in bf16)
#include "cohere_hip.h"
#include "common.h"

#include <algorithm>
#include <string>

namespace {

// a layer's tensors, in the reference's field order (encoder_loop.cpp:34-44, fast_encoder.py:121-130)
enum F {
  LN_FF1_W, LN_FF1_B, LN_ATT_W, LN_ATT_B, LN_CONV_W, LN_CONV_B, LN_FF2_W, LN_FF2_B, LN_OUT_W, LN_OUT_B,
  FF1_W1, FF1_B1, FF1_W2, FF1_B2, FF2_W1, FF2_B1, FF2_W2, FF2_B2,
  WQKV, BQKV, WO, BO, BU, BV, RK, WPW1, BPW1, WDW, BDW, BN_SCALE, BN_SHIFT, WPW2, BPW2,
  Q_FF1_W1, Q_FF1_S1, Q_FF1_W2, Q_FF1_S2, Q_FF2_W1, Q_FF2_S1, Q_FF2_W2, Q_FF2_S2, Q_QKV_W, Q_QKV_S, Q_PW1_W, Q_PW1_S,
  Q_O_W, Q_O_S, Q_PW2_W, Q_PW2_S,
  SP_FF1_W, SP_FF1_E, SP_FF2_W, SP_FF2_E,
  // this library's own: the first feed-forward linears in 2:4 form (the reference keeps them dense)
  SP_FF1_W1, SP_FF1_E1, SP_FF2_W1, SP_FF2_E1,
  N_FIELDS
};
static_assert(N_FIELDS == COHERE_ENC_N_FIELDS, "field count");
enum E { EPS_FF1, EPS_ATT, EPS_CONV, EPS_FF2, EPS_OUT, N_EPS };

constexpr int64_t DM = 1280, DFF = 5120, DQKV = 3 * DM;

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

struct Workspace {
  uint16_t* qkv;  // (rows, 3840) bf16
  uint16_t* a;    // (rows, 1280) bf16: attention output, then the GLU output
  int8_t* hq;     // (rows, 1280)
  int8_t* tq;     // (rows, 5120)
  float* hs;      // (rows)
  float* ts;      // (rows, 5120 / group)
  int64_t bytes;
};

// the bf16 branch's buffers: LayerNorm output, feed-forward hidden, QKV, attention / GLU output, depthwise output
struct WorkspaceBf16 {
  uint16_t *h, *t, *qkv, *a, *z;
  int64_t bytes;
};

WorkspaceBf16 carve_bf16(void* base, int64_t rows) {
  WorkspaceBf16 w{};
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* r = p ? p + off : nullptr;
    off += align256(bytes);
    return reinterpret_cast<uint16_t*>(r);
  };
  w.h = take(rows * DM * 2);
  w.t = take(rows * DFF * 2);
  w.qkv = take(rows * DQKV * 2);
  w.a = take(rows * DM * 2);
  w.z = take(rows * DM * 2);
  w.bytes = off;
  return w;
}

Workspace carve(void* base, int64_t rows, int64_t group) {
  Workspace w{};
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  w.qkv = reinterpret_cast<uint16_t*>(take(rows * DQKV * 2));
  w.a = reinterpret_cast<uint16_t*>(take(rows * DM * 2));
  w.hq = reinterpret_cast<int8_t*>(take(rows * DM));
  w.tq = reinterpret_cast<int8_t*>(take(rows * DFF));
  w.hs = reinterpret_cast<float*>(take(rows * 4));
  w.ts = reinterpret_cast<float*>(take(rows * (DFF / group) * 4));
  w.bytes = off;
  return w;
}

template <typename T>
const T* fld(const void* const* ly, int f) {
  return static_cast<const T*>(ly[f]);
}

}  // namespace

extern "C" int64_t cohere_encoder_workspace_bytes(int64_t rows, int64_t group) {
  if (rows < 0 || group <= 0 || DFF % group) return -1;
  return std::max(carve(nullptr, rows, group).bytes, carve_bf16(nullptr, rows).bytes);
}

extern "C" int64_t cohere_encoder_branch_workspace_bytes(int64_t rows, int64_t group, int32_t int8) {
  if (rows < 0 || group <= 0 || DFF % group) return -1;
  return int8 ? carve(nullptr, rows, group).bytes : carve_bf16(nullptr, rows).bytes;
}

namespace {

// The bf16 branch (reference kernels/csrc/encoder_loop.cpp:101-124): every linear a bf16 GEMM with its epilogue
// fused (SiLU, residual, GLU), the LayerNorms, the attention and the depthwise convolution in bf16.
int encoder_layers_bf16(uint16_t* x, int64_t rows, const void* const* fields, int64_t n_layers, const double* eps,
                        const int32_t* tiles, int64_t n_tiles, const int32_t* lo, const int32_t* hi, int64_t rel_off,
                        int64_t max_len, int64_t rel_rows, double scale, int32_t heads, int32_t head_dim,
                        int64_t c_bf, const WorkspaceBf16& ws, void* stream) {
  static const int required[] = {LN_FF1_W, LN_FF1_B, LN_ATT_W, LN_ATT_B, LN_CONV_W, LN_CONV_B, LN_FF2_W, LN_FF2_B,
                                 LN_OUT_W, LN_OUT_B, FF1_W1, FF1_W2, FF2_W1, FF2_W2, WQKV, WO, BU, BV, RK, WPW1,
                                 WDW, BDW, BN_SCALE, BN_SHIFT, WPW2};
  for (int64_t l = 0; l < n_layers; ++l)
    for (int f : required)
      COHERE_REQUIRE(fields[l * N_FIELDS + f],
                     "encoder_layers (bf16): layer " + std::to_string(l) + " misses field " + std::to_string(f));
  auto ep = [&](int64_t i, int e) { return (float)eps[i * N_EPS + e]; };
  int64_t i = 0;
  auto fail = [&](const char* what) {
    cohere::set_error("encoder_layers (bf16): layer " + std::to_string(i) + ", " + what + ": " + cohere_last_error());
    return 1;
  };
#define RUN(call, what) \
  if ((call) != 0) return fail(what)
  auto gemm = [&](const uint16_t* a, int64_t k, const void* const* ly, int w, int b, uint16_t* out, int64_t ldc,
                  int epi, int64_t n, float alpha) {
    return cohere_gemm_bf16(a, k, fld<uint16_t>(ly, w), fld<uint16_t>(ly, b), out, ldc, epi,
                            epi == COHERE_EPI_RESID ? out : nullptr, ldc, alpha, rows, n, k, (int32_t)c_bf, stream);
  };
  RUN(cohere_layernorm(x, DM, fld<uint16_t>(fields, LN_FF1_W), fld<uint16_t>(fields, LN_FF1_B), ep(0, EPS_FF1),
                       nullptr, nullptr, 0.f, ws.h, DM, rows, DM, stream),
      "first LayerNorm");
  for (i = 0; i < n_layers; ++i) {
    const void* const* ly = fields + i * N_FIELDS;
    RUN(gemm(ws.h, DM, ly, FF1_W1, FF1_B1, ws.t, DFF, COHERE_EPI_SILU, DFF, 1.f), "feed-forward 1 W1");
    RUN(gemm(ws.t, DFF, ly, FF1_W2, FF1_B2, x, DM, COHERE_EPI_RESID, DM, 0.5f), "feed-forward 1 W2");
    RUN(cohere_layernorm(x, DM, fld<uint16_t>(ly, LN_ATT_W), fld<uint16_t>(ly, LN_ATT_B), ep(i, EPS_ATT), nullptr,
                         nullptr, 0.f, ws.h, DM, rows, DM, stream),
        "attention LayerNorm");
    RUN(gemm(ws.h, DM, ly, WQKV, BQKV, ws.qkv, DQKV, COHERE_EPI_BIAS, DQKV, 1.f), "QKV");
    RUN(cohere_relpos_attention(ws.qkv, fld<uint16_t>(ly, RK), rel_rows, fld<uint16_t>(ly, BU),
                                fld<uint16_t>(ly, BV), tiles, n_tiles, heads, head_dim, rel_off, max_len,
                                (float)scale, ws.a, stream),
        "attention");
    RUN(gemm(ws.a, DM, ly, WO, BO, x, DM, COHERE_EPI_RESID, DM, 1.f), "attention output projection");
    RUN(cohere_layernorm(x, DM, fld<uint16_t>(ly, LN_CONV_W), fld<uint16_t>(ly, LN_CONV_B), ep(i, EPS_CONV),
                         nullptr, nullptr, 0.f, ws.h, DM, rows, DM, stream),
        "convolution LayerNorm");
    RUN(gemm(ws.h, DM, ly, WPW1, BPW1, ws.a, DM, COHERE_EPI_GLU, 2 * DM, 1.f), "pointwise conv 1 (GLU)");
    RUN(cohere_dwconv_bn_silu(ws.a, fld<float>(ly, WDW), fld<float>(ly, BDW), fld<float>(ly, BN_SCALE),
                              fld<float>(ly, BN_SHIFT), lo, hi, ws.z, rows, DM, 9, stream),
        "depthwise conv");
    RUN(gemm(ws.z, DM, ly, WPW2, BPW2, x, DM, COHERE_EPI_RESID, DM, 1.f), "pointwise conv 2");
    RUN(cohere_layernorm(x, DM, fld<uint16_t>(ly, LN_FF2_W), fld<uint16_t>(ly, LN_FF2_B), ep(i, EPS_FF2), nullptr,
                         nullptr, 0.f, ws.h, DM, rows, DM, stream),
        "feed-forward 2 LayerNorm");
    RUN(gemm(ws.h, DM, ly, FF2_W1, FF2_B1, ws.t, DFF, COHERE_EPI_SILU, DFF, 1.f), "feed-forward 2 W1");
    RUN(gemm(ws.t, DFF, ly, FF2_W2, FF2_B2, x, DM, COHERE_EPI_RESID, DM, 0.5f), "feed-forward 2 W2");
    if (i + 1 < n_layers) {
      const void* const* nx = ly + N_FIELDS;
      RUN(cohere_layernorm(x, DM, fld<uint16_t>(ly, LN_OUT_W), fld<uint16_t>(ly, LN_OUT_B), ep(i, EPS_OUT),
                           fld<uint16_t>(nx, LN_FF1_W), fld<uint16_t>(nx, LN_FF1_B), ep(i + 1, EPS_FF1), ws.h, DM,
                           rows, DM, stream),
          "output LayerNorm");
    } else {
      RUN(cohere_layernorm(x, DM, fld<uint16_t>(ly, LN_OUT_W), fld<uint16_t>(ly, LN_OUT_B), ep(i, EPS_OUT), nullptr,
                           nullptr, 0.f, x, DM, rows, DM, stream),
          "output LayerNorm");
    }
  }
#undef RUN
  return 0;
}

}  // namespace

extern "C" int cohere_encoder_layers(uint16_t* x, int64_t rows, const void* const* fields, int64_t n_layers,
                                     const double* eps, const int32_t* tiles, int64_t n_tiles, const int32_t* lo,
                                     const int32_t* hi, int64_t rel_off, int64_t max_len, int64_t rel_rows,
                                     double scale, int32_t heads, int32_t head_dim, int32_t int8, const int64_t* cfg,
                                     int64_t n_cfg, void* workspace, int64_t workspace_bytes, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(n_cfg >= 5, "encoder_layers: cfg needs at least 5 entries");
  COHERE_REQUIRE((int64_t)heads * head_dim == DM, "encoder_layers: heads x head size must be 1280");
  COHERE_REQUIRE(rows >= 0 && n_layers >= 0 && x && fields && eps, "encoder_layers: bad arguments");
  const int64_t c_i8 = cfg[1], c_grp = cfg[2], c_ff1 = cfg[3], group = cfg[4];
  const int64_t c_pw1 = n_cfg > 5 ? cfg[5] : c_i8, c_o = n_cfg > 6 ? cfg[6] : c_i8;
  const int64_t c_sp = n_cfg > 7 ? cfg[7] : 0;
  COHERE_REQUIRE(group > 0 && DFF % group == 0, "encoder_layers: the feed-forward group must divide 5120");
  if (rows == 0 || n_layers == 0) return 0;
  const int64_t need = cohere_encoder_branch_workspace_bytes(rows, group, int8);
  COHERE_REQUIRE(workspace && workspace_bytes >= need,
                 "encoder_layers: workspace needs " + std::to_string(need) + " bytes");
  if (!int8) {
    COHERE_REQUIRE(cfg[0] == 3 || cfg[0] == 5 || cfg[0] == 8, "encoder_layers: unknown bf16 GEMM config");
    return encoder_layers_bf16(x, rows, fields, n_layers, eps, tiles, n_tiles, lo, hi, rel_off, max_len, rel_rows,
                               scale, heads, head_dim, cfg[0], carve_bf16(workspace, rows), stream);
  }
  const Workspace ws = carve(workspace, rows, group);
  // biases may be null (the GEMMs then skip them); the 2:4 and dense feed-forward W2 are alternatives
  static const int required[] = {LN_FF1_W, LN_FF1_B, LN_ATT_W, LN_ATT_B, LN_CONV_W, LN_CONV_B, LN_FF2_W, LN_FF2_B,
                                 LN_OUT_W, LN_OUT_B, BU, BV, RK, WDW, BDW, BN_SCALE, BN_SHIFT, Q_FF1_S1,
                                 Q_FF1_S2, Q_FF2_S1, Q_FF2_S2, Q_QKV_W, Q_QKV_S, Q_PW1_W, Q_PW1_S, Q_O_W,
                                 Q_O_S, Q_PW2_W, Q_PW2_S};
  for (int64_t l = 0; l < n_layers; ++l) {
    const void* const* ly = fields + l * N_FIELDS;
    for (int f : required)
      COHERE_REQUIRE(ly[f], "encoder_layers: layer " + std::to_string(l) + " misses field " + std::to_string(f));
    // a 2:4 weight without selectors is in the stage-tiled layout (cohere_pack_24_tiled)
    COHERE_REQUIRE((ly[SP_FF1_W] || ly[Q_FF1_W2]) && (ly[SP_FF2_W] || ly[Q_FF2_W2]) &&
                       (ly[SP_FF1_W1] || ly[Q_FF1_W1]) && (ly[SP_FF2_W1] || ly[Q_FF2_W1]),
                   "encoder_layers: layer " + std::to_string(l) +
                       ": a feed-forward linear has neither dense nor 2:4 weights");
  }

  const int64_t ts_ld = DFF / group;
  auto ep = [&](int64_t i, int e) { return (float)eps[i * N_EPS + e]; };
  auto fail = [&](int64_t i, const char* what) {
    cohere::set_error("encoder_layers: layer " + std::to_string(i) + ", " + what + ": " + cohere_last_error());
    return 1;
  };
#define RUN(call, what) \
  if ((call) != 0) return fail(i, what)

  const void* const* l0 = fields;
  int64_t i = 0;
  RUN(cohere_layernorm_q8(x, DM, fld<uint16_t>(l0, LN_FF1_W), fld<uint16_t>(l0, LN_FF1_B), ep(0, EPS_FF1), nullptr,
                          nullptr, 0.f, ws.hq, DM, ws.hs, rows, DM, stream),
      "first LayerNorm");
  // the 2:4 SILU_Q8 GEMM writes one scale per row and 256 columns: the dense W1's output group must match it
  COHERE_REQUIRE(group == 256 || [&] {
    for (int64_t l = 0; l < n_layers; ++l)
      if (fields[l * N_FIELDS + SP_FF1_W1] || fields[l * N_FIELDS + SP_FF2_W1]) return false;
    return true;
  }(), "encoder_layers: a 2:4 first feed-forward linear needs the feed-forward group 256");
  auto ffn = [&](const void* const* ly, int w1, int s1, int b1, int w2, int s2, int b2, int spw, int spe, int spw1,
                 int spe1) {
    if (ly[spw1] && !ly[spe1]) {
      RUN(cohere_gemm_sp_tiled(ws.hq, DM, ws.hs, 1, DM, fld<uint8_t>(ly, spw1), fld<float>(ly, s1),
                               fld<uint16_t>(ly, b1), ws.tq, DFF, COHERE_EPI_SILU_Q8, nullptr, 0, 1.f, ws.ts, ts_ld,
                               rows, DFF, DM, (int32_t)c_sp, stream),
          "feed-forward W1 (2:4, tiled)");
    } else if (ly[spw1]) {
      RUN(cohere_gemm_sp(ws.hq, DM, ws.hs, 1, DM, fld<int8_t>(ly, spw1), fld<int32_t>(ly, spe1), fld<float>(ly, s1),
                         fld<uint16_t>(ly, b1), ws.tq, DFF, COHERE_EPI_SILU_Q8, nullptr, 0, 1.f, ws.ts, ts_ld, rows,
                         DFF, DM, (int32_t)c_sp, stream),
          "feed-forward W1 (2:4)");
    } else {
      RUN(cohere_gemm_i8(ws.hq, DM, ws.hs, 1, DM, fld<int8_t>(ly, w1), fld<float>(ly, s1), fld<uint16_t>(ly, b1),
                         ws.tq, DFF, COHERE_EPI_SILU_Q8, nullptr, 0, 1.f, ws.ts, ts_ld, rows, DFF, DM,
                         (int32_t)c_ff1, stream),
          "feed-forward W1");
    }
    if (ly[spw] && !ly[spe]) {
      RUN(cohere_gemm_sp_tiled(ws.tq, DFF, ws.ts, ts_ld, group, fld<uint8_t>(ly, spw), fld<float>(ly, s2),
                               fld<uint16_t>(ly, b2), x, DM, COHERE_EPI_RESID, x, DM, 0.5f, nullptr, 0, rows, DM, DFF,
                               (int32_t)c_sp, stream),
          "feed-forward W2 (2:4, tiled)");
    } else if (ly[spw]) {
      RUN(cohere_gemm_sp(ws.tq, DFF, ws.ts, ts_ld, group, fld<int8_t>(ly, spw), fld<int32_t>(ly, spe),
                         fld<float>(ly, s2), fld<uint16_t>(ly, b2), x, DM, COHERE_EPI_RESID, x, DM, 0.5f, nullptr, 0,
                         rows, DM, DFF, (int32_t)c_sp, stream),
          "feed-forward W2 (2:4)");
    } else {
      RUN(cohere_gemm_i8(ws.tq, DFF, ws.ts, ts_ld, group, fld<int8_t>(ly, w2), fld<float>(ly, s2),
                         fld<uint16_t>(ly, b2), x, DM, COHERE_EPI_RESID, x, DM, 0.5f, nullptr, 0, rows, DM, DFF,
                         (int32_t)c_grp, stream),
          "feed-forward W2");
    }
    return 0;
  };
  for (i = 0; i < n_layers; ++i) {
    const void* const* ly = fields + i * N_FIELDS;
    if (ffn(ly, Q_FF1_W1, Q_FF1_S1, FF1_B1, Q_FF1_W2, Q_FF1_S2, FF1_B2, SP_FF1_W, SP_FF1_E, SP_FF1_W1, SP_FF1_E1))
      return 1;
    RUN(cohere_layernorm_q8(x, DM, fld<uint16_t>(ly, LN_ATT_W), fld<uint16_t>(ly, LN_ATT_B), ep(i, EPS_ATT), nullptr,
                            nullptr, 0.f, ws.hq, DM, ws.hs, rows, DM, stream),
        "attention LayerNorm");
    RUN(cohere_gemm_i8(ws.hq, DM, ws.hs, 1, DM, fld<int8_t>(ly, Q_QKV_W), fld<float>(ly, Q_QKV_S),
                       fld<uint16_t>(ly, BQKV), ws.qkv, DQKV, COHERE_EPI_BIAS, nullptr, 0, 1.f, nullptr, 0, rows,
                       DQKV, DM, (int32_t)c_i8, stream),
        "QKV");
    RUN(cohere_relpos_attention(ws.qkv, fld<uint16_t>(ly, RK), rel_rows, fld<uint16_t>(ly, BU),
                                fld<uint16_t>(ly, BV), tiles, n_tiles, heads, head_dim, rel_off, max_len,
                                (float)scale, ws.a, stream),
        "attention");
    RUN(cohere_quantize_rows(ws.a, DM, ws.hq, DM, ws.hs, rows, DM, stream), "attention output quantization");
    RUN(cohere_gemm_i8(ws.hq, DM, ws.hs, 1, DM, fld<int8_t>(ly, Q_O_W), fld<float>(ly, Q_O_S), fld<uint16_t>(ly, BO),
                       x, DM, COHERE_EPI_RESID, x, DM, 1.f, nullptr, 0, rows, DM, DM, (int32_t)c_o, stream),
        "attention output projection");
    RUN(cohere_layernorm_q8(x, DM, fld<uint16_t>(ly, LN_CONV_W), fld<uint16_t>(ly, LN_CONV_B), ep(i, EPS_CONV),
                            nullptr, nullptr, 0.f, ws.hq, DM, ws.hs, rows, DM, stream),
        "convolution LayerNorm");
    RUN(cohere_gemm_i8(ws.hq, DM, ws.hs, 1, DM, fld<int8_t>(ly, Q_PW1_W), fld<float>(ly, Q_PW1_S),
                       fld<uint16_t>(ly, BPW1), ws.a, DM, COHERE_EPI_GLU, nullptr, 0, 1.f, nullptr, 0, rows, 2 * DM,
                       DM, (int32_t)c_pw1, stream),
        "pointwise conv 1 (GLU)");
    // the reference takes a bf16 detour below 512 rows (dwconv_bn_silu + quantize_rows) for speed only: the int8
    // rows and scales are the same, so the fused kernel serves every size here
    RUN(cohere_dwconv_bn_silu_q8(ws.a, fld<float>(ly, WDW), fld<float>(ly, BDW), fld<float>(ly, BN_SCALE),
                                 fld<float>(ly, BN_SHIFT), lo, hi, ws.hq, ws.hs, rows, DM, 9, stream),
        "depthwise conv");
    RUN(cohere_gemm_i8(ws.hq, DM, ws.hs, 1, DM, fld<int8_t>(ly, Q_PW2_W), fld<float>(ly, Q_PW2_S),
                       fld<uint16_t>(ly, BPW2), x, DM, COHERE_EPI_RESID, x, DM, 1.f, nullptr, 0, rows, DM, DM,
                       (int32_t)c_o, stream),
        "pointwise conv 2");
    RUN(cohere_layernorm_q8(x, DM, fld<uint16_t>(ly, LN_FF2_W), fld<uint16_t>(ly, LN_FF2_B), ep(i, EPS_FF2), nullptr,
                            nullptr, 0.f, ws.hq, DM, ws.hs, rows, DM, stream),
        "feed-forward 2 LayerNorm");
    if (ffn(ly, Q_FF2_W1, Q_FF2_S1, FF2_B1, Q_FF2_W2, Q_FF2_S2, FF2_B2, SP_FF2_W, SP_FF2_E, SP_FF2_W1, SP_FF2_E1))
      return 1;
    if (i + 1 < n_layers) {
      const void* const* nx = ly + N_FIELDS;
      RUN(cohere_layernorm_q8(x, DM, fld<uint16_t>(ly, LN_OUT_W), fld<uint16_t>(ly, LN_OUT_B), ep(i, EPS_OUT),
                              fld<uint16_t>(nx, LN_FF1_W), fld<uint16_t>(nx, LN_FF1_B), ep(i + 1, EPS_FF1), ws.hq, DM,
                              ws.hs, rows, DM, stream),
          "output LayerNorm");
    } else {
      RUN(cohere_layernorm(x, DM, fld<uint16_t>(ly, LN_OUT_W), fld<uint16_t>(ly, LN_OUT_B), ep(i, EPS_OUT), nullptr,
                           nullptr, 0.f, x, DM, rows, DM, stream),
          "output LayerNorm");
    }
  }
#undef RUN
  return 0;
}
