// C ABI of the W8A8 int8 GEMMs (include/cohere_hip.h): argument checks, the reference's config-id semantics, the
// choice of gfx950 tile, and dispatch to the kernel instantiations (gemm_q8.h, gemm_q8_dense.hip, gemm_q8_sparse.hip).
#include "cohere_hip.h"
#include "gemm_q8.h"

#include <cstring>
#include <string>

namespace {

using namespace cohere_gemm;

int g_tile_override = -1;

// gfx950 tile choice: the largest tile that still gives (nearly) every CU a workgroup; with fewer tiles than CUs,
// the shape with the most workgroups. SILU_Q8 needs whole scale groups inside a tile.
int num_cus() {
  static int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess || v <= 0)
      v = 256;
    return v;
  }();
  return n;
}

int choose_tile(const GemmArgs& p, bool grouped, bool bf = false) {
  auto fits = [&](int id) {
    const TileInfo& t = TILES[id];
    if (bf && !bf16_tile(id)) return false;
    if (p.N % t.bn) return false;
    if (grouped && !t.grouped_ok) return false;
    if (p.epi == EPI_SILU_Q8 && t.bn % p.qgroup) return false;
    return true;
  };
  if (g_tile_override >= 0 && g_tile_override < N_TILES && fits(g_tile_override)) return g_tile_override;
  auto tiles_of = [&](int id) { return (int64_t)((p.M + TILES[id].bm - 1) / TILES[id].bm) * (p.N / TILES[id].bn); };
  // largest first; the first shape that gives about two thirds of the CUs a workgroup wins (measured on the encoder
  // block's GEMMs at 1504-3000 rows: a large tile on 64 % of the CUs beats a smaller one on all of them). The 128x128
  // tile on 32x32 instructions (12) precedes its 16x16 twin (0). Grouped scales skip 12 and the 8-wave tiles (8, 9,
  // whose fold accumulators spill): 0 is the fastest grouped tile from 3000 to 12032 rows (12032: 154 us against
  // 206-224 us for 8 and 9).
  // The int8 256x256 tile runs 16 waves (15) in place of 8 (6), four per SIMD hiding more latency: SILU_Q8's
  // VALU-heavy epilogue 31.7 -> 30.3 us at config 1; with the grid split into one part per XCD, the bias epilogue too
  // (config 1 up 22.8 -> 21.9 us, config 0 dense 24.5 -> 24.1 us)
  // The stage-tiled 2:4 weights (contiguous kilobyte loads) move the balance: there the 8-wave 256x256 tile (10)
  // beats the 16-wave one (config 1 up 23.9 -> 22.0 us, SILU_Q8 31.4 -> 30.7) and the 16x16 128x128 tile (0) its
  // 32x32 twin (config 1 down 22.8 -> 22.4 us), alternating runs.
  static const int order[] = {6, 9, 1, 8, 2, 12, 0, 4, 3, 5, 7};
  const int64_t want = (int64_t)num_cus() * 64 / 100;
  int best = -1;
  for (int id0 : order) {
    // grouped scales take the 8-wave 128x128 tile (17: 64 tokens x 32 channels a wave, two waves per SIMD) in place
    // of the 4-wave one: the per-group fold's VALU work of one wave then overlaps the other's matrix instructions
    // (config-2 feed-forward W2, 3000 x 1280 x 5120 in groups of 256, 2:4: 33.4 -> 29.3 us)
    const int id = id0 == 6 && !bf ? (p.tiled ? 10 : 15) : (id0 == 0 && grouped ? 17 : id0);
    if (!fits(id) || (grouped && (id == 12 || id == 8 || id == 9)) || (p.tiled && id == 12)) continue;
    if (tiles_of(id) >= want) return id;
    if (best < 0 || tiles_of(id) > tiles_of(best)) best = id;
  }
  return best;
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
  const int out_align = 16;  // the staged epilogues write 16-byte chunks of output rows
  const int esize = p.epi == EPI_SILU_Q8 ? 1 : (p.epi == EPI_I32 ? 4 : 2);
  COHERE_REQUIRE((reinterpret_cast<uintptr_t>(p.C) % out_align) == 0 && (p.ldc * esize) % out_align == 0,
                 nm + ": output rows must be aligned");
  COHERE_REQUIRE(p.epi != EPI_RESID || (aligned16(p.R) && p.ldr % 8 == 0), nm + ": residual rows must be aligned");
  if (p.M == 0) return 0;
  p.group = (int)group;
  const int tile = choose_tile(p, grouped);
  COHERE_REQUIRE(tile >= 0, nm + ": no gfx950 tile fits N=" + std::to_string(p.N));
  if (!launch_gemm<SPARSE>(tile, p.epi, grouped, p, s)) {
    cohere::set_error(nm + ": tile " + std::to_string(tile) + " has no kernel for this epilogue");
    return 1;
  }
  return cohere::check_launch(name);
}

}  // namespace

extern "C" int cohere_set_gemm_tile(int32_t tile) {
  if (tile == -2 || tile == -3) {  // the XCD split off / on
    cohere_gemm::g_xcd_split = tile == -3;
    return N_TILES;
  }
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

extern "C" int cohere_gemm_sp_tiled(const int8_t* x, int64_t ldx, const float* sx, int64_t ldsx, int64_t group,
                                    const uint8_t* wt, const float* sw, const uint16_t* bias, void* out, int64_t ldc,
                                    int32_t epi, const uint16_t* resid, int64_t ldr, float alpha, float* qs,
                                    int64_t ldqs, int64_t M, int64_t N, int64_t K, int32_t cfg, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(cfg >= -1 && cfg <= 4, "gemm_sp_tiled: unknown config " + std::to_string(cfg));
  GemmArgs p{};
  p.X = x; p.sx = sx; p.W = reinterpret_cast<const int8_t*>(wt); p.E = reinterpret_cast<const int32_t*>(wt);
  p.sw = sw; p.bias = bias; p.C = out; p.R = resid; p.qs = qs; p.tiled = 1;
  p.ldx = ldx; p.ldsx = ldsx; p.ldc = ldc; p.ldr = ldr; p.ldqs = ldqs;
  p.M = (int)M; p.N = (int)N; p.K = (int)K; p.qgroup = 256; p.epi = epi; p.alpha = alpha;
  return gemm_entry<true>(p, group, 128, reinterpret_cast<hipStream_t>(stream), "gemm_sp_tiled");
}

extern "C" int64_t cohere_pack_24_tiled_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || N % 16 || K % 128) return -1;
  return N / 16 * (K / 128) * TILED_REC;
}

extern "C" int cohere_pack_24_tiled(const int8_t* wc, const int32_t* e, int64_t N, int64_t K, uint8_t* out) {
  cohere::clear_error();
  COHERE_REQUIRE(wc && e && out, "pack_24_tiled: null pointer");
  COHERE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0, "pack_24_tiled: N % 16 and K % 128 must be 0");
  const int64_t KT = K / 128;
  for (int64_t rb = 0; rb < N / 16; ++rb)
    for (int64_t kt = 0; kt < KT; ++kt) {
      uint8_t* rec = out + (rb * KT + kt) * TILED_REC;
      for (int i = 0; i < 64; ++i) {
        const int64_t row = rb * 16 + i / 4;
        const int c = (i % 4) ^ ((i / 8) % 4);
        std::memcpy(rec + 16 * i, wc + row * (K / 2) + kt * 64 + c * 16, 16);
      }
      // row r's four selector words, words 0-1 and 2-3 swapped in rows 8-15 (see TILED_REC)
      for (int r = 0; r < 16; ++r)
        for (int w = 0; w < 4; ++w)
          std::memcpy(rec + 1024 + 16 * r + 4 * (w ^ (r & 8 ? 2 : 0)), e + (rb * 16 + r) * (K / 32) + kt * 4 + w, 4);
    }
  return 0;
}

extern "C" int cohere_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* w, const uint16_t* bias, uint16_t* out,
                                int64_t ldc, int32_t epi, const uint16_t* resid, int64_t ldr, float alpha, int64_t M,
                                int64_t N, int64_t K, int32_t cfg, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(cfg == 3 || cfg == 5 || cfg == 8, "gemm: unknown config " + std::to_string(cfg));
  COHERE_REQUIRE(M >= 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 30),
                 "gemm: bad sizes");
  COHERE_REQUIRE(a && w && out, "gemm: null pointer");
  COHERE_REQUIRE(K % 32 == 0, "gemm: K must match and be a multiple of 32");
  COHERE_REQUIRE(N % 64 == 0, "gemm: N must be a multiple of 64");
  COHERE_REQUIRE(epi == EPI_BIAS || epi == EPI_SILU || epi == EPI_RELU || epi == EPI_RESID || epi == EPI_GLU ||
                     epi == EPI_CONV_RELU,
                 "gemm: unknown epilogue " + std::to_string(epi));
  COHERE_REQUIRE(epi != EPI_RESID || resid, "gemm: residual epilogue needs resid");
  COHERE_REQUIRE(lda % 8 == 0 && aligned16(a) && aligned16(w), "gemm: operand rows must be 16-byte aligned");
  COHERE_REQUIRE(!bias || (reinterpret_cast<uintptr_t>(bias) & 7) == 0, "gemm: bias must be 8-byte aligned");
  COHERE_REQUIRE(aligned16(out) && ldc % 8 == 0, "gemm: output rows must be 16-byte aligned");
  COHERE_REQUIRE(epi != EPI_RESID || (aligned16(resid) && ldr % 8 == 0), "gemm: residual rows must be aligned");
  if (M == 0) return 0;
  GemmArgs p{};
  // the int8 kernel's byte addressing: K and the row stride in bytes
  p.X = reinterpret_cast<const int8_t*>(a); p.W = reinterpret_cast<const int8_t*>(w); p.bias = bias; p.C = out;
  p.R = resid; p.ldx = 2 * lda; p.ldc = ldc; p.ldr = ldr;
  p.M = (int)M; p.N = (int)N; p.K = (int)(2 * K); p.group = p.K; p.qgroup = 256; p.epi = epi; p.alpha = alpha;
  const int tile = choose_tile(p, false, true);
  COHERE_REQUIRE(tile >= 0, "gemm: no gfx950 tile fits N=" + std::to_string(p.N));
  if (!launch_gemm_bf16(tile, epi, p, reinterpret_cast<hipStream_t>(stream))) {
    cohere::set_error("gemm: tile " + std::to_string(tile) + " has no bf16 kernel for this epilogue");
    return 1;
  }
  return cohere::check_launch("gemm");
}
