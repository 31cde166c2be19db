// cohere_encoder_layers without a caller workspace, for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc). The layer loop's intermediate buffers (QKV,
// attention / GLU output, int8 rows and scales) live in one file-scope device array per GPU, `scratch`, held until
// the process ends. Nothing here allocates: the array's device address is looked up once per device and passed to
// the same launches as the caller's workspace would be.
//
// Every buffer in it is written before it is read within a call, so nothing needs clearing between calls. All
// calls on one GPU share that GPU's array: calls that overlap on one GPU (two streams, two threads) race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "cohere_hip.h"
#include "common.h"

namespace {

static __device__ __align__(256) unsigned char scratch[COHERE_ENC_NOALLOC_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // the array's device address on each GPU (each holds its own copy)

// The device address of this GPU's array (looked up on the first call with that device current).
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    cohere::set_error("encoder_layers_noalloc: no current device");
    return 1;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      cohere::set_error(std::string("encoder_layers_noalloc: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
      return 1;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace

extern "C" int cohere_encoder_layers_noalloc(uint16_t* x, int64_t rows, const void* const* fields, int64_t n_layers,
                                             const double* eps, const int32_t* tiles, int64_t n_tiles,
                                             const int32_t* lo, const int32_t* hi, int64_t rel_off, int64_t max_len,
                                             int64_t rel_rows, double scale, int32_t heads, int32_t head_dim,
                                             int32_t int8, const int64_t* cfg, int64_t n_cfg, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(cfg && n_cfg >= 5, "encoder_layers_noalloc: cfg needs at least 5 entries");
  const int64_t need = cohere_encoder_branch_workspace_bytes(rows, cfg[4], int8);
  COHERE_REQUIRE(need >= 0, "encoder_layers_noalloc: bad rows or feed-forward group");
  COHERE_REQUIRE(need <= (int64_t)COHERE_ENC_NOALLOC_BYTES,
                 "encoder_layers_noalloc: " + std::to_string(rows) + " rows need " + std::to_string(need) +
                     " bytes of scratch, more than the " + std::to_string((int64_t)COHERE_ENC_NOALLOC_BYTES) +
                     " the library holds; use cohere_encoder_layers with a workspace");
  void* ws = nullptr;
  if (scratch_of_current_device(&ws)) return 1;
  return cohere_encoder_layers(x, rows, fields, n_layers, eps, tiles, n_tiles, lo, hi, rel_off, max_len, rel_rows,
                               scale, heads, head_dim, int8, cfg, n_cfg, ws, COHERE_ENC_NOALLOC_BYTES, stream);
}
