// One decoding step's non-GEMM kernels for continuous batching (reference kernels/csrc/decoder_ops.cu,
// kernels/csrc/dec_attn.cuh), for gfx950. Row r of a step works on slot active[r] of the per-slot state and caches,
// so rows join and leave between steps without moving any cache.
//
//   dec_embed       x = LN0(bf16(embed[token] + pos_table[position])), h = LN1(x)           (decoder_ops.cu:24-54)
//   dec_add_ln      x = bf16(x + y), h = LN(x)                                                  (decoder_ops.cu:56-83)
//   dec_attention   softmax(q k^T scale) v of one new token per row over its slot's cache; self-attention first
//                   writes the new key and value at position pos (int8 caches: quantized with one scale per
//                   128-vector) and attends to it unquantized; cross-attention reads the slot's audio frames
//                                                                                               (dec_attn.cuh:84-188)
//   dec_pick        greedy choice (first index of the maximum), the forced prompt, pad once finished, end at the
//                   end-of-text token or the slot's limit; advances the position                (decoder_ops.cu:106-159)
//   dec_scatter_kv  cross-attention keys/values of packed encoder frames into their slots (bf16, or int8 with a
//                   scale per 128-vector)                                                       (decoder_ops.cu:163-204)
#include "cohere_hip.h"
#include "common.h"
#include "rows.h"

#include <string>
#include <type_traits>

namespace {

using namespace cohere_rows;

constexpr int HD = 128;  // head size

// ---- embedding and residual LayerNorms: one wave per row ------------------------------------------------------------

// one row's embedding by one wave: x = LN0(bf16(emb[t] + ptab[p])), h = LN1(x)
// FULL: width == VEC * 512 (the loads then need no per-lane guard)
template <int VEC, bool FULL = false>
DEVI void embed_row(int64_t t, int p, const uint16_t* emb, const uint16_t* ptab, const uint16_t* w0,
                    const uint16_t* b0, float eps0, const uint16_t* w1, const uint16_t* b1, float eps1, uint16_t* xr,
                    uint16_t* hr, int width, int lane) {
  const LnParams<VEC> p0 = load_ln<VEC, FULL>(w0, b0, width, lane), p1 = load_ln<VEC, FULL>(w1, b1, width, lane);
  Row<VEC> e, q;
  load_row<VEC, FULL>(emb + t * width, width, lane, e);
  load_row<VEC, FULL>(ptab + (int64_t)p * width, width, lane, q);
#pragma unroll
  for (int i = 0; i < VEC; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) e.v[i][k] = round_bf(e.v[i][k] + q.v[i][k]);
  ln_row<VEC>(e, width, lane, p0, eps0);
  store_row<VEC>(e, width, lane, xr);
  ln_row<VEC>(e, width, lane, p1, eps1);
  store_row<VEC>(e, width, lane, hr);
}

template <int VEC>
__global__ void __launch_bounds__(256) dec_embed_kernel(const int32_t* __restrict__ active,
                                                        const int64_t* __restrict__ tok, const int32_t* __restrict__ pos,
                                                        const uint16_t* __restrict__ emb, const uint16_t* __restrict__ ptab,
                                                        const uint16_t* w0, const uint16_t* b0, float eps0,
                                                        const uint16_t* w1, const uint16_t* b1, float eps1, uint16_t* x,
                                                        uint16_t* h, int rows, int width) {
  const int row = blockIdx.x * 4 + wave_id(), lane = lane_id();
  if (row >= rows) return;
  const int s = active[row];
  embed_row<VEC>(tok[s], pos[s], emb, ptab, w0, b0, eps0, w1, b1, eps1, x + (int64_t)row * width,
                 h + (int64_t)row * width, width, lane);
}

template <int VEC>
__global__ void __launch_bounds__(256) dec_add_ln_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
                                                         int64_t ldy, const uint16_t* w, const uint16_t* b, float eps,
                                                         uint16_t* h, int rows, int width) {
  const int row = blockIdx.x * 4 + wave_id(), lane = lane_id();
  if (row >= rows) return;
  const LnParams<VEC> lp = load_ln<VEC>(w, b, width, lane);
  Row<VEC> a, d;
  load_row<VEC>(x + (int64_t)row * width, width, lane, a);
  load_row<VEC>(y + (int64_t)row * ldy, width, lane, d);
#pragma unroll
  for (int i = 0; i < VEC; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) a.v[i][k] = round_bf(a.v[i][k] + d.v[i][k]);
  store_row<VEC>(a, width, lane, x + (int64_t)row * width);
  ln_row<VEC>(a, width, lane, lp, eps);
  store_row<VEC>(a, width, lane, h + (int64_t)row * width);
}

// ---- attention of one new token per row ---------------------------------------------------------------------------
// A workgroup of 512 threads per (row, head, split): 64 groups of 8 lanes, each lane 16 of the 128 dims, each group
// taking every 64th key of the split, 7 (int8) or 4 (bf16) keys per pass with all their loads in flight at once (a
// whole 448-token self cache or 375-frame cross cache in one memory round trip). A pass's partial dot products meet
// in one transposed reduction over the group's lanes (lane gl ends with key gl's); the online softmax runs in fp32
// per group, one rescale per pass; the 64 groups are combined through LDS at the end (or, with several splits,
// written as partials (o[128], max, sum) for dec_combine).
struct DecAttnArgs {
  const int32_t* active;
  const uint16_t* q;  // (rows, ldq): head h at column h * 128 (self: q | k | v of the new token)
  int64_t ldq;
  uint16_t* k;        // bf16 caches (slots, H, T, 128)
  uint16_t* v;
  int8_t* k8;         // int8 caches (slots, H, T, 128) with scales (slots, H, T)
  int8_t* v8;
  float* ks;
  float* vs;
  const int32_t* n;   // self: position of the new token per slot; cross: audio frames per slot
  int H, T;
  float scale;
  uint16_t* out;      // (rows, H * 128)
  float* part;        // (rows, H, splits, 130) when split
};

constexpr int AG = 64;  // key groups per workgroup (8 lanes each: 512 threads; one pass covers 448 int8 keys)

DEVI void unpack_q8(const uint4& u, float s, float (&f)[16]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 16; ++k) f[k] = (float)(int8_t)((w[k >> 2] >> (8 * (k & 3))) & 0xff);
  if (s != 1.f) {
#pragma unroll
    for (int k = 0; k < 16; ++k) f[k] *= s;
  }
}

DEVI void unpack_bf(const uint4& a, const uint4& b, float (&f)[16]) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}

// group-of-8 reductions (lanes 8g .. 8g+7 of a wave)
DEVI float group_sum(float v) { return group8_sum(v); }
DEVI float group_max(float v) { return group8_max(v); }

// the 16 values a lane holds of a 128-vector as int8 with the vector's scale (absmax / 127 over the 8 lanes)
DEVI void store16_q8(const float (&f)[16], int8_t* dst, float* scale, int gl) {
  float mx = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) mx = fmaxf(mx, fabsf(f[k]));
  mx = group_max(mx);
  const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
  *reinterpret_cast<uint4*>(dst) = make_uint4(q8x4(f[0], f[1], f[2], f[3], inv), q8x4(f[4], f[5], f[6], f[7], inv),
                                               q8x4(f[8], f[9], f[10], f[11], inv),
                                               q8x4(f[12], f[13], f[14], f[15], inv));
  if (gl == 0) *scale = sc;
}

DEVI void attend_one(const float (&q)[16], const float (&kk)[16], const float (&vv)[16], float scale, float& m,
                     float& l, float (&acc)[16]) {
  float d = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) d = __builtin_fmaf(q[k], kk[k], d);
  d = group_sum(d);
  const float s = d * scale, mn = fmaxf(m, s), a = __expf(m - mn), e = __expf(s - mn);
  l = __builtin_fmaf(l, a, e);
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = __builtin_fmaf(acc[k], a, e * vv[k]);
  m = mn;
}

// LDSV selects where a pass's values wait for the softmax weights: in registers (values loaded with the keys) or in
// LDS, copied global -> LDS by the load unit (global_load_lds), each lane's 16-byte chunks into its own slots and read
// back by the same lane (the copy and read-back add latency, and with copies into LDS and register loads both in
// flight the compiler waits for all of them before the first key). The register form fits two workgroups per CU (113-123 VGPRs with 7 key slots per
// pass) and lets each key and value wait for its own load only; LDSV is taken only by split launches whose grid has
// more workgroups than the GPU has CUs. After the keys, the LDS buffer holds the groups' partial outputs.
// EARLY (cross-attention, register form, one split): the first pass's loads are issued before the slot's frame count
// is read. A template parameter, not a run-time choice: two ways into the first pass would make the compiler wait
// for every load in flight where they join.
template <bool SELF, bool Q8, bool LDSV, bool EARLY = false>
__global__ void __launch_bounds__(AG * 8) __attribute__((amdgpu_waves_per_eu(LDSV ? 4 : 1)))
dec_attention_kernel(const DecAttnArgs p) {
  static_assert(!EARLY || (!SELF && !LDSV), "the early pass is the register form's cross-attention");
  // key slots per group per pass: KL loaded (int8: 7, so that a pass covers 448 keys, the decoder's longest caches,
  // and the register form fits two workgroups per CU), KB in the lanes' reduction (a power of two; slots KL..KB-1
  // are never live)
  constexpr int KB = Q8 ? 8 : 4, KL = Q8 ? 7 : 4;
  constexpr int VB = Q8 ? 1 : 2;  // 16-byte value chunks per lane per key
  constexpr int VBYTES = LDSV ? KL * VB * 8 * 1024 : 0, CBYTES = AG * (HD + 4) * 4;
  __shared__ __attribute__((aligned(16))) char sbuf[VBYTES > CBYTES ? VBYTES : CBYTES];
  __shared__ float sm[AG], sl[AG], sw[AG], sML[2];
  __shared__ float spart[4][HD];
  float(*sacc)[HD + 4] = reinterpret_cast<float(*)[HD + 4]>(sbuf);
  // self-attention: the upper half of the heads takes the rows in reverse order. Workgroups rows * H / 2 apart tend to
  // share a CU; so paired, a CU holds two different rows' caches instead of two heads of one row, which evens the
  // keys per CU when cache lengths differ (config 3, U(1..448): 0.5329 -> 0.5314 ms per step, alternating runs)
  const int r = SELF && blockIdx.y >= gridDim.y / 2 ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
  const int h = blockIdx.y, sp = blockIdx.z, nsp = gridDim.z;
  const int s = p.active[r];
  const int tid = threadIdx.x, grp = tid >> 3, gl = tid & 7, wave = tid >> 6, wl = tid & 63;
  // the query as loaded: converted once the first pass's loads are issued (a conversion ahead of them would make the
  // wave wait for the query before issuing the keys)
  uint4 qr[2];
  {
    const uint16_t* qp = p.q + (int64_t)r * p.ldq + h * HD + gl * 16;
    qr[0] = *reinterpret_cast<const uint4*>(qp);
    qr[1] = *reinterpret_cast<const uint4*>(qp + 8);
  }
  float q[16];
  const int64_t vec0 = ((int64_t)s * p.H + h) * p.T;  // index of key 0's 128-vector
  // LDSV: the wave's LDS block for pass key i, value chunk c (64 lanes x 16 bytes; lane wl's slot at + 16 wl)
  auto vblock = [&](int i, int c) { return sbuf + ((i * VB + c) * 8 + wave) * 1024; };
  uint4 kr[KL][Q8 ? 1 : 2], vr[LDSV ? 1 : KL][Q8 ? 1 : 2];
  // int8 scales: lane gl of a group loads the scales of the group's key gl of the pass (one load each for the key
  // and value scales, where one load per key made 16 narrow loads per lane): the lane that ends up with that key's
  // dot product
  float ksl = 1.f, vsl = 1.f;
  // 32-bit offsets from the layer's cache base (a layer's cache stays below 2^32 elements), so that the loads take
  // the uniform base in scalar registers and one offset register each
  const uint32_t vrow0 = (uint32_t)vec0;
  // key slot i of a pass is live for the wave while its first group's key j0w + i * AG is below the end (the
  // wave's groups are consecutive, so the others' keys of that slot are past it too): slots past the end for the
  // whole wave are not computed (a scalar branch; short caches do a fraction of a pass). They are still loaded (key 0
  // of the slot: one cache line for the wave), so that the loads in flight are the same count everywhere and each
  // key waits only for its own load.
  auto wave_first = [&](int j0) { return __builtin_amdgcn_readfirstlane(j0 - (grp & 7)); };
  // issue order: the scales, the keys, then the values
  auto load_pass = [&](int j0, int limit) {
    if constexpr (Q8) {  // byte offsets in 32 bits: the loads then use the scalar base (one offset register each)
      const int jj = j0 + gl * AG;
      const uint32_t off = (vrow0 + (uint32_t)(jj < limit ? jj : 0)) << 2;
      ksl = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.ks) + off);
      vsl = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.vs) + off);
    }
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int jj = j0 + i * AG;
      const uint32_t vec = vrow0 + (uint32_t)(jj < limit ? jj : 0);
      if constexpr (Q8) {
        kr[i][0] = *reinterpret_cast<const uint4*>(p.k8 + (vec * HD + gl * 16));
      } else {
        kr[i][0] = *reinterpret_cast<const uint4*>(p.k + (vec * HD + gl * 16));
        kr[i][1] = *reinterpret_cast<const uint4*>(p.k + (vec * HD + gl * 16 + 8));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the keys' loads stay ahead of the values': a key waits for keys only
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int jj = j0 + i * AG;
      const uint32_t vec = vrow0 + (uint32_t)(jj < limit ? jj : 0);
      if constexpr (!LDSV) {
        if constexpr (Q8) {
          vr[i][0] = *reinterpret_cast<const uint4*>(p.v8 + (vec * HD + gl * 16));
        } else {
          vr[i][0] = *reinterpret_cast<const uint4*>(p.v + (vec * HD + gl * 16));
          vr[i][1] = *reinterpret_cast<const uint4*>(p.v + (vec * HD + gl * 16 + 8));
        }
      } else if constexpr (Q8) {
        __builtin_amdgcn_global_load_lds(p.v8 + (vec * HD + gl * 16), (LDS_AS void*)vblock(i, 0), 16, 0, 0);
      } else {
        const uint16_t* src = p.v + (vec * HD + gl * 16);
        __builtin_amdgcn_global_load_lds(src, (LDS_AS void*)vblock(i, 0), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(src + 8, (LDS_AS void*)vblock(i, 1), 16, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // nothing that waits for a load is scheduled among the pass's loads
  };
  auto read_v = [&](int i, float (&vv)[16]) {
    uint4 a, b;
    if constexpr (LDSV) {
      a = *reinterpret_cast<const uint4*>(vblock(i, 0) + wl * 16);
      if constexpr (!Q8) b = *reinterpret_cast<const uint4*>(vblock(i, 1) + wl * 16);
    } else {
      a = vr[i][0];
      if constexpr (!Q8) b = vr[i][1];
    }
    if constexpr (Q8) unpack_q8(a, 1.f, vv);
    else unpack_bf(a, b, vv);
  };
  // register form, cross-attention: the first pass is issued before the slot's length is known (clamped to the
  // cache's T frames, masked by the length after), so the key loads do not wait for it; the frame count is close to
  // T anyway. Self-attention lengths grow from 1, so there the length is waited for. (In the LDS form the early pass
  // kept the loaded keys live across the length load and made the kernel spill.)
  constexpr bool early = EARLY;
  if (early) load_pass(grp, p.T);
  const int n = p.n[s];
  float m = -INFINITY, l = 0.f, acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.f;
  // self-attention: the new key and value go into the cache at n and are attended as computed. Their loads are issued
  // here and the work is done after the first pass's cache loads are issued (the cache's keys below n are not
  // touched by it), so the workgroup's first wave does not pay a memory round trip of its own before its pass.
  const bool fresh = SELF && sp == 0 && grp == 0;
  uint4 knr[2], vnr[2];
  const uint16_t* nrow = p.q + (int64_t)r * p.ldq + p.H * HD + h * HD + gl * 16;
  if (fresh) {
    knr[0] = *reinterpret_cast<const uint4*>(nrow);
    knr[1] = *reinterpret_cast<const uint4*>(nrow + 8);
    vnr[0] = *reinterpret_cast<const uint4*>(nrow + p.H * HD);
    vnr[1] = *reinterpret_cast<const uint4*>(nrow + p.H * HD + 8);
  }
  auto new_token = [&]() {
    float kn[16], vn[16];
    unpack_bf(knr[0], knr[1], kn);
    unpack_bf(vnr[0], vnr[1], vn);
    const int64_t vec = vec0 + n;
    if constexpr (Q8) {
      store16_q8(kn, p.k8 + vec * HD + gl * 16, p.ks + vec, gl);
      store16_q8(vn, p.v8 + vec * HD + gl * 16, p.vs + vec, gl);
    } else {
      uint16_t* kd = p.k + vec * HD + gl * 16;
      uint16_t* vd = p.v + vec * HD + gl * 16;
      *reinterpret_cast<uint4*>(kd) = knr[0];
      *reinterpret_cast<uint4*>(kd + 8) = knr[1];
      *reinterpret_cast<uint4*>(vd) = vnr[0];
      *reinterpret_cast<uint4*>(vd + 8) = vnr[1];
    }
    attend_one(q, kn, vn, p.scale, m, l, acc);
  };
  const int chunk = (n + nsp - 1) / nsp, start = sp * chunk, end = min(n, start + chunk);
  // each group takes KL keys per pass (every 64th key), all loads issued before any use: one memory round trip per
  // pass; then one softmax update for the pass
  int j0 = start + grp;
  // a pass's loads are issued at the top of the pass: no registers carry loaded keys across passes, so one pass of KL
  // keys per group fits the register budget. Caches of more than KL * AG = 448 keys pay one more memory round trip
  // per pass. One pass over the loaded keys is a lambda, so that the early pass runs outside the loop (a loop whose
  // first pass could come from registers loaded before it made the compiler copy every loaded register at its back
  // edge).
  // One pass over the loaded keys. Each lane holds its 16 dimensions' partial dot product with every key of the pass;
  // a transposed reduction over the group's 8 lanes (exchange half the keys with the lane 4 away, then 2, then 1)
  // leaves lane gl with the whole dot product of key kx = gl (KB 8) or gl / 2 (KB 4) in 7 (3) lane moves -- the lane
  // that also holds that key's int8 scale. The pass's maximum and sum of weights go over the group's lanes; the
  // weights reach the value loop by a broadcast from the key's lane.
  const int kx = KB == 8 ? gl : gl >> 1;
  auto process = [&](int j0) {
    const int j0w = wave_first(j0);
    float d[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      d[i] = 0.f;
      if (i >= KL || j0w + i * AG >= end) continue;
      float kk[16];
      if constexpr (Q8) unpack_q8(kr[i][0], 1.f, kk);  // the integers; the key's scale multiplies the dot product
      else unpack_bf(kr[i][0], kr[i][1], kk);
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) t = __builtin_fmaf(q[k], kk[k], t);
      d[i] = t;
    }
    // lanes 0-3 of the group keep the first half of the keys, lanes 4-7 the second: send the other half across the
    // half mirror (lane i <-> 7 - i) and add what comes back; then the same within each half across lane ^ 2 and ^ 1
    const bool hi4 = gl & 4, hi2 = gl & 2, hi1 = gl & 1;
    float d1[KB / 2];
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) {
      const float keep = hi4 ? d[j + KB / 2] : d[j], give = hi4 ? d[j] : d[j + KB / 2];
      d1[j] = keep + dpp_mov<DPP_HALF_MIRROR>(give);
    }
    float d2[KB / 4];
#pragma unroll
    for (int j = 0; j < KB / 4; ++j) {
      const float keep = hi2 ? d1[j + KB / 4] : d1[j], give = hi2 ? d1[j] : d1[j + KB / 4];
      d2[j] = keep + dpp_mov<DPP_XOR2>(give);
    }
    float dk;
    if constexpr (KB == 8) {
      const float keep = hi1 ? d2[1] : d2[0], give = hi1 ? d2[0] : d2[1];
      dk = keep + dpp_mov<DPP_XOR1>(give);
    } else {
      dk = d2[0] + dpp_mov<DPP_XOR1>(d2[0]);  // both lanes of a pair hold the key's sum
    }
    if constexpr (Q8) dk *= ksl;
    const float sc = kx < KL && j0 + kx * AG < end ? dk * p.scale : -INFINITY;
    const float mb = fmaxf(m, group_max(sc));
    const float a = __expf(m - mb), e = __expf(sc - mb);
    l = __builtin_fmaf(l, a, group_sum(KB == 8 || !hi1 ? e : 0.f));
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] *= a;
    const float ew = Q8 ? e * vsl : e;  // int8: the value's scale goes into the weight
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      if (j0w + i * AG >= end) break;
      // LDSV: value i has landed in LDS once at most the younger copies are still in flight (stores issued later
      // only make the wait longer)
      if constexpr (LDSV) wait_vm_upto((KL - 1 - i) * VB);
      const float w = group8_bcast(ew, KB == 8 ? i : 2 * i);
      float vv[16];
      read_v(i, vv);
#pragma unroll
      for (int k = 0; k < 16; ++k) acc[k] = __builtin_fmaf(w, vv[k], acc[k]);
      __builtin_amdgcn_sched_barrier(0);
    }
    m = mb;
  };
  // the first pass outside the loop: its loads were issued early (cross, register form) or are issued before the new
  // token's work (self)
  // (for every lane, even past the end: the loads clamp their keys, and a load inside a branch would leave the
  // compiler unable to count the loads in flight after it)
  if (!early) load_pass(j0, end);
  unpack_bf(qr[0], qr[1], q);
  if (fresh) new_token();
  if (j0 < end) process(j0);
  j0 += KL * AG;
  for (; j0 < end; j0 += KL * AG) {
    if constexpr (LDSV) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // last pass's value reads are done
    load_pass(j0, end);
    process(j0);
  }
  // LDSV: every wave is done reading its values before the buffer holds the partial outputs
  if constexpr (LDSV) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  // combine the groups: weights w_g = exp(m_g - M). One wave finds M, the weights and L = sum w_g l_g; then every
  // thread sums 16 groups of one output dimension, and the four partial sums are added in order.
  if (gl == 0) {
    sm[grp] = m;
    sl[grp] = l;
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) sacc[grp][gl * 16 + k] = acc[k];
  __syncthreads();
  static_assert(AG == 64 && AG * 8 == 4 * 128, "one weight per lane of the first wave; four partial sums per dim");
  if (tid < 64) {
    const float mg = sm[tid];
    float M = mg;
    M = wave_max64(M);
    const float w = M == -INFINITY ? 0.f : __expf(mg - M);
    float L = w * sl[tid];
    L = wave_sum64(L);
    sw[tid] = w;
    if (tid == 0) {
      sML[0] = M;
      sML[1] = L;
    }
  }
  __syncthreads();
  {
    const int d = tid & (HD - 1), part = tid >> 7;
    float o = 0.f;
#pragma unroll
    for (int g = part * 16; g < part * 16 + 16; ++g) o = __builtin_fmaf(sw[g], sacc[g][d], o);
    spart[part][d] = o;
  }
  __syncthreads();
  if (tid >= HD) return;
  const float M = sML[0], L = sML[1];
  const float O = (spart[0][tid] + spart[1][tid]) + (spart[2][tid] + spart[3][tid]);
  if (nsp == 1) {
    p.out[(int64_t)r * p.H * HD + h * HD + tid] = f2bf(O / L);
  } else {
    float* part = p.part + (((int64_t)r * p.H + h) * nsp + sp) * (HD + 2);
    part[tid] = O;
    if (tid == 0) {
      part[HD] = M;
      part[HD + 1] = L;
    }
  }
}

__global__ void __launch_bounds__(HD) dec_combine_kernel(const float* __restrict__ part, int nsp, uint16_t* out,
                                                         int H) {
  const int r = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const float* base = part + ((int64_t)r * H + h) * nsp * (HD + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsp; ++s) M = fmaxf(M, base[s * (HD + 2) + HD]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < nsp; ++s) {
    const float* q = base + s * (HD + 2);
    const float w = q[HD] == -INFINITY ? 0.f : __expf(q[HD] - M);
    L = __builtin_fmaf(w, q[HD + 1], L);
    O = __builtin_fmaf(w, q[d], O);
  }
  out[(int64_t)r * H * HD + h * HD + d] = f2bf(O / L);
}

// ---- greedy choice -------------------------------------------------------------------------------------------------
// the next step's embedding of the row, done by the same workgroup after the choice (EVEC > 0), and the end flag
// mirrored into host memory
struct PickEmbed {
  const uint16_t *emb, *ptab, *w0, *b0, *w1, *b1;
  float eps0, eps1;
  uint16_t *x, *h;
  int width;
  uint8_t* flags;  // host-mapped end flags (null: none)
};

template <int EVEC, bool EFULL = false>
__global__ void __launch_bounds__(256) dec_pick_kernel(const uint16_t* __restrict__ logits, int V,
                                                       const int32_t* __restrict__ active, int dummy, int64_t* tok,
                                                       int32_t* pos, uint8_t* finished, const int64_t* forced, int FP,
                                                       const int32_t* plen, const int32_t* limit, int64_t* out, int OUT,
                                                       int64_t pad, int64_t eos, const PickEmbed pe) {
  __shared__ float sb[4];
  __shared__ int sa[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int s = active[r];  // a padding row (the dummy slot) is scanned too and then dropped: its loads do not wait
  const uint16_t* row = logits + (int64_t)r * V;
  // the slot's state, loaded now by the lane that updates it, so that after the scan only the chosen token's
  // embedding is a round trip of its own
  int64_t tok0 = 0, forced0 = 0;
  int pos0 = 0, plen0 = 0, lim0 = 0;
  uint8_t fin0 = 1;
  if (tid == 0) {
    fin0 = finished[s];
    pos0 = pos[s];
    plen0 = plen[s];
    lim0 = limit[s];
    if constexpr (EVEC > 0) tok0 = tok[s];
  }
  float best = -INFINITY;
  int arg = 0x7fffffff;
  // eight 16-byte loads per thread in flight at once (a 16384-entry row in one memory round trip), then the scan in
  // index order per thread
  constexpr int LB = 8;
  for (int i0 = tid * 8; i0 < V; i0 += 256 * 8 * LB) {
    uint4 u[LB];
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int i = i0 + j * 256 * 8;
      u[j] = i < V ? *reinterpret_cast<const uint4*>(row + i) : make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u,
                                                                           0xff80ff80u);  // -inf: never picked
    }
    // the forced token at the next position (used only inside the prompt, so its index is clamped to the row)
    if (tid == 0 && i0 == 0) forced0 = forced[(int64_t)s * FP + min(pos0 + 1, FP - 1)];
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const uint32_t w[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float v = __uint_as_float(k & 1 ? w[k >> 1] & 0xffff0000u : w[k >> 1] << 16);
        if (v > best) {  // strictly greater: the first index of a tie stays
          best = v;
          arg = i0 + j * 256 * 8 + k;
        }
      }
    }
  }
  // the wave's (maximum, first index): pairs combined across lane ^ 1, 2, 4, 8 (DPP lane moves; the combination is
  // symmetric, so each lane group holds one pair before the next level) and ^ 16, 32 (permlane swaps: both results
  // are the group's and its partner's pair, in some order)
  auto take = [&](float ob, int oa) {
    if (ob > best || (ob == best && oa < arg)) {
      best = ob;
      arg = oa;
    }
  };
  auto dpp_i = [](auto ctrl, int v) { return __builtin_amdgcn_update_dpp(0, v, decltype(ctrl)::value, 0xF, 0xF, false); };
  take(dpp_mov<DPP_XOR1>(best), dpp_i(std::integral_constant<int, DPP_XOR1>{}, arg));
  take(dpp_mov<DPP_XOR2>(best), dpp_i(std::integral_constant<int, DPP_XOR2>{}, arg));
  take(dpp_mov<DPP_HALF_MIRROR>(best), dpp_i(std::integral_constant<int, DPP_HALF_MIRROR>{}, arg));
  take(dpp_mov<DPP_ROR8>(best), dpp_i(std::integral_constant<int, DPP_ROR8>{}, arg));
  {
    const auto b2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(best), __float_as_uint(best), false, false);
    const auto a2 = __builtin_amdgcn_permlane16_swap((unsigned)arg, (unsigned)arg, false, false);
    best = __uint_as_float(b2[0]);
    arg = (int)a2[0];
    take(__uint_as_float(b2[1]), (int)a2[1]);
  }
  {
    const auto b2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(best), __float_as_uint(best), false, false);
    const auto a2 = __builtin_amdgcn_permlane32_swap((unsigned)arg, (unsigned)arg, false, false);
    best = __uint_as_float(b2[0]);
    arg = (int)a2[0];
    take(__uint_as_float(b2[1]), (int)a2[1]);
  }
  if ((tid & 63) == 0) {
    sb[tid >> 6] = best;
    sa[tid >> 6] = arg;
  }
  __syncthreads();
  __shared__ int64_t s_tok;
  __shared__ int s_pos;
  if (tid == 0) {
    int64_t t_next = tok0;
    int p_next = EVEC > 0 ? pos0 : 0;
    // ended at an earlier step (or the dummy slot): nothing moves until the host retires the slot
    if (s != dummy && !fin0) {
      for (int w = 1; w < 4; ++w)
        if (sb[w] > best || (sb[w] == best && sa[w] < arg)) {
          best = sb[w];
          arg = sa[w];
        }
      const int at = pos0 + 1;
      const bool in_prompt = at < plen0;
      const int64_t nt = in_prompt ? forced0 : (int64_t)arg;
      const uint8_t fin = (!in_prompt && (nt == eos || at >= lim0)) ? 1 : 0;
      out[(int64_t)s * OUT + at] = nt;
      tok[s] = nt;
      pos[s] = at;
      finished[s] = fin;
      if (pe.flags) pe.flags[s] = fin;
      t_next = nt;
      p_next = at;
    }
    if constexpr (EVEC > 0) {
      s_tok = t_next;
      s_pos = p_next;
    }
  }
  if constexpr (EVEC > 0) {
    __syncthreads();
    if (tid < 64)
      embed_row<EVEC, EFULL>(s_tok, s_pos, pe.emb, pe.ptab, pe.w0, pe.b0, pe.eps0, pe.w1, pe.b1, pe.eps1,
                      pe.x + (int64_t)r * pe.width, pe.h + (int64_t)r * pe.width, pe.width, tid);
  }
  (void)pad;
}

// ---- cross-attention keys and values into their slots --------------------------------------------------------------
// kv (rows, L * 2 * H * 128) of packed frames (per layer: k heads then v heads), row i = frame frame_of[i] of slot
// slot_of[i]; caches (L, S, H, T, 128). 16 threads per 128-vector.
template <bool Q8>
__global__ void __launch_bounds__(256) dec_scatter_kv_kernel(const uint16_t* __restrict__ kv,
                                                             const int32_t* __restrict__ slot_of,
                                                             const int32_t* __restrict__ frame_of, uint16_t* ck,
                                                             uint16_t* cv, int8_t* ck8, int8_t* cv8, float* cks,
                                                             float* cvs, int rows, int L, int S, int H, int T) {
  const int chunks = L * 2 * H * (HD / 8);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // rows * chunks is a multiple of 16
  const bool live = idx < (int64_t)rows * chunks;
  const int row = live ? (int)(idx / chunks) : 0, c = live ? (int)(idx % chunks) : 0;
  const int d8 = c % (HD / 8), h = (c / (HD / 8)) % H, kvi = (c / (HD / 8 * H)) % 2, l = c / (HD / 8 * H * 2);
  uint4 u = make_uint4(0, 0, 0, 0);
  if (live) u = *reinterpret_cast<const uint4*>(kv + (int64_t)row * chunks * 8 + (int64_t)c * 8);
  const int64_t vec = live ? ((((int64_t)l * S + slot_of[row]) * H + h) * T + frame_of[row]) : 0;
  if constexpr (!Q8) {
    if (live) *reinterpret_cast<uint4*>((kvi ? cv : ck) + vec * HD + d8 * 8) = u;
  } else {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    float f[8], mx = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      f[k] = __uint_as_float(k & 1 ? w[k >> 1] & 0xffff0000u : w[k >> 1] << 16);
      mx = fmaxf(mx, fabsf(f[k]));
    }
    mx = row16_max(mx);
    if (!live) return;
    const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
    *reinterpret_cast<uint2*>((kvi ? cv8 : ck8) + vec * HD + d8 * 8) =
        make_uint2(q8x4(f[0], f[1], f[2], f[3], inv), q8x4(f[4], f[5], f[6], f[7], inv));
    if (d8 == 0) (kvi ? cvs : cks)[vec] = sc;
  }
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

int vec_of(int64_t width) { return (int)((width + 511) / 512); }

}  // namespace

extern "C" int cohere_dec_embed(const int32_t* active, int64_t rows, const int64_t* tok, const int32_t* pos,
                                const uint16_t* emb, const uint16_t* ptab, const uint16_t* w0, const uint16_t* b0,
                                float eps0, const uint16_t* w1, const uint16_t* b1, float eps1, uint16_t* x,
                                uint16_t* h, int64_t width, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && width > 0 && width % 8 == 0 && width <= 2048,
                 "dec_embed: width must be a multiple of 8, at most 2048");
  COHERE_REQUIRE(active && tok && pos && emb && ptab && w0 && b0 && w1 && b1 && x && h && al16(emb) && al16(ptab) &&
                     al16(x) && al16(h) && al16(w0) && al16(b0) && al16(w1) && al16(b1),
                 "dec_embed: bad pointer");
  if (rows == 0) return 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int grid = (int)((rows + 3) / 4);
#define EMB(V)                                                                                                      \
  dec_embed_kernel<V><<<grid, 256, 0, st>>>(active, tok, pos, emb, ptab, w0, b0, eps0, w1, b1, eps1, x, h, (int)rows, \
                                            (int)width)
  switch (vec_of(width)) {
    case 1: EMB(1); break;
    case 2: EMB(2); break;
    case 3: EMB(3); break;
    default: EMB(4); break;
  }
#undef EMB
  return cohere::check_launch("dec_embed");
}

extern "C" int cohere_dec_add_ln(uint16_t* x, const uint16_t* y, int64_t ldy, const uint16_t* w, const uint16_t* b,
                                 float eps, uint16_t* h, int64_t rows, int64_t width, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && width > 0 && width % 8 == 0 && width <= 2048,
                 "dec_add_ln: width must be a multiple of 8, at most 2048");
  COHERE_REQUIRE(x && y && w && b && h && al16(x) && al16(y) && ldy % 8 == 0 && al16(w) && al16(b) && al16(h),
                 "dec_add_ln: bad pointer");
  if (rows == 0) return 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int grid = (int)((rows + 3) / 4);
#define ADD(V) dec_add_ln_kernel<V><<<grid, 256, 0, st>>>(x, y, ldy, w, b, eps, h, (int)rows, (int)width)
  switch (vec_of(width)) {
    case 1: ADD(1); break;
    case 2: ADD(2); break;
    case 3: ADD(3); break;
    default: ADD(4); break;
  }
#undef ADD
  return cohere::check_launch("dec_add_ln");
}

namespace {
int num_cus() {
  static const int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess || v <= 0)
      v = 256;
    return v;
  }();
  return n;
}

int attention_entry(bool self, bool q8, DecAttnArgs& p, int64_t rows, int64_t slots, int64_t splits,
                    int64_t part_len, void* stream, const char* name) {
  const std::string nm(name);
  COHERE_REQUIRE(rows >= 0 && p.H > 0 && p.H <= 65535 && p.T > 0 && splits >= 1 && splits <= 64, nm + ": bad sizes");
  // the kernels address a cache with 32-bit element offsets
  COHERE_REQUIRE(slots > 0 && slots * (int64_t)p.H * p.T * HD < (int64_t(1) << 32),
                 nm + ": slots x heads x T x 128 must be positive and below 2^32");
  COHERE_REQUIRE(p.active && p.q && p.n && p.out && al16(p.q) && p.ldq % 8 == 0 && al16(p.out),
                 nm + ": bad pointer");
  COHERE_REQUIRE(q8 ? (p.k8 && p.v8 && p.ks && p.vs && al16(p.k8) && al16(p.v8)) : (p.k && p.v && al16(p.k) && al16(p.v)),
                 nm + ": bad cache pointer");
  COHERE_REQUIRE(splits == 1 || (p.part && part_len >= rows * p.H * splits * (HD + 2)),
                 nm + ": splits > 1 needs part with rows x H x splits x 130 floats");
  if (rows == 0) return 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)rows, (unsigned)p.H, (unsigned)splits);
  // the register form (two workgroups per CU at <= 128 VGPRs, each key and value waiting only for its own load)
  // unless the launch is split over more workgroups than the GPU has CUs: at 64 rows x 8 heads self-attention takes
  // 10.5 us there against 11.7 in the LDS form, cross-attention (with its early pass) 12.0 against 13.6
  const bool ldsv = splits > 1 && rows * p.H * splits > num_cus();
#define COHERE_ATT(SELF_, Q8_)                                                                    \
  (ldsv ? (dec_attention_kernel<SELF_, Q8_, true><<<grid, AG * 8, 0, s>>>(p), 0)                  \
        : (dec_attention_kernel<SELF_, Q8_, false><<<grid, AG * 8, 0, s>>>(p), 0))
  if (self) q8 ? COHERE_ATT(true, true) : COHERE_ATT(true, false);
  else if (splits == 1)
    q8 ? dec_attention_kernel<false, true, false, true><<<grid, AG * 8, 0, s>>>(p)
       : dec_attention_kernel<false, false, false, true><<<grid, AG * 8, 0, s>>>(p);
  else q8 ? COHERE_ATT(false, true) : COHERE_ATT(false, false);
#undef COHERE_ATT
  if (splits > 1) dec_combine_kernel<<<dim3((unsigned)rows, (unsigned)p.H), HD, 0, s>>>(p.part, (int)splits, p.out, p.H);
  return cohere::check_launch(name);
}
}  // namespace

extern "C" int cohere_dec_attention(int32_t self, const int32_t* active, int64_t rows, const uint16_t* q, int64_t ldq,
                                    uint16_t* k, uint16_t* v, const int32_t* n, int64_t slots, int64_t heads, int64_t T,
                                    float scale, int64_t splits, float* part, int64_t part_len, uint16_t* out,
                                    void* stream) {
  cohere::clear_error();
  DecAttnArgs p{};
  p.active = active; p.q = q; p.ldq = ldq; p.k = k; p.v = v; p.n = n; p.H = (int)heads; p.T = (int)T;
  p.scale = scale; p.out = out; p.part = part;
  return attention_entry(self != 0, false, p, rows, slots, splits, part_len, stream, "dec_attention");
}

extern "C" int cohere_dec_attention_q8(int32_t self, const int32_t* active, int64_t rows, const uint16_t* q,
                                       int64_t ldq, int8_t* k8, int8_t* v8, float* ks, float* vs, const int32_t* n,
                                       int64_t slots, int64_t heads, int64_t T, float scale, int64_t splits, float* part,
                                       int64_t part_len, uint16_t* out, void* stream) {
  cohere::clear_error();
  DecAttnArgs p{};
  p.active = active; p.q = q; p.ldq = ldq; p.k8 = k8; p.v8 = v8; p.ks = ks; p.vs = vs; p.n = n; p.H = (int)heads;
  p.T = (int)T; p.scale = scale; p.out = out; p.part = part;
  return attention_entry(self != 0, true, p, rows, slots, splits, part_len, stream, "dec_attention_q8");
}

extern "C" int cohere_dec_pick(const uint16_t* logits, int64_t rows, int64_t V, const int32_t* active, int64_t dummy,
                               int64_t* tok, int32_t* pos, uint8_t* finished, const int64_t* forced, int64_t FP,
                               const int32_t* plen, const int32_t* limit, int64_t* out, int64_t OUT, int64_t pad,
                               int64_t eos, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && V > 0 && V % 8 == 0, "dec_pick: the vocabulary must be a multiple of 8");
  COHERE_REQUIRE(logits && active && tok && pos && finished && forced && plen && limit && out && al16(logits),
                 "dec_pick: bad pointer");
  if (rows == 0) return 0;
  dec_pick_kernel<0><<<(unsigned)rows, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      logits, (int)V, active, (int)dummy, tok, pos, finished, forced, (int)FP, plen, limit, out, (int)OUT, pad, eos,
      PickEmbed{});
  return cohere::check_launch("dec_pick");
}

extern "C" int cohere_dec_pick_embed(const uint16_t* logits, int64_t rows, int64_t V, const int32_t* active,
                                     int64_t dummy, int64_t* tok, int32_t* pos, uint8_t* finished,
                                     const int64_t* forced, int64_t FP, const int32_t* plen, const int32_t* limit,
                                     int64_t* out, int64_t OUT, int64_t pad, int64_t eos, const uint16_t* emb,
                                     const uint16_t* ptab, const uint16_t* w0, const uint16_t* b0, float eps0,
                                     const uint16_t* w1, const uint16_t* b1, float eps1, uint16_t* x, uint16_t* h,
                                     int64_t width, uint8_t* flags_host, void* stream) {
  cohere::clear_error();
  COHERE_REQUIRE(rows >= 0 && V > 0 && V % 8 == 0, "dec_pick_embed: the vocabulary must be a multiple of 8");
  COHERE_REQUIRE(logits && active && tok && pos && finished && forced && plen && limit && out && al16(logits),
                 "dec_pick_embed: bad pointer");
  COHERE_REQUIRE(width > 0 && width % 8 == 0 && width <= 2048,
                 "dec_pick_embed: width must be a multiple of 8, at most 2048");
  COHERE_REQUIRE(emb && ptab && w0 && b0 && w1 && b1 && x && h && al16(emb) && al16(ptab) && al16(x) && al16(h) &&
                     al16(w0) && al16(b0) && al16(w1) && al16(b1),
                 "dec_pick_embed: bad embedding pointer");
  uint8_t* flags_dev = nullptr;
  if (flags_host) {
    void* d = nullptr;
    COHERE_REQUIRE(hipHostGetDevicePointer(&d, flags_host, 0) == hipSuccess && d,
                   "dec_pick_embed: the end flags must be pinned host memory");
    flags_dev = static_cast<uint8_t*>(d);
  }
  if (rows == 0) return 0;
  const PickEmbed pe{emb, ptab, w0, b0, w1, b1, eps0, eps1, x, h, (int)width, flags_dev};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define PICK(VV, F)                                                                                                \
  dec_pick_kernel<VV, F><<<(unsigned)rows, 256, 0, st>>>(logits, (int)V, active, (int)dummy, tok, pos, finished,      \
                                                         forced, (int)FP, plen, limit, out, (int)OUT, pad, eos, pe)
  const bool full = width % 512 == 0;  // vec_of(width) chunks of 512, all whole
  switch (vec_of(width)) {
    case 1: if (full) PICK(1, true); else PICK(1, false); break;
    case 2: if (full) PICK(2, true); else PICK(2, false); break;
    case 3: if (full) PICK(3, true); else PICK(3, false); break;
    default: if (full) PICK(4, true); else PICK(4, false); break;
  }
#undef PICK
  return cohere::check_launch("dec_pick_embed");
}

namespace {
int scatter_entry(bool q8, const uint16_t* kv, int64_t rows, const int32_t* slot_of, const int32_t* frame_of,
                  uint16_t* ck, uint16_t* cv, int8_t* ck8, int8_t* cv8, float* cks, float* cvs, int64_t L, int64_t S,
                  int64_t H, int64_t T, void* stream, const char* name) {
  const std::string nm(name);
  COHERE_REQUIRE(rows >= 0 && L > 0 && S > 0 && H > 0 && T > 0, nm + ": bad sizes");
  COHERE_REQUIRE(kv && slot_of && frame_of && al16(kv), nm + ": bad pointer");
  COHERE_REQUIRE(q8 ? (ck8 && cv8 && cks && cvs) : (ck && cv && al16(ck) && al16(cv)), nm + ": bad cache pointer");
  if (rows == 0) return 0;
  const int64_t n = rows * L * 2 * H * (HD / 8);
  const unsigned grid = (unsigned)((n + 255) / 256);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (q8)
    dec_scatter_kv_kernel<true><<<grid, 256, 0, s>>>(kv, slot_of, frame_of, nullptr, nullptr, ck8, cv8, cks, cvs,
                                                     (int)rows, (int)L, (int)S, (int)H, (int)T);
  else
    dec_scatter_kv_kernel<false><<<grid, 256, 0, s>>>(kv, slot_of, frame_of, ck, cv, nullptr, nullptr, nullptr,
                                                      nullptr, (int)rows, (int)L, (int)S, (int)H, (int)T);
  return cohere::check_launch(name);
}
}  // namespace

extern "C" int cohere_dec_scatter_kv(const uint16_t* kv, int64_t rows, const int32_t* slot_of, const int32_t* frame_of,
                                     uint16_t* ck, uint16_t* cv, int64_t L, int64_t S, int64_t H, int64_t T,
                                     void* stream) {
  cohere::clear_error();
  return scatter_entry(false, kv, rows, slot_of, frame_of, ck, cv, nullptr, nullptr, nullptr, nullptr, L, S, H, T,
                       stream, "dec_scatter_kv");
}

extern "C" int cohere_dec_scatter_kv_q8(const uint16_t* kv, int64_t rows, const int32_t* slot_of,
                                        const int32_t* frame_of, int8_t* ck, int8_t* cv, float* cks, float* cvs,
                                        int64_t L, int64_t S, int64_t H, int64_t T, void* stream) {
  cohere::clear_error();
  return scatter_entry(true, kv, rows, slot_of, frame_of, nullptr, nullptr, ck, cv, cks, cvs, L, S, H, T, stream,
                       "dec_scatter_kv_q8");
}
