/* C ABI of the MI355X (gfx950) quantized-GEMM path of cohere-inference.
 *
 * Every entry point takes raw device pointers, element strides and sizes, and a HIP stream (hipStream_t passed as
 * void*; NULL is the default stream). Every call only enqueues work on that stream: no host synchronisation, no
 * device allocation, so each is safe inside HIP graph capture. Return value: 0 on success, nonzero on a rejected
 * argument or a failed launch; cohere_last_error() then describes it (thread-local, valid until the next call on the
 * same thread).
 *
 * bf16 tensors are passed as uint16_t bit patterns. All matrices are row-major with the given row strides (in
 * elements); the innermost stride is 1.
 *
 * Epilogue codes (kernels/cuda_ext.py:28 of the reference: EPI_BIAS, EPI_SILU, EPI_RELU, EPI_RESID, EPI_GLU,
 * EPI_SILU_Q8, EPI_CONV_RELU = range(7)); the int8 GEMMs accept BIAS, RESID, GLU, SILU_Q8, and COHERE_EPI_I32 (7),
 * which writes the raw int32 accumulators: a parity hook with no counterpart in the reference.
 */
#ifndef COHERE_HIP_H
#define COHERE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  COHERE_EPI_BIAS = 0,
  COHERE_EPI_SILU = 1,
  COHERE_EPI_RELU = 2,
  COHERE_EPI_RESID = 3,
  COHERE_EPI_GLU = 4,
  COHERE_EPI_SILU_Q8 = 5,
  COHERE_EPI_CONV_RELU = 6,
  COHERE_EPI_I32 = 7
};

/* Replaces gemm_i8 (reference kernels/csrc/gemm_int8.cu:351-391, bound at kernels/csrc/bindings.cpp:67).
 * out = epilogue(dequant(a @ w^T) + bias): a int8 [M, K] (lda), sa fp32 [M, K / group] (ldsa), w int8 [N, K]
 * contiguous, sw fp32 [N], bias bf16 [N] or NULL.
 *   BIAS     out bf16 [M, N]
 *   RESID    out = resid + alpha * bf16(v), bf16 [M, N]; out may alias resid
 *   GLU      out bf16 [M, N / 2] from interleaved (a, gate) rows of w
 *   SILU_Q8  out int8 [M, N] and qs fp32 [M, N / G] (ldqs), G = the column tile of the reference config cfg
 *            (64 for cfg 5 and 9, 256 for 4, 6 and 8, else 128; 256 when cfg < 0)
 *   I32      out int32 [M, N] raw accumulators (group == K only)
 * Requirements: K % 64 == 0, group % 64 == 0, K % group == 0, N % 64 == 0; a, w, sw 16-byte aligned with lda % 16 ==
 * 0; out rows 16-byte aligned (out and ldc x element size); bias 8-byte aligned; resid 16-byte aligned, ldr % 8 == 0.
 * cfg is the reference's tile-config id (0, 1, 3-10; unknown ids are rejected) or -1; it never changes the result
 * (tiles are chosen for gfx950 here). */
int cohere_gemm_i8(const int8_t* a, int64_t lda, const float* sa, int64_t ldsa, int64_t group, const int8_t* w,
                   const float* sw, const uint16_t* bias, void* out, int64_t ldc, int32_t epi, const uint16_t* resid,
                   int64_t ldr, float alpha, float* qs, int64_t ldqs, int64_t M, int64_t N, int64_t K, int32_t cfg,
                   void* stream);

/* Replaces gemm_sp (reference kernels/csrc/gemm_sparse.cu:214-253, bound at kernels/csrc/bindings.cpp:68) and
 * widens it to gemm_i8's epilogues. x int8 [M, K] (ldx) with sx fp32 [M, K / group] (ldsx); the 2:4 weights as
 * kernels/sparse.py compress_24 stores them: wc int8 [N, K / 2] kept values, e int32 [N, K / 32] selectors (a nibble
 * i0 | i1 << 2 per group of four, lowest K in the lowest nibble) -- exactly the CDNA4 SMFMAC A operand and index
 * format, used as is. Epilogues, outputs and alignment as cohere_gemm_i8 (e 16-byte aligned too). Requirements:
 * K % 128 == 0, group % 128 == 0, K % group == 0, N % 64 == 0. The result equals cohere_gemm_i8 on the decompressed
 * weights, bit for bit.
 * cfg: the reference's sparse config id (0-4) or -1. */
int cohere_gemm_sp(const int8_t* x, int64_t ldx, const float* sx, int64_t ldsx, int64_t group, const int8_t* wc,
                   const int32_t* e, const float* sw, const uint16_t* bias, void* out, int64_t ldc, int32_t epi,
                   const uint16_t* resid, int64_t ldr, float alpha, float* qs, int64_t ldqs, int64_t M, int64_t N,
                   int64_t K, int32_t cfg, void* stream);

/* No single counterpart in the reference; the same operation as cohere_gemm_sp (reference
 * kernels/csrc/gemm_sparse.cu:214-253, kernels/sparse.py:26-39 for the weight format) with the 2:4 weight in this
 * library's stage-tiled layout wt (cohere_pack_24_tiled of the compressed values and selectors): every DMA
 * instruction then reads one contiguous kilobyte. Same arguments, requirements and results, bit for bit. */
int cohere_gemm_sp_tiled(const int8_t* x, int64_t ldx, const float* sx, int64_t ldsx, int64_t group, const uint8_t* wt,
                         const float* sw, const uint16_t* bias, void* out, int64_t ldc, int32_t epi,
                         const uint16_t* resid, int64_t ldr, float alpha, float* qs, int64_t ldqs, int64_t M,
                         int64_t N, int64_t K, int32_t cfg, void* stream);

/* Load-time weight preparation for cohere_gemm_sp_tiled (host memory, plain loops; no counterpart in the reference):
 * compress_24's kept values wc int8 [N, K/2] and selectors e int32 [N, K/32] into out, cohere_pack_24_tiled_bytes(N, K)
 * bytes (-1 unless N % 16 == 0 and K % 128 == 0). For each block of 16 channels and each 128-wide K stage, one
 * 1280-byte record: 64 chunks of 16 kept bytes (chunk i = row i/4's chunk (i%4) ^ ((i/8)%4) of the stage), then the
 * 16 rows' four selector words of the stage (rows 8-15 with words 0-1 and 2-3 swapped). */
int64_t cohere_pack_24_tiled_bytes(int64_t N, int64_t K);
int cohere_pack_24_tiled(const int8_t* wc, const int32_t* e, int64_t N, int64_t K, uint8_t* out);

/* Replaces gemm (reference kernels/csrc/gemm.cu:246-279, bound at kernels/csrc/bindings.cpp:65): bf16
 * out = epi(a w^T + bias), a bf16 [M, K] (lda), w bf16 [N, K] contiguous, fp32 accumulation, bias bf16 [N] or
 * null added in fp32 before the first rounding. epi: EPI_BIAS, EPI_SILU (silu(bf16(v))), EPI_RELU, EPI_RESID
 * (bf16(alpha * bf16(v) + resid), resid may be out), EPI_GLU (interleaved value/gate rows, out [M, N/2]),
 * EPI_CONV_RELU (relu(bf16(acc) + bias): a convolution whose bias is added after its rounding). Requirements:
 * K % 32 == 0, N % 64 == 0, 16-byte aligned rows. cfg: the reference's config id (3, 5 or 8), validated, otherwise
 * ignored (the gfx950 tile is chosen by shape). */
int cohere_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* w, const uint16_t* bias, uint16_t* out,
                     int64_t ldc, int32_t epi, const uint16_t* resid, int64_t ldr, float alpha, int64_t M, int64_t N,
                     int64_t K, int32_t cfg, void* stream);

/* Replaces quantize_rows (reference kernels/csrc/encoder_ops.cu:545-553, bound at bindings.cpp:69): bf16 rows x
 * [rows, cols] (ldx) -> int8 q [rows, cols] (ldq) and fp32 s [rows]; one scale per row, absmax / 127;
 * cols % 8 == 0, cols <= 8192. */
int cohere_quantize_rows(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* s, int64_t rows, int64_t cols,
                         void* stream);

/* Replaces layernorm_q8 (reference kernels/csrc/encoder_ops.cu:522-543, bound at bindings.cpp:70): h = LN(x) as int8
 * hq with per-row scale hs; with w2 != NULL, x = LN1(x) in place and h = LN2(x). bf16 x [rows, cols] (ldx),
 * weights/biases bf16 [cols]. */
int cohere_layernorm_q8(uint16_t* x, int64_t ldx, const uint16_t* w1, const uint16_t* b1, float eps1,
                        const uint16_t* w2, const uint16_t* b2, float eps2, int8_t* hq, int64_t ldq, float* hs,
                        int64_t rows, int64_t cols, void* stream);

/* Replaces dec_w8_linear (reference kernels/csrc/dec_w8.cu:207-234, bound at bindings.cpp:76). y bf16 [M, N] (ldy) =
 * x bf16 [M, K] (ldx) @ dequant(w)^T + bias (ReLU), M <= 64; w uint8 [N, K] in prepare_w8's layout (int8 + 128,
 * bytes permuted within every 16 of K, reference kernels/stream_decoder.py:38-48), sw fp32 [N]. bn (16, 32, 64) and
 * splits (1..16, K % (128 * splits) == 0) are the reference's tuning knobs, checked as it checks them (splits > 1
 * needs ws, fp32 >= N/bn * splits * 64 * bn elements, and counters, int32 >= N/bn); the gfx950 kernel reduces K
 * inside each workgroup, so it chooses its own tiling and never touches ws or counters. Needs N % 16 == 0 and
 * K % 64 == 0. */
int cohere_dec_w8_linear(const uint16_t* x, int64_t ldx, const uint8_t* w, const float* sw, const uint16_t* bias,
                         uint16_t* y, int64_t ldy, int32_t relu, int64_t bn, int64_t splits, float* ws, int64_t ws_len,
                         int32_t* counters, int64_t counters_len, int64_t M, int64_t N, int64_t K, void* stream);

/* Replaces the bf16 decoder projections (reference kernels/decoder_kernels.py:55-66 `linear`, Triton for <= 32 rows;
 * kernels/stream_decoder.py:23-27 F.linear above): y bf16 [M, N] = x bf16 [M, K] @ w bf16 [N, K]^T + bias (ReLU),
 * M <= 64, fp32 accumulation; N % 16 == 0, K % 64 == 0. */
int cohere_linear_bf16(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* bias, uint16_t* y,
                       int64_t ldy, int32_t relu, int64_t M, int64_t N, int64_t K, void* stream);

/* No single counterpart in the reference: its decoder step (kernels/stream_decoder.py:176-199) runs
 * dec_add_ln (kernels/csrc/decoder_ops.cu:56-83) between the projections; this entry point folds that LayerNorm and
 * residual add into the projections around it, so that a step has three launches per layer fewer. With the same
 * arithmetic as dec_add_ln followed by dec_w8_linear / linear_bf16, its results are bit-identical to theirs.
 *   ln_w non-NULL: the LayerNorm prologue -- h = LN(x) (fp32 statistics, bf16 result, eps) is computed in the
 *                  kernel for the call's rows and used as the GEMM input; 512 <= K <= 1024;
 *   sw non-NULL:   w is int8 in prepare_w8's layout with per-channel scales (dec_w8_linear), else bf16 [N, K];
 *   epilogue:      0 y = r, 1 y = ReLU(r), 2 y = bf16(y + bf16(r)) in place (the residual add; not with ln_w),
 *                  r = x' @ w^T (scaled) + bias.
 * M <= 64, N % 16 == 0, K % 64 == 0. */
int cohere_dec_linear_fused(const uint16_t* x, int64_t ldx, const uint16_t* ln_w, const uint16_t* ln_b, float eps,
                            const void* w, const float* sw, const uint16_t* bias, uint16_t* y, int64_t ldy,
                            int32_t epilogue, int64_t M, int64_t N, int64_t K, void* stream);

/* Replaces layernorm (reference kernels/csrc/encoder_ops.cu:501-520, bound at kernels/csrc/bindings.cpp:73):
 * h = LN1(x) as bf16; with w2 (non-NULL), x = LN1(x) in place and h = LN2(x). h may be x. fp32 statistics, the
 * result rounded to bf16. cols % 8 == 0, cols <= 2048. */
int cohere_layernorm(uint16_t* x, int64_t ldx, const uint16_t* w1, const uint16_t* b1, float eps1, const uint16_t* w2,
                     const uint16_t* b2, float eps2, uint16_t* h, int64_t ldh, int64_t rows, int64_t cols,
                     void* stream);

/* Replaces dwconv_bn_silu (reference kernels/csrc/encoder_ops.cu:643-656, bound at kernels/csrc/bindings.cpp:74):
 * y = bf16(silu(bf16(bn(bf16(dwconv(x)))))) per packed row: x, y bf16 [rows, channels] contiguous; w fp32
 * [channels, 9]; cb, bn_scale, bn_shift fp32 [channels]; seq_lo / seq_hi int32 [rows], the packed-row range of each
 * row's own sequence (taps outside it read zero). channels % 8 == 0, <= 2048; ksize must be 9. */
int cohere_dwconv_bn_silu(const uint16_t* x, const float* w, const float* cb, const float* bn_scale,
                          const float* bn_shift, const int32_t* seq_lo, const int32_t* seq_hi, uint16_t* y,
                          int64_t rows, int64_t channels, int64_t ksize, void* stream);

/* Replaces dwconv_bn_silu_q8 (reference kernels/csrc/encoder_ops.cu:658-674, bound at kernels/csrc/bindings.cpp:75):
 * as cohere_dwconv_bn_silu, the rows written as int8 hq [rows, channels] with one fp32 scale per row hs [rows]
 * (absmax / 127, the arithmetic of cohere_quantize_rows). */
int cohere_dwconv_bn_silu_q8(const uint16_t* x, const float* w, const float* cb, const float* bn_scale,
                             const float* bn_shift, const int32_t* seq_lo, const int32_t* seq_hi, int8_t* hq,
                             float* hs, int64_t rows, int64_t channels, int64_t ksize, void* stream);

/* Replaces relpos_attention (reference kernels/csrc/encoder_ops.cu:676-707, bound at kernels/csrc/bindings.cpp:85).
 * out [rows, H D] bf16 = relative-position self-attention of qkv [rows, 3 H D] bf16 (q | k | v) within each
 * sequence: score[i, j] = ((q_i + bu) . k_j) scale + bf16(bf16((q_i + bv) . rk[i - j + rel_off]) scale), softmax
 * over the sequence's keys, probabilities rounded to bf16 for the value product. rk [rel_rows, H D] bf16, bu / bv
 * [H, D] bf16; tiles int32 [n_tiles, 4] = (sequence start row, sequence length, first query row, 0) for every
 * 64-query tile of every sequence. Head size D = 80 or 160 (the reference: 160 only). Rejects
 * max_len - 1 > rel_off or rel_off + max_len + 62 >= rel_rows, as the reference does. */
int cohere_relpos_attention(const uint16_t* qkv, const uint16_t* rk, int64_t rel_rows, const uint16_t* bu,
                            const uint16_t* bv, const int32_t* tiles, int64_t n_tiles, int64_t heads, int64_t head_dim,
                            int64_t rel_off, int64_t max_len, float scale, uint16_t* out, void* stream);

/* ---- decoder step (reference kernels/csrc/decoder_ops.cu, dec_attn.cuh) ------------------------------------------
 * Row r of a step works on slot active[r] (int32 [rows]) of the per-slot state: tok int64 [slots], pos int32
 * [slots], and caches laid out (slots, heads, T, 128). */

/* Replaces dec_embed (reference kernels/csrc/decoder_ops.cu:24-54, 208-219, bound at kernels/csrc/bindings.cpp:77):
 * x = LN0(bf16(emb[tok[s]] + ptab[pos[s]])), h = LN1(x), bf16 [rows, width] contiguous; emb / ptab bf16 tables with
 * `width` columns. width % 8 == 0, <= 2048. */
int cohere_dec_embed(const int32_t* active, int64_t rows, const int64_t* tok, const int32_t* pos, const uint16_t* emb,
                     const uint16_t* ptab, const uint16_t* w0, const uint16_t* b0, float eps0, const uint16_t* w1,
                     const uint16_t* b1, float eps1, uint16_t* x, uint16_t* h, int64_t width, void* stream);

/* Replaces dec_add_ln (reference kernels/csrc/decoder_ops.cu:56-83, 221-233, bound at kernels/csrc/bindings.cpp:78):
 * x = bf16(x + y) in place (x [rows, width] contiguous, y row stride ldy), h = LN(x). */
int cohere_dec_add_ln(uint16_t* x, const uint16_t* y, int64_t ldy, const uint16_t* w, const uint16_t* b, float eps,
                      uint16_t* h, int64_t rows, int64_t width, void* stream);

/* Replaces dec_attention (reference kernels/csrc/decoder_ops.cu:235-262, dec_attn.cuh:84-188, bound at
 * kernels/csrc/bindings.cpp:80): out bf16 [rows, heads * 128] = softmax(q k^T scale) v for one new token per row.
 * self != 0: q is the qkv projection [rows, ldq] (q | k | v, heads x 128 each), the new key and value are first
 * written into the caches at position n[s] and attended as computed, with keys 0 .. n[s]-1 from the cache; self == 0:
 * q [rows, ldq] over the slot's n[s] audio frames. Caches k, v bf16 (slots, heads, T, 128). splits > 1 splits each
 * (row, head)'s keys over workgroups and needs part with rows x heads x splits x 130 floats. slots is the caches'
 * first dimension: the kernels address a cache with 32-bit element offsets, so slots x heads x T x 128 must stay
 * below 2^32 (refused otherwise). */
int cohere_dec_attention(int32_t self, const int32_t* active, int64_t rows, const uint16_t* q, int64_t ldq,
                         uint16_t* k, uint16_t* v, const int32_t* n, int64_t slots, int64_t heads, int64_t T, float scale,
                         int64_t splits, float* part, int64_t part_len, uint16_t* out, void* stream);

/* Replaces dec_attention_q8 (reference kernels/csrc/decoder_ops.cu:264-290, bound at kernels/csrc/bindings.cpp:81):
 * as cohere_dec_attention over int8 caches k8, v8 (slots, heads, T, 128) with fp32 scales ks, vs (slots, heads, T),
 * one per 128-vector; self-attention writes the new key and value quantized (absmax / 127, round half even) and
 * attends to them unquantized. */
int cohere_dec_attention_q8(int32_t self, const int32_t* active, int64_t rows, const uint16_t* q, int64_t ldq,
                            int8_t* k8, int8_t* v8, float* ks, float* vs, const int32_t* n, int64_t slots, int64_t heads, int64_t T,
                            float scale, int64_t splits, float* part, int64_t part_len, uint16_t* out, void* stream);

/* Replaces dec_pick (reference kernels/csrc/decoder_ops.cu:106-159, 304-314, bound at kernels/csrc/bindings.cpp:83):
 * per row (slot s = active[r], skipped when s == dummy or finished[s]): the first index of the maximum of logits bf16
 * [rows, V]; at = pos[s] + 1; the token is forced[s, at] (int64 [slots, FP]) while at < plen[s], else the argmax;
 * out[s, at] = tok[s] = token (out int64 [slots, OUT]); pos[s] = at; finished[s] = 1 at eos or at >= limit[s]
 * outside the prompt. V % 8 == 0. */
int cohere_dec_pick(const uint16_t* logits, int64_t rows, int64_t V, const int32_t* active, int64_t dummy,
                    int64_t* tok, int32_t* pos, uint8_t* finished, const int64_t* forced, int64_t FP,
                    const int32_t* plen, const int32_t* limit, int64_t* out, int64_t OUT, int64_t pad, int64_t eos,
                    void* stream);

/* No single counterpart in the reference: its step ends with dec_pick (kernels/csrc/decoder_ops.cu:106-159) and the
 * end flags' copy to the host, and the next step starts with dec_embed (decoder_ops.cu:24-54; stream_decoder.py:
 * 176-199). This entry point is dec_pick, then, by the same workgroup, the row's next embedding exactly as dec_embed
 * computes it from the slot's (possibly new) token and position -- x / h [rows, width] -- and, with flags_host
 * non-NULL (pinned host memory, one byte per slot), each stepped slot's end flag written there. Arguments as
 * cohere_dec_pick followed by cohere_dec_embed's tables and LayerNorms. */
int cohere_dec_pick_embed(const uint16_t* logits, int64_t rows, int64_t V, const int32_t* active, int64_t dummy,
                          int64_t* tok, int32_t* pos, uint8_t* finished, const int64_t* forced, int64_t FP,
                          const int32_t* plen, const int32_t* limit, int64_t* out, int64_t OUT, int64_t pad,
                          int64_t eos, const uint16_t* emb, const uint16_t* ptab, const uint16_t* w0,
                          const uint16_t* b0, float eps0, const uint16_t* w1, const uint16_t* b1, float eps1,
                          uint16_t* x, uint16_t* h, int64_t width, uint8_t* flags_host, void* stream);

/* Replaces dec_scatter_kv (reference kernels/csrc/decoder_ops.cu:163-175, 316-327, bound at
 * kernels/csrc/bindings.cpp:84): kv bf16 [rows, L x 2 x H x 128] (per layer: keys of every head, then values) of
 * packed encoder frames, row i = frame frame_of[i] of slot slot_of[i], into caches ck, cv (L, S, H, T, 128). */
int cohere_dec_scatter_kv(const uint16_t* kv, int64_t rows, const int32_t* slot_of, const int32_t* frame_of,
                          uint16_t* ck, uint16_t* cv, int64_t L, int64_t S, int64_t H, int64_t T, void* stream);

/* Replaces dec_scatter_kv_q8 (reference kernels/csrc/decoder_ops.cu:177-204, 292-302, bound at
 * kernels/csrc/bindings.cpp:82): as cohere_dec_scatter_kv into int8 caches with one fp32 scale per 128-vector
 * (cks, cvs (L, S, H, T)). */
int cohere_dec_scatter_kv_q8(const uint16_t* kv, int64_t rows, const int32_t* slot_of, const int32_t* frame_of,
                             int8_t* ck, int8_t* cv, float* cks, float* cvs, int64_t L, int64_t S, int64_t H,
                             int64_t T, void* stream);

/* Number of per-layer tensors of cohere_encoder_layers: the reference's 53 (its enum F,
 * kernels/csrc/encoder_loop.cpp:34-44) followed by 4 of this library's own (the feed-forwards' first linears in 2:4
 * form: ff1 kept bytes, ff1 selectors, ff2 kept bytes, ff2 selectors; NULL keeps the dense first linear, as the
 * reference always does). */
enum { COHERE_ENC_N_REF_FIELDS = 53, COHERE_ENC_N_FIELDS = 57 };

/* Device bytes cohere_encoder_layers needs as workspace for `rows` packed frames and feed-forward scale group
 * `group` (-1 on bad arguments). The reference allocates the same buffers inside the call. */
int64_t cohere_encoder_workspace_bytes(int64_t rows, int64_t group);

/* Device bytes the int8 (int8 nonzero) or bf16 branch of cohere_encoder_layers alone needs (-1 on bad arguments);
 * cohere_encoder_workspace_bytes is the larger of the two. */
int64_t cohere_encoder_branch_workspace_bytes(int64_t rows, int64_t group, int32_t int8);

/* Replaces encoder_layers, int8 branch (reference kernels/csrc/encoder_loop.cpp:50-99, bound at
 * kernels/csrc/bindings.cpp:66): every layer of the FastConformer encoder on packed frames x [rows, 1280] bf16, in
 * place, in the reference's launch order. fields: n_layers x COHERE_ENC_N_FIELDS device pointers in the reference's
 * field order, then the 4 extra 2:4 first-linear fields (NULL for the empty tensors: a dense W1 or W2 whose 2:4 form
 * is given, the 2:4 fields of a dense linear, absent biases). A 2:4 linear whose kept-values field is set and whose
 * selectors field is NULL holds its weight in the stage-tiled layout of cohere_pack_24_tiled there (run by
 * cohere_gemm_sp_tiled; the same results). eps: n_layers x 5 (ff1, att, conv, ff2, out). tiles / lo / hi / rel_off /
 * max_len / scale as in
 * cohere_relpos_attention and cohere_dwconv_bn_silu; rel_rows the table rows. cfg: the reference's list (bf16 config,
 * int8 QKV, grouped FF W2, FF W1, FF group, PW1, O/PW2, 2:4 FF W2). int8 nonzero runs the W8A8 branch on the
 * quantized fields; int8 zero the bf16 branch (reference encoder_loop.cpp:101-124) on the bf16 weight fields with
 * the bf16 GEMM config cfg[0] (3, 5 or 8). workspace: at least cohere_encoder_branch_workspace_bytes(rows, cfg[4],
 * int8) bytes of device memory (cohere_encoder_workspace_bytes is enough for either branch). */
int cohere_encoder_layers(uint16_t* x, int64_t rows, const void* const* fields, int64_t n_layers, const double* eps,
                          const int32_t* tiles, int64_t n_tiles, const int32_t* lo, const int32_t* hi, int64_t rel_off,
                          int64_t max_len, int64_t rel_rows, double scale, int32_t heads, int32_t head_dim,
                          int32_t int8, const int64_t* cfg, int64_t n_cfg, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* No counterpart in the reference. cohere_encoder_layers for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same arguments without the
 * workspace. The loop's buffers live in a file-scope device array of COHERE_ENC_NOALLOC_BYTES (64 MiB) per GPU, held
 * until the process ends; a call whose branch needs more (cohere_encoder_branch_workspace_bytes: above ~3900 rows of
 * the int8 layers or ~2600 of the bf16 ones) fails with an error and launches nothing. The call allocates nothing.
 * All calls on one GPU share its array: calls that overlap on one GPU (two streams, two threads) race. The array
 * costs 64 MiB of device memory on every GPU of a process that loads it (from the first call, when the runtime loads
 * the code object holding it, until the process exits), whether or not the entry point is called again. */
enum { COHERE_ENC_NOALLOC_BYTES = 64 << 20 };
int cohere_encoder_layers_noalloc(uint16_t* x, int64_t rows, const void* const* fields, int64_t n_layers,
                                  const double* eps, const int32_t* tiles, int64_t n_tiles, const int32_t* lo,
                                  const int32_t* hi, int64_t rel_off, int64_t max_len, int64_t rel_rows, double scale,
                                  int32_t heads, int32_t head_dim, int32_t int8, const int64_t* cfg, int64_t n_cfg,
                                  void* stream);

/* Bytes of device workspace cohere_logmel_features needs for total_frames frames (fp32 log-mel values). */
int64_t cohere_logmel_workspace_bytes(int64_t total_frames);

/* Replaces logmel_features (reference kernels/csrc/features.cu:105-132, bound at kernels/csrc/bindings.cpp:79;
 * caller kernels/features.py:76-88): normalized log-mel features of packed pieces, valid frames only. x fp32: the
 * pieces' (dithered) samples back to back; meta int64 [3 pieces + 1]: each piece's first sample, its length, then
 * the cumulative valid-frame counts (a piece of n samples has n / 160 valid frames); window fp32 [512] the Hann
 * window of 400 centred in 512; mel fp32 [128, 257] the filter bank; band int32 [128, 2] each band's first and end
 * nonzero bin; preemph the pre-emphasis coefficient. out bf16 [pieces, T, 128]: frame t < valid of piece p gets
 * (log(mel(|rfft|^2) + 2^-24) - mean) / (std + 1e-5) per band over the piece's valid frames (unbiased variance);
 * other frames are left as they are (the caller zeroes out). work: cohere_logmel_workspace_bytes(total_frames) bytes
 * of device memory. */
int cohere_logmel_features(const float* x, const int64_t* meta, int64_t pieces, int64_t total_frames,
                           const float* window, const float* mel, const int32_t* band, float preemph, uint16_t* out,
                           int64_t T, float* work, void* stream);

/* Replaces sub_conv0_dw (reference kernels/csrc/encoder_ops.cu:709-719, bound at kernels/csrc/bindings.cpp:71;
 * caller kernels/fast_encoder.py:196): the subsampling's conv0 (1 -> C, 3x3, stride 2, padding 1) + bias + ReLU and
 * the first depthwise 3x3 stride-2 convolution + bias, per sequence (zero padding at its ends), channels-last.
 * feats bf16 [B, T, 128] (ld_seq elements between sequences); mel_len int32 [B] frames per sequence; rows int32
 * [n_rows, 2] (sequence, output row t2); w0 / w2 fp32 [C, 9], b0 / b2 fp32 [C]; out bf16 [n_rows, 32, C].
 * C % 64 == 0, C <= 1024. */
int cohere_sub_conv0_dw(const uint16_t* feats, int64_t ld_seq, const int32_t* mel_len, const int32_t* rows,
                        int64_t n_rows, const float* w0, const float* b0, const float* w2, const float* b2,
                        uint16_t* out, int64_t C, void* stream);

/* Replaces sub_dw (reference kernels/csrc/encoder_ops.cu:723-734, bound at kernels/csrc/bindings.cpp:72; caller
 * kernels/fast_encoder.py:199): depthwise 3x3 stride-2 convolution + bias on channels-last sequences. x bf16
 * [sum T_in, F_in, C] with in_start / in_len int32 [B] each sequence's first row and row count; rows int32
 * [n_rows, 2] (sequence, output row); w fp32 [C, 9], b fp32 [C]; out bf16 [n_rows, F_in / 2, C]. C % 8 == 0,
 * 16-byte aligned x and out. */
int cohere_sub_dw(const uint16_t* x, const int32_t* in_start, const int32_t* in_len, const int32_t* rows,
                  int64_t n_rows, const float* w, const float* b, uint16_t* out, int64_t F_in, int64_t C,
                  void* stream);

/* The last error on this thread ("" when none). */
const char* cohere_last_error(void);

/* Library version string. */
const char* cohere_version(void);

/* Tuning hook (no counterpart in the reference): force the gfx950 tile of the int8 GEMMs (-1 = automatic choice by
 * shape; -2 / -3 switch off / on the split of evenly divisible tile grids into one part per XCD, on by default).
 * Used by bench.py's sweeps; results never depend on it. Returns the number of tiles available. */
int cohere_set_gemm_tile(int32_t tile);

/* Tuning hook (no counterpart in the reference): force the skinny projections' workgroup shape -- strips of 16
 * channels per workgroup (1, 2, 4) and waves per workgroup (4, 8, 16); strips <= 0 restores the automatic choice.
 * Results never depend on it. */
int cohere_set_skinny_shape(int32_t strips, int32_t waves);

#ifdef __cplusplus
}
#endif

#endif /* COHERE_HIP_H */
