/*
 * turboquant_hip.h -- C ABI of the MI355X (gfx950) TurboQuant kernels.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream (hipStream_t passed as void*; NULL = the null stream).  Nothing here
 * allocates: scratch memory is passed in by the caller as (workspace,
 * workspace_bytes), sized by the matching *_workspace_bytes() query.  Calls are
 * asynchronous on `stream`; none synchronizes.  Return value: TQ_OK, or an
 * error code with a message available from tq_last_error() (thread-local).
 * Inputs are validated on the host before any launch; an invalid call launches
 * nothing.
 *
 * Layouts follow the reference (turboquant_kv/reference.py:191-224):
 *   packed row = b bit planes of bpp = ceil(d/8) bytes, plane i = bit i of
 *   every code, dim j in byte j>>3 of its plane at bit 7-(j&7); pad bits 0.
 *   QJL sign rows use the same layout with b = 1.
 *
 * The reference binds its kernels through torch.ops (csrc/registration.cpp:84-99);
 * each entry point below names the schema or Python function it replaces.
 */
#ifndef TURBOQUANT_HIP_H
#define TURBOQUANT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQ_OK 0
#define TQ_EINVAL 1       /* bad argument: shape, bit width, null pointer, size */
#define TQ_EHIP 2         /* a HIP runtime call failed */
#define TQ_EUNSUPPORTED 3 /* valid request outside what these kernels cover */

typedef enum tq_dtype { TQ_F32 = 0, TQ_F16 = 1, TQ_BF16 = 2 } tq_dtype;

/* Message for the last failing call on this thread ("" if none). */
const char* tq_last_error(void);
/* Bumped whenever a signature below changes. */
int tq_abi_version(void);

/*
 * Fused normalize -> rotate -> Lloyd-Max quantize -> bit-plane pack.
 * Replaces schema `rotate_and_quantize(Tensor vectors, Tensor rotation,
 * Tensor boundaries, int bit_width) -> (Tensor, Tensor)` (csrc/registration.cpp:86-88)
 * with the arithmetic of quantize_mse (reference.py:263-317):
 *   n = ||x||, u = x / max(n, 1e-10), y = u R^T, code = #{boundaries < y}.
 * in_dtype: element type of `vectors`.  round_dtype: the type every
 * intermediate is rounded to, as reference.py does for low-precision inputs
 * (TQ_F32 = upcast and compute in fp32, which is what the reference's own
 * torch op does).  norms are written as fp32 (holding the rounded value).
 *   vectors [n, d], rotation [d, d] fp32 row-major, boundaries [2^b - 1] fp32,
 *   packed [n, b*ceil(d/8)] u8, norms [n] fp32.   1 <= b <= 4, 1 <= d <= 256.
 */
int tq_rotate_and_quantize(const void* vectors, tq_dtype in_dtype, tq_dtype round_dtype,
                           int64_t n, int32_t d, const float* rotation,
                           const float* boundaries, int32_t bit_width,
                           uint8_t* packed, float* norms, void* stream);

/*
 * TurboQuant_prod quantize (reference.py:392-469): MSE at b-1 bits on the unit
 * vector (normalized a second time inside, reference.py:441 -> 294-295), the
 * residual r = u - c[codes] R, gamma = ||r||, and sign bits of r S^T (>= 0 -> 1).
 *   boundaries [2^(b-1) - 1], centroids [2^(b-1)] (the b-1 bit codebook),
 *   qjl [d, d] fp32 (S), mse_packed [n, (b-1)*ceil(d/8)], signs [n, ceil(d/8)],
 *   res_norms [n] fp32, norms [n] fp32.   2 <= b <= 5.
 */
int tq_quantize_prod(const void* vectors, tq_dtype in_dtype, tq_dtype round_dtype,
                     int64_t n, int32_t d, const float* rotation, const float* boundaries,
                     const float* centroids, const float* qjl, int32_t bit_width,
                     uint8_t* mse_packed, uint8_t* signs, float* res_norms, float* norms,
                     void* stream);

/* Schema `pack_codes(Tensor codes, int bit_width) -> Tensor` (csrc/registration.cpp:98).
 * codes [n, d] u8 (values < 2^b), packed [n, b*ceil(d/8)].  1 <= b <= 8. */
int tq_pack_codes(const uint8_t* codes, int64_t n, int32_t d, int32_t bit_width,
                  uint8_t* packed, void* stream);

/* Schema `unpack_codes(Tensor packed, int bit_width, int dim) -> Tensor`
 * (csrc/registration.cpp:99).  packed [n, b*ceil(d/8)], codes [n, d]. */
int tq_unpack_codes(const uint8_t* packed, int64_t n, int32_t d, int32_t bit_width,
                    uint8_t* codes, void* stream);

/*
 * dequantize_mse (reference.py:320-367): out = (c[codes] R) * n, computed in
 * `out_dtype` rounding (the reference computes in norms.dtype).
 *   packed [n, b*ceil(d/8)], norms [n] fp32 values, centroids [2^b], rotation [d, d],
 *   out [n, d] of out_dtype.
 */
int tq_dequantize_mse(const uint8_t* packed, const float* norms, int64_t n, int32_t d,
                      int32_t bit_width, const float* centroids, const float* rotation,
                      tq_dtype out_dtype, void* out, void* stream);

/*
 * dequantize_prod (reference.py:472-533):
 *   out = (c[codes] R + sqrt(pi/2)/d * gamma * (s S)) * n,  s = +-1 from the sign bits.
 *   centroids: the (b-1)-bit codebook.
 */
int tq_dequantize_prod(const uint8_t* mse_packed, const uint8_t* signs, const float* res_norms,
                       const float* norms, int64_t n, int32_t d, int32_t bit_width,
                       const float* centroids, const float* rotation, const float* qjl,
                       tq_dtype out_dtype, void* out, void* stream);

/*
 * Schema `attention_scores_packed(Tensor query, Tensor packed_keys, Tensor key_norms,
 * Tensor centroids, Tensor rotation, int bit_width) -> Tensor`
 * (csrc/registration.cpp:89-92; csrc/cpu/quant_cpu.cpp:125-192):
 *   scores[q, t] = key_norms[t] * sum_j (R query_q)_j * centroids[code_tj]   (no 1/sqrt(d))
 *   query [nq, d] (nq = batch*heads) of q_dtype, packed_keys [T, b*ceil(d/8)],
 *   key_norms [T] fp32, scores [nq, T] fp32.  Needs tq_scan_workspace_bytes(nq, d, b, 0).
 */
int tq_attention_scores_packed(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                               const uint8_t* packed_keys, const float* key_norms, int64_t T,
                               const float* centroids, const float* rotation, int32_t bit_width,
                               float* scores, void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * Schema `attention_values_packed(Tensor attn_weights, Tensor packed_values,
 * Tensor value_norms, Tensor centroids, Tensor rotation_T, int bit_width) -> Tensor`
 * (csrc/registration.cpp:93-96; csrc/cpu/quant_cpu.cpp:199-266):
 *   out[q] = (sum_t w[q, t] * value_norms[t] * centroids[code_t]) @ rotation_T
 *   (pass R itself as rotation_T to invert y = x R^T).
 *   attn_weights [nq, T] fp32, out [nq, d] fp32.
 *   Needs tq_values_workspace_bytes(nq, d, T).
 */
size_t tq_values_workspace_bytes(int64_t nq, int32_t d, int64_t T);
int tq_attention_values_packed(const float* attn_weights, int64_t nq, int64_t T,
                               const uint8_t* packed_values, const float* value_norms,
                               const float* centroids, const float* rotation_T, int32_t d,
                               int32_t bit_width, float* out, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * Inner-product top-k scan over packed codes: TurboQuantIndex.search / _search_mse
 * (turboquant_kv/search.py:178-227) and _core.search_packed
 * (csrc/core/turboquant_core.cpp:407-514):
 *   score_i = norms[i] * sum_j LUT[j][code_ij],  LUT[j][l] = (R q)_j * centroids[l],
 *   top k by score descending; equal scores keep the lower index first.
 *   queries [nq, d] of q_dtype (fp16/bf16 are upcast to fp32 before rotation),
 *   packed [N, b*ceil(d/8)], norms [N] fp32, out_scores [nq, k] fp32,
 *   out_ids [nq, k] int64.  k > N pads with (-inf, -1).  1 <= b <= 4, d <= 256, k <= 128.
 */
size_t tq_scan_workspace_bytes(int64_t nq, int32_t d, int32_t bit_width, int64_t N, int32_t k);
int tq_ip_scan_topk(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                    const uint8_t* packed, const float* norms, int64_t N,
                    const float* centroids, const float* rotation, int32_t bit_width, int32_t k,
                    float* out_scores, int64_t* out_ids, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * The same scan (and tq_attention_scores_packed) over 4-bit rows in the pair layout:
 * row i is d/2 bytes, byte p = code[i][2p] << 4 | code[i][2p+1] -- the bytes of the
 * bit-plane row rearranged, written by tq_pack_decode_layout (values = 0, one stream,
 * t_cap = N).  Identical scores and ids; each code is one masked nibble, so a lookup
 * costs one address instruction instead of two.  d must be 64 or 128 and `pairs`
 * 16-byte aligned.  Workspace: tq_scan_pairs_workspace_bytes(nq, d, N, k) for the top-k
 * scan, tq_scan_workspace_bytes(nq, d, 4, 0, 0) for the scores.  With two or more queries
 * and that workspace the top-k runs the multi-query filtered scan (64 queries share each
 * table lookup on the matrix cores; candidates rescored with the reference's arithmetic,
 * so ids and scores are the exact scan's); a workspace of only
 * tq_scan_workspace_bytes(nq, d, 4, N, k) runs the exact multi-query scan.
 * TurboQuantIndex keeps 4-bit MSE databases of those dims in this layout.
 * Replaces: the scan of turboquant_core.cpp:407-514 (search_packed) for query batches.
 */
size_t tq_scan_pairs_workspace_bytes(int64_t nq, int32_t d, int64_t N, int32_t k);
int tq_ip_scan_topk_pairs(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                          const uint8_t* pairs, const float* norms, int64_t N,
                          const float* centroids, const float* rotation, int32_t k,
                          float* out_scores, int64_t* out_ids, void* workspace,
                          size_t workspace_bytes, void* stream);
int tq_attention_scores_pairs(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                              const uint8_t* pairs, const float* key_norms, int64_t T,
                              const float* centroids, const float* rotation, float* scores,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * Prod-mode scoring over pair rows: tq_ip_scan_topk_prod / tq_attention_scores_prod
 * (same arguments, scores bit-identical) with the MSE half stored as pair rows
 * (tq_pack_pair_rows of the bit_width - 1 bit codes; bit_width 3 or 4, d 64 or 128) beside
 * the bit-plane sign rows and the residual norms.  Replaces the reference's prod search
 * (turboquant_kv/search.py:229-252: dequantize every row, matmul); pair rows and sign rows
 * 16-byte aligned.
 */
int tq_ip_scan_topk_prod_pair_rows(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                                   const uint8_t* mse_rows, const uint8_t* signs,
                                   const float* res_norms, const float* norms, int64_t N,
                                   const float* centroids, const float* rotation, const float* qjl,
                                   int32_t bit_width, int32_t k, float* out_scores, int64_t* out_ids,
                                   void* workspace, size_t workspace_bytes, void* stream);
int tq_attention_scores_prod_pair_rows(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                                       const uint8_t* mse_rows, const uint8_t* signs,
                                       const float* res_norms, const float* key_norms, int64_t T,
                                       const float* centroids, const float* rotation,
                                       const float* qjl, int32_t bit_width, float* scores,
                                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Pair rows: 2-, 3- or 4-bit codes arranged so one table index covers the codes of a pair
 * of dims (2p, 2p+1), same bytes per row as the bit-plane rows (d * bits / 8), d = 64 or
 * 128.  TurboQuantIndex keeps its MSE databases of those dims in this form.
 *   4 bits: the pair layout above (byte p = code[2p] << 4 | code[2p+1]).
 *   2 bits: byte b = code[4b] << 6 | code[4b+1] << 4 | code[4b+2] << 2 | code[4b+3]
 *           (each nibble the index code[2p] << 2 | code[2p+1] of one pair).
 *   3 bits: per 32 dims (16 pairs) 12 bytes = words X0, X1, X2: the low 6 bits of byte k
 *           of X_i hold pair 4i + k's index code[2p] << 3 | code[2p+1]; pair 12 + k's
 *           index bits 2i, 2i+1 sit in bits 6-7 of byte k of X_i.
 * tq_pack_pair_rows / tq_unpack_pair_rows convert n rows from / to the reference's bit
 * planes (reference.py:191-224).  tq_ip_scan_topk_pair_rows and
 * tq_attention_scores_pair_rows are tq_ip_scan_topk / tq_attention_scores_packed over
 * them, with identical scores and ids (2 and 3 bits: every pair's two products come from
 * one per-query table, so no multiply per row; 4 bits: the pair-layout kernels).
 * Workspace as tq_ip_scan_topk's (2- and 3-bit calls then take at most 65535 queries), or
 * tq_scan_pair_rows_workspace_bytes(nq, d, bits, N, k): with two or more queries the top-k
 * then runs the multi-query filtered scan, as over the pair layout (fp16 centroid pairs
 * from a 2^(2 bits)-entry table as the matrix cores' B operands, candidates rescored with
 * the reference's arithmetic: the exact scan's ids and scores).  No counterpart in the
 * reference for the size function (its search allocates nothing on a device).
 */
size_t tq_scan_pair_rows_workspace_bytes(int64_t nq, int32_t d, int32_t bit_width, int64_t N,
                                         int32_t k);
int tq_pack_pair_rows(const uint8_t* packed, int64_t n, int32_t d, int32_t bit_width, uint8_t* rows,
                      void* stream);
int tq_unpack_pair_rows(const uint8_t* rows, int64_t n, int32_t d, int32_t bit_width, uint8_t* packed,
                        void* stream);
int tq_ip_scan_topk_pair_rows(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                              const uint8_t* rows, const float* norms, int64_t N,
                              const float* centroids, const float* rotation, int32_t bit_width,
                              int32_t k, float* out_scores, int64_t* out_ids, void* workspace,
                              size_t workspace_bytes, void* stream);
int tq_attention_scores_pair_rows(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                                  const uint8_t* rows, const float* key_norms, int64_t T,
                                  const float* centroids, const float* rotation, int32_t bit_width,
                                  float* scores, void* workspace, size_t workspace_bytes,
                                  void* stream);

/*
 * tq_ip_scan_topk_pairs without a workspace argument.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  The candidate lists live in a static device
 * array of TQ_NOALLOC_SCRATCH_BYTES per GPU, held from library load until the process
 * ends; calls that need more (tq_scan_workspace_bytes(nq, d, 4, N, k) above it: about
 * nq * k <= 340 at N >= 2M) return TQ_EINVAL.  Nothing is allocated and nothing has to
 * start at zero.  Every call on one GPU shares the array: calls that overlap on that GPU
 * (other streams or host threads) race.  `stream` must belong to the current device.
 * Same arguments (without workspace), outputs and tie rule as tq_ip_scan_topk_pairs.
 */
#define TQ_NOALLOC_SCRATCH_BYTES (4u << 20)
int tq_ip_scan_topk_pairs_noalloc(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                                  const uint8_t* pairs, const float* norms, int64_t N,
                                  const float* centroids, const float* rotation, int32_t k,
                                  float* out_scores, int64_t* out_ids, void* stream);

/*
 * Prod-mode scoring without reconstruction.  Replaces TurboQuantIndex._search_prod
 * (turboquant_kv/search.py:229-252: dequantize_prod of every row, then queries @ recon^T
 * and topk) and, for prod-mode caches, the dequantize-then-matmul of
 * QuantizedKVCache.attention_scores (cache.py:282-310, without its 1/sqrt(d)):
 *   score[q, i] = norms[i] * ( sum_j (R q)_j c[code_ij]
 *                              + sqrt(pi/2)/d * res_norms[i] * sum_j (S q)_j (2 sign_ij - 1) )
 * which is <q, dequantize_prod(row i)> (reference.py:472-533) rearranged.  Rows are
 * what tq_quantize_prod writes: mse_packed [N, (b-1)*ceil(d/8)], signs [N, ceil(d/8)],
 * res_norms [N], norms [N]; centroids [2^(b-1)] (the (b-1)-bit codebook), rotation R
 * and qjl S [d, d] fp32.  2 <= bit_width <= 4 (the prod bit budget b).  fp32 sums in
 * another order than the reference's GEMM: scores agree to fp32 rounding, not bit for
 * bit.  Top-k: same output and tie rule as tq_ip_scan_topk.  Workspace:
 * tq_scan_workspace_bytes(nq, d, b, N, k) / (nq, d, b, 0, 0).
 */
int tq_ip_scan_topk_prod(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                         const uint8_t* mse_packed, const uint8_t* signs, const float* res_norms,
                         const float* norms, int64_t N, const float* centroids,
                         const float* rotation, const float* qjl, int32_t bit_width, int32_t k,
                         float* out_scores, int64_t* out_ids, void* workspace,
                         size_t workspace_bytes, void* stream);
int tq_attention_scores_prod(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                             const uint8_t* mse_packed, const uint8_t* signs,
                             const float* res_norms, const float* key_norms, int64_t T,
                             const float* centroids, const float* rotation, const float* qjl,
                             int32_t bit_width, float* scores, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Fused GQA decode attention over a packed KV cache (new op: the semantics of
 * QuantizedKVCache.attention_scores -> softmax -> attention_values,
 * turboquant_kv/cache.py:282-339 with turboquant_kv/vllm_plugin/__init__.py:400,
 * extended to grouped KV heads as HF repeat_kv does: q head h reads kv head
 * h / (hq / hkv)):
 *   s_t = scale * kn_t * sum_j (Rk q)_j ck[kcode_tj],  p = softmax_t(s),
 *   out = (sum_t p_t vn_t cv[vcode_t]) Rv
 *   q [B, hq, d] of q_dtype; kpacked [B, hkv, t_max, kb*ceil(d/8)], knorms
 *   [B, hkv, t_max] fp32; vpacked/vnorms likewise with vb; seq_lens [B] int32 on
 *   the device (tokens 0..seq_lens[b]-1 are attended); out [B, hq, d] of q_dtype.
 *   lse: optional fp32 [B, hq] (NULL to skip) receiving max_t s_t + log(sum_t exp(s_t - max)),
 *   -inf for an empty sequence, so callers can merge further tokens by log-sum-exp.
 *   d <= 256; kb, vb in 1..4.  Needs tq_decode_workspace_bytes(...).
 */
size_t tq_decode_workspace_bytes(int32_t B, int32_t hq, int32_t d, int64_t t_max);
int tq_decode_attention_packed(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq,
                               int32_t hkv, int32_t d, const uint8_t* kpacked,
                               const float* knorms, const uint8_t* vpacked, const float* vnorms,
                               int64_t t_max, const int32_t* seq_lens, const float* kcentroids,
                               const float* vcentroids, const float* krotation,
                               const float* vrotation, int32_t kbits, int32_t vbits, float scale,
                               void* out, float* lse, void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * Decode layout: the codes of a packed KV cache with 4-bit keys and 2-, 3- or 4-bit
 * values arranged for the decode kernel, same bytes per token as the bit-plane rows.
 * The reference stores its cache privately (cache.py:81-130), so this arrangement is
 * internal to QuantizedKVCache; these entry points convert it from and to the reference
 * rows.
 *   keys    [streams][t_cap][d/2]:   byte p = (code[2p] << 4) | code[2p+1]
 *   values  [streams][t_cap/64][512*vb] (d = 64): tile T holds tokens 64T..64T+63.  Lane
 *           L = 16*sl + c of a wave owns words 0-3 at tile byte 16*L and words 4.. at
 *           1024 + (8*vb - 16)*L; token t of block 4m + sl (t, m, sl < 4), dim 16dg + c:
 *     vb 2  word m, byte dg, bits 2t
 *     vb 4  word 4*(m/2) + dg, byte 2*(m%2) + t/2, bits 4*(t%2)
 *     vb 3  dg < 3: word 3*(m/2) + dg, the same byte, bits 3*(t%2); dg 3: the byte's
 *           6-bit pair index (code[t even] | code[t odd] << 3) split two bits at a time
 *           into bits 6-7 of that byte of words 3*(m/2) + 0, 1, 2
 *           so each byte is one table index and a lane reads its operand bytes of a tile
 *           with one or two loads (t_cap a multiple of 64)
 * tq_pack_decode_layout writes tokens [pos, pos+n) of every stream from bit-plane rows
 * packed [streams][n][bits*ceil(d/8)] (values: bits of the chunk's other tokens are
 * kept); tq_unpack_decode_layout returns tokens [t0, t0+n) as bit-plane rows.
 * values = 0 for keys (bit_width 4), 1 for values (bit_width 2-4).
 */
int tq_pack_decode_layout(const uint8_t* packed, int64_t n_streams, int64_t n, int32_t d,
                          int32_t bit_width, int32_t values, uint8_t* cache, int64_t t_cap,
                          int64_t pos, void* stream);
int tq_unpack_decode_layout(const uint8_t* cache, int64_t n_streams, int64_t t_cap, int64_t t0,
                            int64_t n, int32_t d, int32_t bit_width, int32_t values,
                            uint8_t* packed, void* stream);

/*
 * One decode step's cache append in one launch: token `pos` of every stream (key and
 * value [n_streams][d], bf16 or fp16, d = 64 or 128) quantized (4-bit keys, vbits-bit
 * values; the codebook boundaries and rotations of tq_rotate_and_quantize) and written
 * into the decode layout above: kpairs [n_streams][t_cap][d/2], vtiles
 * [n_streams][t_cap/64][512*vbits*(d/64)] (only this token's bits change), and the norms
 * knorms / vnorms [n_streams][t_cap] in norm_dtype (TQ_F32, TQ_BF16 or TQ_F16).  Codes
 * and norms equal tq_rotate_and_quantize (rounding in the input type) followed by
 * tq_pack_decode_layout, bit for bit.
 * Replaces: the quantize-and-store of one new token in TurboQuantCache.update
 * (hf_integration.py:319-345 with cache.py:148-210's quantize_mse of keys and values).
 */
int tq_cache_append_dl(const void* key, const void* value, tq_dtype in_dtype, int64_t n_streams,
                       int32_t d, const float* krotation, const float* kboundaries,
                       const float* vrotation, const float* vboundaries, int32_t vbits,
                       uint8_t* kpairs, void* knorms, uint8_t* vtiles, void* vnorms,
                       tq_dtype norm_dtype, int64_t t_cap, int64_t pos, void* stream);

/*
 * tq_decode_attention_packed over a decode-layout cache (same semantics and output):
 * head_dim 64, 4-bit keys, 2-4 bit values (vbits), any number of query heads per KV head
 * (launched four at a time), t_cap a multiple of 64.  kpairs [B, hkv, t_cap, 32],
 * vblocks [B, hkv, t_cap/64, 512*vbits], norms as above.
 * Scores are accurate to about 1e-6 relative (fp16 hi/lo products, fp32 accumulation);
 * fp32 queries get fp32-accurate outputs; fp16/bf16 queries use fp16 value products
 * (relative error about 5e-4, below the output type's own rounding tolerance).
 */
size_t tq_decode_dl_workspace_bytes(int32_t B, int32_t hq, int32_t hkv, int64_t t_cap);
/* kbits must be 4 and vbits 2, 3 or 4 (TQ_EUNSUPPORTED otherwise). */
int tq_decode_attention_dl(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                           int32_t d, const uint8_t* kpairs, const float* knorms,
                           const uint8_t* vblocks, const float* vnorms, int64_t t_cap,
                           const int32_t* seq_lens, const float* kcentroids,
                           const float* vcentroids, const float* krotation,
                           const float* vrotation, int32_t kbits, int32_t vbits, float scale,
                           void* out, float* lse, void* workspace, size_t workspace_bytes,
                           void* stream);
/*
 * tq_decode_attention_dl over a window [seq_starts[b], seq_lens[b]) of each sequence: tokens
 * before seq_starts[b] are masked (a left-padded batch, whose 2-D attention mask hides the
 * first seq_starts[b] positions).  seq_starts may be null (every window starts at 0).
 * knorms / vnorms hold norm_dtype values: TQ_F32, or TQ_BF16 / TQ_F16 for a 16-bit model's
 * cache, which keeps its norms in the model's dtype as the reference's HF cache does
 * (turboquant_kv/hf_integration.py:512-525 counts them so).
 * Replaces: the masked decode step of turboquant_kv/hf_integration.py:319-421 (dequantized
 * history + SDPA with the attention mask).
 */
int tq_decode_attention_dl_window(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq,
                                  int32_t hkv, int32_t d, const uint8_t* kpairs,
                                  const void* knorms, const uint8_t* vblocks,
                                  const void* vnorms, tq_dtype norm_dtype, int64_t t_cap,
                                  const int32_t* seq_lens,
                                  const int32_t* seq_starts, const float* kcentroids,
                                  const float* vcentroids, const float* krotation,
                                  const float* vrotation, int32_t kbits, int32_t vbits,
                                  float scale, void* out, float* lse, void* workspace,
                                  size_t workspace_bytes, void* stream);

/*
 * The exact current token merged into a decode output (o, lse from
 * tq_decode_attention_dl / tq_decode_attention_packed with the lse output) by
 * log-sum-exp: replaces the HF cache's eager composition of that merge
 * (turboquant_kv/hf_integration.py:372-390, which attends the token being decoded to its
 * own unquantized key and value).  o, q, out [B, hq, d] in q_dtype; lse [B, hq] fp32 (natural
 * log); k_new, v_new [B, hkv, d] in kv_dtype.  s = (q . k_new) * scale, m = max(lse, s),
 * out = (o e^(lse - m) + v_new e^(s - m)) / (e^(lse - m) + e^(s - m)) in fp32.  out may be o.
 */
int tq_decode_merge_token(const void* o, const float* lse, const void* q, tq_dtype q_dtype,
                          const void* k_new, const void* v_new, tq_dtype kv_dtype, int32_t B,
                          int32_t hq, int32_t hkv, int32_t d, float scale, void* out, void* stream);

/*
 * Paged KV storage (vLLM block tables).  The reference's vLLM backend keeps one
 * contiguous QuantizedKVCache per model with no block tables
 * (turboquant_kv/vllm_plugin/__init__.py:114-304, 350-412); these entry points give its
 * TurboQuantAttentionImpl what vLLM's cache engine hands an attention backend.
 * A layer's pools hold packed rows and fp32 norms block by block:
 *   pool [num_blocks][hkv][block_size][P] u8, norm_pool [num_blocks][hkv][block_size];
 * token t of sequence s sits in block block_tables[s * bt_stride + t / block_size] at slot
 * t % block_size, and a new token's flat slot is block * block_size + slot (vLLM's
 * slot_mapping).
 *
 * tq_paged_store: rows [n_tokens][hkv][row_bytes] (+ norms [n_tokens][hkv], or both NULL)
 * to the slots slot_mapping[n_tokens] (int64); slots < 0 or >= num_blocks * block_size
 * are skipped (vLLM pads with -1).  Replaces the append of vllm_plugin:395 for a batch
 * of sequences.
 */
int tq_paged_store(const uint8_t* rows, const float* norms, int64_t n_tokens, int32_t hkv,
                   int32_t row_bytes, const int64_t* slot_mapping, uint8_t* pool, float* norm_pool,
                   int64_t num_blocks, int32_t block_size, void* stream);
/*
 * tq_paged_gather: the first min(seq_lens[b], t_max) tokens of batch rows b < B into
 * contiguous out_rows [B][hkv][t_max][row_bytes] (+ out_norms [B][hkv][t_max]); later
 * tokens, and tokens whose block id is outside [0, num_blocks), come out as zero rows.
 * t_max <= bt_stride * block_size.
 */
int tq_paged_gather(const uint8_t* pool, const float* norm_pool, int64_t num_blocks, int32_t hkv,
                    int32_t block_size, int32_t row_bytes, const int32_t* block_tables,
                    int32_t bt_stride, const int32_t* seq_lens, int32_t B, int64_t t_max,
                    uint8_t* out_rows, float* out_norms, void* stream);
/*
 * tq_decode_attention_packed over paged pools (same semantics and outputs): batch row b
 * attends to its first seq_lens[b] tokens, found through block_tables [B][bt_stride]
 * (bt_stride = max_blocks_per_seq).  Head_dim 64, K 1-4 / V 1-2 bits, at most 4 query
 * heads per KV head, fp16/bf16 queries and a power-of-two block_size >= 4 run the fused
 * decode kernel reading the pools directly; other shapes gather the rows into the
 * workspace first.  Pools 16-byte aligned; num_blocks * hkv * block_size < 2^32 rows (pools
 * from 2 GiB on are read with 64-bit addresses, and a block id outside the pool reads the
 * pool's last block instead of memory outside it).
 */
size_t tq_decode_paged_workspace_bytes(tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                                       int32_t d, int32_t kbits, int32_t vbits,
                                       int32_t max_blocks_per_seq, int32_t block_size);
int tq_decode_attention_paged(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                              int32_t d, const uint8_t* kpool, const float* knorm_pool,
                              const uint8_t* vpool, const float* vnorm_pool, int64_t num_blocks,
                              int32_t block_size, const int32_t* block_tables,
                              int32_t max_blocks_per_seq, const int32_t* seq_lens,
                              const float* kcentroids, const float* vcentroids,
                              const float* krotation, const float* vrotation, int32_t kbits,
                              int32_t vbits, float scale, void* out, float* lse, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Paged pools in the decode layout (4-bit keys, vbits = 2-4 bit values, head_dim 64, any
 * number of query heads per KV head): the same kernel as tq_decode_attention_dl with block
 * lookups per 64-token tile (one for block sizes >= 64, one per 16-token group below), for
 * power-of-two block sizes >= 16.  Replaces, like tq_decode_attention_paged, the reference
 * backend's forward (turboquant_kv/vllm_plugin/__init__.py:209-304).
 *   kpairs_pool [num_blocks][hkv][block_size][32]   key pair bytes (tq_pack_decode_layout,
 *                                                   values = 0) stored with tq_paged_store
 *   vtile_pool  block_size >= 64: [num_blocks][hkv][block_size/64][512 * vbits] value
 *               tiles (the byte layout of tq_pack_decode_layout's value tiles);
 *               block_size 16, 32: [num_blocks][hkv][block_size/16][128 * vbits] sub-blocks,
 *               each holding what its 16-token group m of a 64-token tile contributes.
 *               With tt the token's offset in its sub-block, sl = tt/4, r = tt%4, dim
 *               16*dg + c, L = 16*sl + c:
 *                 vbits 2  byte 4L + dg, bits 2r (tile byte 16L + 4m + dg)
 *                 vbits 4  byte 8L + 2dg + r/2, bits 4(r%2) (the two bytes that group m
 *                          fills of tile word 4(m/2) + dg)
 *                 vbits 3  dims below 48: byte 4L + 2dg + r/2 (dg 0, 1) or 256 + 2L + r/2
 *                          (dg 2), bits 3(r%2); dims 48-63: code bit b is bit
 *                          q = 3(r%2) + b of the pair index, stored at bit 6 + q%2 of the
 *                          byte of share q/2 (the tile layout's spread of dim group 3)
 *   knorm_pool, vnorm_pool [num_blocks][hkv][block_size]
 * tq_paged_store_value_tiles writes new tokens' vbits-bit value rows
 * [n_tokens][hkv][8 * vbits] (bit planes) and norms [n_tokens][hkv] into their slots
 * (slot_mapping as in tq_paged_store; negative or out-of-pool slots skipped), leaving the
 * other tokens of each tile as they are.  Workspace: tq_decode_dl_workspace_bytes(B, hq,
 * hkv, max_blocks_per_seq * block_size).  Pools 16-byte aligned; num_blocks * hkv *
 * block_size < 2^32 rows (pools from 2 GiB on are read with 64-bit addresses; a block id
 * outside the pool reads the pool's last block).  Outputs as tq_decode_attention_dl's.
 */
int tq_paged_store_value_tiles(const uint8_t* rows, const float* norms, int64_t n_tokens,
                               int32_t hkv, const int64_t* slot_mapping, uint8_t* vtile_pool,
                               float* vnorm_pool, int64_t num_blocks, int32_t block_size,
                               int32_t vbits, void* stream);
int tq_decode_attention_paged_dl(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                                 int32_t d, const uint8_t* kpairs_pool, const float* knorm_pool,
                                 const uint8_t* vtile_pool, const float* vnorm_pool,
                                 int64_t num_blocks, int32_t block_size, int32_t vbits,
                                 const int32_t* block_tables, int32_t max_blocks_per_seq,
                                 const int32_t* seq_lens, const float* kcentroids,
                                 const float* vcentroids, const float* krotation,
                                 const float* vrotation, float scale, void* out, float* lse,
                                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Causal prefill of one sequence over decode-layout paged pools (the pools of
 * tq_decode_attention_paged_dl): its n new tokens q [n][hq][64] sit at positions
 * T - n .. T - 1 and new token i attends to tokens 0 .. T - n + i, read through
 * block_table [max_blocks] (T <= max_blocks * block_size).  out [n][hq][64] fp32,
 * 16-byte aligned.  Replaces the reference backend's prefill attention over its
 * dequantized cache (vllm_plugin/__init__.py:400 via cache.py:282-339), which has no
 * block tables and no causal mask; one kernel streams each 64-token tile once per 48
 * query rows (32 for fp32 / fp16 queries) instead of once per row.  Pools of any size (64-bit addresses; block ids
 * clamped into the pool).  No workspace.
 */
int tq_prefill_attention_paged_dl(const void* q, tq_dtype q_dtype, int32_t n, int64_t T, int32_t hq,
                                  int32_t hkv, int32_t d, const uint8_t* kpairs_pool,
                                  const float* knorm_pool, const uint8_t* vtile_pool,
                                  const float* vnorm_pool, int64_t num_blocks, int32_t block_size,
                                  int32_t vbits, const int32_t* block_table, int32_t max_blocks,
                                  const float* kcentroids, const float* vcentroids,
                                  const float* krotation, const float* vrotation, float scale,
                                  float* out, void* stream);

/*
 * Host-side tables of the reference's standalone C++ core, for TQIX v1 index files
 * (turboquant_core.cpp:559-618), which record only (dim, bit_width, seed): the reader
 * rebuilds the rotation and codebook the writer used.  No device work; outputs are host
 * memory.  Same matrices and codebooks as the core's, bit for bit.
 *   tq_core_rotation  replaces turboquant::make_rotation_matrix (turboquant_core.cpp:137-213):
 *                     out [dim][dim] fp32 row-major (orthonormal columns; scores use
 *                     q_rot[j] = sum_k q[k] * out[j][k], as search_packed does).
 *   tq_core_codebook  replaces turboquant::Codebook(bits, dim) (turboquant_core.cpp:71-132):
 *                     scaled boundaries [2^bits - 1] and centroids [2^bits] fp32.
 */
int tq_core_rotation(int32_t dim, int32_t seed, float* out);
int tq_core_codebook(int32_t bits, int32_t dim, float* boundaries, float* centroids);

/*
 * Huffman streams of code indices (host memory; the byte format of HuffmanCoder.encode /
 * decode, turboquant_kv/entropy.py:162-231): uint32 LE symbol count, uint32 LE bit count,
 * then the code words most significant bit first, zero-padded to a byte.  The caller
 * supplies the code table (code_words[s] holds code_lens[s] bits, right-aligned).
 * tq_huffman_encode writes 8 + ceil(bits/8) bytes (*out_bytes; TQ_EINVAL when
 * out_capacity is smaller).  tq_huffman_decode matches prefixes against the table
 * (code c -> symbols[c]; a later duplicate entry wins), decodes at most n_symbols (< 0:
 * the header's count) and sets *n_out to the number decoded.
 */
int tq_huffman_encode(const uint8_t* codes, int64_t n, const uint64_t* code_words,
                      const uint8_t* code_lens, int32_t n_levels, uint8_t* out, size_t out_capacity,
                      size_t* out_bytes);
int tq_huffman_decode(const uint8_t* data, size_t data_bytes, int64_t n_symbols,
                      const uint64_t* code_words, const uint8_t* code_lens, const int32_t* symbols,
                      int32_t n_codes, uint8_t* out, int64_t* n_out);

#ifdef __cplusplus
}
#endif

#endif /* TURBOQUANT_HIP_H */
