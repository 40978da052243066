// tq_paged.hip -- paged (vLLM block-table) KV storage for packed codes on gfx950.
//
// Pools hold a layer's packed rows block by block, as vLLM's cache engine lays out its
// blocks: rows [num_blocks][hkv][block_size][P] and fp32 norms [num_blocks][hkv][block_size].
// Token t of a sequence lives in block block_tables[seq][t / block_size], slot
// t % block_size; a new token's flat slot (slot_mapping) is block * block_size + slot.
//
//   paged_store_kernel   scatters freshly quantized rows (and their norms) to their slots
//   paged_gather_kernel  copies sequences' rows out of the pools into contiguous
//                        [B][hkv][t_max][P] buffers (prefill, and decode shapes the fused
//                        kernel does not cover)
//   decode               the fused decode kernel of tq_decode.hip reading the pools
//                        through the block tables (tq_decode_attention_paged)
//
// The reference's vLLM backend keeps one contiguous QuantizedKVCache and has no block
// tables (turboquant_kv/vllm_plugin/__init__.py:114-304, 350-412); the pool layout and
// slot convention here are vLLM's own.

#include "tq_common.h"
#include "tq_decode.h"

#include <climits>

namespace tq {
namespace {

constexpr int kPgThreads = 256;

// One thread per (token, head, byte) of the new rows; the head's norm goes with byte 0.
// Slots outside [0, num_blocks * block_size) are skipped (vLLM pads with -1).
__global__ __launch_bounds__(kPgThreads) void paged_store_kernel(
    const uint8_t* __restrict__ rows, const float* __restrict__ norms, int64_t n_tokens, int hkv,
    int row_bytes, const int64_t* __restrict__ slot_mapping, uint8_t* __restrict__ pool,
    float* __restrict__ norm_pool, int64_t num_slots, int block_size) {
  const int64_t total = n_tokens * hkv * row_bytes;
  for (int64_t e = (int64_t)blockIdx.x * kPgThreads + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kPgThreads) {
    const int64_t th = e / row_bytes;
    const int byte = (int)(e - th * row_bytes);
    const int64_t tok = th / hkv;
    const int h = (int)(th - tok * hkv);
    const int64_t slot = slot_mapping[tok];
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t blk = slot / block_size, off = slot - blk * block_size;
    const int64_t dst = (blk * hkv + h) * block_size + off;
    pool[dst * row_bytes + byte] = rows[e];
    if (byte == 0 && norms) norm_pool[dst] = norms[th];
  }
}

// One thread per (batch row, head, token, byte) of the output; tokens at or past the
// batch row's length are written as zero rows with zero norms.
__global__ __launch_bounds__(kPgThreads) void paged_gather_kernel(
    const uint8_t* __restrict__ pool, const float* __restrict__ norm_pool, int64_t num_blocks,
    int hkv, int block_size, int row_bytes, const int32_t* __restrict__ block_tables,
    int bt_stride, const int32_t* __restrict__ seq_lens, int B, int64_t t_max,
    uint8_t* __restrict__ out_rows, float* __restrict__ out_norms) {
  const int64_t total = (int64_t)B * hkv * t_max * row_bytes;
  for (int64_t e = (int64_t)blockIdx.x * kPgThreads + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kPgThreads) {
    const int64_t r = e / row_bytes;  // (b, h, t) row of the output
    const int byte = (int)(e - r * row_bytes);
    const int64_t bh = r / t_max;
    const int64_t t = r - bh * t_max;
    const int b = (int)(bh / hkv), h = (int)(bh - (int64_t)b * hkv);
    const int64_t len = seq_lens[b] < t_max ? seq_lens[b] : t_max;
    uint8_t v = 0;
    float n = 0.f;
    bool have = false;
    int64_t src = 0;
    if (t < len) {
      const int64_t blk = block_tables[(int64_t)b * bt_stride + t / block_size];
      if (blk >= 0 && blk < num_blocks) {
        src = (blk * hkv + h) * block_size + (t % block_size);
        have = true;
      }
    }
    if (have) v = pool[src * row_bytes + byte];
    out_rows[e] = v;
    if (byte == 0 && out_norms) {
      if (have) n = norm_pool[src];
      out_norms[r] = n;
    }
  }
}

int grid_for(int64_t total) {
  const int64_t cap = (int64_t)device_cu_count() * 16;
  const int64_t b = (total + kPgThreads - 1) / kPgThreads;
  return (int)(b < 1 ? 1 : (b < cap ? b : cap));
}

int log2_exact(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return (1 << l) == v ? l : -1;
}

size_t gather_bytes(int B, int hkv, int64_t t_max, int pk, int pv) {
  const size_t rows = (size_t)B * hkv * (size_t)t_max;
  return align_up(rows * pk, 256) + align_up(rows * 4, 256) + align_up(rows * pv, 256) +
         align_up(rows * 4, 256);
}

bool paged_fused_shape(tq_dtype q_dtype, int hq, int hkv, int d, int kbits, int vbits) {
  FusedDecodeCall c{};
  c.q_dt = (int)q_dtype; c.B = 1; c.hq = hq; c.hkv = hkv; c.d = d; c.kbits = kbits;
  c.vbits = vbits; c.t_max = 64;
  static const float aligned_dummy[4] __attribute__((aligned(16))) = {0.f, 0.f, 0.f, 0.f};
  c.krot = aligned_dummy;
  return fused_decode_covers(c);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int tq_paged_store(const uint8_t* rows, const float* norms, int64_t n_tokens, int32_t hkv,
                   int32_t row_bytes, const int64_t* slot_mapping, uint8_t* pool, float* norm_pool,
                   int64_t num_blocks, int32_t block_size, void* stream) {
  TQ_REQUIRE(n_tokens >= 0 && hkv >= 1 && row_bytes >= 1 && num_blocks >= 0 && block_size >= 1,
             "bad sizes");
  if (n_tokens == 0) return TQ_OK;
  TQ_REQUIRE(rows && slot_mapping && pool, "null pointer argument");
  TQ_REQUIRE(!norms == !norm_pool, "norms and norm_pool go together");
  const int64_t total = n_tokens * hkv * row_bytes;
  hipLaunchKernelGGL(paged_store_kernel, dim3(grid_for(total)), dim3(kPgThreads), 0,
                     as_stream(stream), rows, norms, n_tokens, (int)hkv, (int)row_bytes,
                     slot_mapping, pool, norm_pool, num_blocks * block_size, (int)block_size);
  TQ_LAUNCH_CHECK("paged_store_kernel");
  return TQ_OK;
}

int tq_paged_gather(const uint8_t* pool, const float* norm_pool, int64_t num_blocks, int32_t hkv,
                    int32_t block_size, int32_t row_bytes, const int32_t* block_tables,
                    int32_t bt_stride, const int32_t* seq_lens, int32_t B, int64_t t_max,
                    uint8_t* out_rows, float* out_norms, void* stream) {
  TQ_REQUIRE(B >= 0 && hkv >= 1 && row_bytes >= 1 && block_size >= 1 && num_blocks >= 0 &&
                 t_max >= 0 && bt_stride >= 0,
             "bad sizes");
  TQ_REQUIRE(t_max <= (int64_t)bt_stride * block_size,
             "t_max (%lld) exceeds the block table's reach (%d blocks of %d)", (long long)t_max,
             bt_stride, block_size);
  if (B == 0 || t_max == 0) return TQ_OK;
  TQ_REQUIRE(pool && block_tables && seq_lens && out_rows, "null pointer argument");
  TQ_REQUIRE(!norm_pool == !out_norms, "norm_pool and out_norms go together");
  const int64_t total = (int64_t)B * hkv * t_max * row_bytes;
  hipLaunchKernelGGL(paged_gather_kernel, dim3(grid_for(total)), dim3(kPgThreads), 0,
                     as_stream(stream), pool, norm_pool, num_blocks, (int)hkv, (int)block_size,
                     (int)row_bytes, block_tables, (int)bt_stride, seq_lens, (int)B, t_max, out_rows,
                     out_norms);
  TQ_LAUNCH_CHECK("paged_gather_kernel");
  return TQ_OK;
}

size_t tq_decode_paged_workspace_bytes(tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                                       int32_t d, int32_t kbits, int32_t vbits,
                                       int32_t max_blocks_per_seq, int32_t block_size) {
  if (B <= 0 || hq <= 0 || hkv <= 0 || d <= 0 || max_blocks_per_seq <= 0 || block_size <= 0)
    return 256;
  const int64_t t_max = (int64_t)max_blocks_per_seq * block_size;
  if (paged_fused_shape(q_dtype, hq, hkv, d, kbits, vbits) && log2_exact(block_size) >= 2)
    return fused_decode_workspace_bytes(B, hq, d, t_max);
  const int bpp = (d + 7) / 8;
  return 256 + gather_bytes(B, hkv, t_max, kbits * bpp, vbits * bpp) +
         tq_decode_workspace_bytes(B, hq, d, t_max);
}

int tq_decode_attention_paged(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                              int32_t d, const uint8_t* kpool, const float* knorm_pool,
                              const uint8_t* vpool, const float* vnorm_pool, int64_t num_blocks,
                              int32_t block_size, const int32_t* block_tables,
                              int32_t max_blocks_per_seq, const int32_t* seq_lens,
                              const float* kcentroids, const float* vcentroids,
                              const float* krotation, const float* vrotation, int32_t kbits,
                              int32_t vbits, float scale, void* out, float* lse, void* workspace,
                              size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(kbits >= 1 && kbits <= 4 && vbits >= 1 && vbits <= 4, "bits must be 1-4");
  TQ_REQUIRE(d >= 1 && d <= 256, "head_dim must be in [1, 256], got %d", d);
  TQ_REQUIRE(B >= 0 && hq >= 1 && hkv >= 1 && hq % hkv == 0,
             "num_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  TQ_REQUIRE(block_size >= 1 && max_blocks_per_seq >= 0 && num_blocks >= 0, "bad sizes");
  TQ_REQUIRE(valid_dtype(q_dtype), "unknown dtype");
  if (B == 0) return TQ_OK;
  TQ_REQUIRE(q && out && seq_lens && kcentroids && vcentroids && krotation && vrotation,
             "null pointer argument");
  const int64_t t_max = (int64_t)max_blocks_per_seq * block_size;
  TQ_REQUIRE(t_max == 0 || (kpool && knorm_pool && vpool && vnorm_pool && block_tables),
             "null pointer argument");
  const int bpp = (d + 7) / 8;
  const int pk = kbits * bpp, pv = vbits * bpp;
  const int64_t pool_rows = num_blocks * hkv * block_size;
  TQ_REQUIRE(pool_rows < ((int64_t)1 << 32), "pools hold at most 2^32 rows per layer");
  // pools from 2 GiB of rows on: 64-bit addresses (the buffer path's offsets are 32-bit)
  const bool wide = pool_rows * (pk > pv ? pk : pv) >= (int64_t)INT_MAX;
  TQ_REQUIRE(((reinterpret_cast<uintptr_t>(kpool) | reinterpret_cast<uintptr_t>(vpool) |
               reinterpret_cast<uintptr_t>(knorm_pool) | reinterpret_cast<uintptr_t>(vnorm_pool)) &
              15u) == 0,
             "pools must be 16-byte aligned");
  const size_t need = tq_decode_paged_workspace_bytes(q_dtype, B, hq, hkv, d, kbits, vbits,
                                                      max_blocks_per_seq, block_size);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  hipStream_t st = as_stream(stream);
  const int bsl = log2_exact(block_size);
  FusedDecodeCall fc{q, (int)q_dtype, B, hq, hkv, d, kpool, knorm_pool, vpool, vnorm_pool,
                     t_max, seq_lens, kcentroids, vcentroids, krotation, vrotation,
                     kbits, vbits, scale, out, lse};
  if (t_max > 0 && bsl >= 2 && fused_decode_covers(fc)) {
    const PagedPools pg{block_tables, max_blocks_per_seq, bsl, (uint32_t)pool_rows,
                        (uint32_t)std::max<int64_t>(num_blocks, 1), wide};
    return launch_fused_decode(fc, workspace, workspace_bytes, st, &pg);
  }
  // Other shapes: gather the batch's rows into contiguous buffers and run the general
  // decode path over them.
  char* ws = static_cast<char*>(workspace) + 256;
  const size_t rows = (size_t)B * hkv * (size_t)t_max;
  uint8_t* kr = reinterpret_cast<uint8_t*>(ws);
  ws += align_up(rows * pk, 256);
  float* kn = reinterpret_cast<float*>(ws);
  ws += align_up(rows * 4, 256);
  uint8_t* vr = reinterpret_cast<uint8_t*>(ws);
  ws += align_up(rows * pv, 256);
  float* vn = reinterpret_cast<float*>(ws);
  ws += align_up(rows * 4, 256);
  if (t_max > 0) {
    int rc = tq_paged_gather(kpool, knorm_pool, num_blocks, hkv, block_size, pk, block_tables,
                             max_blocks_per_seq, seq_lens, B, t_max, kr, kn, stream);
    if (rc) return rc;
    rc = tq_paged_gather(vpool, vnorm_pool, num_blocks, hkv, block_size, pv, block_tables,
                         max_blocks_per_seq, seq_lens, B, t_max, vr, vn, stream);
    if (rc) return rc;
  }
  const size_t used = (size_t)(ws - static_cast<char*>(workspace));
  return tq_decode_attention_packed(q, q_dtype, B, hq, hkv, d, kr, kn, vr, vn, t_max, seq_lens,
                                    kcentroids, vcentroids, krotation, vrotation, kbits, vbits,
                                    scale, out, lse, ws, workspace_bytes - used, stream);
}

}  // extern "C"
