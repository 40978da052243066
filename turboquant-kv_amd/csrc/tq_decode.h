// tq_decode.h -- fused single-kernel decode attention (tq_decode.hip), dispatched from
// tq_decode_attention_packed when the shape is one it covers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tq {

struct FusedDecodeCall {
  const void* q;
  int q_dt;
  int B, hq, hkv, d;
  const uint8_t* kpacked;
  const float* knorms;
  const uint8_t* vpacked;
  const float* vnorms;
  int64_t t_max;
  const int32_t* seq_lens;
  const float* kcen;
  const float* vcen;
  const float* krot;
  const float* vrot;
  int kbits, vbits;
  float scale;
  void* out;
  float* lse;
};

// Block pools of a paged cache (vLLM layout): rows [num_blocks][hkv][block_size][P],
// norms [num_blocks][hkv][block_size]; FusedDecodeCall's kpacked/knorms/vpacked/vnorms
// point at the pools and t_max = bt_stride * block_size.
struct PagedPools {
  const int32_t* block_tables;  // [B][bt_stride]
  int bt_stride;
  int bs_log2;
  uint32_t pool_rows;           // num_blocks * hkv * block_size
  uint32_t num_blocks;
  bool wide;                    // rows past 2 GiB: 64-bit addresses
};

// True when the fused kernel covers this call (head_dim 64, K 1-4 bits, V 1-2 bits,
// at most 4 query heads per KV head, fp16/bf16 queries and outputs, 16-byte aligned
// packed rows).
bool fused_decode_covers(const FusedDecodeCall& c);
// Workspace the fused path needs (split partials and split statistics).
size_t fused_decode_workspace_bytes(int B, int hq, int d, int64_t t_max);
// Launches the fused kernel and its split combine on `st`; returns a TQ_* code.
int launch_fused_decode(const FusedDecodeCall& c, void* workspace, size_t workspace_bytes,
                        hipStream_t st, const PagedPools* paged = nullptr);

}  // namespace tq
