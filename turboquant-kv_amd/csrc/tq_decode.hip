// tq_decode.hip -- fused GQA decode attention over a packed KV cache on gfx950.
//
// Semantics: those of tq_decode_attention_packed (QuantizedKVCache.attention_scores ->
// softmax -> attention_values, turboquant_kv/cache.py:282-339, vllm_plugin/__init__.py:400,
// with query head h reading KV head h / (hq / hkv)).
//
// fused_decode_kernel: one workgroup per (batch, kv head, token split); its four waves take
// 64-token tiles in turn and each keeps its own online softmax.  Per tile and wave:
//   q.K    lane l holds token l's packed K row.  The two dims x and x+4 of an octet sit at
//          bits 7-x and 3-x of every plane byte, so one shift, one mask and one v_dot4 over
//          the octet's four plane bytes give 128 * (16 * code_x + code_x+4), the LDS address
//          of a pair table entry (c[code_x], c[code_x+4]) in fp32.  Those values are the A
//          operand (row = token) of v_mfma_f32_4x4x1f32 against B = (R_k q)[dim] of the
//          lane's head: 64 MFMAs leave, in lane (quad, head), that head's scores of the
//          quad's four tokens -- fp32 products, fp32 sums.
//   softmax  log2 domain, exact running maximum per head; a new maximum rescales the
//          accumulators (a handful of times per split).  w = 2^(s - max) * |v_t|.
//   p.V    each lane quad byte-transposes its four V rows (two DPP moves and two v_perm
//          per word), so lane (quad, j) holds the quad's plane bytes of octets j and 4+j.
//          One dim's 2-bit codes of the four tokens form an 8-bit index into a table of
//          four fp16 centroids: the B operand of v_mfma_f32_4x4x4f16 whose A operand is the
//          quad's four weights of one head in fp16 -- the layout q.K left them in.  Each
//          quad accumulates its own partial sums (16 MFMAs per tile cover 64 dims).
// Both tables keep 16 bank-skewed copies (entry stride 128 B, copy = lane % 16): a wave's
// random lookups are then conflict-free.
// fused_combine_kernel: merges the splits by log-sum-exp and applies R_v.
//
// Accuracy: scores are exact fp32 (centroids and rotated query in fp32); the weights and V
// centroids enter the V product in fp16 (relative error of the output about 5e-4), so this
// path serves fp16/bf16 outputs.

#include "tq_common.h"
#include "tq_decode.h"

#include <algorithm>
#include <type_traits>
#include <climits>
#include <cstdlib>

namespace tq {
namespace {

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDim = 64;
constexpr int kTabBytes = 256 * 128;  // 256 indices x 16 copies x 8 bytes
constexpr int kMinSplit = 256;        // tokens; one tile per wave

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct DecodeArgs {
  const void* q;
  int q_dt;
  int hq, hkv, G;
  const uint8_t* kpacked;
  const float* knorms;
  const uint8_t* vpacked;
  const float* vnorms;
  int64_t t_max;
  const int32_t* seq_lens;
  const float* kcen;
  const float* vcen;
  const float* krot;
  float qscale;          // softmax scale * log2(e)
  int64_t split_tokens;  // multiple of kMinSplit
  int nsplit;
  float* part;           // [B*hq][nsplit][64]: sum_t 2^(s_t - max) |v_t| c[code_t]
  float2* stats;         // [B*hq][nsplit]: (max, sum_t 2^(s_t - max)), log2 domain
  // Paged caches (PAGED kernels): K/V rows and norms live in block pools
  // [num_blocks][hkv][block_size][row] and token t of batch row b sits in block
  // block_tables[b * bt_stride + t / block_size], slot t % block_size.
  const int32_t* block_tables;
  int bt_stride;
  int bs_log2;           // log2(block_size), block_size >= 4
  uint32_t pool_rows;    // num_blocks * hkv * block_size
  uint32_t num_blocks;   // wide pools (PG 2): block ids are clamped below it
};

// Raw buffer resource over `bytes` bytes at `p` (gfx9 dword 3); loads past the end
// return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return buf_rsrc(p, bytes);
}

// NB bytes of a packed row (8, 16, 24 or 32) at byte offset `off` as 32-bit words.
template <int NB>
__device__ __forceinline__ void load_row(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                         uint32_t (&w)[NB / 4]) {
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 16 * i, 0);
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 8 * i, 0);
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    }
  }
}

// The same from a global address (row bytes 16-byte aligned when NB is a multiple of 16,
// else 8-byte aligned).
template <int NB>
__device__ __forceinline__ void load_row_at(const uint8_t* p, uint32_t (&w)[NB / 4]) {
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) {
      const u32x2 v = reinterpret_cast<const u32x2*>(p)[i];
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    }
  }
}

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// 4x4 byte transpose inside each lane quad: lane j of a quad returns
// [x3.byte j, x2.byte j, x1.byte j, x0.byte j], x_t being lane t's input.
__device__ __forceinline__ uint32_t quad_transpose(uint32_t x, uint32_t sel1, uint32_t sel2) {
  const uint32_t xp = (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false);  // lane^2
  const uint32_t y = perm(xp, x, sel1);
  const uint32_t yp = (uint32_t)__builtin_amdgcn_mov_dpp((int)y, 0xB1, 0xF, 0xF, false);  // lane^1
  return perm(yp, y, sel2);
}

// PG: 0 contiguous; 1 paged pools read through buffer resources over whole pools (32-bit
// offsets: pools under 2 GiB); 2 paged pools of any size: rows at 64-bit addresses from
// clamped block ids.
template <int KB, int VB, int PG = 0>
__global__ __launch_bounds__(kDecThreads, 2) void fused_decode_kernel(DecodeArgs a) {
  constexpr bool PAGED = PG != 0, WIDE = PG == 2;
  constexpr int PK = KB * 8, PV = VB * 8;  // packed row bytes (d = 64)
  // Tables first; after the tile loop the same bytes hold the cross-quad reduction.
  __shared__ __attribute__((aligned(16))) char tabs[2 * kTabBytes];
  __shared__ __attribute__((aligned(16))) float qr_s[4][kDim];
  __shared__ float qs_s[4][kDim];
  __shared__ float cen_s[20];
  __shared__ float red_m[kDecWaves][4];
  __shared__ float red_l[kDecWaves][4];
  char* const ktab = tabs;
  char* const vtab = tabs + kTabBytes;

  const int split = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / a.hkv;
  const int g = bg - b * a.hkv;
  const int64_t T = min((int64_t)max(a.seq_lens[b], 0), a.t_max);
  const int64_t t_begin = (int64_t)split * a.split_tokens;
  const int64_t t_end = min(T, t_begin + a.split_tokens);
  if (t_begin >= t_end) return;  // uniform; the combine reads only splits below T
  const int64_t qh0 = (int64_t)b * a.hq + (int64_t)g * a.G;

  // ---- prologue: centroids, rotated query rows, tables
  if (threadIdx.x < 16) cen_s[threadIdx.x] = threadIdx.x < (1 << KB) ? a.kcen[threadIdx.x] : 0.f;
  else if (threadIdx.x < 20) {
    const int i = threadIdx.x - 16;
    cen_s[threadIdx.x] = i < (1 << VB) ? a.vcen[i] : 0.f;
  }
  {
    const int h = threadIdx.x >> 6, k = threadIdx.x & 63;
    qs_s[h][k] = h < a.G ? load_as_f32(a.q, (qh0 + h) * kDim + k, a.q_dt) : 0.f;
  }
  __syncthreads();
  {
    const int h = threadIdx.x >> 6, j = threadIdx.x & 63;
    const float4* r4 = reinterpret_cast<const float4*>(a.krot + j * kDim);
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < kDim / 4; ++k) {
      const float4 r = r4[k];
      v = fmaf(r.x, qs_s[h][4 * k], v);
      v = fmaf(r.y, qs_s[h][4 * k + 1], v);
      v = fmaf(r.z, qs_s[h][4 * k + 2], v);
      v = fmaf(r.w, qs_s[h][4 * k + 3], v);
    }
    qr_s[h][j] = v * a.qscale;  // padded heads: 0
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 256 * 16; e += kDecThreads) {
    const int i = e >> 4, c = e & 15;
    *reinterpret_cast<float2*>(ktab + i * 128 + c * 8) = make_float2(cen_s[i >> 4], cen_s[i & 15]);
    v4h v;
    v[0] = (_Float16)cen_s[16 + (i & 3)];
    v[1] = (_Float16)cen_s[16 + ((i >> 2) & 3)];
    v[2] = (_Float16)cen_s[16 + ((i >> 4) & 3)];
    v[3] = (_Float16)cen_s[16 + (i >> 6)];
    *reinterpret_cast<v4h*>(vtab + i * 128 + c * 8) = v;
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int quad = lane >> 2, hn = lane & 3;
  float qv[kDim];
#pragma unroll
  for (int j = 0; j < kDim; j += 4) {
    const float4 t4 = *reinterpret_cast<const float4*>(&qr_s[hn][j]);
    qv[j] = t4.x; qv[j + 1] = t4.y; qv[j + 2] = t4.z; qv[j + 3] = t4.w;
  }
  const uint32_t copy = (uint32_t)(lane & 15) * 8;
  const uint32_t sel1 = hn < 2 ? 0x05040100u : 0x03020706u;
  const uint32_t sel2 = (hn & 1) ? 0x03070105u : 0x06020400u;
  // Contiguous caches: per-stream buffers cover exactly the split's valid tokens, so
  // rows and norms past t_end read as zero (and are masked) -- no load needs a clamp or
  // a branch.  Paged caches: the buffers cover the whole pools; a token's row index
  // comes from the block table, whose buffer covers the blocks holding tokens below
  // t_end (entries past it read as block 0: rows that are loaded and masked).  Block
  // ids outside the pool address rows outside the buffer, which read as zero.
  const size_t sbase = PAGED ? 0 : (size_t)bg * (size_t)a.t_max;
  const uint32_t nrec = PAGED ? a.pool_rows : (uint32_t)t_end;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.kpacked + sbase * PK, nrec * PK);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(a.vpacked + sbase * PV, nrec * PV);
  const __amdgpu_buffer_rsrc_t knrs = make_rsrc(a.knorms + sbase, nrec * 4);
  const __amdgpu_buffer_rsrc_t vnrs = make_rsrc(a.vnorms + sbase, nrec * 4);
  const int bsl = PAGED ? a.bs_log2 : 0;
  const __amdgpu_buffer_rsrc_t btrs =
      make_rsrc(PAGED ? a.block_tables + (size_t)b * a.bt_stride : a.seq_lens,
                PAGED ? (uint32_t)(((t_end + (1 << bsl) - 1) >> bsl) * 4) : 0u);
  const int te = (int)t_end;

  struct Tile {
    uint32_t k[PK / 4];
    uint32_t v[PV / 4];
    float kn[4], vn[4];
  };
  // Paged: block id of token t0 + lane, loaded a tile ahead of its rows.
  auto load_block = [&](int t0) -> uint32_t {
    if constexpr (!PAGED) return 0u;
    return __builtin_amdgcn_raw_buffer_load_b32(btrs, (int)(((uint32_t)(t0 + lane) >> bsl) * 4), 0, 0);
  };
  auto load_tile = [&](int t0, Tile& x, uint32_t blk) {
    uint32_t tr, nr;
    if constexpr (PAGED) {
      // the lane quad's four tokens share a block (block_size >= 4, t0 % 4 == 0); wide
      // pools: an id outside the pool (a corrupt table) reads the last block
      if constexpr (WIDE) blk = blk < a.num_blocks ? blk : a.num_blocks - 1;
      tr = ((blk * (uint32_t)a.hkv + (uint32_t)g) << bsl) | ((uint32_t)(t0 + lane) & ((1u << bsl) - 1));
      nr = tr - (uint32_t)hn;
    } else {
      tr = (uint32_t)(t0 + lane);
      nr = (uint32_t)(t0 + 4 * quad);
    }
    if constexpr (WIDE) {  // pool rows (< 2^32) at 64-bit byte addresses
      load_row_at<PK>(a.kpacked + (size_t)tr * PK, x.k);
      load_row_at<PV>(a.vpacked + (size_t)tr * PV, x.v);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x.kn[r] = a.knorms[(size_t)nr + r];
        x.vn[r] = a.vnorms[(size_t)nr + r];
      }
    } else {
      load_row<PK>(krs, tr * PK, x.k);
      load_row<PV>(vrs, tr * PV, x.v);
      const uint32_t no = nr * 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x.kn[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(knrs, (int)no, 4 * r, 0));
        x.vn[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vnrs, (int)no, 4 * r, 0));
      }
    }
  };

  float M = -INFINITY;  // running max of this lane's head (same in all lanes of the head)
  float l = 0.f;        // this lane's share of sum 2^(s - M)
  tq::VnScale vs;       // value norms scaled into fp16 range
  v4f acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = (v4f){0.f, 0.f, 0.f, 0.f};

  int t0 = (int)t_begin + wave * 64;
  Tile cur, nxt;
  uint32_t blk_nxt = 0;
  if (t0 < te) {
    load_tile(t0, cur, load_block(t0));
    blk_nxt = load_block(t0 + kDecWaves * 64);
  }
  while (t0 < te) {
    const int tn = t0 + kDecWaves * 64;
    load_tile(tn, nxt, blk_nxt);
    blk_nxt = load_block(tn + kDecWaves * 64);

    // ---- q.K: octet words [plane3 | plane2 | plane1 | plane0] bytes
    uint32_t W[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t p0 = cur.k[h];
      const uint32_t p1 = KB > 1 ? cur.k[2 + h] : 0u;
      const uint32_t p2 = KB > 2 ? cur.k[4 + h] : 0u;
      const uint32_t p3 = KB > 3 ? cur.k[6 + h] : 0u;
#pragma unroll
      for (int op = 0; op < 2; ++op) {
        const uint32_t sel = op ? 0x07030602u : 0x05010400u;
        const uint32_t x = perm(p1, p0, sel);
        const uint32_t y = perm(p3, p2, sel);
        W[4 * h + 2 * op] = perm(y, x, 0x05040100u);
        W[4 * h + 2 * op + 1] = perm(y, x, 0x07060302u);
      }
    }
    v4f sk[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) sk[x] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int o = 0; o < 8; ++o) {
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const uint32_t wx = W[o] << x;
        const uint32_t addr = __builtin_amdgcn_udot4(wx & 0x88888888u, 0x80402010u, copy, false);
        const float2 cc = *reinterpret_cast<const float2*>(ktab + addr);
        sk[x] = __builtin_amdgcn_mfma_f32_4x4x1f32(cc.x, qv[8 * o + x], sk[x], 0, 0, 0);
        sk[x] = __builtin_amdgcn_mfma_f32_4x4x1f32(cc.y, qv[8 * o + x + 4], sk[x], 0, 0, 0);
      }
    }

    // ---- online softmax (register r = token t0 + 4 * quad + r)
    const v4f skk = (sk[0] + sk[1]) + (sk[2] + sk[3]);
    float s[4], vn[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = skk[r] * cur.kn[r];
      // contiguous caches: norms past t_end read as zero; paged pools: a stale norm (even
      // NaN) is masked with a select, not a branch (a masked copy of the norms merged
      // from a branch has been miscompiled: registers of the live norms reused before
      // their last read)
      vn[r] = (!PAGED || t0 + 4 * quad + r < te) ? cur.vn[r] : 0.f;
    }
    if (t0 + 64 > te) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (t0 + 4 * quad + r >= te) s[r] = -INFINITY;
    }
    const float lm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    // value norms times the wave's scale (masked tokens 0: a stale pool norm may be NaN)
    float vns[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) vns[r] = vn[r] * vs.s;
    const float vm = fmaxf(fmaxf(fabsf(vns[0]), fabsf(vns[1])), fmaxf(fabsf(vns[2]), fabsf(vns[3])));
    // one branch for both rare events: a running maximum moved, the value scale must drop
    if (__any((lm > M) | (vm > tq::VnScale::kBound))) {
      float m2 = lm;
      m2 = fmaxf(m2, __shfl_xor(m2, 4));
      m2 = fmaxf(m2, __shfl_xor(m2, 8));
      m2 = fmaxf(m2, __shfl_xor(m2, 16));
      m2 = fmaxf(m2, __shfl_xor(m2, 32));
      const float mn = fmaxf(M, m2);
      const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mn);
      l *= f;
      float fs = 1.f;  // the value scale's factor
      if (vs.over(vm)) {
        fs = vs.rescale(fmaxf(fmaxf(fabsf(vn[0]), fabsf(vn[1])), fmaxf(fabsf(vn[2]), fabsf(vn[3]))));
#pragma unroll
        for (int r = 0; r < 4; ++r) vns[r] = vn[r] * vs.s;
      }
      const v4f fv = {__shfl(f, 0) * fs, __shfl(f, 1) * fs, __shfl(f, 2) * fs, __shfl(f, 3) * fs};
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] *= fv;
      M = mn;
    }
    v4h wa;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = __builtin_amdgcn_exp2f(s[r] - M);
      psum += p;
      wa[r] = (_Float16)(p * vns[r]);
    }
    l += psum;
    tq::mfma_operand_fence(wa);  // VALU conversions -> MFMA operand: explicit wait states

    // ---- p.V
    uint32_t Tw[2 * VB];
#pragma unroll
    for (int d = 0; d < 2 * VB; ++d) Tw[d] = quad_transpose(cur.v[d], sel1, sel2);
    uint32_t E[2], O[2];  // bits (2i, 2i+1) of each byte = (plane0, plane1) bits of one dim
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t p0 = Tw[h];
      const uint32_t p1 = VB > 1 ? Tw[2 + h] : 0u;
      E[h] = (p0 & 0x55555555u) | ((p1 << 1) & 0xAAAAAAAAu);
      O[h] = ((p0 >> 1) & 0x55555555u) | (p1 & 0xAAAAAAAAu);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int h = i >> 3, bp = 7 - (i & 7), bpe = bp & ~1;
      const uint32_t word = (bp & 1) ? O[h] : E[h];
      const uint32_t sh = word << (6 - bpe);
      const uint32_t addr = __builtin_amdgcn_udot4(sh & 0xC0C0C0C0u, 0x80200802u, copy, false);
      const v4h bv = *reinterpret_cast<const v4h*>(vtab + addr);
      acc[i] = __builtin_amdgcn_mfma_f32_4x4x4f16(wa, bv, acc[i], 0, 0, 0);
    }

    cur = nxt;
    t0 = tn;
  }

  // ---- reduction: lanes of a head, then quads and waves through LDS
  l += __shfl_xor(l, 4);
  l += __shfl_xor(l, 8);
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (lane < 4) {
    red_m[wave][lane] = M;
    red_l[wave][lane] = l;
  }
  __syncthreads();  // also: every wave is done with the tables
  float mx[4], fw[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    mx[m] = fmaxf(fmaxf(red_m[0][m], red_m[1][m]), fmaxf(red_m[2][m], red_m[3][m]));
    const float mw = red_m[wave][m];
    // this wave's share in true scale: its value-norm scale divided out
    fw[m] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx[m]) * vs.inv();
  }
  float* red = reinterpret_cast<float*>(tabs);  // [wave*16 + quad][i][j][m]
  const v4f fwv = {fw[0], fw[1], fw[2], fw[3]};
#pragma unroll
  for (int i = 0; i < 16; ++i)
    *reinterpret_cast<v4f*>(red + (((wave * 16 + quad) * 16 + i) * 16 + hn * 4)) = acc[i] * fwv;
  __syncthreads();
  {
    const int m = threadIdx.x >> 6, dim = threadIdx.x & 63;
    if (m < a.G) {
      const int oct = dim >> 3;
      const int j = oct & 3, i = (oct >> 2) * 8 + (dim & 7);
      float sum = 0.f;
      for (int wq = 0; wq < kDecWaves * 16; ++wq) sum += red[(wq * 16 + i) * 16 + j * 4 + m];
      a.part[((qh0 + m) * a.nsplit + split) * kDim + dim] = sum;
      if (dim == 0) {
        float L = 0.f;
        for (int w = 0; w < kDecWaves; ++w)
          if (red_m[w][m] != -INFINITY) L += red_l[w][m] * __builtin_amdgcn_exp2f(red_m[w][m] - mx[m]);
        a.stats[(qh0 + m) * a.nsplit + split] = make_float2(mx[m], L);
      }
    }
  }
}

// One D-thread block per query row (D = head_dim, 64 or 128): log-sum-exp merge of the
// splits, o = o_rot / L, out = o @ R_v; lse (natural log) = (max + log2 L) * ln 2.
template <int D = kDim>
__global__ __launch_bounds__(D) void fused_combine_kernel(const float* __restrict__ part,
                                                           const float2* __restrict__ stats,
                                                           int nsplit, int64_t split_tokens,
                                                           const int32_t* __restrict__ seq_lens,
                                                           int64_t t_max, int hq,
                                                           const float* __restrict__ vrot,
                                                           int out_dt, void* __restrict__ out,
                                                           float* __restrict__ lse) {
  __shared__ float o_s[D];
  const int64_t row = blockIdx.x;
  const int b = (int)(row / hq);
  const int j = threadIdx.x;
  // column j of R_v, requested first: its loads overlap the split merge below
  float rcol[D];
#pragma unroll
  for (int k = 0; k < D; ++k) rcol[k] = vrot[k * D + j];
  const int64_t T = min((int64_t)max(seq_lens[b], 0), t_max);
  const int ns = (int)((T + split_tokens - 1) / split_tokens);
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, stats[row * nsplit + s].x);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < ns; ++s) {
    const float2 st = stats[row * nsplit + s];
    const float f = st.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.x - M);
    L += st.y * f;
    o += part[(row * nsplit + s) * D + j] * f;
  }
  const bool any = ns > 0 && L > 0.f;
  o_s[j] = any ? o / L : 0.f;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int k = 0; k < D; ++k) r = fmaf(o_s[k], rcol[k], r);
  store_from_f32(out, row * D + j, r, out_dt);
  if (lse && j == 0) lse[row] = any ? (M + log2f(L)) * 0.69314718055994531f : -INFINITY;
}

// ------------------------------------------------------------------ decode layout
// The decode layout holds the same codes as the bit-plane rows, arranged for the
// decode kernel (4-bit keys; 2-, 3- or 4-bit values; head_dim 64 -- head_dim 128 as two
// 64-dim halves: key bytes 32 h .., value tile half h at byte h * 512 VB, each laid out
// as below for dims 64 h ..):
//   keys    per token d/2 bytes; byte p = (code[2p] << 4) | code[2p+1]
//   values  64-token tiles of 512 * VB bytes.  Lane L = 16 sl + c of a wave reads the
//           words its p.V operands need: words 0-3 at byte 16 L, words 4.. at byte
//           1024 + (8 VB - 16) L.  Token tt of the tile is token t = tt % 4 of block
//           4 m + sl = tt / 4; dim j = 16 dg + c.
//     VB 2  word m, byte dg: the four tokens' codes at bits 2t (one lookup of four values)
//     VB 4  word 4 (m / 2) + dg, byte 2 (m % 2) + t / 2: two tokens' codes, token t at
//           bits 4 (t % 2) (one lookup of a pair)
//     VB 3  dims of dg 0-2: word 3 (m / 2) + dg, the same byte, token t at bits 3 (t % 2);
//           dg 3: the 6-bit pair index of that byte position is spread over the top two
//           bits (6, 7) of the same byte of words 3 (m / 2) + 0, 1, 2 (bits 0-1, 2-3, 4-5)
// Every byte is then one table index: a single v_perm builds its LDS address (the 3-bit
// table repeats each pair under the four values of the top two bits).
constexpr int kDlThreads = 512;  // 8 waves (12 measured slower)
constexpr int kDlWaves = kDlThreads / 64;
constexpr int kDlEntry = 256;                  // bytes per table index (all copies)
constexpr int kDlTab = 256 * kDlEntry;         // 64 KB per table
// K table: hi parts of entry i at kDlTab + i * 256 + 128 (upper half of the slot), lo
// parts kDlKLo bytes further (lower half of slot i + 5).  The distance is neither a
// ds_read2 offset (<= 1020) nor a multiple of 256 (ds_read2st64), so the two reads of an
// entry stay separate ds_read_b32 and each MFMA operand pair is loaded in place.
constexpr int kDlKLo = 1152;
constexpr int kDlTabs = 2 * kDlTab + 5 * kDlEntry;
constexpr int kDlMinSplit = kDlWaves * 64;     // one tile per wave
constexpr int kDlMaxDim = 128;                 // head_dim of the largest (contiguous) layout

struct DlArgs {
  const void* q;
  int q_dt;
  int hq, hkv, G;
  const uint8_t* kpairs;   // [B*hkv][t_cap][32]
  const float* knorms;     // [B*hkv][t_cap] (ND != 0: 16-bit values, read through a cast)
  const uint8_t* vblocks;  // [B*hkv][t_cap/4][64]
  const float* vnorms;
  int64_t t_cap;
  const int32_t* seq_lens;
  // optional [B]: tokens before seq_starts[b] are masked (left-padded batches); the
  // tiles holding them are still read
  const int32_t* seq_starts;
  const float* kcen;  // 16
  const float* vcen;  // 2^VB
  const float* krot;
  float qscale;  // softmax scale * log2(e)
  int64_t split_tokens;
  int nsplit;
  // Query heads of a KV head handled by this launch: heads hofs .. hofs + G - 1 of the
  // Gfull heads that share it (more than four take several launches).
  int Gfull, hofs;
  float* part;
  float2* stats;
  // one split per stream: the kernel writes the output itself
  const float* vrot;
  void* out;
  float* lse;
  // Paged pools (PAGED kernels): block b of a sequence holds its tokens [b*bs, (b+1)*bs);
  // kpairs [num_blocks][hkv][bs][32], knorms/vnorms [num_blocks][hkv][bs], vblocks
  // [num_blocks][hkv][bs/64][1024] for bs a power of two >= 64 (a 64-token tile lies in
  // one block), [num_blocks][hkv][bs/16][256] for bs 16 or 32.
  const int32_t* block_tables;
  int bt_stride;
  int bs_log2;
  uint32_t pool_rows;  // num_blocks * hkv * bs
  uint32_t num_blocks;  // wide pools (PG 3, 4): block ids are clamped below it
  int nstreams;         // B * hkv (two streams per workgroup: the last one may be missing)
};

__device__ __forceinline__ uint32_t byte_addr(uint32_t base_copy, uint32_t w, int byte) {
  // (byte `byte` of w) * 256 + base_copy: base_copy holds the copy offset in byte 0
  // and a multiple of 64 KB in byte 2
  return __builtin_amdgcn_perm(base_copy, w, 0x0c060004u | ((uint32_t)byte << 8));
}

__device__ __forceinline__ v4h as_v4h(uint32_t lo, uint32_t hi) {
  u32x2 t = {lo, hi};
  return __builtin_bit_cast(v4h, t);
}

typedef _Float16 v8h __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v8h as_v8h(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 t = {a, b, c, d};
  return __builtin_bit_cast(v8h, t);
}

__device__ __forceinline__ v8h cat_h(v4h lo, v4h hi) {
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return as_v8h(a.x, a.y, b.x, b.y);
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 lo, _Float16 hi) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, (h2_t){lo, hi});
}

// DPP row shifts of a float within each 16-lane row: row_shl:N -- lane i takes lane
// i + N; row_shr:N -- lane i takes lane i - N (zero where the source leaves the row).
template <int N>
__device__ __forceinline__ float row_shl_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xF, 0xF, true));
}
template <int N>
__device__ __forceinline__ float row_shr_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xF, 0xF, true));
}

// DPP row_shl:N on both words of a v4h: lane i of each 16-lane row takes lane i + N's
// value (zero where i + N leaves the row).
template <int N>
__device__ __forceinline__ v4h row_shl_h(v4h x) {
  const u32x2 w = __builtin_bit_cast(u32x2, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)w.x, 0x100 + N, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)w.y, 0x100 + N, 0xF, 0xF, true);
  return as_v4h(lo, hi);
}

// Scale that brings max |x| into [0.5, 1): 2^-e with x = m * 2^e.
__device__ __forceinline__ float pow2_scale(float amax) {
  int e = 0;
  if (amax > 0.f && amax < INFINITY) frexpf(amax, &e);
  return ldexpf(1.f, -e);
}

// EXACT_V: the weights and V centroids enter as fp16 hi + lo parts (three products,
// about 1e-6 relative), for fp32 outputs; otherwise one fp16 product (about 5e-4).
// PREC_K: q.K from fp16 hi + lo parts of query and centroids (three products, about 1e-6
// relative), for fp32 and fp16 outputs; otherwise (bf16 outputs) one fp16 product per
// term, about 2^-11 relative per operand -- finer than the bf16 arithmetic the reference
// scores bf16 inputs in.
// PG: 0 contiguous caches; 1 paged pools of block_size >= 64 (64-token value tiles);
// 2 paged pools of block_size 16 or 32 (16-token value sub-blocks of 128 VB bytes, each
// the share of its token group m of the tile words: VB 2, lane L's word = tile word m;
// VB 4, lane L's 8 bytes at 8 L = the two bytes of each tile word 4 (m / 2) + dg that
// group m fills (dg = 0..3, two bytes each); VB 3, the two bytes of tile words
// 3 (m / 2) + 0, 1 at 4 L and of word 3 (m / 2) + 2 at 256 + 2 L).
// VB: value code width (2, 3 or 4).
// PG: 0 contiguous; 1 / 2 paged pools (blocks >= 64 tokens / 16- or 32-token blocks) read
// through buffer resources over whole pools (32-bit offsets: pools under 2 GiB); 3 / 4 the
// same for pools of any size: rows at 64-bit addresses from clamped block ids.
// ND: the norms' dtype -- 0 fp32, TQ_F16 or TQ_BF16 (contiguous caches only: a bf16 model's
// cache keeps its norms in bf16, as the reference's quantize returns them).
// NH: 64-dim halves of the head (1: head_dim 64; 2: head_dim 128, contiguous caches).  A
// 128-dim key row is 64 pair bytes, half h at bytes 32 h ..; a 128-dim value tile is two
// 64-dim tiles, half h (dims 64 h ..) at byte h * 512 VB.  Each half runs the 64-dim
// operand layouts below; q.K chains both halves' products into one score, p.V keeps one
// accumulator set per half.
template <bool EXACT_V, bool PREC_K, int PG = 0, int VB = 2, int ND = 0, int NH = 1, int SPW = 1>
__global__ __launch_bounds__(kDlThreads, 1) void dl_decode_kernel(DlArgs a) {
  constexpr bool PAGED = PG != 0, SUB16 = PG == 2 || PG == 4, WIDE = PG >= 3;
  constexpr int D = 64 * NH;  // head_dim
  constexpr int WPS = kDlWaves / SPW;  // waves per stream
  static_assert(VB >= 2 && VB <= 4, "value width");
  static_assert(SPW == 1 || (SPW == 2 && NH == 1 && PG == 0), "two streams: contiguous head_dim 64");
  static_assert(ND == 0 || PG == 0, "16-bit norms: contiguous caches");
  static_assert(NH == 1 || (NH == 2 && PG == 0), "head_dim 128: contiguous caches");
  // value words per lane and tile as loaded (16-token sub-blocks of 3-bit values: the four
  // groups' 4-byte and 2-byte shares, reassembled into tile words at their use)
  constexpr int VW = VB == 2 ? 4 : SUB16 ? 8 : 2 * VB;
  constexpr uint32_t SBB = 128u * VB;       // bytes per 16-token value sub-block
  constexpr uint32_t VTILE = 512u * VB;     // bytes per 64-token value tile
  // V table at 0: index = block byte; 32 copies of 4 fp16 centroids, or (EXACT_V) 16
  // copies of 4 hi + 4 lo halves (VB 3, 4: a pair byte's two fp16 centroids, 32 copies
  // in the first 128 bytes of the entry, the lo halves in the second).  K table at 64 KB: index = pair byte; 32 copies of the
  // fp16 hi parts (c[high nibble], c[low nibble]) * ks, and 32 of the lo parts (layout
  // at kDlKLo).  After the tile loop the bytes hold the reduction.
  __shared__ __attribute__((aligned(16))) char tabs[kDlTabs];
  __shared__ __attribute__((aligned(16))) _Float16 qhl_s[4 * SPW][2][D];  // q * qs2: hi, lo
  __shared__ float qs_s[4 * SPW][D];
  __shared__ float hmax_s[NH == 2 ? kDlWaves : 1];  // head_dim 128: per-wave |q_rot| maxima
  __shared__ float cen_s[32];  // 16 key centroids, then the value centroids
  __shared__ __attribute__((aligned(16))) float rv_s[NH == 1 ? kDim * kDim : 1];  // R_v (one split)
  __shared__ float qs2_s[4 * SPW];  // per-head query scales
  __shared__ float red_m[kDlWaves][4];
  __shared__ float red_l[kDlWaves][4];
  __shared__ u32x2 kst_s[256];  // K table entries (hi, lo words) before replication
  __shared__ u32x4 vst_s[256];  // V table entries
  char* const ktab = tabs + kDlTab;
  char* const vtab = tabs;

  // One-dimensional grid: workgroup L = split + nsplit * stream.
  uint32_t W = blockIdx.x;
  if constexpr (PAGED) {
    // XCD-aware order: workgroups go to the 8 XCDs round-robin in linear order, so linear
    // id L runs on XCD L % 8.  Work item W = (L % 8) * (N / 8) + L / 8 puts consecutive
    // (sequence, kv head) streams on one XCD, where the norm lines that adjacent heads of
    // a block share are fetched into that XCD's L2 once.
    const uint32_t N = gridDim.x;
    if ((N & 7u) == 0) W = (W & 7u) * (N >> 3) + (W >> 3);
  }
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  // SPW 2: waves 0-3 take stream 2W, waves 4-7 stream 2W + 1 (one split; the last
  // workgroup's second stream may not exist: then its waves take no tiles and write nothing)
  const int sw = SPW == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave / WPS);
  const int split = (int)(W % (uint32_t)a.nsplit);
  const int bg0 = (int)(W / (uint32_t)a.nsplit) * SPW + sw;
  const bool live = SPW == 1 || bg0 < a.nstreams;
  const int bg = live ? bg0 : 0;
  const int b = bg / a.hkv;
  const int g = bg - b * a.hkv;
  // The sequence length is requested first, and nothing below is addressed through it
  // until the prologue's loads (query, R_k, the first tiles) are all in flight: their
  // latency and its own then overlap instead of following one another.
  const int32_t slen = live ? a.seq_lens[b] : 0;
  const int32_t sstart = a.seq_starts ? a.seq_starts[b] : 0;
  const int64_t t_begin = (int64_t)split * a.split_tokens;
  const int64_t qh0 = (int64_t)b * a.hq + (int64_t)g * a.Gfull + a.hofs;

  // Lane roles (see the score layout and the tile loads below).
  const int sl = lane >> 4, col = lane & 15;
  const int hh = lane & 3, gq = (lane >> 2) & 3;
  // Contiguous: the buffers cover the stream's capacity (t_cap rows, all allocated).
  // Paged: they cover the whole pools, and a tile's block id comes through a buffer over
  // the sequence's block-table row (entries past the sequence's blocks name whatever
  // block they hold: loaded and masked; ids outside the pool address bytes outside the
  // buffers, which read as zero).  Tokens at or past t_end are masked by selects at their
  // use, so what the loads return for them never matters.
  const size_t sbase = PAGED ? 0 : (size_t)bg * (size_t)a.t_cap;
  const uint32_t nrows = PAGED ? a.pool_rows : (uint32_t)a.t_cap;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.kpairs + sbase * 32 * NH, nrows * 32 * NH);
  const __amdgpu_buffer_rsrc_t vrs =
      make_rsrc(a.vblocks + sbase * (8 * VB * NH),
                PAGED ? nrows * (8 * VB) : (uint32_t)(a.t_cap >> 6) * VTILE * NH);
  // Norms are read four tokens at a time (t_cap % 4 == 0, pools of whole blocks).
  constexpr uint32_t NSZ = ND ? 2 : 4;  // bytes per norm
  const uint32_t nbytes = nrows * NSZ;
  const __amdgpu_buffer_rsrc_t knrs =
      make_rsrc(reinterpret_cast<const char*>(a.knorms) + sbase * NSZ, nbytes);
  const __amdgpu_buffer_rsrc_t vnrs =
      make_rsrc(reinterpret_cast<const char*>(a.vnorms) + sbase * NSZ, nbytes);
  const int bsl = PAGED ? a.bs_log2 : 0;
  const int kvh = g;  // the kv head (the tile loads below name their token groups g)
  const __amdgpu_buffer_rsrc_t btrs =
      make_rsrc(PAGED ? a.block_tables + (size_t)b * a.bt_stride : a.seq_lens,
                PAGED ? (uint32_t)a.bt_stride * 4u : 0u);

  struct Tile {
    u32x2 k[NH][4];      // half h, group g: key bytes 32 h + 8 sl .. + 7 of token 16 g + col
    uint32_t v[NH][VW];  // the lane's value tile words of each half (layout above)
    float kn[4], vn[4];  // tokens 16 gq + 4 sl + r
  };
  // Paged: block id of the tile at t0 (one per tile, the same in every lane; SUB16: one
  // per 16-token group of the tile), requested a tile ahead of the tile's own loads.
  using Blk = typename std::conditional<SUB16, u32x4, uint32_t>::type;
  auto load_block = [&](int t0) -> Blk {
    if constexpr (!PAGED) {
      return Blk{};
    } else if constexpr (!SUB16) {
      return __builtin_amdgcn_raw_buffer_load_b32(btrs, (int)(((uint32_t)t0 >> bsl) * 4), 0, 0);
    } else {
      Blk r;
      r.x = __builtin_amdgcn_raw_buffer_load_b32(btrs, (int)(((uint32_t)t0 >> bsl) * 4), 0, 0);
      r.y = __builtin_amdgcn_raw_buffer_load_b32(btrs, (int)(((uint32_t)(t0 + 16) >> bsl) * 4), 0, 0);
      r.z = __builtin_amdgcn_raw_buffer_load_b32(btrs, (int)(((uint32_t)(t0 + 32) >> bsl) * 4), 0, 0);
      r.w = __builtin_amdgcn_raw_buffer_load_b32(btrs, (int)(((uint32_t)(t0 + 48) >> bsl) * 4), 0, 0);
      return r;
    }
  };
  // wide pools: an id outside the pool (a corrupt table) reads the last block, not memory
  // outside the pool
  const uint32_t blast = a.num_blocks - 1;
  auto clampb = [&](uint32_t x) -> uint32_t { return x < a.num_blocks ? x : blast; };
  // Every tile load covers whole cache lines per instruction (512 B of key rows, 1 KB of a
  // value tile, 256 B of norms) and is read once: non-temporal.
  auto load_tile = [&](int t0, Tile& x, Blk blk) {
    // rg[g]: pool row of the first token of the tile's 16-token group g; vt: value tile
    uint32_t rg[4], vt = (uint32_t)t0 >> 6;
#pragma unroll
    for (int g = 0; g < 4; ++g) rg[g] = (uint32_t)t0 + 16 * g;
    if constexpr (PG == 1 || PG == 3) {
      if constexpr (WIDE) blk = clampb(blk);
      const uint32_t sb = blk * (uint32_t)a.hkv + (uint32_t)kvh;
      const uint32_t in = (uint32_t)t0 & ((1u << bsl) - 1);
#pragma unroll
      for (int g = 0; g < 4; ++g) rg[g] = ((sb << bsl) | in) + 16 * g;
      vt = (sb << (bsl - 6)) | (in >> 6);
    } else if constexpr (SUB16) {
      uint32_t bl[4] = {blk.x, blk.y, blk.z, blk.w};
      if constexpr (WIDE) {
#pragma unroll
        for (int g = 0; g < 4; ++g) bl[g] = clampb(bl[g]);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g)
        rg[g] = ((bl[g] * (uint32_t)a.hkv + (uint32_t)kvh) << bsl) |
                (((uint32_t)t0 + 16 * g) & ((1u << bsl) - 1));
    }
    if constexpr (WIDE) {  // pool rows (< 2^32) at 64-bit byte addresses
#pragma unroll
      for (int g = 0; g < 4; ++g)
        x.k[0][g] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(a.kpairs + (size_t)(rg[g] + col) * 32 + 8 * sl));
      if constexpr (SUB16) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint8_t* sb = a.vblocks + (size_t)(rg[m] >> 4) * SBB;
          if constexpr (VB == 2) {
            x.v[0][m] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(sb + lane * 4));
          } else if constexpr (VB == 4) {
            const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(sb + lane * 8));
            x.v[0][2 * m] = w.x; x.v[0][2 * m + 1] = w.y;
          } else {
            x.v[0][m] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(sb + lane * 4));
            x.v[0][4 + m] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(sb + 256 + lane * 2));
          }
        }
      } else {
        const uint8_t* tb = a.vblocks + (size_t)vt * VTILE;
        const u32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tb + lane * 16));
        x.v[0][0] = v0.x; x.v[0][1] = v0.y; x.v[0][2] = v0.z; x.v[0][3] = v0.w;
        if constexpr (VB == 3) {
          const u32x2 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(tb + 1024 + lane * 8));
          x.v[0][4] = v1.x; x.v[0][5] = v1.y;
        } else if constexpr (VB == 4) {
          const u32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tb + 1024 + lane * 16));
          x.v[0][4] = v1.x; x.v[0][5] = v1.y; x.v[0][6] = v1.z; x.v[0][7] = v1.w;
        }
      }
    } else {
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        x.k[h][g] = __builtin_amdgcn_raw_buffer_load_b64(krs, (int)((rg[g] + col) * 32 * NH + 32 * h + 8 * sl), 0, kNT);
    if constexpr (SUB16) {
      // value sub-block of group m = its first pool row / 16 (rows of a group are 16-aligned)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int so = (int)((rg[m] >> 4) * SBB);
        if constexpr (VB == 2) {
          x.v[0][m] = __builtin_amdgcn_raw_buffer_load_b32(vrs, so + lane * 4, 0, kNT);
        } else if constexpr (VB == 4) {
          const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(vrs, so + lane * 8, 0, kNT);
          x.v[0][2 * m] = w.x; x.v[0][2 * m + 1] = w.y;
        } else {
          x.v[0][m] = __builtin_amdgcn_raw_buffer_load_b32(vrs, so + lane * 4, 0, kNT);
          x.v[0][4 + m] = __builtin_amdgcn_raw_buffer_load_b16(vrs, so + 256 + lane * 2, 0, kNT);
        }
      }
    } else {
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int tb = (int)((vt * NH + h) * VTILE);
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(vrs, tb + lane * 16, 0, kNT);
        x.v[h][0] = v0.x; x.v[h][1] = v0.y; x.v[h][2] = v0.z; x.v[h][3] = v0.w;
        if constexpr (VB == 3) {
          const u32x2 v1 = __builtin_amdgcn_raw_buffer_load_b64(vrs, tb + 1024 + lane * 8, 0, kNT);
          x.v[h][4] = v1.x; x.v[h][5] = v1.y;
        } else if constexpr (VB == 4) {
          const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(vrs, tb + 1024 + lane * 16, 0, kNT);
          x.v[h][4] = v1.x; x.v[h][5] = v1.y; x.v[h][6] = v1.z; x.v[h][7] = v1.w;
        }
      }
    }
    }
    // norms of the lane's four tokens (group gq): 16-byte aligned (t_cap % 64 == 0,
    // aligned base)
    uint32_t rq = rg[0] + 16 * gq;
    if constexpr (SUB16) rq = gq == 0 ? rg[0] : gq == 1 ? rg[1] : gq == 2 ? rg[2] : rg[3];
    const uint32_t no = (rq + 4 * sl) * NSZ;
    u32x4 kn4, vn4;
    if constexpr (WIDE) {
      kn4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.knorms + (size_t)(rq + 4 * sl)));
      vn4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.vnorms + (size_t)(rq + 4 * sl)));
    } else if constexpr (ND != 0) {  // four 16-bit norms, widened to fp32 bit patterns
      const u32x2 k2 = __builtin_amdgcn_raw_buffer_load_b64(knrs, (int)no, 0, kNT);
      const u32x2 v2 = __builtin_amdgcn_raw_buffer_load_b64(vnrs, (int)no, 0, kNT);
      auto wide = [](uint32_t h) -> uint32_t {
        return ND == TQ_BF16 ? h << 16
                             : __float_as_uint(__half2float(__ushort_as_half((unsigned short)h)));
      };
      kn4 = (u32x4){wide(k2.x & 0xFFFFu), wide(k2.x >> 16), wide(k2.y & 0xFFFFu), wide(k2.y >> 16)};
      vn4 = (u32x4){wide(v2.x & 0xFFFFu), wide(v2.x >> 16), wide(v2.y & 0xFFFFu), wide(v2.y >> 16)};
    } else {
      kn4 = __builtin_amdgcn_raw_buffer_load_b128(knrs, (int)no, 0, kNT);
      vn4 = __builtin_amdgcn_raw_buffer_load_b128(vnrs, (int)no, 0, kNT);
    }
    // (__builtin_bit_cast of a vector element would read element 0: convert by value)
    x.kn[0] = __uint_as_float(kn4.x); x.kn[1] = __uint_as_float(kn4.y);
    x.kn[2] = __uint_as_float(kn4.z); x.kn[3] = __uint_as_float(kn4.w);
    x.vn[0] = __uint_as_float(vn4.x); x.vn[1] = __uint_as_float(vn4.y);
    x.vn[2] = __uint_as_float(vn4.z); x.vn[3] = __uint_as_float(vn4.w);
  };

  constexpr int kStep = WPS * 64;
  const int tf = (int)t_begin + (wave % WPS) * 64;
  Tile ta, tb, tc;

  // ---- prologue.  Every global read is issued up front, in the order its data is needed
  // (loads complete in issue order, so waiting for one never waits for a later one): the
  // centroids, the query, R_k and (one split per stream) R_v, the matrices read coalesced.
  // A barrier then holds the first tiles' loads back until every wave has issued those: a
  // wave's tile loads queued ahead of another wave's query load would delay it.  Then:
  // centroids, query and R_k into LDS | staged table entries and the rotated query |
  // the tables' copies and R_v into LDS.
  float cenv = 0.f;
  if (tid < 16) cenv = a.kcen[tid];
  else if (tid < 16 + (1 << VB)) cenv = a.vcen[tid - 16];
  // the query element as the aligned 32-bit word that holds it (one load whatever the
  // dtype, converted after the tables: a dtype branch here made the compiler wait for it
  // before issuing the loads below)
  // thread tid < 4 SPW D: head qh = tid / D (head qh % 4 of the thread's stream), dim
  // qj = tid % D
  const int qh = tid / D, qj = tid % D;
  const int64_t qe = (qh0 + ((qh & 3) < a.G ? (qh & 3) : 0)) * D + qj;
  const int64_t qbyte = qe * (a.q_dt == TQ_F32 ? 4 : 2);
  uint32_t qraw = 0;
  if (tid < 4 * SPW * D)
    qraw = *reinterpret_cast<const uint32_t*>(static_cast<const char*>(a.q) + (qbyte & ~int64_t(3)));
  // Head_dim 64: R_k and (one split per stream, for the epilogue) R_v, read coalesced:
  // thread tid holds floats 8 tid .. 8 tid + 7 of each (row tid / 8, float4 columns
  // 2 (tid % 8) and 2 (tid % 8) + 1).  R_k goes through rv_s for the rotation, R_v after it.
  // (Head_dim 128: R_k is read in the product below, R_v in the epilogue.)
  v4f rk0 = (v4f){0.f, 0.f, 0.f, 0.f}, rk1 = rk0, rv0 = rk0, rv1 = rk0;
  if constexpr (NH == 1) {
    const v4f* k4 = reinterpret_cast<const v4f*>(a.krot) + 2 * tid;
    const v4f* r4 = reinterpret_cast<const v4f*>(a.vrot) + 2 * tid;
    rk0 = k4[0];
    rk1 = k4[1];
    rv0 = r4[0];
    rv1 = r4[1];
  }
  __builtin_amdgcn_s_barrier();
  Blk bnx{};  // paged: block id(s) of the next tile to load
  load_tile(tf, ta, load_block(tf));
  load_tile(tf + kStep, tb, load_block(tf + kStep));
  bnx = load_block(tf + 2 * kStep);

  // ---- the split's token range, now that the sequence length has had its latency
  const int64_t T = min((int64_t)max(slen, 0), a.t_cap);
  const int64_t t_end = min(T, t_begin + a.split_tokens);
  // (SPW 2: one split; an empty stream's waves take no tiles and its epilogue writes zeros
  // and lse -inf)
  if (SPW == 1 && t_begin >= t_end) {  // uniform
    if (a.out != nullptr && T == 0 && tid < a.G * D) {  // empty sequence: zeros, lse -inf
      store_from_f32(a.out, qh0 * D + tid, 0.f, a.q_dt);
      if (a.lse && qj == 0) a.lse[qh0 + qh] = -INFINITY;
    }
    return;
  }
  const int te = (int)t_end;
  const int ts = (int)min((int64_t)max(sstart, 0), T);  // first unmasked token
  const int ntiles = __builtin_amdgcn_readfirstlane(tf < te ? (te - tf + kStep - 1) / kStep : 0);
  if (tid < 32) cen_s[tid] = cenv;
  if (tid < 4 * SPW * D) {
    const uint32_t bits = a.q_dt == TQ_F32 ? qraw : (qraw >> (8 * (qbyte & 2))) & 0xFFFFu;
    const float qv = a.q_dt == TQ_F32 ? __uint_as_float(bits)
                     : a.q_dt == TQ_BF16 ? __uint_as_float(bits << 16)
                                         : __half2float(__ushort_as_half((unsigned short)bits));
    qs_s[qh][qj] = (qh & 3) < a.G ? qv : 0.f;
  }
  if constexpr (NH == 1) {
    // R_k row r, float4 column c at slot 16 r + ((c + r) & 15): the rotation's lane r then
    // reads its row with 16 lanes' 16-byte reads on distinct banks
    const int r = tid >> 3, c = 2 * (tid & 7);
    v4f* rk = reinterpret_cast<v4f*>(rv_s);
    rk[16 * r + ((c + r) & 15)] = rk0;
    rk[16 * r + ((c + 1 + r) & 15)] = rk1;
  }
  __syncthreads();
  // centroid scales: the powers of two that bring each codebook's largest |c| into
  // [0.5, 1) (the same in every lane)
  float km = fabsf(cen_s[lane & 15]);
  float vm = (lane & 15) < (1 << VB) ? fabsf(cen_s[16 + (lane & 15)]) : 0.f;
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) {
    km = fmaxf(km, __shfl_xor(km, o));
    vm = fmaxf(vm, __shfl_xor(vm, o));
  }
  const float ksc = pow2_scale(km), vsc = pow2_scale(vm);
  // Tables: each entry's fp16 words are converted once (a thread per K entry, a thread
  // per V entry) into a small staging table, then stored as 16-byte runs of identical
  // copies, consecutive lanes writing consecutive runs (conflict-free LDS writes).
  // K: entry i, copies 4q .. 4q + 3 of the hi parts (and of the lo parts with PREC_K).
  // V: entry i, copies 2q, 2q + 1 (or, EXACT_V, copy q: hi and lo halves); VB 3, 4: pair
  // entries (c[low code], c[high code]) * vsc as two fp16, copies 4q .. 4q + 3, lo halves
  // 128 bytes further.
  static_assert(kDlThreads == 512, "a thread per K entry and a thread per V entry");
  if (tid < 256) {
    const int i = tid;
    const float x0 = cen_s[i >> 4] * ksc, x1 = cen_s[i & 15] * ksc;
    const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
    kst_s[i] = (u32x2){pack_h2(h0, h1), pack_h2((_Float16)(x0 - (float)h0), (_Float16)(x1 - (float)h1))};
  } else {
    const int i = tid - 256;
    if constexpr (VB == 2) {
      v4h vh, vl;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float x = cen_s[16 + ((i >> (2 * t)) & 3)] * vsc;
        vh[t] = (_Float16)x;
        vl[t] = (_Float16)(x - (float)vh[t]);
      }
      const u32x2 h = __builtin_bit_cast(u32x2, vh), lo = __builtin_bit_cast(u32x2, vl);
      vst_s[i] = EXACT_V ? (u32x4){h.x, h.y, lo.x, lo.y} : (u32x4){h.x, h.y, h.x, h.y};
    } else {
      constexpr int mask = (1 << VB) - 1;
      const float x0 = cen_s[16 + (i & mask)] * vsc, x1 = cen_s[16 + ((i >> VB) & mask)] * vsc;
      const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
      vst_s[i] = (u32x4){pack_h2(h0, h1), pack_h2((_Float16)(x0 - (float)h0), (_Float16)(x1 - (float)h1)), 0u, 0u};
    }
  }
  // the rotated query (the staged entries above are in flight to LDS meanwhile)
  if constexpr (NH == 2) {  // head_dim 128: every wave rotates (head wave / 2, dims 64 (wave % 2) ..)
    const int h = qh, j = qj;
    const float4* r4 = reinterpret_cast<const float4*>(a.krot + j * D);
    float v = 0.f;
#pragma unroll 8
    for (int k = 0; k < D / 4; ++k) {
      const float4 r = r4[k];
      v = fmaf(r.x, qs_s[h][4 * k], v);
      v = fmaf(r.y, qs_s[h][4 * k + 1], v);
      v = fmaf(r.z, qs_s[h][4 * k + 2], v);
      v = fmaf(r.w, qs_s[h][4 * k + 3], v);
    }
    v *= a.qscale;
    const float wm = wave_max(fabsf(v));
    if (lane == 0) hmax_s[wave] = wm;
    __syncthreads();
    // fp16 hi + lo parts, the head's largest element scaled into [0.5, 1) (both halves)
    const float s2 = pow2_scale(fmaxf(hmax_s[2 * h], hmax_s[2 * h + 1]));
    const float x = v * s2;
    const _Float16 xh = (_Float16)x;
    qhl_s[h][0][j] = xh;
    qhl_s[h][1][j] = (_Float16)(x - (float)xh);
    if (j == 0) qs2_s[h] = s2;
  } else if (tid < 4 * SPW * kDim) {  // waves 0-3 (SPW 2: 0-7): head h = wave, dim j = lane (row j of R_k)
    const int h = tid >> 6, j = tid & 63;
    const v4f* rk = reinterpret_cast<const v4f*>(rv_s);
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < kDim / 4; ++k) {
      const v4f r = rk[16 * j + ((k + j) & 15)];
      v = fmaf(r.x, qs_s[h][4 * k], v);
      v = fmaf(r.y, qs_s[h][4 * k + 1], v);
      v = fmaf(r.z, qs_s[h][4 * k + 2], v);
      v = fmaf(r.w, qs_s[h][4 * k + 3], v);
    }
    v *= a.qscale;
    // fp16 hi + lo parts of the rotated query, scaled by a power of two that brings the
    // head's largest element into [0.5, 1) (lo parts stay normal numbers)
    const float s2 = pow2_scale(wave_max(fabsf(v)));
    const float x = v * s2;
    const _Float16 xh = (_Float16)x;
    qhl_s[h][0][j] = xh;
    qhl_s[h][1][j] = (_Float16)(x - (float)xh);
    if (j == 0) qs2_s[h] = s2;
  }
  __syncthreads();
  for (int e = tid; e < 256 * 8; e += kDlThreads) {
    const int i = e >> 3, q = e & 7;
    const u32x2 w = kst_s[i];
    *reinterpret_cast<u32x4*>(ktab + i * kDlEntry + 128 + q * 16) = (u32x4){w.x, w.x, w.x, w.x};
    if constexpr (PREC_K)
      *reinterpret_cast<u32x4*>(ktab + i * kDlEntry + 128 + kDlKLo + q * 16) = (u32x4){w.y, w.y, w.y, w.y};
  }
  if constexpr (VB == 2) {
    for (int e = tid; e < 256 * 16; e += kDlThreads) {
      const int i = e >> 4, q = e & 15;
      *reinterpret_cast<u32x4*>(vtab + i * kDlEntry + q * 16) = vst_s[i];
    }
  } else {
    for (int e = tid; e < 256 * 8; e += kDlThreads) {
      const int i = e >> 3, q = e & 7;
      const u32x4 w = vst_s[i];
      *reinterpret_cast<u32x4*>(vtab + i * kDlEntry + q * 16) = (u32x4){w.x, w.x, w.x, w.x};
      if constexpr (EXACT_V)
        *reinterpret_cast<u32x4*>(vtab + i * kDlEntry + 128 + q * 16) = (u32x4){w.y, w.y, w.y, w.y};
    }
  }
  if constexpr (NH == 1) {  // R_k has been read: rv_s takes R_v
    reinterpret_cast<v4f*>(rv_s)[2 * tid] = rv0;
    reinterpret_cast<v4f*>(rv_s)[2 * tid + 1] = rv1;
  }
  __syncthreads();

  // q.K runs on 16x16x32 MFMAs: rows = 16 tokens, k = 32 dims, cols = (part, head): col
  // h holds the hi halves of head h's (R_k q) * scale * log2(e) * qs2, col 4 + h the lo
  // halves, cols 8-15 zero.  Lane slice sl = lane / 16, chunk c: k = 8 sl + i is dim
  // 16 sl + 8 c + i (the dims of key bytes 8 sl + 4 c .. + 3).  bq[c]: hi and lo columns
  // (multiplies the centroid hi parts); bqh[c]: hi columns only (centroid lo parts).
  // Without PREC_K each token group g has its own columns instead: col 4g + h = head h
  // (hi halves), so one accumulator collects all four groups already in the score layout
  // below.  bcol[c][g]: the lane's hi halves if col / 4 == g, else zero.  Head_dim 128: the
  // same per half h (dims 64 h + ..); without PREC_K the hi halves bhi[h][c] are kept and
  // the per-group columns selected at their use.
  v8h bq[NH][2], bqh[NH][2], bcol[NH == 1 ? 2 : 1][4], bhi[NH][2];
  const v8h vz = (v8h){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int d0 = 64 * h + 16 * sl + 8 * c;
    const v8h z = vz;
    if constexpr (PREC_K) {
      const v8h hi = col < 4 ? *reinterpret_cast<const v8h*>(&qhl_s[4 * sw + col][0][d0]) : z;
      const v8h lo = (col >= 4 && col < 8) ? *reinterpret_cast<const v8h*>(&qhl_s[4 * sw + col - 4][1][d0]) : z;
      bq[h][c] = col < 4 ? hi : lo;
      bqh[h][c] = hi;
    } else {
      const v8h hi = *reinterpret_cast<const v8h*>(&qhl_s[4 * sw + (col & 3)][0][d0]);
      bhi[h][c] = hi;
      if constexpr (NH == 1) {
#pragma unroll
        for (int g = 0; g < 4; ++g) bcol[c][g] = (col >> 2) == g ? hi : z;
      }
    }
  }
  auto bcol_of = [&](int h, int c, int g) -> v8h {
    if constexpr (NH == 1) return bcol[c][g];
    else return (col >> 2) == g ? bhi[h][c] : vz;
  };
  // Score layout after q.K: lane 16 sl + 4 g + h holds tokens 16 g + 4 sl + r (register r)
  // of head h; g = token group of the 16x16x32 MFMA whose rows hold them.
  const float kinv = 1.f / (ksc * qs2_s[4 * sw + hh]);  // a power of two: exact
  // byte 0: copy offset; byte 2 of kcopy: the K table's 64 KB base
  const uint32_t kcopy = (uint32_t)kDlTab | (128u + (uint32_t)(lane & 31) * 4);
  const uint32_t vcopy = VB != 2 ? (uint32_t)(lane & 31) * 4
                          : EXACT_V ? (uint32_t)(lane & 15) * 16 : (uint32_t)(lane & 31) * 8;
  // VB 3, 4: tile word i of half G (16-token sub-blocks: bytes 0-1 from group 2G's share,
  // bytes 2-3 from group 2G + 1's)
  auto tword = [&](const Tile& x, int hd, int G, int i) -> uint32_t {
    const uint32_t* v = x.v[hd];
    if constexpr (!SUB16) {
      return v[(VB == 4 ? 4 : 3) * G + i];
    } else if constexpr (VB == 4) {
      return __builtin_amdgcn_perm(v[2 * (2 * G + 1) + (i >> 1)], v[2 * (2 * G) + (i >> 1)],
                                   (i & 1) ? 0x07060302u : 0x05040100u);
    } else {
      return i == 2 ? __builtin_amdgcn_perm(v[4 + 2 * G + 1], v[4 + 2 * G], 0x05040100u)
                    : __builtin_amdgcn_perm(v[2 * G + 1], v[2 * G], i ? 0x07060302u : 0x05040100u);
    }
  };
  // VB 3, 4: the word whose four bytes index the pair entries of token half G, dim group
  // dg (of head half hd)
  auto vword = [&](const Tile& x, int hd, int G, int dg) -> uint32_t {
    if constexpr (VB == 4) {
      return tword(x, hd, G, dg);
    } else {
      if (dg < 3) return tword(x, hd, G, dg);
      const uint32_t x0 = tword(x, hd, G, 0), x1 = tword(x, hd, G, 1), x2 = tword(x, hd, G, 2);
      return ((x0 >> 6) & 0x03030303u) | ((x1 >> 4) & 0x0C0C0C0Cu) | ((x2 >> 2) & 0x30303030u);
    }
  };
  auto vpair = [&](uint32_t w, int byte) -> uint32_t {
    return *reinterpret_cast<const uint32_t*>(tabs + byte_addr(vcopy, w, byte));
  };

  float M = -INFINITY, l = 0.f;
  tq::VnScale vs;  // value norms scaled into fp16 range
  // half h, dim group dg: lanes 0-15 hold heads 0-3 (registers), dim 64 h + 16 dg + lane
  v4f acc[NH][4];
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[h][i] = (v4f){0.f, 0.f, 0.f, 0.f};

  // One 64-token tile of this wave: x holds its data, loaded one tile ahead.
  auto process = [&](const Tile& cur, int t0) {
    // ---- q.K: per token group g, four 16x16x32 MFMAs: chunks c = 0, 1 of the lane's 8
    // key bytes, centroid hi parts against the (hi | lo) query columns and centroid lo
    // parts against the hi columns: c.q = ch.qh + ch.ql + cl.qh (the cl.ql term is 2^-22
    // relative), accumulated in fp32.  dk[g] (lane 16 sl + n, register r) = token 16 g +
    // 4 sl + r, column n.
    v4f skk;
    if constexpr (!PREC_K) {
      // one product per term; chunk c accumulates in its own chain
      v4f d2[2] = {(v4f){0.f, 0.f, 0.f, 0.f}, (v4f){0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int hd = 0; hd < NH; ++hd)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const uint32_t w = c ? cur.k[hd][g].y : cur.k[hd][g].x;
          uint32_t ad[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) ad[j] = byte_addr(kcopy, w, j);
          const v8h ah = as_v8h(*reinterpret_cast<const uint32_t*>(tabs + ad[0]),
                                *reinterpret_cast<const uint32_t*>(tabs + ad[1]),
                                *reinterpret_cast<const uint32_t*>(tabs + ad[2]),
                                *reinterpret_cast<const uint32_t*>(tabs + ad[3]));
          d2[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bcol_of(hd, c, g), d2[c], 0, 0, 0);
        }
      }
      skk = (d2[0] + d2[1]) * kinv;
    } else {
    v4f dk[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      dk[g] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int hc = 0; hc < 2 * NH; ++hc) {
        const int hd = hc >> 1, c = hc & 1;
        const uint32_t w = c ? cur.k[hd][g].y : cur.k[hd][g].x;
        uint32_t ad[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ad[j] = byte_addr(kcopy, w, j);
        const v8h ah = as_v8h(*reinterpret_cast<const uint32_t*>(tabs + ad[0]),
                              *reinterpret_cast<const uint32_t*>(tabs + ad[1]),
                              *reinterpret_cast<const uint32_t*>(tabs + ad[2]),
                              *reinterpret_cast<const uint32_t*>(tabs + ad[3]));
        const v8h al = as_v8h(*reinterpret_cast<const uint32_t*>(tabs + ad[0] + kDlKLo),
                              *reinterpret_cast<const uint32_t*>(tabs + ad[1] + kDlKLo),
                              *reinterpret_cast<const uint32_t*>(tabs + ad[2] + kDlKLo),
                              *reinterpret_cast<const uint32_t*>(tabs + ad[3] + kDlKLo));
        dk[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[hd][c], dk[g], 0, 0, 0);
        dk[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bqh[hd][c], dk[g], 0, 0, 0);
      }
    }
    // Lane 16 sl + 4 g + h takes group g's column h (lane 16 sl + h) plus column 4 + h
    // (lane 16 sl + 4 + h): row shifts within each 16-lane row, then a select by g.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x0 = dk[0][r] + row_shl_f<4>(dk[0][r]);
      const float x1 = row_shr_f<4>(dk[1][r]) + dk[1][r];
      const float x2 = row_shr_f<8>(dk[2][r]) + row_shr_f<4>(dk[2][r]);
      const float x3 = row_shr_f<12>(dk[3][r]) + row_shr_f<8>(dk[3][r]);
      skk[r] = (gq == 0 ? x0 : gq == 1 ? x1 : gq == 2 ? x2 : x3) * kinv;
    }
    }

    // The value-centroid lookups depend only on the tile's bytes: issued here, their LDS
    // latency runs under the softmax arithmetic.  (p.V below describes the operands.)
    // (head half hd's operands; head_dim 128: half 1's after half 0's products)
    auto value_ops = [&](int hd, v8h (&bv)[8]) {
      if constexpr (VB == 2) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // i = 4 G + dg; value words m = 2G, 2G + 1
          const int G = i >> 2, dg = i & 3;
          bv[i] = cat_h(*reinterpret_cast<const v4h*>(tabs + byte_addr(vcopy, cur.v[hd][2 * G], dg)),
                        *reinterpret_cast<const v4h*>(tabs + byte_addr(vcopy, cur.v[hd][2 * G + 1], dg)));
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // i = 4 G + dg; bytes: blocks 8G + sl, 8G + 4 + sl
          const uint32_t w = vword(cur, hd, i >> 2, i & 3);
          bv[i] = as_v8h(vpair(w, 0), vpair(w, 1), vpair(w, 2), vpair(w, 3));
        }
      }
    };
    v8h bv[8];
    if constexpr (!EXACT_V) value_ops(0, bv);

    // ---- online softmax (register r = token t0 + 16 gq + 4 sl + r, head hh)
    // Tokens at or past te are masked with selects at their use (branch-free: a masked
    // copy of the norms merged from a branch was miscompiled -- registers of the live
    // norms reused before their last read).
    const int nvalid = te - (t0 + 16 * gq + 4 * sl);
    const int nlow = ts - (t0 + 16 * gq + 4 * sl);  // registers below it are masked
    float s[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = ((r < nvalid) & (r >= nlow)) ? skk[r] * cur.kn[r] : -INFINITY;
    const float lm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    // the live tokens' value norms times the wave's scale (masked ones 0)
    float vns[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) vns[r] = ((r < nvalid) & (r >= nlow)) ? cur.vn[r] * vs.s : 0.f;
    const float vm = fmaxf(fmaxf(fabsf(vns[0]), fabsf(vns[1])), fmaxf(fabsf(vns[2]), fabsf(vns[3])));
    // one branch for both rare events: a running maximum moved, the value scale must drop
    if (__any((lm > M) | (vm > tq::VnScale::kBound))) {
      float m2 = lm;
      m2 = fmaxf(m2, __shfl_xor(m2, 4));
      m2 = fmaxf(m2, __shfl_xor(m2, 8));
      m2 = fmaxf(m2, __shfl_xor(m2, 16));
      m2 = fmaxf(m2, __shfl_xor(m2, 32));
      const float mn = fmaxf(M, m2);
      const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mn);
      l *= f;
      float fs = 1.f;  // the value scale's factor
      if (vs.over(vm)) {
        float um = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) um = fmaxf(um, ((r < nvalid) & (r >= nlow)) ? fabsf(cur.vn[r]) : 0.f);
        fs = vs.rescale(um);
#pragma unroll
        for (int r = 0; r < 4; ++r) vns[r] = ((r < nvalid) & (r >= nlow)) ? cur.vn[r] * vs.s : 0.f;
      }
      const v4f fv = {__shfl(f, 0) * fs, __shfl(f, 1) * fs, __shfl(f, 2) * fs, __shfl(f, 3) * fs};
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[h][i] *= fv;
      M = mn;
    }
    // masked tokens: s = -inf, p = 0 (M clamped: M is -inf while every token so far was masked)
    const float Mp = fmaxf(M, -0x1.fffffep127f);
    v4h wh, wl;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = __builtin_amdgcn_exp2f(s[r] - Mp);
      psum += p;
      const float w = p * vns[r];
      if constexpr (EXACT_V) {
        _Float16 h, lo;
        tq::split_f16(w, h, lo);
        wh[r] = h;
        wl[r] = lo;
      } else {
        wh[r] = (_Float16)w;
      }
    }
    l += psum;
    // The weights are written by VALU conversions and read by the MFMAs below as the A
    // operand: explicit wait states between the two (tq::mfma_operand_fence).
    if constexpr (EXACT_V) tq::mfma_operand_fence(wh, wl);
    else tq::mfma_operand_fence(wh);

    // ---- p.V: one 16x16x32 MFMA per (token half G, dim group dg): A rows = heads (rows
    // 4-15 unused), k = 8 sl + j: tokens of block 8G + sl (j < 4) and 8G + 4 + sl (j >= 4),
    // B cols = dims 16 dg + col.  Lane 16 sl + h takes the weights of lanes 16 sl + 8G + h
    // and 16 sl + 8G + 4 + h: row shifts left by 8G and 8G + 4.
    v8h aw[2], awl[2];
    aw[0] = cat_h(wh, row_shl_h<4>(wh));
    aw[1] = cat_h(row_shl_h<8>(wh), row_shl_h<12>(wh));
    if constexpr (EXACT_V) {
      awl[0] = cat_h(wl, row_shl_h<4>(wl));
      awl[1] = cat_h(row_shl_h<8>(wl), row_shl_h<12>(wl));
    }
    if constexpr (!EXACT_V) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[0][i & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[i >> 2], bv[i], acc[0][i & 3], 0, 0, 0);
      if constexpr (NH == 2) {
        value_ops(1, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          acc[1][i & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[i >> 2], bv[i], acc[1][i & 3], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int hG = 0; hG < 2 * NH; ++hG) {
        const int hd = hG >> 1, G = hG & 1;
        v8h bh[4], bl[4];
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) {
          if constexpr (VB == 2) {
            const u32x4 e0 = *reinterpret_cast<const u32x4*>(tabs + byte_addr(vcopy, cur.v[hd][2 * G], dg));
            const u32x4 e1 = *reinterpret_cast<const u32x4*>(tabs + byte_addr(vcopy, cur.v[hd][2 * G + 1], dg));
            bh[dg] = as_v8h(e0.x, e0.y, e1.x, e1.y);
            bl[dg] = as_v8h(e0.z, e0.w, e1.z, e1.w);
          } else {
            const uint32_t w = vword(cur, hd, G, dg);
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const char* e = tabs + byte_addr(vcopy, w, k);
              hi[k] = *reinterpret_cast<const uint32_t*>(e);
              lo[k] = *reinterpret_cast<const uint32_t*>(e + 128);
            }
            bh[dg] = as_v8h(hi[0], hi[1], hi[2], hi[3]);
            bl[dg] = as_v8h(lo[0], lo[1], lo[2], lo[3]);
          }
        }
        if (hG == 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) acc[hd][dg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[G], bh[dg], acc[hd][dg], 0, 0, 0);
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) acc[hd][dg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(awl[G], bh[dg], acc[hd][dg], 0, 0, 0);
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) acc[hd][dg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[G], bl[dg], acc[hd][dg], 0, 0, 0);
      }
    }

  };

  // Tiles are loaded two ahead into three buffers used in turn: one tile of lookahead
  // does not cover the HBM latency under full load (more lookahead measured slower: the
  // extra tiles in flight delay the prologue's own reads).  Loads past te read data that
  // is masked (or zeros past the buffers); the tile count is made wave-uniform explicitly.
  // Head_dim 64: whole groups of three tiles, then the last one or two (in ta, tb).  The
  // loop has no exit inside a group: an exit there joins the back edge, and every
  // iteration then starts by waiting for all loads in flight, the lookahead tile's
  // included.  (Head_dim 128 keeps the exits: two more copies of its tile code spill.
  // With 3- and 4-bit values its three buffers spill too (9 / 28 VGPRs): those take two
  // buffers, one tile ahead -- a 128-dim tile carries twice the bytes of a 64-dim one, and
  // K4/V3 at T = 32K measured 176-177 against 181-182 us; 2-bit values keep three, 155-156
  // against 157-158 us.)
  if constexpr (NH == 1) {
    int it = 0;
    for (; it + 3 <= ntiles; it += 3) {
      const int t = tf + it * kStep;
      const Blk b1 = load_block(t + 3 * kStep);
      load_tile(t + 2 * kStep, tc, bnx);
      process(ta, t);
      const Blk b2 = load_block(t + 4 * kStep);
      load_tile(t + 3 * kStep, ta, b1);
      process(tb, t + kStep);
      bnx = load_block(t + 5 * kStep);
      load_tile(t + 4 * kStep, tb, b2);
      process(tc, t + 2 * kStep);
    }
    if (it < ntiles) process(ta, tf + it * kStep);
    if (it + 1 < ntiles) process(tb, tf + (it + 1) * kStep);
  } else if constexpr (VB != 2) {
    for (int it = 0; it < ntiles; it += 2) {
      const int t = tf + it * kStep;
      process(ta, t);
      if (it + 1 >= ntiles) break;
      load_tile(t + 2 * kStep, ta, bnx);
      process(tb, t + kStep);
      load_tile(t + 3 * kStep, tb, bnx);
    }
  } else {
    for (int it = 0; it < ntiles; it += 3) {
      const int t = tf + it * kStep;
      const Blk b1 = load_block(t + 3 * kStep);
      load_tile(t + 2 * kStep, tc, bnx);
      process(ta, t);
      if (it + 1 >= ntiles) break;
      const Blk b2 = load_block(t + 4 * kStep);
      load_tile(t + 3 * kStep, ta, b1);
      process(tb, t + kStep);
      if (it + 2 >= ntiles) break;
      bnx = load_block(t + 5 * kStep);
      load_tile(t + 4 * kStep, tb, b2);
      process(tc, t + 2 * kStep);
    }
  }

  // ---- reduction: l over the lanes of a head; outputs over the waves (LDS)
  l += __shfl_xor(l, 4);
  l += __shfl_xor(l, 8);
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (lane < 4) {
    red_m[wave][lane] = M;
    red_l[wave][lane] = l;
  }
  __syncthreads();  // also: every wave is done with the tables
  float mx[4], fw[4];
  const int w0 = WPS * sw;  // the stream's first wave
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float v = red_m[w0][m];
#pragma unroll
    for (int w = 1; w < WPS; ++w) v = fmaxf(v, red_m[w0 + w][m]);
    mx[m] = v;
    const float mw = red_m[wave][m];
    // this wave's share in true scale: its value-norm scale divided out
    fw[m] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx[m]) * vs.inv();
  }
  float* red = reinterpret_cast<float*>(tabs);  // [wave][head m][dim]
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int dg = 0; dg < 4; ++dg)
#pragma unroll
      for (int m = 0; m < 4; ++m) red[(wave * 4 + m) * D + 64 * h + 16 * dg + lane] = acc[h][dg][m] * fw[m];
  }
  __syncthreads();
  // thread tid < 4 SPW D: head m of its own wave's stream (tid / (4 D) = sw)
  if (tid < 4 * SPW * D) {
    const int m = (tid / D) & 3, dim = tid % D;
    float sum = 0.f;
    for (int w = w0; w < w0 + WPS; ++w) sum += red[(w * 4 + m) * D + dim];
    float L = 0.f;
    for (int w = w0; w < w0 + WPS; ++w)
      if (red_m[w][m] != -INFINITY) L += red_l[w][m] * __builtin_amdgcn_exp2f(red_m[w][m] - mx[m]);
    if (a.out == nullptr) {  // several splits: partials for the combine kernel
      if (m < a.G) {
        a.part[((qh0 + m) * a.nsplit + split) * D + dim] = sum / vsc;
        if (dim == 0) a.stats[(qh0 + m) * a.nsplit + split] = make_float2(mx[m], L);
      }
    } else {  // the whole sequence: out = (o / L) @ R_v here
      qs_s[4 * sw + m][dim] = L > 0.f ? sum / (vsc * L) : 0.f;
    }
    if (live && a.out != nullptr && m < a.G && dim == 0 && a.lse)
      a.lse[qh0 + m] = L > 0.f ? (mx[m] + log2f(L)) * 0.69314718055994531f : -INFINITY;
  }
  if (a.out != nullptr) {
    __syncthreads();
    if (tid < 4 * SPW * D) {
      const int m = (tid / D) & 3, dim = tid % D;
      if (live && m < a.G) {
        float r = 0.f;
        if constexpr (NH == 1) {
#pragma unroll
          for (int k = 0; k < kDim; ++k) r = fmaf(qs_s[4 * sw + m][k], rv_s[k * kDim + dim], r);
        } else {
#pragma unroll 8
          for (int k = 0; k < D; ++k) r = fmaf(qs_s[4 * sw + m][k], a.vrot[k * D + dim], r);
        }
        store_from_f32(a.out, (qh0 + m) * D + dim, r, a.q_dt);
      }
    }
  }
}

// Byte offset, inside a 64-token value tile of width VB 3 or 4, of byte k of lane L's
// value word w (words 0-3 at 16 L, the rest at 1024 + (8 VB - 16) L).
__device__ __forceinline__ int vt_byte_off(int VB, int L, int w, int k) {
  return w < 4 ? 16 * L + 4 * w + k : 1024 + (8 * VB - 16) * L + 4 * (w - 4) + k;
}

// Bit b of a VB 3 / 4 tile byte (lane L, word w, byte k) holds bit `cbit` of the code of
// tile token `tt`, dim `j`.
__device__ __forceinline__ void vt_bit_source(int VB, int L, int w, int k, int b, int& tt, int& j,
                                              int& cbit) {
  const int sl = L >> 4, c = L & 15;
  int G, e;
  if (VB == 4) {
    G = w >> 2;
    j = 16 * (w & 3) + c;
    e = b >> 2;
    cbit = b & 3;
  } else {
    G = w / 3;
    const int i = w - 3 * G;
    if (b < 6) {
      j = 16 * i + c;
      e = b / 3;
      cbit = b - 3 * e;
    } else {  // bits 2i, 2i + 1 of dim group 3's pair index
      const int q = 2 * i + (b - 6);
      j = 48 + c;
      e = q / 3;
      cbit = q - 3 * e;
    }
  }
  const int m = 2 * G + (k >> 1);
  tt = 4 * (4 * m + sl) + 2 * (k & 1) + e;
}

// Bit-plane rows -> decode layout.  keys: one thread per output byte.  values: one
// thread per byte of the 64-token tiles that tokens [pos, pos + n) touch; bits of
// tokens outside that range are kept.
__global__ void dl_pack_kernel(const uint8_t* __restrict__ packed, int64_t n_streams, int64_t n,
                               int d, int bits, int values, uint8_t* __restrict__ cache,
                               int64_t t_cap, int64_t pos) {
  const int bpp = (d + 7) / 8;
  const int P = bits * bpp;
  auto code = [&](int64_t s, int64_t t, int j) -> uint32_t {  // t relative to pos
    const uint8_t* row = packed + (s * n + t) * P;
    uint32_t c = 0;
    for (int p = 0; p < bits; ++p) c |= ((row[p * bpp + (j >> 3)] >> (7 - (j & 7))) & 1u) << p;
    return c;
  };
  if (!values) {
    const int half = d / 2;
    const int64_t total = n_streams * n * half;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
      const int pidx = (int)(e % half);
      const int64_t r = e / half, s = r / n, t = r - s * n;
      cache[(s * t_cap + pos + t) * half + pidx] =
          (uint8_t)((code(s, t, 2 * pidx) << 4) | code(s, t, 2 * pidx + 1));
    }
  } else if (bits == 2) {
    // value tiles of 64 tokens, a 1024-byte half per 64 dims (d = 64 or 128): byte
    // 16 L + 4 m + dg of half h of tile T, L = 16 sl + c, holds dim 64 h + 16 dg + c of
    // tokens 64 T + 4 (4 m + sl) + t, 2 bits each (t = 0..3)
    const int tbytes = 1024 * (d / 64);
    const int64_t c0 = pos >> 6, c1 = (pos + n + 63) >> 6;
    const int64_t nt = c1 - c0;
    const int64_t total = n_streams * nt * tbytes;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
      const int tb = (int)(e % tbytes), byte = tb & 1023;
      const int64_t r = e / tbytes, s = r / nt, tile = c0 + (r - s * nt);
      const int L = byte >> 4, m = (byte >> 2) & 3, dg = byte & 3;
      const int sl = L >> 4, c = L & 15;
      const int j = 64 * (tb >> 10) + 16 * dg + c;
      uint8_t* dst = cache + (s * (t_cap >> 6) + tile) * tbytes + tb;
      uint32_t v = *dst;
      for (int tt = 0; tt < 4; ++tt) {
        const int64_t t = tile * 64 + 4 * (4 * m + sl) + tt - pos;
        if (t < 0 || t >= n) continue;
        v = (v & ~(3u << (2 * tt))) | (code(s, t, j) << (2 * tt));
      }
      *dst = (uint8_t)v;
    }
  } else {
    // 3- and 4-bit value tiles of 512 * bits bytes per 64-dim half: each byte's bits
    // gathered one by one
    const int tb = 512 * bits, nb = 8 * bits - 16, tbytes = tb * (d / 64);
    const int64_t c0 = pos >> 6, c1 = (pos + n + 63) >> 6;
    const int64_t nt = c1 - c0;
    const int64_t total = n_streams * nt * tbytes;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
      const int toff = (int)(e % tbytes), half = toff / tb, off = toff - half * tb;
      const int64_t r = e / tbytes, s = r / nt, tile = c0 + (r - s * nt);
      int L, w, k;
      if (off < 1024) {
        L = off >> 4; w = (off >> 2) & 3; k = off & 3;
      } else {
        const int o = off - 1024;
        L = o / nb;
        const int rr = o - L * nb;
        w = 4 + (rr >> 2); k = rr & 3;
      }
      uint8_t* dst = cache + (s * (t_cap >> 6) + tile) * tbytes + toff;
      uint32_t v = *dst;
      for (int b = 0; b < 8; ++b) {
        int tt, j, cbit;
        vt_bit_source(bits, L, w, k, b, tt, j, cbit);
        const int64_t t = tile * 64 + tt - pos;
        if (t < 0 || t >= n) continue;
        v = (v & ~(1u << b)) | (((code(s, t, 64 * half + j) >> cbit) & 1u) << b);
      }
      *dst = (uint8_t)v;
    }
  }
}

// One new token per stream quantized and written straight into the decode layout (key
// pair bytes, the token's bits of its value tile, both norms): a decode step's cache
// append in one launch instead of a quantize and a layout pass for each of K and V.
// Arithmetic of quantize_rows_kernel (bf16 / fp16 inputs, rounded in that type), so codes
// and norms equal tq_rotate_and_quantize followed by tq_pack_decode_layout bit for bit.
// One wave per (stream, K or V) row; R_k and R_v, rounded and transposed, in LDS.  A
// stream's token is the only writer of its bits in this launch: every value-tile byte is
// read, merged and written by one lane (3-bit tiles: the lane of dims 16 i + c also
// places dim 48 + c's bits that share its bytes).
struct AppendArgs {
  const void* key;    // [n_streams][D]
  const void* value;  // [n_streams][D]
  int in_dt;          // TQ_BF16 or TQ_F16 (also the rounding type)
  int64_t n_streams;
  const float* krot;  // [D][D]
  const float* kbnd;  // 15
  const float* vrot;
  const float* vbnd;  // 2^VB - 1
  uint8_t* kpairs;    // [n_streams][t_cap][D / 2]
  void* knorms;       // [n_streams][t_cap], norm_dt
  uint8_t* vtiles;    // [n_streams][t_cap / 64][512 VB (D / 64)]
  void* vnorms;
  int norm_dt;
  int64_t t_cap, pos;
};

constexpr int kApThreads = 256;

template <int D, int VB>
__global__ __launch_bounds__(kApThreads) void dl_append_kernel(AppendArgs a) {
  constexpr int C = D / 64;  // dims per lane (lane + 64 c: half c of the head)
  __shared__ float rk_s[D][D + 1];
  __shared__ float rv_s[D][D + 1];
  __shared__ float u_s[kApThreads / 64][D];
  __shared__ float bk_s[16], bv_s[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rdt = a.in_dt;
  if (threadIdx.x < 15) bk_s[threadIdx.x] = round_to(a.kbnd[threadIdx.x], rdt);
  if (threadIdx.x < (1 << VB) - 1) bv_s[threadIdx.x] = round_to(a.vbnd[threadIdx.x], rdt);
  // R_k and R_v: float4 f = i * kApThreads + tid (coalesced), four at a time in flight,
  // stored rounded and transposed (row j = 4 f / D: the 64 lanes' writes hit 64 banks)
  constexpr int NF = D * D / 4 / kApThreads;  // float4 per thread and matrix
#pragma unroll
  for (int c0 = 0; c0 < NF; c0 += 4) {
    v4f rk4[4], rv4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      rk4[i] = reinterpret_cast<const v4f*>(a.krot)[(c0 + i) * kApThreads + threadIdx.x];
      rv4[i] = reinterpret_cast<const v4f*>(a.vrot)[(c0 + i) * kApThreads + threadIdx.x];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = (c0 + i) * kApThreads + threadIdx.x, j = 4 * f / D, k = 4 * f % D;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        rk_s[k + e][j] = round_to(rk4[i][e], rdt);
        rv_s[k + e][j] = round_to(rv4[i][e], rdt);
      }
    }
  }
  __syncthreads();
  const float eps = round_to(1e-10f, rdt);
  const int64_t tile = a.pos >> 6;
  const int tt = (int)(a.pos & 63);  // the token within its tile
  for (int64_t row = (int64_t)blockIdx.x * (kApThreads / 64) + wave; row < 2 * a.n_streams;
       row += (int64_t)gridDim.x * (kApThreads / 64)) {
    const bool val = row >= a.n_streams;  // uniform
    const int64_t s = val ? row - a.n_streams : row;
    float x[C];
#pragma unroll
    for (int c = 0; c < C; ++c) x[c] = load_as_f32(val ? a.value : a.key, s * D + lane + 64 * c, a.in_dt);
    // value rows: this lane's byte of the token's value tile per half (layout above
    // dl_pack_kernel / vt_bit_source), its old contents requested with the row
    const int sl = (tt >> 2) & 3, m = tt >> 4, j = lane, cc = j & 15, L = 16 * sl + cc;
    int off;
    if constexpr (VB == 2) {
      off = 16 * L + 4 * m + (j >> 4);
    } else {
      const int k = 2 * (m & 1) + ((tt >> 1) & 1), G = m >> 1;
      off = VB == 4 ? vt_byte_off(4, L, 4 * G + (j >> 4), k)
                    : vt_byte_off(3, L, 3 * G + ((j >> 4) < 3 ? (j >> 4) : 0), k);
    }
    uint8_t* tb = a.vtiles + (s * (a.t_cap >> 6) + tile) * (int64_t)(512 * VB * C);
    const bool vlane = val && (VB != 3 || j < 48);
    uint32_t old[C];
#pragma unroll
    for (int c = 0; c < C; ++c) old[c] = vlane ? tb[c * (512 * VB) + off] : 0u;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) ss = fmaf(x[c], x[c], ss);
    ss = wave_sum(ss);
    const float nrm = round_to(sqrtf(ss), rdt);
    const float den = fmaxf(nrm, eps);
#pragma unroll
    for (int c = 0; c < C; ++c) u_s[wave][lane + 64 * c] = round_to(x[c] / den, rdt);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float acc[C];
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = 0.f;
    if (!val) {
#pragma unroll 8
      for (int k = 0; k < D; ++k) {
        const float uk = u_s[wave][k];
#pragma unroll
        for (int c = 0; c < C; ++c) acc[c] = fmaf(uk, rk_s[k][lane + 64 * c], acc[c]);
      }
    } else {
#pragma unroll 8
      for (int k = 0; k < D; ++k) {
        const float uk = u_s[wave][k];
#pragma unroll
        for (int c = 0; c < C; ++c) acc[c] = fmaf(uk, rv_s[k][lane + 64 * c], acc[c]);
      }
    }
    uint32_t code[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
      code[c] = (uint32_t)count_below(val ? bv_s : bk_s, val ? 1 << VB : 16, round_to(acc[c], rdt));
    const int64_t slot = s * a.t_cap + a.pos;
    if (lane == 0) store_from_f32(val ? a.vnorms : a.knorms, slot, nrm, a.norm_dt);
    if (!val) {
      // key pair bytes: byte p of half c = code[2p] << 4 | code[2p + 1]
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const uint32_t nx = (uint32_t)__shfl_down((int)code[c], 1);
        if ((lane & 1) == 0) a.kpairs[slot * (D / 2) + 32 * c + (lane >> 1)] = (uint8_t)((code[c] << 4) | nx);
      }
    } else {
      // token tt's bit fields of the tile bytes
      uint32_t code48[C];
#pragma unroll
      for (int c = 0; c < C; ++c) code48[c] = (uint32_t)__shfl((int)code[c], 48 + (lane & 15));
#pragma unroll
      for (int c = 0; c < C; ++c) {
        uint32_t mask, bits;
        if constexpr (VB == 2) {
          const int t2 = tt & 3;
          mask = 3u << (2 * t2);
          bits = code[c] << (2 * t2);
        } else {
          const int e = tt & 1;
          if constexpr (VB == 4) {
            mask = 15u << (4 * e);
            bits = code[c] << (4 * e);
          } else {
            // dims 16 i + c (i < 3): bits 3e .. 3e + 2 of word 3G + i; the same byte's bits
            // 6 and 7 hold bits q - 3e of dim 48 + c's code, q = 2i, 2i + 1
            const int i = j >> 4;
            mask = 7u << (3 * e);
            bits = code[c] << (3 * e);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int cb = 2 * i + h - 3 * e;
              if (cb >= 0 && cb < 3) {
                mask |= 1u << (6 + h);
                bits |= ((code48[c] >> cb) & 1u) << (6 + h);
              }
            }
          }
        }
        if (vlane) tb[c * (512 * VB) + off] = (uint8_t)((old[c] & ~mask) | bits);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // u_s is rewritten by the next row
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Decode layout -> bit-plane rows of tokens [t0, t0 + n): one thread per output byte.
__global__ void dl_unpack_kernel(const uint8_t* __restrict__ cache, int64_t n_streams,
                                 int64_t t_cap, int64_t t0, int64_t n, int d, int bits, int values,
                                 uint8_t* __restrict__ packed) {
  const int bpp = (d + 7) / 8;
  const int P = bits * bpp;
  const int64_t total = n_streams * n * P;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int byte = (int)(e % P);
    const int64_t r = e / P, s = r / n, t = t0 + (r - s * n);
    const int p = byte / bpp, o = byte - p * bpp;
    uint32_t out = 0;
    for (int k = 0; k < 8; ++k) {
      const int j = 8 * o + k;
      if (j >= d) break;
      uint32_t c;
      if (!values) {
        const uint8_t pb = cache[(s * t_cap + t) * (d / 2) + (j >> 1)];
        c = (j & 1) ? (pb & 15u) : (pb >> 4);
      } else if (bits == 2) {
        // tile of 64 tokens and d dims: 64-dim halves of 1024 bytes, dims 64 h + .. in half h
        const int blk = (int)((t >> 2) & 15);  // block within the 64-token tile = 4 m + sl
        const int jh = j & 63;
        const int64_t at = (s * (t_cap >> 6) + (t >> 6)) * (1024 * (d / 64)) + (j >> 6) * 1024 +
                           ((blk & 3) * 16 + (jh & 15)) * 16 + (blk >> 2) * 4 + (jh >> 4);
        c = (cache[at] >> (2 * (t & 3))) & 3u;
      } else {
        const int tt = (int)(t & 63), blk = tt >> 2, m = blk >> 2, sl = blk & 3;
        const int G = m >> 1, kb = 2 * (m & 1) + ((tt >> 1) & 1), eo = tt & 1;
        const int L = 16 * sl + (j & 15), dg = (j & 63) >> 4;
        const uint8_t* tile = cache + (s * (t_cap >> 6) + (t >> 6)) * (512 * bits * (d / 64)) +
                              (j >> 6) * (512 * bits);
        if (bits == 4) {
          c = (tile[vt_byte_off(4, L, 4 * G + dg, kb)] >> (4 * eo)) & 15u;
        } else if (dg < 3) {
          c = (tile[vt_byte_off(3, L, 3 * G + dg, kb)] >> (3 * eo)) & 7u;
        } else {
          uint32_t idx = 0;
          for (int i = 0; i < 3; ++i)
            idx |= (uint32_t)((tile[vt_byte_off(3, L, 3 * G + i, kb)] >> 6) & 3) << (2 * i);
          c = (idx >> (3 * eo)) & 7u;
        }
      }
      out |= ((c >> p) & 1u) << (7 - k);
    }
    packed[e] = (uint8_t)out;
  }
}

struct SplitPlan {
  int64_t split_tokens;
  int nsplit;
};

SplitPlan plan_splits(int B, int hkv, int64_t t_max) {
  // about two workgroups per CU in one round (two fit in LDS and registers)
  const int64_t streams = (int64_t)B * hkv;
  const int64_t want = std::max<int64_t>(1, (2 * (int64_t)device_cu_count() + streams - 1) / streams);
  int64_t split = (t_max + want - 1) / want;
  split = std::max<int64_t>(kMinSplit, (split + kMinSplit - 1) / kMinSplit * kMinSplit);
  return {split, (int)((t_max + split - 1) / split)};
}

template <int KB, int PG = 0>
int launch_kb(int vb, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  if (vb == 1) hipLaunchKernelGGL((fused_decode_kernel<KB, 1, PG>), grid, dim3(kDecThreads), 0, st, a);
  else hipLaunchKernelGGL((fused_decode_kernel<KB, 2, PG>), grid, dim3(kDecThreads), 0, st, a);
  TQ_LAUNCH_CHECK("fused_decode_kernel");
  return TQ_OK;
}

}  // namespace

bool fused_decode_covers(const FusedDecodeCall& c) {
  if (c.d != kDim || c.kbits < 1 || c.kbits > 4 || c.vbits < 1 || c.vbits > 2) return false;
  if (c.hkv < 1 || c.hq % c.hkv != 0 || c.hq / c.hkv > 4) return false;
  if (c.q_dt != TQ_F16 && c.q_dt != TQ_BF16) return false;
  if (c.t_max <= 0 || (int64_t)c.B * c.hkv > 65535) return false;
  if (c.t_max * c.kbits * 8 >= (int64_t)INT_MAX) return false;  // 32-bit buffer offsets
  const uintptr_t ka = reinterpret_cast<uintptr_t>(c.kpacked);
  const uintptr_t va = reinterpret_cast<uintptr_t>(c.vpacked);
  if ((ka & ((c.kbits * 8) % 16 == 0 ? 15u : 7u)) || (va & ((c.vbits * 8) % 16 == 0 ? 15u : 7u)))
    return false;
  if (reinterpret_cast<uintptr_t>(c.krot) & 15u) return false;
  return true;
}

size_t fused_decode_workspace_bytes(int B, int hq, int d, int64_t t_max) {
  if (B <= 0 || hq <= 0 || t_max <= 0) return 256;
  (void)d;
  const int hkv = 1;  // the most splits any kv-head count can ask for
  const SplitPlan p = plan_splits(B, hkv, t_max);
  const size_t rows = (size_t)B * hq;
  return 256 + align_up(rows * p.nsplit * kDim * 4, 256) + align_up(rows * p.nsplit * 8, 256);
}

int launch_fused_decode(const FusedDecodeCall& c, void* workspace, size_t workspace_bytes,
                        hipStream_t st, const PagedPools* pg) {
  const SplitPlan p = plan_splits(c.B, c.hkv, c.t_max);
  const size_t rows = (size_t)c.B * c.hq;
  const size_t part_bytes = align_up(rows * p.nsplit * kDim * 4, 256);
  const size_t need = 256 + part_bytes + align_up(rows * p.nsplit * 8, 256);
  TQ_REQUIRE(workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  char* ws = static_cast<char*>(workspace) + 256;
  DecodeArgs a{};
  a.q = c.q; a.q_dt = c.q_dt; a.hq = c.hq; a.hkv = c.hkv; a.G = c.hq / c.hkv;
  a.kpacked = c.kpacked; a.knorms = c.knorms; a.vpacked = c.vpacked; a.vnorms = c.vnorms;
  a.t_max = c.t_max; a.seq_lens = c.seq_lens; a.kcen = c.kcen; a.vcen = c.vcen; a.krot = c.krot;
  a.qscale = c.scale * 1.4426950408889634f;
  a.split_tokens = p.split_tokens; a.nsplit = p.nsplit;
  a.part = reinterpret_cast<float*>(ws);
  a.stats = reinterpret_cast<float2*>(ws + part_bytes);
  const dim3 grid((unsigned)p.nsplit, (unsigned)(c.B * c.hkv));
  int rc = TQ_OK;
  if (pg) {
    a.block_tables = pg->block_tables; a.bt_stride = pg->bt_stride; a.bs_log2 = pg->bs_log2;
    a.pool_rows = pg->pool_rows;
    a.num_blocks = pg->num_blocks;
    if (!pg->wide) {
      switch (c.kbits) {
        case 1: rc = launch_kb<1, 1>(c.vbits, grid, a, st); break;
        case 2: rc = launch_kb<2, 1>(c.vbits, grid, a, st); break;
        case 3: rc = launch_kb<3, 1>(c.vbits, grid, a, st); break;
        default: rc = launch_kb<4, 1>(c.vbits, grid, a, st); break;
      }
    } else {
      switch (c.kbits) {
        case 1: rc = launch_kb<1, 2>(c.vbits, grid, a, st); break;
        case 2: rc = launch_kb<2, 2>(c.vbits, grid, a, st); break;
        case 3: rc = launch_kb<3, 2>(c.vbits, grid, a, st); break;
        default: rc = launch_kb<4, 2>(c.vbits, grid, a, st); break;
      }
    }
  } else {
    switch (c.kbits) {
      case 1: rc = launch_kb<1>(c.vbits, grid, a, st); break;
      case 2: rc = launch_kb<2>(c.vbits, grid, a, st); break;
      case 3: rc = launch_kb<3>(c.vbits, grid, a, st); break;
      default: rc = launch_kb<4>(c.vbits, grid, a, st); break;
    }
  }
  if (rc != TQ_OK) return rc;
  hipLaunchKernelGGL(fused_combine_kernel<kDim>, dim3((unsigned)rows), dim3(kDim), 0, st, a.part,
                     a.stats, p.nsplit, p.split_tokens, c.seq_lens, c.t_max, c.hq, c.vrot,
                     c.q_dt, c.out, c.lse);
  TQ_LAUNCH_CHECK("fused_combine_kernel");
  return TQ_OK;
}

}  // namespace tq

// ------------------------------------------------------------------ paged value tiles
namespace tq {
namespace {

// New tokens' VB-bit value codes (bit-plane rows [n][hkv][8 VB], d = 64: plane p at bytes
// 8p .. 8p + 7) into the value tiles of a paged pool, one thread per (token, head, dim).
// With tt the token's offset in its 64-token tile (block_size >= 64) or 16-token sub-block
// (below), sl = (tt % 16) / 4, r = tt % 4, m = tt / 16, L = 16 sl + dim % 16, dg = dim / 16,
// the code goes where the decode kernel reads it:
//   VB 2  tile byte 16 L + 4 m + dg, sub-block byte 4 L + dg; bits 2 r
//   VB 4  byte 2 (m % 2) + r / 2 of tile word 4 (m / 2) + dg, sub-block byte
//         8 L + 2 dg + r / 2; bits 4 (r % 2)
//   VB 3  dims below 48: byte 2 (m % 2) + r / 2 of tile word 3 (m / 2) + dg (sub-block
//         byte 4 L + 2 dg + r / 2 for dg 0, 1, 256 + 2 L + r / 2 for dg 2), bits 3 (r % 2);
//         dims 48-63: code bit b is bit q = 3 (r % 2) + b of the pair index, at bit
//         6 + q % 2 of the same byte position of word (or sub-block share) q / 2
// Tokens of one tile share bytes, so each field is cleared and set with 32-bit atomics
// (disjoint bits: concurrent tokens do not interfere); slots outside the pool are skipped.
__global__ __launch_bounds__(256) void paged_vtile_store_kernel(
    const uint8_t* __restrict__ rows, const float* __restrict__ norms, int64_t n, int hkv,
    const int64_t* __restrict__ slot_mapping, uint32_t* __restrict__ vpool,
    float* __restrict__ vnorm_pool, int64_t num_slots, int bs_log2, int vb) {
  const int64_t total = n * hkv * kDim;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int j = (int)(e & (kDim - 1));
    const int64_t th = e >> 6;  // (token, head)
    const int64_t tok = th / hkv;
    const int h = (int)(th - tok * hkv);
    const int64_t slot = slot_mapping[tok];
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t blk = slot >> bs_log2;
    const int off = (int)(slot & ((1 << bs_log2) - 1));
    const uint8_t* row = rows + th * 8 * vb;
    uint32_t code = 0;
    for (int p = 0; p < vb; ++p) code |= ((row[8 * p + (j >> 3)] >> (7 - (j & 7))) & 1u) << p;
    const bool tiles = bs_log2 >= 6;
    const int tt = off & (tiles ? 63 : 15);
    const int sl = (tt >> 2) & 3, r = tt & 3, m = tt >> 4, c = j & 15, L = 16 * sl + c;
    // byte base of the token's tile (64-token tiles of 512 VB bytes) or sub-block (128 VB)
    const int64_t base = tiles ? ((((blk * hkv + h) << (bs_log2 - 6)) + (off >> 6)) * 512 * vb)
                               : (((((blk * hkv + h) << bs_log2) + off) >> 4) * 128 * vb);
    auto put = [&](int byte, int bit, uint32_t mask, uint32_t val) {
      const int64_t at = base + byte;  // base is a multiple of 4
      uint32_t* w = vpool + (at >> 2);
      const int sh = 8 * (int)(at & 3) + bit;
      atomicAnd(w, ~(mask << sh));
      atomicOr(w, val << sh);
    };
    // byte of tile word / sub-block share i (dim group or word index) for this token
    auto byte_of = [&](int i) -> int {
      if (tiles) return vt_byte_off(vb, L, (vb == 4 ? 4 : 3) * (m >> 1) + i, 2 * (m & 1) + (r >> 1));
      if (vb == 4) return 8 * L + 2 * i + (r >> 1);
      return i < 2 ? 4 * L + 2 * i + (r >> 1) : 256 + 2 * L + (r >> 1);
    };
    if (vb == 2) {
      put(tiles ? 16 * L + 4 * m + (j >> 4) : 4 * L + (j >> 4), 2 * r, 3u, code);
    } else if (vb == 4) {
      put(byte_of(j >> 4), 4 * (r & 1), 15u, code);
    } else if (j < 48) {
      put(byte_of(j >> 4), 3 * (r & 1), 7u, code);
    } else {
      for (int b = 0; b < 3; ++b) {
        const int q = 3 * (r & 1) + b;
        put(byte_of(q >> 1), 6 + (q & 1), 1u, (code >> b) & 1u);
      }
    }
    if (j == 0) vnorm_pool[((blk * hkv + h) << bs_log2) + off] = norms[th];
  }
}

}  // namespace
}  // namespace tq

// ------------------------------------------------------------------ decode-layout C ABI
namespace tq {
namespace {

SplitPlan plan_dl_splits(int B, int hkv, int64_t t_cap) {
  // one 512-thread workgroup per CU (132 KB of tables)
  const int64_t streams = (int64_t)B * hkv;
  const int64_t want = std::max<int64_t>(1, ((int64_t)device_cu_count() + streams - 1) / streams);
  int64_t split = (t_cap + want - 1) / want;
  split = std::max<int64_t>(kDlMinSplit, (split + kDlMinSplit - 1) / kDlMinSplit * kDlMinSplit);
  return {split, (int)((t_cap + split - 1) / split)};
}

template <int PG, int VB, int ND = 0, int NH = 1, int SPW = 1>
void launch_dl_kernel(tq_dtype q_dtype, unsigned grid, const DlArgs& a, hipStream_t st) {
  if (q_dtype == TQ_F32)
    hipLaunchKernelGGL((dl_decode_kernel<true, true, PG, VB, ND, NH, SPW>), dim3(grid), dim3(kDlThreads), 0, st, a);
  else if (q_dtype == TQ_F16)
    hipLaunchKernelGGL((dl_decode_kernel<false, true, PG, VB, ND, NH, SPW>), dim3(grid), dim3(kDlThreads), 0, st, a);
  else
    hipLaunchKernelGGL((dl_decode_kernel<false, false, PG, VB, ND, NH, SPW>), dim3(grid), dim3(kDlThreads), 0, st, a);
}

template <int ND, int NH, int SPW>
void launch_dl_contiguous(int vbits, tq_dtype q_dtype, unsigned grid, const DlArgs& a, hipStream_t st) {
  if (vbits == 2) launch_dl_kernel<0, 2, ND, NH, SPW>(q_dtype, grid, a, st);
  else if (vbits == 3) launch_dl_kernel<0, 3, ND, NH, SPW>(q_dtype, grid, a, st);
  else launch_dl_kernel<0, 4, ND, NH, SPW>(q_dtype, grid, a, st);
}

template <int NH, int SPW = 1>
void launch_dl_norms(int norm_dt, int vbits, tq_dtype q_dtype, unsigned grid, const DlArgs& a,
                     hipStream_t st) {
  if (norm_dt == TQ_BF16) launch_dl_contiguous<TQ_BF16, NH, SPW>(vbits, q_dtype, grid, a, st);
  else if (norm_dt == TQ_F16) launch_dl_contiguous<TQ_F16, NH, SPW>(vbits, q_dtype, grid, a, st);
  else launch_dl_contiguous<0, NH, SPW>(vbits, q_dtype, grid, a, st);
}

template <int PG>
void launch_dl_paged(int vbits, tq_dtype q_dtype, unsigned grid, const DlArgs& a, hipStream_t st) {
  if (vbits == 2) launch_dl_kernel<PG, 2>(q_dtype, grid, a, st);
  else if (vbits == 3) launch_dl_kernel<PG, 3>(q_dtype, grid, a, st);
  else launch_dl_kernel<PG, 4>(q_dtype, grid, a, st);
}

// The exact current token merged into a decode output by log-sum-exp (the HF cache's
// rule that the token being decoded attends to its own unquantized key and value,
// hf_integration.py:372-390): one wave per query head h of batch row b, KV head
// h / (hq / hkv).  s = (q . k_new) * scale; m = max(lse, s); out = (o e^(lse - m) +
// v_new e^(s - m)) / (e^(lse - m) + e^(s - m)), in fp32, stored in the query's type.  `out`
// may be `o` (each element is read and then written by the same lane).
__global__ __launch_bounds__(64) void merge_token_kernel(const void* o, const float* __restrict__ lse,
                                                         const void* __restrict__ q,
                                                         const void* __restrict__ knew,
                                                         const void* __restrict__ vnew, int hq,
                                                         int hkv, int d, float scale, int q_dt,
                                                         int kv_dt, void* out) {
  const int64_t row = blockIdx.x;
  const int64_t b = row / hq;
  const int h = (int)(row - b * hq);
  const int64_t kvrow = b * hkv + h / (hq / hkv);
  const int lane = threadIdx.x;
  float dot = 0.f;
  for (int j = lane; j < d; j += 64)
    dot = fmaf(load_as_f32(q, row * d + j, q_dt), load_as_f32(knew, kvrow * d + j, kv_dt), dot);
  dot = wave_sum(dot);
  const float sn = dot * scale;
  const float lh = lse[row];
  const float m = fmaxf(lh, sn);
  const float wh = expf(lh - m), wn = expf(sn - m), den = wh + wn;
  for (int j = lane; j < d; j += 64) {
    const float x = load_as_f32(o, row * d + j, q_dt) * wh + load_as_f32(vnew, kvrow * d + j, kv_dt) * wn;
    store_from_f32(out, row * d + j, x / den, q_dt);
  }
}

// The decode-layout kernel over every (stream, split), in launches of at most four query
// heads per KV head, then (several splits) the log-sum-exp combine.  `a` carries
// everything but the split plan, the head range and the outputs.  d: head_dim (64, or 128
// for contiguous caches).
int run_dl(DlArgs a, tq_dtype q_dtype, int B, int hq, int hkv, int vbits, int pg,
           const SplitPlan& p, void* workspace, void* out, float* lse, hipStream_t st,
           int norm_dt = TQ_F32, int d = kDim) {
  const size_t rows = (size_t)B * hq;
  char* ws = static_cast<char*>(workspace) + 256;
  float* part = reinterpret_cast<float*>(ws);
  float2* stats = reinterpret_cast<float2*>(ws + align_up(rows * p.nsplit * kDlMaxDim * 4, 256));
  const bool single = p.nsplit == 1;
  if (a.t_cap > 0) {
    a.q_dt = (int)q_dtype; a.hq = hq; a.hkv = hkv;
    a.split_tokens = p.split_tokens; a.nsplit = p.nsplit; a.part = part; a.stats = stats;
    a.out = single ? out : nullptr; a.lse = single ? lse : nullptr;
    a.Gfull = hq / hkv;
    a.nstreams = B * hkv;
    // At least two streams per CU (one split each): two streams per workgroup, four waves
    // each, so the tables, R_k and R_v are built once for both and every stream is
    // resident at once (one workgroup per CU: a second round of workgroups would pay the
    // prologue again).
    const bool two = pg == 0 && d == kDim && p.nsplit == 1 &&
                     (int64_t)B * hkv >= 2 * (int64_t)device_cu_count();
    const uint64_t grid = two ? ((uint64_t)B * hkv + 1) / 2
                              : (uint64_t)p.nsplit * (uint64_t)B * (uint64_t)hkv;
    TQ_REQUIRE(grid <= 0xFFFFFFFFull, "too many (stream, split) workgroups");
    for (int h0 = 0; h0 < a.Gfull; h0 += 4) {
      a.hofs = h0;
      a.G = std::min(4, a.Gfull - h0);
      if (pg == 0) {
        if (d == 128) launch_dl_norms<2>(norm_dt, vbits, q_dtype, (unsigned)grid, a, st);
        else if (two) launch_dl_norms<1, 2>(norm_dt, vbits, q_dtype, (unsigned)grid, a, st);
        else launch_dl_norms<1>(norm_dt, vbits, q_dtype, (unsigned)grid, a, st);
      } else if (pg == 1) {
        launch_dl_paged<1>(vbits, q_dtype, (unsigned)grid, a, st);
      } else if (pg == 3) {
        launch_dl_paged<3>(vbits, q_dtype, (unsigned)grid, a, st);
      } else if (pg == 4) {
        launch_dl_paged<4>(vbits, q_dtype, (unsigned)grid, a, st);
      } else {
        launch_dl_paged<2>(vbits, q_dtype, (unsigned)grid, a, st);
      }
      TQ_LAUNCH_CHECK("dl_decode_kernel");
    }
    if (single) return TQ_OK;
  }
  if (d == 128)
    hipLaunchKernelGGL(fused_combine_kernel<128>, dim3((unsigned)rows), dim3(128), 0, st, part, stats,
                       p.nsplit, p.split_tokens, a.seq_lens, a.t_cap, hq, a.vrot, (int)q_dtype, out,
                       lse);
  else
    hipLaunchKernelGGL(fused_combine_kernel<kDim>, dim3((unsigned)rows), dim3(kDim), 0, st, part, stats,
                       p.nsplit, p.split_tokens, a.seq_lens, a.t_cap, hq, a.vrot, (int)q_dtype, out,
                       lse);
  TQ_LAUNCH_CHECK("fused_combine_kernel");
  return TQ_OK;
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

size_t tq_decode_dl_workspace_bytes(int32_t B, int32_t hq, int32_t hkv, int64_t t_cap) {
  if (B <= 0 || hq <= 0 || hkv <= 0 || t_cap <= 0) return 256;
  const SplitPlan p = plan_dl_splits(B, hkv, t_cap);
  const size_t rows = (size_t)B * hq;
  // partial outputs sized for head_dim up to 128
  return 256 + align_up(rows * p.nsplit * kDlMaxDim * 4, 256) + align_up(rows * p.nsplit * 8, 256);
}

int tq_decode_attention_dl_window(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq,
                                  int32_t hkv, int32_t d, const uint8_t* kpairs,
                                  const void* knorms, const uint8_t* vblocks,
                                  const void* vnorms, tq_dtype norm_dtype, int64_t t_cap,
                                  const int32_t* seq_lens,
                                  const int32_t* seq_starts, const float* kcentroids,
                                  const float* vcentroids, const float* krotation,
                                  const float* vrotation, int32_t kbits, int32_t vbits,
                                  float scale, void* out, float* lse, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(valid_dtype(q_dtype) && valid_dtype(norm_dtype), "unknown dtype");
  if ((d != 64 && d != 128) || kbits != 4 || vbits < 2 || vbits > 4)
    return fail(TQ_EUNSUPPORTED, "decode layout covers head_dim 64 and 128 with 4-bit keys and "
                                 "2-4 bit values, got d=%d kbits=%d vbits=%d", d, kbits, vbits);
  TQ_REQUIRE(B >= 0 && hkv >= 1 && hq >= hkv && hq % hkv == 0,
             "num_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  TQ_REQUIRE(t_cap >= 0 && t_cap % 64 == 0, "capacity must be a multiple of 64, got %lld",
             (long long)t_cap);
  TQ_REQUIRE(t_cap * (d / 2) < (int64_t)INT_MAX, "capacity too large for 32-bit offsets");
  if (B == 0) return TQ_OK;
  TQ_REQUIRE(q && out && seq_lens && kcentroids && vcentroids && krotation && vrotation,
             "null pointer argument");
  TQ_REQUIRE(t_cap == 0 || (kpairs && knorms && vblocks && vnorms), "null pointer argument");
  TQ_REQUIRE(((reinterpret_cast<uintptr_t>(krotation) | reinterpret_cast<uintptr_t>(vrotation)) & 15u) == 0,
             "rotations must be 16-byte aligned");
  TQ_REQUIRE(t_cap == 0 || ((reinterpret_cast<uintptr_t>(kpairs) | reinterpret_cast<uintptr_t>(vblocks) |
                             reinterpret_cast<uintptr_t>(knorms) | reinterpret_cast<uintptr_t>(vnorms)) &
                            15u) == 0,
             "decode-layout K/V and norms must be 16-byte aligned");
  const size_t need = tq_decode_dl_workspace_bytes(B, hq, hkv, t_cap);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  const SplitPlan p = t_cap > 0 ? plan_dl_splits(B, hkv, t_cap) : SplitPlan{kDlMinSplit, 1};
  DlArgs a{};
  a.q = q; a.kpairs = kpairs; a.knorms = static_cast<const float*>(knorms); a.vblocks = vblocks;
  a.vnorms = static_cast<const float*>(vnorms); a.t_cap = t_cap; a.seq_lens = seq_lens;
  a.seq_starts = seq_starts; a.kcen = kcentroids; a.vcen = vcentroids; a.krot = krotation;
  a.vrot = vrotation; a.qscale = scale * 1.4426950408889634f;
  return run_dl(a, q_dtype, B, hq, hkv, vbits, 0, p, workspace, out, lse, as_stream(stream),
                (int)norm_dtype, d);
}

int tq_decode_attention_dl(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                           int32_t d, const uint8_t* kpairs, const float* knorms,
                           const uint8_t* vblocks, const float* vnorms, int64_t t_cap,
                           const int32_t* seq_lens, const float* kcentroids,
                           const float* vcentroids, const float* krotation,
                           const float* vrotation, int32_t kbits, int32_t vbits, float scale,
                           void* out, float* lse, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return tq_decode_attention_dl_window(q, q_dtype, B, hq, hkv, d, kpairs, knorms, vblocks, vnorms,
                                       TQ_F32, t_cap, seq_lens, nullptr, kcentroids, vcentroids, krotation,
                                       vrotation, kbits, vbits, scale, out, lse, workspace,
                                       workspace_bytes, stream);
}

int tq_paged_store_value_tiles(const uint8_t* rows, const float* norms, int64_t n_tokens,
                               int32_t hkv, const int64_t* slot_mapping, uint8_t* vpool,
                               float* vnorm_pool, int64_t num_blocks, int32_t block_size,
                               int32_t vbits, void* stream) {
  TQ_REQUIRE(n_tokens >= 0 && hkv >= 1 && num_blocks >= 0, "bad sizes");
  TQ_REQUIRE(vbits >= 2 && vbits <= 4, "value tiles hold 2-4 bit codes, got %d", vbits);
  int bsl = 0;
  while ((1 << bsl) < block_size) ++bsl;
  TQ_REQUIRE(block_size >= 16 && (1 << bsl) == block_size,
             "value tiles need a power-of-two block_size >= 16, got %d", block_size);
  if (n_tokens == 0) return TQ_OK;
  TQ_REQUIRE(rows && norms && slot_mapping && vpool && vnorm_pool, "null pointer argument");
  TQ_REQUIRE((reinterpret_cast<uintptr_t>(vpool) & 3u) == 0, "value pool must be 4-byte aligned");
  const int64_t total = n_tokens * hkv * kDim;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(paged_vtile_store_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     rows, norms, n_tokens, (int)hkv, slot_mapping, reinterpret_cast<uint32_t*>(vpool),
                     vnorm_pool, num_blocks << bsl, bsl, (int)vbits);
  TQ_LAUNCH_CHECK("paged_vtile_store_kernel");
  return TQ_OK;
}

int tq_decode_attention_paged_dl(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                                 int32_t d, const uint8_t* kpairs_pool, const float* knorm_pool,
                                 const uint8_t* vtile_pool, const float* vnorm_pool,
                                 int64_t num_blocks, int32_t block_size, int32_t vbits,
                                 const int32_t* block_tables, int32_t max_blocks_per_seq,
                                 const int32_t* seq_lens, const float* kcentroids,
                                 const float* vcentroids, const float* krotation,
                                 const float* vrotation, float scale, void* out, float* lse,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(valid_dtype(q_dtype), "unknown dtype");
  TQ_REQUIRE(d == kDim, "decode layout covers head_dim 64, got %d", d);
  TQ_REQUIRE(vbits >= 2 && vbits <= 4, "value tiles hold 2-4 bit codes, got %d", vbits);
  TQ_REQUIRE(B >= 0 && hkv >= 1 && hq >= hkv && hq % hkv == 0,
             "num_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  int bsl = 0;
  while ((1 << bsl) < block_size) ++bsl;
  TQ_REQUIRE(block_size >= 16 && (1 << bsl) == block_size,
             "decode-layout pools need a power-of-two block_size >= 16, got %d", block_size);
  TQ_REQUIRE(num_blocks >= 0 && max_blocks_per_seq >= 0, "bad sizes");
  const int64_t t_cap = (int64_t)max_blocks_per_seq * block_size;
  const int64_t pool_rows = num_blocks * hkv * block_size;
  TQ_REQUIRE(pool_rows < ((int64_t)1 << 32), "pools hold at most 2^32 rows per layer");
  // pools from 2 GiB of key rows on: 64-bit addresses (the buffer path's offsets are 32-bit)
  const bool wide = pool_rows * 32 >= (int64_t)INT_MAX;
  if (B == 0) return TQ_OK;
  TQ_REQUIRE(q && out && seq_lens && kcentroids && vcentroids && krotation && vrotation,
             "null pointer argument");
  TQ_REQUIRE(t_cap == 0 || (kpairs_pool && knorm_pool && vtile_pool && vnorm_pool && block_tables),
             "null pointer argument");
  TQ_REQUIRE(((reinterpret_cast<uintptr_t>(krotation) | reinterpret_cast<uintptr_t>(vrotation)) & 15u) == 0,
             "rotations must be 16-byte aligned");
  TQ_REQUIRE(t_cap == 0 || ((reinterpret_cast<uintptr_t>(kpairs_pool) | reinterpret_cast<uintptr_t>(vtile_pool) |
                             reinterpret_cast<uintptr_t>(knorm_pool) | reinterpret_cast<uintptr_t>(vnorm_pool)) &
                            15u) == 0,
             "decode-layout pools must be 16-byte aligned");
  const size_t need = tq_decode_dl_workspace_bytes(B, hq, hkv, t_cap);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  const SplitPlan p = t_cap > 0 ? plan_dl_splits(B, hkv, t_cap) : SplitPlan{kDlMinSplit, 1};
  DlArgs a{};
  a.q = q; a.kpairs = kpairs_pool; a.knorms = knorm_pool; a.vblocks = vtile_pool;
  a.vnorms = vnorm_pool; a.t_cap = t_cap; a.seq_lens = seq_lens; a.kcen = kcentroids;
  a.vcen = vcentroids; a.krot = krotation; a.vrot = vrotation;
  a.qscale = scale * 1.4426950408889634f;
  a.block_tables = block_tables; a.bt_stride = max_blocks_per_seq; a.bs_log2 = bsl;
  a.pool_rows = (uint32_t)pool_rows;
  a.num_blocks = (uint32_t)std::max<int64_t>(num_blocks, 1);
  const int pg = (bsl >= 6 ? 1 : 2) + (wide ? 2 : 0);
  return run_dl(a, q_dtype, B, hq, hkv, vbits, pg, p, workspace, out, lse, as_stream(stream));
}

int tq_decode_merge_token(const void* o, const float* lse, const void* q, tq_dtype q_dtype,
                          const void* k_new, const void* v_new, tq_dtype kv_dtype, int32_t B,
                          int32_t hq, int32_t hkv, int32_t d, float scale, void* out, void* stream) {
  TQ_REQUIRE(valid_dtype(q_dtype) && valid_dtype(kv_dtype), "unknown dtype");
  TQ_REQUIRE(B >= 0 && hkv >= 1 && hq >= hkv && hq % hkv == 0,
             "num_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  TQ_REQUIRE(d >= 1 && d <= 4096, "head_dim must be in [1, 4096], got %d", d);
  const int64_t rows = (int64_t)B * hq;
  TQ_REQUIRE(rows <= 0x7FFFFFFFll, "too many query heads in one call");
  if (rows == 0) return TQ_OK;
  TQ_REQUIRE(o && lse && q && k_new && v_new && out, "null pointer argument");
  hipLaunchKernelGGL(merge_token_kernel, dim3((unsigned)rows), dim3(64), 0, as_stream(stream), o, lse, q,
                     k_new, v_new, (int)hq, (int)hkv, (int)d, scale, (int)q_dtype, (int)kv_dtype, out);
  TQ_LAUNCH_CHECK("merge_token_kernel");
  return TQ_OK;
}

int tq_pack_decode_layout(const uint8_t* packed, int64_t n_streams, int64_t n, int32_t d,
                          int32_t bit_width, int32_t values, uint8_t* cache, int64_t t_cap,
                          int64_t pos, void* stream) {
  TQ_REQUIRE(values == 0 || values == 1, "values must be 0 (keys) or 1 (values)");
  TQ_REQUIRE(d >= 2 && d <= 256 && d % 2 == 0, "dim must be even and at most 256, got %d", d);
  TQ_REQUIRE(values ? (bit_width >= 2 && bit_width <= 4) : bit_width == 4,
             "decode layout holds 4-bit keys and 2-4 bit values");
  TQ_REQUIRE(n_streams >= 0 && n >= 0 && pos >= 0 && pos + n <= t_cap, "bad token range");
  TQ_REQUIRE(!values || (t_cap % 64 == 0 && (d == 64 || d == 128)),
             "value tiles need dim 64 or 128 and a capacity that is a multiple of 64");
  if (n_streams == 0 || n == 0) return TQ_OK;
  TQ_REQUIRE(packed && cache, "null pointer argument");
  const int64_t per = values ? (((pos + n + 63) >> 6) - (pos >> 6)) * 512 * bit_width * (d / 64)
                             : n * (d / 2);
  const int64_t total = n_streams * per;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(dl_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), packed,
                     n_streams, n, d, bit_width, values, cache, t_cap, pos);
  TQ_LAUNCH_CHECK("dl_pack_kernel");
  return TQ_OK;
}

int tq_cache_append_dl(const void* key, const void* value, tq_dtype in_dtype, int64_t n_streams,
                       int32_t d, const float* krotation, const float* kboundaries,
                       const float* vrotation, const float* vboundaries, int32_t vbits,
                       uint8_t* kpairs, void* knorms, uint8_t* vtiles, void* vnorms,
                       tq_dtype norm_dtype, int64_t t_cap, int64_t pos, void* stream) {
  TQ_REQUIRE(in_dtype == TQ_BF16 || in_dtype == TQ_F16, "keys and values must be bf16 or fp16");
  TQ_REQUIRE(d == 64 || d == 128, "dim must be 64 or 128, got %d", d);
  TQ_REQUIRE(vbits >= 2 && vbits <= 4, "value bits must be 2-4, got %d", vbits);
  TQ_REQUIRE(norm_dtype == TQ_F32 || norm_dtype == TQ_BF16 || norm_dtype == TQ_F16, "unknown norm dtype");
  TQ_REQUIRE(n_streams >= 0 && t_cap >= 0 && t_cap % 64 == 0 && pos >= 0 && pos < t_cap,
             "bad position or capacity");
  if (n_streams == 0) return TQ_OK;
  TQ_REQUIRE(key && value && krotation && kboundaries && vrotation && vboundaries && kpairs &&
                 knorms && vtiles && vnorms,
             "null pointer argument");
  AppendArgs a{key, value, (int)in_dtype, n_streams, krotation, kboundaries, vrotation, vboundaries,
               kpairs, knorms, vtiles, vnorms, (int)norm_dtype, t_cap, pos};
  const int64_t want = (2 * n_streams + kApThreads / 64 - 1) / (kApThreads / 64);
  const int64_t cap = (int64_t)device_cu_count() * (d == 64 ? 4 : 1);  // LDS: 33 / 132 KB of R
  const dim3 grid((unsigned)std::min(want, cap));
  hipStream_t st = as_stream(stream);
  if (d == 64) {
    if (vbits == 2) hipLaunchKernelGGL((dl_append_kernel<64, 2>), grid, dim3(kApThreads), 0, st, a);
    else if (vbits == 3) hipLaunchKernelGGL((dl_append_kernel<64, 3>), grid, dim3(kApThreads), 0, st, a);
    else hipLaunchKernelGGL((dl_append_kernel<64, 4>), grid, dim3(kApThreads), 0, st, a);
  } else {
    if (vbits == 2) hipLaunchKernelGGL((dl_append_kernel<128, 2>), grid, dim3(kApThreads), 0, st, a);
    else if (vbits == 3) hipLaunchKernelGGL((dl_append_kernel<128, 3>), grid, dim3(kApThreads), 0, st, a);
    else hipLaunchKernelGGL((dl_append_kernel<128, 4>), grid, dim3(kApThreads), 0, st, a);
  }
  TQ_LAUNCH_CHECK("dl_append_kernel");
  return TQ_OK;
}

int tq_unpack_decode_layout(const uint8_t* cache, int64_t n_streams, int64_t t_cap, int64_t t0,
                            int64_t n, int32_t d, int32_t bit_width, int32_t values,
                            uint8_t* packed, void* stream) {
  TQ_REQUIRE(values == 0 || values == 1, "values must be 0 (keys) or 1 (values)");
  TQ_REQUIRE(d >= 2 && d <= 256 && d % 2 == 0, "dim must be even and at most 256, got %d", d);
  TQ_REQUIRE(values ? (bit_width >= 2 && bit_width <= 4) : bit_width == 4,
             "decode layout holds 4-bit keys and 2-4 bit values");
  TQ_REQUIRE(n_streams >= 0 && n >= 0 && t0 >= 0 && t0 + n <= t_cap, "bad token range");
  TQ_REQUIRE(!values || (t_cap % 64 == 0 && (d == 64 || d == 128)),
             "value tiles need dim 64 or 128 and a capacity that is a multiple of 64");
  if (n_streams == 0 || n == 0) return TQ_OK;
  TQ_REQUIRE(packed && cache, "null pointer argument");
  const int64_t total = n_streams * n * bit_width * ((d + 7) / 8);
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(dl_unpack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     cache, n_streams, t_cap, t0, n, d, bit_width, values, packed);
  TQ_LAUNCH_CHECK("dl_unpack_kernel");
  return TQ_OK;
}

}  // extern "C"
