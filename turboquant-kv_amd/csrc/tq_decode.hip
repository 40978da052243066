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
};

// Raw buffer resource over `bytes` bytes at `p` (gfx9 dword 3); loads past the end
// return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
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

template <int KB, int VB>
__global__ __launch_bounds__(kDecThreads, 2) void fused_decode_kernel(DecodeArgs a) {
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
  // Per-stream buffers cover exactly the split's valid tokens: rows and norms past
  // t_end read as zero (and are masked), so no load needs a clamp or a branch.
  const size_t sbase = (size_t)bg * (size_t)a.t_max;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.kpacked + sbase * PK, (uint32_t)t_end * PK);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(a.vpacked + sbase * PV, (uint32_t)t_end * PV);
  const __amdgpu_buffer_rsrc_t knrs = make_rsrc(a.knorms + sbase, (uint32_t)t_end * 4);
  const __amdgpu_buffer_rsrc_t vnrs = make_rsrc(a.vnorms + sbase, (uint32_t)t_end * 4);
  const int te = (int)t_end;

  struct Tile {
    uint32_t k[PK / 4];
    uint32_t v[PV / 4];
    float kn[4], vn[4];
  };
  auto load_tile = [&](int t0, Tile& x) {
    const uint32_t tr = (uint32_t)(t0 + lane);
    load_row<PK>(krs, tr * PK, x.k);
    load_row<PV>(vrs, tr * PV, x.v);
    const uint32_t no = (uint32_t)(t0 + 4 * quad) * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x.kn[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(knrs, (int)no, 4 * r, 0));
      x.vn[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vnrs, (int)no, 4 * r, 0));
    }
  };

  float M = -INFINITY;  // running max of this lane's head (same in all lanes of the head)
  float l = 0.f;        // this lane's share of sum 2^(s - M)
  v4f acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = (v4f){0.f, 0.f, 0.f, 0.f};

  int t0 = (int)t_begin + wave * 64;
  Tile cur, nxt;
  if (t0 < te) load_tile(t0, cur);
  while (t0 < te) {
    const int tn = t0 + kDecWaves * 64;
    load_tile(tn, nxt);

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
    float s[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = skk[r] * cur.kn[r];
    if (t0 + 64 > te) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (t0 + 4 * quad + r >= te) s[r] = -INFINITY;
    }
    const float lm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    if (__any(lm > M)) {
      float m2 = lm;
      m2 = fmaxf(m2, __shfl_xor(m2, 4));
      m2 = fmaxf(m2, __shfl_xor(m2, 8));
      m2 = fmaxf(m2, __shfl_xor(m2, 16));
      m2 = fmaxf(m2, __shfl_xor(m2, 32));
      const float mn = fmaxf(M, m2);
      const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mn);
      l *= f;
      const v4f fv = {__shfl(f, 0), __shfl(f, 1), __shfl(f, 2), __shfl(f, 3)};
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
      wa[r] = (_Float16)(p * cur.vn[r]);
    }
    l += psum;

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
    fw[m] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx[m]);
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

// One 64-thread block per query row: log-sum-exp merge of the splits, o = o_rot / L,
// out = o @ R_v; lse (natural log) = (max + log2 L) * ln 2.
__global__ __launch_bounds__(64) void fused_combine_kernel(const float* __restrict__ part,
                                                           const float2* __restrict__ stats,
                                                           int nsplit, int64_t split_tokens,
                                                           const int32_t* __restrict__ seq_lens,
                                                           int64_t t_max, int hq,
                                                           const float* __restrict__ vrot,
                                                           int out_dt, void* __restrict__ out,
                                                           float* __restrict__ lse) {
  __shared__ float o_s[kDim];
  const int64_t row = blockIdx.x;
  const int b = (int)(row / hq);
  const int j = threadIdx.x;
  const int64_t T = min((int64_t)max(seq_lens[b], 0), t_max);
  const int ns = (int)((T + split_tokens - 1) / split_tokens);
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, stats[row * nsplit + s].x);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < ns; ++s) {
    const float2 st = stats[row * nsplit + s];
    const float f = st.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.x - M);
    L += st.y * f;
    o += part[(row * nsplit + s) * kDim + j] * f;
  }
  const bool any = ns > 0 && L > 0.f;
  o_s[j] = any ? o / L : 0.f;
  __syncthreads();
  float r = 0.f;
#pragma unroll 8
  for (int k = 0; k < kDim; ++k) r = fmaf(o_s[k], vrot[k * kDim + j], r);
  store_from_f32(out, row * kDim + j, r, out_dt);
  if (lse && j == 0) lse[row] = any ? (M + log2f(L)) * 0.69314718055994531f : -INFINITY;
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

bool fused_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("TQ_DECODE_FUSED");
    return !(e && e[0] == '0');
  }();
  return on;
}

template <int KB>
int launch_kb(int vb, dim3 grid, const DecodeArgs& a, hipStream_t st) {
  if (vb == 1) hipLaunchKernelGGL((fused_decode_kernel<KB, 1>), grid, dim3(kDecThreads), 0, st, a);
  else hipLaunchKernelGGL((fused_decode_kernel<KB, 2>), grid, dim3(kDecThreads), 0, st, a);
  TQ_LAUNCH_CHECK("fused_decode_kernel");
  return TQ_OK;
}

}  // namespace

bool fused_decode_covers(const FusedDecodeCall& c) {
  if (!fused_enabled()) return false;
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
                        hipStream_t st) {
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
  switch (c.kbits) {
    case 1: rc = launch_kb<1>(c.vbits, grid, a, st); break;
    case 2: rc = launch_kb<2>(c.vbits, grid, a, st); break;
    case 3: rc = launch_kb<3>(c.vbits, grid, a, st); break;
    default: rc = launch_kb<4>(c.vbits, grid, a, st); break;
  }
  if (rc != TQ_OK) return rc;
  hipLaunchKernelGGL(fused_combine_kernel, dim3((unsigned)rows), dim3(kDim), 0, st, a.part,
                     a.stats, p.nsplit, p.split_tokens, c.seq_lens, c.t_max, c.hq, c.vrot,
                     c.q_dt, c.out, c.lse);
  TQ_LAUNCH_CHECK("fused_combine_kernel");
  return TQ_OK;
}

}  // namespace tq
