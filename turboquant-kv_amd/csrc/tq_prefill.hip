// tq_prefill.hip -- causal prefill attention over decode-layout paged pools on gfx950.
//
// Semantics: one sequence's n new tokens at positions T - n .. T - 1 attend causally to
// its first T tokens: new token i sees tokens 0 .. T - n + i (the mask of vLLM's prefill;
// the reference's backend attends over its dequantized cache, vllm_plugin/__init__.py:400
// with cache.py:282-339 for the scores and values).  score = scale * n_k <R_k q, c_k[code]>,
// softmax over the visible tokens, out = (sum_t w_t n_v,t c_v[code_t]) R_v.
//
// One workgroup of four waves per (64 NGR query rows, KV head h); query row r of h is
// query head h G + r % G of new token r / G.  Each wave owns NGR groups of 16 rows (three
// for bf16 queries, two otherwise) and streams the 64-token tiles its last row can see,
// once for all of them (the per-token decode launch reads the history once per row); each
// tile's key and value operands are looked up once and feed every group's MFMAs.  Online
// softmax in the log2 domain.  Per tile, wave and row group:
//   S^T = K Qrot^T  v_mfma_f32_16x16x32_f16, one 16-token group b per MFMA chain.  A: lane
//                   (c, g) = (lane % 16, lane / 16) holds token 16 b + c, dims 8 g .. 8 g + 7
//                   and 32 + 8 g .. : one 4-byte read of its pair bytes each, four pair-
//                   table lookups (c[hi], c[lo]) as fp16.  B: the rotated query (fp16 hi +
//                   lo parts); c.q = ch qh + ch ql + cl qh, accumulated in fp32.  Lane
//                   (c, g) gets tokens 16 b + 4 g + r of query row c.
//   softmax         per query row over the four lanes c, c + 16, c + 32, c + 48.
//   O^T += V^T P^T  A: value centroids of dim 16 nb + c for the 8 tokens lane (c, g) holds
//                   weights of -- the decode layout's value words of lane 16 g + c carry
//                   exactly those tokens' codes, so no data moves between lanes: 2-bit
//                   values, byte nb of words 2 s and 2 s + 1 (tokens 16 m + 4 g .. + 3,
//                   one lookup of four centroids each); 3- and 4-bit values, the four bytes
//                   of tile word (4 s + nb), or the dim-group word of half s (3 bits), one
//                   lookup of a (c[low code], c[high code]) pair each.  B: weights times
//                   value norms, the layout S^T left them in (hi + lo).
// Rotations in fp32 on v_mfma_f32_16x16x4f32: Qrot = q R_k^T (rows of R_k permuted so the
// result lands in the B layout above), out = O R_v.  Each row's query and the centroid
// tables are scaled by powers of two into [0.5, 1) before the fp16 split (exact), which
// the fp32 results undo.  Accuracy: fp32 and fp16 queries take hi + lo parts (the dropped
// lo x lo terms are 2^-22 relative: fp32-accurate scores and sums); bf16 queries one fp16
// product per term (2^-11 relative per operand, below the bf16 rounding of their outputs).
// Outputs fp32.
//
// Pools: rows at 64-bit addresses from block ids clamped into the pool (any pool size; a
// corrupt table reads the pool's last block, never memory outside it).  Tokens past a
// row's limit are masked by selects, so stale rows and norms (even NaN) contribute 0.

#include "tq_common.h"

#include <climits>
#include <type_traits>

namespace tq {
namespace {

constexpr int kPfThreads = 256;
constexpr int kPfRows = 64;  // query rows per workgroup and row group, 16 per wave

typedef float pf_v4f __attribute__((ext_vector_type(4)));
typedef _Float16 pf_v8h __attribute__((ext_vector_type(8)));
typedef uint32_t pf_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pf_u32x2 __attribute__((ext_vector_type(2)));

struct PfArgs {
  const void* q;  // [n][hq][64]
  int q_dt;
  int n, hq, hkv, G;
  int64_t past;  // T - n
  const uint8_t* kpairs;  // [num_blocks][hkv][bs][32]
  const float* knorms;    // [num_blocks][hkv][bs]
  const uint8_t* vtiles;  // [num_blocks][hkv][bs/64][512 VB] or [num_blocks][hkv][bs/16][128 VB]
  const float* vnorms;
  const int32_t* block_table;  // the sequence's row
  int max_blocks;
  int bs_log2;
  uint32_t num_blocks;
  const float* kcen;  // 16
  const float* vcen;  // 2^VB
  const float* krot;  // [64][64]
  const float* vrot;
  float qscale;  // softmax scale * log2(e)
  float* out;    // [n][hq][64]
};

__device__ __forceinline__ pf_v8h pf_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  pf_u32x4 t = {a, b, c, d};
  return __builtin_bit_cast(pf_v8h, t);
}

__device__ __forceinline__ uint32_t pf_pack(_Float16 lo, _Float16 hi) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, (h2_t){lo, hi});
}

// 2^-e with amax = m 2^e, m in [0.5, 1) (1 for 0, inf or NaN)
__device__ __forceinline__ float pf_pow2_scale(float amax) {
  int e = 0;
  if (amax > 0.f && amax < INFINITY) frexpf(amax, &e);
  return ldexpf(1.f, -e);
}

// SUB: value sub-blocks of 16 tokens (block_size 16 or 32), else 64-token value tiles.
// PREC: fp16 hi + lo parts of every operand (three products per term, fp32-accurate);
// otherwise one fp16 product per term (about 2^-11 relative per operand), for bf16 queries
// whose outputs are consumed in bf16 (2^-9).
// VB: value code width (2, 3 or 4); tiles and sub-blocks as the decode kernel reads them.
template <bool SUB, bool PREC, int VB>
__global__ __launch_bounds__(kPfThreads, 2) void dl_prefill_kernel(PfArgs a) {
#pragma clang fp contract(off)
  // Tables, KC / VC copies of each entry (lane L reads copy L % KC, L % VC, so a wave's
  // random lookups spread over the banks instead of piling onto a 1 KB table's):
  //   tk[p][i KC + j]  key byte i -> (c[i >> 4], c[i & 15]) as two fp16, part p (hi, lo)
  //   tv[p][i VC + j]  VB 2: value byte i -> its four 2-bit codes' centroids as four fp16;
  //                    VB 3, 4: (in tw, 2 VC copies) byte i -> (c[low code], c[high code])
  //                    as two fp16 (3 bits: the top two bits of i ignored)
  constexpr int KC = PREC ? 4 : 8, VC = PREC ? 2 : 4, NP = PREC ? 2 : 1;
  constexpr int WC = 2 * VC;  // copies of a VB 3 / 4 pair entry (the same 8 KB)
  constexpr int NGR = PREC ? 2 : 3;  // 16-row groups per wave (sharing each tile's operands)
  static_assert(VB >= 2 && VB <= 4, "value width");
  __shared__ __attribute__((aligned(16))) uint32_t tk[NP][256 * KC];
  __shared__ __attribute__((aligned(16))) pf_u32x2 tv[VB == 2 ? NP : 1][VB == 2 ? 256 * VC : 1];
  __shared__ __attribute__((aligned(16))) uint32_t tw[VB == 2 ? 1 : NP][VB == 2 ? 1 : 256 * WC];
  __shared__ float sc_s[2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int hkv = a.hkv;
  const int nG = a.n * a.G;
  const int nrt = (nG + kPfRows * NGR - 1) / (kPfRows * NGR);
  const int h = (int)(blockIdx.x % (unsigned)hkv);
  const int rt = nrt - 1 - (int)(blockIdx.x / (unsigned)hkv);  // longest rows first

  // ---- centroid tables scaled by powers of two, fp16 hi (+ lo)
  if (wave == 0) {
    float km = lane < 16 ? fabsf(a.kcen[lane]) : 0.f;
    float vm = lane < (1 << VB) ? fabsf(a.vcen[lane]) : 0.f;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      km = fmaxf(km, __shfl_xor(km, o, 64));
      vm = fmaxf(vm, __shfl_xor(vm, o, 64));
    }
    if (lane == 0) {
      sc_s[0] = pf_pow2_scale(km);
      sc_s[1] = pf_pow2_scale(vm);
    }
  }
  __syncthreads();
  const float ksc = sc_s[0], vsc = sc_s[1];
  {
    const int e = tid;  // one entry per thread
    const float c0 = a.kcen[e >> 4] * ksc, c1 = a.kcen[e & 15] * ksc;
    const _Float16 h0 = (_Float16)c0, h1 = (_Float16)c1;
    const uint32_t kh = pf_pack(h0, h1);
    const uint32_t kl = pf_pack((_Float16)(c0 - (float)h0), (_Float16)(c1 - (float)h1));
#pragma unroll
    for (int j = 0; j < KC; j += 4) {
      *reinterpret_cast<pf_u32x4*>(&tk[0][e * KC + j]) = (pf_u32x4){kh, kh, kh, kh};
      if constexpr (PREC) *reinterpret_cast<pf_u32x4*>(&tk[NP - 1][e * KC + j]) = (pf_u32x4){kl, kl, kl, kl};
    }
    if constexpr (VB == 2) {
      _Float16 vh[4], vl[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float v = a.vcen[(e >> (2 * t)) & 3] * vsc;
        vh[t] = (_Float16)v;
        vl[t] = (_Float16)(v - (float)vh[t]);
      }
      const uint32_t v0 = pf_pack(vh[0], vh[1]), v1 = pf_pack(vh[2], vh[3]);
      const uint32_t w0 = pf_pack(vl[0], vl[1]), w1 = pf_pack(vl[2], vl[3]);
#pragma unroll
      for (int j = 0; j < VC; j += 2) {
        *reinterpret_cast<pf_u32x4*>(&tv[0][e * VC + j]) = (pf_u32x4){v0, v1, v0, v1};
        if constexpr (PREC) *reinterpret_cast<pf_u32x4*>(&tv[NP - 1][e * VC + j]) = (pf_u32x4){w0, w1, w0, w1};
      }
    } else {
      constexpr int mask = (1 << VB) - 1;
      const float x0 = a.vcen[e & mask] * vsc, x1 = a.vcen[(e >> VB) & mask] * vsc;
      const _Float16 y0 = (_Float16)x0, y1 = (_Float16)x1;
      const uint32_t vhw = pf_pack(y0, y1);
      const uint32_t vlw = pf_pack((_Float16)(x0 - (float)y0), (_Float16)(x1 - (float)y1));
#pragma unroll
      for (int j = 0; j < WC; j += 4) {
        *reinterpret_cast<pf_u32x4*>(&tw[0][e * WC + j]) = (pf_u32x4){vhw, vhw, vhw, vhw};
        if constexpr (PREC) *reinterpret_cast<pf_u32x4*>(&tw[NP - 1][e * WC + j]) = (pf_u32x4){vlw, vlw, vlw, vlw};
      }
    }
  }
  const int kcp = lane & (KC - 1), vcp = lane & (VC - 1), wcp = lane & (WC - 1);
  __syncthreads();  // the last barrier: from here on every wave runs on its own

  // rows of this wave: group j holds rows row0 + 16 j + c
  const int row0 = rt * (kPfRows * NGR) + wave * (16 * NGR);
  if (row0 >= nG) return;
  int row[NGR];
  int64_t qoff[NGR], lim[NGR];
#pragma unroll
  for (int j = 0; j < NGR; ++j) {
    row[j] = row0 + 16 * j + c;
    const int rowc = row[j] < nG ? row[j] : nG - 1;
    const int ti = rowc / a.G;
    const int qh = h * a.G + (rowc - ti * a.G);
    qoff[j] = ((int64_t)ti * a.hq + qh) * 64;
    lim[j] = row[j] < nG ? a.past + ti + 1 : 0;  // tokens this row sees
  }
  const int64_t limw = a.past + (min(row0 + 16 * NGR - 1, nG - 1) / a.G) + 1;
  const int ntiles = (int)((limw + 63) >> 6);

  // ---- Qrot = (q * qscale) R_k^T.  MFMA mb, k-step s: lane (c, g) supplies A[c][g] =
  // R_k[pi(16 mb + c)][16 g + s] and B[g][c] = q_c[16 g + s] (the contraction runs over the
  // input dims in the order 16 g + s, so each lane reads 16 consecutive floats of a row);
  // register r of lane (c, g) gets Qrot_c[pi(16 mb + 4 g + r)] with
  // pi(16 mb + 4 g + r) = 32 (mb / 2) + 8 g + 4 (mb % 2) + r: dims 8 g + i and 32 + 8 g + i.
  pf_v8h qhi[NGR][2], qlo[NGR][2];
  float kinv[NGR];
  {
    float rk[4][16];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int dim = 32 * (mb >> 1) + 8 * (c >> 2) + 4 * (mb & 1) + (c & 3);
      const pf_v4f* src = reinterpret_cast<const pf_v4f*>(a.krot + dim * 64 + 16 * g);
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const pf_v4f v = src[j4];
        rk[mb][4 * j4] = v.x; rk[mb][4 * j4 + 1] = v.y; rk[mb][4 * j4 + 2] = v.z; rk[mb][4 * j4 + 3] = v.w;
      }
    }
#pragma unroll
    for (int j = 0; j < NGR; ++j) {
      float qv[16];
      if (a.q_dt == TQ_F32) {
        const pf_v4f* src = reinterpret_cast<const pf_v4f*>(static_cast<const float*>(a.q) + qoff[j] + 16 * g);
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const pf_v4f v = src[j4];
          qv[4 * j4] = v.x; qv[4 * j4 + 1] = v.y; qv[4 * j4 + 2] = v.z; qv[4 * j4 + 3] = v.w;
        }
      } else {
        const pf_u32x4* src = reinterpret_cast<const pf_u32x4*>(static_cast<const uint16_t*>(a.q) + qoff[j] + 16 * g);
        const bool bf = a.q_dt == TQ_BF16;
#pragma unroll
        for (int j8 = 0; j8 < 2; ++j8) {
          const pf_u32x4 v = src[j8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t hb = (v[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            qv[8 * j8 + e] = bf ? __uint_as_float(hb << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
          }
        }
      }
      pf_v4f d[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) d[mb] = (pf_v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s16 = 0; s16 < 16; ++s16) {
        const float b = qv[s16] * a.qscale;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) d[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(rk[mb][s16], b, d[mb], 0, 0, 0);
      }
      float qm = 0.f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) qm = fmaxf(qm, fabsf(d[mb][r]));
      qm = fmaxf(qm, __shfl_xor(qm, 16, 64));
      qm = fmaxf(qm, __shfl_xor(qm, 32, 64));
      const float qsc = pf_pow2_scale(qm);
      kinv[j] = 1.f / (qsc * ksc);  // a power of two
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = d[2 * s + (i >> 2)][i & 3] * qsc;
          const _Float16 hv = (_Float16)v;
          qhi[j][s][i] = hv;
          qlo[j][s][i] = (_Float16)(v - (float)hv);
        }
    }
  }

  const int bsl = a.bs_log2;
  const int64_t bsm = ((int64_t)1 << bsl) - 1;
  float m[NGR], l[NGR];
  pf_v4f o[NGR][4];

  // pool row of token t0 + 16 b (a 16-token group never straddles a block)
  auto tile_rows = [&](int64_t t0, int64_t* base) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t tb = t0 + 16 * b;
      const int bi = (int)min<int64_t>(tb >> bsl, (int64_t)a.max_blocks - 1);
      const uint32_t blk = min((uint32_t)a.block_table[bi], a.num_blocks - 1u);
      base[b] = (((int64_t)blk * hkv + h) << bsl) + (tb & bsm);
    }
  };
  // this lane's largest |v| over tile kt's tokens that some row of the wave sees
  auto tile_vmax = [&](int kt) -> float {
    int64_t base[4];
    tile_rows((int64_t)kt * 64, base);
    float vm = 0.f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const pf_v4f x = *reinterpret_cast<const pf_v4f*>(a.vnorms + base[b] + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        vm = fmaxf(vm, (int64_t)kt * 64 + 16 * b + 4 * g + r < limw ? fabsf(x[r]) : 0.f);
    }
    return vm;
  };
  // The value-norm scale comes from tile 0 (its largest |v| lands in [2^11, 2^12), so
  // later norms up to 16 times larger still give finite fp16 weights); a wave whose
  // accumulators end non-finite runs its tiles again with the scale of all its tiles.
  tq::VnScale vs;
  vs.fit(tile_vmax(0), 12);

  // Tiles every row of the wave sees whole need no mask (all but the last one or two).
  const int64_t limlo = a.past + row0 / a.G + 1;
  auto tile = [&](auto masked_tag, int kt) {
    constexpr bool MASK = decltype(masked_tag)::value;
    const int64_t t0 = (int64_t)kt * 64;
    // tokens of this tile each of the lane's rows sees (rows past the end: none)
    int rel[NGR];
#pragma unroll
    for (int j = 0; j < NGR; ++j) rel[j] = MASK ? (int)max<int64_t>(0, min<int64_t>(lim[j] - t0, 64)) : 64;
    int64_t base[4];
    tile_rows(t0, base);
    uint32_t kw[4][2];
    pf_v4f nk[4], nv[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint8_t* kr = a.kpairs + (base[b] + c) * 32 + 4 * g;
      kw[b][0] = *reinterpret_cast<const uint32_t*>(kr);
      kw[b][1] = *reinterpret_cast<const uint32_t*>(kr + 16);
      nk[b] = *reinterpret_cast<const pf_v4f*>(a.knorms + base[b] + 4 * g);
      nv[b] = *reinterpret_cast<const pf_v4f*>(a.vnorms + base[b] + 4 * g);
    }
    // value words (8 VB bytes per pool row; a sub-block starts at its group's first row):
    // VB 2 tile words 0-3; VB 3 / 4 tiles: words 0-3, then 4-5 / 4-7; sub-blocks of VB 3 /
    // 4: each group's shares, reassembled by vword below
    constexpr int NV = VB == 2 ? 4 : (SUB ? 8 : 2 * VB);
    uint32_t vw[NV];
    if constexpr (SUB) {
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const uint8_t* sb = a.vtiles + base[mm] * (8 * VB);
        if constexpr (VB == 2) {
          vw[mm] = *reinterpret_cast<const uint32_t*>(sb + 4 * lane);
        } else if constexpr (VB == 4) {
          const pf_u32x2 w = *reinterpret_cast<const pf_u32x2*>(sb + 8 * lane);
          vw[2 * mm] = w.x; vw[2 * mm + 1] = w.y;
        } else {
          vw[mm] = *reinterpret_cast<const uint32_t*>(sb + 4 * lane);
          vw[4 + mm] = *reinterpret_cast<const uint16_t*>(sb + 256 + 2 * lane);
        }
      }
    } else {
      const uint8_t* tb = a.vtiles + base[0] * (8 * VB);
      const pf_u32x4 v = *reinterpret_cast<const pf_u32x4*>(tb + 16 * lane);
      vw[0] = v.x; vw[1] = v.y; vw[2] = v.z; vw[3] = v.w;
      if constexpr (VB == 3) {
        const pf_u32x2 v1 = *reinterpret_cast<const pf_u32x2*>(tb + 1024 + 8 * lane);
        vw[4] = v1.x; vw[5] = v1.y;
      } else if constexpr (VB == 4) {
        const pf_u32x4 v1 = *reinterpret_cast<const pf_u32x4*>(tb + 1024 + 16 * lane);
        vw[4] = v1.x; vw[5] = v1.y; vw[6] = v1.z; vw[7] = v1.w;
      }
    }
    // VB 3 / 4: tile word i of half s (sub-blocks: bytes 0-1 from group 2 s's share, 2-3
    // from group 2 s + 1's), then the word whose bytes index the pair entries of dim group nb
    auto tword = [&](int s, int i) -> uint32_t {
      if constexpr (!SUB) {
        return vw[(VB == 4 ? 4 : 3) * s + i];
      } else if constexpr (VB == 4) {
        return __builtin_amdgcn_perm(vw[2 * (2 * s + 1) + (i >> 1)], vw[2 * (2 * s) + (i >> 1)],
                                     (i & 1) ? 0x07060302u : 0x05040100u);
      } else {
        return i == 2 ? __builtin_amdgcn_perm(vw[4 + 2 * s + 1], vw[4 + 2 * s], 0x05040100u)
                      : __builtin_amdgcn_perm(vw[2 * s + 1], vw[2 * s], i ? 0x07060302u : 0x05040100u);
      }
    };
    auto vword = [&](int s, int nb) -> uint32_t {
      if constexpr (VB == 4) {
        return tword(s, nb);
      } else {
        if (nb < 3) return tword(s, nb);
        const uint32_t x0 = tword(s, 0), x1 = tword(s, 1), x2 = tword(s, 2);
        return ((x0 >> 6) & 0x03030303u) | ((x1 >> 4) & 0x0C0C0C0Cu) | ((x2 >> 2) & 0x30303030u);
      }
    };

    // ---- scores (log2 domain), masked past each row's limit; one key operand per (b, s)
    // serves every row group
    pf_v4f sv[NGR][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      pf_v4f acc[NGR];
#pragma unroll
      for (int j = 0; j < NGR; ++j) acc[j] = (pf_v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t w = kw[b][s];
        const uint32_t i0 = w & 255u, i1 = (w >> 8) & 255u, i2 = (w >> 16) & 255u, i3 = w >> 24;
        const pf_v8h ah = pf_h8(tk[0][i0 * KC + kcp], tk[0][i1 * KC + kcp], tk[0][i2 * KC + kcp],
                                tk[0][i3 * KC + kcp]);
#pragma unroll
        for (int j = 0; j < NGR; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qhi[j][s], acc[j], 0, 0, 0);
        if constexpr (PREC) {
          const pf_v8h al = pf_h8(tk[NP - 1][i0 * KC + kcp], tk[NP - 1][i1 * KC + kcp],
                                  tk[NP - 1][i2 * KC + kcp], tk[NP - 1][i3 * KC + kcp]);
#pragma unroll
          for (int j = 0; j < NGR; ++j) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qlo[j][s], acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, qhi[j][s], acc[j], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < NGR; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // score / kinv (kinv a power of two: scaling it out is exact)
          const float x = acc[j][r] * nk[b][r];
          sv[j][b][r] = (!MASK || 16 * b + 4 * g + r < rel[j]) ? x : -INFINITY;
        }
    }
    // value norms times the wave's scale (masked tokens are selected away below)
    float nvs[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) nvs[b][r] = nv[b][r] * vs.s;
    pf_v8h bh[NGR][2], bl[NGR][2];
#pragma unroll
    for (int j = 0; j < NGR; ++j) {
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sv[j][b][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m[j], mx * kinv[j]);
      const float ms = mn == -INFINITY ? 0.f : mn;
      // 2^x on the hardware's exp2 (results below 2^-126 flush to 0: weights that small
      // against the running maximum's 1 do not change an fp32 sum).  The accumulators are
      // rescaled only when some row's maximum moved (a few tiles per row).
      if (__any(mn != m[j])) {
        const float alpha = __builtin_amdgcn_exp2f(m[j] - ms);
        l[j] *= alpha;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) o[j][nb] *= alpha;
      }
      m[j] = mn;
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sv[j][b][r], kinv[j], -ms));
          l[j] += p;
          // masked tokens' norms may be stale (even NaN): selected away, not multiplied
          const float v = (!MASK || 16 * b + 4 * g + r < rel[j]) ? p * nvs[b][r] : 0.f;
          if constexpr (PREC) {
            _Float16 hv, lv;
            tq::split_f16(v, hv, lv);
            bh[j][b >> 1][4 * (b & 1) + r] = hv;
            bl[j][b >> 1][4 * (b & 1) + r] = lv;
          } else {
            bh[j][b >> 1][4 * (b & 1) + r] = (_Float16)v;
          }
        }
    }

    // The weights are written by VALU conversions and read by the MFMAs below as the B
    // operand: explicit wait states between the two (tq::mfma_operand_fence).
    if constexpr (NGR == 3 && !PREC) {
      tq::mfma_operand_fence6(bh[0][0], bh[0][1], bh[1][0], bh[1][1], bh[2][0], bh[2][1]);
    } else if constexpr (NGR == 2 && PREC) {
      tq::mfma_operand_fence8(bh[0][0], bh[0][1], bh[1][0], bh[1][1], bl[0][0], bl[0][1],
                              bl[1][0], bl[1][1]);
    } else {
#pragma unroll
      for (int j = 0; j < NGR; ++j) {
        if constexpr (PREC) tq::mfma_operand_fence(bh[j][0], bh[j][1], bl[j][0], bl[j][1]);
        else tq::mfma_operand_fence(bh[j][0], bh[j][1]);
      }
    }

    // ---- O^T += V^T P^T over the tile's two 32-token halves; one value operand per
    // (s, nb) serves every row group
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        pf_v8h ah, al{};
        if constexpr (VB == 2) {
          const uint32_t b0 = (vw[2 * s] >> (8 * nb)) & 255u, b1 = (vw[2 * s + 1] >> (8 * nb)) & 255u;
          const pf_u32x2 h0 = tv[0][b0 * VC + vcp], h1 = tv[0][b1 * VC + vcp];
          ah = pf_h8(h0.x, h0.y, h1.x, h1.y);
          if constexpr (PREC) {
            const pf_u32x2 l0 = tv[NP - 1][b0 * VC + vcp], l1 = tv[NP - 1][b1 * VC + vcp];
            al = pf_h8(l0.x, l0.y, l1.x, l1.y);
          }
        } else {
          const uint32_t w = vword(s, nb);
          const uint32_t i0 = w & 255u, i1 = (w >> 8) & 255u, i2 = (w >> 16) & 255u, i3 = w >> 24;
          ah = pf_h8(tw[0][i0 * WC + wcp], tw[0][i1 * WC + wcp], tw[0][i2 * WC + wcp], tw[0][i3 * WC + wcp]);
          if constexpr (PREC)
            al = pf_h8(tw[NP - 1][i0 * WC + wcp], tw[NP - 1][i1 * WC + wcp], tw[NP - 1][i2 * WC + wcp],
                       tw[NP - 1][i3 * WC + wcp]);
        }
#pragma unroll
        for (int j = 0; j < NGR; ++j)
          o[j][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j][s], o[j][nb], 0, 0, 0);
        if constexpr (PREC) {
#pragma unroll
          for (int j = 0; j < NGR; ++j) {
            o[j][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[j][s], o[j][nb], 0, 0, 0);
            o[j][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j][s], o[j][nb], 0, 0, 0);
          }
        }
      }
    }
  };
  for (int pass = 0;; ++pass) {
#pragma unroll
    for (int j = 0; j < NGR; ++j) {
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) o[j][nb] = (pf_v4f){0.f, 0.f, 0.f, 0.f};
    }
    for (int kt = 0; kt < ntiles; ++kt) {
      if ((int64_t)kt * 64 + 64 <= limlo) tile(std::false_type{}, kt);
      else tile(std::true_type{}, kt);
    }
    if (pass == 1) break;
    bool bad = false;  // an fp16 weight overflowed (or the inputs hold inf / NaN)
#pragma unroll
    for (int j = 0; j < NGR; ++j)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) bad |= !(fabsf(o[j][nb][r]) <= 0x1.fffffep127f);
    if (!__any(bad)) break;
    float vm = 0.f;
    for (int kt = 0; kt < ntiles; ++kt) vm = fmaxf(vm, tile_vmax(kt));
    vs.fit(vm, 12);
  }

  // ---- out = (O / l) R_v.  o[j][nb][r] of lane (c, g) = O_c[16 nb + 4 g + r]: the B
  // operand of k-step (nb, r); A[m][k] = R_v[16 nb + 4 k + r][16 ob + m]; lane (c, g)
  // register r gets out_c[16 ob + 4 g + r].
  // this lane's R_v entries, all requested before the first product
  float rv[4][16];
#pragma unroll
  for (int ob = 0; ob < 4; ++ob)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) rv[ob][4 * nb + r] = a.vrot[(16 * nb + 4 * g + r) * 64 + 16 * ob + c];
#pragma unroll
  for (int j = 0; j < NGR; ++j) {
    float lt = l[j];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const float inv = lt > 0.f ? 1.f / (lt * vsc) * vs.inv() : 0.f;
    float* dst = a.out + qoff[j];
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      pf_v4f acc = (pf_v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(rv[ob][4 * nb + r], o[j][nb][r] * inv, acc, 0, 0, 0);
      if (row[j] < nG) *reinterpret_cast<pf_v4f*>(dst + 16 * ob + 4 * g) = acc;
    }
  }
}

template <bool SUB, bool PREC>
void launch_prefill(int vbits, dim3 grid, const PfArgs& a, hipStream_t st) {
  if (vbits == 2) hipLaunchKernelGGL((dl_prefill_kernel<SUB, PREC, 2>), grid, dim3(kPfThreads), 0, st, a);
  else if (vbits == 3) hipLaunchKernelGGL((dl_prefill_kernel<SUB, PREC, 3>), grid, dim3(kPfThreads), 0, st, a);
  else hipLaunchKernelGGL((dl_prefill_kernel<SUB, PREC, 4>), grid, dim3(kPfThreads), 0, st, a);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int tq_prefill_attention_paged_dl(const void* q, tq_dtype q_dtype, int32_t n, int64_t T, int32_t hq,
                                  int32_t hkv, int32_t d, const uint8_t* kpairs_pool,
                                  const float* knorm_pool, const uint8_t* vtile_pool,
                                  const float* vnorm_pool, int64_t num_blocks, int32_t block_size,
                                  int32_t vbits, const int32_t* block_table, int32_t max_blocks,
                                  const float* kcentroids, const float* vcentroids,
                                  const float* krotation, const float* vrotation, float scale,
                                  float* out, void* stream) {
  TQ_REQUIRE(valid_dtype(q_dtype), "unknown dtype");
  TQ_REQUIRE(d == 64, "decode layout covers head_dim 64, got %d", d);
  TQ_REQUIRE(vbits >= 2 && vbits <= 4, "value tiles hold 2-4 bit codes, got %d", vbits);
  TQ_REQUIRE(hkv >= 1 && hq >= hkv && hq % hkv == 0,
             "num_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  int bsl = 0;
  while (bsl < 30 && (1 << bsl) < block_size) ++bsl;
  TQ_REQUIRE(block_size >= 16 && (1 << bsl) == block_size,
             "decode-layout pools need a power-of-two block_size >= 16, got %d", block_size);
  TQ_REQUIRE(n >= 0 && T >= n && max_blocks >= 0 && num_blocks >= 0, "bad sizes");
  TQ_REQUIRE(T <= (int64_t)max_blocks * block_size,
             "context of %lld tokens exceeds the block table (%d blocks of %d)", (long long)T,
             max_blocks, block_size);
  const int64_t rows = (int64_t)n * (hq / hkv);
  TQ_REQUIRE(rows <= INT_MAX - kPfRows, "too many query rows in one call");
  // bf16 queries: one product per term (their outputs are consumed in bf16), three 16-row
  // groups per wave; fp32 / fp16 queries: hi + lo parts, two groups per wave
  const bool prec = q_dtype != TQ_BF16;
  const int wg_rows = prec ? 2 * kPfRows : 3 * kPfRows;
  const int64_t grid = (rows + wg_rows - 1) / wg_rows * hkv;
  TQ_REQUIRE(grid <= INT_MAX, "too many query rows in one call");
  TQ_REQUIRE(num_blocks <= (int64_t)UINT_MAX, "too many blocks");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(num_blocks >= 1, "empty pools");
  TQ_REQUIRE(q && out && block_table && kpairs_pool && knorm_pool && vtile_pool && vnorm_pool &&
                 kcentroids && vcentroids && krotation && vrotation,
             "null pointer argument");
  TQ_REQUIRE(((reinterpret_cast<uintptr_t>(kpairs_pool) | reinterpret_cast<uintptr_t>(vtile_pool) |
               reinterpret_cast<uintptr_t>(knorm_pool) | reinterpret_cast<uintptr_t>(vnorm_pool) |
               reinterpret_cast<uintptr_t>(out)) & 15u) == 0,
             "pools and output must be 16-byte aligned");
  PfArgs a{};
  a.q = q; a.q_dt = (int)q_dtype; a.n = n; a.hq = hq; a.hkv = hkv; a.G = hq / hkv;
  a.past = T - n;
  a.kpairs = kpairs_pool; a.knorms = knorm_pool; a.vtiles = vtile_pool; a.vnorms = vnorm_pool;
  a.block_table = block_table; a.max_blocks = max_blocks; a.bs_log2 = bsl;
  a.num_blocks = (uint32_t)num_blocks;
  a.kcen = kcentroids; a.vcen = vcentroids; a.krot = krotation; a.vrot = vrotation;
  a.qscale = scale * 1.4426950408889634f;
  a.out = out;
  const dim3 gr((unsigned)grid);
  hipStream_t st = as_stream(stream);
  if (bsl >= 6) {
    if (prec) launch_prefill<false, true>(vbits, gr, a, st);
    else launch_prefill<false, false>(vbits, gr, a, st);
  } else {
    if (prec) launch_prefill<true, true>(vbits, gr, a, st);
    else launch_prefill<true, false>(vbits, gr, a, st);
  }
  TQ_LAUNCH_CHECK("dl_prefill_kernel");
  return TQ_OK;
}

}  // extern "C"
