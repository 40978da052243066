// tq_scan.hip -- scoring over packed codes on gfx950.
//
// Kernels
//   scan_kernel     ADC scan.  Each block first builds its queries' tables in LDS:
//                   q_rot = R q (sequential fp32 mul/add per output, like
//                   csrc/core/turboquant_core.cpp:429-437) and LUT[j][l] = q_rot[j] * c[l]
//                   (core.cpp:440-446; triton_kernels.py:437).  Then one lane = one
//                   packed row: the row's bit planes are loaded with 16-byte loads,
//                   transposed to per-octet words with v_perm_b32, and every dim's
//                   code becomes an LDS byte address (code*8) with one v_and + one
//                   v_dot4_u32_u8.  The table for dim j sits in LDS with an 8-byte
//                   stride per code (two dims share a 128-byte block), so a wave's 64
//                   lookups of one dim touch 16 distinct banks or broadcast:
//                   conflict-free.  Sums run over j in increasing order and are scaled
//                   by the row norm last, the reference's own order (core.cpp:455-483).
//                   Modes: TOPK keeps per-wave candidate lists in LDS (insert when
//                   score beats the wave's k-th best, strict '>' with lower index
//                   winning ties, as the core's heap does: core.cpp:487-494) and
//                   writes each workgroup's sorted top-k; ALL writes every score
//                   (attention_scores_packed, attn_scores.cu:31-104 semantics).
//   merge_kernel    per query: prunes the block lists with the k-th best of the
//                   per-block maxima, rank-sorts the survivors and writes top-k
//                   (int64 ids, (-inf, -1) pads).  A launch of its own: merging in the
//                   scan's last block would need an agent-scope release per block,
//                   i.e. an L2 write-back on every one of the 8 XCDs' caches.
//   softmax_stats   per query: max and sum of exp over its valid scores.
//   values_kernel   o_part[q][j] = sum_t w[q][t] * vn[t] * c[code_tj] over one
//                   split of the tokens; 16 fp32 accumulators per thread (4 queries
//                   x 4 dims), V rows staged in LDS.
//   combine_kernel  sum of the split partials, then o = o_rot @ M (M = R).

#include "tq_common.h"
#include "tq_decode.h"

#include <atomic>
#include <climits>
#include <mutex>
#include <utility>

namespace tq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxK = 128;           // top-k of the fused scans
constexpr int kSmallK = 32;          // the one-query filter and the small-list paths
// Candidate slots per (wave, query) of the exact scans' top-k lists, in dynamic LDS: room
// for the k kept entries plus one 64-row step of new ones.
__host__ __device__ constexpr int cand_cap(int k) { return k <= kSmallK ? 96 : 192; }
constexpr int kCandRegs = cand_cap(kMaxK) / 64;  // list entries per lane in wave_compact
constexpr int kValTokens = 256;       // tokens staged per values chunk
constexpr int kSplitTokens = 1024;    // tokens per values split (decode / values op)

// ------------------------------------------------------------------ scan
struct ScanArgs {
  const uint8_t* packed;    // rows of stream s start at packed + s * stream_rows * P
  const float* norms;       // stream s starts at norms + s * stream_rows
  int64_t stream_rows;      // row stride between streams
  int64_t nrows;            // rows per stream when seq_lens == nullptr
  const int32_t* seq_lens;  // per batch row counts (decode); stream s -> batch s / spb
  int spb;                  // streams per batch
  int bpp;                  // bytes per plane (runtime; used by the generic loader)
  const void* q;            // [nq_total][d] queries (q_dt); the table is built per block
  int q_dt;
  int d;
  const float* rot;         // [d][d]
  const float* cen;         // [2^bits]
  // Prod mode (signs != nullptr): rows also carry a QJL sign row (bpp bytes, the 1-bit
  // bit-plane layout) and a residual norm gamma, and score
  // n * (sum_j q_rot[j] c[code_j] + gamma * qjl_scale * sum_j (S q)_j (+-1)_j).
  const uint8_t* signs;     // stream s starts at signs + s * stream_rows * bpp
  const float* gammas;      // stream s starts at gammas + s * stream_rows
  const float* qjl;         // [d][d] S
  float qjl_scale;          // sqrt(pi/2) / d
  int qps;                  // queries per stream
  float post_scale;         // multiplies norm * sum (decode: softmax scale)
  int k;
  int ccap;                 // TOPK: cand_cap(k), the dynamic LDS lists' slots
  float* part_s;            // TOPK: [nq_total][gridDim.x][k]
  int32_t* part_i;
  float* scores;            // ALL:  [nq_total][stream_rows]
  float* out_s;             // [nq_total][k] (TOPK: written by merge_kernel)
  int64_t* out_i;
  const int32_t* qflag;     // optional [qps]: a block whose queries are all 0 here returns
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int BITS, int BPP>
struct RowLoader {
  static constexpr int P = BITS * BPP;
  static constexpr int NW = (P + 3) / 4;  // 32-bit words per row (fast path: P % 4 == 0)
  // Plane p, word w of the row: bytes [p*BPP + 4w, +4) (dims 32w..32w+31 of plane p).
  __device__ static __forceinline__ void load(const uint8_t* __restrict__ row, uint32_t (&wd)[NW]) {
    if constexpr (P % 16 == 0) {
      const u32x4* r4 = reinterpret_cast<const u32x4*>(row);
#pragma unroll
      for (int i = 0; i < P / 16; ++i) {
        const u32x4 v = r4[i];
        wd[4 * i + 0] = v.x; wd[4 * i + 1] = v.y; wd[4 * i + 2] = v.z; wd[4 * i + 3] = v.w;
      }
    } else if constexpr (P % 8 == 0) {
      const u32x2* r2 = reinterpret_cast<const u32x2*>(row);
#pragma unroll
      for (int i = 0; i < P / 8; ++i) {
        const u32x2 v = r2[i];
        wd[2 * i + 0] = v.x; wd[2 * i + 1] = v.y;
      }
    } else {
      const uint32_t* r1 = reinterpret_cast<const uint32_t*>(row);
#pragma unroll
      for (int i = 0; i < NW; ++i) wd[i] = r1[i];
    }
  }
};

// Generic loader for any bytes-per-plane (<= 32): assembles the plane words of a
// BPP_T=32 layout from byte loads; missing bytes are zero (pad dims decode to code 0,
// whose table entries are zero).
template <int BITS>
__device__ __forceinline__ void load_generic(const uint8_t* __restrict__ row, int bpp,
                                             uint32_t (&wd)[BITS * 8]) {
#pragma unroll
  for (int p = 0; p < BITS; ++p) {
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t v = 0;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int kb = 4 * w + m;
        if (kb < bpp) v |= (uint32_t)row[p * bpp + kb] << (8 * m);
      }
      wd[p * 8 + w] = v;
    }
  }
}

// Byte address (code * SC) of every dim of one 32-dim word group.
// A[p] = word w of plane p.  Calls f(dim_in_group, addr8) for dims 0..31 in order.
template <int BITS, int SC, typename F, typename G>
__device__ __forceinline__ void decode_group(const uint32_t (&A)[4], F&& f, G&& after_octet) {
  static_assert(SC == 8 || SC == 16, "code stride");
  const uint32_t a0 = A[0];
  const uint32_t a1 = BITS > 1 ? A[1] : 0u;
  const uint32_t a2 = BITS > 2 ? A[2] : 0u;
  const uint32_t a3 = BITS > 3 ? A[3] : 0u;
  const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
  const uint32_t hi01 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
  const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
  uint32_t X[4];
  X[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
  X[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  X[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  X[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
  // X[m] byte p = plane p's byte m (dims 8m..8m+7, dim 8m+i at bit 7-i).
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t xh = X[m];
    const uint32_t xl = X[m] >> 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // shift s of dim i's bit within each byte after choosing xh (i>=4) or xl (i<4)
      const int s = (i >= 4) ? (7 - i) : (3 - i);
      const uint32_t src = (i >= 4) ? xh : xl;
      const uint32_t z = src & (0x01010101u << s);
      // byte p of the weight = SC * 2^p / 2^s, so the dot product is code * SC
      const uint32_t w = SC == 8 ? ((s == 0) ? 0x40201008u : (s == 1) ? 0x20100804u
                                  : (s == 2) ? 0x10080402u : 0x08040201u)
                                 : ((s == 0) ? 0x80402010u : (s == 1) ? 0x40201008u
                                  : (s == 2) ? 0x20100804u : 0x10080402u);
      f(8 * m + i, __builtin_amdgcn_udot4(z, w, 0u, false));
    }
    after_octet();
  }
}

// Written with bitwise operators: short-circuit forms compile to exec-mask branches,
// which cost about a hundred cycles per comparison in the single-block merges.
__device__ __forceinline__ bool better(float sa, int ia, float sb, int ib) {
  return (sa > sb) | ((sa == sb) & (ia < ib));
}

// Reduce a wave's candidate list (cs/ci, `count` entries, count <= 64 R) to its best
// min(count, k) entries in sorted order: every entry counts the entries better than it
// and moves to that rank.  Wave-uniform arguments.
template <int R>
__device__ __forceinline__ void wave_compact_r(float* cs, int* ci, int& count, int k, float& th,
                                               int& thi) {
  const int lane = threadIdx.x & 63;
  float s[R];
  int id[R], rk[R];
  bool v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    v[r] = lane + 64 * r < count;
    s[r] = v[r] ? cs[lane + 64 * r] : 0.f;
    id[r] = v[r] ? ci[lane + 64 * r] : 0;
    rk[r] = 0;
  }
  for (int e = 0; e < count; ++e) {
    const float se = cs[e];
    const int ie = ci[e];
#pragma unroll
    for (int r = 0; r < R; ++r) rk[r] += better(se, ie, s[r], id[r]);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (v[r] && rk[r] < k) { cs[rk[r]] = s[r]; ci[rk[r]] = id[r]; }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  count = count < k ? count : k;
  if (count == k) {
    th = cs[k - 1];
    thi = ci[k - 1];
  }
}

// wave_compact_r for lists of up to cand_cap(kMaxK) entries.
__device__ __forceinline__ void wave_compact(float* cs, int* ci, int& count, int k, float& th,
                                             int& thi) {
  if (count <= 128) wave_compact_r<2>(cs, ci, count, k, th, thi);  // uniform
  else wave_compact_r<kCandRegs>(cs, ci, count, k, th, thi);
}

// Rank of (s, id) among the n entries of a best-first list: the entries better than it,
// by binary search (ids are distinct, so no entry of another list equals it).
__device__ __forceinline__ int sorted_rank(const float* ls, const int* li, int n, float s, int id) {
  int lo = 0, hi = n;  // entries [0, lo) are better, [hi, n) are not
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (better(ls[mid], li[mid], s, id)) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// The block's query tables in LDS.  q_rot[j] = sum_k q[k] * R[j][k] with k ascending and
// separate multiply and add roundings, table entry = q_rot[j] * c[l] -- the arithmetic
// of csrc/core/turboquant_core.cpp:429-446, so scores match the reference bit for bit.
// Layout: QB == 1: entry (j, l) at (j>>1)*NLEV*8 + l*8 + (j&1)*4 (two dims interleaved,
// 8-byte code stride); QB > 1: the QB queries' entries of (j, l) contiguous at
// (j*NLEV + l)*QB*4, so one 8/16-byte read serves every query.  Dims d..DP-1 are zero.
//
// PROD adds the QJL term of every query as a table over groups of 4 sign bits:
// qs = S q (qs[j] = sum_k S[j][k] q[k], computed in the same pass over k as q_rot);
// entry (g, v) = qjl_scale * sum_{i<4, 4g+i<d} (bit 3-i of v ? +qs[4g+i] : -qs[4g+i]),
// v being the nibble that holds the signs of dims 4g..4g+3 (MSB first, as in the packed
// sign row).  So sum_g T[g][nibble_g] = qjl_scale * <S q, +-1> = qjl_scale * <q, (+-1) S>,
// the residual term of reference.py:522-529 dotted with q.  Groups past d are zero, as
// are pad dims.  Layout as the pair-layout tables (16 entries per group): QB == 1: entry
// (g, v) at (g>>1)*128 + v*8 + (g&1)*4; QB > 1: the QB queries' entries contiguous at
// (g*16 + v)*QB*4.
template <int NLEV, int DP, int QB, bool PROD = false>
__device__ __forceinline__ void build_tables(const ScanArgs& a, int q0, int nq, char* lut_s,
                                             char* sgn_s = nullptr) {
#pragma clang fp contract(off)
  __shared__ float qs[QB][256];
  __shared__ float qss[PROD ? QB : 1][PROD ? DP : 1];
  const int d = a.d;
  for (int idx = threadIdx.x; idx < QB * d; idx += kThreads) {
    const int qi = idx / d, k = idx - qi * d;
    qs[qi][k] = qi < nq ? load_as_f32(a.q, (int64_t)(q0 + qi) * d + k, a.q_dt) : 0.f;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < QB * DP; idx += kThreads) {
    const int qi = idx / DP, j = idx - qi * DP;
    float v = 0.f, w = 0.f;
    if (qi < nq && j < d) {
      const float* r = a.rot + (size_t)j * d;
      const float* sr = PROD ? a.qjl + (size_t)j * d : nullptr;
      if ((d & 3) == 0) {
        for (int k = 0; k < d; k += 4) {
          const float4 r4 = *reinterpret_cast<const float4*>(r + k);
          v = v + qs[qi][k] * r4.x;
          v = v + qs[qi][k + 1] * r4.y;
          v = v + qs[qi][k + 2] * r4.z;
          v = v + qs[qi][k + 3] * r4.w;
          if constexpr (PROD) {
            const float4 s4 = *reinterpret_cast<const float4*>(sr + k);
            w = fmaf(qs[qi][k], s4.x, w);
            w = fmaf(qs[qi][k + 1], s4.y, w);
            w = fmaf(qs[qi][k + 2], s4.z, w);
            w = fmaf(qs[qi][k + 3], s4.w, w);
          }
        }
      } else {
        for (int k = 0; k < d; ++k) {
          v = v + qs[qi][k] * r[k];
          if constexpr (PROD) w = fmaf(qs[qi][k], sr[k], w);
        }
      }
    }
    if constexpr (PROD) qss[qi][j] = w;
    for (int l = 0; l < NLEV; ++l) {
      const float e = (qi < nq && j < d) ? v * a.cen[l] : 0.f;
      const int off = QB == 1 ? (j >> 1) * NLEV * 8 + l * 8 + (j & 1) * 4
                              : (j * NLEV + l) * QB * 4 + qi * 4;
      *reinterpret_cast<float*>(lut_s + off) = e;
    }
  }
  __syncthreads();
  if constexpr (PROD) {
    for (int idx = threadIdx.x; idx < QB * DP * 4; idx += kThreads) {
      const int qi = idx / (DP * 4), e = idx - qi * (DP * 4);
      const int g = e >> 4, v = e & 15;
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = qss[qi][4 * g + i];
        t += ((v >> (3 - i)) & 1) ? x : -x;
      }
      const int off = QB == 1 ? (g >> 1) * 128 + v * 8 + (g & 1) * 4 : (g * 16 + v) * QB * 4 + qi * 4;
      *reinterpret_cast<float*>(sgn_s + off) = t * a.qjl_scale;
    }
    __syncthreads();
  }
}

// Calls f(dim, addr) for the 8 dims of one 32-bit word of pair-layout bytes (byte p =
// code[2p] << 4 | code[2p+1]), in dim order; addr = code * SC.  Two shift-and-mask pairs
// per word put every code of one nibble position at the SC scale, then one v_perm per dim
// moves its byte into an otherwise zero register.  (A 16-byte code stride would save one
// shift but puts codes l and l+8 in one LDS bank: 2-way conflicts on every lookup.)
template <int SC, typename F>
__device__ __forceinline__ void decode_pairs(uint32_t w, int j0, F&& f) {
  static_assert(SC == 8 || SC == 16, "code stride");
  const uint32_t wh = SC == 8 ? (w >> 1) & 0x78787878u : w & 0xF0F0F0F0u;
  const uint32_t wl = SC == 8 ? (w << 3) & 0x78787878u : (w << 4) & 0xF0F0F0F0u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f(j0 + 2 * k, __builtin_amdgcn_perm(0u, wh, 0x0c0c0c00u | k));
    f(j0 + 2 * k + 1, __builtin_amdgcn_perm(0u, wl, 0x0c0c0c00u | k));
  }
}

// One-query top-k prod scans over the fast layouts are held to 80 VGPRs: six 4-wave
// blocks per CU (scan_blocks' grid) are then all resident.
template <int BITS, int BPP, int QB, bool TOPK, bool GENERIC, bool PAIRS, bool PROD>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(
    (PROD && TOPK && !GENERIC && QB == 1) ? 6 : 0))) void scan_kernel(ScanArgs a) {
  static_assert(!PAIRS || (BITS == 4 && !GENERIC), "pair layout: 4-bit fast rows only");
  static_assert(!PROD || (!PAIRS && BITS <= 3), "prod rows: bit-plane MSE codes of 1-3 bits");
  constexpr int NLEV = 1 << BITS;
  constexpr int BPPT = GENERIC ? 32 : BPP;          // layout the decoder sees
  constexpr int DP = 8 * BPPT;                      // dims covered by the decoder
  constexpr int QSTRIDE = DP * NLEV * 4;            // bytes per query table
  constexpr int NW = GENERIC ? BITS * 8 : RowLoader<BITS, BPP>::NW;
  constexpr int WPP = BPPT / 4;                     // words per plane
  // Static LDS: the table's base address is a link-time constant, so every lookup is a
  // ds_read with an immediate offset and no address add.
  __shared__ __attribute__((aligned(16))) char lut_s[QB * QSTRIDE];
  constexpr int SW = GENERIC ? 8 : BPP / 4;         // sign-row words (prod mode)
  __shared__ __attribute__((aligned(16))) char sgn_s[PROD ? QB * DP * 16 : 16];
  // TOPK: kWaves * QB lists of a.ccap (score, id) slots in dynamic LDS
  extern __shared__ __attribute__((aligned(16))) char dyn_s[];
  const int ccap = TOPK ? a.ccap : 0;
  float* cand_s = reinterpret_cast<float*>(dyn_s);
  int* cand_i = reinterpret_cast<int*>(dyn_s) + kWaves * QB * ccap;
  __shared__ int cnt_s[TOPK ? kWaves * QB : 1];

  const int s = blockIdx.z;
  const int qb = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  int64_t nrows = a.nrows;
  if (a.seq_lens) {
    const int64_t sl = a.seq_lens[s / a.spb];
    nrows = sl < a.stream_rows ? sl : a.stream_rows;
  }
  const int q0 = s * a.qps + qb * QB;            // first global query of this block
  const int nq = min(QB, a.qps - qb * QB);       // valid queries in this block
  if (a.qflag) {  // only flagged queries are scanned (uniform)
    int any = 0;
    for (int j = 0; j < nq; ++j) any |= a.qflag[qb * QB + j];
    if (!any) return;
  }
  const int P = BITS * a.bpp;

  build_tables<NLEV, DP, QB, PROD>(a, q0, nq, lut_s, sgn_s);

  // Contiguous row range of this block, 64-row steps interleaved over the waves.
  const int64_t per_block = ((nrows + gridDim.x - 1) / gridDim.x + 63) / 64 * 64;
  const int64_t rbeg = (int64_t)blockIdx.x * per_block;
  const int64_t rend = min(nrows, rbeg + per_block);
  const uint8_t* base = a.packed + (size_t)s * a.stream_rows * P;
  const float* nbase = a.norms + (size_t)s * a.stream_rows;

  float th[QB];
  int thi[QB];
  int cnt[QB];
#pragma unroll
  for (int qi = 0; qi < QB; ++qi) { th[qi] = -INFINITY; thi[qi] = INT_MAX; cnt[qi] = 0; }
  float* my_cs = cand_s + wave * QB * ccap;
  int* my_ci = cand_i + wave * QB * ccap;

  int64_t row = rbeg + wave * 64 + lane;
  // Loads are unconditional (rows past the end re-read the last row and are masked
  // when scored): a branch around them would make the compiler wait for every
  // outstanding load, including the next row's prefetch, before each row.
  const int64_t rlast = rend - 1;
  // A row's words and its norm, loaded together: a norm load issued inside the step
  // would make the step wait (loads complete in issue order) for every row prefetched
  // before it.
  struct RowBuf {
    uint32_t w[NW];
    float n;
    uint32_t sw[PROD ? SW : 1];  // prod: sign row
    float g;                     // prod: residual norm
  };
  // Fast layouts load through per-block buffer resources: 32-bit offsets from the
  // block's first row, and rows at or past rend read as zeros (no clamp).
  const uint32_t nbr = (uint32_t)(rend > rbeg ? rend - rbeg : 0);
  const __amdgpu_buffer_rsrc_t rows_rs = buf_rsrc(base + rbeg * P, nbr * (uint32_t)P);
  const __amdgpu_buffer_rsrc_t norm_rs = buf_rsrc(nbase + rbeg, nbr * 4u);
  const uint8_t* sbase = PROD ? a.signs + (size_t)s * a.stream_rows * a.bpp : nullptr;
  const float* gbase = PROD ? a.gammas + (size_t)s * a.stream_rows : nullptr;
  const __amdgpu_buffer_rsrc_t sgn_rs =
      buf_rsrc(PROD ? sbase + rbeg * BPP : a.packed, PROD ? nbr * (uint32_t)BPP : 0u);
  const __amdgpu_buffer_rsrc_t gam_rs = buf_rsrc(PROD ? gbase + rbeg : a.norms, PROD ? nbr * 4u : 0u);
  auto load_row = [&](int64_t r, RowBuf& b) {
    if constexpr (GENERIC) {
      const int64_t rl = r < rend ? r : rlast;
      load_generic<BITS>(base + rl * P, a.bpp, b.w);
      b.n = __builtin_nontemporal_load(nbase + rl);
      if constexpr (PROD) {
        uint32_t sw[8];
        load_generic<1>(sbase + rl * a.bpp, a.bpp, sw);
#pragma unroll
        for (int i = 0; i < 8; ++i) b.sw[i] = sw[i];
        b.g = __builtin_nontemporal_load(gbase + rl);
      }
    } else {
      constexpr int PB = BITS * BPP;
      const uint32_t rr = (uint32_t)(r - rbeg);
      const int off = (int)(rr * (uint32_t)PB);
      if constexpr (PB % 16 == 0) {
#pragma unroll
        for (int i = 0; i < PB / 16; ++i) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rows_rs, off, 16 * i, 0);
          b.w[4 * i + 0] = v.x; b.w[4 * i + 1] = v.y; b.w[4 * i + 2] = v.z; b.w[4 * i + 3] = v.w;
        }
      } else {
        static_assert(PB % 8 == 0, "fast rows are a whole number of 8-byte units");
#pragma unroll
        for (int i = 0; i < PB / 8; ++i) {
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rows_rs, off, 8 * i, 0);
          b.w[2 * i + 0] = v.x; b.w[2 * i + 1] = v.y;
        }
      }
      b.n = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(norm_rs, (int)(rr * 4u), 0, kNT));
      if constexpr (PROD) {
        const int soff = (int)(rr * (uint32_t)BPP);
        if constexpr (BPP == 16) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(sgn_rs, soff, 0, 0);
          b.sw[0] = v.x; b.sw[1] = v.y; b.sw[2] = v.z; b.sw[3] = v.w;
        } else {
          static_assert(BPP == 8, "fast prod rows: 64 or 128 dims");
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(sgn_rs, soff, 0, 0);
          b.sw[0] = v.x; b.sw[1] = v.y;
        }
        b.g = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(gam_rs, (int)(rr * 4u), 0, kNT));
      }
    }
  };
  // One 64-row step of this wave: score row `row` from its plane words `rb.w`.
  auto step = [&](const RowBuf& rb, const int64_t row) {
    const uint32_t (&cur)[NW] = rb.w;
    const float nrm = rb.n;

    float acc[QB];
#pragma unroll
    for (int qi = 0; qi < QB; ++qi) acc[qi] = 0.f;
    if constexpr (PAIRS) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        decode_pairs<QB == 4 ? 16 : 8>(cur[w], 8 * w, [&](int j, uint32_t addr) {
          if constexpr (QB == 1) {
            acc[0] += *reinterpret_cast<const float*>(lut_s + (j >> 1) * NLEV * 8 + (j & 1) * 4 + addr);
          } else if constexpr (QB == 2) {
            const float2 v = *reinterpret_cast<const float2*>(lut_s + j * NLEV * 8 + addr);
            acc[0] += v.x;
            acc[1] += v.y;
          } else {
            const float4 v = *reinterpret_cast<const float4*>(lut_s + j * NLEV * 16 + addr);
            acc[0] += v.x;
            acc[1] += v.y;
            acc[2] += v.z;
            acc[3] += v.w;
          }
        });
        if constexpr (QB == 2) asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
        if constexpr (QB == 4) asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
      }
    } else {
#pragma unroll
    for (int w = 0; w < WPP; ++w) {
      uint32_t A[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) A[p] = (p < BITS) ? cur[p * WPP + w] : 0u;
      constexpr int SC = QB == 4 ? 16 : 8;
      decode_group<BITS, SC>(A, [&](int di, uint32_t addr) {
        const int j = 32 * w + di;
        if constexpr (QB == 1) {
          acc[0] += *reinterpret_cast<const float*>(lut_s + (j >> 1) * NLEV * 8 + (j & 1) * 4 + addr);
        } else if constexpr (QB == 2) {
          const float2 v = *reinterpret_cast<const float2*>(lut_s + j * NLEV * 8 + addr);
          acc[0] += v.x;
          acc[1] += v.y;
        } else {
          const float4 v = *reinterpret_cast<const float4*>(lut_s + j * NLEV * 16 + addr);
          acc[0] += v.x;
          acc[1] += v.y;
          acc[2] += v.z;
          acc[3] += v.w;
        }
      }, [&]() {
        // Multi-query tables return 8-16 bytes per lookup; without this the compiler
        // issues every lookup of the row before the adds and spills.  Pinning the
        // accumulators here makes each octet's adds complete in order.
        if constexpr (QB == 2) asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
        if constexpr (QB == 4) asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
      });
    }
    }
    if constexpr (PROD) {
      // QJL term: one lookup per 4 sign bits (decode_pairs reads a sign byte's two
      // nibbles as groups 2p and 2p+1), added to the MSE sum scaled by gamma.
      float sacc[QB];
#pragma unroll
      for (int qi = 0; qi < QB; ++qi) sacc[qi] = 0.f;
#pragma unroll
      for (int w = 0; w < SW; ++w) {
        decode_pairs<QB == 4 ? 16 : 8>(rb.sw[w], 8 * w, [&](int g, uint32_t addr) {
          if constexpr (QB == 1) {
            sacc[0] += *reinterpret_cast<const float*>(sgn_s + (g >> 1) * 128 + (g & 1) * 4 + addr);
          } else if constexpr (QB == 2) {
            const float2 v = *reinterpret_cast<const float2*>(sgn_s + g * 128 + addr);
            sacc[0] += v.x;
            sacc[1] += v.y;
          } else {
            const float4 v = *reinterpret_cast<const float4*>(sgn_s + g * 256 + addr);
            sacc[0] += v.x;
            sacc[1] += v.y;
            sacc[2] += v.z;
            sacc[3] += v.w;
          }
        });
        if constexpr (QB == 2) asm volatile("" : "+v"(sacc[0]), "+v"(sacc[1]));
        if constexpr (QB == 4) asm volatile("" : "+v"(sacc[0]), "+v"(sacc[1]), "+v"(sacc[2]), "+v"(sacc[3]));
      }
#pragma unroll
      for (int qi = 0; qi < QB; ++qi) acc[qi] = fmaf(rb.g, sacc[qi], acc[qi]);
    }

    if constexpr (TOPK) {
      const bool valid = row < rend;
#pragma unroll
      for (int qi = 0; qi < QB; ++qi) {
        if (QB > 1 && qi >= nq) break;  // a one-query block always has its query
        const float sc = acc[qi] * nrm * a.post_scale;
        const int id = (int)row;
        bool pred = valid & better(sc, id, th[qi], thi[qi]);
        uint64_t mask = __ballot(pred);
        int nnew = __popcll(mask);
        if (nnew == 0) continue;
        float* cs = my_cs + qi * ccap;
        int* ci = my_ci + qi * ccap;
        if (cnt[qi] + nnew > ccap) {
          wave_compact(cs, ci, cnt[qi], a.k, th[qi], thi[qi]);
          pred = valid & better(sc, id, th[qi], thi[qi]);
          mask = __ballot(pred);
          nnew = __popcll(mask);
        }
        if (pred) {
          const int pos = cnt[qi] + (int)__builtin_amdgcn_mbcnt_hi(
                                        (uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
          cs[pos] = sc;
          ci[pos] = id;
        }
        cnt[qi] += nnew;
      }
    } else {
      if (row < rend) {
#pragma unroll
        for (int qi = 0; qi < QB; ++qi)
          if (qi < nq) a.scores[(size_t)(q0 + qi) * a.stream_rows + row] = acc[qi] * nrm * a.post_scale;
      }
    }
  };
  // Pair-layout rows are loaded two steps ahead, others one, into rotating register
  // buffers: a row loaded from HBM under full load takes longer than one step to
  // arrive.  (A copy between buffers would wait for the loads in flight.)
  // The next step's rows are loaded before the current step is scored, into the other
  // of two register buffers (a copy between them would wait for the loads in flight;
  // a third buffer measured slower).  The step count is made wave-uniform explicitly:
  // a loop on the per-lane row index compiles to an exec-masked loop whose merged
  // states make the load waits conservative.
  constexpr int64_t kStride = kWaves * 64;
  const int64_t first = rbeg + wave * 64;
  const int nsteps = __builtin_amdgcn_readfirstlane(
      first < rend ? (int)((rend - first + kStride - 1) / kStride) : 0);
  RowBuf ta, tb;
  if (nsteps > 0) load_row(row, ta);
  for (int it = 0; it < nsteps; it += 2) {
    load_row(row + kStride, tb);
    step(ta, row);
    row += kStride;
    if (it + 1 >= nsteps) break;
    load_row(row + kStride, ta);
    step(tb, row);
    row += kStride;
  }

  if constexpr (TOPK) {
#pragma unroll
    for (int qi = 0; qi < QB; ++qi) {
      if (qi >= nq) break;
      // every wave list leaves sorted (best first) with at most k entries
      if (cnt[qi] > 1) wave_compact(my_cs + qi * ccap, my_ci + qi * ccap, cnt[qi], a.k, th[qi], thi[qi]);
      if (lane == 0) cnt_s[wave * QB + qi] = cnt[qi];
    }
    __syncthreads();
    // Merge the 4 wave lists of query qi (<= 4k entries): wave qi % 4.
    for (int qi = wave; qi < nq; qi += kWaves) {
      int total = 0;
      int off[kWaves];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) { off[w] = total; total += cnt_s[w * QB + qi]; }
      // entry e of the union -> (wave w, slot e - off[w])
      auto fetch = [&](int e, float& sc, int& id) {
        int w = 0;
#pragma unroll
        for (int t = 1; t < kWaves; ++t) w += (e >= off[t]);
        const int slot = e - off[w];
        sc = cand_s[(w * QB + qi) * ccap + slot];
        id = cand_i[(w * QB + qi) * ccap + slot];
      };
      float* ps = a.part_s + ((size_t)(q0 + qi) * gridDim.x + blockIdx.x) * a.k;
      int32_t* pi = a.part_i + ((size_t)(q0 + qi) * gridDim.x + blockIdx.x) * a.k;
      if (total <= 128) {  // uniform
        for (int e = lane; e < 2 * 64; e += 64) {
          if (e < total) {
            float se; int ie;
            fetch(e, se, ie);
            int rank = 0;
            for (int f = 0; f < total; ++f) {
              float sf; int jf;
              fetch(f, sf, jf);
              rank += better(sf, jf, se, ie);
            }
            if (rank < a.k) { ps[rank] = se; pi[rank] = ie; }
          }
        }
      } else {
        // long lists: an entry's rank is its slot in its own sorted list plus, per other
        // wave's list, the entries better than it (binary search)
        for (int e = lane; e < total; e += 64) {
          int w = 0;
#pragma unroll
          for (int t = 1; t < kWaves; ++t) w += (e >= off[t]);
          const int slot = e - off[w];
          const float se = cand_s[(w * QB + qi) * ccap + slot];
          const int ie = cand_i[(w * QB + qi) * ccap + slot];
          int rank = slot;
#pragma unroll
          for (int t = 0; t < kWaves; ++t)
            if (t != w)
              rank += sorted_rank(cand_s + (t * QB + qi) * ccap, cand_i + (t * QB + qi) * ccap,
                                  cnt_s[t * QB + qi], se, ie);
          if (rank < a.k) { ps[rank] = se; pi[rank] = ie; }
        }
      }
      for (int e = total + lane; e < a.k; e += 64) { ps[e] = -INFINITY; pi[e] = -1; }
    }
  }
}

// ------------------------------------------------------------------ pair-layout scan, one query
// The same scores as scan_kernel<4, *, 1, *, false, true>, with half the LDS reads.  A
// 256-entry table indexed by a whole pair byte returns both centroids of the byte's two
// dims in one 8-byte read (32 copies, one per lane of a half-wave: conflict-free); the
// products q_rot[j] * c[code] are formed in registers with q_rot[j] broadcast from the
// lane that holds it (DPP row_newbcast, folded into v_mul_f32).  Each product is rounded
// to fp32 on its own and added in dim order: the reference's arithmetic, as with the
// per-dim table (csrc/core/turboquant_core.cpp:440-446, 455-483).  A lookup of a wave64
// 4-byte read costs about as much LDS time as an 8-byte one, so the per-dim table's 128
// reads per row bounded the scan near the HBM time; here it is 64.
constexpr int kPsThreads = 768;                 // two blocks per CU (the table is 64 KB)
constexpr int kPsWaves = kPsThreads / 64;
constexpr int kPsBlocksPerScan = 3;             // kThreads-sized scan blocks per pair block
constexpr int kCtabBytes = 256 * 256;           // byte value x 32 copies x (c_hi, c_lo)

// q_rot[j] (row j of this block's broadcast set) from lane (j & 15) of each 16-lane row.
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + N, 0xF, 0xF, false));
}

// acc += q_rot[2P] * c[hi(P)], then acc += q_rot[2P+1] * c[lo(P)] for pair byte P.
template <int P, int NQ>
__device__ __forceinline__ void pair_byte(float& acc, const uint32_t* wds, uint32_t copy8,
                                          const char* ctab, const float (&qv)[NQ]) {
#pragma clang fp contract(off)
  // address = byte << 8 | copy offset: v_perm picks the byte into bits 8-15
  const uint32_t addr = __builtin_amdgcn_perm(wds[P >> 2], copy8, 0x0c0c0000u | ((4u + (P & 3)) << 8));
  const float2 cc = *reinterpret_cast<const float2*>(ctab + addr);
  const float p0 = row_bcast<(2 * P) & 15>(qv[(2 * P) >> 4]) * cc.x;
  acc = acc + p0;
  const float p1 = row_bcast<(2 * P + 1) & 15>(qv[(2 * P) >> 4]) * cc.y;
  acc = acc + p1;
}

// Bytes [G0, G0 + kPairGroup) of a row; a schedule barrier after each group keeps the
// compiler from issuing every table read of the row ahead of the adds (each holds two
// registers until its adds).
constexpr int kPairGroup = 16;
template <int G0, int NQ, int... Ps>
__device__ __forceinline__ void pair_group(float& acc, const uint32_t* wds, uint32_t copy8,
                                           const char* ctab, const float (&qv)[NQ],
                                           std::integer_sequence<int, Ps...>) {
  (pair_byte<G0 + Ps, NQ>(acc, wds, copy8, ctab, qv), ...);
  __builtin_amdgcn_sched_barrier(0);
}

template <int NQ, int... Gs>
__device__ __forceinline__ float pair_row(const uint32_t* wds, uint32_t copy8, const char* ctab,
                                          const float (&qv)[NQ], std::integer_sequence<int, Gs...>) {
  float acc = 0.f;
  (pair_group<Gs * kPairGroup, NQ>(acc, wds, copy8, ctab, qv,
                                   std::make_integer_sequence<int, kPairGroup>{}), ...);
  return acc;
}

// ------------------------------------------------------------------ 2- and 3-bit pair rows
// Rows of 2- or 3-bit codes where each table index covers the two codes of a pair of dims
// (2p, 2p + 1): index = code[2p] << BITS | code[2p + 1].  Bytes per row = the bit-plane
// row's (d * BITS / 8).
//   2 bits: byte b = the indices of pairs 2b (high nibble) and 2b + 1 (low nibble).
//   3 bits: per 32 dims (16 pairs) 12 bytes = words X0, X1, X2: the low 6 bits of byte k of
//           X_i hold pair 4i + k; pair 12 + k's index is spread over bits 6-7 of byte k of
//           X0 (index bits 0-1), X1 (bits 2-3) and X2 (bits 4-5).
// The block's table holds, per pair, every index's two products (fl(q_rot[2p] * c[hi]),
// fl(q_rot[2p + 1] * c[lo])) -- the reference's per-dim LUT values
// (csrc/core/turboquant_core.cpp:440-446) -- so a row costs one 8-byte read and two adds
// (in dim order) per pair and no multiply.  Lanes reading one pair's table touch at most
// 2^(2 BITS) distinct 8-byte entries: conflict-free at 2 bits (128 bytes); at 3 bits the
// 512 bytes wrap the 64 banks twice (indices i and i + 32 share banks), which measured
// faster than splitting each entry over two 256-byte halves read as two b32.
template <int BITS>
constexpr int pmp_pair_bytes() { return (1 << (2 * BITS)) * 8; }

// The row's table reads in groups of 8 pairs, each group's reads issued before the previous
// group's adds (two register buffers), so LDS latency overlaps the add chain; a schedule
// barrier per group keeps the compiler from hoisting every read of the row (128 registers).
// Products are added in pair order: the reference's per-dim order.
template <int BITS>
constexpr int pmp_group() { return BITS == 2 ? 8 : 4; }  // pairs per pipelined group

template <int BITS, int D>
__device__ __forceinline__ void pmp_fetch(const uint32_t* w, const char* ctab, int g,
                                          float2 (&e)[pmp_group<BITS>()]) {
  if constexpr (BITS == 2) {
    // group g = word g: bytes k = 0..3, pairs 8g + 2k (high nibble), 8g + 2k + 1 (low)
    const uint32_t wh = (w[g] >> 1) & 0x78787878u, wl = (w[g] << 3) & 0x78787878u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int p = 8 * g + 2 * k;
      e[2 * k] = *reinterpret_cast<const float2*>(
          ctab + p * pmp_pair_bytes<2>() + __builtin_amdgcn_perm(0u, wh, 0x0c0c0c00u | k));
      e[2 * k + 1] = *reinterpret_cast<const float2*>(
          ctab + (p + 1) * pmp_pair_bytes<2>() + __builtin_amdgcn_perm(0u, wl, 0x0c0c0c00u | k));
    }
  } else {
    // group g = word i of 16-pair block t: pairs 16t + 4i + k (X3 rebuilt from the top bits
    // of X0..X2)
    const int t = g >> 2, i = g & 3;
    const uint32_t* X = w + 3 * t;
    const uint32_t wi = i < 3 ? X[i]
                              : ((X[0] >> 6) & 0x03030303u) | ((X[1] >> 4) & 0x0C0C0C0Cu) |
                                    ((X[2] >> 2) & 0x30303030u);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t idx = __builtin_amdgcn_ubfe(wi, 8 * k, 6);
      e[k] = *reinterpret_cast<const float2*>(ctab + (16 * t + 4 * i + k) * pmp_pair_bytes<3>() + idx * 8);
    }
  }
}

template <int BITS, int D>
__device__ __forceinline__ float pmp_row(const uint32_t* w, const char* ctab) {
#pragma clang fp contract(off)
  constexpr int GP = pmp_group<BITS>();
  constexpr int NG = D / 2 / GP;  // groups per row (even)
  float acc = 0.f;
  float2 ea[GP], eb[GP];
  pmp_fetch<BITS, D>(w, ctab, 0, ea);
#pragma unroll
  for (int g = 0; g < NG; g += 2) {
    pmp_fetch<BITS, D>(w, ctab, g + 1, eb);
#pragma unroll
    for (int q = 0; q < GP; ++q) {
      acc = acc + ea[q].x;
      acc = acc + ea[q].y;
    }
    asm volatile("" : "+v"(acc));  // the adds stay in this group (pure ops float otherwise)
    __builtin_amdgcn_sched_barrier(0);
    if (g + 2 < NG) pmp_fetch<BITS, D>(w, ctab, g + 2, ea);
#pragma unroll
    for (int q = 0; q < GP; ++q) {
      acc = acc + eb[q].x;
      acc = acc + eb[q].y;
    }
    asm volatile("" : "+v"(acc));
    __builtin_amdgcn_sched_barrier(0);
  }
  return acc;
}

// Bitonic sort of one (score, id) per lane over the 64 lanes, best first (score desc, id
// asc).  Pads are (-inf, INT_MAX): every entry is better than a pad.
__device__ __forceinline__ void wave_sort64(float& s, int& id) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float ps = __shfl_xor(s, stride);
      const int pid = __shfl_xor(id, stride);
      // within a best-first run the lower lane keeps the better entry; runs alternate
      const bool keep_better = ((lane & stride) == 0) == ((lane & size) == 0 || size == 64);
      if (keep_better == better(ps, pid, s, id)) { s = ps; id = pid; }
    }
  }
}

// Bitonic sort of 128 entries, element e = lane + 64 r in register r, best first.
__device__ __forceinline__ void wave_sort128(float (&s)[2], int (&id)[2]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 128; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride == 64) {  // partner in this lane's other register; one best-first run
        if (better(s[1], id[1], s[0], id[0])) {
          const float ts = s[0]; s[0] = s[1]; s[1] = ts;
          const int ti = id[0]; id[0] = id[1]; id[1] = ti;
        }
        continue;
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = lane + 64 * r;
        const float ps = __shfl_xor(s[r], stride);
        const int pid = __shfl_xor(id[r], stride);
        const bool keep_better = ((e & stride) == 0) == ((e & size) == 0 || size == 128);
        if (keep_better == better(ps, pid, s[r], id[r])) { s[r] = ps; id[r] = pid; }
      }
    }
  }
}

// Reduce a wave's candidate list to its best min(count, k) in sorted order; th/thi become
// the k-th best once there are k.  Up to 128 entries: a bitonic sort in registers; longer
// lists (k above 64): wave_compact_r's ranking.  Wave-uniform arguments.
__device__ __forceinline__ void wave_compact_sort(float* cs, int* ci, int& count, int k, float& th,
                                                  int& thi) {
  if (count > 128) {  // uniform
    wave_compact_r<kCandRegs>(cs, ci, count, k, th, thi);
    return;
  }
  const int lane = threadIdx.x & 63;
  float s[2];
  int id[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int e = lane + 64 * r;
    s[r] = e < count ? cs[e] : -INFINITY;
    id[r] = e < count ? ci[e] : INT_MAX;
  }
  if (count <= 64) wave_sort64(s[0], id[0]);  // uniform
  else wave_sort128(s, id);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (lane < k && lane < count) { cs[lane] = s[0]; ci[lane] = id[0]; }
  if (lane + 64 < k && lane + 64 < count) { cs[lane + 64] = s[1]; ci[lane + 64] = id[1]; }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  count = count < k ? count : k;
  if (count == k) {
    const bool hi = k > 64;  // uniform: entry k - 1 is in register hi, lane (k - 1) & 63
    th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hi ? s[1] : s[0]), (k - 1) & 63));
    thi = __builtin_amdgcn_readlane(hi ? id[1] : id[0], (k - 1) & 63);
  }
}

// BITS 4: the pair layout with the centroid-pair table and register products above; BITS 2,
// 3: pair rows with the per-block table of products (pmp_row).
// PROD (BITS 2, 3): prod rows -- the MSE half as pair rows, the sign row and the residual
// norm gamma beside it -- scored as scan_kernel<BITS, ..., PROD> scores them, bit for bit:
// the same MSE sum (per-dim LUT products in dim order), the QJL term as a sum of
// build_tables' sign-nibble entries in group order, acc = fma(gamma, sacc, acc).
// Occupancy: two blocks per CU (6 waves per SIMD, 80 VGPRs); the prod variant's sign rows
// need more registers, and spilling them (7 VGPRs, 44.7 MB of scratch writes per 10M-row
// scan) cost more than running one block per CU (190 -> 169 us at 10M x 128).
template <int D, bool TOPK, int BITS = 4, bool PROD = false>
__global__ __launch_bounds__(kPsThreads, PROD ? 4 : 6) void pair_scan_kernel(ScanArgs a) {
#pragma clang fp contract(off)
  static_assert(D == 64 || D == 128, "pair scan dims");
  static_assert(BITS >= 2 && BITS <= 4, "pair rows of 2-4 bit codes");
  static_assert(!PROD || BITS <= 3, "prod pair rows: 2- or 3-bit MSE codes");
  constexpr int SB = D / 8;  // sign bytes per row
  constexpr int RB = D * BITS / 8;  // bytes per row
  constexpr int NW = RB / 4;        // 32-bit words per row
  constexpr int NQ = D / 16;        // q_rot registers
  static_assert(BITS != 4 || RB % kPairGroup == 0, "whole byte groups per row");
  constexpr int CT = BITS == 4 ? kCtabBytes : (D / 2) * pmp_pair_bytes<BITS>();
  __shared__ __attribute__((aligned(16))) char ctab[CT];
  __shared__ __attribute__((aligned(16))) char sgn_s[PROD ? D * 16 : 16];  // (D/4) x 16 entries
  __shared__ float qs_s[D];
  __shared__ float qr_s[D];
  __shared__ float qss_s[PROD ? D : 1];
  __shared__ float cen_s[16];
  // TOPK: kPsWaves lists of a.ccap (score, id) slots in dynamic LDS
  extern __shared__ __attribute__((aligned(16))) char dyn_s[];
  const int ccap = TOPK ? a.ccap : 0;
  float* cand_s = reinterpret_cast<float*>(dyn_s);
  int* cand_i = reinterpret_cast<int*>(dyn_s) + kPsWaves * ccap;
  __shared__ int cnt_s[TOPK ? kPsWaves : 1];
  __shared__ float bnd_s;
  __shared__ int bnd_i;

  const int s = blockIdx.z;
  const int q0 = s * a.qps + blockIdx.y;  // this block's query
  if (a.qflag && !a.qflag[blockIdx.y]) return;  // only flagged queries are scanned (uniform)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int tid = threadIdx.x;

  // ---- this wave's rows
  int64_t nrows = a.nrows;
  if (a.seq_lens) {
    const int64_t sl = a.seq_lens[s / a.spb];
    nrows = sl < a.stream_rows ? sl : a.stream_rows;
  }
  const int64_t per_block = ((nrows + gridDim.x - 1) / gridDim.x + 63) / 64 * 64;
  const int64_t rbeg = (int64_t)blockIdx.x * per_block;
  const int64_t rend = min(nrows, rbeg + per_block);
  const uint8_t* base = a.packed + (size_t)s * a.stream_rows * RB;
  const float* nbase = a.norms + (size_t)s * a.stream_rows;

  struct RowBuf {
    uint32_t w[NW];
    float n;
    uint32_t sw[PROD ? SB / 4 : 1];  // prod: sign row
    float g;                          // prod: residual norm
  };
  const uint32_t nbr = (uint32_t)(rend > rbeg ? rend - rbeg : 0);
  const __amdgpu_buffer_rsrc_t rows_rs = buf_rsrc(base + rbeg * RB, nbr * (uint32_t)RB);
  const __amdgpu_buffer_rsrc_t norm_rs = buf_rsrc(nbase + rbeg, nbr * 4u);
  const __amdgpu_buffer_rsrc_t sgn_rs =
      buf_rsrc(PROD ? a.signs + ((size_t)s * a.stream_rows + rbeg) * SB : a.packed, PROD ? nbr * (uint32_t)SB : 0u);
  const __amdgpu_buffer_rsrc_t gam_rs =
      buf_rsrc(PROD ? a.gammas + (size_t)s * a.stream_rows + rbeg : a.norms, PROD ? nbr * 4u : 0u);
  auto load_row = [&](int64_t r, RowBuf& b) {
    const uint32_t rr = (uint32_t)(r - rbeg);
    const int off = (int)(rr * (uint32_t)RB);
#pragma unroll
    for (int i = 0; i < RB / 16; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rows_rs, off, 16 * i, 0);
      b.w[4 * i + 0] = v.x; b.w[4 * i + 1] = v.y; b.w[4 * i + 2] = v.z; b.w[4 * i + 3] = v.w;
    }
    if constexpr (RB % 16 == 8) {  // 3-bit rows of 64 dims: 24 bytes
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rows_rs, off, RB - 8, 0);
      b.w[NW - 2] = v.x; b.w[NW - 1] = v.y;
    }
    b.n = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(norm_rs, (int)(rr * 4u), 0, kNT));
    if constexpr (PROD) {
      if constexpr (SB == 16) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(sgn_rs, (int)(rr * 16u), 0, 0);
        b.sw[0] = v.x; b.sw[1] = v.y; b.sw[2] = v.z; b.sw[3] = v.w;
      } else {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(sgn_rs, (int)(rr * 8u), 0, 0);
        b.sw[0] = v.x; b.sw[1] = v.y;
      }
      b.g = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(gam_rs, (int)(rr * 4u), 0, kNT));
    }
  };

  constexpr int64_t kStride = kPsWaves * 64;
  const int64_t first = rbeg + wave * 64;
  int64_t row = first + lane;
  const int nsteps = __builtin_amdgcn_readfirstlane(
      first < rend ? (int)((rend - first + kStride - 1) / kStride) : 0);
  // ---- query rotation (build_tables' arithmetic) and the centroid-pair table
  if (tid < D) qs_s[tid] = load_as_f32(a.q, (int64_t)q0 * D + tid, a.q_dt);
  else if (tid < D + 16) cen_s[tid - D] = a.cen[tid - D];
  __syncthreads();
  if (tid < D) {
    const float* r = a.rot + (size_t)tid * D;
    float v = 0.f;
#pragma unroll 4
    for (int k = 0; k < D; k += 4) {
      const float4 r4 = *reinterpret_cast<const float4*>(r + k);
      v = v + qs_s[k] * r4.x;
      v = v + qs_s[k + 1] * r4.y;
      v = v + qs_s[k + 2] * r4.z;
      v = v + qs_s[k + 3] * r4.w;
    }
    qr_s[tid] = v;
  } else if (PROD && tid >= 2 * D && tid < 3 * D) {  // S q, build_tables' arithmetic
    const int j = tid - 2 * D;
    const float* sr = a.qjl + (size_t)j * D;
    float w = 0.f;
    for (int k = 0; k < D; k += 4) {
      const float4 s4 = *reinterpret_cast<const float4*>(sr + k);
      w = fmaf(qs_s[k], s4.x, w);
      w = fmaf(qs_s[k + 1], s4.y, w);
      w = fmaf(qs_s[k + 2], s4.z, w);
      w = fmaf(qs_s[k + 3], s4.w, w);
    }
    qss_s[j] = w;
  }
  if constexpr (BITS == 4) {
    for (int e = tid; e < 256 * 16; e += kPsThreads) {  // entry b, copies 2c and 2c + 1
      const int b = e >> 4, c = e & 15;
      const float hi = cen_s[b >> 4], lo = cen_s[b & 15];
      *reinterpret_cast<float4*>(ctab + b * 256 + c * 16) = make_float4(hi, lo, hi, lo);
    }
  }
  __syncthreads();
  if constexpr (BITS != 4) {  // products of pair p, index i (i = hi << BITS | lo)
    constexpr int L = 1 << BITS;
    for (int e = tid; e < (D / 2) * L * L; e += kPsThreads) {
      const int pp = e / (L * L), i = e - pp * (L * L);
      *reinterpret_cast<float2*>(ctab + e * 8) =
          make_float2(qr_s[2 * pp] * cen_s[i >> BITS], qr_s[2 * pp + 1] * cen_s[i & (L - 1)]);
    }
    if constexpr (PROD) {  // sign-nibble entries (g, v), layout (g>>1)*128 + v*8 + (g&1)*4
      for (int e = tid; e < D * 4; e += kPsThreads) {
        const int g = e >> 4, v = e & 15;
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = qss_s[4 * g + i];
          t += ((v >> (3 - i)) & 1) ? x : -x;
        }
        *reinterpret_cast<float*>(sgn_s + (g >> 1) * 128 + v * 8 + (g & 1) * 4) = t * a.qjl_scale;
      }
    }
    __syncthreads();
  }
  float qv[NQ];
#pragma unroll
  for (int m = 0; m < NQ; ++m) qv[m] = qr_s[16 * m + (lane & 15)];
  const uint32_t copy8 = (uint32_t)(lane & 31) * 8;

  float th = -INFINITY;
  int thi = INT_MAX;
  int cnt = 0;
  float* cs = cand_s + wave * ccap;
  int* ci = cand_i + wave * ccap;

  auto score = [&](const RowBuf& rb) {
    float acc;
    if constexpr (BITS == 4) {
      // The broadcasts of qv are loop-invariant: hoisted, each would hold a register of its
      // own (128 for d = 128).  Redefining qv here keeps them inside the multiplies.
#pragma unroll
      for (int m = 0; m < NQ; ++m) asm volatile("" : "+v"(qv[m]));
      acc = pair_row<NQ>(rb.w, copy8, ctab, qv, std::make_integer_sequence<int, RB / kPairGroup>{});
    } else {
      acc = pmp_row<BITS, D>(rb.w, ctab);
    }
    if constexpr (PROD) {
      float sacc = 0.f;
#pragma unroll
      for (int w = 0; w < SB / 4; ++w)
        decode_pairs<8>(rb.sw[w], 8 * w, [&](int g, uint32_t addr) {
          sacc += *reinterpret_cast<const float*>(sgn_s + (g >> 1) * 128 + (g & 1) * 4 + addr);
        });
      acc = fmaf(rb.g, sacc, acc);
    }
    float sc = acc * rb.n * a.post_scale;
    // materialized here: sunk into a branch that uses it, the products would be split
    // from their broadcasts (a DPP move cannot move into divergent code)
    asm volatile("" : "+v"(sc));
    return sc;
  };
  // Steps after the first: list the rows that beat the bound (th, thi).
  auto step = [&](const RowBuf& rb, const int64_t row) {
    const float sc = score(rb);
    const bool valid = row < rend;
    if constexpr (TOPK) {
      const int id = (int)row;
      bool pred = valid & better(sc, id, th, thi);
      uint64_t mask = __ballot(pred);
      int nnew = __popcll(mask);
      if (nnew == 0) return;
      if (cnt + nnew > ccap) {
        const float bs = th;
        const int bi = thi;
        wave_compact_sort(cs, ci, cnt, a.k, th, thi);
        if (better(bs, bi, th, thi)) { th = bs; thi = bi; }  // keep the block bound
        pred = valid & better(sc, id, th, thi);
        mask = __ballot(pred);
        nnew = __popcll(mask);
      }
      if (pred) {
        const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
        cs[pos] = sc;
        ci[pos] = id;
      }
      cnt += nnew;
    } else {
      if (valid) a.scores[(size_t)q0 * a.stream_rows + row] = sc;
    }
  };

  RowBuf ta, tb;
  if (nsteps > 0) load_row(row, ta);
  if (nsteps > 1) load_row(row + kStride, tb);
  // ---- step 0 of every wave (waves without rows take part with nothing valid)
  {
    const float sc = nsteps > 0 ? score(ta) : 0.f;
    const bool valid = nsteps > 0 && row < rend;
    if constexpr (TOPK) {
      // Keep the best k of the wave's first 64 rows (a sort across the lanes).  NaN
      // scores are never listed: no comparison with a bound holds for them.
      const bool real = valid && !__builtin_isnan(sc);
      float ss = real ? sc : -INFINITY;
      int ii = real ? (int)row : INT_MAX;
      wave_sort64(ss, ii);
      const int nreal = __popcll(__ballot(real));
      if (lane < a.k && lane < nreal) { cs[lane] = ss; ci[lane] = ii; }
      cnt = nreal < a.k ? nreal : a.k;
      if (cnt == a.k) {
        th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), a.k - 1));
        thi = __builtin_amdgcn_readlane(ii, a.k - 1);
      }
      if (lane == 0) cnt_s[wave] = cnt;
      __syncthreads();
      // Block bound: the k-th best of the waves' first-step lists (up to 10 entries from
      // each, sorted) bounds the block's answer from below, so every wave lists only rows
      // that beat it: about 20 more per wave instead of a refill of its list.
      constexpr int kTake = 128 / kPsWaves;
      if (wave == 0) {
        float sv[2];
        int iv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int e = lane + 64 * r;
          const int w = e / kTake, j = e - w * kTake;
          const bool ok = w < kPsWaves && j < cnt_s[w < kPsWaves ? w : 0];
          sv[r] = ok ? cand_s[w * ccap + j] : -INFINITY;
          iv[r] = ok ? cand_i[w * ccap + j] : INT_MAX;
        }
        wave_sort128(sv, iv);
        const bool hi = a.k > 64;  // uniform: entry k - 1 in register hi
        const float bs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hi ? sv[1] : sv[0]), (a.k - 1) & 63));
        const int bi = __builtin_amdgcn_readlane(hi ? iv[1] : iv[0], (a.k - 1) & 63);
        if (lane == 0) { bnd_s = bs; bnd_i = bi; }  // (-inf, INT_MAX): fewer than k rows
      }
      __syncthreads();
      const float bs = bnd_s;
      const int bi = bnd_i;
      if (bi != INT_MAX && better(bs, bi, th, thi)) { th = bs; thi = bi; }
    } else {
      if (valid) a.scores[(size_t)q0 * a.stream_rows + row] = sc;
    }
  }
  row += kStride;
  // tb holds step 1's rows
  for (int it = 1; it < nsteps; it += 2) {
    load_row(row + kStride, ta);
    step(tb, row);
    row += kStride;
    if (it + 1 >= nsteps) break;
    load_row(row + kStride, tb);
    step(ta, row);
    row += kStride;
  }

  if constexpr (TOPK) {
    // every wave list leaves sorted (best first) with at most k entries
    if (cnt > 1) wave_compact_sort(cs, ci, cnt, a.k, th, thi);
    if (lane == 0) cnt_s[wave] = cnt;
    __syncthreads();
    int total = 0;
    int off[kPsWaves];
#pragma unroll
    for (int w = 0; w < kPsWaves; ++w) { off[w] = total; total += cnt_s[w]; }
    float* ps = a.part_s + ((size_t)q0 * gridDim.x + blockIdx.x) * a.k;
    int32_t* pi = a.part_i + ((size_t)q0 * gridDim.x + blockIdx.x) * a.k;
    if (total <= 128) {  // uniform; wave 0 sorts the union
      if (wave == 0) {
        float sv[2];
        int iv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int e = lane + 64 * r;
          int w = 0;
#pragma unroll
          for (int t = 1; t < kPsWaves; ++t) w += (e >= off[t]);
          const bool ok = e < total;
          sv[r] = ok ? cand_s[w * ccap + e - off[w]] : -INFINITY;
          iv[r] = ok ? cand_i[w * ccap + e - off[w]] : INT_MAX;
        }
        wave_sort128(sv, iv);
        if (lane < a.k) {
          ps[lane] = lane < total ? sv[0] : -INFINITY;
          pi[lane] = lane < total ? iv[0] : -1;
        }
        if (lane + 64 < a.k) {
          ps[lane + 64] = lane + 64 < total ? sv[1] : -INFINITY;
          pi[lane + 64] = lane + 64 < total ? iv[1] : -1;
        }
      }
    } else {
      // an entry's rank: its slot in its own sorted list plus, per other wave's list, the
      // entries better than it (binary search); total > 128 >= k, so no pads
      for (int e = threadIdx.x; e < total; e += kPsThreads) {
        int w = 0;
#pragma unroll
        for (int t = 1; t < kPsWaves; ++t) w += (e >= off[t]);
        const int slot = e - off[w];
        const float se = cand_s[w * ccap + slot];
        const int ie = cand_i[w * ccap + slot];
        int rank = slot;
#pragma unroll
        for (int t = 0; t < kPsWaves; ++t)
          if (t != w) rank += sorted_rank(cand_s + t * ccap, cand_i + t * ccap, cnt_s[t], se, ie);
        if (rank < a.k) { ps[rank] = se; pi[rank] = ie; }
      }
    }
  }
}

// ------------------------------------------------------------------ merge
constexpr int kMergeCap = 512;       // survivors kept for the rank sort (more: exact fallback)
constexpr int kMaxBlocksPerLane = 8;  // merge handles up to 64 * 4 * 8 = 2048 block lists

// Wave-wide arg-best over per-lane candidates (score desc, id asc); returns the
// winner's (score, id) in every lane.  Lanes with id == INT_MAX hold nothing.  Uses DPP
// row operations (quad swaps, row mirrors, row broadcasts), a few cycles each, rather than
// LDS-routed shuffles: this runs in single-block kernels where latency is the cost.
template <int CTRL, int ROWS>
__device__ __forceinline__ void best_step(float& s, int& id) {
  const int so_bits = __builtin_amdgcn_update_dpp(__float_as_int(s), __float_as_int(s), CTRL, ROWS, 0xF, false);
  const int io = __builtin_amdgcn_update_dpp(id, id, CTRL, ROWS, 0xF, false);
  const float so = __int_as_float(so_bits);
  const bool take = (io != INT_MAX) & ((id == INT_MAX) | better(so, io, s, id));
  s = take ? so : s;
  id = take ? io : id;
}

__device__ __forceinline__ void wave_best(float& s, int& id) {
  best_step<0xB1, 0xF>(s, id);   // quad_perm [1,0,3,2]
  best_step<0x4E, 0xF>(s, id);   // quad_perm [2,3,0,1]
  best_step<0x141, 0xF>(s, id);  // row_half_mirror: 8-lane groups
  best_step<0x140, 0xF>(s, id);  // row_mirror: 16-lane rows
  best_step<0x142, 0xA>(s, id);  // row_bcast15 into rows 1 and 3
  best_step<0x143, 0xC>(s, id);  // row_bcast31 into rows 2 and 3
  s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 63));
  id = __builtin_amdgcn_readlane(id, 63);
}

// Per query.  tau = the k-th best of 64 group maxima (group = the block lists of 4
// adjacent threads) is a lower bound of the k-th best score overall: those k maxima are
// k distinct rows.  Only list entries at or above tau can be in the answer; they are
// rank-sorted.  Every step is a fixed number of passes (no per-k rounds of wave
// reductions, whose DPP chains cost about a microsecond each).
// Runs on all kThreads threads of a block (it synchronizes), for query q.
__device__ void merge_query(const float* __restrict__ part_s, const int32_t* __restrict__ part_i,
                            int nblocks, int k, int q, float* __restrict__ out_s,
                            int64_t* __restrict__ out_i) {
  static_assert(kThreads == 256, "64 groups of 4 threads");
  __shared__ __attribute__((aligned(16))) float gs[64];
  __shared__ __attribute__((aligned(16))) int gi[64];
  __shared__ float ss[kMergeCap];
  __shared__ int si[kMergeCap];
  __shared__ int nsurv;
  __shared__ int nlists;
  __shared__ int lists[kMergeCap];
  __shared__ float tau_s;
  __syncthreads();  // the shared buffers may still be read by a previous call
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float* ps = part_s + (size_t)q * nblocks * k;
  const int32_t* pi = part_i + (size_t)q * nblocks * k;
  // 1. block maxima (block b's list is sorted, entry 0 = its max), then each group's best
  float ms[kMaxBlocksPerLane];
  int mi[kMaxBlocksPerLane];
  // Every load is issued unconditionally (clamped index) so all of them are in flight
  // together: these lists were just written on other XCDs and each load is a far miss.
#pragma unroll
  for (int r = 0; r < kMaxBlocksPerLane; ++r) {
    const int b = threadIdx.x + r * kThreads;
    const size_t bc = (size_t)(b < nblocks ? b : nblocks - 1) * k;
    const int id = pi[bc];
    const float sc = ps[bc];
    const bool ok = b < nblocks && id >= 0;
    ms[r] = ok ? sc : -INFINITY;
    mi[r] = ok ? id : INT_MAX;
  }
  float bs = -INFINITY;
  int bi = INT_MAX;
#pragma unroll
  for (int t = 0; t < kMaxBlocksPerLane; ++t) {
    const bool take = (mi[t] != INT_MAX) & ((bi == INT_MAX) | better(ms[t], mi[t], bs, bi));
    bs = take ? ms[t] : bs;
    bi = take ? mi[t] : bi;
  }
  best_step<0xB1, 0xF>(bs, bi);  // quad_perm [1,0,3,2]
  best_step<0x4E, 0xF>(bs, bi);  // quad_perm [2,3,0,1]
  if ((lane & 3) == 0) { gs[threadIdx.x >> 2] = bs; gi[threadIdx.x >> 2] = bi; }
  if (threadIdx.x == 0) { nsurv = 0; nlists = 0; tau_s = -INFINITY; }
  __syncthreads();
  // 2. wave 0: rank of each group maximum among the 64 (a strict order: score, then id);
  // the one ranked k-1 is tau.  With fewer than k non-empty groups tau stays -inf.
  if (wave == 0) {
    const float s0 = gs[lane];
    const int i0 = gi[lane];
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < 64; j += 4) {
      const float4 s4 = *reinterpret_cast<const float4*>(gs + j);
      const int4 i4 = *reinterpret_cast<const int4*>(gi + j);
      rank += (i4.x != INT_MAX) & better(s4.x, i4.x, s0, i0);
      rank += (i4.y != INT_MAX) & better(s4.y, i4.y, s0, i0);
      rank += (i4.z != INT_MAX) & better(s4.z, i4.z, s0, i0);
      rank += (i4.w != INT_MAX) & better(s4.w, i4.w, s0, i0);
    }
    if (i0 != INT_MAX && rank == k - 1) tau_s = s0;
  }
  __syncthreads();
  const float tau = tau_s;
  // 3. survivors: only lists whose maximum reaches tau can hold any.  Collect those
  // lists, then read all their entries at once.
  const int total = nblocks * k;
#pragma unroll
  for (int r = 0; r < kMaxBlocksPerLane; ++r) {
    const int b = threadIdx.x + r * kThreads;
    if (b < nblocks && mi[r] != INT_MAX && ms[r] >= tau) {
      const int pos = atomicAdd(&nlists, 1);
      if (pos < kMergeCap) lists[pos] = b;
    }
  }
  __syncthreads();
  const int nl_all = nlists;
  const int nl = min(nl_all, kMergeCap);
  for (int e = threadIdx.x; e < nl * k; e += kThreads) {
    const int li = e / k;
    const size_t at = (size_t)lists[li] * k + (e - li * k);
    const int id = pi[at];
    const float sc = ps[at];
    if (id >= 0 && sc >= tau) {
      const int pos = atomicAdd(&nsurv, 1);
      if (pos < kMergeCap) { ss[pos] = sc; si[pos] = id; }
    }
  }
  __syncthreads();
  const int m = nsurv;
  float* os = out_s + (size_t)q * k;
  int64_t* oi = out_i + (size_t)q * k;
  // More than kMergeCap lists (or survivors) means many rows tie at tau: exact fallback.
  if (m <= kMergeCap && nl_all <= kMergeCap) {
    for (int e = threadIdx.x; e < m; e += kThreads) {
      const float se = ss[e];
      const int ie = si[e];
      int rank = 0;
      for (int f = 0; f < m; ++f) rank += better(ss[f], si[f], se, ie);
      if (rank < k) { os[rank] = se; oi[rank] = ie; }
    }
    for (int e = m + threadIdx.x; e < k; e += kThreads) { os[e] = -INFINITY; oi[e] = -1; }
    return;  // uniform: every thread of the block takes the same branch
  }
  // 4. more than kMergeCap rows tie at tau: k rounds of block arg-best over everything
  __shared__ float bs_s[kWaves];
  __shared__ int bi_s[kWaves];
  float last_s = INFINITY;
  int last_i = -1;
  for (int r = 0; r < k; ++r) {
    float cs = -INFINITY;
    int ci = INT_MAX;
    for (int e = threadIdx.x; e < total; e += kThreads) {
      const int id = pi[e];
      const float sc = ps[e];
      if (id < 0 || !better(last_s, last_i, sc, id)) continue;  // emitted already
      if (ci == INT_MAX || better(sc, id, cs, ci)) { cs = sc; ci = id; }
    }
    wave_best(cs, ci);
    if (lane == 0) { bs_s[wave] = cs; bi_s[wave] = ci; }
    __syncthreads();
    cs = bs_s[0];
    ci = bi_s[0];
    for (int w = 1; w < kWaves; ++w)
      if ((bi_s[w] != INT_MAX) & ((ci == INT_MAX) | better(bs_s[w], bi_s[w], cs, ci))) { cs = bs_s[w]; ci = bi_s[w]; }
    __syncthreads();
    last_s = cs;
    last_i = ci;
    if (threadIdx.x == 0) {
      os[r] = ci == INT_MAX ? -INFINITY : cs;
      oi[r] = ci == INT_MAX ? -1 : ci;
    }
  }
}

// merge_query for at most kThreads * kMergeRegs list entries: every entry is loaded
// once, in one round of coalesced loads, and stays in registers -- tau (as in
// merge_query, from 64 group maxima, a group being the entries of 4 adjacent threads) and
// the survivors come from there without a second round trip to memory.
constexpr int kMergeRegs = 24;
__device__ void merge_query_regs(const float* __restrict__ part_s, const int32_t* __restrict__ part_i,
                                 int nblocks, int k, int q, float* __restrict__ out_s,
                                 int64_t* __restrict__ out_i) {
  __shared__ __attribute__((aligned(16))) float gs[64];
  __shared__ __attribute__((aligned(16))) int gi[64];
  __shared__ float ss[kMergeCap];
  __shared__ int si[kMergeCap];
  __shared__ int nsurv;
  __shared__ float tau_s;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int total = nblocks * k;
  const float* ps = part_s + (size_t)q * total;
  const int32_t* pi = part_i + (size_t)q * total;
  float es[kMergeRegs];
  int ei[kMergeRegs];
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) {
    const int e = threadIdx.x + r * kThreads;
    const int ec = e < total ? e : total - 1;
    const float sc = ps[ec];
    const int id = pi[ec];
    const bool ok = (e < total) & (id >= 0);
    es[r] = ok ? sc : -INFINITY;
    ei[r] = ok ? id : INT_MAX;
  }
  float bs = -INFINITY;
  int bi = INT_MAX;
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) {
    const bool take = (ei[r] != INT_MAX) & ((bi == INT_MAX) | better(es[r], ei[r], bs, bi));
    bs = take ? es[r] : bs;
    bi = take ? ei[r] : bi;
  }
  best_step<0xB1, 0xF>(bs, bi);  // quad_perm [1,0,3,2]
  best_step<0x4E, 0xF>(bs, bi);  // quad_perm [2,3,0,1]
  if ((lane & 3) == 0) { gs[threadIdx.x >> 2] = bs; gi[threadIdx.x >> 2] = bi; }
  if (threadIdx.x == 0) { nsurv = 0; tau_s = -INFINITY; }
  __syncthreads();
  if (wave == 0) {
    const float s0 = gs[lane];
    const int i0 = gi[lane];
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < 64; j += 4) {
      const float4 s4 = *reinterpret_cast<const float4*>(gs + j);
      const int4 i4 = *reinterpret_cast<const int4*>(gi + j);
      rank += (i4.x != INT_MAX) & better(s4.x, i4.x, s0, i0);
      rank += (i4.y != INT_MAX) & better(s4.y, i4.y, s0, i0);
      rank += (i4.z != INT_MAX) & better(s4.z, i4.z, s0, i0);
      rank += (i4.w != INT_MAX) & better(s4.w, i4.w, s0, i0);
    }
    if ((i0 != INT_MAX) & (rank == k - 1)) tau_s = s0;
  }
  __syncthreads();
  const float tau = tau_s;
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) {
    if (ei[r] != INT_MAX && es[r] >= tau) {
      const int pos = atomicAdd(&nsurv, 1);
      if (pos < kMergeCap) { ss[pos] = es[r]; si[pos] = ei[r]; }
    }
  }
  __syncthreads();
  const int m = nsurv;
  float* os = out_s + (size_t)q * k;
  int64_t* oi = out_i + (size_t)q * k;
  if (m <= kMergeCap) {
    for (int e = threadIdx.x; e < m; e += kThreads) {
      const float se = ss[e];
      const int ie = si[e];
      int rank = 0;
      for (int f = 0; f < m; ++f) rank += better(ss[f], si[f], se, ie);
      if (rank < k) { os[rank] = se; oi[rank] = ie; }
    }
    for (int e = m + threadIdx.x; e < k; e += kThreads) { os[e] = -INFINITY; oi[e] = -1; }
    return;  // uniform
  }
  // more than kMergeCap rows tie at tau: the general path (its exact fallback)
  merge_query(part_s, part_i, nblocks, k, q, out_s, out_i);
}

__device__ void merge_query_big(const float* __restrict__ part_s, const int32_t* __restrict__ part_i,
                                int nblocks, int k, int q, float* __restrict__ out_s,
                                int64_t* __restrict__ out_i);

__global__ __launch_bounds__(kThreads) void merge_kernel(const float* __restrict__ part_s,
                                                         const int32_t* __restrict__ part_i,
                                                         int nblocks, int k,
                                                         float* __restrict__ out_s,
                                                         int64_t* __restrict__ out_i,
                                                         const int32_t* __restrict__ qflag) {
  if (qflag && !qflag[blockIdx.x]) return;  // only flagged queries (uniform)
  if (k > kSmallK)  // uniform
    merge_query_big(part_s, part_i, nblocks, k, blockIdx.x, out_s, out_i);
  else if (nblocks * k <= kThreads * kMergeRegs)  // uniform
    merge_query_regs(part_s, part_i, nblocks, k, blockIdx.x, out_s, out_i);
  else
    merge_query(part_s, part_i, nblocks, k, blockIdx.x, out_s, out_i);
}

// ------------------------------------------------------------------ filtered pair scan
// One-query top-k over 4-bit pair-layout rows (d = 64 / 128) whose answer carries the
// reference's exact scores (csrc/core/turboquant_core.cpp:455-494: per-dim products
// q_rot[j] * c[code] rounded one by one, added in dim order, times the norm; strict '>'
// with the lower index winning ties).
//
// Filter.  An approximate score per row on the matrix cores.  A code byte is a table
// index; one 4-byte LDS read returns the fp16 centroid pair (c[hi], c[lo]), which is
// exactly what v_mfma_f32_16x16x32_f16 takes as B operand (16 rows x 32 dims per MFMA).
// The A operand holds the rotated query, scaled by a power of two and split into fp16 hi
// + lo parts, in rows 0 and 1.  Per 64 rows that is 64 table reads, 16 MFMAs and a few
// dozen VALU instructions, against 128 multiplies and 128 dependent adds per row for the
// reference's arithmetic: the scan runs at the HBM streaming rate instead of the VALU
// rate.
//   Bound: |approx - exact| <= |n| * beta with
//     beta = ||q_rot||_1 * (e_c + 2^-14 max|c|) * (1 + 2^-10),  e_c = max_i |c_i - fp16(c_i)|.
//   Terms, each times ||q_rot||_1: the fp16 centroids e_c (computed, not assumed: inf when a
//   centroid overflows fp16, which turns the filter off); the hi + lo query split 2^-22
//   max|c| (plus 128 * 2^-25 / scale, far below); fp32 accumulation of the 256 exact
//   products of the MFMAs, 256 * 2^-23 max|c|; the reference's own sequential sum,
//   128 * 2^-24 max|c|; the two final multiplies by n, 2^-23 max|c|: 2^-14.5 max|c| in all
//   but e_c.  The (1 + 2^-10) covers the rounding of ||q_rot||_1 and of sa +- B (B >= 2^-14
//   |sa| / (1 + 2^-10), so rounding sa + B moves it by less than 2^-10 B).  For the 4-bit
//   Lloyd-Max tables e_c = 2^-12.1 max|c| (d = 128) and 2^-11.6 max|c| (d = 64); the worst
//   |approx - exact| measured on 12M random and adversarial rows was 2^-12.3 ||q||_1 max|c|.
//   Each row gets lo = approx - B and hi = approx + B.  Every wave keeps (th, thi) = the
//   k-th best (lo, id) over the rows it has seen -- k distinct rows score at least their
//   lo, so the k-th best exact (score, id) is at least (th, thi) -- and lists a row only
//   when (hi, id) reaches it; a row below it cannot be in the answer.  A listed row's code
//   bytes and norm are copied from the registers they arrived in to LDS beside its list
//   entry, so rescoring it exactly never reads memory again.  A list that stays full after
//   pruning (near-ties, duplicate rows) is rescored exactly in place, which leaves at most
//   k entries.  Waves share th through LDS.  At the end every wave rescores its list
//   exactly (at most k entries remain), each entry is ranked against the block's other
//   waves' entries, and the block writes its exact top k.
// Merge (filter_merge_kernel): the top k of the block lists.
constexpr int kFsThreads = 512;   // 8 waves; one block per CU
constexpr int kFsWaves = kFsThreads / 64;
constexpr int kFsCap = 128;       // candidate slots per wave
constexpr int kFsEager = 48;      // a list this long is pruned (and th published) at once
constexpr int kHtabBytes = 256 * 256;  // byte value x 64 lane copies x fp16 centroid pair

struct FilterArgs {
  const uint8_t* rows;  // [n][D / 2] pair layout
  const float* norms;   // [n]
  int64_t n;
  const void* q;        // [nq][D]
  int q_dt;
  const float* rot;     // [D][D]
  const float* cen;     // [16]
  int k;
  float* bs;            // [nq][nblocks][k] block lists: exact scores, best first
  int32_t* bi;          // ids; -1 past the list's length
  float* out_s;         // [nq][k]
  int64_t* out_i;
};

typedef _Float16 fs_v8h __attribute__((ext_vector_type(8)));
typedef float fs_v4f __attribute__((ext_vector_type(4)));

// Exact score of one pair-layout row (byte p = codes 2p (high nibble) and 2p + 1): the
// reference's arithmetic, as pair_scan_kernel.  `row` is 16-byte aligned (LDS here).
template <int D>
__device__ __forceinline__ float exact_pair_score(const uint8_t* __restrict__ row, float n,
                                                  const float* qr, const float* cen) {
#pragma clang fp contract(off)
  float acc = 0.f;
  const u32x4* r4 = reinterpret_cast<const u32x4*>(row);
#pragma unroll 1
  for (int i = 0; i < D / 32; ++i) {
    const u32x4 v = r4[i];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int p = 16 * i + 4 * wi + b;
        const uint32_t byte = (w[wi] >> (8 * b)) & 0xFFu;
        const float p0 = qr[2 * p] * cen[byte >> 4];
        acc = acc + p0;
        const float p1 = qr[2 * p + 1] * cen[byte & 15u];
        acc = acc + p1;
      }
    }
  }
  return acc * n;
}

// exact_pair_score from a product table: ptab[16 j + i] = qr[j] * cen[i] (the same fp32
// products), so each dim costs one table read (the row's nibbles pre-shifted to byte
// offsets, the dim's 64-byte stride in the read's immediate offset) and the add, in the
// same order.  `row` and `ptab` in LDS, `row` 16-byte aligned.
template <int D>
__device__ __forceinline__ float exact_pair_score_ptab(const uint32_t* row, float n,
                                                       const float* ptab) {
#pragma clang fp contract(off)
  const char* pt = reinterpret_cast<const char*>(ptab);
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    const u32x4 v = reinterpret_cast<const u32x4*>(row)[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      const uint32_t h4 = (w[wi] >> 2) & 0x3C3C3C3Cu;  // byte b: 4 * (high nibble)
      const uint32_t l4 = (w[wi] << 2) & 0x3C3C3C3Cu;  // byte b: 4 * (low nibble)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int pg = 16 * c + 4 * wi + b;
        acc = acc + *reinterpret_cast<const float*>(pt + 128 * pg + ((h4 >> (8 * b)) & 0xFFu));
        acc = acc + *reinterpret_cast<const float*>(pt + 128 * pg + 64 + ((l4 >> (8 * b)) & 0xFFu));
      }
    }
  }
  return acc * n;
}

// exact_pair_score for a row held in registers (word w = bytes 4w .. 4w + 3).
template <int D>
__device__ __forceinline__ float exact_pair_score_regs(const uint32_t (&rw)[D / 8], float n,
                                                       const float* qr, const float* cen) {
#pragma clang fp contract(off)
  float acc = 0.f;
#pragma unroll
  for (int w = 0; w < D / 8; ++w)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int p = 4 * w + b;
      const uint32_t byte = (rw[w] >> (8 * b)) & 0xFFu;
      const float p0 = qr[2 * p] * cen[byte >> 4];
      acc = acc + p0;
      const float p1 = qr[2 * p + 1] * cen[byte & 15u];
      acc = acc + p1;
    }
  return acc * n;
}

// The same for a pair row of BITS-bit codes (layouts above pmp_row): products
// q_rot[j] * c[code_j] added in dim order, then times the norm.
template <int D, int BITS>
__device__ __forceinline__ float exact_row_score_regs(const uint32_t (&rw)[D * BITS / 32], float n,
                                                      const float* qr, const float* cen) {
#pragma clang fp contract(off)
  if constexpr (BITS == 4) {
    return exact_pair_score_regs<D>(rw, n, qr, cen);
  } else if constexpr (BITS == 2) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < D / 16; ++w)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (rw[w] >> (8 * b)) & 0xFFu;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float p = qr[16 * w + 4 * b + c] * cen[(byte >> (6 - 2 * c)) & 3u];
          acc = acc + p;
        }
      }
    return acc * n;
  } else {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < D / 32; ++t) {
      const uint32_t* X = rw + 3 * t;
      const uint32_t x3 = ((X[0] >> 6) & 0x03030303u) | ((X[1] >> 4) & 0x0C0C0C0Cu) |
                          ((X[2] >> 2) & 0x30303030u);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wi = i < 3 ? X[i] : x3;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int p = 16 * t + 4 * i + k;
          const uint32_t idx = (wi >> (8 * k)) & 63u;
          const float p0 = qr[2 * p] * cen[idx >> 3];
          acc = acc + p0;
          const float p1 = qr[2 * p + 1] * cen[idx & 7u];
          acc = acc + p1;
        }
      }
    }
    return acc * n;
  }
}

__device__ __forceinline__ bool fs_keep(float hi, int id, float th, int thi) {
  return (hi > th) | ((hi == th) & (id <= thi));
}

// One wave's candidate list in LDS: (lo, hi, id, norm) per entry, the entry's row codes
// (RW words) in rw, and the wave-uniform count and threshold.
struct FsList {
  float* lo;
  float* hi;
  int* id;
  float* nr;
  uint32_t* rw;
  int cnt;
  float th;
  int thi;
};

__device__ __forceinline__ int lane_prefix(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Order-preserving 32-bit key of a non-NaN float (-0 and +0 get the same key).
__device__ __forceinline__ uint32_t fs_fkey(float x) {
  const uint32_t b = __float_as_uint(x + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float fs_unkey(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// The k-th best (score desc, id asc) of the wave's valid entries, NV per lane (at least k
// of them, no NaN scores, distinct ids >= 0).  The k-th largest score key comes from a
// 32-step binary search on counts (a compare mask and a scalar popcount per entry
// register and step); when several entries share that score, the needed smallest id among
// them from a 31-step search.  About 2 NV VALU ops per step, against n per entry for
// ranking every entry against every other.
template <int NV>
__device__ __forceinline__ void wave_kth(const float* s, const int* id, const bool* v, int k,
                                         float& ts, int& ti) {
  uint32_t u[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) u[j] = v[j] ? fs_fkey(s[j]) : 0u;  // every real key is > 0
  uint32_t x = 0;
#pragma unroll 4
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t t = x | (1u << bit);
    int c = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) c += __popcll(__ballot(u[j] >= t));
    if (c >= k) x = t;
  }
  int cg = 0, ce = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    cg += __popcll(__ballot(u[j] > x));
    ce += __popcll(__ballot(u[j] == x));
  }
  ts = fs_unkey(x);
  if (ce == 1) {
    int t = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const uint64_t m = __ballot(u[j] == x);
      if (m) t = __builtin_amdgcn_readlane(id[j], __ffsll((long long)m) - 1);
    }
    ti = t;
  } else {  // the (k - cg)-th smallest id among the ties: largest y with fewer below it
    const int need = k - cg;
    uint32_t y = 0;
#pragma unroll 1
    for (int bit = 30; bit >= 0; --bit) {
      const uint32_t t = y | (1u << bit);
      int c = 0;
#pragma unroll
      for (int j = 0; j < NV; ++j) c += __popcll(__ballot((u[j] == x) & ((uint32_t)id[j] < t)));
      if (c < need) y = t;
    }
    ti = (int)y;
  }
}

__device__ __forceinline__ int rank1(const float* s, const int* id, int n, float s0, int i0);

// Ranks of the m LDS entries (cs[c], ci[c]) among themselves (entries with ci == INT_MAX
// hold nothing and rank nowhere), with NT threads: each entry is ranked by up to 8
// threads against a slice of the others (16-byte aligned slices: cs / ci readable and
// padded with (-inf, INT_MAX) up to m rounded up to 4), the slices' counts summed into
// rk[c] (zero on entry) with LDS atomics.  The caller syncs before reading rk.
template <int NT>
__device__ __forceinline__ void block_rank(const float* cs, const int* ci, int m, int* rk, int tid) {
  if (m <= 0) return;
  const int P = m >= NT ? 1 : (NT / m < 8 ? NT / m : 8);
  const int chunk = (((m + P - 1) / P) + 3) & ~3;
  for (int t = tid; t < m * P; t += NT) {
    const int c = t % m, part = t / m, lo = part * chunk;
    const int n = m - lo < chunk ? m - lo : chunk;
    if ((n > 0) & (ci[c] != INT_MAX)) {
      const int r = rank1(cs + lo, ci + lo, n, cs[c], ci[c]);
      if (r) atomicAdd(rk + c, r);
    }
  }
}

__device__ __forceinline__ int rank1(const float* s, const int* id, int n, float s0, int i0) {
  int r0 = 0;
#pragma unroll 4
  for (int f = 0; f < n; f += 4) {
    const float4 a = *reinterpret_cast<const float4*>(s + f);
    const int4 b = *reinterpret_cast<const int4*>(id + f);
    r0 += (f + 0 < n) & better(a.x, b.x, s0, i0);
    r0 += (f + 1 < n) & better(a.y, b.y, s0, i0);
    r0 += (f + 2 < n) & better(a.z, b.z, s0, i0);
    r0 += (f + 3 < n) & better(a.w, b.w, s0, i0);
  }
  return r0;
}

// The entries of (cs, ci)[0, m) that can be among the k best, ranked among themselves (ci
// == INT_MAX: no entry).  When more than S = max(64, 2k rounded up to 64) are given, the
// first S -- in no particular order of score -- are ranked among themselves first, and only
// the entries reaching their k-th best (k distinct entries do, so every entry of the answer
// does; about k m / S of them) move to the front and are ranked: S^2 + (k m / S)^2
// comparisons instead of m^2.  Returns the number of entries ranked (the front of cs / ci);
// rk[c] = the rank of entry c among them.  cs / ci are padded with (-inf, INT_MAX) from m
// up to m rounded to 4 and have room for that; EPT >= capacity / NT.  shf: one float,
// shi: two ints of LDS.  Every thread of the block calls it; it ends with a barrier.
template <int NT, int EPT>
__device__ __forceinline__ int rank_best(float* cs, int* ci, int m, int k, int* rk, int tid,
                                         float* shf, int* shi) {
  const int S = min(m, max(64, (2 * k + 63) & ~63));
  int mr = m;
  if (S < m) {  // uniform
    for (int c = tid; c < S; c += NT) rk[c] = 0;
    if (tid == 0) { shf[0] = -INFINITY; shi[0] = INT_MAX; shi[1] = 0; }
    __syncthreads();
    block_rank<NT>(cs, ci, S, rk, tid);
    __syncthreads();
    for (int c = tid; c < S; c += NT)
      if ((ci[c] != INT_MAX) & (rk[c] == k - 1)) { shf[0] = cs[c]; shi[0] = ci[c]; }
    __syncthreads();
    const float ts = shf[0];
    const int ti = shi[0];
    if (ti != INT_MAX) {  // uniform: the sample holds k entries
      float vs[EPT];
      int vi[EPT];
#pragma unroll
      for (int j = 0; j < EPT; ++j) {  // every entry is read before any is written
        const int e = j * NT + tid;
        const bool kp = (e < m) && (ci[e] != INT_MAX) && !better(ts, ti, cs[e], ci[e]);
        vs[j] = kp ? cs[e] : 0.f;
        vi[j] = kp ? ci[e] : INT_MAX;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < EPT; ++j)
        if (vi[j] != INT_MAX) {
          const int p = atomicAdd(&shi[1], 1);
          cs[p] = vs[j];
          ci[p] = vi[j];
        }
      __syncthreads();
      mr = shi[1];
      for (int c = mr + tid; c < ((mr + 3) & ~3); c += NT) { cs[c] = -INFINITY; ci[c] = INT_MAX; }
    }
  }
  for (int c = tid; c < mr; c += NT) rk[c] = 0;
  __syncthreads();
  block_rank<NT>(cs, ci, mr, rk, tid);
  __syncthreads();
  return mr;
}

// merge_query for k above kSmallK, where 64 group maxima no longer bound the k-th best.
// Per query, for all kThreads threads of a block:
//   1. tau = the k-th largest score among the leading ceil(k / nblocks) entries of every
//      block list (a 32-step binary search on order-preserving keys): those are k distinct
//      rows, so the k-th best score overall is at least tau.
//   2. Per list, the entries scoring at least tau (a prefix: the lists are best first, pads
//      (-inf, -1) last) are counted by binary search and gathered into LDS.
//   3. The survivors are ranked (score desc, id asc) and the best k written.
// More than kBigMergeCap survivors (many rows tied at tau) fall back to merge_query.
constexpr int kBigMergeCap = 2048;
__device__ void merge_query_big(const float* __restrict__ part_s, const int32_t* __restrict__ part_i,
                                int nblocks, int k, int q, float* __restrict__ out_s,
                                int64_t* __restrict__ out_i) {
  constexpr int CR = (kThreads * kMaxBlocksPerLane + kMaxK + kThreads - 1) / kThreads;  // candidates / thread
  __shared__ __attribute__((aligned(16))) float bss[kBigMergeCap + 4];
  __shared__ __attribute__((aligned(16))) int bsi[kBigMergeCap + 4];
  __shared__ int brk[kBigMergeCap];
  __shared__ int bcnt[33];
  __shared__ int bpart[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* ps = part_s + (size_t)q * nblocks * k;
  const int32_t* pi = part_i + (size_t)q * nblocks * k;
  const int depth = (k + nblocks - 1) / nblocks;
  const int ncand = nblocks * depth;
  // 1. candidate keys (0: a pad, below every real key), all loads in flight together
  uint32_t u[CR];
#pragma unroll
  for (int j = 0; j < CR; ++j) {
    const int c = tid + j * kThreads;
    const int cc = c < ncand ? c : ncand - 1;
    const int b = cc / depth, pos = cc - b * depth;
    const int id = pi[(size_t)b * k + pos];
    const float sc = ps[(size_t)b * k + pos];
    u[j] = ((c < ncand) & (id >= 0)) ? fs_fkey(sc) : 0u;
  }
  if (tid < 33) bcnt[tid] = 0;
  __syncthreads();
  uint32_t x = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t t = x | (1u << bit);
    int c = 0;  // wave-uniform
#pragma unroll
    for (int j = 0; j < CR; ++j) c += __popcll(__ballot(u[j] >= t));
    if (lane == 0 && c) atomicAdd(&bcnt[bit], c);
    __syncthreads();
    if (bcnt[bit] >= k) x = t;
  }
  const float tau = x ? fs_unkey(x) : -INFINITY;
  // 2. survivors per list: the prefix whose entries are real and score >= tau
  int cnt[kMaxBlocksPerLane];
  int mine = 0;
#pragma unroll
  for (int r = 0; r < kMaxBlocksPerLane; ++r) {
    const int b = tid + r * kThreads;
    int lo = 0;
    if (b < nblocks) {
      const float* ls = ps + (size_t)b * k;
      const int32_t* li = pi + (size_t)b * k;
      if ((li[0] >= 0) & (ls[0] >= tau)) {
        int hi = k;  // entries [0, lo) pass, [hi, k) do not
        lo = 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if ((li[mid] >= 0) & (ls[mid] >= tau)) lo = mid + 1; else hi = mid;
        }
      }
    }
    cnt[r] = lo;
    mine += lo;
  }
  // block exclusive prefix sum of the per-thread counts
  int incl = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) bpart[wave] = incl;
  __syncthreads();
  int base = incl - mine;
  int S = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    base += w < wave ? bpart[w] : 0;
    S += bpart[w];
  }
  if (S > kBigMergeCap) {  // uniform
    merge_query(part_s, part_i, nblocks, k, q, out_s, out_i);
    return;
  }
#pragma unroll
  for (int r = 0; r < kMaxBlocksPerLane; ++r) {
    const int b = tid + r * kThreads;
    for (int e = 0; e < cnt[r]; ++e) {
      bss[base + e] = ps[(size_t)b * k + e];
      bsi[base + e] = pi[(size_t)b * k + e];
    }
    base += cnt[r];
  }
  for (int e = S + tid; e < ((S + 3) & ~3); e += kThreads) { bss[e] = -INFINITY; bsi[e] = INT_MAX; }
  for (int e = tid; e < S; e += kThreads) brk[e] = 0;
  __syncthreads();
  // 3. ranks, then the best k
  block_rank<kThreads>(bss, bsi, S, brk, tid);
  __syncthreads();
  float* os = out_s + (size_t)q * k;
  int64_t* oi = out_i + (size_t)q * k;
  for (int e = tid; e < S; e += kThreads)
    if (brk[e] < k) { os[brk[e]] = bss[e]; oi[brk[e]] = bsi[e]; }
  for (int e = S + tid; e < k; e += kThreads) { os[e] = -INFINITY; oi[e] = -1; }
}

// (th, thi) from the list's k-th best (lo, id) when it holds k entries or more (kept if
// it beats the current one), then the entries whose (hi, id) fall below it are dropped
// (the rest, with their row codes, move down to close the gaps).
template <int RW>
__device__ __forceinline__ void fs_prune(FsList& L, int k) {
  const int lane = threadIdx.x & 63;
  float lo[2], hi[2], nr[2];
  int id[2];
  bool v[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int e = lane + 64 * r;
    v[r] = e < L.cnt;
    lo[r] = v[r] ? L.lo[e] : -INFINITY;
    hi[r] = v[r] ? L.hi[e] : -INFINITY;
    id[r] = v[r] ? L.id[e] : INT_MAX;
    nr[r] = v[r] ? L.nr[e] : 0.f;
  }
  if (L.cnt >= k) {
    float ts;
    int ti;
    wave_kth<2>(lo, id, v, k, ts, ti);
    if (better(ts, ti, L.th, L.thi)) { L.th = ts; L.thi = ti; }
  }
  const bool k0 = v[0] & fs_keep(hi[0], id[0], L.th, L.thi);
  const bool k1 = v[1] & fs_keep(hi[1], id[1], L.th, L.thi);
  const uint64_t m0 = __ballot(k0), m1 = __ballot(k1);
  const int n0 = __popcll(m0);
  const int p0 = lane_prefix(m0), p1 = n0 + lane_prefix(m1);
  // rows that move are read before any entry is written (a destination slot may hold a
  // row that has yet to move)
  const bool mv0 = k0 & (p0 != lane), mv1 = k1 & (p1 != lane + 64);
  u32x4 w0[RW / 4], w1[RW / 4];
  const u32x4* s0 = reinterpret_cast<const u32x4*>(L.rw + lane * RW);
  const u32x4* s1 = reinterpret_cast<const u32x4*>(L.rw + (lane + 64) * RW);
#pragma unroll
  for (int j = 0; j < RW / 4; ++j) {
    w0[j] = mv0 ? s0[j] : (u32x4){0u, 0u, 0u, 0u};
    w1[j] = mv1 ? s1[j] : (u32x4){0u, 0u, 0u, 0u};
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (k0) {
    L.lo[p0] = lo[0]; L.hi[p0] = hi[0]; L.id[p0] = id[0]; L.nr[p0] = nr[0];
    if (mv0) {
      u32x4* d = reinterpret_cast<u32x4*>(L.rw + p0 * RW);
#pragma unroll
      for (int j = 0; j < RW / 4; ++j) d[j] = w0[j];
    }
  }
  if (k1) {
    L.lo[p1] = lo[1]; L.hi[p1] = hi[1]; L.id[p1] = id[1]; L.nr[p1] = nr[1];
    if (mv1) {
      u32x4* d = reinterpret_cast<u32x4*>(L.rw + p1 * RW);
#pragma unroll
      for (int j = 0; j < RW / 4; ++j) d[j] = w1[j];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  L.cnt = n0 + __popcll(m1);
}

// Rescore every entry with the reference's arithmetic from its row codes in LDS (lo = hi
// = the exact score; NaN scores are never listed), then prune: at most k entries remain.
template <int D>
__device__ __forceinline__ void fs_exact(FsList& L, int k, const float* qr, const float* cen) {
  constexpr int RW = D / 8;
  const int lane = threadIdx.x & 63;
#pragma unroll 1
  for (int r = 0; r < 2; ++r) {
    const int e = lane + 64 * r;
    if (e < L.cnt) {
      const float s = exact_pair_score<D>(reinterpret_cast<const uint8_t*>(L.rw + e * RW), L.nr[e], qr, cen);
      const bool nan = __builtin_isnan(s);
      L.lo[e] = nan ? -INFINITY : s;
      L.hi[e] = nan ? __builtin_nanf("") : s;  // fs_keep fails for NaN: dropped
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  fs_prune<RW>(L, k);
}

// Best of this wave's threshold and the ones the block's other waves published (a
// published th alone is the weaker (th, INT_MAX): every row with hi == th passes it).
__device__ __forceinline__ void fs_share(FsList& L, float* th_s, int wave) {
  if ((threadIdx.x & 63) == 0) th_s[wave] = L.th;
#pragma unroll
  for (int w = 0; w < kFsWaves; ++w) {
    const float t = th_s[w];
    if (t > L.th) { L.th = t; L.thi = INT_MAX; }
  }
}

// fp16 centroid pair of byte K of w: LDS entry (byte << 8) | lane * 4 (64 lane copies).
template <int K>
__device__ __forceinline__ uint32_t fs_hlook(uint32_t w, uint32_t lane4, const char* htab) {
  const uint32_t addr = __builtin_amdgcn_perm(w, lane4, 0x0c0c0000u | ((4u + K) << 8));
  return *reinterpret_cast<const uint32_t*>(htab + addr);
}

// Per query, one kFmThreads block after the filter: the block lists (k exact (score, id)
// per block, best first, id -1 past a list's length) are loaded in one round into
// registers, NR slots per thread.  tau = the best over the waves of the k-th best of the
// wave's share of the block bests (ranked by register broadcast within the wave): k
// distinct rows score at least tau, so every row of the answer does too.  The entries at
// or above tau (tens on real data) are ranked among themselves by all threads, with
// (-inf, -1) pads; more than kFmCap of them (ties across blocks) take k rounds of a
// block-wide arg-best instead.
constexpr int kFmThreads = 512;
constexpr int kFmWaves = kFmThreads / 64;
constexpr int kFmRegs = 40;    // list slots per thread
constexpr int kFmCap = 512;    // survivors ranked in LDS

template <int NR>
__global__ __launch_bounds__(kFmThreads) void filter_merge_kernel(FilterArgs a, int nblocks) {
  __shared__ __attribute__((aligned(16))) float ss[kFmCap + 4];
  __shared__ __attribute__((aligned(16))) int si[kFmCap + 4];
  __shared__ int rk[kFmCap];
  __shared__ float wb_s[kFmWaves];
  __shared__ int wb_i[kFmWaves];
  __shared__ int cnt_s;
  const int q = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int k = a.k;
  const int nslots = nblocks * k;
  const size_t base = (size_t)q * nslots;
  float* os = a.out_s + (size_t)q * k;
  int64_t* oi = a.out_i + (size_t)q * k;
  float es[NR];
  int ei[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int e = tid + kFmThreads * r;
    const size_t ec = base + (size_t)(e < nslots ? e : nslots - 1);
    const float s = a.bs[ec];
    const int id = a.bi[ec];
    const bool ok = (e < nslots) & (id >= 0);
    es[r] = ok ? s : -INFINITY;
    ei[r] = ok ? id : INT_MAX;
  }
  // this wave's share of the block bests: blocks wave * per .. + per - 1, one per lane
  const int per = (nblocks + kFmWaves - 1) / kFmWaves;
  float bs = -INFINITY;
  int bi = INT_MAX;
  {
    const int b = wave * per + lane;
    const bool in = (lane < per) & (b < nblocks);
    const size_t ec = base + (size_t)(in ? b : 0) * k;
    const float x = a.bs[ec];
    const int id = a.bi[ec];
    if (in & (id >= 0)) { bs = x; bi = id; }
  }
  if (tid == 0) cnt_s = 0;
  {  // rank of each lane's block best among the wave's (per <= 64 of them)
    int r = 0;
    for (int j = 0; j < per && j < 64; ++j) {
      const float sj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), j));
      const int ij = __builtin_amdgcn_readlane(bi, j);
      r += (ij != INT_MAX) & better(sj, ij, bs, bi);
    }
    const uint64_t hit = __ballot((bi != INT_MAX) & (r == k - 1));
    float ts = -INFINITY;
    int ti = INT_MAX;
    if (hit) {
      const int src = __ffsll((long long)hit) - 1;
      ts = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), src));
      ti = __builtin_amdgcn_readlane(bi, src);
    }
    if (lane == 0) { wb_s[wave] = ts; wb_i[wave] = ti; }
  }
  __syncthreads();
  float tau = -INFINITY;
  int taui = INT_MAX;  // no wave holds k lists: every entry survives
#pragma unroll
  for (int w = 0; w < kFmWaves; ++w)
    if ((wb_i[w] != INT_MAX) & ((taui == INT_MAX) | better(wb_s[w], wb_i[w], tau, taui))) { tau = wb_s[w]; taui = wb_i[w]; }
#pragma unroll
  for (int r = 0; r < NR; ++r) {  // one LDS atomic per wave and register
    const bool kp = (ei[r] != INT_MAX) & fs_keep(es[r], ei[r], tau, taui);
    const uint64_t km = __ballot(kp);
    if (km) {
      int p0 = 0;
      if (lane == 0) p0 = atomicAdd(&cnt_s, __popcll(km));
      p0 = __builtin_amdgcn_readfirstlane(p0);
      const int p = p0 + lane_prefix(km);
      if (kp & (p < kFmCap)) { ss[p] = es[r]; si[p] = ei[r]; rk[p] = 0; }
    }
  }
  __syncthreads();
  const int m = cnt_s;
  if (m <= kFmCap) {
    if (tid < (((m + 3) & ~3) - m)) { ss[m + tid] = -INFINITY; si[m + tid] = INT_MAX; }
    __syncthreads();
    block_rank<kFmThreads>(ss, si, m, rk, tid);
    __syncthreads();
    for (int e = tid; e < m; e += kFmThreads)
      if (rk[e] < k) { os[rk[e]] = ss[e]; oi[rk[e]] = si[e]; }
    for (int e = m + tid; e < k; e += kFmThreads) { os[e] = -INFINITY; oi[e] = -1; }
    return;  // uniform
  }
  // k rounds: the best survivor not emitted yet (every entry strictly below the last one)
  float last_s = INFINITY;
  int last_i = -1;
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    float cs = -INFINITY;
    int ci = INT_MAX;
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const bool c = (ei[u] != INT_MAX) & fs_keep(es[u], ei[u], tau, taui) &
                     better(last_s, last_i, es[u], ei[u]);
      if (c & ((ci == INT_MAX) | better(es[u], ei[u], cs, ci))) { cs = es[u]; ci = ei[u]; }
    }
    wave_best(cs, ci);
    __syncthreads();
    if (lane == 0) { wb_s[wave] = cs; wb_i[wave] = ci; }
    __syncthreads();
    cs = wb_s[0];
    ci = wb_i[0];
#pragma unroll
    for (int w = 1; w < kFmWaves; ++w)
      if ((wb_i[w] != INT_MAX) & ((ci == INT_MAX) | better(wb_s[w], wb_i[w], cs, ci))) { cs = wb_s[w]; ci = wb_i[w]; }
    last_s = cs;
    last_i = ci;
    if (tid == 0) {
      os[r] = ci == INT_MAX ? -INFINITY : cs;
      oi[r] = ci == INT_MAX ? -1 : ci;
    }
  }
}

// BIG: rows or norms past 2^32 bytes -- a buffer resource per 64-row group (64-bit base);
// otherwise one resource over the whole database and 32-bit offsets.
template <int D, bool BIG>
__global__ __launch_bounds__(kFsThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void
pair_filter_kernel(FilterArgs a) {
#pragma clang fp contract(off)
  static_assert(D == 64 || D == 128, "pair filter dims");
  constexpr int RB = D / 2;   // bytes per row
  constexpr int KT = D / 32;  // MFMA k tiles per row
  constexpr int LW = D / 32;  // 32-bit words per lane per 16-row tile (16 B at D=128, 8 B at 64)
  constexpr int RW = D / 8;   // 32-bit words per row
  __shared__ __attribute__((aligned(16))) char htab[kHtabBytes];
  __shared__ float qs_s[D];
  __shared__ float qr_s[D];
  __shared__ float cen_s[16];
  __shared__ float red_s[2 * kFsWaves];
  __shared__ float th_s[kFsWaves];
  __shared__ int thi_s[kFsWaves];
  __shared__ int ncand_s, nvalid_s, rbi_s[2];
  __shared__ float rbf_s;
  __shared__ __attribute__((aligned(16))) float lo_s[kFsWaves * kFsCap];
  __shared__ float hi_s[kFsWaves * kFsCap];
  __shared__ __attribute__((aligned(16))) int id_s[kFsWaves * kFsCap];
  __shared__ float nr_s[kFsWaves * kFsCap];
  __shared__ __attribute__((aligned(16))) uint32_t rw_s[kFsWaves * kFsCap * RW];  // row codes
  __shared__ int cnt_s[kFsWaves];

  const int q = blockIdx.y;
  // wave-uniform (readfirstlane) so row offsets and buffer resources live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  const uint32_t W = gridDim.x * kFsWaves;
  const uint32_t gw = blockIdx.x * kFsWaves + wave;
  const uint32_t n = (uint32_t)a.n;  // < 2^31 (ids are int32)
  const uint32_t ngroups = (n + 63) / 64;
  const int nsteps = gw < ngroups ? (int)((ngroups - 1 - gw) / W + 1) : 0;

  // ---- query, centroids and the rotation first, so that waiting for them does not wait
  // for the row prefetch behind them
  // (the query as a raw dword through a bounded buffer: no dtype branch, so no wait, here)
  float cload = 0.f;
  const int esz = a.q_dt == TQ_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t qrs =
      buf_rsrc(static_cast<const char*>(a.q) + (size_t)q * D * esz, (uint32_t)(D * esz));
  const uint32_t qraw = __builtin_amdgcn_raw_buffer_load_b32(qrs, (tid * esz) & ~3, 0, 0);
  // R read coalesced (load i: float4 i * kFsThreads + tid), staged in the table's LDS
  // before the table is built: row r, float4 column c at slot (D/4) r + ((c + r) mod (D/4)),
  // so the rotation's thread r reads its row with 16 lanes per pass on distinct banks
  // (row-per-thread global reads touched 64 cache lines per load instruction)
  constexpr int RC = D / 4;                     // float4 per row
  constexpr int RV = D * RC / kFsThreads;       // float4 per thread
  static_assert(D * D * 4 <= kHtabBytes, "R fits in the table's LDS");
  fs_v4f rv[RV];
#pragma unroll
  for (int i = 0; i < RV; ++i) rv[i] = reinterpret_cast<const fs_v4f*>(a.rot)[i * kFsThreads + tid];
  if (tid < 16) cload = a.cen[tid];

  // Rows of step t: the 64-row group t * W + gw (grid stride: all waves sweep memory
  // together).  Lane 16 g + i reads LW words of row 16 rt + i at byte 4 LW g, one load per
  // 16-row tile rt: each load instruction covers 16 whole rows, so the loads are
  // non-temporal (the rows stream through once; 10M x 128 went 130 -> 120 us per op).
  // Loads past the last row return zeros (the resource's range check).
  struct RowBuf {
    uint32_t w[4 * LW];
    float n;
  };
  const uint32_t loff = (lane & 15) * RB + (lane >> 4) * (4 * LW);
  const __amdgpu_buffer_rsrc_t rows_all = buf_rsrc(a.rows, BIG ? 0u : n * (uint32_t)RB);
  const __amdgpu_buffer_rsrc_t norms_all = buf_rsrc(a.norms, BIG ? 0u : n * 4u);
  auto load = [&](int t, RowBuf& b) {
    const uint32_t g = (uint32_t)t * W + gw;
    __amdgpu_buffer_rsrc_t rs = rows_all, ns = norms_all;
    uint32_t roff = loff, noff = lane * 4u;
    if constexpr (BIG) {
      const int64_t r0 = (int64_t)g * 64;
      const int64_t left = a.n - r0;
      const uint32_t nr = (uint32_t)(left < 64 ? (left > 0 ? left : 0) : 64);
      rs = buf_rsrc(a.rows + r0 * RB, nr * (uint32_t)RB);
      ns = buf_rsrc(a.norms + r0, nr * 4u);
    } else {
      const uint32_t gl = g < ngroups ? g : ngroups;  // groups past the end: an empty range
      roff += gl * (64u * RB);
      noff += gl * 256u;
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      if constexpr (LW == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(roff + 16 * RB * rt), 0, kNT);
        b.w[4 * rt + 0] = v.x; b.w[4 * rt + 1] = v.y; b.w[4 * rt + 2] = v.z; b.w[4 * rt + 3] = v.w;
      } else {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(roff + 16 * RB * rt), 0, kNT);
        b.w[2 * rt + 0] = v.x; b.w[2 * rt + 1] = v.y;
      }
    }
    b.n = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ns, (int)noff, 0, kNT));
  };
  RowBuf ta, tb;
  __builtin_amdgcn_sched_barrier(0);
  load(0, ta);
  // the loop issues each buffer's loads as one group (rows, then norm); the prologue keeps
  // that order, so the per-register wait counts agree on both paths into the loop
  __builtin_amdgcn_sched_barrier(0);
  load(1, tb);
  __builtin_amdgcn_sched_barrier(0);

  // ---- query rotation (pair_scan_kernel's arithmetic), tables, bound
  if (tid < D) {
    const uint32_t h = (tid & 1) ? qraw >> 16 : qraw & 0xFFFFu;  // 2-byte types: this half
    qs_s[tid] = a.q_dt == TQ_F32 ? __uint_as_float(qraw)
              : a.q_dt == TQ_BF16 ? __uint_as_float(h << 16)
                                  : __half2float(__ushort_as_half((unsigned short)h));
  }
  if (tid < 16) cen_s[tid] = cload;
  if (tid < kFsWaves) th_s[tid] = -INFINITY;
  {
    fs_v4f* rs_l = reinterpret_cast<fs_v4f*>(htab);
#pragma unroll
    for (int i = 0; i < RV; ++i) {
      const int f = i * kFsThreads + tid, r = f / RC, c = f % RC;
      rs_l[RC * r + ((c + r) & (RC - 1))] = rv[i];
    }
  }
  __syncthreads();
  float qv = 0.f;
  if (tid < D) {
    const fs_v4f* rs_l = reinterpret_cast<const fs_v4f*>(htab);
#pragma unroll
    for (int i = 0; i < D / 4; ++i) {
      const fs_v4f r = rs_l[RC * tid + ((i + tid) & (RC - 1))];
      qv = qv + qs_s[4 * i] * r.x;
      qv = qv + qs_s[4 * i + 1] * r.y;
      qv = qv + qs_s[4 * i + 2] * r.z;
      qv = qv + qs_s[4 * i + 3] * r.w;
    }
    qr_s[tid] = qv;
  }
  __syncthreads();  // R read: the table takes its LDS
  for (int e = tid; e < 256 * 16; e += kFsThreads) {  // entry b, copies 4c..4c+3
    const int b = e >> 4, c = e & 15;
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    const uint32_t v = __builtin_bit_cast(uint32_t, (h2_t){(_Float16)cen_s[b >> 4], (_Float16)cen_s[b & 15]});
    *reinterpret_cast<u32x4*>(htab + b * 256 + c * 16) = (u32x4){v, v, v, v};
  }
  // max |q_rot| and ||q_rot||_1 (threads >= D contribute 0)
  {
    float am = fabsf(qv), l1 = fabsf(qv);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      am = fmaxf(am, __shfl_xor(am, off));
      l1 = l1 + __shfl_xor(l1, off);
    }
    if (lane == 0) { red_s[wave] = am; red_s[kFsWaves + wave] = l1; }
  }
  __syncthreads();
  float amax = 0.f, l1 = 0.f, cmax = 0.f;
#pragma unroll
  for (int w = 0; w < kFsWaves; ++w) { amax = fmaxf(amax, red_s[w]); l1 = l1 + red_s[kFsWaves + w]; }
#pragma unroll
  for (int i = 0; i < 16; ++i) cmax = fmaxf(cmax, fabsf(cen_s[i]));
  float ec = 0.f;  // largest fp16 rounding error of a centroid (inf if one overflows fp16)
#pragma unroll
  for (int i = 0; i < 16; ++i) ec = fmaxf(ec, fabsf(cen_s[i] - (float)(_Float16)cen_s[i]));
  // scale: max |q_rot| * scale in [2^14, 2^15); a query whose scale would leave fp32's
  // range gets beta = inf (every row is then rescored exactly).
  int ex = 0;
  const bool scalable = amax > 0.f && amax < INFINITY;
  if (scalable) frexpf(amax, &ex);
  const bool ok = scalable && ex > -100 && ex < 100;
  const float scale = ok ? ldexpf(1.f, 15 - ex) : 1.f;
  const float inv_scale = ok ? ldexpf(1.f, ex - 15) : 1.f;
  const float beta = ok ? l1 * (ec + cmax * 0x1p-14f) * (1.f + 0x1p-10f) : (amax == 0.f ? 0.f : INFINITY);
  fs_v8h qa[KT];
  {
    const int m = lane & 15, g = lane >> 4;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = qr_s[(D == 128 ? 32 : 16) * g + 8 * kt + e] * scale;
        const _Float16 h = (_Float16)x;
        const _Float16 l = (_Float16)(x - (float)h);
        qa[kt][e] = m == 0 ? h : (m == 1 ? l : (_Float16)0.f);
      }
    }
  }
  const uint32_t lane4 = (uint32_t)lane * 4;

  // Approximate scores of the wave's 64 rows, lane = row: tile rt's rows are the columns of
  // its MFMAs; rows 0 / 1 of the result (hi / lo query part) sit in lanes 0-15, and three
  // row swaps bring tile rt's 16 scores to lanes 16 rt .. 16 rt + 15.
  auto approx = [&](const RowBuf& rb) -> float {
    float t[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      fs_v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const uint32_t x = rb.w[LW * rt + kt];
        const u32x4 bw = {fs_hlook<0>(x, lane4, htab), fs_hlook<1>(x, lane4, htab),
                          fs_hlook<2>(x, lane4, htab), fs_hlook<3>(x, lane4, htab)};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[kt], __builtin_bit_cast(fs_v8h, bw), acc, 0, 0, 0);
      }
      t[rt] = acc[0] + acc[1];
    }
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(t[0]), __float_as_uint(t[1]), false, false);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(t[2]), __float_as_uint(t[3]), false, false);
    const auto s = __builtin_amdgcn_permlane32_swap(p[0], r[0], false, false);
    return __uint_as_float(s[0]);
  };

  FsList L{lo_s + wave * kFsCap, hi_s + wave * kFsCap, id_s + wave * kFsCap,
           nr_s + wave * kFsCap, rw_s + wave * kFsCap * RW, 0, -INFINITY, INT_MAX};
  // Per step the common case costs two multiplies, an fma and a compare: hi >= th can only
  // hold for a row that beats th's float (NaN passes too); the rest -- row validity, the
  // exact (hi, id) test, lo, non-finite scores -- runs only when some lane passes.
  auto step = [&](const RowBuf& rb, int t) {
    const float sa = approx(rb) * inv_scale * rb.n;
    const float hq = __builtin_fmaf(fabsf(rb.n), beta, sa);
    if (__ballot(!(hq < L.th)) == 0) return;
    const uint32_t row = ((uint32_t)t * W + gw) * 64u + lane;
    const bool valid = row < n;
    const float B = fabsf(rb.n) * beta;
    const bool fin = (fabsf(sa) < INFINITY) & (B < INFINITY);
    const float lo = fin ? sa - B : -INFINITY;
    const float hi = fin ? sa + B : INFINITY;
    const int id = (int)row;
    bool ins = valid & fs_keep(hi, id, L.th, L.thi);
    uint64_t mask = __ballot(ins);
    if (mask == 0) return;
    int nnew = __popcll(mask);
    if (L.cnt + nnew > kFsCap) {
      fs_share(L, th_s, wave);
      fs_prune<RW>(L, a.k);
      ins = valid & fs_keep(hi, id, L.th, L.thi);
      mask = __ballot(ins);
      nnew = __popcll(mask);
      if (L.cnt + nnew > kFsCap) {
        fs_exact<D>(L, a.k, qr_s, cen_s);
        ins = valid & fs_keep(hi, id, L.th, L.thi);
        mask = __ballot(ins);
        nnew = __popcll(mask);
      }
      if (mask == 0) return;
    }
    if (ins) {
      const int p = L.cnt + lane_prefix(mask);
      L.lo[p] = lo; L.hi[p] = hi; L.id[p] = id; L.nr[p] = rb.n;
    }
    // the listed rows' codes, from the lanes that loaded them: in tile rt this lane holds
    // LW words of row 16 rt + (lane & 15) at word LW (lane >> 4)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int r = 16 * rt + (lane & 15);
      if ((mask >> r) & 1) {
        const int p = L.cnt + __popcll(mask & ((1ull << r) - 1));
        uint32_t* d = L.rw + p * RW + LW * (lane >> 4);
        if constexpr (LW == 4) {
          *reinterpret_cast<u32x4*>(d) = (u32x4){rb.w[4 * rt], rb.w[4 * rt + 1], rb.w[4 * rt + 2], rb.w[4 * rt + 3]};
        } else {
          *reinterpret_cast<u32x2*>(d) = (u32x2){rb.w[2 * rt], rb.w[2 * rt + 1]};
        }
      }
    }
    L.cnt += nnew;
    // raise th early -- from the first k rows, then whenever the list grows long -- and
    // share it with the block's other waves: fewer inserts for all of them
    if ((L.cnt >= kFsEager) | ((L.th == -INFINITY) & (L.cnt >= a.k))) {
      fs_share(L, th_s, wave);
      fs_prune<RW>(L, a.k);
      fs_share(L, th_s, wave);
    }
  };

  // Loads past the last step address an empty range (zeros, no memory access); issuing
  // them unconditionally keeps every path's load order the same, so each step waits only
  // for its own rows.  After the first step the list is pruned once, which sets the
  // threshold from 64 rows instead of letting 128 rows in first.
  // Loads past the last step address an empty range (zeros, no memory access); issuing
  // them unconditionally keeps every path's load order the same, so each step waits only
  // for its own rows.
  for (int t = 0; t < nsteps; t += 2) {
    step(ta, t);
    load(t + 2, ta);
    if (t + 1 >= nsteps) break;
    step(tb, t + 1);
    load(t + 3, tb);
  }

  // ---- block list.  (bt, bti) = the best of the waves' thresholds (each is the k-th best
  // (lo, id) of some rows of its wave, so it bounds the block's answer from below).  The
  // entries whose (hi, id) reach it (about 50 on random data) are gathered, rescored
  // exactly one per thread from their row codes in LDS, and ranked among themselves; the
  // block's top k go to its slots in rank order, with (-inf, -1) past the end.  The
  // candidate arrays reuse the table's LDS, which no wave reads after its loop.
  if (lane == 0) { th_s[wave] = L.th; thi_s[wave] = L.thi; }
  if (tid == 0) { ncand_s = 0; nvalid_s = 0; }
  __syncthreads();
  float bt = th_s[0];
  int bti = thi_s[0];
#pragma unroll
  for (int w = 1; w < kFsWaves; ++w)
    if (better(th_s[w], thi_s[w], bt, bti)) { bt = th_s[w]; bti = thi_s[w]; }
  int* cslot = reinterpret_cast<int*>(htab);                                  // [kFsWaves * kFsCap]
  float* cs = reinterpret_cast<float*>(htab + 4 * kFsWaves * kFsCap);        // exact scores
  int* ci = reinterpret_cast<int*>(htab + 8 * kFsWaves * kFsCap);            // ids (INT_MAX: NaN)
  int* rk = reinterpret_cast<int*>(htab + 12 * kFsWaves * kFsCap);           // ranks
  // exact products for the rescoring: ptab[16 j + i] = qr[j] * cen[i] (D x 16 floats)
  float* ptab = reinterpret_cast<float*>(htab + 16 * kFsWaves * kFsCap);
  static_assert(16 * kFsWaves * kFsCap + D * 16 * 4 <= kHtabBytes, "product table fits");
  for (int e = tid; e < D * 16; e += kFsThreads) ptab[e] = qr_s[e >> 4] * cen_s[e & 15];
#pragma unroll
  for (int r = 0; r < 2; ++r) {  // one LDS atomic per wave and half
    const int e = lane + 64 * r;
    const bool kp = (e < L.cnt) && fs_keep(L.hi[e], L.id[e], bt, bti);
    const uint64_t km = __ballot(kp);
    if (km) {
      int p0 = 0;
      if (lane == 0) p0 = atomicAdd(&ncand_s, __popcll(km));
      p0 = __builtin_amdgcn_readfirstlane(p0);
      if (kp) cslot[p0 + lane_prefix(km)] = wave * kFsCap + e;
    }
  }
  __syncthreads();
  const int m = ncand_s;
  for (int t = tid; t < m; t += kFsThreads) {
    const int sl = cslot[t];
    const float x = exact_pair_score_ptab<D>(rw_s + sl * RW, nr_s[sl], ptab);
    const bool ok = !__builtin_isnan(x);
    cs[t] = ok ? x : -INFINITY;
    ci[t] = ok ? id_s[sl] : INT_MAX;  // (-inf, INT_MAX) ranks below every listed row
    rk[t] = 0;
    if (ok) atomicAdd(&nvalid_s, 1);
  }
  for (int t = m + tid; t < ((m + 3) & ~3); t += kFsThreads) { cs[t] = -INFINITY; ci[t] = INT_MAX; }
  const int mr = rank_best<kFsThreads, (kFsWaves * kFsCap + kFsThreads - 1) / kFsThreads>(
      cs, ci, m, a.k, rk, tid, &rbf_s, rbi_s);
  const size_t base = ((size_t)q * gridDim.x + blockIdx.x) * a.k;
  for (int t = tid; t < mr; t += kFsThreads) {
    const int id = ci[t], rank = rk[t];
    if ((id != INT_MAX) & (rank < a.k)) { a.bs[base + rank] = cs[t]; a.bi[base + rank] = id; }
  }
  for (int e = nvalid_s + tid; e < a.k; e += kFsThreads) { a.bs[base + e] = -INFINITY; a.bi[base + e] = -1; }
}

// ------------------------------------------------------------------ multi-query filtered pair scan
// Top-k over 4-bit pair-layout rows (d = 64 / 128) for batches of queries, with the
// reference's exact scores and tie order (csrc/core/turboquant_core.cpp:407-514), as the
// one-query filter above; here 64 queries share every table lookup.
//
// A wave takes 64 queries x 64 rows per step on v_mfma_f32_16x16x32_f16: A = 16 queries'
// rotated vectors (one tile-wide power-of-two scale, rounded to fp16) per M tile, B = 16
// rows' fp16 centroid pairs per N tile from one LDS lookup per code byte -- the lookups
// of a row serve all 64 queries.  Lane (n, g) of N tile rt gets queries 16 mt + 4 g + r of
// row 16 rt + n.  Bound (per tile, with l1 = max over its queries of ||q_rot||_1, e_c the
// largest fp16 rounding error of a centroid, s the scale):
//   |approx - exact| <= |n| beta + 2^-100,
//   beta = (l1 (e_c (1 + 2^-11) + max|c| (2^-11 + 2^-15)) + d (max|c| + e_c) 2^-25 / s) (1 + 2^-9).
// Terms: fp16 rounding of the scaled query (2^-11 relative, or 2^-25 absolute below fp16's
// normal range, the last term), the centroids' fp16 errors, fp32 accumulation of the d
// exact products (d 2^-24 <= 2^-17 relative) and the reference's own sequential sum and
// final multiply (2^-17 + 2^-24); the (1 + 2^-9) covers rounding l1, beta, |n| beta and the
// fma that adds it (each under 2^-12 of the bound); the absolute 2^-100 covers n / s
// underflowing in m = n / s (an error below |acc| 2^-150 <= 2^-125).
// Pipeline (one call):
//   mq_rotate_kernel  q_rot with the reference's arithmetic (kept for the exact rescoring).
//   mq_tile_kernel    per 64-query tile: the fp16 A operands, 1/s and beta.
//   mq_sample_kernel  lo = approx - bound of 4096 evenly spaced 64-row groups; per query,
//                     the maximum over each block's 16 groups (a bucket of 1024 rows).
//   mq_filter_kernel  prologue: per query, tau = the k-th largest bucket maximum.  Buckets
//                     are disjoint row sets, so k distinct rows score at least tau; a row
//                     whose upper bound hi = approx + bound is below tau is not in the
//                     answer.  Then every row: hi against tau per (query, row); the rows
//                     that reach it (a few hundred per query at 10M rows) are listed per
//                     (block, query) with (hi, lo, id).
//   mq_merge_kernel   per query: tau' = the k-th best lo of the list, the entries whose hi
//                     reaches it are rescored exactly (rows re-read from memory) and
//                     ranked; the answer is the exact scan's, ties included.  A list that
//                     overflowed (ties, duplicated rows, degenerate queries) flags the query
//                     instead, and the exact multi-query scan then runs for flagged queries
//                     only (its blocks for unflagged queries return at once).
constexpr int kMqQ = 64;                 // queries per tile
constexpr int kMqThreads = 512;          // 8 waves; one block per CU
constexpr int kMqWaves = kMqThreads / 64;
constexpr int kMqCap = 64;               // listed rows per (block, query)
constexpr int kMqSampleGroups = 4096;    // 64-row groups sampled for tau
constexpr int kMqGroupsPerWave = 2;      // sampled groups per wave (one bucket per wave)
constexpr int kMqMaxBuckets = 256;       // bucket maxima per query (one per sample block)
constexpr int kMqMergeCap = 6144;        // listed entries a query's merge holds in LDS
constexpr int kMqMergeCapBig = 12288;    // the same for k above kSmallK (147 KB of LDS)
constexpr int kMqTilesPerRound = 8;      // query tiles per filter launch
constexpr int kMqFallbackBlocks = 128;   // row blocks of the exact fallback scan
static_assert(kMqSampleGroups / (kMqWaves * kMqGroupsPerWave) <= kMqMaxBuckets, "bucket count");

struct MqArgs {
  const uint8_t* rows;  // [n][D * BITS / 8] pair rows (4 bits: the pair layout)
  const float* norms;   // [n]
  int64_t n;
  const void* q;        // [nq][D]
  int q_dt;
  int nq;
  const float* rot;     // [D][D]
  const float* cen;     // [2^BITS]
  int k;
  float* qrot;          // [nq][D] rotated queries (reference arithmetic)
  uint32_t* qa;         // per tile [KT][4][64 lanes][4 words]: fp16 A operands
  float* tparam;        // per tile {1 / s, beta}
  float* buckets;       // [round queries][nbk]
  float* tau;           // [nq]
  int nbk;              // buckets per query
  int sstride;          // sampled group stride
  int nsgroups;         // sampled groups
  int nb;               // filter blocks
  int tile0;            // first tile of the round
  int* cnt;             // [round tiles][nb][64] listed rows per (block, query)
  float* chi;           // [round tiles][nb][64][kMqCap]
  float* clo;
  int* cid;
  int* flag;            // [nq] 1: the exact fallback answers this query
  float* out_s;         // [nq][k]
  int64_t* out_i;
};

// Rows of one 64-row group for the MFMA B operands: lane 16 g + i holds NW words of row
// 16 rt + i per 16-row tile rt, and the norm of row `lane`.  The words hold the dims of
// lane group g's A operands (dims (D / 4) g ..):
//   4 bits: D / 32 words at byte 4 NW g;
//   3 bits: the 12-byte block of 32 dims holding them, at byte 12 g (D 128) or 12 (g / 2)
//           (D 64: the odd group's pairs 12-15 are rebuilt from all three words);
//   2 bits: D / 64 words at byte 4 NW g.
// Rows past n read as zeros (the buffer's range check).
template <int D, int BITS, bool BIG>
struct MqRows {
  static constexpr int RB = D * BITS / 8;
  static constexpr int NW = BITS == 4 ? D / 32 : BITS == 3 ? 3 : D / 64;
  uint32_t w[4 * NW];
  float n;
  __device__ __forceinline__ void load(const MqArgs& a, uint32_t g, uint32_t ngroups,
                                       __amdgpu_buffer_rsrc_t rows_all,
                                       __amdgpu_buffer_rsrc_t norms_all, int lane, int cpol) {
    __amdgpu_buffer_rsrc_t rs = rows_all, ns = norms_all;
    const uint32_t lg = (uint32_t)lane >> 4;
    const uint32_t gofs = BITS == 3 ? 12u * (D == 128 ? lg : lg >> 1) : 4u * NW * lg;
    uint32_t roff = (lane & 15) * RB + gofs, noff = lane * 4u;
    if constexpr (BIG) {
      const int64_t r0 = (int64_t)g * 64;
      const int64_t left = a.n - r0;
      const uint32_t nr = (uint32_t)(left < 64 ? (left > 0 ? left : 0) : 64);
      rs = buf_rsrc(a.rows + r0 * RB, nr * (uint32_t)RB);
      ns = buf_rsrc(a.norms + r0, nr * 4u);
    } else {
      const uint32_t gl = g < ngroups ? g : ngroups;
      roff += gl * (64u * RB);
      noff += gl * 256u;
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int o = (int)(roff + 16 * RB * rt);
      if constexpr (NW == 4) {
        const u32x4 v = cpol ? __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, kNT)
                             : __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
        w[4 * rt + 0] = v.x; w[4 * rt + 1] = v.y; w[4 * rt + 2] = v.z; w[4 * rt + 3] = v.w;
      } else if constexpr (NW == 3) {
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 v = cpol ? __builtin_amdgcn_raw_buffer_load_b96(rs, o, 0, kNT)
                             : __builtin_amdgcn_raw_buffer_load_b96(rs, o, 0, 0);
        w[3 * rt + 0] = v.x; w[3 * rt + 1] = v.y; w[3 * rt + 2] = v.z;
      } else if constexpr (NW == 2) {
        const u32x2 v = cpol ? __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, kNT)
                             : __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, 0);
        w[2 * rt + 0] = v.x; w[2 * rt + 1] = v.y;
      } else {
        w[rt] = cpol ? __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, kNT)
                     : __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, 0);
      }
    }
    n = __uint_as_float(cpol ? __builtin_amdgcn_raw_buffer_load_b32(ns, (int)noff, 0, kNT)
                             : __builtin_amdgcn_raw_buffer_load_b32(ns, (int)noff, 0, 0));
  }
};

// Maximum over each 16-lane row of the wave (DPP: quad swaps, then half-row and row mirrors).
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  return v;
}

// The fp16 centroid-pair table: entry (p << 8) | lane * 4 holds (c[p >> BITS],
// c[p & (2^BITS - 1)]) in 64 lane copies for each pair index p of two BITS-bit codes (the
// first dim's code in the high bits): 64 KB for 4 bits, as pair_filter_kernel builds it,
// 16 KB for 3 bits, 4 KB for 2 bits.
template <int BITS>
__device__ __forceinline__ void mq_fill_htab(char* htab, const float* cen_s, int tid, int nthreads) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  constexpr int M = (1 << BITS) - 1;
  for (int e = tid; e < (1 << (2 * BITS)) * 16; e += nthreads) {
    const int b = e >> 4, c = e & 15;
    const uint32_t v = __builtin_bit_cast(uint32_t, (h2_t){(_Float16)cen_s[b >> BITS], (_Float16)cen_s[b & M]});
    *reinterpret_cast<u32x4*>(htab + b * 256 + c * 16) = (u32x4){v, v, v, v};
  }
}

// Pair indices of k tile kt of N tile rt (dims 8 kt .. 8 kt + 7 of the lane group's
// share), one per byte in dim order.
template <int D, int BITS, bool BIG>
__device__ __forceinline__ uint32_t mq_pair_indices(const MqRows<D, BITS, BIG>& rb, int rt, int kt,
                                                    uint32_t lane) {
  constexpr int NW = MqRows<D, BITS, BIG>::NW;
  const uint32_t* w = rb.w + NW * rt;
  if constexpr (BITS == 4) {
    return w[kt];  // a byte per pair of dims
  } else if constexpr (BITS == 3) {
    // word i of the block: pairs 4 i .. 4 i + 3, six bits each; word 3 from the top bits
    const uint32_t x3 = ((w[0] >> 6) & 0x03030303u) | ((w[1] >> 4) & 0x0C0C0C0Cu) |
                        ((w[2] >> 2) & 0x30303030u);
    if constexpr (D == 128) {
      return kt < 3 ? w[kt] & 0x3F3F3F3Fu : x3;
    } else {  // lane group g: words 2 (g % 2) + kt
      const bool odd = (lane >> 4) & 1u;
      return odd ? (kt ? x3 : w[2] & 0x3F3F3F3Fu) : w[kt] & 0x3F3F3F3Fu;
    }
  } else {
    // bytes 2 kt, 2 kt + 1 of the lane's words, each two 4-bit pair indices (high nibble
    // first): [b0 >> 4, b0 & 15, b1 >> 4, b1 & 15]
    const uint32_t x = w[D == 128 ? kt >> 1 : 0];
    const int h = D == 128 ? kt & 1 : kt;
    const uint32_t t = __builtin_amdgcn_perm(x, x, h ? 0x03030202u : 0x01010000u);
    return ((t >> 4) & 0x000F000Fu) | (t & 0x0F000F00u);
  }
}

// B operands of N tile rt of the group in `rb`: per k tile, the fp16 centroid pairs of the
// lane's four pair indices (one LDS lookup each).
template <int D, int BITS, bool BIG>
__device__ __forceinline__ void mq_fetch_b(const MqRows<D, BITS, BIG>& rb, int rt, uint32_t lane4,
                                           const char* htab, u32x4 (&bw)[D / 32]) {
  constexpr int KT = D / 32;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const uint32_t x = mq_pair_indices<D, BITS, BIG>(rb, rt, kt, lane4 >> 2);
    bw[kt] = (u32x4){fs_hlook<0>(x, lane4, htab), fs_hlook<1>(x, lane4, htab),
                     fs_hlook<2>(x, lane4, htab), fs_hlook<3>(x, lane4, htab)};
  }
}

// Approximate scores (in units of the scaled query) of 16 rows x 64 queries from one N
// tile's B operands: acc[mt][r] = query 16 mt + 4 (lane >> 4) + r, row 16 rt + (lane & 15).
template <int D>
__device__ __forceinline__ void mq_mfma(const u32x4 (&bw)[D / 32], const fs_v8h (&qa)[4][D / 32],
                                        fs_v4f (&acc)[4]) {
  constexpr int KT = D / 32;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) acc[mt] = (fs_v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const fs_v8h b = __builtin_bit_cast(fs_v8h, bw[kt]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[mt][kt], b, acc[mt], 0, 0, 0);
  }
}

template <int D, int BITS, bool BIG>
__device__ __forceinline__ void mq_tile_scores(const MqRows<D, BITS, BIG>& rb, int rt,
                                               const fs_v8h (&qa)[4][D / 32], uint32_t lane4,
                                               const char* htab, fs_v4f (&acc)[4]) {
  u32x4 bw[D / 32];
  mq_fetch_b<D, BITS, BIG>(rb, rt, lane4, htab, bw);
  mq_mfma<D>(bw, qa, acc);
}

// q_rot of four queries per block (reference arithmetic: q_rot[j] = sum over i in order
// of q[i] * R[j][i], each product rounded; csrc/core/turboquant_core.cpp:429-437).
// Thread j holds row j of R; the queries are read from LDS as 16-byte broadcasts.
constexpr int kMqRotQ = 4;
template <int D>
__global__ __launch_bounds__(D) void mq_rotate_kernel(MqArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float qs[kMqRotQ][D];
  const int j = threadIdx.x;
  const int q0 = blockIdx.x * kMqRotQ;
  const int nv = min(kMqRotQ, a.nq - q0);
  float4 rrow[D / 4];
  const float4* r4 = reinterpret_cast<const float4*>(a.rot + (size_t)j * D);
#pragma unroll
  for (int i = 0; i < D / 4; ++i) rrow[i] = r4[i];
#pragma unroll
  for (int qi = 0; qi < kMqRotQ; ++qi)
    qs[qi][j] = qi < nv ? load_as_f32(a.q, (int64_t)(q0 + qi) * D + j, a.q_dt) : 0.f;
  __syncthreads();
  float v[kMqRotQ];
#pragma unroll
  for (int qi = 0; qi < kMqRotQ; ++qi) v[qi] = 0.f;
#pragma unroll
  for (int i = 0; i < D / 4; ++i) {
#pragma unroll
    for (int qi = 0; qi < kMqRotQ; ++qi) {
      const float4 x = *reinterpret_cast<const float4*>(&qs[qi][4 * i]);
      v[qi] = v[qi] + x.x * rrow[i].x;
      v[qi] = v[qi] + x.y * rrow[i].y;
      v[qi] = v[qi] + x.z * rrow[i].z;
      v[qi] = v[qi] + x.w * rrow[i].w;
    }
  }
#pragma unroll
  for (int qi = 0; qi < kMqRotQ; ++qi)
    if (qi < nv) a.qrot[(size_t)(q0 + qi) * D + j] = v[qi];
}

// Per 64-query tile: the scale, beta and the fp16 A operands from the rotated queries.
template <int D, int BITS>
__global__ __launch_bounds__(kMqThreads) void mq_tile_kernel(MqArgs a) {
  constexpr int NC = 1 << BITS;  // centroids
  constexpr int KT = D / 32;
  __shared__ float qr[kMqQ][D + 1];
  __shared__ float red[2][kMqQ];
  __shared__ float cen_s[16];
  const int tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int q0 = tile * kMqQ;
  const int nvalid = min(kMqQ, a.nq - q0);
  for (int e = tid; e < kMqQ * D; e += kMqThreads) {
    const int qi = e / D, j = e % D;
    qr[qi][j] = qi < nvalid ? a.qrot[(size_t)(q0 + qi) * D + j] : 0.f;
  }
  if (tid < NC) cen_s[tid] = a.cen[tid];
  __syncthreads();
  {  // max |q_rot| and ||q_rot||_1 per query: 8 threads per query
    const int qi = tid >> 3, part = tid & 7;
    float am = 0.f, l1 = 0.f;
    for (int j = part; j < D; j += 8) {
      const float x = fabsf(qr[qi][j]);
      am = fmaxf(am, x);
      l1 = l1 + x;
    }
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
      am = fmaxf(am, __shfl_xor(am, off));
      l1 = l1 + __shfl_xor(l1, off);
    }
    if (part == 0) {
      const bool v = qi < nvalid;
      red[0][qi] = v ? am : 0.f;
      // a NaN anywhere in a valid query turns the filter off for the tile
      red[1][qi] = v ? (l1 < INFINITY ? l1 : INFINITY) : 0.f;
    }
  }
  __syncthreads();
  float amax = 0.f, l1 = 0.f;
  for (int i = 0; i < kMqQ; ++i) { amax = fmaxf(amax, red[0][i]); l1 = fmaxf(l1, red[1][i]); }
  float cmax = 0.f, ec = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    cmax = fmaxf(cmax, fabsf(cen_s[i]));
    ec = fmaxf(ec, fabsf(cen_s[i] - (float)(_Float16)cen_s[i]));
  }
  int ex = 0;
  const bool scalable = amax > 0.f && amax < INFINITY;
  if (scalable) frexpf(amax, &ex);
  const bool ok = scalable && ex > -60 && ex < 60 && l1 < INFINITY && ec < INFINITY;
  const float scale = ok ? ldexpf(1.f, 15 - ex) : 0.f;
  const float inv_s = ok ? ldexpf(1.f, ex - 15) : 0.f;
  float beta = INFINITY;
  if (ok) {
    beta = (l1 * (ec * (1.f + 0x1p-11f) + cmax * (0x1p-11f + 0x1p-15f)) +
            (float)D * (cmax + ec) * 0x1p-25f * inv_s) * (1.f + 0x1p-9f);
    if (!(beta < INFINITY)) beta = INFINITY;
  }
  if (tid == 0) {
    a.tparam[2 * tile] = inv_s;
    a.tparam[2 * tile + 1] = beta;
  }
  // A operand of (kt, mt), lane (m, g): query 16 mt + m, dims (D == 128 ? 32 : 16) g + 8 kt + e
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  for (int it = tid; it < KT * 4 * 64; it += kMqThreads) {
    const int l = it & 63, mt = (it >> 6) & 3, kt = it >> 8;
    const int qi = 16 * mt + (l & 15), g = l >> 4;
    const int dim0 = (D == 128 ? 32 : 16) * g + 8 * kt;
    uint32_t wv[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const _Float16 h0 = (_Float16)(qr[qi][dim0 + 2 * w] * scale);
      const _Float16 h1 = (_Float16)(qr[qi][dim0 + 2 * w + 1] * scale);
      wv[w] = __builtin_bit_cast(uint32_t, (h2_t){h0, h1});
    }
    *reinterpret_cast<u32x4*>(a.qa + (((size_t)tile * KT + kt) * 4 + mt) * 256 + l * 4) =
        (u32x4){wv[0], wv[1], wv[2], wv[3]};
  }
  (void)lane;
}

// The tile's A operands, 1/s and beta for this lane.
template <int D>
__device__ __forceinline__ void mq_load_tile(const MqArgs& a, int tile, int lane, fs_v8h (&qa)[4][D / 32],
                                             float& inv_s, float& beta) {
  constexpr int KT = D / 32;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(a.qa + (((size_t)tile * KT + kt) * 4 + mt) * 256 + lane * 4);
      qa[mt][kt] = __builtin_bit_cast(fs_v8h, v);
    }
  inv_s = a.tparam[2 * tile];
  beta = a.tparam[2 * tile + 1];
}

// Buckets: wave (block b, wave w) takes sampled groups (8 b + w) * 4 + u; lane (n, g) keeps
// per query 16 mt + 4 g + r the largest lo over its rows 16 rt + n of those groups.
template <int D, int BITS, bool BIG>
__global__ __launch_bounds__(kMqThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void
mq_sample_kernel(MqArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) char htab[256 << (2 * BITS)];
  __shared__ float cen_s[16];
  constexpr uint32_t RB = D * BITS / 8;
  __shared__ float wmax_s[kMqWaves][kMqQ];
  const int rtile = blockIdx.y, tile = a.tile0 + rtile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t n = (uint32_t)a.n;
  const uint32_t ngroups = (n + 63) / 64;
  fs_v8h qa[4][D / 32];
  float inv_s, beta;
  mq_load_tile<D>(a, tile, lane, qa, inv_s, beta);
  if (tid < (1 << BITS)) cen_s[tid] = a.cen[tid];
  __syncthreads();
  mq_fill_htab<BITS>(htab, cen_s, tid, kMqThreads);
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rows_all = buf_rsrc(a.rows, BIG ? 0u : n * RB);
  const __amdgpu_buffer_rsrc_t norms_all = buf_rsrc(a.norms, BIG ? 0u : n * 4u);
  const uint32_t lane4 = (uint32_t)lane * 4;
  float bmax[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) bmax[mt][r] = -INFINITY;
  const int sw = blockIdx.x * kMqWaves + wave;
  // every group's loads first (a sampled group past nsgroups reads the empty range past
  // the last row: zeros, and its rows are not valid)
  MqRows<D, BITS, BIG> rbs[kMqGroupsPerWave];
  uint32_t gs[kMqGroupsPerWave];
#pragma unroll
  for (int u = 0; u < kMqGroupsPerWave; ++u) {
    const int s = sw * kMqGroupsPerWave + u;
    gs[u] = s < a.nsgroups ? (uint32_t)s * (uint32_t)a.sstride : ngroups;
    rbs[u].load(a, gs[u], ngroups, rows_all, norms_all, lane, 0);
  }
#pragma unroll
  for (int u = 0; u < kMqGroupsPerWave; ++u) {
    const uint32_t g = gs[u];
    const MqRows<D, BITS, BIG>& rb = rbs[u];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      fs_v4f acc[4];
      mq_tile_scores<D, BITS, BIG>(rb, rt, qa, lane4, htab, acc);
      const float nr = __shfl(rb.n, 16 * rt + (lane & 15));
      const bool valid = g * 64u + 16u * rt + (uint32_t)(lane & 15) < n;
      const float m = inv_s * nr;
      const float L = valid ? -__builtin_fmaf(fabsf(nr), beta, 0x1p-100f) : -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) bmax[mt][r] = fmaxf(bmax[mt][r], __builtin_fmaf(acc[mt][r], m, L));
    }
  }
  // The block's rows make one bucket per query: the maximum over the 16 lanes of the
  // query's row group, then over the waves.  +inf (an overflowed approximation) hides the
  // other rows of its lane: no bound from that lane.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = row_max16(bmax[mt][r] < INFINITY ? bmax[mt][r] : -INFINITY);
      const int ql = 16 * mt + 4 * (lane >> 4) + r;
      if ((lane & 15) == 0) wmax_s[wave][ql] = v;
    }
  __syncthreads();
  if (tid < kMqQ) {
    float v = wmax_s[0][tid];
#pragma unroll
    for (int w = 1; w < kMqWaves; ++w) v = fmaxf(v, wmax_s[w][tid]);
    a.buckets[(size_t)(rtile * kMqQ + tid) * a.nbk + blockIdx.x] = v;
  }
}

// tau of each of the tile's 64 queries (eight threads per query): the k-th largest of its
// nbk bucket maxima, -inf when fewer than k are above -inf -- a 32-step binary search on
// order-preserving keys.  Buckets are disjoint row sets, so k distinct rows score at
// least tau.
__device__ __forceinline__ void mq_tau(const MqArgs& a, int rtile, int tid, float* tau_s) {
  constexpr int PER = kMqMaxBuckets / 8;
  const int ql = tid >> 3, part = tid & 7;
  const float* src = a.buckets + (size_t)(rtile * kMqQ + ql) * a.nbk;
  float vals[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) vals[j] = src[min(8 * j + part, a.nbk - 1)];
  uint32_t u[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j)
    u[j] = ((8 * j + part < a.nbk) & (vals[j] > -INFINITY)) ? fs_fkey(vals[j]) : 0u;
  uint32_t x = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t t = x | (1u << bit);
    int c = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) c += (u[j] >= t);
    c += __shfl_xor(c, 1);
    c += __shfl_xor(c, 2);
    c += __shfl_xor(c, 4);
    if (c >= a.k) x = t;
  }
  if (part == 0) tau_s[ql] = x ? fs_unkey(x) : -INFINITY;
}

// Every row against tau per query; rows whose upper bound reaches it are listed.
template <int D, int BITS, bool BIG>
__global__ __launch_bounds__(kMqThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void
mq_filter_kernel(MqArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) char htab[256 << (2 * BITS)];
  __shared__ float cen_s[16];
  constexpr uint32_t RB = D * BITS / 8;
  __shared__ int cnt_s[kMqQ];
  __shared__ float tau_s[kMqQ];
  const int rtile = blockIdx.y, tile = a.tile0 + rtile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t W = gridDim.x * kMqWaves;
  const uint32_t gw = blockIdx.x * kMqWaves + wave;
  const uint32_t n = (uint32_t)a.n;
  const uint32_t ngroups = (n + 63) / 64;
  const int nsteps = gw < ngroups ? (int)((ngroups - 1 - gw) / W + 1) : 0;
  const __amdgpu_buffer_rsrc_t rows_all = buf_rsrc(a.rows, BIG ? 0u : n * RB);
  const __amdgpu_buffer_rsrc_t norms_all = buf_rsrc(a.norms, BIG ? 0u : n * 4u);
  MqRows<D, BITS, BIG> ta, tb;
  ta.load(a, gw, ngroups, rows_all, norms_all, lane, 1);
  tb.load(a, gw + W, ngroups, rows_all, norms_all, lane, 1);

  fs_v8h qa[4][D / 32];
  float inv_s, beta;
  mq_load_tile<D>(a, tile, lane, qa, inv_s, beta);
  if (tid < (1 << BITS)) cen_s[tid] = a.cen[tid];
  if (tid < kMqQ) cnt_s[tid] = 0;
  mq_tau(a, rtile, tid, tau_s);
  __syncthreads();
  if (blockIdx.x == 0 && tid < kMqQ && tile * kMqQ + tid < a.nq) a.tau[tile * kMqQ + tid] = tau_s[tid];
  float th[4][4];
  uint32_t qv = 0;  // bit 4 mt + r: query 16 mt + 4 (lane >> 4) + r is a real query
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ql = 16 * mt + 4 * (lane >> 4) + r;
      const bool v = tile * kMqQ + ql < a.nq;
      th[mt][r] = v ? tau_s[ql] : INFINITY;
      qv |= (uint32_t)v << (4 * mt + r);
    }
  mq_fill_htab<BITS>(htab, cen_s, tid, kMqThreads);
  __syncthreads();
  const uint32_t lane4 = (uint32_t)lane * 4;
  const size_t lbase = ((size_t)rtile * a.nb + blockIdx.x) * kMqQ;

  // Per row tile: the MFMAs, then hi = acc * m + H of (query 16 mt + 4 (lane >> 4) + r, row
  // 16 rt + (lane & 15)) against the queries' tau.  The next tile's table lookups are issued
  // before this tile's tests, so their latency runs under the tests and the branch.
  auto step = [&](const MqRows<D, BITS, BIG>& rb, int t) {
    const uint32_t g = (uint32_t)t * W + gw;
    u32x4 bw[2][D / 32];
    mq_fetch_b<D, BITS, BIG>(rb, 0, lane4, htab, bw[0]);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      fs_v4f acc[4];
      mq_mfma<D>(bw[rt & 1], qa, acc);
      if (rt < 3) mq_fetch_b<D, BITS, BIG>(rb, rt + 1, lane4, htab, bw[(rt + 1) & 1]);
      const float nr = __shfl(rb.n, 16 * rt + (lane & 15));
      const uint32_t row = g * 64u + 16u * rt + (uint32_t)(lane & 15);
      const bool valid = row < n;
      const float m = inv_s * nr;
      const float H = valid ? __builtin_fmaf(fabsf(nr), beta, 0x1p-100f) : -INFINITY;
      bool any = false;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) any |= !(__builtin_fmaf(acc[mt][r], m, H) < th[mt][r]);
      if (__ballot(any) == 0) continue;
      // a row reaches some query's tau (NaN bounds reach every tau): list it there
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float hi = __builtin_fmaf(acc[mt][r], m, H);
          const bool p = !(hi < th[mt][r]) & valid & ((qv >> (4 * mt + r)) & 1u);
          if (__ballot(p) == 0) continue;
          if (p) {
            const int ql = 16 * mt + 4 * (lane >> 4) + r;
            const int slot = atomicAdd(&cnt_s[ql], 1);
            if (slot < kMqCap) {
              const size_t e = (lbase + ql) * kMqCap + slot;
              a.chi[e] = hi;
              a.clo[e] = __builtin_fmaf(acc[mt][r], m, -H);
              a.cid[e] = (int)row;
            }
          }
        }
    }
  };
  for (int t = 0; t < nsteps; t += 2) {
    step(ta, t);
    ta.load(a, (uint32_t)(t + 2) * W + gw, ngroups, rows_all, norms_all, lane, 1);
    if (t + 1 >= nsteps) break;
    step(tb, t + 1);
    tb.load(a, (uint32_t)(t + 3) * W + gw, ngroups, rows_all, norms_all, lane, 1);
  }
  __syncthreads();
  if (tid < kMqQ) a.cnt[lbase + tid] = cnt_s[tid];
}

// Per query: the listed rows of every block, tau' = their k-th best lo, the rows whose hi
// reaches it rescored exactly and ranked.  More than kMqCap rows listed by one block, or
// more than MCAP in all, flags the query for the exact fallback instead.
template <int D, int BITS, int MCAP>
__global__ __launch_bounds__(kMqThreads) void mq_merge_kernel(MqArgs a) {
  __shared__ __attribute__((aligned(16))) float ehi[MCAP];
  __shared__ __attribute__((aligned(16))) float elo[MCAP];
  __shared__ __attribute__((aligned(16))) int eid[MCAP];
  __shared__ int off_s[kMqThreads + 1];
  __shared__ int part[kMqWaves];
  __shared__ int tcnt[32];
  __shared__ int bad_s, m2_s, nvalid_s, shi_s[2];
  __shared__ float ts_s;
  __shared__ float qr_s[D];
  __shared__ float cen_s[16];
  const int ql = blockIdx.x % kMqQ, rtile = blockIdx.x / kMqQ;
  const int q = (a.tile0 + rtile) * kMqQ + ql;
  if (q >= a.nq) return;  // uniform
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nb = a.nb, k = a.k;
  // listed counts per block and their prefix sums (nb <= kMqThreads)
  int c = 0;
  if (tid < nb) c = a.cnt[((size_t)rtile * nb + tid) * kMqQ + ql];
  if (tid == 0) bad_s = 0;
  __syncthreads();
  if (c > kMqCap) bad_s = 1;
  int incl = c;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) part[wave] = incl;
  __syncthreads();
  int wofs = 0;
  for (int w = 0; w < wave; ++w) wofs += part[w];
  off_s[tid] = wofs + incl - c;
  if (tid == kMqThreads - 1) off_s[kMqThreads] = wofs + incl;
  __syncthreads();
  const int M = off_s[kMqThreads];
  if (bad_s || M > MCAP) {
    if (tid == 0) a.flag[q] = 1;
    return;  // uniform
  }
  if (tid == 0) a.flag[q] = 0;
  // gather the lists: entry e of the concatenation is slot e - off_s[b] of block b, found by
  // a binary search over the prefix sums (every load of the gather in flight at once)
  for (int e = tid; e < M; e += kMqThreads) {
    int lo = 0, hi = nb;  // off_s[lo] <= e < off_s[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off_s[mid] <= e) lo = mid; else hi = mid;
    }
    const size_t src = (((size_t)rtile * nb + lo) * kMqQ + ql) * kMqCap + (e - off_s[lo]);
    const float l = a.clo[src];
    ehi[e] = a.chi[src];
    elo[e] = l == l ? l : -INFINITY;
    eid[e] = a.cid[src];
  }
  if (tid < D) qr_s[tid] = a.qrot[(size_t)q * D + tid];
  if (tid < (1 << BITS)) cen_s[tid] = a.cen[tid];
  __syncthreads();
  // tau' = max(tau, k-th best lo): a 32-step binary search on keys, every thread holding
  // its EPT entries' keys (per step a compare mask and a popcount per register, one LDS
  // add per wave).  Up to one entry per thread every entry is rescored anyway: no search.
  constexpr int EPT = (MCAP + kMqThreads - 1) / kMqThreads;
  if (tid < 32) tcnt[tid] = 0;
  uint32_t x = 0;
  if (M > kMqThreads) {  // uniform
    uint32_t u[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int e = j * kMqThreads + tid;
      u[j] = (e < M && elo[e] > -INFINITY) ? fs_fkey(elo[e]) : 0u;
    }
    __syncthreads();
#pragma unroll 1
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t t = x | (1u << bit);
      int cc = 0;  // wave-uniform
#pragma unroll
      for (int j = 0; j < EPT; ++j)
        if (j * kMqThreads < M) cc += __popcll(__ballot(u[j] >= t));
      if (lane == 0 && cc) atomicAdd(&tcnt[bit], cc);
      __syncthreads();
      if (tcnt[bit] >= k) x = t;
    }
  }
  const float tk = x ? fs_unkey(x) : -INFINITY;
  const float tau2 = fmaxf(a.tau[q], tk);
  // survivors: entries whose hi reaches tau'; their ids move to the front of eid (every
  // entry is read before any is overwritten; order does not matter, the ranking orders them)
  if (tid == 0) { m2_s = 0; nvalid_s = 0; }
  __syncthreads();
  int my[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = j * kMqThreads + tid;
    my[j] = (e < M && !(ehi[e] < tau2)) ? eid[e] : -1;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if (my[j] >= 0) eid[atomicAdd(&m2_s, 1)] = my[j];
  __syncthreads();
  const int m2 = m2_s;
  // exact rescoring of the survivors: the row's codes and norm from memory
  constexpr int RB = D * BITS / 8;
  for (int s = tid; s < m2; s += kMqThreads) {
    const int id = eid[s];
    // the row's bytes (8-byte aligned) and norm requested together, then scored from
    // registers
    uint32_t rw[RB / 4];
    const u32x2* r2 = reinterpret_cast<const u32x2*>(a.rows + (size_t)id * RB);
#pragma unroll
    for (int i = 0; i < RB / 8; ++i) {
      const u32x2 v = r2[i];
      rw[2 * i] = v.x; rw[2 * i + 1] = v.y;
    }
    const float nrm = a.norms[id];
    const float sc = exact_row_score_regs<D, BITS>(rw, nrm, qr_s, cen_s);
    const bool ok = !__builtin_isnan(sc);
    ehi[s] = ok ? sc : -INFINITY;
    if (!ok) eid[s] = INT_MAX;  // ranks below every listed row
    else atomicAdd(&nvalid_s, 1);
  }
  for (int s = m2 + tid; s < ((m2 + 3) & ~3); s += kMqThreads) { ehi[s] = -INFINITY; eid[s] = INT_MAX; }
  int* rk = reinterpret_cast<int*>(elo);
  // only the survivors that can be among the k best are ranked
  const int m3 = rank_best<kMqThreads, EPT>(ehi, eid, m2, k, rk, tid, &ts_s, shi_s);
  float* os = a.out_s + (size_t)q * k;
  int64_t* oi = a.out_i + (size_t)q * k;
  for (int s = tid; s < m3; s += kMqThreads) {
    const int id = eid[s], rank = rk[s];
    if ((id != INT_MAX) & (rank < k)) { os[rank] = ehi[s]; oi[rank] = id; }
  }
  for (int e = nvalid_s + tid; e < k; e += kMqThreads) { os[e] = -INFINITY; oi[e] = -1; }
}

// ------------------------------------------------------------------ softmax stats
// stats[q] = (max_t s, sum_t exp(s - max)) over the valid tokens of query q's stream.
__global__ __launch_bounds__(kThreads) void softmax_stats_kernel(const float* __restrict__ scores,
                                                                 int64_t t_max,
                                                                 const int32_t* __restrict__ seq_lens,
                                                                 int q_per_batch,
                                                                 float2* __restrict__ stats) {
  __shared__ float red[kThreads];
  const int q = blockIdx.x;
  const int64_t n = min<int64_t>(seq_lens[q / q_per_batch], t_max);
  const float* sp = scores + (size_t)q * t_max;
  float m = -INFINITY;
  for (int64_t t = threadIdx.x; t < n; t += kThreads) m = fmaxf(m, sp[t]);
  red[threadIdx.x] = m;
  __syncthreads();
  for (int st = kThreads / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
    __syncthreads();
  }
  m = red[0];
  __syncthreads();
  float l = 0.f;
  for (int64_t t = threadIdx.x; t < n; t += kThreads) l += __expf(sp[t] - m);
  red[threadIdx.x] = l;
  __syncthreads();
  for (int st = kThreads / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  if (threadIdx.x == 0) stats[q] = make_float2(m, red[0]);
}

// ------------------------------------------------------------------ values
struct ValuesArgs {
  const uint8_t* packed;    // stream s rows at packed + s * stream_rows * P
  const float* vnorms;      // stream s at vnorms + s * stream_rows
  int64_t stream_rows;
  int64_t nrows;            // when seq_lens == nullptr
  const int32_t* seq_lens;
  int spb;
  int d;
  int bits;
  const float* cen;
  int qps;                  // queries per stream
  // weights: explicit [nq_total][w_stride] (op), or exp(s - m) / l from scores + stats
  const float* w;
  int64_t w_stride;
  const float* scores;      // [nq_total][stream_rows]
  const float2* stats;
  float* part;              // [nq_total][nsplit][d]
  int nsplit;
};

template <bool kDecode>
__global__ __launch_bounds__(kThreads) void values_kernel(ValuesArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t rows_s[kValTokens * 4 * 32];
  __shared__ __attribute__((aligned(16))) float w_s[kValTokens][4];
  __shared__ float cen_s[16];
  __shared__ float red_s[kThreads / 4 * 16];
  const int sp = blockIdx.x, qb = blockIdx.y, s = blockIdx.z;
  const int d = a.d, bits = a.bits;
  const int bpp = (d + 7) >> 3;
  const int P = bits * bpp;
  int64_t nrows = a.nrows;
  if (a.seq_lens) {
    const int64_t sl = a.seq_lens[s / a.spb];
    nrows = sl < a.stream_rows ? sl : a.stream_rows;
  }
  const int q0 = s * a.qps + qb * 4;
  const int nq = min(4, a.qps - qb * 4);
  const int64_t t0 = (int64_t)sp * kSplitTokens;
  const int64_t t1 = min<int64_t>(t0 + kSplitTokens, nrows);
  const int ng = (d + 3) >> 2;          // dim groups of 4
  const int nsl = kThreads / ng;        // token slices
  const int tid = threadIdx.x;
  const int g = tid % ng, sl = tid / ng;
  const bool active = sl < nsl;
  if (tid < (1 << bits)) cen_s[tid] = a.cen[tid];
  float2 st[4];
  if (kDecode) {
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) st[qi] = qi < nq ? a.stats[q0 + qi] : make_float2(0.f, 1.f);
  }
  float acc[4][4];
#pragma unroll
  for (int qi = 0; qi < 4; ++qi)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[qi][i] = 0.f;

  const uint8_t* base = a.packed + (size_t)s * a.stream_rows * P;
  const float* vn = a.vnorms + (size_t)s * a.stream_rows;
  for (int64_t c0 = t0; c0 < t1; c0 += kValTokens) {
    const int nt = (int)min<int64_t>(kValTokens, t1 - c0);
    __syncthreads();
    for (int idx = tid; idx < nt * P; idx += kThreads) rows_s[idx] = base[(size_t)c0 * P + idx];
    for (int idx = tid; idx < nt * 4; idx += kThreads) {
      const int t = idx >> 2, qi = idx & 3;
      float w = 0.f;
      if (qi < nq) {
        const int64_t tt = c0 + t;
        if (kDecode) {
          const float sc = a.scores[(size_t)(q0 + qi) * a.stream_rows + tt];
          w = __expf(sc - st[qi].x) / st[qi].y;
        } else {
          w = a.w[(size_t)(q0 + qi) * a.w_stride + tt];
        }
        w *= vn[tt];
      }
      w_s[t][qi] = w;
    }
    __syncthreads();
    if (active) {
      const int kb = g >> 1;
      const int sh = (g & 1) ? 0 : 4;
      for (int t = sl; t < nt; t += nsl) {
        const uint8_t* r = rows_s + t * P;
        uint32_t nib[4];
        for (int p = 0; p < 4; ++p) nib[p] = p < bits ? (r[p * bpp + kb] >> sh) & 0xFu : 0u;
        const float4 w4 = *reinterpret_cast<const float4*>(&w_s[t][0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t code = ((nib[0] >> (3 - i)) & 1u) | (((nib[1] >> (3 - i)) & 1u) << 1) |
                                (((nib[2] >> (3 - i)) & 1u) << 2) | (((nib[3] >> (3 - i)) & 1u) << 3);
          const float v = cen_s[code];
          acc[0][i] = fmaf(w4.x, v, acc[0][i]);
          acc[1][i] = fmaf(w4.y, v, acc[1][i]);
          acc[2][i] = fmaf(w4.z, v, acc[2][i]);
          acc[3][i] = fmaf(w4.w, v, acc[3][i]);
        }
      }
    }
  }
  // reduce over slices: red_s[g][qi*4+i] accumulated slice by slice
  __syncthreads();
  for (int slice = 0; slice < nsl; ++slice) {
    if (active && sl == slice) {
#pragma unroll
      for (int qi = 0; qi < 4; ++qi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float& dst = red_s[g * 16 + qi * 4 + i];
          dst = (slice == 0) ? acc[qi][i] : dst + acc[qi][i];
        }
    }
    __syncthreads();
  }
  for (int idx = tid; idx < nq * d; idx += kThreads) {
    const int qi = idx / d, j = idx - qi * d;
    const float v = (t0 < t1) ? red_s[(j >> 2) * 16 + qi * 4 + (j & 3)] : 0.f;
    a.part[((size_t)(q0 + qi) * a.nsplit + sp) * d + j] = v;
  }
}

// out[q][k] = sum_j (sum_sp part[q][sp][j]) * M[j][k], cast to out_dt; optionally the
// log-sum-exp of the query's scores from its softmax stats.
__global__ void combine_kernel(const float* __restrict__ part, int nsplit, int d,
                               const float* __restrict__ M, const int32_t* __restrict__ seq_lens,
                               int q_per_batch, int out_dt, void* __restrict__ out,
                               const float2* __restrict__ stats, float* __restrict__ lse) {
  __shared__ float o_s[256];
  const int q = blockIdx.x;
  if (lse && threadIdx.x == 0) {
    const bool empty = seq_lens && seq_lens[q / q_per_batch] <= 0;
    lse[q] = (empty || !stats) ? -INFINITY : stats[q].x + logf(stats[q].y);
  }
  int ns = nsplit;
  if (seq_lens) {
    const int64_t n = seq_lens[q / q_per_batch];
    const int64_t need = (n + kSplitTokens - 1) / kSplitTokens;
    ns = (int)min<int64_t>(need, nsplit);
  }
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    float v = 0.f;
    for (int sp = 0; sp < ns; ++sp) v += part[((size_t)q * nsplit + sp) * d + j];
    o_s[j] = v;
  }
  __syncthreads();
  for (int kk = threadIdx.x; kk < d; kk += blockDim.x) {
    float v = 0.f;
    for (int j = 0; j < d; ++j) v = fmaf(o_s[j], M[(size_t)j * d + kk], v);
    store_from_f32(out, (int64_t)q * d + kk, v, out_dt);
  }
}

// ------------------------------------------------------------------ host helpers

int scan_blocks(int64_t nrows) {
  const int64_t want = (nrows + 64 * 8 * kWaves - 1) / (64 * 8 * kWaves);  // >= 8 steps per wave
  // Six 4-wave blocks per CU (the 64/128-dim scan kernels stay under 80 VGPRs, so all
  // six are resident); measured faster than four or eight.
  int64_t cap = (int64_t)device_cu_count() * 6;
  if (cap > (int64_t)kThreads * kMaxBlocksPerLane) cap = (int64_t)kThreads * kMaxBlocksPerLane;
  int64_t b = want < cap ? want : cap;
  return (int)(b < 1 ? 1 : b);
}

template <int BITS, int BPP, int QB, bool TOPK, bool GENERIC, bool PAIRS = false, bool PROD = false>
int launch_scan_t(const ScanArgs& a, dim3 grid, hipStream_t st) {
  static_assert(QB * 8 * (GENERIC ? 32 : BPP) * ((1 << BITS) * 4 + (PROD ? 16 : 0)) <= 48 * 1024,
                "table too large");
  ScanArgs b = a;
  b.ccap = TOPK ? cand_cap(a.k) : 0;
  const size_t lds = TOPK ? (size_t)kWaves * QB * b.ccap * 8 : 0;  // the top-k lists
  hipLaunchKernelGGL((scan_kernel<BITS, BPP, QB, TOPK, GENERIC, PAIRS, PROD>), grid, dim3(kThreads), lds,
                     st, b);
  TQ_LAUNCH_CHECK("scan_kernel");
  return TQ_OK;
}

// Queries per block: 4 for the 64/128-dim layouts, 2 for the generic (256-dim) one.
inline int queries_per_block(const ScanArgs& a) {
  const bool fast = a.bpp == 8 || a.bpp == 16;
  if (a.qps < 2) return 1;
  return fast ? 4 : 2;
}

// The fast loaders issue 8/16-byte loads: they need 16-byte aligned bases (row strides
// of the fast layouts keep that alignment).
inline bool fast_aligned(const ScanArgs& a) {
  return ((reinterpret_cast<uintptr_t>(a.packed) | reinterpret_cast<uintptr_t>(a.signs)) & 15u) == 0;
}

template <int BITS, bool TOPK, bool PROD = false>
int launch_scan_bits(const ScanArgs& a, int qb, dim3 grid, hipStream_t st) {
  const bool aligned = fast_aligned(a);
  if (aligned && a.bpp == 16) {
    return qb == 4 ? launch_scan_t<BITS, 16, 4, TOPK, false, false, PROD>(a, grid, st)
                   : launch_scan_t<BITS, 16, 1, TOPK, false, false, PROD>(a, grid, st);
  }
  if (aligned && a.bpp == 8) {
    return qb == 4 ? launch_scan_t<BITS, 8, 4, TOPK, false, false, PROD>(a, grid, st)
                   : launch_scan_t<BITS, 8, 1, TOPK, false, false, PROD>(a, grid, st);
  }
  return qb >= 2 ? launch_scan_t<BITS, 32, 2, TOPK, true, false, PROD>(a, grid, st)
                 : launch_scan_t<BITS, 32, 1, TOPK, true, false, PROD>(a, grid, st);
}

// Pair-layout rows: 4-bit codes, 64 or 128 dims, 16-byte aligned base (checked by callers).
template <bool TOPK>
int launch_scan_pairs(const ScanArgs& a, int qb, dim3 grid, hipStream_t st) {
  if (a.bpp == 16) {
    return qb == 4 ? launch_scan_t<4, 16, 4, TOPK, false, true>(a, grid, st)
                   : launch_scan_t<4, 16, 1, TOPK, false, true>(a, grid, st);
  }
  return qb == 4 ? launch_scan_t<4, 8, 4, TOPK, false, true>(a, grid, st)
                 : launch_scan_t<4, 8, 1, TOPK, false, true>(a, grid, st);
}

// Row blocks of a pair-layout one-query scan: pair_scan_kernel's blocks are three
// scan_kernel blocks in size (the same waves in all).
int pair_scan_blocks(int64_t nrows) {
  const int b = (scan_blocks(nrows) + kPsBlocksPerScan - 1) / kPsBlocksPerScan;
  return b < 1 ? 1 : b;
}

template <bool TOPK, int BITS, bool PROD = false>
int launch_pair_scan_b(const ScanArgs& a, dim3 grid, hipStream_t st) {
  ScanArgs b = a;
  b.ccap = TOPK ? cand_cap(a.k) : 0;
  const size_t lds = TOPK ? (size_t)kPsWaves * b.ccap * 8 : 0;  // the top-k lists
  if (a.bpp == 16) hipLaunchKernelGGL((pair_scan_kernel<128, TOPK, BITS, PROD>), grid, dim3(kPsThreads), lds, st, b);
  else hipLaunchKernelGGL((pair_scan_kernel<64, TOPK, BITS, PROD>), grid, dim3(kPsThreads), lds, st, b);
  TQ_LAUNCH_CHECK("pair_scan_kernel");
  return TQ_OK;
}

template <bool TOPK>
int launch_pair_scan(const ScanArgs& a, dim3 grid, hipStream_t st, int bits = 4) {
  if (a.signs) {  // prod rows: `bits` is the MSE half's width
    if (bits == 2) return launch_pair_scan_b<TOPK, 2, true>(a, grid, st);
    if (bits == 3) return launch_pair_scan_b<TOPK, 3, true>(a, grid, st);
    return fail(TQ_EINVAL, "prod pair rows hold 2- or 3-bit MSE codes, got %d", bits);
  }
  if (bits == 2) return launch_pair_scan_b<TOPK, 2>(a, grid, st);
  if (bits == 3) return launch_pair_scan_b<TOPK, 3>(a, grid, st);
  return launch_pair_scan_b<TOPK, 4>(a, grid, st);
}

// *nblocks_out: the grid's row blocks (TOPK: the lists merge_kernel reads per query).
int launch_scan(const ScanArgs& a, int bits, bool topk, int nstreams, hipStream_t st,
                bool pairs = false, int* nblocks_out = nullptr) {
  const bool aligned = fast_aligned(a);
  int qb = queries_per_block(a);
  if (!aligned && qb > 2) qb = 2;
  // 2- and 3-bit pair rows: one query per block row of the pair scan, at any query count
  if (pairs && bits != 4) qb = 1;
  const int64_t rows_hint = a.seq_lens ? a.stream_rows : a.nrows;
  const bool pair1 = pairs && qb == 1;
  dim3 grid(pair1 ? (unsigned)pair_scan_blocks(rows_hint) : (unsigned)scan_blocks(rows_hint),
            (unsigned)((a.qps + qb - 1) / qb), (unsigned)nstreams);
  if (nblocks_out) *nblocks_out = (int)grid.x;
  // The fast loaders address a block's rows with 32-bit buffer offsets.
  const int64_t per_block = ((rows_hint + grid.x - 1) / grid.x + 63) / 64 * 64;
  if (per_block * (int64_t)(bits * a.bpp) >= ((int64_t)1 << 32))
    return fail(TQ_EINVAL, "too many rows per scan block");
  if (pairs) {
    if (bits < 2 || bits > 4 || !aligned || (a.bpp != 8 && a.bpp != 16))
      return fail(TQ_EINVAL, "pair-row scan needs 2-4 bit codes, dim 64 or 128 and a 16-byte aligned base");
    if (a.signs && !pair1) return fail(TQ_EINVAL, "prod pair rows need 2- or 3-bit MSE codes");
    if (pair1) return topk ? launch_pair_scan<true>(a, grid, st, bits) : launch_pair_scan<false>(a, grid, st, bits);
    return topk ? launch_scan_pairs<true>(a, qb, grid, st) : launch_scan_pairs<false>(a, qb, grid, st);
  }
  if (a.signs) {
    // Prod rows: `bits` is the MSE code width (the prod bit budget minus the sign bit).
    switch (bits) {
      case 1: return topk ? launch_scan_bits<1, true, true>(a, qb, grid, st) : launch_scan_bits<1, false, true>(a, qb, grid, st);
      case 2: return topk ? launch_scan_bits<2, true, true>(a, qb, grid, st) : launch_scan_bits<2, false, true>(a, qb, grid, st);
      case 3: return topk ? launch_scan_bits<3, true, true>(a, qb, grid, st) : launch_scan_bits<3, false, true>(a, qb, grid, st);
    }
    return fail(TQ_EINVAL, "prod bit_width must be 2-4, got %d", bits + 1);
  }
  switch (bits) {
    case 1: return topk ? launch_scan_bits<1, true>(a, qb, grid, st) : launch_scan_bits<1, false>(a, qb, grid, st);
    case 2: return topk ? launch_scan_bits<2, true>(a, qb, grid, st) : launch_scan_bits<2, false>(a, qb, grid, st);
    case 3: return topk ? launch_scan_bits<3, true>(a, qb, grid, st) : launch_scan_bits<3, false>(a, qb, grid, st);
    case 4: return topk ? launch_scan_bits<4, true>(a, qb, grid, st) : launch_scan_bits<4, false>(a, qb, grid, st);
  }
  return fail(TQ_EINVAL, "bit_width must be 1-4, got %d", bits);
}

// Row blocks of the filtered pair scan: one 8-wave block per CU, fewer when there are
// fewer 64-row groups than waves.
int filter_blocks(int64_t nrows) {
  const int64_t groups = (nrows + 63) / 64;
  const int64_t want = (groups + kFsWaves - 1) / kFsWaves;
  const int64_t cap = (int64_t)device_cu_count();
  const int64_t b = want < cap ? want : cap;
  return (int)(b < 1 ? 1 : b);
}

// Workspace of the filtered pair scan: the block lists, k (score, id) per block and query.
size_t filter_workspace_bytes(int64_t nq, int d, int64_t N, int k) {
  (void)d;
  const size_t nb = (size_t)filter_blocks(N);
  return align_up((size_t)nq * nb * k * 4, 256) * 2;
}

template <int D>
int launch_filter_d(const FilterArgs& f, int nb, int nq, bool big, hipStream_t st) {
  const dim3 grid((unsigned)nb, (unsigned)nq);
  if (big) hipLaunchKernelGGL((pair_filter_kernel<D, true>), grid, dim3(kFsThreads), 0, st, f);
  else hipLaunchKernelGGL((pair_filter_kernel<D, false>), grid, dim3(kFsThreads), 0, st, f);
  TQ_LAUNCH_CHECK("pair_filter_kernel");
  const int nslots = nb * f.k;
  const dim3 mg((unsigned)nq);
  if (nslots <= 4 * kFmThreads) hipLaunchKernelGGL((filter_merge_kernel<4>), mg, dim3(kFmThreads), 0, st, f, nb);
  else if (nslots <= 8 * kFmThreads) hipLaunchKernelGGL((filter_merge_kernel<8>), mg, dim3(kFmThreads), 0, st, f, nb);
  else if (nslots <= 16 * kFmThreads) hipLaunchKernelGGL((filter_merge_kernel<16>), mg, dim3(kFmThreads), 0, st, f, nb);
  else hipLaunchKernelGGL((filter_merge_kernel<kFmRegs>), mg, dim3(kFmThreads), 0, st, f, nb);
  TQ_LAUNCH_CHECK("filter_merge_kernel");
  return TQ_OK;
}

int launch_filter(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d, const uint8_t* pairs,
                  const float* norms, int64_t N, const float* centroids, const float* rotation,
                  int32_t k, float* out_scores, int64_t* out_ids, char* ws, hipStream_t st) {
  TQ_REQUIRE(nq <= 65535, "too many queries in one call");
  const int nb = filter_blocks(N);
  TQ_REQUIRE(nb * k <= kFmRegs * kFmThreads && nb <= 64 * kFmWaves, "too many block lists for the merge");
  FilterArgs f{};
  f.rows = pairs; f.norms = norms; f.n = N; f.q = queries; f.q_dt = q_dtype; f.rot = rotation;
  f.cen = centroids; f.k = k;
  f.bs = reinterpret_cast<float*>(ws);
  ws += align_up((size_t)nq * nb * k * 4, 256);
  f.bi = reinterpret_cast<int32_t*>(ws);
  f.out_s = out_scores; f.out_i = out_ids;
  // 32-bit offsets while rows and norms stay under 2^32 bytes
  const bool big = N * (d / 2) >= ((int64_t)1 << 32) - 4096 || N * 4 >= ((int64_t)1 << 32) - 4096;
  return d == 128 ? launch_filter_d<128>(f, nb, (int)nq, big, st)
                  : launch_filter_d<64>(f, nb, (int)nq, big, st);
}

// ------------------------------------------------------------------ multi-query filtered scan: host
// Workspace layout of the multi-query filtered pair scan.  Per call: rotated queries, A
// operands, tile parameters, tau and flags for every query; per round of at most
// kMqTilesPerRound tiles (reused round after round): bucket maxima, listed rows and the
// exact fallback's block lists.
struct MqLayout {
  int ntiles, tiles_round, nbk, nsgroups, sstride, nb, fbx;
  size_t qrot, qa, tparam, tau, flag, buckets, cnt, chi, clo, cid, fps, fpi, total;
};

int pair_scan_blocks(int64_t nrows);

MqLayout mq_layout(int64_t nq, int d, int64_t N, int k, int bits) {
  MqLayout L{};
  const int KT = d / 32;
  L.ntiles = (int)((nq + kMqQ - 1) / kMqQ);
  L.tiles_round = L.ntiles < kMqTilesPerRound ? L.ntiles : kMqTilesPerRound;
  const int64_t ngroups = (N + 63) / 64;
  L.nsgroups = (int)(ngroups < kMqSampleGroups ? ngroups : kMqSampleGroups);
  if (L.nsgroups < 1) L.nsgroups = 1;
  L.sstride = (int)(ngroups / L.nsgroups);
  if (L.sstride < 1) L.sstride = 1;
  const int sblocks = (L.nsgroups + kMqWaves * kMqGroupsPerWave - 1) / (kMqWaves * kMqGroupsPerWave);
  L.nbk = sblocks;
  L.nb = filter_blocks(N);
  // row blocks of the exact fallback: the 4-bit multi-query scan, or the pair-row scan
  const int fb = bits == 4 ? scan_blocks(N) : pair_scan_blocks(N);
  L.fbx = fb < kMqFallbackBlocks ? fb : kMqFallbackBlocks;
  const size_t rq = (size_t)L.tiles_round * kMqQ;
  size_t o = 256;
  auto take = [&](size_t bytes) { const size_t at = o; o = align_up(o + bytes, 256); return at; };
  L.qrot = take((size_t)nq * d * 4);
  L.qa = take((size_t)L.ntiles * KT * 4 * 64 * 16);
  L.tparam = take((size_t)L.ntiles * 2 * 4);
  L.tau = take((size_t)nq * 4);
  L.flag = take((size_t)nq * 4);
  L.buckets = take(rq * L.nbk * 4);
  L.cnt = take((size_t)L.tiles_round * L.nb * kMqQ * 4);
  const size_t slots = (size_t)L.tiles_round * L.nb * kMqQ * kMqCap;
  L.chi = take(slots * 4);
  L.clo = take(slots * 4);
  L.cid = take(slots * 4);
  L.fps = take(rq * L.fbx * k * 4);
  L.fpi = take(rq * L.fbx * k * 4);
  L.total = o;
  return L;
}

// The multi-query filter applies to pair rows of d 64 / 128 with at least two queries; for
// 4-bit rows also to one query with k above the one-query filter's kSmallK.
bool mq_applies(int64_t nq, int d, int64_t N, int k, int bits) {
  return (nq >= 2 || (bits == 4 && nq == 1 && k > kSmallK)) && N > 0 && (d == 64 || d == 128) &&
         bits >= 2 && bits <= 4;
}

template <int D, int BITS>
int launch_mq_d(const MqArgs& base, const MqLayout& L, const void* queries, size_t qbytes,
                char* ws, bool big, hipStream_t st) {
  hipLaunchKernelGGL((mq_rotate_kernel<D>), dim3((unsigned)((base.nq + kMqRotQ - 1) / kMqRotQ)),
                     dim3(D), 0, st, base);
  TQ_LAUNCH_CHECK("mq_rotate_kernel");
  hipLaunchKernelGGL((mq_tile_kernel<D, BITS>), dim3((unsigned)L.ntiles), dim3(kMqThreads), 0, st, base);
  TQ_LAUNCH_CHECK("mq_tile_kernel");
  const int sblocks = L.nbk;
  for (int t0 = 0; t0 < L.ntiles; t0 += L.tiles_round) {
    MqArgs a = base;
    a.tile0 = t0;
    const int nt = L.ntiles - t0 < L.tiles_round ? L.ntiles - t0 : L.tiles_round;
    const dim3 sg((unsigned)sblocks, (unsigned)nt), fg((unsigned)L.nb, (unsigned)nt);
    if (big) {
      hipLaunchKernelGGL((mq_sample_kernel<D, BITS, true>), sg, dim3(kMqThreads), 0, st, a);
    } else {
      hipLaunchKernelGGL((mq_sample_kernel<D, BITS, false>), sg, dim3(kMqThreads), 0, st, a);
    }
    TQ_LAUNCH_CHECK("mq_sample_kernel");
    if (big) {
      hipLaunchKernelGGL((mq_filter_kernel<D, BITS, true>), fg, dim3(kMqThreads), 0, st, a);
    } else {
      hipLaunchKernelGGL((mq_filter_kernel<D, BITS, false>), fg, dim3(kMqThreads), 0, st, a);
    }
    TQ_LAUNCH_CHECK("mq_filter_kernel");
    if (a.k > kSmallK)
      hipLaunchKernelGGL((mq_merge_kernel<D, BITS, kMqMergeCapBig>), dim3((unsigned)(nt * kMqQ)), dim3(kMqThreads), 0, st, a);
    else
      hipLaunchKernelGGL((mq_merge_kernel<D, BITS, kMqMergeCap>), dim3((unsigned)(nt * kMqQ)), dim3(kMqThreads), 0, st, a);
    TQ_LAUNCH_CHECK("mq_merge_kernel");
    // The exact scan for the round's flagged queries (blocks of unflagged ones return).
    const int q0 = t0 * kMqQ;
    const int rq = (int)(a.nq - q0 < nt * kMqQ ? a.nq - q0 : nt * kMqQ);
    ScanArgs s{};
    s.packed = a.rows; s.norms = a.norms; s.stream_rows = a.n; s.nrows = a.n; s.seq_lens = nullptr;
    s.spb = 1; s.bpp = D / 8; s.q = static_cast<const char*>(queries) + (size_t)q0 * qbytes;
    s.q_dt = a.q_dt; s.d = D; s.rot = a.rot; s.cen = a.cen; s.qps = rq; s.post_scale = 1.f;
    s.k = a.k;
    s.part_s = reinterpret_cast<float*>(ws + L.fps);
    s.part_i = reinterpret_cast<int32_t*>(ws + L.fpi);
    s.scores = nullptr;
    s.out_s = a.out_s + (size_t)q0 * a.k;
    s.out_i = a.out_i + (size_t)q0 * a.k;
    s.qflag = a.flag + q0;
    int rc;
    if constexpr (BITS == 4) {
      rc = launch_scan_pairs<true>(s, 4, dim3((unsigned)L.fbx, (unsigned)((rq + 3) / 4), 1u), st);
    } else {  // the pair-row scan: one query per block row
      rc = launch_pair_scan<true>(s, dim3((unsigned)L.fbx, (unsigned)rq, 1u), st, BITS);
    }
    if (rc != TQ_OK) return rc;
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)rq), dim3(kThreads), 0, st, s.part_s, s.part_i,
                       L.fbx, a.k, s.out_s, s.out_i, (const int32_t*)s.qflag);
    TQ_LAUNCH_CHECK("merge_kernel");
  }
  return TQ_OK;
}

int launch_mq(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d, const uint8_t* pairs,
              const float* norms, int64_t N, const float* centroids, const float* rotation,
              int32_t bits, int32_t k, float* out_scores, int64_t* out_ids, char* ws, hipStream_t st) {
  const MqLayout L = mq_layout(nq, d, N, k, bits);
  TQ_REQUIRE(L.nb <= kMqThreads, "too many filter blocks");
  MqArgs a{};
  a.rows = pairs; a.norms = norms; a.n = N; a.q = queries; a.q_dt = q_dtype; a.nq = (int)nq;
  a.rot = rotation; a.cen = centroids; a.k = k;
  a.qrot = reinterpret_cast<float*>(ws + L.qrot);
  a.qa = reinterpret_cast<uint32_t*>(ws + L.qa);
  a.tparam = reinterpret_cast<float*>(ws + L.tparam);
  a.tau = reinterpret_cast<float*>(ws + L.tau);
  a.flag = reinterpret_cast<int*>(ws + L.flag);
  a.buckets = reinterpret_cast<float*>(ws + L.buckets);
  a.cnt = reinterpret_cast<int*>(ws + L.cnt);
  a.chi = reinterpret_cast<float*>(ws + L.chi);
  a.clo = reinterpret_cast<float*>(ws + L.clo);
  a.cid = reinterpret_cast<int*>(ws + L.cid);
  a.nbk = L.nbk; a.sstride = L.sstride; a.nsgroups = L.nsgroups; a.nb = L.nb;
  a.out_s = out_scores; a.out_i = out_ids;
  const size_t qbytes = (size_t)d * dtype_size(q_dtype);
  // 32-bit offsets while rows and norms stay under 2^32 bytes
  const bool big = N * (d * bits / 8) >= ((int64_t)1 << 32) - 4096 || N * 4 >= ((int64_t)1 << 32) - 4096;
  if (d == 128) {
    if (bits == 2) return launch_mq_d<128, 2>(a, L, queries, qbytes, ws, big, st);
    if (bits == 3) return launch_mq_d<128, 3>(a, L, queries, qbytes, ws, big, st);
    return launch_mq_d<128, 4>(a, L, queries, qbytes, ws, big, st);
  }
  if (bits == 2) return launch_mq_d<64, 2>(a, L, queries, qbytes, ws, big, st);
  if (bits == 3) return launch_mq_d<64, 3>(a, L, queries, qbytes, ws, big, st);
  return launch_mq_d<64, 4>(a, L, queries, qbytes, ws, big, st);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

size_t tq_scan_workspace_bytes(int64_t nq, int32_t d, int32_t bit_width, int64_t N, int32_t k) {
  if (nq <= 0 || d <= 0 || bit_width < 1 || bit_width > 4) return 0;
  size_t bytes = 256;
  if (k > 0) {
    const size_t nb = (size_t)scan_blocks(N);
    bytes += align_up((size_t)nq * nb * k * 4, 256) * 2;
    if (bit_width == 4 && (d == 64 || d == 128)) {  // the filtered pair scan's lists
      const size_t fb = 256 + filter_workspace_bytes(nq, d, N, k);
      if (fb > bytes) bytes = fb;
    }
  }
  return bytes;
}

size_t tq_scan_pair_rows_workspace_bytes(int64_t nq, int32_t d, int32_t bit_width, int64_t N,
                                         int32_t k) {
  size_t bytes = tq_scan_workspace_bytes(nq, d, bit_width, N, k);
  if (k >= 1 && k <= kMaxK && mq_applies(nq, d, N, k, bit_width)) {
    const size_t mq = mq_layout(nq, d, N, k, bit_width).total;
    if (mq > bytes) bytes = mq;
  }
  return bytes;
}

size_t tq_scan_pairs_workspace_bytes(int64_t nq, int32_t d, int64_t N, int32_t k) {
  return tq_scan_pair_rows_workspace_bytes(nq, d, 4, N, k);
}

}  // extern "C"

namespace {

// The QJL half of prod rows (reference.py:392-469 outputs beside the MSE codes).
struct ProdRows {
  const uint8_t* signs;   // [rows][ceil(d/8)] sign bits, 1-bit bit-plane layout
  const float* gammas;    // [rows] residual norms
  const float* qjl;       // [d][d] S
};

void set_prod(ScanArgs& a, const ProdRows& p) {
  a.signs = p.signs; a.gammas = p.gammas; a.qjl = p.qjl;
  a.qjl_scale = (float)(1.2533141373155002512 / a.d);  // sqrt(pi/2) / d, as reference.py:527
}

int ip_scan_topk(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                 const uint8_t* packed, const float* norms, int64_t N, const float* centroids,
                 const float* rotation, int32_t bit_width, int32_t k, float* out_scores,
                 int64_t* out_ids, void* workspace, size_t workspace_bytes, void* stream,
                 bool pairs, const ProdRows* prod = nullptr) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4, got %d", bit_width);
  TQ_REQUIRE(!prod || bit_width >= 2, "prod bit_width must be 2-4, got %d", bit_width);
  TQ_REQUIRE(!prod || N == 0 || (prod->signs && prod->gammas), "null pointer argument");
  TQ_REQUIRE(!prod || prod->qjl, "null pointer argument");
  TQ_REQUIRE(d >= 1 && d <= 256, "dim must be in [1, 256], got %d", d);
  TQ_REQUIRE(k >= 1 && k <= kMaxK, "k must be in [1, %d], got %d", kMaxK, k);
  TQ_REQUIRE(nq >= 0 && N >= 0, "bad sizes");
  TQ_REQUIRE(N <= INT_MAX, "N must fit in int32 ids");
  TQ_REQUIRE(valid_dtype(q_dtype), "unknown dtype");
  if (nq == 0) return TQ_OK;
  TQ_REQUIRE(queries && out_scores && out_ids && centroids && rotation, "null pointer argument");
  TQ_REQUIRE(N == 0 || (packed && norms), "null pointer argument");
  const size_t need = tq_scan_workspace_bytes(nq, d, bit_width, N, k);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  hipStream_t st = as_stream(stream);
  // Several queries over pair rows: the multi-query filtered scan, when the workspace
  // holds its buffers (tq_scan_pair_rows_workspace_bytes); the exact scans below otherwise.
  if (pairs && !prod && mq_applies(nq, d, N, k, bit_width) && nq <= INT_MAX &&
      workspace_bytes >= mq_layout(nq, d, N, k, bit_width).total)
    return launch_mq(queries, q_dtype, nq, d, packed, norms, N, centroids, rotation, bit_width, k,
                     out_scores, out_ids, static_cast<char*>(workspace), st);
  char* ws = static_cast<char*>(workspace) + 256;
  // The lists are laid out for scan_blocks(N) blocks; a launch uses at most that many.
  const int nb_max = scan_blocks(N);
  float* ps = reinterpret_cast<float*>(ws);
  ws += align_up((size_t)nq * nb_max * k * 4, 256);
  int32_t* pi = reinterpret_cast<int32_t*>(ws);
  ScanArgs a{};
  a.packed = packed; a.norms = norms; a.stream_rows = N; a.nrows = N; a.seq_lens = nullptr; a.spb = 1;
  a.bpp = (d + 7) / 8; a.q = queries; a.q_dt = q_dtype; a.d = d; a.rot = rotation; a.cen = centroids;
  a.qps = (int)nq; a.post_scale = 1.f; a.k = k;
  a.part_s = ps; a.part_i = pi; a.scores = nullptr;
  a.out_s = out_scores; a.out_i = out_ids;
  if (prod) set_prod(a, *prod);
  // One query over 4-bit pair rows: the filtered scan (approximate scores on the matrix
  // cores, the candidates rescored exactly).
  if (pairs && bit_width == 4 && !prod && nq == 1 && (d == 64 || d == 128) && k <= kSmallK)
    return launch_filter(queries, q_dtype, nq, d, packed, norms, N, centroids, rotation, k,
                         out_scores, out_ids, static_cast<char*>(workspace) + 256, st);
  TQ_REQUIRE(nq <= 65535 * 4, "too many queries in one call");
  TQ_REQUIRE(!pairs || (prod ? bit_width - 1 : bit_width) == 4 || nq <= 65535, "too many queries in one call");
  int nb = 0;
  const int rc = launch_scan(a, prod ? bit_width - 1 : bit_width, true, 1, st, pairs, &nb);
  if (rc != TQ_OK) return rc;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)nq), dim3(kThreads), 0, st, ps, pi, nb, k,
                     out_scores, out_ids, (const int32_t*)nullptr);
  TQ_LAUNCH_CHECK("merge_kernel");
  return TQ_OK;
}

int attention_scores(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                     const uint8_t* packed_keys, const float* key_norms, int64_t T,
                     const float* centroids, const float* rotation, int32_t bit_width,
                     float* scores, void* workspace, size_t workspace_bytes, void* stream,
                     bool pairs, const ProdRows* prod = nullptr) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4, got %d", bit_width);
  TQ_REQUIRE(!prod || bit_width >= 2, "prod bit_width must be 2-4, got %d", bit_width);
  TQ_REQUIRE(!prod || T == 0 || (prod->signs && prod->gammas), "null pointer argument");
  TQ_REQUIRE(!prod || prod->qjl, "null pointer argument");
  TQ_REQUIRE(d >= 1 && d <= 256, "dim must be in [1, 256], got %d", d);
  TQ_REQUIRE(nq >= 0 && T >= 0, "bad sizes");
  TQ_REQUIRE(valid_dtype(q_dtype), "unknown dtype");
  if (nq == 0 || T == 0) return TQ_OK;
  TQ_REQUIRE(query && packed_keys && key_norms && centroids && rotation && scores,
             "null pointer argument");
  const size_t need = tq_scan_workspace_bytes(nq, d, bit_width, T, 0);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  hipStream_t st = as_stream(stream);
  ScanArgs a{};
  a.packed = packed_keys; a.norms = key_norms; a.stream_rows = T; a.nrows = T; a.seq_lens = nullptr;
  a.spb = 1; a.bpp = (d + 7) / 8; a.q = query; a.q_dt = q_dtype; a.d = d; a.rot = rotation;
  a.cen = centroids; a.qps = (int)nq; a.post_scale = 1.f;
  a.k = 0; a.scores = scores;
  if (prod) set_prod(a, *prod);
  TQ_REQUIRE(nq <= 65535 * 4, "too many queries in one call");
  TQ_REQUIRE(!pairs || (prod ? bit_width - 1 : bit_width) == 4 || nq <= 65535, "too many queries in one call");
  return launch_scan(a, prod ? bit_width - 1 : bit_width, false, 1, st, pairs);
}

}  // namespace

extern "C" {

int tq_ip_scan_topk(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                    const uint8_t* packed, const float* norms, int64_t N, const float* centroids,
                    const float* rotation, int32_t bit_width, int32_t k, float* out_scores,
                    int64_t* out_ids, void* workspace, size_t workspace_bytes, void* stream) {
  return ip_scan_topk(queries, q_dtype, nq, d, packed, norms, N, centroids, rotation, bit_width,
                      k, out_scores, out_ids, workspace, workspace_bytes, stream, false);
}

int tq_ip_scan_topk_pairs(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                          const uint8_t* pairs, const float* norms, int64_t N,
                          const float* centroids, const float* rotation, int32_t k,
                          float* out_scores, int64_t* out_ids, void* workspace,
                          size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(d == 64 || d == 128, "pair-layout scan needs dim 64 or 128, got %d", d);
  TQ_REQUIRE(N == 0 || (reinterpret_cast<uintptr_t>(pairs) & 15u) == 0,
             "pair-layout rows must be 16-byte aligned");
  return ip_scan_topk(queries, q_dtype, nq, d, pairs, norms, N, centroids, rotation, 4, k,
                      out_scores, out_ids, workspace, workspace_bytes, stream, true);
}

int tq_attention_scores_packed(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                               const uint8_t* packed_keys, const float* key_norms, int64_t T,
                               const float* centroids, const float* rotation, int32_t bit_width,
                               float* scores, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return attention_scores(query, q_dtype, nq, d, packed_keys, key_norms, T, centroids, rotation,
                          bit_width, scores, workspace, workspace_bytes, stream, false);
}

int tq_ip_scan_topk_prod(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                         const uint8_t* mse_packed, const uint8_t* signs, const float* res_norms,
                         const float* norms, int64_t N, const float* centroids,
                         const float* rotation, const float* qjl, int32_t bit_width, int32_t k,
                         float* out_scores, int64_t* out_ids, void* workspace,
                         size_t workspace_bytes, void* stream) {
  const ProdRows p{signs, res_norms, qjl};
  return ip_scan_topk(queries, q_dtype, nq, d, mse_packed, norms, N, centroids, rotation,
                      bit_width, k, out_scores, out_ids, workspace, workspace_bytes, stream,
                      false, &p);
}

int tq_attention_scores_prod(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                             const uint8_t* mse_packed, const uint8_t* signs,
                             const float* res_norms, const float* key_norms, int64_t T,
                             const float* centroids, const float* rotation, const float* qjl,
                             int32_t bit_width, float* scores, void* workspace,
                             size_t workspace_bytes, void* stream) {
  const ProdRows p{signs, res_norms, qjl};
  return attention_scores(query, q_dtype, nq, d, mse_packed, key_norms, T, centroids, rotation,
                          bit_width, scores, workspace, workspace_bytes, stream, false, &p);
}

int tq_attention_scores_pairs(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                              const uint8_t* pairs, const float* key_norms, int64_t T,
                              const float* centroids, const float* rotation, float* scores,
                              void* workspace, size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(d == 64 || d == 128, "pair-layout scan needs dim 64 or 128, got %d", d);
  TQ_REQUIRE(T == 0 || (reinterpret_cast<uintptr_t>(pairs) & 15u) == 0,
             "pair-layout rows must be 16-byte aligned");
  return attention_scores(query, q_dtype, nq, d, pairs, key_norms, T, centroids, rotation, 4,
                          scores, workspace, workspace_bytes, stream, true);
}

size_t tq_values_workspace_bytes(int64_t nq, int32_t d, int64_t T) {
  if (nq <= 0 || d <= 0) return 0;
  const int64_t ns = (T + kSplitTokens - 1) / kSplitTokens;
  return align_up((size_t)nq * (ns > 0 ? ns : 1) * d * 4, 256);
}

int tq_attention_values_packed(const float* attn_weights, int64_t nq, int64_t T,
                               const uint8_t* packed_values, const float* value_norms,
                               const float* centroids, const float* rotation_T, int32_t d,
                               int32_t bit_width, float* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4, got %d", bit_width);
  TQ_REQUIRE(d >= 1 && d <= 256, "dim must be in [1, 256], got %d", d);
  TQ_REQUIRE(nq >= 0 && T >= 0, "bad sizes");
  if (nq == 0) return TQ_OK;
  TQ_REQUIRE(attn_weights || T == 0, "null pointer argument");
  TQ_REQUIRE(out && centroids && rotation_T, "null pointer argument");
  TQ_REQUIRE(T == 0 || (packed_values && value_norms), "null pointer argument");
  const size_t need = tq_values_workspace_bytes(nq, d, T);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  hipStream_t st = as_stream(stream);
  float* part = static_cast<float*>(workspace);
  const int ns = (int)((T + kSplitTokens - 1) / kSplitTokens);
  TQ_REQUIRE(nq <= 65535 * 4, "too many queries in one call");
  if (ns > 0) {
    ValuesArgs a{};
    a.packed = packed_values; a.vnorms = value_norms; a.stream_rows = T; a.nrows = T;
    a.seq_lens = nullptr; a.spb = 1; a.d = d; a.bits = bit_width; a.cen = centroids;
    a.qps = (int)nq; a.w = attn_weights; a.w_stride = T; a.scores = nullptr; a.stats = nullptr;
    a.part = part; a.nsplit = ns;
    hipLaunchKernelGGL(values_kernel<false>, dim3((unsigned)ns, (unsigned)((nq + 3) / 4), 1),
                       dim3(kThreads), 0, st, a);
    TQ_LAUNCH_CHECK("values_kernel");
  }
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)nq), dim3(256), 0, st, part, ns, d, rotation_T,
                     nullptr, 1, (int)TQ_F32, out, nullptr, nullptr);
  TQ_LAUNCH_CHECK("combine_kernel");
  return TQ_OK;
}

size_t tq_decode_workspace_bytes(int32_t B, int32_t hq, int32_t d, int64_t t_max) {
  if (B <= 0 || hq <= 0 || d <= 0) return 0;
  const size_t nq = (size_t)B * hq;
  const int64_t ns = (t_max + kSplitTokens - 1) / kSplitTokens;
  size_t bytes = 256;
  bytes += align_up(nq * (size_t)(t_max > 0 ? t_max : 1) * 4, 256);   // scores
  bytes += align_up(nq * sizeof(float2), 256);                        // stats
  bytes += align_up(nq * (size_t)(ns > 0 ? ns : 1) * d * 4, 256);     // partials
  const size_t fused = fused_decode_workspace_bytes(B, hq, d, t_max);
  return bytes > fused ? bytes : fused;
}

int tq_decode_attention_packed(const void* q, tq_dtype q_dtype, int32_t B, int32_t hq, int32_t hkv,
                               int32_t d, const uint8_t* kpacked, const float* knorms,
                               const uint8_t* vpacked, const float* vnorms, int64_t t_max,
                               const int32_t* seq_lens, const float* kcentroids,
                               const float* vcentroids, const float* krotation,
                               const float* vrotation, int32_t kbits, int32_t vbits, float scale,
                               void* out, float* lse, void* workspace, size_t workspace_bytes,
                               void* stream) {
  TQ_REQUIRE(kbits >= 1 && kbits <= 4 && vbits >= 1 && vbits <= 4, "bits must be 1-4");
  TQ_REQUIRE(d >= 1 && d <= 256, "head_dim must be in [1, 256], got %d", d);
  TQ_REQUIRE(B >= 0 && hq >= 1 && hkv >= 1 && hq % hkv == 0,
             "num_heads (%d) must be a multiple of num_kv_heads (%d)", hq, hkv);
  TQ_REQUIRE(t_max >= 0, "bad t_max");
  TQ_REQUIRE(valid_dtype(q_dtype), "unknown dtype");
  if (B == 0) return TQ_OK;
  TQ_REQUIRE(q && out && seq_lens && kcentroids && vcentroids && krotation && vrotation,
             "null pointer argument");
  TQ_REQUIRE(t_max == 0 || (kpacked && knorms && vpacked && vnorms), "null pointer argument");
  const size_t need = tq_decode_workspace_bytes(B, hq, d, t_max);
  TQ_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need %zu bytes", need);
  TQ_REQUIRE((int64_t)B * hkv <= 65535, "too many (batch, kv head) streams");
  hipStream_t st = as_stream(stream);
  const FusedDecodeCall fc{q, (int)q_dtype, B, hq, hkv, d, kpacked, knorms, vpacked, vnorms,
                           t_max, seq_lens, kcentroids, vcentroids, krotation, vrotation,
                           kbits, vbits, scale, out, lse};
  if (fused_decode_covers(fc)) return launch_fused_decode(fc, workspace, workspace_bytes, st);
  const int64_t nq = (int64_t)B * hq;
  const int G = hq / hkv;
  const int ns = (int)((t_max + kSplitTokens - 1) / kSplitTokens);
  char* ws = static_cast<char*>(workspace) + 256;
  float* scores = reinterpret_cast<float*>(ws);
  ws += align_up((size_t)nq * (size_t)(t_max > 0 ? t_max : 1) * 4, 256);
  float2* stats = reinterpret_cast<float2*>(ws);
  ws += align_up((size_t)nq * sizeof(float2), 256);
  float* part = reinterpret_cast<float*>(ws);
  if (t_max > 0) {
    ScanArgs a{};
    a.packed = kpacked; a.norms = knorms; a.stream_rows = t_max; a.nrows = t_max;
    a.seq_lens = seq_lens; a.spb = hkv; a.bpp = (d + 7) / 8; a.q = q; a.q_dt = q_dtype; a.d = d;
    a.rot = krotation; a.cen = kcentroids;
    a.qps = G; a.post_scale = scale; a.k = 0; a.scores = scores;
    int rc = launch_scan(a, kbits, false, B * hkv, st);
    if (rc) return rc;
    hipLaunchKernelGGL(softmax_stats_kernel, dim3((unsigned)nq), dim3(kThreads), 0, st, scores,
                       t_max, seq_lens, hq, stats);
    TQ_LAUNCH_CHECK("softmax_stats_kernel");
    ValuesArgs v{};
    v.packed = vpacked; v.vnorms = vnorms; v.stream_rows = t_max; v.nrows = t_max;
    v.seq_lens = seq_lens; v.spb = hkv; v.d = d; v.bits = vbits; v.cen = vcentroids; v.qps = G;
    v.w = nullptr; v.w_stride = 0; v.scores = scores; v.stats = stats; v.part = part; v.nsplit = ns;
    hipLaunchKernelGGL(values_kernel<true>,
                       dim3((unsigned)ns, (unsigned)((G + 3) / 4), (unsigned)(B * hkv)),
                       dim3(kThreads), 0, st, v);
    TQ_LAUNCH_CHECK("values_kernel");
  }
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)nq), dim3(256), 0, st, part, ns, d, vrotation,
                     seq_lens, hq, (int)q_dtype, out, t_max > 0 ? stats : nullptr, lse);
  TQ_LAUNCH_CHECK("combine_kernel");
  return TQ_OK;
}

}  // extern "C"

// ------------------------------------------------------------------ pair rows <-> bit planes
namespace tq {
namespace {

// Code of dim j in a bit-plane row (reference.py:191-224 layout).
__device__ __forceinline__ uint32_t plane_code(const uint8_t* row, int bpp, int bits, int j) {
  uint32_t c = 0;
  for (int p = 0; p < bits; ++p) c |= ((row[p * bpp + (j >> 3)] >> (7 - (j & 7))) & 1u) << p;
  return c;
}

// Code of dim j in a pair row of d dims (layout above pmp_row; 4 bits: byte j/2, high
// nibble for even j).
__device__ __forceinline__ uint32_t pair_row_code(const uint8_t* row, int bits, int j) {
  if (bits == 4) return (j & 1) ? (row[j >> 1] & 15u) : (row[j >> 1] >> 4);
  if (bits == 2) return (row[j >> 2] >> (6 - 2 * (j & 3))) & 3u;
  const int pp = j >> 1, t = pp >> 4, q = pp & 15;
  uint32_t idx;
  if (q < 12) {
    idx = row[12 * t + q] & 63u;
  } else {
    idx = 0;
    for (int i = 0; i < 3; ++i) idx |= (uint32_t)((row[12 * t + 4 * i + (q - 12)] >> 6) & 3) << (2 * i);
  }
  return (j & 1) ? (idx & 7u) : (idx >> 3);
}

// One thread per output byte of the pair rows.
__global__ void pack_pair_rows_kernel(const uint8_t* __restrict__ packed, int64_t n, int d, int bits,
                                      uint8_t* __restrict__ rows) {
  const int bpp = (d + 7) / 8, P = bits * bpp, RB = d * bits / 8;
  const int64_t total = n * RB;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / RB;
    const int b = (int)(e - r * RB);
    const uint8_t* src = packed + r * P;
    uint32_t v;
    if (bits == 4) {
      v = plane_code(src, bpp, 4, 2 * b) << 4 | plane_code(src, bpp, 4, 2 * b + 1);
    } else if (bits == 2) {
      v = 0;
      for (int k = 0; k < 4; ++k) v |= plane_code(src, bpp, 2, 4 * b + k) << (6 - 2 * k);
    } else {
      const int t = b / 12, q = b - 12 * t, i = q >> 2, k = q & 3;
      const int plo = 16 * t + q, phi = 16 * t + 12 + k;
      const uint32_t ilo = plane_code(src, bpp, 3, 2 * plo) << 3 | plane_code(src, bpp, 3, 2 * plo + 1);
      const uint32_t ihi = plane_code(src, bpp, 3, 2 * phi) << 3 | plane_code(src, bpp, 3, 2 * phi + 1);
      v = ilo | ((ihi >> (2 * i)) & 3u) << 6;
    }
    rows[e] = (uint8_t)v;
  }
}

// One thread per output byte of the bit-plane rows.
__global__ void unpack_pair_rows_kernel(const uint8_t* __restrict__ rows, int64_t n, int d, int bits,
                                        uint8_t* __restrict__ packed) {
  const int bpp = (d + 7) / 8, P = bits * bpp, RB = d * bits / 8;
  const int64_t total = n * P;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / P;
    const int byte = (int)(e - r * P), pl = byte / bpp, o = byte - pl * bpp;
    uint32_t out = 0;
    for (int k = 0; k < 8 && 8 * o + k < d; ++k)
      out |= ((pair_row_code(rows + r * RB, bits, 8 * o + k) >> pl) & 1u) << (7 - k);
    packed[e] = (uint8_t)out;
  }
}

int check_pair_rows(int64_t n, int32_t d, int32_t bits) {
  TQ_REQUIRE(d == 64 || d == 128, "pair rows need dim 64 or 128, got %d", d);
  TQ_REQUIRE(bits >= 2 && bits <= 4, "pair rows hold 2-4 bit codes, got %d", bits);
  TQ_REQUIRE(n >= 0, "bad sizes");
  return TQ_OK;
}

}  // namespace
}  // namespace tq

extern "C" {

int tq_pack_pair_rows(const uint8_t* packed, int64_t n, int32_t d, int32_t bit_width, uint8_t* rows,
                      void* stream) {
  const int rc = check_pair_rows(n, d, bit_width);
  if (rc != TQ_OK) return rc;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(packed && rows, "null pointer argument");
  const int64_t total = n * d * bit_width / 8;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(pack_pair_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     packed, n, (int)d, (int)bit_width, rows);
  TQ_LAUNCH_CHECK("pack_pair_rows_kernel");
  return TQ_OK;
}

int tq_unpack_pair_rows(const uint8_t* rows, int64_t n, int32_t d, int32_t bit_width, uint8_t* packed,
                        void* stream) {
  const int rc = check_pair_rows(n, d, bit_width);
  if (rc != TQ_OK) return rc;
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(packed && rows, "null pointer argument");
  const int64_t total = n * bit_width * ((d + 7) / 8);
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(unpack_pair_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     rows, n, (int)d, (int)bit_width, packed);
  TQ_LAUNCH_CHECK("unpack_pair_rows_kernel");
  return TQ_OK;
}

int tq_ip_scan_topk_pair_rows(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                              const uint8_t* rows, const float* norms, int64_t N,
                              const float* centroids, const float* rotation, int32_t bit_width,
                              int32_t k, float* out_scores, int64_t* out_ids, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const int rc = check_pair_rows(N, d, bit_width);
  if (rc != TQ_OK) return rc;
  TQ_REQUIRE(N == 0 || (reinterpret_cast<uintptr_t>(rows) & 15u) == 0,
             "pair rows must be 16-byte aligned");
  return ip_scan_topk(queries, q_dtype, nq, d, rows, norms, N, centroids, rotation, bit_width, k,
                      out_scores, out_ids, workspace, workspace_bytes, stream, true);
}

int tq_ip_scan_topk_prod_pair_rows(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                                   const uint8_t* mse_rows, const uint8_t* signs,
                                   const float* res_norms, const float* norms, int64_t N,
                                   const float* centroids, const float* rotation, const float* qjl,
                                   int32_t bit_width, int32_t k, float* out_scores, int64_t* out_ids,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(bit_width == 3 || bit_width == 4,
             "prod pair rows hold 2- or 3-bit MSE codes (bit_width 3 or 4), got %d", bit_width);
  const int rc = check_pair_rows(N, d, bit_width - 1);
  if (rc != TQ_OK) return rc;
  TQ_REQUIRE(N == 0 || ((reinterpret_cast<uintptr_t>(mse_rows) | reinterpret_cast<uintptr_t>(signs)) & 15u) == 0,
             "pair rows and sign rows must be 16-byte aligned");
  const ProdRows p{signs, res_norms, qjl};
  return ip_scan_topk(queries, q_dtype, nq, d, mse_rows, norms, N, centroids, rotation, bit_width, k,
                      out_scores, out_ids, workspace, workspace_bytes, stream, true, &p);
}

int tq_attention_scores_prod_pair_rows(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                                       const uint8_t* mse_rows, const uint8_t* signs,
                                       const float* res_norms, const float* key_norms, int64_t T,
                                       const float* centroids, const float* rotation,
                                       const float* qjl, int32_t bit_width, float* scores,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  TQ_REQUIRE(bit_width == 3 || bit_width == 4,
             "prod pair rows hold 2- or 3-bit MSE codes (bit_width 3 or 4), got %d", bit_width);
  const int rc = check_pair_rows(T, d, bit_width - 1);
  if (rc != TQ_OK) return rc;
  TQ_REQUIRE(T == 0 || ((reinterpret_cast<uintptr_t>(mse_rows) | reinterpret_cast<uintptr_t>(signs)) & 15u) == 0,
             "pair rows and sign rows must be 16-byte aligned");
  const ProdRows p{signs, res_norms, qjl};
  return attention_scores(query, q_dtype, nq, d, mse_rows, key_norms, T, centroids, rotation,
                          bit_width, scores, workspace, workspace_bytes, stream, true, &p);
}

int tq_attention_scores_pair_rows(const void* query, tq_dtype q_dtype, int64_t nq, int32_t d,
                                  const uint8_t* rows, const float* key_norms, int64_t T,
                                  const float* centroids, const float* rotation, int32_t bit_width,
                                  float* scores, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const int rc = check_pair_rows(T, d, bit_width);
  if (rc != TQ_OK) return rc;
  TQ_REQUIRE(T == 0 || (reinterpret_cast<uintptr_t>(rows) & 15u) == 0,
             "pair rows must be 16-byte aligned");
  return attention_scores(query, q_dtype, nq, d, rows, key_norms, T, centroids, rotation, bit_width,
                          scores, workspace, workspace_bytes, stream, true);
}

}  // extern "C"

// ------------------------------------------------------------------ no-allocation scan
// tq_ip_scan_topk_pairs_noalloc: the pair-layout top-k scan with its per-block candidate
// lists in a file-scope device array instead of a caller workspace.  Each GPU holds its
// own copy of `scratch` (TQ_NOALLOC_SCRATCH_BYTES) from the moment the library's code is
// loaded on it until the process ends.  Host code never passes `scratch` itself to a
// kernel (its name is a host-side stand-in, not a device address): the device address is
// looked up once per device with hipGetSymbolAddress and kept in scratch_dev[].
// Every scan block writes all k slots of its lists before merge_kernel reads them, so
// nothing in the array has to start at zero; calls that overlap on one GPU race on it.
static __device__ __align__(256) unsigned char scratch[TQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxScratchDevices];

// Device address of `scratch` on the stream's device, which must be the current one (the
// symbol lookup answers for the current device).
int scratch_address(hipStream_t st, void** out) {
  int cur = 0;
  TQ_HIP_TRY(hipGetDevice(&cur));
  hipDevice_t sdev = cur;
  if (st != nullptr) TQ_HIP_TRY(hipStreamGetDevice(st, &sdev));
  if ((int)sdev != cur)
    return fail(TQ_EINVAL, "the stream belongs to device %d, but device %d is current",
                (int)sdev, cur);
  if (cur < 0 || cur >= kMaxScratchDevices)
    return fail(TQ_EUNSUPPORTED, "device ordinal %d above %d", cur, kMaxScratchDevices - 1);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[cur] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(TQ_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", cur,
                  hipGetErrorString(e));
    scratch_dev[cur] = p;
  }
  *out = scratch_dev[cur];
  return TQ_OK;
}

}  // namespace

extern "C" {

int tq_ip_scan_topk_pairs_noalloc(const void* queries, tq_dtype q_dtype, int64_t nq, int32_t d,
                                  const uint8_t* pairs, const float* norms, int64_t N,
                                  const float* centroids, const float* rotation, int32_t k,
                                  float* out_scores, int64_t* out_ids, void* stream) {
  TQ_REQUIRE(d == 64 || d == 128, "pair-layout scan needs dim 64 or 128, got %d", d);
  TQ_REQUIRE(k >= 1 && k <= kMaxK, "k must be in [1, %d], got %d", kMaxK, k);
  TQ_REQUIRE(nq >= 0 && N >= 0, "bad sizes");
  const size_t need = tq_scan_workspace_bytes(nq, d, 4, N, k);
  TQ_REQUIRE(need <= (size_t)TQ_NOALLOC_SCRATCH_BYTES,
             "%lld queries x k=%d over %lld rows need %zu bytes of scratch, above the static "
             "%u bytes; use tq_ip_scan_topk_pairs with a workspace",
             (long long)nq, k, (long long)N, need, (unsigned)TQ_NOALLOC_SCRATCH_BYTES);
  if (nq == 0) return TQ_OK;
  void* ws = nullptr;
  const int rc = scratch_address(as_stream(stream), &ws);
  if (rc != TQ_OK) return rc;
  return tq_ip_scan_topk_pairs(queries, q_dtype, nq, d, pairs, norms, N, centroids, rotation, k,
                               out_scores, out_ids, ws, TQ_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
