// tq_quantize.hip -- quantize-on-write kernels for gfx950.
//
//   rotate_and_quantize : n = ||x||, u = x/max(n,1e-10), y = u R^T, code = #{bnd < y}, pack
//                         (reference.py:263-317; registration.cpp:86-88)
//   quantize_prod       : MSE at b-1 bits + 1-bit QJL sign residual (reference.py:392-469)
//   pack / unpack       : bit-plane layout (reference.py:191-255)
//   dequantize_mse/prod : c[codes] R * n (+ QJL correction) (reference.py:320-367, 472-533)
//
// Work decomposition.  A 256-thread workgroup owns a tile of ROWS=16 rows at a
// time (grid-stride over tiles).  The tile's rows are staged in LDS as fp32, the
// per-row reductions (norms, residual norms) are one wave per 4 rows, and every
// d x d contraction is an item loop: item = (output column j, group of 8 rows);
// the thread keeps 8 fp32 accumulators, streams row j of the matrix from L1/L2
// in float4 pieces and reads the 8 staged rows as LDS broadcasts, summing k in
// increasing order.  Codes land in an LDS byte tile and are packed to bit planes
// by one thread per output byte, so the packed rows leave as contiguous stores.
//
// Rounding.  `rdt` is the element type every intermediate is rounded to; the
// reference computes in the input tensor's dtype (bf16 inputs give bf16 norms,
// bf16 unit vectors, a bf16 GEMM output and bf16 boundaries).  With rdt=F32 all
// rounding helpers are the identity.

#include "tq_common.h"

namespace tq {

std::string& last_error() {
  static thread_local std::string msg;
  return msg;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

namespace {

constexpr int kRows = 16;       // rows per tile
constexpr int kThreads = 256;   // 4 waves
constexpr int kRowsPerItem = 8; // accumulators per contraction item
constexpr int kMaxD = 256;
constexpr int kDPad = kMaxD + 4;  // LDS row stride (floats); keeps rows 16-byte aligned

struct QuantArgs {
  const void* x;
  int in_dt;
  int rdt;
  int64_t n;
  int d;
  const float* rot;     // [d, d]
  const float* bnd;     // [2^bits - 1]
  const float* cen;     // [2^bits] (prod only)
  const float* qjl;     // [d, d]   (prod only)
  int bits;             // bits of the MSE codes written
  uint8_t* packed;      // [n, bits*bpp]
  uint8_t* signs;       // [n, bpp] (prod only)
  float* res_norms;     // [n]     (prod only)
  float* norms;         // [n]
};

// acc[i] = sum_k A[row0+i][k] * M[col][k] for i < 8, k ascending.  A rows in LDS
// (stride kDPad), M row-major in global memory.  `rdt` rounds M's elements.
__device__ __forceinline__ void contract_rows(const float (*A)[kDPad], int row0,
                                              const float* __restrict__ M, int col, int d,
                                              int rdt, float acc[kRowsPerItem]) {
#pragma unroll
  for (int i = 0; i < kRowsPerItem; ++i) acc[i] = 0.f;
  const float* mrow = M + (size_t)col * d;
  if ((d & 3) == 0) {
    for (int k = 0; k < d; k += 4) {
      float4 m4 = *reinterpret_cast<const float4*>(mrow + k);
      if (rdt != TQ_F32) {
        m4.x = round_to(m4.x, rdt); m4.y = round_to(m4.y, rdt);
        m4.z = round_to(m4.z, rdt); m4.w = round_to(m4.w, rdt);
      }
#pragma unroll
      for (int i = 0; i < kRowsPerItem; ++i) {
        const float4 a4 = *reinterpret_cast<const float4*>(&A[row0 + i][k]);
        float s = acc[i];
        s = fmaf(a4.x, m4.x, s);
        s = fmaf(a4.y, m4.y, s);
        s = fmaf(a4.z, m4.z, s);
        s = fmaf(a4.w, m4.w, s);
        acc[i] = s;
      }
    }
  } else {
    for (int k = 0; k < d; ++k) {
      const float m = round_to(mrow[k], rdt);
#pragma unroll
      for (int i = 0; i < kRowsPerItem; ++i) acc[i] = fmaf(A[row0 + i][k], m, acc[i]);
    }
  }
}

// Same contraction with the matrix read down a column: acc[i] = sum_j C[row0+i][j] * M[j][col].
// C holds centroid values already (fp32); j ascending.
__device__ __forceinline__ void contract_cols(const float (*C)[kDPad], int row0,
                                              const float* __restrict__ M, int col, int d,
                                              int rdt, float acc[kRowsPerItem]) {
#pragma unroll
  for (int i = 0; i < kRowsPerItem; ++i) acc[i] = 0.f;
  for (int j = 0; j < d; ++j) {
    const float m = round_to(M[(size_t)j * d + col], rdt);
#pragma unroll
    for (int i = 0; i < kRowsPerItem; ++i) acc[i] = fmaf(C[row0 + i][j], m, acc[i]);
  }
}

// Pack the LDS code tile rows [0, rows) into bit planes and store them.
__device__ __forceinline__ void pack_tile(const uint8_t (*codes)[kDPad], int rows, int64_t row_base,
                                          int d, int bits, uint8_t* __restrict__ out) {
  const int bpp = (d + 7) >> 3;
  const int P = bits * bpp;
  for (int idx = threadIdx.x; idx < rows * P; idx += kThreads) {
    const int r = idx / P;
    const int byte = idx - r * P;
    const int plane = byte / bpp;
    const int kb = byte - plane * bpp;
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = kb * 8 + i;
      if (j < d) v |= ((uint32_t)(codes[r][j] >> plane) & 1u) << (7 - i);
    }
    out[(row_base + r) * (int64_t)P + byte] = (uint8_t)v;
  }
}

// Row norms of the staged tile: wave w reduces rows 4w..4w+3.  Returns nothing;
// writes nrm[r] = round(sqrt(sum x^2)).
__device__ __forceinline__ void tile_norms(const float (*X)[kDPad], int d, int rdt, float* nrm) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int rr = 0; rr < kRows / 4; ++rr) {
    const int r = wave * (kRows / 4) + rr;
    float s = 0.f;
    for (int c = lane; c < d; c += 64) s = fmaf(X[r][c], X[r][c], s);
    s = wave_sum(s);
    if (lane == 0) nrm[r] = round_to(sqrtf(s), rdt);
  }
}

template <bool kProd>
__global__ __launch_bounds__(kThreads) void quantize_kernel(QuantArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kRows][kDPad];   // x, then unit u
  __shared__ __attribute__((aligned(16))) float us[kRows][kDPad];   // u / ||u||, then residual
  __shared__ uint8_t cs[kRows][kDPad];                              // codes
  __shared__ float bnd_s[32];
  __shared__ float cen_s[32];
  __shared__ float nrm_s[kRows];
  __shared__ float nrm2_s[kRows];

  const int d = a.d;
  const int rdt = a.rdt;
  const int nlev = 1 << a.bits;
  if (threadIdx.x < nlev - 1) bnd_s[threadIdx.x] = round_to(a.bnd[threadIdx.x], rdt);
  if (kProd && threadIdx.x < nlev) cen_s[threadIdx.x] = round_to(a.cen[threadIdx.x], rdt);
  const float eps = round_to(1e-10f, rdt);
  const int64_t ntiles = (a.n + kRows - 1) / kRows;
  const int items = d * (kRows / kRowsPerItem);

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r0 = tile * kRows;
    const int rows = (int)min<int64_t>(kRows, a.n - r0);
    __syncthreads();  // previous tile fully consumed
    for (int idx = threadIdx.x; idx < kRows * d; idx += kThreads) {
      const int r = idx / d, c = idx - r * d;
      xs[r][c] = (r < rows) ? load_as_f32(a.x, (r0 + r) * (int64_t)d + c, a.in_dt) : 0.f;
    }
    __syncthreads();
    tile_norms(xs, d, rdt, nrm_s);
    __syncthreads();
    // unit = x / max(n, eps)
    for (int idx = threadIdx.x; idx < kRows * d; idx += kThreads) {
      const int r = idx / d, c = idx - r * d;
      const float den = fmaxf(nrm_s[r], eps);
      xs[r][c] = round_to(xs[r][c] / den, rdt);
    }
    if (threadIdx.x < rows) a.norms[r0 + threadIdx.x] = nrm_s[threadIdx.x];
    __syncthreads();
    if (kProd) {
      // quantize_mse normalizes its (already unit) input again.
      tile_norms(xs, d, rdt, nrm2_s);
      __syncthreads();
      for (int idx = threadIdx.x; idx < kRows * d; idx += kThreads) {
        const int r = idx / d, c = idx - r * d;
        us[r][c] = round_to(xs[r][c] / fmaxf(nrm2_s[r], eps), rdt);
      }
      __syncthreads();
    }
    const float (*U)[kDPad] = kProd ? us : xs;
    // y = u R^T and codes.
    for (int it = threadIdx.x; it < items; it += kThreads) {
      const int g = it / d, j = it - g * d;
      float acc[kRowsPerItem];
      contract_rows(U, g * kRowsPerItem, a.rot, j, d, rdt, acc);
#pragma unroll
      for (int i = 0; i < kRowsPerItem; ++i) {
        const float y = round_to(acc[i], rdt);
        cs[g * kRowsPerItem + i][j] = (uint8_t)count_below(bnd_s, nlev, y);
      }
    }
    __syncthreads();
    pack_tile(cs, rows, r0, d, a.bits, a.packed);
    if (kProd) {
      // us <- centroid values of the codes (reads cs, writes us: u/||u|| is dead now)
      for (int idx = threadIdx.x; idx < kRows * d; idx += kThreads) {
        const int r = idx / d, c = idx - r * d;
        us[r][c] = cen_s[cs[r][c]];
      }
      __syncthreads();
      // residual = u - round(c[codes] R); kept in registers until all reads of us end.
      // items <= 2 * kMaxD = 2 * kThreads, so each thread owns at most two items.
      float resv[2][kRowsPerItem];
#pragma unroll
      for (int rep = 0; rep < 2; ++rep) {
        const int it = threadIdx.x + rep * kThreads;
        if (it < items) {
          const int g = it / d, k = it - g * d;
          float acc[kRowsPerItem];
          contract_cols(us, g * kRowsPerItem, a.rot, k, d, rdt, acc);
#pragma unroll
          for (int i = 0; i < kRowsPerItem; ++i)
            resv[rep][i] = round_to(xs[g * kRowsPerItem + i][k] - round_to(acc[i], rdt), rdt);
        }
      }
      __syncthreads();
#pragma unroll
      for (int rep = 0; rep < 2; ++rep) {
        const int it = threadIdx.x + rep * kThreads;
        if (it < items) {
          const int g = it / d, k = it - g * d;
#pragma unroll
          for (int i = 0; i < kRowsPerItem; ++i) us[g * kRowsPerItem + i][k] = resv[rep][i];
        }
      }
      __syncthreads();
      tile_norms(us, d, rdt, nrm2_s);
      // signs of residual S^T
      for (int it = threadIdx.x; it < items; it += kThreads) {
        const int g = it / d, j = it - g * d;
        float acc[kRowsPerItem];
        contract_rows(us, g * kRowsPerItem, a.qjl, j, d, rdt, acc);
#pragma unroll
        for (int i = 0; i < kRowsPerItem; ++i)
          cs[g * kRowsPerItem + i][j] = (round_to(acc[i], rdt) >= 0.f) ? 1 : 0;
      }
      __syncthreads();
      if (threadIdx.x < rows) a.res_norms[r0 + threadIdx.x] = nrm2_s[threadIdx.x];
      pack_tile(cs, rows, r0, d, 1, a.signs);
    }
  }
}

// ---------------------------------------------------------------- MFMA quantize (fp32, d 64/128)
// The same arithmetic as quantize_kernel for fp32 inputs, with every d x d contraction on
// v_mfma_f32_16x16x4f32 (exact fp32 products, fp32 sums; the summation order differs
// from the reference's like any GEMM's, which the decision band of the codes allows).
// A workgroup of d / 16 waves stays on its CU and takes 64-row tiles in turn.
//  * GEMMs: wave w computes output columns [16 w, 16 w + 16) of all 64 rows, so the matrix
//    operand of each of its contractions -- rows 16 w.. of R (u R^T), columns 16 w.. of R
//    (c[codes] R), rows 16 w.. of S (r S^T) -- is fixed: it is held in registers for the
//    whole kernel and only the tile operand comes from LDS, one read per four MFMAs.  A
//    k-step takes the four k = s, s+16, s+32, s+48 of a 64-wide block: with the tiles at a
//    row stride of d + 1 (= 1 mod 64 words) those reads hit 64 distinct banks.
//  * Row work (norms, normalization, bit-plane packing): thread t owns 16 consecutive dims
//    of row t / (d/16), from registers; a row's partial sums meet over d/16 adjacent lanes.
//    x / n is formed as q0 = x y, q = q0 + (x - q0 n) y with y the reciprocal of n refined
//    by one Newton step: the correctly rounded quotient (checked against IEEE division on
//    8e7 random pairs) at 3 operations per element instead of a full division each.
// The next tile's rows are loaded into registers while the current one is processed.
//
// Wider rows (RELOAD: d up to 256, padded to D = a multiple of 16) do not fit three
// register-resident operands: each wave reloads the operand of every contraction from
// global memory (L2: R and S stay cached) just before it, one matrix at a time.  A
// 64-row tile is tens of microseconds of MFMA work per CU, against a few kilobytes of
// operand per wave.  Dims d..D-1 are zero in the tile and in the operands, so the
// padded columns add nothing to any sum; their codes and signs are not stored.
constexpr int kQmRows = 64;
template <int D> constexpr int qm_threads() { return 64 * (D / 16); }

// 1/b correctly rounded (b normal): hardware reciprocal plus one Newton step
__device__ __forceinline__ float qm_recip(float b) {
  const float y0 = __builtin_amdgcn_rcpf(b);
  return fmaf(fmaf(-b, y0, 1.f), y0, y0);
}
// a / b from y = qm_recip(b)
__device__ __forceinline__ float qm_div(float a, float b, float y) {
  const float q0 = a * y;
  return fmaf(fmaf(-q0, b, a), y, q0);
}
// Plane p of 16 codes (bytes of w[0..3], dim order) as two bit-plane bytes, dim 8i+j at
// bit 7-j: four codes' bits gather into a nibble with one multiply.
__device__ __forceinline__ uint32_t qm_plane16(const uint32_t (&w)[4], int p) {
  uint32_t nib[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) nib[i] = ((((w[i] >> p) & 0x01010101u) * 0x08040201u) >> 24) & 0xFu;
  return (nib[0] << 4 | nib[1]) | (nib[2] << 4 | nib[3]) << 8;
}

template <bool kProd, int D, int NB, bool RELOAD = false>
__global__ __launch_bounds__(qm_threads<D>()) void quantize_mfma_kernel(QuantArgs a) {
#pragma clang fp contract(off)
  constexpr int kQmThreads = qm_threads<D>();
  constexpr int TPR = kQmThreads / kQmRows;      // threads per row (16 dims each)
  constexpr int LD = D + 1;                      // LDS row stride in floats
  constexpr int KS = D / 4;                      // k-steps per contraction
  constexpr int RB = kQmRows / 16;               // 16-row blocks per tile
  constexpr int BPP = D / 8;  // RELOAD: the row's bytes per plane are (d + 7) / 8
  static_assert(TPR * 16 == D, "16 dims per thread");
  const int d = RELOAD ? a.d : D;  // real dim (RELOAD: d % 4 == 0, d <= D)
  typedef float v4f_t __attribute__((ext_vector_type(4)));
  __shared__ float ta[kQmRows * LD];             // u -> residual
  __shared__ float tb[kProd ? kQmRows * LD : 1]; // u / ||u|| -> centroid values
  __shared__ __attribute__((aligned(16))) uint8_t cs[kQmRows * D];  // codes, then signs
  __shared__ float cen_s[16];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int col = wave * 16 + c16;         // this lane's GEMM output column
  const int trow = tid / TPR, part = tid % TPR;  // row work: row, dims 16 part..
  // k index of lane group g at k-step t: the four k = s, s+16, s+32, s+48 of a 64-wide
  // block (conflict-free tile reads); a last 16-wide block (D % 64 == 16) takes four
  // consecutive k per step
  constexpr int KF = (D / 64) * 16;  // k-steps in whole 64-wide blocks
  static_assert(D % 64 == 0 || D % 64 == 16, "D: whole 64-wide blocks plus at most 16");
  auto kof = [&](int t) {
    return t < KF ? 64 * (t >> 4) + (t & 15) + 16 * g : 64 * (D / 64) + 4 * (t - KF) + g;
  };
  float bnd_r[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) bnd_r[i] = a.bnd[i];
  if (kProd && tid < 16) cen_s[tid] = tid <= NB ? a.cen[tid] : 0.f;
  // matrix operands: bR[t] = R[col][k_t] (u R^T), bC[t] = R[k_t][col] (c R), bS[t] = S[col][k_t]
  // (RELOAD: one array, refilled before each contraction; zero outside d x d)
  constexpr bool kHold = !RELOAD;
  // RELOAD: each contraction's operand comes in two halves of k-steps (the second loaded
  // after the first half's MFMAs), so a wave holds KS / 2 operand registers: with 13-16
  // waves per workgroup a wave has 128 VGPRs, and a whole operand spilled.  The MFMAs
  // keep their k order, so the sums are unchanged.
  constexpr int KH = RELOAD ? KS / 2 : KS;
  static_assert(!RELOAD || KS % 2 == 0, "two halves of k-steps");
  float bR[KH], bC[kProd && kHold ? KS : 1], bS[kProd && kHold ? KS : 1];
  // (RELOAD: half h of the k-steps, t = h KH .. h KH + KH - 1)
  auto load_op = [&](float (&bm)[KH], const float* __restrict__ M, bool transposed, int h = 0) {
    if constexpr (RELOAD) {
      // Buffer loads of the d x d matrix: an offset past its end reads 0 (the hardware's
      // range check), one inside it but outside row/column d is zeroed by the select.
      // Element (r, c) of M sits at byte 4 (r d + c).  Per load one 32-bit offset: the
      // lane part (its column, its k group g) in a register, the k-step's constant part
      // as the instruction's immediate (M[col][k]) or added to it (M[k][col]).  The
      // column and d pass through an empty asm so the offsets are formed per call, not
      // hoisted out of the tile loop (held across it they would need KS registers each).
      const __amdgpu_buffer_rsrc_t rs = buf_rsrc(M, (uint32_t)(d * d) * 4u);
      int cc = col < d ? col : d - 1, dd = d;
      asm volatile("" : "+v"(cc), "+v"(dd));
#pragma unroll
      for (int i = 0; i < KH; ++i) {
        const int t = h * KH + i, k = kof(t);
        const int kc = t < KF ? 64 * (t >> 4) + (t & 15) : 64 * (D / 64) + 4 * (t - KF);  // k - lane part
        const int kl = t < KF ? 16 * g : g;
        uint32_t v;
        if (transposed) v = __builtin_amdgcn_raw_buffer_load_b32(rs, ((kl + kc) * dd + cc) * 4, 0, 0);
        else v = __builtin_amdgcn_raw_buffer_load_b32(rs, (cc * dd + kl) * 4, kc * 4, 0);
        bm[i] = (col < d && k < d) ? __uint_as_float(v) : 0.f;
      }
    } else {
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        const int k = kof(t);
        bm[t] = transposed ? M[k * D + col] : M[col * D + k];
      }
    }
  };
  if constexpr (kHold) load_op(bR, a.rot, false);
  if constexpr (kProd && kHold) {
    load_op(bC, a.rot, true);
    load_op(bS, a.qjl, false);
  }
  const float eps = 1e-10f;
  const int64_t ntiles = (a.n + kQmRows - 1) / kQmRows;
  const float* xin = static_cast<const float*>(a.x);

  float4 xr[4];  // this thread's 16 dims of its row of the next tile
  auto load_tile = [&](int64_t tile) {
    const int64_t row = tile * kQmRows + trow;
    const float4* src = reinterpret_cast<const float4*>(xin + row * d + 16 * part);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xr[i] = (row < a.n && (!RELOAD || 16 * part + 4 * i < d)) ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  // sum over the row's TPR threads (every thread of the row gets it).  A power-of-two
  // TPR keeps a row inside a wave (butterfly over adjacent lanes); otherwise (d padded to
  // 192 or 208: 12 or 13 threads, rows straddling waves) the partials meet in LDS.  Called
  // by every thread of the workgroup at the same point.
  constexpr bool kPow2Row = (TPR & (TPR - 1)) == 0;
  __shared__ float rsum_s[kPow2Row ? 1 : kQmRows * TPR];
  auto row_sum = [&](float v) {
    if constexpr (kPow2Row) {
#pragma unroll
      for (int o = 1; o < TPR; o <<= 1) v += __shfl_xor(v, o, 64);
      return v;
    } else {
      rsum_s[trow * TPR + part] = v;
      __syncthreads();
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < TPR; ++i) t += rsum_s[trow * TPR + i];
      __syncthreads();
      return t;
    }
  };
  auto row_norm = [&](const float (&v)[16]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = fmaf(v[i], v[i], s);
    return sqrtf(row_sum(s));
  };
  // acc[rb] = rows 16 rb.. of T (LDS tile, the k index along a row) times the register
  // operand b: D[row][col] = sum_k T[row][k] b(k).
  auto gemm = [&](const float* T, const float (&bm)[KS], v4f_t (&acc)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = (v4f_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const int k = kof(t);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(T[(16 * rb + c16) * LD + k], bm[t], acc[rb], 0, 0, 0);
      if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // bounds the tile reads in flight
    }
  };
  // RELOAD: the same product with the operand M (transposed or not) loaded half by half.
  auto gemm_reload = [&](const float* T, const float* __restrict__ M, bool transposed,
                         v4f_t (&acc)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = (v4f_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __builtin_amdgcn_sched_barrier(0);  // the second half's loads wait for the first's MFMAs
      load_op(bR, M, transposed, h);
#pragma unroll
      for (int i = 0; i < KH; ++i) {
        const int t = h * KH + i, k = kof(t);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(T[(16 * rb + c16) * LD + k], bR[i], acc[rb], 0, 0, 0);
        if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // Bit planes of row r0 + trow's codes in cs, stored to `out`.  Whole planes (an output
  // aligned to them): each thread's 16-bit share of every plane goes over the row's own
  // codes in LDS (only the row's threads read those, all from one wave, and each holds
  // its codes in registers by then), and the threads part < bits copy plane `part` out
  // with one 16-byte (D 64: 8-byte) store.  Otherwise 2-byte stores (RELOAD: bytes).
  auto pack_cs = [&](int rows, int64_t r0, int bits, uint8_t* __restrict__ out) {
    const uint4 c = *reinterpret_cast<const uint4*>(&cs[trow * D + 16 * part]);
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    if constexpr (!RELOAD) {
      if ((reinterpret_cast<uintptr_t>(out) & (BPP - 1)) == 0) {
        uint8_t* srow = &cs[trow * D];  // bits * BPP <= D bytes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        for (int p = 0; p < bits; ++p)
          *reinterpret_cast<uint16_t*>(srow + p * BPP + 2 * part) = (uint16_t)qm_plane16(w, p);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (trow < rows && part < bits) {
          uint8_t* dst = out + (r0 + trow) * (int64_t)(bits * BPP) + part * BPP;
          if constexpr (D == 128) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(srow + part * BPP);
          } else {
            *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(srow + part * BPP);
          }
        }
        return;
      }
    }
    if (trow < rows) {
      if constexpr (RELOAD) {  // odd plane widths: byte stores, dims below d only
        const int bpp = (d + 7) >> 3;
        uint8_t* dst = out + (r0 + trow) * (int64_t)(bits * bpp) + 2 * part;
        for (int p = 0; p < bits; ++p) {
          const uint32_t v = qm_plane16(w, p);
          if (2 * part < bpp) dst[p * bpp] = (uint8_t)v;
          if (2 * part + 1 < bpp) dst[p * bpp + 1] = (uint8_t)(v >> 8);
        }
      } else {
        uint8_t* dst = out + (r0 + trow) * (int64_t)(bits * BPP) + 2 * part;
        for (int p = 0; p < bits; ++p)
          *reinterpret_cast<uint16_t*>(dst + p * BPP) = (uint16_t)qm_plane16(w, p);
      }
    }
  };

  // RELOAD: a tile's rows are loaded when it starts (a prefetched tile would stay live
  // through the three contractions; a tile is long enough to absorb one load latency)
  if (!RELOAD && blockIdx.x < ntiles) load_tile(blockIdx.x);
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    if constexpr (RELOAD) load_tile(tile);
    const int64_t r0 = tile * kQmRows;
    const int rows = (int)min<int64_t>(kQmRows, a.n - r0);
    float u[16];
    {
      float x[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) { x[4 * i] = xr[i].x; x[4 * i + 1] = xr[i].y; x[4 * i + 2] = xr[i].z; x[4 * i + 3] = xr[i].w; }
      if (!RELOAD && tile + gridDim.x < ntiles) load_tile(tile + gridDim.x);
      const float n = row_norm(x);
      if (part == 0 && trow < rows) a.norms[r0 + trow] = n;
      const float den = fmaxf(n, eps), y = qm_recip(den);
#pragma unroll
      for (int i = 0; i < 16; ++i) u[i] = qm_div(x[i], den, y);  // u = x / max(n, eps)
    }
    __syncthreads();  // the previous tile is fully consumed
#pragma unroll
    for (int i = 0; i < 16; ++i) ta[trow * LD + 16 * part + i] = u[i];
    if constexpr (kProd) {
      // quantize_mse normalizes its (already unit) input again
      const float den = fmaxf(row_norm(u), eps), y = qm_recip(den);
#pragma unroll
      for (int i = 0; i < 16; ++i) tb[trow * LD + 16 * part + i] = qm_div(u[i], den, y);
    }
    __syncthreads();
    // ---- y = u R^T, codes = #{bnd < y}
    v4f_t acc[RB];
    if constexpr (RELOAD) gemm_reload(kProd ? tb : ta, a.rot, false, acc);
    else gemm(kProd ? tb : ta, bR, acc);
    if (kProd) __syncthreads();  // every wave is done reading tb before it takes c[codes]
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * rb + 4 * g + r;
        const float yv = acc[rb][r];
        int code = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i) code += (bnd_r[i] < yv) ? 1 : 0;
        cs[row * D + col] = (uint8_t)((RELOAD && col >= d) ? 0 : code);  // pad bits stay 0
        if (kProd) tb[row * LD + col] = cen_s[code];
      }
    }
    __syncthreads();
    pack_cs(rows, r0, a.bits, a.packed);
    if constexpr (kProd) {
      // ---- residual = u - c[codes] R (ta, u, is no operand of this product: each lane
      // rewrites its own elements)
      if constexpr (RELOAD) {
        gemm_reload(tb, a.rot, true, acc);
      } else {
        gemm(tb, bC, acc);
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * rb + 4 * g + r;
          ta[row * LD + col] = ta[row * LD + col] - acc[rb][r];
        }
      }
      __syncthreads();  // residual complete; the code pack is done with cs
      {
        float rv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) rv[i] = ta[trow * LD + 16 * part + i];
        const float gam = row_norm(rv);
        if (part == 0 && trow < rows) a.res_norms[r0 + trow] = gam;
      }
      // ---- signs of residual S^T
      if constexpr (RELOAD) {
        gemm_reload(ta, a.qjl, false, acc);
      } else {
        gemm(ta, bS, acc);
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cs[(16 * rb + 4 * g + r) * D + col] = (acc[rb][r] >= 0.f && (!RELOAD || col < d)) ? 1 : 0;
      }
      __syncthreads();
      pack_cs(rows, r0, 1, a.signs);
    }
  }
}

// ---------------------------------------------------------------- pack / unpack
__global__ void pack_kernel(const uint8_t* __restrict__ codes, int64_t n, int d, int bits,
                            uint8_t* __restrict__ packed) {
  const int bpp = (d + 7) >> 3;
  const int P = bits * bpp;
  const int64_t total = n * (int64_t)P;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx / P;
    const int byte = (int)(idx - r * P);
    const int plane = byte / bpp;
    const int kb = byte - plane * bpp;
    const uint8_t* crow = codes + r * d;
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = kb * 8 + i;
      if (j < d) v |= ((uint32_t)(crow[j] >> plane) & 1u) << (7 - i);
    }
    packed[idx] = (uint8_t)v;
  }
}

__global__ void unpack_kernel(const uint8_t* __restrict__ packed, int64_t n, int d, int bits,
                              uint8_t* __restrict__ codes) {
  const int bpp = (d + 7) >> 3;
  const int P = bits * bpp;
  const int64_t total = n * (int64_t)d;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx / d;
    const int j = (int)(idx - r * d);
    const uint8_t* prow = packed + r * P;
    uint32_t c = 0;
    for (int p = 0; p < bits; ++p) c |= ((uint32_t)(prow[p * bpp + (j >> 3)] >> (7 - (j & 7))) & 1u) << p;
    codes[idx] = (uint8_t)c;
  }
}

// ---------------------------------------------------------------- dequantize
struct DequantArgs {
  const uint8_t* packed;
  const uint8_t* signs;     // prod only
  const float* res_norms;   // prod only
  const float* norms;
  int64_t n;
  int d;
  int bits;                 // bits of `packed`
  const float* cen;
  const float* rot;
  const float* qjl;         // prod only
  int out_dt;
  void* out;
};

template <bool kProd>
__global__ __launch_bounds__(kThreads) void dequant_kernel(DequantArgs a) {
  __shared__ __attribute__((aligned(16))) float cv[kRows][kDPad];   // centroid values
  __shared__ __attribute__((aligned(16))) float sv[kRows][kDPad];   // +-1 signs (prod)
  __shared__ float cen_s[32];
  const int d = a.d;
  const int rdt = a.out_dt;
  const int nlev = 1 << a.bits;
  const int bpp = (d + 7) >> 3;
  const int P = a.bits * bpp;
  if (threadIdx.x < nlev) cen_s[threadIdx.x] = round_to(a.cen[threadIdx.x], rdt);
  const int64_t ntiles = (a.n + kRows - 1) / kRows;
  const int items = d * (kRows / kRowsPerItem);
  const float qscale = 1.2533141373155003f / (float)d;  // sqrt(pi/2) / d
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r0 = tile * kRows;
    const int rows = (int)min<int64_t>(kRows, a.n - r0);
    __syncthreads();
    for (int idx = threadIdx.x; idx < kRows * d; idx += kThreads) {
      const int r = idx / d, j = idx - r * d;
      float v = 0.f, s = 0.f;
      if (r < rows) {
        const uint8_t* prow = a.packed + (r0 + r) * (int64_t)P;
        uint32_t c = 0;
        for (int p = 0; p < a.bits; ++p)
          c |= ((uint32_t)(prow[p * bpp + (j >> 3)] >> (7 - (j & 7))) & 1u) << p;
        v = cen_s[c];
        if (kProd) {
          const uint8_t sb = a.signs[(r0 + r) * (int64_t)bpp + (j >> 3)];
          s = ((sb >> (7 - (j & 7))) & 1u) ? 1.f : -1.f;
        }
      }
      cv[r][j] = v;
      if (kProd) sv[r][j] = s;
    }
    __syncthreads();
    for (int it = threadIdx.x; it < items; it += kThreads) {
      const int g = it / d, k = it - g * d;
      float acc[kRowsPerItem];
      contract_cols(cv, g * kRowsPerItem, a.rot, k, d, rdt, acc);
      float corr[kRowsPerItem];
      if (kProd) contract_cols(sv, g * kRowsPerItem, a.qjl, k, d, TQ_F32, corr);
#pragma unroll
      for (int i = 0; i < kRowsPerItem; ++i) {
        const int r = g * kRowsPerItem + i;
        if (r >= rows) continue;
        const int64_t row = r0 + r;
        float v = round_to(acc[i], rdt);
        if (kProd) {
          const float t = qscale * a.res_norms[row];
          v = v + t * corr[i];
        }
        v = round_to(v * a.norms[row], rdt);
        store_from_f32(a.out, row * (int64_t)d + k, v, rdt);
      }
    }
  }
}

// ---------------------------------------------------------------- one row per wave (few rows)
// quantize_kernel<false>'s arithmetic, bit for bit, for bf16/fp16 inputs of d = 64 / 128,
// with one wave per row (lane j owns output dims j and j + 64): a decode step appends one
// token per (sequence, KV head) -- a few hundred rows -- which 16-row tiles would spread
// over a few dozen workgroups, each walking its tile through five barriers.  Here R (its
// elements rounded to the input type, transposed: Rt[k][j]) sits in LDS; per row the norm
// (fmaf over the lane's dims, then the wave sum: tile_norms' order), the unit vector
// (rounded), y_j = sum_k fmaf(u_k, R[j][k]) for k ascending (contract_rows' order), the
// code (count_below) and the bit planes from ballots (dim j at bit 7 - j % 8 of byte j / 8).
constexpr int kQrThreads = 256;
constexpr int64_t kQrMaxRows = 16384;  // above this the tiled kernel is as fast

template <int D>
__global__ __launch_bounds__(kQrThreads) void quantize_rows_kernel(QuantArgs a) {
  constexpr int C = D / 64;  // output dims per lane
  constexpr int BPP = D / 8;
  __shared__ float rt_s[D][D + 1];  // padded: the transposing writes hit distinct banks
  __shared__ float u_s[kQrThreads / 64][D];
  __shared__ float bnd_s[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rdt = a.rdt;
  const int nlev = 1 << a.bits;
  if (threadIdx.x < nlev - 1) bnd_s[threadIdx.x] = round_to(a.bnd[threadIdx.x], rdt);
  for (int e = threadIdx.x; e < D * D; e += kQrThreads) {  // coalesced read of R row j
    const int j = e / D, k = e - j * D;
    rt_s[k][j] = round_to(a.rot[e], rdt);
  }
  __syncthreads();
  const float eps = round_to(1e-10f, rdt);
  const int P = a.bits * BPP;
  for (int64_t row = (int64_t)blockIdx.x * (kQrThreads / 64) + wave; row < a.n;
       row += (int64_t)gridDim.x * (kQrThreads / 64)) {
    float x[C];
#pragma unroll
    for (int c = 0; c < C; ++c) x[c] = load_as_f32(a.x, row * D + lane + 64 * c, a.in_dt);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) ss = fmaf(x[c], x[c], ss);
    ss = wave_sum(ss);
    const float nrm = round_to(sqrtf(ss), rdt);
    if (lane == 0) a.norms[row] = nrm;
    const float den = fmaxf(nrm, eps);
#pragma unroll
    for (int c = 0; c < C; ++c) u_s[wave][lane + 64 * c] = round_to(x[c] / den, rdt);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float acc[C];
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = 0.f;
#pragma unroll 8
    for (int k = 0; k < D; ++k) {
      const float uk = u_s[wave][k];
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] = fmaf(uk, rt_s[k][lane + 64 * c], acc[c]);
    }
    uint32_t code[C];
#pragma unroll
    for (int c = 0; c < C; ++c) code[c] = (uint32_t)count_below(bnd_s, nlev, round_to(acc[c], rdt));
    // lane L < P writes byte L of the row: plane L / BPP, dims 8 (L % BPP) .. + 7
    uint8_t out = 0;
#pragma unroll
    for (int pl = 0; pl < 4; ++pl) {
      if (pl < a.bits) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const uint64_t m = __ballot((code[c] >> pl) & 1u);
          const int b = lane - pl * BPP - 8 * c;  // byte of this plane held in mask c
          if (b >= 0 && b < 8)
            out = (uint8_t)(__builtin_bitreverse32((uint32_t)(m >> (8 * b)) & 0xFFu) >> 24);
        }
      }
    }
    if (lane < P) a.packed[row * P + lane] = out;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // u_s is rewritten by the next row
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

int grid_for_tiles(int64_t n) {
  const int64_t tiles = (n + kRows - 1) / kRows;
  const int64_t cap = (int64_t)device_cu_count() * 6;
  return (int)(tiles < cap ? tiles : cap);
}

// The MFMA quantize kernel covers fp32 inputs kept in fp32, d = 64 or 128, 16-byte
// aligned rows; its workgroups stay on their CUs (at most one per tile).
// Padded width of the operand-reloading MFMA kernel for d, 0 if none applies.
int qm_reload_dim(int d) {
  if (d % 4 != 0 || d <= 128 || d > 256) return 0;
  return d <= 192 ? 192 : d <= 208 ? 208 : 256;
}

bool use_mfma_quantize(const void* x, tq_dtype in_dt, tq_dtype rdt, int d) {
  return in_dt == TQ_F32 && rdt == TQ_F32 && (d == 64 || d == 128 || qm_reload_dim(d) > 0) &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

template <bool kProd, int D>
void launch_qm_reload(const QuantArgs& a, dim3 grid, hipStream_t st) {
  switch (a.bits) {
    case 1: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, D, 1, true>), grid, dim3(qm_threads<D>()), 0, st, a); break;
    case 2: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, D, 3, true>), grid, dim3(qm_threads<D>()), 0, st, a); break;
    case 3: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, D, 7, true>), grid, dim3(qm_threads<D>()), 0, st, a); break;
    default: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, D, 15, true>), grid, dim3(qm_threads<D>()), 0, st, a); break;
  }
}

template <bool kProd>
void launch_quantize_mfma(const QuantArgs& a, hipStream_t st) {
  const int64_t tiles = (a.n + kQmRows - 1) / kQmRows;
  // workgroups per CU that the registers (matrix operands held per wave) allow; the
  // reloading kernel's 12-16 waves and its tiles' LDS take one CU each
  const int rd = qm_reload_dim(a.d);
  const int per_cu = rd ? 1 : a.d == 128 ? (kProd ? 1 : 2) : (kProd ? 2 : 4);
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  const dim3 grid((unsigned)(tiles < cap ? tiles : cap));
  if (rd == 192) {
    launch_qm_reload<kProd, 192>(a, grid, st);
  } else if (rd == 208) {
    launch_qm_reload<kProd, 208>(a, grid, st);
  } else if (rd == 256) {
    launch_qm_reload<kProd, 256>(a, grid, st);
  } else if (a.d == 128) {
    switch (a.bits) {
      case 1: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 128, 1>), grid, dim3(qm_threads<128>()), 0, st, a); break;
      case 2: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 128, 3>), grid, dim3(qm_threads<128>()), 0, st, a); break;
      case 3: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 128, 7>), grid, dim3(qm_threads<128>()), 0, st, a); break;
      default: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 128, 15>), grid, dim3(qm_threads<128>()), 0, st, a); break;
    }
  } else {
    switch (a.bits) {
      case 1: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 64, 1>), grid, dim3(qm_threads<64>()), 0, st, a); break;
      case 2: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 64, 3>), grid, dim3(qm_threads<64>()), 0, st, a); break;
      case 3: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 64, 7>), grid, dim3(qm_threads<64>()), 0, st, a); break;
      default: hipLaunchKernelGGL((quantize_mfma_kernel<kProd, 64, 15>), grid, dim3(qm_threads<64>()), 0, st, a); break;
    }
  }
}

int grid_for_elems(int64_t total, int threads) {
  const int64_t blocks = (total + threads - 1) / threads;
  const int64_t cap = (int64_t)device_cu_count() * 16;
  return (int)(blocks < cap ? blocks : cap);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

const char* tq_last_error(void) { return tq::last_error().c_str(); }

int tq_abi_version(void) { return 4; }

int tq_rotate_and_quantize(const void* vectors, tq_dtype in_dtype, tq_dtype round_dtype, int64_t n,
                           int32_t d, const float* rotation, const float* boundaries,
                           int32_t bit_width, uint8_t* packed, float* norms, void* stream) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4, got %d", bit_width);
  TQ_REQUIRE(d >= 1 && d <= kMaxD, "dim must be in [1, %d], got %d", kMaxD, d);
  TQ_REQUIRE(n >= 0, "n must be >= 0");
  TQ_REQUIRE(valid_dtype(in_dtype) && valid_dtype(round_dtype), "unknown dtype");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(vectors && rotation && boundaries && packed && norms, "null pointer argument");
  QuantArgs a{vectors, in_dtype, round_dtype, n, d, rotation, boundaries, nullptr, nullptr,
              bit_width, packed, nullptr, nullptr, norms};
  if (use_mfma_quantize(vectors, in_dtype, round_dtype, d)) {
    launch_quantize_mfma<false>(a, as_stream(stream));
    TQ_LAUNCH_CHECK("quantize_mfma_kernel<mse>");
    return TQ_OK;
  }
  if ((d == 64 || d == 128) && in_dtype != TQ_F32 && n <= kQrMaxRows) {  // few rows: a wave each
    const int64_t waves_per_cu = d == 64 ? 16 : 8;  // LDS: 16 / 64 KB of R per workgroup
    const int64_t cap = (int64_t)device_cu_count() * waves_per_cu / (kQrThreads / 64);
    const int64_t want = (n + kQrThreads / 64 - 1) / (kQrThreads / 64);
    const dim3 grid((unsigned)(want < cap ? want : cap));
    if (d == 64) hipLaunchKernelGGL(quantize_rows_kernel<64>, grid, dim3(kQrThreads), 0, as_stream(stream), a);
    else hipLaunchKernelGGL(quantize_rows_kernel<128>, grid, dim3(kQrThreads), 0, as_stream(stream), a);
    TQ_LAUNCH_CHECK("quantize_rows_kernel");
    return TQ_OK;
  }
  hipLaunchKernelGGL(quantize_kernel<false>, dim3(grid_for_tiles(n)), dim3(kThreads), 0,
                     as_stream(stream), a);
  TQ_LAUNCH_CHECK("quantize_kernel<mse>");
  return TQ_OK;
}

int tq_quantize_prod(const void* vectors, tq_dtype in_dtype, tq_dtype round_dtype, int64_t n,
                     int32_t d, const float* rotation, const float* boundaries,
                     const float* centroids, const float* qjl, int32_t bit_width,
                     uint8_t* mse_packed, uint8_t* signs, float* res_norms, float* norms,
                     void* stream) {
  TQ_REQUIRE(bit_width >= 2 && bit_width <= 5, "Prod mode requires bits in [2, 5], got %d",
             bit_width);
  TQ_REQUIRE(d >= 1 && d <= kMaxD, "dim must be in [1, %d], got %d", kMaxD, d);
  TQ_REQUIRE(n >= 0, "n must be >= 0");
  TQ_REQUIRE(valid_dtype(in_dtype) && valid_dtype(round_dtype), "unknown dtype");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(vectors && rotation && boundaries && centroids && qjl && mse_packed && signs &&
                 res_norms && norms,
             "null pointer argument");
  QuantArgs a{vectors, in_dtype, round_dtype, n, d, rotation, boundaries, centroids, qjl,
              bit_width - 1, mse_packed, signs, res_norms, norms};
  if (use_mfma_quantize(vectors, in_dtype, round_dtype, d)) {
    launch_quantize_mfma<true>(a, as_stream(stream));
    TQ_LAUNCH_CHECK("quantize_mfma_kernel<prod>");
    return TQ_OK;
  }
  hipLaunchKernelGGL(quantize_kernel<true>, dim3(grid_for_tiles(n)), dim3(kThreads), 0,
                     as_stream(stream), a);
  TQ_LAUNCH_CHECK("quantize_kernel<prod>");
  return TQ_OK;
}

int tq_pack_codes(const uint8_t* codes, int64_t n, int32_t d, int32_t bit_width, uint8_t* packed,
                  void* stream) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 8, "bit_width must be 1-8, got %d", bit_width);
  TQ_REQUIRE(d >= 1 && n >= 0, "bad shape");
  const int64_t total = n * (int64_t)(bit_width * ((d + 7) / 8));
  if (total == 0) return TQ_OK;
  TQ_REQUIRE(codes && packed, "null pointer argument");
  hipLaunchKernelGGL(pack_kernel, dim3(grid_for_elems(total, 256)), dim3(256), 0,
                     as_stream(stream), codes, n, d, bit_width, packed);
  TQ_LAUNCH_CHECK("pack_kernel");
  return TQ_OK;
}

int tq_unpack_codes(const uint8_t* packed, int64_t n, int32_t d, int32_t bit_width, uint8_t* codes,
                    void* stream) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 8, "bit_width must be 1-8, got %d", bit_width);
  TQ_REQUIRE(d >= 1 && n >= 0, "bad shape");
  const int64_t total = n * (int64_t)d;
  if (total == 0) return TQ_OK;
  TQ_REQUIRE(codes && packed, "null pointer argument");
  hipLaunchKernelGGL(unpack_kernel, dim3(grid_for_elems(total, 256)), dim3(256), 0,
                     as_stream(stream), packed, n, d, bit_width, codes);
  TQ_LAUNCH_CHECK("unpack_kernel");
  return TQ_OK;
}

int tq_dequantize_mse(const uint8_t* packed, const float* norms, int64_t n, int32_t d,
                      int32_t bit_width, const float* centroids, const float* rotation,
                      tq_dtype out_dtype, void* out, void* stream) {
  TQ_REQUIRE(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4, got %d", bit_width);
  TQ_REQUIRE(d >= 1 && d <= kMaxD, "dim must be in [1, %d], got %d", kMaxD, d);
  TQ_REQUIRE(valid_dtype(out_dtype), "unknown dtype");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(packed && norms && centroids && rotation && out, "null pointer argument");
  DequantArgs a{packed, nullptr, nullptr, norms, n, d, bit_width, centroids, rotation, nullptr,
                out_dtype, out};
  hipLaunchKernelGGL(dequant_kernel<false>, dim3(grid_for_tiles(n)), dim3(kThreads), 0,
                     as_stream(stream), a);
  TQ_LAUNCH_CHECK("dequant_kernel<mse>");
  return TQ_OK;
}

int tq_dequantize_prod(const uint8_t* mse_packed, const uint8_t* signs, const float* res_norms,
                       const float* norms, int64_t n, int32_t d, int32_t bit_width,
                       const float* centroids, const float* rotation, const float* qjl,
                       tq_dtype out_dtype, void* out, void* stream) {
  TQ_REQUIRE(bit_width >= 2 && bit_width <= 5, "Prod mode requires bits in [2, 5], got %d",
             bit_width);
  TQ_REQUIRE(d >= 1 && d <= kMaxD, "dim must be in [1, %d], got %d", kMaxD, d);
  TQ_REQUIRE(out_dtype == TQ_F32, "dequantize_prod computes in fp32 only");
  if (n == 0) return TQ_OK;
  TQ_REQUIRE(mse_packed && signs && res_norms && norms && centroids && rotation && qjl && out,
             "null pointer argument");
  DequantArgs a{mse_packed, signs, res_norms, norms, n, d, bit_width - 1, centroids, rotation, qjl,
                out_dtype, out};
  hipLaunchKernelGGL(dequant_kernel<true>, dim3(grid_for_tiles(n)), dim3(kThreads), 0,
                     as_stream(stream), a);
  TQ_LAUNCH_CHECK("dequant_kernel<prod>");
  return TQ_OK;
}

}  // extern "C"
