// tq_common.h -- shared host/device helpers for the gfx950 TurboQuant kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/turboquant_hip.h"

namespace tq {

// ---------------------------------------------------------------- errors
// One message per host thread; entry points return a code and leave the text here.
std::string& last_error();

int fail(int code, const char* fmt, ...);

#define TQ_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::tq::fail(TQ_EINVAL, __VA_ARGS__);     \
  } while (0)

#define TQ_HIP_TRY(expr)                                                          \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess)                                                         \
      return ::tq::fail(TQ_EHIP, "%s: %s", #expr, hipGetErrorString(e_));         \
  } while (0)

// Checks the launch that was just issued on this thread.
#define TQ_LAUNCH_CHECK(name)                                                     \
  do {                                                                            \
    hipError_t e_ = hipGetLastError();                                            \
    if (e_ != hipSuccess)                                                         \
      return ::tq::fail(TQ_EHIP, "launch of %s failed: %s", name,                 \
                        hipGetErrorString(e_));                                   \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device).
int device_cu_count();

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------- buffer loads
// Raw buffer resource over [p, p + bytes): loads through it take 32-bit byte offsets and
// return zeros for any access that reaches past `bytes` (the hardware range check), so
// tails need no clamp.  Cache-policy argument of the raw loads: 0 = default, kNT =
// non-temporal (only for accesses that cover whole cache lines per instruction).
constexpr int kNT = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

// ---------------------------------------------------------------- dtype helpers
// Round an fp32 value to the nearest bf16 / fp16 value (ties to even) and return it
// widened back to fp32.  This is how the reference's torch ops round every
// intermediate when the input tensor is bf16 or fp16.
__device__ __forceinline__ float round_bf16(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7f800000u) == 0x7f800000u) {              // inf / nan: keep, quiet nan
    return (u & 0x007fffffu) ? __uint_as_float(u | 0x00400000u) : v;
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

__device__ __forceinline__ float round_f16(float v) {
  return __half2float(__float2half_rn(v));
}

__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == TQ_BF16) return round_bf16(v);
  if (dt == TQ_F16) return round_f16(v);
  return v;
}

__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == TQ_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == TQ_BF16) {
    uint32_t h = reinterpret_cast<const uint16_t*>(p)[i];
    return __uint_as_float(h << 16);
  }
  return __half2float(reinterpret_cast<const __half*>(p)[i]);
}

// Store an fp32 value that already holds a representable value of `dt`.
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v, int dt) {
  if (dt == TQ_F32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else if (dt == TQ_BF16) {
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)(__float_as_uint(round_bf16(v)) >> 16);
  } else {
    reinterpret_cast<__half*>(p)[i] = __float2half_rn(v);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// fp16 hi + lo parts of x (hi + lo = x to about 2^-22).  x is pinned as an fp32 value
// first: when x is a product, the compiler may otherwise fold the multiply into each
// conversion separately (one part rounded once from the exact product, the other via its
// fp32 rounding), and in the rare case where the two roundings differ the parts describe
// numbers one fp16 ulp apart.
__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
  asm("" : "+v"(x));
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// ---------------------------------------------------------------- value-norm scale
// The attention kernels hand the weights p |v| (p <= 1: softmax weights against the
// running maximum) to the matrix cores as fp16, whose range (2^-24 .. 65504) is far
// narrower than the norms' fp32.  A wave keeps a power of two S = 2^e such that every
// |v| S it has seen is at most 2^14, so the weights stay finite for any finite norm and
// keep fp16's full precision for small ones.  Decode: a tile that breaks the bound lowers
// e (the accumulators are rescaled by 2^(e' - e), exactly); prefill: e comes from the
// wave's first tile (fit) and a wave that overflows runs again with the scale of all its
// tiles.  The wave's result is multiplied by 2^-e at the end.  Scaling by a power of two
// commutes with rounding, so weights that were normal fp16 numbers without it give the
// same bits with it.  Wave-uniform.
struct VnScale {
  static constexpr float kBound = 16384.f;  // |v| S at most 2^14
  int e = 126;  // the first tile with a norm above 2^-112 sets it
  float s = 0x1p126f;
  // vsmax: this lane's largest |v| S over the tile's live tokens (0 for none)
  __device__ __forceinline__ bool over(float vsmax) const { return __any(vsmax > kBound); }
  // Lowers e so that the wave's largest |v| lands in [2^13, 2^14); returns the factor for
  // the accumulators.  vmax: this lane's largest |v| over the tile's live tokens.
  __device__ __forceinline__ float rescale(float vmax) {
    const float wm = wave_max(vmax);
    const int en = __builtin_amdgcn_readfirstlane(14 - __builtin_amdgcn_frexp_expf(wm));
    const float f = __builtin_amdgcn_ldexpf(1.f, en - e);
    e = en;
    s = __builtin_amdgcn_ldexpf(1.f, en);
    return f;
  }
  __device__ __forceinline__ float inv() const { return __builtin_amdgcn_ldexpf(1.f, -e); }
  // Sets e so that the wave's largest |v| (vmax on every lane) lands in
  // [2^(top-1), 2^top) (e at most 126: a wave of zero norms keeps 2^top).
  __device__ __forceinline__ void fit(float vmax, int top) {
    const float wm = wave_max(vmax);
    e = min(126, __builtin_amdgcn_readfirstlane(top - __builtin_amdgcn_frexp_expf(wm)));
    s = __builtin_amdgcn_ldexpf(1.f, e);
  }
};

// #{ bnd[i] < y } for sorted bnd of length 2^bits - 1 (torch.searchsorted, right=False).
__device__ __forceinline__ int count_below(const float* bnd, int nlev, float y) {
  int lo = 0;
  for (int step = nlev >> 1; step >= 1; step >>= 1) {
    if (y > bnd[lo + step - 1]) lo += step;
  }
  return lo;
}

// ---------------------------------------------------------------- MFMA operand fence
// Explicit wait states between VALU fp32 -> fp16 conversions and the MFMAs that read
// their results as an A/B operand.  On gfx950 an MFMA issued directly after the
// v_cvt_pk_f16_f32 that wrote its operand has read stale registers.  The asm below
// redefines the operand registers, so every MFMA that reads them is ordered after it
// whatever the scheduler does, and its two s_nop 7 put 16 wait states between the last
// conversion that wrote them and that MFMA.  (A copy the register allocator might insert
// after it is a plain move, whose VALU -> MFMA hazard the compiler tracks itself.)  The asm
// is not volatile: it has no side effects, so memory operations (the table lookups) may
// still be scheduled across it; its outputs are used, so it is never dropped.
template <typename A>
__device__ __forceinline__ void mfma_operand_fence(A& a) {
  asm("s_nop 7\n\ts_nop 7" : "+v"(a));
}
template <typename A, typename B>
__device__ __forceinline__ void mfma_operand_fence(A& a, B& b) {
  asm("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b));
}
template <typename A, typename B, typename C, typename D>
__device__ __forceinline__ void mfma_operand_fence(A& a, B& b, C& c, D& d) {
  asm("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
template <typename A>
__device__ __forceinline__ void mfma_operand_fence6(A& a, A& b, A& c, A& d, A& e, A& f) {
  asm("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f));
}
template <typename A>
__device__ __forceinline__ void mfma_operand_fence8(A& a, A& b, A& c, A& d, A& e, A& f, A& g,
                                                    A& h) {
  asm("s_nop 7\n\ts_nop 7"
               : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h));
}

inline bool valid_dtype(int dt) { return dt == TQ_F32 || dt == TQ_F16 || dt == TQ_BF16; }
inline size_t dtype_size(int dt) { return dt == TQ_F32 ? 4 : 2; }

}  // namespace tq
