// tq_core_tables.hip -- host-side tables of the reference's standalone C++ core, so that
// indexes stored in its TQIX v1 files (turboquant_core.cpp:559-618) search on the GPU
// with the rotation and codebook the core used to write them.
//
// A TQIX file records only (dim, bit_width, seed); the core rebuilds the rest:
//   rotation  turboquant_core.cpp:137-213: a dim x dim Gaussian matrix drawn row-major from
//             std::mt19937(seed) through std::normal_distribution<float>(0, 1), its columns
//             orthonormalized by modified Gram-Schmidt with two passes per column (dot
//             products accumulated in double, updates rounded to float), each column then
//             flipped so that its diagonal entry is non-negative.
//   codebook  turboquant_core.cpp:71-132: Lloyd-Max on N(0, 1) in double, centroids
//             started at -3 + 6 i / (L - 1), the normal CDF from Abramowitz & Stegun 26.2.17
//             (|error| < 7.5e-8), at most 200 iterations, stop when no centroid moves by
//             1e-12 or more; boundaries = midpoints; both scaled by 1/sqrt(dim) in double
//             and rounded to float.
// The arithmetic follows those steps in the same order (identical matrices and
// codebooks are the point).  std::mt19937 and std::normal_distribution come from the
// C++ standard library both builds use.  No fused multiply-add: the reference's
// compiled core rounds every product and sum.

#include "tq_common.h"

#include <cmath>
#include <limits>
#include <random>
#include <vector>

#pragma clang fp contract(off)

namespace tq {
namespace {

constexpr double kPi = 3.14159265358979323846;

double normal_pdf(double x) { return std::exp(-0.5 * x * x) / std::sqrt(2.0 * kPi); }

// Abramowitz & Stegun 26.2.17: P(x) = 1 - Z(x) (b1 t + b2 t^2 + b3 t^3 + b4 t^4 + b5 t^5),
// t = 1 / (1 + p x) for x >= 0; clamped to 0 / 1 beyond |x| = 8.
double normal_cdf(double x) {
  if (x < -8.0) return 0.0;
  if (x > 8.0) return 1.0;
  const double z = x < 0.0 ? -x : x;
  const double t = 1.0 / (1.0 + 0.2316419 * z);
  const double t2 = t * t, t3 = t2 * t, t4 = t3 * t, t5 = t4 * t;
  const double poly = 0.319381530 * t + -0.356563782 * t2 + 1.781477937 * t3 +
                      -1.821255978 * t4 + 1.330274429 * t5;
  const double upper = 1.0 - normal_pdf(z) * poly;
  return x < 0.0 ? 1.0 - upper : upper;
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int tq_core_rotation(int32_t dim, int32_t seed, float* out) {
  TQ_REQUIRE(dim >= 1 && dim <= 4096, "dim must be in [1, 4096], got %d", dim);
  TQ_REQUIRE(out != nullptr, "null pointer argument");
  const int n = dim;
  std::mt19937 gen(static_cast<uint32_t>(seed));
  std::normal_distribution<float> gauss(0.0f, 1.0f);
  // Column-major working copy: col[c][r] = element (r, c) of the row-major draw.
  std::vector<float> col((size_t)n * n);
  for (int r = 0; r < n; ++r)
    for (int c = 0; c < n; ++c) col[(size_t)c * n + r] = gauss(gen);
  auto dot = [&](int a, int b) {
    const float* x = &col[(size_t)a * n];
    const float* y = &col[(size_t)b * n];
    double acc = 0.0;
    for (int r = 0; r < n; ++r) acc += (double)x[r] * (double)y[r];
    return acc;
  };
  for (int j = 0; j < n; ++j) {
    float* cj = &col[(size_t)j * n];
    for (int pass = 0; pass < 2; ++pass) {
      for (int i = 0; i < j; ++i) {
        const double proj = dot(j, i);
        const float* ci = &col[(size_t)i * n];
        for (int r = 0; r < n; ++r) cj[r] -= (float)(proj * ci[r]);
      }
    }
    const double len = std::sqrt(dot(j, j));
    if (len < 1e-12) return fail(TQ_EINVAL, "rotation: degenerate column %d", j);
    const double inv = 1.0 / len;
    for (int r = 0; r < n; ++r) cj[r] = (float)((double)cj[r] * inv);
  }
  for (int j = 0; j < n; ++j) {
    float* cj = &col[(size_t)j * n];
    if (cj[j] < 0.0f)
      for (int r = 0; r < n; ++r) cj[r] = -cj[r];
  }
  for (int r = 0; r < n; ++r)
    for (int c = 0; c < n; ++c) out[(size_t)r * n + c] = col[(size_t)c * n + r];
  return TQ_OK;
}

int tq_core_codebook(int32_t bits, int32_t dim, float* boundaries, float* centroids) {
  TQ_REQUIRE(bits >= 1 && bits <= 8, "bits must be in [1, 8], got %d", bits);
  TQ_REQUIRE(dim >= 1, "dim must be positive, got %d", dim);
  TQ_REQUIRE(boundaries != nullptr && centroids != nullptr, "null pointer argument");
  const int L = 1 << bits;
  std::vector<double> c(L), nc(L), edge(L + 1);
  for (int i = 0; i < L; ++i) c[i] = -3.0 + 6.0 * i / (L - 1);
  edge[0] = -std::numeric_limits<double>::infinity();
  edge[L] = std::numeric_limits<double>::infinity();
  for (int iter = 0; iter < 200; ++iter) {
    for (int i = 0; i + 1 < L; ++i) edge[i + 1] = (c[i] + c[i + 1]) / 2.0;
    double moved = 0.0;
    for (int i = 0; i < L; ++i) {
      const double mass = normal_cdf(edge[i + 1]) - normal_cdf(edge[i]);
      nc[i] = mass < 1e-15 ? c[i] : (normal_pdf(edge[i]) - normal_pdf(edge[i + 1])) / mass;
      moved = std::max(moved, std::abs(nc[i] - c[i]));
    }
    c.swap(nc);
    if (moved < 1e-12) break;
  }
  const double scale = 1.0 / std::sqrt(static_cast<double>(dim));
  for (int i = 0; i + 1 < L; ++i) boundaries[i] = (float)(((c[i] + c[i + 1]) / 2.0) * scale);
  for (int i = 0; i < L; ++i) centroids[i] = (float)(c[i] * scale);
  return TQ_OK;
}

}  // extern "C"
