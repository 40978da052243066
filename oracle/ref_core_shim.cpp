// ref_core_shim.cpp -- extern "C" entry points over the reference's standalone C++
// core (csrc/core/turboquant_core.cpp), compiled from its sources where they lie in
// the reference checkout.  TEST INFRASTRUCTURE ONLY (bench.py cpu_baseline with
// kind "reference", and a checker in tests/).  Output: oracle/_ref/libtqcore_ref.so.
#include <cstdint>
#include <vector>

#include "turboquant_core.h"

extern "C" {

// turboquant::search_packed (turboquant_core.h / turboquant_core.cpp:407-514).
void ref_search_packed(const float* queries, int Q, const uint8_t* packed, const float* norms,
                       int N, int dim, int bits, const float* rotation,
                       const float* scaled_centroids, int k, float* out_scores,
                       int64_t* out_ids) {
  turboquant::search_packed(queries, Q, packed, norms, N, dim, bits, rotation, scaled_centroids,
                            k, out_scores, out_ids);
}

// turboquant::pack_codes / unpack_codes (turboquant_core.cpp:223-271).
void ref_pack_codes(const uint8_t* codes, int N, int dim, int bits, uint8_t* packed) {
  turboquant::pack_codes(codes, N, dim, bits, packed);
}

void ref_unpack_codes(const uint8_t* packed, int N, int dim, int bits, uint8_t* codes) {
  turboquant::unpack_codes(packed, N, dim, bits, codes);
}

}  // extern "C"

// Rotation, codebook and index persistence of the core (turboquant_core.cpp:71-213,
// 519-618), for the TQIX fixtures of tests/golden/make_tqix_golden.py.
#include <cstring>
#include <memory>
#include <stdexcept>

extern "C" {

void ref_make_rotation(int dim, int seed, float* out) {
  const std::vector<float> R = turboquant::make_rotation_matrix(dim, seed);
  std::memcpy(out, R.data(), sizeof(float) * R.size());
}

void ref_codebook(int bits, int dim, float* boundaries, float* centroids) {
  const turboquant::Codebook cb(bits, dim);
  std::memcpy(boundaries, cb.scaled_boundaries.data(), sizeof(float) * cb.scaled_boundaries.size());
  std::memcpy(centroids, cb.scaled_centroids.data(), sizeof(float) * cb.scaled_centroids.size());
}

int ref_index_build_save(int dim, int bits, int seed, const float* vectors, int N, const char* path) {
  try {
    turboquant::TurboQuantIndex idx(dim, bits, seed);
    idx.add(vectors, N);
    idx.save(path);
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

int ref_index_load_search(const char* path, const float* queries, int Q, int k, float* out_scores,
                          int64_t* out_ids) {
  try {
    auto idx = turboquant::TurboQuantIndex::load(path);
    idx->search(queries, Q, k, out_scores, out_ids);
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

}  // extern "C"
