// ref_core_shim.cpp -- extern "C" entry points over the reference's standalone C++
// core (csrc/core/turboquant_core.cpp), compiled from its sources where they lie in
// the reference checkout.  TEST INFRASTRUCTURE ONLY (bench.py cpu_baseline with
// kind "reference", and a checker in tests/).  Output: oracle/_ref/libtqcore_ref.so.
#include <cstdint>

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
