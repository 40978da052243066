// ref_quant_cpu_shim.cpp -- extern "C" entry points over the reference's CPU kernels
// (csrc/cpu/quant_cpu.cpp), compiled from that source where it lies in the reference
// checkout, against the installed torch.  TEST INFRASTRUCTURE ONLY (a checker in tests/
// and bench.py's config-0 CPU leg with kind "reference").  Output:
// oracle/_ref/libquant_cpu_ref.so.  Inputs are wrapped without copies (torch::from_blob);
// each entry point returns 0, or 1 after printing the reference's error.
#include <torch/torch.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <tuple>

// The reference's CPU kernels (quant_cpu.cpp:44, 125, 199), as its registration binds them.
std::tuple<torch::Tensor, torch::Tensor> rotate_and_quantize_cpu(torch::Tensor vectors,
                                                                 torch::Tensor rotation,
                                                                 torch::Tensor boundaries,
                                                                 int64_t bit_width);
torch::Tensor attention_scores_packed_cpu(torch::Tensor query, torch::Tensor packed_keys,
                                          torch::Tensor key_norms, torch::Tensor centroids,
                                          torch::Tensor rotation, int64_t bit_width);
torch::Tensor attention_values_packed_cpu(torch::Tensor attn_weights, torch::Tensor packed_values,
                                          torch::Tensor value_norms, torch::Tensor centroids,
                                          torch::Tensor rotation_T, int64_t bit_width);

namespace {

torch::Tensor wrap_f32(const float* p, at::IntArrayRef shape) {
  return torch::from_blob(const_cast<float*>(p), shape, torch::TensorOptions().dtype(torch::kFloat32));
}

torch::Tensor wrap_u8(const uint8_t* p, at::IntArrayRef shape) {
  return torch::from_blob(const_cast<uint8_t*>(p), shape, torch::TensorOptions().dtype(torch::kUInt8));
}

int packed_width(int d, int bits) { return bits * ((d + 7) / 8); }

}  // namespace

extern "C" {

// rotate_and_quantize_cpu: x [n][d], R [d][d], bnd [2^bits - 1] -> packed [n][bits *
// ceil(d / 8)], norms [n].
int ref_cpu_rotate_and_quantize(const float* x, int64_t n, int d, const float* R, const float* bnd,
                                int bits, uint8_t* packed, float* norms) {
  try {
    auto out = rotate_and_quantize_cpu(wrap_f32(x, {n, d}), wrap_f32(R, {d, d}),
                                       wrap_f32(bnd, {(1 << bits) - 1}), bits);
    auto p = std::get<0>(out).contiguous();
    auto nm = std::get<1>(out).to(torch::kFloat32).contiguous();
    std::memcpy(packed, p.data_ptr<uint8_t>(), (size_t)n * packed_width(d, bits));
    std::memcpy(norms, nm.data_ptr<float>(), (size_t)n * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_cpu_rotate_and_quantize: %s\n", e.what());
    return 1;
  }
}

// attention_scores_packed_cpu: q [batch][heads][d], keys [T][bits * ceil(d / 8)] ->
// scores [batch][heads][T].
int ref_cpu_attention_scores(const float* q, int batch, int heads, int d, const uint8_t* keys,
                             const float* key_norms, int64_t T, const float* cen, const float* R,
                             int bits, float* scores) {
  try {
    auto s = attention_scores_packed_cpu(wrap_f32(q, {batch, heads, d}),
                                         wrap_u8(keys, {T, packed_width(d, bits)}),
                                         wrap_f32(key_norms, {T}), wrap_f32(cen, {1 << bits}),
                                         wrap_f32(R, {d, d}), bits)
                 .contiguous();
    std::memcpy(scores, s.data_ptr<float>(), (size_t)batch * heads * T * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_cpu_attention_scores: %s\n", e.what());
    return 1;
  }
}

// attention_values_packed_cpu: w [batch][heads][T], values [T][bits * ceil(d / 8)],
// R_T [d][d] -> out [batch][heads][d].
int ref_cpu_attention_values(const float* w, int batch, int heads, int64_t T, const uint8_t* values,
                             const float* value_norms, int d, const float* cen, const float* R_T,
                             int bits, float* out) {
  try {
    auto o = attention_values_packed_cpu(wrap_f32(w, {batch, heads, T}),
                                         wrap_u8(values, {T, packed_width(d, bits)}),
                                         wrap_f32(value_norms, {T}), wrap_f32(cen, {1 << bits}),
                                         wrap_f32(R_T, {d, d}), bits)
                 .contiguous();
    std::memcpy(out, o.data_ptr<float>(), (size_t)batch * heads * d * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_cpu_attention_values: %s\n", e.what());
    return 1;
  }
}

}  // extern "C"
