// torch_ops.cpp -- registers the `turboquant` operator namespace with the PyTorch
// dispatcher and forwards every op to the C ABI in include/turboquant_hip.h.
//
// It takes the place of csrc/registration.cpp: the five reference schemas
// (registration.cpp:84-99) are kept verbatim, and the fused ops the reference's
// signatures cannot express are added.  Ops are registered for the CUDA dispatch
// key, which is where PyTorch-ROCm files HIP tensors.  There is no CPU
// implementation and no fallback: a CPU tensor raises.
//
// Conventions (registration.cpp, quant_cpu.cpp, rotate_fused.cu): inputs are made
// contiguous (and upcast to fp32 where the reference op does), outputs are freshly
// allocated on the input's device, kernels run asynchronously on the current
// stream under a device guard, errors raise RuntimeError with the kernel's message.

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cmath>

#include "../../include/turboquant_hip.h"

namespace {

void check_rc(int rc) { TORCH_CHECK(rc == TQ_OK, "turboquant: ", tq_last_error()); }

void* cur_stream(const at::Tensor& t) {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

tq_dtype to_tq(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return TQ_F32;
    case at::kHalf: return TQ_F16;
    case at::kBFloat16: return TQ_BF16;
    default: TORCH_CHECK(false, "turboquant: unsupported dtype ", t);
  }
  return TQ_F32;
}

at::ScalarType from_tq(tq_dtype t) {
  return t == TQ_F32 ? at::kFloat : t == TQ_F16 ? at::kHalf : at::kBFloat16;
}

void require_gpu(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), "turboquant: ", name,
              " must be on a HIP device (this build has no CPU kernels)");
}

at::Tensor f32c(const at::Tensor& t, const at::Device& dev) {
  return t.to(dev, at::kFloat).contiguous();
}

// Input of a supported float dtype, contiguous, on `dev`.
at::Tensor floatc(const at::Tensor& t, const at::Device& dev) {
  auto st = t.scalar_type();
  if (st != at::kFloat && st != at::kHalf && st != at::kBFloat16) return t.to(dev, at::kFloat).contiguous();
  return t.to(dev).contiguous();
}

at::Tensor workspace(size_t bytes, const at::Device& dev) {
  return at::empty({(int64_t)(bytes > 0 ? bytes : 1)}, at::TensorOptions().dtype(at::kByte).device(dev));
}

int64_t packed_width(int64_t bits, int64_t d) { return bits * ((d + 7) / 8); }

// ------------------------------------------------------------ reference schemas

std::tuple<at::Tensor, at::Tensor> rotate_and_quantize(const at::Tensor& vectors,
                                                       const at::Tensor& rotation,
                                                       const at::Tensor& boundaries,
                                                       int64_t bit_width) {
  require_gpu(vectors, "vectors");
  TORCH_CHECK(vectors.dim() == 2, "vectors must be [N, d]");
  c10::DeviceGuard g(vectors.device());
  const auto dev = vectors.device();
  auto x = f32c(vectors, dev);  // the reference op upcasts (rotate_fused.cu:148)
  auto R = f32c(rotation, dev);
  auto bnd = f32c(boundaries, dev);
  const int64_t n = x.size(0), d = x.size(1);
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "Rotation matrix must be [d, d]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  TORCH_CHECK(bnd.numel() == (1 << bit_width) - 1, "boundaries length must be 2^bit_width - 1");
  auto packed = at::zeros({n, packed_width(bit_width, d)}, x.options().dtype(at::kByte));
  auto norms = at::empty({n}, x.options());
  check_rc(tq_rotate_and_quantize(x.data_ptr(), TQ_F32, TQ_F32, n, (int32_t)d, R.data_ptr<float>(),
                                  bnd.data_ptr<float>(), (int32_t)bit_width,
                                  packed.data_ptr<uint8_t>(), norms.data_ptr<float>(),
                                  cur_stream(x)));
  return {packed, norms};
}

at::Tensor attention_scores_packed(const at::Tensor& query, const at::Tensor& packed_keys,
                                   const at::Tensor& key_norms, const at::Tensor& centroids,
                                   const at::Tensor& rotation, int64_t bit_width) {
  require_gpu(query, "query");
  TORCH_CHECK(query.dim() == 3, "query must be [batch, heads, head_dim]");
  TORCH_CHECK(packed_keys.dim() == 2, "packed_keys must be [seq_len, packed_dim]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  c10::DeviceGuard g(query.device());
  const auto dev = query.device();
  auto q = f32c(query, dev);
  auto pk = packed_keys.to(dev).contiguous();
  auto kn = f32c(key_norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  const int64_t B = q.size(0), H = q.size(1), d = q.size(2), T = pk.size(0);
  TORCH_CHECK(pk.scalar_type() == at::kByte, "packed_keys must be uint8");
  TORCH_CHECK(pk.size(1) == packed_width(bit_width, d), "packed dim mismatch: expected ",
              packed_width(bit_width, d), " got ", pk.size(1));
  TORCH_CHECK(kn.numel() == T, "key_norms must have seq_len entries");
  TORCH_CHECK(cen.numel() == (1 << bit_width), "centroids length must be 2^bit_width");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto scores = at::empty({B, H, T}, q.options());
  if (B * H == 0 || T == 0) return scores;
  auto ws = workspace(tq_scan_workspace_bytes(B * H, (int32_t)d, (int32_t)bit_width, T, 0), dev);
  check_rc(tq_attention_scores_packed(q.data_ptr(), TQ_F32, B * H, (int32_t)d, pk.data_ptr<uint8_t>(),
                                      kn.data_ptr<float>(), T, cen.data_ptr<float>(),
                                      R.data_ptr<float>(), (int32_t)bit_width,
                                      scores.data_ptr<float>(), ws.data_ptr(), ws.numel(),
                                      cur_stream(q)));
  return scores;
}

at::Tensor attention_values_packed(const at::Tensor& attn_weights, const at::Tensor& packed_values,
                                   const at::Tensor& value_norms, const at::Tensor& centroids,
                                   const at::Tensor& rotation_T, int64_t bit_width) {
  require_gpu(attn_weights, "attn_weights");
  TORCH_CHECK(attn_weights.dim() == 3, "attn_weights must be [batch, heads, seq_len]");
  TORCH_CHECK(packed_values.dim() == 2, "packed_values must be [seq_len, packed_dim]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  c10::DeviceGuard g(attn_weights.device());
  const auto dev = attn_weights.device();
  auto w = f32c(attn_weights, dev);
  auto pv = packed_values.to(dev).contiguous();
  auto vn = f32c(value_norms, dev);
  auto cen = f32c(centroids, dev);
  auto RT = f32c(rotation_T, dev);
  const int64_t B = w.size(0), H = w.size(1), T = w.size(2), d = RT.size(0);
  TORCH_CHECK(RT.dim() == 2 && RT.size(1) == d, "rotation_T must be [d, d]");
  TORCH_CHECK(pv.scalar_type() == at::kByte, "packed_values must be uint8");
  TORCH_CHECK(pv.size(0) == T, "packed_values must have seq_len rows");
  TORCH_CHECK(pv.size(1) == packed_width(bit_width, d), "packed dim mismatch: expected ",
              packed_width(bit_width, d), " got ", pv.size(1));
  TORCH_CHECK(vn.numel() == T, "value_norms must have seq_len entries");
  TORCH_CHECK(cen.numel() == (1 << bit_width), "centroids length must be 2^bit_width");
  auto out = at::empty({B, H, d}, w.options());
  if (B * H == 0) return out;
  auto ws = workspace(tq_values_workspace_bytes(B * H, (int32_t)d, T), dev);
  check_rc(tq_attention_values_packed(w.data_ptr<float>(), B * H, T, pv.data_ptr<uint8_t>(),
                                      vn.data_ptr<float>(), cen.data_ptr<float>(),
                                      RT.data_ptr<float>(), (int32_t)d, (int32_t)bit_width,
                                      out.data_ptr<float>(), ws.data_ptr(), ws.numel(),
                                      cur_stream(w)));
  return out;
}

at::Tensor pack_codes(const at::Tensor& codes, int64_t bit_width) {
  require_gpu(codes, "codes");
  TORCH_CHECK(codes.scalar_type() == at::kByte, "codes must be uint8");
  TORCH_CHECK(codes.dim() == 2, "codes must be 2D [N, d]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 8, "bit_width must be 1-8");
  c10::DeviceGuard g(codes.device());
  auto c = codes.contiguous();
  const int64_t n = c.size(0), d = c.size(1);
  auto packed = at::empty({n, packed_width(bit_width, d)}, c.options());
  if (d == 0) return packed;
  check_rc(tq_pack_codes(c.data_ptr<uint8_t>(), n, (int32_t)d, (int32_t)bit_width,
                         packed.data_ptr<uint8_t>(), cur_stream(c)));
  return packed;
}

at::Tensor unpack_codes(const at::Tensor& packed, int64_t bit_width, int64_t dim) {
  require_gpu(packed, "packed");
  TORCH_CHECK(packed.scalar_type() == at::kByte, "packed must be uint8");
  TORCH_CHECK(packed.dim() == 2, "packed must be 2D");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 8, "bit_width must be 1-8");
  TORCH_CHECK(dim >= 1, "dim must be >= 1");
  c10::DeviceGuard g(packed.device());
  auto p = packed.contiguous();
  TORCH_CHECK(p.size(1) == packed_width(bit_width, dim), "packed dim mismatch: expected ",
              packed_width(bit_width, dim), " got ", p.size(1));
  auto codes = at::empty({p.size(0), dim}, p.options());
  check_rc(tq_unpack_codes(p.data_ptr<uint8_t>(), p.size(0), (int32_t)dim, (int32_t)bit_width,
                           codes.data_ptr<uint8_t>(), cur_stream(p)));
  return codes;
}

// ------------------------------------------------------------ fused ops (new)

// quantize_mse with the reference's rounding points: intermediates in vectors.dtype,
// norms returned in vectors.dtype (reference.py:263-317).
std::tuple<at::Tensor, at::Tensor> quantize_mse_packed(const at::Tensor& vectors,
                                                       const at::Tensor& rotation,
                                                       const at::Tensor& boundaries,
                                                       int64_t bit_width) {
  require_gpu(vectors, "vectors");
  TORCH_CHECK(vectors.dim() == 2, "vectors must be [N, d]");
  c10::DeviceGuard g(vectors.device());
  const auto dev = vectors.device();
  auto x = floatc(vectors, dev);
  const tq_dtype dt = to_tq(x.scalar_type());
  auto R = f32c(rotation, dev);
  auto bnd = f32c(boundaries, dev);
  const int64_t n = x.size(0), d = x.size(1);
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  TORCH_CHECK(bnd.numel() == (1 << bit_width) - 1, "boundaries length must be 2^bit_width - 1");
  auto packed = at::empty({n, packed_width(bit_width, d)}, x.options().dtype(at::kByte));
  auto norms = at::empty({n}, x.options().dtype(at::kFloat));
  check_rc(tq_rotate_and_quantize(x.data_ptr(), dt, dt, n, (int32_t)d, R.data_ptr<float>(),
                                  bnd.data_ptr<float>(), (int32_t)bit_width,
                                  packed.data_ptr<uint8_t>(), norms.data_ptr<float>(),
                                  cur_stream(x)));
  return {packed, norms.to(x.scalar_type())};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> quantize_prod_packed(
    const at::Tensor& vectors, const at::Tensor& rotation, const at::Tensor& boundaries,
    const at::Tensor& centroids, const at::Tensor& qjl, int64_t bit_width) {
  require_gpu(vectors, "vectors");
  TORCH_CHECK(vectors.dim() == 2, "vectors must be [N, d]");
  TORCH_CHECK(bit_width >= 2, "Prod mode requires bits >= 2, got ", bit_width);
  TORCH_CHECK(bit_width <= 5, "Prod mode supports bits <= 5");
  c10::DeviceGuard g(vectors.device());
  const auto dev = vectors.device();
  auto x = floatc(vectors, dev);
  const tq_dtype dt = to_tq(x.scalar_type());
  auto R = f32c(rotation, dev);
  auto bnd = f32c(boundaries, dev);
  auto cen = f32c(centroids, dev);
  auto S = f32c(qjl, dev);
  const int64_t n = x.size(0), d = x.size(1);
  const int64_t mb = bit_width - 1;
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  TORCH_CHECK(S.dim() == 2 && S.size(0) == d && S.size(1) == d, "S_matrix must be [d, d]");
  TORCH_CHECK(bnd.numel() == (1 << mb) - 1, "boundaries length must be 2^(bits-1) - 1");
  TORCH_CHECK(cen.numel() == (1 << mb), "centroids length must be 2^(bits-1)");
  auto ob = x.options().dtype(at::kByte);
  auto of = x.options().dtype(at::kFloat);
  auto mp = at::empty({n, packed_width(mb, d)}, ob);
  auto sg = at::empty({n, (d + 7) / 8}, ob);
  auto rn = at::empty({n}, of);
  auto nm = at::empty({n}, of);
  check_rc(tq_quantize_prod(x.data_ptr(), dt, dt, n, (int32_t)d, R.data_ptr<float>(),
                            bnd.data_ptr<float>(), cen.data_ptr<float>(), S.data_ptr<float>(),
                            (int32_t)bit_width, mp.data_ptr<uint8_t>(), sg.data_ptr<uint8_t>(),
                            rn.data_ptr<float>(), nm.data_ptr<float>(), cur_stream(x)));
  return {mp, sg, rn.to(x.scalar_type()), nm.to(x.scalar_type())};
}

at::Tensor dequantize_mse_packed(const at::Tensor& packed, const at::Tensor& norms,
                                 const at::Tensor& centroids, const at::Tensor& rotation,
                                 int64_t bit_width, int64_t dim) {
  require_gpu(packed, "packed_codes");
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.dim() == 2, "packed must be uint8 [N, P]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  c10::DeviceGuard g(packed.device());
  const auto dev = packed.device();
  auto p = packed.contiguous();
  const int64_t n = p.size(0);
  TORCH_CHECK(p.size(1) == packed_width(bit_width, dim), "packed dim mismatch");
  auto nf = norms.to(dev).contiguous();
  const tq_dtype odt = to_tq(nf.scalar_type());
  auto n32 = nf.to(at::kFloat).contiguous();
  TORCH_CHECK(n32.numel() == n, "norms must have N entries");
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  TORCH_CHECK(cen.numel() == (1 << bit_width), "centroids length must be 2^bit_width");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == dim && R.size(1) == dim, "rotation must be [d, d]");
  auto out = at::empty({n, dim}, p.options().dtype(from_tq(odt)));
  check_rc(tq_dequantize_mse(p.data_ptr<uint8_t>(), n32.data_ptr<float>(), n, (int32_t)dim,
                             (int32_t)bit_width, cen.data_ptr<float>(), R.data_ptr<float>(), odt,
                             out.data_ptr(), cur_stream(p)));
  return out;
}

at::Tensor dequantize_prod_packed(const at::Tensor& mse_packed, const at::Tensor& signs,
                                  const at::Tensor& res_norms, const at::Tensor& norms,
                                  const at::Tensor& centroids, const at::Tensor& rotation,
                                  const at::Tensor& qjl, int64_t bit_width, int64_t dim) {
  require_gpu(mse_packed, "mse_packed");
  TORCH_CHECK(bit_width >= 2 && bit_width <= 5, "Prod mode requires bits in [2, 5]");
  c10::DeviceGuard g(mse_packed.device());
  const auto dev = mse_packed.device();
  auto mp = mse_packed.contiguous();
  auto sg = signs.to(dev).contiguous();
  const int64_t n = mp.size(0);
  TORCH_CHECK(norms.scalar_type() == at::kFloat,
              "dequantize_prod computes in float32 (the reference's signs @ S needs fp32 S)");
  TORCH_CHECK(mp.size(1) == packed_width(bit_width - 1, dim), "packed dim mismatch");
  TORCH_CHECK(sg.scalar_type() == at::kByte && sg.size(0) == n && sg.size(1) == (dim + 7) / 8,
              "signs must be uint8 [N, ceil(d/8)]");
  auto rn = f32c(res_norms, dev);
  auto nm = f32c(norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  auto S = f32c(qjl, dev);
  TORCH_CHECK(rn.numel() == n && nm.numel() == n, "norms must have N entries");
  TORCH_CHECK(cen.numel() == (1 << (bit_width - 1)), "centroids length must be 2^(bits-1)");
  auto out = at::empty({n, dim}, mp.options().dtype(at::kFloat));
  check_rc(tq_dequantize_prod(mp.data_ptr<uint8_t>(), sg.data_ptr<uint8_t>(), rn.data_ptr<float>(),
                              nm.data_ptr<float>(), n, (int32_t)dim, (int32_t)bit_width,
                              cen.data_ptr<float>(), R.data_ptr<float>(), S.data_ptr<float>(),
                              TQ_F32, out.data_ptr(), cur_stream(mp)));
  return out;
}

std::tuple<at::Tensor, at::Tensor> ip_scan_topk(const at::Tensor& queries, const at::Tensor& packed,
                                                const at::Tensor& norms, const at::Tensor& centroids,
                                                const at::Tensor& rotation, int64_t bit_width,
                                                int64_t k) {
  require_gpu(queries, "queries");
  TORCH_CHECK(queries.dim() == 2, "queries must be [Q, d]");
  TORCH_CHECK(packed.dim() == 2 && packed.scalar_type() == at::kByte, "packed must be uint8 [N, P]");
  c10::DeviceGuard g(queries.device());
  const auto dev = queries.device();
  auto q = floatc(queries, dev);
  auto p = packed.to(dev).contiguous();
  auto nm = f32c(norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  const int64_t Q = q.size(0), d = q.size(1), N = p.size(0);
  TORCH_CHECK(p.size(1) == packed_width(bit_width, d), "packed dim mismatch");
  TORCH_CHECK(nm.numel() == N, "norms must have N entries");
  TORCH_CHECK(cen.numel() == (1 << bit_width), "centroids length must be 2^bit_width");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto os = at::empty({Q, k}, q.options().dtype(at::kFloat));
  auto oi = at::empty({Q, k}, q.options().dtype(at::kLong));
  if (Q == 0) return {os, oi};
  auto ws = workspace(tq_scan_workspace_bytes(Q, (int32_t)d, (int32_t)bit_width, N, (int32_t)k), dev);
  check_rc(tq_ip_scan_topk(q.data_ptr(), to_tq(q.scalar_type()), Q, (int32_t)d, p.data_ptr<uint8_t>(),
                           nm.data_ptr<float>(), N, cen.data_ptr<float>(), R.data_ptr<float>(),
                           (int32_t)bit_width, (int32_t)k, os.data_ptr<float>(),
                           oi.data_ptr<int64_t>(), ws.data_ptr(), ws.numel(), cur_stream(q)));
  return {os, oi};
}

// Same scan over 4-bit pair-layout rows [N, d/2] (d = 64 or 128).
std::tuple<at::Tensor, at::Tensor> ip_scan_topk_pairs(const at::Tensor& queries,
                                                      const at::Tensor& pairs,
                                                      const at::Tensor& norms,
                                                      const at::Tensor& centroids,
                                                      const at::Tensor& rotation, int64_t k) {
  require_gpu(queries, "queries");
  TORCH_CHECK(queries.dim() == 2, "queries must be [Q, d]");
  TORCH_CHECK(pairs.dim() == 2 && pairs.scalar_type() == at::kByte, "pairs must be uint8 [N, d/2]");
  c10::DeviceGuard g(queries.device());
  const auto dev = queries.device();
  auto q = floatc(queries, dev);
  auto p = pairs.to(dev).contiguous();
  auto nm = f32c(norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  const int64_t Q = q.size(0), d = q.size(1), N = p.size(0);
  TORCH_CHECK(p.size(1) * 2 == d, "pairs must hold d/2 bytes per row");
  TORCH_CHECK(nm.numel() == N, "norms must have N entries");
  TORCH_CHECK(cen.numel() == 16, "pair layout holds 4-bit codes: 16 centroids");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto os = at::empty({Q, k}, q.options().dtype(at::kFloat));
  auto oi = at::empty({Q, k}, q.options().dtype(at::kLong));
  if (Q == 0) return {os, oi};
  auto ws = workspace(tq_scan_pairs_workspace_bytes(Q, (int32_t)d, N, (int32_t)k), dev);
  check_rc(tq_ip_scan_topk_pairs(q.data_ptr(), to_tq(q.scalar_type()), Q, (int32_t)d,
                                 p.data_ptr<uint8_t>(), nm.data_ptr<float>(), N,
                                 cen.data_ptr<float>(), R.data_ptr<float>(), (int32_t)k,
                                 os.data_ptr<float>(), oi.data_ptr<int64_t>(), ws.data_ptr(),
                                 ws.numel(), cur_stream(q)));
  return {os, oi};
}

// Prod rows (quantize_prod_packed's outputs): checks shared by the two prod scoring ops.
struct ProdRowsT {
  at::Tensor mp, sg, rn, nm, cen, R, S;
};
ProdRowsT prod_rows(const at::Tensor& mse_packed, const at::Tensor& signs,
                    const at::Tensor& res_norms, const at::Tensor& norms,
                    const at::Tensor& centroids, const at::Tensor& rotation, const at::Tensor& qjl,
                    int64_t bit_width, int64_t d, c10::Device dev) {
  TORCH_CHECK(bit_width >= 2 && bit_width <= 4, "prod scoring supports bit_width 2-4");
  TORCH_CHECK(mse_packed.dim() == 2 && mse_packed.scalar_type() == at::kByte,
              "mse_packed must be uint8 [N, P]");
  ProdRowsT r;
  r.mp = mse_packed.to(dev).contiguous();
  const int64_t n = r.mp.size(0);
  TORCH_CHECK(r.mp.size(1) == packed_width(bit_width - 1, d), "packed dim mismatch");
  r.sg = signs.to(dev).contiguous();
  TORCH_CHECK(r.sg.scalar_type() == at::kByte && r.sg.dim() == 2 && r.sg.size(0) == n &&
                  r.sg.size(1) == (d + 7) / 8,
              "signs must be uint8 [N, ceil(d/8)]");
  r.rn = f32c(res_norms, dev);
  r.nm = f32c(norms, dev);
  r.cen = f32c(centroids, dev);
  r.R = f32c(rotation, dev);
  r.S = f32c(qjl, dev);
  TORCH_CHECK(r.rn.numel() == n && r.nm.numel() == n, "norms must have N entries");
  TORCH_CHECK(r.cen.numel() == (1 << (bit_width - 1)), "centroids length must be 2^(bits-1)");
  TORCH_CHECK(r.R.dim() == 2 && r.R.size(0) == d && r.R.size(1) == d, "rotation must be [d, d]");
  TORCH_CHECK(r.S.dim() == 2 && r.S.size(0) == d && r.S.size(1) == d, "S_matrix must be [d, d]");
  return r;
}

// <q, dequantize_prod(row)> for every row, top-k (search.py:229-252 without the
// reconstruction).
// pairs: the MSE half as pair rows (tq_ip_scan_topk_prod_pair_rows; same row width).
std::tuple<at::Tensor, at::Tensor> ip_scan_topk_prod_impl(const at::Tensor& queries,
                                                          const at::Tensor& mse_packed,
                                                          const at::Tensor& signs,
                                                          const at::Tensor& res_norms,
                                                          const at::Tensor& norms,
                                                          const at::Tensor& centroids,
                                                          const at::Tensor& rotation,
                                                          const at::Tensor& qjl, int64_t bit_width,
                                                          int64_t k, bool pairs) {
  require_gpu(queries, "queries");
  TORCH_CHECK(queries.dim() == 2, "queries must be [Q, d]");
  c10::DeviceGuard g(queries.device());
  const auto dev = queries.device();
  auto q = floatc(queries, dev);
  const int64_t Q = q.size(0), d = q.size(1);
  auto r = prod_rows(mse_packed, signs, res_norms, norms, centroids, rotation, qjl, bit_width, d, dev);
  const int64_t N = r.mp.size(0);
  auto os = at::empty({Q, k}, q.options().dtype(at::kFloat));
  auto oi = at::empty({Q, k}, q.options().dtype(at::kLong));
  if (Q == 0) return {os, oi};
  auto ws = workspace(tq_scan_workspace_bytes(Q, (int32_t)d, (int32_t)bit_width, N, (int32_t)k), dev);
  check_rc((pairs ? tq_ip_scan_topk_prod_pair_rows : tq_ip_scan_topk_prod)(
      q.data_ptr(), to_tq(q.scalar_type()), Q, (int32_t)d, r.mp.data_ptr<uint8_t>(),
      r.sg.data_ptr<uint8_t>(), r.rn.data_ptr<float>(), r.nm.data_ptr<float>(), N,
      r.cen.data_ptr<float>(), r.R.data_ptr<float>(), r.S.data_ptr<float>(), (int32_t)bit_width,
      (int32_t)k, os.data_ptr<float>(), oi.data_ptr<int64_t>(), ws.data_ptr(), ws.numel(),
      cur_stream(q)));
  return {os, oi};
}

std::tuple<at::Tensor, at::Tensor> ip_scan_topk_prod(const at::Tensor& queries, const at::Tensor& mse_packed,
                                                     const at::Tensor& signs, const at::Tensor& res_norms,
                                                     const at::Tensor& norms, const at::Tensor& centroids,
                                                     const at::Tensor& rotation, const at::Tensor& qjl,
                                                     int64_t bit_width, int64_t k) {
  return ip_scan_topk_prod_impl(queries, mse_packed, signs, res_norms, norms, centroids, rotation,
                                qjl, bit_width, k, false);
}

std::tuple<at::Tensor, at::Tensor> ip_scan_topk_prod_pair_rows(
    const at::Tensor& queries, const at::Tensor& mse_rows, const at::Tensor& signs,
    const at::Tensor& res_norms, const at::Tensor& norms, const at::Tensor& centroids,
    const at::Tensor& rotation, const at::Tensor& qjl, int64_t bit_width, int64_t k) {
  return ip_scan_topk_prod_impl(queries, mse_rows, signs, res_norms, norms, centroids, rotation,
                                qjl, bit_width, k, true);
}

// attention_scores_packed for prod-mode keys: query [B, H, d] -> [B, H, T] fp32.
at::Tensor attention_scores_prod_impl(const at::Tensor& query, const at::Tensor& mse_packed,
                                      const at::Tensor& signs, const at::Tensor& res_norms,
                                      const at::Tensor& key_norms, const at::Tensor& centroids,
                                      const at::Tensor& rotation, const at::Tensor& qjl,
                                      int64_t bit_width, bool pairs) {
  require_gpu(query, "query");
  TORCH_CHECK(query.dim() == 3, "query must be [batch, heads, head_dim]");
  c10::DeviceGuard g(query.device());
  const auto dev = query.device();
  auto q = f32c(query, dev);
  const int64_t B = q.size(0), H = q.size(1), d = q.size(2);
  auto r = prod_rows(mse_packed, signs, res_norms, key_norms, centroids, rotation, qjl, bit_width,
                     d, dev);
  const int64_t T = r.mp.size(0);
  auto scores = at::empty({B, H, T}, q.options());
  if (B * H == 0 || T == 0) return scores;
  auto ws = workspace(tq_scan_workspace_bytes(B * H, (int32_t)d, (int32_t)bit_width, T, 0), dev);
  check_rc((pairs ? tq_attention_scores_prod_pair_rows : tq_attention_scores_prod)(
      q.data_ptr(), TQ_F32, B * H, (int32_t)d, r.mp.data_ptr<uint8_t>(), r.sg.data_ptr<uint8_t>(),
      r.rn.data_ptr<float>(), r.nm.data_ptr<float>(), T, r.cen.data_ptr<float>(),
      r.R.data_ptr<float>(), r.S.data_ptr<float>(), (int32_t)bit_width, scores.data_ptr<float>(),
      ws.data_ptr(), ws.numel(), cur_stream(q)));
  return scores;
}

at::Tensor attention_scores_prod(const at::Tensor& query, const at::Tensor& mse_packed,
                                 const at::Tensor& signs, const at::Tensor& res_norms,
                                 const at::Tensor& key_norms, const at::Tensor& centroids,
                                 const at::Tensor& rotation, const at::Tensor& qjl, int64_t bit_width) {
  return attention_scores_prod_impl(query, mse_packed, signs, res_norms, key_norms, centroids,
                                    rotation, qjl, bit_width, false);
}

at::Tensor attention_scores_prod_pair_rows(const at::Tensor& query, const at::Tensor& mse_rows,
                                           const at::Tensor& signs, const at::Tensor& res_norms,
                                           const at::Tensor& key_norms, const at::Tensor& centroids,
                                           const at::Tensor& rotation, const at::Tensor& qjl,
                                           int64_t bit_width) {
  return attention_scores_prod_impl(query, mse_rows, signs, res_norms, key_norms, centroids,
                                    rotation, qjl, bit_width, true);
}

// Pair rows of 2-4 bit codes (d * bits / 8 bytes per row, d = 64 or 128): conversion
// from / to bit-plane rows and the top-k scan over them.
at::Tensor pack_pair_rows(const at::Tensor& packed, int64_t bit_width, int64_t dim) {
  require_gpu(packed, "packed");
  c10::DeviceGuard g(packed.device());
  auto pk = packed.contiguous();
  TORCH_CHECK(pk.dim() == 2 && pk.scalar_type() == at::kByte && pk.size(1) == packed_width(bit_width, dim),
              "packed must be uint8 [n, bits * ceil(dim / 8)]");
  auto rows = at::empty({pk.size(0), dim * bit_width / 8}, pk.options());
  check_rc(tq_pack_pair_rows(pk.data_ptr<uint8_t>(), pk.size(0), (int32_t)dim, (int32_t)bit_width,
                             rows.data_ptr<uint8_t>(), cur_stream(pk)));
  return rows;
}

at::Tensor unpack_pair_rows(const at::Tensor& rows, int64_t bit_width, int64_t dim) {
  require_gpu(rows, "rows");
  c10::DeviceGuard g(rows.device());
  auto r = rows.contiguous();
  TORCH_CHECK(r.dim() == 2 && r.scalar_type() == at::kByte && r.size(1) * 8 == dim * bit_width,
              "rows must be uint8 [n, dim * bits / 8]");
  auto out = at::empty({r.size(0), packed_width(bit_width, dim)}, r.options());
  check_rc(tq_unpack_pair_rows(r.data_ptr<uint8_t>(), r.size(0), (int32_t)dim, (int32_t)bit_width,
                               out.data_ptr<uint8_t>(), cur_stream(r)));
  return out;
}

std::tuple<at::Tensor, at::Tensor> ip_scan_topk_pair_rows(const at::Tensor& queries,
                                                          const at::Tensor& rows,
                                                          const at::Tensor& norms,
                                                          const at::Tensor& centroids,
                                                          const at::Tensor& rotation,
                                                          int64_t bit_width, int64_t k) {
  require_gpu(queries, "queries");
  TORCH_CHECK(queries.dim() == 2, "queries must be [Q, d]");
  TORCH_CHECK(rows.dim() == 2 && rows.scalar_type() == at::kByte, "rows must be uint8 [N, d * bits / 8]");
  c10::DeviceGuard g(queries.device());
  const auto dev = queries.device();
  auto q = floatc(queries, dev);
  auto p = rows.to(dev).contiguous();
  auto nm = f32c(norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  const int64_t Q = q.size(0), d = q.size(1), N = p.size(0);
  TORCH_CHECK(p.size(1) * 8 == d * bit_width, "rows must hold d * bits / 8 bytes");
  TORCH_CHECK(nm.numel() == N, "norms must have N entries");
  TORCH_CHECK(cen.numel() == (int64_t(1) << bit_width), "centroids must have 2^bits entries");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto os = at::empty({Q, k}, q.options().dtype(at::kFloat));
  auto oi = at::empty({Q, k}, q.options().dtype(at::kLong));
  if (Q == 0) return {os, oi};
  auto ws = workspace(tq_scan_pair_rows_workspace_bytes(Q, (int32_t)d, (int32_t)bit_width, N, (int32_t)k), dev);
  check_rc(tq_ip_scan_topk_pair_rows(q.data_ptr(), to_tq(q.scalar_type()), Q, (int32_t)d,
                                     p.data_ptr<uint8_t>(), nm.data_ptr<float>(), N,
                                     cen.data_ptr<float>(), R.data_ptr<float>(), (int32_t)bit_width,
                                     (int32_t)k, os.data_ptr<float>(), oi.data_ptr<int64_t>(),
                                     ws.data_ptr(), ws.numel(), cur_stream(q)));
  return {os, oi};
}

at::Tensor attention_scores_pair_rows(const at::Tensor& query, const at::Tensor& rows,
                                      const at::Tensor& key_norms, const at::Tensor& centroids,
                                      const at::Tensor& rotation, int64_t bit_width) {
  require_gpu(query, "query");
  TORCH_CHECK(query.dim() == 3, "query must be [batch, heads, head_dim]");
  TORCH_CHECK(rows.dim() == 2 && rows.scalar_type() == at::kByte, "rows must be uint8 [T, d * bits / 8]");
  c10::DeviceGuard g(query.device());
  const auto dev = query.device();
  auto q = f32c(query, dev);
  auto pk = rows.to(dev).contiguous();
  auto kn = f32c(key_norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  const int64_t B = q.size(0), H = q.size(1), d = q.size(2), T = pk.size(0);
  TORCH_CHECK(pk.size(1) * 8 == d * bit_width, "rows must hold d * bits / 8 bytes");
  TORCH_CHECK(kn.numel() == T, "key_norms must have seq_len entries");
  TORCH_CHECK(cen.numel() == (int64_t(1) << bit_width), "centroids must have 2^bits entries");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto scores = at::empty({B, H, T}, q.options());
  if (B * H == 0 || T == 0) return scores;
  auto ws = workspace(tq_scan_workspace_bytes(B * H, (int32_t)d, (int32_t)bit_width, T, 0), dev);
  check_rc(tq_attention_scores_pair_rows(q.data_ptr(), TQ_F32, B * H, (int32_t)d,
                                         pk.data_ptr<uint8_t>(), kn.data_ptr<float>(), T,
                                         cen.data_ptr<float>(), R.data_ptr<float>(),
                                         (int32_t)bit_width, scores.data_ptr<float>(),
                                         ws.data_ptr(), ws.numel(), cur_stream(q)));
  return scores;
}

at::Tensor attention_scores_pairs(const at::Tensor& query, const at::Tensor& pairs,
                                  const at::Tensor& key_norms, const at::Tensor& centroids,
                                  const at::Tensor& rotation) {
  require_gpu(query, "query");
  TORCH_CHECK(query.dim() == 3, "query must be [batch, heads, head_dim]");
  TORCH_CHECK(pairs.dim() == 2 && pairs.scalar_type() == at::kByte, "pairs must be uint8 [T, d/2]");
  c10::DeviceGuard g(query.device());
  const auto dev = query.device();
  auto q = f32c(query, dev);
  auto pk = pairs.to(dev).contiguous();
  auto kn = f32c(key_norms, dev);
  auto cen = f32c(centroids, dev);
  auto R = f32c(rotation, dev);
  const int64_t B = q.size(0), H = q.size(1), d = q.size(2), T = pk.size(0);
  TORCH_CHECK(pk.size(1) * 2 == d, "pairs must hold d/2 bytes per row");
  TORCH_CHECK(kn.numel() == T, "key_norms must have seq_len entries");
  TORCH_CHECK(cen.numel() == 16, "pair layout holds 4-bit codes: 16 centroids");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto scores = at::empty({B, H, T}, q.options());
  if (B * H == 0 || T == 0) return scores;
  auto ws = workspace(tq_scan_workspace_bytes(B * H, (int32_t)d, 4, T, 0), dev);
  check_rc(tq_attention_scores_pairs(q.data_ptr(), TQ_F32, B * H, (int32_t)d,
                                     pk.data_ptr<uint8_t>(), kn.data_ptr<float>(), T,
                                     cen.data_ptr<float>(), R.data_ptr<float>(),
                                     scores.data_ptr<float>(), ws.data_ptr(), ws.numel(),
                                     cur_stream(q)));
  return scores;
}

std::tuple<at::Tensor, at::Tensor> decode_attention_packed_lse(
    const at::Tensor& q, const at::Tensor& kpacked,
                                   const at::Tensor& knorms, const at::Tensor& vpacked,
                                   const at::Tensor& vnorms, const at::Tensor& seq_lens,
                                   const at::Tensor& kcentroids, const at::Tensor& vcentroids,
    const at::Tensor& krotation, const at::Tensor& vrotation,
    int64_t kbits, int64_t vbits, double scale) {
  require_gpu(q, "q");
  TORCH_CHECK(q.dim() == 3, "q must be [B, Hq, d]");
  TORCH_CHECK(kpacked.dim() == 4 && vpacked.dim() == 4, "packed K/V must be [B, Hkv, T, P]");
  c10::DeviceGuard g(q.device());
  const auto dev = q.device();
  auto qq = floatc(q, dev);
  const int64_t B = qq.size(0), Hq = qq.size(1), d = qq.size(2);
  const int64_t Hkv = kpacked.size(1), Tm = kpacked.size(2);
  TORCH_CHECK(kpacked.scalar_type() == at::kByte && vpacked.scalar_type() == at::kByte,
              "packed K/V must be uint8");
  TORCH_CHECK(kpacked.is_contiguous() && vpacked.is_contiguous() && knorms.is_contiguous() &&
                  vnorms.is_contiguous(),
              "packed K/V and norms must be contiguous");
  TORCH_CHECK(kpacked.device() == dev && vpacked.device() == dev && knorms.device() == dev &&
                  vnorms.device() == dev,
              "K/V must be on the query's device");
  TORCH_CHECK(kpacked.size(0) == B && vpacked.size(0) == B && vpacked.size(1) == Hkv &&
                  vpacked.size(2) == Tm,
              "K/V batch/head/length mismatch");
  TORCH_CHECK(kpacked.size(3) == packed_width(kbits, d), "packed key width mismatch");
  TORCH_CHECK(vpacked.size(3) == packed_width(vbits, d), "packed value width mismatch");
  TORCH_CHECK(knorms.scalar_type() == at::kFloat && vnorms.scalar_type() == at::kFloat,
              "norms must be float32");
  TORCH_CHECK(knorms.numel() == B * Hkv * Tm && vnorms.numel() == B * Hkv * Tm, "norms shape");
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "num_heads must be a multiple of num_kv_heads");
  auto sl = seq_lens.to(dev, at::kInt).contiguous();
  TORCH_CHECK(sl.numel() == B, "seq_lens must have B entries");
  auto kc = f32c(kcentroids, dev);
  auto vc = f32c(vcentroids, dev);
  auto Rk = f32c(krotation, dev);
  auto Rv = f32c(vrotation, dev);
  TORCH_CHECK(kc.numel() == (1 << kbits) && vc.numel() == (1 << vbits), "centroid lengths");
  auto out = at::empty({B, Hq, d}, qq.options());
  auto lse = at::empty({B, Hq}, qq.options().dtype(at::kFloat));
  if (B == 0) return {out, lse};
  auto ws = workspace(tq_decode_workspace_bytes((int32_t)B, (int32_t)Hq, (int32_t)d, Tm), dev);
  check_rc(tq_decode_attention_packed(
      qq.data_ptr(), to_tq(qq.scalar_type()), (int32_t)B, (int32_t)Hq, (int32_t)Hkv, (int32_t)d,
      kpacked.data_ptr<uint8_t>(), knorms.data_ptr<float>(), vpacked.data_ptr<uint8_t>(),
      vnorms.data_ptr<float>(), Tm, sl.data_ptr<int32_t>(), kc.data_ptr<float>(),
      vc.data_ptr<float>(), Rk.data_ptr<float>(), Rv.data_ptr<float>(), (int32_t)kbits,
      (int32_t)vbits, (float)scale, out.data_ptr(), lse.data_ptr<float>(), ws.data_ptr(),
      ws.numel(), cur_stream(qq)));
  return {out, lse};
}

at::Tensor decode_attention_packed(const at::Tensor& q, const at::Tensor& kpacked,
                                   const at::Tensor& knorms, const at::Tensor& vpacked,
                                   const at::Tensor& vnorms, const at::Tensor& seq_lens,
                                   const at::Tensor& kcentroids, const at::Tensor& vcentroids,
                                   const at::Tensor& krotation, const at::Tensor& vrotation,
                                   int64_t kbits, int64_t vbits, double scale) {
  return std::get<0>(decode_attention_packed_lse(q, kpacked, knorms, vpacked, vnorms, seq_lens,
                                                 kcentroids, vcentroids, krotation, vrotation,
                                                 kbits, vbits, scale));
}

// ------------------------------------------------------------ the C++ core's tables (TQIX files)

at::Tensor core_rotation(int64_t dim, int64_t seed) {
  auto R = at::empty({dim, dim}, at::TensorOptions().dtype(at::kFloat));
  check_rc(tq_core_rotation((int32_t)dim, (int32_t)seed, R.data_ptr<float>()));
  return R;
}

std::tuple<at::Tensor, at::Tensor> core_codebook(int64_t bits, int64_t dim) {
  TORCH_CHECK(bits >= 1 && bits <= 8, "bits must be in [1, 8]");
  auto o = at::TensorOptions().dtype(at::kFloat);
  auto bnd = at::empty({(1 << bits) - 1}, o);
  auto cen = at::empty({1 << bits}, o);
  check_rc(tq_core_codebook((int32_t)bits, (int32_t)dim, bnd.data_ptr<float>(), cen.data_ptr<float>()));
  return {bnd, cen};
}

// ------------------------------------------------------------ Huffman streams (host tensors)

at::Tensor huffman_encode(const at::Tensor& codes, const at::Tensor& code_words,
                          const at::Tensor& code_lens) {
  TORCH_CHECK(!codes.is_cuda() && !code_words.is_cuda() && !code_lens.is_cuda(),
              "huffman_encode works on host tensors");
  auto c = codes.to(at::kByte).contiguous().reshape({-1});
  auto w = code_words.to(at::kLong).contiguous();
  auto l = code_lens.to(at::kByte).contiguous();
  TORCH_CHECK(w.numel() == l.numel(), "one code word and length per symbol");
  uint64_t nbits = 0;
  const uint8_t* cp = c.data_ptr<uint8_t>();
  const uint8_t* lp = l.data_ptr<uint8_t>();
  for (int64_t i = 0; i < c.numel(); ++i) {
    TORCH_CHECK(cp[i] < l.numel(), "symbol out of range");
    nbits += lp[cp[i]];
  }
  auto out = at::empty({(int64_t)(8 + (nbits + 7) / 8)}, at::TensorOptions().dtype(at::kByte));
  size_t nb = 0;
  check_rc(tq_huffman_encode(cp, c.numel(), reinterpret_cast<const uint64_t*>(w.data_ptr<int64_t>()),
                             lp, (int32_t)l.numel(), out.data_ptr<uint8_t>(), out.numel(), &nb));
  return out;
}

at::Tensor huffman_decode(const at::Tensor& data, int64_t n_symbols, const at::Tensor& code_words,
                          const at::Tensor& code_lens, const at::Tensor& symbols) {
  TORCH_CHECK(!data.is_cuda(), "huffman_decode works on host tensors");
  auto d = data.to(at::kByte).contiguous();
  auto w = code_words.to(at::kLong).contiguous();
  auto l = code_lens.to(at::kByte).contiguous();
  auto sy = symbols.to(at::kInt).contiguous();
  TORCH_CHECK(w.numel() == l.numel() && w.numel() == sy.numel(), "code table sizes differ");
  TORCH_CHECK(d.numel() >= 8, "stream shorter than its header");
  int64_t n = n_symbols;
  if (n < 0) {
    const uint8_t* p = d.data_ptr<uint8_t>();
    n = (int64_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
  }
  // Every code word is at least one bit long, so the body holds at most 8 symbols per
  // byte: a corrupt or truncated header cannot make the output larger than that.
  n = std::min<int64_t>(n, 8 * (d.numel() - 8));
  auto out = at::empty({n}, at::TensorOptions().dtype(at::kByte));
  int64_t got = 0;
  check_rc(tq_huffman_decode(d.data_ptr<uint8_t>(), d.numel(), n,
                             reinterpret_cast<const uint64_t*>(w.data_ptr<int64_t>()),
                             l.data_ptr<uint8_t>(), sy.data_ptr<int32_t>(), (int32_t)sy.numel(),
                             out.data_ptr<uint8_t>(), &got));
  return out.narrow(0, 0, got).clone();
}

// ------------------------------------------------------------ paged pools (vLLM block tables)

// rows [n, hkv, P] u8 (+ norms [n, hkv] f32) to the slots slot_mapping [n] of
// pool [num_blocks, hkv, block_size, P] (+ norm_pool [num_blocks, hkv, block_size]).
void paged_store(const at::Tensor& rows, const c10::optional<at::Tensor>& norms,
                 const at::Tensor& slot_mapping, at::Tensor& pool,
                 const c10::optional<at::Tensor>& norm_pool) {
  require_gpu(pool, "pool");
  TORCH_CHECK(pool.dim() == 4 && pool.scalar_type() == at::kByte && pool.is_contiguous(),
              "pool must be contiguous uint8 [num_blocks, hkv, block_size, P]");
  TORCH_CHECK(rows.dim() == 3 && rows.scalar_type() == at::kByte, "rows must be uint8 [n, hkv, P]");
  TORCH_CHECK(norms.has_value() == norm_pool.has_value(), "norms and norm_pool go together");
  c10::DeviceGuard g(pool.device());
  const auto dev = pool.device();
  const int64_t n = rows.size(0), hkv = pool.size(1), bs = pool.size(2), P = pool.size(3);
  TORCH_CHECK(rows.size(1) == hkv && rows.size(2) == P, "rows must be [n, hkv, P] of the pool's hkv, P");
  auto r = rows.to(dev).contiguous();
  auto sm = slot_mapping.to(dev, at::kLong).contiguous();
  TORCH_CHECK(sm.numel() == n, "slot_mapping must have one entry per token");
  at::Tensor nm, np;
  if (norms.has_value()) {
    nm = f32c(*norms, dev);
    np = *norm_pool;
    TORCH_CHECK(nm.numel() == n * hkv, "norms must be [n, hkv]");
    TORCH_CHECK(np.device() == dev && np.scalar_type() == at::kFloat && np.is_contiguous() &&
                    np.numel() == pool.size(0) * hkv * bs,
                "norm_pool must be contiguous float32 [num_blocks, hkv, block_size]");
  }
  check_rc(tq_paged_store(r.data_ptr<uint8_t>(), nm.defined() ? nm.data_ptr<float>() : nullptr, n,
                          (int32_t)hkv, (int32_t)P, sm.data_ptr<int64_t>(), pool.data_ptr<uint8_t>(),
                          np.defined() ? np.data_ptr<float>() : nullptr, pool.size(0), (int32_t)bs,
                          cur_stream(pool)));
}

// The first seq_lens[b] tokens of each batch row as contiguous [B, hkv, t_max, P] rows
// (+ [B, hkv, t_max] norms; empty without norm_pool).
std::tuple<at::Tensor, at::Tensor> paged_gather(const at::Tensor& pool,
                                                const c10::optional<at::Tensor>& norm_pool,
                                                const at::Tensor& block_tables,
                                                const at::Tensor& seq_lens, int64_t t_max) {
  require_gpu(pool, "pool");
  TORCH_CHECK(pool.dim() == 4 && pool.scalar_type() == at::kByte && pool.is_contiguous(),
              "pool must be contiguous uint8 [num_blocks, hkv, block_size, P]");
  c10::DeviceGuard g(pool.device());
  const auto dev = pool.device();
  const int64_t hkv = pool.size(1), bs = pool.size(2), P = pool.size(3);
  auto bt = block_tables.to(dev, at::kInt).contiguous();
  TORCH_CHECK(bt.dim() == 2, "block_tables must be [B, max_blocks]");
  auto sl = seq_lens.to(dev, at::kInt).contiguous();
  const int64_t B = bt.size(0);
  TORCH_CHECK(sl.numel() == B, "seq_lens must have B entries");
  auto rows = at::empty({B, hkv, t_max, P}, pool.options());
  at::Tensor np, on;
  if (norm_pool.has_value()) {
    np = *norm_pool;
    TORCH_CHECK(np.device() == dev && np.scalar_type() == at::kFloat && np.is_contiguous() &&
                    np.numel() == pool.size(0) * hkv * bs,
                "norm_pool must be contiguous float32 [num_blocks, hkv, block_size]");
    on = at::empty({B, hkv, t_max}, pool.options().dtype(at::kFloat));
  } else {
    on = at::empty({0}, pool.options().dtype(at::kFloat));
  }
  check_rc(tq_paged_gather(pool.data_ptr<uint8_t>(), np.defined() ? np.data_ptr<float>() : nullptr,
                           pool.size(0), (int32_t)hkv, (int32_t)bs, (int32_t)P, bt.data_ptr<int32_t>(),
                           (int32_t)bt.size(1), sl.data_ptr<int32_t>(), (int32_t)B, t_max,
                           rows.data_ptr<uint8_t>(), np.defined() ? on.data_ptr<float>() : nullptr,
                           cur_stream(pool)));
  return {rows, on};
}

std::tuple<at::Tensor, at::Tensor> decode_attention_paged(
    const at::Tensor& q, const at::Tensor& kpool, const at::Tensor& knorm_pool,
    const at::Tensor& vpool, const at::Tensor& vnorm_pool, const at::Tensor& block_tables,
    const at::Tensor& seq_lens, const at::Tensor& kcentroids, const at::Tensor& vcentroids,
    const at::Tensor& krotation, const at::Tensor& vrotation, int64_t kbits, int64_t vbits,
    double scale) {
  require_gpu(q, "q");
  TORCH_CHECK(q.dim() == 3, "q must be [B, Hq, d]");
  TORCH_CHECK(kpool.dim() == 4 && vpool.dim() == 4, "pools must be [num_blocks, hkv, block_size, P]");
  c10::DeviceGuard g(q.device());
  const auto dev = q.device();
  auto qq = floatc(q, dev);
  const int64_t B = qq.size(0), Hq = qq.size(1), d = qq.size(2);
  const int64_t nb = kpool.size(0), Hkv = kpool.size(1), bs = kpool.size(2);
  for (const at::Tensor* t : {&kpool, &vpool, &knorm_pool, &vnorm_pool})
    TORCH_CHECK(t->device() == dev && t->is_contiguous(), "pools must be contiguous on the query's device");
  TORCH_CHECK(kpool.scalar_type() == at::kByte && vpool.scalar_type() == at::kByte, "pools must be uint8");
  TORCH_CHECK(vpool.size(0) == nb && vpool.size(1) == Hkv && vpool.size(2) == bs, "K/V pool shapes differ");
  TORCH_CHECK(kpool.size(3) == packed_width(kbits, d) && vpool.size(3) == packed_width(vbits, d),
              "pool row widths must be bits * ceil(d/8)");
  TORCH_CHECK(knorm_pool.scalar_type() == at::kFloat && vnorm_pool.scalar_type() == at::kFloat &&
                  knorm_pool.numel() == nb * Hkv * bs && vnorm_pool.numel() == nb * Hkv * bs,
              "norm pools must be float32 [num_blocks, hkv, block_size]");
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "num_heads must be a multiple of num_kv_heads");
  auto bt = block_tables.to(dev, at::kInt).contiguous();
  TORCH_CHECK(bt.dim() == 2 && bt.size(0) == B, "block_tables must be [B, max_blocks]");
  auto sl = seq_lens.to(dev, at::kInt).contiguous();
  TORCH_CHECK(sl.numel() == B, "seq_lens must have B entries");
  auto kc = f32c(kcentroids, dev);
  auto vc = f32c(vcentroids, dev);
  auto Rk = f32c(krotation, dev);
  auto Rv = f32c(vrotation, dev);
  TORCH_CHECK(kc.numel() == (1 << kbits) && vc.numel() == (1 << vbits), "centroid lengths");
  auto out = at::empty({B, Hq, d}, qq.options());
  auto lse = at::empty({B, Hq}, qq.options().dtype(at::kFloat));
  if (B == 0) return {out, lse};
  const tq_dtype qdt = to_tq(qq.scalar_type());
  auto ws = workspace(tq_decode_paged_workspace_bytes(qdt, (int32_t)B, (int32_t)Hq, (int32_t)Hkv,
                                                      (int32_t)d, (int32_t)kbits, (int32_t)vbits,
                                                      (int32_t)bt.size(1), (int32_t)bs),
                      dev);
  check_rc(tq_decode_attention_paged(
      qq.data_ptr(), qdt, (int32_t)B, (int32_t)Hq, (int32_t)Hkv, (int32_t)d,
      kpool.data_ptr<uint8_t>(), knorm_pool.data_ptr<float>(), vpool.data_ptr<uint8_t>(),
      vnorm_pool.data_ptr<float>(), nb, (int32_t)bs, bt.data_ptr<int32_t>(), (int32_t)bt.size(1),
      sl.data_ptr<int32_t>(), kc.data_ptr<float>(), vc.data_ptr<float>(), Rk.data_ptr<float>(),
      Rv.data_ptr<float>(), (int32_t)kbits, (int32_t)vbits, (float)scale, out.data_ptr(),
      lse.data_ptr<float>(), ws.data_ptr(), ws.numel(), cur_stream(qq)));
  return {out, lse};
}

// ------------------------------------------------------------ decode layout

void pack_decode_layout(const at::Tensor& packed, at::Tensor& cache, int64_t dim,
                        int64_t bit_width, int64_t values, int64_t pos) {
  require_gpu(cache, "cache");
  c10::DeviceGuard g(cache.device());
  const auto dev = cache.device();
  TORCH_CHECK(cache.scalar_type() == at::kByte && cache.is_contiguous() && cache.dim() == 3,
              "cache must be contiguous uint8 [streams, rows, width]");
  auto pk = packed.to(dev, at::kByte).contiguous();
  TORCH_CHECK(pk.dim() == 3 && pk.size(0) == cache.size(0), "packed must be [streams, n, P]");
  TORCH_CHECK(pk.size(2) == packed_width(bit_width, dim), "packed width mismatch");
  const int64_t t_cap = values ? cache.size(1) * 64 : cache.size(1);
  TORCH_CHECK(cache.size(2) == (values ? 8 * bit_width * dim : dim / 2), "cache width mismatch");
  check_rc(tq_pack_decode_layout(pk.data_ptr<uint8_t>(), pk.size(0), pk.size(1), (int32_t)dim,
                                 (int32_t)bit_width, (int32_t)values, cache.data_ptr<uint8_t>(),
                                 t_cap, pos, cur_stream(cache)));
}

at::Tensor unpack_decode_layout(const at::Tensor& cache, int64_t dim, int64_t bit_width,
                                int64_t values, int64_t t0, int64_t n) {
  require_gpu(cache, "cache");
  c10::DeviceGuard g(cache.device());
  TORCH_CHECK(cache.scalar_type() == at::kByte && cache.is_contiguous() && cache.dim() == 3,
              "cache must be contiguous uint8 [streams, rows, width]");
  const int64_t t_cap = values ? cache.size(1) * 64 : cache.size(1);
  auto out = at::empty({cache.size(0), n, packed_width(bit_width, dim)}, cache.options());
  check_rc(tq_unpack_decode_layout(cache.data_ptr<uint8_t>(), cache.size(0), t_cap, t0, n,
                                   (int32_t)dim, (int32_t)bit_width, (int32_t)values,
                                   out.data_ptr<uint8_t>(), cur_stream(cache)));
  return out;
}

std::tuple<at::Tensor, at::Tensor> decode_attention_dl_lse(
    const at::Tensor& q, const at::Tensor& kpairs, const at::Tensor& knorms,
    const at::Tensor& vblocks, const at::Tensor& vnorms, const at::Tensor& seq_lens,
    const at::Tensor& kcentroids, const at::Tensor& vcentroids, const at::Tensor& krotation,
    const at::Tensor& vrotation, double scale, const c10::optional<at::Tensor>& seq_starts) {
  require_gpu(q, "q");
  TORCH_CHECK(q.dim() == 3, "q must be [B, Hq, d]");
  TORCH_CHECK(kpairs.dim() == 4 && vblocks.dim() == 4,
              "kpairs must be [B, Hkv, T, d/2] and vblocks [B, Hkv, T/64, 8 * vbits * d]");
  c10::DeviceGuard g(q.device());
  const auto dev = q.device();
  auto qq = floatc(q, dev);
  const int64_t B = qq.size(0), Hq = qq.size(1), d = qq.size(2);
  const int64_t Hkv = kpairs.size(1), Tc = kpairs.size(2);
  TORCH_CHECK(kpairs.scalar_type() == at::kByte && vblocks.scalar_type() == at::kByte,
              "kpairs/vblocks must be uint8");
  TORCH_CHECK(kpairs.is_contiguous() && vblocks.is_contiguous() && knorms.is_contiguous() &&
                  vnorms.is_contiguous(),
              "K/V and norms must be contiguous");
  TORCH_CHECK(kpairs.device() == dev && vblocks.device() == dev && knorms.device() == dev &&
                  vnorms.device() == dev,
              "K/V must be on the query's device");
  // value tiles of 8 * vbits * d bytes per 64 tokens: the width names the value code width
  const int64_t vbits = d > 0 ? vblocks.size(3) / (8 * d) : 0;
  TORCH_CHECK(kpairs.size(0) == B && kpairs.size(3) == d / 2 && vblocks.size(0) == B &&
                  vblocks.size(1) == Hkv && vblocks.size(2) * 64 == Tc &&
                  vblocks.size(3) == 8 * vbits * d && vbits >= 2 && vbits <= 4,
              "decode-layout K/V shape mismatch");
  const auto ndt = knorms.scalar_type();
  TORCH_CHECK((ndt == at::kFloat || ndt == at::kBFloat16 || ndt == at::kHalf) &&
                  vnorms.scalar_type() == ndt && knorms.numel() == B * Hkv * Tc &&
                  vnorms.numel() == B * Hkv * Tc,
              "norms must be [B, Hkv, T], both float32, bfloat16 or float16");
  auto sl = seq_lens.to(dev, at::kInt).contiguous();
  TORCH_CHECK(sl.numel() == B, "seq_lens must have B entries");
  at::Tensor ss;
  if (seq_starts.has_value() && seq_starts->defined()) {
    ss = seq_starts->to(dev, at::kInt).contiguous();
    TORCH_CHECK(ss.numel() == B, "seq_starts must have B entries");
  }
  auto kc = f32c(kcentroids, dev);
  auto vc = f32c(vcentroids, dev);
  auto Rk = f32c(krotation, dev);
  auto Rv = f32c(vrotation, dev);
  TORCH_CHECK(kc.numel() == 16 && vc.numel() == (1 << vbits),
              "decode layout: 16 key centroids and 2^vbits value centroids");
  auto out = at::empty({B, Hq, d}, qq.options());
  auto lse = at::empty({B, Hq}, qq.options().dtype(at::kFloat));
  if (B == 0) return {out, lse};
  auto ws = workspace(tq_decode_dl_workspace_bytes((int32_t)B, (int32_t)Hq, (int32_t)Hkv, Tc), dev);
  check_rc(tq_decode_attention_dl_window(
      qq.data_ptr(), to_tq(qq.scalar_type()), (int32_t)B, (int32_t)Hq, (int32_t)Hkv, (int32_t)d,
      kpairs.data_ptr<uint8_t>(), knorms.data_ptr(), vblocks.data_ptr<uint8_t>(),
      vnorms.data_ptr(), to_tq(ndt), Tc, sl.data_ptr<int32_t>(),
      ss.defined() ? ss.data_ptr<int32_t>() : nullptr, kc.data_ptr<float>(),
      vc.data_ptr<float>(), Rk.data_ptr<float>(), Rv.data_ptr<float>(), 4, (int32_t)vbits,
      (float)scale, out.data_ptr(), lse.data_ptr<float>(), ws.data_ptr(), ws.numel(),
      cur_stream(qq)));
  return {out, lse};
}

// Value widths of decode-layout value pools: tile_bytes = 64-token tiles of 512 * VB bytes
// (block_size >= 64) or 16-token sub-blocks of 128 * VB (block_size 16, 32); 0 if neither.
int value_tile_bits(int64_t tile_bytes, bool tiles64) {
  const int64_t unit = tiles64 ? 512 : 128;
  if (tile_bytes % unit != 0) return 0;
  const int64_t vb = tile_bytes / unit;
  return vb >= 2 && vb <= 4 ? (int)vb : 0;
}

// VB-bit value rows [n, hkv, 8 VB] + norms [n, hkv] into the value tiles
// vtile_pool [num_blocks, hkv, block_size/64, 512 VB] (block_size >= 64) or
// [num_blocks, hkv, block_size/16, 128 VB] (+ vnorm_pool [num_blocks, hkv, block_size]).
void paged_store_value_tiles(const at::Tensor& rows, const at::Tensor& norms,
                             const at::Tensor& slot_mapping, at::Tensor& vtile_pool,
                             at::Tensor& vnorm_pool) {
  require_gpu(vtile_pool, "vtile_pool");
  // 64-token tiles are 1024-2048 bytes, 16-token sub-blocks 256-512: the width tells them apart
  const bool tiles64 = vtile_pool.dim() == 4 && vtile_pool.size(3) >= 1024;
  const int vb = vtile_pool.dim() == 4 ? value_tile_bits(vtile_pool.size(3), tiles64) : 0;
  TORCH_CHECK(vtile_pool.dim() == 4 && vtile_pool.scalar_type() == at::kByte &&
                  vtile_pool.is_contiguous() && vb != 0,
              "vtile_pool must be contiguous uint8 [num_blocks, hkv, block_size/64, 512 VB] "
              "(block_size >= 64) or [num_blocks, hkv, block_size/16, 128 VB] (block_size 16, 32)");
  c10::DeviceGuard g(vtile_pool.device());
  const auto dev = vtile_pool.device();
  const int64_t nb = vtile_pool.size(0), hkv = vtile_pool.size(1);
  const int64_t bs = vtile_pool.size(2) * (tiles64 ? 64 : 16);
  TORCH_CHECK(tiles64 == (bs >= 64), "value tile shape does not match block_size");
  TORCH_CHECK(rows.dim() == 3 && rows.scalar_type() == at::kByte && rows.size(1) == hkv &&
                  rows.size(2) == 8 * vb,
              "rows must be uint8 [n, hkv, 8 * value bits] (bit planes of d = 64)");
  const int64_t n = rows.size(0);
  auto r = rows.to(dev).contiguous();
  auto nm = f32c(norms, dev);
  TORCH_CHECK(nm.numel() == n * hkv, "norms must be [n, hkv]");
  auto sm = slot_mapping.to(dev, at::kLong).contiguous();
  TORCH_CHECK(sm.numel() == n, "slot_mapping must have one entry per token");
  TORCH_CHECK(vnorm_pool.device() == dev && vnorm_pool.scalar_type() == at::kFloat &&
                  vnorm_pool.is_contiguous() && vnorm_pool.numel() == nb * hkv * bs,
              "vnorm_pool must be contiguous float32 [num_blocks, hkv, block_size]");
  check_rc(tq_paged_store_value_tiles(r.data_ptr<uint8_t>(), nm.data_ptr<float>(), n, (int32_t)hkv,
                                      sm.data_ptr<int64_t>(), vtile_pool.data_ptr<uint8_t>(),
                                      vnorm_pool.data_ptr<float>(), nb, (int32_t)bs, (int32_t)vb,
                                      cur_stream(vtile_pool)));
}

std::tuple<at::Tensor, at::Tensor> decode_attention_paged_dl(
    const at::Tensor& q, const at::Tensor& kpairs_pool, const at::Tensor& knorm_pool,
    const at::Tensor& vtile_pool, const at::Tensor& vnorm_pool, const at::Tensor& block_tables,
    const at::Tensor& seq_lens, const at::Tensor& kcentroids, const at::Tensor& vcentroids,
    const at::Tensor& krotation, const at::Tensor& vrotation, double scale) {
  require_gpu(q, "q");
  TORCH_CHECK(q.dim() == 3, "q must be [B, Hq, d]");
  TORCH_CHECK(kpairs_pool.dim() == 4 && vtile_pool.dim() == 4,
              "kpairs_pool must be [num_blocks, hkv, block_size, d/2] and vtile_pool "
              "[num_blocks, hkv, block_size/64, 16d]");
  c10::DeviceGuard g(q.device());
  const auto dev = q.device();
  auto qq = floatc(q, dev);
  const int64_t B = qq.size(0), Hq = qq.size(1), d = qq.size(2);
  const int64_t nb = kpairs_pool.size(0), Hkv = kpairs_pool.size(1), bs = kpairs_pool.size(2);
  for (const at::Tensor* t : {&kpairs_pool, &vtile_pool, &knorm_pool, &vnorm_pool})
    TORCH_CHECK(t->device() == dev && t->is_contiguous(), "pools must be contiguous on the query's device");
  TORCH_CHECK(kpairs_pool.scalar_type() == at::kByte && vtile_pool.scalar_type() == at::kByte,
              "pools must be uint8");
  const int64_t tile_tokens = bs >= 64 ? 64 : 16;
  const int vb = d == 64 ? value_tile_bits(vtile_pool.size(3), bs >= 64) : 0;
  TORCH_CHECK(kpairs_pool.size(3) == d / 2 && vtile_pool.size(0) == nb && vtile_pool.size(1) == Hkv &&
                  vtile_pool.size(2) * tile_tokens == bs && vb != 0,
              "decode-layout pool shapes mismatch: value tiles [num_blocks, hkv, block_size/64, "
              "512 VB] (block_size >= 64) or [num_blocks, hkv, block_size/16, 128 VB] (block_size "
              "16, 32), VB = 2-4 value bits, head_dim 64");
  TORCH_CHECK(knorm_pool.scalar_type() == at::kFloat && vnorm_pool.scalar_type() == at::kFloat &&
                  knorm_pool.numel() == nb * Hkv * bs && vnorm_pool.numel() == nb * Hkv * bs,
              "norm pools must be float32 [num_blocks, hkv, block_size]");
  auto bt = block_tables.to(dev, at::kInt).contiguous();
  TORCH_CHECK(bt.dim() == 2 && bt.size(0) == B, "block_tables must be [B, max_blocks]");
  auto sl = seq_lens.to(dev, at::kInt).contiguous();
  TORCH_CHECK(sl.numel() == B, "seq_lens must have B entries");
  auto kc = f32c(kcentroids, dev);
  auto vc = f32c(vcentroids, dev);
  auto Rk = f32c(krotation, dev);
  auto Rv = f32c(vrotation, dev);
  TORCH_CHECK(kc.numel() == 16 && vc.numel() == (1 << vb),
              "decode layout: 4-bit keys (16 centroids) and 2^VB value centroids for the pool's "
              "VB-bit value tiles");
  auto out = at::empty({B, Hq, d}, qq.options());
  auto lse = at::empty({B, Hq}, qq.options().dtype(at::kFloat));
  if (B == 0) return {out, lse};
  auto ws = workspace(tq_decode_dl_workspace_bytes((int32_t)B, (int32_t)Hq, (int32_t)Hkv,
                                                   bt.size(1) * bs),
                      dev);
  check_rc(tq_decode_attention_paged_dl(
      qq.data_ptr(), to_tq(qq.scalar_type()), (int32_t)B, (int32_t)Hq, (int32_t)Hkv, (int32_t)d,
      kpairs_pool.data_ptr<uint8_t>(), knorm_pool.data_ptr<float>(), vtile_pool.data_ptr<uint8_t>(),
      vnorm_pool.data_ptr<float>(), nb, (int32_t)bs, (int32_t)vb, bt.data_ptr<int32_t>(), (int32_t)bt.size(1),
      sl.data_ptr<int32_t>(), kc.data_ptr<float>(), vc.data_ptr<float>(), Rk.data_ptr<float>(),
      Rv.data_ptr<float>(), (float)scale, out.data_ptr(), lse.data_ptr<float>(), ws.data_ptr(),
      ws.numel(), cur_stream(qq)));
  return {out, lse};
}

at::Tensor prefill_attention_paged_dl(
    const at::Tensor& q, const at::Tensor& kpairs_pool, const at::Tensor& knorm_pool,
    const at::Tensor& vtile_pool, const at::Tensor& vnorm_pool, const at::Tensor& block_table,
    int64_t T, const at::Tensor& kcentroids, const at::Tensor& vcentroids,
    const at::Tensor& krotation, const at::Tensor& vrotation, double scale) {
  require_gpu(q, "q");
  TORCH_CHECK(q.dim() == 3, "q must be [n, Hq, d]");
  TORCH_CHECK(kpairs_pool.dim() == 4 && vtile_pool.dim() == 4,
              "kpairs_pool must be [num_blocks, hkv, block_size, d/2] and vtile_pool "
              "[num_blocks, hkv, block_size/64, 16d]");
  c10::DeviceGuard g(q.device());
  const auto dev = q.device();
  auto qq = floatc(q, dev);
  const int64_t n = qq.size(0), Hq = qq.size(1), d = qq.size(2);
  const int64_t nb = kpairs_pool.size(0), Hkv = kpairs_pool.size(1), bs = kpairs_pool.size(2);
  for (const at::Tensor* t : {&kpairs_pool, &vtile_pool, &knorm_pool, &vnorm_pool})
    TORCH_CHECK(t->device() == dev && t->is_contiguous(), "pools must be contiguous on the query's device");
  TORCH_CHECK(kpairs_pool.scalar_type() == at::kByte && vtile_pool.scalar_type() == at::kByte,
              "pools must be uint8");
  const int64_t tile_tokens = bs >= 64 ? 64 : 16;
  const int vb = d == 64 ? value_tile_bits(vtile_pool.size(3), bs >= 64) : 0;
  TORCH_CHECK(kpairs_pool.size(3) == d / 2 && vtile_pool.size(0) == nb && vtile_pool.size(1) == Hkv &&
                  vtile_pool.size(2) * tile_tokens == bs && vb != 0,
              "decode-layout pool shapes mismatch: value tiles [num_blocks, hkv, block_size/64, "
              "512 VB] (block_size >= 64) or [num_blocks, hkv, block_size/16, 128 VB] (block_size "
              "16, 32), VB = 2-4 value bits, head_dim 64");
  TORCH_CHECK(knorm_pool.scalar_type() == at::kFloat && vnorm_pool.scalar_type() == at::kFloat &&
                  knorm_pool.numel() == nb * Hkv * bs && vnorm_pool.numel() == nb * Hkv * bs,
              "norm pools must be float32 [num_blocks, hkv, block_size]");
  auto bt = block_table.to(dev, at::kInt).contiguous().view(-1);
  auto kc = f32c(kcentroids, dev);
  auto vc = f32c(vcentroids, dev);
  auto Rk = f32c(krotation, dev);
  auto Rv = f32c(vrotation, dev);
  TORCH_CHECK(kc.numel() == 16 && vc.numel() == (1 << vb),
              "decode layout: 4-bit keys (16 centroids) and 2^VB value centroids for the pool's "
              "VB-bit value tiles");
  TORCH_CHECK(Rk.numel() == d * d && Rv.numel() == d * d, "rotations must be [d, d]");
  auto out = at::empty({n, Hq, d}, qq.options().dtype(at::kFloat));
  check_rc(tq_prefill_attention_paged_dl(
      qq.data_ptr(), to_tq(qq.scalar_type()), (int32_t)n, T, (int32_t)Hq, (int32_t)Hkv, (int32_t)d,
      kpairs_pool.data_ptr<uint8_t>(), knorm_pool.data_ptr<float>(), vtile_pool.data_ptr<uint8_t>(),
      vnorm_pool.data_ptr<float>(), nb, (int32_t)bs, (int32_t)vb, bt.data_ptr<int32_t>(), (int32_t)bt.numel(),
      kc.data_ptr<float>(), vc.data_ptr<float>(), Rk.data_ptr<float>(), Rv.data_ptr<float>(),
      (float)scale, out.data_ptr<float>(), cur_stream(qq)));
  return out;
}

at::Tensor decode_attention_dl(const at::Tensor& q, const at::Tensor& kpairs,
                               const at::Tensor& knorms, const at::Tensor& vblocks,
                               const at::Tensor& vnorms, const at::Tensor& seq_lens,
                               const at::Tensor& kcentroids, const at::Tensor& vcentroids,
                               const at::Tensor& krotation, const at::Tensor& vrotation,
                               double scale) {
  return std::get<0>(decode_attention_dl_lse(q, kpairs, knorms, vblocks, vnorms, seq_lens,
                                             kcentroids, vcentroids, krotation, vrotation, scale,
                                             c10::nullopt));
}

// Appends s new tokens of every (batch row, KV head) to a decode-layout cache at token
// position pos: keys [B, H, s, d] and values quantized as quantize_mse_packed does
// (rounding in their own dtype), written into kp [B, H, t_cap, d/2] / vp [B, H, t_cap/64,
// 8 vbits d] and their fp32 norms into kn / vn [B, H, t_cap] -- the HF cache's append
// (hf_integration.py: quantize + pack + norm store for K and V) in one call.
void cache_append_dl(const at::Tensor& key, const at::Tensor& value, at::Tensor& kp, at::Tensor& kn,
                     at::Tensor& vp, at::Tensor& vn, int64_t pos, const at::Tensor& krotation,
                     const at::Tensor& kboundaries, const at::Tensor& vrotation,
                     const at::Tensor& vboundaries, int64_t kbits, int64_t vbits) {
  require_gpu(key, "key");
  TORCH_CHECK(key.dim() == 4 && value.sizes() == key.sizes(), "key / value must be [B, H, s, d]");
  c10::DeviceGuard g(key.device());
  const auto dev = key.device();
  const int64_t B = key.size(0), H = key.size(1), n = key.size(2), d = key.size(3);
  TORCH_CHECK(kp.dim() == 4 && vp.dim() == 4 && kp.size(0) == B && kp.size(1) == H &&
                  vp.size(0) == B && vp.size(1) == H && kp.is_contiguous() && vp.is_contiguous(),
              "kp / vp must be contiguous [B, H, ...] decode-layout caches");
  TORCH_CHECK(kn.dim() == 3 && vn.dim() == 3 &&
                  (kn.scalar_type() == at::kFloat || kn.scalar_type() == key.scalar_type()) &&
                  vn.scalar_type() == kn.scalar_type() && kn.size(0) == B && kn.size(1) == H &&
                  vn.sizes() == kn.sizes(),
              "kn / vn must be [B, H, t_cap], float32 or the key's dtype");
  TORCH_CHECK(pos >= 0 && pos + n <= kn.size(2), "tokens past the cache's capacity");
  if (B * H * n == 0) return;
  const auto kdt = key.scalar_type();
  if (n == 1 && kbits == 4 && vbits >= 2 && vbits <= 4 && (d == 64 || d == 128) &&
      (kdt == at::kBFloat16 || kdt == at::kHalf) && value.scalar_type() == kdt &&
      kn.is_contiguous() && vn.is_contiguous()) {
    // one token per stream (a decode step): quantized and stored in one launch
    auto k1 = key.to(dev).reshape({B * H, d}).contiguous();
    auto v1 = value.to(dev).reshape({B * H, d}).contiguous();
    auto Rk = f32c(krotation, dev), Rv = f32c(vrotation, dev);
    auto bk = f32c(kboundaries, dev), bv = f32c(vboundaries, dev);
    TORCH_CHECK(Rk.dim() == 2 && Rk.size(0) == d && Rk.size(1) == d && Rv.sizes() == Rk.sizes(),
                "rotations must be [d, d]");
    TORCH_CHECK(bk.numel() == 15 && bv.numel() == (1 << vbits) - 1,
                "boundaries length must be 2^bit_width - 1");
    TORCH_CHECK(kp.size(3) == d / 2 && vp.size(3) == 8 * vbits * d, "cache width mismatch");
    const int64_t t_cap = kp.size(2);
    TORCH_CHECK(vp.size(2) * 64 == t_cap && kn.size(2) == t_cap, "cache capacities differ");
    check_rc(tq_cache_append_dl(k1.data_ptr(), v1.data_ptr(), to_tq(kdt), B * H, (int32_t)d,
                                Rk.data_ptr<float>(), bk.data_ptr<float>(), Rv.data_ptr<float>(),
                                bv.data_ptr<float>(), (int32_t)vbits, kp.data_ptr<uint8_t>(),
                                kn.data_ptr(), vp.data_ptr<uint8_t>(), vn.data_ptr(),
                                to_tq(kn.scalar_type()), t_cap, pos, cur_stream(k1)));
    return;
  }
  for (int values = 0; values < 2; ++values) {
    const at::Tensor& t = values ? value : key;
    at::Tensor& cache = values ? vp : kp;
    at::Tensor& norm_cache = values ? vn : kn;
    const int64_t bits = values ? vbits : kbits;
    auto x = floatc(t.reshape({B * H * n, d}), dev);
    const tq_dtype dt = to_tq(x.scalar_type());
    auto R = f32c(values ? vrotation : krotation, dev);
    auto bnd = f32c(values ? vboundaries : kboundaries, dev);
    TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
    TORCH_CHECK(bits >= 1 && bits <= 4 && bnd.numel() == (1 << bits) - 1,
                "boundaries length must be 2^bit_width - 1");
    auto packed = at::empty({B * H * n, packed_width(bits, d)}, x.options().dtype(at::kByte));
    auto norms = at::empty({B * H * n}, x.options().dtype(at::kFloat));
    check_rc(tq_rotate_and_quantize(x.data_ptr(), dt, dt, B * H * n, (int32_t)d, R.data_ptr<float>(),
                                    bnd.data_ptr<float>(), (int32_t)bits, packed.data_ptr<uint8_t>(),
                                    norms.data_ptr<float>(), cur_stream(x)));
    const int64_t t_cap = values ? cache.size(2) * 64 : cache.size(2);
    TORCH_CHECK(cache.size(3) == (values ? 8 * bits * d : d / 2), "cache width mismatch");
    check_rc(tq_pack_decode_layout(packed.data_ptr<uint8_t>(), B * H, n, (int32_t)d, (int32_t)bits,
                                   values, cache.data_ptr<uint8_t>(), t_cap, pos, cur_stream(x)));
    norm_cache.narrow(2, pos, n).copy_(norms.view({B, H, n}));
  }
}

// The exact current token merged into a decode output by log-sum-exp
// (hf_integration.py:372-390): o [B, Hq, d] and lse [B, Hq] from a *_lse decode op, q
// [B, Hq, d], k_new / v_new [B, Hkv, d]; returns [B, Hq, d] in q.dtype.
at::Tensor decode_merge_token(const at::Tensor& o, const at::Tensor& lse, const at::Tensor& q,
                              const at::Tensor& k_new, const at::Tensor& v_new, double scale) {
  require_gpu(q, "q");
  TORCH_CHECK(q.dim() == 3 && o.dim() == 3 && k_new.dim() == 3 && v_new.dim() == 3,
              "q / o must be [B, Hq, d] and k_new / v_new [B, Hkv, d]");
  c10::DeviceGuard g(q.device());
  const auto dev = q.device();
  auto qq = floatc(q, dev);
  auto oo = o.to(dev, qq.scalar_type()).contiguous();
  auto ls = f32c(lse, dev);
  auto kn = floatc(k_new, dev);
  auto vn = v_new.to(dev, kn.scalar_type()).contiguous();
  const int64_t B = qq.size(0), Hq = qq.size(1), d = qq.size(2), Hkv = kn.size(1);
  TORCH_CHECK(oo.sizes() == qq.sizes(), "o must match q's shape");
  TORCH_CHECK(ls.numel() == B * Hq, "lse must be [B, Hq]");
  TORCH_CHECK(kn.size(0) == B && kn.size(2) == d && vn.sizes() == kn.sizes(),
              "k_new / v_new must be [B, Hkv, d]");
  auto out = at::empty_like(qq);
  check_rc(tq_decode_merge_token(oo.data_ptr(), ls.data_ptr<float>(), qq.data_ptr(),
                                 to_tq(qq.scalar_type()), kn.data_ptr(), vn.data_ptr(),
                                 to_tq(kn.scalar_type()), (int32_t)B, (int32_t)Hq, (int32_t)Hkv,
                                 (int32_t)d, (float)scale, out.data_ptr(), cur_stream(qq)));
  return out;
}

// One decode step of a decode-layout cache in one op: attention over the cached history
// (decode_attention_dl_lse) merged with the token being decoded, which attends to its own
// exact key and value (decode_merge_token) -- the same two launches, one dispatch.
at::Tensor decode_attention_dl_merged(
    const at::Tensor& q, const at::Tensor& kpairs, const at::Tensor& knorms,
    const at::Tensor& vblocks, const at::Tensor& vnorms, const at::Tensor& seq_lens,
    const at::Tensor& kcentroids, const at::Tensor& vcentroids, const at::Tensor& krotation,
    const at::Tensor& vrotation, double scale, const c10::optional<at::Tensor>& seq_starts,
    const at::Tensor& k_new, const at::Tensor& v_new) {
  auto ol = decode_attention_dl_lse(q, kpairs, knorms, vblocks, vnorms, seq_lens, kcentroids,
                                    vcentroids, krotation, vrotation, scale, seq_starts);
  return decode_merge_token(std::get<0>(ol), std::get<1>(ol), q, k_new, v_new, scale);
}

}  // namespace

TORCH_LIBRARY(turboquant, m) {
  // The reference's schemas (csrc/registration.cpp:84-99), verbatim.
  m.def("rotate_and_quantize(Tensor vectors, Tensor rotation, Tensor boundaries, int bit_width)"
        " -> (Tensor, Tensor)");
  m.def("attention_scores_packed(Tensor query, Tensor packed_keys, Tensor key_norms,"
        " Tensor centroids, Tensor rotation, int bit_width) -> Tensor");
  m.def("attention_values_packed(Tensor attn_weights, Tensor packed_values, Tensor value_norms,"
        " Tensor centroids, Tensor rotation_T, int bit_width) -> Tensor");
  m.def("pack_codes(Tensor codes, int bit_width) -> Tensor");
  m.def("unpack_codes(Tensor packed, int bit_width, int dim) -> Tensor");
  // Fused ops the reference's signatures cannot express.
  m.def("quantize_mse_packed(Tensor vectors, Tensor rotation, Tensor boundaries, int bit_width)"
        " -> (Tensor, Tensor)");
  m.def("quantize_prod_packed(Tensor vectors, Tensor rotation, Tensor boundaries,"
        " Tensor centroids, Tensor qjl, int bit_width) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("dequantize_mse_packed(Tensor packed, Tensor norms, Tensor centroids, Tensor rotation,"
        " int bit_width, int dim) -> Tensor");
  m.def("dequantize_prod_packed(Tensor mse_packed, Tensor signs, Tensor res_norms, Tensor norms,"
        " Tensor centroids, Tensor rotation, Tensor qjl, int bit_width, int dim) -> Tensor");
  m.def("ip_scan_topk(Tensor queries, Tensor packed, Tensor norms, Tensor centroids,"
        " Tensor rotation, int bit_width, int k) -> (Tensor, Tensor)");
  m.def("ip_scan_topk_pairs(Tensor queries, Tensor pairs, Tensor norms, Tensor centroids,"
        " Tensor rotation, int k) -> (Tensor, Tensor)");
  m.def("attention_scores_pairs(Tensor query, Tensor pairs, Tensor key_norms, Tensor centroids,"
        " Tensor rotation) -> Tensor");
  m.def("pack_pair_rows(Tensor packed, int bit_width, int dim) -> Tensor");
  m.def("unpack_pair_rows(Tensor rows, int bit_width, int dim) -> Tensor");
  m.def("ip_scan_topk_pair_rows(Tensor queries, Tensor rows, Tensor norms, Tensor centroids,"
        " Tensor rotation, int bit_width, int k) -> (Tensor, Tensor)");
  m.def("attention_scores_pair_rows(Tensor query, Tensor rows, Tensor key_norms, Tensor centroids,"
        " Tensor rotation, int bit_width) -> Tensor");
  // host-side tables (no tensor arguments: registered with catch-all kernels)
  m.def("core_rotation(int dim, int seed) -> Tensor", &core_rotation);
  m.def("core_codebook(int bits, int dim) -> (Tensor, Tensor)", &core_codebook);
  m.def("huffman_encode(Tensor codes, Tensor code_words, Tensor code_lens) -> Tensor", &huffman_encode);
  m.def("huffman_decode(Tensor data, int n_symbols, Tensor code_words, Tensor code_lens,"
        " Tensor symbols) -> Tensor", &huffman_decode);
  m.def("paged_store(Tensor rows, Tensor? norms, Tensor slot_mapping, Tensor(a!) pool,"
        " Tensor(b!)? norm_pool) -> ()");
  m.def("paged_gather(Tensor pool, Tensor? norm_pool, Tensor block_tables, Tensor seq_lens,"
        " int t_max) -> (Tensor, Tensor)");
  m.def("decode_attention_paged(Tensor q, Tensor kpool, Tensor knorm_pool, Tensor vpool,"
        " Tensor vnorm_pool, Tensor block_tables, Tensor seq_lens, Tensor kcentroids,"
        " Tensor vcentroids, Tensor krotation, Tensor vrotation, int kbits, int vbits,"
        " float scale) -> (Tensor, Tensor)");
  m.def("ip_scan_topk_prod(Tensor queries, Tensor mse_packed, Tensor signs, Tensor res_norms,"
        " Tensor norms, Tensor centroids, Tensor rotation, Tensor qjl, int bit_width, int k)"
        " -> (Tensor, Tensor)");
  m.def("attention_scores_prod(Tensor query, Tensor mse_packed, Tensor signs, Tensor res_norms,"
        " Tensor key_norms, Tensor centroids, Tensor rotation, Tensor qjl, int bit_width) -> Tensor");
  m.def("ip_scan_topk_prod_pair_rows(Tensor queries, Tensor mse_rows, Tensor signs, Tensor res_norms,"
        " Tensor norms, Tensor centroids, Tensor rotation, Tensor qjl, int bit_width, int k)"
        " -> (Tensor, Tensor)");
  m.def("attention_scores_prod_pair_rows(Tensor query, Tensor mse_rows, Tensor signs,"
        " Tensor res_norms, Tensor key_norms, Tensor centroids, Tensor rotation, Tensor qjl,"
        " int bit_width) -> Tensor");
  m.def("decode_attention_packed(Tensor q, Tensor kpacked, Tensor knorms, Tensor vpacked,"
        " Tensor vnorms, Tensor seq_lens, Tensor kcentroids, Tensor vcentroids,"
        " Tensor krotation, Tensor vrotation, int kbits, int vbits, float scale) -> Tensor");
  m.def("decode_attention_packed_lse(Tensor q, Tensor kpacked, Tensor knorms, Tensor vpacked,"
        " Tensor vnorms, Tensor seq_lens, Tensor kcentroids, Tensor vcentroids,"
        " Tensor krotation, Tensor vrotation, int kbits, int vbits, float scale)"
        " -> (Tensor, Tensor)");
  m.def("pack_decode_layout(Tensor packed, Tensor(a!) cache, int dim, int bit_width, int values,"
        " int pos) -> ()");
  m.def("unpack_decode_layout(Tensor cache, int dim, int bit_width, int values, int t0, int n)"
        " -> Tensor");
  m.def("decode_attention_dl(Tensor q, Tensor kpairs, Tensor knorms, Tensor vblocks,"
        " Tensor vnorms, Tensor seq_lens, Tensor kcentroids, Tensor vcentroids,"
        " Tensor krotation, Tensor vrotation, float scale) -> Tensor");
  m.def("decode_attention_dl_lse(Tensor q, Tensor kpairs, Tensor knorms, Tensor vblocks,"
        " Tensor vnorms, Tensor seq_lens, Tensor kcentroids, Tensor vcentroids,"
        " Tensor krotation, Tensor vrotation, float scale, Tensor? seq_starts=None)"
        " -> (Tensor, Tensor)");
  m.def("decode_merge_token(Tensor o, Tensor lse, Tensor q, Tensor k_new, Tensor v_new,"
        " float scale) -> Tensor");
  m.def("decode_attention_dl_merged(Tensor q, Tensor kpairs, Tensor knorms, Tensor vblocks,"
        " Tensor vnorms, Tensor seq_lens, Tensor kcentroids, Tensor vcentroids,"
        " Tensor krotation, Tensor vrotation, float scale, Tensor? seq_starts, Tensor k_new,"
        " Tensor v_new) -> Tensor");
  m.def("cache_append_dl(Tensor key, Tensor value, Tensor(a!) kp, Tensor(b!) kn, Tensor(c!) vp,"
        " Tensor(d!) vn, int pos, Tensor krotation, Tensor kboundaries, Tensor vrotation,"
        " Tensor vboundaries, int kbits, int vbits) -> ()");
  m.def("paged_store_value_tiles(Tensor rows, Tensor norms, Tensor slot_mapping,"
        " Tensor(a!) vtile_pool, Tensor(b!) vnorm_pool) -> ()");
  m.def("decode_attention_paged_dl(Tensor q, Tensor kpairs_pool, Tensor knorm_pool,"
        " Tensor vtile_pool, Tensor vnorm_pool, Tensor block_tables, Tensor seq_lens,"
        " Tensor kcentroids, Tensor vcentroids, Tensor krotation, Tensor vrotation,"
        " float scale) -> (Tensor, Tensor)");
  m.def("prefill_attention_paged_dl(Tensor q, Tensor kpairs_pool, Tensor knorm_pool,"
        " Tensor vtile_pool, Tensor vnorm_pool, Tensor block_table, int T,"
        " Tensor kcentroids, Tensor vcentroids, Tensor krotation, Tensor vrotation,"
        " float scale) -> Tensor");
}

TORCH_LIBRARY_IMPL(turboquant, CUDA, m) {
  m.impl("rotate_and_quantize", &rotate_and_quantize);
  m.impl("attention_scores_packed", &attention_scores_packed);
  m.impl("attention_values_packed", &attention_values_packed);
  m.impl("pack_codes", &pack_codes);
  m.impl("unpack_codes", &unpack_codes);
  m.impl("quantize_mse_packed", &quantize_mse_packed);
  m.impl("quantize_prod_packed", &quantize_prod_packed);
  m.impl("dequantize_mse_packed", &dequantize_mse_packed);
  m.impl("dequantize_prod_packed", &dequantize_prod_packed);
  m.impl("ip_scan_topk", &ip_scan_topk);
  m.impl("ip_scan_topk_pairs", &ip_scan_topk_pairs);
  m.impl("attention_scores_pairs", &attention_scores_pairs);
  m.impl("pack_pair_rows", &pack_pair_rows);
  m.impl("unpack_pair_rows", &unpack_pair_rows);
  m.impl("ip_scan_topk_pair_rows", &ip_scan_topk_pair_rows);
  m.impl("attention_scores_pair_rows", &attention_scores_pair_rows);
  m.impl("ip_scan_topk_prod", &ip_scan_topk_prod);
  m.impl("paged_store", &paged_store);
  m.impl("paged_gather", &paged_gather);
  m.impl("decode_attention_paged", &decode_attention_paged);
  m.impl("paged_store_value_tiles", &paged_store_value_tiles);
  m.impl("decode_attention_paged_dl", &decode_attention_paged_dl);
  m.impl("prefill_attention_paged_dl", &prefill_attention_paged_dl);
  m.impl("attention_scores_prod", &attention_scores_prod);
  m.impl("ip_scan_topk_prod_pair_rows", &ip_scan_topk_prod_pair_rows);
  m.impl("attention_scores_prod_pair_rows", &attention_scores_prod_pair_rows);
  m.impl("decode_attention_packed", &decode_attention_packed);
  m.impl("decode_attention_packed_lse", &decode_attention_packed_lse);
  m.impl("pack_decode_layout", &pack_decode_layout);
  m.impl("unpack_decode_layout", &unpack_decode_layout);
  m.impl("decode_attention_dl", &decode_attention_dl);
  m.impl("decode_attention_dl_lse", &decode_attention_dl_lse);
  m.impl("decode_merge_token", &decode_merge_token);
  m.impl("decode_attention_dl_merged", &decode_attention_dl_merged);
  m.impl("cache_append_dl", &cache_append_dl);
}
