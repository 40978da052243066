// cpu_ops.cpp -- the five reference schemas for CPU tensors (the CPU dispatch key).
//
// The reference registers CPU kernels for rotate_and_quantize, attention_scores_packed,
// attention_values_packed, pack_codes and unpack_codes (csrc/registration.cpp:106-112,
// kernels in csrc/cpu/quant_cpu.cpp).  These serve callers whose tensors live in host
// memory; tensors on a HIP device always take the gfx950 kernels (torch_ops.cpp), never
// these.  The arithmetic is the reference CPU kernels' own, element for element:
//   rotate_and_quantize  n = sqrt(sum_k v_k^2) (k ascending), u_k = v_k * (1 / n) (0 when
//                        n <= 1e-10), y_j = sum_k u_k R[j][k] (k ascending, separate
//                        multiply and add), code = number of leading boundaries below y_j
//                        (quant_cpu.cpp:44-118);
//   attention_scores     q_rot_j = sum_k R[j][k] q_k (k ascending), s = (sum_j q_rot_j
//                        c[code_j]) * n (j ascending) (quant_cpu.cpp:125-192);
//   attention_values     r_j = sum_t (w_t c[code_tj]) n_t (t ascending), out_k = sum_j r_j
//                        R_T[j][k] (j ascending) (quant_cpu.cpp:199-266);
//   pack / unpack        bit-plane rows: plane i holds bit i of every code, dim j at bit
//                        7 - j % 8 of byte j / 8 (quant_cpu.cpp:273-345).
// so a CPU caller gets the reference CPU path's bits.  The loops are arranged for the host
// instead of restated: each sum keeps its order, but the independent sums of a row run
// side by side (the j loop innermost, which the compiler vectorises), codes are unpacked
// once per row rather than once per (row, head), and rows are spread over ATen's
// intra-op thread pool.

#include <ATen/ATen.h>
#include <ATen/Parallel.h>
#include <torch/library.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <tuple>
#include <vector>

namespace {

#pragma clang fp contract(off)

int64_t planes_width(int64_t bits, int64_t d) { return bits * ((d + 7) / 8); }

void require_cpu(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.device().is_cpu(), "turboquant CPU kernel: ", name, " must be a CPU tensor");
}

at::Tensor f32_cpu(const at::Tensor& t) { return t.to(at::kCPU, at::kFloat).contiguous(); }

// Codes of one bit-plane row (`bits` planes of `bpp` bytes) into out[0 .. d).
inline void unpack_row(const uint8_t* row, int64_t d, int64_t bits, int64_t bpp, uint8_t* out) {
  for (int64_t j = 0; j < d; ++j) out[j] = 0;
  for (int64_t i = 0; i < bits; ++i) {
    const uint8_t* plane = row + i * bpp;
    for (int64_t j = 0; j < d; ++j) out[j] |= (uint8_t)(((plane[j >> 3] >> (7 - (j & 7))) & 1u) << i);
  }
}

// Bit-plane row of codes[0 .. d) (row zeroed first).
inline void pack_row(const uint8_t* codes, int64_t d, int64_t bits, int64_t bpp, uint8_t* row) {
  std::memset(row, 0, (size_t)(bits * bpp));
  for (int64_t j = 0; j < d; ++j) {
    const uint32_t c = codes[j];
    const uint8_t m = (uint8_t)(1u << (7 - (j & 7)));
    for (int64_t i = 0; i < bits; ++i)
      if ((c >> i) & 1u) row[i * bpp + (j >> 3)] |= m;
  }
}

std::tuple<at::Tensor, at::Tensor> rotate_and_quantize_cpu(const at::Tensor& vectors,
                                                           const at::Tensor& rotation,
                                                           const at::Tensor& boundaries,
                                                           int64_t bit_width) {
  require_cpu(vectors, "vectors");
  TORCH_CHECK(vectors.dim() == 2, "vectors must be [N, d]");
  auto x = f32_cpu(vectors);
  auto R = f32_cpu(rotation);
  auto bnd = f32_cpu(boundaries);
  const int64_t n = x.size(0), d = x.size(1);
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "Rotation matrix must be [d, d]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  TORCH_CHECK(bnd.numel() == (1 << bit_width) - 1, "boundaries length must be 2^bit_width - 1");
  const int64_t bpp = (d + 7) / 8, width = bit_width * bpp, nb = bnd.numel();
  auto packed = at::zeros({n, width}, x.options().dtype(at::kByte));
  auto norms = at::empty({n}, x.options());
  if (n == 0 || d == 0) return {packed, norms};
  const auto RT = R.t().contiguous();  // RT[k][j] = R[j][k]: row k of the sum's k-th terms
  const float* xp = x.data_ptr<float>();
  const float* rt = RT.data_ptr<float>();
  const float* bp = bnd.data_ptr<float>();
  uint8_t* pp = packed.data_ptr<uint8_t>();
  float* np_ = norms.data_ptr<float>();
  at::parallel_for(0, n, 16, [&](int64_t r0, int64_t r1) {
    std::vector<float> u((size_t)d), y((size_t)d);
    std::vector<uint8_t> code((size_t)d);
    for (int64_t r = r0; r < r1; ++r) {
      const float* v = xp + r * d;
      float ss = 0.f;
      for (int64_t k = 0; k < d; ++k) ss = ss + v[k] * v[k];
      const float nv = std::sqrt(ss);
      np_[r] = nv;
      const float inv = nv > 1e-10f ? 1.0f / nv : 0.0f;
      for (int64_t k = 0; k < d; ++k) u[k] = v[k] * inv;
      for (int64_t j = 0; j < d; ++j) y[j] = 0.f;
      for (int64_t k = 0; k < d; ++k) {  // y_j += u_k R[j][k], k ascending for every j
        const float uk = u[k];
        const float* rk = rt + k * d;
        float* yp = y.data();
        for (int64_t j = 0; j < d; ++j) yp[j] = yp[j] + uk * rk[j];
      }
      for (int64_t j = 0; j < d; ++j) {
        int c = 0;
        while (c < nb && y[j] > bp[c]) ++c;  // leading boundaries below y (NaN: none)
        code[j] = (uint8_t)c;
      }
      pack_row(code.data(), d, bit_width, bpp, pp + r * width);
    }
  });
  return {packed, norms};
}

at::Tensor attention_scores_packed_cpu(const at::Tensor& query, const at::Tensor& packed_keys,
                                       const at::Tensor& key_norms, const at::Tensor& centroids,
                                       const at::Tensor& rotation, int64_t bit_width) {
  require_cpu(query, "query");
  TORCH_CHECK(query.dim() == 3, "query must be [batch, heads, head_dim]");
  TORCH_CHECK(packed_keys.dim() == 2, "packed_keys must be [seq_len, packed_dim]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  auto q = f32_cpu(query);
  require_cpu(packed_keys, "packed_keys");
  auto pk = packed_keys.contiguous();
  auto kn = f32_cpu(key_norms);
  auto cen = f32_cpu(centroids);
  auto R = f32_cpu(rotation);
  const int64_t B = q.size(0), H = q.size(1), d = q.size(2), T = pk.size(0);
  TORCH_CHECK(pk.scalar_type() == at::kByte, "packed_keys must be uint8");
  TORCH_CHECK(pk.size(1) == planes_width(bit_width, d), "packed dim mismatch: expected ",
              planes_width(bit_width, d), " got ", pk.size(1));
  TORCH_CHECK(kn.numel() == T, "key_norms must have seq_len entries");
  TORCH_CHECK(cen.numel() == (1 << bit_width), "centroids length must be 2^bit_width");
  TORCH_CHECK(R.dim() == 2 && R.size(0) == d && R.size(1) == d, "rotation must be [d, d]");
  auto scores = at::empty({B, H, T}, q.options());
  const int64_t BH = B * H;
  if (BH == 0 || T == 0) return scores;
  const int64_t L = cen.numel(), bpp = (d + 7) / 8, width = bit_width * bpp;
  // Per (batch, head): the rotated query, then the table lut[j][c] = q_rot_j * c[c] -- the
  // very products the reference forms inside its sum.
  std::vector<float> lut((size_t)(BH * d * L));
  {
    const float* qp = q.data_ptr<float>();
    const float* rp = R.data_ptr<float>();
    const float* cp = cen.data_ptr<float>();
    at::parallel_for(0, BH, 1, [&](int64_t h0, int64_t h1) {
      for (int64_t h = h0; h < h1; ++h) {
        const float* qh = qp + h * d;
        for (int64_t j = 0; j < d; ++j) {
          float acc = 0.f;
          for (int64_t k = 0; k < d; ++k) acc = acc + rp[j * d + k] * qh[k];
          for (int64_t c = 0; c < L; ++c) lut[(size_t)((h * d + j) * L + c)] = acc * cp[c];
        }
      }
    });
  }
  const uint8_t* pkp = pk.data_ptr<uint8_t>();
  const float* knp = kn.data_ptr<float>();
  float* sp = scores.data_ptr<float>();
  constexpr int64_t kRows = 64;  // rows unpacked once and scored for every head
  at::parallel_for(0, (T + kRows - 1) / kRows, 1, [&](int64_t b0, int64_t b1) {
    std::vector<uint8_t> codes((size_t)(kRows * d));
    for (int64_t blk = b0; blk < b1; ++blk) {
      const int64_t t0 = blk * kRows, nt = std::min<int64_t>(kRows, T - t0);
      for (int64_t i = 0; i < nt; ++i) unpack_row(pkp + (t0 + i) * width, d, bit_width, bpp, codes.data() + i * d);
      for (int64_t h = 0; h < BH; ++h) {
        const float* lh = lut.data() + (size_t)(h * d * L);
        float* out = sp + h * T + t0;
        int64_t i = 0;
        for (; i + 4 <= nt; i += 4) {  // four rows' sums side by side, each in j order
          const uint8_t* c0 = codes.data() + i * d;
          float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
          for (int64_t j = 0; j < d; ++j) {
            const float* lj = lh + j * L;
            a0 = a0 + lj[c0[j]];
            a1 = a1 + lj[c0[d + j]];
            a2 = a2 + lj[c0[2 * d + j]];
            a3 = a3 + lj[c0[3 * d + j]];
          }
          out[i] = a0 * knp[t0 + i];
          out[i + 1] = a1 * knp[t0 + i + 1];
          out[i + 2] = a2 * knp[t0 + i + 2];
          out[i + 3] = a3 * knp[t0 + i + 3];
        }
        for (; i < nt; ++i) {
          const uint8_t* ci = codes.data() + i * d;
          float a = 0.f;
          for (int64_t j = 0; j < d; ++j) a = a + lh[j * L + ci[j]];
          out[i] = a * knp[t0 + i];
        }
      }
    }
  });
  return scores;
}

at::Tensor attention_values_packed_cpu(const at::Tensor& attn_weights, const at::Tensor& packed_values,
                                       const at::Tensor& value_norms, const at::Tensor& centroids,
                                       const at::Tensor& rotation_T, int64_t bit_width) {
  require_cpu(attn_weights, "attn_weights");
  TORCH_CHECK(attn_weights.dim() == 3, "attn_weights must be [batch, heads, seq_len]");
  TORCH_CHECK(packed_values.dim() == 2, "packed_values must be [seq_len, packed_dim]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 4, "bit_width must be 1-4");
  auto w = f32_cpu(attn_weights);
  require_cpu(packed_values, "packed_values");
  auto pv = packed_values.contiguous();
  auto vn = f32_cpu(value_norms);
  auto cen = f32_cpu(centroids);
  auto RT = f32_cpu(rotation_T);
  const int64_t B = w.size(0), H = w.size(1), T = w.size(2), d = RT.size(0);
  TORCH_CHECK(RT.dim() == 2 && RT.size(1) == d, "rotation_T must be [d, d]");
  TORCH_CHECK(pv.scalar_type() == at::kByte, "packed_values must be uint8");
  TORCH_CHECK(pv.size(0) == T, "packed_values must have seq_len rows");
  TORCH_CHECK(pv.size(1) == planes_width(bit_width, d), "packed dim mismatch: expected ",
              planes_width(bit_width, d), " got ", pv.size(1));
  TORCH_CHECK(vn.numel() == T, "value_norms must have seq_len entries");
  TORCH_CHECK(cen.numel() == (1 << bit_width), "centroids length must be 2^bit_width");
  auto out = at::empty({B, H, d}, w.options());
  const int64_t BH = B * H;
  if (BH == 0 || d == 0) return out;
  const int64_t bpp = (d + 7) / 8, width = bit_width * bpp;
  // every row's codes, unpacked once for all heads
  std::vector<uint8_t> codes((size_t)(T * d));
  const uint8_t* pvp = pv.data_ptr<uint8_t>();
  at::parallel_for(0, T, 256, [&](int64_t t0, int64_t t1) {
    for (int64_t t = t0; t < t1; ++t) unpack_row(pvp + t * width, d, bit_width, bpp, codes.data() + t * d);
  });
  const float* wp = w.data_ptr<float>();
  const float* vnp = vn.data_ptr<float>();
  const float* cp = cen.data_ptr<float>();
  const float* rtp = RT.data_ptr<float>();
  float* op = out.data_ptr<float>();
  at::parallel_for(0, BH, 1, [&](int64_t h0, int64_t h1) {
    std::vector<float> acc((size_t)d);
    for (int64_t h = h0; h < h1; ++h) {
      const float* wh = wp + h * T;
      for (int64_t j = 0; j < d; ++j) acc[j] = 0.f;
      for (int64_t t = 0; t < T; ++t) {  // r_j += (w_t c[code_tj]) n_t, t ascending for every j
        const float wt = wh[t], nt = vnp[t];
        const uint8_t* ct = codes.data() + t * d;
        float* ap = acc.data();
        for (int64_t j = 0; j < d; ++j) ap[j] = ap[j] + (wt * cp[ct[j]]) * nt;
      }
      float* oh = op + h * d;
      for (int64_t k = 0; k < d; ++k) oh[k] = 0.f;
      for (int64_t j = 0; j < d; ++j) {  // out_k += r_j R_T[j][k], j ascending for every k
        const float rj = acc[j];
        const float* row = rtp + j * d;
        for (int64_t k = 0; k < d; ++k) oh[k] = oh[k] + rj * row[k];
      }
    }
  });
  return out;
}

at::Tensor pack_codes_cpu(const at::Tensor& codes, int64_t bit_width) {
  require_cpu(codes, "codes");
  TORCH_CHECK(codes.scalar_type() == at::kByte, "codes must be uint8");
  TORCH_CHECK(codes.dim() == 2, "codes must be 2D [N, d]");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 8, "bit_width must be 1-8");
  auto c = codes.contiguous();
  const int64_t n = c.size(0), d = c.size(1), bpp = (d + 7) / 8, width = bit_width * bpp;
  auto packed = at::empty({n, width}, c.options());
  if (n == 0 || d == 0) return packed;
  const uint8_t* cp = c.data_ptr<uint8_t>();
  uint8_t* pp = packed.data_ptr<uint8_t>();
  at::parallel_for(0, n, 1024, [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) pack_row(cp + r * d, d, bit_width, bpp, pp + r * width);
  });
  return packed;
}

at::Tensor unpack_codes_cpu(const at::Tensor& packed, int64_t bit_width, int64_t dim) {
  require_cpu(packed, "packed");
  TORCH_CHECK(packed.scalar_type() == at::kByte, "packed must be uint8");
  TORCH_CHECK(packed.dim() == 2, "packed must be 2D");
  TORCH_CHECK(bit_width >= 1 && bit_width <= 8, "bit_width must be 1-8");
  TORCH_CHECK(dim >= 1, "dim must be >= 1");
  auto p = packed.contiguous();
  const int64_t bpp = (dim + 7) / 8, width = bit_width * bpp;
  TORCH_CHECK(p.size(1) == width, "packed dim mismatch: expected ", width, " got ", p.size(1));
  const int64_t n = p.size(0);
  auto codes = at::empty({n, dim}, p.options());
  if (n == 0) return codes;
  const uint8_t* pp = p.data_ptr<uint8_t>();
  uint8_t* cp = codes.data_ptr<uint8_t>();
  at::parallel_for(0, n, 1024, [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) unpack_row(pp + r * width, dim, bit_width, bpp, cp + r * dim);
  });
  return codes;
}

}  // namespace

TORCH_LIBRARY_IMPL(turboquant, CPU, m) {
  m.impl("rotate_and_quantize", &rotate_and_quantize_cpu);
  m.impl("attention_scores_packed", &attention_scores_packed_cpu);
  m.impl("attention_values_packed", &attention_values_packed_cpu);
  m.impl("pack_codes", &pack_codes_cpu);
  m.impl("unpack_codes", &unpack_codes_cpu);
}
