/*
 * tq_cpu.c -- C/OpenMP restatement of the reference's CPU kernels.
 *
 * TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py and a checker in
 * tests/.  The product never links it.
 *
 *   tqo_rotate_and_quantize  loop structure of rotate_and_quantize_cpu
 *                            (csrc/cpu/quant_cpu.cpp:44-118): per-vector omp dynamic,
 *                            scalar dot with R, linear searchsorted (val > bnd),
 *                            bit-set packing.  Like that function it multiplies by
 *                            1/norm instead of dividing.
 *   tqo_search_packed        LUT + min-heap top-k of _core.search_packed
 *                            (csrc/core/turboquant_core.cpp:407-514): per-query omp,
 *                            q_rot by sequential float mul/add, table[j][c] =
 *                            q_rot[j]*c[c], byte-wise plane decode, strict '>'
 *                            replacement (the lower index wins ties), results
 *                            sorted by (score desc, index asc), padded (-inf, -1).
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline int better(float sa, int64_t ia, float sb, int64_t ib) {
  return sa > sb || (sa == sb && ia < ib);
}

void tqo_rotate_and_quantize(const float* vec, int64_t n, int d, const float* rot,
                             const float* bnd, int bits, uint8_t* packed, float* norms) {
  const int nb = (1 << bits) - 1;
  const int bpp = (d + 7) / 8;
  const int P = bits * bpp;
  memset(packed, 0, (size_t)n * P);
#pragma omp parallel for schedule(dynamic)
  for (int64_t r = 0; r < n; ++r) {
    const float* v = vec + r * d;
    float ss = 0.f;
    for (int k = 0; k < d; ++k) ss += v[k] * v[k];
    const float nv = sqrtf(ss);
    norms[r] = nv;
    const float inv = (nv > 1e-10f) ? 1.0f / nv : 0.0f;
    uint8_t* row = packed + r * P;
    for (int j = 0; j < d; ++j) {
      float val = 0.f;
      for (int k = 0; k < d; ++k) val += (v[k] * inv) * rot[j * d + k];
      int code = 0;
      for (int b = 0; b < nb; ++b) {
        if (val > bnd[b]) code = b + 1;
        else break;
      }
      for (int i = 0; i < bits; ++i)
        if ((code >> i) & 1) row[i * bpp + (j >> 3)] |= (uint8_t)(1u << (7 - (j & 7)));
    }
  }
}

/* min-heap on (score, index) ordered by `better` reversed: root = worst kept entry */
static void heap_sift_down(float* hs, int64_t* hi, int n, int i) {
  for (;;) {
    int l = 2 * i + 1, r = l + 1, w = i;
    if (l < n && better(hs[w], hi[w], hs[l], hi[l])) w = l;
    if (r < n && better(hs[w], hi[w], hs[r], hi[r])) w = r;
    if (w == i) return;
    float ts = hs[i]; hs[i] = hs[w]; hs[w] = ts;
    int64_t ti = hi[i]; hi[i] = hi[w]; hi[w] = ti;
    i = w;
  }
}

static void heap_sift_up(float* hs, int64_t* hi, int i) {
  while (i > 0) {
    int p = (i - 1) / 2;
    if (!better(hs[p], hi[p], hs[i], hi[i])) return;
    float ts = hs[i]; hs[i] = hs[p]; hs[p] = ts;
    int64_t ti = hi[i]; hi[i] = hi[p]; hi[p] = ti;
    i = p;
  }
}

void tqo_search_packed(const float* queries, int Q, const uint8_t* packed, const float* norms,
                       int64_t N, int d, int bits, const float* rot, const float* cen, int k,
                       float* out_s, int64_t* out_i) {
  const int L = 1 << bits;
  const int bpp = (d + 7) / 8;
  const int P = bits * bpp;
#pragma omp parallel for schedule(dynamic, 1)
  for (int q = 0; q < Q; ++q) {
    const float* qv = queries + (size_t)q * d;
    float* qr = (float*)malloc(sizeof(float) * d);
    float* tab = (float*)malloc(sizeof(float) * d * L);
    float* hs = (float*)malloc(sizeof(float) * (k > 0 ? k : 1));
    int64_t* hi = (int64_t*)malloc(sizeof(int64_t) * (k > 0 ? k : 1));
    for (int j = 0; j < d; ++j) {
      float v = 0.f;
      for (int kk = 0; kk < d; ++kk) v += qv[kk] * rot[(size_t)j * d + kk];
      qr[j] = v;
    }
    for (int j = 0; j < d; ++j)
      for (int c = 0; c < L; ++c) tab[j * L + c] = qr[j] * cen[c];
    int hn = 0;
    for (int64_t i = 0; i < N; ++i) {
      const uint8_t* row = packed + i * P;
      float dot = 0.f;
      for (int kb = 0; kb < bpp; ++kb) {
        uint8_t pb[8];
        for (int p = 0; p < bits; ++p) pb[p] = row[p * bpp + kb];
        const int base = kb * 8;
        const int nd = d - base < 8 ? d - base : 8;
        for (int b = 0; b < nd; ++b) {
          int code = 0;
          for (int p = 0; p < bits; ++p) code |= ((pb[p] >> (7 - b)) & 1) << p;
          dot += tab[(base + b) * L + code];
        }
      }
      const float s = dot * norms[i];
      if (hn < k) {
        hs[hn] = s; hi[hn] = i;
        heap_sift_up(hs, hi, hn);
        ++hn;
      } else if (k > 0 && better(s, i, hs[0], hi[0])) {
        hs[0] = s; hi[0] = i;
        heap_sift_down(hs, hi, hn, 0);
      }
    }
    /* pop worst-first into the tail */
    float* os = out_s + (size_t)q * k;
    int64_t* oi = out_i + (size_t)q * k;
    for (int r = hn - 1; r >= 0; --r) {
      os[r] = hs[0]; oi[r] = hi[0];
      hs[0] = hs[hn - 1]; hi[0] = hi[hn - 1];
      --hn;
      heap_sift_down(hs, hi, hn, 0);
    }
    for (int r = (int)(N < k ? N : k); r < k; ++r) { os[r] = -INFINITY; oi[r] = -1; }
    free(qr); free(tab); free(hs); free(hi);
  }
}
