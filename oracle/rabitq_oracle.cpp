// rabitq_oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// CPU restatement of rabitq_quantize<1> (reference include/jasper/rabitq/
// quantize.cuh:144-383, layout.cuh:43-143) at one bit per dimension.
//
// At SIZE_PER_DIM = 1 the multi-bit code collapses: calc_multi_code clamps
// every value to 0 (quantize.cuh:156-160), so t_const (and the curand draw
// behind it) does not enter the result; the sign pass sets bit i = [r_i >= 0]
// (:166-175). Per vector, with r = P^T x - P c:
//   l2_sqr = sum r_i^2, l2_norm = sqrt(l2_sqr)
//   ip_norm = sum 0.5 * |r_i / l2_norm|, ip_norm_inv = 1 / ip_norm (NaN -> 1)
//   xucb_i = b_i - 0.5
//   ip_resi_xucb = sum r_i xucb_i (0 -> +inf), ip_cent_xucb = sum c'_i xucb_i,
//   ip_resi_cent = sum r_i c'_i          (c' = P c, the rotated centroid)
//   L2: f_add = l2_sqr + 2 l2_sqr ip_cent_xucb / ip_resi_xucb,
//       f_rescale = ip_norm_inv * -2 * l2_norm
//   IP: f_add = 1 - ip_resi_cent + l2_sqr ip_cent_xucb / ip_resi_xucb,
//       f_rescale = ip_norm_inv * -l2_norm
// Node = code bytes (ceil(dim/8) rounded up to 4, bits LSB-first) + f_add +
// f_rescale (fp32). The data goes through P^T (rotate_data_vec, CUBLAS_OP_T)
// but the centroid through P (rotate_single_data_vec, CUBLAS_OP_N,
// rotation.cuh:136-138 versus 169-171); both are kept as written.
//
// Sums run in index order in fp32 (the reference's cuBLAS and cg::reduce
// orders are unspecified); parity with the device is a tolerance.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <utility>
#include <vector>

#include <omp.h>

extern "C" {

uint32_t jo_rabitq_code_bytes(int dim) {
  const uint32_t raw = ((uint32_t)dim + 7u) / 8u;
  return (raw + 3u) / 4u * 4u;
}

// x: [n, dim] fp32 rows; P: [dim*dim] column-major; c: [dim] (may be null:
// zero centroid); metric 0 = L2, 1 = IP; out: [n, code_bytes + 8].
// rotated_out (optional): [n, dim] residuals r.
void jo_rabitq_quantize(const float* x, int64_t n, int dim, const float* P, const float* c, int metric, uint8_t* out,
                        float* resid_out, int nthreads) {
  const uint32_t cb = jo_rabitq_code_bytes(dim);
  const size_t node = cb + 8;
  std::vector<float> rc((size_t)dim, 0.0f);
  if (c) {
    for (int i = 0; i < dim; ++i) {
      float acc = 0.0f;
      for (int k = 0; k < dim; ++k) acc = std::fmaf(P[(size_t)i + (size_t)k * dim], c[k], acc);
      rc[(size_t)i] = acc;
    }
  }
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    std::vector<float> r((size_t)dim);
#pragma omp for schedule(static)
    for (int64_t v = 0; v < n; ++v) {
      const float* xv = x + (size_t)v * dim;
      for (int i = 0; i < dim; ++i) {
        float acc = 0.0f;
        for (int k = 0; k < dim; ++k) acc = std::fmaf(P[(size_t)k + (size_t)i * dim], xv[k], acc);
        r[(size_t)i] = acc - rc[(size_t)i];
      }
      float l2_sqr = 0.0f;
      for (int i = 0; i < dim; ++i) l2_sqr = std::fmaf(r[(size_t)i], r[(size_t)i], l2_sqr);
      const float l2_norm = std::sqrt(l2_sqr);
      float ip_norm = 0.0f;
      for (int i = 0; i < dim; ++i) ip_norm += 0.5f * std::fabs(r[(size_t)i] / l2_norm);
      float ip_norm_inv = 1.0f / ip_norm;
      if (std::isnan(ip_norm_inv)) ip_norm_inv = 1.0f;
      float s_rx = 0.0f, s_cx = 0.0f, s_rc = 0.0f;
      uint8_t* o = out + (size_t)v * node;
      std::memset(o, 0, cb);
      for (int i = 0; i < dim; ++i) {
        const bool bit = r[(size_t)i] >= 0.0f;
        const float xucb = bit ? 0.5f : -0.5f;
        s_rx = std::fmaf(r[(size_t)i], xucb, s_rx);
        s_cx = std::fmaf(rc[(size_t)i], xucb, s_cx);
        s_rc = std::fmaf(r[(size_t)i], rc[(size_t)i], s_rc);
        if (bit) o[i >> 3] |= (uint8_t)(1u << (i & 7));
      }
      if (s_rx == 0.0f) s_rx = std::numeric_limits<float>::infinity();
      float f_add, f_rescale;
      if (metric == 0) {
        f_add = l2_sqr + 2.0f * l2_sqr * s_cx / s_rx;
        f_rescale = ip_norm_inv * -2.0f * l2_norm;
      } else {
        f_add = 1.0f - s_rc + l2_sqr * s_cx / s_rx;
        f_rescale = ip_norm_inv * -l2_norm;
      }
      std::memcpy(o + cb, &f_add, 4);
      std::memcpy(o + cb + 4, &f_rescale, 4);
      if (resid_out) std::memcpy(resid_out + (size_t)v * dim, r.data(), (size_t)dim * 4);
    }
  }
}

// best_rescale_factor (reference quantize.cuh:22-82), the host routine behind
// get_const_scaling_factors (:89-131). For o = |x| of a unit vector and
// ex_bits bits it returns the scale t at which o_bar(t) = the per-dimension
// counters, stepped one at a time in increasing order of their step
// thresholds (o_bar_i + 1) / o_i, maximise <o_bar + 1/2, o> / |o_bar + 1/2|.
// Counters start at floor(t0 * o_i + 1e-5), t0 = t_end * tight[ex_bits],
// t_end = (2^ex_bits - 1 + 10) / max(o). Every dimension's first step is
// taken; a later one only while the counter is below 2^ex_bits - 1 and its
// threshold below t_end. Here all steps are listed first and swept in
// (threshold, dimension) order, which is the order the reference's min-heap
// pops them in. Sums are in double, as the reference's.
double jo_best_rescale_factor(const float* o, int64_t dim, int ex_bits) {
  static const double kTight[9] = {0, 0.15, 0.20, 0.52, 0.59, 0.71, 0.75, 0.77, 0.81};
  const int top = (1 << ex_bits) - 1;
  double mx = 0.0;
  for (int64_t i = 0; i < dim; ++i) mx = std::max(mx, (double)o[i]);
  const double t_end = (double)(top + 10) / mx;
  const double t0 = t_end * kTight[ex_bits];
  std::vector<int> bar((size_t)dim);
  double num = 0.0, den = 0.25 * (double)dim;
  for (int64_t i = 0; i < dim; ++i) {
    const int b = (int)(t0 * (double)o[i] + 1e-5);
    bar[(size_t)i] = b;
    den += (double)b * b + b;
    num += (b + 0.5) * (double)o[i];
  }
  // every step: the first one per dimension, then the ones its counter
  // takes while below top with a threshold below t_end
  std::vector<std::pair<double, int64_t>> steps;
  for (int64_t i = 0; i < dim; ++i) {
    int b = bar[(size_t)i] + 1;
    steps.emplace_back((double)b / (double)o[i], i);
    while (b < top) {
      const double t = (double)(b + 1) / (double)o[i];
      if (!(t < t_end)) break;
      steps.emplace_back(t, i);
      ++b;
    }
  }
  std::sort(steps.begin(), steps.end());
  double best_ip = 0.0, best_t = 0.0;
  for (const auto& st : steps) {
    const int b = ++bar[(size_t)st.second];
    den += 2.0 * b;
    num += (double)o[st.second];
    const double ip = num / std::sqrt(den);
    if (ip > best_ip) {
      best_ip = ip;
      best_t = st.first;
    }
  }
  return best_t;
}

// get_const_scaling_factors' host loop (quantize.cuh:124-130): the mean of
// best_rescale_factor over n rows of o = |x| (rows of length dim).
double jo_const_scaling_factor(const float* rows, int64_t n, int64_t dim, int ex_bits) {
  double sum = 0.0;
  for (int64_t r = 0; r < n; ++r) sum += jo_best_rescale_factor(rows + (size_t)r * dim, dim, ex_bits);
  return sum / (double)n;
}

}  // extern "C"
