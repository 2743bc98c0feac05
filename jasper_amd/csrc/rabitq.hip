// rabitq.hip -- one-bit RaBitQ codes (reference rabitq/quantize.cuh:144-383,
// rabitq/layout.cuh:43-143).
//
// At one bit per dimension the quantizer reduces to a closed form (the
// multi-bit code is clamped to 0, so t_const does not matter): with
// r = P^T x - P c, bit_i = [r_i >= 0] and two fp32 factors per vector
// (f_add, f_rescale). The rotation P^T x is a GEMM; here it runs on the
// matrix cores in fp32 (v_mfma_f32_16x16x4_f32), one wave per 16 vectors:
// the MFMA's M side is 16 output coordinates, its N side 16 vectors, and the
// four K slots of each MFMA take coordinates k = 32b + 8q + s (q = lane/16,
// s = 0..7 across eight MFMAs), so each lane feeds the MFMA from one 32-byte
// (fp16: 16-byte) run of its vector. All residuals of a vector stay in the
// registers of the four lanes that hold it; the factor sums are reduced
// across those lanes with two xor shuffles.
//
// Node layout (rabitq_data_store<float>): code bytes = ceil(dim/8) rounded
// up to 4, bits LSB-first, then f_add and f_rescale.
#include "common.hpp"
#include "graph.hpp"
#include "rabitq.hpp"

#include <cmath>
#include <limits>
#include <stdexcept>

namespace jasper_amd {

typedef float float4v __attribute__((ext_vector_type(4)));

uint32_t rabitq_code_bytes(uint32_t dim) { return ((dim + 7u) / 8u + 3u) / 4u * 4u; }

// rc[i] = sum_k P[i + k*dim] c[k] (P times c: the centroid goes through
// CUBLAS_OP_N, rotation.cuh:160-176).
__global__ void rotate_centroid_kernel(const float* __restrict__ P, const float* __restrict__ c, uint32_t dim,
                                       float* __restrict__ rc) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim) return;
  float acc = 0.0f;
  for (uint32_t k = 0; k < dim; ++k) acc = __builtin_fmaf(P[(size_t)i + (size_t)k * dim], c[k], acc);
  rc[i] = acc;
}

// Pt[i][k] = P[k + i*dim] for i < dim, k < dim; zero padding to [mp][kp].
__global__ void transpose_pad_kernel(const float* __restrict__ P, uint32_t dim, uint32_t mp, uint32_t kp,
                                     float* __restrict__ pt) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)mp * kp) return;
  const uint32_t i = (uint32_t)(t / kp), k = (uint32_t)(t % kp);
  pt[t] = (i < dim && k < dim) ? P[(size_t)k + (size_t)i * dim] : 0.0f;
}

template <bool F16>
__device__ __forceinline__ void load_run8(const void* x, size_t row, uint32_t stride, uint32_t k, uint32_t dim,
                                          bool ok, float (&v)[8]) {
  if constexpr (F16) {
    const uint16_t* xr = (const uint16_t*)x + row * stride;
    if (ok && k + 8 <= stride) {
      const uint4 w = *reinterpret_cast<const uint4*>(xr + k);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = h2f_lo(ws[j]);
        v[2 * j + 1] = h2f_hi(ws[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k + j >= dim) v[j] = 0.0f;
  } else {
    const float* xr = (const float*)x + row * stride;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (ok && k + j < dim) ? xr[k + j] : 0.0f;
  }
}

// KT = number of 16-wide output tiles (mp = 16 * KT <= 256).
template <int KT, bool F16>
__global__ __launch_bounds__(256) void rabitq_kernel(const void* __restrict__ x, int64_t n, uint32_t stride,
                                                     uint32_t dim, const float* __restrict__ pt, uint32_t kp,
                                                     const float* __restrict__ rc, int metric,
                                                     uint8_t* __restrict__ out, uint32_t code_bytes) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t col = lane & 15u;  // vector within the tile
  const uint32_t q = lane >> 4;     // K slot / output quarter
  const uint32_t node_bytes = code_bytes + 8;
  const int64_t tiles = (n + 15) / 16;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < tiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t v = tile * 16 + col;
    const bool ok = v < n;
    float4v acc[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) acc[t] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t b = 0; b < kp; b += 32) {
      float xv[8];
      load_run8<F16>(x, (size_t)(ok ? v : 0), stride, b + 8 * q, dim, ok, xv);
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const float4* pr = reinterpret_cast<const float4*>(pt + (size_t)(16 * t + col) * kp + b + 8 * q);
        const float4 p0 = pr[0], p1 = pr[1];
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[s], xv[s], acc[t], 0, 0, 0);
      }
    }
    // lane holds r_i for vector v at i = 16t + 4q + j
    float l2 = 0.0f;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t i = 16u * t + 4u * q + j;
        const float r = i < dim ? acc[t][j] - rc[i] : 0.0f;
        acc[t][j] = r;
        l2 = __builtin_fmaf(r, r, l2);
      }
    l2 += __shfl_xor(l2, 16, 64);
    l2 += __shfl_xor(l2, 32, 64);
    const float l2_norm = sqrt_rn(l2);
    float ipn = 0.0f, s_rx = 0.0f, s_cx = 0.0f, s_rc = 0.0f;
    uint32_t nib[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      nib[t] = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t i = 16u * t + 4u * q + j;
        if (i < dim) {
          const float r = acc[t][j];
          const float c = rc[i];
          ipn += 0.5f * fabsf(div_rn(r, l2_norm));
          const bool bit = r >= 0.0f;
          const float xucb = bit ? 0.5f : -0.5f;
          s_rx = __builtin_fmaf(r, xucb, s_rx);
          s_cx = __builtin_fmaf(c, xucb, s_cx);
          s_rc = __builtin_fmaf(r, c, s_rc);
          nib[t] |= (bit ? 1u : 0u) << j;
        }
      }
    }
#pragma unroll
    for (int m = 16; m <= 32; m <<= 1) {
      ipn += __shfl_xor(ipn, m, 64);
      s_rx += __shfl_xor(s_rx, m, 64);
      s_cx += __shfl_xor(s_cx, m, 64);
      s_rc += __shfl_xor(s_rc, m, 64);
    }
    float ipn_inv = div_rn(1.0f, ipn);
    if (isnan(ipn_inv)) ipn_inv = 1.0f;
    if (s_rx == 0.0f) s_rx = __builtin_inff();
    float f_add, f_rescale;
    if (metric == kL2) {
      f_add = l2 + div_rn(2.0f * l2 * s_cx, s_rx);
      f_rescale = ipn_inv * -2.0f * l2_norm;
    } else {
      f_add = (1.0f - s_rc) + div_rn(l2 * s_cx, s_rx);
      f_rescale = ipn_inv * -l2_norm;
    }
    // byte 2t + (q >> 1) = nibble of q even | nibble of q odd << 4; the
    // shuffles run on every lane (lanes l and l ^ 16 hold the same vector)
    uint32_t bytes[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) bytes[t] = nib[t] | ((uint32_t)__shfl_xor((int)nib[t], 16, 64) << 4);
    if (ok) {
      uint8_t* node = out + (size_t)v * node_bytes;
      if ((q & 1u) == 0) {
#pragma unroll
        for (int t = 0; t < KT; ++t) node[2u * t + (q >> 1)] = (uint8_t)bytes[t];
      }
      if (q == 0) {
        for (uint32_t byte = 2u * KT; byte < code_bytes; ++byte) node[byte] = 0;
        *reinterpret_cast<float*>(node + code_bytes) = f_add;
        *reinterpret_cast<float*>(node + code_bytes + 4) = f_rescale;
      }
    }
  }
}

void rabitq_quantize(const void* x, bool f16, int64_t n, uint32_t dim, uint32_t stride, const float* P,
                     const float* centroid, int metric, void* out, hipStream_t s) {
  if (dim == 0 || dim > 256) throw std::invalid_argument("rabitq_quantize supports 1 <= dim <= 256");
  if (stride < dim) throw std::invalid_argument("row stride below dim");
  if (f16 && (stride % 8 != 0 || ((uintptr_t)x & 15u) != 0))
    throw std::invalid_argument("fp16 rows must be 16-byte aligned with a stride that is a multiple of 8");
  if (n <= 0) return;
  const uint32_t kp = (dim + 31u) & ~31u, mp = (dim + 15u) & ~15u, kt = mp / 16;
  float* pt = nullptr;
  float* rc = nullptr;
  hip_check(hipMallocAsync((void**)&pt, (size_t)mp * kp * 4, s), "alloc rabitq rotation");
  hip_check(hipMallocAsync((void**)&rc, (size_t)mp * 4, s), "alloc rotated centroid");
  hip_check(hipMemsetAsync(rc, 0, (size_t)mp * 4, s), "clear rotated centroid");
  const uint64_t total = (uint64_t)mp * kp;
  hipLaunchKernelGGL(transpose_pad_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, P, dim, mp, kp, pt);
  if (centroid)
    hipLaunchKernelGGL(rotate_centroid_kernel, dim3((dim + 63) / 64), dim3(64), 0, s, P, centroid, dim, rc);
  hip_check(hipGetLastError(), "launch rabitq set-up");
  const int64_t tiles = (n + 15) / 16;
  const uint32_t grid = (uint32_t)std::min<int64_t>((tiles + 3) / 4, 16384);
  const uint32_t cb = rabitq_code_bytes(dim);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, s, x, n, stride, dim, (const float*)pt, kp,
                       (const float*)rc, metric, (uint8_t*)out, cb);
  };
#define JA_RQ_CASE(K)                                        \
  case K:                                                    \
    if (f16) go(rabitq_kernel<K, true>);                     \
    else go(rabitq_kernel<K, false>);                        \
    break;
  switch (kt) {
    JA_RQ_CASE(1) JA_RQ_CASE(2) JA_RQ_CASE(3) JA_RQ_CASE(4) JA_RQ_CASE(5) JA_RQ_CASE(6) JA_RQ_CASE(7)
    JA_RQ_CASE(8) JA_RQ_CASE(9) JA_RQ_CASE(10) JA_RQ_CASE(11) JA_RQ_CASE(12) JA_RQ_CASE(13) JA_RQ_CASE(14)
    JA_RQ_CASE(15) JA_RQ_CASE(16)
    default: throw std::invalid_argument("rabitq_quantize: unsupported dim");
  }
#undef JA_RQ_CASE
  hip_check(hipGetLastError(), "launch rabitq_kernel");
  (void)hipFreeAsync(pt, s);
  (void)hipFreeAsync(rc, s);
}

}  // namespace jasper_amd
