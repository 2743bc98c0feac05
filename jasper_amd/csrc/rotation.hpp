// rotation.hpp -- the prerotation matrix and the MFMA row rotation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstring>
#include <memory>
#include <vector>

namespace jasper_amd {

// Host fp32 -> fp16 bits, round to nearest even.
inline uint16_t f2h_rn(float f) {
  const _Float16 h = (_Float16)f;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

// Random orthogonal matrix of set_rotation_matrix (rotation.cuh:28-111),
// column-major [dim * dim] fp32.
std::vector<float> rotation_matrix(uint32_t dim, uint64_t seed);

// P as the MFMA kernel reads it: Pt[i][k] = fp16(P[k + i*dim]), i padded to
// mp = roundup(dim, 16), k to kp = roundup(dim, 32), zero padded.
struct RotationMatrix {
  uint32_t dim = 0, kp = 0, mp = 0;
  void* pt = nullptr;  // device fp16 [mp][kp]
  ~RotationMatrix();
};

std::unique_ptr<RotationMatrix> make_rotation(const std::vector<float>& P, uint32_t dim);

// out[r][i] = fp16(sum_k P[k + i*dim] * x[r][k]) for i < dim (fp32
// accumulation on the matrix cores); x rows have stride dp_in (a multiple of
// 8, entries past dim zero), out rows stride dp_out >= dim. Columns of out in
// [dim, roundup(dim, 16)) that fit in dp_out are written as zero.
void rotate_rows(const RotationMatrix& r, const void* x, int64_t n, uint32_t dp_in, void* out, uint32_t dp_out,
                 hipStream_t s);

// Any row strides / alignment / host input (staged through padded buffers).
void rotate_rows_any(const RotationMatrix& r, const void* x, int64_t n, int64_t x_stride, void* out,
                     int64_t out_stride, hipStream_t s);

}  // namespace jasper_amd
