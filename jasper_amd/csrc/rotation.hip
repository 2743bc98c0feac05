// rotation.hip -- row rotation x' = P^T x on the matrix cores.
//
// Reference: construct.cuh:1021-1112 (cublasGemmEx, fp16 in/out, fp32
// compute, stride padded_dim) and rotation.cuh:122-151 (rotate_data_vec,
// queries). Here one wave computes a 16-row tile with
// v_mfma_f32_16x16x32_f16: the MFMA's M side is 16 outputs i, its N side the
// 16 rows, K runs over the input coordinates. P is held transposed and
// K-padded (Pt[i][k] = P[k + i*dim], zero for i or k >= dim) so that both
// operands are 16-byte loads along K. Each lane ends with four consecutive
// outputs of one row per M tile, rounded to fp16 (round to nearest even).
#include "common.hpp"
#include "graph.hpp"
#include "rotation.hpp"

#include <cmath>
#include <cstdlib>
#include <random>
#include <stdexcept>
#include <vector>

namespace jasper_amd {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half8 as_half8(uint4 v) {
  half8 h;
  __builtin_memcpy(&h, &v, 16);
  return h;
}

// KS = number of 32-wide K steps held in registers (Kp = 32 * KS). With
// KS == 0 the K loop runs over kp32 steps and reloads operands per M tile.
template <int KS, bool PT_LDS>
__global__ __launch_bounds__(256) void rotate_mfma_kernel(const uint16_t* __restrict__ x, int64_t n, uint32_t dp_in,
                                                          const uint16_t* __restrict__ pt, uint32_t kp,
                                                          uint32_t dim, uint16_t* __restrict__ out,
                                                          uint32_t dp_out) {
  extern __shared__ uint4 pt_lds[];  // [mp][kp/8] when PT_LDS
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t mp = (dim + 15u) & ~15u;  // outputs padded to the M tile
  const uint32_t kc = kp / 8;               // uint4 chunks per Pt row
  const uint4* ptg = reinterpret_cast<const uint4*>(pt);
  if constexpr (PT_LDS) {
    for (uint32_t i = threadIdx.x; i < mp * kc; i += blockDim.x) pt_lds[i] = ptg[i];
    __syncthreads();
  }
  const uint4* ptv = PT_LDS ? pt_lds : ptg;
  const uint32_t col = lane & 15u;   // row of the tile (MFMA N index)
  const uint32_t kq = lane >> 4;     // which 8-wide K slice of the 32-wide step
  const uint32_t in_chunks = dp_in / 8;
  const int64_t tiles = (n + 15) / 16;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < tiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t row = tile * 16 + col;
    const bool row_ok = row < n;
    const uint4* xr = reinterpret_cast<const uint4*>(x) + (size_t)(row_ok ? row : 0) * in_chunks;
    uint16_t* orow = out + (size_t)(row_ok ? row : 0) * dp_out;
    if constexpr (KS > 0) {
      uint4 xf[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = (uint32_t)s * 4 + kq;
        xf[s] = (row_ok && c < in_chunks) ? xr[c] : make_uint4(0, 0, 0, 0);
      }
      for (uint32_t m0 = 0; m0 < mp; m0 += 16) {
        float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const uint4 pf = ptv[(size_t)(m0 + col) * kc + (uint32_t)s * 4 + kq];
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(pf), as_half8(xf[s]), acc, 0, 0, 0);
        }
        if (row_ok) {
          const uint32_t i0 = m0 + 4 * kq;
          if (i0 + 3 < dp_out) {
            uint2 w;
            w.x = (uint32_t)__half_as_ushort(__float2half_rn(acc[0])) |
                  ((uint32_t)__half_as_ushort(__float2half_rn(acc[1])) << 16);
            w.y = (uint32_t)__half_as_ushort(__float2half_rn(acc[2])) |
                  ((uint32_t)__half_as_ushort(__float2half_rn(acc[3])) << 16);
            *reinterpret_cast<uint2*>(orow + i0) = w;
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (i0 + j < dp_out) orow[i0 + j] = __half_as_ushort(__float2half_rn(acc[j]));
          }
        }
      }
    } else {
      const uint32_t ksteps = kp / 32;
      for (uint32_t m0 = 0; m0 < mp; m0 += 16) {
        float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t s = 0; s < ksteps; ++s) {
          const uint32_t c = s * 4 + kq;
          const uint4 xv = (row_ok && c < in_chunks) ? xr[c] : make_uint4(0, 0, 0, 0);
          const uint4 pf = ptv[(size_t)(m0 + col) * kc + c];
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(pf), as_half8(xv), acc, 0, 0, 0);
        }
        if (row_ok) {
          const uint32_t i0 = m0 + 4 * kq;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (i0 + j < dp_out) orow[i0 + j] = __half_as_ushort(__float2half_rn(acc[j]));
        }
      }
    }
  }
}

// The common case (P and four 16-row output tiles fit in LDS). P is staged
// once per block; after that each wave works alone: tiles gw, gw + stride,
// ... (gw its index in the grid), the next tile's rows loaded before the
// current tile's MFMAs. Each wave rounds its 16 x dim results to fp16 into
// its own LDS tile (row stride dp_out + 8 halves, 16-byte aligned, 2-way bank
// conflicts at most) and writes whole rows with 16-byte stores; a wave's LDS
// operations execute in order, so the tile needs no block barrier.
template <int KS, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void rotate_tile_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                                 uint32_t dp_in, const uint16_t* __restrict__ pt,
                                                                 uint32_t kp, uint32_t dim,
                                                                 uint16_t* __restrict__ out, uint32_t dp_out) {
  extern __shared__ uint4 lds4[];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t mp = (dim + 15u) & ~15u;
  const uint32_t kc = kp / 8;
  // Pt rows in LDS one chunk apart from 256-byte alignment: the 16 lanes that
  // read one K slice of 16 rows then hit 16 different bank groups (with rows
  // kc chunks apart, kc a multiple of 16 at d = 128, they all hit one; the
  // kernel ran 1.5x slower)
  const uint32_t kcl = kc + 1;
  const uint32_t ostride = dp_out + 8;  // halves
  uint4* pt_lds = lds4;
  uint16_t* otile = reinterpret_cast<uint16_t*>(lds4 + (size_t)mp * kcl) + (size_t)wave * 16 * ostride;
  const uint4* ptg = reinterpret_cast<const uint4*>(pt);
  for (uint32_t i = threadIdx.x; i < mp * kc; i += blockDim.x) pt_lds[(i / kc) * kcl + i % kc] = ptg[i];
  __syncthreads();
  const uint32_t col = lane & 15u, kq = lane >> 4;
  const uint32_t in_chunks = dp_in / 8, out_chunks = dp_out / 8;
  const int64_t tiles = (n + 15) / 16;
  const int64_t stride = (int64_t)gridDim.x * WAVES;
  auto load_tile = [&](int64_t tile, uint4 (&xf)[KS]) {
    const int64_t row = tile * 16 + col;
    const bool row_ok = tile < tiles && row < n;
    const uint4* xr = reinterpret_cast<const uint4*>(x) + (size_t)(row_ok ? row : 0) * in_chunks;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t c = (uint32_t)s * 4 + kq;
      xf[s] = (row_ok && c < in_chunks) ? xr[c] : make_uint4(0, 0, 0, 0);
    }
  };
  uint4 xf[KS];
  int64_t tile = (int64_t)blockIdx.x * WAVES + wave;
  load_tile(tile, xf);
  for (; tile < tiles; tile += stride) {
    uint4 xn[KS];
    load_tile(tile + stride, xn);
    for (uint32_t m0 = 0; m0 < mp; m0 += 16) {
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint4 pf = pt_lds[(size_t)(m0 + col) * kcl + (uint32_t)s * 4 + kq];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(pf), as_half8(xf[s]), acc, 0, 0, 0);
      }
      const uint32_t i0 = m0 + 4 * kq;
      if (i0 + 3 < dp_out) {
        // one 8-byte write of the lane's four outputs: a half wave's 32
        // lanes cover the 64 banks once
        uint2 w;
        w.x = (uint32_t)__half_as_ushort(__float2half_rn(acc[0])) |
              ((uint32_t)__half_as_ushort(__float2half_rn(acc[1])) << 16);
        w.y = (uint32_t)__half_as_ushort(__float2half_rn(acc[2])) |
              ((uint32_t)__half_as_ushort(__float2half_rn(acc[3])) << 16);
        *reinterpret_cast<uint2*>(otile + col * ostride + i0) = w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (i0 + j < dp_out) otile[col * ostride + i0 + j] = __half_as_ushort(__float2half_rn(acc[j]));
      }
    }
    lds_wave_sync();
    const int64_t row0 = tile * 16;
    for (uint32_t idx = lane; idx < 16 * out_chunks; idx += 64) {
      const uint32_t r = idx / out_chunks, c = idx % out_chunks;
      if (row0 + r < n) {
        // output columns in [mp, dp_out) never reach here (dp_out <= mp); zero-fill above dim came from
        // the zero rows of Pt
        reinterpret_cast<uint4*>(out + (size_t)(row0 + r) * dp_out)[c] =
            *reinterpret_cast<const uint4*>(otile + r * ostride + c * 8);
      }
    }
    lds_wave_sync();
#pragma unroll
    for (int s = 0; s < KS; ++s) xf[s] = xn[s];
  }
}

// Long rows (P too large for LDS, d > 192; config 4's d = 960): an
// LDS-tiled GEMM out[r][i] = sum_k Pt[i][k] x[r][k]. A block of 4 waves owns
// 128 outputs i x 128 rows r; each wave 64 x 64 as 2 x 2 tiles of
// v_mfma_f32_32x32x16_f16 (A = Pt: M = outputs, B = x: N = rows, both read
// along K). K runs in chunks of 64 staged through LDS, the next chunk's
// global loads in flight while the current one is on the matrix cores.
// Blocks are mapped so that the output-column blocks of one row block land
// on one XCD (work-groups are dealt to the 8 XCDs round-robin): they read the
// same x tile, which that XCD's L2 then serves.
constexpr uint32_t kRgTile = 128;  // outputs and rows per block
constexpr uint32_t kRgK = 64;      // K per LDS chunk
constexpr uint32_t kRgStride = kRgK / 8 + 1;  // uint4 per LDS row (one chunk of padding)

typedef float float16v_r __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void rotate_gemm_kernel(const uint16_t* __restrict__ x, int64_t n, uint32_t dp_in,
                                                          const uint16_t* __restrict__ pt, uint32_t kp,
                                                          uint32_t dim, uint16_t* __restrict__ out,
                                                          uint32_t dp_out, uint32_t col_blocks, int64_t row_blocks) {
  __shared__ uint4 sa[2][kRgTile * kRgStride];  // Pt chunk: [output][k]
  __shared__ uint4 sb[2][kRgTile * kRgStride];  // x chunk: [row][k]
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t mp = (dim + 15u) & ~15u;
  // block p runs on XCD p % 8; the col_blocks blocks of one row block are
  // p = xcd + 8 * (c + col_blocks * j) for c < col_blocks
  const int64_t p = blockIdx.x;
  const int64_t xcd = p & 7, q = p >> 3;
  const uint32_t cb = (uint32_t)(q % col_blocks);
  const int64_t rb = (q / col_blocks) * 8 + xcd;
  if (rb >= row_blocks) return;
  const uint32_t i_base = cb * kRgTile;
  const int64_t r_base = rb * kRgTile;
  const uint32_t kc = kp / 8, in_chunks = dp_in / 8;
  // staging: thread element e = tid + 256 j is (row e / 8, chunk e % 8)
  auto gload = [&](uint32_t k0, uint4 (&ga)[4], uint4 (&gb)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t e = tid + 256u * (uint32_t)j, rr = e >> 3, c = (k0 / 8) + (e & 7u);
      const uint32_t i = i_base + rr;
      ga[j] = (i < mp && c < kc) ? reinterpret_cast<const uint4*>(pt)[(size_t)i * kc + c] : make_uint4(0, 0, 0, 0);
      const int64_t r = r_base + rr;
      gb[j] = (r < n && c < in_chunks) ? reinterpret_cast<const uint4*>(x)[(size_t)r * in_chunks + c]
                                       : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](uint32_t buf, const uint4 (&ga)[4], const uint4 (&gb)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t e = tid + 256u * (uint32_t)j, rr = e >> 3, c = e & 7u;
      sa[buf][rr * kRgStride + c] = ga[j];
      sb[buf][rr * kRgStride + c] = gb[j];
    }
  };
  const uint32_t wm = wave & 1u, wn = wave >> 1;  // the wave's 64 outputs and 64 rows
  const uint32_t l32 = lane & 31u, lh = lane >> 5;
  float16v_r acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = float16v_r{};
  uint4 ga[4], gb[4];
  gload(0, ga, gb);
  sstore(0, ga, gb);
  __syncthreads();
  const uint32_t nchunk = (kp + kRgK - 1) / kRgK;
  for (uint32_t ch = 0; ch < nchunk; ++ch) {
    const uint32_t buf = ch & 1u;
    if (ch + 1 < nchunk) gload((ch + 1) * kRgK, ga, gb);
#pragma unroll
    for (uint32_t ks = 0; ks < kRgK / 16; ++ks) {
      // lane: row/output l32 of the tile, K slice 8 * lh of the 16-wide step
      const uint32_t c = ks * 2 + lh;
      uint4 fa[2], fb[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) fa[a] = sa[buf][(wm * 64 + 32 * a + l32) * kRgStride + c];
#pragma unroll
      for (int b = 0; b < 2; ++b) fb[b] = sb[buf][(wn * 64 + 32 * b + l32) * kRgStride + c];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_half8(fa[a]), as_half8(fb[b]), acc[a][b], 0, 0, 0);
    }
    if (ch + 1 < nchunk) {
      sstore(buf ^ 1u, ga, gb);
      __syncthreads();
    }
  }
  // acc[a][b][4g + e]: output i_base + 64 wm + 32 a + 8 g + 4 lh + e, row
  // r_base + 64 wn + 32 b + l32; four consecutive outputs per 8-byte store
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int64_t r = r_base + wn * 64 + 32 * b + l32;
    if (r >= n) continue;
    uint16_t* orow = out + (size_t)r * dp_out;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t i0 = i_base + wm * 64 + 32 * a + 8 * g + 4 * lh;
        const float v[4] = {acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
        if (i0 + 3 < mp && i0 + 3 < dp_out) {
          uint2 w;
          w.x = (uint32_t)__half_as_ushort(__float2half_rn(v[0])) |
                ((uint32_t)__half_as_ushort(__float2half_rn(v[1])) << 16);
          w.y = (uint32_t)__half_as_ushort(__float2half_rn(v[2])) |
                ((uint32_t)__half_as_ushort(__float2half_rn(v[3])) << 16);
          *reinterpret_cast<uint2*>(orow + i0) = w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (i0 + e < mp && i0 + e < dp_out) orow[i0 + e] = __half_as_ushort(__float2half_rn(v[e]));
        }
      }
    }
  }
}

// Zero the output pad columns [dim, dp_out) that the tiles do not cover.
__global__ void clear_pad_kernel(uint16_t* out, int64_t n, uint32_t mp, uint32_t dp_out) {
  const uint32_t w = dp_out - mp;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * (int64_t)w) return;
  out[(size_t)(t / w) * dp_out + mp + (uint32_t)(t % w)] = 0;
}

// Host restatement of householder_qr + set_rotation_matrix
// (rotation.cuh:28-111): the matrix must be the reference's, bit for bit, for
// graphs built with prerotation to be searched with the same rotation.
std::vector<float> rotation_matrix(uint32_t dd, uint64_t seed) {
  const int d = (int)dd;
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> N(0, 1);
  std::vector<float> A((size_t)d * d);
  for (int j = 0; j < d; j++)
    for (int i = 0; i < d; i++) A[(size_t)i + (size_t)j * d] = N(rng);
  std::vector<float> Q((size_t)d * d, 0.0f);
  for (int i = 0; i < d; i++) Q[(size_t)i + (size_t)i * d] = 1.0f;
  std::vector<float> v((size_t)d);
  for (int k = 0; k < d; k++) {
    float norm_sq = 0;
    for (int i = k; i < d; i++) {
      v[i] = A[(size_t)i + (size_t)k * d];
      norm_sq += v[i] * v[i];
    }
    const float norm = std::sqrt(norm_sq);
    if (norm < 1e-12f) continue;
    const float sign = (A[(size_t)k + (size_t)k * d] >= 0) ? 1.0f : -1.0f;
    v[k] += sign * norm;
    float v_norm_sq = 0;
    for (int i = k; i < d; i++) v_norm_sq += v[i] * v[i];
    const float tau = 2.0f / v_norm_sq;
    for (int j = k; j < d; j++) {
      float dot = 0;
      for (int i = k; i < d; i++) dot += v[i] * A[(size_t)i + (size_t)j * d];
      for (int i = k; i < d; i++) A[(size_t)i + (size_t)j * d] -= tau * v[i] * dot;
    }
    for (int j = 0; j < d; j++) {
      float dot = 0;
      for (int i = k; i < d; i++) dot += v[i] * Q[(size_t)i + (size_t)j * d];
      for (int i = k; i < d; i++) Q[(size_t)i + (size_t)j * d] -= tau * v[i] * dot;
    }
  }
  for (int i = 0; i < d; i++)
    if (A[(size_t)i + (size_t)i * d] < 0.0f)
      for (int j = 0; j < d; j++) Q[(size_t)j + (size_t)i * d] *= -1.0f;
  return Q;
}

RotationMatrix::~RotationMatrix() {
  if (pt) (void)hipFree(pt);
}

std::unique_ptr<RotationMatrix> make_rotation(const std::vector<float>& P, uint32_t dim) {
  auto r = std::make_unique<RotationMatrix>();
  r->dim = dim;
  r->kp = (dim + 31u) & ~31u;
  r->mp = (dim + 15u) & ~15u;
  std::vector<uint16_t> h((size_t)r->mp * r->kp, 0);
  for (uint32_t i = 0; i < dim; ++i)
    for (uint32_t k = 0; k < dim; ++k) h[(size_t)i * r->kp + k] = f2h_rn(P[(size_t)k + (size_t)i * dim]);
  hip_check(hipMalloc(&r->pt, h.size() * 2), "alloc rotation matrix");
  hip_check(hipMemcpy(r->pt, h.data(), h.size() * 2, hipMemcpyHostToDevice), "upload rotation matrix");
  return r;
}

void rotate_rows(const RotationMatrix& r, const void* x, int64_t n, uint32_t dp_in, void* out, uint32_t dp_out,
                 hipStream_t s) {
  if (n <= 0) return;
  if (dp_in % 8 != 0 || dp_out < r.dim) throw std::invalid_argument("rotate_rows: bad row strides");
  const uint32_t ks = r.kp / 32;
  const size_t lds = (size_t)r.mp * r.kp * 2;
  const bool use_lds = lds <= 64 * 1024;
  const int64_t tiles = (n + 15) / 16;
  const uint32_t grid = (uint32_t)std::min<int64_t>((tiles + 3) / 4, 8192);
  const uint16_t* xi = (const uint16_t*)x;
  uint16_t* o = (uint16_t*)out;
  auto launch = [&](auto kern, size_t shm) {
    if (shm > 64 * 1024)
      hip_check(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm),
                "rotation LDS");
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), shm, s, xi, n, dp_in, (const uint16_t*)r.pt, r.kp, r.dim, o,
                       dp_out);
  };
  // eight waves share one staged P where the LDS allows (1M x 128: 98 us
  // against 105 us with four; two blocks of 69.6 KB per CU)
  auto lds_for = [&](int w) { return (size_t)r.mp * (r.kp / 8 + 1) * 16 + (size_t)w * 16 * (dp_out + 8) * 2; };
  const int waves = lds_for(8) <= 96 * 1024 ? 8 : 4;
  const size_t tile_lds = lds_for(waves);
  if (tile_lds <= 96 * 1024 && dp_out <= r.mp && ks <= 6) {
    // whole rounds of resident blocks (LDS allows floor(160 KB / tile_lds)
    // per CU): every wave then walks the same number of tiles, give or take one
    static const int cus = [] {
      int dev = 0, c = 256;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
        c = 256;
      return c;
    }();
    const int64_t per_cu = std::max<int64_t>(1, (int64_t)(160 * 1024) / (int64_t)tile_lds);
    const uint32_t g2 = (uint32_t)std::min<int64_t>((tiles + waves - 1) / waves, per_cu * cus);
    auto go = [&](auto kern) {
      if (tile_lds > 64 * 1024)
        hip_check(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)tile_lds),
                  "rotation LDS");
      hipLaunchKernelGGL(kern, dim3(g2), dim3(64 * waves), tile_lds, s, xi, n, dp_in, (const uint16_t*)r.pt, r.kp,
                         r.dim, o, dp_out);
    };
    if (waves == 8) {
      switch (ks) {
        case 1: go(rotate_tile_kernel<1, 8>); break;
        case 2: go(rotate_tile_kernel<2, 8>); break;
        case 3: go(rotate_tile_kernel<3, 8>); break;
        case 4: go(rotate_tile_kernel<4, 8>); break;
        case 5: go(rotate_tile_kernel<5, 8>); break;
        default: go(rotate_tile_kernel<6, 8>); break;
      }
    } else {
      switch (ks) {
        case 1: go(rotate_tile_kernel<1, 4>); break;
        case 2: go(rotate_tile_kernel<2, 4>); break;
        case 3: go(rotate_tile_kernel<3, 4>); break;
        case 4: go(rotate_tile_kernel<4, 4>); break;
        case 5: go(rotate_tile_kernel<5, 4>); break;
        default: go(rotate_tile_kernel<6, 4>); break;
      }
    }
  } else if (ks > 6) {
    const uint32_t col_blocks = (r.mp + kRgTile - 1) / kRgTile;
    const int64_t row_blocks = (n + kRgTile - 1) / kRgTile;
    // grid: col_blocks blocks per row block, row blocks in groups of 8 (one per XCD)
    const int64_t blocks = ((row_blocks + 7) / 8) * 8 * col_blocks;
    hipLaunchKernelGGL(rotate_gemm_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, xi, n, dp_in,
                       (const uint16_t*)r.pt, r.kp, r.dim, o, dp_out, col_blocks, row_blocks);
  } else if (use_lds) {
    switch (ks) {
      case 1: launch(rotate_mfma_kernel<1, true>, lds); break;
      case 2: launch(rotate_mfma_kernel<2, true>, lds); break;
      case 3: launch(rotate_mfma_kernel<3, true>, lds); break;
      case 4: launch(rotate_mfma_kernel<4, true>, lds); break;
      case 5: launch(rotate_mfma_kernel<5, true>, lds); break;
      case 6: launch(rotate_mfma_kernel<6, true>, lds); break;
      default: launch(rotate_mfma_kernel<0, true>, lds); break;
    }
  } else {
    launch(rotate_mfma_kernel<0, false>, 0);
  }
  hip_check(hipGetLastError(), "launch rotate_mfma_kernel");
  if (dp_out > r.mp) {
    const int64_t total = n * (int64_t)(dp_out - r.mp);
    hipLaunchKernelGGL(clear_pad_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, o, n, r.mp, dp_out);
    hip_check(hipGetLastError(), "launch clear_pad_kernel");
  }
}

// Rotation as a stand-alone operator: x [n, dim] fp16 rows with stride
// x_stride elements (device or host memory) -> out [n, dim] with stride
// out_stride (device). Rows that are not 16-byte aligned multiples of 8
// elements go through padded staging buffers.
void rotate_rows_any(const RotationMatrix& r, const void* x, int64_t n, int64_t x_stride, void* out,
                     int64_t out_stride, hipStream_t s) {
  if (n <= 0) return;
  const uint32_t dp = (r.dim + 7u) & ~7u;
  const bool in_ok = x_stride % 8 == 0 && ((uintptr_t)x & 15u) == 0 && x_stride >= (int64_t)dp;
  const bool out_ok = out_stride % 8 == 0 && ((uintptr_t)out & 15u) == 0 && out_stride >= (int64_t)dp;
  hipPointerAttribute_t attr{};
  const bool in_dev = hipPointerGetAttributes(&attr, x) == hipSuccess && attr.type == hipMemoryTypeDevice;
  (void)hipGetLastError();
  void* xin = const_cast<void*>(x);
  void* xs = nullptr;
  void* os = nullptr;
  if (!in_ok || !in_dev) {
    hip_check(hipMallocAsync(&xs, (size_t)n * dp * 2, s), "alloc rotation input");
    hip_check(hipMemsetAsync(xs, 0, (size_t)n * dp * 2, s), "clear rotation input");
    hip_check(hipMemcpy2DAsync(xs, (size_t)dp * 2, x, (size_t)x_stride * 2, (size_t)r.dim * 2, (size_t)n,
                               hipMemcpyDefault, s),
              "stage rotation input");
    xin = xs;
  }
  const int64_t in_stride = xs ? dp : x_stride;
  if (out_ok) {
    rotate_rows(r, xin, n, (uint32_t)in_stride, out, (uint32_t)out_stride, s);
  } else {
    hip_check(hipMallocAsync(&os, (size_t)n * dp * 2, s), "alloc rotation output");
    rotate_rows(r, xin, n, (uint32_t)in_stride, os, dp, s);
    hip_check(hipMemcpy2DAsync(out, (size_t)out_stride * 2, os, (size_t)dp * 2, (size_t)r.dim * 2, (size_t)n,
                               hipMemcpyDefault, s),
              "copy rotation output");
  }
  if (xs) (void)hipFreeAsync(xs, s);
  if (os) (void)hipFreeAsync(os, s);
}

}  // namespace jasper_amd

extern "C" int64_t jasperx_rotate_rows(int64_t dim, int64_t seed, const void* x, int64_t n, int64_t x_stride,
                                       void* out, int64_t out_stride, void* stream);
