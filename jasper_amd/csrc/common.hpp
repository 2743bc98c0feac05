// common.hpp -- device primitives shared by the search and build kernels.
//
// Wave64-first building blocks for gfx950:
//   * 64-bit candidate keys that sort with one unsigned compare,
//   * quad (4-lane) distance evaluation that reproduces the reference
//     arithmetic bit for bit (reference include/jasper/distance/distance.cuh),
//   * wave-wide bitonic sort of 64 keys held one per lane,
//   * an LDS bitonic sort for up to 512 keys (one wave).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace jasper_amd {

constexpr uint32_t kInvalid32 = 0xFFFFFFFFu;
constexpr uint64_t kEmptyKey = ~0ull;

enum Metric : int { kL2 = 0, kIP = 1 };

// ----------------------------------------------------------------- keys --
// A candidate is one u64: [63:32] order-preserving image of the fp32
// distance, [31:1] the 31-bit vertex id, [0] the visited flag. Unsigned
// comparison of (key >> 1) is the reference order "distance ascending, then
// id ascending" (beam_search/device_kernels.cuh:132-151); -0.0 is folded onto
// +0.0 so that the image agrees with the float comparison.

__host__ __device__ __forceinline__ uint32_t dist_to_ord(float d) {
  uint32_t b = __float_as_uint(d + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__host__ __device__ __forceinline__ float ord_to_dist(uint32_t o) {
  uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
  return __uint_as_float(b);
}

__host__ __device__ __forceinline__ uint64_t make_key(float d, uint32_t id) {
  return ((uint64_t)dist_to_ord(d) << 32) | ((uint64_t)(id & 0x7FFFFFFFu) << 1);
}

__host__ __device__ __forceinline__ uint32_t key_id(uint64_t k) { return (uint32_t)(k >> 1) & 0x7FFFFFFFu; }
__host__ __device__ __forceinline__ float key_dist(uint64_t k) { return ord_to_dist((uint32_t)(k >> 32)); }
__host__ __device__ __forceinline__ bool key_visited(uint64_t k) { return (k & 1ull) != 0; }
__host__ __device__ __forceinline__ uint64_t key_rank(uint64_t k) { return k >> 1; }

// fp32 -> bf16 bits, round to nearest even (the reference stores edge
// distances with `(__nv_bfloat16)float`, index/graph.cuh:494).
__host__ __device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__host__ __device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ float h2f_lo(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w & 0xFFFFu))); }
__device__ __forceinline__ float h2f_hi(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w >> 16))); }

// Correctly rounded fp32 square root and quotient. The hardware v_sqrt_f32
// is not correctly rounded (and HIP's __fsqrt_rn maps to it), so both go
// through f64, whose LLVM lowering is correctly rounded; rounding the f64
// result to f32 is then exact-then-round (53 >= 2 * 24 + 2).
__device__ __forceinline__ float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }

// ----------------------------------------------------------- wave helpers --

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// number of set bits of m below this lane
__device__ __forceinline__ uint32_t mbcnt(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// LDS visibility between lanes of the one wave that owns a work-group.
__device__ __forceinline__ void wave_sync() { __syncthreads(); }

// LDS ordering for a work-group of one wave, without the workgroup fence of
// __syncthreads (which also waits for every outstanding global load): waits
// for this wave's LDS operations, which execute in order, and keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A value every lane holds alike, marked as such for the compiler (it is
// then kept in an SGPR and branches on it are scalar branches).
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// v with lane l replaced by s (v_writelane_b32); s and l are wave-uniform.
// The lane select goes through m0: an SGPR data operand and an SGPR lane
// select together exceed gfx9's one scalar operand per VALU instruction.
__device__ __forceinline__ uint32_t writelane(uint32_t v, uint32_t s, uint32_t l) {
  asm("v_writelane_b32 %0, %1, m0"
      : "+v"(v)
      : "s"(__builtin_amdgcn_readfirstlane(s)), "{m0}"(__builtin_amdgcn_readfirstlane(l)));
  return v;
}

// Per-lane select by a wave-uniform lane mask held in SGPRs: bit set -> b.
__device__ __forceinline__ uint32_t select_by_mask(uint32_t a, uint32_t b, uint64_t mask) {
  uint32_t r;
  asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
  return r;
}

// Value of lane (lane ^ J), without the LDS crossbar: xor 1 and 2 are DPP
// quad permutations, xor 4 a row half-mirror followed by a quad mirror,
// xor 8 a row rotation by 8, xor 16 and 32 v_permlane16/32_swap.
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  static_assert(J == 1 || J == 2 || J == 4 || J == 8 || J == 16 || J == 32, "xor mask");
  if constexpr (J == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // [1,0,3,2]
  else if constexpr (J == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // [2,3,0,1]
  else if constexpr (J == 4) {
    const int m8 = __builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);  // row_half_mirror: i <-> 7 - i
    return (uint32_t)__builtin_amdgcn_mov_dpp(m8, 0x1B, 0xF, 0xF, false);    // quad_perm [3,2,1,0]
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return select_by_mask(r[1], r[0], 0xFFFF0000FFFF0000ull);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return select_by_mask(r[1], r[0], 0xFFFFFFFF00000000ull);
  }
}

// Value of lane 63 - lane: a mirror within each row of 16 lanes (DPP)
// composed with xor 16 and xor 32.
__device__ __forceinline__ uint32_t reverse_lanes(uint32_t v) {
  const uint32_t m = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);  // row_mirror
  return xor_lane<32>(xor_lane<16>(m));
}

__device__ __forceinline__ uint64_t reverse_lanes64(uint64_t v) {
  return (uint64_t)reverse_lanes((uint32_t)v) | ((uint64_t)reverse_lanes((uint32_t)(v >> 32)) << 32);
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  return (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l) |
         ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l) << 32);
}

template <int J>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
  return (uint64_t)xor_lane<J>((uint32_t)v) | ((uint64_t)xor_lane<J>((uint32_t)(v >> 32)) << 32);
}

template <int J>
__device__ __forceinline__ float xor_lane_f(float v) {
  return __uint_as_float(xor_lane<J>(__float_as_uint(v)));
}

// Quad butterfly (offset 2, then 1): every lane of the quad gets
// (l0 + l2) + (l1 + l3), the combine order of cg::reduce over a 4-lane tile.
__device__ __forceinline__ float quad_sum(float v) {
  v = v + xor_lane_f<2>(v);
  v = v + xor_lane_f<1>(v);
  return v;
}

// Broadcast lane s of each quad to the whole quad (DPP quad_perm).
template <int S>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  constexpr int ctrl = S | (S << 2) | (S << 4) | (S << 6);
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, false);
}

// One compare-exchange stage of a bitonic sort: partner lane ^ J, blocks of
// K lanes alternate direction. Keep the min when (lower == up), else the
// max: take the partner exactly when (o < x) agrees with "keep min" (equal
// keys are interchangeable).
// Lanes that keep the minimum in stage (K, J): ((l & K) == 0) == ((l & J) == 0).
constexpr uint64_t bitonic_min_lanes(int K, int J) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if (((l & K) == 0) == ((l & J) == 0)) m |= 1ull << l;
  return m;
}

template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_stage(uint64_t x, uint32_t /*lane*/) {
  const uint64_t o = xor_lane64<J>(x);
  // take the partner where (o < x) agrees with "keep the minimum"
  const uint64_t take = ~(ballot(o < x) ^ bitonic_min_lanes(K, J));
  const uint32_t lo = select_by_mask((uint32_t)x, (uint32_t)o, take);
  const uint32_t hi = select_by_mask((uint32_t)(x >> 32), (uint32_t)(o >> 32), take);
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_merge_steps(uint64_t x, uint32_t lane) {
  x = bitonic_stage<K, J>(x, lane);
  if constexpr (J > 1) x = bitonic_merge_steps<K, J / 2>(x, lane);
  return x;
}

// Ascending bitonic sort of one key per lane over aligned blocks of W lanes
// (W a power of two <= 64); lanes of other blocks are sorted independently.
template <int W, int K = 2>
__device__ __forceinline__ uint64_t wave_bitonic_sort(uint64_t x) {
  x = bitonic_merge_steps<K, K / 2>(x, lane_id());
  if constexpr (K < W) x = wave_bitonic_sort<W, K * 2>(x);
  return x;
}

// Ascending bitonic sort of 128 keys held two per lane (element r * 64 +
// lane in register r). Stages with partner distance 64 compare a lane's two
// registers; the others exchange within each register as above.
constexpr uint64_t bitonic_min_lanes2(int K, int J, int r) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l) {
    const int i = r * 64 + l;
    if (((i & K) == 0) == ((i & J) == 0)) m |= 1ull << l;
  }
  return m;
}

template <int K, int J>
__device__ __forceinline__ void bitonic_stage128(uint64_t& x0, uint64_t& x1) {
  if constexpr (J == 64) {
    const uint64_t lo = x0 < x1 ? x0 : x1, hi = x0 < x1 ? x1 : x0;
    x0 = lo;
    x1 = hi;
  } else {
    const uint64_t o0 = xor_lane64<J>(x0), o1 = xor_lane64<J>(x1);
    const uint64_t t0 = ~(ballot(o0 < x0) ^ bitonic_min_lanes2(K, J, 0));
    const uint64_t t1 = ~(ballot(o1 < x1) ^ bitonic_min_lanes2(K, J, 1));
    x0 = (uint64_t)select_by_mask((uint32_t)x0, (uint32_t)o0, t0) |
         ((uint64_t)select_by_mask((uint32_t)(x0 >> 32), (uint32_t)(o0 >> 32), t0) << 32);
    x1 = (uint64_t)select_by_mask((uint32_t)x1, (uint32_t)o1, t1) |
         ((uint64_t)select_by_mask((uint32_t)(x1 >> 32), (uint32_t)(o1 >> 32), t1) << 32);
  }
  if constexpr (J > 1) bitonic_stage128<K, J / 2>(x0, x1);
}

template <int K = 2>
__device__ __forceinline__ void wave_bitonic_sort128(uint64_t& x0, uint64_t& x1) {
  bitonic_stage128<K, K / 2>(x0, x1);
  if constexpr (K < 128) wave_bitonic_sort128<K * 2>(x0, x1);
}

__device__ __forceinline__ uint64_t wave_sort_upto(uint64_t x, uint32_t n) {
  if (n <= 1) return x;
  if (n <= 2) return wave_bitonic_sort<2>(x);
  if (n <= 4) return wave_bitonic_sort<4>(x);
  if (n <= 8) return wave_bitonic_sort<8>(x);
  if (n <= 16) return wave_bitonic_sort<16>(x);
  if (n <= 32) return wave_bitonic_sort<32>(x);
  return wave_bitonic_sort<64>(x);
}

// Ascending bitonic sort of buf[0..N) in LDS by one wave (N power of two).
__device__ __forceinline__ void lds_bitonic_sort(uint64_t* buf, uint32_t N) {
  const uint32_t lane = lane_id();
  for (uint32_t k = 2; k <= N; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t t = lane; t < N / 2; t += 64) {
        // t-th compare-exchange pair of this stage
        const uint32_t lo = ((t & ~(j - 1)) << 1) | (t & (j - 1));
        const uint32_t hi = lo | j;
        const uint64_t a = buf[lo], b = buf[hi];
        const bool up = (lo & k) == 0;
        const bool swap = up ? (a > b) : (a < b);
        if (swap) { buf[lo] = b; buf[hi] = a; }
      }
      wave_sync();
    }
  }
}

// Number of entries of sorted keys[0..cnt) whose rank is below `r`
// (branch-free lower bound; `top` is a power of two >= cnt).
__device__ __forceinline__ uint32_t lds_lower_bound(const uint64_t* keys, uint32_t cnt, uint32_t top,
                                                    uint64_t r) {
  uint32_t lo = 0;
  for (uint32_t step = top; step > 0; step >>= 1) {
    const uint32_t probe = lo + step;
    if (probe <= cnt && key_rank(keys[probe - 1]) < r) lo = probe;
  }
  return lo;
}

__host__ __device__ __forceinline__ uint32_t pow2_ceil(uint32_t x) {
  uint32_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

// -------------------------------------------------------------- distances --
// Quad layout: the 4 lanes of a quad evaluate one distance. For L2, quad
// lane l owns the 16-byte chunks l, l+4, l+8, ... (distance.cuh:40-84) and
// accumulates fma(d, d, acc), d = f32(a) - f32(b), over the 8 halves of each
// chunk in order; the quad sum is (l0 + l2) + (l1 + l3). For IP, reference
// lane l owns the elements l, l+4, l+8, ... (distance.cuh:94-106); chunks
// are loaded as for L2 and every chunk is broadcast across the quad so that
// lane l can accumulate its two elements of each chunk in element order.

// Load the query fragment a quad lane needs into fp32 registers.
// src is a row of fp16 with at least nchunks*8 readable elements.
template <int CPL, int METRIC>
__device__ __forceinline__ void load_query_frag(const uint4* src, uint32_t ql, uint32_t nchunks,
                                                float (&qf)[CPL * 8]) {
  if constexpr (METRIC == kL2) {
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const uint32_t c = ql + 4u * (uint32_t)t;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (c < nchunks) x = src[c];
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        qf[t * 8 + 2 * k] = h2f_lo(w[k]);
        qf[t * 8 + 2 * k + 1] = h2f_hi(w[k]);
      }
    }
  } else {
    // IP: 2 elements per chunk for every chunk c < 4*CPL.
#pragma unroll
    for (int c = 0; c < 4 * CPL; ++c) {
      uint4 x = make_uint4(0, 0, 0, 0);
      if ((uint32_t)c < nchunks) x = src[c];
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
      const uint32_t e0 = ql, e1 = ql + 4u;
      const uint32_t w0 = w[e0 >> 1], w1 = w[e1 >> 1];
      qf[2 * c] = (e0 & 1u) ? h2f_hi(w0) : h2f_lo(w0);
      qf[2 * c + 1] = (e1 & 1u) ? h2f_hi(w1) : h2f_lo(w1);
    }
  }
}

// A quad lane's view of one vector row: its chunks ql, ql+4, ... held in
// registers (CPL = chunks per lane, rows of up to 32 chunks), or for longer
// rows (CPL = 0) the row's address, read chunk by chunk while scoring.
template <int CPL>
struct RowFrag {
  uint4 x[CPL];
};
template <>
struct RowFrag<0> {
  const uint4* row;
};

// Issue the chunk loads of one vector row for quad lane ql. Every lane loads
// (inactive lanes pass a valid row and ignore the result), and a chunk past
// the row's end re-reads chunk 0: the partial sums skip chunks >= their
// limit, so no masking or zero-fill is needed.
template <int CPL>
__device__ __forceinline__ void load_row_frag(const uint4* row, uint32_t ql, uint32_t nchunks, bool /*active*/,
                                              RowFrag<CPL>& f) {
  if constexpr (CPL == 0) {
    f.row = row;
  } else {
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const uint32_t c = ql + 4u * (uint32_t)t;
      f.x[t] = row[c < nchunks ? c : 0u];
    }
  }
}

// Partial (per quad lane) accumulation; returns the lane partial.
// L2: nlimit = number of chunks in the sum (dim / 8 of the reference call).
// IP: nlimit = number of elements in the sum (the reference `dim`).
template <int CPL, int METRIC>
__device__ __forceinline__ float quad_partial(const float (&qf)[CPL * 8], const RowFrag<CPL>& xf, uint32_t ql,
                                              uint32_t nlimit) {
  const uint4 (&x)[CPL] = xf.x;
  float acc = 0.0f;
  if constexpr (METRIC == kL2) {
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const uint32_t c = ql + 4u * (uint32_t)t;
      if (t < CPL - 1 || c < nlimit) {  // only the last slot can pass the row (CPL = ceil(chunks / 4))
        const uint32_t w[4] = {x[t].x, x[t].y, x[t].z, x[t].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float d0 = qf[t * 8 + 2 * k] - h2f_lo(w[k]);
          acc = __builtin_fmaf(d0, d0, acc);
          const float d1 = qf[t * 8 + 2 * k + 1] - h2f_hi(w[k]);
          acc = __builtin_fmaf(d1, d1, acc);
        }
      }
    }
  } else {
    // element order within reference lane ql: chunk 0 (ql, ql+4), chunk 1, ...
    // Rows and queries are zero-padded to whole chunks, so an element past
    // nlimit inside the last chunk adds fma(0, 0, acc) == acc: acc starts at
    // +0.0f and (+0) + (+-0) is +0 under round to nearest, so it is never
    // -0.0f. Only chunks past the row are left out; with CPL = ceil(chunks
    // / 4) those are among the last 4 slots, one uniform test each (a test
    // per element was one mask per element, which the compiler held in
    // scalar registers across the search loop and spilled).
    const uint32_t nck = (nlimit + 7u) >> 3;
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int c = 4 * t + s;  // chunk index, held by quad lane s in slot t
        if (c >= 4 * (CPL - 1) && (uint32_t)c >= nck) continue;
        uint32_t w[4];
        const uint32_t src[4] = {x[t].x, x[t].y, x[t].z, x[t].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (s == 0) w[k] = quad_bcast<0>(src[k]);
          else if (s == 1) w[k] = quad_bcast<1>(src[k]);
          else if (s == 2) w[k] = quad_bcast<2>(src[k]);
          else w[k] = quad_bcast<3>(src[k]);
        }
        const uint32_t e0 = ql, e1 = ql + 4u;
        const uint32_t w0 = (e0 >> 1) == 0 ? w[0] : w[1];
        const uint32_t w1 = (e1 >> 1) == 2 ? w[2] : w[3];
        const float v0 = (e0 & 1u) ? h2f_hi(w0) : h2f_lo(w0);
        const float v1 = (e1 & 1u) ? h2f_hi(w1) : h2f_lo(w1);
        acc = __builtin_fmaf(qf[2 * c], v0, acc);
        acc = __builtin_fmaf(qf[2 * c + 1], v1, acc);
      }
    }
  }
  return acc;
}

// f32(a) - f32(b) for the low (or high) fp16 halves of two words, rounded
// once: v_fma_mix_f32 converts the fp16 operands inside the instruction and
// computes a * 1.0 + (-b) exactly before rounding, which is the fp32
// subtraction of the converted values bit for bit, subnormals included.
__device__ __forceinline__ float mix_diff_lo(uint32_t a, uint32_t b) {
  float d;
  asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ float mix_diff_hi(uint32_t a, uint32_t b) {
  float d;
  asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  return d;
}

// L2 lane partial with the query fragment kept as fp16 chunks (the lane's
// chunks ql, ql+4, ... as load_row_frag reads them): the same accumulation
// order as quad_partial<CPL, kL2>, two VALU operations per element.
template <int CPL>
__device__ __forceinline__ float quad_partial_l2h(const RowFrag<CPL>& qf, const RowFrag<CPL>& xf, uint32_t ql,
                                                  uint32_t nlimit) {
  const uint4 (&qh)[CPL] = qf.x;
  const uint4 (&x)[CPL] = xf.x;
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < CPL; ++t) {
    const uint32_t c = ql + 4u * (uint32_t)t;
    if (t < CPL - 1 || c < nlimit) {  // only the last slot can pass the row (CPL = ceil(chunks / 4))
      const uint32_t qw[4] = {qh[t].x, qh[t].y, qh[t].z, qh[t].w};
      const uint32_t w[4] = {x[t].x, x[t].y, x[t].z, x[t].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float d0 = mix_diff_lo(qw[k], w[k]);
        acc = __builtin_fmaf(d0, d0, acc);
        const float d1 = mix_diff_hi(qw[k], w[k]);
        acc = __builtin_fmaf(d1, d1, acc);
      }
    }
  }
  return acc;
}

template <int METRIC>
__device__ __forceinline__ float quad_finish(float partial) {
  const float s = quad_sum(partial);
  return METRIC == kL2 ? s : -s;
}

// ------------------------------------------------- rows longer than 32 chunks
// Streamed forms of the lane partials: both rows are read from memory
// (global or LDS) chunk by chunk, in the same per-lane order as the register
// forms above, so the sums are identical bit for bit.

__device__ __forceinline__ void l2_chunk(const uint4& q, const uint4& x, float& acc) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float d0 = mix_diff_lo(qw[k], w[k]);
    acc = __builtin_fmaf(d0, d0, acc);
    const float d1 = mix_diff_hi(qw[k], w[k]);
    acc = __builtin_fmaf(d1, d1, acc);
  }
}

// L2 lane partial over chunks ql, ql+4, ... < nlimit.
__device__ __forceinline__ float stream_partial_l2(const uint4* a, const uint4* b, uint32_t ql, uint32_t nlimit) {
  float acc = 0.0f;
  uint32_t c = ql;
  for (; c + 28 < nlimit; c += 32) {  // 8 chunks per lane in flight
    uint4 qa[8], xb[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      qa[u] = a[c + 4u * (uint32_t)u];
      xb[u] = b[c + 4u * (uint32_t)u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) l2_chunk(qa[u], xb[u], acc);
  }
  for (; c < nlimit; c += 4) l2_chunk(a[c], b[c], acc);
  return acc;
}

// IP lane partial in the reference's element order (lane l: elements l,
// l+4, l+8, ... below nlimit): lane s of the quad loads chunk 4t+s of both
// rows and each chunk is broadcast across the quad. Every lane of a quad
// must call this with the same arguments.
__device__ __forceinline__ float stream_partial_ip(const uint4* a, const uint4* b, uint32_t ql, uint32_t nchunks,
                                                   uint32_t nlimit) {
  float acc = 0.0f;
  const uint32_t groups = (nchunks + 3u) / 4u;
  const uint32_t e0 = ql, e1 = ql + 4u;
  for (uint32_t t = 0; t < groups; ++t) {
    const uint32_t c = 4u * t + ql;
    uint4 xa = make_uint4(0, 0, 0, 0), xb = make_uint4(0, 0, 0, 0);
    if (c < nchunks) {
      xa = a[c];
      xb = b[c];
    }
    const uint32_t sa[4] = {xa.x, xa.y, xa.z, xa.w}, sb[4] = {xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint32_t wa[4], wb[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (s == 0) { wa[k] = quad_bcast<0>(sa[k]); wb[k] = quad_bcast<0>(sb[k]); }
        else if (s == 1) { wa[k] = quad_bcast<1>(sa[k]); wb[k] = quad_bcast<1>(sb[k]); }
        else if (s == 2) { wa[k] = quad_bcast<2>(sa[k]); wb[k] = quad_bcast<2>(sb[k]); }
        else { wa[k] = quad_bcast<3>(sa[k]); wb[k] = quad_bcast<3>(sb[k]); }
      }
      const uint32_t a0 = (e0 >> 1) == 0 ? wa[0] : wa[1], b0 = (e0 >> 1) == 0 ? wb[0] : wb[1];
      const uint32_t a1 = (e1 >> 1) == 2 ? wa[2] : wa[3], b1 = (e1 >> 1) == 2 ? wb[2] : wb[3];
      const float qa0 = (e0 & 1u) ? h2f_hi(a0) : h2f_lo(a0), xb0 = (e0 & 1u) ? h2f_hi(b0) : h2f_lo(b0);
      const float qa1 = (e1 & 1u) ? h2f_hi(a1) : h2f_lo(a1), xb1 = (e1 & 1u) ? h2f_hi(b1) : h2f_lo(b1);
      const uint32_t base = 8u * (4u * t + (uint32_t)s);
      if (base + e0 < nlimit) acc = __builtin_fmaf(qa0, xb0, acc);
      if (base + e1 < nlimit) acc = __builtin_fmaf(qa1, xb1, acc);
    }
  }
  return acc;
}

// ------------------------------------------------------ integer-valued data
// When every value is an integer and the values span at most 2,048 (see
// int_exact_l2), each fp16 difference a - b is exact, each square is an
// exact fp32 integer and every partial sum stays below 2^24: the reference's
// ordered fp32 sum then equals the exact integer whatever the order. The
// fast form takes the differences of two halves at once (v_pk_add_f16) and
// adds both squares with one v_dot2_f32_f16: one VALU per element instead of
// two, and the same bits as quad_partial_l2h on such data.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// a - b on two fp16 values at once (v_pk_add_f16)
__device__ __forceinline__ uint32_t sub_half2(uint32_t a, uint32_t b) {
  half2_t x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  const half2_t d = x - y;
  uint32_t r;
  __builtin_memcpy(&r, &d, 4);
  return r;
}

__device__ __forceinline__ float dot2_sqdiff(uint32_t a, uint32_t b, float acc) {
  half2_t x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  const half2_t d = x - y;
  return __builtin_amdgcn_fdot2(d, d, acc, false);
}

template <int CPL>
__device__ __forceinline__ float quad_partial_l2_int(const RowFrag<CPL>& qf, const RowFrag<CPL>& xf, uint32_t ql,
                                                     uint32_t nlimit) {
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < CPL; ++t) {
    const uint32_t c = ql + 4u * (uint32_t)t;
    if (t < CPL - 1 || c < nlimit) {  // only the last slot can pass the row (CPL = ceil(chunks / 4))
      acc = dot2_sqdiff(qf.x[t].x, xf.x[t].x, acc);
      acc = dot2_sqdiff(qf.x[t].y, xf.x[t].y, acc);
      acc = dot2_sqdiff(qf.x[t].z, xf.x[t].z, acc);
      acc = dot2_sqdiff(qf.x[t].w, xf.x[t].w, acc);
    }
  }
  return acc;
}

// ---- byte rows. A row of integers that spans at most 255 values can be
// held as bytes b = x - lo; an operand that qualifies for the packed-difference
// form is scored against the bytes instead of the fp16 row, reading half the
// bytes. Quad lane ql takes byte chunks ql and ql + 4 (16 values each). The
// left operand (a query) is held shifted, q' = q - lo + 1024,
// and a byte b becomes the fp16 value 1024 + b by placing 0x64 above it
// (one v_perm_b32 per two values), so q' - (1024 + b) = q - x: the same
// exact fp16 difference, and with it the same exact sum of squares, as the
// fp16 rows give.
struct RowBytes {
  uint4 x[2];
};

// q: byte chunk ql in q[0..1], byte chunk ql + 4 in q[2..3] (fp16 q')
__device__ __forceinline__ void load_query_bytes(const uint4* qrow, uint32_t nb8, uint32_t qsh2, uint32_t ql,
                                                 uint4 (&q)[4]) {
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint32_t c = ql + 4u * u;
    const uint32_t c0 = c < nb8 ? 2u * c : 0u;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      uint4 w = qrow[c0 + h];
      w.x = sub_half2(w.x, qsh2);
      w.y = sub_half2(w.y, qsh2);
      w.z = sub_half2(w.z, qsh2);
      w.w = sub_half2(w.w, qsh2);
      q[2 * u + h] = w;
    }
  }
}

__device__ __forceinline__ void load_row_bytes(const uint4* vecs8, uint32_t nb8, uint32_t v, uint32_t ql,
                                               RowBytes& r) {
  const uint4* row = vecs8 + (size_t)v * nb8;
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint32_t c = ql + 4u * u;
    r.x[u] = row[c < nb8 ? c : 0u];
  }
}

// bytes b0..b3 of w to fp16 pairs (1024 + b0, 1024 + b1) and (1024 + b2, 1024 + b3)
__device__ __forceinline__ uint32_t bytes_lo_pair(uint32_t w) { return __builtin_amdgcn_perm(w, 0x64646464u, 0x00050004u); }
__device__ __forceinline__ uint32_t bytes_hi_pair(uint32_t w) { return __builtin_amdgcn_perm(w, 0x64646464u, 0x00070006u); }

__device__ __forceinline__ float score_bytes(uint32_t nb8, const uint4 (&q)[4], const RowBytes& r, uint32_t ql) {
  float acc = 0.0f;
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    if (ql + 4u * u < nb8) {
      const uint4 b = r.x[u];
      const uint4 q0 = q[2 * u], q1 = q[2 * u + 1];
      acc = dot2_sqdiff(q0.x, bytes_lo_pair(b.x), acc);
      acc = dot2_sqdiff(q0.y, bytes_hi_pair(b.x), acc);
      acc = dot2_sqdiff(q0.z, bytes_lo_pair(b.y), acc);
      acc = dot2_sqdiff(q0.w, bytes_hi_pair(b.y), acc);
      acc = dot2_sqdiff(q1.x, bytes_lo_pair(b.z), acc);
      acc = dot2_sqdiff(q1.y, bytes_hi_pair(b.z), acc);
      acc = dot2_sqdiff(q1.z, bytes_lo_pair(b.w), acc);
      acc = dot2_sqdiff(q1.w, bytes_hi_pair(b.w), acc);
    }
  }
  return quad_finish<kL2>(acc);
}

// A left operand whose own values also lie in [lo, lo + 255] (every half of
// its q' words is 0x64bb) becomes bytes b_q = q - lo in the byte rows'
// layout (qb[0]: byte chunk ql, qb[1]: byte chunk ql + 4), with qn the sum
// of b_q^2 over the lane's values. Then per lane sum (q - x)^2 = qn + sum
// b_x^2 - 2 sum b_q b_x, all exact in u32 with v_dot4_u32_u8 (four values
// per instruction, against one v_perm, v_pk_add_f16 and v_dot2 per two values
// of score_bytes), and the quad sum of these integers (each below 2^24, their
// total too) is the same float. Returns whether the operand qualifies
// (wave-uniform).
__device__ __forceinline__ bool left_bytes_u8(uint32_t nb8, const uint4 (&q)[4], uint32_t ql, uint4 (&qb)[2],
                                              uint32_t& qn) {
  bool ok = true;
  qn = 0;
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint4 q0 = q[2 * u], q1 = q[2 * u + 1];
    qb[u] = make_uint4(__builtin_amdgcn_perm(q0.y, q0.x, 0x06040200u), __builtin_amdgcn_perm(q0.w, q0.z, 0x06040200u),
                       __builtin_amdgcn_perm(q1.y, q1.x, 0x06040200u), __builtin_amdgcn_perm(q1.w, q1.z, 0x06040200u));
    if (ql + 4u * u < nb8) {
      // every half's high byte is 0x64: the and of the words has all of
      // 0x64's bits there and their or no other bit
      const uint32_t wa = q0.x & q0.y & q0.z & q0.w & q1.x & q1.y & q1.z & q1.w;
      const uint32_t wo = q0.x | q0.y | q0.z | q0.w | q1.x | q1.y | q1.z | q1.w;
      ok = ok && (wa & 0xFF00FF00u) == 0x64006400u && (wo & 0xFF00FF00u) == 0x64006400u;
      qn = __builtin_amdgcn_udot4(qb[u].x, qb[u].x, qn, false);
      qn = __builtin_amdgcn_udot4(qb[u].y, qb[u].y, qn, false);
      qn = __builtin_amdgcn_udot4(qb[u].z, qb[u].z, qn, false);
      qn = __builtin_amdgcn_udot4(qb[u].w, qb[u].w, qn, false);
    }
  }
  return ballot(!ok) == 0;
}

__device__ __forceinline__ float score_bytes_u8(uint32_t nb8, const uint4& qb0, const uint4& qb1, uint32_t qn,
                                                const RowBytes& r, uint32_t ql) {
  uint32_t qx = 0, xx = 0;
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    if (ql + 4u * u < nb8) {
      const uint4 b = r.x[u];
      const uint4 q = u == 0 ? qb0 : qb1;
      qx = __builtin_amdgcn_udot4(q.x, b.x, qx, false);
      qx = __builtin_amdgcn_udot4(q.y, b.y, qx, false);
      qx = __builtin_amdgcn_udot4(q.z, b.z, qx, false);
      qx = __builtin_amdgcn_udot4(q.w, b.w, qx, false);
      xx = __builtin_amdgcn_udot4(b.x, b.x, xx, false);
      xx = __builtin_amdgcn_udot4(b.y, b.y, xx, false);
      xx = __builtin_amdgcn_udot4(b.z, b.z, xx, false);
      xx = __builtin_amdgcn_udot4(b.w, b.w, xx, false);
    }
  }
  return quad_finish<kL2>((float)(qn + xx - 2u * qx));  // the lane's exact sum of (q - x)^2
}

// ----------------------------------------------------------- left operands
// The operand a row is compared against (a query, or a pruning candidate):
// L2 keeps its fp16 chunks (v_fma_mix converts them), IP its fp32 elements
// in quad_partial's broadcast layout, and long rows (CPL = 0) their address.
template <int CPL, int METRIC>
struct LeftFrag {
  float f[CPL * 8];
};
template <int CPL>
struct LeftFrag<CPL, kL2> {
  RowFrag<CPL> h;
};
template <>
struct LeftFrag<0, kL2> {
  const uint4* row;
};
template <>
struct LeftFrag<0, kIP> {
  const uint4* row;
};

// The left operand of a row held in memory (queries).
template <int CPL, int METRIC>
__device__ __forceinline__ void load_left(const uint4* row, uint32_t ql, uint32_t nchunks, LeftFrag<CPL, METRIC>& l) {
  if constexpr (CPL == 0) l.row = row;
  else if constexpr (METRIC == kL2) load_row_frag<CPL>(row, ql, nchunks, true, l.h);
  else load_query_frag<CPL, METRIC>(row, ql, nchunks, l.f);
}

// Distance between a left operand and a row fragment (nlimit: L2 chunks,
// IP elements), in the reference's per-lane order and quad combine.
// INTX: the rows are integer-valued within the exact range (int_exact_l2).
template <int CPL, int METRIC, bool INTX = false>
__device__ __forceinline__ float left_distance(const LeftFrag<CPL, METRIC>& l, const RowFrag<CPL>& x, uint32_t ql,
                                               uint32_t nchunks, uint32_t nlimit) {
  if constexpr (INTX && CPL > 0 && METRIC == kL2) {
    return quad_finish<METRIC>(quad_partial_l2_int<CPL>(l.h, x, ql, nlimit));
  } else if constexpr (CPL == 0) {
    if constexpr (METRIC == kL2) return quad_finish<METRIC>(stream_partial_l2(l.row, x.row, ql, nlimit));
    else return quad_finish<METRIC>(stream_partial_ip(l.row, x.row, ql, nchunks, nlimit));
  } else if constexpr (METRIC == kL2) {
    return quad_finish<METRIC>(quad_partial_l2h<CPL>(l.h, x, ql, nlimit));
  } else {
    return quad_finish<METRIC>(quad_partial<CPL, METRIC>(l.f, x, ql, nlimit));
  }
}

}  // namespace jasper_amd
