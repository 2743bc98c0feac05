// prune.hpp -- wave-level RobustPrune over a sorted candidate list in LDS.
//
// Reference semantics (index/construct.cuh:419-472 and :680-729): walk the
// candidates in (distance, id) order; stop once R are selected; skip the
// node itself; drop c when some already selected s has d(c, s) * alpha <
// d_c; otherwise select c.
//
// Wave formulation: candidates are taken in blocks of 16, one per quad.
// Each quad first tests its candidate against the members selected before
// the block (vectors cached in LDS), then the block is resolved in order:
// the lowest surviving quad is selected, its vector is added to the cache,
// and every later quad tests against it. A candidate is therefore dropped
// exactly when a member selected before it prunes it -- the reference rule.
#pragma once

#include "common.hpp"

namespace jasper_amd {

struct PruneCtx {
  const uint4* vecs;
  uint32_t nchunks;  // row length in 16-byte chunks
  uint32_t nlimit;   // L2: chunks summed (dim / 8); IP: elements summed (dim)
  uint32_t R;
  float alpha;
  uint32_t lo2;      // integer-valued rows: the smallest value, as two fp16
  float margin_scale;  // >= 1: widens the Gram prune's proof margin (testing)
  // partitioned build merges: the two id ranges whose vectors the merge may
  // read ([r1_lo, r1_lo + r1_n) and [r2_lo, r2_lo + r2_n))
  uint32_t r1_lo, r1_n, r2_lo, r2_n;
  // the graph's byte rows (value - lo, nb8 16-byte chunks per row) and the
  // shift lo - 1024 as two fp16, when it keeps them; null otherwise
  const uint4* vecs8;
  uint32_t nb8, qsh2;
  // staged merge (the partitioned build with its partitions in host memory,
  // two on the device): range 1's rows at vecs, range 2's at vecs_b, each
  // from its first id; no other rows are on the device (byte rows off)
  uint32_t staged;
  const uint4* vecs_b;
};

// Row of vector id: the flat array, or in a staged merge the device slot of
// the id's range (callers pass only ids of the two ranges there).
__device__ __forceinline__ const uint4* vec_row(const PruneCtx& p, uint32_t id) {
  if (p.staged) {
    if (id - p.r2_lo < p.r2_n) return p.vecs_b + (size_t)(id - p.r2_lo) * p.nchunks;
    return p.vecs + (size_t)(id - p.r1_lo) * p.nchunks;
  }
  return p.vecs + (size_t)id * p.nchunks;
}

// Whether the merge prune resolves id's vector (robust_prune_kernel_scale,
// reference index/construct_scale_kernels.cuh:69-74: b1_graph.is_valid or
// b2_graph.is_valid).
__device__ __forceinline__ bool resolvable(const PruneCtx& p, uint32_t id) {
  return id - p.r1_lo < p.r1_n || id - p.r2_lo < p.r2_n;
}

// id, or range 1's first row for an id the merge does not resolve: rows
// that are read but whose values are not used (a staged merge has only the
// two ranges' rows on the device).
__device__ __forceinline__ uint32_t readable_id(const PruneCtx& p, uint32_t id) {
  return p.staged && !resolvable(p, id) ? p.r1_lo : id;
}

// The left operand of a loaded row: L2 keeps the fp16 chunks; IP converts
// the load layout (lane l: chunks l, l+4, ...) to quad_partial's fp32
// broadcast layout; long rows (CPL = 0) keep the address.
template <int CPL, int METRIC>
__device__ __forceinline__ void left_from_row(const RowFrag<CPL>& xf, uint32_t ql, LeftFrag<CPL, METRIC>& l) {
  if constexpr (CPL == 0) {
    l.row = xf.row;
  } else if constexpr (METRIC == kL2) {
    l.h = xf;
  } else {
    float (&f)[CPL * 8] = l.f;
    const uint4 (&x)[CPL] = xf.x;
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int c = 4 * t + s;
        const uint32_t src[4] = {x[t].x, x[t].y, x[t].z, x[t].w};
        uint32_t w[4];
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
        f[2 * c] = (e0 & 1u) ? h2f_hi(w0) : h2f_lo(w0);
        f[2 * c + 1] = (e1 & 1u) ? h2f_hi(w1) : h2f_lo(w1);
      }
    }
  }
}

// A selected member's row, read from the vector array by id. The 16 quads
// of a wave read the same member, so each chunk load is one wave-wide
// request served from L1/L2; keeping members in LDS instead (R x dim x 2
// bytes per wave) cut residency to 1.5 waves per SIMD and measured 1.6x
// slower on the build.
template <int CPL>
__device__ __forceinline__ void load_member(const PruneCtx& p, const uint32_t* S_ids, uint32_t s, uint32_t ql,
                                            RowFrag<CPL>& x) {
  load_row_frag<CPL>(vec_row(p, readable_id(p, S_ids[s])), ql, p.nchunks, true, x);
}

// C: sorted keys [0, nc) in LDS. Writes the selection to S_ids / S_dist.
// Returns |S|. INTX: rows are integer-valued within the exact range
// (int_exact_l2), so pair distances take the packed-difference form.
// SCALE: the merge prune of the partitioned build (reference
// index/construct_scale_kernels.cuh:54-126): a candidate whose vector is
// not resolvable is selected without a test, and a selected member that is
// not resolvable prunes nothing.
template <int CPL, int METRIC, bool INTX, bool SCALE = false>
__device__ uint32_t robust_prune_wave(const PruneCtx& p, const uint64_t* C, uint32_t nc, uint32_t self,
                                      uint32_t* S_ids, float* S_dist) {
  const uint32_t lane = lane_id();
  const uint32_t ql = lane & 3u, qg = lane >> 2;
  uint32_t ns = 0;
  for (uint32_t b = 0; b < nc && ns < p.R; b += 16) {
    const uint32_t j = b + qg;
    bool valid = j < nc;
    const uint64_t ck = valid ? C[j] : kEmptyKey;
    const uint32_t cid = key_id(ck);
    const float cd = key_dist(ck);
    valid = valid && cid != self;
    // tested against members (SCALE: only when its vector is resolvable)
    const bool tested = !SCALE || resolvable(p, cid);
    RowFrag<CPL> xc;
    load_row_frag<CPL>(vec_row(p, valid ? readable_id(p, cid) : p.r1_lo), ql, p.nchunks, valid, xc);
    LeftFrag<CPL, METRIC> cf;
    left_from_row<CPL, METRIC>(xc, ql, cf);
    bool pruned = false;
    // members selected before this block: ids held one per lane and read
    // with v_readlane, the next member's row loading while this one scores
    const uint32_t ns0 = ns;
    if (ns0) {
      const uint32_t sid_lane = lane < ns0 ? S_ids[lane] : 0u;
      RowFrag<CPL> xn;
      load_row_frag<CPL>(vec_row(p, readable_id(p, (uint32_t)__builtin_amdgcn_readlane((int)sid_lane, 0))), ql,
                         p.nchunks, true, xn);
      for (uint32_t s = 0; s < ns0; ++s) {
        const RowFrag<CPL> xs = xn;
        if (s + 1 < ns0)
          load_row_frag<CPL>(
              vec_row(p, readable_id(p, (uint32_t)__builtin_amdgcn_readlane((int)sid_lane, (int)(s + 1)))), ql,
              p.nchunks, true, xn);
        if constexpr (SCALE) {
          if (!resolvable(p, (uint32_t)__builtin_amdgcn_readlane((int)sid_lane, (int)s))) continue;
        }
        const float d = left_distance<CPL, METRIC, INTX>(cf, xs, ql, p.nchunks, p.nlimit);
        if (tested && d * p.alpha < cd) pruned = true;
        if ((s & 7u) == 7u && ballot(valid && !pruned) == 0) break;
      }
    }
    // resolve the block in candidate order
    uint64_t live = ballot(valid && !pruned && ql == 0);
    while (live && ns < p.R) {
      const uint32_t g = (uint32_t)__builtin_ctzll(live) >> 2;
      // SCALE: the new member prunes only when its vector is resolvable
      const bool g_prunes = !SCALE || (ballot(tested && qg == g) != 0);
      if (qg == g) {
        if (ql == 0) {
          S_ids[ns] = cid;
          S_dist[ns] = cd;
        }
      }
      wave_sync();
      RowFrag<CPL> xs;
      if constexpr (CPL == 0) {
        load_member<CPL>(p, S_ids, ns, ql, xs);
      } else {
        // the selected row is quad g's: lane 4g + ql holds the chunks this lane needs
        const int src = (int)(g * 4u + ql);
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
          xs.x[t].x = (uint32_t)__shfl((int)xc.x[t].x, src, 64);
          xs.x[t].y = (uint32_t)__shfl((int)xc.x[t].y, src, 64);
          xs.x[t].z = (uint32_t)__shfl((int)xc.x[t].z, src, 64);
          xs.x[t].w = (uint32_t)__shfl((int)xc.x[t].w, src, 64);
        }
      }
      if (g_prunes) {
        const float d = left_distance<CPL, METRIC, INTX>(cf, xs, ql, p.nchunks, p.nlimit);
        if (qg > g && tested && d * p.alpha < cd) pruned = true;
      }
      ns += 1;
      live = ballot(valid && !pruned && ql == 0 && qg > g);
    }
  }
  wave_sync();
  return ns;
}

// robust_prune_wave on byte rows (CPL 4, L2, pc.vecs8 set: integer rows
// spanning at most 255 values): candidates and members are read as byte
// rows and every pair distance is sum b_c^2 + sum b_m^2 - 2 sum b_c b_m in
// u32 (score_bytes_u8: two independent chains of eight v_dot4_u32_u8 per
// lane instead of one chain of sixteen v_dot2), the exact integer of the
// packed-difference form, so the selection is the same. A member selected
// in this block is taken from its quad's registers. SCALE: the merge prune's
// rule, as robust_prune_wave's.
template <bool SCALE = false>
__device__ uint32_t robust_prune_wave_u8(const PruneCtx& p, const uint64_t* C, uint32_t nc, uint32_t self,
                                         uint32_t* S_ids, float* S_dist) {
  const uint32_t lane = lane_id();
  const uint32_t ql = lane & 3u, qg = lane >> 2;
  uint32_t ns = 0;
  for (uint32_t b = 0; b < nc && ns < p.R; b += 16) {
    const uint32_t j = b + qg;
    bool valid = j < nc;
    const uint64_t ck = valid ? C[j] : kEmptyKey;
    const uint32_t cid = key_id(ck);
    const float cd = key_dist(ck);
    valid = valid && cid != self;
    const bool tested = !SCALE || resolvable(p, cid);
    RowBytes cb;
    load_row_bytes(p.vecs8, p.nb8, valid ? cid : 0u, ql, cb);
    uint32_t cn = 0;
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u) {
      if (ql + 4u * u < p.nb8) {
        cn = __builtin_amdgcn_udot4(cb.x[u].x, cb.x[u].x, cn, false);
        cn = __builtin_amdgcn_udot4(cb.x[u].y, cb.x[u].y, cn, false);
        cn = __builtin_amdgcn_udot4(cb.x[u].z, cb.x[u].z, cn, false);
        cn = __builtin_amdgcn_udot4(cb.x[u].w, cb.x[u].w, cn, false);
      }
    }
    bool pruned = false;
    const uint32_t ns0 = ns;
    if (ns0) {
      const uint32_t sid_lane = lane < ns0 ? S_ids[lane] : 0u;
      RowBytes xn;
      load_row_bytes(p.vecs8, p.nb8, (uint32_t)__builtin_amdgcn_readlane((int)sid_lane, 0), ql, xn);
      for (uint32_t s = 0; s < ns0; ++s) {
        const RowBytes xs = xn;
        if (s + 1 < ns0)
          load_row_bytes(p.vecs8, p.nb8, (uint32_t)__builtin_amdgcn_readlane((int)sid_lane, (int)(s + 1)), ql, xn);
        if constexpr (SCALE) {
          if (!resolvable(p, (uint32_t)__builtin_amdgcn_readlane((int)sid_lane, (int)s))) continue;
        }
        const float d = score_bytes_u8(p.nb8, cb.x[0], cb.x[1], cn, xs, ql);
        if (tested && d * p.alpha < cd) pruned = true;
        if ((s & 7u) == 7u && ballot(valid && !pruned) == 0) break;
      }
    }
    // resolve the block in candidate order
    uint64_t live = ballot(valid && !pruned && ql == 0);
    while (live && ns < p.R) {
      const uint32_t g = (uint32_t)__builtin_ctzll(live) >> 2;
      // SCALE: the new member prunes only when its vector is resolvable
      const bool g_prunes = !SCALE || (ballot(tested && qg == g) != 0);
      if (qg == g && ql == 0) {
        S_ids[ns] = cid;
        S_dist[ns] = cd;
      }
      wave_sync();
      const int src = (int)(g * 4u + ql);
      RowBytes xs;
#pragma unroll
      for (uint32_t u = 0; u < 2; ++u) {
        xs.x[u].x = (uint32_t)__shfl((int)cb.x[u].x, src, 64);
        xs.x[u].y = (uint32_t)__shfl((int)cb.x[u].y, src, 64);
        xs.x[u].z = (uint32_t)__shfl((int)cb.x[u].z, src, 64);
        xs.x[u].w = (uint32_t)__shfl((int)cb.x[u].w, src, 64);
      }
      if (g_prunes) {
        const float d = score_bytes_u8(p.nb8, cb.x[0], cb.x[1], cn, xs, ql);
        if (qg > g && tested && d * p.alpha < cd) pruned = true;
      }
      ns += 1;
      live = ballot(valid && !pruned && ql == 0 && qg > g);
    }
  }
  wave_sync();
  return ns;
}

// ------------------------------------------------ integer rows: Gram form
// On integer-valued rows within the exact range (int_exact_l2), shifted by
// their smallest value lo to a' = a - lo in [0, span] (exact in fp16), every
// product and partial sum of a'_i . a'_j and |a'_i|^2 is an integer below
// 2^24, so the matrix cores' fp32 accumulation is exact in any order, and
//   d(i, j) = (|a'_i|^2 - a'_i.a'_j) + (|a'_j|^2 - a'_i.a'_j)
// is the exact integer the reference's fp32 chain produces: each bracket is
// an exact integer of magnitude below 2^24 and so is the sum. One
// v_mfma_f32_32x32x16_f16 chain per pair of 32-candidate tiles gives all
// pair distances of up to 96 candidates; the prune then works on bits:
// dom(i, j) = [j < i and d(i, j) * alpha < d_i], and candidate i is
// selected when no selected j has dom(i, j) -- the reference rule, as each
// selection settles every candidate before it.
constexpr uint32_t kGramMaxCands = 96;    // three tiles of 32
constexpr uint32_t kGramMaxChunks = 16;   // rows of up to 128 fp16 values

typedef _Float16 gram_h8 __attribute__((ext_vector_type(8)));
typedef float gram_f16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ gram_h8 as_gram_h8(const uint4& x) {
  gram_h8 r;
  __builtin_memcpy(&r, &x, 16);
  return r;
}

typedef int gram_i4 __attribute__((ext_vector_type(4)));
typedef int gram_i16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ gram_i4 as_gram_i4(const uint4& x) {
  gram_i4 r;
  __builtin_memcpy(&r, &x, 16);
  return r;
}

// C: sorted keys [0, nc) in LDS, nc <= 32 * T; p.nlimit <= kGramMaxChunks.
// gn: LDS scratch of kGramLdsWords words. Writes the selection to S_ids /
// S_dist and returns |S| (the selection robust_prune_wave makes).
constexpr uint32_t kGramLdsWords = 2 * kGramMaxCands;

// Spreads 16 bits (bit 4g + q) to bit 8g + q of a word.
__device__ __forceinline__ uint32_t spread_nibbles(uint32_t w) {
  return (w & 0xFu) | ((w & 0xF0u) << 4) | ((w & 0xF00u) << 8) | ((w & 0xF000u) << 12);
}

// The prune test d * alpha < cd (fp32) on an exact integer distance d is
// d < T for one integer T per candidate: fl(d * alpha) is non-decreasing in
// d for alpha >= 0, so the passing d form a prefix. T is the smallest d >= 0
// that fails, or 2^30 when every d below it passes. Callers route alpha < 0
// and NaN elsewhere; inv_alpha is any estimate of 1 / alpha (it only places
// the search).
//
// With d0 = floor(cd * inv_alpha) and b = max(d0 - 2, 0) the test is made
// at b .. b + 5: when it passes at b and fails at b + 5 (or fails at b = 0)
// the prefix ends among them, and T = b + (the passes among b .. b + 4).
// For cd / alpha below 2^23 and inv_alpha within an ulp, T lies in
// [d0 - 1, d0 + 3], so that window always holds it; otherwise the search
// steps one value at a time to the boundary from floor(cd / alpha), as it
// did before the window.
__device__ __forceinline__ int prune_int_threshold(float cd, float alpha, float inv_alpha) {
  if (!(cd > 0.0f)) return 0;            // 0 * alpha < cd fails, and so does every d
  if (!(alpha > 0.0f)) return 1 << 30;   // alpha == 0: every d passes
  const float q = cd * inv_alpha;
  int d = q >= 1073741824.0f ? (1 << 30) : (int)q;
  const int b = max(d - 2, 0);
  int n = 0;
#pragma unroll
  for (int k = 0; k < 5; ++k) n += (float)(b + k) * alpha < cd ? 1 : 0;
  const bool past = (float)(b + 5) * alpha < cd;
  if (!past && (n > 0 || b == 0)) return min(b + n, 1 << 30);
  // the stepped search from the quotient itself (cd * inv_alpha can be far
  // off, e.g. infinite for a subnormal alpha, where cd / alpha is not)
  const float q2 = cd / alpha;
  d = q2 >= 1073741824.0f ? (1 << 30) : (int)q2;
  while (d < (1 << 30) && (float)d * alpha < cd) ++d;
  while (d > 0 && !((float)(d - 1) * alpha < cd)) --d;
  return d;
}

// I8: rows whose values span at most 255 (int8_rows) as bytes v - 128,
// v = x - lo in [0, 255], on v_mfma_i32_32x32x32_i8: half the operand
// registers of the fp16 form and half its MFMA steps. The Gram form's pair
// distance is the same exact integer (|a_i - a_j|^2 does not depend on the
// shift, and stays below 2^24), so the decisions are the fp16 form's.
template <int T, int I8 = 0>
__device__ uint32_t robust_prune_gram(const PruneCtx& p, const uint64_t* C, uint32_t nc, uint32_t self,
                                      uint32_t* S_ids, float* S_dist, float* gn) {
  static_assert(T >= 1 && T <= 3, "one to three tiles");
  // fp16: 16 values per step, lane half h holds chunk 2s + h; int8: 32
  // values per step, lane half h holds chunks 4s + 2h and 4s + 2h + 1 (byte
  // chunk 2s + h of a byte row)
  constexpr int KS = I8 ? kGramMaxChunks / 4 : kGramMaxChunks / 2;
  const uint32_t lane = lane_id();
  const uint32_t r = lane & 31u, h = lane >> 5;
  // per candidate i: U_i = T_i - |a_i|^2 (prune_int_threshold) in the
  // registers of the lanes that hold i's column, |a_i|^2 in gu[i], so that
  // "i prunes j" is |a_i|^2 - 2 a_i.a_j < U_j in exact integers
  int* gu = reinterpret_cast<int*>(gn);
  int ucol[T];
  const float inv_alpha = 1.0f / p.alpha;  // places the threshold search

  // MFMA operand of tile t, step s for candidate 32t + r, shifted; chunks
  // past the summed length are zero
  uint4 fr[T][KS];
  int nrm[T];
  if constexpr (I8 == 2) {
    // the byte rows already hold v = x - lo: one 16-byte load per step
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t i = 32u * (uint32_t)t + r;
      const uint64_t key = i < nc ? C[i] : kEmptyKey;
      const uint32_t id = i < nc ? key_id(key) : self;
      const uint4* row8 = p.vecs8 + (size_t)id * p.nb8;
      uint4 raw[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = 2u * (uint32_t)s + h;  // fp16 chunks 2c and 2c + 1
        raw[s] = row8[min(c, p.nb8 - 1u)];
      }
      int acc = 0;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = 2u * (uint32_t)s + h;
        const uint32_t keep = 2u * c + 1u < p.nlimit ? ~0u : 0u;
        const uint4 x = raw[s];
        const uint32_t wd[4] = {(x.x ^ 0x80808080u) & keep, (x.y ^ 0x80808080u) & keep,
                                (x.z ^ 0x80808080u) & keep, (x.w ^ 0x80808080u) & keep};
        fr[t][s] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_sdot4((int)wd[u], (int)wd[u], acc, false);
      }
      nrm[t] = acc + __shfl_xor(acc, 32, 64);  // below 2^24
      ucol[t] = prune_int_threshold(key_dist(key), p.alpha, inv_alpha) - nrm[t];
      if (h == 0) gu[i] = nrm[t];
    }
  } else if constexpr (I8 == 1) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t i = 32u * (uint32_t)t + r;
      const uint64_t key = i < nc ? C[i] : kEmptyKey;
      const uint32_t id = i < nc ? key_id(key) : self;
      const uint4* row = p.vecs + (size_t)id * p.nchunks;
      uint4 raw[2 * KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = 4u * (uint32_t)s + 2u * h;
        raw[2 * s] = row[min(c, p.nchunks - 1u)];
        raw[2 * s + 1] = row[min(c + 1u, p.nchunks - 1u)];
      }
      int acc = 0;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        uint32_t wd[4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t c = 4u * (uint32_t)s + 2u * h + (uint32_t)u;
          const uint32_t keep = c < p.nlimit ? ~0u : 0u;
          const uint4 x = raw[2 * s + u];
          // x - lo + 1024 = 0x6400 | v exactly (v < 1024): v is the low byte
          const uint32_t a0 = sub_half2(sub_half2(x.x, p.lo2), 0xE400E400u);
          const uint32_t a1 = sub_half2(sub_half2(x.y, p.lo2), 0xE400E400u);
          const uint32_t a2 = sub_half2(sub_half2(x.z, p.lo2), 0xE400E400u);
          const uint32_t a3 = sub_half2(sub_half2(x.w, p.lo2), 0xE400E400u);
          wd[2 * u] = (__builtin_amdgcn_perm(a1, a0, 0x06040200u) ^ 0x80808080u) & keep;
          wd[2 * u + 1] = (__builtin_amdgcn_perm(a3, a2, 0x06040200u) ^ 0x80808080u) & keep;
        }
        fr[t][s] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_sdot4((int)wd[u], (int)wd[u], acc, false);
      }
      nrm[t] = acc + __shfl_xor(acc, 32, 64);  // below 2^24
      ucol[t] = prune_int_threshold(key_dist(key), p.alpha, inv_alpha) - nrm[t];
      if (h == 0) gu[i] = nrm[t];
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t i = 32u * (uint32_t)t + r;
      const uint64_t key = i < nc ? C[i] : kEmptyKey;
      const uint32_t id = i < nc ? key_id(key) : self;
      const uint4* row = p.vecs + (size_t)id * p.nchunks;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = 2u * (uint32_t)s + h;
        fr[t][s] = row[min(c, p.nchunks - 1u)];
      }
      ucol[t] = prune_int_threshold(key_dist(key), p.alpha, inv_alpha);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = 2u * (uint32_t)s + h;
        const uint32_t keep = c < p.nlimit ? ~0u : 0u;  // per word: no struct select
        uint4 x = fr[t][s];
        x.x = sub_half2(x.x, p.lo2) & keep;
        x.y = sub_half2(x.y, p.lo2) & keep;
        x.z = sub_half2(x.z, p.lo2) & keep;
        x.w = sub_half2(x.w, p.lo2) & keep;
        fr[t][s] = x;
        acc = dot2_sqdiff(x.x, 0u, acc);
        acc = dot2_sqdiff(x.y, 0u, acc);
        acc = dot2_sqdiff(x.z, 0u, acc);
        acc = dot2_sqdiff(x.w, 0u, acc);
      }
      nrm[t] = (int)(acc + xor_lane_f<32>(acc));  // exact: integers below 2^24
    }
    wave_sync();
#pragma unroll
    for (int t = 0; t < T; ++t) {
      ucol[t] -= nrm[t];
      if (h == 0) gu[32u * (uint32_t)t + r] = nrm[t];
    }
  }
  wave_sync();
  // rows 8g + 4h + q of a diagonal block that precede this lane's column r,
  // at bit 8g + q: the bits below r - 4h that lie in the low nibbles
  const int dm = (int)r - 4 * (int)h;
  const uint32_t diagm8 = dm > 0 ? ((1u << dm) - 1u) & 0x0F0F0F0Fu : 0u;

  // W[t][t2] (t <= t2), lane (r, h): bit b set when candidate 32 t + b
  // prunes candidate 32 t2 + r (which follows it): the block of rows t and
  // columns t2 (the Gram matrix is symmetric), so the lanes of a candidate's
  // column hold the candidates that prune it
  uint32_t W[T][T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int t2 = 0; t2 < T; ++t2) W[t][t2] = 0u;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int t2 = t; t2 < T; ++t2) {
      gram_i16 ai;
      if constexpr (I8 != 0) {
        ai = gram_i16{};
#pragma unroll
        for (int s = 0; s < KS; ++s)
          ai = __builtin_amdgcn_mfma_i32_32x32x32_i8(as_gram_i4(fr[t][s]), as_gram_i4(fr[t2][s]), ai, 0, 0, 0);
      } else {
        gram_f16 acc = gram_f16{};
#pragma unroll
        for (int s = 0; s < KS; ++s)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_gram_h8(fr[t][s]), as_gram_h8(fr[t2][s]), acc, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) ai[e] = (int)acc[e];  // exact: |a_i . a_j| < 2^24
      }
      // lane holds column j = 32 t2 + r (whose U_j it holds) and rows i =
      // 32 t + 8g + 4h + q; bit 8g + q: i prunes j, i.e. the sign of
      // |a_i|^2 - (2 a_i.a_j + U_j) (no overflow: |a_i|^2 and |a_i.a_j| are
      // below 2^24, U_j below 2^30), shifted in from the top bit down by one
      // v_alignbit each, with a zero nibble between groups
      const uint32_t uj = (uint32_t)ucol[t2];
      uint32_t w = 0u;
#pragma unroll
      for (int g = 3; g >= 0; --g) {
        const int4 nn = *reinterpret_cast<const int4*>(gu + 32 * t + 8 * g + 4 * h);
        if (g < 3) w <<= 4;
#pragma unroll
        for (int q = 3; q >= 0; --q) {
          const uint32_t ni = (uint32_t)(q == 0 ? nn.x : q == 1 ? nn.y : q == 2 ? nn.z : nn.w);
          // (the barrier keeps 2 a_i.a_j + U_j one v_lshl_add_u32, not
          // reassociated into a shift, a subtraction and an addition)
          uint32_t t2u = ((uint32_t)ai[4 * g + q] << 1) + uj;
          asm volatile("" : "+v"(t2u));
          w = __builtin_amdgcn_alignbit(w, ni - t2u, 31u);  // (w << 1) | sign bit
        }
      }
      if (t == t2) w &= diagm8;
      w <<= 4u * h;  // rows 8g + 4h + q
      W[t][t2] = w | xor_lane<32>(w);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // row words by candidate: lane i % 64 of set A (candidates 0..63) or set
  // B (64..95) holds, per row tile t, the candidates of tile t that prune it
  uint32_t rowA[T], rowB[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t w0 = t == 0 ? W[0][0] : 0u;
    const uint32_t w1 = T >= 2 && t <= 1 ? W[t][T >= 2 ? 1 : 0] : 0u;
    rowA[t] = T >= 2 && h ? w1 : w0;
    rowB[t] = T == 3 ? W[t][T - 1] : 0u;
  }

  // selection (RobustPrune's greedy: a candidate is taken when no taken
  // candidate before it prunes it) as the fixed point of S = {valid j : no
  // i in S prunes j}: the relation only runs from earlier to later
  // candidates, so the fixed point is unique and it is the greedy's set;
  // iterating from S = every valid candidate reaches it in at most (the
  // longest chain of the relation) + 1 rounds, each a few ANDs and two
  // ballots. The cap of R keeps the first R of the set.
  const bool validA = lane < nc && key_id(C[lane]) != self;
  const bool validB = T == 3 && lane < 32u && 64u + lane < nc && key_id(C[64u + lane]) != self;
  uint64_t selA = ballot(validA), selB = ballot(validB);
  for (uint32_t round = 0; round <= kGramMaxCands; ++round) {
    const uint32_t s0 = (uint32_t)selA, s1 = (uint32_t)(selA >> 32), s2 = (uint32_t)selB;
    uint32_t hitA = rowA[0] & s0, hitB = rowB[0] & s0;
    if constexpr (T >= 2) {
      hitA |= rowA[1] & s1;
      hitB |= rowB[1] & s1;
    }
    if constexpr (T == 3) {
      hitA |= rowA[2] & s2;
      hitB |= rowB[2] & s2;
    }
    const uint64_t nA = ballot(validA && hitA == 0u), nB = ballot(validB && hitB == 0u);
    if (nA == selA && nB == selB) break;
    selA = nA;
    selB = nB;
  }
  const uint32_t allA = (uint32_t)__builtin_popcountll(selA);
  const uint32_t ns = min(p.R, allA + (uint32_t)__builtin_popcountll(selB));
  selA = ballot(((selA >> lane) & 1ull) && mbcnt(selA) < p.R);
  selB = ballot(lane < 32u && ((selB >> lane) & 1ull) && allA + mbcnt(selB) < p.R);
  // the selection in candidate order
  const uint32_t nA = (uint32_t)__builtin_popcountll(selA);
  if ((selA >> lane) & 1ull) {
    const uint32_t k = mbcnt(selA);
    const uint64_t key = C[lane];
    S_ids[k] = key_id(key);
    S_dist[k] = key_dist(key);
  }
  if (lane < 32u && ((selB >> lane) & 1ull)) {
    const uint32_t k = nA + mbcnt(selB);
    const uint64_t key = C[64u + lane];
    S_ids[k] = key_id(key);
    S_dist[k] = key_dist(key);
  }
  wave_sync();
  return ns;
}

// ------------------------------------------- any fp16 rows: Gram + proof
// For rows that are not integer-valued the matrix cores' sums are not the
// reference's fp32 chain bit for bit, so the Gram matrix only decides the
// pairs it can prove. With S = sum |a_i,k a_j,k| <= (|a_i|^2 + |a_j|^2) / 2,
// the Gram form d~ = (|a_i|^2 - a_i.a_j) + (|a_j|^2 - a_i.a_j) (L2; -a_i.a_j
// for IP) and the chain's own result are both within a few n*u (u = 2^-24,
// n summed values) of the exact real value: the matrix-core sum of products
// within n*u*S, the norms within (n/2+2)*u*|a|^2, the chain within
// (n/4+8)*u*d (L2: nonnegative terms) or (n/4+8)*u*S (IP). The margin M
// takes four times those bounds (plus 2^-13 per unit of sqrt(n)*|a| in case
// fp16 subnormals are flushed, and the roundings of d*alpha and of the
// comparison). A pair with |d~*alpha - d_i| > M has the chain's decision;
// the others are settled by the chain itself when they matter: when their
// row becomes the first live candidate, the exact d(i, j) to each selected
// member j of an unproved pair is computed in the reference's order.
template <int T, int CPL, int METRIC>
__device__ uint32_t robust_prune_gram_f(const PruneCtx& p, const uint64_t* C, uint32_t nc, uint32_t self,
                                        uint32_t* S_ids, float* S_dist, float* gn) {
  static_assert(T >= 1 && T <= 3, "one to three tiles");
  static_assert(CPL >= 1, "rows held in registers");
  constexpr int KS = kGramMaxChunks / 2;
  const uint32_t lane = lane_id();
  const uint32_t r = lane & 31u, h = lane >> 5;
  // chunks summed: L2 counts chunks, IP elements (padding past dim is zero)
  const uint32_t climit = METRIC == kL2 ? p.nlimit : (p.nlimit + 7u) / 8u;
  const float nsum = 8.0f * (float)climit;
  constexpr float U = 5.9604645e-8f;  // 2^-24
  const float sub = 1.2207031e-4f * sqrtf(nsum);  // 2^-13 * sqrt(n)

  uint4 fr[T][KS];
  float nrm[T], cdc[T];  // the norm and distance of this lane's candidate 32 t + r
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t i = 32u * (uint32_t)t + r;
    const uint64_t key = i < nc ? C[i] : kEmptyKey;
    const uint32_t id = i < nc ? key_id(key) : self;
    const uint4* row = p.vecs + (size_t)id * p.nchunks;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t c = 2u * (uint32_t)s + h;
      fr[t][s] = row[min(c, p.nchunks - 1u)];
    }
    cdc[t] = key_dist(key);
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t c = 2u * (uint32_t)s + h;
      const uint32_t keep = c < climit ? ~0u : 0u;
      uint4 x = fr[t][s];
      x.x &= keep;
      x.y &= keep;
      x.z &= keep;
      x.w &= keep;
      fr[t][s] = x;
      acc = dot2_sqdiff(x.x, 0u, acc);
      acc = dot2_sqdiff(x.y, 0u, acc);
      acc = dot2_sqdiff(x.z, 0u, acc);
      acc = dot2_sqdiff(x.w, 0u, acc);
    }
    nrm[t] = acc + xor_lane_f<32>(acc);
    if (h == 0) gn[32u * (uint32_t)t + r] = nrm[t];
  }
  wave_sync();

  // The margin, linear in a row term, a column term and |d|: with c1, c2
  // the coefficients of e (L2: U (1.5 n + 16) and U (0.25 n + 8); IP:
  // U (1.25 n + 16) and no |d| term), K1 = 4 ms |alpha| and
  //   e = c1 (n_i + n_j) + c2 |d| + sub (sqrt n_i + sqrt n_j),
  //   M = 4 ms (|alpha| e + 2 U (|alpha| |d| + |c_j|))
  //     = a_i + C_j + K2 |d|,  a_i = K1 (c1 n_i + sub sqrt n_i),
  //   C_j = K1 (c1 n_j + sub sqrt n_j) + 8 ms U |c_j|, K2 = K1 c2 + 8 ms U |alpha|
  // (|alpha|: a sound bound for either sign). a_i sits in gn[96 + i].
  const float aalpha = fabsf(p.alpha);
  const float K1 = p.margin_scale * 4.0f * aalpha;
  const float c1 = METRIC == kL2 ? U * (1.5f * nsum + 16.0f) : U * (1.25f * nsum + 16.0f);
  const float c2 = METRIC == kL2 ? U * (0.25f * nsum + 8.0f) : 0.0f;
  const float K2 = K1 * c2 + p.margin_scale * 8.0f * U * aalpha;
  float ccol[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float sn = sqrtf(nrm[t]);
    ccol[t] = K1 * (c1 * nrm[t] + sub * sn) + p.margin_scale * 8.0f * U * fabsf(cdc[t]);
    if (h == 0) gn[kGramMaxCands + 32u * (uint32_t)t + r] = K1 * (c1 * nrm[t] + sub * sn);
  }
  wave_sync();
  // rows 8g + 4h + q of a diagonal block that precede this lane's column r,
  // at bit 8g + q
  const int dm = (int)r - 4 * (int)h;
  const uint32_t diagm8 = dm > 0 ? ((1u << dm) - 1u) & 0x0F0F0F0Fu : 0u;

  // P: proved "i prunes j", A: not proved either way, for rows i of tile
  // t <= column tile t2 (rows precede columns; the Gram matrix is
  // symmetric): the lanes of column j = 32 t2 + r hold the bits of rows i =
  // 32 t + 8g + 4h + q, so a candidate's lanes hold the candidates that may
  // prune it. With x = d alpha - c_j: proved when x + M < 0, not proved
  // when additionally M - x >= 0 fails neither (NaN sums count as not
  // proved); each bit is a sign shifted in by one v_alignbit.
  uint32_t WP[T][T], WA[T][T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int t2 = 0; t2 < T; ++t2) {
      WP[t][t2] = 0u;
      WA[t][t2] = 0u;
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int t2 = t; t2 < T; ++t2) {
      gram_f16 acc = {};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_gram_h8(fr[t][s]), as_gram_h8(fr[t2][s]), acc, 0, 0, 0);
      const float nj = nrm[t2];
      const float cdj = cdc[t2];
      const float cj = ccol[t2];
      uint32_t wy = 0u, wz = 0u;
#pragma unroll
      for (int g = 3; g >= 0; --g) {
        const float4 ni = *reinterpret_cast<const float4*>(gn + 32 * t + 8 * g + 4 * h);
        const float4 ai = *reinterpret_cast<const float4*>(gn + kGramMaxCands + 32 * t + 8 * g + 4 * h);
        if (g < 3) {
          wy <<= 4;
          wz <<= 4;
        }
#pragma unroll
        for (int q = 3; q >= 0; --q) {
          const float gij = acc[4 * g + q];
          const float niq = q == 0 ? ni.x : q == 1 ? ni.y : q == 2 ? ni.z : ni.w;
          const float aiq = q == 0 ? ai.x : q == 1 ? ai.y : q == 2 ? ai.z : ai.w;
          const float d = METRIC == kL2 ? (niq - gij) + (nj - gij) : -gij;
          const float x = __builtin_fmaf(d, p.alpha, -cdj);
          const float m = __builtin_fmaf(K2, fabsf(d), aiq + cj);
          const float y = fminf(x + m, __builtin_inff());  // NaN -> +inf: not proved
          const float z = fminf(m - x, __builtin_inff());
          wy = __builtin_amdgcn_alignbit(wy, __float_as_uint(y), 31u);
          wz = __builtin_amdgcn_alignbit(wz, __float_as_uint(z), 31u);
        }
      }
      uint32_t wp = wy, wa = ~(wy | wz) & 0x0F0F0F0Fu;
      if (t == t2) {
        wp &= diagm8;
        wa &= diagm8;
      }
      const uint32_t sp = wp << (4u * h);
      const uint32_t sa = wa << (4u * h);
      WP[t][t2] = sp | xor_lane<32>(sp);
      WA[t][t2] = sa | xor_lane<32>(sa);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // row words by candidate (lane i % 64 of set A, candidates 0..63, or set
  // B, 64..95): per row tile t, the candidates of tile t that prune it
  // (pA, pB) or may (aA, aB)
  uint32_t pA[T], pB[T], aA[T], aB[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t tA = T >= 2 && h ? 1u : 0u;
    pA[t] = (uint32_t)t <= tA ? (tA ? WP[t][T >= 2 ? 1 : 0] : WP[t][0]) : 0u;
    aA[t] = (uint32_t)t <= tA ? (tA ? WA[t][T >= 2 ? 1 : 0] : WA[t][0]) : 0u;
    pB[t] = T == 3 ? WP[t][T - 1] : 0u;
    aB[t] = T == 3 ? WA[t][T - 1] : 0u;
  }

  const bool validA = lane < nc && key_id(C[lane]) != self;
  const bool validB = T == 3 && lane < 32u && 64u + lane < nc && key_id(C[64u + lane]) != self;
  // Every pair the margin leaves open is settled by the chain (the
  // reference's order, one quad per pair, 16 pairs per pass): its bit moves
  // to the proved words when i prunes j.
  const uint32_t ql = lane & 3u, qg = lane >> 2;
  for (;;) {
    uint32_t anyA = 0u, anyB = 0u;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      anyA |= aA[t];
      anyB |= aB[t];
    }
    uint64_t openA = ballot(validA && anyA != 0u), openB = ballot(validB && anyB != 0u);
    if (!(openA | openB)) break;
    // up to 16 pairs (i, j) in lane order of j, then row order of i
    uint32_t iq = 0xFFFFFFFFu, jq = 0xFFFFFFFFu;
    uint32_t cur_j = 0xFFFFFFFFu, w0 = 0u, w1 = 0u, w2 = 0u;
    for (uint32_t g = 0; g < 16u; ++g) {
      if (cur_j == 0xFFFFFFFFu || !(w0 | w1 | w2)) {
        if (!(openA | openB)) break;
        uint32_t src;
        const bool inA = openA != 0;
        if (inA) {
          src = (uint32_t)__builtin_ctzll(openA);
          openA &= openA - 1u;
          cur_j = src;
        } else {
          src = (uint32_t)__builtin_ctzll(openB);
          openB &= openB - 1u;
          cur_j = 64u + src;
        }
        w0 = (uint32_t)__builtin_amdgcn_readlane((int)(inA ? aA[0] : aB[0]), (int)src);
        w1 = T >= 2 ? (uint32_t)__builtin_amdgcn_readlane((int)(inA ? aA[T >= 2 ? 1 : 0] : aB[T >= 2 ? 1 : 0]), (int)src)
                    : 0u;
        w2 = T == 3 ? (uint32_t)__builtin_amdgcn_readlane((int)(inA ? aA[T - 1] : aB[T - 1]), (int)src) : 0u;
      }
      uint32_t i;
      if (w0) {
        i = (uint32_t)__builtin_ctz(w0);
        w0 &= w0 - 1u;
      } else if (w1) {
        i = 32u + (uint32_t)__builtin_ctz(w1);
        w1 &= w1 - 1u;
      } else {
        i = 64u + (uint32_t)__builtin_ctz(w2);
        w2 &= w2 - 1u;
      }
      if (qg == g) {
        iq = i;
        jq = cur_j;
      }
    }
    const bool act = jq != 0xFFFFFFFFu;
    const uint64_t ki = act ? C[iq] : C[0];
    const uint64_t kj = act ? C[jq] : C[0];
    RowFrag<CPL> xj, xi;
    load_row_frag<CPL>(p.vecs + (size_t)key_id(kj) * p.nchunks, ql, p.nchunks, true, xj);
    load_row_frag<CPL>(p.vecs + (size_t)key_id(ki) * p.nchunks, ql, p.nchunks, true, xi);
    LeftFrag<CPL, METRIC> lj;
    left_from_row<CPL, METRIC>(xj, ql, lj);
    // d(j, i) in the order the sequential prune computes it: the candidate
    // j as the left operand, the member i as the row
    const float d = left_distance<CPL, METRIC, false>(lj, xi, ql, p.nchunks, p.nlimit);
    const uint64_t prq = ballot(act && ql == 0u && d * p.alpha < key_dist(kj));
    const uint64_t doneq = ballot(act && ql == 0u);
    // each settled pair: the owner lanes of j clear the open bit of i and
    // set the proved bit when i prunes j
    for (uint64_t m = doneq; m; m &= m - 1u) {
      const uint32_t l = (uint32_t)__builtin_ctzll(m);
      const uint32_t pi = (uint32_t)__builtin_amdgcn_readlane((int)iq, (int)l);
      const uint32_t pj = (uint32_t)__builtin_amdgcn_readlane((int)jq, (int)l);
      const bool pruned = (prq >> l) & 1ull;
      const uint32_t ti = pi >> 5, bit = 1u << (pi & 31u);
      const bool own = pj < 64u ? lane == pj : lane == pj - 64u;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        if ((uint32_t)t != ti || !own) continue;
        if (pj < 64u) {
          aA[t] &= ~bit;
          if (pruned) pA[t] |= bit;
        } else {
          aB[t] &= ~bit;
          if (pruned) pB[t] |= bit;
        }
      }
    }
  }
  // selection as the fixed point of S = {valid j : no i in S prunes j}
  // (robust_prune_gram): the greedy's set, capped at the first R
  uint64_t selA = ballot(validA), selB = ballot(validB);
  for (uint32_t round = 0; round <= kGramMaxCands; ++round) {
    const uint32_t s0 = (uint32_t)selA, s1 = (uint32_t)(selA >> 32), s2 = (uint32_t)selB;
    uint32_t hitA = pA[0] & s0, hitB = pB[0] & s0;
    if constexpr (T >= 2) {
      hitA |= pA[1] & s1;
      hitB |= pB[1] & s1;
    }
    if constexpr (T == 3) {
      hitA |= pA[2] & s2;
      hitB |= pB[2] & s2;
    }
    const uint64_t nA = ballot(validA && hitA == 0u), nB = ballot(validB && hitB == 0u);
    if (nA == selA && nB == selB) break;
    selA = nA;
    selB = nB;
  }
  const uint32_t allA = (uint32_t)__builtin_popcountll(selA);
  const uint32_t ns = min(p.R, allA + (uint32_t)__builtin_popcountll(selB));
  selA = ballot(((selA >> lane) & 1ull) && mbcnt(selA) < p.R);
  selB = ballot(lane < 32u && ((selB >> lane) & 1ull) && allA + mbcnt(selB) < p.R);
  const uint32_t nA = (uint32_t)__builtin_popcountll(selA);
  if ((selA >> lane) & 1ull) {
    const uint32_t k = mbcnt(selA);
    const uint64_t key = C[lane];
    S_ids[k] = key_id(key);
    S_dist[k] = key_dist(key);
  }
  if (lane < 32u && ((selB >> lane) & 1ull)) {
    const uint32_t k = nA + mbcnt(selB);
    const uint64_t key = C[64u + lane];
    S_ids[k] = key_id(key);
    S_dist[k] = key_dist(key);
  }
  wave_sync();
  return ns;
}

}  // namespace jasper_amd
