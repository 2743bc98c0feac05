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
};

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
  load_row_frag<CPL>(p.vecs + (size_t)S_ids[s] * p.nchunks, ql, p.nchunks, true, x);
}

// C: sorted keys [0, nc) in LDS. Writes the selection to S_ids / S_dist.
// Returns |S|. INTX: rows are integer-valued within the exact range
// (int_exact_l2), so pair distances take the packed-difference form.
template <int CPL, int METRIC, bool INTX>
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
    RowFrag<CPL> xc;
    load_row_frag<CPL>(p.vecs + (size_t)(valid ? cid : 0u) * p.nchunks, ql, p.nchunks, valid, xc);
    LeftFrag<CPL, METRIC> cf;
    left_from_row<CPL, METRIC>(xc, ql, cf);
    bool pruned = false;
    // members selected before this block: ids held one per lane and read
    // with v_readlane, the next member's row loading while this one scores
    const uint32_t ns0 = ns;
    if (ns0) {
      const uint32_t sid_lane = lane < ns0 ? S_ids[lane] : 0u;
      RowFrag<CPL> xn;
      load_row_frag<CPL>(p.vecs + (size_t)(uint32_t)__builtin_amdgcn_readlane((int)sid_lane, 0) * p.nchunks, ql,
                         p.nchunks, true, xn);
      for (uint32_t s = 0; s < ns0; ++s) {
        const RowFrag<CPL> xs = xn;
        if (s + 1 < ns0)
          load_row_frag<CPL>(p.vecs + (size_t)(uint32_t)__builtin_amdgcn_readlane((int)sid_lane, (int)(s + 1)) *
                                          p.nchunks,
                             ql, p.nchunks, true, xn);
        const float d = left_distance<CPL, METRIC, INTX>(cf, xs, ql, p.nchunks, p.nlimit);
        if (d * p.alpha < cd) pruned = true;
        if ((s & 7u) == 7u && ballot(valid && !pruned) == 0) break;
      }
    }
    // resolve the block in candidate order
    uint64_t live = ballot(valid && !pruned && ql == 0);
    while (live && ns < p.R) {
      const uint32_t g = (uint32_t)__builtin_ctzll(live) >> 2;
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
      const float d = left_distance<CPL, METRIC, INTX>(cf, xs, ql, p.nchunks, p.nlimit);
      if (qg > g && d * p.alpha < cd) pruned = true;
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

__device__ __forceinline__ uint32_t sub_half2(uint32_t a, uint32_t b) {
  half2_t x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  const half2_t d = x - y;
  uint32_t r;
  __builtin_memcpy(&r, &d, 4);
  return r;
}

__device__ __forceinline__ gram_h8 as_gram_h8(const uint4& x) {
  gram_h8 r;
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

template <int T>
__device__ uint32_t robust_prune_gram(const PruneCtx& p, const uint64_t* C, uint32_t nc, uint32_t self,
                                      uint32_t* S_ids, float* S_dist, float* gn) {
  static_assert(T >= 1 && T <= 3, "one to three tiles");
  constexpr int KS = kGramMaxChunks / 2;  // 16 fp16 values per step
  const uint32_t lane = lane_id();
  const uint32_t r = lane & 31u, h = lane >> 5;
  float* gcd = gn + kGramMaxCands;

  // MFMA operand of tile t, step s: lane (r, h) holds values 16s + 8h .. +8
  // of candidate 32t + r, shifted; steps past the summed length are zero
  uint4 fr[T][KS];
  float nrm[T];
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
    if (h == 0) gcd[i] = key_dist(key);
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
    nrm[t] = acc + xor_lane_f<32>(acc);  // exact: integers below 2^24
    if (h == 0) gn[32u * (uint32_t)t + r] = nrm[t];
  }
  wave_sync();

  // W[t][t2], lane (r, h): bit b set when candidate 32 t + b is pruned by
  // candidate 32 t2 + r (which precedes it): the column of the pair block
  uint32_t W[T][T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int t2 = 0; t2 < T; ++t2) W[t][t2] = 0u;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int t2 = 0; t2 <= t; ++t2) {
      gram_f16 acc = {};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_gram_h8(fr[t][s]), as_gram_h8(fr[t2][s]), acc, 0, 0, 0);
      // lane holds column j = 32 t2 + r (whose norm it holds) and rows
      // 32 t + 8g + 4h + q
      const float nj = nrm[t2];
      uint32_t w16 = 0u;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 ni = *reinterpret_cast<const float4*>(gn + 32 * t + 8 * g + 4 * h);
        const float4 cd = *reinterpret_cast<const float4*>(gcd + 32 * t + 8 * g + 4 * h);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float gij = acc[4 * g + q];
          const float niq = q == 0 ? ni.x : q == 1 ? ni.y : q == 2 ? ni.z : ni.w;
          const float cdq = q == 0 ? cd.x : q == 1 ? cd.y : q == 2 ? cd.z : cd.w;
          const float d = (niq - gij) + (nj - gij);
          bool bit = d * p.alpha < cdq;
          if (t == t2) bit = bit && r < (uint32_t)(8 * g + 4 * (int)h + q);
          w16 |= bit ? (1u << (4 * g + q)) : 0u;
        }
      }
      const uint32_t w = spread_nibbles(w16) << (4u * h);  // rows 8g + 4h + q
      W[t][t2] = w | xor_lane<32>(w);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // column words by candidate: lane i % 64 of set A (candidates 0..63) or
  // set B (64..95) holds, per row tile t, the rows that candidate prunes
  uint32_t colA[T], colB[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    colA[t] = T >= 2 && h ? W[t][T >= 2 ? 1 : 0] : W[t][0];
    colB[t] = T == 3 ? W[t][T - 1] : 0u;
  }

  // selection: the first live candidate is taken and the candidates it
  // prunes leave the live set (every one before it is already settled)
  const bool validA = lane < nc && key_id(C[lane]) != self;
  const bool validB = T == 3 && lane < 32u && 64u + lane < nc && key_id(C[64u + lane]) != self;
  uint64_t liveA = ballot(validA), liveB = ballot(validB);
  uint64_t selA = 0, selB = 0;
  uint32_t ns = 0;
  while (ns < p.R && (liveA | liveB)) {
    uint32_t p0, p1, p2;
    if (liveA) {
      const uint32_t i = (uint32_t)__builtin_ctzll(liveA);
      liveA &= liveA - 1u;
      selA |= 1ull << i;
      p0 = (uint32_t)__builtin_amdgcn_readlane((int)colA[0], (int)i);
      p1 = T >= 2 ? (uint32_t)__builtin_amdgcn_readlane((int)colA[T >= 2 ? 1 : 0], (int)i) : 0u;
      p2 = T == 3 ? (uint32_t)__builtin_amdgcn_readlane((int)colA[T - 1], (int)i) : 0u;
    } else {
      const uint32_t i = (uint32_t)__builtin_ctzll(liveB);
      liveB &= liveB - 1u;
      selB |= 1ull << i;
      p0 = 0u;  // rows before the candidate are settled
      p1 = 0u;
      p2 = (uint32_t)__builtin_amdgcn_readlane((int)colB[T - 1], (int)i);
    }
    liveA &= ~((uint64_t)p0 | ((uint64_t)p1 << 32));
    liveB &= ~(uint64_t)p2;
    ns += 1;
  }
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

}  // namespace jasper_amd
