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

}  // namespace jasper_amd
