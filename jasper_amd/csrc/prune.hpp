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

// Convert a row fragment in load layout (lane l: chunks l, l+4, ...) to the
// fp32 "left operand" layout quad_partial expects.
template <int CPL, int METRIC>
__device__ __forceinline__ void frag_from_rows(const uint4 (&x)[CPL], uint32_t ql, float (&f)[CPL * 8]) {
  if constexpr (METRIC == kL2) {
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const uint32_t w[4] = {x[t].x, x[t].y, x[t].z, x[t].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        f[t * 8 + 2 * k] = h2f_lo(w[k]);
        f[t * 8 + 2 * k + 1] = h2f_hi(w[k]);
      }
    }
  } else {
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

// Distance between a left row (fp16 chunks xl; for IP also its fp32 layout
// fl) and a right row xr, in the reference's per-lane order.
template <int CPL, int METRIC>
__device__ __forceinline__ float pair_distance(const uint4 (&xl)[CPL], const float (&fl)[CPL * 8],
                                               const uint4 (&xr)[CPL], uint32_t ql, uint32_t nlimit) {
  if constexpr (METRIC == kL2) return quad_finish<METRIC>(quad_partial_l2h<CPL>(xl, xr, ql, nlimit));
  else return quad_finish<METRIC>(quad_partial<CPL, METRIC>(fl, xr, ql, nlimit));
}

template <int CPL>
__device__ __forceinline__ void load_cache_frag(const uint4* cache_row, uint32_t ql, uint32_t nchunks,
                                                uint4 (&x)[CPL]) {
#pragma unroll
  for (int t = 0; t < CPL; ++t) {
    const uint32_t c = ql + 4u * (uint32_t)t;
    x[t] = c < nchunks ? cache_row[c] : make_uint4(0, 0, 0, 0);
  }
}

// C: sorted keys [0, nc) in LDS. Writes the selection to S_ids / S_dist and
// the selected vectors to Scache ([R][nchunks] uint4, LDS). Returns |S|.
template <int CPL, int METRIC>
__device__ uint32_t robust_prune_wave(const PruneCtx& p, const uint64_t* C, uint32_t nc, uint32_t self,
                                      uint32_t* S_ids, float* S_dist, uint4* Scache) {
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
    uint4 xc[CPL];
    load_row_frag<CPL>(p.vecs + (size_t)(valid ? cid : 0u) * p.nchunks, ql, p.nchunks, valid, xc);
    float cf[CPL * 8];
    if constexpr (METRIC != kL2) frag_from_rows<CPL, METRIC>(xc, ql, cf);
    bool pruned = false;
    // members selected before this block
    const uint32_t ns0 = ns;
    for (uint32_t s = 0; s < ns0; ++s) {
      uint4 xs[CPL];
      load_cache_frag<CPL>(Scache + (size_t)s * p.nchunks, ql, p.nchunks, xs);
      const float d = pair_distance<CPL, METRIC>(xc, cf, xs, ql, p.nlimit);
      if (d * p.alpha < cd) pruned = true;
      if ((s & 7u) == 7u && ballot(valid && !pruned) == 0) break;
    }
    // resolve the block in candidate order
    uint64_t live = ballot(valid && !pruned && ql == 0);
    while (live && ns < p.R) {
      const uint32_t g = (uint32_t)__builtin_ctzll(live) >> 2;
      if (qg == g) {
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
          const uint32_t c = ql + 4u * (uint32_t)t;
          if (c < p.nchunks) Scache[(size_t)ns * p.nchunks + c] = xc[t];
        }
        if (ql == 0) {
          S_ids[ns] = cid;
          S_dist[ns] = cd;
        }
      }
      wave_sync();
      uint4 xs[CPL];
      load_cache_frag<CPL>(Scache + (size_t)ns * p.nchunks, ql, p.nchunks, xs);
      const float d = pair_distance<CPL, METRIC>(xc, cf, xs, ql, p.nlimit);
      if (qg > g && d * p.alpha < cd) pruned = true;
      ns += 1;
      live = ballot(valid && !pruned && ql == 0 && qg > g);
    }
  }
  wave_sync();
  return ns;
}

}  // namespace jasper_amd
