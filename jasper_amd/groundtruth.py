"""Exact brute-force k-NN ground truth (reference python/jasper/__init__.py:828-926).

Same arithmetic as the reference utility: L2 distances as
||q||^2 + ||v||^2 - 2 q.v in float32, clamped at 0; inner product as -(q.v)
with float16 inputs; a running top-k over streamed vector batches.
"""

from __future__ import annotations

import torch


def generate_groundtruth(vectors: torch.Tensor, queries: torch.Tensor, k: int = 100,
                         distance: str = "l2", query_batch_size: int = 1024,
                         vector_batch_size: int = 100_000, device: str = "cuda",
                         verbose: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    assert vectors.dtype in (torch.float32, torch.float16)
    assert queries.dtype in (torch.float32, torch.float16)
    assert vectors.size(1) == queries.size(1)
    use_fp16 = vectors.dtype == torch.float16 and queries.dtype == torch.float16
    compute_dtype = torch.float16 if (use_fp16 and distance == "ip") else torch.float32
    n, _ = vectors.shape
    nq = queries.size(0)
    final_ids = torch.empty(nq, k, dtype=torch.int32)
    final_dists = torch.empty(nq, k, dtype=torch.float32)
    v_sq_all = None
    for q_start in range(0, nq, query_batch_size):
        q_end = min(q_start + query_batch_size, nq)
        q_batch = queries[q_start:q_end].to(device=device, dtype=compute_dtype)
        qbs = q_batch.size(0)
        if distance == "l2":
            q_sq = (q_batch * q_batch).sum(dim=1, keepdim=True)
        top_dists = torch.full((qbs, k), float("inf"), dtype=torch.float32, device=device)
        top_ids = torch.zeros((qbs, k), dtype=torch.int64, device=device)
        for v_start in range(0, n, vector_batch_size):
            v_end = min(v_start + vector_batch_size, n)
            v_batch = vectors[v_start:v_end].to(device=device, dtype=compute_dtype)
            if distance == "l2":
                v_sq = (v_batch * v_batch).sum(dim=1)
                dists = q_sq + v_sq.unsqueeze(0) - 2.0 * (q_batch @ v_batch.T)
                dists.clamp_(min=0.0)
            elif distance == "ip":
                dists = -(q_batch @ v_batch.T)
            else:
                raise ValueError(f"Unknown distance: {distance}")
            dists = dists.float()
            local_ids = torch.arange(v_start, v_end, device=device).unsqueeze(0).expand(qbs, -1)
            merged_d = torch.cat([top_dists, dists], dim=1)
            merged_i = torch.cat([top_ids, local_ids], dim=1)
            top_dists, sel = merged_d.topk(k, dim=1, largest=False)
            top_ids = merged_i.gather(1, sel)
            del v_batch, dists, local_ids, merged_d, merged_i, sel
        final_ids[q_start:q_end] = top_ids.to(torch.int32).cpu()
        final_dists[q_start:q_end] = top_dists.cpu()
        if verbose:
            print(f"\r[groundtruth] {q_end}/{nq} queries", end="", flush=True)
    if verbose:
        print()
    del v_sq_all
    return final_ids, final_dists
