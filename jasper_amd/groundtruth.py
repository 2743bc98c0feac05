"""Exact brute-force k-NN ground truth (reference python/jasper/__init__.py:828-926).

Same arithmetic as the reference utility: L2 distances as
(||q||^2 + ||v||^2) - 2 q.v in float32, clamped at 0; inner product as
-(q.v) where fp16 inputs give an fp16 matmul result. Results are ordered by
(distance, id).

fp16 inputs with k <= 64 and dim <= 512 run on the matrix-core kernel of the
HIP library (`jasperx_bruteforce_knn`), with the whole base resident in HBM.
Other inputs (fp32 data, larger k or dim, or device="cpu") use the
reference's formulation in torch, streaming vector batches.
"""

from __future__ import annotations

import torch

_HIP_MAX_K = 64
_HIP_MAX_DIM = 512


def _padded_rows(x: torch.Tensor, dp: int, device) -> torch.Tensor:
    if (x.dtype == torch.float16 and x.device == torch.device(device) and x.size(1) == dp
            and x.is_contiguous() and x.data_ptr() % 16 == 0):
        return x
    out = torch.zeros((x.size(0), dp), dtype=torch.float16, device=device)
    out[:, :x.size(1)] = x.to(device=device, dtype=torch.float16)
    return out


def bruteforce_knn(vectors: torch.Tensor, queries: torch.Tensor, k: int, distance: str = "l2",
                   device: str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """k nearest base rows per query on the matrix cores; fp16 inputs,
    k <= 64, dim <= 512. Returns device tensors (int32 ids [nq, k], float32
    distances [nq, k]); missing neighbours are (-1, FLT_MAX)."""
    from . import _agnostic, _stream_ptr, _tensor_ptr
    if vectors.dtype != torch.float16 or queries.dtype != torch.float16:
        raise ValueError("bruteforce_knn takes float16 vectors and queries")
    if distance not in ("l2", "ip"):
        raise ValueError(f"Unknown distance: {distance}")
    n, dim = vectors.shape
    nq = queries.size(0)
    if queries.size(1) != dim:
        raise ValueError("vectors and queries differ in dim")
    if not (0 < k <= _HIP_MAX_K) or dim > _HIP_MAX_DIM:
        raise ValueError(f"bruteforce_knn supports 1 <= k <= {_HIP_MAX_K} and dim <= {_HIP_MAX_DIM}")
    dev = torch.device(device)
    dp = (dim + 7) // 8 * 8
    base = _padded_rows(vectors, dp, dev)
    qs = _padded_rows(queries, dp, dev)
    ids = torch.empty((nq, k), dtype=torch.int32, device=dev)
    dists = torch.empty((nq, k), dtype=torch.float32, device=dev)
    if nq:
        _agnostic("jasperx_bruteforce_knn")(_tensor_ptr(base), n, dim, dp, _tensor_ptr(qs), nq, dp, k,
                                            0 if distance == "l2" else 1, _tensor_ptr(ids), _tensor_ptr(dists),
                                            _stream_ptr(dev))
    return ids, dists


def generate_groundtruth(vectors: torch.Tensor, queries: torch.Tensor, k: int = 100,
                         distance: str = "l2", query_batch_size: int = 1024,
                         vector_batch_size: int = 100_000, device: str = "cuda",
                         verbose: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (int32 ids [nq, k], float32 distances [nq, k]) on the CPU."""
    assert vectors.dtype in (torch.float32, torch.float16)
    assert queries.dtype in (torch.float32, torch.float16)
    assert vectors.size(1) == queries.size(1)
    n, dim = vectors.shape
    nq = queries.size(0)
    if (torch.device(device).type == "cuda" and vectors.dtype == torch.float16
            and queries.dtype == torch.float16 and k <= _HIP_MAX_K and dim <= _HIP_MAX_DIM and n > 0):
        ids, d = bruteforce_knn(vectors, queries, k, distance, device)
        if verbose:
            print(f"[groundtruth] done — {nq} queries, {n} vectors, k={k}")
        return ids.cpu(), d.cpu()

    use_fp16 = vectors.dtype == torch.float16 and queries.dtype == torch.float16
    compute_dtype = torch.float16 if (use_fp16 and distance == "ip") else torch.float32
    final_ids = torch.empty(nq, k, dtype=torch.int32)
    final_dists = torch.empty(nq, k, dtype=torch.float32)
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
            # (distance, id) order: stable sort by id, then by distance
            order = torch.argsort(merged_i, dim=1, stable=True)
            merged_d = merged_d.gather(1, order)
            merged_i = merged_i.gather(1, order)
            order = torch.argsort(merged_d, dim=1, stable=True)[:, :k]
            top_dists = merged_d.gather(1, order)
            top_ids = merged_i.gather(1, order)
            del v_batch, dists, local_ids, merged_d, merged_i, order
        final_ids[q_start:q_end] = top_ids.to(torch.int32).cpu()
        final_dists[q_start:q_end] = top_dists.cpu()
        if verbose:
            print(f"\r[groundtruth] {q_end}/{nq} queries", end="", flush=True)
    if verbose:
        print()
    return final_ids, final_dists
