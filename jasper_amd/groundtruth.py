"""Exact brute-force k-NN ground truth (reference python/jasper/__init__.py:828-926).

Same arithmetic as the reference utility: L2 distances as
(||q||^2 + ||v||^2) - 2 q.v in float32, clamped at 0; inner product as
-(q.v) where fp16 inputs give an fp16 matmul result. Results are ordered by
(distance, id).

fp16 inputs with k <= 128 and dim <= 4096 (the reference's default k = 100
and config 4's dim 960 included) run on the matrix-core kernel of the HIP
library (`jasperx_bruteforce_knn`), with the whole base resident in HBM.
Other inputs (fp32 data, larger k or dim, or device="cpu") take a torch
path that streams query and base blocks with the same arithmetic and keeps
the k nearest of each query as (distance, id) keys.
"""

from __future__ import annotations

import torch

_HIP_MAX_K = 128
_HIP_MAX_DIM = 4096


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
    k <= 128, dim <= 4096. Returns device tensors (int32 ids [nq, k], float32
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

    return _keyed_knn(vectors, queries, k, distance, torch.device(device), query_batch_size,
                      vector_batch_size, verbose)


# Keys for the (distance, id) order: the float's bits mapped to a signed int32
# that orders like the float (negative values have their magnitude bits
# flipped), shifted above the 32-bit id. Keys are unique, so the k smallest
# keys are the k nearest rows in (distance, id) order whatever order topk
# visits ties in.
_NO_KEY = torch.iinfo(torch.int64).max


def _to_keys(d: torch.Tensor, first_id: int) -> torch.Tensor:
    bits = (d + 0.0).contiguous().view(torch.int32)  # + 0.0 folds -0.0 into +0.0
    bits = torch.where(bits < 0, bits ^ 0x7FFFFFFF, bits).to(torch.int64)
    ids = torch.arange(first_id, first_id + d.size(1), dtype=torch.int64, device=d.device)
    return (bits << 32) | ids.unsqueeze(0)


def _from_keys(keys: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    missing = keys == _NO_KEY
    bits = (keys >> 32).to(torch.int32)
    bits = torch.where(bits < 0, bits ^ 0x7FFFFFFF, bits)
    d = bits.view(torch.float32).masked_fill(missing, torch.finfo(torch.float32).max)
    ids = (keys & 0xFFFFFFFF).to(torch.int32).masked_fill(missing, -1)
    return ids, d


def _block_distances(q: torch.Tensor, q_sq, v: torch.Tensor, distance: str) -> torch.Tensor:
    """Distances of a query block to a base block with the ground-truth
    arithmetic: L2 = (|q|^2 + |v|^2) - 2 q.v in float32 clamped at 0;
    IP = -(q.v) in the operands' precision (an fp16 product for fp16
    inputs), then widened to float32."""
    if distance == "l2":
        v_sq = (v * v).sum(dim=1)
        return (q_sq + v_sq[None, :] - 2.0 * (q @ v.T)).clamp_(min=0.0)
    return (-(q @ v.T)).float()


def _keyed_knn(vectors, queries, k, distance, dev, q_step, v_step, verbose):
    if distance not in ("l2", "ip"):
        raise ValueError(f"Unknown distance: {distance}")
    # fp16 inner products stay fp16, everything else is computed in float32
    fp16_ip = distance == "ip" and vectors.dtype == queries.dtype == torch.float16
    dtype = torch.float16 if fp16_ip else torch.float32
    n, nq = vectors.size(0), queries.size(0)
    out_ids = torch.empty((nq, k), dtype=torch.int32)
    out_d = torch.empty((nq, k), dtype=torch.float32)
    for q0 in range(0, nq, q_step):
        q = queries[q0:q0 + q_step].to(device=dev, dtype=dtype)
        q_sq = (q * q).sum(dim=1, keepdim=True) if distance == "l2" else None
        best = torch.full((q.size(0), k), _NO_KEY, dtype=torch.int64, device=dev)
        for v0 in range(0, n, v_step):
            v = vectors[v0:v0 + v_step].to(device=dev, dtype=dtype)
            keys = torch.cat([best, _to_keys(_block_distances(q, q_sq, v, distance), v0)], dim=1)
            best = torch.topk(keys, k, dim=1, largest=False, sorted=True).values
        ids, d = _from_keys(best)
        out_ids[q0:q0 + q.size(0)] = ids.cpu()
        out_d[q0:q0 + q.size(0)] = d.cpu()
        if verbose:
            print(f"\r[groundtruth] {q0 + q.size(0)}/{nq} queries", end="", flush=True)
    if verbose:
        print()
    return out_ids, out_d
