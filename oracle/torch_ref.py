"""The reference's torch-level SVOO call on the CPU, in float32: the "reference torch CPU path" the benchmark times
beside the GPU.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: only ``bench.py``'s ``cpu_baseline`` leg and ``tests/``
use it.  It restates, with torch tensor operations on the CPU, what the reference computes on the GPU with
Triton and FlashInfer; no reference code is imported.  Unlike :mod:`oracle.svoo_oracle` (the exact-arithmetic
checker of the HIP kernels) it computes in float32 and uses torch's own kernels (multi-threaded matmuls,
``index_add_``, ``sort``, ``scaled_dot_product_attention``), so it is the throughput a CPU reaches with the
reference's formulation, not a bit-exact contract.  ``tests/test_torch_ref.py`` checks it against the numpy
oracle's float32 contract on small shapes.

Steps of one call (``svoo/models/wan/attention.py:958-1088, 1110-1216``):
  * co-clustering (``svoo/co_clustering.py:2402-2451``): per iteration the key labels by the profile-space
    argmin ``2 - 2 (x C^T / |x C^T|) . P_j`` with ``P = l2norm(K_c Q_c^T)`` (``:2086-2255``), the key centroid
    update (the member mean; an empty cluster keeps its centroid, ``:181-303``), then the query side in the new
    key-centroid space;
  * the block mask (``:556-633``): weighted softmax of ``Q_c K_c^T / sqrt(D)`` by the key cluster sizes, sorted
    descending, top-p with the per-head minimum;
  * stable permutes of Q by query label and K, V by key label, attention of each query cluster over the tokens
    of its kept key clusters (``:949-1108``), the inverse permutation and ``[1, S, H*D]``.
"""

from __future__ import annotations

import math
from typing import Sequence, Tuple

import torch
import torch.nn.functional as F


def _profiles(cent: torch.Tensor, basis: torch.Tensor) -> torch.Tensor:
    """Row-normalised ``cent @ basis^T`` (``svoo/co_clustering.py:2427-2441``): [H, C, B]."""
    p = torch.matmul(cent, basis.transpose(1, 2))
    return p / torch.sqrt((p * p).sum(-1, keepdim=True) + 1e-8)


def _assign(x: torch.Tensor, basis: torch.Tensor, prof: torch.Tensor, chunk: int = 16384) -> torch.Tensor:
    """Profile-space nearest centroid of every token (``svoo/co_clustering.py:2146-2255``): [H, N] int64."""
    h, n, _ = x.shape
    out = torch.empty(h, n, dtype=torch.int64)
    pt = prof.transpose(1, 2)
    for s0 in range(0, n, chunk):
        y = torch.matmul(x[:, s0:s0 + chunk], basis.transpose(1, 2))
        y = y / torch.sqrt((y * y).sum(-1, keepdim=True) + 1e-8)
        dist = 2.0 - 2.0 * torch.matmul(y, pt)
        out[:, s0:s0 + chunk] = dist.argmin(-1)
    return out


def _update(x: torch.Tensor, labels: torch.Tensor, old: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Member means (``svoo/co_clustering.py:181-303``); an empty cluster keeps its old centroid."""
    h, c, d = old.shape
    sums = torch.zeros(h, c, d, dtype=x.dtype)
    counts = torch.zeros(h, c, dtype=torch.int64)
    for hi in range(h):
        sums[hi].index_add_(0, labels[hi], x[hi])
        counts[hi] = torch.bincount(labels[hi], minlength=c)
    new = torch.where(counts[..., None] > 0, sums / counts.clamp(min=1)[..., None].to(x.dtype), old)
    return new, counts


def co_cluster_tokens(q: torch.Tensor, k: torch.Tensor, num_q: int, num_k: int, iters: int,
                      init_q_centroids: torch.Tensor, init_k_centroids: torch.Tensor):
    """[H, N, D] float32 queries and keys -> (q labels, q centroids, q sizes, k labels, k centroids, k sizes)."""
    qc, kc = init_q_centroids.clone(), init_k_centroids.clone()
    ql = kl = qs = ks = None
    for _ in range(iters):
        kl = _assign(k, qc, _profiles(kc, qc))
        kc, ks = _update(k, kl, kc)
        ql = _assign(q, kc, _profiles(qc, kc))
        qc, qs = _update(q, ql, qc)
    return ql, qc, qs, kl, kc, ks


def identify_dynamic_map(qc: torch.Tensor, kc: torch.Tensor, k_sizes: torch.Tensor, p: float,
                         min_kc_ratio: Sequence[float]) -> torch.Tensor:
    """Top-p block map with a per-head minimum (``svoo/co_clustering.py:556-633``): [H, Qc, Kc] bool."""
    h, qn, d = qc.shape
    kn = kc.shape[1]
    if p >= 1.0:
        return torch.ones(h, qn, kn, dtype=torch.bool)
    s = torch.matmul(qc, kc.transpose(1, 2)) / math.sqrt(d)
    w = k_sizes[:, None, :].to(s.dtype) * torch.exp(s - s.max(-1, keepdim=True).values)
    prob = w / w.sum(-1, keepdim=True).clamp(min=1e-12)
    sp, order = torch.sort(prob, dim=-1, descending=True, stable=True)
    remove = torch.cumsum(sp, -1) > p
    remove[..., 1:] = remove[..., :-1].clone()
    remove[..., 0] = False
    for hi in range(h):
        keep = int(float(min_kc_ratio[hi]) * kn)
        if keep > 0:
            remove[hi, :, :keep] = False
    out = torch.zeros(h, qn, kn, dtype=torch.bool)
    out.scatter_(-1, order, ~remove)
    return out


def block_sparse_attention(qp: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, dmap: torch.Tensor,
                           q_sizes: torch.Tensor, k_sizes: torch.Tensor) -> torch.Tensor:
    """Cluster-contiguous [H, S, D] inputs: each query cluster attends the tokens of its kept key clusters
    (``svoo/co_clustering.py:949-1108``); a cluster with none gets zero rows."""
    h, s, d = qp.shape
    out = torch.zeros_like(qp)
    qoff = torch.cat([torch.zeros(h, 1, dtype=torch.int64), torch.cumsum(q_sizes, -1)], -1)
    koff = torch.cat([torch.zeros(h, 1, dtype=torch.int64), torch.cumsum(k_sizes, -1)], -1)
    for hi in range(h):
        key_cluster = torch.repeat_interleave(torch.arange(k_sizes.shape[-1]), k_sizes[hi])
        for i in range(q_sizes.shape[-1]):
            a, e = int(qoff[hi, i]), int(qoff[hi, i + 1])
            if e == a:
                continue
            rows = torch.nonzero(dmap[hi, i][key_cluster]).flatten()
            if rows.numel() == 0:
                continue
            out[hi, a:e] = F.scaled_dot_product_attention(qp[hi, a:e][None], kp[hi, rows][None], vp[hi, rows][None])[0]
    return out


def svoo_attention_call(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, num_q: int, num_k: int,
                        iters: int, top_p: float, min_kc_ratio: Sequence[float], init_q_centroids: torch.Tensor,
                        init_k_centroids: torch.Tensor) -> torch.Tensor:
    """One Wan ``attention_core_logic`` call: [1, H, S, D] float32 in, [1, S, H*D] out."""
    b, h, s, d = query.shape
    q, k, v = query[0], key[0], value[0]
    ql, qc, qs, kl, kc, ks = co_cluster_tokens(q, k, num_q, num_k, iters, init_q_centroids, init_k_centroids)
    qidx = torch.sort(ql, dim=-1, stable=True).indices
    kidx = torch.sort(kl, dim=-1, stable=True).indices
    gather = lambda x, idx: torch.gather(x, 1, idx[..., None].expand(-1, -1, d))  # noqa: E731
    qp, kp, vp = gather(q, qidx), gather(k, kidx), gather(v, kidx)
    dmap = identify_dynamic_map(qc, kc, ks, top_p, min_kc_ratio)
    op = block_sparse_attention(qp, kp, vp, dmap, qs, ks)
    o = torch.empty_like(op).scatter_(1, qidx[..., None].expand(-1, -1, d), op)
    return o.transpose(0, 1).reshape(1, s, h * d)


def hunyuan_attention_call(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, num_q: int, num_k: int,
                           iters: int, top_p: float, min_kc_ratio: Sequence[float], prompt_length: int,
                           context_length: int, init_q_centroids: torch.Tensor,
                           init_k_centroids: torch.Tensor) -> torch.Tensor:
    """One HunyuanVideo ``attention_core_logic`` call (``svoo/models/hunyuan10/attention.py:977-1110``): the video
    part clustered and masked, the prompt (a cluster attending and attended by everything) and the padding (a
    cluster of itself) appended; [1, H, S, D] float32 in, [1, H, S, D] out."""
    b, h, s, d = query.shape
    vl = s - context_length
    q, k, v = query[0], key[0], value[0]
    ql, qc, qs, kl, kc, ks = co_cluster_tokens(q[:, :vl], k[:, :vl], num_q, num_k, iters, init_q_centroids,
                                               init_k_centroids)
    dmap = identify_dynamic_map(qc, kc, ks, top_p, min_kc_ratio)
    m2 = torch.zeros(h, num_q + 2, num_k + 2, dtype=torch.bool)
    m2[:, :num_q, :num_k] = dmap
    m2[:, num_q, :num_k + 1] = True
    m2[:, :num_q + 1, num_k] = True
    m2[:, num_q + 1, num_k + 1] = True
    tail = torch.tensor([prompt_length, context_length - prompt_length], dtype=torch.int64).expand(h, 2)
    qs2, ks2 = torch.cat([qs, tail], -1), torch.cat([ks, tail], -1)
    text = torch.arange(vl, s).expand(h, context_length)
    qidx = torch.cat([torch.sort(ql, dim=-1, stable=True).indices, text], -1)
    kidx = torch.cat([torch.sort(kl, dim=-1, stable=True).indices, text], -1)
    gather = lambda x, idx: torch.gather(x, 1, idx[..., None].expand(-1, -1, d))  # noqa: E731
    op = block_sparse_attention(gather(q, qidx), gather(k, kidx), gather(v, kidx), m2, qs2, ks2)
    return torch.empty_like(op).scatter_(1, qidx[..., None].expand(-1, -1, d), op)[None]
