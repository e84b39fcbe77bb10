"""EAR: error-aware block routing with centroid compensation, on MI355X.

Names, arguments and results follow the EAR functions of ``svoo/co_clustering.py`` (lines
1314-2050) and the value-centroid helper of ``svoo/models/wan/attention.py:593-610``:

* :func:`error_estimation_triton` - per (query cluster i, key cluster j) the log error of replacing
  the tokens of key cluster j by its centroid pair, minus ``gamma`` log block area;
* :func:`identify_dynamic_map_estimated` - the area budget from centroid attention and the greedy
  selection by that efficiency;
* :func:`dynamic_block_sparse_prune_fwd_flashinfer` - attention over the selected token blocks with
  the pruned clusters compensated by their (key, value) centroids, in one HIP kernel (the reference
  runs FlashInfer with ``return_lse`` and merges in a second Triton kernel).

Everything runs as HIP kernels through the C ABI (``include/svoo_hip.h``); only the per-head
minimum counts are derived on the host, as the reference also does.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .co_clustering import _bf16_value, _check_host_sizes, _ratio_values

__all__ = [
    "ear_row_params",
    "value_centroids_from_permuted",
    "compute_value_centroids",
    "centroid_logits",
    "error_estimation_triton",
    "identify_dynamic_map_estimated",
    "dynamic_block_sparse_prune_fwd",
    "dynamic_block_sparse_prune_fwd_flashinfer",
]

EAR_EPS = 1e-8  # identify_dynamic_map_estimated's eps (svoo/co_clustering.py:1725)


def _bf16_4d(x: torch.Tensor, name: str) -> torch.Tensor:
    """``x [B, H, N, D]`` (D <= 128) as the kernels' bf16 operand ``[B, H, N, 128]`` (fp16 / fp32 rounded to bf16,
    to nearest even; columns past D zero)."""
    if isinstance(x, torch.Tensor) and x.dim() != 4:
        raise ValueError(f"{name}: expected [B, H, N, D], got {tuple(x.shape)}")
    return _lib.as_rows128(x, name).contiguous()


def _sizes(x: torch.Tensor, dev, bh: int, n: int) -> torch.Tensor:
    return x.to(device=dev, dtype=torch.int32).reshape(bh, n).contiguous()


def _offsets(ks: torch.Tensor) -> torch.Tensor:
    """Exclusive prefix of int32 sizes ``[BH, K]``."""
    return (torch.cumsum(ks, dim=-1, dtype=torch.int32) - ks).contiguous()


def ear_row_params(h: int, kc_num: int, min_kc_ratio=0.0) -> Tuple[list, list]:
    """Per-head ``(preserve, budget_preserve)`` of the EAR selection (``svoo/co_clustering.py:1740-1781``):
    ``max(1, int(r * Kc))`` and ``max(1, int(r * Kc * 2))`` for ``r > 0``.  A tensor or sequence of H
    ratios is read through float32; one of length 1, or a number, in double precision; other lengths
    give no minimum."""
    if isinstance(min_kc_ratio, torch.Tensor):
        n = min_kc_ratio.numel()
        if n == h:
            rs = _ratio_values(min_kc_ratio.flatten(), h)
        elif n == 1:
            rs = [float(min_kc_ratio.item())] * h
        else:
            rs = [0.0] * h
    elif isinstance(min_kc_ratio, (list, tuple)):
        if len(min_kc_ratio) == h:
            rs = _ratio_values(min_kc_ratio, h)
        elif len(min_kc_ratio) == 1:
            rs = [float(min_kc_ratio[0])] * h
        else:
            rs = [0.0] * h
    elif isinstance(min_kc_ratio, (int, float)):
        rs = [float(min_kc_ratio)] * h
    else:
        rs = [0.0] * h
    pre = [max(1, int(r * kc_num)) if r > 0 else 0 for r in rs]
    bpre = [max(1, int(r * kc_num * 2)) if r > 0 else 0 for r in rs]
    return pre, bpre


# ------------------------------------------------------------------------------------------------ value side
def _value_stats(v_perm: torch.Tensor, ks: torch.Tensor, koff: torch.Tensor, vc: Optional[torch.Tensor]):
    bh, n, d = v_perm.shape
    kn = ks.shape[-1]
    dev = v_perm.device
    compute = vc is None
    vc_out = torch.empty(bh, kn, d, dtype=torch.bfloat16, device=dev) if compute else vc.reshape(bh, kn, d).contiguous()
    vc_sq = torch.empty(bh, kn, dtype=torch.float32, device=dev)
    stats = torch.empty(bh, n, 2, dtype=torch.float32, device=dev)
    _lib.call("svoo_ear_value_stats", v_perm.data_ptr(), koff.data_ptr(), ks.data_ptr(), bh, n, kn, d, int(compute),
              vc_out.data_ptr(), vc_sq.data_ptr(), stats.data_ptr(), _lib.stream_of(dev))
    return vc_out, vc_sq, stats


def value_centroids_from_permuted(v_perm: torch.Tensor, k_cluster_sizes: torch.Tensor) -> torch.Tensor:
    """Value centroids ``[B, H, Kc, D]`` of cluster-contiguous values ``v_perm [B, H, S, D]``:
    ``bf16(bf16(member sum) / bf16(max(|K_j|, 1)))``, zero for an empty cluster; in v_perm's dtype."""
    vp = _bf16_4d(v_perm, "v_perm")
    b, h, s, d = vp.shape
    kn = k_cluster_sizes.shape[-1]
    ks = _sizes(k_cluster_sizes, vp.device, b * h, kn)
    vc, _, _ = _value_stats(vp.reshape(b * h, s, d), ks, _offsets(ks), None)
    return _lib.from_rows128(vc.reshape(b, h, kn, d), v_perm.shape[-1], v_perm.dtype)


def compute_value_centroids(tokens: torch.Tensor, labels: torch.Tensor, cluster_sizes: torch.Tensor,
                            num_clusters: int) -> torch.Tensor:
    """``_compute_value_centroids`` (``svoo/models/wan/attention.py:593-610``) from unpermuted tokens
    ``[BH, S, D]`` and their key labels ``[BH, S]``: ``[BH, Kc, D]``."""
    from .permute import cluster_sort

    _lib.require_gpu_tensor(tokens, "tokens")
    bh, s, d = tokens.shape
    sorted_idx, sizes, _ = cluster_sort(labels.reshape(bh, s), num_clusters)
    vp = torch.empty(bh, s, d, dtype=tokens.dtype, device=tokens.device)
    tok = tokens.contiguous()
    _lib.call("svoo_permute_rows", tok.data_ptr(), sorted_idx.data_ptr(), vp.data_ptr(), bh, s, s,
              d * tok.element_size(), _lib.stream_of(tok.device))
    return value_centroids_from_permuted(vp.reshape(1, bh, s, d), sizes.reshape(1, bh, num_clusters))[0]


# ------------------------------------------------------------------------------------------------ scores
def centroid_logits(query_centroids: torch.Tensor, key_centroids: torch.Tensor) -> torch.Tensor:
    """``einsum("bhqd,bhkd->bhqk", Qc, Kc) * D**-0.5`` on bf16 centroids (``co_clustering.py:1725``):
    the exact dot rounded to bf16, times ``float32(D**-0.5)``, rounded to bf16."""
    c = _centroid_logits(_bf16_4d(query_centroids, "query_centroids"), _bf16_4d(key_centroids, "key_centroids"),
                         query_centroids.shape[-1])
    return _lib.convert(c, query_centroids.dtype)


def _centroid_logits(qc: torch.Tensor, kc: torch.Tensor, hd: int) -> torch.Tensor:
    """The bf16 logits of padded centroids ``[B, H, *, 128]`` with the scale of head dim ``hd``."""
    b, h, qn, _ = qc.shape
    kn = kc.shape[2]
    c = torch.empty(b, h, qn, kn, dtype=torch.bfloat16, device=qc.device)
    _lib.call("svoo_ear_centroid_logits", qc.data_ptr(), kc.data_ptr(), b * h, qn, kn, hd, c.data_ptr(),
              _lib.stream_of(qc.device))
    return c


def _efficiency(qc, kp, c, stats, vc_sq, qs, ks, koff, gamma: float, eps: float, hd: int) -> torch.Tensor:
    b, h, qn, _ = qc.shape
    n = kp.shape[2]
    kn = ks.shape[-1]
    eff = torch.empty(b, h, qn, kn, dtype=torch.float32, device=qc.device)
    _lib.call("svoo_ear_efficiency", qc.data_ptr(), kp.data_ptr(), c.contiguous().data_ptr(), stats.data_ptr(),
              vc_sq.data_ptr(), qs.data_ptr(), ks.data_ptr(), koff.data_ptr(), b * h, n, qn, kn, hd, float(gamma),
              float(eps), eff.data_ptr(), _lib.stream_of(qc.device))
    return eff


def error_estimation_triton(query_centroids, key_centroids, value_centroids, permuted_K, permuted_V, qc_sz, kc_sz,
                            c_logits, gamma: float, eps: float, BLOCK_SIZE_Q: int = 64, BLOCK_SIZE_K: int = 32):
    """Log-efficiency scores ``[B, H, Qc, Kc]`` (fp32) for every (query cluster, key cluster) pair
    (``svoo/co_clustering.py:1570-1689``).  ``BLOCK_SIZE_*`` are accepted for signature compatibility;
    the HIP kernels choose their own tiles."""
    qc = _bf16_4d(query_centroids, "query_centroids")
    kp = _bf16_4d(permuted_K, "permuted_K")
    vp = _bf16_4d(permuted_V, "permuted_V")
    b, h, qn, d = qc.shape
    s = kp.shape[2]
    kn = key_centroids.shape[2]
    dev = qc.device
    ks = _sizes(kc_sz, dev, b * h, kn)
    qs = _sizes(qc_sz, dev, b * h, qn)
    koff = _offsets(ks)
    vc = _bf16_4d(value_centroids, "value_centroids")
    _, vc_sq, stats = _value_stats(vp.reshape(b * h, s, d), ks, koff, vc)
    c = _lib.as_bf16(c_logits, "c_logits").contiguous()
    return _efficiency(qc, kp, c, stats, vc_sq, qs, ks, koff, gamma, eps, query_centroids.shape[-1])


# ------------------------------------------------------------------------------------------------ selection
def _select(c, eff, qs, ks, b, h, qn, kn, top_p: float, min_kc_ratio) -> torch.Tensor:
    dev = eff.device
    pre, bpre = ear_row_params(h, kn, min_kc_ratio)
    pc = torch.tensor(pre + bpre, dtype=torch.int32).to(dev, non_blocking=True)
    dmap = torch.empty(b, h, qn, kn, dtype=torch.bool, device=dev)
    _lib.call("svoo_ear_select", c.data_ptr(), eff.data_ptr(), qs.data_ptr(), ks.data_ptr(), pc.data_ptr(),
              pc[h:].data_ptr(), b, h, qn, kn, _bf16_value(top_p), dmap.data_ptr(), _lib.stream_of(dev))
    return dmap


@torch.inference_mode()
def identify_dynamic_map_estimated(q_perm, k_perm, v_perm, qc_sz, kc_sz, qcentroids, kcentroids, vcentroids,
                                   top_p=0.9, gamma=1.0, min_kc_ratio=0.0):
    """EAR block map ``bool [B, H, Qc, Kc]`` (``svoo/co_clustering.py:1692-1797``).

    Budget: the area of the top-``top_p`` prefix (at least ``2 r Kc`` clusters) of the centroid
    attention weighted by key-cluster size; the first ``r Kc`` of that order are kept; the others are
    added in descending estimated-error efficiency while the area before them is below the remaining
    budget.  Sorts are stable (ties to the lower cluster index) and areas exact integers.
    """
    qc = _bf16_4d(qcentroids, "qcentroids")
    b, h, qn, d = qc.shape
    kn = kcentroids.shape[2]
    dev = qc.device
    kp = _bf16_4d(k_perm, "k_perm")
    vp = _bf16_4d(v_perm, "v_perm")
    s = kp.shape[2]
    ks = _sizes(kc_sz, dev, b * h, kn)
    qs = _sizes(qc_sz, dev, b * h, qn)
    koff = _offsets(ks)
    hd = qcentroids.shape[-1]
    c = _centroid_logits(qc, _bf16_4d(kcentroids, "kcentroids"), hd)
    vc = _bf16_4d(vcentroids, "vcentroids")
    _, vc_sq, stats = _value_stats(vp.reshape(b * h, s, d), ks, koff, vc)
    eff = _efficiency(qc, kp, c, stats, vc_sq, qs, ks, koff, gamma, EAR_EPS, hd)
    return _select(c, eff, qs, ks, b, h, qn, kn, top_p, min_kc_ratio)


def ear_map_and_value_centroids(q_perm, k_perm, v_perm, qc_sz, kc_sz, qcentroids, kcentroids, top_p=0.9,
                                gamma=1.0, min_kc_ratio=0.0, return_parts: bool = False):
    """Value centroids and EAR map in one pass over ``v_perm`` (the processor's path): returns
    ``(v_centroids [B, H, Kc, D] in v_perm's dtype, map)``, plus ``{"c", "eff"}`` with ``return_parts``."""
    qc = _bf16_4d(qcentroids, "qcentroids")
    b, h, qn, d = qc.shape
    kn = kcentroids.shape[2]
    dev = qc.device
    kp = _bf16_4d(k_perm, "k_perm")
    vp = _bf16_4d(v_perm, "v_perm")
    s = kp.shape[2]
    ks = _sizes(kc_sz, dev, b * h, kn)
    qs = _sizes(qc_sz, dev, b * h, qn)
    koff = _offsets(ks)
    vc, vc_sq, stats = _value_stats(vp.reshape(b * h, s, d), ks, koff, None)
    hd = qcentroids.shape[-1]
    c = _centroid_logits(qc, _bf16_4d(kcentroids, "kcentroids"), hd)
    eff = _efficiency(qc, kp, c, stats, vc_sq, qs, ks, koff, gamma, EAR_EPS, hd)
    dmap = _select(c, eff, qs, ks, b, h, qn, kn, top_p, min_kc_ratio)
    vc = _lib.from_rows128(vc.reshape(b, h, kn, d), v_perm.shape[-1], v_perm.dtype)
    if return_parts:
        return vc, dmap, {"c": c, "eff": eff}
    return vc, dmap


# ------------------------------------------------------------------------------------------------ attention
def dynamic_block_sparse_prune_fwd(q, k, v, k_centroids, v_centroids, block_mask_map, block_row_sz, block_col_sz,
                                   *, validate: bool = True):
    """Compensated variable-block-sparse attention ``[B, H, S, D]``.

    Query cluster ``i`` attends, in one softmax, to the tokens of its active key clusters and to the
    centroid pairs ``(Kc_j, Vc_j)`` of its inactive ones with logit ``q . Kc_j / sqrt(D) +
    log(|K_j| + 1e-6)``.  With ``validate`` the sizes of every head must sum to ``S``; host-side sizes
    are checked before the launch, and without ``validate`` inconsistent device sizes give NaN rows."""
    assert q.is_cuda and k.is_cuda and v.is_cuda, "Inputs must be CUDA tensors"
    assert q.dtype == k.dtype == v.dtype, "Input dtypes must match"
    in_dtype, hd = q.dtype, q.shape[-1]
    assert k_centroids.shape[-1] == hd and v_centroids.shape[-1] == hd, "centroids must have the head dim of q"
    q, k, v = (_lib.as_rows128(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    b, h, s, d = q.shape
    qn = block_row_sz.shape[-1]
    kn = block_col_sz.shape[-1]
    assert k.shape == q.shape and v.shape == q.shape, "q, k, v must share one shape"
    assert block_mask_map.shape == (b, h, qn, kn)
    assert k_centroids.shape == (b, h, kn, hd) and v_centroids.shape == (b, h, kn, hd)
    _check_host_sizes(block_row_sz, s, "block_row_sz")
    _check_host_sizes(block_col_sz, s, "block_col_sz")
    dev = q.device
    bh = b * h
    qq, kk, vv = (t.reshape(bh, s, d).contiguous() for t in (q, k, v))
    kc = _bf16_4d(k_centroids, "k_centroids")
    vc = _bf16_4d(v_centroids, "v_centroids")
    m = block_mask_map.to(device=dev, dtype=torch.bool).reshape(bh, qn, kn).contiguous()
    qs = _sizes(block_row_sz, dev, bh, qn)
    ks = _sizes(block_col_sz, dev, bh, kn)
    out = torch.empty_like(qq)
    L = _lib.lib()
    ws = _lib.workspace(L.svoo_vbsa_workspace_size(bh, s, qn, kn), dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if validate else None
    _lib.call("svoo_vbsa_ear_fwd", qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), kc.data_ptr(), vc.data_ptr(),
              m.data_ptr(), qs.data_ptr(), ks.data_ptr(), out.data_ptr(), bh, s, hd, qn, kn, ws.data_ptr(), ws.numel(),
              _lib.ptr(status), _lib.stream_of(dev))
    if validate and int(status.item()) != 0:
        raise AssertionError("cluster sizes of every head must sum to S (block_row_sz / block_col_sz)")
    return _lib.from_rows128(out.reshape(b, h, s, d), hd, in_dtype)


def dynamic_block_sparse_prune_fwd_flashinfer(q, k, v, k_centroids, v_centroids, block_mask_map, block_row_sz,
                                              block_col_sz, is_cpu: bool = True):
    """Drop-in for ``dynamic_block_sparse_prune_fwd_flashinfer`` (``svoo/co_clustering.py:1924-2050``): the
    reference's size asserts hold; ``is_cpu`` only says where the map and sizes live."""
    return dynamic_block_sparse_prune_fwd(q, k, v, k_centroids, v_centroids, block_mask_map, block_row_sz,
                                          block_col_sz, validate=True)
