"""SVOO hot-path operators on MI355X: co-clustering, block mask, variable-block-sparse attention.

Names, arguments and return values follow ``svoo/co_clustering.py`` of the reference so that the
functions drop into the same call sites.  Every function enqueues HIP kernels on the current
stream through the C ABI (``include/svoo_hip.h``); nothing here computes on the host except the
per-head keep/cap counts of the mask, which the reference also derives on the host.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

__all__ = [
    "co_cluster_tokens",
    "co_cluster_tokens_full",
    "cocluster_profile",
    "cocluster_assign",
    "centroid_update",
    "triton_l2norm_forward",
    "weighted_softmax",
    "mask_row_params",
    "identify_dynamic_map",
    "block_mask_lengths",
    "dynamic_block_sparse_fwd",
    "dynamic_block_sparse_fwd_fused",
    "dynamic_block_sparse_fwd_flashinfer",
    "dynamic_block_sparse_fwd_triton",
    "vbsa_segments",
]

_ASSIGN_CHUNK = 64  # E rows staged per step by the assign kernel; padded cluster counts are multiples of it


def _pad(v: int, m: int = _ASSIGN_CHUNK) -> int:
    return (v + m - 1) // m * m


def _bf16_3d(x: torch.Tensor, name: str) -> torch.Tensor:
    """``x [BH, N, D]`` (D <= 128) as the kernels' bf16 operand ``[BH, N, 128]`` (fp16 / fp32 rounded to bf16, to
    nearest even; columns past D zero, which leaves every dot, centroid and label as on the D columns)."""
    if isinstance(x, torch.Tensor) and x.dim() != 3:
        raise ValueError(f"{name}: expected [BH, N, D], got {tuple(x.shape)}")
    return _lib.as_rows128(x, name).contiguous()


# ------------------------------------------------------------------------------------------------
# Co-clustering
# ------------------------------------------------------------------------------------------------
def _gather_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """``x[b, idx[b, c]]`` for ``x [BH, N, D]`` and ``idx [BH, C]`` via the HIP row gather."""
    bh, n, d = x.shape
    c = idx.shape[1]
    idx32 = idx.to(device=x.device, dtype=torch.int32).contiguous()
    out = torch.empty(bh, c, d, dtype=x.dtype, device=x.device)
    _lib.call("svoo_permute_rows", x.data_ptr(), idx32.data_ptr(), out.data_ptr(), bh, n, c, d * x.element_size(),
              _lib.stream_of(x.device))
    return out


def co_cluster_tokens_full(
    q_flat: torch.Tensor,
    k_flat: torch.Tensor,
    num_q_centroids: int,
    num_k_centroids: int,
    max_iters: int = 10,
    *,
    init_q_idx: Optional[torch.Tensor] = None,
    init_k_idx: Optional[torch.Tensor] = None,
    init_q_centroids: Optional[torch.Tensor] = None,
    init_k_centroids: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
) -> dict:
    """:func:`co_cluster_tokens` returning every device output in a dict.

    Keys: ``qlabels, klabels`` (int32), ``qcentroids, kcentroids`` (in the tokens' dtype), ``qsizes, ksizes``,
    ``q_sorted_idx, k_sorted_idx`` and ``q_offsets, k_offsets`` (int32; the stable cluster sort of
    the final labels, ready for the permutes).  fp16 / fp32 tokens and centroids are rounded to bf16, the type
    the kernels compute in; the centroids come back in the tokens' dtype (bf16 values).
    """
    assert q_flat.shape == k_flat.shape, "q_flat and k_flat must have the same shape"
    q = _bf16_3d(q_flat, "q_flat")
    k = _bf16_3d(k_flat, "k_flat")
    if max_iters < 1:
        # svoo/co_clustering.py:2451 returns qlabels, which the loop never bound.
        raise UnboundLocalError("co_cluster_tokens needs max_iters >= 1")
    bh, n, d = q.shape
    hd = q_flat.shape[-1]
    dev = q.device

    def _init(x, idx, cents, nc):
        if cents is not None:
            c = _lib.as_rows128(cents.to(device=dev).reshape(bh, nc, hd), "init centroids")
            return c.clone()
        if idx is None:
            # svoo/co_clustering.py:2417-2421: uniform random token indices (with replacement).
            idx = torch.randint(0, n, (bh, nc), device=dev, generator=generator)
        return _gather_rows(x, idx.reshape(bh, nc))

    qc = _init(q, init_q_idx, init_q_centroids, num_q_centroids).contiguous()
    kc = _init(k, init_k_idx, init_k_centroids, num_k_centroids).contiguous()
    i32 = dict(dtype=torch.int32, device=dev)
    out = dict(
        qlabels=torch.empty(bh, n, **i32), klabels=torch.empty(bh, n, **i32),
        qsizes=torch.empty(bh, num_q_centroids, **i32), ksizes=torch.empty(bh, num_k_centroids, **i32),
        q_sorted_idx=torch.empty(bh, n, **i32), k_sorted_idx=torch.empty(bh, n, **i32),
        q_offsets=torch.empty(bh, num_q_centroids, **i32), k_offsets=torch.empty(bh, num_k_centroids, **i32),
    )
    L = _lib.lib()
    ws = _lib.workspace(L.svoo_co_cluster_workspace_size(bh, n, num_q_centroids, num_k_centroids, d), dev)
    _lib.call(
        "svoo_co_cluster", q.data_ptr(), k.data_ptr(), bh, n, hd, num_q_centroids, num_k_centroids, max_iters,
        qc.data_ptr(), kc.data_ptr(), out["qlabels"].data_ptr(), out["klabels"].data_ptr(), out["qsizes"].data_ptr(),
        out["ksizes"].data_ptr(), out["q_sorted_idx"].data_ptr(), out["k_sorted_idx"].data_ptr(),
        out["q_offsets"].data_ptr(), out["k_offsets"].data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(dev),
    )
    out["qcentroids"] = _lib.from_rows128(qc, hd, q_flat.dtype)
    out["kcentroids"] = _lib.from_rows128(kc, hd, q_flat.dtype)
    return out


def co_cluster_tokens(
    q_flat,
    k_flat,
    num_q_centroids,
    num_k_centroids,
    max_iters=10,
    *,
    init_q_idx=None,
    init_k_idx=None,
    init_q_centroids=None,
    init_k_centroids=None,
    generator=None,
):
    """Cluster query/key tokens by alternating profile-space k-means (``svoo/co_clustering.py:2402-2451``).

    Returns ``(qlabels int64, qcentroids, qsizes int32, klabels int64, kcentroids, ksizes int32)``.
    The keyword-only ``init_*`` arguments fix the initial centroids (token indices or explicit
    centroids, e.g. a warm start); without them the indices are drawn with ``torch.randint`` on the
    device as in the reference.
    """
    r = co_cluster_tokens_full(
        q_flat, k_flat, num_q_centroids, num_k_centroids, max_iters,
        init_q_idx=init_q_idx, init_k_idx=init_k_idx, init_q_centroids=init_q_centroids,
        init_k_centroids=init_k_centroids, generator=generator,
    )
    return (r["qlabels"].long(), r["qcentroids"], r["qsizes"], r["klabels"].long(), r["kcentroids"], r["ksizes"])


def cocluster_profile(centroids: torch.Tensor, basis: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Profile centroids ``P = l2norm(bf16(A B^T))`` and the split assignment matrix ``E = P B``.

    ``centroids`` is ``A [BH, J, D]``, ``basis`` is ``B [BH, KP, D]`` (D <= 128).  Returns
    ``(P fp32 [BH, J, KP], E_hi bf16 [BH, Jpad, 128], E_lo bf16 [BH, Jpad, 128])`` (E zero past D); follows
    ``svoo/co_clustering.py:2427-2428`` (profile) and the reduction of ``:2146-2255`` (assignment).
    """
    a = _bf16_3d(centroids, "centroids")
    b = _bf16_3d(basis, "basis")
    bh, j, _ = a.shape
    kp = b.shape[1]
    jpad = _pad(j)
    prof = torch.empty(bh, j, kp, dtype=torch.float32, device=a.device)
    e_hi = torch.empty(bh, jpad, 128, dtype=torch.bfloat16, device=a.device)
    e_lo = torch.empty_like(e_hi)
    _lib.call("svoo_cocluster_prep", a.data_ptr(), b.data_ptr(), e_hi.data_ptr(), e_lo.data_ptr(), prof.data_ptr(),
              bh, j, kp, centroids.shape[-1], jpad, _lib.stream_of(a.device))
    return prof, e_hi, e_lo


def cocluster_assign(x: torch.Tensor, centroids: torch.Tensor, basis: torch.Tensor) -> torch.Tensor:
    """Labels of tokens ``x`` among ``centroids`` in the profile space spanned by ``basis`` (int32 [BH, N]).

    One assignment half-step of ``co_cluster_tokens``: ``profile_norm_triton`` +
    ``fused_cocluster_assign_triton`` (``svoo/co_clustering.py:2257-2400``) with the profiles of
    ``centroids`` built from ``basis``.
    """
    xx = _bf16_3d(x, "x")
    _, e_hi, e_lo = cocluster_profile(centroids, basis)
    bh, n, _ = xx.shape
    j = centroids.shape[1]
    labels = torch.empty(bh, n, dtype=torch.int32, device=xx.device)
    _lib.call("svoo_cocluster_assign", xx.data_ptr(), e_hi.data_ptr(), e_lo.data_ptr(), labels.data_ptr(), bh, n, j,
              e_hi.shape[1], x.shape[-1], _lib.stream_of(xx.device))
    return labels


def centroid_update(x: torch.Tensor, labels: torch.Tensor, old_centroids: torch.Tensor):
    """Cluster means of ``x`` by ``labels``; empty clusters keep ``old_centroids``.

    Mirrors ``triton_centroid_update_sorted_euclid`` (``svoo/co_clustering.py:253-303``): returns
    ``(centroids [BH, K, D] in x's dtype, counts int32 [BH, K])``; fp16 / fp32 inputs are rounded to bf16.
    """
    from .permute import cluster_sort  # local import keeps module load order simple

    xx = _bf16_3d(x, "x")
    old = _bf16_3d(old_centroids, "old_centroids")
    bh, n, d = xx.shape
    k = old.shape[1]
    lab = labels.to(device=xx.device, dtype=torch.int32).contiguous()
    sorted_idx, sizes, _, sorted_lab = cluster_sort(lab, k, with_sorted_labels=True)
    new = torch.empty_like(old)
    L = _lib.lib()
    ws = _lib.workspace(L.svoo_centroid_update_workspace_size(bh, k, d), xx.device)
    _lib.call("svoo_centroid_update", xx.data_ptr(), sorted_idx.data_ptr(), sorted_lab.data_ptr(), sizes.data_ptr(),
              old.data_ptr(), new.data_ptr(), bh, n, k, x.shape[-1], ws.data_ptr(), ws.numel(),
              _lib.stream_of(xx.device))
    return _lib.from_rows128(new, x.shape[-1], x.dtype), sizes


def triton_l2norm_forward(x: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    """Normalise the last dimension to unit L2 norm, fp32 output (``svoo/kernels/triton/l2norm.py:44-80``)."""
    _lib.require_gpu_tensor(x, "x")
    assert x.dim() in (2, 3), "Input tensors must be batched (3D) or not batched (2D)"
    xx = x.contiguous()
    if xx.dtype not in (torch.bfloat16, torch.float32):
        xx = _lib.convert(xx, torch.float32)
    y = torch.empty(xx.shape, dtype=torch.float32, device=xx.device)
    rows = xx.numel() // xx.shape[-1]
    _lib.call("svoo_l2norm_rows", xx.data_ptr(), int(xx.dtype == torch.bfloat16), y.data_ptr(), rows, xx.shape[-1],
              float(eps), _lib.stream_of(xx.device))
    return y


# ------------------------------------------------------------------------------------------------
# Block mask
# ------------------------------------------------------------------------------------------------
def weighted_softmax(scores: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """Softmax after weighting each key cluster by its size (``svoo/co_clustering.py:544-553``).  Computed on bf16
    scores (fp16 / fp32 scores are rounded to bf16) with a bf16 result, returned in the scores' dtype."""
    s = _lib.as_bf16(scores, "scores").contiguous()
    cols = s.shape[-1]
    rows = s.numel() // cols
    w = weights.to(device=s.device, dtype=torch.float32)
    w = torch.broadcast_to(w, s.shape).contiguous()
    out = torch.empty_like(s)
    _lib.call("svoo_weighted_softmax", s.data_ptr(), w.data_ptr(), cols, out.data_ptr(), rows, cols,
              _lib.stream_of(s.device))
    return _lib.convert(out, scores.dtype)


def _ratio_values(v, h: int):
    # A per-head ratio goes through a float32 tensor and .item() (svoo/co_clustering.py:590-594).
    if isinstance(v, torch.Tensor):
        v = v.detach().to("cpu", torch.float32)
        return [float(v[i]) for i in range(h)]
    import numpy as np

    return [float(np.float32(float(v[i]))) for i in range(h)]


def _per_head(v, h: int) -> bool:
    return isinstance(v, (list, tuple)) or (hasattr(v, "__len__") and len(v) == h)


def mask_row_params(h: int, kc_num: int, min_kc_ratio=0, max_kc_ratio=0) -> Tuple[list, list]:
    """Per-head ``(preserve, cap)`` counts of ``identify_dynamic_map`` (``svoo/co_clustering.py:589-627``).

    ``preserve[h] = int(ratio_h * Kc)`` for ``ratio_h > 0``; ``cap[h] = max(1, int(max_ratio * Kc))``
    raised to the head's minimum, or 0 when no cap applies.
    """
    preserve = [0] * h
    cap = [0] * h
    mins = None
    if _per_head(min_kc_ratio, h):
        mins = _ratio_values(min_kc_ratio, h)
        for i in range(h):
            if mins[i] > 0:
                preserve[i] = int(mins[i] * kc_num)
    elif isinstance(min_kc_ratio, (int, float)) and min_kc_ratio > 0:
        preserve = [int(min_kc_ratio * kc_num)] * h
    if max_kc_ratio is not None:
        if _per_head(max_kc_ratio, h):
            mx = _ratio_values(max_kc_ratio, h)
            for i in range(h):
                if mx[i] > 0:
                    c = max(1, int(mx[i] * kc_num))
                    if mins is not None:
                        c = max(c, int(mins[i] * kc_num))
                    cap[i] = c
        elif isinstance(max_kc_ratio, (int, float)) and float(max_kc_ratio) > 0:
            c = max(1, int(float(max_kc_ratio) * kc_num))
            if mins is not None:
                for i in range(h):
                    ch = c
                    if mins[i] > 0:
                        ch = max(ch, int(mins[i] * kc_num))
                    cap[i] = max(1, ch)
            else:
                if isinstance(min_kc_ratio, (int, float)) and float(min_kc_ratio) > 0:
                    c = max(c, int(float(min_kc_ratio) * kc_num))
                cap = [c] * h
    return preserve, cap


def _bf16_value(p: float) -> float:
    """``p`` rounded to float32 then bfloat16 (a Python scalar compared with a bf16 tensor)."""
    return float(torch.tensor(float(p), dtype=torch.float32).to(torch.bfloat16).float())


def block_mask_lengths(query_centroids, key_centroids, q_cluster_sizes, k_cluster_sizes, p, min_kc_ratio=0,
                       max_kc_ratio=0) -> Tuple[torch.Tensor, torch.Tensor]:
    """:func:`identify_dynamic_map` that also returns the kept count per row (int32 ``[B, H, Qc]``)."""
    qc = query_centroids
    kc = key_centroids
    _lib.require_gpu_tensor(qc, "query_centroids")
    b, h, qn, d = qc.shape
    kn = kc.shape[2]
    dev = qc.device
    dmap = torch.empty(b, h, qn, kn, dtype=torch.bool, device=dev)
    lengths = torch.empty(b, h, qn, dtype=torch.int32, device=dev)
    full = p >= 1.0
    if full:
        _lib.call("svoo_block_mask", None, None, None, None, None, b, h, qn, kn, d, 0.0, 1, dmap.data_ptr(),
                  lengths.data_ptr(), None, _lib.stream_of(dev))
        return dmap, lengths
    qc = _lib.as_rows128(qc, "query_centroids")
    kc = _lib.as_rows128(kc, "key_centroids")
    preserve, cap = mask_row_params(h, kn, min_kc_ratio, max_kc_ratio)
    pc = torch.tensor(preserve + cap, dtype=torch.int32).to(dev, non_blocking=True)
    ks = k_cluster_sizes.to(device=dev, dtype=torch.int32).reshape(b * h, kn).contiguous()
    scores = torch.empty(b, h, qn, kn, dtype=torch.bfloat16, device=dev)
    _lib.call("svoo_block_mask", qc.contiguous().data_ptr(), kc.contiguous().data_ptr(), ks.data_ptr(),
              pc.data_ptr(), pc[h:].data_ptr(), b, h, qn, kn, d, _bf16_value(p), 0, dmap.data_ptr(),
              lengths.data_ptr(), scores.data_ptr(), _lib.stream_of(dev))
    return dmap, lengths


def centroid_scores(query_centroids, key_centroids) -> torch.Tensor:
    """Scaled centroid attention scores ``matmul(Qc, Kc^T) / D**0.5`` of the block mask on bf16 centroids
    (``svoo/co_clustering.py:578``): the exact dot rounded to bf16, times ``float32(1 / sqrt(D))``, rounded to
    bf16.  ``[B, H, Qc, D]`` x ``[B, H, Kc, D]`` -> ``[B, H, Qc, Kc]`` bf16."""
    qc = _lib.as_rows128(query_centroids, "query_centroids")
    kc = _lib.as_rows128(key_centroids, "key_centroids")
    b, h, qn, _ = qc.shape
    d = query_centroids.shape[-1]
    kn = kc.shape[2]
    out = torch.empty(b, h, qn, kn, dtype=torch.bfloat16, device=qc.device)
    _lib.call("svoo_centroid_scores", qc.contiguous().data_ptr(), kc.contiguous().data_ptr(), b * h, qn, kn, d,
              out.data_ptr(), _lib.stream_of(qc.device))
    return out


def identify_dynamic_map(query_centroids, key_centroids, q_cluster_sizes, k_cluster_sizes, p, min_kc_ratio=0,
                         max_kc_ratio=0):
    """Boolean block map ``[B, H, Qc, Kc]`` by top-p over centroid attention (``svoo/co_clustering.py:556-633``).

    ``min_kc_ratio`` / ``max_kc_ratio``: scalar or per-head ratios (0 disables).  Ties in the
    descending probability order go to the lower key-cluster index.
    """
    return block_mask_lengths(query_centroids, key_centroids, q_cluster_sizes, k_cluster_sizes, p, min_kc_ratio,
                              max_kc_ratio)[0]


# ------------------------------------------------------------------------------------------------
# Variable-block-sparse attention
# ------------------------------------------------------------------------------------------------
def _check_host_sizes(sizes, s: int, name: str) -> None:
    """Sizes that live on the host (the reference's ``is_cpu=True`` case) are checked before they are
    copied, at no cost to the GPU stream (``svoo/co_clustering.py:1138-1139``).  Device sizes are
    checked by the plan kernel: the rows of a head whose sizes do not sum to ``S`` come back NaN."""
    if isinstance(sizes, torch.Tensor) and sizes.is_cuda:
        return
    tot = torch.as_tensor(sizes).to(torch.int64)
    if tot.dim() == 0 or bool((tot < 0).any()) or not bool((tot.sum(-1) == s).all()):
        raise AssertionError(f"{name}: cluster sizes of every head must sum to S={s}")


def dynamic_block_sparse_fwd(q, k, v, dynamic_map, qc_size, kc_size, *, validate: bool = True):
    """Variable-block-sparse attention over cluster-contiguous tokens.

    ``q, k, v [B, H, S, D]`` (bf16, D = 128), ``dynamic_map bool [B, H, Qc, Kc]``, ``qc_size [B, H, Qc]``,
    ``kc_size [B, H, Kc]``.  Query cluster ``i`` attends to the concatenation of its active key
    clusters with ``scale = D ** -0.5``; clusters without active keys produce zeros.  With
    ``validate`` the sizes of every head must sum to ``S`` (checked on the host after the call, as
    the reference asserts, ``svoo/co_clustering.py:1138-1139``).  Sizes passed as host tensors are
    checked before the launch in either case; without ``validate`` a head whose device sizes are
    inconsistent comes back as NaN rows (no host read-back).
    """
    assert q.is_cuda and k.is_cuda and v.is_cuda, "Inputs must be CUDA tensors"
    assert q.dtype == k.dtype == v.dtype, "Input dtypes must match"
    in_dtype, hd = q.dtype, q.shape[-1]
    q, k, v = (_lib.as_rows128(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    b, h, s, d = q.shape
    assert k.shape == q.shape and v.shape == q.shape, "q, k, v must share one shape"
    qn = qc_size.shape[-1]
    kn = kc_size.shape[-1]
    assert dynamic_map.shape == (b, h, qn, kn), "dynamic_map must be [B, H, Qc, Kc]"
    _check_host_sizes(qc_size, s, "qc_size")
    _check_host_sizes(kc_size, s, "kc_size")
    dev = q.device
    bh = b * h
    qq = q.reshape(bh, s, d).contiguous()
    kk = k.reshape(bh, s, d).contiguous()
    vv = v.reshape(bh, s, d).contiguous()
    m = dynamic_map.to(device=dev, dtype=torch.bool).reshape(bh, qn, kn).contiguous()
    qs = qc_size.to(device=dev, dtype=torch.int32).reshape(bh, qn).contiguous()
    ks = kc_size.to(device=dev, dtype=torch.int32).reshape(bh, kn).contiguous()
    out = torch.empty_like(qq)
    L = _lib.lib()
    ws = _lib.workspace(L.svoo_vbsa_workspace_size(bh, s, qn, kn), dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if validate else None
    _lib.call("svoo_vbsa_fwd", qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), m.data_ptr(), qs.data_ptr(),
              ks.data_ptr(), out.data_ptr(), bh, s, hd, qn, kn, ws.data_ptr(), ws.numel(), _lib.ptr(status),
              _lib.stream_of(dev))
    if validate and int(status.item()) != 0:
        raise AssertionError("cluster sizes of every head must sum to S (qc_size / kc_size)")
    return _lib.from_rows128(out.reshape(b, h, s, d), hd, in_dtype)


def dynamic_block_sparse_fwd_fused(query, key, value, dynamic_map, qc_size, kc_size, q_sorted_idx, k_sorted_idx,
                                   *, validate: bool = True):
    """Permute, variable-block-sparse attention and inverse permutation in one kernel.

    ``query, key, value [B, H, S, D]`` in token order; ``q_sorted_idx`` / ``k_sorted_idx [B*H, S]`` are the stable
    cluster sorts (``co_cluster_tokens_full``'s ``q_sorted_idx`` / ``k_sorted_idx``).  Returns ``[B, S, H*D]``,
    equal to :func:`dynamic_block_sparse_fwd` on the permuted tensors followed by the inverse permutation and
    ``transpose(1, 2).flatten(2, 3)`` (``svoo/models/wan/attention.py:1037-1042, 1196-1215``).
    """
    assert query.is_cuda and key.is_cuda and value.is_cuda, "Inputs must be CUDA tensors"
    assert query.dtype == key.dtype == value.dtype, "Input dtypes must match"
    in_dtype, hd = query.dtype, query.shape[-1]
    query, key, value = (_lib.as_rows128(t, n) for t, n in ((query, "query"), (key, "key"), (value, "value")))
    b, h, s, d = query.shape
    assert key.shape == query.shape and value.shape == query.shape, "q, k, v must share one shape"
    qn = qc_size.shape[-1]
    kn = kc_size.shape[-1]
    assert dynamic_map.shape == (b, h, qn, kn), "dynamic_map must be [B, H, Qc, Kc]"
    _check_host_sizes(qc_size, s, "qc_size")
    _check_host_sizes(kc_size, s, "kc_size")
    dev = query.device
    bh = b * h
    qq, kk, vv = (t.reshape(bh, s, d).contiguous() for t in (query, key, value))
    qi = q_sorted_idx.to(device=dev, dtype=torch.int32).reshape(bh, s).contiguous()
    ki = k_sorted_idx.to(device=dev, dtype=torch.int32).reshape(bh, s).contiguous()
    m = dynamic_map.to(device=dev, dtype=torch.bool).reshape(bh, qn, kn).contiguous()
    qs = qc_size.to(device=dev, dtype=torch.int32).reshape(bh, qn).contiguous()
    ks = kc_size.to(device=dev, dtype=torch.int32).reshape(bh, kn).contiguous()
    out = torch.empty(b, s, h * d, dtype=query.dtype, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(L.svoo_vbsa_workspace_size(bh, s, qn, kn), dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if validate else None
    _lib.call("svoo_vbsa_fused_fwd", qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), qi.data_ptr(), ki.data_ptr(),
              m.data_ptr(), qs.data_ptr(), ks.data_ptr(), out.data_ptr(), bh, h, s, hd, qn, kn, ws.data_ptr(),
              ws.numel(), _lib.ptr(status), _lib.stream_of(dev))
    if validate and int(status.item()) != 0:
        raise AssertionError("cluster sizes of every head must sum to S (qc_size / kc_size)")
    return _lib.from_rows128(out.view(b, s, h, d), hd, in_dtype).reshape(b, s, h * hd)


def dynamic_block_sparse_fwd_flashinfer(q, k, v, block_mask_map, block_row_sz, block_col_sz, is_cpu: bool = True):
    """Drop-in for ``dynamic_block_sparse_fwd_flashinfer`` (``svoo/co_clustering.py:1231-1311``).

    The plan is built on the device, so ``is_cpu`` only states where the map and sizes live; they
    are moved to the GPU if needed.  No 128 MiB workspace and no host round trip per call.  Host-side
    sizes are checked before the copy; inconsistent device sizes give NaN rows for that head.
    """
    return dynamic_block_sparse_fwd(q, k, v, block_mask_map, block_row_sz, block_col_sz, validate=False)


def dynamic_block_sparse_fwd_triton(q, k, v, dynamic_map, qc_size, kc_size):
    """Drop-in for ``dynamic_block_sparse_fwd_triton`` (``svoo/co_clustering.py:1111-1228``), with its size asserts."""
    return dynamic_block_sparse_fwd(q, k, v, dynamic_map, qc_size, kc_size, validate=True)


def vbsa_segments(block_mask_map: torch.Tensor, block_col_sz: torch.Tensor):
    """Active key segments per ``(bh, q-cluster)`` as walked by the attention kernel.

    Returns ``(start int32 [BH, Qc, Kc], length int32 [BH, Qc, Kc], count int32 [BH, Qc])``: entries
    ``< count`` are the active non-empty key clusters in ascending order, as (first key row,
    key count) of the cluster-contiguous K.  Expanding them reproduces the token list of the
    reference's plan (``svoo/utils/flashinfer_sparse.py:43-97``) without the head offset.
    """
    m = block_mask_map.to(torch.bool)
    bh = m.numel() // (m.shape[-1] * m.shape[-2])
    qn, kn = m.shape[-2], m.shape[-1]
    m = m.reshape(bh, qn, kn).contiguous()
    ks = block_col_sz.to(device=m.device, dtype=torch.int32).reshape(bh, kn).contiguous()
    start = torch.zeros(bh, qn, kn, dtype=torch.int32, device=m.device)
    length = torch.zeros_like(start)
    count = torch.empty(bh, qn, dtype=torch.int32, device=m.device)
    _lib.call("svoo_vbsa_segments", m.data_ptr(), ks.data_ptr(), bh, qn, kn, start.data_ptr(), length.data_ptr(),
              count.data_ptr(), _lib.stream_of(m.device))
    return start, length, count
