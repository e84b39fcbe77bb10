"""numpy restatement of the SVOO hot path (test infrastructure, see package docstring).

Array conventions
-----------------
* Token tensors are ``[BH, N, D]`` (or ``[B, H, S, D]`` where the reference uses
  that shape).  "bf16" data is carried as float32 arrays whose values are exactly
  representable in bfloat16; :func:`bf16_round` produces such arrays.
* Labels are int64, cluster sizes and offsets int32, as in the reference.

Rounding contract (applies to the GPU implementation as well)
-------------------------------------------------------------
* Dot products of stored (bf16 or fp32) values are evaluated exactly (float64
  sums of exactly representable products) and rounded to float32, then to the
  storage dtype, where the reference rounds a matmul output.
* Centroid sums are float64, rounded to float32, divided by the count in
  float32 (IEEE division) and rounded to the storage dtype.  A float64 sum of
  bf16 values is exact while, per cluster and dimension, the members' exponent
  span plus log2(member count) stays within 45 bits (53-bit significand minus
  bf16's 8; about 28 binades at N = 75600); beyond that it rounds, and sums
  taken in another order can differ in the last float64 bits.
* Sorting is stable: ties go to the lower original index (-0.0 and +0.0 tie).
* EAR (error-aware routing): value centroids are the exact member sum rounded to
  bf16, divided by the bf16-rounded count (the reference's bf16 tensor ops); the
  efficiency scores are evaluated in float64 (the reference's fp32 expansion is
  ill-conditioned where a centroid reproduces its block); budget and greedy areas
  are exact integers (the reference sums them in float32).
"""

from __future__ import annotations

import math
from typing import Iterable, Optional, Sequence, Tuple

import numpy as np

__all__ = [
    "bf16_round",
    "bf16_bits",
    "bf16_from_bits",
    "storage_round",
    "cluster_sort",
    "permute_rows",
    "unpermute_rows",
    "centroid_update",
    "l2norm_rows",
    "profile_centroids",
    "cocluster_assign",
    "reduced_assign",
    "co_cluster_tokens",
    "centroid_scores",
    "weighted_softmax",
    "mask_row_params",
    "identify_dynamic_map",
    "kv_plan_indices",
    "block_sparse_attention",
    "dense_attention",
    "svoo_attention_call",
    "hunyuan_post_process",
    "hunyuan_attention_call",
    "hunyuan_dense_attention",
    "sparsity_weights",
    "exact_sparsity_counts",
    "exact_attention_sparsity",
    "value_centroids",
    "value_stats",
    "ear_centroid_logits",
    "ear_efficiency_scores",
    "ear_row_params",
    "ear_select",
    "ear_compensated_attention",
    "ear_attention_call",
]

_FIX_SHIFT = 60  # fixed-point scale of the top-p prefix sums (2**60)


# --------------------------------------------------------------------------------------
# bf16 helpers
# --------------------------------------------------------------------------------------
def bf16_bits(x) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even) and return the 16-bit patterns.

    Mirrors ``Tensor.to(torch.bfloat16)`` used throughout the reference
    (e.g. ``svoo/co_clustering.py:303``, ``:553``).  NaN maps to a quiet NaN.
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) & np.uint64(0xFFFF)
    r = r.astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = np.uint16(0x7FC0)
    return r


def bf16_from_bits(b) -> np.ndarray:
    """Expand 16-bit bfloat16 patterns to float32 values (exact)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """float32 array holding the bf16-rounded (RNE) values of ``x`` (float32 input)."""
    return bf16_from_bits(bf16_bits(x))


def storage_round(x, dtype: str) -> np.ndarray:
    """Round float values to the storage dtype: ``"bf16"`` via float32 then bf16, ``"fp32"`` to float32."""
    x32 = np.asarray(x).astype(np.float32)
    if dtype == "bf16":
        return bf16_round(x32)
    if dtype == "fp32":
        return x32
    raise ValueError(f"unsupported storage dtype {dtype!r}")


def _exact_matmul_nt(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """``a @ b.T`` in float64 over the last dim (exact for bf16 operands of bounded exponent span)."""
    return np.matmul(a.astype(np.float64), np.swapaxes(b.astype(np.float64), -1, -2))


# --------------------------------------------------------------------------------------
# A9 / A10: cluster sort, permute, unpermute
# --------------------------------------------------------------------------------------
def cluster_sort(labels, num_clusters: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Stable sort of token labels per row: ``sorted_idx``, cluster ``sizes`` and ``offsets``.

    Follows ``svoo/kernels/triton/permute.py:90`` (``torch.argsort(labels)``) and
    ``svoo/co_clustering.py:273-274`` (``torch.sort(cluster_ids)``).  The reference
    sorts are unstable; the contract here is stable (ascending original index
    within a cluster).  ``sizes == bincount(labels, minlength=K)``;
    ``offsets`` is the exclusive prefix sum of ``sizes``.
    """
    labels = np.asarray(labels)
    bh, n = labels.shape
    sorted_idx = np.empty((bh, n), dtype=np.int32)
    sizes = np.empty((bh, num_clusters), dtype=np.int32)
    for r in range(bh):
        lab = labels[r].astype(np.int64)
        if n and (lab.min() < 0 or lab.max() >= num_clusters):
            raise ValueError("label out of range")
        # Counting sort: positions are filled in ascending token order per cluster.
        cnt = np.bincount(lab, minlength=num_clusters)
        start = np.concatenate([[0], np.cumsum(cnt)[:-1]])
        order = np.empty(n, dtype=np.int64)
        fill = start.copy()
        for t in range(n):
            c = lab[t]
            order[fill[c]] = t
            fill[c] += 1
        sorted_idx[r] = order
        sizes[r] = cnt
    offsets = (np.cumsum(sizes, axis=1) - sizes).astype(np.int32)
    return sorted_idx, sizes, offsets


def permute_rows(x, sorted_idx) -> np.ndarray:
    """``y[bh, s, :] = x[bh, sorted_idx[bh, s], :]`` (``svoo/kernels/triton/permute.py:9-35``)."""
    x = np.asarray(x)
    idx = np.asarray(sorted_idx).astype(np.int64)
    return np.take_along_axis(x, idx[:, :, None], axis=1)


def unpermute_rows(y, sorted_idx) -> np.ndarray:
    """``x[bh, sorted_idx[bh, s], :] = y[bh, s, :]`` (``svoo/kernels/triton/permute.py:38-65``)."""
    y = np.asarray(y)
    idx = np.asarray(sorted_idx).astype(np.int64)
    out = np.empty_like(y)
    for r in range(y.shape[0]):
        out[r, idx[r]] = y[r]
    return out


# --------------------------------------------------------------------------------------
# A5: centroid update
# --------------------------------------------------------------------------------------
def centroid_update(x, labels, old_centroids, dtype: str = "bf16") -> Tuple[np.ndarray, np.ndarray]:
    """Per-cluster mean of member tokens; empty clusters keep their old centroid.

    Follows ``svoo/co_clustering.py:253-303`` (``triton_centroid_update_sorted_euclid``):
    ``sums / max(count, 1)`` in float32, ``torch.where(count == 0, old, mean)``,
    cast to the token dtype.  Contract: the member sum is taken in float64 (exact
    under the exponent-span condition of the module docstring), rounded to float32,
    then divided by ``float32(count)``.
    """
    x = np.asarray(x)
    labels = np.asarray(labels).astype(np.int64)
    old = np.asarray(old_centroids)
    bh, n, d = x.shape
    k = old.shape[1]
    out = np.empty((bh, k, d), dtype=np.float32)
    counts = np.empty((bh, k), dtype=np.int32)
    for r in range(bh):
        sums = np.zeros((k, d), dtype=np.float64)
        np.add.at(sums, labels[r], x[r].astype(np.float64))
        cnt = np.bincount(labels[r], minlength=k)
        mean32 = sums.astype(np.float32) / np.maximum(cnt, 1).astype(np.float32)[:, None]
        mean = storage_round(mean32, dtype)
        empty = cnt == 0
        mean[empty] = old[r][empty].astype(np.float32)
        out[r] = mean
        counts[r] = cnt
    return out, counts


# --------------------------------------------------------------------------------------
# A3 / A4: profile centroids and profile-space assignment
# --------------------------------------------------------------------------------------
def l2norm_rows(x, eps: float = 1e-8) -> np.ndarray:
    """Row L2 normalisation ``x / sqrt(sum(x**2) + eps)`` in float64.

    Follows ``svoo/kernels/triton/l2norm.py:8-41`` (eps inside the square root).
    """
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + eps)


def profile_centroids(a, b, dtype: str = "bf16") -> np.ndarray:
    """``P = l2norm(rnd(A @ B^T))``: profiles of the centroids ``A`` in the space of ``B``.

    Follows ``svoo/co_clustering.py:2427-2428`` (key step, ``A = Kc``, ``B = Qc``)
    and ``:2440-2441`` (query step, ``A = Qc``, ``B = Kc``).  The matmul output is
    rounded to the storage dtype as ``torch.matmul`` on bf16 does.
    """
    raw = storage_round(_exact_matmul_nt(a, b), dtype)
    return l2norm_rows(raw, 1e-8)


def cocluster_assign(x, c, p, chunk: int = 8192) -> Tuple[np.ndarray, np.ndarray]:
    """Literal profile-space nearest centroid, in float64.

    Follows ``svoo/co_clustering.py:2086-2144`` (``norm = sqrt(sum_k (x.C_k)^2 + 1e-8)``)
    and ``:2146-2255`` (``dist_j = 2 - 2 * sum_k (x.C_k / norm) * P[j, k]``,
    ``label = argmin_j dist_j``, first index on ties).

    Returns ``(labels int64 [BH, N], margin float64 [BH, N])`` where ``margin`` is
    the gap between the second-best and best distance (inf when ``J == 1``).
    """
    x = np.asarray(x, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    p = np.asarray(p, dtype=np.float64)
    bh, n, _ = x.shape
    j = p.shape[1]
    labels = np.empty((bh, n), dtype=np.int64)
    margin = np.empty((bh, n), dtype=np.float64)
    for r in range(bh):
        for s in range(0, n, chunk):
            xs = x[r, s : s + chunk]
            dots = xs @ c[r].T
            norm = np.sqrt(np.sum(dots * dots, axis=1) + 1e-8)
            dist = 2.0 - 2.0 * ((dots / norm[:, None]) @ p[r].T)
            best = np.argmin(dist, axis=1)
            labels[r, s : s + chunk] = best
            if j > 1:
                part = np.partition(dist, 1, axis=1)
                margin[r, s : s + chunk] = part[:, 1] - part[:, 0]
            else:
                margin[r, s : s + chunk] = np.inf
    return labels, margin


def reduced_assign(x, c, p) -> np.ndarray:
    """Reduced form of :func:`cocluster_assign`: ``argmax_j x . E_j`` with ``E = P @ C``.

    Equal to the literal form wherever the literal margin is not a near-tie,
    because ``norm > 0`` is a per-token constant.  The GPU kernel computes this form.
    """
    x = np.asarray(x, dtype=np.float64)
    e = np.matmul(np.asarray(p, dtype=np.float64), np.asarray(c, dtype=np.float64))
    return np.argmax(np.matmul(x, np.swapaxes(e, -1, -2)), axis=-1).astype(np.int64)


def co_cluster_tokens(
    q_flat,
    k_flat,
    num_q_centroids: int,
    num_k_centroids: int,
    max_iters: int = 10,
    *,
    init_q_idx=None,
    init_k_idx=None,
    init_q_centroids=None,
    init_k_centroids=None,
    dtype: str = "bf16",
    trace: Optional[list] = None,
):
    """Alternating key/query profile-space k-means.

    Follows ``svoo/co_clustering.py:2402-2451``: initial centroids are tokens
    gathered at ``init_*_idx`` (the reference draws them with ``torch.randint``,
    ``:2417-2421``; here they are explicit) or explicit ``init_*_centroids``;
    each iteration runs the key step (profiles in query-centroid space) and then
    the query step with the *new* key centroids.  ``max_iters == 0`` raises, as
    the reference does (its ``qlabels`` is unbound).

    Returns ``(qlabels, qcentroids, qsizes, klabels, kcentroids, ksizes)``.
    ``trace`` (a list) collects ``(side, labels, margin, centroids_in, profile)``
    per half-step for tests.
    """
    q = np.asarray(q_flat, dtype=np.float32)
    k = np.asarray(k_flat, dtype=np.float32)
    bh, n, d = q.shape
    if max_iters < 1:
        raise UnboundLocalError("co_cluster_tokens needs max_iters >= 1 (reference leaves qlabels unbound)")

    def _init(x, idx, cents, kc):
        if cents is not None:
            return np.asarray(cents, dtype=np.float32).copy()
        if idx is None:
            raise ValueError("explicit init indices or centroids are required")
        idx = np.asarray(idx).astype(np.int64)
        assert idx.shape == (bh, kc)
        return np.take_along_axis(x, idx[:, :, None], axis=1).copy()

    qc = _init(q, init_q_idx, init_q_centroids, num_q_centroids)
    kc = _init(k, init_k_idx, init_k_centroids, num_k_centroids)
    for _ in range(max_iters):
        pk = profile_centroids(kc, qc, dtype)
        klabels, kmargin = cocluster_assign(k, qc, pk)
        if trace is not None:
            trace.append(("k", klabels.copy(), kmargin, kc.copy(), qc.copy()))
        kc, ksizes = centroid_update(k, klabels, kc, dtype)
        pq = profile_centroids(qc, kc, dtype)
        qlabels, qmargin = cocluster_assign(q, kc, pq)
        if trace is not None:
            trace.append(("q", qlabels.copy(), qmargin, qc.copy(), kc.copy()))
        qc, qsizes = centroid_update(q, qlabels, qc, dtype)
    return qlabels, qc, qsizes, klabels, kc, ksizes


# --------------------------------------------------------------------------------------
# A6 / A7: weighted softmax and the block mask
# --------------------------------------------------------------------------------------
def centroid_scores(qc, kc, dtype: str = "bf16") -> np.ndarray:
    """Scaled centroid attention scores ``rnd(rnd(Qc @ Kc^T) * (1 / sqrt(D)))``.

    Follows ``svoo/co_clustering.py:578``: ``torch.matmul(...) / (D ** 0.5)`` on
    bf16 tensors.  The division by a Python scalar executes on the GPU as a
    multiplication by the float32 reciprocal of ``float32(sqrt(D))``; the
    product is formed in float32 and rounded to the storage dtype.
    """
    d = np.asarray(qc).shape[-1]
    s = storage_round(_exact_matmul_nt(qc, kc), dtype)
    inv = np.float32(1.0) / np.float32(d ** 0.5)
    return storage_round((s.astype(np.float32) * inv).astype(np.float32), dtype)


def weighted_softmax(scores, weights, dtype: str = "bf16") -> np.ndarray:
    """``w * exp(s - max) / max(sum(w * exp(s - max)), 1e-12)`` rounded to the storage dtype.

    Follows ``svoo/co_clustering.py:544-553``.  Contract: evaluated in float64,
    rounded to float32 and then to the storage dtype (the reference evaluates
    in float32 and casts back to the input dtype).
    """
    s = np.asarray(scores, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    m = np.max(s, axis=-1, keepdims=True)
    we = w * np.exp(s - m)
    den = np.maximum(np.sum(we, axis=-1, keepdims=True), 1e-12)
    return storage_round(we / den, dtype)


def _ratio_list(v, h: int):
    """Per-head ratio values as the reference reads them: float32 tensor elements via ``.item()``."""
    return [float(np.float32(float(v[i]))) for i in range(h)]


def _is_per_head(v, h: int) -> bool:
    # svoo/co_clustering.py:589: list/tuple, or any sized object whose length is H.
    return isinstance(v, (list, tuple)) or (hasattr(v, "__len__") and len(v) == h)


def mask_row_params(h: int, kc_num: int, min_kc_ratio=0, max_kc_ratio=0) -> Tuple[np.ndarray, np.ndarray]:
    """Per-head ``(preserve, cap)`` key-cluster counts (``cap == 0`` means no cap).

    Follows the branches of ``svoo/co_clustering.py:589-627``: a per-head ratio is
    read through a float32 tensor (``.item()`` of float32), a scalar ratio in
    double precision; ``preserve = int(ratio * Kc)`` when ``ratio > 0``;
    ``cap = max(1, int(max_ratio * Kc))``, raised to the head's preserve count
    when per-head minima exist (or to the scalar minimum's count).
    """
    preserve = np.zeros(h, dtype=np.int64)
    cap = np.zeros(h, dtype=np.int64)
    min_tensor = None
    if _is_per_head(min_kc_ratio, h):
        min_tensor = _ratio_list(min_kc_ratio, h)
        for i in range(h):
            if min_tensor[i] > 0:
                preserve[i] = int(min_tensor[i] * kc_num)
    elif isinstance(min_kc_ratio, (int, float)) and min_kc_ratio > 0:
        preserve[:] = int(min_kc_ratio * kc_num)

    if max_kc_ratio is not None:
        if _is_per_head(max_kc_ratio, h):
            mx = _ratio_list(max_kc_ratio, h)
            for i in range(h):
                if mx[i] > 0:
                    c = max(1, int(mx[i] * kc_num))
                    if min_tensor is not None:
                        c = max(c, int(min_tensor[i] * kc_num))
                    cap[i] = c
        elif isinstance(max_kc_ratio, (int, float)) and float(max_kc_ratio) > 0:
            c = max(1, int(float(max_kc_ratio) * kc_num))
            if min_tensor is not None:
                for i in range(h):
                    ch = c
                    if min_tensor[i] > 0:
                        ch = max(ch, int(min_tensor[i] * kc_num))
                    cap[i] = max(1, ch)
            else:
                if isinstance(min_kc_ratio, (int, float)) and float(min_kc_ratio) > 0:
                    c = max(c, int(float(min_kc_ratio) * kc_num))
                cap[:] = c
    return preserve, cap


def _fixed_point(pb: np.ndarray) -> np.ndarray:
    """floor(pb * 2**60) as int64 for bf16-valued probabilities in [0, 1]."""
    out = np.zeros(pb.shape, dtype=np.int64)
    flat = pb.reshape(-1)
    o = out.reshape(-1)
    for i, v in enumerate(flat.tolist()):
        if v > 0.0:
            o[i] = math.floor(math.ldexp(v, _FIX_SHIFT))
    return out


def _prefix_to_bf16(prefix: np.ndarray) -> np.ndarray:
    """bf16(float32(float64(prefix) * 2**-60)) with round-to-nearest at each conversion."""
    as_f64 = prefix.astype(np.float64) * math.ldexp(1.0, -_FIX_SHIFT)
    return bf16_round(as_f64.astype(np.float32))


def identify_dynamic_map(
    query_centroids,
    key_centroids,
    q_cluster_sizes,
    k_cluster_sizes,
    p,
    min_kc_ratio=0,
    max_kc_ratio=0,
    dtype: str = "bf16",
    return_lengths: bool = False,
):
    """Top-p block mask over centroid attention with per-head minimum keep and optional cap.

    Follows ``svoo/co_clustering.py:556-633``:
    ``p >= 1`` gives an all-true map (``:575-576``); otherwise the weighted softmax
    of the scaled centroid scores is sorted in descending order, ``remove =
    cumsum > p`` is shifted right by one with position 0 always kept
    (``:582-587``), the first ``preserve`` sorted positions are kept and
    positions from ``cap`` on are removed (``:589-627``), and the kept set is
    scattered back (``:629-632``).

    Contract for the reference's non-deterministic pieces: the sort is stable
    (probability descending, key-cluster index ascending); the running sum is
    exact in fixed point (``floor(p * 2**60)`` summed in int64), rounded to the
    storage dtype before the comparison with ``p`` rounded to the storage dtype
    (the reference compares a bf16 cumsum with a Python float in bf16).
    ``q_cluster_sizes`` is accepted for signature parity and, as in the
    reference, unused.
    """
    qc = np.asarray(query_centroids, dtype=np.float32)
    kc = np.asarray(key_centroids, dtype=np.float32)
    b, h, qn, _ = qc.shape
    kn = kc.shape[2]
    if p >= 1.0:
        m = np.ones((b, h, qn, kn), dtype=bool)
        return (m, np.full((b, h, qn), kn, dtype=np.int64)) if return_lengths else m
    t = centroid_scores(qc, kc, dtype)
    w = np.asarray(k_cluster_sizes, dtype=np.float64)[:, :, None, :]
    pb = weighted_softmax(t, np.broadcast_to(w, t.shape), dtype)
    preserve, cap = mask_row_params(h, kn, min_kc_ratio, max_kc_ratio)
    p_st = storage_round(np.float32(p), dtype)
    out = np.zeros((b, h, qn, kn), dtype=bool)
    lengths = np.zeros((b, h, qn), dtype=np.int64)
    j_idx = np.arange(kn)
    for bi in range(b):
        for hi in range(h):
            for i in range(qn):
                row = pb[bi, hi, i]
                order = np.lexsort((j_idx, -row.astype(np.float64)))  # stable: prob desc, index asc
                srt = row[order]
                if dtype == "bf16":
                    prefix = np.cumsum(_fixed_point(srt))
                    cum = _prefix_to_bf16(prefix)
                else:
                    cum = np.cumsum(srt.astype(np.float64)).astype(np.float32)
                le = cum[: kn - 1] <= p_st
                # Number of leading positions t >= 1 whose predecessor prefix is <= p.
                lead = int(np.argmin(le)) if not le.all() else kn - 1
                length = 1 + lead
                length = max(length, int(preserve[hi]))
                if cap[hi] > 0:
                    length = min(length, int(cap[hi]))
                length = min(length, kn)
                out[bi, hi, i, order[:length]] = True
                lengths[bi, hi, i] = length
    return (out, lengths) if return_lengths else out


# --------------------------------------------------------------------------------------
# A11 / A12: plan indices and variable-block-sparse attention
# --------------------------------------------------------------------------------------
def kv_plan_indices(block_mask_map, block_col_sz) -> Tuple[np.ndarray, np.ndarray]:
    """Token-level KV plan of the reference's FlashInfer wrapper.

    Follows ``svoo/utils/flashinfer_sparse.py:43-97``: ``kv_indptr`` is the
    exclusive prefix of per-row active key counts over ``(head, q-cluster)``
    rows; ``kv_indices`` lists, row by row and key cluster by key cluster in
    ascending index, ``head_offset[h] + col_offset[h, c] + t``.
    """
    m = np.asarray(block_mask_map, dtype=bool)
    cs = np.asarray(block_col_sz).astype(np.int64)
    bh, qn, kn = m.shape
    row_len = (m * cs[:, None, :]).sum(-1)
    kv_indptr = np.concatenate([[0], np.cumsum(row_len.reshape(-1))]).astype(np.int64)
    col_off = np.cumsum(cs, axis=1) - cs
    head_len = cs.sum(1)
    head_off = np.cumsum(head_len) - head_len
    out = []
    for r in range(bh):
        for i in range(qn):
            for c in np.nonzero(m[r, i])[0]:
                base = head_off[r] + col_off[r, c]
                out.append(np.arange(base, base + cs[r, c], dtype=np.int64))
    kv_indices = np.concatenate(out) if out else np.zeros(0, dtype=np.int64)
    return kv_indptr, kv_indices


def block_sparse_attention(q, k, v, dynamic_map, qc_size, kc_size, compute_dtype=np.float64) -> np.ndarray:
    """Variable-block-sparse attention over cluster-contiguous (permuted) tokens.

    Follows the semantic spec ``svoo/co_clustering.py:949-1108``: query cluster
    ``i`` (rows ``qoff[i] .. qoff[i] + qs[i]``) attends to the concatenation of the
    active key clusters ``j`` (ascending) with ``scale = D ** -0.5``; a query
    cluster with no active keys outputs zeros (``:1102-1104``).  Computed in
    ``compute_dtype`` without intermediate rounding.
    """
    q = np.asarray(q)
    b, h, s, d = q.shape
    k = np.asarray(k)
    v = np.asarray(v)
    m = np.asarray(dynamic_map, dtype=bool)
    qs = np.asarray(qc_size).astype(np.int64)
    ks = np.asarray(kc_size).astype(np.int64)
    out = np.zeros((b, h, s, d), dtype=compute_dtype)
    scale = float(d) ** -0.5
    for bi in range(b):
        for hi in range(h):
            qoff = np.concatenate([[0], np.cumsum(qs[bi, hi])])
            koff = np.concatenate([[0], np.cumsum(ks[bi, hi])])
            kk = k[bi, hi].astype(compute_dtype)
            vv = v[bi, hi].astype(compute_dtype)
            for i in range(qs.shape[-1]):
                a, e = qoff[i], qoff[i + 1]
                if e == a:
                    continue
                act = np.nonzero(m[bi, hi, i])[0]
                rows = np.concatenate([np.arange(koff[j], koff[j + 1]) for j in act]) if len(act) else np.zeros(0, np.int64)
                if rows.size == 0:
                    continue
                qi = q[bi, hi, a:e].astype(compute_dtype)
                sc = (qi @ kk[rows].T) * compute_dtype(scale)
                sc -= sc.max(axis=1, keepdims=True)
                pr = np.exp(sc)
                pr /= pr.sum(axis=1, keepdims=True)
                out[bi, hi, a:e] = pr @ vv[rows]
    return out


def dense_attention(q, k, v, compute_dtype=np.float64) -> np.ndarray:
    """Dense softmax attention, ``F.scaled_dot_product_attention`` semantics (``svoo/models/wan/attention.py:329-331``)."""
    q = np.asarray(q, dtype=compute_dtype)
    k = np.asarray(k, dtype=compute_dtype)
    v = np.asarray(v, dtype=compute_dtype)
    sc = np.matmul(q, np.swapaxes(k, -1, -2)) * compute_dtype(q.shape[-1] ** -0.5)
    sc -= sc.max(axis=-1, keepdims=True)
    pr = np.exp(sc)
    pr /= pr.sum(axis=-1, keepdims=True)
    return np.matmul(pr, v)


# --------------------------------------------------------------------------------------
# A13: the whole SAP attention call
# --------------------------------------------------------------------------------------
def svoo_attention_call(
    query,
    key,
    value,
    num_q_centroids: int,
    num_k_centroids: int,
    kmeans_iters: int,
    top_p: float,
    min_kc_ratio=0,
    max_kc_ratio=0,
    *,
    init_q_idx=None,
    init_k_idx=None,
    init_q_centroids=None,
    init_k_centroids=None,
    dtype: str = "bf16",
    attn_dtype=np.float64,
    return_parts: bool = False,
):
    """One sparse ``attention_core_logic`` call (``svoo/models/wan/attention.py:1110-1216``).

    ``semantic_aware_permutation`` (``:958-1088``): co-cluster, per-head ratios,
    permute Q by query labels and K/V by key labels, ``identify_dynamic_map``;
    then block-sparse attention, inverse permutation of the output and the
    ``[1, S, H*D]`` reshape (``:1211-1215``).
    """
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, h, s, d = q.shape
    assert b == 1, "Batch size must be 1 for kmeans block sparse attention"
    qf, kf, vf = q.reshape(h, s, d), k.reshape(h, s, d), v.reshape(h, s, d)
    ql, qcent, qsz, kl, kcent, ksz = co_cluster_tokens(
        qf, kf, num_q_centroids, num_k_centroids, kmeans_iters,
        init_q_idx=init_q_idx, init_k_idx=init_k_idx,
        init_q_centroids=init_q_centroids, init_k_centroids=init_k_centroids, dtype=dtype,
    )
    qidx, _, _ = cluster_sort(ql, num_q_centroids)
    kidx, _, _ = cluster_sort(kl, num_k_centroids)
    qp, kp, vp = permute_rows(qf, qidx), permute_rows(kf, kidx), permute_rows(vf, kidx)
    dmap = identify_dynamic_map(
        qcent.reshape(1, h, num_q_centroids, d), kcent.reshape(1, h, num_k_centroids, d),
        qsz.reshape(1, h, -1), ksz.reshape(1, h, -1), top_p, min_kc_ratio, max_kc_ratio, dtype,
    )
    op = block_sparse_attention(
        qp[None], kp[None], vp[None], dmap, qsz.reshape(1, h, -1), ksz.reshape(1, h, -1), attn_dtype
    )[0]
    o = unpermute_rows(op, qidx)
    out = np.transpose(o[None], (0, 2, 1, 3)).reshape(1, s, h * d)
    if return_parts:
        return out, dict(qlabels=ql, klabels=kl, qcentroids=qcent, kcentroids=kcent,
                         qsizes=qsz, ksizes=ksz, map=dmap, qidx=qidx, kidx=kidx)
    return out


# --------------------------------------------------------------------------------------
# HunyuanVideo text-dense variant
# --------------------------------------------------------------------------------------
def hunyuan_post_process(dyn_map, q_sizes, k_sizes, q_sorted_idx, video_length: int, context_length: int,
                         prompt_length: int):
    """Append the prompt and padding clusters to a video block map.

    Follows ``svoo/models/hunyuan10/attention.py:977-1021``: the map gains two rows and columns;
    row ``Qc`` (prompt) attends columns ``0..Kc`` (every video cluster and the prompt), column
    ``Kc`` (prompt) is attended by rows ``0..Qc``, and the padding cluster ``Kc+1`` pairs only with
    itself.  Sizes gain ``[prompt_length, context_length - prompt_length]``; the query sort order
    gains the identity over the text tokens.
    """
    m = np.asarray(dyn_map, dtype=bool)
    b, h, qn, kn = m.shape
    out = np.zeros((b, h, qn + 2, kn + 2), dtype=bool)
    out[:, :, :qn, :kn] = m
    out[:, :, qn, : kn + 1] = True      # prompt row: video clusters and the prompt
    out[:, :, : qn + 1, kn] = True      # prompt column: every video row and the prompt row
    out[:, :, qn + 1, kn + 1] = True    # padding only with itself
    tail = np.array([prompt_length, context_length - prompt_length], dtype=np.int64)
    qs = np.concatenate([np.asarray(q_sizes), np.broadcast_to(tail, (b, h, 2))], axis=-1)
    ks = np.concatenate([np.asarray(k_sizes), np.broadcast_to(tail, (b, h, 2))], axis=-1)
    idx = np.asarray(q_sorted_idx)
    text = np.arange(video_length, video_length + context_length)
    qidx = np.concatenate([idx, np.broadcast_to(text, (idx.shape[0], context_length))], axis=1)
    return out, qs, ks, qidx


def hunyuan_attention_call(query, key, value, num_q_centroids: int, num_k_centroids: int, kmeans_iters: int,
                           top_p: float, min_kc_ratio, prompt_length: int, context_length: int, *,
                           init_q_idx=None, init_k_idx=None, init_q_centroids=None, init_k_centroids=None,
                           dtype: str = "bf16", attn_dtype=np.float64):
    """One sparse Hunyuan ``attention_core_logic`` call, output ``[1, H, S, D]``.

    Follows ``svoo/models/hunyuan10/attention.py:1031-1110``: co-cluster the video part (the first
    ``S - context_length`` tokens), mask it, permute video Q by query labels and video K/V by key
    labels with the text kept last, extend the map and sizes (:func:`hunyuan_post_process`),
    block-sparse attention over the whole sequence and the inverse permutation.
    """
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, h, s, d = q.shape
    assert b == 1
    vl = s - context_length
    qv, kv = q[0, :, :vl], k[0, :, :vl]
    ql, qcent, qsz, kl, kcent, ksz = co_cluster_tokens(qv, kv, num_q_centroids, num_k_centroids, kmeans_iters,
                                                       init_q_idx=init_q_idx, init_k_idx=init_k_idx,
                                                       init_q_centroids=init_q_centroids,
                                                       init_k_centroids=init_k_centroids, dtype=dtype)
    qidx, _, _ = cluster_sort(ql, num_q_centroids)
    kidx, _, _ = cluster_sort(kl, num_k_centroids)
    dmap = identify_dynamic_map(qcent[None], kcent[None], qsz[None], ksz[None], top_p, min_kc_ratio, 0, dtype)
    m2, qs2, ks2, qidx2 = hunyuan_post_process(dmap, qsz[None], ksz[None], qidx, vl, context_length, prompt_length)
    _, _, _, kidx2 = hunyuan_post_process(dmap, qsz[None], ksz[None], kidx, vl, context_length, prompt_length)
    qp = permute_rows(q[0], qidx2)
    kp = permute_rows(k[0], kidx2)
    vp = permute_rows(v[0], kidx2)
    op = block_sparse_attention(qp[None], kp[None], vp[None], m2, qs2, ks2, attn_dtype)[0]
    return unpermute_rows(op, qidx2)[None]


def hunyuan_dense_attention(query, key, value, valid_length: int, compute_dtype=np.float64):
    """The full-precision gate (``svoo/models/hunyuan10/attention.py:1113-1185``): tokens ``< valid_length``
    attend each other, the rest (prompt padding) attend each other; ``[1, H, S, D]``."""
    q = np.asarray(query)
    b, h, s, d = q.shape
    m = np.zeros((b, h, 2, 2), dtype=bool)
    m[:, :, 0, 0] = m[:, :, 1, 1] = True
    sz = np.broadcast_to(np.array([valid_length, s - valid_length]), (b, h, 2))
    return block_sparse_attention(query, key, value, m, sz, sz, compute_dtype)


# --------------------------------------------------------------------------------------
# Offline profile producer: exact attention sparsity
# --------------------------------------------------------------------------------------
def sparsity_weights(scores, scale: float) -> np.ndarray:
    """Unnormalised softmax weights of score rows: ``float32(exp(float64(s - m)))`` with
    ``s = float32(score) * float32(scale)`` and ``m`` the row max (fp32 subtraction).  The reference
    softmaxes ``matmul(q, k^T).float() * scale`` (``svoo/sparsity/exact.py:216-221``); counts depend
    only on ratios of weights, so the normalisation by the row sum is left out."""
    s = np.asarray(scores, dtype=np.float32) * np.float32(scale)
    m = s.max(axis=-1, keepdims=True)
    return np.exp((s - m).astype(np.float64)).astype(np.float32)


def exact_sparsity_counts(scores, scale: float, threshold: float) -> np.ndarray:
    """Per-row key count covering ``threshold`` of the mass: weights sorted descending, fp64 cumulative
    sum, ``searchsorted(cumsum, threshold * total, right=False) + 1``
    (``svoo/sparsity/exact.py:110-155``, in fp64 where the reference's cumsum is fp32)."""
    e = sparsity_weights(scores, scale).astype(np.float64)
    w = -np.sort(-e, axis=-1)
    cum = np.cumsum(w, axis=-1)
    target = threshold * cum[..., -1:]
    return (cum < target).sum(axis=-1).astype(np.int64) + 1


def exact_attention_sparsity(query, key, threshold: float = 0.95, query_sample_size: int = 0):
    """``compute_exact_attention_sparsity`` (``svoo/sparsity/exact.py:177-246``): bf16 scores
    ``bf16(q . k)`` (exact dots rounded like a bf16 matmul output), per-row counts, per-head mean of
    ``count / Sk``.  Returns ``(avg, per_head, counts)``; query rows are sampled as the reference
    does (uniform ``linspace`` positions, rounded, duplicates dropped)."""
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    b, h, sq, d = q.shape
    sk = k.shape[2]
    if query_sample_size and 0 < query_sample_size < sq:
        if query_sample_size == 1:
            pos = np.array([sq // 2])
        else:
            # torch.linspace in float32, then round-half-even and unique_consecutive
            pos = np.unique(np.round(np.linspace(0, sq - 1, query_sample_size, dtype=np.float32)).astype(np.int64))
        q = q[:, :, pos]
    scores = bf16_round(np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64)).astype(np.float32))
    counts = exact_sparsity_counts(scores, d ** -0.5, threshold)
    per_head = (counts / float(sk)).mean(axis=(0, 2))
    return float(per_head.mean()), per_head.tolist(), counts


# --------------------------------------------------------------------------------------
# EAR: error-aware routing with centroid compensation (svoo/co_clustering.py:1314-2050)
# --------------------------------------------------------------------------------------
def value_centroids(v_perm, k_sizes, dtype: str = "bf16") -> np.ndarray:
    """Mean value row of each key cluster over the cluster-contiguous ``v_perm`` ``[BH, N, D]``
    (``_compute_value_centroids``, ``svoo/models/wan/attention.py:593-610``): the reference scatter-adds the
    members into a bf16 tensor and divides by ``bf16(max(count, 1))``.  Contract: the member sum is exact,
    rounded (via float32) to the storage dtype, then divided in float32 by the storage-rounded count and rounded
    again; an empty cluster gives 0."""
    v = np.asarray(v_perm, np.float32)
    ks = np.asarray(k_sizes, np.int64)
    bh, _, d = v.shape
    kn = ks.shape[-1]
    out = np.zeros((bh, kn, d), np.float32)
    for b in range(bh):
        off = np.concatenate([[0], np.cumsum(ks[b])])
        for j in range(kn):
            sm = v[b, off[j]:off[j + 1]].astype(np.float64).sum(axis=0)
            s_st = storage_round(sm.astype(np.float32), dtype).astype(np.float32)
            den = storage_round(np.float32(max(int(ks[b, j]), 1)), dtype).astype(np.float32)
            out[b, j] = storage_round((s_st / den).astype(np.float32), dtype)
    return out


def value_stats(v_perm, vc, k_sizes) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Per-token ``|v_t|^2`` and ``vc_j . v_t`` (t in cluster j) and per-cluster ``|vc_j|^2``
    (``_precompute_v_stats_kernel``, ``co_clustering.py:1315-1396``), in float64."""
    v = np.asarray(v_perm, np.float64)
    c = np.asarray(vc, np.float64)
    ks = np.asarray(k_sizes, np.int64)
    labels = np.stack([np.repeat(np.arange(ks.shape[-1]), ks[b]) for b in range(ks.shape[0])])
    vn = (v * v).sum(-1)
    cvd = np.einsum("bnd,bnd->bn", v, np.take_along_axis(c, labels[..., None], axis=1))
    return vn, cvd, (c * c).sum(-1)


def ear_centroid_logits(qc, kc, dtype: str = "bf16") -> np.ndarray:
    """``einsum(Qc, Kc) * D**-0.5`` on bf16 tensors (``co_clustering.py:1725``): the bf16 product times the
    float32 scale, rounded to bf16."""
    d = np.asarray(qc).shape[-1]
    s = storage_round(_exact_matmul_nt(qc, kc), dtype)
    return storage_round((s.astype(np.float32) * np.float32(d ** -0.5)).astype(np.float32), dtype)


def ear_efficiency_scores(qc, c_logits, k_perm, v_perm, vc, q_sizes, k_sizes, gamma: float, eps: float = 1e-8):
    """``log(err_ij) - gamma * log(max(|Q_i| |K_j|, eps))`` (``co_clustering.py:1399-1567``) with
    ``err_ij = max(sum_t || e^{a_t} v_t - e^{c_ij} vc_j ||^2, eps)`` over the tokens t of key cluster j,
    ``a_t = (qc_i . k_t) / sqrt(D)`` and ``c_ij`` the bf16 centroid logit; evaluated in float64 with the
    exponents shifted by ``max(c_ij, max_t a_t)``.  Inputs ``[BH, ...]``; returns float32 ``[BH, Qc, Kc]``."""
    qc = np.asarray(qc, np.float64)
    c = np.asarray(c_logits, np.float64)
    kp = np.asarray(k_perm, np.float64)
    vp = np.asarray(v_perm, np.float64)
    vcv = np.asarray(vc, np.float64)
    qs = np.asarray(q_sizes, np.int64)
    ks = np.asarray(k_sizes, np.int64)
    bh, qn, d = qc.shape
    kn = ks.shape[-1]
    scale = d ** -0.5
    out = np.empty((bh, qn, kn), np.float32)
    for b in range(bh):
        koff = np.concatenate([[0], np.cumsum(ks[b])])
        a_all = (qc[b] @ kp[b].T) * scale  # [Qc, N]
        vn = (vp[b] ** 2).sum(axis=1)
        for j in range(kn):
            t0, t1 = koff[j], koff[j + 1]
            cj = c[b, :, j]
            if t1 > t0:
                a = a_all[:, t0:t1]
                m = np.maximum(cj, a.max(axis=1))
                e = np.exp(a - m[:, None])
                cvd = vp[b, t0:t1] @ vcv[b, j]
                s2 = (e * e * vn[None, t0:t1]).sum(axis=1)
                x = (e * cvd[None, :]).sum(axis=1)
            else:
                m = cj
                s2 = x = np.zeros(qn)
            pc = np.exp(cj - m)
            err = s2 - 2.0 * pc * x + pc * pc * float(vcv[b, j] @ vcv[b, j]) * (t1 - t0)
            with np.errstate(divide="ignore", invalid="ignore"):
                lerr = np.where(err > 0, np.log(np.where(err > 0, err, 1.0)) + 2.0 * m, -np.inf)
            lerr = np.maximum(lerr, np.log(eps))
            area = np.maximum(qs[b].astype(np.float64) * (t1 - t0), eps)
            out[b, :, j] = (lerr - gamma * np.log(area)).astype(np.float32)
    return out


def ear_row_params(h: int, kc_num: int, min_kc_ratio=0) -> Tuple[np.ndarray, np.ndarray]:
    """Per-head ``(preserve, budget_preserve)`` of the EAR selection (``co_clustering.py:1740-1781``):
    ``max(1, int(r * Kc))`` and ``max(1, int(r * Kc * 2))`` for ``r > 0``, else 0.  A sequence (or tensor)
    of H ratios is read through float32; one of length 1, or a number, in double precision; any other length
    gives no minimum."""
    pre = np.zeros(h, np.int64)
    bpre = np.zeros(h, np.int64)
    if isinstance(min_kc_ratio, (int, float, np.floating, np.integer)) or np.ndim(min_kc_ratio) == 0:
        rs = [float(min_kc_ratio)] * h
    else:
        n = len(min_kc_ratio)
        if n == h:
            rs = _ratio_list(min_kc_ratio, h)
        elif n == 1:
            rs = [float(min_kc_ratio[0])] * h
        else:
            rs = [0.0] * h
    for i, r in enumerate(rs):
        if r > 0:
            pre[i] = max(1, int(r * kc_num))
            bpre[i] = max(1, int(r * kc_num * 2))
    return pre, bpre


def ear_select(eff, c_logits, q_sizes, k_sizes, top_p: float, min_kc_ratio=0, dtype: str = "bf16") -> np.ndarray:
    """EAR block map (``identify_dynamic_map_estimated``, ``co_clustering.py:1692-1797``), per (b, h, i) row:

    1. budget probabilities ``softmax(bf16(c + bf16(log(bf16(|K_j|) + 1e-8))))`` rounded to bf16, sorted
       (descending, stable); the budget keeps position 0 and every later position whose predecessor's
       cumulative probability is ``<= top_p`` (exact fixed-point prefix, rounded to bf16, as the SVOO mask),
       at least ``budget_preserve`` positions; ``budget = sum |Q_i||K_j|`` over them;
    2. the first ``preserve`` budget-ordered clusters are guaranteed; ``remaining = max(budget - their area, 0)``;
    3. the other clusters in descending efficiency order (stable) are kept while the area before them is
       ``< remaining``.
    Areas are exact integers (the reference sums them in float32)."""
    eff = np.asarray(eff, np.float32)
    c = np.asarray(c_logits, np.float32)
    qs = np.asarray(q_sizes, np.int64)
    ks = np.asarray(k_sizes, np.int64)
    b, h, qn, kn = eff.shape
    pre, bpre = ear_row_params(h, kn, min_kc_ratio)
    p_st = storage_round(np.float32(top_p), dtype)
    # torch.log(kc_sz.to(bf16) + eps): the sum is a bf16 tensor, rounded before the log
    ks_eps = storage_round(storage_round(ks.astype(np.float32), dtype).astype(np.float32) + np.float32(1e-8), dtype)
    lks = storage_round(np.log(ks_eps.astype(np.float64)).astype(np.float32), dtype)  # exact log, rounded
    logits = storage_round(c + lks[:, :, None, :].astype(np.float32), dtype).astype(np.float64)
    out = np.zeros((b, h, qn, kn), bool)
    j_idx = np.arange(kn)
    for bi in range(b):
        for hi in range(h):
            for i in range(qn):
                lg = logits[bi, hi, i]
                e = np.exp(lg - lg.max())
                pb = storage_round((e / e.sum()).astype(np.float32), dtype)
                order = np.lexsort((j_idx, -pb.astype(np.float64)))
                prefix = np.cumsum(_fixed_point(pb[order]))
                cum = _prefix_to_bf16(prefix)
                le = cum[: kn - 1] <= p_st
                lead = int(np.argmin(le)) if not le.all() else kn - 1
                length = max(1 + lead, int(bpre[hi]))
                length = min(length, kn)
                area = qs[bi, hi, i] * ks[bi, hi]
                budget = int(area[order[:length]].sum())
                guar = order[: int(pre[hi])]
                remaining = max(budget - int(area[guar].sum()), 0)
                e2 = eff[bi, hi, i].astype(np.float64).copy()
                e2[guar] = -1e10
                order2 = np.lexsort((j_idx, -e2))
                cum2 = np.cumsum(area[order2])
                keep = (cum2 - area[order2]) < remaining
                out[bi, hi, i, guar] = True
                out[bi, hi, i, order2[keep]] = True
    return out


def ear_compensated_attention(q, k, v, k_centroids, v_centroids, dynamic_map, qc_size, kc_size,
                              compute_dtype=np.float64) -> np.ndarray:
    """Sparse attention over the active blocks plus centroid compensation of the pruned ones
    (``dynamic_block_sparse_prune_fwd_flashinfer`` + ``_fused_qc_kernel_opt``, ``co_clustering.py:1801-2050``):
    query cluster i attends to the tokens of its active key clusters and, for every inactive key cluster j,
    to the centroid pair ``(Kc_j, Vc_j)`` with logit ``q . Kc_j / sqrt(D) + log(|K_j| + 1e-6)``; one softmax
    over both.  ``[B, H, S, D]`` in, ``[B, H, S, D]`` out."""
    q = np.asarray(q)
    b, h, s, d = q.shape
    kk_all = np.asarray(k)
    vv_all = np.asarray(v)
    kcv = np.asarray(k_centroids)
    vcv = np.asarray(v_centroids)
    m = np.asarray(dynamic_map, bool)
    qs = np.asarray(qc_size).astype(np.int64)
    ks = np.asarray(kc_size).astype(np.int64)
    out = np.zeros((b, h, s, d), compute_dtype)
    scale = float(d) ** -0.5
    for bi in range(b):
        for hi in range(h):
            qoff = np.concatenate([[0], np.cumsum(qs[bi, hi])])
            koff = np.concatenate([[0], np.cumsum(ks[bi, hi])])
            kk = kk_all[bi, hi].astype(compute_dtype)
            vv = vv_all[bi, hi].astype(compute_dtype)
            kcc = kcv[bi, hi].astype(compute_dtype)
            vcc = vcv[bi, hi].astype(compute_dtype)
            bias = np.log(ks[bi, hi].astype(np.float32) + np.float32(1e-6)).astype(compute_dtype)
            for i in range(qs.shape[-1]):
                a, e = qoff[i], qoff[i + 1]
                if e == a:
                    continue
                act = np.nonzero(m[bi, hi, i])[0]
                ina = np.nonzero(~m[bi, hi, i])[0]
                rows = np.concatenate([np.arange(koff[j], koff[j + 1]) for j in act]) if len(act) else np.zeros(0, np.int64)
                qi = q[bi, hi, a:e].astype(compute_dtype)
                keys = np.concatenate([kk[rows], kcc[ina]])
                vals = np.concatenate([vv[rows], vcc[ina]])
                sc = (qi @ keys.T) * compute_dtype(scale)
                sc[:, len(rows):] += bias[ina][None, :]
                sc -= sc.max(axis=1, keepdims=True)
                pr = np.exp(sc)
                pr /= pr.sum(axis=1, keepdims=True)
                out[bi, hi, a:e] = pr @ vals
    return out


def ear_attention_call(query, key, value, num_q_centroids: int, num_k_centroids: int, kmeans_iters: int,
                       top_p: float, min_kc_ratio=0, gamma: float = 1.0, *, init_q_idx=None, init_k_idx=None,
                       init_q_centroids=None, init_k_centroids=None, dtype: str = "bf16", attn_dtype=np.float64,
                       return_parts: bool = False):
    """One EAR ``attention_core_logic`` call (``svoo/models/wan/attention.py:1040-1071, 1180-1215``):
    co-cluster, permute, value centroids by key label, EAR block map, compensated sparse attention, inverse
    permutation, ``[1, S, H*D]``."""
    q = np.asarray(query, np.float32)
    k = np.asarray(key, np.float32)
    v = np.asarray(value, np.float32)
    b, h, s, d = q.shape
    assert b == 1
    ql, qcent, qsz, kl, kcent, ksz = co_cluster_tokens(q[0], k[0], num_q_centroids, num_k_centroids, kmeans_iters,
                                                       init_q_idx=init_q_idx, init_k_idx=init_k_idx,
                                                       init_q_centroids=init_q_centroids,
                                                       init_k_centroids=init_k_centroids, dtype=dtype)
    qidx, _, _ = cluster_sort(ql, num_q_centroids)
    kidx, _, _ = cluster_sort(kl, num_k_centroids)
    qp = permute_rows(q[0], qidx)
    kp = permute_rows(k[0], kidx)
    vp = permute_rows(v[0], kidx)
    vc = value_centroids(vp, ksz, dtype)
    c = ear_centroid_logits(qcent, kcent, dtype)
    eff = ear_efficiency_scores(qcent, c, kp, vp, vc, qsz, ksz, gamma)
    dmap = ear_select(eff[None], c[None], qsz[None], ksz[None], top_p, min_kc_ratio, dtype)
    op = ear_compensated_attention(qp[None], kp[None], vp[None], kcent[None], vc[None], dmap, qsz[None], ksz[None],
                                   attn_dtype)[0]
    o = unpermute_rows(op, qidx)
    out = o.transpose(1, 0, 2).reshape(1, s, h * d)
    if return_parts:
        return out, dict(map=dmap, eff=eff, c=c, vc=vc, qsizes=qsz, ksizes=ksz, qidx=qidx, kidx=kidx,
                         qcent=qcent, kcent=kcent, qlabels=ql, klabels=kl)
    return out
