"""Token permutation by cluster labels (HIP).

Mirrors ``svoo/kernels/triton/permute.py:68-130`` (``permute_tensor_by_labels_triton``,
``apply_inverse_permutation_triton``): same names, arguments, return values and asserts.  The
sort behind it is a stable HIP counting sort (ascending token index inside a cluster), where the
reference uses the unstable ``torch.argsort``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def cluster_sort(labels: torch.Tensor, num_clusters: int, *, with_sorted_labels: bool = False):
    """Stable counting sort of ``labels[BH, N]``: ``(sorted_idx int32, sizes int32 [BH, K], offsets int32 [BH, K])``.

    With ``with_sorted_labels`` a fourth output holds the labels in sorted order.  Labels must lie in
    ``[0, num_clusters)``; tokens with labels outside are dropped by the kernel.
    """
    _lib.require_gpu_tensor(labels, "labels")
    assert labels.dim() == 2, "labels must be [BH, N]"
    bh, n = labels.shape
    lab = labels.to(torch.int32).contiguous()
    dev = lab.device
    sorted_idx = torch.empty(bh, n, dtype=torch.int32, device=dev)
    sizes = torch.empty(bh, num_clusters, dtype=torch.int32, device=dev)
    offsets = torch.empty(bh, num_clusters, dtype=torch.int32, device=dev)
    sorted_lab = torch.empty(bh, n, dtype=torch.int32, device=dev) if with_sorted_labels else None
    if n == 0:
        sizes.zero_()
        offsets.zero_()
        return (sorted_idx, sizes, offsets, sorted_lab) if with_sorted_labels else (sorted_idx, sizes, offsets)
    L = _lib.lib()
    nbytes = L.svoo_cluster_sort_workspace_size(bh, n, num_clusters)
    ws = _lib.workspace(nbytes, dev)
    _lib.call("svoo_cluster_sort", lab.data_ptr(), bh, n, num_clusters, sorted_idx.data_ptr(), sizes.data_ptr(),
              offsets.data_ptr(), _lib.ptr(sorted_lab), ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    if with_sorted_labels:
        return sorted_idx, sizes, offsets, sorted_lab
    return sorted_idx, sizes, offsets


def _row_bytes(t: torch.Tensor) -> int:
    rb = t.shape[-1] * t.element_size()
    if rb % 16 or (256 % (rb // 16)) or rb // 16 > 256:
        raise ValueError(f"row of {rb} bytes is not supported (needs 16 * 2^i bytes, at most 4096)")
    return rb


def permute_tensor_by_labels(
    tensor: torch.Tensor,
    labels: Optional[torch.Tensor],
    dim: int,
    *,
    sorted_indices: Optional[torch.Tensor] = None,
    num_clusters: Optional[int] = None,
):
    """Permute a ``[B, H, S, D]`` tensor along the sequence dimension so clusters are contiguous.

    Returns ``(permuted, sorted_indices int32 [B*H, S])``.  With ``sorted_indices`` given, the labels
    are ignored (``svoo/kernels/triton/permute.py:83-85``).  ``num_clusters`` bounds the label values;
    without it the maximum label is read back from the device.
    """
    assert dim == 2, "permute_tensor_by_labels currently only supports dim==2 (sequence dimension)"
    assert tensor.dim() == 4, "Expected tensor shape [B,H,S,D]"
    assert tensor.is_cuda, "permute_tensor_by_labels requires CUDA tensors"
    b, h, s, d = tensor.shape
    bh = b * h
    if sorted_indices is not None:
        sorted_indices = sorted_indices.to(device=tensor.device, dtype=torch.int32).contiguous()
    else:
        assert labels is not None, "Either `labels` or `sorted_indices` must be provided."
        labels = labels.to(tensor.device).reshape(bh, s)
        if num_clusters is None:
            lo, hi = int(labels.min()), int(labels.max())
            if lo < 0:
                raise ValueError("labels must be non-negative")
            num_clusters = hi + 1
        sorted_indices, _, _ = cluster_sort(labels, num_clusters)
    inp = tensor.reshape(bh, s, d).contiguous()
    out = torch.empty_like(inp)
    if s:
        _lib.call("svoo_permute_rows", inp.data_ptr(), sorted_indices.data_ptr(), out.data_ptr(), bh, s, s,
                  _row_bytes(inp), _lib.stream_of(inp.device))
    return out.reshape(b, h, s, d), sorted_indices


def permute_pair_by_indices(x0: torch.Tensor, x1: torch.Tensor, sorted_indices: torch.Tensor):
    """Permute two ``[B, H, S, D]`` tensors with one index (K and V) in a single pass."""
    assert x0.shape == x1.shape and x0.dtype == x1.dtype and x0.dim() == 4
    b, h, s, d = x0.shape
    a = x0.reshape(b * h, s, d).contiguous()
    c = x1.reshape(b * h, s, d).contiguous()
    ya, yc = torch.empty_like(a), torch.empty_like(c)
    idx = sorted_indices.to(device=a.device, dtype=torch.int32).contiguous()
    if s:
        _lib.call("svoo_permute_rows2", a.data_ptr(), c.data_ptr(), idx.data_ptr(), ya.data_ptr(), yc.data_ptr(),
                  b * h, s, _row_bytes(a), _lib.stream_of(a.device))
    return ya.reshape(b, h, s, d), yc.reshape(b, h, s, d)


def apply_inverse_permutation(permuted_tensor: torch.Tensor, sorted_indices: torch.Tensor, dim: int):
    """Undo :func:`permute_tensor_by_labels` for ``[B, H, S, D]`` tensors (``permute.py:105-130``)."""
    assert dim == 2, "apply_inverse_permutation currently only supports dim==2"
    assert permuted_tensor.dim() == 4, "Expected tensor shape [B,H,S,D]"
    assert permuted_tensor.is_cuda, "apply_inverse_permutation requires CUDA tensors"
    b, h, s, d = permuted_tensor.shape
    idx = sorted_indices.to(device=permuted_tensor.device, dtype=torch.int32).reshape(b * h, s).contiguous()
    inp = permuted_tensor.reshape(b * h, s, d).contiguous()
    out = torch.empty_like(inp)
    if s:
        _lib.call("svoo_unpermute_rows", inp.data_ptr(), idx.data_ptr(), out.data_ptr(), b * h, s, _row_bytes(inp),
                  _lib.stream_of(inp.device))
    return out.reshape(b, h, s, d)


# Reference names (the Triton suffix is kept for drop-in use).
permute_tensor_by_labels_triton = permute_tensor_by_labels
apply_inverse_permutation_triton = apply_inverse_permutation


def apply_inverse_permutation_bshd(permuted_tensor: torch.Tensor, sorted_indices: torch.Tensor) -> torch.Tensor:
    """``apply_inverse_permutation(x, idx, 2).transpose(1, 2).flatten(2, 3)`` in one HIP pass: ``[B, S, H*D]``."""
    assert permuted_tensor.dim() == 4 and permuted_tensor.is_cuda
    b, h, s, d = permuted_tensor.shape
    idx = sorted_indices.to(device=permuted_tensor.device, dtype=torch.int32).reshape(b * h, s).contiguous()
    inp = permuted_tensor.reshape(b * h, s, d).contiguous()
    out = torch.empty(b, s, h * d, dtype=inp.dtype, device=inp.device)
    if s:
        _lib.call("svoo_unpermute_rows_bshd", inp.data_ptr(), idx.data_ptr(), out.data_ptr(), b * h, s, h,
                  _row_bytes(inp), _lib.stream_of(inp.device))
    return out
