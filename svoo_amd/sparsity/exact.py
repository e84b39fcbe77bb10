"""Exact attention-sparsity profiling on the GPU (the producer of the per-head profiles).

``compute_exact_attention_sparsity`` keeps the name, arguments and return value of
``svoo/sparsity/exact.py:177-246``: the sparsity of a head is the mean over query rows of
``count / seq_len_k``, where ``count`` is the smallest number of keys whose softmax weights hold
``threshold`` of the row's mass.  The reference materialises fp32 probabilities, sorts every row
and searches a cumulative sum; here the score matmul stays a library GEMM (bf16 scores, as the
reference's ``torch.matmul`` of bf16 inputs) and ``svoo_exact_sparsity_counts`` finds each row's
count with two histogram passes over the bf16 scores (no sort, no fp32 probability tensor).

Counting contract: weights ``e_j = float(exp(double(s_j - m)))`` with ``s_j = float(score_j) *
scale`` in fp32 and ``m`` the row max; prefix masses in fp64 over the weights in descending order;
``count = #{prefix < threshold * total} + 1`` (``torch.searchsorted(..., right=False) + 1``).  The
reference's own fp32 softmax and cumsum can move a count by one key where the target falls within
fp32 rounding of a prefix sum.
"""

from __future__ import annotations

import os
import re
from typing import List, Tuple

import torch

from .. import _lib

DEFAULT_SPARSITY_THRESHOLD = 0.95
DEFAULT_AUTO_MEMORY_FRACTION = 0.45
# bf16 scores plus the GEMM's own workspace, per score (the counts need no per-score scratch)
_BYTES_PER_SCORE = 4
_SPARSITY_HEADER_RE = re.compile(r"\[Sparsity\] Layer (\d+) \| Type: \w+ \| Step: (\d+)")
_SPARSITY_HEAD_RE = re.compile(r"\s*Head\s+(\d+):\s+Sparsity=")


def _auto_query_chunk_size(query: torch.Tensor, key: torch.Tensor) -> int:
    """Largest query chunk whose bf16 scores fit a fraction of free device memory (``exact.py:21-47``)."""
    batch, num_heads, seq_len_q, _ = query.size()
    seq_len_k = key.size(2)
    try:
        free_bytes, _ = torch.cuda.mem_get_info(query.device)
    except Exception:
        return min(128, seq_len_q)
    try:
        frac = float(os.environ.get("SVOO_SPARSITY_AUTO_MEM_FRACTION", DEFAULT_AUTO_MEMORY_FRACTION))
    except ValueError:
        frac = DEFAULT_AUTO_MEMORY_FRACTION
    frac = min(0.90, max(0.05, frac))
    per_query = max(1, batch * num_heads * seq_len_k * _BYTES_PER_SCORE)
    chunk = int(free_bytes * frac / per_query)
    if chunk >= 16:
        chunk = (chunk // 8) * 8
    return max(1, min(seq_len_q, chunk))


def _sample_query_rows(query: torch.Tensor, sample_size: int):
    """Deterministic uniform subset of query rows, or all rows (``exact.py:158-174``)."""
    seq_len_q = query.size(2)
    sample_size = int(sample_size or 0)
    if sample_size <= 0 or sample_size >= seq_len_q:
        return query, seq_len_q
    if sample_size == 1:
        positions = torch.tensor([seq_len_q // 2], device=query.device, dtype=torch.long)
    else:
        positions = torch.linspace(0, seq_len_q - 1, steps=sample_size, device=query.device)
        positions = torch.unique_consecutive(positions.round().long())
    return query.index_select(2, positions), int(positions.numel())


def exact_counts_from_scores(scores: torch.Tensor, scale: float, threshold: float) -> torch.Tensor:
    """Per-row counts of a bf16 score tensor ``[..., n]`` (rows = every leading index); int32 ``[...]``."""
    if scores.dtype != torch.bfloat16 or not scores.is_cuda:
        raise ValueError("exact_counts_from_scores needs bf16 scores on a HIP device")
    scores = scores.contiguous()
    n = scores.size(-1)
    rows = scores.numel() // n
    counts = torch.empty(scores.shape[:-1], dtype=torch.int32, device=scores.device)
    _lib.call("svoo_exact_sparsity_counts", scores.data_ptr(), rows, n, float(scale), float(threshold),
              counts.data_ptr(), _lib.stream_of(scores.device))
    return counts


@torch.no_grad()
def compute_exact_attention_sparsity(
    query: torch.Tensor,
    key: torch.Tensor,
    *,
    batch_size: int = 0,
    threshold: float = DEFAULT_SPARSITY_THRESHOLD,
    query_sample_size: int = 0,
) -> Tuple[float, List[float], dict]:
    """Per-head attention sparsity (the minimal key ratio covering ``threshold`` of the mass).

    ``query``/``key`` are bf16 ``[B, H, S, D]`` on a HIP device.  ``batch_size <= 0`` picks the query
    chunk from free memory; ``query_sample_size > 0`` estimates from a uniform row subset.  Returns
    ``(avg_sparsity, per_head_list, stats)`` like ``svoo/sparsity/exact.py:177-246``.
    """
    batch, num_heads, seq_len_q, dim = query.size()
    seq_len_k = key.size(2)
    threshold = float(threshold)
    if threshold <= 0.0 or threshold > 1.0:
        raise ValueError(f"sparsity threshold must be in (0, 1], got {threshold}")
    if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16:
        raise ValueError("compute_exact_attention_sparsity needs bf16 query and key (the SVOO attention dtype)")
    if not query.is_cuda:
        raise ValueError("compute_exact_attention_sparsity runs on a HIP device")
    query, sampled = _sample_query_rows(query, query_sample_size)
    rows_q = query.size(2)
    if batch_size is None or batch_size <= 0:
        batch_size = _auto_query_chunk_size(query, key)
    else:
        batch_size = min(int(batch_size), rows_q)
    scale = dim ** -0.5
    key_t = key.transpose(-2, -1)
    parts = []
    for q0 in range(0, rows_q, batch_size):
        qb = query[:, :, q0:q0 + batch_size, :]
        scores = torch.matmul(qb, key_t)  # bf16 [B, H, c, Sk]
        parts.append(exact_counts_from_scores(scores, scale, threshold))
        del scores
    counts = torch.cat(parts, dim=2)
    per_query = counts.double() / float(seq_len_k)
    per_head = per_query.mean(dim=(0, 2))
    avg = float(per_head.mean().item())
    stats = {
        "attn_scores_shape": [batch, num_heads, sampled, seq_len_k],
        "seq_len": seq_len_q,
        "sampled_seq_len": sampled,
        "chunk_size": batch_size,
    }
    return avg, per_head.cpu().tolist(), stats


_COMPLETION_CACHE: dict = {}


def _resume_enabled() -> bool:
    return os.environ.get("SVOO_SPARSITY_RESUME", "0") not in ("0", "", "false", "False")


def has_completed_sparsity_entry(output_file: str, layer_idx: int, step: int, num_heads: int) -> bool:
    """Opt-in resume guard (``SVOO_SPARSITY_RESUME``): True when the raw log already holds every head of
    this layer/step (``svoo/sparsity/exact.py:58-107``).  The file is read incrementally."""
    if not _resume_enabled() or not output_file or not os.path.exists(output_file):
        return False
    try:
        st = os.stat(output_file)
        ident = (st.st_dev, st.st_ino)
        cache = _COMPLETION_CACHE.get(output_file)
        if cache is None or cache["id"] != ident or st.st_size < cache["offset"]:
            cache = {"id": ident, "offset": 0, "key": None, "heads": {}}
            _COMPLETION_CACHE[output_file] = cache
        with open(output_file, "r", encoding="utf-8") as f:
            f.seek(cache["offset"])
            for line in f:
                m = _SPARSITY_HEADER_RE.match(line)
                if m:
                    cache["key"] = (int(m.group(1)), int(m.group(2)))
                    cache["heads"].setdefault(cache["key"], set())
                    continue
                if cache["key"] is not None:
                    hm = _SPARSITY_HEAD_RE.match(line)
                    if hm:
                        cache["heads"][cache["key"]].add(int(hm.group(1)))
            cache["offset"] = f.tell()
        return set(range(int(num_heads))) <= cache["heads"].get((int(layer_idx), int(step)), set())
    except OSError:
        return False


def format_sparsity_log(layer_idx: int, attn_type: str, step: int, threshold: float, avg: float,
                        per_head: List[float], seq_len: int, sampled: int) -> List[str]:
    """Raw log lines of one layer/step (the format ``merge`` and the resume guard parse,
    ``svoo/models/wan/attention.py:480-489``)."""
    sample_text = f" | Query Samples: {sampled}/{seq_len}" if sampled != seq_len else ""
    lines = [f"[Sparsity] Layer {layer_idx} | Type: {attn_type} | Step: {step} | Threshold: {threshold:.2%} | "
             f"Avg Sparsity: {avg:.4f} | n={seq_len}{sample_text}"]
    lines += [f"  Head {h:2d}: Sparsity={v:.4f}" for h, v in enumerate(per_head)]
    return lines
