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
from typing import Dict, List, Set, Tuple

import torch

from .. import _lib

DEFAULT_SPARSITY_THRESHOLD = 0.95
# Share of the device's free memory one query chunk's bf16 scores may take when the chunk is sized
# automatically; SVOO_SPARSITY_AUTO_MEM_FRACTION overrides it (the reference's knob, same meaning).
DEFAULT_AUTO_MEMORY_FRACTION = 0.45
# Above this many score bytes per chunk the count kernel, not the GEMM launch count, sets the time,
# so larger chunks buy nothing and only hold memory.
_MAX_CHUNK_SCORE_BYTES = 4 << 30
_SCORE_BYTES = 2  # bf16 scores; the counts need no per-score scratch
_SPARSITY_HEADER_RE = re.compile(r"\[Sparsity\] Layer (\d+) \| Type: \w+ \| Step: (\d+)")
_SPARSITY_HEAD_RE = re.compile(r"\s*Head\s+(\d+):\s+Sparsity=")


def _memory_share() -> float:
    """The free-memory share from the environment, or the default when unset or not a number in (0, 1)."""
    raw = os.environ.get("SVOO_SPARSITY_AUTO_MEM_FRACTION")
    try:
        share = float(raw) if raw is not None else DEFAULT_AUTO_MEMORY_FRACTION
    except ValueError:
        return DEFAULT_AUTO_MEMORY_FRACTION
    return share if 0.0 < share < 1.0 else DEFAULT_AUTO_MEMORY_FRACTION


def _query_chunk_rows(query: torch.Tensor, key: torch.Tensor) -> int:
    """Query rows per chunk when the caller leaves it to us (``svoo/sparsity/exact.py:19-42`` sizes the
    reference's fp32 sort workspace the same way).

    One chunk of ``r`` rows holds ``B * H * r * S_k`` bf16 scores.  The budget is the smaller of
    ``_MAX_CHUNK_SCORE_BYTES`` and a share of free device memory; rows come in multiples of 64 (whole
    MFMA tiles of the score GEMM) once the budget allows 64.
    """
    b, h, rows_q, _ = query.shape
    bytes_per_row = max(1, b * h * key.size(2) * _SCORE_BYTES)
    try:
        free = torch.cuda.mem_get_info(query.device)[0]
    except Exception:
        # No free-memory figure (the query itself failed): a small fixed chunk, as the reference falls back to.
        return int(min(128, rows_q))
    budget = min(_MAX_CHUNK_SCORE_BYTES, int(free * _memory_share()))
    rows = budget // bytes_per_row
    if rows >= 64:
        rows -= rows % 64
    return int(min(rows_q, max(1, rows)))


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
    auto = batch_size is None or batch_size <= 0
    chunk = _query_chunk_rows(query, key) if auto else min(int(batch_size), rows_q)
    scale = dim ** -0.5
    key_t = key.transpose(-2, -1)
    parts = []
    q0 = 0
    while q0 < rows_q:
        try:
            scores = torch.matmul(query[:, :, q0:q0 + chunk, :], key_t)  # bf16 [B, H, c, Sk]
            part = exact_counts_from_scores(scores, scale, threshold)
        except torch.cuda.OutOfMemoryError:
            # Free memory can shrink between the sizing and the GEMM (other streams, the caching
            # allocator's fragmentation): an automatic chunk halves and the same rows are retried
            # (svoo/sparsity/exact.py:218-230).  An explicit chunk size is the caller's to fix.
            if not auto or chunk == 1:
                raise
            scores = None
            torch.cuda.empty_cache()
            chunk = max(1, chunk // 2)
            continue
        del scores
        parts.append(part)
        q0 += chunk
    counts = torch.cat(parts, dim=2)
    per_query = counts.double() / float(seq_len_k)
    per_head = per_query.mean(dim=(0, 2))
    avg = float(per_head.mean().item())
    stats = {
        "attn_scores_shape": [batch, num_heads, sampled, seq_len_k],
        "seq_len": seq_len_q,
        "sampled_seq_len": sampled,
        "chunk_size": chunk,
    }
    return avg, per_head.cpu().tolist(), stats


def resume_requested() -> bool:
    """The resume guard is on unless ``SVOO_SPARSITY_RESUME`` is unset or one of ``0``, the empty string,
    ``false`` and ``False`` (``svoo/sparsity/exact.py:50-51``, ``svoo/models/wan/inference.py:334``): any
    other value keeps the raw log and skips what it already holds."""
    return os.environ.get("SVOO_SPARSITY_RESUME", "0") not in ("0", "", "false", "False")


class SparsityLogIndex:
    """The (layer, step) -> heads entries of one raw sparsity log.

    Each query stats the file: when its identity (device, inode) changed or it shrank below what was read,
    the index is rebuilt from the start; when it grew, only the new complete lines are parsed (the reference's
    cache, ``svoo/sparsity/exact.py:54-102``).  An unterminated last line is left for a later read, so a
    line being written is never taken in half.  :meth:`add` records this process's own appends at once.
    """

    def __init__(self, path: str):
        self.path = path
        self.heads: Dict[Tuple[int, int], Set[int]] = {}
        self._file_id = None
        self._offset = 0
        self._entry = None
        self.refresh()

    def _reset(self, file_id) -> None:
        self.heads = {}
        self._file_id = file_id
        self._offset = 0
        self._entry = None

    def refresh(self) -> None:
        """Bring the index up to the file's current contents."""
        try:
            st = os.stat(self.path)
        except OSError:
            return
        file_id = (st.st_dev, st.st_ino)
        if file_id != self._file_id or st.st_size < self._offset:
            self._reset(file_id)
        if st.st_size == self._offset:
            return
        try:
            with open(self.path, "rb") as f:
                f.seek(self._offset)
                data = f.read()
        except OSError:
            return
        end = data.rfind(b"\n") + 1
        for raw in data[:end].splitlines():
            line = raw.decode("utf-8", errors="replace")
            m = _SPARSITY_HEADER_RE.match(line)
            if m:
                self._entry = self.heads.setdefault((int(m.group(1)), int(m.group(2))), set())
            elif self._entry is not None:
                hm = _SPARSITY_HEAD_RE.match(line)
                if hm:
                    self._entry.add(int(hm.group(1)))
        self._offset += end

    def add(self, layer_idx: int, step: int, heads) -> None:
        self.heads.setdefault((int(layer_idx), int(step)), set()).update(int(h) for h in heads)

    def complete(self, layer_idx: int, step: int, num_heads: int) -> bool:
        have = self.heads.get((int(layer_idx), int(step)), ())
        return all(h in have for h in range(int(num_heads)))


_LOG_INDEX: Dict[str, SparsityLogIndex] = {}


def _log_index(output_file: str) -> SparsityLogIndex:
    key = os.path.realpath(output_file)
    if key not in _LOG_INDEX:
        _LOG_INDEX[key] = SparsityLogIndex(key)
    return _LOG_INDEX[key]


def has_completed_sparsity_entry(output_file: str, layer_idx: int, step: int, num_heads: int) -> bool:
    """Opt-in resume guard (``SVOO_SPARSITY_RESUME``): True when the raw log already holds every head of
    this layer/step, so the measurement can be skipped (``svoo/sparsity/exact.py:54-102``)."""
    if not resume_requested() or not output_file or not os.path.exists(output_file):
        return False
    index = _log_index(output_file)
    index.refresh()
    return index.complete(layer_idx, step, num_heads)


def record_sparsity_entry(output_file: str, layer_idx: int, step: int, heads) -> None:
    """Tell the resume guard about lines this process appended to ``output_file``."""
    if output_file and os.path.realpath(output_file) in _LOG_INDEX:
        _log_index(output_file).add(layer_idx, step, heads)


def format_sparsity_log(layer_idx: int, attn_type: str, step: int, threshold: float, avg: float,
                        per_head: List[float], seq_len: int, sampled: int) -> List[str]:
    """Raw log lines of one layer/step (the format ``merge`` and the resume guard parse,
    ``svoo/models/wan/attention.py:480-489``)."""
    sample_text = f" | Query Samples: {sampled}/{seq_len}" if sampled != seq_len else ""
    lines = [f"[Sparsity] Layer {layer_idx} | Type: {attn_type} | Step: {step} | Threshold: {threshold:.2%} | "
             f"Avg Sparsity: {avg:.4f} | n={seq_len}{sample_text}"]
    lines += [f"  Head {h:2d}: Sparsity={v:.4f}" for h, v in enumerate(per_head)]
    return lines
