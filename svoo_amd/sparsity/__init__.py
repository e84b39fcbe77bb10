"""Per-head sparsity profiles: the lookup the online mask reads, the exact GPU profiler that
produces them, and the merge of raw profiling logs into the profile CSV."""

from .lookup import SparsityLookup
from .exact import (
    DEFAULT_SPARSITY_THRESHOLD,
    compute_exact_attention_sparsity,
    exact_counts_from_scores,
    format_sparsity_log,
    has_completed_sparsity_entry,
    record_sparsity_entry,
)
from .merge import merge_sparsity_data, parse_sparsity_file, save_to_csv

__all__ = [
    "SparsityLookup",
    "DEFAULT_SPARSITY_THRESHOLD",
    "compute_exact_attention_sparsity",
    "exact_counts_from_scores",
    "format_sparsity_log",
    "has_completed_sparsity_entry",
    "record_sparsity_entry",
    "merge_sparsity_data",
    "parse_sparsity_file",
    "save_to_csv",
]
