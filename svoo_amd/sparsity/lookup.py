"""Per-(step, layer, head) sparsity profile lookup.

Same interface and semantics as ``svoo/sparsity/lookup.py:9-45``: a ``Step,Layer,Head,Sparsity``
CSV (1-based steps) loaded into a dict; missing entries read as ``None`` (``get_sparsity``) or
``0.0`` (``get_sparsity_batch``).
"""

from __future__ import annotations

import csv
from pathlib import Path
from typing import Dict, List, Optional, Tuple


class SparsityLookup:
    """In-memory lookup table for per-step, per-layer, per-head sparsity."""

    def __init__(self, csv_path: str, verbose: bool = True):
        self.lookup_dict: Dict[Tuple[int, int, int], float] = {}
        self._load_csv(csv_path, verbose)

    def _load_csv(self, csv_path: str, verbose: bool) -> None:
        path = Path(csv_path)
        if not path.exists():
            raise FileNotFoundError(f"Sparsity CSV file not found: {csv_path}")
        with open(path, "r", encoding="utf-8") as f:
            for row in csv.DictReader(f):
                key = (int(row["Step"]), int(row["Layer"]), int(row["Head"]))
                self.lookup_dict[key] = float(row["Sparsity"])
        if verbose:
            print(f"Loaded {len(self.lookup_dict)} sparsity entries from {csv_path}")

    def get_sparsity(self, step: int, layer: int, head: int) -> Optional[float]:
        """One value, or ``None`` when the entry is missing."""
        return self.lookup_dict.get((step, layer, head))

    def get_sparsity_batch(self, step: int, layer: int, num_heads: int) -> List[float]:
        """Values of every head of one step/layer; missing (or zero) entries read as ``0.0``."""
        return [self.get_sparsity(step, layer, h) or 0.0 for h in range(num_heads)]

    def has_data_for_step_layer(self, step: int, layer: int, num_heads: int = 12) -> bool:
        """True only when every expected head exists for this step/layer."""
        return all(self.get_sparsity(step, layer, h) is not None for h in range(num_heads))
