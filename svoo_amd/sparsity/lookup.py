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
    """A profile CSV held as a ``{(step, layer, head): ratio}`` dict, read by the online mask every step.

    The CSV is parsed once at construction; lookups are plain dict reads, so the processors can query
    it per call without touching the file or the GPU.
    """

    def __init__(self, csv_path: str, verbose: bool = True):
        self.lookup_dict: Dict[Tuple[int, int, int], float] = {}
        self._load_csv(csv_path, verbose)

    def _load_csv(self, csv_path: str, verbose: bool) -> None:
        path = Path(csv_path)
        if not path.exists():
            raise FileNotFoundError(f"Sparsity CSV file not found: {csv_path}")
        with open(path, "r", encoding="utf-8") as f:
            self.lookup_dict.update(
                ((int(r["Step"]), int(r["Layer"]), int(r["Head"])), float(r["Sparsity"])) for r in csv.DictReader(f))
        if verbose:
            print(f"Loaded {len(self.lookup_dict)} sparsity entries from {csv_path}")

    def get_sparsity(self, step: int, layer: int, head: int) -> Optional[float]:
        """The ratio stored for ``(step, layer, head)``; ``None`` if the profile has no such row."""
        return self.lookup_dict.get((step, layer, head))

    def get_sparsity_batch(self, step: int, layer: int, num_heads: int) -> List[float]:
        """Ratios of heads ``0 .. num_heads - 1`` at one step and layer; an absent or zero row gives ``0.0``."""
        return [self.get_sparsity(step, layer, h) or 0.0 for h in range(num_heads)]

    def has_data_for_step_layer(self, step: int, layer: int, num_heads: int = 12) -> bool:
        """Whether the profile covers all ``num_heads`` heads of this step and layer (a partial layer is
        treated as absent by the processors, which then fall back to the scalar ratio)."""
        return all(self.get_sparsity(step, layer, h) is not None for h in range(num_heads))
