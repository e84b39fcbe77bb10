"""Merge raw sparsity logs into the ``Step,Layer,Head,Sparsity`` profile CSV.

Same log format and merge rule as ``svoo/sparsity/merge.py:16-106``: each raw log holds blocks of
``[Sparsity] Layer L | Type: T | Step: S ...`` followed by ``  Head H: Sparsity=V`` lines; the merged
profile keeps, per (step, layer, head), the maximum over the input logs (prompt samples).

    python -m svoo_amd.sparsity.merge -i run1.txt run2.txt -o profile.csv
"""

from __future__ import annotations

import argparse
import csv
import re
from pathlib import Path
from typing import Dict, Iterable, Tuple

_HEADER = re.compile(r"\[Sparsity\] Layer (\d+) \| Type: \w+ \| Step: (\d+)")
_HEAD = re.compile(r"\s*Head\s+(\d+):\s+Sparsity=([\d.]+)")

Key = Tuple[int, int, int]  # (step, layer, head)


def parse_sparsity_file(file_path) -> Dict[Key, float]:
    """``{(step, layer, head): sparsity}`` of one raw log (the maximum when an entry repeats);
    an unreadable file gives ``{}``."""
    data: Dict[Key, float] = {}
    try:
        with open(file_path, "r", encoding="utf-8") as f:
            step = layer = None
            for line in f:
                m = _HEADER.match(line)
                if m:
                    layer, step = int(m.group(1)), int(m.group(2))
                    continue
                hm = _HEAD.match(line)
                if hm and step is not None:
                    k = (step, layer, int(hm.group(1)))
                    data[k] = max(data.get(k, 0.0), float(hm.group(2)))
    except OSError as e:
        print(f"Error reading {file_path}: {e}")
        return {}
    return data


def merge_sparsity_data(file_paths: Iterable) -> Dict[Key, float]:
    """Maximum over the logs of every (step, layer, head) entry."""
    merged: Dict[Key, float] = {}
    for p in file_paths:
        for k, v in parse_sparsity_file(p).items():
            merged[k] = max(merged.get(k, v), v)
    return merged


def save_to_csv(data: Dict[Key, float], output_path) -> None:
    """Write the profile sorted by (step, layer, head)."""
    out = Path(output_path)
    out.parent.mkdir(parents=True, exist_ok=True)
    with open(out, "w", newline="", encoding="utf-8") as f:
        w = csv.writer(f)
        w.writerow(["Step", "Layer", "Head", "Sparsity"])
        for (step, layer, head), v in sorted(data.items()):
            w.writerow([step, layer, head, v])


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Merge raw attention-sparsity logs into a profile CSV")
    ap.add_argument("-i", "--inputs", nargs="+", required=True)
    ap.add_argument("-o", "--output", required=True)
    args = ap.parse_args(argv)
    data = merge_sparsity_data(args.inputs)
    if not data:
        print("no sparsity entries found")
        return 1
    save_to_csv(data, args.output)
    vals = list(data.values())
    print(f"{len(data)} entries, mean {sum(vals) / len(vals):.6f}, min {min(vals):.6f}, max {max(vals):.6f} "
          f"-> {args.output}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
