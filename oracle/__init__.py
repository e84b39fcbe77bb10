"""CPU oracle for the SVOO online sparse-attention hot path.

TEST INFRASTRUCTURE ONLY.  This package is a numpy (float64) restatement of the
reference algorithm, written from the reference source text.  It exists to
check the HIP implementation in ``svoo_amd`` and to time a CPU baseline.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed baseline.
The product path (``svoo_amd``) never imports, calls or falls back to it.

Every function cites the reference ``file:line`` it follows (paths relative to
the reference repository root).  Where the reference's own arithmetic is not
deterministic (fp32 atomics, unstable sorts, TF32 dots, bf16 tree scans), the
oracle fixes one deterministic contract and says so in the docstring.

Pinning status of each function (what independent check fixes it) is recorded
in the module docstrings of ``tests/test_oracle.py`` and ``tests/test_oracle_ear.py``.
Each public function there has at least one check that does not restate its
formula (hand-computed values, closed forms, library routines, brute force), so
none is "parity unpinned"; the scaled centroid scores of the block mask are
pinned by hand-computed bf16 values and by torch's own bf16 matmul.
"""

from .svoo_oracle import *  # noqa: F401,F403
