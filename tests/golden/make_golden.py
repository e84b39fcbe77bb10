"""Write the committed fixtures under tests/golden/ (run here, never on the GPU box).

* ``sparsity_wan_1.3B_t2v_steps1-3.csv``: the first three denoising steps of the reference's shipped
  Wan2.1-1.3B profile (``sparsity_profiles/sparsity_wan_1.3B_t2v.csv``, Apache-2.0 data), as a
  parsing fixture for the ``Step,Layer,Head,Sparsity`` format.
* ``golden_small.npz``: one small seeded SVOO attention call (inputs regenerated from the seed by
  ``svoo_amd.synth``; expected outputs from the oracle): labels, centroids, sizes, sorted indices,
  block maps for several mask settings and the attention output.

    python tests/golden/make_golden.py [--reference /root/reference]
"""

from __future__ import annotations

import argparse
import csv
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import svoo_oracle as O  # noqa: E402
from svoo_amd import synth  # noqa: E402

SMALL = synth.SynthConfig("golden-small", 37, 2, 2, 12, 16, 128, 24, 12, 40, 3, 0.1, 0.4, True, "bf16")
MASK_CASES = [
    # (top_p, min_kc_ratio, max_kc_ratio)
    (0.9, [0.15, 0.3], 0),
    (0.0, [0.1, 0.25], 0),
    (0.5, 0.2, 0),
    (0.88, [0.2, 0.2], [0.3, 0.05]),
    (0.95, 0, 0.1),
    (1.0, 0, 0),
]


def small_inputs():
    q, k, v = synth.make_qkv(SMALL)
    import torch

    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    qb, kb, vb = bits(q[0]), bits(k[0]), bits(v[0])
    h, n = SMALL.heads, SMALL.tokens
    qi = synth.init_indices(SMALL, h, SMALL.num_q_centroids, n, 1).numpy()
    ki = synth.init_indices(SMALL, h, SMALL.num_k_centroids, n, 2).numpy()
    return qb, kb, vb, qi, ki


def write_csv(reference: Path):
    src = reference / "sparsity_profiles" / "sparsity_wan_1.3B_t2v.csv"
    dst = HERE / "sparsity_wan_1.3B_t2v_steps1-3.csv"
    with open(src, newline="") as f, open(dst, "w", newline="") as g:
        r = csv.reader(f)
        w = csv.writer(g, lineterminator="\n")
        w.writerow(next(r))
        for row in r:
            if int(row[0]) <= 3:
                w.writerow(row)
    print("wrote", dst)


def write_small():
    qb, kb, vb, qi, ki = small_inputs()
    q, k, v = (O.bf16_from_bits(x) for x in (qb, kb, vb))
    h, n, d = q.shape
    out = dict(q_init=qi, k_init=ki)
    ql, qc, qs, kl, kc, ks = O.co_cluster_tokens(q, k, SMALL.num_q_centroids, SMALL.num_k_centroids,
                                                 SMALL.kmeans_iters, init_q_idx=qi, init_k_idx=ki)
    out.update(qlabels=ql.astype(np.int32), klabels=kl.astype(np.int32), qsizes=qs, ksizes=ks,
               qcent=O.bf16_bits(qc), kcent=O.bf16_bits(kc))
    qidx, _, _ = O.cluster_sort(ql, SMALL.num_q_centroids)
    kidx, _, _ = O.cluster_sort(kl, SMALL.num_k_centroids)
    out.update(q_sorted_idx=qidx, k_sorted_idx=kidx)
    for ci, (p, mn, mx) in enumerate(MASK_CASES):
        m, lens = O.identify_dynamic_map(qc[None], kc[None], qs[None], ks[None], p, mn, mx, return_lengths=True)
        out[f"map{ci}"] = m[0]
        out[f"len{ci}"] = lens[0].astype(np.int32)
    m = out["map0"][None]
    qp, kp, vp = O.permute_rows(q, qidx), O.permute_rows(k, kidx), O.permute_rows(v, kidx)
    o = O.block_sparse_attention(qp[None], kp[None], vp[None], m, qs[None], ks[None])[0]
    out["out_perm"] = o.astype(np.float16)
    np.savez_compressed(HERE / "golden_small.npz", **out)
    print("wrote", HERE / "golden_small.npz")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    if Path(args.reference).exists():
        write_csv(Path(args.reference))
    write_small()
