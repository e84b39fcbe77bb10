"""Shared checks of the full-size GPU parity tests (imported by the ``test_gpu_*`` modules; not a test module).

* :func:`replay_clustering` re-runs the GPU co-clustering of one head for 1, 2, ... iterations from the same
  start and checks every half-step against the oracle evaluated on the GPU's own input centroids: labels equal
  the literal profile-space argmin except at near-ties, and the centroids equal an exact recount of the GPU's
  labels bit for bit (the first iteration sums sorted clusters, later ones move only the changed tokens, so this
  pins the incremental update against a full recount).
* :func:`check_clustering` checks the clustering outputs against each other (sizes, stable sort, offsets).
* :func:`sampled_rows_vs_float64` compares output rows with a float64 softmax over exactly the keys the map keeps.
"""

import numpy as np
import torch

from oracle import svoo_oracle as O

MAX_ABS = 2e-2  # bf16 attention tolerance (max-abs) from the north-star contract
MIN_COS = 0.999
NEAR_TIE = 1e-4  # literal-distance margin below which the GPU's label may differ from the literal argmin
MAX_TIE_FRACTION = 1e-3


def say(*a):
    print("[case]", *a, flush=True)


def bits(x):
    return O.bf16_bits(np.asarray(x, np.float32))


def _assign_agrees(gpu_labels, x, centroids, profile, what):
    want, margin = O.cocluster_assign(x, centroids, profile)
    bad = gpu_labels != want
    assert (margin[bad] < NEAR_TIE).all(), (what, "label differs from the literal argmin away from a near-tie",
                                           float(margin[bad].max()))
    assert bad.mean() <= MAX_TIE_FRACTION, (what, float(bad.mean()))
    return int(bad.sum())


def replay_clustering(q, k, num_q, num_k, iters, *, init_q_idx=None, init_k_idx=None, init_q_centroids=None,
                      init_k_centroids=None, check_labels=True, final=None):
    """Per-half-step parity of the GPU co-clustering of one head (``svoo/co_clustering.py:2402-2451``).

    ``q``, ``k``: ``[1, N, 128]`` bf16 on the device.  The start is given by token indices or centroids
    (``[1, C]`` / ``[1, C, 128]``).  Iteration ``i`` of the reference: key labels from the key centroids'
    profiles in the previous query-centroid space, key centroid update, query labels from the query centroids'
    profiles in the *new* key-centroid space, query centroid update.  ``final`` (a ``co_cluster_tokens_full``
    result of the same head and start after ``iters`` iterations) must equal the replay's last state.
    Returns the number of near-tie label differences.
    """
    from svoo_amd.co_clustering import co_cluster_tokens_full

    qn = q[0].float().cpu().numpy()[None]
    kn = k[0].float().cpu().numpy()[None]
    if init_q_centroids is not None:
        prev_q = init_q_centroids.float().cpu().numpy()
        prev_k = init_k_centroids.float().cpu().numpy()
    else:
        prev_q = np.take_along_axis(qn, init_q_idx.cpu().numpy()[:, :, None], axis=1)
        prev_k = np.take_along_axis(kn, init_k_idx.cpu().numpy()[:, :, None], axis=1)
    ties = 0
    r = None
    for it in range(1, iters + 1):
        say("clustering replay, iteration", it, "of", iters, "N =", qn.shape[1], "Qc =", num_q, "Kc =", num_k)
        r = co_cluster_tokens_full(q, k, num_q, num_k, it, init_q_idx=init_q_idx, init_k_idx=init_k_idx,
                                   init_q_centroids=init_q_centroids, init_k_centroids=init_k_centroids)
        torch.cuda.synchronize()
        kl = r["klabels"].cpu().numpy().astype(np.int64)
        ql = r["qlabels"].cpu().numpy().astype(np.int64)
        kc = r["kcentroids"].float().cpu().numpy()
        qc = r["qcentroids"].float().cpu().numpy()
        if check_labels:
            ties += _assign_agrees(kl, kn, prev_q, O.profile_centroids(prev_k, prev_q), f"key step {it}")
        okc, oks = O.centroid_update(kn, kl, prev_k)
        np.testing.assert_array_equal(bits(kc), bits(okc), err_msg=f"key centroids, iteration {it}")
        np.testing.assert_array_equal(r["ksizes"].cpu().numpy(), oks)
        if check_labels:
            ties += _assign_agrees(ql, qn, kc, O.profile_centroids(prev_q, kc), f"query step {it}")
        oqc, oqs = O.centroid_update(qn, ql, prev_q)
        np.testing.assert_array_equal(bits(qc), bits(oqc), err_msg=f"query centroids, iteration {it}")
        np.testing.assert_array_equal(r["qsizes"].cpu().numpy(), oqs)
        prev_q, prev_k = qc, kc
    if final is not None:
        for key in ("qlabels", "klabels", "qcentroids", "kcentroids", "qsizes", "ksizes"):
            assert torch.equal(final[key], r[key]), key
    return ties


def check_clustering(labels, sizes, order, offsets, nc):
    """Sizes are the label counts, the sort is a stable grouping permutation, offsets are exclusive sums."""
    bh, n = labels.shape
    lab = labels.to(torch.int64)
    assert int(lab.min()) >= 0 and int(lab.max()) < nc
    counts = torch.zeros(bh, nc, dtype=torch.int64, device=lab.device).scatter_add_(1, lab, torch.ones_like(lab))
    assert torch.equal(counts, sizes.reshape(bh, nc).to(torch.int64))
    o = order.to(torch.int64)
    ar = torch.arange(n, device=lab.device).expand(bh, n)
    assert torch.equal(torch.sort(o, dim=1).values, ar)  # a permutation of every head's tokens
    sl = torch.gather(lab, 1, o)
    assert bool((sl[:, 1:] >= sl[:, :-1]).all())  # grouped by label
    same = sl[:, 1:] == sl[:, :-1]
    assert bool((o[:, 1:] > o[:, :-1])[same].all())  # stable: token order within a cluster
    excl = torch.cumsum(counts, 1) - counts
    assert torch.equal(offsets.reshape(bh, nc).to(torch.int64), excl)


def sampled_rows_vs_float64(out_rows, q, k, v, q_cluster, k_cluster, dmap, heads, tokens_per_head, seed):
    """``out_rows(head, toks) -> [T, D]`` output rows; ``q, k, v [1, H, S, D]``; ``q_cluster(head)`` /
    ``k_cluster(head)`` the cluster index of every token ``[S]`` (int64, device); ``dmap [H, Qn, Kn]`` bool.
    Each sampled row must equal ``softmax(q K_sel^T / sqrt(d)) V_sel`` in float64, where ``K_sel`` are the keys
    whose cluster the query's cluster keeps."""
    rng = np.random.default_rng(seed)
    s, d = q.shape[2], q.shape[3]
    o_all, r_all = [], []
    for head in heads:
        toks = torch.from_numpy(rng.choice(s, size=tokens_per_head, replace=False)).to(q.device)
        qrows = q[0, head, toks].double()
        sel = dmap[head][q_cluster(head)[toks]][:, k_cluster(head)]  # [T, S] kept keys per row
        sc = (qrows @ k[0, head].double().T) / np.sqrt(d)
        sc = sc.masked_fill(~sel, float("-inf"))
        ref = torch.softmax(sc, dim=1) @ v[0, head].double()
        ref = torch.where(sel.any(1, keepdim=True), ref, torch.zeros_like(ref))  # no kept key -> 0
        o_all.append(out_rows(head, toks).double())
        r_all.append(ref)
    o = torch.cat(o_all).cpu().numpy().reshape(-1)
    ref = torch.cat(r_all).cpu().numpy().reshape(-1)
    err = float(np.abs(o - ref).max())
    cos = float(o @ ref / (np.linalg.norm(o) * np.linalg.norm(ref)))
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)
    return err, cos
