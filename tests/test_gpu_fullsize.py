"""GPU checks at the full Wan2.1-14B 720p layer shape (H=40, N=75600, d=128, bf16; 100 query / 1000 key
clusters, per-head density in [0.05, 0.3]) through size-independent properties:

* clustering outputs are consistent with each other (sizes = label counts, the sort is a stable
  permutation that groups labels, offsets = exclusive prefix sums), bit-exact;
* the block mask equals the oracle's on the same centroids and sizes, bit-exact;
* permute then inverse permute returns the input bits, and the permute is the indexed gather;
* sampled output rows equal a float64 recomputation over exactly the keys the mask selects
  (the north-star bf16 tolerance), for the separate-permute and the fused paths, which agree bitwise;
* with one cluster per head and a full mask the kernel equals torch's dense bf16 attention.

The oracle runs only on small pieces here (the mask over centroids); the rest are properties that hold
at any size.
"""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2  # bf16 attention tolerance (max-abs) from the north-star contract
MIN_COS = 0.999


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def c3(gpu):
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    cfg = synth.CONFIGS["C3"]
    say("C3 inputs", cfg.heads, cfg.tokens)
    q, k, v = synth.make_qkv_device(cfg, gpu)
    qi = synth.init_indices(cfg, cfg.heads, cfg.num_q_centroids, cfg.tokens, 1).to(gpu)
    ki = synth.init_indices(cfg, cfg.heads, cfg.num_k_centroids, cfg.tokens, 2).to(gpu)
    rho = synth.head_densities(cfg)
    res = {}
    for fused in (False, True):
        class P(WanAttn_SAPAttn_Processor):
            pass

        P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
        P.num_q_centroids, P.num_k_centroids = cfg.num_q_centroids, cfg.num_k_centroids
        P.top_p_kmeans, P.min_kc_ratio, P.max_kc_ratio = 0.0, rho, 0
        P.kmeans_iter_init = P.kmeans_iter_step = cfg.kmeans_iters
        P.first_times_fp, P.first_layers_fp = float("inf"), 0
        P.kmeans_init_idx = (qi, ki)
        P.fuse_permutes = fused
        say("C3 processor call, fused" if fused else "C3 processor call, separate permutes")
        proc = P(layer_idx=0)
        out = proc.attention_core_logic(q, k, v, None)
        torch.cuda.synchronize()
        res["fused" if fused else "separate"] = (out, proc._last_call)
    yield dict(cfg=cfg, q=q, k=k, v=v, rho=rho, **res)


def _check_clustering(labels, sizes, order, offsets, nc):
    bh, n = labels.shape
    lab = labels.to(torch.int64)
    assert int(lab.min()) >= 0 and int(lab.max()) < nc
    counts = torch.zeros(bh, nc, dtype=torch.int64, device=lab.device).scatter_add_(1, lab, torch.ones_like(lab))
    assert torch.equal(counts, sizes.reshape(bh, nc).to(torch.int64))
    assert torch.equal(sizes.reshape(bh, nc).sum(1), torch.full((bh,), n, device=lab.device, dtype=torch.int64))
    o = order.to(torch.int64)
    ar = torch.arange(n, device=lab.device).expand(bh, n)
    assert torch.equal(torch.sort(o, dim=1).values, ar)  # a permutation of every head's tokens
    sl = torch.gather(lab, 1, o)
    assert bool((sl[:, 1:] >= sl[:, :-1]).all())  # grouped by label
    same = sl[:, 1:] == sl[:, :-1]
    assert bool((o[:, 1:] > o[:, :-1])[same].all())  # stable: token order within a cluster
    excl = torch.cumsum(counts, 1) - counts
    assert torch.equal(offsets.reshape(bh, nc).to(torch.int64), excl)


def test_c3_clustering_invariants(c3):
    cfg = c3["cfg"]
    r = c3["separate"][1]["clustering"]
    say("C3 clustering invariants")
    _check_clustering(r["qlabels"], r["qsizes"], r["q_sorted_idx"], r["q_offsets"], cfg.num_q_centroids)
    _check_clustering(r["klabels"], r["ksizes"], r["k_sorted_idx"], r["k_offsets"], cfg.num_k_centroids)
    f = c3["fused"][1]["clustering"]
    for key in ("qlabels", "klabels", "q_sorted_idx", "k_sorted_idx"):
        assert torch.equal(r[key], f[key])  # the same deterministic clustering on both paths


def test_c3_block_mask_matches_oracle(c3):
    cfg = c3["cfg"]
    last = c3["separate"][1]
    r = last["clustering"]
    say("C3 block mask vs oracle")
    h, d = cfg.heads, cfg.head_dim
    qc = r["qcentroids"].float().cpu().numpy().reshape(1, h, cfg.num_q_centroids, d)
    kc = r["kcentroids"].float().cpu().numpy().reshape(1, h, cfg.num_k_centroids, d)
    qs = last["q_sizes"].cpu().numpy()
    ks = last["k_sizes"].cpu().numpy()
    om, olens = O.identify_dynamic_map(qc, kc, qs, ks, 0.0, c3["rho"], 0, return_lengths=True)
    np.testing.assert_array_equal(last["map"].cpu().numpy(), om)
    np.testing.assert_array_equal(last["lengths"].cpu().numpy(), olens)


def test_c3_permute_round_trip(c3):
    from svoo_amd.permute import apply_inverse_permutation, permute_pair_by_indices

    say("C3 permute / inverse permute round trip")
    k, v = c3["k"], c3["v"]
    order = c3["separate"][1]["clustering"]["k_sorted_idx"]
    kp, vp = permute_pair_by_indices(k, v, order)
    idx = order.to(torch.int64)[None, :, :, None].expand_as(k)
    assert torch.equal(kp, torch.gather(k, 2, idx))
    assert torch.equal(vp, torch.gather(v, 2, idx))
    assert torch.equal(apply_inverse_permutation(kp, order, dim=2), k)
    assert torch.equal(apply_inverse_permutation(vp, order, dim=2), v)


def test_c3_fused_equals_separate(c3):
    say("C3 fused vs separate output")
    assert torch.equal(c3["separate"][0], c3["fused"][0])


@pytest.mark.parametrize("path", ["separate", "fused"])
def test_c3_sampled_rows_match_float64(c3, path):
    """Rows of every fifth head, 24 tokens each, against softmax(q K_sel^T / sqrt(d)) V_sel in float64,
    where K_sel are the keys whose cluster the query's cluster keeps."""
    cfg = c3["cfg"]
    out, last = c3[path]
    r = last["clustering"]
    h, n, d = cfg.heads, cfg.tokens, cfg.head_dim
    rng = np.random.default_rng(33)
    dmap = last["map"].reshape(h, cfg.num_q_centroids, cfg.num_k_centroids)
    o_all, r_all = [], []
    for head in range(0, h, 5):
        say("C3 sampled rows", path, "head", head)
        toks = torch.from_numpy(rng.choice(n, size=24, replace=False)).to(out.device)
        qrows = c3["q"][0, head, toks].double()
        kl = r["klabels"][head].to(torch.int64)
        sel = dmap[head][r["qlabels"][head, toks].to(torch.int64)][:, kl]  # [24, N] kept keys per row
        kh, vh = c3["k"][0, head].double(), c3["v"][0, head].double()
        s = (qrows @ kh.T) / np.sqrt(d)
        s = s.masked_fill(~sel, float("-inf"))
        ref = torch.softmax(s, dim=1) @ vh
        o_all.append(out[0, toks, head * d:(head + 1) * d].double())
        r_all.append(ref)
    o = torch.cat(o_all).cpu().numpy().reshape(-1)
    ref = torch.cat(r_all).cpu().numpy().reshape(-1)
    err = np.abs(o - ref).max()
    cos = float(o @ ref / (np.linalg.norm(o) * np.linalg.norm(ref)))
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)


def test_c3_dense_mask_equals_sdpa(c3):
    """One cluster per head with its block kept: the kernel is dense attention at the full shape."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    cfg = c3["cfg"]
    h, n = cfg.heads, cfg.tokens
    say("C3 dense mask vs torch bf16 attention")
    sizes = torch.full((1, h, 1), n, dtype=torch.int32, device=c3["q"].device)
    m = torch.ones(1, h, 1, 1, dtype=torch.bool, device=c3["q"].device)
    out = dynamic_block_sparse_fwd(c3["q"], c3["k"], c3["v"], m, sizes, sizes)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        ref = torch.nn.functional.scaled_dot_product_attention(c3["q"], c3["k"], c3["v"])
    torch.cuda.synchronize()
    o, rf = out.double().reshape(-1), ref.double().reshape(-1)
    err = float((o - rf).abs().max())
    cos = float(o @ rf / (o.norm() * rf.norm()))
    # both sides are bf16 outputs of float32 accumulations: each within half a bf16 ulp of the exact value
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)
