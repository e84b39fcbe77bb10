"""GPU checks at the full BASELINE layer shapes, through properties that hold at any size and oracle pieces that
finish in seconds:

* C2 (Wan2.1-1.3B 480p: H=12, N=32760, 100/500 clusters, density in [0.05, 0.4]) and C3 (Wan2.1-14B 720p:
  H=40, N=75600, 100/1000 clusters, density in [0.05, 0.3]) through the Wan processor, fused and separate;
* C4 (HunyuanVideo 720p: H=24, 118800 video + 256 text tokens, 200/1000 clusters) through the Hunyuan
  processor, fused and separate, with the whole text as the prompt and with a padded prompt.

For each: the clustering outputs agree with each other (bit-exact); one head's clustering replays half-step by
half-step against the oracle on the GPU's own inputs (labels up to near-ties, centroids bit-exact); the block
mask equals the oracle's on the same centroids (bit-exact); the fused and separate paths give identical bits;
sampled output rows equal a float64 softmax over exactly the keys the mask keeps (bf16 tolerance).  C3 also
checks the permute round trip and the dense one-cluster map against torch's bf16 attention.

Each shape runs in two mask modes: density mode (top_p 0, the per-head profile ratio as the minimum) and the
mode the reference's Wan launchers ship (top_p 0.9, the profile ratios clipped to [0.15, 0.20];
scripts/inference/wan/wan_t2v_720p_svoo.sh:77-84 and :98-105).  The clustering does not depend on the mode, so
the clustering-only checks run in density mode.
"""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O
from parity_helpers import (MAX_ABS, MIN_COS, check_clustering, replay_clustering, sampled_rows_vs_float64,
                            say)

pytestmark = pytest.mark.gpu


TOP_P_SHIPPED = 0.9
RATIO_CLIP = (0.15, 0.20)


def mask_mode(mode, rho):
    """``(top_p, per-head minimum ratios)`` of a mask mode."""
    if mode == "density":
        return 0.0, rho
    return TOP_P_SHIPPED, [min(max(r, RATIO_CLIP[0]), RATIO_CLIP[1]) for r in rho]


def density_only(case):
    if case["mode"] != "density":
        pytest.skip("the clustering does not depend on the mask mode; checked in density mode")


def _wan_calls(cfg, gpu, q, k, v, qi, ki, top_p, ratios):
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    res = {}
    for fused in (False, True):
        class P(WanAttn_SAPAttn_Processor):
            pass

        P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
        P.num_q_centroids, P.num_k_centroids = cfg.num_q_centroids, cfg.num_k_centroids
        P.top_p_kmeans, P.min_kc_ratio, P.max_kc_ratio = top_p, ratios, 0
        P.kmeans_iter_init = P.kmeans_iter_step = cfg.kmeans_iters
        P.first_times_fp, P.first_layers_fp = float("inf"), 0
        P.kmeans_init_idx = (qi, ki)
        P.fuse_permutes = fused
        say(cfg.name, "processor call, top_p", top_p, "fused" if fused else "separate permutes")
        proc = P(layer_idx=0)
        out = proc.attention_core_logic(q, k, v, None)
        torch.cuda.synchronize()
        res["fused" if fused else "separate"] = (out, proc._last_call)
    return res


@pytest.fixture(scope="module", params=["C2", "C3", "C2-topp", "C3-topp"])
def wan(request, gpu):
    from svoo_amd import synth

    name, _, mode = request.param.partition("-")
    mode = mode or "density"
    cfg = synth.CONFIGS[name]
    say(cfg.name, "inputs", cfg.heads, cfg.tokens, "mask mode", mode)
    q, k, v = synth.make_qkv_device(cfg, gpu)
    qi = synth.init_indices(cfg, cfg.heads, cfg.num_q_centroids, cfg.tokens, 1).to(gpu)
    ki = synth.init_indices(cfg, cfg.heads, cfg.num_k_centroids, cfg.tokens, 2).to(gpu)
    rho = synth.head_densities(cfg)
    top_p, ratios = mask_mode(mode, rho)
    res = _wan_calls(cfg, gpu, q, k, v, qi, ki, top_p, ratios)
    yield dict(name=name, mode=mode, cfg=cfg, q=q, k=k, v=v, qi=qi, ki=ki, rho=rho, top_p=top_p, ratios=ratios,
               **res)
    del res, q, k, v
    torch.cuda.empty_cache()


def test_wan_clustering_invariants(wan):
    cfg = wan["cfg"]
    r = wan["separate"][1]["clustering"]
    say(wan["name"], "clustering invariants")
    check_clustering(r["qlabels"], r["qsizes"], r["q_sorted_idx"], r["q_offsets"], cfg.num_q_centroids)
    check_clustering(r["klabels"], r["ksizes"], r["k_sorted_idx"], r["k_offsets"], cfg.num_k_centroids)
    f = wan["fused"][1]["clustering"]
    for key in ("qlabels", "klabels", "q_sorted_idx", "k_sorted_idx"):
        assert torch.equal(r[key], f[key])  # the same deterministic clustering on both paths


def test_wan_clustering_replays_against_oracle(wan):
    """Head 0, every half-step of the 5 iterations: labels vs the literal argmin (near-ties excepted), key
    centroids and query centroids bit-exact against an exact recount (iterations 2-5 are the incremental
    update), and the last state equal to the processor's clustering of that head."""
    density_only(wan)
    cfg = wan["cfg"]
    r = wan["separate"][1]["clustering"]
    head0 = {key: r[key][:1] for key in ("qlabels", "klabels", "qcentroids", "kcentroids", "qsizes", "ksizes")}
    ties = replay_clustering(wan["q"][0, :1], wan["k"][0, :1], cfg.num_q_centroids, cfg.num_k_centroids,
                             cfg.kmeans_iters, init_q_idx=wan["qi"][:1], init_k_idx=wan["ki"][:1], final=head0)
    say(wan["name"], "near-tie label differences over", cfg.kmeans_iters, "iterations:", ties)


@pytest.mark.parametrize("start", ["random", "warm"])
def test_wan_key_candidate_pass_changes_nothing(wan, start, monkeypatch):
    """The key side's candidate pass (exact triangle-inequality pruning in profile space, iterations 2-5) gives
    bit-identical clustering outputs to full passes, from a random start (many label moves, long candidate lists,
    recounts) and from a warm start (the benchmark's case)."""
    density_only(wan)
    from svoo_amd import synth
    from svoo_amd.co_clustering import co_cluster_tokens_full

    cfg = wan["cfg"]
    qf, kf = wan["q"][0], wan["k"][0]
    if start == "random":
        kw = dict(init_q_idx=wan["qi"], init_k_idx=wan["ki"])
    else:
        prev = co_cluster_tokens_full(qf, kf, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters,
                                      init_q_idx=wan["qi"], init_k_idx=wan["ki"])
        kw = dict(init_q_centroids=synth.perturb_centroids(cfg, prev["qcentroids"], 3),
                  init_k_centroids=synth.perturb_centroids(cfg, prev["kcentroids"], 4))
    res = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("SVOO_KEY_CANDIDATES", flag)
        say(wan["name"], start, "clustering, key candidate pass", "on" if flag == "1" else "off")
        res[flag] = co_cluster_tokens_full(qf, kf, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters, **kw)
        torch.cuda.synchronize()
    for key in res["0"]:
        assert torch.equal(res["0"][key], res["1"][key]), key


@pytest.mark.parametrize("start", ["random", "warm"])
def test_wan_query_pruning_changes_nothing(wan, start, monkeypatch):
    """The query side's pruning of later passes (tokens whose bounds prove their label cannot change are
    skipped) gives the same clustering outputs as unpruned passes.  A pruned token keeps the exact argmax of x.E;
    an unpruned one gets the certified fp16 label or the hi + lo kernel's, which equal the exact argmax except
    where two scores lie within the hi + lo rounding, and a pruned token's bounds separate its scores by more."""
    density_only(wan)
    from svoo_amd import synth
    from svoo_amd.co_clustering import co_cluster_tokens_full

    cfg = wan["cfg"]
    qf, kf = wan["q"][0], wan["k"][0]
    if start == "random":
        kw = dict(init_q_idx=wan["qi"], init_k_idx=wan["ki"])
    else:
        prev = co_cluster_tokens_full(qf, kf, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters,
                                      init_q_idx=wan["qi"], init_k_idx=wan["ki"])
        kw = dict(init_q_centroids=synth.perturb_centroids(cfg, prev["qcentroids"], 3),
                  init_k_centroids=synth.perturb_centroids(cfg, prev["kcentroids"], 4))
    res = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("SVOO_QUERY_PRUNE", flag)
        say(wan["name"], start, "clustering, query pruning", "on" if flag == "1" else "off")
        res[flag] = co_cluster_tokens_full(qf, kf, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters, **kw)
        torch.cuda.synchronize()
    for key in res["0"]:
        assert torch.equal(res["0"][key], res["1"][key]), key


def test_wan_block_mask_matches_oracle(wan):
    cfg = wan["cfg"]
    last = wan["separate"][1]
    r = last["clustering"]
    say(wan["name"], wan["mode"], "block mask vs oracle")
    h, d = cfg.heads, cfg.head_dim
    qc = r["qcentroids"].float().cpu().numpy().reshape(1, h, cfg.num_q_centroids, d)
    kc = r["kcentroids"].float().cpu().numpy().reshape(1, h, cfg.num_k_centroids, d)
    om, olens = O.identify_dynamic_map(qc, kc, last["q_sizes"].cpu().numpy(), last["k_sizes"].cpu().numpy(),
                                       wan["top_p"], wan["ratios"], 0, return_lengths=True)
    np.testing.assert_array_equal(last["map"].cpu().numpy(), om)
    np.testing.assert_array_equal(last["lengths"].cpu().numpy(), olens)


def test_wan_fused_equals_separate(wan):
    say(wan["name"], "fused vs separate output")
    assert torch.equal(wan["separate"][0], wan["fused"][0])


@pytest.mark.parametrize("path", ["separate", "fused"])
def test_wan_sampled_rows_match_float64(wan, path):
    """Rows of every fifth head (every head at C2), 24 tokens each, against a float64 softmax over the kept keys."""
    cfg = wan["cfg"]
    out, last = wan[path]
    r = last["clustering"]
    h, d = cfg.heads, cfg.head_dim
    dmap = last["map"].reshape(h, cfg.num_q_centroids, cfg.num_k_centroids)
    say(wan["name"], "sampled rows vs float64,", path)
    sampled_rows_vs_float64(lambda hd, toks: out[0, toks, hd * d:(hd + 1) * d], wan["q"], wan["k"], wan["v"],
                            lambda hd: r["qlabels"][hd].to(torch.int64), lambda hd: r["klabels"][hd].to(torch.int64),
                            dmap, range(0, h, 5 if h > 12 else 1), 24, 33)


def test_c3_permute_round_trip(wan):
    from svoo_amd.permute import apply_inverse_permutation, permute_pair_by_indices

    if wan["name"] != "C3" or wan["mode"] != "density":
        pytest.skip("C3 density case only (the check does not depend on the mask mode)")
    say("C3 permute / inverse permute round trip")
    k, v = wan["k"], wan["v"]
    order = wan["separate"][1]["clustering"]["k_sorted_idx"]
    kp, vp = permute_pair_by_indices(k, v, order)
    idx = order.to(torch.int64)[None, :, :, None].expand_as(k)
    assert torch.equal(kp, torch.gather(k, 2, idx))
    assert torch.equal(vp, torch.gather(v, 2, idx))
    assert torch.equal(apply_inverse_permutation(kp, order, dim=2), k)
    assert torch.equal(apply_inverse_permutation(vp, order, dim=2), v)


def test_c3_dense_mask_equals_sdpa(wan):
    """One cluster per head with its block kept: the kernel is dense attention at the full shape."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    if wan["name"] != "C3" or wan["mode"] != "density":
        pytest.skip("C3 density case only (the check does not depend on the mask mode)")
    cfg = wan["cfg"]
    h, n = cfg.heads, cfg.tokens
    say("C3 dense mask vs torch bf16 attention")
    sizes = torch.full((1, h, 1), n, dtype=torch.int32, device=wan["q"].device)
    m = torch.ones(1, h, 1, 1, dtype=torch.bool, device=wan["q"].device)
    out = dynamic_block_sparse_fwd(wan["q"], wan["k"], wan["v"], m, sizes, sizes)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        ref = torch.nn.functional.scaled_dot_product_attention(wan["q"], wan["k"], wan["v"])
    torch.cuda.synchronize()
    o, rf = out.double().reshape(-1), ref.double().reshape(-1)
    err = float((o - rf).abs().max())
    cos = float(o @ rf / (o.norm() * rf.norm()))
    # both sides are bf16 outputs of float32 accumulations: each within half a bf16 ulp of the exact value
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)


# ------------------------------------------------------------------------------------------ C4 (HunyuanVideo)
@pytest.fixture(scope="module", params=["density", "topp"])
def c4(request, gpu):
    from svoo_amd import synth
    from svoo_amd.processor import Hunyuan_SAPAttn_Processor

    mode = request.param
    cfg = synth.CONFIGS["C4"]
    say(cfg.name, "inputs", cfg.heads, cfg.tokens, "mask mode", mode)
    q, k, v = synth.make_qkv_device(cfg, gpu)
    nv = cfg.video_tokens
    qi = synth.init_indices(cfg, cfg.heads, cfg.num_q_centroids, nv, 1).to(gpu)
    ki = synth.init_indices(cfg, cfg.heads, cfg.num_k_centroids, nv, 2).to(gpu)
    rho = synth.head_densities(cfg)
    top_p, ratios = mask_mode(mode, rho)
    res = {}
    for prompt in (cfg.text_tokens, 200):  # whole text as prompt (empty padding cluster); 56 padding tokens
        for fused in (False, True):
            class P(Hunyuan_SAPAttn_Processor):
                pass

            P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, cfg.text_tokens
            P.prompt_length = prompt
            P.num_q_centroids, P.num_k_centroids = cfg.num_q_centroids, cfg.num_k_centroids
            P.top_p_kmeans, P.min_kc_ratio, P.max_kc_ratio = top_p, ratios, 0
            P.kmeans_iter_init = P.kmeans_iter_step = cfg.kmeans_iters
            P.first_times_fp, P.first_layers_fp = float("inf"), 0
            P.kmeans_init_idx = (qi, ki)
            P.fuse_permutes = fused
            say(cfg.name, "processor call, prompt", prompt, "top_p", top_p,
                "fused" if fused else "separate permutes")
            proc = P(layer_idx=0)
            out = proc.attention_core_logic(q, k, v, 0.0, 0)
            torch.cuda.synchronize()
            res[(prompt, fused)] = (out.contiguous(), proc._last_call)
    yield dict(cfg=cfg, mode=mode, q=q, k=k, v=v, qi=qi, ki=ki, rho=rho, top_p=top_p, ratios=ratios, res=res)
    del res, q, k, v
    torch.cuda.empty_cache()


@pytest.mark.parametrize("prompt", [256, 200])
def test_c4_fused_equals_separate(c4, prompt):
    say("C4 fused vs separate, prompt", prompt)
    a, la = c4["res"][(prompt, False)]
    b, lb = c4["res"][(prompt, True)]
    assert torch.equal(a, b)
    assert torch.equal(la["map"], lb["map"]) and torch.equal(la["q_sizes"], lb["q_sizes"])
    assert not torch.isnan(a).any()


def test_c4_clustering_and_masks_match_oracle(c4):
    """Video clustering invariants, the video mask against the oracle and the text-extended map, sizes and
    sort orders against the oracle's post-processing (svoo/models/hunyuan10/attention.py:977-1021)."""
    cfg = c4["cfg"]
    h, d, nv, ctx = cfg.heads, cfg.head_dim, cfg.video_tokens, cfg.text_tokens
    qn, kn = cfg.num_q_centroids, cfg.num_k_centroids
    for prompt in (256, 200):
        last = c4["res"][(prompt, True)][1]
        r = last["clustering"]
        say("C4", c4["mode"], "clustering and masks vs oracle, prompt", prompt)
        check_clustering(r["qlabels"], r["qsizes"], r["q_sorted_idx"], r["q_offsets"], qn)
        check_clustering(r["klabels"], r["ksizes"], r["k_sorted_idx"], r["k_offsets"], kn)
        qs, ks = r["qsizes"].cpu().numpy().reshape(1, h, qn), r["ksizes"].cpu().numpy().reshape(1, h, kn)
        om, olens = O.identify_dynamic_map(r["qcentroids"].float().cpu().numpy().reshape(1, h, qn, d),
                                           r["kcentroids"].float().cpu().numpy().reshape(1, h, kn, d), qs, ks,
                                           c4["top_p"], c4["ratios"], 0, return_lengths=True)
        np.testing.assert_array_equal(last["video_lengths"].cpu().numpy(), olens)
        m2, qs2, ks2, qidx2 = O.hunyuan_post_process(om, qs, ks, r["q_sorted_idx"].cpu().numpy(), nv, ctx, prompt)
        _, _, _, kidx2 = O.hunyuan_post_process(om, qs, ks, r["k_sorted_idx"].cpu().numpy(), nv, ctx, prompt)
        np.testing.assert_array_equal(last["map"].cpu().numpy(), m2)
        np.testing.assert_array_equal(last["q_sizes"].cpu().numpy(), qs2)
        np.testing.assert_array_equal(last["k_sizes"].cpu().numpy(), ks2)
        np.testing.assert_array_equal(last["q_idx"].cpu().numpy(), qidx2)
        np.testing.assert_array_equal(last["k_idx"].cpu().numpy(), kidx2)


def test_c4_clustering_replays_against_oracle(c4):
    """Head 0 of the video part, every half-step of the 5 iterations, ending in the processor's clustering."""
    density_only(c4)
    cfg = c4["cfg"]
    nv = cfg.video_tokens
    r = c4["res"][(256, True)][1]["clustering"]
    head0 = {key: r[key][:1] for key in ("qlabels", "klabels", "qcentroids", "kcentroids", "qsizes", "ksizes")}
    q0, k0 = c4["q"][0, :1, :nv].contiguous(), c4["k"][0, :1, :nv].contiguous()
    ties = replay_clustering(q0, k0, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters,
                             init_q_idx=c4["qi"][:1], init_k_idx=c4["ki"][:1], final=head0)
    say("C4 near-tie label differences over", cfg.kmeans_iters, "iterations:", ties)


@pytest.mark.parametrize("prompt", [256, 200])
def test_c4_sampled_rows_match_float64(c4, prompt):
    """Video rows of every sixth head plus prompt and padding rows, against a float64 softmax over the kept keys
    of the text-extended map (prompt tokens form cluster Qc / Kc, padding tokens cluster Qc+1 / Kc+1)."""
    cfg = c4["cfg"]
    h, d, nv, s = cfg.heads, cfg.head_dim, cfg.video_tokens, cfg.tokens
    qn, kn = cfg.num_q_centroids, cfg.num_k_centroids
    out, last = c4["res"][(prompt, True)]
    r = last["clustering"]
    dmap = last["map"].reshape(h, qn + 2, kn + 2)
    dev = out.device
    text_q = torch.where(torch.arange(s - nv, device=dev) < prompt, qn, qn + 1)
    text_k = torch.where(torch.arange(s - nv, device=dev) < prompt, kn, kn + 1)
    qlab = lambda hd: torch.cat([r["qlabels"][hd].to(torch.int64), text_q])  # noqa: E731
    klab = lambda hd: torch.cat([r["klabels"][hd].to(torch.int64), text_k])  # noqa: E731
    say("C4 sampled rows vs float64, prompt", prompt)
    heads = range(0, h, 6)
    sampled_rows_vs_float64(lambda hd, toks: out[0, hd, toks], c4["q"], c4["k"], c4["v"], qlab, klab, dmap, heads,
                            24, 44 + prompt)
    # text rows: the first and last prompt rows and, with padding, padding rows
    rows = [nv, nv + prompt - 1] + ([nv + prompt, s - 1] if prompt < s - nv else [])
    toks = torch.tensor(rows, device=dev)
    for hd in heads:
        sel = dmap[hd][qlab(hd)[toks]][:, klab(hd)]
        sc = (c4["q"][0, hd, toks].double() @ c4["k"][0, hd].double().T) / np.sqrt(d)
        ref = torch.softmax(sc.masked_fill(~sel, float("-inf")), 1) @ c4["v"][0, hd].double()
        got = out[0, hd, toks].double()
        assert float((got - ref).abs().max()) <= MAX_ABS, (hd, rows)
