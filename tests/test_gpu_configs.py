"""GPU parity at the BASELINE workloads not covered by the full-size layer tests: C1 (the reference's CPU-sized
call, H=2, N=4680, 32/64 clusters, density 0.25) end to end against the oracle, C5 (one random-init
Wan2.1-1.3B DiT with SVOO in all 30 blocks, three steps with carried centroids), and the incremental centroid
update against a full recount on an input whose magnitudes span 40 binades.

C1 is specified in fp32; the MI355X path computes in bf16, so here the inputs are rounded to bf16 and the oracle runs
on the rounded values (its attention in float64).  The fp32 call itself equals this call bit for bit
(``test_gpu_dtypes.py::test_c1_processor_call_in_fp32``)."""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O
from parity_helpers import MAX_ABS, MIN_COS, bits, replay_clustering, sampled_rows_vs_float64, say

pytestmark = pytest.mark.gpu


def _close(got, ref):
    o = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    err = float(np.abs(o - r).max())
    cos = float(o @ r / (np.linalg.norm(o) * np.linalg.norm(r) + 1e-30))
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)
    return err, cos


@pytest.mark.parametrize("mode", ["density", "reference"])
def test_c1_processor_call_matches_oracle(gpu, mode):
    """The Wan processor's sparse call at C1 through the C ABI.  Per head, every half-step of the 5 iterations
    replays against the oracle (labels up to near-ties, centroids bit-exact); the block map equals the oracle's on
    the GPU's centroids; the output equals the oracle's block-sparse attention over the GPU's clusters; and where
    the labels follow the oracle's own trajectory, the whole call equals ``svoo_attention_call``."""
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    cfg = synth.CONFIGS["C1"]
    h, n, d = cfg.heads, cfg.tokens, cfg.head_dim
    qn, kn, iters = cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters
    top_p, ratios = (0.0, [0.25] * h) if mode == "density" else (0.9, [0.25] * h)
    say("C1", mode, "inputs (fp32 spec, rounded to bf16)")
    q, k, v = (x.to(torch.bfloat16) for x in synth.make_qkv(cfg))
    qi = synth.init_indices(cfg, h, qn, n, 1)
    ki = synth.init_indices(cfg, h, kn, n, 2)

    class P(WanAttn_SAPAttn_Processor):
        pass

    P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
    P.num_q_centroids, P.num_k_centroids = qn, kn
    P.top_p_kmeans, P.min_kc_ratio, P.max_kc_ratio = top_p, ratios, 0
    P.kmeans_iter_init = P.kmeans_iter_step = iters
    P.first_times_fp, P.first_layers_fp = float("inf"), 0
    P.kmeans_init_idx = (qi.to(gpu), ki.to(gpu))
    proc = P(layer_idx=0)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    say("C1", mode, "processor call")
    out = proc.attention_core_logic(qd, kd, vd, None)
    torch.cuda.synchronize()
    last = proc._last_call
    r = last["clustering"]

    for head in range(h):
        final = {key: r[key][head:head + 1] for key in ("qlabels", "klabels", "qcentroids", "kcentroids", "qsizes",
                                                        "ksizes")}
        replay_clustering(qd[0, head:head + 1], kd[0, head:head + 1], qn, kn, iters,
                          init_q_idx=qi[head:head + 1].to(gpu), init_k_idx=ki[head:head + 1].to(gpu), final=final)

    # the mask and the attention on the GPU's own clustering
    qc = r["qcentroids"].float().cpu().numpy().reshape(1, h, qn, d)
    kc = r["kcentroids"].float().cpu().numpy().reshape(1, h, kn, d)
    qs, ks = r["qsizes"].cpu().numpy().reshape(1, h, qn), r["ksizes"].cpu().numpy().reshape(1, h, kn)
    om = O.identify_dynamic_map(qc, kc, qs, ks, top_p, ratios, 0)
    np.testing.assert_array_equal(last["map"].cpu().numpy(), om)
    qidx, kidx = r["q_sorted_idx"].cpu().numpy(), r["k_sorted_idx"].cpu().numpy()
    qf, kf, vf = (x[0].float().numpy() for x in (q, k, v))
    op = O.block_sparse_attention(O.permute_rows(qf, qidx)[None], O.permute_rows(kf, kidx)[None],
                                  O.permute_rows(vf, kidx)[None], om, qs, ks)[0]
    want = np.transpose(O.unpermute_rows(op, qidx), (1, 0, 2)).reshape(1, n, h * d)
    got = out.float().cpu().numpy()
    say("C1", mode, "output vs oracle attention on the GPU clustering:", _close(got, want))

    # the oracle's whole call from the same start
    ref, parts = O.svoo_attention_call(qf[None], kf[None], vf[None], qn, kn, iters, top_p, ratios,
                                       init_q_idx=qi.numpy(), init_k_idx=ki.numpy(), return_parts=True)
    same_q = (parts["qlabels"] == r["qlabels"].cpu().numpy()).mean()
    same_k = (parts["klabels"] == r["klabels"].cpu().numpy()).mean()
    say("C1", mode, "labels equal to the oracle trajectory: q", same_q, "k", same_k)
    assert same_q >= 0.999 and same_k >= 0.999
    if same_q == 1.0 and same_k == 1.0:
        np.testing.assert_array_equal(bits(qc), bits(parts["qcentroids"].reshape(qc.shape)))
        np.testing.assert_array_equal(last["map"].cpu().numpy(), parts["map"])
        say("C1", mode, "whole call vs svoo_attention_call:", _close(got, ref))


def test_delta_centroids_equal_recount_on_wide_range_input(gpu):
    """Iterations 2+ move only the tokens whose label changed between persistent float64 sums.  That equals a
    recount bit for bit while every cluster's member values span fewer than 53 - 8 - log2(N) binades (the sums
    are then exact).  Here token magnitudes span 2^-40 .. 2^0 (N = 32768: beyond the 29-binade bound), so the
    float64 sums can round; the rounding (below 2^-40 of a sum) still leaves every bf16 centroid equal to the
    recount's.  Labels of tokens near 2^-40 are near-ties of the literal distance and are not compared."""
    r = np.random.default_rng(404)
    n = 32768
    scale = np.exp2(r.uniform(-40.0, 0.0, size=(n, 1)))
    q = torch.from_numpy((r.standard_normal((n, 128)) * scale).astype(np.float32)).to(torch.bfloat16)[None]
    k = torch.from_numpy((r.standard_normal((n, 128)) * scale + 0.5 * scale).astype(np.float32)).to(torch.bfloat16)
    k = k[None]
    qi = torch.from_numpy(r.integers(0, n, size=(1, 64))).to(gpu)
    ki = torch.from_numpy(r.integers(0, n, size=(1, 256))).to(gpu)
    say("wide-range input: delta centroid update vs recount, 4 iterations")
    replay_clustering(q.to(gpu), k.to(gpu), 64, 256, 4, init_q_idx=qi, init_k_idx=ki, check_labels=False)


def test_c5_full_dit_three_steps(gpu, tmp_path):
    """C5: a random-init Wan2.1-1.3B DiT (30 blocks, dim 1536, 12 heads, FFN 8960, 480x832x81 -> N = 32760) with
    the SVOO processor in every block (the 1.3B launcher's 256 / 1024 clusters, 2 iterations per clustering),
    the per-(step, layer, head) profile rho ~ U[0.05, 0.4] read from a CSV, density mode, centroids carried from
    step to step.  Every step, every layer: each query cluster keeps exactly max(1, floor(rho * Kc)) key
    clusters and the output is finite; layer 7 at step 3 (warm-started twice) matches a float64 recomputation on
    sampled rows of every third head."""
    from svoo_amd import dit
    from svoo_amd.inference import replace_wan_attention
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    cfg = dit.WanDiTConfig()
    layers, heads, qn, kn = cfg.num_layers, cfg.num_attention_heads, 256, 1024
    say("C5 DiT build (30 blocks)")
    pipe = dit.make_pipe(cfg, device=gpu, dtype=torch.bfloat16, seed=5)
    g = torch.Generator(device=gpu).manual_seed(5)
    lat = torch.randn(dit.latent_shape(cfg, 480, 832, 81), generator=g, device=gpu).to(torch.bfloat16)
    txt = torch.randn(1, 512, cfg.text_dim, generator=g, device=gpu).to(torch.bfloat16)
    rho = np.random.default_rng(5).uniform(0.05, 0.4, size=(3, layers, heads))
    csv = tmp_path / "profile.csv"
    with open(csv, "w") as f:
        f.write("Step,Layer,Head,Sparsity\n")
        for st in range(3):
            for ly in range(layers):
                for hd in range(heads):
                    f.write(f"{st + 1},{ly},{hd},{rho[st, ly, hd]:.4f}\n")
    cls = type("P", (WanAttn_SAPAttn_Processor,), {"kmeans_warm_start": True})
    procs = replace_wan_attention(pipe, 480, 832, 81, first_layers_fp=0, first_times_fp=1000.0, num_q_centroids=qn,
                                  num_k_centroids=kn, top_p_kmeans=0.0, min_kc_ratio=0.1, kmeans_iter_init=2,
                                  kmeans_iter_step=2, start_reuse_step=None, use_dynamic_min_kc_ratio=True,
                                  sparsity_csv_path=str(csv), processor_cls=cls)
    assert len(procs) == layers and cls.num_frame * cls.frame_size == 32760
    probe = procs[7]
    seen = {}
    core = probe.attention_core_logic

    def capture(query, key, value, timestep):
        seen["qkv"] = (query, key, value)
        seen["out"] = core(query, key, value, timestep)
        return seen["out"]

    probe.attention_core_logic = capture
    clusterings = {p.layer_idx: [] for p in procs}
    with torch.no_grad():
        for step, tval in enumerate((999.0, 979.0, 959.0), start=1):
            say("C5 DiT step", step)
            out = pipe.transformer(lat, torch.tensor([tval], device=gpu), txt)
            torch.cuda.synchronize()
            assert torch.isfinite(out.float()).all()
            for p in procs:
                assert p.current_inference_step == step
                lc = p._last_call
                preserve, _ = O.mask_row_params(heads, kn, [float(f"{rho[step - 1, p.layer_idx, hd]:.4f}")
                                                            for hd in range(heads)])
                rows = lc["lengths"][0].cpu().numpy()
                assert (rows == np.maximum(1, preserve)[:, None]).all(), (step, p.layer_idx)
                assert torch.equal(lc["map"][0].sum(-1, dtype=torch.int32), lc["lengths"][0])
                clusterings[p.layer_idx].append(lc["clustering"])
    for cl in clusterings.values():  # no reuse configured: every step re-clusters (warm-started)
        assert cl[0] is not cl[1] and cl[1] is not cl[2] and cl[0] is not cl[2]
    q, k, v = seen["qkv"]
    r = probe._last_call["clustering"]
    dmap = probe._last_call["map"].reshape(heads, qn, kn)
    o = seen["out"]
    d = cfg.attention_head_dim
    say("C5 layer 7, step 3: sampled rows vs float64")
    sampled_rows_vs_float64(lambda hd, toks: o[0, toks, hd * d:(hd + 1) * d], q, k, v,
                            lambda hd: r["qlabels"][hd].to(torch.int64), lambda hd: r["klabels"][hd].to(torch.int64),
                            dmap, range(0, heads, 3), 24, 55)
