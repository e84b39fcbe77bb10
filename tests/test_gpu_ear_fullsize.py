"""EAR (error-aware routing with centroid compensation) at the full BASELINE layer shapes, through the Wan EAR
processor (``svoo/models/wan/attention.py:1047-1071, 1180-1222``; ``svoo/co_clustering.py:1314-2050``):

* C2 (H=12, N=32760, 100/500 clusters) in density mode and in the shipped top-p mode, every head;
* C3 (H=40, N=75600, 100/1000 clusters) in density mode, the maps of every head and the efficiency of every
  tenth head.

On the GPU's own clustering: value centroids and centroid logits bit-exact against the oracle; the oracle's
selection on the GPU's own efficiency scores and logits equals the GPU's map (bit-exact); the efficiency scores
within their tolerance of the float64 oracle; and sampled output rows within the bf16 attention tolerance of a
float64 softmax over the kept tokens plus the (Kc_j, Vc_j) pairs of the pruned clusters with the
``log(|K_j| + 1e-6)`` prior.
"""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O
from parity_helpers import MAX_ABS, MIN_COS, say

pytestmark = pytest.mark.gpu

EFF_ABS = 2e-3  # fp32 MFMA dots and fp32 sums against the fp64 restatement, in log units
GAMMA = 1.0


def _f32(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="module", params=["C2", "C2-topp", "C3"])
def ear_case(request, gpu):
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_EARAttn_Processor

    name, _, mode = request.param.partition("-")
    mode = mode or "density"
    cfg = synth.CONFIGS[name]
    say("EAR", cfg.name, "inputs", cfg.heads, cfg.tokens, "mask mode", mode)
    q, k, v = synth.make_qkv_device(cfg, gpu)
    qi = synth.init_indices(cfg, cfg.heads, cfg.num_q_centroids, cfg.tokens, 1).to(gpu)
    ki = synth.init_indices(cfg, cfg.heads, cfg.num_k_centroids, cfg.tokens, 2).to(gpu)
    rho = synth.head_densities(cfg)
    if mode == "density":
        top_p, ratios = 0.0, rho
    else:
        top_p, ratios = 0.9, [min(max(r, 0.15), 0.20) for r in rho]

    class P(WanAttn_EARAttn_Processor):
        pass

    P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
    P.num_q_centroids, P.num_k_centroids = cfg.num_q_centroids, cfg.num_k_centroids
    P.top_p_kmeans, P.min_kc_ratio, P.ear_gamma = top_p, ratios, GAMMA
    P.kmeans_iter_init = P.kmeans_iter_step = cfg.kmeans_iters
    P.first_times_fp, P.first_layers_fp = float("inf"), 0
    P.kmeans_init_idx = (qi, ki)
    say("EAR", cfg.name, "processor call, top_p", top_p)
    proc = P(layer_idx=0)
    out = proc.attention_core_logic(q, k, v, None)
    torch.cuda.synchronize()
    last = proc._last_call
    r = last["clustering"]
    h, d = cfg.heads, cfg.head_dim
    kidx = r["k_sorted_idx"].to(torch.int64)[:, :, None].expand(h, cfg.tokens, d)
    kp = torch.gather(k[0], 1, kidx)
    vp = torch.gather(v[0], 1, kidx)
    yield dict(name=name, mode=mode, cfg=cfg, q=q, k=k, v=v, out=out, last=last, kp=kp, vp=vp, top_p=top_p,
               ratios=ratios)
    del out, last, q, k, v, kp, vp
    torch.cuda.empty_cache()


def test_ear_value_centroids_and_logits_bit_exact(ear_case):
    cfg, last = ear_case["cfg"], ear_case["last"]
    r = last["clustering"]
    h, d, qn, kn = cfg.heads, cfg.head_dim, cfg.num_q_centroids, cfg.num_k_centroids
    say("EAR", ear_case["name"], ear_case["mode"], "value centroids and centroid logits vs oracle")
    ks = last["k_sizes"].cpu().numpy().reshape(h, kn)
    want_vc = O.value_centroids(_f32(ear_case["vp"]), ks)
    np.testing.assert_array_equal(_f32(last["v_centroids"]).reshape(h, kn, d), want_vc)
    qc = _f32(r["qcentroids"]).reshape(1, h, qn, d)
    kc = _f32(r["kcentroids"]).reshape(1, h, kn, d)
    np.testing.assert_array_equal(_f32(last["c"]).reshape(1, h, qn, kn), O.ear_centroid_logits(qc, kc))


def test_ear_selection_on_gpu_scores_equals_gpu_map(ear_case):
    cfg, last = ear_case["cfg"], ear_case["last"]
    h, qn, kn = cfg.heads, cfg.num_q_centroids, cfg.num_k_centroids
    say("EAR", ear_case["name"], ear_case["mode"], "selection vs oracle on the GPU's efficiency and logits")
    want = O.ear_select(_f32(last["eff"]).reshape(1, h, qn, kn), _f32(last["c"]).reshape(1, h, qn, kn),
                        last["q_sizes"].cpu().numpy().reshape(1, h, qn), last["k_sizes"].cpu().numpy().reshape(1, h, kn),
                        ear_case["top_p"], ear_case["ratios"])
    got = last["map"].cpu().numpy().reshape(1, h, qn, kn)
    np.testing.assert_array_equal(got, want)
    say("EAR", ear_case["name"], "kept block fraction", float(got.mean()))


def test_ear_efficiency_matches_float64(ear_case):
    cfg, last = ear_case["cfg"], ear_case["last"]
    r = last["clustering"]
    h, d, qn, kn = cfg.heads, cfg.head_dim, cfg.num_q_centroids, cfg.num_k_centroids
    heads = list(range(0, h, 10 if h > 12 else 1))
    say("EAR", ear_case["name"], ear_case["mode"], "efficiency vs float64 oracle, heads", heads)
    qc = _f32(r["qcentroids"]).reshape(h, qn, d)[heads]
    c = _f32(last["c"]).reshape(h, qn, kn)[heads]
    vc = _f32(last["v_centroids"]).reshape(h, kn, d)[heads]
    qs = last["q_sizes"].cpu().numpy().reshape(h, qn)[heads]
    ks = last["k_sizes"].cpu().numpy().reshape(h, kn)[heads]
    hsel = torch.tensor(heads, device=ear_case["kp"].device)
    kp = _f32(ear_case["kp"].index_select(0, hsel))
    vp = _f32(ear_case["vp"].index_select(0, hsel))
    want = O.ear_efficiency_scores(qc, c, kp, vp, vc, qs, ks, GAMMA)
    got = _f32(last["eff"]).reshape(h, qn, kn)[heads]
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=0, atol=EFF_ABS)


def test_ear_sampled_rows_match_float64(ear_case):
    """24 tokens of every head (every fifth head at C3) against a float64 softmax over the tokens of the kept key
    clusters and the centroid pairs of the pruned ones, on the GPU's map and value centroids
    (``co_clustering.py:1801-2050``)."""
    cfg, last = ear_case["cfg"], ear_case["last"]
    r = last["clustering"]
    h, d, qn, kn, s = cfg.heads, cfg.head_dim, cfg.num_q_centroids, cfg.num_k_centroids, cfg.tokens
    q, k, v, out = ear_case["q"], ear_case["k"], ear_case["v"], ear_case["out"]
    dmap = last["map"].reshape(h, qn, kn)
    kcent = r["kcentroids"].reshape(h, kn, d).double()
    vcent = last["v_centroids"].reshape(h, kn, d).double()
    ksz = last["k_sizes"].reshape(h, kn)
    rng = np.random.default_rng(71)
    say("EAR", ear_case["name"], ear_case["mode"], "sampled rows vs float64 compensated attention")
    o_all, r_all = [], []
    for hd in range(0, h, 5 if h > 12 else 1):
        toks = torch.from_numpy(rng.choice(s, size=24, replace=False)).to(q.device)
        qrows = q[0, hd, toks].double()
        qcl = r["qlabels"][hd].to(torch.int64)[toks]
        kcl = r["klabels"][hd].to(torch.int64)
        keep = dmap[hd][qcl]  # [T, Kc]
        sel = keep[:, kcl]  # [T, S] tokens of kept clusters
        sc = (qrows @ k[0, hd].double().T) / np.sqrt(d)
        sc = sc.masked_fill(~sel, float("-inf"))
        prior = torch.log(ksz[hd].float() + 1e-6).double()
        cs = (qrows @ kcent[hd].T) / np.sqrt(d) + prior[None, :]
        cs = cs.masked_fill(keep, float("-inf"))  # centroids stand in for the pruned clusters only
        p = torch.softmax(torch.cat([sc, cs], 1), dim=1)
        ref = p[:, :s] @ v[0, hd].double() + p[:, s:] @ vcent[hd]
        o_all.append(out[0, toks, hd * d:(hd + 1) * d].double())
        r_all.append(ref)
    o = torch.cat(o_all).cpu().numpy().reshape(-1)
    ref = torch.cat(r_all).cpu().numpy().reshape(-1)
    err = float(np.abs(o - ref).max())
    cos = float(o @ ref / (np.linalg.norm(o) * np.linalg.norm(ref)))
    say("EAR", ear_case["name"], "max|err|", err, "cos", cos)
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)
