"""Head dims below 128.  Every kernel works on rows of 128 elements; the operators pad rows of a head dim D < 128 with
zeros (``svoo_convert_rows``) and pass D, which sets the score and softmax scale 1/sqrt(D).  Zero columns change no
dot, centroid or label, so the padded computation is the reference's computation on D columns; these tests check it
against the oracle evaluated on the D-column inputs: the clustering per half-step, the mask and centroid scores bit
for bit, the attention (plain and EAR-compensated) within the bf16 tolerance, and the Wan SAP and EAR processors'
whole calls at D = 64.  The reference's Triton kernels take D as a compile-time parameter
(``svoo/co_clustering.py:949-1108``, ``kernels/triton/permute.py:9-65``)."""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O
from parity_helpers import MAX_ABS, MIN_COS, bits, replay_clustering, say

pytestmark = pytest.mark.gpu


def f32(t):
    return t.float().cpu().numpy()


def _close(got, ref):
    o = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    err = float(np.abs(o - r).max())
    cos = float(o @ r / (np.linalg.norm(o) * np.linalg.norm(r) + 1e-30))
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)
    return err, cos


def test_row_padding_round_trip(gpu):
    from svoo_amd import _lib

    say("svoo_convert_rows: pad to 128 and back")
    g = torch.Generator().manual_seed(3)
    for d, dtype in ((64, torch.float32), (96, torch.bfloat16), (8, torch.float16), (128, torch.float32)):
        x = (torch.randn(7, 5, d, generator=g) * 3).to(dtype).to(gpu)
        p = _lib.as_rows128(x, "x")
        assert p.shape == (7, 5, 128) and p.dtype == torch.bfloat16
        assert torch.equal(p[..., :d], x.to(torch.bfloat16)) and not bool(p[..., d:].any())
        back = _lib.from_rows128(p, d, dtype)
        assert back.dtype == dtype and torch.equal(back, x.to(torch.bfloat16).to(dtype))


def _sizes(h, s, c, r):
    cuts = np.sort(r.integers(0, s + 1, size=(h, c - 1)), axis=1)
    return np.diff(np.concatenate([np.zeros((h, 1), int), cuts, np.full((h, 1), s)], axis=1), axis=1)


@pytest.mark.parametrize("d", [64, 96, 32])
def test_attention_and_mask_at_head_dim(gpu, d):
    from svoo_amd.co_clustering import (block_mask_lengths, centroid_scores, dynamic_block_sparse_fwd,
                                        dynamic_block_sparse_fwd_fused)
    from svoo_amd.ear import dynamic_block_sparse_prune_fwd

    say("attention, mask and EAR attention at D =", d)
    r = np.random.default_rng(d)
    h, s, qn, kn = 3, 1800, 10, 36
    q, k, v = (O.bf16_round(r.standard_normal((1, h, s, d)).astype(np.float32)) for _ in range(3))
    qs, ks = _sizes(h, s, qn, r)[None], _sizes(h, s, kn, r)[None]
    m = r.random((1, h, qn, kn)) < 0.4
    m[0, 0, 0] = False  # one query cluster may keep nothing (zero rows) when the row is all False
    qt, kt, vt = (torch.from_numpy(x).to(gpu) for x in (q, k, v))
    mt = torch.from_numpy(m).to(gpu)
    qst, kst = torch.from_numpy(qs).int().to(gpu), torch.from_numpy(ks).int().to(gpu)
    want = O.block_sparse_attention(q, k, v, m, qs, ks)
    out = dynamic_block_sparse_fwd(qt.bfloat16(), kt.bfloat16(), vt.bfloat16(), mt, qst, kst)
    assert out.shape == (1, h, s, d)
    say("D =", d, "attention vs float64:", _close(f32(out), want))
    # the fused form on token order equals the permuted form bit for bit
    perm = torch.stack([torch.randperm(s, generator=torch.Generator().manual_seed(9 + i)) for i in range(h)])
    perm = perm.int().to(gpu)
    fused = dynamic_block_sparse_fwd_fused(qt.bfloat16(), kt.bfloat16(), vt.bfloat16(), mt, qst, kst, perm, perm)
    qp = torch.gather(qt.bfloat16(), 2, perm.long()[None, :, :, None].expand(-1, -1, -1, d))
    kp = torch.gather(kt.bfloat16(), 2, perm.long()[None, :, :, None].expand(-1, -1, -1, d))
    vp = torch.gather(vt.bfloat16(), 2, perm.long()[None, :, :, None].expand(-1, -1, -1, d))
    op = dynamic_block_sparse_fwd(qp, kp, vp, mt, qst, kst)
    unperm = torch.empty_like(op).scatter_(2, perm.long()[None, :, :, None].expand(-1, -1, -1, d), op)
    assert torch.equal(fused, unperm.transpose(1, 2).reshape(1, s, h * d))

    # centroid scores and the mask (scale 1/sqrt(D)), bit for bit
    qc = O.bf16_round(r.standard_normal((1, h, qn, d)).astype(np.float32))
    kc = O.bf16_round(r.standard_normal((1, h, kn, d)).astype(np.float32))
    qct, kct = torch.from_numpy(qc).to(gpu).bfloat16(), torch.from_numpy(kc).to(gpu).bfloat16()
    np.testing.assert_array_equal(bits(f32(centroid_scores(qct, kct))), bits(O.centroid_scores(qc, kc)))
    for top_p, ratios in ((0.9, [0.1] * h), (0.0, [0.3] * h)):
        dm, _ = block_mask_lengths(qct, kct, qst, kst, top_p, ratios)
        np.testing.assert_array_equal(dm.cpu().numpy(), O.identify_dynamic_map(qc, kc, qs, ks, top_p, ratios, 0))

    # the EAR-compensated attention on the cluster-contiguous inputs
    vc = O.bf16_round(r.standard_normal((1, h, kn, d)).astype(np.float32))
    ear = dynamic_block_sparse_prune_fwd(qt.bfloat16(), kt.bfloat16(), vt.bfloat16(), kct,
                                         torch.from_numpy(vc).to(gpu).bfloat16(), mt, qst, kst)
    say("D =", d, "EAR attention vs float64:",
        _close(f32(ear), O.ear_compensated_attention(q, k, v, kc, vc, m, qs, ks)))


def _cfg(name, head_dim):
    from svoo_amd import synth

    return synth.SynthConfig(name, 61, 2, 3, 16, 24, head_dim, 24, 12, 32, 3, 0.1, 0.4, True, "bf16")


def test_sap_processor_at_head_dim_64(gpu):
    """The Wan SAP processor's sparse call at D = 64: every clustering half-step against the oracle on the
    64-column inputs, the mask bit for bit on the GPU's centroids, and the output against the oracle's block-sparse
    attention over the GPU's clusters."""
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    cfg = _cfg("sap-d64", 64)
    h, n, d = cfg.heads, cfg.video_tokens, cfg.head_dim
    qn, kn, iters = cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters
    q, k, v = synth.make_qkv(cfg)
    assert q.shape == (1, h, n, 64)
    qi = synth.init_indices(cfg, h, qn, n, 1)
    ki = synth.init_indices(cfg, h, kn, n, 2)
    top_p, ratios = 0.9, [0.2] * h

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
    say("SAP processor at D = 64")
    out = proc.attention_core_logic(qd, kd, vd, None)
    torch.cuda.synchronize()
    assert out.shape == (1, n, h * d)
    last = proc._last_call
    r = last["clustering"]
    assert r["qcentroids"].shape[-1] == 64
    for head in range(h):
        final = {key: r[key][head:head + 1] for key in ("qlabels", "klabels", "qcentroids", "kcentroids", "qsizes",
                                                        "ksizes")}
        replay_clustering(qd[0, head:head + 1], kd[0, head:head + 1], qn, kn, iters,
                          init_q_idx=qi[head:head + 1].to(gpu), init_k_idx=ki[head:head + 1].to(gpu), final=final)
    qc = f32(r["qcentroids"]).reshape(1, h, qn, d)
    kc = f32(r["kcentroids"]).reshape(1, h, kn, d)
    qs, ks = r["qsizes"].cpu().numpy().reshape(1, h, qn), r["ksizes"].cpu().numpy().reshape(1, h, kn)
    om = O.identify_dynamic_map(qc, kc, qs, ks, top_p, ratios, 0)
    np.testing.assert_array_equal(last["map"].cpu().numpy(), om)
    qidx, kidx = r["q_sorted_idx"].cpu().numpy(), r["k_sorted_idx"].cpu().numpy()
    qf, kf, vf = (x[0].float().numpy() for x in (q, k, v))
    op = O.block_sparse_attention(O.permute_rows(qf, qidx)[None], O.permute_rows(kf, kidx)[None],
                                  O.permute_rows(vf, kidx)[None], om, qs, ks)[0]
    want = np.transpose(O.unpermute_rows(op, qidx), (1, 0, 2)).reshape(1, n, h * d)
    say("SAP D = 64 output vs oracle attention on the GPU clustering:", _close(f32(out), want))


def test_ear_processor_at_head_dim_64(gpu):
    """The Wan EAR processor at D = 64 against the oracle's whole EAR call (labels, value centroids and logits
    exact, efficiencies within tolerance, the map exact on the GPU's scores, the output within tolerance)."""
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_EARAttn_Processor

    cfg = _cfg("ear-d64", 64)
    q, k, v = synth.make_qkv(cfg)
    h, s = cfg.heads, cfg.video_tokens
    r = np.random.default_rng(5)
    qi = r.integers(0, s, size=(h, 12))
    ki = r.integers(0, s, size=(h, 32))

    class P(WanAttn_EARAttn_Processor):
        pass

    P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
    P.num_q_centroids, P.num_k_centroids = 12, 32
    P.top_p_kmeans, P.min_kc_ratio, P.ear_gamma = 0.6, 0.1, 1.0
    P.kmeans_iter_init = P.kmeans_iter_step = 3
    P.first_times_fp, P.first_layers_fp = 1e9, 0
    P.kmeans_init_idx = (torch.from_numpy(qi).to(gpu), torch.from_numpy(ki).to(gpu))
    proc = P(layer_idx=0)
    say("EAR processor at D = 64")
    out = proc.attention_core_logic(*(x.to(gpu) for x in (q, k, v)), torch.tensor([100.0], device=gpu))
    torch.cuda.synchronize()
    last = proc._last_call
    ref, parts = O.ear_attention_call(q.float().numpy(), k.float().numpy(), v.float().numpy(), 12, 32, 3, 0.6, 0.1,
                                      1.0, init_q_idx=qi, init_k_idx=ki, return_parts=True)
    np.testing.assert_array_equal(last["clustering"]["klabels"].cpu().numpy(), parts["klabels"])
    np.testing.assert_array_equal(f32(last["v_centroids"])[0], parts["vc"])
    np.testing.assert_array_equal(f32(last["c"])[0], parts["c"])
    np.testing.assert_allclose(f32(last["eff"])[0], parts["eff"], rtol=0, atol=2e-3)
    want_map = O.ear_select(f32(last["eff"]), f32(last["c"]), parts["qsizes"][None], parts["ksizes"][None], 0.6, 0.1)
    np.testing.assert_array_equal(last["map"].cpu().numpy(), want_map)
    assert out.shape == (1, s, h * 64)
    if np.array_equal(want_map, parts["map"]):
        say("EAR D = 64 whole call vs oracle:", _close(f32(out), ref))
    else:
        qp = O.permute_rows(q.float().numpy()[0], parts["qidx"])
        kp = O.permute_rows(k.float().numpy()[0], parts["kidx"])
        vp = O.permute_rows(v.float().numpy()[0], parts["kidx"])
        op = O.ear_compensated_attention(qp[None], kp[None], vp[None], parts["kcent"][None], parts["vc"][None],
                                         want_map, parts["qsizes"][None], parts["ksizes"][None])[0]
        say("EAR D = 64 output vs oracle on the GPU map:",
            _close(f32(out), O.unpermute_rows(op, parts["qidx"]).transpose(1, 0, 2).reshape(1, s, h * 64)))
