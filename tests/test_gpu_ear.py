"""GPU parity of the EAR path (error-aware routing with centroid compensation) against the oracle:
value centroids, centroid logits and the selection bit-exact; the fp32 efficiency scores within a
log-domain tolerance; the compensated attention within the bf16 attention tolerance; and the
processor end to end.  Each test prints its case before launching."""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O

pytestmark = pytest.mark.gpu

ATTN_MAX_ABS = 2e-2  # bf16 attention tolerance (max-abs) from the north-star contract
ATTN_MIN_COS = 0.999
EFF_ABS = 2e-3  # fp32 MFMA dots and fp32 sums against the fp64 restatement, in log units


def say(*a):
    print("[case]", *a, flush=True)


def bf16(x_np, dev):
    return torch.from_numpy(np.ascontiguousarray(x_np, dtype=np.float32)).to(torch.bfloat16).to(dev)


def f32(t):
    return t.detach().float().cpu().numpy()


def rand_bf16(shape, seed, dev, scale=1.0):
    r = np.random.default_rng(seed)
    x = O.bf16_round((r.standard_normal(shape) * scale).astype(np.float32))
    return x, bf16(x, dev)


def rand_sizes(r, bh, c, s):
    cuts = np.sort(r.integers(0, s + 1, size=(bh, c - 1)), axis=1)
    z = np.concatenate([np.zeros((bh, 1), int), cuts, np.full((bh, 1), s)], axis=1)
    return np.diff(z, axis=1).astype(np.int32)


def _attn_check(out, ref):
    o = f32(out).astype(np.float64).reshape(-1)
    rr = np.asarray(ref, np.float64).reshape(-1)
    err = np.abs(o - rr).max()
    cos = float(o @ rr / (np.linalg.norm(o) * np.linalg.norm(rr) + 1e-30))
    assert err <= ATTN_MAX_ABS and cos >= ATTN_MIN_COS, (err, cos)
    return err, cos


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)


# ------------------------------------------------------------------------------------------ value side
@pytest.mark.parametrize("bh,s,kn,seed", [(3, 700, 20, 1), (2, 1500, 3, 2), (1, 97, 64, 3)])
def test_value_stats_match_oracle(gpu, bh, s, kn, seed):
    from svoo_amd import ear

    say("ear value stats", bh, s, kn)
    r = np.random.default_rng(seed)
    ks = rand_sizes(r, bh, kn, s)
    if kn == 3:
        ks[0] = [0, 301, s - 301]  # a count above 256 rounds in bf16; an empty cluster
    vp, vpt = rand_bf16((bh, s, 128), seed, gpu)
    kst = _i32(ks, gpu)
    vc, vc_sq, stats = ear._value_stats(vpt, kst, ear._offsets(kst), None)
    want = O.value_centroids(vp, ks)
    np.testing.assert_array_equal(f32(vc), want)
    vn, cvd, vcsq = O.value_stats(vp, want, ks)
    np.testing.assert_allclose(f32(vc_sq), vcsq, rtol=1e-5, atol=1e-6)
    # the kernel keeps u = v - vc: |u|^2 = |v|^2 - 2 vc.v + |vc|^2 and u.vc = vc.v - |vc|^2
    labels = np.stack([np.repeat(np.arange(kn), ks[b]) for b in range(bh)])
    vcsq_t = np.take_along_axis(vcsq, labels, axis=1)
    st = f32(stats)
    np.testing.assert_allclose(st[..., 0], vn - 2 * cvd + vcsq_t, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(st[..., 1], cvd - vcsq_t, rtol=1e-4, atol=1e-4)
    # given centroids: the statistics only
    _, vc_sq2, stats2 = ear._value_stats(vpt, kst, ear._offsets(kst), vc)
    assert torch.equal(vc_sq2, vc_sq) and torch.equal(stats2, stats)
    # from unpermuted tokens and labels (the processor helper's signature)
    perm = r.permutation(s)
    tok = np.empty_like(vp)
    tok[:, perm] = vp
    lab = np.empty_like(labels)
    lab[:, perm] = labels
    got = ear.compute_value_centroids(bf16(tok, gpu), _i32(lab, gpu), kst, kn)
    np.testing.assert_array_equal(f32(got), want)


@pytest.mark.parametrize("qn,kn", [(37, 300), (100, 1000), (1, 7)])
def test_centroid_logits_bit_exact(gpu, qn, kn):
    from svoo_amd.ear import centroid_logits

    say("ear centroid logits", qn, kn)
    qc, qct = rand_bf16((1, 2, qn, 128), 5, gpu, 0.3)
    kc, kct = rand_bf16((1, 2, kn, 128), 6, gpu, 0.3)
    np.testing.assert_array_equal(f32(centroid_logits(qct, kct)), O.ear_centroid_logits(qc, kc))


# ------------------------------------------------------------------------------------------ efficiency
@pytest.mark.parametrize("h,s,qn,kn,gamma,qscale,seed", [
    (2, 3000, 37, 40, 1.0, 0.4, 1),     # several token tiles per cluster
    (1, 2000, 70, 203, 0.5, 0.4, 2),    # three query tiles; clusters of 0..~30 tokens
    (2, 1200, 256, 24, 1.0, 0.4, 3),    # eight query tiles (two per wave)
    (1, 900, 20, 9, 0.0, 40.0, 4),      # logits far above 44: the shifted evaluation stays finite
])
def test_efficiency_matches_oracle(gpu, h, s, qn, kn, gamma, qscale, seed):
    from svoo_amd import ear

    say("ear efficiency", h, s, qn, kn, gamma, qscale)
    r = np.random.default_rng(seed)
    ks = rand_sizes(r, h, kn, s)
    qs = rand_sizes(r, h, qn, s)
    ks[0, min(2, kn - 1)] += ks[0, 0]
    ks[0, 0] = 0  # an empty key cluster
    qc, qct = rand_bf16((1, h, qn, 128), seed + 10, gpu, qscale)
    kc, kct = rand_bf16((1, h, kn, 128), seed + 11, gpu, 0.4)
    kp, kpt = rand_bf16((1, h, s, 128), seed + 12, gpu, 1.0)
    vp, vpt = rand_bf16((1, h, s, 128), seed + 13, gpu, 1.0)
    kst, qst = _i32(ks[None], gpu), _i32(qs[None], gpu)
    c = ear.centroid_logits(qct, kct)
    vc = ear.value_centroids_from_permuted(vpt, kst)
    eff = ear.error_estimation_triton(qct, kct, vc, kpt, vpt, qst, kst, c, gamma, 1e-8)
    torch.cuda.synchronize()
    want = np.stack([O.ear_efficiency_scores(qc[0], f32(c)[0], kp[0], vp[0], f32(vc)[0], qs, ks, gamma)], 0)
    got = f32(eff)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=0, atol=EFF_ABS)


def test_efficiency_of_one_member_clusters(gpu):
    """A one-member cluster's key centroid is its member and its value centroid its value, so the error is
    ``(pc expm1(a - c))^2 |vc|^2`` with ``a - c`` the bf16 rounding of the logit: the score must carry the exact
    ``a``, not an fp32 dot's (which moves the log error by percents)."""
    from svoo_amd import ear

    say("ear efficiency, one-member clusters")
    r = np.random.default_rng(21)
    h, qn, kn = 2, 64, 200
    ks = np.ones((h, kn), np.int32)
    ks[:, ::7] = r.integers(2, 40, size=ks[:, ::7].shape)  # a few larger clusters among the singletons
    s = int(ks.sum(1).max())
    ks[:, -1] += s - ks.sum(1)
    qs = rand_sizes(r, h, qn, s)
    kp, kpt = rand_bf16((1, h, s, 128), 22, gpu, 1.0)
    vp, vpt = rand_bf16((1, h, s, 128), 23, gpu, 1.0)
    qc, qct = rand_bf16((1, h, qn, 128), 24, gpu, 1.0)
    kst, qst = _i32(ks[None], gpu), _i32(qs[None], gpu)
    vc = ear.value_centroids_from_permuted(vpt, kst)
    # key centroids as the clustering leaves them: the member mean, which is the member itself for one member
    kc = np.zeros((1, h, kn, 128), np.float32)
    for b in range(h):
        off = np.concatenate([[0], np.cumsum(ks[b])])
        for j in range(kn):
            kc[0, b, j] = O.bf16_round(kp[0, b, off[j]:off[j + 1]].mean(0).astype(np.float32))
    kct = bf16(kc, gpu)
    c = ear.centroid_logits(qct, kct)
    eff = ear.error_estimation_triton(qct, kct, vc, kpt, vpt, qst, kst, c, 1.0, 1e-8)
    torch.cuda.synchronize()
    want = O.ear_efficiency_scores(qc[0], f32(c)[0], kp[0], vp[0], f32(vc)[0], qs, ks, 1.0)[None]
    np.testing.assert_allclose(f32(eff), want, rtol=0, atol=EFF_ABS)


# ------------------------------------------------------------------------------------------ selection
@pytest.mark.parametrize("kn", [7, 256, 300, 1000, 2100])
@pytest.mark.parametrize("top_p,ratio", [(0.9, 0.0), (0.5, 0.1), (1.0, [0.05, 0.3]), (0.7, [0.2])])
def test_select_bit_exact(gpu, kn, top_p, ratio):
    from svoo_amd import ear

    say("ear select", kn, top_p, ratio)
    r = np.random.default_rng(kn + int(top_p * 10))
    b, h, qn = 1, 2, 9
    c = O.bf16_round((r.standard_normal((b, h, qn, kn)) * 2).astype(np.float32))
    eff = (np.round(r.standard_normal((b, h, qn, kn)) * 4) / 2).astype(np.float32)  # many ties
    qs = r.integers(0, 50, (b, h, qn)).astype(np.int32)
    qs[0, 0, 0] = 0
    ks = r.integers(0, 80, (b, h, kn)).astype(np.int32)
    ks[..., : max(1, kn // 10)] = 0
    got = ear._select(bf16(c, gpu), torch.from_numpy(eff).to(gpu), _i32(qs.reshape(b * h, qn), gpu),
                      _i32(ks.reshape(b * h, kn), gpu), b, h, qn, kn, top_p, ratio)
    want = O.ear_select(eff, c, qs, ks, top_p, ratio)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


# ------------------------------------------------------------------------------------------ attention
@pytest.mark.parametrize("h,qn,kn,s,density,seed", [
    (2, 12, 40, 3000, 0.3, 1), (1, 5, 9, 700, 0.6, 2), (3, 30, 200, 4096, 0.1, 3), (2, 4, 100, 333, 0.05, 4),
])
def test_compensated_attention_matches_oracle(gpu, h, qn, kn, s, density, seed):
    from svoo_amd.ear import dynamic_block_sparse_prune_fwd

    say("ear attention", h, qn, kn, s, density)
    r = np.random.default_rng(seed)
    qs, ks = rand_sizes(r, h, qn, s)[None], rand_sizes(r, h, kn, s)[None]
    m = r.random((1, h, qn, kn)) < density
    m[0, 0, 0, :] = False  # no active tokens: centroids only
    m[0, -1, -1, :] = True  # no inactive cluster: tokens only
    q, qt = rand_bf16((1, h, s, 128), seed, gpu, 0.5)
    k, kt = rand_bf16((1, h, s, 128), seed + 1, gpu, 0.5)
    v, vt = rand_bf16((1, h, s, 128), seed + 2, gpu)
    kc, kct = rand_bf16((1, h, kn, 128), seed + 3, gpu, 0.5)
    vc, vct = rand_bf16((1, h, kn, 128), seed + 4, gpu)
    out = dynamic_block_sparse_prune_fwd(qt, kt, vt, kct, vct, torch.from_numpy(m).to(gpu), _i32(qs, gpu),
                                         _i32(ks, gpu))
    _attn_check(out, O.ear_compensated_attention(q, k, v, kc, vc, m, qs, ks))


def test_compensation_of_point_mass_clusters_is_dense(gpu):
    from svoo_amd.ear import dynamic_block_sparse_prune_fwd

    say("ear attention point-mass clusters vs sdpa")
    r = np.random.default_rng(9)
    h, kn, s = 2, 30, 2048
    ks = rand_sizes(r, h, kn, s)[None]
    kc, kct = rand_bf16((1, h, kn, 128), 31, gpu, 0.5)
    vc, vct = rand_bf16((1, h, kn, 128), 32, gpu)
    k = np.stack([np.repeat(kc[0, i], ks[0, i], axis=0) for i in range(h)])[None]
    v = np.stack([np.repeat(vc[0, i], ks[0, i], axis=0) for i in range(h)])[None]
    q, qt = rand_bf16((1, h, s, 128), 33, gpu, 0.5)
    qs = np.array([[[s // 2, s - s // 2]] * h], np.int32)
    m = r.random((1, h, 2, kn)) < 0.3
    out = dynamic_block_sparse_prune_fwd(qt, bf16(k, gpu), bf16(v, gpu), kct, vct, torch.from_numpy(m).to(gpu),
                                         _i32(qs, gpu), _i32(ks, gpu))
    ref = torch.nn.functional.scaled_dot_product_attention(qt.float(), bf16(k, gpu).float(), bf16(v, gpu).float())
    _attn_check(out, ref.cpu().numpy())


def test_compensated_attention_rejects_inconsistent_sizes(gpu):
    from svoo_amd.ear import dynamic_block_sparse_prune_fwd_flashinfer

    say("ear attention size validation")
    _, qt = rand_bf16((1, 1, 256, 128), 1, gpu)
    _, kc = rand_bf16((1, 1, 2, 128), 2, gpu)
    m = torch.ones(1, 1, 2, 2, dtype=torch.bool, device=gpu)
    with pytest.raises(AssertionError):
        dynamic_block_sparse_prune_fwd_flashinfer(qt, qt, qt, kc, kc, m, _i32([[[128, 100]]], gpu),
                                                  _i32([[[128, 128]]], gpu), is_cpu=False)


# ------------------------------------------------------------------------------------------ end to end
def test_identify_dynamic_map_estimated_api(gpu):
    from svoo_amd import ear

    say("identify_dynamic_map_estimated api")
    r = np.random.default_rng(12)
    h, s, qn, kn = 2, 1500, 16, 50
    qs, ks = rand_sizes(r, h, qn, s)[None], rand_sizes(r, h, kn, s)[None]
    _, qct = rand_bf16((1, h, qn, 128), 40, gpu, 0.4)
    _, kct = rand_bf16((1, h, kn, 128), 41, gpu, 0.4)
    _, qpt = rand_bf16((1, h, s, 128), 42, gpu)
    _, kpt = rand_bf16((1, h, s, 128), 43, gpu)
    _, vpt = rand_bf16((1, h, s, 128), 44, gpu)
    qst, kst = _i32(qs, gpu), _i32(ks, gpu)
    vc, m1, parts = ear.ear_map_and_value_centroids(qpt, kpt, vpt, qst, kst, qct, kct, 0.8, 1.0, [0.1, 0.2],
                                                    return_parts=True)
    m2 = ear.identify_dynamic_map_estimated(qpt, kpt, vpt, qst, kst, qct, kct, vc, 0.8, 1.0, [0.1, 0.2])
    assert torch.equal(m1, m2)
    want = O.ear_select(f32(parts["eff"]), f32(parts["c"]), qs, ks, 0.8, [0.1, 0.2])
    np.testing.assert_array_equal(m1.cpu().numpy(), want)


def test_ear_processor_matches_oracle(gpu):
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_EARAttn_Processor

    say("ear processor attention_core_logic vs oracle")
    cfg = synth.SynthConfig("ear-small", 51, 2, 3, 16, 20, 128, 24, 12, 32, 3, 0.1, 0.4, True, "bf16")
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
    qt, kt, vt = (x.to(gpu) for x in (q, k, v))
    out = proc.attention_core_logic(qt, kt, vt, torch.tensor([100.0], device=gpu))
    torch.cuda.synchronize()
    last = proc._last_call
    ref, parts = O.ear_attention_call(q.float().numpy(), k.float().numpy(), v.float().numpy(), 12, 32, 3, 0.6, 0.1,
                                      1.0, init_q_idx=qi, init_k_idx=ki, return_parts=True)
    # clustering, value centroids and logits are exact; the efficiency within tolerance
    np.testing.assert_array_equal(last["clustering"]["klabels"].cpu().numpy(), parts["klabels"])
    np.testing.assert_array_equal(f32(last["v_centroids"])[0], parts["vc"])
    np.testing.assert_array_equal(f32(last["c"])[0], parts["c"])
    np.testing.assert_allclose(f32(last["eff"])[0], parts["eff"], rtol=0, atol=EFF_ABS)
    # the selection is exact on the scores it was given
    want_map = O.ear_select(f32(last["eff"]), f32(last["c"]), parts["qsizes"][None], parts["ksizes"][None], 0.6, 0.1)
    np.testing.assert_array_equal(last["map"].cpu().numpy(), want_map)
    assert out.shape == (1, s, h * 128)
    if np.array_equal(want_map, parts["map"]):
        _attn_check(out, ref)
    else:  # an efficiency near-tie flipped a block: compare on the GPU's map
        qp = O.permute_rows(q.float().numpy()[0], parts["qidx"])
        kp = O.permute_rows(k.float().numpy()[0], parts["kidx"])
        vp = O.permute_rows(v.float().numpy()[0], parts["kidx"])
        op = O.ear_compensated_attention(qp[None], kp[None], vp[None], parts["kcent"][None], parts["vc"][None],
                                         want_map, parts["qsizes"][None], parts["ksizes"][None])[0]
        _attn_check(out, O.unpermute_rows(op, parts["qidx"]).transpose(1, 0, 2).reshape(1, s, h * 128))
