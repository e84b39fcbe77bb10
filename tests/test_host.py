"""Host-side logic and the C ABI surface (CPU only, no kernel launches)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"


def _header_symbols():
    text = (ROOT / "include" / "svoo_hip.h").read_text()
    return sorted(set(re.findall(r"\b(svoo_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from svoo_amd import _lib

    syms = _header_symbols()
    assert len(syms) >= 20
    h = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in syms if not hasattr(h, s)]
    assert not missing, missing
    assert set(syms) == set(_lib.EXPORTED_SYMBOLS), set(syms) ^ set(_lib.EXPORTED_SYMBOLS)


def test_library_reports_errors_without_launching():
    from svoo_amd import _lib

    L = _lib.lib()
    assert L.svoo_version() == 100
    rc = L.svoo_vbsa_fwd(None, None, None, None, None, None, None, 1, 1, 128, 1, 1, None, 0, None, None)
    assert rc == -1 and "null pointer" in _lib.last_error()
    rc = L.svoo_block_mask(1, 1, 1, 1, 1, 1, 1, 1, 1, 160, 0.5, 0, 1, None, 1, None)
    assert rc == -2 and "D=160" in _lib.last_error()
    rc = L.svoo_block_mask(1, 1, 1, 1, 1, 1, 1, 1, 1, 128, 0.5, 0, 1, None, None, None)
    assert rc == -1 and "null pointer" in _lib.last_error()  # the scores buffer is required
    rc = L.svoo_centroid_scores(1, 1, 1, 1, 1, 0, 1, None)
    assert rc == -2 and "D=0" in _lib.last_error()
    rc = L.svoo_convert_rows(1, 0, 0, 1, 0, 128, 4, None)
    assert rc == -1 and "src_cols=0" in _lib.last_error()
    assert L.svoo_co_cluster_workspace_size(40, 75600, 100, 1000, 128) > 0
    rc = L.svoo_convert(1, 0, 1, 3, 8, None)
    assert rc == -1 and "element types" in _lib.last_error()
    rc = L.svoo_convert(None, 0, 1, 2, 8, None)
    assert rc == -1 and "null pointer" in _lib.last_error()
    assert L.svoo_convert(1, 2, 1, 0, 0, None) == 0  # nothing to convert: no launch


def test_operators_reject_non_float_inputs_before_any_call():
    """Operands are bf16, fp16 or fp32 (fp16 / fp32 are rounded to bf16 on the GPU); anything else is refused
    on the host, before a GPU is touched."""
    from svoo_amd import _lib
    from svoo_amd.co_clustering import co_cluster_tokens_full, dynamic_block_sparse_fwd

    with pytest.raises(TypeError, match="bfloat16, float16 or float32"):
        _lib.as_bf16(torch.zeros(2, 3, 128, dtype=torch.int32), "x")
    with pytest.raises(TypeError, match="float64"):
        co_cluster_tokens_full(torch.zeros(1, 64, 128, dtype=torch.float64), torch.zeros(1, 64, 128), 4, 4, 1)
    with pytest.raises(AssertionError, match="GPU"):
        _lib.as_bf16(torch.zeros(2, 3, 128), "x")  # a float tensor on the CPU
    with pytest.raises(AssertionError, match="CUDA"):
        dynamic_block_sparse_fwd(*(torch.zeros(1, 1, 8, 128),) * 3, None, None, None)
    with pytest.raises(ValueError, match="head dim 192"):
        _lib.as_rows128(torch.zeros(2, 3, 192), "x")


def test_noalloc_attention_rejects_plans_above_its_scratch():
    """The allocation-free attention checks its plan size against the static scratch before any HIP call."""
    from svoo_amd import _lib

    L = _lib.lib()
    limit = 4 << 20  # SVOO_NOALLOC_SCRATCH_BYTES
    assert L.svoo_vbsa_workspace_size(40, 75600, 100, 1000) <= limit  # the Wan2.1-14B 720p layer fits
    bh = 2048
    assert L.svoo_vbsa_workspace_size(bh, 75600, 100, 1000) > limit
    rc = L.svoo_vbsa_fused_fwd_noalloc(1, 1, 1, 1, 1, 1, 1, 1, 1, bh, 1, 75600, 128, 100, 1000, None, None)
    assert rc == -3 and "static scratch" in _lib.last_error()
    rc = L.svoo_vbsa_fused_fwd_noalloc(1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 1, 75600, 128, 100, 1000, None, None)
    assert rc == -1 and "bad dims" in _lib.last_error()


def test_product_code_never_touches_the_oracle():
    for p in (ROOT / "svoo_amd").rglob("*.py"):
        text = p.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), p
        assert "svoo_oracle" not in text, p


@pytest.mark.parametrize("mn,mx", [
    (0, 0), (0.2, 0), ([0.7, 0.15, 0.3], 0), ([0.2, 0.0, 0.05], [0.1, 0.3, 0.0]), (0.1, 0.05), (0, 0.001),
    ([0.25, 0.25, 0.25], 0.1), (torch.tensor([0.1, 0.2, 0.3]), None), (np.array([0.3, 0.33, 0.7]), 0),
])
def test_mask_row_params_matches_oracle(mn, mx):
    from svoo_amd.co_clustering import mask_row_params

    for kn in (64, 500, 1000):
        pre, cap = mask_row_params(3, kn, mn, mx)
        opre, ocap = O.mask_row_params(3, kn, mn, mx)
        assert pre == opre.tolist() and cap == ocap.tolist()


def test_sparsity_lookup_fixture():
    from svoo_amd.sparsity import SparsityLookup

    lk = SparsityLookup(str(GOLDEN / "sparsity_wan_1.3B_t2v_steps1-3.csv"), verbose=False)
    assert len(lk.lookup_dict) == 3 * 30 * 12
    assert lk.get_sparsity(1, 0, 0) == pytest.approx(0.7382)
    assert lk.get_sparsity(1, 0, 1) == pytest.approx(0.0411)
    assert lk.get_sparsity(4, 0, 0) is None
    assert lk.has_data_for_step_layer(2, 29, 12)
    assert not lk.has_data_for_step_layer(4, 0, 12)
    assert lk.get_sparsity_batch(9, 0, 3) == [0.0, 0.0, 0.0]
    with pytest.raises(FileNotFoundError):
        SparsityLookup(str(GOLDEN / "missing.csv"))


def _proc(**kw):
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    cls = type("P", (WanAttn_SAPAttn_Processor,), dict(kw))
    return cls(layer_idx=3)


def test_reuse_schedule():
    p = _proc(start_reuse_step=11, reuse_interval=40)
    p._cached_clustering_results = {"x": 1}
    got = []
    for step in range(1, 51):
        p.current_inference_step = step
        got.append(p.should_recluster())
    # Steps 1..10 always cluster, step 11 is the reuse anchor, 12..50 reuse (next recluster would be 51).
    assert [s for s, r in zip(range(1, 51), got) if r] == list(range(1, 12))
    p2 = _proc(start_reuse_step=11, reuse_interval=40)
    p2.current_inference_step = 30
    assert p2.should_recluster()  # nothing cached yet -> forced


def test_reuse_debug_trace(monkeypatch, capsys):
    """SVG_REUSE_DEBUG prints the reference's [reuse] lines from kmeans_clustering's decision
    (svoo/models/wan/attention.py:682-704); should_recluster() alone stays silent."""
    p = _proc(start_reuse_step=2, reuse_interval=2)
    p.current_inference_step = 3
    monkeypatch.setenv("SVG_REUSE_DEBUG", "1")
    assert p.should_recluster()
    assert capsys.readouterr().out == ""
    assert p.should_recluster(trace=True)  # offset 1: reuse, but nothing cached -> forced
    assert capsys.readouterr().out.splitlines() == [
        "[reuse] current_step=3, start_reuse_step=2, reuse_interval=2",
        "[reuse] offset=1, should_recluster=False",
        "[reuse] No cached clustering results, forcing recluster",
    ]
    p._cached_clustering_results = {"x": 1}
    assert not p.should_recluster(trace=True)
    assert capsys.readouterr().out.splitlines()[-1] == "[reuse] Reusing cached clustering results"
    p.current_inference_step = 1  # before the reuse anchor: offset None, recluster
    assert p.should_recluster(trace=True)
    assert "[reuse] offset=None, should_recluster=True" in capsys.readouterr().out
    monkeypatch.setenv("SVG_REUSE_DEBUG", "false")
    p.should_recluster(trace=True)
    assert capsys.readouterr().out == ""


def test_reuse_similarity_report(monkeypatch, capsys):
    """COMPUTE_REUSE_SIMILARITY: per (layer, head), the NMI of this clustering's labels against the previous
    recorded step's (svoo/models/wan/attention.py:821-861), checked against a plug-in computation of NMI."""
    r = np.random.default_rng(7)
    n, heads = 500, 2
    p = _proc()

    def labels(seed):
        g = np.random.default_rng(seed)
        return {"qlabels": torch.from_numpy(g.integers(0, 8, (heads, n)).astype(np.int32)),
                "klabels": torch.from_numpy(g.integers(0, 16, (heads, n)).astype(np.int32))}

    def nmi(a, b):  # arithmetic-mean normalised mutual information from the contingency table
        ua, ia = np.unique(a, return_inverse=True)
        ub, ib = np.unique(b, return_inverse=True)
        c = np.zeros((len(ua), len(ub)))
        np.add.at(c, (ia, ib), 1.0)
        pij = c / c.sum()
        pi, pj = pij.sum(1), pij.sum(0)
        nz = pij > 0
        mi = (pij[nz] * np.log(pij[nz] / np.outer(pi, pj)[nz])).sum()
        h = lambda q: -(q[q > 0] * np.log(q[q > 0])).sum()  # noqa: E731
        return mi / ((h(pi) + h(pj)) / 2.0)

    r1 = labels(1)
    p.current_inference_step = 4
    assert p.report_reuse_similarity(r1, 3, heads) == {}  # nothing earlier
    r2 = labels(2)
    # the second clustering keeps most labels of the first
    keep = r.random((heads, n)) < 0.8
    for k_ in ("qlabels", "klabels"):
        r2[k_] = torch.where(torch.from_numpy(keep), r1[k_], r2[k_])
    p.current_inference_step = 9
    got = p.report_reuse_similarity(r2, 3, heads)
    out = capsys.readouterr().out.splitlines()
    assert len(out) == heads and out[0].startswith("[Reuse Similarity] Step 4->9, Layer 3, Head 0: Q=")
    for h in range(heads):
        ps, qn, kn = got[h]
        assert ps == 4
        assert qn == pytest.approx(nmi(r1["qlabels"][h].numpy(), r2["qlabels"][h].numpy()), rel=1e-9)
        assert kn == pytest.approx(nmi(r1["klabels"][h].numpy(), r2["klabels"][h].numpy()), rel=1e-9)
        assert 0.2 < qn < 1.0
    # identical labels give 1
    p.current_inference_step = 10
    got = p.report_reuse_similarity(r2, 3, heads)
    assert got[0][0] == 9 and got[0][1] == pytest.approx(1.0) and got[0][2] == pytest.approx(1.0)


def test_save_qk_dump(monkeypatch, tmp_path):
    """SAVE_QK writes {dir}/step{timestep}/layer{l}.pt with q, k, timestep, layer_idx from the scheduler
    timestep SAVE_QK_START_STEP on (svoo/models/wan/attention.py:217-240)."""
    from svoo_amd.processor import save_qk

    q, k = torch.randn(1, 2, 6, 4), torch.randn(1, 2, 6, 4)
    assert save_qk(q, k, torch.tensor([999.0]), 3) is None  # switched off
    monkeypatch.setenv("SAVE_QK", "1")
    assert save_qk(q, k, torch.tensor([999.0]), 3) is None  # no directory
    monkeypatch.setenv("SAVE_QK_DIR", str(tmp_path))
    monkeypatch.setenv("SAVE_QK_START_STEP", "500")
    assert save_qk(q, k, torch.tensor([400.0]), 3) is None  # before the start step
    assert save_qk(q, k, None, 3) is None  # dense (no timestep) calls are not captured
    path = save_qk(q, k, torch.tensor([999.0, 999.0]), 3)
    assert path == str(tmp_path / "step999.0" / "layer3.pt")
    d = torch.load(path, weights_only=True)
    assert torch.equal(d["q"], q) and torch.equal(d["k"], k) and d["timestep"] == 999.0 and d["layer_idx"] == 3


def test_candidate_exclusion_bound():
    """The key-side candidate pass (cocluster.hip) drops cluster j of a token with anchor a when
    D_aj = |P_a - P_j| >= 2 d_a + m, d_a = |u - P_a|, u = y / |y|.  Its argument: then
    P_a . y - P_j . y >= |y| (m^2 - nu) / 2 with nu >= max_j n_j - n_a for rows of squared norm n_j <= 1 (the
    l2norm's eps).  Checked on random profiles with non-unit rows, including the extreme of the bound; a
    plausible slip (d_a instead of 2 d_a in the radius) is caught by the same data."""
    rng = np.random.default_rng(11)
    worst = np.inf
    slip_caught = False
    for _ in range(400):
        kp, J = int(rng.integers(2, 24)), int(rng.integers(2, 96))
        P = rng.normal(size=(J, kp))
        P /= np.linalg.norm(P, axis=1, keepdims=True)
        P *= np.sqrt(1.0 - rng.uniform(0.0, 1e-3, size=J))[:, None]
        n = (P * P).sum(1)
        y = rng.normal(size=kp) * rng.uniform(0.01, 100.0)
        yn = np.linalg.norm(y)
        a = int(rng.integers(J))
        # anchors near the token too (the candidate pass's usual case)
        if rng.random() < 0.5:
            y = yn * (P[a] + rng.normal(size=kp) * rng.uniform(0.0, 0.5))
            yn = np.linalg.norm(y)
        u = y / yn
        d_a = np.linalg.norm(u - P[a])
        D = np.linalg.norm(P - P[a], axis=1)
        nu = n.max() - n[a]
        m = rng.uniform(0.0, 0.3)
        excl = D >= 2.0 * d_a + m
        if excl.any():
            margin = (P[a] @ y - P[excl] @ y) - yn * (m * m - nu) / 2.0
            worst = min(worst, margin.min() / yn)
        slip = (D >= d_a + m) & ~excl
        if slip.any() and ((P[slip] @ y) > P[a] @ y).any():
            slip_caught = True
    assert worst >= -1e-12
    assert slip_caught


def test_dynamic_ratio_from_profile():
    from svoo_amd.sparsity import SparsityLookup

    lk = SparsityLookup(str(GOLDEN / "sparsity_wan_1.3B_t2v_steps1-3.csv"), verbose=False)
    p = _proc(use_dynamic_min_kc_ratio=True, sparsity_lookup=lk, dynamic_min_kc_ratio_min=0.15,
              dynamic_min_kc_ratio_max=0.20, min_kc_ratio=0.1)
    vals = p._get_min_kc_ratio_for_heads_from_step(1, 12)
    raw = lk.get_sparsity_batch(1, 3, 12)
    assert vals == [min(max(v, 0.15), 0.20) for v in raw]
    assert p._get_min_kc_ratio_for_heads_from_step(7, 12) == 0.1  # step missing -> scalar
    assert p._get_min_kc_ratio_for_heads_from_step(None, 12) == 0.1


def test_inference_step_counter():
    p = _proc(_current_internal_timestep=None, _inference_step_counter=0, _seen_timesteps=set())
    steps = [p._get_inference_step(t) for t in (999, 999, 980, 980, 950)]
    assert steps == [1, 1, 2, 2, 3]
    assert p._get_inference_step(999) == 1  # a larger timestep starts a new generation


def test_synth_is_deterministic_and_head_separable():
    from svoo_amd import synth

    cfg = synth.SynthConfig("t", 5, 3, 2, 4, 4, 128, 8, 4, 6, 2, 0.1, 0.3, True, "bf16")
    a = synth.make_qkv(cfg)
    b = synth.make_qkv(cfg, heads=[2])
    for x, y in zip(a, b):
        assert torch.equal(x[:, 2:3], y)
    c = synth.make_qkv(cfg)
    assert all(torch.equal(x, y) for x, y in zip(a, c))
    d = synth.head_densities(cfg)
    assert all(0.1 <= r <= 0.3 for r in d) and d == synth.head_densities(cfg)


def test_golden_fixture_matches_oracle():
    from tests.golden.make_golden import MASK_CASES, SMALL, small_inputs

    g = np.load(GOLDEN / "golden_small.npz")
    qb, kb, vb, qi, ki = small_inputs()
    np.testing.assert_array_equal(qi, g["q_init"])
    q, k = O.bf16_from_bits(qb), O.bf16_from_bits(kb)
    ql, qc, qs, kl, kc, ks = O.co_cluster_tokens(q, k, SMALL.num_q_centroids, SMALL.num_k_centroids,
                                                 SMALL.kmeans_iters, init_q_idx=qi, init_k_idx=ki)
    np.testing.assert_array_equal(ql, g["qlabels"])
    np.testing.assert_array_equal(O.bf16_bits(kc), g["kcent"])
    for ci, (p, mn, mx) in enumerate(MASK_CASES):
        m = O.identify_dynamic_map(qc[None], kc[None], qs[None], ks[None], p, mn, mx)
        np.testing.assert_array_equal(m[0], g[f"map{ci}"])


def test_hunyuan_processor_post_processing_matches_oracle():
    import torch

    from svoo_amd.processor import Hunyuan_SAPAttn_Processor

    r = np.random.default_rng(3)
    m = r.random((1, 2, 5, 7)) < 0.4
    qs = r.integers(1, 9, size=(1, 2, 5)).astype(np.int32)
    ks = r.integers(0, 9, size=(1, 2, 7)).astype(np.int32)
    idx = np.stack([r.permutation(30) for _ in range(2)]).astype(np.int32)
    proc = Hunyuan_SAPAttn_Processor(layer_idx=0)
    got = proc.dynamic_map_post_processing(torch.from_numpy(m), torch.from_numpy(qs), torch.from_numpy(ks),
                                           torch.from_numpy(idx), 30, 12, 7, 5)
    want = O.hunyuan_post_process(m, qs, ks, idx, 30, 12, 7)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.numpy(), w)


def _tiny_pipe(layers=2, with_second=False):
    from svoo_amd import dit

    cfg = dit.WanDiTConfig(num_attention_heads=2, ffn_dim=64, num_layers=layers, text_dim=32)
    pipe = dit.make_pipe(cfg, dtype=torch.float32)
    if with_second:
        pipe.transformer_2 = dit.make_pipe(cfg, dtype=torch.float32, seed=6).transformer
    return pipe


def test_replace_wan_attention_configures_and_installs():
    from svoo_amd.inference import replace_wan_attention, wan_token_geometry
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    pipe = _tiny_pipe(layers=3, with_second=True)
    # inference.py:81-83: 81 frames, 480x832 -> 21 latent frames of 30x52 patches
    assert wan_token_geometry(pipe, 480, 832, 81) == (21, 1560)
    cls = type("P", (WanAttn_SAPAttn_Processor,), {})
    procs = replace_wan_attention(
        pipe, 480, 832, 81, first_layers_fp=1, first_times_fp=900, num_q_centroids=100, num_k_centroids=500,
        top_p_kmeans=0.9, min_kc_ratio=0.1, kmeans_iter_init=2, kmeans_iter_step=2, start_reuse_step=11,
        reuse_interval=20, use_dynamic_min_kc_ratio=True,
        sparsity_csv_path=str(GOLDEN / "sparsity_wan_1.3B_t2v_steps1-3.csv"),
        dynamic_min_kc_ratio_min=0.15, dynamic_min_kc_ratio_max=0.2, processor_cls=cls)
    assert len(procs) == 6  # both transformers
    for t in (pipe.transformer, pipe.transformer_2):
        assert [b.attn1.processor.layer_idx for b in t.blocks] == [0, 1, 2]
        assert all(isinstance(b.attn1.processor, cls) for b in t.blocks)
        assert not any(isinstance(b.attn2.processor, cls) for b in t.blocks)  # cross-attention stays dense
    assert (cls.num_frame, cls.frame_size, cls.context_length, cls.num_layers) == (21, 1560, 0, 3)
    assert (cls.num_q_centroids, cls.num_k_centroids, cls.top_p_kmeans, cls.min_kc_ratio) == (100, 500, 0.9, 0.1)
    assert (cls.start_reuse_step, cls.reuse_interval, cls.first_layers_fp, cls.first_times_fp) == (11, 20, 1, 900)
    assert cls.use_dynamic_min_kc_ratio and cls.sparsity_lookup is not None
    p = procs[4]
    assert p._get_min_kc_ratio_for_heads_from_step(2, 12) == [
        min(max(v, 0.15), 0.2) for v in cls.sparsity_lookup.get_sparsity_batch(2, 1, 12)]
    # the base class is untouched
    assert WanAttn_SAPAttn_Processor.num_frame == 0


def test_replace_wan_attention_fallbacks_and_rejections():
    from svoo_amd.inference import replace_wan_attention
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    pipe = _tiny_pipe()
    cls = type("P", (WanAttn_SAPAttn_Processor,), {})
    replace_wan_attention(pipe, 480, 832, 81, 0, 900, num_q_centroids=8, num_k_centroids=16, top_p_kmeans=0.9,
                          min_kc_ratio=0.1, use_dynamic_min_kc_ratio=True,
                          sparsity_csv_path=str(GOLDEN / "missing.csv"), processor_cls=cls)
    assert not cls.use_dynamic_min_kc_ratio and cls.sparsity_lookup is None  # unreadable profile -> scalar ratio
    with pytest.raises(ValueError):
        replace_wan_attention(pipe, 480, 832, 81, 0, 900, pattern="SVG", processor_cls=cls)
    with pytest.raises(ValueError):
        replace_wan_attention(pipe, 480, 832, 81, 0, 900, use_svoo=False, processor_cls=cls)
    with pytest.raises(NotImplementedError):
        replace_wan_attention(pipe, 480, 832, 81, 0, 900, use_global_constraints=True, processor_cls=cls)


def test_replace_wan_attention_ear_and_dense_patterns():
    from svoo_amd.inference import replace_wan_attention
    from svoo_amd.processor import WanAttn_DenseAttn_Processor, WanAttn_EARAttn_Processor, WanAttn_SAPAttn_Processor

    pipe = _tiny_pipe()
    cls = type("E", (WanAttn_EARAttn_Processor,), {})
    procs = replace_wan_attention(pipe, 480, 832, 81, 0, 900, pattern="EAR", num_q_centroids=8, num_k_centroids=16,
                                  top_p_kmeans=0.9, min_kc_ratio=0.1, ear_gamma=0.5, processor_cls=cls)
    assert all(isinstance(p, cls) for p in procs)
    assert cls.use_ear and cls.ear_gamma == 0.5 and cls.num_frame == 21
    assert not WanAttn_SAPAttn_Processor.use_ear and WanAttn_EARAttn_Processor.use_ear
    sap = type("S", (WanAttn_EARAttn_Processor,), {})
    replace_wan_attention(pipe, 480, 832, 81, 0, 900, pattern="SAP", num_q_centroids=8, num_k_centroids=16,
                          top_p_kmeans=0.9, processor_cls=sap)
    assert not sap.use_ear  # inference.py:282 sets use_ear from the pattern
    # "dense": the diagnostic processor class (dense attention on every layer)
    procs = replace_wan_attention(pipe, 480, 832, 81, 0, 900, pattern="dense")
    assert all(type(p) is WanAttn_DenseAttn_Processor for p in procs)


@pytest.mark.parametrize("ratio", [0, 0.0, 0.1, 0.35, [0.1], [0.0, 0.05, 0.35], [0.2, 0.3], (0.25, 0.5, 0.01)])
def test_ear_row_params_matches_oracle(ratio):
    from svoo_amd.ear import ear_row_params

    for kn in (16, 100, 1000):
        pre, bpre = ear_row_params(3, kn, ratio)
        opre, obpre = O.ear_row_params(3, kn, ratio)
        assert pre == list(opre) and bpre == list(obpre), (ratio, kn)
    pre, bpre = ear_row_params(3, 100, torch.tensor([0.0, 0.05, 0.35]))
    assert (pre, bpre) == ([0, 5, 34], [0, 10, 69])  # float32 reads of a tensor (0.35 -> 0.34999999)



def test_replace_hunyuan_attention_numbers_double_then_single_blocks():
    """HunyuanVideo 1.0 has 20 double-stream and 40 single-stream blocks; the profile CSV's layer index runs
    over the double-stream blocks first (svoo/models/hunyuan10/inference.py:207-231)."""
    from types import SimpleNamespace

    from svoo_amd.inference import replace_hunyuan10_attention, replace_hunyuan_attention
    from svoo_amd.processor import Hunyuan_SAPAttn_Processor

    assert replace_hunyuan10_attention is replace_hunyuan_attention
    blk = lambda: SimpleNamespace(attn=SimpleNamespace(processor=None))  # noqa: E731
    pipe = SimpleNamespace(transformer=SimpleNamespace(transformer_blocks=[blk() for _ in range(20)],
                                                       single_transformer_blocks=[blk() for _ in range(40)]))
    cls = type("H", (Hunyuan_SAPAttn_Processor,), {})
    procs = replace_hunyuan_attention(
        pipe, 720, 1280, 129, prompt_length=200, first_layers_fp=0.025, first_times_fp=0.075, num_q_centroids=400,
        num_k_centroids=1000, top_p_kmeans=0.9, min_kc_ratio=0.1, kmeans_iter_init=50, kmeans_iter_step=2,
        context_length=512, start_reuse_step=11, reuse_interval=0, use_dynamic_min_kc_ratio=True,
        sparsity_csv_path=str(GOLDEN / "sparsity_wan_1.3B_t2v_steps1-3.csv"), dynamic_min_kc_ratio_min=0.15,
        dynamic_min_kc_ratio_max=0.2, processor_cls=cls)
    assert [b.attn.processor.layer_idx for b in pipe.transformer.transformer_blocks] == list(range(20))
    assert [b.attn.processor.layer_idx for b in pipe.transformer.single_transformer_blocks] == list(range(20, 60))
    assert [p.layer_idx for p in procs] == list(range(60)) and all(type(p) is cls for p in procs)
    # 129 frames -> 33 latent frames of 45 x 80 patches; the text context is fixed at 256 tokens
    assert (cls.num_frame, cls.frame_size, cls.context_length, cls.prompt_length) == (33, 3600, 256, 200)
    assert (cls.num_q_centroids, cls.num_k_centroids, cls.kmeans_iter_init, cls.kmeans_iter_step) == (400, 1000, 50, 2)
    assert cls.reuse_interval == 1 and cls.start_reuse_step == 11 and cls.num_layers == 60
    assert cls.use_dynamic_min_kc_ratio and cls.sparsity_lookup.get_sparsity(1, 0, 0) is not None
    assert Hunyuan_SAPAttn_Processor.prompt_length == 0  # the base class is untouched
    with pytest.raises(ValueError):
        replace_hunyuan_attention(pipe, 720, 1280, 129, 10, 0, 0, pattern="SVG", processor_cls=cls)
    with pytest.raises(ValueError):
        replace_hunyuan_attention(pipe, 720, 1280, 129, 300, 0, 0, processor_cls=cls)  # prompt longer than the text
    replace_hunyuan_attention(pipe, 720, 1280, 129, 10, 0, 0, use_dynamic_min_kc_ratio=True,
                              sparsity_csv_path=str(GOLDEN / "missing.csv"), processor_cls=cls)
    assert not cls.use_dynamic_min_kc_ratio and cls.sparsity_lookup is None


def test_hunyuan_processor_rejects_prompt_longer_than_context():
    from svoo_amd.processor import Hunyuan_SAPAttn_Processor

    cls = type("H", (Hunyuan_SAPAttn_Processor,), {"prompt_length": 300, "context_length": 256, "num_frame": 1,
                                                   "frame_size": 4})
    x = torch.zeros(1, 2, 260, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="prompt_length"):
        cls(layer_idx=0).attention_core_logic(x, x, x, None)

def test_tiny_dit_dense_forward_shapes():
    from svoo_amd import dit

    pipe = _tiny_pipe()
    cfg = pipe.transformer.config
    lat = torch.randn(dit.latent_shape(cfg, 64, 96, 9))
    with torch.no_grad():
        out = pipe.transformer(lat, torch.tensor([900.0]), torch.randn(1, 8, cfg.text_dim))
    assert out.shape == lat.shape and torch.isfinite(out).all()
    cos, sin = dit.rope_tables(cfg, 3, 4, 6, "cpu")
    assert cos.shape == (1, 72, 1, 128)
    # pairs share one angle; the t-axis channels of token 0 (position 0) do not rotate
    assert torch.equal(cos[..., 0::2], cos[..., 1::2]) and torch.all(cos[0, 0, 0] == 1)


def test_sparsity_log_merge_roundtrip(tmp_path):
    from svoo_amd.sparsity import SparsityLookup, format_sparsity_log, merge_sparsity_data, parse_sparsity_file, save_to_csv

    a, b = tmp_path / "run_a.txt", tmp_path / "run_b.txt"
    with open(a, "w") as f:
        f.write("\n".join(format_sparsity_log(0, "self", 1, 0.95, 0.2, [0.1, 0.3], 100, 100)) + "\n")
        f.write("\n".join(format_sparsity_log(1, "self", 1, 0.95, 0.5, [0.5, 0.5], 100, 10)) + "\n")
    with open(b, "w") as f:
        f.write("\n".join(format_sparsity_log(0, "self", 1, 0.95, 0.25, [0.2, 0.3], 100, 100)) + "\n")
    pa = parse_sparsity_file(a)
    assert pa[(1, 0, 0)] == 0.1 and pa[(1, 1, 1)] == 0.5 and len(pa) == 4
    merged = merge_sparsity_data([a, b, tmp_path / "missing.txt"])
    assert merged[(1, 0, 0)] == 0.2 and merged[(1, 0, 1)] == 0.3  # maximum over the runs
    out = tmp_path / "profile.csv"
    save_to_csv(merged, out)
    lk = SparsityLookup(str(out), verbose=False)
    assert lk.get_sparsity(1, 0, 0) == 0.2 and lk.get_sparsity_batch(1, 1, 2) == [0.5, 0.5]
    assert open(out).readline().strip() == "Step,Layer,Head,Sparsity"


def test_sparsity_resume_guard(tmp_path, monkeypatch):
    from svoo_amd.sparsity import format_sparsity_log, has_completed_sparsity_entry, record_sparsity_entry

    log = tmp_path / "raw.txt"
    log.write_text("\n".join(format_sparsity_log(3, "self", 7, 0.95, 0.1, [0.1] * 4, 50, 50)) + "\n")
    monkeypatch.delenv("SVOO_SPARSITY_RESUME", raising=False)
    assert not has_completed_sparsity_entry(str(log), 3, 7, 4)  # opt-in only
    for off in ("0", "false", "False", ""):  # the reference's off values (svoo/sparsity/exact.py:50-51)
        monkeypatch.setenv("SVOO_SPARSITY_RESUME", off)
        assert not has_completed_sparsity_entry(str(log), 3, 7, 4)
    for on in ("2", "y", "enabled", "FALSE", "no"):  # any other value is on there, so it is here
        monkeypatch.setenv("SVOO_SPARSITY_RESUME", on)
        assert has_completed_sparsity_entry(str(log), 3, 7, 4), on
    monkeypatch.setenv("SVOO_SPARSITY_RESUME", "True")
    assert has_completed_sparsity_entry(str(log), 3, 7, 4)
    assert not has_completed_sparsity_entry(str(log), 3, 7, 5)
    assert not has_completed_sparsity_entry(str(log), 3, 8, 4)
    # this process's own appends reach the guard through record_sparsity_entry, without a re-read
    with open(log, "a") as f:
        f.write("\n".join(format_sparsity_log(3, "self", 8, 0.95, 0.1, [0.1] * 4, 50, 50)) + "\n")
    record_sparsity_entry(str(log), 3, 8, range(4))
    assert has_completed_sparsity_entry(str(log), 3, 8, 4)
    # a resumed run (a fresh index) parses the file once, including partial entries
    from svoo_amd.sparsity import exact

    part = tmp_path / "partial.txt"
    part.write_text("\n".join(format_sparsity_log(0, "self", 2, 0.95, 0.1, [0.1] * 3, 50, 50)[:3]) + "\n")
    assert exact.SparsityLogIndex(str(part)).complete(0, 2, 2)
    assert not exact.SparsityLogIndex(str(part)).complete(0, 2, 3)
    assert not exact.SparsityLogIndex(str(tmp_path / "absent.txt")).complete(0, 1, 1)
    # another writer's appends are read on the next query; an unterminated line waits for its newline
    lines = format_sparsity_log(5, "self", 1, 0.95, 0.1, [0.1] * 2, 50, 50)
    with open(log, "a") as f:
        f.write("\n".join(lines[:2]) + "\n" + lines[2][:9])
    assert not has_completed_sparsity_entry(str(log), 5, 1, 2)
    with open(log, "a") as f:
        f.write(lines[2][9:] + "\n")
    assert has_completed_sparsity_entry(str(log), 5, 1, 2)
    # a truncated or replaced log is read again from the start: its old entries are gone
    log.write_text("\n".join(format_sparsity_log(9, "self", 1, 0.95, 0.1, [0.1], 50, 50)) + "\n")
    assert not has_completed_sparsity_entry(str(log), 3, 7, 4)
    assert has_completed_sparsity_entry(str(log), 9, 1, 1)
    repl = tmp_path / "raw_new.txt"
    repl.write_text("\n".join(format_sparsity_log(3, "self", 7, 0.95, 0.1, [0.1] * 4, 50, 50)) + "\n" * 40)
    import os

    os.replace(repl, log)  # same path, new inode, larger file
    assert has_completed_sparsity_entry(str(log), 3, 7, 4)
    assert not has_completed_sparsity_entry(str(log), 9, 1, 1)


def test_sparsity_chunk_rows_and_oom_backoff(monkeypatch):
    """Automatic query chunks fill a share of free memory in whole 64-row steps, capped at 4 GiB of bf16
    scores; an out-of-memory error in a chunk halves it and retries the same rows (the counts equal one
    unchunked pass), while an explicit chunk size re-raises."""
    from svoo_amd.sparsity import exact

    q = torch.zeros(1, 2, 5000, 128)
    k = torch.zeros(1, 2, 3000, 128)
    per_row = 2 * 3000 * 2
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda dev=None: (per_row * 1000, 1 << 40))
    monkeypatch.delenv("SVOO_SPARSITY_AUTO_MEM_FRACTION", raising=False)
    assert exact._query_chunk_rows(q, k) == 448  # 0.45 * 1000 rows -> 450 -> 448
    monkeypatch.setenv("SVOO_SPARSITY_AUTO_MEM_FRACTION", "0.05")
    assert exact._query_chunk_rows(q, k) == 50  # below 64 rows: no rounding
    for bad in ("x", "0", "1.5"):
        monkeypatch.setenv("SVOO_SPARSITY_AUTO_MEM_FRACTION", bad)
        assert exact._query_chunk_rows(q, k) == 448
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda dev=None: (1 << 45, 1 << 46))
    assert exact._query_chunk_rows(q, k) == 5000  # the 4 GiB cap holds 357913 rows: all 5000 fit
    q_long = torch.zeros(1, 2, 10 ** 6, 128)
    assert exact._query_chunk_rows(q_long, k) == ((4 << 30) // per_row) // 64 * 64

    def no_info(dev=None):
        raise RuntimeError("hipMemGetInfo failed")

    monkeypatch.setattr(torch.cuda, "mem_get_info", no_info)
    assert exact._query_chunk_rows(q, k) == 128  # the reference's fallback, min(128, rows)
    assert exact._query_chunk_rows(q[:, :, :50], k) == 50

    # the loop, with the score GEMM's output on the CPU and a count stand-in (no device here)
    calls = []

    def fake_counts(scores, scale, threshold):
        calls.append(scores.shape[2])
        if scores.shape[2] > 100:
            raise torch.cuda.OutOfMemoryError("HIP out of memory")
        return (scores.float() > 0).sum(-1).to(torch.int32)

    monkeypatch.setattr(exact, "exact_counts_from_scores", fake_counts)
    monkeypatch.setattr(exact, "_query_chunk_rows", lambda qq, kk: 448)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    g = torch.Generator().manual_seed(0)
    qq = torch.randn(1, 2, 1000, 128, generator=g).to(torch.bfloat16)
    kk = torch.randn(1, 2, 300, 128, generator=g).to(torch.bfloat16)
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))
    avg, per_head, stats = exact.compute_exact_attention_sparsity(qq, kk)
    assert calls[:3] == [448, 224, 112] and stats["chunk_size"] == 56
    ref = (torch.matmul(qq, kk.transpose(-2, -1)).float() > 0).sum(-1).double() / 300
    assert per_head == pytest.approx(ref.mean(dim=(0, 2)).tolist(), abs=1e-12)
    calls.clear()
    with pytest.raises(torch.cuda.OutOfMemoryError):
        exact.compute_exact_attention_sparsity(qq, kk, batch_size=400)


def test_sparsity_query_sampling_positions():
    from svoo_amd.sparsity.exact import _sample_query_rows

    q = torch.arange(64, dtype=torch.float32).view(1, 1, 64, 1)
    sub, n = _sample_query_rows(q, 5)
    assert n == 5 and sub.flatten().tolist() == [0, 16, 32, 47, 63]
    assert _sample_query_rows(q, 1)[0].flatten().tolist() == [32]
    assert _sample_query_rows(q, 0)[1] == 64 and _sample_query_rows(q, 99)[1] == 64


def test_exact_sparsity_rejects_bad_inputs():
    from svoo_amd.sparsity import compute_exact_attention_sparsity

    q = torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        compute_exact_attention_sparsity(q, q, threshold=1.5)
    with pytest.raises(ValueError):
        compute_exact_attention_sparsity(q.float(), q.float())
    with pytest.raises(ValueError):  # no CPU fallback: the counts run on the HIP device only
        compute_exact_attention_sparsity(q, q)
