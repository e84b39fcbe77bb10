"""fp16 and fp32 inputs.  Every kernel here computes in bf16 (its MFMA operand type); the operators round fp16 and
fp32 tensors to bf16 on the GPU (``svoo_convert``, to nearest even) and return results in the caller's dtype.  The
reference's Triton kernels load any float input as fp32 (``svoo/co_clustering.py:2121``, ``:2197``) and FlashInfer
takes fp16 or bf16 (``svoo/utils/flashinfer_sparse.py:117-124``); this path instead fixes the arithmetic type.

The tests pin that boundary: the conversion kernel against torch's round-to-nearest-even casts (special values,
ties, subnormals, overflow), and each operator on fp32 / fp16 inputs against the same operator on the
bf16-rounded inputs, bit for bit, up to the Wan processor's whole call at C1, which the benchmark configuration
specifies in fp32.  The bf16 results themselves are pinned against the oracle by the other GPU tests."""

import numpy as np
import pytest
import torch

from parity_helpers import say

pytestmark = pytest.mark.gpu


def _same_bits(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape, (a.dtype, b.dtype, a.shape, b.shape)
    ai, bi = (x.contiguous().view(torch.int16 if x.element_size() == 2 else torch.int32) for x in (a, b))
    nan = torch.isnan(a) & torch.isnan(b)
    bad = (ai != bi) & ~nan
    assert not bool(bad.any()), (int(bad.sum()), a[bad][:4].tolist(), b[bad][:4].tolist())


def _specials_f32():
    r = np.random.default_rng(31)
    base = [0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 3.0e38, -3.0e38, 3.4028235e38, 1e-45, -1e-45, 1e-40,
            1.1754944e-38, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20, 65504.0, 65520.0,
            70000.0, 2.0 ** -24, 2.0 ** -25, 2.0 ** -14, 6.0e-8]
    x = np.concatenate([np.array(base, np.float32), (r.standard_normal(100000) * np.exp2(
        r.uniform(-30, 30, 100000))).astype(np.float32)])
    return torch.from_numpy(x)


def test_convert_matches_torch_rounding(gpu):
    from svoo_amd import _lib

    say("svoo_convert against torch casts")
    x32 = _specials_f32().to(gpu)
    _same_bits(_lib.convert(x32, torch.bfloat16), x32.to(torch.bfloat16))
    x16 = x32.to(torch.float16)
    _same_bits(_lib.convert(x16, torch.bfloat16), x16.float().to(torch.bfloat16))
    xb = x32.to(torch.bfloat16)
    _same_bits(_lib.convert(xb, torch.float32), xb.float())
    _same_bits(_lib.convert(xb, torch.float16), xb.float().to(torch.float16))
    _same_bits(_lib.convert(x16, torch.float32), x16.float())
    _same_bits(_lib.convert(x32, torch.float16), x32.to(torch.float16))
    assert _lib.convert(torch.empty(0, device=gpu), torch.bfloat16).numel() == 0
    # a strided view is read in logical order
    v = x32[: 2 * 1000].view(1000, 2).t()
    _same_bits(_lib.convert(v, torch.bfloat16), v.contiguous().to(torch.bfloat16))


def _rand(shape, dtype, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * 1.7).to(dtype).to(gpu)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_co_cluster_on_rounded_inputs(gpu, dtype):
    from svoo_amd.co_clustering import co_cluster_tokens_full

    say("co_cluster_tokens_full", dtype)
    bh, n, qn, kn = 2, 3000, 24, 80
    q, k = _rand((bh, n, 128), dtype, 1, gpu), _rand((bh, n, 128), dtype, 2, gpu)
    g = torch.Generator(device=gpu).manual_seed(5)
    qi = torch.randint(0, n, (bh, qn), device=gpu, generator=g)
    ki = torch.randint(0, n, (bh, kn), device=gpu, generator=g)
    got = co_cluster_tokens_full(q, k, qn, kn, 3, init_q_idx=qi, init_k_idx=ki)
    want = co_cluster_tokens_full(q.to(torch.bfloat16), k.to(torch.bfloat16), qn, kn, 3, init_q_idx=qi,
                                  init_k_idx=ki)
    for key in want:
        if key in ("qcentroids", "kcentroids"):
            assert got[key].dtype == dtype
            _same_bits(got[key], want[key].to(dtype))
        else:
            assert torch.equal(got[key], want[key]), key
    # explicit fp32 warm-start centroids equal their bf16 rounding as a start
    qc0, kc0 = got["qcentroids"].float() * 1.01, got["kcentroids"].float() * 0.99
    a = co_cluster_tokens_full(q, k, qn, kn, 2, init_q_centroids=qc0, init_k_centroids=kc0)
    b = co_cluster_tokens_full(q.to(torch.bfloat16), k.to(torch.bfloat16), qn, kn, 2,
                               init_q_centroids=qc0.to(torch.bfloat16), init_k_centroids=kc0.to(torch.bfloat16))
    assert torch.equal(a["qlabels"], b["qlabels"]) and torch.equal(a["klabels"], b["klabels"])


@pytest.mark.parametrize("n,qn,kn", [(30, 20, 8), (3000, 24, 80)])
def test_co_cluster_final_sorts_are_stable_sorts_of_the_labels(gpu, n, qn, kn):
    """The last step of the co-clustering sorts both sides' final labels: as one set of launches when the query
    side's chunk counts fit the change list's buffer (n = 3000), one sort after the other when they do not
    (n = 30).  Either way sizes, offsets and sorted indices are those of a stable sort of the returned labels."""
    from svoo_amd.co_clustering import co_cluster_tokens_full

    say("co_cluster final sorts", n, qn, kn)
    bh = 2
    q, k = _rand((bh, n, 128), torch.bfloat16, 11, gpu), _rand((bh, n, 128), torch.bfloat16, 12, gpu)
    g = torch.Generator(device=gpu).manual_seed(7)
    qi = torch.stack([torch.randperm(n, device=gpu, generator=g)[:qn] for _ in range(bh)])
    ki = torch.stack([torch.randperm(n, device=gpu, generator=g)[:kn] for _ in range(bh)])
    r = co_cluster_tokens_full(q, k, qn, kn, 3, init_q_idx=qi, init_k_idx=ki)
    for side, c in (("q", qn), ("k", kn)):
        lab = r[f"{side}labels"].cpu().numpy().astype(np.int64)
        for b in range(bh):
            sizes = np.bincount(lab[b], minlength=c)
            np.testing.assert_array_equal(r[f"{side}sizes"][b].cpu().numpy(), sizes)
            np.testing.assert_array_equal(r[f"{side}_offsets"][b].cpu().numpy(),
                                          np.concatenate([[0], np.cumsum(sizes)[:-1]]))
            np.testing.assert_array_equal(r[f"{side}_sorted_idx"][b].cpu().numpy(),
                                          np.argsort(lab[b], kind="stable"))


def _clusters(b, h, s, qn, kn, seed):
    r = np.random.default_rng(seed)

    def sizes(c):
        cuts = np.sort(r.integers(0, s + 1, size=(b * h, c - 1)), axis=1)
        return np.diff(np.concatenate([np.zeros((b * h, 1), int), cuts, np.full((b * h, 1), s)], axis=1), axis=1)

    qs, ks = sizes(qn).reshape(b, h, qn), sizes(kn).reshape(b, h, kn)
    m = r.random((b, h, qn, kn)) < 0.35
    m[..., 0] = True
    return torch.from_numpy(m), torch.from_numpy(qs).int(), torch.from_numpy(ks).int()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_attention_ops_on_rounded_inputs(gpu, dtype):
    from svoo_amd.co_clustering import (block_mask_lengths, centroid_scores, dynamic_block_sparse_fwd,
                                        dynamic_block_sparse_fwd_fused, weighted_softmax)
    from svoo_amd.ear import dynamic_block_sparse_prune_fwd, identify_dynamic_map_estimated

    say("attention, mask and EAR operators", dtype)
    b, h, s, d, qn, kn = 1, 3, 1500, 128, 12, 40
    q, k, v = (_rand((b, h, s, d), dtype, 10 + i, gpu) for i in range(3))
    qb, kb, vb = (x.to(torch.bfloat16) for x in (q, k, v))
    m, qs, ks = _clusters(b, h, s, qn, kn, 3)
    m, qs, ks = m.to(gpu), qs.to(gpu), ks.to(gpu)
    out = dynamic_block_sparse_fwd(q, k, v, m, qs, ks)
    assert out.dtype == dtype
    _same_bits(out, dynamic_block_sparse_fwd(qb, kb, vb, m, qs, ks).to(dtype))
    perm = torch.stack([torch.randperm(s, generator=torch.Generator().manual_seed(7 + i)) for i in range(b * h)])
    perm = perm.int().to(gpu)
    out = dynamic_block_sparse_fwd_fused(q, k, v, m, qs, ks, perm, perm.flip(-1).contiguous())
    _same_bits(out, dynamic_block_sparse_fwd_fused(qb, kb, vb, m, qs, ks, perm, perm.flip(-1).contiguous()).to(dtype))

    qc, kc, vc = (_rand((b, h, n_, d), dtype, 20 + i, gpu) for i, n_ in enumerate((qn, kn, kn)))
    qcb, kcb, vcb = (x.to(torch.bfloat16) for x in (qc, kc, vc))
    _same_bits(centroid_scores(qc, kc), centroid_scores(qcb, kcb))
    dm, ln = block_mask_lengths(qc, kc, qs, ks, 0.9, [0.1] * h)
    dmb, lnb = block_mask_lengths(qcb, kcb, qs, ks, 0.9, [0.1] * h)
    assert torch.equal(dm, dmb) and torch.equal(ln, lnb)
    sc = centroid_scores(qcb, kcb).to(dtype)
    _same_bits(weighted_softmax(sc, ks[:, :, None, :].float()),
               weighted_softmax(sc.to(torch.bfloat16), ks[:, :, None, :].float()).to(dtype))
    em = identify_dynamic_map_estimated(q, k, v, qs, ks, qc, kc, vc, top_p=0.9, min_kc_ratio=0.1)
    emb = identify_dynamic_map_estimated(qb, kb, vb, qs, ks, qcb, kcb, vcb, top_p=0.9, min_kc_ratio=0.1)
    assert torch.equal(em, emb)
    out = dynamic_block_sparse_prune_fwd(q, k, v, kc, vc, em, qs, ks)
    assert out.dtype == dtype
    _same_bits(out, dynamic_block_sparse_prune_fwd(qb, kb, vb, kcb, vcb, em, qs, ks).to(dtype))


def test_c1_processor_call_in_fp32(gpu):
    """C1 as specified (fp32 Q/K/V): the Wan processor's sparse call returns fp32, equal bit for bit to the call on
    the bf16-rounded inputs (whose parity with the oracle test_gpu_configs pins)."""
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    cfg = synth.CONFIGS["C1"]
    h, n = cfg.heads, cfg.tokens
    qn, kn, iters = cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters
    q, k, v = (x.to(gpu) for x in synth.make_qkv(cfg))
    assert q.dtype == torch.float32
    qi = synth.init_indices(cfg, h, qn, n, 1).to(gpu)
    ki = synth.init_indices(cfg, h, kn, n, 2).to(gpu)

    def call(qq, kk, vv):
        class P(WanAttn_SAPAttn_Processor):
            pass

        P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
        P.num_q_centroids, P.num_k_centroids = qn, kn
        P.top_p_kmeans, P.min_kc_ratio, P.max_kc_ratio = 0.9, [0.25] * h, 0
        P.kmeans_iter_init = P.kmeans_iter_step = iters
        P.first_times_fp, P.first_layers_fp = float("inf"), 0
        P.kmeans_init_idx = (qi, ki)
        return P(layer_idx=0).attention_core_logic(qq, kk, vv, None)

    say("C1 in fp32 through the Wan processor")
    out = call(q, k, v)
    ref = call(*(x.to(torch.bfloat16) for x in (q, k, v)))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and ref.dtype == torch.bfloat16
    _same_bits(out, ref.float())
