"""GPU parity of every HIP kernel against the oracle (bit-exact for integer/index/mask work,
tolerance-bounded for floating point).  Each test prints the case it runs before launching."""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O

pytestmark = pytest.mark.gpu

ATTN_MAX_ABS = 2e-2  # bf16 attention tolerance (max-abs) from the north-star contract
ATTN_MIN_COS = 0.999


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


def test_mfma_operand_layout(gpu):
    from svoo_amd import _lib

    say("mfma layout probe")
    o32 = torch.zeros(64 * 16, dtype=torch.float32, device=gpu)
    o16 = torch.zeros(64 * 4, dtype=torch.float32, device=gpu)
    _lib.call("svoo_probe_mfma_layout", o32.data_ptr(), o16.data_ptr(), _lib.stream_of(gpu))
    torch.cuda.synchronize()
    c32 = o32.cpu().numpy().reshape(64, 16)
    c16 = o16.cpu().numpy().reshape(64, 4)
    for l in range(64):
        for r in range(16):
            m, n = (r // 4) * 8 + (l // 32) * 4 + r % 4, l % 32
            assert c32[l, r] == 64 * m + n, (l, r, c32[l, r])
        for r in range(4):
            m, n = 4 * (l // 16) + r, l % 16
            assert c16[l, r] == 16 * m + n, (l, r, c16[l, r])


def test_mfma_f64_operand_layout(gpu):
    from svoo_amd import _lib

    say("mfma f64 layout probe")
    o = torch.zeros(64 * 4, dtype=torch.float64, device=gpu)
    _lib.call("svoo_probe_mfma_f64_layout", o.data_ptr(), _lib.stream_of(gpu))
    torch.cuda.synchronize()
    c = o.cpu().numpy().reshape(64, 4)
    want = np.array([[64 * (4 * r + l // 16) + l % 16 for r in range(4)] for l in range(64)], np.float64)
    assert np.array_equal(c, want), c.tolist()


@pytest.mark.parametrize("bh,n,k", [(3, 5000, 37), (2, 1024, 1), (1, 1, 1), (2, 777, 2000), (4, 2049, 1000)])
def test_cluster_sort_bit_exact(gpu, bh, n, k):
    from svoo_amd.permute import cluster_sort

    say("cluster_sort", bh, n, k)
    r = np.random.default_rng(n + k)
    labels = r.integers(0, k, size=(bh, n))
    idx, sizes, offs, slab = cluster_sort(torch.from_numpy(labels).to(gpu), k, with_sorted_labels=True)
    oidx, osz, ooff = O.cluster_sort(labels, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_array_equal(sizes.cpu().numpy(), osz)
    np.testing.assert_array_equal(offs.cpu().numpy(), ooff)
    np.testing.assert_array_equal(slab.cpu().numpy(), np.take_along_axis(labels, oidx.astype(np.int64), 1))


@pytest.mark.parametrize("d", [128, 32, 256])  # rows of 256 B (one step per block), 64 B, 512 B
def test_permute_unpermute_bit_exact(gpu, d):
    from svoo_amd.permute import (apply_inverse_permutation, apply_inverse_permutation_bshd,
                                  permute_pair_by_indices, permute_tensor_by_labels)

    say("permute 1x3x3001x", d)
    x, xt = rand_bf16((1, 3, 3001, d), 1, gpu)
    v, vt = rand_bf16((1, 3, 3001, d), 2, gpu)
    labels = np.random.default_rng(3).integers(0, 50, size=(3, 3001))
    y, idx = permute_tensor_by_labels(xt, torch.from_numpy(labels).to(gpu), 2)
    oidx, _, _ = O.cluster_sort(labels, 50)
    np.testing.assert_array_equal(idx.cpu().numpy(), oidx)
    np.testing.assert_array_equal(f32(y)[0], O.permute_rows(x[0], oidx))
    ky, vy = permute_pair_by_indices(xt, vt, idx)
    assert torch.equal(ky, y)
    np.testing.assert_array_equal(f32(vy)[0], O.permute_rows(v[0], oidx))
    back = apply_inverse_permutation(y, idx, 2)
    assert torch.equal(back, xt)
    bshd = apply_inverse_permutation_bshd(y, idx)
    assert torch.equal(bshd, xt.transpose(1, 2).flatten(2, 3))
    # given sorted indices, labels are ignored
    y2, idx2 = permute_tensor_by_labels(xt, None, 2, sorted_indices=idx)
    assert torch.equal(y2, y) and torch.equal(idx2, idx)


def test_centroid_update_bit_exact(gpu):
    from svoo_amd.co_clustering import centroid_update

    for bh, n, k in [(2, 3000, 100), (3, 700, 1000), (1, 64, 3)]:
        say("centroid_update", bh, n, k)
        x, xt = rand_bf16((bh, n, 128), n, gpu, scale=2.0)
        old, oldt = rand_bf16((bh, k, 128), k, gpu)
        labels = np.random.default_rng(7).integers(0, k, size=(bh, n))
        labels[0][labels[0] == 1] = 0  # cluster 1 empty in row 0
        new, cnt = centroid_update(xt, torch.from_numpy(labels).to(gpu), oldt)
        onew, ocnt = O.centroid_update(x, labels, old)
        np.testing.assert_array_equal(cnt.cpu().numpy(), ocnt)
        np.testing.assert_array_equal(f32(new), onew)


def test_l2norm(gpu):
    from svoo_amd.co_clustering import triton_l2norm_forward

    say("l2norm")
    x, xt = rand_bf16((3, 100, 1000), 5, gpu)
    y = triton_l2norm_forward(xt, 1e-8)
    np.testing.assert_allclose(f32(y), O.l2norm_rows(x), rtol=2e-6, atol=1e-7)


def test_profile_prep(gpu):
    from svoo_amd.co_clustering import cocluster_profile

    for j, kp in [(1000, 100), (100, 1000), (70, 33), (5, 1800), (300, 520), (3, 3900)]:
        say("cocluster_prep", j, kp)
        a, at = rand_bf16((2, j, 128), j, gpu)
        b, btt = rand_bf16((2, kp, 128), kp + 1, gpu)
        prof, e_hi, e_lo = cocluster_profile(at, btt)
        ref = O.profile_centroids(a, b)
        np.testing.assert_allclose(f32(prof), ref, rtol=1e-6, atol=1e-7)
        e = (e_hi.double() + e_lo.double()).cpu().numpy()[:, :j]
        e_ref = ref @ b.astype(np.float64)
        scale = np.abs(e_ref).max()
        assert np.abs(e - e_ref).max() <= 3e-5 * scale
        # padding rows repeat row j - 1 (a padding row can only tie with it in the assignment)
        assert torch.equal(e_hi[:, j:], e_hi[:, j - 1 : j].expand_as(e_hi[:, j:]))
        assert torch.equal(e_lo[:, j:], e_lo[:, j - 1 : j].expand_as(e_lo[:, j:]))


def test_assign_matches_literal_argmin(gpu):
    from svoo_amd.co_clustering import cocluster_assign

    for n, j, kp in [(5000, 1000, 100), (4000, 100, 1000), (333, 7, 5)]:
        say("cocluster_assign", n, j, kp)
        x, xt = rand_bf16((2, n, 128), n, gpu)
        cent, ct = rand_bf16((2, j, 128), j + 7, gpu)
        basis, bt = rand_bf16((2, kp, 128), kp + 9, gpu)
        lab = cocluster_assign(xt, ct, bt).cpu().numpy()
        ref, margin = O.cocluster_assign(x, basis, O.profile_centroids(cent, basis))
        diff = lab != ref
        # a mismatch is allowed only at a near-tie of the literal distance
        assert np.all(margin[diff] < 1e-4), (diff.sum(), margin[diff].max() if diff.any() else None)
        assert diff.mean() < 1e-3



@pytest.mark.parametrize("cfg_name,heads,zero01", [("C3", 4, False), ("C2", 3, False), ("C4", 2, False),
                                                   ("C2", 3, True)])
def test_certified_fp16_pass_equals_hi_lo_labels(gpu, cfg_name, heads, zero01):
    """Inside svoo_co_cluster the assignment runs one fp16 MFMA pass and certifies a label when the best score
    beats the second by more than twice a rigorous error bound; the other tokens go to the hi + lo kernel.
    One iteration from seeded starts: the key labels equal the hi + lo kernel's (svoo_cocluster_assign) on the
    initial centroids, and the query labels equal it in the space of the updated key centroids.

    With zero01 the token components d = 0, 1 (mod 8) are zero: the bound scales with the token norm, and a
    norm taken from those components alone (the first 32-bit word of each 16-byte operand) is zero, which
    certifies every near-tie the fp16 rounding can flip."""
    from svoo_amd import synth
    from svoo_amd.co_clustering import cocluster_assign, co_cluster_tokens_full

    cfg = synth.CONFIGS[cfg_name]
    say("certified fp16 pass vs hi+lo labels", cfg_name, heads, "zero d%8 in {0,1}" if zero01 else "")
    q, k, _ = synth.make_qkv_device(cfg, gpu)
    nv = cfg.video_tokens
    q, k = q[0, :heads, :nv].contiguous(), k[0, :heads, :nv].contiguous()
    if zero01:
        dims = torch.arange(128, device=gpu)
        keep = ((dims % 8) >= 2).to(q.dtype)
        q, k = (q * keep).contiguous(), (k * keep).contiguous()
    qi = synth.init_indices(cfg, heads, cfg.num_q_centroids, nv, 1).to(gpu)
    ki = synth.init_indices(cfg, heads, cfg.num_k_centroids, nv, 2).to(gpu)
    r = co_cluster_tokens_full(q, k, cfg.num_q_centroids, cfg.num_k_centroids, 1, init_q_idx=qi, init_k_idx=ki)
    qc0 = torch.gather(q, 1, qi[:, :, None].expand(-1, -1, 128))
    kc0 = torch.gather(k, 1, ki[:, :, None].expand(-1, -1, 128))
    klab = cocluster_assign(k, kc0, qc0)
    qlab = cocluster_assign(q, qc0, r["kcentroids"])
    torch.cuda.synchronize()
    assert torch.equal(r["klabels"], klab)
    assert torch.equal(r["qlabels"], qlab)

def test_weighted_softmax_bit_exact(gpu):
    from svoo_amd.co_clustering import weighted_softmax

    say("weighted_softmax")
    s, st = rand_bf16((2, 3, 7, 1000), 11, gpu, scale=3.0)
    w = np.random.default_rng(12).integers(0, 200, size=(2, 3, 1, 1000)).astype(np.float32)
    out = weighted_softmax(st, torch.from_numpy(w).to(gpu))
    ref = O.weighted_softmax(s, np.broadcast_to(w, s.shape))
    np.testing.assert_array_equal(f32(out), ref)


def _mask_case(gpu, h, qn, kn, seed):
    r = np.random.default_rng(seed)
    qc = O.bf16_round((r.standard_normal((1, h, qn, 128)) * 0.5).astype(np.float32))
    kc = O.bf16_round((r.standard_normal((1, h, kn, 128)) * 0.5).astype(np.float32))
    qs = r.integers(1, 400, size=(1, h, qn)).astype(np.int32)
    ks = r.integers(0, 200, size=(1, h, kn)).astype(np.int32)
    return (qc, kc, qs, ks), (bf16(qc, gpu), bf16(kc, gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu))


@pytest.mark.parametrize("p,mn,mx", [
    (0.9, [0.15, 0.2, 0.18], 0), (0.0, [0.05, 0.3, 0.17], 0), (0.5, 0.2, 0), (0.88, 0, [0.1, 0.0, 0.05]),
    (0.97, 0.0, 0.15), (1.0, 0, 0), (0.3, 0.7, 0),
])
@pytest.mark.parametrize("qn,kn", [(100, 1000), (20, 300), (7, 2500)])
def test_block_mask_bit_exact(gpu, p, mn, mx, qn, kn):
    from svoo_amd.co_clustering import block_mask_lengths

    say("block_mask", p, mn, mx, qn, kn)
    (qc, kc, qs, ks), (qct, kct, qst, kst) = _mask_case(gpu, 3, qn, kn, qn * kn)
    m, lens = block_mask_lengths(qct, kct, qst, kst, p, mn, mx)
    om, olens = O.identify_dynamic_map(qc, kc, qs, ks, p, mn, mx, return_lengths=True)
    np.testing.assert_array_equal(m.cpu().numpy(), om)
    np.testing.assert_array_equal(lens.cpu().numpy(), olens)


def _score_cases():
    """(name, qc, kc) float32 arrays of bf16 values [1, H, n, 128] for the centroid-score kernel."""
    r = np.random.default_rng(77)
    cases = []
    for scale in (0.05, 0.5, 30.0):
        qc = O.bf16_round((r.standard_normal((1, 3, 100, 128)) * scale).astype(np.float32))
        kc = O.bf16_round((r.standard_normal((1, 3, 1000, 128)) * scale).astype(np.float32))
        cases.append((f"gaussian x{scale}", qc, kc))
    # small integers: dots are exact in fp32, many land on bf16 rounding midpoints (ties to even)
    qi = r.integers(-4, 5, size=(1, 2, 37, 128)).astype(np.float32)
    ki = r.integers(-4, 5, size=(1, 2, 301, 128)).astype(np.float32)
    cases.append(("small integers", qi, ki))
    # subnormal bf16 entries next to large ones; overflowing products; zero rows
    qs = O.bf16_round((r.standard_normal((1, 1, 40, 128))).astype(np.float32))
    ks = O.bf16_round((r.standard_normal((1, 1, 70, 128))).astype(np.float32))
    qs[0, 0, :5, :3] = np.float32(3e-39)
    ks[0, 0, 7, 10:20] = np.float32(-1.5e-39)
    qs[0, 0, 6, 0] = np.float32(1e30)
    ks[0, 0, 8, 0] = np.float32(2e25)
    qs[0, 0, 9] = 0.0
    ks[0, 0, 11] = 0.0
    cases.append(("subnormal / large / zero", O.bf16_round(qs), O.bf16_round(ks)))
    return cases


@pytest.mark.parametrize("case", range(5))
def test_centroid_scores_bit_exact(gpu, case):
    """bf16(bf16(Qc.Kc^T) * f32(1/sqrt(D))) from the certified MFMA pass (with its exact fp64 fallback) equals the
    oracle's exact-dot scores bit for bit, on Gaussian centroids, integer dots on bf16 midpoints, bf16
    subnormals, large values and zero rows."""
    from svoo_amd.co_clustering import centroid_scores
    from svoo_amd.ear import centroid_logits

    name, qc, kc = _score_cases()[case]
    say("centroid scores", name, qc.shape, kc.shape)
    got = centroid_scores(bf16(qc, gpu), bf16(kc, gpu))
    want = O.centroid_scores(qc, kc)
    np.testing.assert_array_equal(O.bf16_bits(f32(got)), O.bf16_bits(want))
    assert torch.equal(centroid_logits(bf16(qc, gpu), bf16(kc, gpu)), got)  # EAR's logits are the same values


def _attn_check(out, ref):
    o = f32(out).astype(np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    err = np.abs(o - r).max()
    cos = float(o @ r / (np.linalg.norm(o) * np.linalg.norm(r) + 1e-30))
    assert err <= ATTN_MAX_ABS and cos >= ATTN_MIN_COS, (err, cos)
    return err, cos


@pytest.mark.parametrize("h,qn,kn,s,density,seed", [
    (2, 12, 40, 3000, 0.3, 1), (1, 5, 9, 700, 0.6, 2), (3, 30, 200, 4096, 0.1, 3), (2, 4, 4, 333, 1.0, 4),
])
def test_vbsa_matches_oracle(gpu, h, qn, kn, s, density, seed):
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    say("vbsa", h, qn, kn, s, density)
    r = np.random.default_rng(seed)

    def sizes(c):
        cuts = np.sort(r.integers(0, s + 1, size=(h, c - 1)), axis=1)
        z = np.concatenate([np.zeros((h, 1), int), cuts, np.full((h, 1), s)], axis=1)
        return np.diff(z, axis=1).astype(np.int32)[None]

    qs, ks = sizes(qn), sizes(kn)
    m = r.random((1, h, qn, kn)) < density
    m[0, 0, 0, :] = False  # an empty row
    q, qt = rand_bf16((1, h, s, 128), seed, gpu)
    k, kt = rand_bf16((1, h, s, 128), seed + 1, gpu)
    v, vt = rand_bf16((1, h, s, 128), seed + 2, gpu)
    out = dynamic_block_sparse_fwd(qt, kt, vt, torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu),
                                   torch.from_numpy(ks).to(gpu))
    ref = O.block_sparse_attention(q, k, v, m, qs, ks)
    _attn_check(out, ref)
    a = int(qs[0, 0, 0])
    assert torch.all(out[0, 0, :a] == 0)


def _half_item_case(kn, r, h=2):
    """Query cluster sizes around the 128 / 256 item boundaries (last tiles of 1 to 128 queries become half
    items), random key cuts and per-row map densities from one short cluster to all-true."""
    qsz = np.array([1, 31, 32, 33, 100, 128, 129, 255, 256, 257, 300, 384, 385, 640, 700], np.int32)
    s = int(qsz.sum())
    qs = np.stack([qsz, qsz[::-1]])[None]
    cuts = np.sort(np.stack([r.choice(np.arange(1, s), size=kn - 1, replace=False) for _ in range(h)]), axis=1)
    ks = np.diff(np.concatenate([np.zeros((h, 1), int), cuts, np.full((h, 1), s)], axis=1), axis=1).astype(np.int32)
    ks = ks[None]
    qn = len(qsz)
    m = np.zeros((1, h, qn, kn), bool)
    for b in range(h):
        small = int(np.argmin(ks[0, b]))
        for i in range(qn):
            mode = (i + b) % 5
            if mode == 0:
                m[0, b, i, small] = True  # one short cluster: a single KV tile
            else:
                m[0, b, i] = r.random(kn) < (0.05, 0.15, 0.4, 1.0)[mode - 1]
                m[0, b, i, small] = True
    return h, s, qs, ks, m


@pytest.mark.parametrize("ear,kn", [(False, 24), (True, 24), (True, 2000)])
def test_vbsa_half_items_match_oracle(gpu, ear, kn):
    """Query clusters whose last 256-query tile holds at most 128 queries (the kernel splits such a
    tile's KV stream over its two wave groups and merges the two softmax states), for KV streams of
    1 to several 64-key tiles.  kn = 2000 with EAR leaves no LDS for the second stream: the same
    sizes then run as full items."""
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd
    from svoo_amd.ear import dynamic_block_sparse_prune_fwd

    say("vbsa half items", "ear" if ear else "sap", kn)
    r = np.random.default_rng(40 + kn)
    h, s, qs, ks, m = _half_item_case(kn, r)
    q, qt = rand_bf16((1, h, s, 128), 41, gpu, 0.5)
    k, kt = rand_bf16((1, h, s, 128), 42, gpu, 0.5)
    v, vt = rand_bf16((1, h, s, 128), 43, gpu)
    mt, qst, kst = torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    if ear:
        kc, kct = rand_bf16((1, h, kn, 128), 44, gpu, 0.5)
        vc, vct = rand_bf16((1, h, kn, 128), 45, gpu)
        out = dynamic_block_sparse_prune_fwd(qt, kt, vt, kct, vct, mt, qst, kst)
        ref = O.ear_compensated_attention(q, k, v, kc, vc, m, qs, ks)
    else:
        out = dynamic_block_sparse_fwd(qt, kt, vt, mt, qst, kst)
        ref = O.block_sparse_attention(q, k, v, m, qs, ks)
    _attn_check(out, ref)


_BCHUNK_QSZ = (129, 150, 160, 161, 180, 192, 193, 385, 448, 650, 1, 64, 128, 256)
_BCHUNK_LEN = (0, 1, 5, 31, 32, 33, 63, 64, 65, 96, 97, 127, 128, 129, 160, 191, 192, 193, 255, 256, 257, 700)


def _b_chunked_case(r, h=4):
    """Last tiles of 129 to 192 queries (group B's two waves per 32 queries take the two 32-key halves of every
    tile) next to half, full and larger items.  Key clusters of one token each make a map row's stream exactly
    as long as the number of clusters it selects: lengths on both sides of every 32-key chunk edge, 0 (an empty
    row) and the whole sequence."""
    qsz = np.array(_BCHUNK_QSZ, np.int32)
    s = int(qsz.sum())
    qn, kn = len(qsz), s
    qs = np.stack([qsz, qsz[::-1], np.roll(qsz, 5), np.roll(qsz[::-1], 9)][:h])[None]
    ks = np.ones((1, h, kn), np.int32)
    m = np.zeros((1, h, qn, kn), bool)
    lens = _BCHUNK_LEN + (kn,)
    for b in range(h):
        for i in range(qn):
            m[0, b, i, r.choice(kn, size=lens[(i + 9 * b) % len(lens)], replace=False)] = True
    return h, s, qs, ks, m


def test_vbsa_b_chunked_items_match_oracle(gpu):
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    say("vbsa B-chunked items")
    r = np.random.default_rng(100)
    h, s, qs, ks, m = _b_chunked_case(r)
    q, qt = rand_bf16((1, h, s, 128), 101, gpu, 0.5)
    k, kt = rand_bf16((1, h, s, 128), 102, gpu, 0.5)
    v, vt = rand_bf16((1, h, s, 128), 103, gpu)
    mt, qst, kst = torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    out = dynamic_block_sparse_fwd(qt, kt, vt, mt, qst, kst)
    ref = O.block_sparse_attention(q, k, v, m, qs, ks)
    _attn_check(out, ref)
    # per query cluster, so that a wrong cluster cannot hide in the whole tensor's cosine
    o = f32(out)
    for b in range(h):
        off = np.concatenate([[0], np.cumsum(qs[0, b])])
        for i in range(qs.shape[-1]):
            a, e = int(off[i]), int(off[i + 1])
            got, want = o[0, b, a:e].astype(np.float64), np.asarray(ref[0, b, a:e], np.float64)
            assert np.abs(got - want).max(initial=0.0) <= ATTN_MAX_ABS, (b, i, e - a, int(m[0, b, i].sum()))
            if not m[0, b, i].any():
                assert np.all(got == 0), (b, i)


def test_fused_b_chunked_items_equal_separate_passes(gpu):
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd, dynamic_block_sparse_fwd_fused
    from svoo_amd.permute import apply_inverse_permutation_bshd, permute_pair_by_indices
    from svoo_amd.processor import _permute_rows

    say("fused vbsa B-chunked items")
    r = np.random.default_rng(105)
    h, s, qs, ks, m = _b_chunked_case(r)
    qi = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(gpu)
    ki = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(gpu)
    _, q = rand_bf16((1, h, s, 128), 106, gpu, 0.5)
    _, k = rand_bf16((1, h, s, 128), 107, gpu, 0.5)
    _, v = rand_bf16((1, h, s, 128), 108, gpu)
    mt, qst, kst = torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    out = dynamic_block_sparse_fwd_fused(q, k, v, mt, qst, kst, qi, ki)
    qp = _permute_rows(q, qi)
    kp, vp = permute_pair_by_indices(k, v, ki)
    ref = apply_inverse_permutation_bshd(dynamic_block_sparse_fwd(qp, kp, vp, mt, qst, kst), qi)
    assert torch.equal(out, ref)


def test_vbsa_dense_equals_sdpa(gpu):
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    say("vbsa dense vs sdpa")
    h, s = 4, 2048
    q, qt = rand_bf16((1, h, s, 128), 21, gpu)
    k, kt = rand_bf16((1, h, s, 128), 22, gpu)
    v, vt = rand_bf16((1, h, s, 128), 23, gpu)
    qs = torch.full((1, h, 1), s, dtype=torch.int32, device=gpu)
    m = torch.ones(1, h, 1, 1, dtype=torch.bool, device=gpu)
    out = dynamic_block_sparse_fwd(qt, kt, vt, m, qs, qs)
    ref = torch.nn.functional.scaled_dot_product_attention(qt.float(), kt.float(), vt.float())
    _attn_check(out, ref.cpu().numpy())


def test_vbsa_rejects_inconsistent_sizes(gpu):
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd_triton

    say("vbsa bad sizes")
    _, qt = rand_bf16((1, 1, 64, 128), 1, gpu)
    qs = torch.tensor([[[30, 30]]], dtype=torch.int32, device=gpu)  # sums to 60 != 64
    m = torch.ones(1, 1, 2, 2, dtype=torch.bool, device=gpu)
    with pytest.raises(AssertionError):
        dynamic_block_sparse_fwd_triton(qt, qt, qt, m, qs, qs)
    with pytest.raises(AssertionError):  # sizes on the host are checked before any launch
        dynamic_block_sparse_fwd_triton(qt, qt, qt, m, qs.cpu(), qs)


def test_vbsa_fills_heads_with_inconsistent_sizes_with_nan(gpu):
    """Without the host check (the processors' path: no read-back), a head whose sizes do not sum to S
    comes back as NaN in every row, on the separate and the fused kernel; the other heads are computed."""
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd, dynamic_block_sparse_fwd_fused

    say("vbsa bad sizes in one of two heads -> NaN rows")
    s = 300
    q, qt = rand_bf16((1, 2, s, 128), 11, gpu)
    k, kt = rand_bf16((1, 2, s, 128), 12, gpu)
    v, vt = rand_bf16((1, 2, s, 128), 13, gpu)
    qs = np.array([[[100, 200], [100, 200]]], np.int32)
    ks = np.array([[[150, 150], [150, 140]]], np.int32)  # head 1: 290 != 300
    m = np.ones((1, 2, 2, 2), bool)
    qst, kst, mt = torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu), torch.from_numpy(m).to(gpu)
    out = dynamic_block_sparse_fwd(qt, kt, vt, mt, qst, kst, validate=False)
    torch.cuda.synchronize()
    assert torch.isnan(out[0, 1]).all()
    assert not torch.isnan(out[0, 0]).any()
    _attn_check(out[:, :1], O.block_sparse_attention(q[:, :1], k[:, :1], v[:, :1], m[:, :1], qs[:, :1], ks[:, :1]))
    ident = torch.arange(s, dtype=torch.int32, device=gpu).expand(2, s).contiguous()
    fused = dynamic_block_sparse_fwd_fused(qt, kt, vt, mt, qst, kst, ident, ident, validate=False)
    torch.cuda.synchronize()
    fo = fused.view(s, 2, 128)
    assert torch.isnan(fo[:, 1]).all()
    assert torch.equal(fo[:, 0], out[0, 0])


def _many_heads_case(bh, s, seed):
    """bh heads of s tokens with 1 to 3 non-empty query clusters, random maps (so the heads' work and launch
    ranks differ) and, on every 37th head, key sizes that do not sum to S."""
    r = np.random.default_rng(seed)
    patterns = np.array([[s, 0, 0], [s // 2, s - s // 2, 0], [1, 1, s - 2], [0, s, 0], [13, 14, s - 27]], np.int32)
    qs = patterns[r.integers(0, len(patterns), bh)][None]
    cut = r.integers(1, s, bh)
    ks = np.stack([cut, s - cut], axis=1).astype(np.int32)[None]
    bad = np.arange(bh) % 37 == 5
    ks[0, bad, 1] -= 1
    m = r.random((1, bh, 3, 2)) < 0.6
    m[..., r.integers(0, 2)] = True
    return qs, ks, m, bad


@pytest.mark.parametrize("bh", [300, 4100])
def test_vbsa_work_list_over_many_heads(gpu, bh):
    """The work list the order kernel builds: heads ranked by work in chunks of 256 (bh = 300), or in their
    own order past 4096 heads (bh = 4100), each contributing its items, or NaN-filling slots when its sizes
    do not sum to S, with no slot lost or repeated."""
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    s = 40
    say("vbsa work list over", bh, "heads")
    qs, ks, m, bad = _many_heads_case(bh, s, 60 + bh)
    q, qt = rand_bf16((1, bh, s, 128), 61, gpu)
    k, kt = rand_bf16((1, bh, s, 128), 62, gpu)
    v, vt = rand_bf16((1, bh, s, 128), 63, gpu)
    mt, qst, kst = torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    out = dynamic_block_sparse_fwd(qt, kt, vt, mt, qst, kst, validate=False)
    torch.cuda.synchronize()
    o = out[0]
    assert torch.isnan(o[torch.from_numpy(bad).to(gpu)]).all()
    good = ~bad
    assert not torch.isnan(o[torch.from_numpy(good).to(gpu)]).any()
    # the oracle on every good head at bh = 300, on every 13th of 4100
    pick = good & (np.arange(bh) % (1 if bh < 1000 else 13) == 0)
    ref = O.block_sparse_attention(q[:, pick], k[:, pick], v[:, pick], m[:, pick], qs[:, pick], ks[:, pick])
    _attn_check(out[:, torch.from_numpy(pick).to(gpu)], ref)


def test_vbsa_many_query_clusters_keep_cluster_order(gpu):
    """A head with more than 4096 query clusters is planned in cluster order (the longest-first sort covers
    up to 4096): one head of 5000 clusters, most of 1-3 queries (half items), a few of 150-700 (B-chunked, full
    and half last tiles), against the oracle."""
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd

    say("vbsa 5000 query clusters")
    r = np.random.default_rng(81)
    qn, kn = 5000, 24
    qsz = r.integers(1, 4, qn).astype(np.int32)
    qsz[[7, 1000, 2500, 4000, 4999]] = [150, 420, 700, 300, 192]
    s = int(qsz.sum())
    cuts = np.sort(r.choice(np.arange(1, s), size=kn - 1, replace=False))
    ks = np.diff(np.concatenate([[0], cuts, [s]])).astype(np.int32)[None, None]
    qs = qsz[None, None]
    m = r.random((1, 1, qn, kn)) < 0.3
    m[..., 0] = True
    q, qt = rand_bf16((1, 1, s, 128), 82, gpu)
    k, kt = rand_bf16((1, 1, s, 128), 83, gpu)
    v, vt = rand_bf16((1, 1, s, 128), 84, gpu)
    mt, qst, kst = torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    out = dynamic_block_sparse_fwd(qt, kt, vt, mt, qst, kst)
    _attn_check(out, O.block_sparse_attention(q, k, v, m, qs, ks))


def test_vbsa_segments_expand_to_reference_plan(gpu):
    from svoo_amd.co_clustering import vbsa_segments

    say("vbsa segments")
    r = np.random.default_rng(8)
    bh, qn, kn = 3, 6, 50
    m = r.random((bh, qn, kn)) < 0.3
    cs = r.integers(0, 9, size=(bh, kn)).astype(np.int32)
    start, length, count = vbsa_segments(torch.from_numpy(m).to(gpu), torch.from_numpy(cs).to(gpu))
    start, length, count = start.cpu().numpy(), length.cpu().numpy(), count.cpu().numpy()
    indptr, ind = O.kv_plan_indices(m, cs)
    head_off = np.concatenate([[0], np.cumsum(cs.sum(1))[:-1]])
    row = 0
    for b in range(bh):
        for i in range(qn):
            toks = [np.arange(start[b, i, c], start[b, i, c] + length[b, i, c]) for c in range(count[b, i])]
            toks = np.concatenate(toks) if toks else np.zeros(0, int)
            np.testing.assert_array_equal(toks + head_off[b], ind[indptr[row]:indptr[row + 1]])
            row += 1


def test_golden_small_end_to_end(gpu):
    """Co-clustering, mask and attention of the committed small case through the C ABI."""
    from svoo_amd.co_clustering import block_mask_lengths, co_cluster_tokens_full, dynamic_block_sparse_fwd
    from svoo_amd.permute import permute_pair_by_indices
    from tests.golden.make_golden import MASK_CASES, SMALL, small_inputs
    from pathlib import Path

    say("golden small end to end")
    g = np.load(Path(__file__).parent / "golden" / "golden_small.npz")
    qb, kb, vb, qi, ki = small_inputs()
    to_t = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(gpu)  # noqa: E731
    q, k, v = to_t(qb), to_t(kb), to_t(vb)
    r = co_cluster_tokens_full(q, k, SMALL.num_q_centroids, SMALL.num_k_centroids, SMALL.kmeans_iters,
                               init_q_idx=torch.from_numpy(qi).to(gpu), init_k_idx=torch.from_numpy(ki).to(gpu))
    ql, kl = r["qlabels"].cpu().numpy(), r["klabels"].cpu().numpy()
    # well-separated synthetic mixture: the labels must match the oracle exactly
    np.testing.assert_array_equal(ql, g["qlabels"])
    np.testing.assert_array_equal(kl, g["klabels"])
    np.testing.assert_array_equal(r["qcentroids"].view(torch.int16).cpu().numpy().view(np.uint16), g["qcent"])
    np.testing.assert_array_equal(r["kcentroids"].view(torch.int16).cpu().numpy().view(np.uint16), g["kcent"])
    np.testing.assert_array_equal(r["qsizes"].cpu().numpy(), g["qsizes"])
    np.testing.assert_array_equal(r["k_sorted_idx"].cpu().numpy(), g["k_sorted_idx"])
    h = SMALL.heads
    for ci, (p, mn, mx) in enumerate(MASK_CASES):
        m, lens = block_mask_lengths(r["qcentroids"][None], r["kcentroids"][None], r["qsizes"][None],
                                     r["ksizes"][None], p, mn, mx)
        np.testing.assert_array_equal(m[0].cpu().numpy(), g[f"map{ci}"])
        np.testing.assert_array_equal(lens[0].cpu().numpy(), g[f"len{ci}"])
    qp = torch.empty_like(q)
    from svoo_amd import _lib

    _lib.call("svoo_permute_rows", q.data_ptr(), r["q_sorted_idx"].data_ptr(), qp.data_ptr(), h, q.shape[1],
              q.shape[1], 256, _lib.stream_of(gpu))
    kp, vp = permute_pair_by_indices(k[None], v[None], r["k_sorted_idx"])
    m0 = torch.from_numpy(g["map0"]).to(gpu)[None]
    out = dynamic_block_sparse_fwd(qp[None], kp, vp, m0, r["qsizes"][None], r["ksizes"][None])
    _attn_check(out[0], g["out_perm"].astype(np.float64))


@pytest.mark.parametrize("h,qn,kn,s,density,seed", [(2, 12, 40, 3000, 0.3, 1), (3, 30, 200, 4096, 0.1, 3),
                                                    (2, 4, 4, 333, 1.0, 4)])
def test_fused_attention_equals_separate_passes(gpu, h, qn, kn, s, density, seed):
    """Permute + attention + inverse permutation in one kernel gives the same bits as the three passes."""
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd, dynamic_block_sparse_fwd_fused
    from svoo_amd.permute import apply_inverse_permutation_bshd, permute_pair_by_indices
    from svoo_amd.processor import _permute_rows

    say("fused vbsa", h, qn, kn, s, density)
    r = np.random.default_rng(seed)

    def sizes(c):
        cuts = np.sort(r.integers(0, s + 1, size=(h, c - 1)), axis=1)
        z = np.concatenate([np.zeros((h, 1), int), cuts, np.full((h, 1), s)], axis=1)
        return np.diff(z, axis=1).astype(np.int32)[None]

    qs, ks = sizes(qn), sizes(kn)
    m = torch.from_numpy(r.random((1, h, qn, kn)) < density).to(gpu)
    m[0, 0, 0, :] = False  # an empty row
    qi = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(gpu)
    ki = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(gpu)
    _, q = rand_bf16((1, h, s, 128), seed, gpu)
    _, k = rand_bf16((1, h, s, 128), seed + 1, gpu)
    _, v = rand_bf16((1, h, s, 128), seed + 2, gpu)
    qst, kst = torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    out = dynamic_block_sparse_fwd_fused(q, k, v, m, qst, kst, qi, ki)
    qp = _permute_rows(q, qi)
    kp, vp = permute_pair_by_indices(k, v, ki)
    ref = apply_inverse_permutation_bshd(dynamic_block_sparse_fwd(qp, kp, vp, m, qst, kst), qi)
    assert out.shape == (1, s, h * 128)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("kn", [24, 700])
def test_fused_half_items_equal_separate_passes(gpu, kn):
    """The fused kernel on half items (each wave group resolving every other table, its index loads one
    table ahead) gives the same bits as permute + attention + inverse permutation."""
    from svoo_amd.co_clustering import dynamic_block_sparse_fwd, dynamic_block_sparse_fwd_fused
    from svoo_amd.permute import apply_inverse_permutation_bshd, permute_pair_by_indices
    from svoo_amd.processor import _permute_rows

    say("fused vbsa half items", kn)
    r = np.random.default_rng(70 + kn)
    h, s, qs, ks, m = _half_item_case(kn, r)
    qi = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(gpu)
    ki = torch.from_numpy(np.stack([r.permutation(s) for _ in range(h)]).astype(np.int32)).to(gpu)
    _, q = rand_bf16((1, h, s, 128), 71, gpu, 0.5)
    _, k = rand_bf16((1, h, s, 128), 72, gpu, 0.5)
    _, v = rand_bf16((1, h, s, 128), 73, gpu)
    mt, qst, kst = torch.from_numpy(m).to(gpu), torch.from_numpy(qs).to(gpu), torch.from_numpy(ks).to(gpu)
    out = dynamic_block_sparse_fwd_fused(q, k, v, mt, qst, kst, qi, ki)
    qp = _permute_rows(q, qi)
    kp, vp = permute_pair_by_indices(k, v, ki)
    ref = apply_inverse_permutation_bshd(dynamic_block_sparse_fwd(qp, kp, vp, mt, qst, kst), qi)
    assert torch.equal(out, ref)
