"""Pins every oracle function with checks that do not restate it: library routines, closed forms,
special cases, invariants and brute force on tiny inputs (CPU only).

Pinning map (oracle function -> independent checks):
  bf16_round / bf16_bits      torch's float32 -> bfloat16 conversion; hand-picked tie cases
  cluster_sort                numpy stable argsort + bincount; edge cases (one cluster, K > N)
  permute_rows / unpermute    fancy indexing; round trip; identity labels
  centroid_update             exact rational means (fractions.Fraction); empty cluster keeps old
  l2norm_rows                 numpy.linalg.norm
  profile_centroids           unit rows; bf16-rounded matmul entries
  cocluster_assign            brute force with math.fsum; reduced form argmax x.E; K == 1
  co_cluster_tokens           well-separated mixture recovered exactly; fixed point of the update
  centroid_scores             hand-computed bf16 values of bf16(Qc.Kc^T) * fl32(1/sqrt(D)) for integer
                              dots that bf16 cannot hold; torch's CPU bf16 matmul and scalar division
  weighted_softmax            scipy softmax (unit weights); closed form w / sum(w) for equal scores
  identify_dynamic_map        p >= 1 all-true; p = 0 keeps max(1, int(r*Kc)); hand-computed top-p
                              cut; prefix property; top-1 kept; float32 ratio semantics (0.7 -> 699);
                              a hand-worked row whose kept set at p = 0.9 changes if the dot is not
                              rounded to bf16 or the scale is 1/D
  kv_plan_indices             brute force on a hand-made map
  block_sparse_attention      dense SDPA (torch, float64) for an all-true map; block-diagonal map;
                              empty row -> 0
  svoo_attention_call         one cluster + p >= 1 reduces to dense attention
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch
from scipy.special import softmax as sp_softmax

from oracle import svoo_oracle as O

RNG = np.random.default_rng(1234)


def test_bf16_round_matches_torch():
    x = np.concatenate([
        RNG.standard_normal(10000).astype(np.float32) * 10.0,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], np.float32),
    ])
    ours = O.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, ref)
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1 (even mantissa)
    assert O.bf16_round(np.float32(1.0 + 2 ** -8)) == np.float32(1.0)
    assert O.bf16_round(np.float32(1.0 + 3 * 2 ** -8)) == np.float32(1.0 + 2 ** -6)
    assert np.isnan(O.bf16_round(np.float32(np.nan)))


@pytest.mark.parametrize("bh,n,k", [(3, 1000, 7), (2, 50, 64), (1, 1, 1), (2, 300, 1)])
def test_cluster_sort_is_stable_counting_sort(bh, n, k):
    labels = RNG.integers(0, k, size=(bh, n))
    idx, sizes, offsets = O.cluster_sort(labels, k)
    for r in range(bh):
        np.testing.assert_array_equal(idx[r], np.argsort(labels[r], kind="stable"))
        np.testing.assert_array_equal(sizes[r], np.bincount(labels[r], minlength=k))
        np.testing.assert_array_equal(offsets[r], np.concatenate([[0], np.cumsum(sizes[r])[:-1]]))
        assert np.all(np.diff(labels[r][idx[r]]) >= 0)


def test_permute_unpermute_round_trip():
    x = RNG.standard_normal((2, 97, 8)).astype(np.float32)
    labels = RNG.integers(0, 5, size=(2, 97))
    idx, _, _ = O.cluster_sort(labels, 5)
    y = O.permute_rows(x, idx)
    for r in range(2):
        np.testing.assert_array_equal(y[r], x[r][idx[r]])
    np.testing.assert_array_equal(O.unpermute_rows(y, idx), x)
    ident = np.tile(np.arange(97), (2, 1))
    idx2, _, _ = O.cluster_sort(ident, 97)
    np.testing.assert_array_equal(O.permute_rows(x, idx2), x)


def test_centroid_update_exact_means():
    x = O.bf16_round(RNG.standard_normal((2, 60, 16)).astype(np.float32))
    labels = RNG.integers(0, 6, size=(2, 60))
    labels[1][labels[1] == 3] = 4  # cluster 3 of row 1 is empty
    old = O.bf16_round(RNG.standard_normal((2, 6, 16)).astype(np.float32))
    cent, cnt = O.centroid_update(x, labels, old)
    for r in range(2):
        for c in range(6):
            members = x[r][labels[r] == c]
            assert cnt[r, c] == len(members)
            if len(members) == 0:
                np.testing.assert_array_equal(cent[r, c], old[r, c])
                continue
            for d in range(16):
                s = sum(Fraction(float(v)) for v in members[:, d])
                s32 = np.float32(float(s))  # exact sum rounded once (these sums are exact in float64)
                expect = O.bf16_round(np.float32(s32 / np.float32(len(members))))
                assert cent[r, c, d] == expect


def test_l2norm_rows():
    x = RNG.standard_normal((5, 33))
    np.testing.assert_allclose(O.l2norm_rows(x, 0.0), x / np.linalg.norm(x, axis=1, keepdims=True), rtol=1e-14)
    z = np.zeros((1, 4))
    np.testing.assert_array_equal(O.l2norm_rows(z), z)


def test_profile_centroids_unit_rows_and_bf16_entries():
    a = O.bf16_round(RNG.standard_normal((1, 9, 128)).astype(np.float32))
    b = O.bf16_round(RNG.standard_normal((1, 5, 128)).astype(np.float32))
    p = O.profile_centroids(a, b)
    np.testing.assert_allclose(np.linalg.norm(p, axis=-1), 1.0, rtol=1e-9)
    raw = torch.from_numpy(a).double() @ torch.from_numpy(b).double().transpose(-1, -2)
    raw_bf = raw.float().to(torch.bfloat16).double().numpy()
    np.testing.assert_allclose(p * np.linalg.norm(raw_bf, axis=-1, keepdims=True), raw_bf, rtol=1e-7, atol=1e-6)


def test_cocluster_assign_brute_force_and_reduced_form():
    x = O.bf16_round(RNG.standard_normal((1, 40, 128)).astype(np.float32))
    c = O.bf16_round(RNG.standard_normal((1, 6, 128)).astype(np.float32))
    cent = O.bf16_round(RNG.standard_normal((1, 9, 128)).astype(np.float32))
    p = O.profile_centroids(cent, c)
    labels, margin = O.cocluster_assign(x, c, p)
    for n in range(40):
        dots = [math.fsum(float(a) * float(b) for a, b in zip(x[0, n], c[0, kk])) for kk in range(6)]
        norm = math.sqrt(math.fsum(d * d for d in dots) + 1e-8)
        dist = [2.0 - 2.0 * math.fsum(dots[kk] / norm * p[0, j, kk] for kk in range(6)) for j in range(9)]
        assert labels[0, n] == int(np.argmin(dist))
        srt = sorted(dist)
        assert margin[0, n] == pytest.approx(srt[1] - srt[0], abs=1e-12)
    red = O.reduced_assign(x, c, p)
    ok = margin > 1e-9
    np.testing.assert_array_equal(red[ok], labels[ok])
    one, _ = O.cocluster_assign(x, c, p[:, :1])
    assert np.all(one == 0)


def test_co_cluster_recovers_separated_mixture():
    # Four far-apart components; queries and keys share the component -> exact recovery.
    h, n, m = 1, 400, 4
    mu = RNG.standard_normal((m, 128)) * 6.0
    z = np.repeat(np.arange(m), n // m)
    q = O.bf16_round((mu[z] + 0.05 * RNG.standard_normal((n, 128))).astype(np.float32))[None]
    k = O.bf16_round((mu[z] + 0.05 * RNG.standard_normal((n, 128))).astype(np.float32))[None]
    init = np.array([[0, 100, 200, 300]])
    ql, qc, qs, kl, kc, ks = O.co_cluster_tokens(q, k, 4, 4, 3, init_q_idx=init, init_k_idx=init)
    np.testing.assert_array_equal(ql[0], z)
    np.testing.assert_array_equal(kl[0], z)
    np.testing.assert_array_equal(qs[0], [100] * 4)
    # Fixed point: centroids are the member means of the final labels.
    again, _ = O.centroid_update(q, ql, qc)
    np.testing.assert_array_equal(again, qc)
    with pytest.raises(UnboundLocalError):
        O.co_cluster_tokens(q, k, 4, 4, 0, init_q_idx=init, init_k_idx=init)



def _brute_labels(x, centroids, basis):
    """Literal profile-space argmin in pure Python (svoo/co_clustering.py:2086-2255): the token's profile is its
    dot products with the basis centroids, normalised with eps 1e-8 inside the root; a centroid's profile is the
    bf16-rounded dot products with the basis, L2-normalised; the label minimises 2 - 2 <profiles>, first index
    on ties."""
    import math

    def dot(a, b):
        return math.fsum(float(u) * float(v) for u, v in zip(a, b))

    prof = []
    for c in centroids:
        raw = [float(O.bf16_round(np.array([dot(c, b)], np.float32))[0]) for b in basis]
        nrm = math.sqrt(math.fsum(r * r for r in raw) + 1e-8)
        prof.append([r / nrm for r in raw])
    labels = []
    for t in x:
        d = [dot(t, b) for b in basis]
        nrm = math.sqrt(math.fsum(v * v for v in d) + 1e-8)
        dist = [2.0 - 2.0 * math.fsum(v / nrm * pj for v, pj in zip(d, pr)) for pr in prof]
        labels.append(min(range(len(dist)), key=lambda j: (dist[j], j)))
    return np.array(labels)


def test_co_cluster_wiring_key_step_then_query_step_on_new_key_centroids():
    """Each iteration assigns keys in the space of the previous query centroids, updates the key centroids, then
    assigns queries in the space of the *updated* key centroids (svoo/co_clustering.py:2423-2449).  The oracle's
    trace shows each half-step's basis; a pure-Python brute force on a tiny case where a stale key-centroid
    basis gives other query labels pins which one the oracle uses."""
    rng = np.random.default_rng(77)
    found = False
    for attempt in range(200):
        n, d, qn, kn = 12, 4, 3, 3
        q = O.bf16_round(rng.standard_normal((1, n, d)).astype(np.float32))
        k = O.bf16_round(rng.standard_normal((1, n, d)).astype(np.float32))
        qi = rng.choice(n, size=(1, qn), replace=False)
        ki = rng.choice(n, size=(1, kn), replace=False)
        trace = []
        ql, qc, qs, kl, kc, ks = O.co_cluster_tokens(q, k, qn, kn, 2, init_q_idx=qi, init_k_idx=ki, trace=trace)
        assert [t[0] for t in trace] == ["k", "q", "k", "q"]
        qc_run, kc_run = q[0, qi[0]], k[0, ki[0]]
        for it in range(2):
            (_, klab, _, kc_in, k_basis), (_, qlab, _, qc_in, q_basis) = trace[2 * it], trace[2 * it + 1]
            np.testing.assert_array_equal(kc_in[0], kc_run)
            np.testing.assert_array_equal(k_basis[0], qc_run)  # keys: previous query centroids
            np.testing.assert_array_equal(klab[0], _brute_labels(k[0], kc_run, qc_run))
            kc_new = O.centroid_update(k, klab, kc_in)[0][0]
            np.testing.assert_array_equal(q_basis[0], kc_new)  # queries: the key centroids just updated
            np.testing.assert_array_equal(qc_in[0], qc_run)
            np.testing.assert_array_equal(qlab[0], _brute_labels(q[0], qc_run, kc_new))
            stale = _brute_labels(q[0], qc_run, kc_run)
            found = found or not np.array_equal(stale, qlab[0])
            qc_run = O.centroid_update(q, qlab, qc_in)[0][0]
            kc_run = kc_new
        np.testing.assert_array_equal(qc[0], qc_run)
        np.testing.assert_array_equal(kc[0], kc_run)
        if found and attempt >= 4:
            break
    assert found, "no case where a stale key-centroid basis changes the query labels"

def test_weighted_softmax_closed_forms():
    s = O.bf16_round(RNG.standard_normal((3, 50)).astype(np.float32))
    w = np.ones((3, 50))
    np.testing.assert_array_equal(O.weighted_softmax(s, w), O.bf16_round(sp_softmax(s.astype(np.float64), axis=-1)))
    eq = np.zeros((1, 7), np.float32)
    wts = np.array([[1, 2, 3, 4, 0, 6, 7]], np.float64)
    np.testing.assert_array_equal(O.weighted_softmax(eq, wts), O.bf16_round(wts / wts.sum()))
    zero_w = O.weighted_softmax(eq, np.zeros((1, 7)))
    np.testing.assert_array_equal(zero_w, np.zeros((1, 7), np.float32))


def _centroids(h, qn, kn, seed=0):
    r = np.random.default_rng(seed)
    qc = O.bf16_round(r.standard_normal((1, h, qn, 128)).astype(np.float32))
    kc = O.bf16_round(r.standard_normal((1, h, kn, 128)).astype(np.float32))
    qs = r.integers(1, 50, size=(1, h, qn)).astype(np.int32)
    ks = r.integers(0, 50, size=(1, h, kn)).astype(np.int32)
    return qc, kc, qs, ks


def test_mask_special_cases():
    qc, kc, qs, ks = _centroids(2, 5, 40)
    assert O.identify_dynamic_map(qc, kc, qs, ks, 1.0).all()
    assert O.identify_dynamic_map(qc, kc, qs, ks, 0.5, min_kc_ratio=1.0).all()
    m = O.identify_dynamic_map(qc, kc, qs, ks, 0.0, min_kc_ratio=[0.1, 0.35])
    np.testing.assert_array_equal(m.sum(-1)[0, 0], [4] * 5)
    # .item() of a float32 tensor gives float64(float32(0.35)) = 0.3499999940..., times 40 -> 13.99999976 -> 13
    np.testing.assert_array_equal(m.sum(-1)[0, 1], [13] * 5)
    m0 = O.identify_dynamic_map(qc, kc, qs, ks, 0.0)
    np.testing.assert_array_equal(m0.sum(-1), np.ones((1, 2, 5)))


def test_mask_keeps_top1_and_prefix():
    qc, kc, qs, ks = _centroids(2, 6, 64, seed=3)
    t = O.centroid_scores(qc, kc)
    pb = O.weighted_softmax(t, np.broadcast_to(ks[:, :, None, :].astype(np.float64), t.shape))
    for p in (0.3, 0.7, 0.9, 0.99):
        m = O.identify_dynamic_map(qc, kc, qs, ks, p)
        for h in range(2):
            for i in range(6):
                row = pb[0, h, i]
                order = np.lexsort((np.arange(64), -row.astype(np.float64)))
                kept = m[0, h, i][order]
                nk = kept.sum()
                assert kept[:nk].all() and not kept[nk:].any()  # a prefix of the stable order
                assert kept[0]


def test_mask_hand_computed_top_p():
    # Equal centroid scores: p_j = w_j / sum(w) exactly; weights 8,4,2,1,1 (sum 16):
    # probabilities 0.5, 0.25, 0.125, 0.0625, 0.0625 (all exact in bf16), prefix 0.5, 0.75, 0.875, 0.9375, 1.
    qc = np.zeros((1, 1, 1, 128), np.float32)
    kc = np.zeros((1, 1, 5, 128), np.float32)
    ks = np.array([[[1, 2, 8, 4, 1]]], np.int32)  # sorted (stable) order: j=2,3,1,0,4
    qs = np.ones((1, 1, 1), np.int32)
    expect = {0.0: [2], 0.5: [2, 3], 0.74: [2, 3], 0.75: [2, 3, 1], 0.9: [2, 3, 1, 0], 0.99: [2, 3, 1, 0, 4]}
    for p, keep in expect.items():
        m = O.identify_dynamic_map(qc, kc, qs, ks, p)[0, 0, 0]
        assert sorted(np.nonzero(m)[0].tolist()) == sorted(keep), p
    # ties 0 and 4 (both 1/16): stable order keeps j=0 before j=4 at p = 0.9
    m = O.identify_dynamic_map(qc, kc, qs, ks, 0.0, min_kc_ratio=0.8)[0, 0, 0]
    assert np.nonzero(m)[0].tolist() == [0, 1, 2, 3]


def _int_row(a, b, e):
    v = np.zeros(128, np.float32)
    v[:3] = (a, b, e)
    return v


def test_centroid_scores_hand_computed():
    # svoo/co_clustering.py:578: bf16 matmul, then "/ (D ** 0.5)" on the bf16 result.
    # q = (16, 16, 1, 0, ...), so q.k = 16*k0 + 16*k1 + k2, exact small integers.
    # bf16 keeps 8 significant bits: in [1024, 2048) its spacing is 8, in [256, 512) it is 2.
    # fl32(1/sqrt(128)) = fl32(1 / fl32(11.3137...)) = 0.088388346; in [64, 128) bf16's spacing is 0.5,
    # in [16, 32) 0.125.
    #   dot 1027 -> bf16 1024 -> 1024 * 0.088388346 = 90.5097 -> bf16 90.5
    #        (unrounded dot: 1027 * 0.0883883 = 90.775 -> 91.0; scaled by 1/128: 8.0)
    #   dot 1029 -> bf16 1032 -> 91.2168 -> 91.0  (unrounded: 90.952 -> 91.0)
    #   dot 1032 -> bf16 1032 -> 91.0
    #   dot  257 -> bf16 256 (tie, even mantissa) -> 22.6274 -> bf16 22.625 (unrounded: 22.7158 -> 22.75)
    #   dot -1027 -> -90.5
    #   dot    5 -> 0.441942 -> bf16 0.44140625 (= 113/256)
    q = _int_row(16, 16, 1)
    keys = [_int_row(32, 32, 3), _int_row(32, 32, 5), _int_row(32, 32, 8), _int_row(8, 8, 1),
            _int_row(-32, -32, -3), _int_row(0, 0, 5)]
    qc = q[None, None, None, :]
    kc = np.stack(keys)[None, None]
    expect = np.array([90.5, 91.0, 91.0, 22.625, -90.5, 0.44140625], np.float32)
    np.testing.assert_array_equal(O.centroid_scores(qc, kc)[0, 0, 0], expect)
    # torch's own bf16 matmul and scalar division on the CPU give the same values.
    tq = torch.from_numpy(qc).bfloat16()
    tk = torch.from_numpy(kc).bfloat16()
    ref = (torch.matmul(tq, tk.transpose(-2, -1)) / (128 ** 0.5)).float().numpy()
    np.testing.assert_array_equal(ref[0, 0, 0], expect)


def test_mask_kept_set_depends_on_score_rounding_and_scale():
    # Key clusters j0, j1, jT with dots 1027, 1029, 1032 (scores 90.5, 91.0, 91.0 as above) and sizes 3, 2, 24.
    # Weighted masses in units of e^91: jT 24, j1 2, j0 3 e^-0.5 = 1.8196; total 27.8196.
    #   sorted: jT 0.8627 (bf16 0.86328125 <= bf16(0.9) = 0.8984375), j1 0.0719, j0 0.0654
    #   prefix after jT = 0.863 <= 0.898: keep j1; prefix after j1 = 0.935 > 0.898: drop j0  => {j1, jT}
    # Without the rounding of the dot j0 scores 91.0: masses 24, 3, 2 -> order jT, j0, j1 => {j0, jT}.
    # With 1/D for 1/sqrt(D) the scores are 8.0, 8.0625, 8.0625: masses 24, 2, 3 e^-0.0625 = 2.818
    #   -> order jT, j0, j1 => {j0, jT}.
    q = _int_row(16, 16, 1)
    kc = np.stack([_int_row(32, 32, 3), _int_row(32, 32, 5), _int_row(32, 32, 8)])[None, None]
    qc = q[None, None, None, :]
    ks = np.array([[[3, 2, 24]]], np.int32)
    m = O.identify_dynamic_map(qc, kc, np.ones((1, 1, 1), np.int32), ks, 0.9)[0, 0, 0]
    assert m.tolist() == [False, True, True]
    t = O.centroid_scores(qc, kc)
    pb = O.weighted_softmax(t, np.broadcast_to(ks[:, :, None, :].astype(np.float64), t.shape))[0, 0, 0]
    # bf16 of 1.8196/27.8196 = 0.06541, 2/27.8196 = 0.07189, 24/27.8196 = 0.86270 (spacing 2^-11 below 0.125)
    np.testing.assert_array_equal(pb, np.array([134 / 2048, 147 / 2048, 221 / 256], np.float32))


def test_mask_row_params_float32_ratio_semantics():
    pre, cap = O.mask_row_params(2, 1000, [0.7, 0.15])
    assert pre.tolist() == [699, 150]  # float32(0.7) * 1000 = 699.99998
    pre, _ = O.mask_row_params(2, 1000, 0.7)
    assert pre.tolist() == [700, 700]
    pre, cap = O.mask_row_params(2, 1000, [0.2, 0.0], [0.1, 0.3])
    assert cap.tolist() == [200, 300]
    pre, cap = O.mask_row_params(2, 1000, 0.1, 0.05)
    assert cap.tolist() == [100, 100]
    pre, cap = O.mask_row_params(2, 100, 0, 0.001)
    assert cap.tolist() == [1, 1]


def test_kv_plan_indices_brute_force():
    m = np.zeros((2, 2, 3), bool)
    m[0, 0, [0, 2]] = True
    m[1, 1, [1]] = True
    cs = np.array([[2, 3, 1], [1, 1, 4]])
    indptr, ind = O.kv_plan_indices(m, cs)
    assert indptr.tolist() == [0, 3, 3, 3, 4]
    assert ind.tolist() == [0, 1, 5, 7]


def test_block_sparse_attention_closed_forms():
    q = RNG.standard_normal((1, 2, 30, 128))
    k = RNG.standard_normal((1, 2, 30, 128))
    v = RNG.standard_normal((1, 2, 30, 128))
    qs = np.array([[[10, 20], [15, 15]]])
    ks = np.array([[[12, 18], [30, 0]]])
    full = np.ones((1, 2, 2, 2), bool)
    o = O.block_sparse_attention(q, k, v, full, qs, ks)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v)).numpy()
    np.testing.assert_allclose(o, ref, rtol=1e-10, atol=1e-12)
    diag = np.zeros((1, 2, 2, 2), bool)
    diag[0, 0, 0, 0] = diag[0, 0, 1, 1] = True
    diag[0, 1, 0, 0] = True  # head 1: cluster 1 has no active keys -> zeros
    o = O.block_sparse_attention(q, k, v, diag, qs, ks)
    blk = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q[:, :1, :10]), torch.from_numpy(k[:, :1, :12]), torch.from_numpy(v[:, :1, :12])).numpy()
    np.testing.assert_allclose(o[:, :1, :10], blk, rtol=1e-10, atol=1e-12)
    assert np.all(o[0, 1, 15:] == 0)


def test_attention_call_reduces_to_dense():
    h, n = 2, 64
    q = O.bf16_round(RNG.standard_normal((1, h, n, 128)).astype(np.float32))
    k = O.bf16_round(RNG.standard_normal((1, h, n, 128)).astype(np.float32))
    v = O.bf16_round(RNG.standard_normal((1, h, n, 128)).astype(np.float32))
    init = np.zeros((h, 1), np.int64)
    out = O.svoo_attention_call(q, k, v, 1, 1, 2, 1.0, init_q_idx=init, init_k_idx=init)
    dense = O.dense_attention(q, k, v)
    np.testing.assert_allclose(out, np.transpose(dense, (0, 2, 1, 3)).reshape(1, n, h * 128), rtol=1e-9, atol=1e-12)


def test_hunyuan_post_process_rules():
    # 2 video q-clusters x 3 video k-clusters; prompt 5 of 8 text tokens.
    m = np.array([[[[1, 0, 1], [0, 1, 0]]]], dtype=bool)
    qs = np.array([[[4, 6]]])
    ks = np.array([[[3, 3, 4]]])
    idx = np.array([[3, 1, 0, 2, 4, 5, 9, 8, 7, 6]])
    m2, qs2, ks2, idx2 = O.hunyuan_post_process(m, qs, ks, idx, 10, 8, 5)
    expect = np.array([[1, 0, 1, 1, 0],
                       [0, 1, 0, 1, 0],
                       [1, 1, 1, 1, 0],
                       [0, 0, 0, 0, 1]], dtype=bool)
    np.testing.assert_array_equal(m2[0, 0], expect)
    np.testing.assert_array_equal(qs2[0, 0], [4, 6, 5, 3])
    np.testing.assert_array_equal(ks2[0, 0], [3, 3, 4, 5, 3])
    np.testing.assert_array_equal(idx2[0], [3, 1, 0, 2, 4, 5, 9, 8, 7, 6, 10, 11, 12, 13, 14, 15, 16, 17])


def test_hunyuan_dense_gate_closed_form():
    q, k, v = (RNG.standard_normal((1, 2, 40, 128)) for _ in range(3))
    out = O.hunyuan_dense_attention(q, k, v, 31)
    sd = lambda a, b, c: torch.nn.functional.scaled_dot_product_attention(  # noqa: E731
        torch.from_numpy(a), torch.from_numpy(b), torch.from_numpy(c)).numpy()
    np.testing.assert_allclose(out[:, :, :31], sd(q[:, :, :31], k[:, :, :31], v[:, :, :31]), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(out[:, :, 31:], sd(q[:, :, 31:], k[:, :, 31:], v[:, :, 31:]), rtol=1e-10, atol=1e-12)


def test_hunyuan_call_with_all_blocks_is_dense_varlen():
    # top_p >= 1 keeps every video block, so video + prompt form one dense block and the padding another.
    h, vl, ctx, prompt = 2, 96, 16, 11
    q, k, v = (O.bf16_round(RNG.standard_normal((1, h, vl + ctx, 128)).astype(np.float32)) for _ in range(3))
    init_q = RNG.integers(0, vl, size=(h, 4))
    init_k = RNG.integers(0, vl, size=(h, 6))
    out = O.hunyuan_attention_call(q, k, v, 4, 6, 2, 1.0, 0, prompt, ctx, init_q_idx=init_q, init_k_idx=init_k)
    np.testing.assert_allclose(out, O.hunyuan_dense_attention(q, k, v, vl + prompt), rtol=1e-9, atol=1e-12)


# ---------------------------------------------------------------- exact sparsity (profile producer)
def _torch_reference_counts(scores, scale, threshold):
    """The reference's fp32 formulation (svoo/sparsity/exact.py:110-155) restated in torch on the CPU:
    softmax, descending sort, cumsum, searchsorted(right=False) + 1."""
    import torch

    t = torch.from_numpy(np.asarray(scores, np.float32)) * scale
    w = torch.softmax(t, dim=-1)
    cs = torch.cumsum(torch.sort(w, dim=-1, descending=True).values, dim=-1)
    target = (threshold * cs[..., -1:]).contiguous()
    return (torch.searchsorted(cs, target, right=False, out_int32=True).squeeze(-1) + 1).numpy()


def test_exact_sparsity_closed_forms():
    # equal scores: every weight is 1, so c keys hold c/n of the mass -> ceil(threshold * n)
    for n in (1, 7, 100, 4096):
        for thr in (0.5, 0.9, 0.95, 1.0):
            c = O.exact_sparsity_counts(np.zeros((3, n), np.float32), 0.088, thr)
            assert (c == int(np.ceil(thr * n - 1e-12))).all(), (n, thr, c)
    # one dominant key holds almost all of the mass
    s = np.full((2, 1000), -60.0, np.float32)
    s[:, 123] = 60.0
    assert (O.exact_sparsity_counts(s, 1.0, 0.95) == 1).all()
    # two keys of equal weight above a negligible tail: 0.6 of the mass needs both
    s = np.full((1, 50), -200.0, np.float32)
    s[0, [3, 9]] = 0.0
    assert O.exact_sparsity_counts(s, 1.0, 0.6)[0] == 2
    assert O.exact_sparsity_counts(s, 1.0, 0.5)[0] == 1
    # threshold 1: exactly the keys whose fp32 weight is non-zero (exp(-120) underflows)
    s = np.zeros((1, 10), np.float32)
    s[0, :4] = -120.0
    assert O.exact_sparsity_counts(s, 1.0, 1.0)[0] == 6


def test_exact_sparsity_matches_reference_formulation_and_brute_force():
    import math

    rng = np.random.default_rng(7)
    for scale_in, n in ((3.0, 3000), (0.5, 777), (8.0, 256)):
        sc = O.bf16_round((rng.standard_normal((48, n)) * scale_in).astype(np.float32))
        mine = O.exact_sparsity_counts(sc, 0.0884, 0.95)
        ref = _torch_reference_counts(sc, 0.0884, 0.95)
        # fp32 softmax/cumsum in the reference can move a count by one key at a rounding boundary
        assert np.abs(mine - ref).max() <= 1 and (mine == ref).mean() >= 0.97
    # brute force with exact (fsum) prefix sums on small rows
    sc = O.bf16_round((rng.standard_normal((6, 40)) * 4).astype(np.float32))
    w = O.sparsity_weights(sc, 0.5)
    for r in range(6):
        vals = sorted((float(x) for x in w[r]), reverse=True)
        tot = math.fsum(vals)
        c = next(i + 1 for i in range(len(vals)) if math.fsum(vals[: i + 1]) >= 0.9 * tot)
        assert O.exact_sparsity_counts(sc[r : r + 1], 0.5, 0.9)[0] == c


def test_exact_attention_sparsity_per_head_mean():
    rng = np.random.default_rng(3)
    q = O.bf16_round(rng.standard_normal((1, 2, 64, 128)).astype(np.float32))
    k = O.bf16_round(rng.standard_normal((1, 2, 96, 128)).astype(np.float32))
    avg, per_head, counts = O.exact_attention_sparsity(q, k, 0.9)
    assert counts.shape == (1, 2, 64)
    assert np.allclose(per_head, counts[0].mean(axis=1) / 96.0) and abs(avg - np.mean(per_head)) < 1e-12
    # sampled rows: linspace positions of the sampled query rows only
    _, _, c5 = O.exact_attention_sparsity(q, k, 0.9, query_sample_size=5)
    pos = [0, 16, 32, 47, 63]
    assert np.array_equal(c5, counts[:, :, pos])
