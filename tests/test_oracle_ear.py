"""Pinning of the EAR restatement (error-aware routing with centroid compensation) on the CPU.

The reference ships no test, golden vector or known-answer test for this path, so each oracle
function is pinned by what the mathematics fixes: brute force from the definition on tiny inputs,
hand-worked selections, and closed forms (dense attention where nothing is pruned, exact
compensation where every pruned cluster is a point mass at its centroid).

Pinning map (oracle function -> independent checks):
  value_centroids             small-integer means; empty cluster -> 0; the bf16 count rounding (301 -> 300)
  value_stats                 per-token dot products in float64
  ear_centroid_logits         exact small-integer dots times float32(D**-0.5)
  ear_efficiency_scores       brute force from the vector-norm definition (no expansion), gamma 0 / 0.5 / 1;
                              empty cluster; logits of 100 stay finite (log err = 200)
  ear_row_params              scalar / per-head / length-1 / other-length branches; float32 reads
  ear_select                  hand-worked budgets and greedy fills; ties by index; random invariants
  ear_compensated_attention   all-active map = dense attention; all-inactive = centroid attention with the
                              log|K| prior; point-mass clusters = dense attention for any map
  ear_attention_call          min ratio 1 keeps every block: the call equals dense attention
"""

import numpy as np
import pytest

from oracle import svoo_oracle as O


def _bf(x):
    return O.bf16_round(np.asarray(x, np.float32))


def _dense(q, k, v):
    s = (q.astype(np.float64) @ k.astype(np.float64).T) / np.sqrt(q.shape[-1])
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v.astype(np.float64)


# ------------------------------------------------------------------------------------------ value side
def test_value_centroids_small_integer_means():
    v = np.zeros((1, 7, 4), np.float32)
    v[0, :3] = [[1, 2, 3, 4], [3, 2, 1, 0], [2, 2, 2, 2]]  # cluster 0: mean (2, 2, 2, 2)
    v[0, 3:7] = [[4, 0, 0, 8], [0, 4, 0, 8], [0, 0, 4, 8], [0, 0, 0, 8]]  # cluster 2 (cluster 1 empty)
    vc = O.value_centroids(v, np.array([[3, 0, 4]]))
    np.testing.assert_array_equal(vc[0, 0], [2, 2, 2, 2])
    np.testing.assert_array_equal(vc[0, 1], [0, 0, 0, 0])  # empty: zero sum / 1
    np.testing.assert_array_equal(vc[0, 2], [1, 1, 1, 8])


def test_value_centroids_divide_by_storage_rounded_count():
    # 301 members equal to 1: sum 301 rounds to bf16 300, the count 301 rounds to 300 -> mean exactly 1;
    # 259 members: sum 259 -> bf16 260, count -> 260 -> 1.  A float32 count would give 300/301 and 260/259.
    for n in (301, 259):
        vc = O.value_centroids(np.ones((1, n, 2), np.float32), np.array([[n]]))
        np.testing.assert_array_equal(vc[0, 0], [1, 1])
    # 3 members: sum 3 / count 3 -> 1 exactly; and a mean that is not a bf16 value rounds once
    vc = O.value_centroids(np.array([[[1.0], [1.0], [2.0]]], np.float32), np.array([[3]]))
    assert vc[0, 0, 0] == _bf(np.float32(4.0) / np.float32(3.0))


def test_value_stats_brute_force():
    rng = np.random.default_rng(0)
    v = _bf(rng.standard_normal((2, 9, 8)))
    ks = np.array([[4, 0, 5], [2, 6, 1]])
    vc = O.value_centroids(v, ks)
    vn, cvd, vcsq = O.value_stats(v, vc, ks)
    v, vc = v.astype(np.float64), vc.astype(np.float64)
    for b in range(2):
        off = np.concatenate([[0], np.cumsum(ks[b])])
        for j in range(3):
            assert vcsq[b, j] == pytest.approx(float(np.dot(vc[b, j], vc[b, j])), rel=1e-12)
            for t in range(off[j], off[j + 1]):
                assert vn[b, t] == pytest.approx(float(np.dot(v[b, t], v[b, t])), rel=1e-12)
                assert cvd[b, t] == pytest.approx(float(np.dot(v[b, t], vc[b, j])), rel=1e-12)


# ------------------------------------------------------------------------------------------ scores
def test_centroid_logits_exact_on_small_integers():
    qc = np.array([[[1, 2] + [0] * 126, [3, -1] + [0] * 126]], np.float32)
    kc = np.array([[[4, 4] + [0] * 126]], np.float32)
    c = O.ear_centroid_logits(qc, kc)
    scale = np.float32(128 ** -0.5)
    np.testing.assert_array_equal(c[0, :, 0], _bf([np.float32(12) * scale, np.float32(8) * scale]))


def _err_brute(qc_i, c_ij, k_rows, v_rows, vc_j):
    """sum_t || e^{a_t} v_t - e^{c} vc ||^2 as explicit vector norms (no expansion)."""
    d = qc_i.shape[0]
    tot = 0.0
    for kt, vt in zip(k_rows.astype(np.float64), v_rows.astype(np.float64)):
        a = float(qc_i.astype(np.float64) @ kt) / np.sqrt(d)
        diff = np.exp(a) * vt - np.exp(float(c_ij)) * vc_j.astype(np.float64)
        tot += float(diff @ diff)
    return tot


@pytest.mark.parametrize("gamma", [0.0, 1.0, 0.5])
def test_efficiency_scores_match_vector_norm_definition(gamma):
    rng = np.random.default_rng(1)
    d = 128
    ks = np.array([[3, 0, 5, 1]])
    qs = np.array([[2, 7, 0]])
    n = int(ks.sum())
    kp = _bf(rng.standard_normal((1, n, d)) * 0.5)
    vp = _bf(rng.standard_normal((1, n, d)))
    qc = _bf(rng.standard_normal((1, 3, d)) * 0.5)
    kc = _bf(rng.standard_normal((1, 4, d)) * 0.5)
    vc = O.value_centroids(vp, ks)
    c = O.ear_centroid_logits(qc, kc)
    eff = O.ear_efficiency_scores(qc, c, kp, vp, vc, qs, ks, gamma)
    off = np.concatenate([[0], np.cumsum(ks[0])])
    eps = 1e-8
    for i in range(3):
        for j in range(4):
            err = _err_brute(qc[0, i], c[0, i, j], kp[0, off[j]:off[j + 1]], vp[0, off[j]:off[j + 1]], vc[0, j])
            want = np.log(max(err, eps)) - gamma * np.log(max(qs[0, i] * ks[0, j], eps))
            assert eff[0, i, j] == pytest.approx(want, abs=2e-5), (i, j)
    # an empty key cluster has zero error and zero area
    assert eff[0, 0, 1] == pytest.approx(np.log(eps) - gamma * np.log(eps), abs=1e-5)


def test_efficiency_scores_large_logits_stay_finite():
    # logits near 100 overflow exp() in float32; the shifted evaluation keeps log(err) exact
    d = 128
    kp = np.zeros((1, 2, d), np.float32)
    kp[0, :, 0] = [1.0, 0.5]
    vp = np.zeros((1, 2, d), np.float32)
    vp[0, :, 1] = [1.0, 3.0]
    qc = np.zeros((1, 1, d), np.float32)
    qc[0, 0, 0] = 100.0 * np.sqrt(d)  # a_t = 100, 50
    c = np.full((1, 1, 1), 60.0, np.float32)
    vc = O.value_centroids(vp, np.array([[2]]))
    eff = O.ear_efficiency_scores(qc, c, kp, vp, vc, np.array([[1]]), np.array([[2]]), 0.0)
    # err ~ e^{200} * |v_0|^2 dominates: log err ~ 200
    assert np.isfinite(eff).all() and eff[0, 0, 0] == pytest.approx(200.0, abs=1e-3)


# ------------------------------------------------------------------------------------------ selection
def test_row_params_branches():
    pre, bpre = O.ear_row_params(3, 10, 0.25)
    assert list(pre) == [2, 2, 2] and list(bpre) == [5, 5, 5]
    # per head, read through float32: a tiny ratio still keeps 1, and float32(0.35) < 0.35 gives
    # int(3.4999999) = 3 and int(6.9999998) = 6 (a scalar 0.35 gives 3 and 7)
    pre, bpre = O.ear_row_params(3, 10, [0.0, 0.01, 0.35])
    assert list(pre) == [0, 1, 3] and list(bpre) == [0, 1, 6]
    pre, bpre = O.ear_row_params(3, 10, 0.35)
    assert list(pre) == [3, 3, 3] and list(bpre) == [7, 7, 7]
    pre, bpre = O.ear_row_params(3, 10, [0.3])  # length 1: a scalar
    assert list(pre) == [3, 3, 3] and list(bpre) == [6, 6, 6]
    pre, bpre = O.ear_row_params(3, 10, [0.3, 0.3])  # any other length: no minimum
    assert list(pre) == [0, 0, 0] and list(bpre) == [0, 0, 0]


def _select_one(eff, c, qs, ks, top_p, ratio):
    return O.ear_select(np.asarray(eff, np.float32)[None, None, None], np.asarray(c, np.float32)[None, None, None],
                        np.array([[[qs]]]), np.array([ks])[None], top_p, ratio)[0, 0, 0]


def test_select_hand_worked_budget_and_greedy():
    # Kc = 4, |Q_i| = 1, |K| = (10, 20, 30, 40).  Logits chosen so that c_j + log|K_j| = (0, 0, -20, -20):
    # budget probabilities ~ (0.5, 0.5, 0, 0) -> sorted (0, 1, 2, 3); with top_p 0.4 the prefix after the
    # first entry (0.5) exceeds p, so the budget keeps only cluster 0: budget = 10.
    ks = [10, 20, 30, 40]
    c = [0 - np.log(10), 0 - np.log(20), -20 - np.log(30), -20 - np.log(40)]
    c = list(_bf(c))
    # efficiency order 2 > 3 > 1 > 0: greedy keeps 2 (cost before it 0 < 10), then 3 (30 >= 10 stops)
    m = _select_one([0.0, 1.0, 3.0, 2.0], c, 1, ks, 0.4, 0)
    assert list(m) == [False, False, True, False]
    # top_p 0.6: budget keeps clusters 0 and 1 (30); greedy: 2 (0 < 30), 3 (30 >= 30: no)
    m = _select_one([0.0, 1.0, 3.0, 2.0], c, 1, ks, 0.6, 0)
    assert list(m) == [False, False, True, False]
    # min ratio 0.25 -> preserve 1 (cluster 0 guaranteed), budget_preserve 2 -> budget 30, remaining 20;
    # greedy over the others: 2 (0 < 20), then 3 (30 >= 20) stop
    m = _select_one([0.0, 1.0, 3.0, 2.0], c, 1, ks, 0.4, 0.25)
    assert list(m) == [True, False, True, False]
    # cheap high-efficiency blocks first: 1 (0 < 30), 0 (20 < 30), then 2 (30 >= 30) stop
    m = _select_one([2.0, 3.0, 1.0, 0.0], c, 1, ks, 0.6, 0)
    assert list(m) == [True, True, False, False]


def test_select_ties_break_by_cluster_index():
    ks = [5, 5, 5, 5]
    c = [0.0, 0.0, 0.0, 0.0]  # equal budget probabilities 0.25
    # top_p 0.3: prefix 0.25 <= 0.3 keeps position 1 too: budget 10; equal efficiency -> clusters 0, 1
    m = _select_one([1.0, 1.0, 1.0, 1.0], c, 1, ks, 0.3, 0)
    assert list(m) == [True, True, False, False]
    # preserve 1 guarantees the first budget-ordered cluster (index 0 on ties)
    m = _select_one([0.0, 0.0, 5.0, 0.0], c, 1, ks, 0.3, 0.25)
    assert list(m) == [True, False, True, False]


def test_select_invariants_random():
    rng = np.random.default_rng(3)
    b, h, qn, kn = 1, 3, 5, 40
    eff = rng.standard_normal((b, h, qn, kn)).astype(np.float32) * 3
    c = _bf(rng.standard_normal((b, h, qn, kn)))
    qs = rng.integers(0, 30, (b, h, qn))
    ks = rng.integers(0, 50, (b, h, kn))
    ratios = [0.0, 0.05, 0.2]
    m = O.ear_select(eff, c, qs, ks, 0.8, ratios)
    pre, _ = O.ear_row_params(h, kn, ratios)
    for hi in range(h):
        for i in range(qn):
            row = m[0, hi, i]
            assert row.sum() >= pre[hi]
            area = qs[0, hi, i] * ks[0, hi]
            # the kept candidates are a prefix of the efficiency order (ties by index)
            order = np.lexsort((np.arange(kn), -eff[0, hi, i].astype(np.float64)))
            kept_rank = [r for r, j in enumerate(order) if row[j]]
            if qs[0, hi, i] > 0 and pre[hi] == 0:
                assert kept_rank == list(range(len(kept_rank)))
            # the guaranteed clusters plus the greedy ones: the cost before the last kept candidate is
            # below the budget, so the kept area exceeds it by at most one block
            assert area[row].sum() <= area.sum()


# ------------------------------------------------------------------------------------------ compensation
def _clustered_inputs(rng, qs, ks, d=128):
    s = int(sum(qs))
    q = _bf(rng.standard_normal((1, 1, s, d)) * 0.3)
    k = _bf(rng.standard_normal((1, 1, s, d)) * 0.3)
    v = _bf(rng.standard_normal((1, 1, s, d)))
    return q, k, v


def test_compensated_attention_all_active_is_dense():
    rng = np.random.default_rng(4)
    qs, ks = [5, 9, 2], [4, 7, 5]
    q, k, v = _clustered_inputs(rng, qs, ks)
    kc = _bf(rng.standard_normal((1, 1, 3, 128)))
    vc = _bf(rng.standard_normal((1, 1, 3, 128)))
    m = np.ones((1, 1, 3, 3), bool)
    out = O.ear_compensated_attention(q, k, v, kc, vc, m, np.array([[qs]]), np.array([[ks]]))
    np.testing.assert_allclose(out[0, 0], _dense(q[0, 0], k[0, 0], v[0, 0]), atol=1e-12)


def test_compensated_attention_all_inactive_is_centroid_attention():
    rng = np.random.default_rng(5)
    qs, ks = [6, 10], [3, 13]
    q, k, v = _clustered_inputs(rng, qs, ks)
    kc = _bf(rng.standard_normal((1, 1, 2, 128)) * 0.3)
    vc = _bf(rng.standard_normal((1, 1, 2, 128)))
    m = np.zeros((1, 1, 2, 2), bool)
    out = O.ear_compensated_attention(q, k, v, kc, vc, m, np.array([[qs]]), np.array([[ks]]))
    s = q[0, 0].astype(np.float64) @ kc[0, 0].astype(np.float64).T / np.sqrt(128)
    s += np.log(np.array(ks, np.float32) + np.float32(1e-6)).astype(np.float64)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(out[0, 0], p @ vc[0, 0].astype(np.float64), atol=1e-12)


def test_compensation_exact_for_point_mass_clusters():
    # every key cluster holds |K_j| copies of (kc_j, vc_j): pruning any subset and compensating with the
    # centroid and the log|K_j| prior reproduces dense attention (up to the 1e-6 inside the log)
    rng = np.random.default_rng(6)
    qs, ks = [7, 5, 9], [5, 1, 9, 6]
    kc = _bf(rng.standard_normal((1, 1, 4, 128)) * 0.4)
    vc = _bf(rng.standard_normal((1, 1, 4, 128)))
    k = np.concatenate([np.repeat(kc[0, 0, j:j + 1], ks[j], 0) for j in range(4)])[None, None]
    v = np.concatenate([np.repeat(vc[0, 0, j:j + 1], ks[j], 0) for j in range(4)])[None, None]
    q = _bf(rng.standard_normal((1, 1, sum(qs), 128)) * 0.4)
    m = rng.integers(0, 2, (1, 1, 3, 4)).astype(bool)
    m[..., 0] = True
    out = O.ear_compensated_attention(q, k, v, kc, vc, m, np.array([[qs]]), np.array([[ks]]))
    np.testing.assert_allclose(out[0, 0], _dense(q[0, 0], k[0, 0], v[0, 0]), atol=2e-6)


def test_ear_attention_call_full_budget_is_dense():
    # min_kc_ratio 1 guarantees every key cluster: the call reduces to dense attention
    rng = np.random.default_rng(7)
    h, s, d = 2, 96, 128
    q = _bf(rng.standard_normal((1, h, s, d)) * 0.5)
    k = _bf(rng.standard_normal((1, h, s, d)) * 0.5)
    v = _bf(rng.standard_normal((1, h, s, d)))
    out = O.ear_attention_call(q, k, v, 4, 8, 2, 0.5, 1.0, 1.0, init_q_idx=rng.integers(0, s, (h, 4)),
                               init_k_idx=rng.integers(0, s, (h, 8)))
    want = np.stack([_dense(q[0, i], k[0, i], v[0, i]) for i in range(h)], 1).reshape(1, s, h * d)
    np.testing.assert_allclose(out, want, atol=1e-10)
