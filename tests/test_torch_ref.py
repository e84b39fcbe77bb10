"""The float32 torch restatement of the reference call (``oracle/torch_ref.py``, the CPU baseline the benchmark
times) against the numpy oracle's float32 contract, on the CPU."""

import numpy as np
import torch

from oracle import svoo_oracle as O
from oracle import torch_ref as T


def _mixture(h, n, centers, scale, noise, seed):
    r = np.random.default_rng(seed)
    mu = r.standard_normal((h, centers, 128)) * scale
    z = r.integers(0, centers, size=(h, n))
    out = []
    for _ in range(3):
        x = np.take_along_axis(mu, z[:, :, None], axis=1) + noise * r.standard_normal((h, n, 128))
        out.append(x.astype(np.float32)[None])
    return out, z


def test_torch_call_equals_oracle_on_separated_clusters():
    (q, k, v), z = _mixture(2, 1500, 6, 3.0, 0.05, 1)
    # initial centroids: one member of each component (the same for both sides' mixtures)
    first = np.stack([[int(np.nonzero(z[h] == c)[0][0]) for c in range(6)] for h in range(2)])
    qi = np.stack([q[0, h, first[h]] for h in range(2)])
    ki = np.stack([k[0, h, first[h]] for h in range(2)])
    ratios = [0.3, 0.5]
    out, parts = O.svoo_attention_call(q, k, v, 6, 6, 3, 0.9, ratios, init_q_centroids=qi, init_k_centroids=ki,
                                       dtype="fp32", attn_dtype=np.float64, return_parts=True)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    ql, qc, qs, kl, kc, ks = T.co_cluster_tokens(tq[0], tk[0], 6, 6, 3, torch.from_numpy(qi), torch.from_numpy(ki))
    np.testing.assert_array_equal(ql.numpy(), parts["qlabels"])
    np.testing.assert_array_equal(kl.numpy(), parts["klabels"])
    np.testing.assert_allclose(qc.numpy(), parts["qcentroids"], rtol=0, atol=1e-5)
    dmap = T.identify_dynamic_map(qc, kc, ks, 0.9, ratios)
    np.testing.assert_array_equal(dmap.numpy(), parts["map"][0])
    got = T.svoo_attention_call(tq, tk, tv, 6, 6, 3, 0.9, ratios, torch.from_numpy(qi), torch.from_numpy(ki))
    np.testing.assert_allclose(got.numpy(), out, rtol=0, atol=2e-5)


def test_torch_block_sparse_attention_matches_oracle():
    r = np.random.default_rng(3)
    h, s, qn, kn = 2, 700, 5, 9

    def sizes(c):
        cuts = np.sort(r.integers(0, s + 1, size=(h, c - 1)), axis=1)
        return np.diff(np.concatenate([np.zeros((h, 1), int), cuts, np.full((h, 1), s)], axis=1), axis=1)

    qs, ks = sizes(qn), sizes(kn)
    m = r.random((h, qn, kn)) < 0.4
    m[0, 0] = False  # a query cluster with no kept key cluster -> zero rows
    q, k, v = (r.standard_normal((h, s, 128)).astype(np.float32) for _ in range(3))
    want = O.block_sparse_attention(q[None], k[None], v[None], m[None], qs[None], ks[None])[0]
    got = T.block_sparse_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), torch.from_numpy(m),
                                   torch.from_numpy(qs), torch.from_numpy(ks))
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=2e-5)


def test_torch_hunyuan_call_matches_oracle():
    (q, k, v), z = _mixture(1, 900 + 40, 4, 3.0, 0.05, 7)
    vl = 900
    first = [int(np.nonzero(z[0, :vl] == c)[0][0]) for c in range(4)]
    qi, ki = q[0][:, first], k[0][:, first]
    want = O.hunyuan_attention_call(q, k, v, 4, 4, 2, 0.9, [0.5], 30, 40, init_q_centroids=qi, init_k_centroids=ki,
                                    dtype="fp32", attn_dtype=np.float64)
    got = T.hunyuan_attention_call(*(torch.from_numpy(x) for x in (q, k, v)), 4, 4, 2, 0.9, [0.5], 30, 40,
                                   torch.from_numpy(qi), torch.from_numpy(ki))
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=2e-5)
