"""GPU tests of the offline profile producer: exact sparsity counts through the C ABI against the oracle,
the full ``compute_exact_attention_sparsity`` call, and the processor's logging hook end to end (raw log ->
merged profile CSV -> ``SparsityLookup``)."""

import numpy as np
import pytest
import torch

from oracle import svoo_oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _scores(rng, rows, n, kind):
    if kind == "normal":
        x = rng.standard_normal((rows, n)) * 3.0
    elif kind == "heavy":
        x = rng.standard_cauchy((rows, n)).clip(-200, 200)
    elif kind == "ties":
        x = rng.integers(-3, 4, size=(rows, n)).astype(np.float64)  # few distinct values, many ties
    elif kind == "peaked":
        x = rng.standard_normal((rows, n)) * 0.5
        x[:, : max(1, n // 50)] += 12.0
    else:
        x = np.zeros((rows, n))
    return O.bf16_round(x.astype(np.float32))


@pytest.mark.parametrize("n", [1, 7, 256, 300, 4099])
@pytest.mark.parametrize("kind", ["normal", "heavy", "ties", "peaked", "equal"])
def test_counts_match_oracle(gpu, n, kind):
    from svoo_amd.sparsity import exact_counts_from_scores

    say("exact counts", kind, n)
    rng = np.random.default_rng(n * 7 + len(kind))
    rows = 37
    sc = _scores(rng, rows, n, kind)
    t = torch.from_numpy(sc).to(torch.bfloat16).to(gpu)
    # threshold 1 asks for the whole mass, which fp64 summation only pins when no weight is below
    # 2^-53 of the total (the heavy-tailed rows have weights near 1e-16 of the total)
    for thr in (0.5, 0.9, 0.95) + ((1.0,) if kind != "heavy" else ()):
        got = exact_counts_from_scores(t, 0.0884, thr).cpu().numpy()
        want = O.exact_sparsity_counts(sc, 0.0884, thr)
        assert np.array_equal(got, want), (kind, n, thr, np.nonzero(got != want), got[:5], want[:5])


def test_counts_long_rows(gpu):
    from svoo_amd.sparsity import exact_counts_from_scores

    say("exact counts, rows of 75600 keys")
    rng = np.random.default_rng(11)
    sc = _scores(rng, 6, 75600, "normal")
    got = exact_counts_from_scores(torch.from_numpy(sc).to(torch.bfloat16).to(gpu), 0.0884, 0.95).cpu().numpy()
    assert np.array_equal(got, O.exact_sparsity_counts(sc, 0.0884, 0.95))


def test_compute_exact_attention_sparsity(gpu):
    from svoo_amd.sparsity import compute_exact_attention_sparsity

    say("compute_exact_attention_sparsity")
    rng = np.random.default_rng(5)
    q = O.bf16_round((rng.standard_normal((1, 3, 500, 128)) * 1.5).astype(np.float32))
    k = O.bf16_round((rng.standard_normal((1, 3, 700, 128)) * 1.5).astype(np.float32))
    qt, kt = (torch.from_numpy(a).to(torch.bfloat16).to(gpu) for a in (q, k))
    for bs, samples in ((0, 0), (128, 0), (64, 33)):
        avg, per_head, stats = compute_exact_attention_sparsity(qt, kt, batch_size=bs, threshold=0.9,
                                                                query_sample_size=samples)
        assert stats["sampled_seq_len"] == (samples or 500) and stats["attn_scores_shape"][2] == (samples or 500)
        # exact against the oracle on the same bf16 scores (the library GEMM's rounding)
        qs = qt if not samples else qt[:, :, np.unique(np.round(np.linspace(0, 499, samples, dtype=np.float32)))
                                         .astype(np.int64)]
        cs = stats["chunk_size"]  # the same GEMM chunks as the call (bf16 rounding may depend on the shape)
        s_gpu = torch.cat([torch.matmul(qs[:, :, i:i + cs], kt.transpose(-2, -1)) for i in range(0, qs.shape[2], cs)],
                          dim=2).float().cpu().numpy()
        want = O.exact_sparsity_counts(s_gpu, 128 ** -0.5, 0.9).mean(axis=2)[0] / 700.0
        np.testing.assert_allclose(per_head, want, rtol=0, atol=1e-12)
        assert abs(avg - float(np.mean(want))) < 1e-12
        # against exact-dot bf16 scores: a score can round to the neighbouring bf16 value
        o_avg, o_heads, _ = O.exact_attention_sparsity(q, k, 0.9, samples)
        np.testing.assert_allclose(per_head, o_heads, atol=2e-3)


def test_processor_logs_profile_end_to_end(gpu, tmp_path):
    from svoo_amd import dit
    from svoo_amd.inference import replace_wan_attention
    from svoo_amd.processor import WanAttn_SAPAttn_Processor
    from svoo_amd.sparsity import SparsityLookup, merge_sparsity_data, save_to_csv

    say("processor sparsity log -> merged profile -> lookup")
    cfg = dit.WanDiTConfig(num_attention_heads=2, ffn_dim=256, num_layers=2, text_dim=32)
    pipe = dit.make_pipe(cfg, device=gpu, dtype=torch.bfloat16, seed=9)
    g = torch.Generator().manual_seed(2)
    lat = torch.randn(dit.latent_shape(cfg, 128, 128, 5), generator=g).to(gpu, torch.bfloat16)
    txt = torch.randn(1, 8, 32, generator=g).to(gpu, torch.bfloat16)
    log = tmp_path / "raw.txt"
    cls = type("P", (WanAttn_SAPAttn_Processor,), {})
    replace_wan_attention(pipe, 128, 128, 5, first_layers_fp=0, first_times_fp=1000, num_q_centroids=4,
                          num_k_centroids=8, top_p_kmeans=0.9, min_kc_ratio=0.1, kmeans_iter_init=2,
                          kmeans_iter_step=2, measure_attention_sparsity=True, sparsity_output_file=str(log),
                          sparsity_threshold=0.95, processor_cls=cls)
    with torch.no_grad():
        for t in (999.0, 979.0):
            pipe.transformer(lat, torch.tensor([t], device=gpu), txt)
    torch.cuda.synchronize()
    data = merge_sparsity_data([log])
    assert sorted({(s, l) for s, l, _ in data}) == [(1, 0), (1, 1), (2, 0), (2, 1)]
    assert all(0.0 < v <= 1.0 for v in data.values())
    csv = tmp_path / "profile.csv"
    save_to_csv(data, csv)
    lk = SparsityLookup(str(csv), verbose=False)
    assert lk.has_data_for_step_layer(2, 1, 2)
