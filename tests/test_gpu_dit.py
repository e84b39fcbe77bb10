"""GPU tests of the processors inside a random-init Wan-shaped DiT (the C5 harness): processors installed by
``replace_wan_attention``, called from the blocks exactly as a pipeline calls them, over consecutive steps."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _pipe(gpu, layers=2, heads=2):
    from svoo_amd import dit

    cfg = dit.WanDiTConfig(num_attention_heads=heads, ffn_dim=512, num_layers=layers, text_dim=64)
    return dit.make_pipe(cfg, device=gpu, dtype=torch.bfloat16, seed=5)


def _inputs(pipe, gpu, h=256, w=256, frames=9, seed=0):
    from svoo_amd import dit

    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(dit.latent_shape(pipe.transformer.config, h, w, frames), generator=g)
    txt = torch.randn(1, 16, pipe.transformer.config.text_dim, generator=g)
    return lat.to(gpu, torch.bfloat16), txt.to(gpu, torch.bfloat16)


def _cls():
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    return type("P", (WanAttn_SAPAttn_Processor,), {})


def test_dit_one_cluster_matches_dense_dit(gpu):
    from svoo_amd import dit
    from svoo_amd.inference import replace_wan_attention

    say("tiny DiT, one cluster, all-true map vs dense processors")
    pipe = _pipe(gpu)
    lat, txt = _inputs(pipe, gpu)
    t = torch.tensor([500.0], device=gpu)
    with torch.no_grad():
        ref = pipe.transformer(lat, t, txt).float()
        cls = _cls()
        replace_wan_attention(pipe, 256, 256, 9, first_layers_fp=0, first_times_fp=1e9, num_q_centroids=1,
                              num_k_centroids=1, top_p_kmeans=1.0, min_kc_ratio=0, kmeans_iter_init=2,
                              kmeans_iter_step=2, processor_cls=cls)
        out = pipe.transformer(lat, t, txt).float()
        torch.cuda.synchronize()
    assert all(isinstance(b.attn1.processor, cls) for b in pipe.transformer.blocks)
    assert all(b.attn1.processor._last_call is not None for b in pipe.transformer.blocks)  # sparse path ran
    err = (out - ref).abs().max().item() / ref.abs().max().item()
    cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0).item()
    assert err <= 2e-2 and cos >= 0.999, (err, cos)
    for b in pipe.transformer.blocks:
        b.attn1.set_processor(dit.DenseWanAttnProcessor())


def test_dit_three_steps_profile_reuse_and_warm_start(gpu, tmp_path):
    from svoo_amd.inference import replace_wan_attention

    say("tiny DiT, 3 steps, per-(layer, head) profile, reuse from step 3, warm start")
    layers, heads, kc = 2, 2, 16
    rng = np.random.default_rng(5)
    rho = rng.uniform(0.05, 0.4, size=(3, layers, heads))
    csv = tmp_path / "profile.csv"
    with open(csv, "w") as f:
        f.write("Step,Layer,Head,Sparsity\n")
        for s in range(3):
            for l in range(layers):
                for h in range(heads):
                    f.write(f"{s + 1},{l},{h},{rho[s, l, h]:.4f}\n")
    pipe = _pipe(gpu, layers, heads)
    lat, txt = _inputs(pipe, gpu, seed=1)
    cls = _cls()
    cls.kmeans_warm_start = True
    procs = replace_wan_attention(pipe, 256, 256, 9, first_layers_fp=0, first_times_fp=1000, num_q_centroids=8,
                                  num_k_centroids=kc, top_p_kmeans=0.0, min_kc_ratio=0.1, kmeans_iter_init=3,
                                  kmeans_iter_step=2, start_reuse_step=2, reuse_interval=10,
                                  use_dynamic_min_kc_ratio=True, sparsity_csv_path=str(csv), processor_cls=cls)
    cached = {}
    with torch.no_grad():
        for step, tval in enumerate((999.0, 979.0, 959.0), start=1):
            out = pipe.transformer(lat, torch.tensor([tval], device=gpu), txt)
            torch.cuda.synchronize()
            assert torch.isfinite(out.float()).all()
            for p in procs:
                assert p.current_inference_step == step
                lc = p._last_call
                # density mode: each q-cluster keeps exactly max(1, floor(rho * Kc)) key clusters
                rows = lc["map"][0].sum(-1).cpu().numpy()
                want = [max(1, int(float(np.float32(float(f"{rho[step - 1, p.layer_idx, h]:.4f}"))) * kc))
                        for h in range(heads)]
                assert (rows == np.array(want)[:, None]).all(), (step, p.layer_idx, rows, want)
                cached.setdefault(p.layer_idx, []).append(id(p._cached_clustering_results))
                assert p.centroids_init and p.q_centroids is not None
    for ids in cached.values():
        assert ids[0] != ids[1]  # step 2 re-clusters (the reuse anchor), warm-started from step 1's centroids
        assert ids[1] == ids[2]  # step 3 reuses step 2's clustering
