"""GPU tests of the attention processors (the drop-in boundary): the Wan and Hunyuan processors run
through the HIP library and are compared with the oracle or with a float32 torch computation of the
same projections, norms, RoPE and attention."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import svoo_oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2  # bf16 attention tolerance (max-abs) from the north-star contract
MIN_COS = 0.999


def say(*a):
    print("[case]", *a, flush=True)


def check(out, ref, scale=1.0):
    o = out.detach().double().cpu().numpy().reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    err = np.abs(o - r).max() / scale
    cos = float(o @ r / (np.linalg.norm(o) * np.linalg.norm(r) + 1e-30))
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)


class FakeWanAttn(torch.nn.Module):
    """The attributes the Wan processor reads from a diffusers ``WanAttention``."""

    def __init__(self, dim, heads):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = (torch.nn.Linear(dim, dim) for _ in range(3))
        self.norm_q, self.norm_k = torch.nn.RMSNorm(dim, eps=1e-6), torch.nn.RMSNorm(dim, eps=1e-6)
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(dim, dim), torch.nn.Identity()])
        self.add_k_proj = None


def _rope_tables(s, d, dev):
    pos = torch.arange(s, dtype=torch.float64)[:, None]
    freq = 1.0 / (10000 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = (pos * freq).repeat_interleave(2, dim=1)  # [S, D], pairs share an angle
    return ang.cos().float().to(dev), ang.sin().float().to(dev)


def _rope_ref(x, cos, sin):
    # interleaved pairs: (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    c, s_ = cos[..., 0::2], sin[..., 0::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s_
    out[..., 1::2] = x0 * s_ + x1 * c
    return out


def test_wan_processor_call_single_cluster_is_dense(gpu):
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    say("wan __call__ one cluster")
    torch.manual_seed(0)
    h, d, frames, fsize = 2, 128, 2, 96
    s = frames * fsize
    attn = FakeWanAttn(h * d, h).to(gpu)
    x = torch.randn(1, s, h * d, device=gpu)
    cos, sin = _rope_tables(s, d, gpu)
    with torch.no_grad():
        # float32 reference of the same computation
        q = attn.norm_q(attn.to_q(x)).unflatten(2, (h, d))
        k = attn.norm_k(attn.to_k(x)).unflatten(2, (h, d))
        v = attn.to_v(x).unflatten(2, (h, d))
        q = _rope_ref(q, cos[None, :, None], sin[None, :, None])
        k = _rope_ref(k, cos[None, :, None], sin[None, :, None])
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
        ref = attn.to_out[0](o.transpose(1, 2).flatten(2, 3))

        class P(WanAttn_SAPAttn_Processor):
            pass

        P.num_frame, P.frame_size, P.context_length = frames, fsize, 0
        P.num_q_centroids = P.num_k_centroids = 1
        P.top_p_kmeans, P.min_kc_ratio = 1.0, 0
        P.kmeans_iter_init = P.kmeans_iter_step = 2
        P.first_times_fp, P.first_layers_fp = 1e9, 0
        proc = P(layer_idx=0)
        attn_bf = attn.to(torch.bfloat16)
        out = proc(attn_bf, x.to(torch.bfloat16), rotary_emb=(cos[None, :, None], sin[None, :, None]),
                   timestep=torch.tensor([500.0], device=gpu))
    assert out.shape == (1, s, h * d)
    check(out, ref.cpu().numpy(), scale=float(ref.abs().max()))


def _hunyuan_proc(frames, fsize, ctx, prompt, qc, kc, iters, top_p, ratios, qi=None, ki=None, full=False):
    from svoo_amd.processor import Hunyuan_SAPAttn_Processor

    class P(Hunyuan_SAPAttn_Processor):
        pass

    P.num_frame, P.frame_size, P.context_length, P.prompt_length = frames, fsize, ctx, prompt
    P.num_q_centroids, P.num_k_centroids = qc, kc
    P.top_p_kmeans, P.min_kc_ratio = top_p, ratios
    P.kmeans_iter_init = P.kmeans_iter_step = iters
    P.first_times_fp = 1e9
    P.first_layers_fp = 1 if full else 0
    if qi is not None:
        P.kmeans_init_idx = (qi, ki)
    return P(layer_idx=0)


def _bf(shape, seed, dev):
    r = np.random.default_rng(seed)
    x = O.bf16_round(r.standard_normal(shape).astype(np.float32))
    return x, torch.from_numpy(x).to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("d", [128, 64])
def test_hunyuan_sparse_call_matches_oracle(gpu, d):
    say("hunyuan attention_core_logic sparse, head dim", d)
    from svoo_amd import synth

    # video tokens from the seeded Gaussian mixture (well separated: labels agree with the oracle),
    # text tokens appended
    cfg = synth.SynthConfig("hy-small", 41, 2, 2, 12, 16, d, 24, 12, 24, 3, 0.1, 0.4, True, "bf16")
    h, frames, fsize, ctx, prompt = cfg.heads, cfg.frames, cfg.frame_size, 32, 20
    s = frames * fsize + ctx
    vids = synth.make_qkv(cfg)
    txt = [_bf((1, h, ctx, d), seed, gpu)[0] for seed in (1, 2, 3)]
    full = [np.concatenate([vt_.float().numpy(), tx], axis=2) for vt_, tx in zip(vids, txt)]
    q, k, v = full
    qt, kt, vt = (torch.from_numpy(a).to(torch.bfloat16).to(gpu) for a in full)
    r = np.random.default_rng(4)
    qi = r.integers(0, frames * fsize, size=(h, 12))
    ki = r.integers(0, frames * fsize, size=(h, 24))
    ratios = [0.2, 0.3]
    proc = _hunyuan_proc(frames, fsize, ctx, prompt, 12, 24, 3, 0.9, ratios,
                         torch.from_numpy(qi).to(gpu), torch.from_numpy(ki).to(gpu))
    out = proc.attention_core_logic(qt, kt, vt, torch.tensor([100.0], device=gpu), 0)
    torch.cuda.synchronize()
    ref = O.hunyuan_attention_call(q, k, v, 12, 24, 3, 0.9, ratios, prompt, ctx, init_q_idx=qi, init_k_idx=ki)
    assert out.shape == (1, h, s, d)
    check(out, ref)


def test_hunyuan_dense_gate_matches_oracle(gpu):
    say("hunyuan attention_core_logic dense gate")
    h, frames, fsize, ctx, prompt = 2, 2, 96, 32, 9
    s = frames * fsize + ctx
    q, qt = _bf((1, h, s, 128), 5, gpu)
    k, kt = _bf((1, h, s, 128), 6, gpu)
    v, vt = _bf((1, h, s, 128), 7, gpu)
    proc = _hunyuan_proc(frames, fsize, ctx, prompt, 4, 8, 2, 0.9, 0.2, full=True)
    mask = torch.zeros(s, dtype=torch.bool, device=gpu)
    mask[: frames * fsize + prompt] = True
    out = proc.attention_core_logic(qt, kt, vt, torch.tensor([100.0], device=gpu), 0,
                                    proc.get_cu_max_seqlen(mask, gpu))
    check(out, O.hunyuan_dense_attention(q, k, v, frames * fsize + prompt))


class FakeHunyuanDoubleAttn(torch.nn.Module):
    """The attributes the Hunyuan processor reads from a diffusers double-stream ``Attention``."""

    def __init__(self, dim, heads, head_dim):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = (torch.nn.Linear(dim, dim) for _ in range(3))
        self.add_q_proj, self.add_k_proj, self.add_v_proj = (torch.nn.Linear(dim, dim) for _ in range(3))
        self.norm_q, self.norm_k = torch.nn.RMSNorm(head_dim, eps=1e-6), torch.nn.RMSNorm(head_dim, eps=1e-6)
        self.norm_added_q, self.norm_added_k = torch.nn.RMSNorm(head_dim, eps=1e-6), torch.nn.RMSNorm(head_dim, eps=1e-6)
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(dim, dim), torch.nn.Identity()])
        self.to_add_out = torch.nn.Linear(dim, dim)


def test_hunyuan_double_stream_call_dense_gate(gpu):
    say("hunyuan __call__ double stream, dense gate")
    torch.manual_seed(1)
    h, d, frames, fsize, ctx, prompt = 2, 128, 2, 64, 16, 10
    vl = frames * fsize
    dim = h * d
    attn = FakeHunyuanDoubleAttn(dim, h, d).to(gpu)
    x = torch.randn(1, vl, dim, device=gpu)
    enc = torch.randn(1, ctx, dim, device=gpu)
    cos, sin = _rope_tables(vl, d, gpu)
    mask = torch.zeros(vl + ctx, dtype=torch.bool, device=gpu)
    mask[: vl + prompt] = True
    with torch.no_grad():
        t = lambda y: y.unflatten(2, (h, d)).transpose(1, 2)  # noqa: E731
        q = _rope_ref(attn.norm_q(t(attn.to_q(x))), cos, sin)
        k = _rope_ref(attn.norm_k(t(attn.to_k(x))), cos, sin)
        v = t(attn.to_v(x))
        q = torch.cat([q, attn.norm_added_q(t(attn.add_q_proj(enc)))], dim=2)
        k = torch.cat([k, attn.norm_added_k(t(attn.add_k_proj(enc)))], dim=2)
        v = torch.cat([v, t(attn.add_v_proj(enc))], dim=2)
        allowed = mask[:, None] == mask[None, :]
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=allowed)
        o = o.transpose(1, 2).flatten(2, 3)
        ref_h, ref_e = attn.to_out[0](o[:, :vl]), attn.to_add_out(o[:, vl:])

        proc = _hunyuan_proc(frames, fsize, ctx, prompt, 4, 8, 2, 0.9, 0.2, full=True)
        attn_bf = attn.to(torch.bfloat16)
        out_h, out_e = proc(attn_bf, x.to(torch.bfloat16), enc.to(torch.bfloat16), mask, (cos, sin),
                            torch.tensor([100.0], device=gpu))
    assert out_h.shape == (1, vl, dim) and out_e.shape == (1, ctx, dim)
    check(out_h, ref_h.cpu().numpy(), scale=float(ref_h.abs().max()))
    check(out_e, ref_e.cpu().numpy(), scale=float(ref_e.abs().max()))


def test_wan_processor_fused_path_equals_separate_passes(gpu):
    """``fuse_permutes`` runs the same attention in one kernel: identical output bits."""
    from svoo_amd import synth
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    say("wan attention_core_logic fused vs separate permutes")
    cfg = synth.SynthConfig("fuse-small", 61, 2, 3, 16, 20, 128, 24, 12, 32, 3, 0.1, 0.4, True, "bf16")
    q, k, v = (x.to(gpu) for x in synth.make_qkv(cfg))
    r = np.random.default_rng(6)
    qi = torch.from_numpy(r.integers(0, cfg.video_tokens, size=(cfg.heads, 12))).to(gpu)
    ki = torch.from_numpy(r.integers(0, cfg.video_tokens, size=(cfg.heads, 32))).to(gpu)
    outs = []
    for fused in (False, True):
        class P(WanAttn_SAPAttn_Processor):
            pass

        P.num_frame, P.frame_size, P.context_length = cfg.frames, cfg.frame_size, 0
        P.num_q_centroids, P.num_k_centroids = 12, 32
        P.top_p_kmeans, P.min_kc_ratio = 0.7, 0.1
        P.kmeans_iter_init = P.kmeans_iter_step = 3
        P.first_times_fp, P.first_layers_fp = 1e9, 0
        P.kmeans_init_idx = (qi, ki)
        P.fuse_permutes = fused
        outs.append(P(layer_idx=0).attention_core_logic(q, k, v, torch.tensor([100.0], device=gpu)))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
