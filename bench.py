#!/usr/bin/env python3
"""Benchmark of the SVOO attention call on one MI355X.

One step is one full ``attention_core_logic`` call of the SVOO processor at the Wan2.1-14B 720p
layer shape (H=40, N=75600, d=128, bf16): 5 warm-started co-clustering iterations (100 query /
1000 key clusters), per-head block mask, permutes of Q/K/V, variable-block-sparse attention and
the inverse permutation.  Inputs are synthetic (seeded Gaussian mixture with per-frame drift, drawn
on the device) and resident in HBM before timing starts.

Prints ONE JSON line: ``value`` is the dense-equivalent throughput ``4*H*N^2*d / t_call``
(TFLOP/s), ``ms_per_step`` the call latency.  Extra fields give the stage breakdown (HIP events on
the stream the kernels run on), the dense SDPA comparator at equal shape, the roofline of the
dominant kernel (the sparse attention) and a CPU baseline (the numpy oracle on a bounded sample of
the same inputs, rank 0 only).

    python bench.py [--steps K] [--warmup W] [--config C3] [--mode density|reference]
"""

from __future__ import annotations

import argparse
import contextlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "SVOO attention-call latency (ms) + effective TFLOP/s, Wan-14B 720p shape, 1 GPU"
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C3", choices=["C2", "C3", "C4", "C5"],
                    help="C2-C4: one SVOO attention call; C5: one denoising step of a random-init Wan2.1-1.3B DiT")
    ap.add_argument("--mode", default="density", choices=["density", "reference"],
                    help="density: top_p=0, min_kc_ratio=rho_h; reference: top_p=0.9, min_kc_ratio=clip(rho_h,0.15,0.2)")
    ap.add_argument("--pattern", default="SAP", choices=["SAP", "EAR"],
                    help="SAP: top-p block mask (the headline); EAR: error-aware routing with centroid compensation "
                         "(Wan configs)")
    ap.add_argument("--sparsity-profile", action="store_true",
                    help="time the offline profile producer (exact per-head sparsity of one layer) instead")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense SDPA comparator")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-kernel-table", action="store_true",
                    help="skip the per-kernel table (one extra call under torch.profiler)")
    ap.add_argument("--cpu-heads", type=int, default=2,
                    help="heads in the CPU baseline sample (a fixed subset spread over the heads)")
    ap.add_argument("--traffic", default=str(ROOT / "profiles" / "vbsa_attn_C3_traffic.json"),
                    help="measured HBM traffic of the attention kernel (from rocprofv3 --pmc), if present")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run three 1 GiB device copies (the known-size reference for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE scaling) and exit")
    return ap.parse_args()


def cpu_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        n = [i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"]
        if n:
            return int(max(n))
    except Exception:
        pass
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the SVOO call is per-head independent and this build runs on "
              "a single MI355X (multi-GPU sharding is design-only); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        import torch

        src = torch.empty((1 << 30) // 2, dtype=torch.bfloat16, device="cuda:0").normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("three 1 GiB copies done")
        return
    if args.config == "C5":
        return main_dit(args)
    if args.sparsity_profile:
        return main_profile(args)

    import numpy as np
    import torch

    from svoo_amd import _lib, synth
    from svoo_amd.co_clustering import co_cluster_tokens_full
    from svoo_amd.processor import Hunyuan_SAPAttn_Processor, WanAttn_EARAttn_Processor, WanAttn_SAPAttn_Processor

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    _lib.lib()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS[args.config]
    h, n, d = cfg.heads, cfg.tokens, cfg.head_dim
    qcn, kcn, iters = cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters
    hunyuan = cfg.text_tokens > 0
    nv = cfg.video_tokens
    ear = args.pattern == "EAR"
    if ear and hunyuan:
        raise SystemExit("EAR is wired for the Wan processor only (as in the reference)")

    log(f"config {cfg.name}: H={h} N={n} d={d} Qc={qcn} Kc={kcn} iters={iters} mode={args.mode} "
        f"pattern={args.pattern}")
    t0 = time.time()
    q, k, v = synth.make_qkv_device(cfg, dev)
    torch.cuda.synchronize()
    log(f"inputs drawn on device in {time.time() - t0:.1f}s")

    rho = synth.head_densities(cfg)
    if args.mode == "density":
        top_p, ratios = 0.0, rho
    else:
        top_p, ratios = 0.9, [min(max(r, 0.15), 0.20) for r in rho]

    # "Previous step": a clustering from seeded random token indices; the timed calls warm-start
    # from its centroids perturbed by N(0, (0.05 rms)^2).
    qv, kv = (x[0, :, :nv].contiguous() for x in (q, k))
    qi = synth.init_indices(cfg, h, qcn, nv, 1).to(dev)
    ki = synth.init_indices(cfg, h, kcn, nv, 2).to(dev)
    prev = co_cluster_tokens_full(qv, kv, qcn, kcn, iters, init_q_idx=qi, init_k_idx=ki)
    del qv, kv
    q_init = synth.perturb_centroids(cfg, prev["qcentroids"], 3)
    k_init = synth.perturb_centroids(cfg, prev["kcentroids"], 4)
    del prev

    class Proc(Hunyuan_SAPAttn_Processor if hunyuan else (WanAttn_EARAttn_Processor if ear else
                                                         WanAttn_SAPAttn_Processor)):
        pass

    Proc.num_frame, Proc.frame_size = cfg.frames, cfg.frame_size
    Proc.context_length = cfg.text_tokens
    if hunyuan:
        # all text tokens are the valid prompt: the padding cluster is empty
        Proc.prompt_length = cfg.text_tokens
        Proc.first_times_fp = float("inf")
    Proc.num_q_centroids, Proc.num_k_centroids = qcn, kcn
    Proc.top_p_kmeans, Proc.min_kc_ratio, Proc.max_kc_ratio = top_p, ratios, 0
    Proc.kmeans_iter_init = Proc.kmeans_iter_step = iters
    Proc.kmeans_warm_start = True
    Proc.centroids_init = True
    Proc.enable_mem_save = True
    proc = Proc(layer_idx=0)

    def step(events=None):
        proc.q_centroids, proc.k_centroids = q_init, k_init
        proc._cached_clustering_results = None
        proc.current_inference_step = None
        proc.stage_events = events
        if hunyuan:
            return proc.attention_core_logic(q, k, v, 0.0, 0)
        return proc.attention_core_logic(q, k, v, timestep=None)

    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize()
    log("warmup done")

    # Timed region: K full calls; stage events are recorded on the current stream inside each call.
    all_events = []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        ev = []
        out = step(ev)
        all_events.append(ev)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    t_call_ms = start.elapsed_time(end) / args.steps
    log(f"timed {args.steps} calls: {t_call_ms:.3f} ms/call (host wall {1e3 * wall / args.steps:.3f} ms/call)")

    # stage = time between a mark and the previous one, in the order the call records them
    stage = {}
    for ev in all_events:
        for (_, e0), (nm, e1) in zip(ev[:-1], ev[1:]):
            stage.setdefault(nm, []).append(e0.elapsed_time(e1))
    stages_ms = {nm: float(np.median(vals)) for nm, vals in stage.items()}
    attn_ms_avg = float(np.mean(stage["attention"]))
    # each call's span from its first to its last stage mark (the same stream): the spread over the K calls
    per_call = [ev[0][1].elapsed_time(ev[-1][1]) for ev in all_events]

    # Work of the last call (every call starts from the same centroids, so all calls are equal).
    last = proc._last_call
    qs = last["q_sizes"].to(torch.int64)
    ks = last["k_sizes"].to(torch.int64)
    dmap = last["map"]
    pairs = int((dmap.to(torch.int64) * qs[..., :, None] * ks[..., None, :]).sum().item())
    # EAR: every query row also scores the centroids of its inactive clusters
    cent_pairs = int(((~dmap).to(torch.int64).sum(-1) * qs).sum().item()) if ear else 0
    active_flop = 4.0 * d * (pairs + cent_pairs)
    dense_flop = cfg.dense_flops()
    realized_density = pairs / (h * float(n) ** 2)
    active_tflops = active_flop / (attn_ms_avg * 1e-3) / 1e12
    permute_bytes = 4 * (2 * h * n * d * 2 + h * n * 4)
    if "permute" in stages_ms:
        permute_ms = stages_ms["permute"] + stages_ms["unpermute"]
        permute_fused = False
    else:
        # The SAP call (Wan, HunyuanVideo) reads Q/K/V through the sorted indices inside the attention kernel; the permute
        # operators (the reference's separate passes) are timed on their own at the same size.
        from svoo_amd.permute import apply_inverse_permutation_bshd, permute_pair_by_indices
        from svoo_amd.processor import _permute_rows

        clu = last["clustering"]
        # HunyuanVideo: the whole sequence's indices (text rows map to themselves)
        qix, kix = last.get("q_idx", clu["q_sorted_idx"]), last.get("k_idx", clu["k_sorted_idx"])

        def permutes():
            qp = _permute_rows(q, qix)
            permute_pair_by_indices(k, v, kix)
            apply_inverse_permutation_bshd(qp, qix)

        permutes()
        torch.cuda.synchronize()
        ps_, pe_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ps_.record()
        for _ in range(3):
            permutes()
        pe_.record()
        torch.cuda.synchronize()
        permute_ms = ps_.elapsed_time(pe_) / 3
        permute_fused = True
    eff_tflops = dense_flop / (t_call_ms * 1e-3) / 1e12

    # Reuse step: clustering cached, mask + permutes + attention + unpermute only.
    proc._step_from_callback = 2
    Proc.start_reuse_step, Proc.reuse_interval = 1, 1000
    proc.stage_events = None
    call = (lambda: proc.attention_core_logic(q, k, v, 0.0, 0)) if hunyuan else (
        lambda: proc.attention_core_logic(q, k, v, timestep=None))
    call()  # warm-up; reuses the last timed call's clustering
    assert proc.should_recluster() is False
    torch.cuda.synchronize()
    rs, re_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    nreuse = max(3, args.steps // 2)
    rs.record()
    for _ in range(nreuse):
        call()
    re_.record()
    torch.cuda.synchronize()
    reuse_ms = rs.elapsed_time(re_) / nreuse
    del proc._step_from_callback
    log(f"reuse step {reuse_ms:.3f} ms")

    # Dense comparators at equal shape, each timed per repetition: torch SDPA (flash / memory-efficient kernels
    # only, the reference's dense path) and this library's attention kernel on an all-true one-cluster map.
    def timed_reps(fn, reps):
        fn()
        torch.cuda.synchronize()
        out_ms = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            out_ms.append(a.elapsed_time(b))
        return out_ms

    sdpa_reps, own_reps = None, None
    if not args.no_dense:
        try:
            from torch.nn.attention import SDPBackend, sdpa_kernel

            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                sdpa_reps = timed_reps(lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v), 3)
            log(f"dense SDPA {np.median(sdpa_reps):.2f} ms (reps {[round(x, 2) for x in sdpa_reps]})")
        except Exception as e:  # the comparator is informative only
            log(f"dense SDPA comparator unavailable: {e!r}")
        from svoo_amd.co_clustering import dynamic_block_sparse_fwd

        full_sz = torch.full((1, h, 1), n, dtype=torch.int32, device=dev)
        full_map = torch.ones(1, h, 1, 1, dtype=torch.bool, device=dev)
        own_reps = timed_reps(lambda: dynamic_block_sparse_fwd(q, k, v, full_map, full_sz, full_sz, validate=False), 3)
        log(f"dense (this library's kernel, all-true map) {np.median(own_reps):.2f} ms")
    t_sdpa_ms = None if sdpa_reps is None else float(np.median(sdpa_reps))
    t_own_ms = None if own_reps is None else float(np.median(own_reps))

    kernels = None
    if not args.no_kernel_table:
        try:
            kernels = kernel_table(step, cfg, h, nv, d, qcn, kcn, iters)
        except Exception as e:  # informative only
            log(f"per-kernel table unavailable: {e!r}")

    traffic = None
    tpath = Path(args.traffic)
    if tpath.exists():
        try:
            tj = json.loads(tpath.read_text())
            if tj.get("workload") == cfg.name and tj.get("mode") == args.mode:
                traffic = float(tj["hbm_bytes_per_launch"])
        except Exception as e:
            log(f"traffic file unreadable: {e!r}")

    roofline = {
        "kernel": "vbsa_attn_kernel" + ("<EAR>" if ear else ""),
        "bound": "mfma",
        "achieved": round(active_tflops, 2),
        "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(active_tflops / BF16_PEAK_TFLOPS, 4),
        "traffic": traffic,
        "avg_launch_ms": round(attn_ms_avg, 4),
        "flop_per_launch": active_flop,
    }

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, q, k, v, q_init, k_init, top_p, ratios, args.cpu_heads, t_call_ms, hunyuan, ear)

    line = {
        "metric": METRIC,
        "value": round(eff_tflops, 2),
        "unit": "TFLOP/s (dense-equivalent, 4*H*N^2*d / t_call)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_call_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Gaussian mixture with per-frame drift, drawn on device)",
        "config": {
            "workload": f"{cfg.name}: one SVOO{'-EAR' if ear else ''} attention call, H={h} N={n} d={d} "
                        f"Qc={qcn} Kc={kcn}, {iters} warm-started k-means iterations, {args.mode} mask mode",
            "heads": h, "tokens": n, "head_dim": d, "q_clusters": qcn, "k_clusters": kcn,
            "kmeans_iters": iters, "top_p": top_p, "mask_mode": args.mode, "pattern": args.pattern,
        },
        "latency_ms": round(t_call_ms, 4),
        "reuse_step_ms": round(reuse_ms, 4),
        "stages_ms": {kk: round(vv, 4) for kk, vv in stages_ms.items()},
        "text_tokens": cfg.text_tokens,
        "realized_density": round(realized_density, 5),
        "centroid_pairs": cent_pairs,
        "active_tflops": round(active_tflops, 2),
        "permute_gbps": round(permute_bytes / (permute_ms * 1e-3) / 1e9, 1),
        "permutes_fused_into_attention": permute_fused,
        "permute_frac_hbm": round(permute_bytes / (permute_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "call_ms_spread": {"min": round(min(per_call), 4), "median": round(float(np.median(per_call)), 4),
                           "max": round(max(per_call), 4), "calls": len(per_call)},
        "t_sdpa_ms": None if t_sdpa_ms is None else round(t_sdpa_ms, 3),
        "t_sdpa_ms_reps": None if sdpa_reps is None else [round(x, 3) for x in sdpa_reps],
        "speedup_vs_dense": None if t_sdpa_ms is None else round(t_sdpa_ms / t_call_ms, 3),
        "speedup_vs_dense_spread": None if sdpa_reps is None else {
            "min": round(min(sdpa_reps) / max(per_call), 3), "max": round(max(sdpa_reps) / min(per_call), 3)},
        "t_dense_own_kernel_ms": None if t_own_ms is None else round(t_own_ms, 3),
        "dense_own_kernel_tflops": None if t_own_ms is None else round(dense_flop / (t_own_ms * 1e-3) / 1e12, 1),
        "speedup_vs_dense_own_kernel": None if t_own_ms is None else round(t_own_ms / t_call_ms, 3),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def kernel_table(step, cfg, h, nv, d, qcn, kcn, iters):
    """Device time of every kernel of one call, from one extra call under torch.profiler (outside the timed
    region), and roofline figures for the clustering kernels: the assignment's key side (J = Kc, MFMA bound:
    2*d*J FLOP per token of the reduced form) and query side (J = Qc, HBM bound: a 256-byte token row read and
    a 4-byte label written), the sorted centroid sums (HBM: the row, its index and label per token) and the
    incremental update.  Launch order inside the co-clustering alternates key side, query side."""
    import torch
    from torch.profiler import ProfilerActivity, profile

    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        step()
        torch.cuda.synchronize()
    evs = [e for e in prof.events() if getattr(e, "device_type", None) is not None
           and str(e.device_type).endswith("CUDA") and e.time_range.elapsed_us() > 0]
    evs.sort(key=lambda e: e.time_range.start)

    def short(name):
        base = name.split("(")[0].replace("void ", "").strip()
        return base.split("::")[-1].split("<")[0]

    table = {}
    for e in evs:
        t = table.setdefault(short(e.name), {"count": 0, "total_us": 0.0})
        t["count"] += 1
        t["total_us"] += e.time_range.elapsed_us()
    for t in table.values():
        t["avg_us"] = round(t["total_us"] / t["count"], 2)
        t["total_us"] = round(t["total_us"], 1)

    def launches(name):
        return [e.time_range.elapsed_us() for e in evs if short(e.name) == name]

    out = {"per_kernel": dict(sorted(table.items(), key=lambda kv: -kv[1]["total_us"]))}
    bh = h
    stage = {}
    # Passes of the co-clustering, in launch order: each starts with its prep kernel and alternates key side,
    # query side.  A key-side pass from the second iteration on is the candidate pass (radius, lists, score
    # kernels) when the library takes it, else the full pass; each ends with the hi/lo kernel on the tokens it
    # left (cocluster_assign_kernel).
    passes = []
    for e in evs:
        nm = short(e.name)
        if nm.startswith("cocluster_prep"):
            passes.append({"side": "key" if len(passes) % 2 == 0 else "query", "k": {}})
        if passes and nm.startswith("cocluster_"):
            passes[-1]["k"].setdefault(nm, []).append(e.time_range.elapsed_us())
    tot = lambda pz, names: sum(sum(pz["k"].get(nm, [])) for nm in names)  # noqa: E731
    key_passes = [pz for pz in passes if pz["side"] == "key"]
    qry_passes = [pz for pz in passes if pz["side"] == "query"]
    full_names = ("cocluster_assign16_kernel", "cocluster_assign_kernel")
    cand_names = ("cocluster_nu_kernel", "cocluster_radius_kernel", "cocluster_lists_kernel",
                  "cocluster_score_kernel", "cocluster_assign_kernel")
    if key_passes and "cocluster_assign16_kernel" in key_passes[0]["k"]:
        # the first key-side pass scores every cluster for every token: its MFMA roofline
        key_us = tot(key_passes[0], full_names)
        key_flop = 2.0 * bh * nv * d * kcn
        stage["assign_key_side"] = {"bound": "mfma", "achieved": round(key_flop / (key_us * 1e-6) / 1e12, 1),
                                    "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(key_flop / (key_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                                    "full_pass_us": round(key_us, 2),
                                    "fallback_us": round(tot(key_passes[0], ("cocluster_assign_kernel",)), 2),
                                    "note": "first iteration: fp16 certified pass + hi/lo fallback; algorithmic "
                                            "FLOP of the reduced form"}
        cand = [pz for pz in key_passes[1:] if "cocluster_score_kernel" in pz["k"]]
        full_later = [pz for pz in key_passes[1:] if "cocluster_assign16_kernel" in pz["k"]]
        if cand:
            # the first candidate pass measures the radii (radius kernel); later ones check each token's radius in
            # the score kernel against the one its anchor's list was built for
            def part(pzs, names):
                return round(sum(tot(pz, names) for pz in pzs) / len(pzs), 2) if pzs else None

            first, later = cand[:1], cand[1:]
            stage["key_candidate_passes"] = {
                "passes": len(cand), "avg_us": part(cand, cand_names),
                "first_pass_us": part(first, cand_names), "later_passes_avg_us": part(later, cand_names),
                "radius_us": part(first, ("cocluster_radius_kernel",)),
                "lists_us": part(cand, ("cocluster_lists_kernel",)),
                "score_first_us": part(first, ("cocluster_score_kernel",)),
                "score_later_us": part(later, ("cocluster_score_kernel",)),
                "fallback_us": part(cand, ("cocluster_assign_kernel",)),
                "note": "iterations 2+: triangle-inequality candidates in profile space, exact (same labels)"}
        if full_later:
            stage["key_full_passes_later_avg_us"] = round(
                sum(tot(pz, full_names) for pz in full_later) / len(full_later), 2)
    if qry_passes and "cocluster_assign16_kernel" in qry_passes[0]["k"]:
        # the query side's later passes run only on the tokens the pruning test left, so its HBM roofline is
        # taken on the first iteration's full pass
        qry_full_us = tot(qry_passes[0], full_names)
        qry_later = [tot(pz, full_names) for pz in qry_passes[1:]]
        qry_bytes = bh * nv * (2 * d + 4)
        stage["assign_query_side"] = {"bound": "hbm", "achieved": round(qry_bytes / (qry_full_us * 1e-6) / 1e9, 1),
                                      "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                                      "frac": round(qry_bytes / (qry_full_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                                      "first_pass_us": round(qry_full_us, 2),
                                      "pruned_passes_avg_us": round(sum(qry_later) / len(qry_later), 2)
                                      if qry_later else None}
    pr = launches("cocluster_prune_kernel")
    if pr:
        stage["prune"] = {"avg_us": round(sum(pr) / len(pr), 2), "launches": len(pr),
                          "note": "exact bound test before each later query-side pass"}
    acc = launches("centroid_accumulate_kernel")
    if acc:
        # the first iteration's two launches sum every token (sorted order)
        full = acc[:2]
        acc_bytes = bh * nv * (2 * d + 8) * len(full)
        ach = acc_bytes / (sum(full) * 1e-6) / 1e9
        stage["centroid_accumulate"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                                        "full_pass_avg_us": round(sum(full) / len(full), 2)}
    mv = launches("centroid_move_kernel")
    if mv:
        stage["centroid_move"] = {"avg_us": round(sum(mv) / len(mv), 2), "launches": len(mv),
                                  "note": "later iterations: moves only the tokens whose label changed, or "
                                          "recounts from the sorted labels when many changed (chosen on the device)"}
    out["clustering"] = stage
    return out


def main_dit(args):
    """C5: denoising steps of a random-init Wan2.1-T2V-1.3B-shaped DiT (30 blocks, dim 1536, 12 heads, FFN 8960,
    480x832x81 video -> N = 21 x 30 x 52 = 32760 tokens) with the SVOO processor in every block's self-attention,
    installed by ``replace_wan_attention`` with the reference launcher's 1.3B settings (Qc=256, Kc=1024, 2 k-means
    iterations per clustering).  The per-(step, layer, head) profile is synthetic, rho ~ U[0.05, 0.4], read through
    ``SparsityLookup`` from a CSV.  Centroids are carried from step to step (warm start).  Three kinds of step are
    timed: a re-clustering step, a reuse step (clustering cached) and the same DiT with dense SDPA self-attention."""
    import tempfile

    import numpy as np
    import torch

    from svoo_amd import _lib, dit
    from svoo_amd.inference import replace_wan_attention
    from svoo_amd.processor import WanAttn_SAPAttn_Processor

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    _lib.lib()
    dev = torch.device("cuda:0")
    cfg = dit.WanDiTConfig()
    height, width, frames = 480, 832, 81
    t0 = time.time()
    pipe = dit.make_pipe(cfg, device=dev, dtype=torch.bfloat16, seed=5)
    model = pipe.transformer
    g = torch.Generator(device=dev).manual_seed(5)
    lat = torch.randn(dit.latent_shape(cfg, height, width, frames), generator=g, device=dev).to(torch.bfloat16)
    txt = torch.randn(1, 512, cfg.text_dim, generator=g, device=dev).to(torch.bfloat16)
    torch.cuda.synchronize()
    log(f"C5 DiT built ({sum(p.numel() for p in model.parameters()) / 1e9:.2f} B params) in {time.time() - t0:.1f}s")

    nsteps = args.warmup + 2 * args.steps + 4  # every step the run takes has a profile row
    layers, heads = cfg.num_layers, cfg.num_attention_heads
    rho = np.random.default_rng(5).uniform(0.05, 0.4, size=(nsteps + 1, layers, heads))
    if args.mode == "density":
        top_p, dmin, dmax = 0.0, None, None
    else:
        top_p, dmin, dmax = 0.9, 0.15, 0.20

    class Proc(WanAttn_SAPAttn_Processor):
        kmeans_warm_start = True

    with tempfile.TemporaryDirectory() as tdir:
        csv = Path(tdir) / "profile.csv"
        with open(csv, "w") as f:
            f.write("Step,Layer,Head,Sparsity\n")
            for st in range(nsteps + 1):
                for ly in range(layers):
                    for hd in range(heads):
                        f.write(f"{st + 1},{ly},{hd},{rho[st, ly, hd]:.4f}\n")
        # the profile loader reports on stdout; keep stdout for the one JSON line
        with contextlib.redirect_stdout(sys.stderr):
            procs = replace_wan_attention(
                pipe, height, width, frames, first_layers_fp=0, first_times_fp=1000.0, num_q_centroids=256,
                num_k_centroids=1024, top_p_kmeans=top_p, min_kc_ratio=0.10, kmeans_iter_init=2, kmeans_iter_step=2,
                start_reuse_step=None, reuse_interval=1, use_dynamic_min_kc_ratio=True, sparsity_csv_path=str(csv),
                dynamic_min_kc_ratio_min=dmin, dynamic_min_kc_ratio_max=dmax, processor_cls=Proc)
    n = Proc.num_frame * Proc.frame_size
    assert n == 32760, n
    timesteps = iter(np.linspace(999.0, 600.0, 10 * nsteps))

    def fwd(events=False):
        for p in procs:
            p.stage_events = [] if events else None
        t = torch.tensor([float(next(timesteps))], device=dev)
        with torch.no_grad():
            return model(lat, t, txt)

    def timed(k, events=False):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        calls = []
        for _ in range(k):
            fwd(events)
            if events:
                calls.append([p.stage_events for p in procs])
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / k, calls

    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    log("warmup done")
    # re-clustering steps (2 warm-started iterations per block), stage events on every block
    t_step, calls = timed(args.steps, events=True)
    call_ms = [ev[0][1].elapsed_time(ev[-1][1]) for step in calls for ev in step]
    stage = {}
    for step in calls:
        for ev in step:
            for (_, e0), (nm, e1) in zip(ev[:-1], ev[1:]):
                stage.setdefault(nm, []).append(e0.elapsed_time(e1))
    stages_ms = {nm: float(np.sum(v)) / args.steps for nm, v in stage.items()}
    svoo_ms = float(np.sum(call_ms)) / args.steps
    pairs = 0
    for p in procs:
        lc = p._last_call
        qs, ks = lc["q_sizes"].to(torch.int64), lc["k_sizes"].to(torch.int64)
        pairs += int((lc["map"].to(torch.int64) * qs[..., :, None] * ks[..., None, :]).sum().item())
    density = pairs / (layers * heads * float(n) ** 2)
    log(f"re-clustering step {t_step:.2f} ms (SVOO calls {svoo_ms:.2f} ms over {layers} blocks)")

    # reuse steps: the clustering of the last step is reused by every block
    Proc.start_reuse_step, Proc.reuse_interval = procs[0].current_inference_step + 1, 10 ** 6
    fwd()
    t_reuse, _ = timed(args.steps)
    assert not any(p.should_recluster() for p in procs)
    log(f"reuse step {t_reuse:.2f} ms")

    t_dense = None
    if not args.no_dense:
        for b in model.blocks:
            b.attn1.set_processor(dit.DenseWanAttnProcessor())
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            fwd()
            t_dense, _ = timed(max(2, args.steps // 2))
        log(f"dense step {t_dense:.2f} ms")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_dit(model, lat, txt, rho, top_p, dmin, dmax, args.cpu_heads, t_step, dev)

    line = {
        "metric": "Wan2.1-1.3B DiT denoising-step latency with SVOO self-attention (ms), 1 GPU",
        "value": round(t_step, 3),
        "unit": "ms per denoising step (re-clustering step)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, Gaussian latents and text embeddings, U[0.05,0.4] profile)",
        "config": {
            "workload": f"C5-wan2.1-1.3B-dit-step: 30 blocks, dim 1536, 12 heads, FFN 8960, N={n}, 512 text tokens, "
                        f"Qc=256 Kc=1024, 2 warm-started k-means iterations per block, {args.mode} mask mode",
            "layers": layers, "heads": heads, "tokens": n, "q_clusters": 256, "k_clusters": 1024,
            "kmeans_iters": 2, "top_p": top_p, "mask_mode": args.mode,
        },
        "reuse_step_ms": round(t_reuse, 3),
        "dense_step_ms": None if t_dense is None else round(t_dense, 3),
        "speedup_vs_dense": None if t_dense is None else round(t_dense / t_step, 3),
        "reuse_speedup_vs_dense": None if t_dense is None else round(t_dense / t_reuse, 3),
        "svoo_calls_ms": round(svoo_ms, 3),
        "stages_ms": {kk: round(vv, 3) for kk, vv in stages_ms.items()},
        "realized_density": round(density, 5),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def main_profile(args):
    """Offline profile producer on one layer of the chosen config (default inputs of C2/C3/C4): exact
    per-head sparsity (threshold 0.95, every query row) with ``compute_exact_attention_sparsity``.
    Timed: the whole call, and inside it the score GEMMs and the HIP count kernel separately; beside
    it, the reference's own formulation (fp32 softmax, sort, cumsum, searchsorted) on the same GPU
    and inputs for a sample of rows, and the numpy oracle on the host for a sample of rows."""
    import numpy as np
    import torch

    from svoo_amd import _lib, synth
    from svoo_amd.sparsity import compute_exact_attention_sparsity, exact_counts_from_scores

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    _lib.lib()
    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS[args.config]
    h, n, d = cfg.heads, cfg.tokens, cfg.head_dim
    q, k, _ = synth.make_qkv_device(cfg, dev)
    torch.cuda.synchronize()
    thr = 0.95
    scale = d ** -0.5
    # warm-up on a slice, then the timed full call
    compute_exact_attention_sparsity(q[:, :, :256], k, threshold=thr)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    avg, per_head, stats = compute_exact_attention_sparsity(q, k, threshold=thr)
    e1.record()
    torch.cuda.synchronize()
    t_call = e0.elapsed_time(e1)
    chunk = stats["chunk_size"]
    log(f"profile producer {cfg.name}: {t_call:.1f} ms per layer (chunk {chunk} rows), avg sparsity {avg:.4f}")

    # split: GEMM and count kernel on one chunk, scaled by the number of chunks
    rows = min(chunk, n)
    kt = k.transpose(-2, -1)
    g0, g1, c1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    g0.record()
    sc = torch.matmul(q[:, :, :rows], kt)
    g1.record()
    exact_counts_from_scores(sc, scale, thr)
    c1.record()
    torch.cuda.synchronize()
    nchunks = (n + rows - 1) // rows
    t_gemm = g0.elapsed_time(g1) * n / rows
    t_count = g1.elapsed_time(c1) * n / rows
    count_bytes = 3 * 2.0 * h * rows * n  # three passes over bf16 scores
    count_gbps = count_bytes / (g1.elapsed_time(c1) * 1e-3) / 1e9

    # the reference formulation on the same GPU for a sample of rows (fp32 probabilities, sort, cumsum)
    sample = min(512, n)
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record()
    w = torch.softmax(torch.matmul(q[:, :, :sample], kt).float() * scale, dim=-1)
    cs = torch.cumsum(torch.sort(w, dim=-1, descending=True).values, dim=-1)
    ref_counts = torch.searchsorted(cs, (thr * cs[..., -1:]).contiguous(), right=False, out_int32=True).squeeze(-1) + 1
    r1.record()
    torch.cuda.synchronize()
    t_ref = r0.elapsed_time(r1) * n / sample
    mine = exact_counts_from_scores(torch.matmul(q[:, :, :sample], kt), scale, thr)
    agree = float((mine == ref_counts).float().mean().item())
    maxdiff = int((mine - ref_counts).abs().max().item())
    del w, cs
    log(f"reference formulation on the GPU: {t_ref:.1f} ms per layer (from {sample} rows); counts agree on "
        f"{agree * 100:.2f}% of rows, max difference {maxdiff}")

    cpu = None
    if not args.no_cpu:
        from oracle import svoo_oracle as O

        rows_cpu = 8
        s_cpu = torch.matmul(q[:, :1, :rows_cpu], kt[:, :1]).float().cpu().numpy()
        t0 = time.perf_counter()
        O.exact_sparsity_counts(s_cpu, scale, thr)
        t_host = time.perf_counter() - t0
        per_layer_s = t_host * h * n / rows_cpu
        cpu = {"value": round(per_layer_s * 1e3, 1), "unit": "ms per layer", "cores": cpu_threads(), "kind": "port",
               "sample": f"{rows_cpu} query rows of 1 head (scores from the GPU GEMM) through the numpy oracle's "
                         f"sort/cumsum count: {t_host:.3f} s, scaled x{h * n // rows_cpu} to {per_layer_s:.1f} s"}

    line = {
        "metric": "exact per-head attention sparsity of one layer (offline profile producer), ms, 1 GPU",
        "value": round(t_call, 3),
        "unit": "ms per layer (all query rows, threshold 0.95)",
        "n_gpus": 1, "steps": 1, "warmup": 1, "ms_per_step": round(t_call, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded Gaussian mixture with per-frame drift, drawn on device)",
        "config": {"workload": f"{cfg.name}: exact sparsity profile of one layer, H={h} Sq=Sk={n} d={d}",
                   "heads": h, "tokens": n, "threshold": thr, "chunk_rows": chunk},
        "gemm_ms": round(t_gemm, 3), "count_kernel_ms": round(t_count, 3),
        "count_kernel_gbps": round(count_gbps, 1), "count_kernel_frac_hbm": round(count_gbps / HBM_PEAK_GBPS, 4),
        "reference_formulation_ms": round(t_ref, 3), "speedup_vs_reference_formulation": round(t_ref / t_call, 2),
        "counts_agree_with_reference_formulation": round(agree, 5),
        "avg_sparsity": round(avg, 6),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline_dit(model, lat, txt, rho, top_p, dmin, dmax, nheads, t_step_ms, dev):
    """One block of the same DiT on the host in float32, its self-attention through the numpy oracle on
    ``nheads`` heads (scaled to all heads); the block time is scaled by the number of blocks."""
    import copy

    import numpy as np
    import torch

    from oracle import torch_ref as T
    from svoo_amd import dit

    cfg = model.config
    heads, d = cfg.num_attention_heads, cfg.attention_head_dim
    with torch.no_grad():
        x = model.patch_embedding(lat).flatten(2).transpose(1, 2).float().cpu()
        wdt = model.time_embedder[0].weight.dtype
        temb = model.time_embedder(dit.timestep_embedding(torch.tensor([700.0], device=dev), cfg.freq_dim).to(wdt))
        tproj = model.time_proj(temb).unflatten(1, (6, -1)).float().cpu()
        ctx = model.text_embedder(txt).float().cpu()
        f, hh, ww = lat.shape[2], lat.shape[3] // 2, lat.shape[4] // 2
        rot = tuple(t.cpu() for t in dit.rope_tables(cfg, f, hh, ww, "cpu"))
    block = copy.deepcopy(model.blocks[0]).float().cpu()
    ratios = [float(r) for r in rho[0, 0]]
    if dmin is not None:
        ratios = [min(max(r, dmin), dmax) for r in ratios]
    timing = {}

    class OracleProc:
        def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, rotary_emb=None,
                     timestep=None):
            q = attn.norm_q(attn.to_q(hidden_states)).unflatten(2, (attn.heads, -1))
            k = attn.norm_k(attn.to_k(hidden_states)).unflatten(2, (attn.heads, -1))
            v = attn.to_v(hidden_states).unflatten(2, (attn.heads, -1))
            q, k = dit.apply_rope(q, *rotary_emb), dit.apply_rope(k, *rotary_emb)
            sel = list(range(nheads))
            qt, kt, vt = (t.transpose(1, 2)[:, sel].contiguous() for t in (q, k, v))
            n = qt.shape[2]
            r = np.random.default_rng(0)
            qi = torch.from_numpy(r.integers(0, n, (nheads, 256)))
            ki = torch.from_numpy(r.integers(0, n, (nheads, 1024)))
            qc0 = torch.gather(qt[0], 1, qi[..., None].expand(-1, -1, d))
            kc0 = torch.gather(kt[0], 1, ki[..., None].expand(-1, -1, d))
            t0 = time.perf_counter()
            o = T.svoo_attention_call(qt, kt, vt, 256, 1024, 2, top_p, ratios[:nheads], qc0, kc0)
            timing["attn"] = time.perf_counter() - t0
            out = torch.zeros(1, n, heads * d)
            out[..., : nheads * d] = o.reshape(1, n, nheads * d)
            return attn.to_out[0](out)

    block.attn1.set_processor(OracleProc())
    t0 = time.perf_counter()
    with torch.no_grad():
        block(x, ctx, tproj, rot, timestep=None)
    t_block = time.perf_counter() - t0
    t_rest = t_block - timing["attn"]
    t_block_scaled = t_rest + timing["attn"] * heads / nheads
    step_s = t_block_scaled * cfg.num_layers
    log(f"CPU: block {t_block:.1f}s (SVOO attention {timing['attn']:.1f}s for {nheads} head(s)) -> "
        f"{step_s:.0f}s per step")
    return {
        "value": round(step_s * 1e3, 1),
        "unit": "ms per denoising step",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"block 0 on the host in float32 (torch for projections, norms, cross-attention and FFN; the torch "
                  f"restatement of the reference's SVOO self-attention on {nheads} of {heads} heads): {t_block:.1f} s, attention "
                  f"scaled x{heads / nheads:g}, block scaled x{cfg.num_layers} = {step_s:.0f} s per step = "
                  f"{step_s * 1e3 / t_step_ms:.0f}x the GPU step",
        "step_s_scaled": round(step_s, 1),
    }


CPU_BUDGET_S = 30.0  # the CPU sample repeats (up to 3 runs, median) while its total stays in this budget


def cpu_baseline(cfg, q, k, v, q_init, k_init, top_p, ratios, nheads, t_call_ms, hunyuan=False, ear=False):
    """The reference's call on the host on a fixed subset of ``nheads`` heads of the same inputs (heads spread
    evenly: 0 and H/2 for two), timed up to 3 times within CPU_BUDGET_S (median); latency scaled linearly to all
    heads.  SAP (Wan and HunyuanVideo): the float32 torch restatement of the reference's operations
    (``oracle/torch_ref.py``, torch's multi-threaded CPU kernels); EAR: the numpy oracle."""
    import numpy as np
    import torch

    from oracle import svoo_oracle as O
    from oracle import torch_ref as T

    h, n, d = cfg.heads, cfg.tokens, cfg.head_dim
    nheads = max(1, min(nheads, h))
    sel = sorted({(i * h) // nheads for i in range(nheads)})
    nheads = len(sel)
    f = lambda t: t[:, sel].float().cpu().contiguous()  # noqa: E731
    qt, kt, vt = f(q), f(k), f(v)
    qit = q_init.view(h, -1, d)[sel].float().cpu().contiguous()
    kit = k_init.view(h, -1, d)[sel].float().cpu().contiguous()
    qn, kn, vn, qi, ki = (x.numpy() for x in (qt, kt, vt, qit, kit))
    rs = [ratios[i] for i in sel]
    what = "the numpy oracle" if ear else "the float32 torch restatement of the reference's operations"

    def one_run():
        t0 = time.perf_counter()
        with torch.no_grad():
            if hunyuan:
                T.hunyuan_attention_call(qt, kt, vt, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters,
                                         top_p, rs, cfg.text_tokens, cfg.text_tokens, qit, kit)
            elif ear:
                O.ear_attention_call(qn, kn, vn, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters, top_p,
                                     rs, 1.0, init_q_centroids=qi, init_k_centroids=ki, attn_dtype=np.float32)
            else:
                T.svoo_attention_call(qt, kt, vt, cfg.num_q_centroids, cfg.num_k_centroids, cfg.kmeans_iters, top_p,
                                      rs, qit, kit)
        return time.perf_counter() - t0

    runs = [one_run()]
    while len(runs) < 3 and sum(runs) + runs[0] <= CPU_BUDGET_S:
        runs.append(one_run())
    t = float(np.median(runs))
    per_head = t / nheads
    call_s = per_head * h
    log(f"CPU ({what}): {[round(x, 2) for x in runs]} s for heads {sel} -> {call_s:.1f}s per {h}-head call")
    return {
        "value": round(4.0 * nheads * float(n) ** 2 * d / t / 1e12, 5),
        "unit": "TFLOP/s (dense-equivalent)",
        "cores": torch.get_num_threads() if not ear else cpu_threads(),
        "kind": "port",
        "sample": f"heads {sel} of {h} of the same inputs, full call (k-means {cfg.kmeans_iters} warm-started "
                  f"iterations, {'EAR scoring and selection' if ear else 'mask'}, permutes, fp32 "
                  f"{'compensated ' if ear else ''}block-sparse attention) in {what}: median of "
                  f"{len(runs)} run(s) {t:.2f} s; scaled x{h / nheads:g} to {call_s:.1f} s per call = "
                  f"{call_s * 1e3 / t_call_ms:.0f}x the GPU latency",
        "call_s_scaled": round(call_s, 3),
        "runs_s": [round(x, 3) for x in runs],
    }


if __name__ == "__main__":
    main()
