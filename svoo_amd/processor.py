"""SVOO attention processors (the drop-in boundary) on the MI355X hot path.

``WanAttn_SAPAttn_Processor`` keeps the diffusers attention-processor protocol and the class-level
configuration of ``svoo/models/wan/attention.py:546-1216``:

* ``__call__(attn, hidden_states, encoder_hidden_states=None, attention_mask=None, rotary_emb=None,
  timestep=None)`` projects Q/K/V, applies the q/k norms and RoPE, and routes self-attention with a
  timestep to :meth:`attention_core_logic`;
* ``attention_core_logic(query, key, value, timestep)`` takes ``[1, H, S, D]`` bf16 tensors and
  returns ``[1, S, H*D]``: dense SDPA on the configured full-precision layers/timesteps, otherwise
  co-clustering (or the reuse cache), per-head profile ratios, block mask, permutes, variable-block
  sparse attention and the inverse permutation.

``WanAttn_EARAttn_Processor`` swaps the top-p mask for EAR routing (an area budget filled by estimated
pruning error) and the attention for its centroid-compensated form
(``svoo/models/wan/attention.py:1047-1071, 1180-1196, 1219-1222``).

``Hunyuan_SAPAttn_Processor`` adds the text-dense post-processing of
``svoo/models/hunyuan10/attention.py:977-1110`` on the same kernels.
"""

from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn.functional as F

from .co_clustering import (block_mask_lengths, co_cluster_tokens_full, dynamic_block_sparse_fwd,
                            dynamic_block_sparse_fwd_fused)
from .ear import dynamic_block_sparse_prune_fwd, ear_map_and_value_centroids
from .sparsity.exact import (compute_exact_attention_sparsity, format_sparsity_log, has_completed_sparsity_entry,
                             record_sparsity_entry)
from .permute import apply_inverse_permutation, apply_inverse_permutation_bshd, permute_pair_by_indices
from . import _lib


def _env_on(name: str) -> bool:
    """Truthiness of a diagnostic switch as the reference reads ``SVG_REUSE_DEBUG``: anything but unset, ``0``,
    empty, ``false`` or ``False``."""
    return os.getenv(name, "0") not in ("0", "", "false", "False")


def save_qk(query, key, timestep, layer_idx) -> Optional[str]:
    """Activation capture of the self-attention inputs (``svoo/models/wan/attention.py:217-240``).

    With ``SAVE_QK=1``, a ``timestep`` (the scheduler's value, ``timestep[0]`` of a tensor) at or above
    ``SAVE_QK_START_STEP`` (default 0) and ``SAVE_QK_DIR`` set, writes ``{dir}/step{timestep}/layer{layer_idx}.pt``
    holding ``{"q", "k"}`` (host copies of the ``[B, H, S, D]`` tensors after norm and RoPE), ``"timestep"`` and
    ``"layer_idx"``.  Returns the file written, or None.
    """
    if os.getenv("SAVE_QK", "0") != "1" or timestep is None:
        return None
    if isinstance(timestep, torch.Tensor):
        step = timestep[0].item() if timestep.dim() > 0 else timestep.item()
    else:
        step = timestep
    save_dir = os.getenv("SAVE_QK_DIR", "")
    if step < int(os.getenv("SAVE_QK_START_STEP", "0")) or not save_dir:
        return None
    step_dir = os.path.join(save_dir, f"step{step}")
    os.makedirs(step_dir, exist_ok=True)
    path = os.path.join(step_dir, f"layer{layer_idx}.pt")
    torch.save({"q": query.detach().cpu(), "k": key.detach().cpu(), "timestep": step, "layer_idx": layer_idx}, path)
    return path


def _permute_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    b, h, s, d = x.shape
    inp = x.reshape(b * h, s, d).contiguous()
    out = torch.empty_like(inp)
    _lib.call("svoo_permute_rows", inp.data_ptr(), idx.data_ptr(), out.data_ptr(), b * h, s, s, d * inp.element_size(),
              _lib.stream_of(inp.device))
    return out.reshape(b, h, s, d)


def _apply_rotary_emb(hidden_states: torch.Tensor, freqs_cos: torch.Tensor, freqs_sin: torch.Tensor) -> torch.Tensor:
    # Interleaved-pair RoPE of the Wan processor (svoo/models/wan/attention.py:179-190).
    x1, x2 = hidden_states.unflatten(-1, (-1, 2)).unbind(-1)
    cos = freqs_cos[..., 0::2]
    sin = freqs_sin[..., 1::2]
    out = torch.empty_like(hidden_states)
    out[..., 0::2] = x1 * cos - x2 * sin
    out[..., 1::2] = x1 * sin + x2 * cos
    return out.type_as(hidden_states)


class WanAttn_SAPAttn_Processor:
    """Semantic-aware-permutation sparse attention for Wan DiT self-attention (SVOO)."""

    # Sequence geometry (set by replace_wan_attention).
    context_length = 0
    num_frame = 0
    frame_size = 0
    # Dense gates.
    first_layers_fp = 0
    first_times_fp = 0
    # Clustering and mask.
    num_layers = 0
    num_q_centroids = 0
    num_k_centroids = 0
    top_p_kmeans = 0
    min_kc_ratio = 0
    max_kc_ratio = 0
    kmeans_iter_init = 0
    kmeans_iter_step = 0
    zero_step_kmeans_init = False
    centroids_init = False
    # Start each re-clustering from the previous centroids instead of random tokens.  The reference
    # SVOO path always draws random tokens (svoo/models/wan/attention.py:641-649); off by default.
    kmeans_warm_start = False
    kmeans_generator: Optional[torch.Generator] = None
    # Optional fixed initial token indices ``(q_idx [BH, Qc], k_idx [BH, Kc])`` for the random-init
    # clusterings (reproducible runs; the reference draws them with torch.randint).
    kmeans_init_idx = None
    # Reuse cache.
    start_reuse_step = None
    reuse_interval = 1
    # Per-head profile ratios.
    use_dynamic_min_kc_ratio = False
    sparsity_lookup = None
    dynamic_min_kc_ratio_min = None
    dynamic_min_kc_ratio_max = None
    # Variants: EAR routing is built (WanAttn_EARAttn_Processor); the global-constraint and
    # routing-transformer clusterings are not.
    use_svoo = True
    use_ear = False
    ear_gamma = 1.0
    # Run the SAP attention on token-order Q/K/V through the sorted indices (one kernel instead of
    # permute + attention + inverse permutation; the same bits, and no permuted copies of Q/K/V/O).
    # At the Wan-14B 720p shape the gathered rows cost the attention 0.25 ms and save the 1.1 ms of
    # permute passes; False runs the separate passes, as the reference does.
    fuse_permutes = True
    use_global_constraints = False
    use_routing_transformer_strategy = False
    enable_mem_save = bool(int(os.environ.get("SVOO_ENABLE_MEM_SAVE", "1")))
    # Offline profiling: exact per-head sparsity of self-attention, appended to a raw log
    # (svoo/models/wan/attention.py:395-489); merged into the profile CSV by sparsity.merge.
    measure_attention_sparsity = False
    sparsity_output_file = None
    sparsity_batch_size = 0
    sparsity_query_samples = 0
    sparsity_threshold = 0.95
    sparsity_start_step = 1

    # Inference-step tracking shared by all instances (svoo/models/wan/attention.py:84-86).
    _current_internal_timestep = None
    _inference_step_counter = 0
    _seen_timesteps = set()

    def __init__(self, layer_idx: int):
        self.layer_idx = layer_idx
        self.q_centroids = None
        self.k_centroids = None
        self._cached_clustering_results = None
        self.current_inference_step = None
        self._last_call = None
        # When set to a list, the sparse path appends (stage name, recorded torch.cuda.Event) at each
        # stage boundary on the current stream: start, cluster, permute, mask, attention, unpermute.
        self.stage_events = None
        self._last_logged_step = None

    def _mark(self, name: str) -> None:
        if self.stage_events is not None:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self.stage_events.append((name, ev))

    # ---------------------------------------------------------------- diffusers glue
    def get_qkv(self, attn, hidden_states, encoder_hidden_states):
        if encoder_hidden_states is None:
            encoder_hidden_states = hidden_states
        if getattr(attn, "fused_projections", False):
            if getattr(attn, "cross_attention_dim_head", None) is None:
                return attn.to_qkv(hidden_states).chunk(3, dim=-1)
            query = attn.to_q(hidden_states)
            key, value = attn.to_kv(encoder_hidden_states).chunk(2, dim=-1)
            return query, key, value
        return attn.to_q(hidden_states), attn.to_k(encoder_hidden_states), attn.to_v(encoder_hidden_states)

    def get_qk_norm(self, attn, query, key):
        if getattr(attn, "norm_q", None) is not None:
            query = attn.norm_q(query)
        if getattr(attn, "norm_k", None) is not None:
            key = attn.norm_k(key)
        return query, key

    def get_transpose_qkv(self, attn, query, key, value):
        return (query.transpose(1, 2).contiguous(), key.transpose(1, 2).contiguous(),
                value.transpose(1, 2).contiguous())

    def get_o(self, attn, query, hidden_states, hidden_states_img):
        if hidden_states.dim() == 4:
            hidden_states = hidden_states.transpose(1, 2).flatten(2, 3)
        hidden_states = hidden_states.type_as(query)
        if hidden_states_img is not None:
            if hidden_states_img.dim() == 4:
                hidden_states_img = hidden_states_img.transpose(1, 2).flatten(2, 3)
            hidden_states = hidden_states + hidden_states_img
        hidden_states = attn.to_out[0](hidden_states)
        hidden_states = attn.to_out[1](hidden_states)
        return hidden_states

    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, rotary_emb=None,
                 timestep=None):
        """Diffusers processor entry (``svoo/models/wan/attention.py:153-260``)."""
        encoder_hidden_states_img = None
        if getattr(attn, "add_k_proj", None) is not None:
            image_context_length = encoder_hidden_states.shape[1] - 512
            encoder_hidden_states_img = encoder_hidden_states[:, :image_context_length]
            encoder_hidden_states = encoder_hidden_states[:, image_context_length:]
        query, key, value = self.get_qkv(attn, hidden_states, encoder_hidden_states)
        query, key = self.get_qk_norm(attn, query, key)
        query = query.unflatten(2, (attn.heads, -1))
        key = key.unflatten(2, (attn.heads, -1))
        value = value.unflatten(2, (attn.heads, -1))
        if rotary_emb is not None:
            query = _apply_rotary_emb(query, *rotary_emb)
            key = _apply_rotary_emb(key, *rotary_emb)
        query, key, value = self.get_transpose_qkv(attn, query, key, value)

        hidden_states_img = None
        if encoder_hidden_states_img is not None:
            key_img = attn.add_k_proj(encoder_hidden_states_img)
            value_img = attn.add_v_proj(encoder_hidden_states_img)
            key_img = attn.norm_added_k(key_img)
            key_img = key_img.unflatten(2, (attn.heads, -1)).transpose(1, 2)
            value_img = value_img.unflatten(2, (attn.heads, -1)).transpose(1, 2)
            hidden_states_img = F.scaled_dot_product_attention(query, key_img, value_img, dropout_p=0.0,
                                                               is_causal=False)
            hidden_states_img = hidden_states_img.transpose(1, 2).flatten(2, 3).type_as(query)

        save_qk(query, key, timestep, self.layer_idx)
        if timestep is None:
            hidden_states = F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask,
                                                           dropout_p=0.0, is_causal=False)
        else:
            if self.measure_attention_sparsity:
                self.log_attention_sparsity(query, key, value, timestep, "self")
            hidden_states = self.attention_core_logic(query, key, value, timestep)
        return self.get_o(attn, query, hidden_states, hidden_states_img)

    # ---------------------------------------------------------------- step bookkeeping
    def _get_inference_step(self, timestep):
        """1-based denoising step from scheduler timesteps (``svoo/models/wan/attention.py:423-444``)."""
        cls = self.__class__
        internal_t = timestep[0].item() if isinstance(timestep, torch.Tensor) else timestep
        if cls._current_internal_timestep is not None and internal_t > cls._current_internal_timestep:
            cls._inference_step_counter = 0
            cls._seen_timesteps = set()
        if internal_t not in cls._seen_timesteps:
            cls._seen_timesteps.add(internal_t)
            cls._inference_step_counter += 1
            cls._current_internal_timestep = internal_t
        return cls._inference_step_counter

    @torch.no_grad()
    def compute_attention_sparsity(self, query, key, value, attn_type="self", batch_size=0, threshold=0.95,
                                   query_sample_size=0):
        """Exact per-head sparsity of this call's attention (``svoo/models/wan/attention.py:395-417``)."""
        return compute_exact_attention_sparsity(query, key, batch_size=batch_size, threshold=threshold,
                                                query_sample_size=query_sample_size)

    def log_attention_sparsity(self, query, key, value, timestep, attn_type="self"):
        """Measure once per (layer, step) from ``sparsity_start_step`` on and append the raw log lines
        (``svoo/models/wan/attention.py:446-489``); completed entries are skipped on resume."""
        if not self.measure_attention_sparsity:
            return
        step = self._get_inference_step(timestep)
        if step is None or step < self.sparsity_start_step or self._last_logged_step == step:
            return
        self._last_logged_step = step
        out = self.sparsity_output_file
        if has_completed_sparsity_entry(out, self.layer_idx, step, query.size(1)):
            return
        avg, per_head, stats = self.compute_attention_sparsity(
            query, key, value, attn_type, batch_size=self.sparsity_batch_size, threshold=self.sparsity_threshold,
            query_sample_size=self.sparsity_query_samples)
        lines = format_sparsity_log(self.layer_idx, attn_type, step, self.sparsity_threshold, avg, per_head,
                                    stats["seq_len"], stats["sampled_seq_len"])
        for line in lines:
            print(line)
        if out:
            d = os.path.dirname(out)
            if d:
                os.makedirs(d, exist_ok=True)
            with open(out, "a") as f:
                f.write("\n".join(lines) + "\n")
            record_sparsity_entry(out, self.layer_idx, step, range(len(per_head)))

    def flash_attention(self, query, key, value):
        """Dense attention of the full-precision gate (``svoo/models/wan/attention.py:329-331``)."""
        return F.scaled_dot_product_attention(query, key, value, dropout_p=0.0, is_causal=False)

    # ---------------------------------------------------------------- clustering
    def _check_variant(self):
        if not self.use_svoo:
            raise ValueError("Only the SVOO co-clustering path is supported (use_svoo=True).")
        if self.use_global_constraints or self.use_routing_transformer_strategy:
            raise NotImplementedError("global-constraint and routing-transformer variants are not built here.")

    def _co_cluster(self, query, key, iters, warm):
        cfg, num_heads, seq_len, dim = query.size()
        q_flat = query.reshape(cfg * num_heads, seq_len, dim)
        k_flat = key.reshape(cfg * num_heads, seq_len, dim)
        kw = {}
        if warm and self.q_centroids is not None and self.k_centroids is not None:
            kw = dict(init_q_centroids=self.q_centroids, init_k_centroids=self.k_centroids)
        elif self.kmeans_init_idx is not None:
            kw = dict(init_q_idx=self.kmeans_init_idx[0], init_k_idx=self.kmeans_init_idx[1])
        r = co_cluster_tokens_full(q_flat, k_flat, self.num_q_centroids, self.num_k_centroids, iters,
                                   generator=self.kmeans_generator, **kw)
        self.q_centroids = r["qcentroids"]
        self.k_centroids = r["kcentroids"]
        return r

    def kmeans_init(self, query, key, layer_idx):
        self._check_variant()
        return self._co_cluster(query, key, self.kmeans_iter_init, warm=False)

    def kmeans_step(self, query, key, layer_idx):
        self._check_variant()
        return self._co_cluster(query, key, self.kmeans_iter_step, warm=self.kmeans_warm_start)

    def should_recluster(self, trace: bool = False) -> bool:
        """Reuse schedule of ``svoo/models/wan/attention.py:682-711``.  With ``trace`` and ``SVG_REUSE_DEBUG`` set,
        prints the reference's ``[reuse]`` lines (the offset is None before ``start_reuse_step``, and an interval
        below 1 counts as 1, as in ``svoo/models/hunyuan10/attention.py:851-884``)."""
        debug = trace and _env_on("SVG_REUSE_DEBUG")
        step = self.current_inference_step
        recluster = True
        if debug:
            print(f"[reuse] current_step={step}, start_reuse_step={self.start_reuse_step}, "
                  f"reuse_interval={self.reuse_interval}")
        if step is not None and self.start_reuse_step is not None and self.start_reuse_step > 0:
            offset = None
            if step >= self.start_reuse_step:
                offset = step - self.start_reuse_step
                recluster = offset % max(1, int(self.reuse_interval)) == 0
            if debug:
                print(f"[reuse] offset={offset}, should_recluster={recluster}")
        if not recluster:
            if self._cached_clustering_results is None:
                if debug:
                    print("[reuse] No cached clustering results, forcing recluster")
                recluster = True
            elif debug:
                print("[reuse] Reusing cached clustering results")
        return recluster

    def kmeans_clustering(self, query, key, layer_idx):
        """Co-cluster (or return the cached clustering) and refresh the reuse cache (``:669-863``)."""
        if not self.should_recluster(trace=True):
            return self._cached_clustering_results
        if not self.centroids_init:
            r = self.kmeans_init(query, key, layer_idx)
            self.centroids_init = True
        else:
            r = self.kmeans_step(query, key, layer_idx)
        self._cached_clustering_results = r
        if os.getenv("COMPUTE_REUSE_SIMILARITY", "0") == "1":
            self.report_reuse_similarity(r, layer_idx, query.size(1))
        return r

    def report_reuse_similarity(self, r, layer_idx, num_heads):
        """Label agreement between this clustering and the previous one of the same (layer, head)
        (``svoo/models/wan/attention.py:821-861``): the normalised mutual information (arithmetic mean) of the
        query labels and of the key labels of the first batch element, printed as ``[Reuse Similarity]`` lines
        and returned as ``{head: (prev_step, q_nmi, k_nmi)}``.  Needs scikit-learn (skipped without it, as in the
        reference)."""
        step = self.current_inference_step
        out = {}
        if step is None:
            return out
        hist = self.__dict__.setdefault("_clustering_history", {})
        ql, kl = r["qlabels"], r["klabels"]
        if ql.dim() != 2 or kl.dim() != 2 or ql.size(0) // num_heads < 1:
            return out
        try:
            from sklearn.metrics import normalized_mutual_info_score
        except ImportError:
            normalized_mutual_info_score = None
        for h in range(num_heads):
            q_now, k_now = ql[h].cpu().clone(), kl[h].cpu().clone()
            key_ = (layer_idx, h)
            prev = [st for st in hist.get(key_, {}) if st < step]
            if step > 0 and prev and normalized_mutual_info_score is not None:
                ps = max(prev)
                pq, pk = hist[key_][ps]
                q_nmi = normalized_mutual_info_score(pq.numpy(), q_now.numpy(), average_method="arithmetic")
                k_nmi = normalized_mutual_info_score(pk.numpy(), k_now.numpy(), average_method="arithmetic")
                print(f"[Reuse Similarity] Step {ps}->{step}, Layer {layer_idx}, Head {h}: "
                      f"Q={q_nmi:.4f}, K={k_nmi:.4f}, Avg={(q_nmi + k_nmi) / 2.0:.4f}")
                out[h] = (ps, float(q_nmi), float(k_nmi))
            hist.setdefault(key_, {})[step] = (q_now, k_now)
        return out

    def _get_min_kc_ratio_for_heads_from_step(self, inference_step, num_heads):
        """Per-head ratios from the profile, clipped, or the scalar ratio (``:931-956``)."""
        if self.use_dynamic_min_kc_ratio and self.sparsity_lookup is not None and inference_step is not None:
            if not self.sparsity_lookup.has_data_for_step_layer(inference_step, self.layer_idx, num_heads):
                return self.min_kc_ratio
            values = []
            for value in self.sparsity_lookup.get_sparsity_batch(inference_step, self.layer_idx, num_heads):
                if self.dynamic_min_kc_ratio_min is not None:
                    value = max(value, self.dynamic_min_kc_ratio_min)
                if self.dynamic_min_kc_ratio_max is not None:
                    value = min(value, self.dynamic_min_kc_ratio_max)
                values.append(value)
            return values
        return self.min_kc_ratio

    def semantic_aware_permutation(self, query, key, value, timestep=None):
        """Cluster, build the block map and permute Q/K/V (``svoo/models/wan/attention.py:958-1088``).

        Returns ``(q_perm, k_perm, v_perm, dynamic_map, q_cluster_sizes, k_cluster_sizes, q_sorted_indices)``,
        with EAR also ``(k_centroids, v_centroids)``.
        """
        cfg, num_heads, seq_len, dim = query.size()
        r = self.kmeans_clustering(query, key, self.layer_idx)
        self._mark("cluster")
        min_kc_ratio = self._get_min_kc_ratio_for_heads_from_step(self.current_inference_step, num_heads)
        q_sizes = r["qsizes"].view(cfg, num_heads, self.num_q_centroids)
        k_sizes = r["ksizes"].view(cfg, num_heads, self.num_k_centroids)
        q_perm = _permute_rows(query, r["q_sorted_idx"])
        k_perm, v_perm = permute_pair_by_indices(key, value, r["k_sorted_idx"])
        self._mark("permute")
        if self.use_ear:
            qcv = r["qcentroids"].view(cfg, num_heads, self.num_q_centroids, dim)
            kcv = r["kcentroids"].view(cfg, num_heads, self.num_k_centroids, dim)
            v_cent, dynamic_map, parts = ear_map_and_value_centroids(
                q_perm, k_perm, v_perm, q_sizes, k_sizes, qcv, kcv, self.top_p_kmeans, gamma=self.ear_gamma,
                min_kc_ratio=min_kc_ratio, return_parts=True)
            self._last_call = dict(clustering=r, map=dynamic_map, lengths=dynamic_map.sum(-1, dtype=torch.int32),
                                   min_kc_ratio=min_kc_ratio, q_sizes=q_sizes, k_sizes=k_sizes, v_centroids=v_cent,
                                   **parts)
            return q_perm, k_perm, v_perm, dynamic_map, q_sizes, k_sizes, r["q_sorted_idx"], kcv, v_cent
        dynamic_map = self._block_mask(r, cfg, num_heads, dim, q_sizes, k_sizes, min_kc_ratio)
        return q_perm, k_perm, v_perm, dynamic_map, q_sizes, k_sizes, r["q_sorted_idx"]

    def _block_mask(self, r, cfg, num_heads, dim, q_sizes, k_sizes, min_kc_ratio):
        dynamic_map, lengths = block_mask_lengths(
            r["qcentroids"].view(cfg, num_heads, self.num_q_centroids, dim),
            r["kcentroids"].view(cfg, num_heads, self.num_k_centroids, dim),
            q_sizes, k_sizes, self.top_p_kmeans, min_kc_ratio, self.max_kc_ratio,
        )
        self._last_call = dict(clustering=r, map=dynamic_map, lengths=lengths, min_kc_ratio=min_kc_ratio,
                               q_sizes=q_sizes, k_sizes=k_sizes)
        return dynamic_map

    def fused_sparse_attention(self, query, key, value):
        """The SAP path of :meth:`attention_core_logic` without separate permute passes: cluster, block mask,
        then one kernel that reads Q/K/V through the sorted indices and writes ``[1, S, H*D]`` in token order
        (the same values as permute + ``dynamic_block_sparse_fwd`` + inverse permutation)."""
        cfg, num_heads, seq_len, dim = query.size()
        r = self.kmeans_clustering(query, key, self.layer_idx)
        self._mark("cluster")
        min_kc_ratio = self._get_min_kc_ratio_for_heads_from_step(self.current_inference_step, num_heads)
        q_sizes = r["qsizes"].view(cfg, num_heads, self.num_q_centroids)
        k_sizes = r["ksizes"].view(cfg, num_heads, self.num_k_centroids)
        dynamic_map = self._block_mask(r, cfg, num_heads, dim, q_sizes, k_sizes, min_kc_ratio)
        self._mark("mask")
        out = dynamic_block_sparse_fwd_fused(query, key, value, dynamic_map, q_sizes, k_sizes, r["q_sorted_idx"],
                                             r["k_sorted_idx"], validate=False)
        self._mark("attention")
        return out

    def attention_core_logic(self, query, key, value, timestep):
        """SVOO attention for ``[1, H, S, D]`` Q/K/V; returns ``[1, S, H*D]`` (``:1110-1216``)."""
        cfg, num_heads, seq_len, dim = query.size()
        assert cfg == 1, "Batch size must be 1 for kmeans block sparse attention"
        cb_step = getattr(self, "_step_from_callback", None)
        if cb_step is not None:
            self.current_inference_step = cb_step
        elif timestep is not None:
            self.current_inference_step = self._get_inference_step(timestep)
        else:
            self.current_inference_step = None
        assert seq_len == self.context_length + self.num_frame * self.frame_size, (
            f"Query Shape: {seq_len} is not equivalent to {self.context_length} + {self.num_frame} * {self.frame_size}"
        )
        full = self.layer_idx < self.first_layers_fp
        if timestep is not None:
            if isinstance(timestep, torch.Tensor):
                tval = timestep[0].item() if timestep.numel() > 0 else None
            else:
                tval = timestep
            if tval is not None and tval > self.first_times_fp:
                full = True
        if full:
            if self.zero_step_kmeans_init:
                video_length = self.num_frame * self.frame_size
                self.kmeans_clustering(query[:, :, :video_length].contiguous(), key[:, :, :video_length].contiguous(),
                                       self.layer_idx)
            out = self.flash_attention(query, key, value)
            return out.transpose(1, 2).flatten(2, 3)

        self._mark("start")
        if not self.use_ear and self.fuse_permutes:
            return self.fused_sparse_attention(query, key, value)
        perm = self.semantic_aware_permutation(query, key, value, timestep)
        q_perm, k_perm, v_perm, dyn_map, qc_sz, kc_sz, q_sorted_indices = perm[:7]
        self._mark("mask")
        if len(perm) == 9:  # EAR: centroid-compensated attention
            out_perm = dynamic_block_sparse_prune_fwd(q_perm, k_perm, v_perm, perm[7], perm[8], dyn_map, qc_sz, kc_sz,
                                                      validate=False)
        else:
            out_perm = dynamic_block_sparse_fwd(q_perm, k_perm, v_perm, dyn_map, qc_sz, kc_sz, validate=False)
        self._mark("attention")
        if self.enable_mem_save:
            del q_perm, k_perm, v_perm
        out = apply_inverse_permutation_bshd(out_perm, q_sorted_indices)
        self._mark("unpermute")
        return out


class WanAttn_EARAttn_Processor(WanAttn_SAPAttn_Processor):
    """Wan SAP processor with EAR (error-aware routing, centroid compensation) enabled
    (``svoo/models/wan/attention.py:1219-1222``)."""

    use_ear = True


class WanAttn_DenseAttn_Processor(WanAttn_SAPAttn_Processor):
    """Dense self-attention on every layer and step, with the optional sparsity logging: the
    ``pattern="dense"`` diagnostic that produces the per-head profiles (``svoo/models/wan/inference.py:398-440``
    with ``WanAttn_SVGAttn_Processor2_0.attention_core_logic`` and ``attention_masks = None``,
    ``svoo/models/wan/attention.py:337-355``)."""

    def attention_core_logic(self, query, key, value, timestep):
        cfg, num_heads, seq_len, dim = query.size()
        assert seq_len == self.context_length + self.num_frame * self.frame_size, (
            f"Query Shape: {seq_len} is not equivalent to {self.context_length} + {self.num_frame} * {self.frame_size}"
        )
        return self.flash_attention(query, key, value).transpose(1, 2).flatten(2, 3)


def _apply_rotary_emb_real(x: torch.Tensor, freqs_cis) -> torch.Tensor:
    """RoPE with real ``(cos, sin)`` tables of shape ``[S, D]`` on interleaved pairs, ``[B, H, S, D]`` input.

    The rotary form HunyuanVideo uses through diffusers' ``apply_rotary_emb(use_real=True,
    use_real_unbind_dim=-1)`` (called at ``svoo/models/hunyuan10/attention.py:305-353``).
    """
    cos, sin = freqs_cis
    cos = cos[None, None].to(x.device)
    sin = sin[None, None].to(x.device)
    x_real, x_imag = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    x_rot = torch.stack([-x_imag, x_real], dim=-1).flatten(3)
    return (x.float() * cos + x_rot.float() * sin).to(x.dtype)


def _extend_with_text(sorted_indices: torch.Tensor, video_length: int, context_length: int) -> torch.Tensor:
    """``[BH, V]`` video sort order -> ``[BH, V + C]`` with the text tokens ``V .. V+C-1`` in place
    (``svoo/models/hunyuan10/attention.py:1013-1017``)."""
    text = torch.arange(video_length, video_length + context_length, dtype=sorted_indices.dtype,
                        device=sorted_indices.device)
    return torch.cat([sorted_indices, text.expand(sorted_indices.shape[0], context_length)], dim=1).contiguous()


class Hunyuan_SAPAttn_Processor(WanAttn_SAPAttn_Processor):
    """Semantic-aware-permutation attention for HunyuanVideo (``svoo/models/hunyuan10/attention.py:757-1110``).

    The sequence is ``num_frame * frame_size`` video tokens followed by ``context_length`` text
    tokens, of which the first ``prompt_length`` are the valid prompt.  The video part is
    co-clustered, masked and permuted as in Wan; the text stays at the end and becomes two extra
    clusters (``dynamic_map_post_processing``, ``:977-1021``): the prompt attends every video
    cluster and itself, every video cluster attends the prompt, and the unused padding attends only
    itself.  ``attention_core_logic`` returns ``[1, H, S, D]``.
    """

    prompt_length = 0
    context_length = 256
    num_frame = 33
    frame_size = 3600

    # ---------------------------------------------------------------- diffusers glue (hunyuan10/attention.py:459-575)
    def get_qkv(self, attn, hidden_states, encoder_hidden_states=None):
        return attn.to_q(hidden_states), attn.to_k(hidden_states), attn.to_v(hidden_states)

    def get_transpose_qkv(self, attn, query, key, value):
        t = lambda x: x.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()  # noqa: E731
        return t(query), t(key), t(value)

    def get_rotary_emb(self, attn, query, key, image_rotary_emb, encoder_hidden_states):
        if image_rotary_emb is None:
            return query, key
        if getattr(attn, "add_q_proj", None) is None and encoder_hidden_states is not None:
            # Single-stream block: RoPE on the video part, text (last) untouched.
            txt = encoder_hidden_states.shape[1]
            query = torch.cat([_apply_rotary_emb_real(query[:, :, :-txt], image_rotary_emb), query[:, :, -txt:]], dim=2)
            key = torch.cat([_apply_rotary_emb_real(key[:, :, :-txt], image_rotary_emb), key[:, :, -txt:]], dim=2)
            return query, key
        return _apply_rotary_emb_real(query, image_rotary_emb), _apply_rotary_emb_real(key, image_rotary_emb)

    def get_encoder_condition_and_concat(self, attn, query, key, value, encoder_hidden_states):
        if getattr(attn, "add_q_proj", None) is not None and encoder_hidden_states is not None:
            t = lambda x: x.unflatten(2, (attn.heads, -1)).transpose(1, 2)  # noqa: E731
            eq = t(attn.add_q_proj(encoder_hidden_states))
            ek = t(attn.add_k_proj(encoder_hidden_states))
            ev = t(attn.add_v_proj(encoder_hidden_states))
            if getattr(attn, "norm_added_q", None) is not None:
                eq = attn.norm_added_q(eq)
            if getattr(attn, "norm_added_k", None) is not None:
                ek = attn.norm_added_k(ek)
            query = torch.cat([query, eq], dim=2)
            key = torch.cat([key, ek], dim=2)
            value = torch.cat([value, ev], dim=2)
        return query.contiguous(), key.contiguous(), value.contiguous()

    def get_cu_max_seqlen(self, attention_mask, device):
        """``([0, valid, total]`` for q and kv, max lengths); built on the device (no host read-back)."""
        mask = attention_mask.to(device)
        total = mask.numel()
        cu = torch.zeros(3, dtype=torch.int32, device=device)
        cu[1] = mask.sum().to(torch.int32)
        cu[2] = total
        return cu, cu.clone(), total, total

    def get_o(self, attn, hidden_states, encoder_hidden_states):
        if encoder_hidden_states is not None:
            n_txt = encoder_hidden_states.shape[1]
            hidden_states, encoder_hidden_states = hidden_states[:, :-n_txt], hidden_states[:, -n_txt:]
            if getattr(attn, "to_out", None) is not None:
                hidden_states = attn.to_out[0](hidden_states)
                hidden_states = attn.to_out[1](hidden_states)
            if getattr(attn, "to_add_out", None) is not None:
                encoder_hidden_states = attn.to_add_out(encoder_hidden_states)
        return hidden_states, encoder_hidden_states

    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, image_rotary_emb=None,
                 timestep=None):
        """Diffusers processor entry (``svoo/models/hunyuan10/attention.py:536-575``); returns ``(hidden, encoder_hidden)``."""
        if getattr(attn, "add_q_proj", None) is None and encoder_hidden_states is not None:
            hidden_states = torch.cat([hidden_states, encoder_hidden_states], dim=1)
        query, key, value = self.get_qkv(attn, hidden_states)
        query, key, value = self.get_transpose_qkv(attn, query, key, value)
        query, key = self.get_qk_norm(attn, query, key)
        query, key = self.get_rotary_emb(attn, query, key, image_rotary_emb, encoder_hidden_states)
        query, key, value = self.get_encoder_condition_and_concat(attn, query, key, value, encoder_hidden_states)
        if attention_mask is None:
            attention_mask = torch.ones(query.shape[2], dtype=torch.bool, device=query.device)
        cu_max_seqlens = self.get_cu_max_seqlen(attention_mask, query.device)
        out = self.attention_core_logic(query, key, value, timestep, self.layer_idx, cu_max_seqlens)
        out = out.transpose(1, 2).flatten(2, 3).to(query.dtype)
        return self.get_o(attn, out, encoder_hidden_states)

    # ---------------------------------------------------------------- attention
    def flashinfer_attention(self, query, key, value, cu_max_seqlens):
        """Dense attention of the full-precision gate (``:639-645``, ``:1113-1185``): valid tokens attend each
        other, the padding attends itself; a 2x2 block map on the same sparse kernel."""
        cu_q, cu_kv = cu_max_seqlens[0], cu_max_seqlens[1]
        b, h = query.shape[:2]
        dev = query.device
        rs = (cu_q[1:] - cu_q[:-1]).to(device=dev, dtype=torch.int32).repeat(b, h, 1)
        cs = (cu_kv[1:] - cu_kv[:-1]).to(device=dev, dtype=torch.int32).repeat(b, h, 1)
        bmap = torch.eye(2, dtype=torch.bool, device=dev).repeat(b, h, 1, 1)
        return dynamic_block_sparse_fwd(query, key, value, bmap, rs, cs, validate=False)

    flash_attention = flashinfer_attention

    def dynamic_map_post_processing(self, dyn_map, qc_sz, kc_sz, q_sorted_indices, video_length, context_length,
                                    prompt_length, unprompt_length):
        """Append the prompt and padding clusters (``:977-1021``), on the device.

        ``dyn_map [B, H, Qc, Kc] -> [B, H, Qc+2, Kc+2]``: row ``Qc`` (prompt) attends key clusters
        ``0..Kc`` (video and prompt), column ``Kc`` (prompt) is attended by rows ``0..Qc``, row and
        column ``Kc+1`` (padding) only by each other.  Sizes gain ``[prompt_length, unprompt_length]``;
        ``q_sorted_indices [BH, V]`` gains the identity over the text tokens.
        """
        dyn_map = F.pad(dyn_map, (0, 2, 0, 2), value=False)
        dyn_map[:, :, -2, :-1] = True
        dyn_map[:, :, :-1, -2] = True
        dyn_map[:, :, -1, -1] = True
        tail = torch.tensor([prompt_length, unprompt_length], dtype=qc_sz.dtype, device=qc_sz.device)
        qc_sz = torch.cat([qc_sz, tail.expand(*qc_sz.shape[:-1], 2)], dim=-1)
        kc_sz = torch.cat([kc_sz, tail.to(kc_sz.dtype).expand(*kc_sz.shape[:-1], 2)], dim=-1)
        return dyn_map, qc_sz, kc_sz, _extend_with_text(q_sorted_indices, video_length, context_length)

    def attention_core_logic(self, query, key, value, timestep, layer_idx=None, cu_max_seqlens=None):
        """Hunyuan SVOO attention for ``[1, H, S, D]`` Q/K/V (``:1031-1110``); returns ``[1, H, S, D]``.

        Layout: with ``fuse_permutes`` (the default) the result is the ``transpose(1, 2)`` view of a
        contiguous ``[1, S, H, D]`` buffer, so the caller's ``transpose(1, 2).flatten(2, 3)`` is free;
        it is not contiguous, so a caller that needs ``.view`` on it calls ``.contiguous()`` first (the
        reference returns a contiguous ``[1, H, S, D]``).  With ``fuse_permutes = False`` it is
        contiguous.  The values are identical either way.

        ``_last_call`` holds the post-processed ``map``, ``q_sizes`` and ``k_sizes`` (``Qc + 2`` /
        ``Kc + 2`` clusters, text last) and ``video_lengths``, the kept key clusters per row of the
        video-only map before the text clusters are added."""
        cfg, num_heads, seq_len, dim = query.size()
        assert cfg == 1, "Batch size must be 1 for kmeans block sparse attention"
        prompt_length, context_length = int(self.prompt_length), int(self.context_length)
        if not 0 <= prompt_length <= context_length:
            # A prompt longer than the text context would make the padding cluster's size negative and
            # every head's plan invalid.
            raise ValueError(f"prompt_length={prompt_length} must lie in [0, context_length={context_length}]")
        video_length = self.num_frame * self.frame_size
        assert seq_len == context_length + video_length, (
            f"Query Shape: {seq_len} is not equivalent to {context_length} + {self.num_frame} * {self.frame_size}"
        )
        self.current_inference_step = getattr(self, "_step_from_callback", None)
        full = self.layer_idx < self.first_layers_fp
        if timestep is not None:
            tval = timestep[0].item() if isinstance(timestep, torch.Tensor) else timestep
            if tval > self.first_times_fp:
                full = True
        if full:
            if self.zero_step_kmeans_init:
                self.kmeans_clustering(query[:, :, :video_length].contiguous(), key[:, :, :video_length].contiguous(),
                                       self.layer_idx)
            if cu_max_seqlens is None:
                valid = video_length + prompt_length
                cu = torch.tensor([0, valid, seq_len], dtype=torch.int32, device=query.device)
                cu_max_seqlens = (cu, cu, seq_len, seq_len)
            return self.flashinfer_attention(query, key, value, cu_max_seqlens).reshape(cfg, num_heads, seq_len, dim)

        # 1. Video part: cluster (or reuse), per-head ratios, block mask.
        self._mark("start")
        q_video = query[:, :, :video_length].contiguous()
        k_video = key[:, :, :video_length].contiguous()
        r = self.kmeans_clustering(q_video, k_video, self.layer_idx)
        del q_video, k_video
        self._mark("cluster")
        min_kc_ratio = self._get_min_kc_ratio_for_heads_from_step(self.current_inference_step, num_heads)
        q_sizes = r["qsizes"].view(cfg, num_heads, self.num_q_centroids)
        k_sizes = r["ksizes"].view(cfg, num_heads, self.num_k_centroids)
        dyn_map, lengths = block_mask_lengths(
            r["qcentroids"].view(cfg, num_heads, self.num_q_centroids, dim),
            r["kcentroids"].view(cfg, num_heads, self.num_k_centroids, dim),
            q_sizes, k_sizes, self.top_p_kmeans, min_kc_ratio, self.max_kc_ratio,
        )
        self._mark("mask")
        # 2. Text clusters; permutes over the whole sequence with the text rows mapped to themselves.
        unprompt_length = context_length - prompt_length
        dyn_map, qc_sz, kc_sz, q_idx = self.dynamic_map_post_processing(
            dyn_map, q_sizes, k_sizes, r["q_sorted_idx"], video_length, context_length, prompt_length, unprompt_length)
        k_idx = _extend_with_text(r["k_sorted_idx"], video_length, context_length)
        if self.fuse_permutes:
            # One kernel on token-order Q/K/V through q_idx / k_idx (text rows map to themselves); it writes
            # [1, S, H*D] in token order, returned as its [1, H, S, D] transposed view (the same values as the
            # separate passes; the caller's transpose(1, 2).flatten(2, 3) is then a view, not a copy).
            self._last_call = dict(clustering=r, map=dyn_map, video_lengths=lengths, min_kc_ratio=min_kc_ratio,
                                   q_sizes=qc_sz, k_sizes=kc_sz, q_idx=q_idx, k_idx=k_idx)
            out = dynamic_block_sparse_fwd_fused(query.contiguous(), key.contiguous(), value.contiguous(), dyn_map,
                                                 qc_sz, kc_sz, q_idx, k_idx, validate=False)
            self._mark("attention")
            return out.view(cfg, seq_len, num_heads, dim).transpose(1, 2)
        q_perm = _permute_rows(query.contiguous(), q_idx)
        k_perm, v_perm = permute_pair_by_indices(key.contiguous(), value.contiguous(), k_idx)
        self._mark("permute")
        self._last_call = dict(clustering=r, map=dyn_map, video_lengths=lengths, min_kc_ratio=min_kc_ratio,
                               q_sizes=qc_sz, k_sizes=kc_sz, q_idx=q_idx, k_idx=k_idx)
        out_perm = dynamic_block_sparse_fwd(q_perm, k_perm, v_perm, dyn_map, qc_sz, kc_sz, validate=False)
        self._mark("attention")
        if self.enable_mem_save:
            del q_perm, k_perm, v_perm
        out = apply_inverse_permutation(out_perm, q_idx, 2)
        self._mark("unpermute")
        return out
