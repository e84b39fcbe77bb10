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

``Hunyuan_SAPAttn_Processor`` adds the text-dense post-processing of
``svoo/models/hunyuan10/attention.py:977-1110`` on the same kernels.
"""

from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn.functional as F

from .co_clustering import block_mask_lengths, co_cluster_tokens_full, dynamic_block_sparse_fwd
from .permute import apply_inverse_permutation, apply_inverse_permutation_bshd, permute_pair_by_indices
from . import _lib


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
    # Variants of the reference that this build does not carry (see DESIGN.md scope).
    use_svoo = True
    use_ear = False
    use_global_constraints = False
    use_routing_transformer_strategy = False
    enable_mem_save = bool(int(os.environ.get("SVOO_ENABLE_MEM_SAVE", "1")))
    measure_attention_sparsity = False

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

        if timestep is None:
            hidden_states = F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask,
                                                           dropout_p=0.0, is_causal=False)
        else:
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

    def flash_attention(self, query, key, value):
        """Dense attention of the full-precision gate (``svoo/models/wan/attention.py:329-331``)."""
        return F.scaled_dot_product_attention(query, key, value, dropout_p=0.0, is_causal=False)

    # ---------------------------------------------------------------- clustering
    def _check_variant(self):
        if not self.use_svoo:
            raise ValueError("Only the SVOO co-clustering path is supported (use_svoo=True).")
        if self.use_ear or self.use_global_constraints or self.use_routing_transformer_strategy:
            raise NotImplementedError("EAR, global-constraint and routing-transformer variants are not built here.")

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

    def should_recluster(self) -> bool:
        """Reuse schedule of ``svoo/models/wan/attention.py:682-711``."""
        step = self.current_inference_step
        recluster = True
        if step is not None and self.start_reuse_step is not None and self.start_reuse_step > 0:
            if step >= self.start_reuse_step:
                recluster = (step - self.start_reuse_step) % self.reuse_interval == 0
        if not recluster and self._cached_clustering_results is None:
            recluster = True
        return recluster

    def kmeans_clustering(self, query, key, layer_idx):
        """Co-cluster (or return the cached clustering) and refresh the reuse cache (``:669-863``)."""
        if not self.should_recluster():
            return self._cached_clustering_results
        if not self.centroids_init:
            r = self.kmeans_init(query, key, layer_idx)
            self.centroids_init = True
        else:
            r = self.kmeans_step(query, key, layer_idx)
        self._cached_clustering_results = r
        return r

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

        Returns ``(q_perm, k_perm, v_perm, dynamic_map, q_cluster_sizes, k_cluster_sizes, q_sorted_indices)``.
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
        dynamic_map, lengths = block_mask_lengths(
            r["qcentroids"].view(cfg, num_heads, self.num_q_centroids, dim),
            r["kcentroids"].view(cfg, num_heads, self.num_k_centroids, dim),
            q_sizes, k_sizes, self.top_p_kmeans, min_kc_ratio, self.max_kc_ratio,
        )
        self._last_call = dict(clustering=r, map=dynamic_map, lengths=lengths, min_kc_ratio=min_kc_ratio)
        return q_perm, k_perm, v_perm, dynamic_map, q_sizes, k_sizes, r["q_sorted_idx"]

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
        q_perm, k_perm, v_perm, dyn_map, qc_sz, kc_sz, q_sorted_indices = self.semantic_aware_permutation(
            query, key, value, timestep)
        self._mark("mask")
        out_perm = dynamic_block_sparse_fwd(q_perm, k_perm, v_perm, dyn_map, qc_sz, kc_sz, validate=False)
        self._mark("attention")
        if self.enable_mem_save:
            del q_perm, k_perm, v_perm
        out = apply_inverse_permutation_bshd(out_perm, q_sorted_indices)
        self._mark("unpermute")
        return out
