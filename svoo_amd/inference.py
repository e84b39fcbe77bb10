"""Install the SVOO attention processors into a Wan or HunyuanVideo pipeline (the reference's configuration surface).

``replace_wan_attention`` follows ``svoo/models/wan/inference.py:23-440`` (the SAP, EAR and dense
patterns): it derives the token geometry from the pipeline, writes the configuration as class
attributes of the pattern's processor class (shared by every layer, as in the reference) and
registers one processor instance per transformer block (``transformer_2`` too, for Wan2.2).  The pipeline is
duck-typed: ``pipe.transformer.blocks[i].attn1.set_processor``, ``pipe.transformer.config``
(``patch_size``, ``num_attention_heads``, ``attention_head_dim``) and ``pipe.vae_scale_factor_*``.
No kernel warm-up is needed: the HIP kernels are compiled ahead of time.

``replace_hunyuan_attention`` (also under the reference's name ``replace_hunyuan10_attention``) does
the same for HunyuanVideo 1.0 (``svoo/models/hunyuan10/inference.py:31-231``): one
:class:`Hunyuan_SAPAttn_Processor` per double-stream block (layers ``0 .. D-1``), then per
single-stream block (layers ``D ..``), the numbering the per-layer profile CSV is indexed by.
"""

from __future__ import annotations

import os

from .processor import (Hunyuan_SAPAttn_Processor, WanAttn_DenseAttn_Processor, WanAttn_EARAttn_Processor,
                        WanAttn_SAPAttn_Processor)
from .sparsity import SparsityLookup
from .sparsity.exact import resume_requested


def wan_token_geometry(pipe, height: int, width: int, num_frames: int):
    """``(num_frame_patches, frame_patches_one_frame)`` of a Wan pipeline (``inference.py:81-83``)."""
    patch = pipe.transformer.config.patch_size
    num_frame_patches = 1 + num_frames // (pipe.vae_scale_factor_temporal * patch[0])
    mod_value = pipe.vae_scale_factor_spatial * patch[1]
    frame_patches_one_frame = int(height // mod_value) * int(width // mod_value)
    return num_frame_patches, frame_patches_one_frame


def replace_wan_attention(
    pipe,
    height,
    width,
    num_frames,
    first_layers_fp,
    first_times_fp,
    num_inference_steps=None,
    attention_backend="flexattn",
    pattern="SAP",
    num_q_centroids=None,
    num_k_centroids=None,
    top_p_kmeans=None,
    min_kc_ratio=0,
    max_kc_ratio=0,
    ear_gamma=1.0,
    kmeans_iter_init=0,
    kmeans_iter_step=0,
    zero_step_kmeans_init=False,
    use_global_constraints=False,
    use_routing_transformer_strategy=False,
    use_svoo=True,
    start_reuse_step=None,
    reuse_interval=1,
    use_dynamic_min_kc_ratio=False,
    sparsity_csv_path=None,
    dynamic_min_kc_ratio_min=None,
    dynamic_min_kc_ratio_max=None,
    measure_attention_sparsity=False,
    sparsity_output_file="attention_sparsity.txt",
    sparsity_batch_size=0,
    sparsity_query_samples=0,
    sparsity_threshold=0.95,
    sparsity_start_step=1,
    processor_cls=None,
    **unused,
):
    """Configure SVOO attention and install one processor per Wan DiT block.

    Arguments keep the reference's names and meaning (``svoo/models/wan/inference.py:23-74``);
    ``first_layers_fp`` is a layer count and ``first_times_fp`` a timestep threshold, as the CLI
    passes them.  ``max_kc_ratio`` is forwarded to the SAP mask (EAR has no cap).  Patterns:
    ``"SAP"`` (:class:`WanAttn_SAPAttn_Processor`), ``"EAR"`` (:class:`WanAttn_EARAttn_Processor`, with
    ``ear_gamma``) and the ``"dense"`` diagnostic (:class:`WanAttn_DenseAttn_Processor`: dense attention,
    used to record sparsity profiles); anything else, or ``use_svoo=False``, raises ``ValueError`` as the
    reference does (``:77-78``), and the global-constraint / routing variants raise
    ``NotImplementedError``.  ``processor_cls`` overrides the pattern's class (a subclass keeps the
    configuration local to it).  A missing or unreadable profile CSV disables the dynamic ratios
    (``:308-320``).  With ``measure_attention_sparsity`` every processor also appends the exact per-head
    sparsity of each (layer, step) to ``sparsity_output_file`` (the offline profile producer).  Returns the
    processors.
    """
    if pattern not in ("SAP", "EAR", "dense") or not use_svoo:
        raise ValueError("Only SVOO, EAR and dense diagnostic patterns are supported in this release.")
    if use_global_constraints or use_routing_transformer_strategy:
        raise NotImplementedError("global-constraint and routing-transformer variants are not built here")
    num_frame_patches, frame_patches_one_frame = wan_token_geometry(pipe, height, width, num_frames)
    blocks = pipe.transformer.blocks
    num_layers = len(blocks)

    cls = processor_cls or {"SAP": WanAttn_SAPAttn_Processor, "EAR": WanAttn_EARAttn_Processor,
                            "dense": WanAttn_DenseAttn_Processor}[pattern]
    if pattern != "dense":
        cls.use_ear = pattern == "EAR"  # inference.py:282
        cls.ear_gamma = ear_gamma
    cls.first_layers_fp = first_layers_fp
    cls.first_times_fp = first_times_fp
    cls.context_length = 0
    cls.num_frame = num_frame_patches
    cls.frame_size = frame_patches_one_frame
    cls.num_q_centroids = num_q_centroids
    cls.num_k_centroids = num_k_centroids
    cls.top_p_kmeans = top_p_kmeans
    cls.min_kc_ratio = min_kc_ratio
    cls.max_kc_ratio = max_kc_ratio
    cls.num_layers = num_layers
    cls.kmeans_iter_init = kmeans_iter_init
    cls.kmeans_iter_step = kmeans_iter_step
    cls.zero_step_kmeans_init = zero_step_kmeans_init
    cls.use_svoo = True
    cls.start_reuse_step = start_reuse_step
    cls.reuse_interval = reuse_interval
    cls.use_dynamic_min_kc_ratio = False
    cls.sparsity_lookup = None
    # a fresh step counter for this pipeline (the class-level state the processors share)
    cls._current_internal_timestep = None
    cls._inference_step_counter = 0
    cls._seen_timesteps = set()
    if use_dynamic_min_kc_ratio and sparsity_csv_path:
        try:
            cls.sparsity_lookup = SparsityLookup(sparsity_csv_path)
            cls.use_dynamic_min_kc_ratio = True
            cls.dynamic_min_kc_ratio_min = dynamic_min_kc_ratio_min
            cls.dynamic_min_kc_ratio_max = dynamic_min_kc_ratio_max
        except Exception:  # the reference silently falls back to the scalar ratio
            cls.use_dynamic_min_kc_ratio = False
            cls.sparsity_lookup = None

    # offline profiling (inference.py:322-341): a fresh raw log unless SVOO_SPARSITY_RESUME keeps it
    cls.measure_attention_sparsity = measure_attention_sparsity
    cls.sparsity_output_file = sparsity_output_file
    cls.sparsity_batch_size = sparsity_batch_size
    cls.sparsity_query_samples = sparsity_query_samples
    cls.sparsity_threshold = sparsity_threshold
    cls.sparsity_start_step = sparsity_start_step
    if measure_attention_sparsity and sparsity_output_file:
        d = os.path.dirname(sparsity_output_file)
        if d:
            os.makedirs(d, exist_ok=True)
        if not resume_requested():
            open(sparsity_output_file, "w", encoding="utf-8").close()

    processors = []
    for transformer in (pipe.transformer, getattr(pipe, "transformer_2", None)):
        if transformer is None:
            continue
        for layer_idx, block in enumerate(transformer.blocks):
            if hasattr(block.attn1, "set_processor"):
                proc = cls(layer_idx=layer_idx)
                proc.num_layers = num_layers
                block.attn1.set_processor(proc)
                processors.append(proc)
    return processors


def _configure_profile(cls, use_dynamic_min_kc_ratio, sparsity_csv_path, dynamic_min_kc_ratio_min,
                       dynamic_min_kc_ratio_max) -> None:
    """Per-head ratios from a profile CSV; a missing or unreadable CSV leaves the scalar ratio in force."""
    cls.use_dynamic_min_kc_ratio = False
    cls.sparsity_lookup = None
    cls.dynamic_min_kc_ratio_min = None
    cls.dynamic_min_kc_ratio_max = None
    if use_dynamic_min_kc_ratio and sparsity_csv_path:
        try:
            cls.sparsity_lookup = SparsityLookup(sparsity_csv_path)
        except Exception:
            return
        cls.use_dynamic_min_kc_ratio = True
        cls.dynamic_min_kc_ratio_min = dynamic_min_kc_ratio_min
        cls.dynamic_min_kc_ratio_max = dynamic_min_kc_ratio_max


def replace_hunyuan_attention(
    pipe,
    height,
    width,
    num_frames,
    prompt_length,
    first_layers_fp,
    first_times_fp,
    pattern="SAP",
    num_q_centroids=None,
    num_k_centroids=None,
    top_p_kmeans=None,
    min_kc_ratio=0,
    max_kc_ratio=0,
    kmeans_iter_init=0,
    kmeans_iter_step=0,
    zero_step_kmeans_init=False,
    context_length=256,
    use_svoo=True,
    start_reuse_step=None,
    reuse_interval=1,
    use_dynamic_min_kc_ratio=False,
    sparsity_csv_path=None,
    dynamic_min_kc_ratio_min=None,
    dynamic_min_kc_ratio_max=None,
    measure_attention_sparsity=False,
    sparsity_output_file="attention_sparsity.txt",
    sparsity_batch_size=0,
    sparsity_query_samples=0,
    sparsity_threshold=0.95,
    sparsity_start_step=1,
    processor_cls=None,
    **unused,
):
    """Configure SVOO attention and install one processor per HunyuanVideo 1.0 transformer block.

    Arguments keep the names and meaning of ``replace_hunyuan10_attention``
    (``svoo/models/hunyuan10/inference.py:31-65``).  The token geometry is HunyuanVideo's: ``1 +
    num_frames // 4`` latent frames of ``height * width // 256`` patches, and 256 text tokens (the
    reference fixes the text length at 256 whatever ``context_length`` says, ``:68-70``; so does this
    function).  Only the SAP pattern with ``use_svoo`` exists for HunyuanVideo (``:66-67``); anything
    else raises ``ValueError``.  ``prompt_length`` (the valid text tokens) must lie in ``[0, 256]``.

    Processors go to ``block.attn.processor`` of every ``pipe.transformer.transformer_blocks`` entry
    (double stream, layers ``0 .. D-1``) and then of every ``single_transformer_blocks`` entry (layers
    ``D + i``, ``:207-231``).  The blocks must pass ``timestep`` to their attention, as the reference's
    patched block forwards do (``custom_models.py:383-390``; the pipeline side is not part of this
    package).  ``processor_cls`` overrides the class (a subclass keeps the configuration local).
    Returns the processors in layer order.
    """
    if pattern != "SAP" or not use_svoo:
        raise ValueError("Only SVOO (pattern='SAP') is supported for HunyuanVideo in this release.")
    context_length = 256
    if not 0 <= int(prompt_length) <= context_length:
        raise ValueError(f"prompt_length={prompt_length} must lie in [0, {context_length}]")
    tr = pipe.transformer
    double = list(tr.transformer_blocks)
    single = list(getattr(tr, "single_transformer_blocks", []))

    cls = processor_cls or Hunyuan_SAPAttn_Processor
    cls.first_layers_fp = first_layers_fp
    cls.first_times_fp = first_times_fp
    cls.prompt_length = int(prompt_length)
    cls.context_length = context_length
    cls.num_frame = 1 + num_frames // 4
    cls.frame_size = height * width // 256
    cls.num_layers = len(double) + len(single)
    cls.num_q_centroids = num_q_centroids
    cls.num_k_centroids = num_k_centroids
    cls.top_p_kmeans = top_p_kmeans
    cls.min_kc_ratio = min_kc_ratio
    cls.max_kc_ratio = max_kc_ratio
    cls.kmeans_iter_init = kmeans_iter_init
    cls.kmeans_iter_step = kmeans_iter_step
    cls.zero_step_kmeans_init = zero_step_kmeans_init
    cls.use_svoo = True
    cls.start_reuse_step = start_reuse_step
    cls.reuse_interval = 1 if reuse_interval is None else max(1, int(reuse_interval))
    _configure_profile(cls, use_dynamic_min_kc_ratio, sparsity_csv_path, dynamic_min_kc_ratio_min,
                       dynamic_min_kc_ratio_max)
    cls.measure_attention_sparsity = measure_attention_sparsity
    cls.sparsity_output_file = sparsity_output_file
    cls.sparsity_batch_size = sparsity_batch_size
    cls.sparsity_query_samples = sparsity_query_samples
    cls.sparsity_threshold = sparsity_threshold
    cls.sparsity_start_step = sparsity_start_step

    processors = []
    for layer_idx, block in enumerate(double + single):
        proc = cls(layer_idx=layer_idx)
        proc.num_layers = cls.num_layers
        block.attn.processor = proc
        processors.append(proc)
    return processors


replace_hunyuan10_attention = replace_hunyuan_attention
