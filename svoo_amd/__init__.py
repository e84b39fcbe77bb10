"""MI355X-native SVOO online sparse-attention hot path.

QK co-clustering, cluster permutes, profile-driven block masks and variable-block-sparse
attention as hand-written HIP kernels for gfx950 behind a C ABI (``include/svoo_hip.h``), with
the reference's Python operator and attention-processor API on top.
"""

from .co_clustering import (  # noqa: F401
    block_mask_lengths,
    co_cluster_tokens,
    co_cluster_tokens_full,
    dynamic_block_sparse_fwd,
    dynamic_block_sparse_fwd_flashinfer,
    dynamic_block_sparse_fwd_triton,
    identify_dynamic_map,
    triton_l2norm_forward,
    weighted_softmax,
)
from .permute import (  # noqa: F401
    apply_inverse_permutation,
    apply_inverse_permutation_triton,
    cluster_sort,
    permute_tensor_by_labels,
    permute_tensor_by_labels_triton,
)
from .sparsity import SparsityLookup  # noqa: F401

__version__ = "0.1.0"
