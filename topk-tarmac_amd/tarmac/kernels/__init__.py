"""HIP kernel entry points, one module per reference module of ``src/kernels``."""

from .backward import (dense_attention_backward, dense_attention_forward_stats,
                       fixedset_attention_backward)
from .fused_dense_attention import fused_dense_attention
from .fused_prescore_attention import fused_prescore_attention
from .fused_topk_attention import (fused_topk_attention, fused_topk_attention_masked,
                                   fused_topk_attention_sort, fused_topk_attention_tiled,
                                   reference_topk_attention, topk_attention,
                                   topk_variant_attention)
from .prescore_selection import (SELECTORS, _morton_code, grid_knn_recall, grid_knn_shape,
                                 prescore_attention, prescore_full, select_grid_knn,
                                 select_morton_window, select_radius_knn, zorder_attention)
from .streaming_topk_attention import streaming_topk_attention

__all__ = [
    "dense_attention_backward", "dense_attention_forward_stats", "fixedset_attention_backward",
    "fused_dense_attention", "fused_prescore_attention", "fused_topk_attention",
    "fused_topk_attention_masked", "fused_topk_attention_sort", "fused_topk_attention_tiled",
    "reference_topk_attention", "topk_attention", "topk_variant_attention",
    "prescore_attention", "prescore_full", "select_morton_window", "select_radius_knn",
    "select_grid_knn", "grid_knn_shape", "grid_knn_recall", "SELECTORS",
    "zorder_attention", "streaming_topk_attention", "_morton_code",
]
