"""genie_tk — pair-representation hot path (triangle multiplicative update,
triangle attention, LayerNorm) on hand-written gfx950 (MI355X) HIP kernels.

The public names are those of the reference package (src/genie_tk/__init__.py:35-50).
"""

__version__ = "0.1.0"

from genie_tk.triangle_mul import (
    TriangleMultiplicativeUpdate,
    TriangleMultiplicationOutgoing,
    TriangleMultiplicationIncoming,
)
from genie_tk.triangle_attention import (
    TriangleAttention,
    TriangleAttentionStartingNode,
    TriangleAttentionEndingNode,
)
from genie_tk.pair_transform import PairTransformLayer, PairTransformNet
from genie_tk.utils import has_cuda_kernels, get_device_info

__all__ = [
    "TriangleMultiplicativeUpdate",
    "TriangleMultiplicationOutgoing",
    "TriangleMultiplicationIncoming",
    "TriangleAttention",
    "TriangleAttentionStartingNode",
    "TriangleAttentionEndingNode",
    "PairTransformLayer",
    "PairTransformNet",
    "has_cuda_kernels",
    "get_device_info",
]
