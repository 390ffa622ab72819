"""
Wide primitives: N independent copies of a torch.nn layer executed as one HIP kernel family
(mirror of wide_compiler/core/primitives/__init__.py).  All inputs and outputs are N-first.
"""

from .wide_conv1d import WideConv1d, Conv1dStrategy
from .wide_conv2d import (
    WideConv2d,
    ConvStrategy,
    select_strategy as select_conv_strategy,
    create_wide_conv2d,
    STRATEGY_THRESHOLDS as CONV_THRESHOLDS,
)
from .wide_conv3d import WideConv3d, Conv3dStrategy
from .wide_linear import WideLinear, WideMLP2, LinearStrategy, select_linear_strategy, LINEAR_THRESHOLDS
from .wide_batchnorm_1d import WideBatchNorm1d
from .wide_batchnorm_2d import WideBatchNorm2d
from .wide_layernorm import WideLayerNorm
from .wide_groupnorm import WideGroupNorm, GroupNormStrategy
from .wide_instancenorm import WideInstanceNorm1d, WideInstanceNorm2d, InstanceNormStrategy
from .wide_embedding import WideEmbedding, EmbeddingStrategy
from .wide_attention import WideAttention, AttentionStrategy
from .wide_gru import WideGRU, GRUStrategy
from .wide_lstm import WideLSTM, LSTMStrategy

__all__ = [
    "WideConv1d", "Conv1dStrategy", "WideConv2d", "ConvStrategy", "select_conv_strategy",
    "create_wide_conv2d", "CONV_THRESHOLDS", "WideConv3d", "Conv3dStrategy",
    "WideLinear", "WideMLP2", "LinearStrategy", "select_linear_strategy", "LINEAR_THRESHOLDS",
    "WideBatchNorm1d", "WideBatchNorm2d", "WideLayerNorm", "WideGroupNorm", "GroupNormStrategy",
    "WideInstanceNorm1d", "WideInstanceNorm2d", "InstanceNormStrategy",
    "WideEmbedding", "EmbeddingStrategy", "WideAttention", "AttentionStrategy",
    "WideGRU", "GRUStrategy", "WideLSTM", "LSTMStrategy",
]
