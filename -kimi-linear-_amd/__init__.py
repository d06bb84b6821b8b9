"""MI355X-native (gfx950) Kimi Delta Attention core.

Drop-in replacements for the reference's ``kimi_linear.kda_chunkwise`` and
``kimi_linear.kda_recurrent`` (kimi_linear/__init__.py:9), running hand-written
HIP kernels behind the C ABI in ``include/kda_hip.h``, and the reference's
``KimiDeltaAttention`` layer (kimi_linear/kda.py:331-536) around that core.
"""

from .kda import (FP16_MAX_SAFE, KdaError, kda_chunkwise, kda_chunkwise_fused,  # noqa: F401
                  kda_chunkwise_gated, kda_recurrent, kda_recurrent_gated)
from .layer import HeadwiseRMSNorm, KimiDeltaAttention, ShortConv, l2norm, linear_attn_config  # noqa: F401

__all__ = ["kda_chunkwise", "kda_recurrent", "kda_chunkwise_gated", "kda_recurrent_gated", "kda_chunkwise_fused",
           "KdaError", "FP16_MAX_SAFE", "KimiDeltaAttention", "ShortConv", "HeadwiseRMSNorm", "l2norm",
           "linear_attn_config"]
