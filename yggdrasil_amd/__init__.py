"""yggdrasil_amd -- MI355X-native (gfx950) MoE-HLM expert layer.

A from-scratch HIP implementation of Yggdrasil's MoE-HLM expert layer
(``holograph/models/hlm_block.py:154-183``): CliffordRouter top-k gating,
token dispatch, grouped CliffordLinear expert products with the grade-wise
activation fused, and the weighted combine, behind the C ABI declared in
``include/ygg_moe.h`` and the torch module ``CliffordMoELayer``; the pre-norm
and residual around it (``hlm_block.py:144-151``) as ``CliffordMoEBlockFFN``.
"""

from .layers import (CliffordLayerNorm, CliffordLinear, CliffordMoEBlockFFN, CliffordMoELayer,  # noqa: F401
                     MoEHLMConfig)
from . import ops  # noqa: F401

__all__ = ["CliffordMoELayer", "CliffordMoEBlockFFN", "CliffordLayerNorm", "CliffordLinear", "MoEHLMConfig", "ops"]
