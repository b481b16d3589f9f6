"""MI355X-native (gfx950) prefix-LM attention for Mimir2.

Drop-in replacement for ``mimir.model.layers.flash_attn_varlen_prefixlm``
(src/mimir/model/flash_attention_prefixlm_v2.py:286-306) backed by hand-written
HIP kernels behind a C ABI (include/mimir_prefixlm.h), and the attention
layer's core around it (``gated_attention``: gqkv split, RoPE, the operator and
the sigmoid output gate of src/mimir/model/layers.py:182-239).
"""

from .metadata import (
    PrefixLMSeqInfo,
    allowed_pairs,
    compute_aux_seq_tensors_scalars,
    prefixlm_seq_info_from_tensors,
)
from .layer import gated_attention, rope
from .prefixlm import (
    PrefixLMAttention,
    check_metadata,
    flash_attn_varlen_prefixlm,
    prefixlm_attn_bwd,
    prefixlm_attn_fwd,
    set_dscore_workspace_limit,
    set_validate_metadata,
)

__all__ = [
    "PrefixLMAttention",
    "PrefixLMSeqInfo",
    "allowed_pairs",
    "check_metadata",
    "compute_aux_seq_tensors_scalars",
    "flash_attn_varlen_prefixlm",
    "gated_attention",
    "prefixlm_attn_bwd",
    "prefixlm_attn_fwd",
    "prefixlm_seq_info_from_tensors",
    "rope",
    "set_dscore_workspace_limit",
    "set_validate_metadata",
]
