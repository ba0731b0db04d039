"""Drop-ins for ``molt_stream.methods`` on the NF4 QLoRA hot path."""
from .gated_replay import (asymmetric_gated_nf4_lora, enable_asymmetric_gated_replay,
                           enable_fused_gated_nf4_lora, enable_rmsnorm_replay, fused_gated_nf4_lora_mlp)
from .nf4_backward import packed_nf4_backward_input, packed_nf4_lora_backward_input, resolved_nf4_scales
from .nf4_layer_cache import dense_nf4_layer_cache
from .nf4_lora import enable_scheduled_nf4_lora, scheduled_nf4_lora
from .stacked_lora import enable_stacked_nf4_lora, stacked_nf4_lora

__all__ = [
    "asymmetric_gated_nf4_lora", "enable_asymmetric_gated_replay", "enable_fused_gated_nf4_lora", "enable_rmsnorm_replay",
    "fused_gated_nf4_lora_mlp", "packed_nf4_backward_input", "packed_nf4_lora_backward_input",
    "resolved_nf4_scales", "dense_nf4_layer_cache", "enable_scheduled_nf4_lora", "scheduled_nf4_lora",
    "enable_stacked_nf4_lora", "stacked_nf4_lora",
]
