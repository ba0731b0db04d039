"""Drop-ins for ``molt_stream.kernels`` on the NF4 QLoRA hot path."""
from .gated_activation import enable_fused_silu_mlp, fused_silu_multiply

__all__ = ["enable_fused_silu_mlp", "fused_silu_multiply"]
