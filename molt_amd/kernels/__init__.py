"""Drop-ins for ``molt_stream.kernels`` on the NF4 QLoRA hot path."""
from .frozen_rmsnorm import FrozenRMSNormBF16, enable_frozen_rmsnorm_bf16, enable_qwen2_frozen_rmsnorm_bf16
from .gated_activation import enable_fused_silu_mlp, fused_silu_multiply

__all__ = ["FrozenRMSNormBF16", "enable_frozen_rmsnorm_bf16", "enable_fused_silu_mlp", "enable_qwen2_frozen_rmsnorm_bf16",
           "fused_silu_multiply"]
