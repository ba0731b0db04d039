"""MI355X-native NF4 QLoRA linear and gated-MLP hot path (drop-in for MOLT's
``molt_stream`` NF4-LoRA methods), on hand-written HIP kernels for gfx950."""
from .errors import CapabilityError, MoltError, MoltStreamError
from .nf4 import (NF4_CODEBOOK, NF4DevicePayload, NF4Tensor, QuantState, dequantize_4bit, dynamic_map,
                  quantize_4bit, resolved_nf4_scales)

__version__ = "0.3.0"

__all__ = [
    "CapabilityError", "MoltError", "MoltStreamError", "NF4_CODEBOOK", "NF4DevicePayload", "NF4Tensor",
    "QuantState", "dequantize_4bit", "dynamic_map", "quantize_4bit", "resolved_nf4_scales",
]
