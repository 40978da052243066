"""TurboQuant configuration (same fields and defaults as turboquant_kv/config.py:6-30)."""

from dataclasses import dataclass


@dataclass
class TurboQuantConfig:
    """Configuration for TurboQuant KV cache compression.

    Attributes:
        key_bits: Quantization bit width for keys (default 4).
        value_bits: Quantization bit width for values (default 2).
        mode: "mse" (Algorithm 1) or "prod" (Algorithm 2).
        rotation: "dense_qr" (exact paper) or "rht" (Hadamard-based).
        outlier_channels: Accepted for compatibility; builds no separate codebook use.
        protected_layers: First N layers kept at full precision.
        quantize_on_append: Quantize on append (always True in practice).
        block_size: 0 = per-token quantization (the only mode implemented).
        seed: Random seed for rotation matrices (keys use seed, values seed + 1).
    """

    key_bits: int = 4
    value_bits: int = 2
    mode: str = "mse"
    rotation: str = "dense_qr"
    outlier_channels: int = 0
    protected_layers: int = 0
    quantize_on_append: bool = True
    block_size: int = 0
    seed: int = 42
