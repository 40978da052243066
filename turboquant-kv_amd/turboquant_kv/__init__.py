"""turboquant_kv -- TurboQuant KV-cache compression and vector search on MI355X (gfx950).

Drop-in for the reference package's quantize-and-score path (turboquant_kv/__init__.py:7-61):
the quantize/dequantize functions, QuantizedKVCache, TurboQuantIndex, the HF
TurboQuantCache and the vLLM backend, computed by hand-written HIP kernels behind
torch.ops.turboquant; the Huffman storage of code indices (entropy.py) and the C++
core's TQIX index files (formats.py).  The multi-GPU wrapper is not part of this package.
"""

from turboquant_kv.config import TurboQuantConfig
from turboquant_kv.cache import QuantizedKVCache
from turboquant_kv.search import TurboQuantIndex
from turboquant_kv.quantizers import TurboQuantMSE, TurboQuantProd
from turboquant_kv.entropy import HuffmanCoder, EntropyPackedStorage, compute_codeword_probabilities
from turboquant_kv.reference import (
    quantize_mse,
    dequantize_mse,
    quantize_prod,
    dequantize_prod,
)

try:
    from turboquant_kv.hf_integration import TurboQuantCache
except ImportError:  # transformers missing
    TurboQuantCache = None  # type: ignore[assignment,misc]

try:
    from turboquant_kv.vllm_plugin import (
        TurboQuantKVCacheConfig,
        TurboQuantPagedKVCache,
        TurboQuantAttentionBackend,
    )
except ImportError:
    TurboQuantKVCacheConfig = None  # type: ignore[assignment,misc]
    TurboQuantPagedKVCache = None  # type: ignore[assignment,misc]
    TurboQuantAttentionBackend = None  # type: ignore[assignment,misc]

__version__ = "0.1.0"

__all__ = [
    "TurboQuantConfig",
    "QuantizedKVCache",
    "TurboQuantIndex",
    "TurboQuantMSE",
    "TurboQuantProd",
    "HuffmanCoder",
    "EntropyPackedStorage",
    "compute_codeword_probabilities",
    "quantize_mse",
    "dequantize_mse",
    "quantize_prod",
    "dequantize_prod",
    "TurboQuantCache",
    "TurboQuantKVCacheConfig",
    "TurboQuantPagedKVCache",
    "TurboQuantAttentionBackend",
]
