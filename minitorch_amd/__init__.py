"""minitorch_amd -- MI355X-native causal-attention hot path for minitorch.

The public surface mirrors the reference package (minitorch/__init__.py):
Tensor, no_grad, Module, Sequential, Linear, LayerNorm, Embedding, GELU,
Dropout, GPT, TransformerBlock, MultiHeadAttention, cross_entropy_loss, Adam,
F.  Every operation runs in libmtx_hip.so (HIP, gfx950) through the C ABI in
include/mtx.h, device memory included (the library's caching allocator):
no other GPU framework is imported.
"""
__version__ = "0.1.0"

from . import functional as F  # noqa: E402
from .graphs import CapturedStep  # noqa: E402
from .layers import GELU, Dropout, Embedding, LayerNorm, Linear  # noqa: E402
from .loss import cross_entropy_loss  # noqa: E402
from .module import Module, Sequential  # noqa: E402
from .optim import Adam  # noqa: E402
from .tensor import Tensor, no_grad  # noqa: E402
from .transformer import GPT, MultiHeadAttention, TransformerBlock  # noqa: E402

__all__ = [
    "Tensor", "no_grad",
    "Module", "Sequential",
    "Linear", "Dropout", "GELU", "LayerNorm", "Embedding",
    "GPT", "TransformerBlock", "MultiHeadAttention",
    "cross_entropy_loss",
    "Adam",
    "CapturedStep",
    "F",
]
