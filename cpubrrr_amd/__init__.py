"""cpubrrr_amd -- MI355X (gfx950) MoE expert-FFN decode path of arizqi/cpubrrr.

The product is libcpb_moe.so (HIP kernels + C ABI, include/cpb_moe.h); this
package is its Python host mirror (`MoeBlock`) and workload synthesiser.
"""
from .moe import MoeBlock, MoeConfig  # noqa: F401
from . import synth  # noqa: F401
from .gguf import GgufFile  # noqa: F401
from .head import LmHead  # noqa: F401
from .attn import Attention  # noqa: F401

__all__ = ["MoeBlock", "MoeConfig", "synth", "GgufFile", "LmHead", "Attention"]
