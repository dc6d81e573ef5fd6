"""MI355X (gfx950) memory-efficient causal attention block.

Drop-in for ``fused_attn`` / ``FusedAttentionFunction`` of
xTimeCrystal/memory_efficient_attn_layer (fast_triton_attn.py:373-697), backed
by hand-written HIP kernels in libmea.so (C ABI: include/mea.h).
"""
from .attention import FusedAttentionFunction, FusedAttentionVarlenFunction, fused_attn, fused_attn_varlen
from .decode import DecodeGraph, KVCache, decode_step, prefill
from .module import CausalSoftmaxAttention
from .yarn import Yarn, rotary_tables, swap_even_odd

__all__ = [
    "FusedAttentionFunction",
    "fused_attn",
    "FusedAttentionVarlenFunction",
    "fused_attn_varlen",
    "CausalSoftmaxAttention",
    "KVCache",
    "DecodeGraph",
    "prefill",
    "decode_step",
    "Yarn",
    "rotary_tables",
    "swap_even_odd",
]
__version__ = "0.1.0"
