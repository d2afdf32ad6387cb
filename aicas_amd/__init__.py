"""aicas_amd — MI355X-native KV-cache append and q_len=1 GQA decode attention for the Qwen3-VL-2B text
decoder, a drop-in for the decode path of Frun1na/AICAS's ``triton_qwen3vl`` package.

Same import surface as ``triton_qwen3vl/__init__.py:1-16`` for this path: the backend keys,
``TRITON_AVAILABLE`` (False: nothing here is Triton), ``gqa_decode_attention`` and
``install_qwen3vl_triton_attention``; plus the HF cache (``AicasDecodeCache``) whose ``update`` runs the HIP
append kernel, and ``install_fused_decode``, which runs a text layer's whole decode step (q/k norms, rotary
embedding, cache update, attention) in one launch, and ``AicasGraphDecodeRunner``, which captures a whole
decode step of the text model as a HIP graph. The kernels live in ``libaicas_decode.so`` (C ABI in
include/aicas_decode.h).
"""

from .backends import TEXT_BACKEND_KEY, VISION_BACKEND_KEY, text_triton_attention, vision_triton_attention
from .gqa_decode_attention import can_use_gqa_decode_attention, gqa_decode_attention
from .patch import TRITON_AVAILABLE, install_qwen3vl_triton_attention

__all__ = [
    "TEXT_BACKEND_KEY",
    "TRITON_AVAILABLE",
    "VISION_BACKEND_KEY",
    "can_use_gqa_decode_attention",
    "gqa_decode_attention",
    "install_qwen3vl_triton_attention",
    "text_triton_attention",
    "vision_triton_attention",
]


def __getattr__(name):
    # the cache classes and the attention patch import transformers; load them on first use
    if name in ("AicasDecodeCache", "AicasKVCacheLayer"):
        from . import kv_cache

        return getattr(kv_cache, name)
    if name in ("install_fused_decode", "uninstall_fused_decode"):
        from . import fused_attention

        return getattr(fused_attention, name)
    if name == "AicasGraphDecodeRunner":
        from . import graph_runner

        return graph_runner.AicasGraphDecodeRunner
    raise AttributeError(name)
