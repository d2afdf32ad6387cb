"""Backend installer (drop-in for triton_qwen3vl/patch.py).

``install_qwen3vl_triton_attention(model)`` does what the reference's does (triton_qwen3vl/patch.py:23-63):
registers the text and vision attention functions under the same keys in HF's ``ALL_ATTENTION_FUNCTIONS``,
aliases both mask functions to ``flash_attention_2``'s (which returns ``None`` when there is no padding, so
decode reaches the kernel), points the four config objects' ``_attn_implementation`` at the keys when they
exist, and returns the same state-dict keys. ``triton_available`` is False (there is no Triton here); the
``*_enabled`` flags report what runs on the HIP library.
"""

from __future__ import annotations

from typing import Any

from . import _lib
from .backends import TEXT_BACKEND_KEY, VISION_BACKEND_KEY, text_triton_attention, vision_triton_attention

TRITON_AVAILABLE = False


def _load_attention_registries():
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    return ALL_ATTENTION_FUNCTIONS, ALL_MASK_ATTENTION_FUNCTIONS


def _set_attr_if_present(target: Any, attr_name: str, value: str) -> bool:
    if target is None or not hasattr(target, attr_name):
        return False
    setattr(target, attr_name, value)
    return True


def hip_decode_available() -> bool:
    """True if libaicas_decode.so is built and loads."""
    try:
        _lib.lib()
    except _lib.AicasError:
        return False
    return True


def install_qwen3vl_triton_attention(model: Any) -> dict[str, Any]:
    attention_registry, mask_registry = _load_attention_registries()

    if VISION_BACKEND_KEY not in attention_registry:
        attention_registry.register(VISION_BACKEND_KEY, vision_triton_attention)
    if TEXT_BACKEND_KEY not in attention_registry:
        attention_registry.register(TEXT_BACKEND_KEY, text_triton_attention)

    if VISION_BACKEND_KEY not in mask_registry:
        mask_registry.register(VISION_BACKEND_KEY, mask_registry["flash_attention_2"])
    if TEXT_BACKEND_KEY not in mask_registry:
        mask_registry.register(TEXT_BACKEND_KEY, mask_registry["flash_attention_2"])

    base_model = getattr(model, "model", None)
    visual = getattr(base_model, "visual", None)
    language_model = getattr(base_model, "language_model", None)
    model_config = getattr(model, "config", None)

    mutated = {
        "model.model.visual.config": _set_attr_if_present(
            getattr(visual, "config", None), "_attn_implementation", VISION_BACKEND_KEY
        ),
        "model.model.language_model.config": _set_attr_if_present(
            getattr(language_model, "config", None), "_attn_implementation", TEXT_BACKEND_KEY
        ),
        "model.config.vision_config": _set_attr_if_present(
            getattr(model_config, "vision_config", None), "_attn_implementation", VISION_BACKEND_KEY
        ),
        "model.config.text_config": _set_attr_if_present(
            getattr(model_config, "text_config", None), "_attn_implementation", TEXT_BACKEND_KEY
        ),
    }

    hip = hip_decode_available()
    return {
        "installed": True,
        "triton_available": TRITON_AVAILABLE,
        "vision_backend_key": VISION_BACKEND_KEY,
        "text_backend_key": TEXT_BACKEND_KEY,
        "vision_varlen_triton_enabled": False,
        "text_prefill_gqa_triton_enabled": False,
        "text_decode_triton_enabled": hip,
        "mutated_configs": mutated,
    }
