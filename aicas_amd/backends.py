"""HF attention-interface functions (drop-in for triton_qwen3vl/backends.py).

``text_triton_attention`` keeps the reference's signature, return convention and routing
(triton_qwen3vl/backends.py:179-289):
  * ``output_attentions`` -> SDPA (backends.py:194-205);
  * q_len == 1, no mask, no dropout and ``can_use_gqa_decode_attention`` -> the HIP decode kernel, output
    transposed to ``[B, 1, Hq, D]`` contiguous (backends.py:207-227). Unlike the reference there is no
    try/except around the kernel: a failure raises instead of warning once and falling back to SDPA
    (backends.py:228-233);
  * everything else (prefill, masked calls, CPU tensors) -> SDPA (backends.py:235-260). The reference's
    Triton prefill kernel (gqa_flash_attention.py) is outside this package's scope.

``vision_triton_attention`` keeps the reference's signature (backends.py:90-176) and serves the vision
encoder through the reference's own SDPA-per-chunk route (backends.py:41-87); vision attention is outside
this package's scope.
"""

from __future__ import annotations

import torch

from .fallback import sdpa_fallback
from .gqa_decode_attention import can_use_gqa_decode_attention, gqa_decode_attention, kv_descriptor

TEXT_BACKEND_KEY = "qwen3vl_triton_flash_text"
VISION_BACKEND_KEY = "qwen3vl_triton_flash_vision"


def _resolve_is_causal(module: torch.nn.Module, is_causal: bool | None) -> bool:
    if is_causal is not None:
        return is_causal
    return bool(getattr(module, "is_causal", True))


def _resolve_scale(module: torch.nn.Module, scaling: float | None) -> float:
    if scaling is not None:
        return scaling
    return float(getattr(module, "scaling"))


def _split_lengths(cu_seq_lens: torch.Tensor) -> list[int]:
    return (cu_seq_lens[1:] - cu_seq_lens[:-1]).detach().cpu().tolist()


def _vision_varlen_sdpa(
    module, query, key, value, *, dropout, scaling, cu_seq_lens_q, cu_seq_lens_k, is_causal, **kwargs
) -> tuple[torch.Tensor, None]:
    """Packed vision attention as independent SDPA calls per cu_seq_lens chunk (backends.py:41-87)."""
    if cu_seq_lens_q is None or cu_seq_lens_k is None:
        return sdpa_fallback(
            module, query, key, value, attention_mask=None, dropout=dropout, scaling=scaling,
            is_causal=is_causal, **kwargs,
        )
    q_chunks = torch.split(query, _split_lengths(cu_seq_lens_q), dim=2)
    k_lengths = _split_lengths(cu_seq_lens_k)
    k_chunks = torch.split(key, k_lengths, dim=2)
    v_chunks = torch.split(value, k_lengths, dim=2)
    outputs = []
    for q_chunk, k_chunk, v_chunk in zip(q_chunks, k_chunks, v_chunks):
        out, _ = sdpa_fallback(
            module, q_chunk, k_chunk, v_chunk, attention_mask=None, dropout=dropout, scaling=scaling,
            is_causal=is_causal, **kwargs,
        )
        outputs.append(out)
    return torch.cat(outputs, dim=1), None


def vision_triton_attention(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
    dropout: float = 0.0,
    scaling: float | None = None,
    cu_seq_lens_q: torch.Tensor | None = None,
    cu_seq_lens_k: torch.Tensor | None = None,
    max_length_q: int | torch.Tensor | None = None,
    max_length_k: int | torch.Tensor | None = None,
    is_causal: bool | None = None,
    **kwargs,
) -> tuple[torch.Tensor, None]:
    del attention_mask, max_length_q, max_length_k
    is_causal = _resolve_is_causal(module, is_causal)
    sm_scale = _resolve_scale(module, scaling)
    return _vision_varlen_sdpa(
        module, query, key, value, dropout=dropout, scaling=sm_scale, cu_seq_lens_q=cu_seq_lens_q,
        cu_seq_lens_k=cu_seq_lens_k, is_causal=is_causal, **kwargs,
    )


def text_triton_attention(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None,
    dropout: float = 0.0,
    scaling: float | None = None,
    is_causal: bool | None = None,
    **kwargs,
) -> tuple[torch.Tensor, None]:
    is_causal = _resolve_is_causal(module, is_causal)
    sm_scale = _resolve_scale(module, scaling)
    num_key_value_groups = int(getattr(module, "num_key_value_groups", 1))

    if kwargs.get("output_attentions", False):
        return sdpa_fallback(
            module, query, key, value, attention_mask, dropout=dropout, scaling=sm_scale, is_causal=is_causal,
            **kwargs,
        )

    meta = kv_descriptor(key)
    # The decode kernel has no per-token mask. HF hands an attention function a mask only when some position is
    # padding (flash_attention_mask returns None for an all-ones mask), so a masked call takes the SDPA route
    # with the mask, as the reference does (backends.py:235-260): dense caches as they are, paged or fp8 caches
    # through aicas_kv_gather. A ragged aicas cache defines visibility through its own per-sequence lengths,
    # which a padding mask over a common length cannot describe: refused rather than silently ignored.
    if attention_mask is not None and meta is not None and not meta.dense and meta.min_seq_len != meta.max_seq_len:
        raise ValueError(
            "a padding mask reached an aicas cache whose sequences have different lengths: use a cache whose "
            "sequences advance together (HF's left padding) or no mask"
        )
    can_use_decode = (
        attention_mask is None
        and query.shape[2] == 1
        and dropout == 0.0
        and can_use_gqa_decode_attention(query, key, value, num_key_value_groups=num_key_value_groups)
    )
    if can_use_decode:
        attn_output = gqa_decode_attention(
            query, key, value, sm_scale=sm_scale, num_key_value_groups=num_key_value_groups
        )
        return attn_output.transpose(1, 2).contiguous(), None

    return sdpa_fallback(
        module, query, key, value, attention_mask, dropout=dropout, scaling=sm_scale, is_causal=is_causal,
        **kwargs,
    )
