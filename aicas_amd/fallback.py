"""SDPA route for the attention calls that are not q_len=1 decode (prefill, masked or
``output_attentions`` calls, CPU tensors).

These calls are outside the decode path this package accelerates; like the reference
(triton_qwen3vl/fallback.py:23-64, routing in triton_qwen3vl/backends.py:194-205, 249-260) they go to HF's
``sdpa_attention_forward`` when transformers is importable, else to ``F.scaled_dot_product_attention`` over
``repeat_kv``. The decode path never reaches this module: a decode call that the HIP kernel cannot serve
fails loudly instead.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, Hkv, L, D] -> [B, Hkv*n_rep, L, D]; q head i reads kv head i // n_rep (fallback.py:7-12)."""
    batch, num_key_value_heads, seq_len, head_dim = hidden_states.shape
    if n_rep == 1:
        return hidden_states
    expanded = hidden_states[:, :, None, :, :].expand(batch, num_key_value_heads, n_rep, seq_len, head_dim)
    return expanded.reshape(batch, num_key_value_heads * n_rep, seq_len, head_dim)


def _load_sdpa_attention_forward():
    try:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
    except Exception:
        return None
    return sdpa_attention_forward


def _padding_mask_4d(attention_mask: torch.Tensor, q_len: int, kv_len: int, causal: bool) -> torch.Tensor:
    """The 2-D padding mask ``[B, kv]`` an attention function receives when its mask interface is
    flash_attention_2's (transformers/masking_utils.py:607-647, what install_qwen3vl_triton_attention aliases) ->
    the 4-D boolean ``[B, 1, q, kv]`` mask HF's own SDPA path builds for the same step
    (masking_utils.sdpa_mask, queries at the last q_len positions). SDPA cannot broadcast a 2-D ``[B, kv]`` mask
    over ``[B, H, q, kv]`` scores for B > 1, which is what the reference's fallback would hand it."""
    from transformers.masking_utils import bidirectional_mask_function, causal_mask_function, sdpa_mask

    return sdpa_mask(batch_size=attention_mask.shape[0], q_length=q_len, kv_length=kv_len, q_offset=kv_len - q_len,
                     kv_offset=0, mask_function=causal_mask_function if causal else bidirectional_mask_function,
                     attention_mask=attention_mask.bool(), allow_is_causal_skip=False, device=attention_mask.device)


def _causal_continuation_mask(batch: int, q_len: int, kv_len: int, device: torch.device) -> torch.Tensor:
    """Boolean [B, 1, q, kv] visibility of q_len queries that follow kv_len - q_len cached tokens: query i sits
    at position kv_len - q_len + i and sees keys j <= that position (the alignment of HF's own causal mask for a
    cache, transformers/masking_utils.py causal_mask_function with q_offset = kv_len - q_len)."""
    i = torch.arange(q_len, device=device)[:, None]
    j = torch.arange(kv_len, device=device)[None, :]
    return (j <= i + (kv_len - q_len))[None, None].expand(batch, 1, q_len, kv_len)


def sdpa_fallback(
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
    meta = getattr(key, "_aicas_kv", None)
    if meta is not None and not meta.dense:
        # a paged or fp8 aicas cache: its rows as dense 16-bit K/V (fp8 dequantised), every sequence being
        # max_seq_len long; a ragged one has no single causal offset for the new queries and is refused
        if meta.min_seq_len != meta.max_seq_len:
            raise RuntimeError(
                "this aicas KV cache holds sequences of different lengths; only the decode kernel reads it "
                "(attention_mask=None, q_len=1)"
            )
        from . import ops

        key, value = ops.kv_gather(meta.cache, meta.seq_lens, meta.max_seq_len, dtype=query.dtype)
    causal = bool(is_causal if is_causal is not None else getattr(module, "is_causal", True))
    q_len, kv_len = query.shape[2], key.shape[2]
    sdpa_attention_forward = _load_sdpa_attention_forward()
    if attention_mask is None and causal and 1 < q_len < kv_len:
        # queries continuing a cached prefix: SDPA's is_causal would align them with the first keys
        attention_mask = _causal_continuation_mask(query.shape[0], q_len, kv_len, query.device)
    elif sdpa_attention_forward is not None and attention_mask is not None and attention_mask.dim() == 2:
        attention_mask = _padding_mask_4d(attention_mask, q_len, kv_len, causal)
    if sdpa_attention_forward is not None:
        return sdpa_attention_forward(
            module, query, key, value, attention_mask, dropout=dropout, scaling=scaling, is_causal=is_causal,
            **kwargs,
        )

    if hasattr(module, "num_key_value_groups"):
        key = repeat_kv(key, module.num_key_value_groups)
        value = repeat_kv(value, module.num_key_value_groups)
    is_causal = is_causal if is_causal is not None else getattr(module, "is_causal", True)
    is_causal = query.shape[2] > 1 and attention_mask is None and is_causal
    attn_output = F.scaled_dot_product_attention(
        query, key, value, attn_mask=attention_mask, dropout_p=dropout, scale=scaling, is_causal=is_causal
    )
    return attn_output.transpose(1, 2).contiguous(), None
