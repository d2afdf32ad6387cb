"""q_len=1 GQA decode attention on the HIP kernel (drop-in for triton_qwen3vl/gqa_decode_attention.py).

Public surface mirrors the reference module:
  * ``can_use_gqa_decode_attention(query, key, value, *, num_key_value_groups)`` — the same gate as
    triton_qwen3vl/gqa_decode_attention.py:8-41. The Triton-availability condition becomes "the tensors are
    on a GPU"; whether the HIP library is present is not a gate condition: if it is missing, the call
    below raises instead of silently taking another path.
  * ``gqa_decode_attention(query, key, value, *, sm_scale, num_key_value_groups)`` -> ``[B, Hq, 1, D]``
    (gqa_decode_attention.py:413-430). Raises ``ValueError`` on inputs the gate rejects, with the
    reference's message (gqa_decode_attention.py:282). The backward pass (gqa_decode_attention.py:143-265,
    330-410) is training-only and not provided: a call that needs gradients raises.

``key``/``value`` are either plain ``[B, Hkv, L, D]`` tensors (every sequence has L tokens, as with HF's
DynamicCache) or tensors returned by :class:`aicas_amd.kv_cache.AicasKVCacheLayer.update`, which carry
an ``_aicas_kv`` descriptor: per-sequence lengths on the device, and for paged or fp8 caches the block
table and scales (HF's attention interface forwards only q, k, v and the mask, so the descriptor travels
on the key tensor itself).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops

SUPPORTED_HEAD_DIMS = ops.SUPPORTED_HEAD_DIMS


@dataclass
class AicasKV:
    """Descriptor attached to cache tensors as ``tensor._aicas_kv``."""

    cache: ops.KVCacheView
    seq_lens: torch.Tensor      # int32 [B] on device, lengths after the latest append
    max_seq_len: int            # host-side upper bound on seq_lens
    batch: int
    min_seq_len: int = 0        # host-side lower bound on seq_lens
    workspace: torch.Tensor | None = None
    dense: bool = True          # the tensor itself is a [B, Hkv, L, D] view usable by other backends


def kv_descriptor(key: torch.Tensor) -> AicasKV | None:
    return getattr(key, "_aicas_kv", None)


def can_use_gqa_decode_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    num_key_value_groups: int,
) -> bool:
    if num_key_value_groups < 1 or num_key_value_groups not in ops.SUPPORTED_GROUP_SIZES:
        return False
    if not (query.is_cuda and key.is_cuda and value.is_cuda):
        return False
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        return False
    if query.shape[2] != 1:
        return False
    if query.dtype not in (torch.float16, torch.bfloat16):
        return False
    meta = kv_descriptor(key)
    if meta is not None:
        c = meta.cache
        if query.shape[0] != meta.batch:
            return False
        if query.shape[1] != c.num_kv_heads * num_key_value_groups:
            return False
        if query.shape[-1] != c.head_dim or query.shape[-1] not in SUPPORTED_HEAD_DIMS:
            return False
        if not c.is_fp8 and c.k.dtype != query.dtype:
            return False
        return True
    if query.shape[0] != key.shape[0] or key.shape[0] != value.shape[0]:
        return False
    if key.shape[2] != value.shape[2]:
        return False
    if key.shape[1] != value.shape[1]:
        return False
    if query.shape[1] != key.shape[1] * num_key_value_groups:
        return False
    if query.shape[-1] != key.shape[-1] or key.shape[-1] != value.shape[-1]:
        return False
    if query.shape[-1] not in SUPPORTED_HEAD_DIMS:
        return False
    if key.dtype != query.dtype or value.dtype != query.dtype:
        return False
    return True


def _row_aligned(x: torch.Tensor) -> bool:
    es = x.element_size()
    return (
        x.stride(3) == 1
        and x.data_ptr() % 16 == 0
        and all((x.stride(i) * es) % 16 == 0 for i in range(3))
    )


def gqa_decode_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    sm_scale: float,
    num_key_value_groups: int,
) -> torch.Tensor:
    if torch.is_grad_enabled() and (query.requires_grad or key.requires_grad or value.requires_grad):
        raise NotImplementedError("aicas decode attention is inference-only (no backward pass)")
    if not can_use_gqa_decode_attention(query, key, value, num_key_value_groups=num_key_value_groups):
        raise ValueError("GQA decode attention only supports GPU fp16/bf16 q_len==1 inference.")

    q = query if _row_aligned(query) else query.contiguous()
    meta = kv_descriptor(key)
    if meta is not None:
        return ops.decode_attention(
            q, meta.cache, sm_scale=sm_scale, seq_lens=meta.seq_lens, max_seq_len=meta.max_seq_len,
            min_seq_len=meta.min_seq_len, workspace=meta.workspace,
        )
    k, v = key, value
    if not (_row_aligned(k) and _row_aligned(v) and k.stride() == v.stride()):
        # the reference makes q/k/v contiguous unconditionally (gqa_decode_attention.py:284-286);
        # here only layouts the kernel cannot address are copied
        k, v = k.contiguous(), v.contiguous()
    view = ops.KVCacheView(k, v)
    return ops.decode_attention(q, view, sm_scale=sm_scale, max_seq_len=k.shape[2])
