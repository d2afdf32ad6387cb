"""Drop-in for dujunbaoV1's native decode entry (dujunbaoV1/native_cuda_ops/__init__.py:17-20), the call its
evaluation wrapper makes per layer and decode step (dujunbaoV1/evaluation_wrapper.py:518-538).

``decode_q1_gqa_forward(query, key_cache, value_cache, visible_len, softmax_scale)`` attends the q_len=1 query
``[B, Hq, D]`` to the first ``visible_len`` tokens of a fixed-capacity cache ``[B, Hkv, capacity, D]`` and
returns ``[B, Hq, D]``. It keeps the reference's argument checks and their error type (``TORCH_CHECK`` raises
``RuntimeError``, decode_q1_gqa.cpp:65-92) and runs the HIP decode kernel of ``libaicas_decode.so``, which also
takes bf16, any head_dim in {16, 32, 64, 128} and any capacity (the reference's CUDA kernel is fp16, D=128,
capacity <= 1024). Nothing falls back: if the library is missing, the call raises.
"""

from __future__ import annotations

import torch

from . import _lib, ops


def is_available() -> bool:
    """True when libaicas_decode.so loads (dujunbaoV1/native_cuda_ops/__init__.py:13-14)."""
    try:
        _lib.lib()
    except _lib.AicasError:
        return False
    return True


def _check(tensor: torch.Tensor, name: str) -> None:
    if not tensor.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not tensor.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if tensor.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError(f"{name} must be float16 or bfloat16")


def decode_q1_gqa_forward(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                          visible_len: int, softmax_scale: float) -> torch.Tensor:
    """query [B, Hq, D], key_cache / value_cache [B, Hkv, capacity, D] -> out [B, Hq, D]: softmax(q K^T *
    softmax_scale) V over the first visible_len cached tokens of every sequence (decode_q1_gqa.cpp:73-95)."""
    _check(query, "query")
    _check(key_cache, "key_cache")
    _check(value_cache, "value_cache")
    if query.dim() != 3:
        raise RuntimeError("query must have shape [batch, num_heads, head_dim]")
    if key_cache.dim() != 4:
        raise RuntimeError("key_cache must have shape [batch, num_kv_heads, seq_len, head_dim]")
    if value_cache.dim() != 4:
        raise RuntimeError("value_cache must have shape [batch, num_kv_heads, seq_len, head_dim]")
    if query.size(0) != key_cache.size(0) or query.size(0) != value_cache.size(0):
        raise RuntimeError("batch size mismatch")
    if key_cache.shape != value_cache.shape:
        raise RuntimeError("key/value cache shape mismatch")
    if query.size(2) != key_cache.size(3):
        raise RuntimeError("head_dim mismatch")
    if query.size(1) % key_cache.size(1) != 0:
        raise RuntimeError("num_heads must be divisible by num_kv_heads")
    if visible_len <= 0:
        raise RuntimeError("visible_len must be positive")
    if visible_len > key_cache.size(2):
        raise RuntimeError("visible_len exceeds cache length")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise RuntimeError("query, key_cache and value_cache must share a dtype")
    out = ops.decode_attention(query, ops.KVCacheView(key_cache, value_cache), sm_scale=float(softmax_scale),
                               max_seq_len=int(visible_len))
    return out.squeeze(2)
