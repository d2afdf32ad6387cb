"""Qwen3-VL text attention with the whole decode step of a layer in one HIP launch.

``install_fused_decode(model)`` replaces the forward of every ``Qwen3VLTextAttention`` module (the method the
reference's KV wrappers patch, with the same signature: ``forward(self, hidden_states, position_embeddings,
attention_mask, past_key_values=None, **kwargs) -> (attn_output, attn_weights)``, new KV
cache/evaluation_wrapper.py:365-497). On a decode step (one new token, no attention mask, weights not asked
for) whose cache is an :class:`~aicas_amd.kv_cache.AicasDecodeCache`, the patched forward runs the q/k/v
projections and then ``aicas_decode_attention_append_qk``: q_norm, k_norm and the rotary embedding
(transformers/models/qwen3_vl/modeling_qwen3_vl.py:481-486), the cache update (:487-488) and the attention
(:490-501), in one launch, before ``o_proj``. Every other call runs the module's own forward.
"""

from __future__ import annotations

import types

import torch

from . import ops
from .kv_cache import AicasDecodeCache, AicasKVCacheLayer


def _fused_forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None, **kwargs):
    layer = None
    if isinstance(past_key_values, AicasDecodeCache) and self.layer_idx < len(past_key_values.layers):
        layer = past_key_values.layers[self.layer_idx]
    decode = (
        isinstance(layer, AicasKVCacheLayer) and layer.is_initialized and hidden_states.shape[1] == 1
        and attention_mask is None and not kwargs.get("output_attentions", False) and not self.training
        and hidden_states.is_cuda
    )
    if not decode:
        return self._aicas_original_forward(hidden_states, position_embeddings, attention_mask, past_key_values,
                                            **kwargs)
    B = hidden_states.shape[0]
    D = self.head_dim
    q = self.q_proj(hidden_states).view(B, 1, -1, D).transpose(1, 2)
    k = self.k_proj(hidden_states).view(B, 1, -1, D).transpose(1, 2)
    v = self.v_proj(hidden_states).view(B, 1, -1, D).transpose(1, 2)
    cos, sin = position_embeddings
    if self.q_norm.variance_epsilon != self.k_norm.variance_epsilon:
        raise ValueError("q_norm and k_norm must share eps for the fused step")
    qk = ops.QKPrologue(q_norm_weight=self.q_norm.weight, k_norm_weight=self.k_norm.weight,
                        eps=self.q_norm.variance_epsilon, cos=cos, sin=sin)
    out = layer.fused_decode_step(q, k, v, sm_scale=self.scaling, qk=qk)
    attn_output = out.transpose(1, 2).reshape(B, 1, -1).contiguous()
    return self.o_proj(attn_output), None


def install_fused_decode(model: torch.nn.Module) -> int:
    """Patch every Qwen3VLTextAttention module of ``model`` (idempotent); returns the number patched."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextAttention

    n = 0
    for module in model.modules():
        if isinstance(module, Qwen3VLTextAttention):
            if not hasattr(module, "_aicas_original_forward"):
                module._aicas_original_forward = module.forward
                module.forward = types.MethodType(_fused_forward, module)
            n += 1
    return n


def uninstall_fused_decode(model: torch.nn.Module) -> int:
    """Undo :func:`install_fused_decode`; returns the number of modules restored."""
    n = 0
    for module in model.modules():
        if hasattr(module, "_aicas_original_forward"):
            module.forward = module._aicas_original_forward
            del module._aicas_original_forward
            n += 1
    return n
