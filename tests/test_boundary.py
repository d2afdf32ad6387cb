"""The drop-in boundary: backend installer and attention-function routing (CPU, monkeypatch-based).

Ported from the reference's routing tests (test/test_qwen3vl_triton_patch.py:22-97, 236-276) with the same
fakes (DummyRegistry, DummyAttentionModule, the SimpleNamespace model tree), plus the behaviour this build has
instead of the reference's warn-once SDPA fallback: decode-kernel errors propagate.
"""

from types import SimpleNamespace

import pytest
import torch

import aicas_amd
from aicas_amd import _lib, backends, patch
from aicas_amd.backends import text_triton_attention, vision_triton_attention
from aicas_amd.fallback import repeat_kv
from aicas_amd.gqa_decode_attention import AicasKV, can_use_gqa_decode_attention, gqa_decode_attention


class DummyRegistry(dict):
    def register(self, name, fn):
        self[name] = fn


class DummyAttentionModule(torch.nn.Module):
    def __init__(self, *, num_key_value_groups: int = 1, scaling: float = 0.125, is_causal: bool = True):
        super().__init__()
        self.num_key_value_groups = num_key_value_groups
        self.scaling = scaling
        self.is_causal = is_causal


def _build_fake_model():
    return SimpleNamespace(
        model=SimpleNamespace(
            visual=SimpleNamespace(config=SimpleNamespace(_attn_implementation="sdpa")),
            language_model=SimpleNamespace(config=SimpleNamespace(_attn_implementation="sdpa")),
        ),
        config=SimpleNamespace(
            vision_config=SimpleNamespace(_attn_implementation="sdpa"),
            text_config=SimpleNamespace(_attn_implementation="sdpa"),
        ),
    )


def test_package_exports_match_reference_surface():
    # triton_qwen3vl/__init__.py:1-16 exports for this path
    for name in ("TEXT_BACKEND_KEY", "VISION_BACKEND_KEY", "TRITON_AVAILABLE", "gqa_decode_attention",
                 "install_qwen3vl_triton_attention"):
        assert hasattr(aicas_amd, name)
    assert aicas_amd.TEXT_BACKEND_KEY == "qwen3vl_triton_flash_text"
    assert aicas_amd.VISION_BACKEND_KEY == "qwen3vl_triton_flash_vision"
    assert aicas_amd.TRITON_AVAILABLE is False


def test_install_registers_backends_and_mutates_configs(monkeypatch):
    attention_registry = DummyRegistry()
    mask_registry = DummyRegistry({"flash_attention_2": object()})
    monkeypatch.setattr(patch, "_load_attention_registries", lambda: (attention_registry, mask_registry))
    model = _build_fake_model()
    state = patch.install_qwen3vl_triton_attention(model)

    assert attention_registry[patch.VISION_BACKEND_KEY] is vision_triton_attention
    assert attention_registry[patch.TEXT_BACKEND_KEY] is text_triton_attention
    assert mask_registry[patch.VISION_BACKEND_KEY] is mask_registry["flash_attention_2"]
    assert mask_registry[patch.TEXT_BACKEND_KEY] is mask_registry["flash_attention_2"]
    assert model.model.visual.config._attn_implementation == patch.VISION_BACKEND_KEY
    assert model.model.language_model.config._attn_implementation == patch.TEXT_BACKEND_KEY
    assert model.config.vision_config._attn_implementation == patch.VISION_BACKEND_KEY
    assert model.config.text_config._attn_implementation == patch.TEXT_BACKEND_KEY
    assert state["installed"] is True
    # same state keys as triton_qwen3vl/patch.py:54-63
    assert set(state) == {
        "installed", "triton_available", "vision_backend_key", "text_backend_key", "vision_varlen_triton_enabled",
        "text_prefill_gqa_triton_enabled", "text_decode_triton_enabled", "mutated_configs",
    }
    assert all(state["mutated_configs"].values())
    assert state["text_decode_triton_enabled"] is patch.hip_decode_available()


def test_install_skips_missing_configs_and_keeps_existing_registrations(monkeypatch):
    existing = object()
    attention_registry = DummyRegistry({patch.TEXT_BACKEND_KEY: existing})
    mask_registry = DummyRegistry({"flash_attention_2": object()})
    monkeypatch.setattr(patch, "_load_attention_registries", lambda: (attention_registry, mask_registry))
    state = patch.install_qwen3vl_triton_attention(SimpleNamespace(model=None, config=None))
    assert attention_registry[patch.TEXT_BACKEND_KEY] is existing
    assert not any(state["mutated_configs"].values())


def test_install_against_real_hf_registries():
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    patch.install_qwen3vl_triton_attention(_build_fake_model())
    assert ALL_ATTENTION_FUNCTIONS[patch.TEXT_BACKEND_KEY] is text_triton_attention
    assert ALL_MASK_ATTENTION_FUNCTIONS[patch.TEXT_BACKEND_KEY] is ALL_MASK_ATTENTION_FUNCTIONS["flash_attention_2"]


def test_text_attention_uses_sdpa_fallback_on_cpu(monkeypatch):
    sentinel = torch.randn(1, 4, 2, 8)
    recorded = {}

    def fake_sdpa(*args, **kwargs):
        recorded["called"] = True
        return sentinel, None

    monkeypatch.setattr(backends, "sdpa_fallback", fake_sdpa)
    module = DummyAttentionModule(num_key_value_groups=2, is_causal=True)
    output, attn_weights = text_triton_attention(
        module, torch.randn(1, 4, 4, 8), torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8),
        attention_mask=None, dropout=0.0, scaling=None,
    )
    assert recorded["called"] is True
    assert attn_weights is None
    assert output is sentinel


def test_text_attention_uses_decode_kernel_fast_path(monkeypatch):
    sentinel = torch.arange(1 * 4 * 1 * 4, dtype=torch.float32).reshape(1, 4, 1, 4)
    recorded = {}
    monkeypatch.setattr(backends, "can_use_gqa_decode_attention", lambda *args, **kwargs: True)

    def fake_decode(query, key, value, **kwargs):
        recorded.update(kwargs)
        return sentinel

    monkeypatch.setattr(backends, "gqa_decode_attention", fake_decode)

    def unexpected_fallback(*args, **kwargs):
        raise AssertionError("decode fast path should not fall back to sdpa")

    monkeypatch.setattr(backends, "sdpa_fallback", unexpected_fallback)
    module = DummyAttentionModule(num_key_value_groups=2, scaling=0.25, is_causal=True)
    output, attn_weights = text_triton_attention(
        module, torch.randn(1, 4, 1, 4), torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4),
        attention_mask=None, dropout=0.0, scaling=None,
    )
    assert recorded["sm_scale"] == module.scaling
    assert recorded["num_key_value_groups"] == 2
    assert attn_weights is None
    assert torch.equal(output, sentinel.transpose(1, 2).contiguous())


def test_decode_kernel_errors_propagate_instead_of_falling_back(monkeypatch):
    monkeypatch.setattr(backends, "can_use_gqa_decode_attention", lambda *args, **kwargs: True)

    def failing_decode(*args, **kwargs):
        raise _lib.AicasError(_lib.ERR_LAUNCH, "boom")

    def unexpected_fallback(*args, **kwargs):
        raise AssertionError("no SDPA fallback on the decode path")

    monkeypatch.setattr(backends, "gqa_decode_attention", failing_decode)
    monkeypatch.setattr(backends, "sdpa_fallback", unexpected_fallback)
    with pytest.raises(_lib.AicasError):
        text_triton_attention(DummyAttentionModule(num_key_value_groups=2), torch.randn(1, 4, 1, 4),
                              torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4), attention_mask=None)


@pytest.mark.parametrize("case", ["prefill", "masked", "dropout", "output_attentions"])
def test_non_decode_calls_route_to_sdpa(monkeypatch, case):
    calls = []
    monkeypatch.setattr(backends, "can_use_gqa_decode_attention", lambda *a, **k: True)
    monkeypatch.setattr(backends, "gqa_decode_attention", lambda *a, **k: pytest.fail("decode kernel called"))
    monkeypatch.setattr(backends, "sdpa_fallback", lambda *a, **k: (calls.append(k) or torch.zeros(1), None))
    q = torch.randn(1, 4, 3 if case == "prefill" else 1, 8)
    kwargs = dict(attention_mask=torch.zeros(1, 1, 1, 5) if case == "masked" else None,
                  dropout=0.1 if case == "dropout" else 0.0)
    if case == "output_attentions":
        kwargs["output_attentions"] = True
    text_triton_attention(DummyAttentionModule(num_key_value_groups=2), q, torch.randn(1, 2, 5, 8),
                          torch.randn(1, 2, 5, 8), **kwargs)
    assert len(calls) == 1


def test_sdpa_route_matches_reference_numerics_on_cpu():
    """The non-decode route is HF's SDPA forward, i.e. the reference's fallback: [B, S, Hq, D] output."""
    module = DummyAttentionModule(num_key_value_groups=2, scaling=8 ** -0.5, is_causal=True)
    q, k, v = torch.randn(2, 4, 3, 8), torch.randn(2, 2, 3, 8), torch.randn(2, 2, 3, 8)
    out, w = text_triton_attention(module, q, k, v, attention_mask=None)
    expect = torch.nn.functional.scaled_dot_product_attention(
        q, repeat_kv(k, 2), repeat_kv(v, 2), is_causal=True, scale=8 ** -0.5).transpose(1, 2)
    assert w is None and out.is_contiguous()
    torch.testing.assert_close(out, expect)


def test_vision_attention_chunks_packed_sequences():
    module = DummyAttentionModule(num_key_value_groups=1, scaling=0.5, is_causal=False)
    q, k, v = torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4)
    cu = torch.tensor([0, 2, 5])
    out, _ = vision_triton_attention(module, q, k, v, cu_seq_lens_q=cu, cu_seq_lens_k=cu)
    parts = []
    for a, b in ((0, 2), (2, 5)):
        parts.append(torch.nn.functional.scaled_dot_product_attention(
            q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], scale=0.5).transpose(1, 2))
    torch.testing.assert_close(out, torch.cat(parts, dim=1))


def test_gate_mirrors_reference_conditions():
    """triton_qwen3vl/gqa_decode_attention.py:8-41 on CPU tensors and mismatched shapes: False."""
    q, k, v = torch.randn(1, 4, 1, 64), torch.randn(1, 2, 5, 64), torch.randn(1, 2, 5, 64)
    assert can_use_gqa_decode_attention(q.half(), k.half(), v.half(), num_key_value_groups=2) is False  # CPU
    with pytest.raises(ValueError):
        gqa_decode_attention(q.half(), k.half(), v.half(), sm_scale=0.125, num_key_value_groups=2)
    assert can_use_gqa_decode_attention(q, k, v, num_key_value_groups=0) is False
    assert can_use_gqa_decode_attention(q, k, v, num_key_value_groups=3) is False


def test_training_calls_are_refused():
    q = torch.randn(1, 4, 1, 64, requires_grad=True)
    with pytest.raises(NotImplementedError):
        gqa_decode_attention(q, torch.randn(1, 2, 5, 64), torch.randn(1, 2, 5, 64), sm_scale=0.1,
                             num_key_value_groups=2)


def test_sdpa_route_refuses_kernel_only_caches():
    """A paged / fp8 cache's pools cannot be read by SDPA: a masked or prefill call on them raises."""
    from aicas_amd import fallback

    k = torch.randn(4, 2, 16, 8)
    k._aicas_kv = AicasKV(cache=None, seq_lens=None, max_seq_len=5, batch=1, dense=False)
    with pytest.raises(RuntimeError):
        fallback.sdpa_fallback(DummyAttentionModule(num_key_value_groups=2), torch.randn(1, 4, 2, 8), k, k,
                               attention_mask=None)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.AicasError, match="not built"):
        _lib.lib()
    assert patch.hip_decode_available() is False
