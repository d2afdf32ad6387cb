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


def test_padding_mask_routes_to_sdpa_or_is_refused(monkeypatch):
    """A padding mask never reaches the decode kernel (it attends to every cached token of a sequence). On a cache
    whose sequences advance together — dense, or paged / fp8 read through aicas_kv_gather — the call takes the
    SDPA route with the mask, as the reference's does; on a ragged aicas cache the attention function raises
    instead of dropping the mask."""
    from aicas_amd.gqa_decode_attention import AicasKV

    monkeypatch.setattr(backends, "can_use_gqa_decode_attention", lambda *args, **kwargs: True)
    monkeypatch.setattr(backends, "gqa_decode_attention",
                        lambda *a, **k: (_ for _ in ()).throw(AssertionError("kernel must not run with a mask")))
    module = DummyAttentionModule(num_key_value_groups=2)
    q, k, v = torch.randn(2, 4, 1, 8), torch.randn(2, 2, 6, 8), torch.randn(2, 2, 6, 8)
    mask = torch.tensor([[0, 1, 1, 1, 1, 1], [1, 1, 1, 1, 1, 1]], dtype=torch.bool)
    k._aicas_kv = AicasKV(cache=None, seq_lens=None, max_seq_len=6, min_seq_len=4, batch=2, dense=False)
    with pytest.raises(ValueError, match="padding mask"):
        text_triton_attention(module, q, k, v, attention_mask=mask)
    recorded = {}

    def fake_sdpa(*args, **kwargs):
        recorded["mask"] = args[4] if len(args) > 4 else kwargs.get("attention_mask")
        return torch.zeros(2, 1, 4, 8), None

    monkeypatch.setattr(backends, "sdpa_fallback", fake_sdpa)
    for dense in (True, False):  # dense 16-bit; paged or fp8 with every sequence 6 tokens long
        recorded.clear()
        k._aicas_kv = AicasKV(cache=None, seq_lens=None, max_seq_len=6, min_seq_len=6, batch=2, dense=dense)
        text_triton_attention(module, q, k, v, attention_mask=mask)
        assert recorded["mask"] is mask


def test_continuing_prefill_mask_is_bottom_right_causal():
    """Queries that follow cached tokens (q_len > 1, no mask) see every cached key and the new ones up to their
    own position — HF's causal alignment for a cache — not SDPA's top-left is_causal."""
    from aicas_amd.fallback import _causal_continuation_mask

    m = _causal_continuation_mask(2, 3, 7, torch.device("cpu"))
    assert m.shape == (2, 1, 3, 7)
    expect = torch.tensor([[1, 1, 1, 1, 1, 0, 0], [1, 1, 1, 1, 1, 1, 0], [1, 1, 1, 1, 1, 1, 1]], dtype=torch.bool)
    assert torch.equal(m[0, 0], expect) and torch.equal(m[1, 0], expect)
    # a fresh prompt (q_len == kv_len) is the plain lower triangle
    assert torch.equal(_causal_continuation_mask(1, 4, 4, torch.device("cpu"))[0, 0],
                       torch.ones(4, 4, dtype=torch.bool).tril())


def test_continuing_prefill_through_sdpa_fallback_matches_full_attention():
    """A prompt split in two prefills (the second continuing the first through a dense cache) gives the rows a
    single prefill over the whole prompt gives, on the CPU SDPA route."""
    torch.manual_seed(3)
    module = DummyAttentionModule(num_key_value_groups=2)
    q = torch.randn(1, 4, 7, 8)
    k, v = torch.randn(1, 2, 7, 8), torch.randn(1, 2, 7, 8)
    whole, _ = backends.sdpa_fallback(module, q, k, v, None, scaling=8 ** -0.5)
    tail, _ = backends.sdpa_fallback(module, q[:, :, 4:], k, v, None, scaling=8 ** -0.5)
    torch.testing.assert_close(tail, whole[:, 4:], rtol=1e-5, atol=1e-6)


def test_cache_layer_refuses_beam_reordering():
    """Beam search would reorder HF's keys/values and leave the kernels' descriptor behind: refused."""
    from aicas_amd.kv_cache import AicasKVCacheLayer

    layer = AicasKVCacheLayer(max_cache_len=16)
    for call in (lambda: layer.reorder_cache(torch.tensor([1, 0])), lambda: layer.crop(4),
                 lambda: layer.batch_repeat_interleave(2), lambda: layer.batch_select_indices(torch.tensor([0]))):
        with pytest.raises(NotImplementedError):
            call()


def test_column_sliced_block_table_is_refused():
    """The kernels take a block-table row's width to be its stride: a column-sliced table is refused."""
    from aicas_amd import ops

    pool = torch.zeros((8, 2, 16, 64), dtype=torch.bfloat16)
    table = torch.arange(8, dtype=torch.int32).view(2, 4)
    ops.KVCacheView(pool, pool.clone(), block_table=table)
    ops.KVCacheView(pool, pool.clone(), block_table=table[1:2])
    with pytest.raises(_lib.AicasError, match="contiguous"):
        ops.KVCacheView(pool, pool.clone(), block_table=table[:, :2])


def test_left_padded_batch_matches_hf_sdpa_on_cpu():
    """A left-padded batch through the installed backend (whose mask interface hands attention functions HF's 2-D
    padding mask) gives HF's own SDPA path's hidden states, prefill and decode, on the CPU route."""
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    from aicas_amd import patch
    from aicas_amd.backends import TEXT_BACKEND_KEY

    cfg = Qwen3VLTextConfig(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=256)
    torch.manual_seed(0)
    model = Qwen3VLTextModel(cfg).eval()
    patch.install_qwen3vl_triton_attention(model)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(1, 128, (2, 12), generator=g)
    mask = torch.ones((2, 12), dtype=torch.long)
    mask[0, :5] = 0
    ids[0, :5] = 0
    steps = torch.randint(1, 128, (2, 3), generator=g)
    outs = {}
    for impl in ("sdpa", TEXT_BACKEND_KEY):
        cfg._attn_implementation = impl
        cache, m, res = DynamicCache(config=cfg), mask.clone(), []
        with torch.no_grad():
            res.append(model(input_ids=ids, attention_mask=m, past_key_values=cache).last_hidden_state[:, -1])
            for s in range(steps.shape[1]):
                m = torch.cat([m, torch.ones((2, 1), dtype=m.dtype)], 1)
                res.append(model(input_ids=steps[:, s : s + 1], attention_mask=m,
                                 past_key_values=cache).last_hidden_state[:, -1])
        outs[impl] = torch.stack(res)
    cfg._attn_implementation = "sdpa"
    torch.testing.assert_close(outs[TEXT_BACKEND_KEY], outs["sdpa"], atol=1e-5, rtol=1e-5)


def test_native_decode_entry_keeps_reference_checks():
    """decode_q1_gqa_forward (dujunbaoV1/native_cuda_ops) refuses what the reference's TORCH_CHECKs refuse,
    with RuntimeError, before anything reaches a device."""
    from aicas_amd import native_ops

    q, k = torch.zeros(1, 4, 64, dtype=torch.float16), torch.zeros(1, 2, 16, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        native_ops.decode_q1_gqa_forward(q, k, k, 8, 0.125)
    assert native_ops.is_available()
