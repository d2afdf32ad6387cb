"""End to end through HF: a small randomly initialised Qwen3-VL text decoder (3 layers, 4 q / 2 kv heads,
head_dim 64) runs a prefill and decode steps with the aicas cache and backend installed, against the same
model with HF's DynamicCache and SDPA (the reference path). Also the golden c1 fixture through every entry
point, and quantize-on-write of the fixture's fp8 rows.
"""

import math
import os
import sys

import pytest
import torch
from safetensors.torch import load_file

from aicas_amd import AicasDecodeCache, ops, patch
from aicas_amd.backends import TEXT_BACKEND_KEY
from aicas_amd.gqa_decode_attention import gqa_decode_attention

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402

FIX = load_file(os.path.join(GOLDEN, "fixtures.safetensors"))


def _model(dev, layers=3):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    cfg = Qwen3VLTextConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=4096)
    torch.manual_seed(0)
    return Qwen3VLTextModel(cfg).to(dev, torch.bfloat16).eval(), cfg


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


@pytest.mark.parametrize("kv_dtype, page_size", [(None, None), (None, 16), (torch.float8_e4m3fn, None),
                                                  (torch.float8_e4m3fn, 16)])
def test_qwen3vl_text_decode_matches_dynamic_cache_sdpa(dev, kv_dtype, page_size):
    from transformers.cache_utils import DynamicCache
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    model, cfg = _model(dev)
    patch.install_qwen3vl_triton_attention(model)  # registers the backend keys (no .model tree here)
    assert TEXT_BACKEND_KEY in ALL_ATTENTION_FUNCTIONS and TEXT_BACKEND_KEY in ALL_MASK_ATTENTION_FUNCTIONS
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 512, (2, 37), generator=g).to(dev)
    steps = torch.randint(0, 512, (2, 6), generator=g).to(dev)
    with torch.no_grad():
        cfg._attn_implementation = "sdpa"
        ref_cache = DynamicCache(config=cfg)
        ref_outs = [model(input_ids=prompt, past_key_values=ref_cache, use_cache=True).last_hidden_state[:, -1]]
        for s in range(steps.shape[1]):
            ref_outs.append(model(input_ids=steps[:, s : s + 1], past_key_values=ref_cache,
                                  use_cache=True).last_hidden_state[:, -1])

        cfg._attn_implementation = TEXT_BACKEND_KEY
        cache = AicasDecodeCache(num_layers=cfg.num_hidden_layers, max_cache_len=64, kv_dtype=kv_dtype,
                                 page_size=page_size)
        calls = {"n": 0}
        import aicas_amd.backends as backends

        real = backends.gqa_decode_attention

        def counting(*a, **k):
            calls["n"] += 1
            return real(*a, **k)

        backends.gqa_decode_attention = counting
        try:
            outs = [model(input_ids=prompt, past_key_values=cache, use_cache=True).last_hidden_state[:, -1]]
            for s in range(steps.shape[1]):
                outs.append(model(input_ids=steps[:, s : s + 1], past_key_values=cache,
                                  use_cache=True).last_hidden_state[:, -1])
        finally:
            backends.gqa_decode_attention = real
            cfg._attn_implementation = "sdpa"
    assert calls["n"] == steps.shape[1] * cfg.num_hidden_layers  # every decode step took the HIP kernel
    assert cache.get_seq_length() == ref_cache.get_seq_length() == 37 + steps.shape[1]
    tol = 3e-2 if kv_dtype is None else 8e-2
    for a, b in zip(outs, ref_outs):
        assert _rel(a, b) < tol
    if kv_dtype is None and page_size is None:
        # The 16-bit cache holds bit for bit what DynamicCache concatenated wherever the inputs are the same:
        # every layer's prefill rows (both runs prefill through SDPA) and all of layer 0 (its K/V depend on the
        # token embeddings only). Later layers' decode rows inherit the attention outputs' rounding
        # differences and are compared within the tolerance.
        for i, (layer, ref_layer) in enumerate(zip(cache.layers, ref_cache.layers)):
            L = ref_layer.keys.shape[2]
            upto = L if i == 0 else 37
            for got, want in ((layer.keys, ref_layer.keys), (layer.values, ref_layer.values)):
                assert torch.equal(got[:, :, :upto].view(torch.int16), want[:, :, :upto].view(torch.int16))
                assert _rel(got[:, :, :L], want) < tol


def test_golden_c1_through_every_entry_point(dev):
    cache_k, cache_v, k_new, v_new, q = (t.to(dev) for t in make_golden.c1_inputs())
    expect = FIX["c1.out_fp64"]
    scale = 1 / math.sqrt(128)

    def check(out):
        err = (out.double().cpu() - expect).abs()
        assert float(err.max()) < 2e-2 and bool((err <= 2e-2 + 1e-2 * expect.abs()).all())

    # 1. plain gqa_decode_attention over the concatenated cache (the reference's call)
    full_k, full_v = torch.cat([cache_k, k_new], 2), torch.cat([cache_v, v_new], 2)
    check(gqa_decode_attention(q, full_k, full_v, sm_scale=scale, num_key_value_groups=2))
    # 2. HF cache layer: prefix load, append through update(), decode through the descriptor
    from aicas_amd.kv_cache import AicasKVCacheLayer

    layer = AicasKVCacheLayer(max_cache_len=1100)
    layer.load_prefix(cache_k, cache_v)
    k, v = layer.update(k_new, v_new)
    assert k.shape[2] == 1025
    assert torch.equal(k.cpu().view(torch.int16), full_k.cpu().view(torch.int16))
    check(gqa_decode_attention(q, k, v, sm_scale=scale, num_key_value_groups=2))
    # 3. fused append + attend
    kb = torch.zeros((1, 8, 1100, 128), dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    kb[:, :, :1024], vb[:, :, :1024] = cache_k, cache_v
    pos = torch.full((1,), 1024, dtype=torch.int32, device=dev)
    check(ops.decode_attention_append(q, ops.KVCacheView(kb, vb), k_new, v_new, pos, sm_scale=scale,
                                      max_seq_len=1025, min_seq_len=1024, seq_lens_out=pos))
    assert int(pos.item()) == 1025
    assert torch.equal(kb[:, :, :1025].cpu().view(torch.int16), full_k.cpu().view(torch.int16))


def test_golden_tiny_case(dev):
    out = gqa_decode_attention(FIX["tiny.q"].to(dev), FIX["tiny.k"].to(dev), FIX["tiny.v"].to(dev), sm_scale=0.25,
                               num_key_value_groups=2)
    assert float((out.double().cpu() - FIX["tiny.out_fp64"]).abs().max()) < 2e-2


def test_golden_fp8_rows_quantize_on_write(dev):
    """The fixture rows (ties, subnormals, the 448 clamp, a zero row, outliers) through aicas_kv_append into an
    fp8 cache: codes and scales bit-exact."""
    x = FIX["fp8.rows_x"]  # [6, 16]
    R = x.shape[0]
    src = x.view(R, 1, 1, 16).to(dev)
    k = torch.zeros((R, 1, 4, 16), dtype=torch.float8_e4m3fn, device=dev)
    ks = torch.zeros((R, 1, 4), dtype=torch.float32, device=dev)
    view = ops.KVCacheView(k, k.clone(), ks, ks.clone())
    pos = torch.full((R,), 2, dtype=torch.int32, device=dev)
    ops.kv_append(view, src, src, pos)
    assert torch.equal(view.k[:, 0, 2].cpu().view(torch.uint8), FIX["fp8.rows_codes"])
    assert torch.equal(view.v[:, 0, 2].cpu().view(torch.uint8), FIX["fp8.rows_codes"])
    assert torch.equal(view.k_scale[:, 0, 2].cpu(), FIX["fp8.rows_scale"])


@pytest.mark.parametrize("kv_dtype, page_size", [(None, None), (torch.float8_e4m3fn, None), (None, 16),
                                                  (torch.float8_e4m3fn, 16)])
def test_left_padded_batch(dev, kv_dtype, page_size):
    """A left-padded batch (HF hands the attention function its 2-D padding mask): the masked calls take the SDPA
    route with HF's own 4-D mask, over the cache as it is (dense bf16) or as aicas_kv_gather reads it (paged, fp8:
    dequantised), and give HF's DynamicCache + SDPA hidden states within the cache's bar."""
    from transformers.cache_utils import DynamicCache

    model, cfg = _model(dev)
    patch.install_qwen3vl_triton_attention(model)
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(1, 512, (3, 40), generator=g)
    mask = torch.ones((3, 40), dtype=torch.long)
    for b, pad in enumerate((7, 0, 19)):
        ids[b, :pad] = 0
        mask[b, :pad] = 0
    ids, mask = ids.to(dev), mask.to(dev)
    steps = torch.randint(1, 512, (3, 4), generator=g).to(dev)

    def run(impl, cache):
        cfg._attn_implementation = impl
        m, res = mask.clone(), []
        try:
            with torch.no_grad():
                res.append(model(input_ids=ids, attention_mask=m, past_key_values=cache).last_hidden_state[:, -1])
                for s in range(steps.shape[1]):
                    m = torch.cat([m, torch.ones((3, 1), dtype=m.dtype, device=dev)], 1)
                    res.append(model(input_ids=steps[:, s : s + 1], attention_mask=m,
                                     past_key_values=cache).last_hidden_state[:, -1])
        finally:
            cfg._attn_implementation = "sdpa"
        return res

    ref_outs = run("sdpa", DynamicCache(config=cfg))
    cache = AicasDecodeCache(num_layers=cfg.num_hidden_layers, max_cache_len=64, kv_dtype=kv_dtype,
                             page_size=page_size)
    outs = run(TEXT_BACKEND_KEY, cache)
    tol = 3e-2 if kv_dtype is None else 8e-2
    for a, b in zip(outs, ref_outs):
        assert _rel(a, b) < tol


@pytest.mark.parametrize("kv_dtype, page_size", [(None, None), (None, 16), (torch.float8_e4m3fn, None),
                                                  (torch.float8_e4m3fn, 16)])
def test_second_prefill_continues_the_cache(dev, kv_dtype, page_size):
    """A multi-turn continuation: prompt, decode steps, a second multi-token prefill into the same cache, more
    decode steps. The second prefill's queries attend to every cached token and, causally, to each other (over
    the cache as aicas_kv_gather reads it for paged and fp8 caches), as with HF's DynamicCache + SDPA."""
    from transformers.cache_utils import DynamicCache

    model, cfg = _model(dev)
    patch.install_qwen3vl_triton_attention(model)
    g = torch.Generator().manual_seed(21)
    turns = [torch.randint(0, 512, (2, n), generator=g).to(dev) for n in (29, 1, 1, 1, 11, 1, 1)]

    def run(impl, cache):
        cfg._attn_implementation = impl
        res = []
        try:
            with torch.no_grad():
                for ids in turns:
                    res.append(model(input_ids=ids, past_key_values=cache, use_cache=True).last_hidden_state)
        finally:
            cfg._attn_implementation = "sdpa"
        return res

    ref_outs = run("sdpa", DynamicCache(config=cfg))
    cache = AicasDecodeCache(num_layers=cfg.num_hidden_layers, max_cache_len=64, kv_dtype=kv_dtype,
                             page_size=page_size)
    outs = run(TEXT_BACKEND_KEY, cache)
    assert cache.get_seq_length() == sum(t.shape[1] for t in turns)
    tol = 3e-2 if kv_dtype is None else 8e-2
    for a, b in zip(outs, ref_outs):
        assert _rel(a, b) < tol
