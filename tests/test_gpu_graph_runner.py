"""The HIP-graph-captured decode step (AicasGraphDecodeRunner) on the GPU.

A 3-layer Qwen3-VL text decoder with the model's real vocabulary (151936, so that lm_head and the argmax run
at their real width) is prefilled by HF with DynamicCache + SDPA; the runner loads that prefix, captures its
step once and generates greedily by replays. Every replay's logits are checked against HF's own eager decode
step fed the same tokens (DynamicCache + SDPA), with host synchronisations and eager work between replays:
within 3e-2 (bf16 cache) / 8e-2 (fp8) of the logits' norm, and the replayed token equal to the eager argmax
wherever the eager top-2 margin exceeds that error.
"""

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(dev, vocab):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    cfg = Qwen3VLTextConfig(vocab_size=vocab, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=4096)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    model = Qwen3VLTextModel(cfg).to(dev, torch.bfloat16).eval()
    for m in model.modules():
        if m.__class__.__name__ == "Qwen3VLTextRMSNorm":
            with torch.no_grad():
                m.weight.copy_(1 + 0.1 * torch.randn_like(m.weight))
    lm_head = torch.nn.Linear(256, vocab, bias=False).to(dev, torch.bfloat16)
    return cfg, model, lm_head


@pytest.mark.parametrize("B, kv_dtype, page_size, block_pool", [
    (1, None, None, False), (2, None, None, False), (2, torch.float8_e4m3fn, 16, False), (2, None, 4, True),
    (100, None, None, False)])  # 200 (batch row, kv head) pairs: the launches take the row order
def test_graph_runner_matches_eager_decode(dev, B, kv_dtype, page_size, block_pool):
    from transformers.cache_utils import DynamicCache

    from aicas_amd.graph_runner import AicasGraphDecodeRunner
    import aicas_amd.fused_attention as fa

    vocab, P, steps = 151936, 29, 12
    cfg, model, lm_head = _model(dev, vocab)
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, vocab, (B, P), generator=g).to(dev)
    tol = 3e-2 if kv_dtype is None else 8e-2
    with torch.no_grad():
        prefix = DynamicCache(config=cfg)
        h = model(input_ids=prompt, past_key_values=prefix, use_cache=True).last_hidden_state
        tok = lm_head(h[:, -1:, :]).argmax(-1)  # [B, 1]
        eager_cache = copy.deepcopy(prefix)

        runner = AicasGraphDecodeRunner(model, lm_head, max_cache_len=P + steps + 3, batch_size=B,
                                        kv_dtype=kv_dtype, page_size=page_size, block_pool=block_pool)
        pos = torch.full((B, 1), P, dtype=torch.long, device=dev)
        assert runner.maybe_capture(prefix, P, tok, pos)
        assert runner.cache.get_seq_length() == P
        try:
            for s in range(steps):
                runner.prepare_step(tok, pos)
                nxt = runner.replay().clone()
                got = runner.static_logits.float().clone()
                # eager HF decode of the same token (its own attention and cache), between replays
                fa.uninstall_fused_decode(model)
                h = model(input_ids=tok, past_key_values=eager_cache, use_cache=True,
                          position_ids=pos).last_hidden_state
                want = lm_head(h[:, -1:, :]).float()
                fa.install_fused_decode(model)
                err = float((got - want).norm() / want.norm())
                assert err < tol, (s, err)
                top2 = want[:, -1].topk(2, dim=-1).values
                clear = (top2[:, 0] - top2[:, 1]) > 4 * tol * want[:, -1].abs().max(dim=-1).values
                assert torch.equal(nxt[clear], want[:, -1].argmax(-1, keepdim=True)[clear]), s
                tok = nxt
                pos = pos + 1
        finally:
            runner.release()
            fa.uninstall_fused_decode(model)
    assert runner.cache.get_seq_length() == P + steps
    lens = runner.cache.layers[0].seq_lens.cpu().tolist()
    assert lens == [P + steps] * B
    if block_pool:  # pages were handed out inside the captured steps, one block per page reached
        layer = runner.cache.layers[0]
        reached = -(-(P + steps) // page_size)
        assert layer.pool.available() == layer.pool.num_blocks - B * reached


def test_graph_runner_back_to_back_replays(dev):
    """Replays issued back to back with the token fed back on the device (no host synchronisation in between,
    as a serving loop runs them), then checked against HF's eager decode fed the same tokens."""
    from transformers.cache_utils import DynamicCache

    from aicas_amd.graph_runner import AicasGraphDecodeRunner
    import aicas_amd.fused_attention as fa

    vocab, P, steps = 151936, 17, 24
    cfg, model, lm_head = _model(dev, vocab)
    prompt = torch.randint(0, vocab, (1, P), generator=torch.Generator().manual_seed(9)).to(dev)
    with torch.no_grad():
        prefix = DynamicCache(config=cfg)
        h = model(input_ids=prompt, past_key_values=prefix, use_cache=True).last_hidden_state
        tok = lm_head(h[:, -1:, :]).argmax(-1)
        eager_cache = copy.deepcopy(prefix)
        runner = AicasGraphDecodeRunner(model, lm_head, max_cache_len=P + steps + 2)
        pos = torch.full((1, 1), P, dtype=torch.long, device=dev)
        assert runner.maybe_capture(prefix, P, tok, pos)
        fed = torch.empty((steps, 1, 1), dtype=torch.long, device=dev)
        logits = torch.empty((steps, 1, 1, vocab), dtype=torch.bfloat16, device=dev)
        fed[0].copy_(tok)
        try:
            for s in range(steps):
                runner.prepare_step(fed[s], pos + s)
                nxt = runner.replay()
                logits[s].copy_(runner.static_logits)
                if s + 1 < steps:
                    fed[s + 1].copy_(nxt)
            torch.cuda.synchronize()
        finally:
            runner.release()
            fa.uninstall_fused_decode(model)
        assert int(fed.max()) < vocab and int(fed.min()) >= 0
        for s in range(steps):
            h = model(input_ids=fed[s], past_key_values=eager_cache, use_cache=True, position_ids=pos + s).last_hidden_state
            want = lm_head(h[:, -1:, :]).float()
            err = float((logits[s].float() - want).norm() / want.norm())
            assert err < 3e-2, (s, err)


def test_graph_runner_rejects_mismatched_shapes(dev):
    from transformers.cache_utils import DynamicCache

    from aicas_amd.graph_runner import AicasGraphDecodeRunner

    cfg, model, lm_head = _model(dev, 512)
    with torch.no_grad():
        prefix = DynamicCache(config=cfg)
        model(input_ids=torch.zeros((2, 5), dtype=torch.long, device=dev), past_key_values=prefix, use_cache=True)
    runner = AicasGraphDecodeRunner(model, lm_head, max_cache_len=16, batch_size=1)
    tok = torch.zeros((2, 1), dtype=torch.long, device=dev)
    assert not runner.maybe_capture(prefix, 5, tok, tok)      # batch 2 into a batch-1 runner
    assert runner.capture_failed and not runner.is_captured
    with pytest.raises(RuntimeError):
        runner.replay()
