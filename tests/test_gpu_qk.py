"""The fused decode step with the model's q/k preparation (aicas_decode_attention_append_qk) on the GPU.

Against the oracle (reference_path.prepare_qk: Qwen3VLTextRMSNorm then apply_rotary_pos_emb, pinned bit for bit
to transformers' own modules in test_oracle.py):
  * q as prepared (q_out) and the K row written to the cache: within one unit in the last place of the 16-bit
    type (the norm's fp32 sum of squares may be ordered differently from torch's), and equal on nearly every
    element; fp8 caches: the written codes dequantise to within one e4m3 step of the oracle's K row;
  * the V row: bit for bit (16-bit), code for code (fp8) — V is not prepared;
  * the attention output: within the decode bar (2e-2 / 1e-2 for 16-bit caches, 6e-2 for fp8) of the oracle's
    decode over the oracle's cache.
And end to end: a 3-layer Qwen3-VL text decoder whose attention modules run install_fused_decode, against the
same model with HF's DynamicCache and SDPA.
"""

import pytest
import torch

from aicas_amd import ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

ATOL_16, RTOL_16, ATOL_FP8 = 2e-2, 1e-2, 6e-2


def _rope_rows(B, D, positions, dtype):
    """cos/sin [B, 1, D] as the model's rotary embedding gives them at these text positions."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRotaryEmbedding

    cfg = Qwen3VLTextConfig(hidden_size=256, num_attention_heads=16, num_key_value_heads=8, head_dim=D)
    x = torch.zeros(1, dtype=dtype)
    return Qwen3VLTextRotaryEmbedding(cfg)(x, torch.tensor(positions).view(B, 1))


def _ulps(got, want):
    """|got - want| in units of the 16-bit type's spacing at want (float tensors of 16-bit values)."""
    info = torch.finfo(got.dtype)
    g, w = got.double(), want.double()
    spacing = torch.where(w == 0, torch.full_like(w, info.smallest_normal),
                          2.0 ** (torch.floor(torch.log2(w.abs())) - (info.bits - 1 - (8 if got.dtype == torch.bfloat16 else 5))))
    return ((g - w).abs() / spacing)


@pytest.mark.parametrize("parts", ["norm+rope", "norm", "rope"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kind", ["bf16", "fp16", "bf16_fp8", "bf16_paged", "fp16_fp8_paged"])
def test_fused_qk_step_matches_oracle(dev, status, kind, D, parts):
    qdt = torch.float16 if kind.startswith("fp16") else torch.bfloat16
    fp8, paged = "fp8" in kind, "paged" in kind
    B, Hkv, G, page = 3, 8, 2, 16
    Hq = Hkv * G
    lens = [5, 200, 777]
    g = torch.Generator().manual_seed(sum(map(ord, kind + parts)) + D)
    q = (3 * torch.randn((B, Hq, 1, D), generator=g)).to(qdt)
    k = (3 * torch.randn((B, Hkv, 1, D), generator=g)).to(qdt)
    v = torch.randn((B, Hkv, 1, D), generator=g).to(qdt)
    qw = (1 + 0.2 * torch.randn(D, generator=g)).to(qdt) if "norm" in parts else None
    kw = (1 + 0.2 * torch.randn(D, generator=g)).to(qdt) if "norm" in parts else None
    cos, sin = _rope_rows(B, D, lens, qdt) if "rope" in parts else (None, None)
    eps = 1e-6
    # the cache: lens[b] cached rows drawn at random, written through the append kernel
    cap = max(lens) + 1
    prefix_k = torch.randn((B, Hkv, max(lens), D), generator=g).to(qdt)
    prefix_v = torch.randn((B, Hkv, max(lens), D), generator=g).to(qdt)
    store = ops.FP8_DTYPE if fp8 else qdt
    if paged:
        per_seq = (cap + page - 1) // page
        bt = torch.randperm(B * per_seq, generator=g).to(torch.int32).view(B, per_seq).to(dev)
        shape, sshape = (B * per_seq, Hkv, page, D), (B * per_seq, Hkv, page)
    else:
        bt, shape, sshape = None, (B, Hkv, cap, D), (B, Hkv, cap)
    kc, vc = torch.zeros(shape, dtype=store, device=dev), torch.zeros(shape, dtype=store, device=dev)
    ks = torch.zeros(sshape, dtype=torch.float32, device=dev) if fp8 else None
    vs = torch.zeros(sshape, dtype=torch.float32, device=dev) if fp8 else None
    view = ops.KVCacheView(kc, vc, ks, vs, bt)
    ops.kv_append(view, prefix_k.to(dev), prefix_v.to(dev), torch.zeros(B, dtype=torch.int32, device=dev))
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    q_out = torch.zeros((B, Hq, 1, D), dtype=qdt, device=dev)
    qk = ops.QKPrologue(
        q_norm_weight=None if qw is None else qw.to(dev), k_norm_weight=None if kw is None else kw.to(dev), eps=eps,
        cos=None if cos is None else cos.to(dev), sin=None if sin is None else sin.to(dev), q_out=q_out)
    out = ops.decode_attention_append(q.to(dev), view, k.to(dev), v.to(dev), pos, sm_scale=D ** -0.5,
                                      max_seq_len=cap, seq_lens_out=pos, status=status, qk=qk)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert pos.cpu().tolist() == [L + 1 for L in lens]

    eq, ek = ref.prepare_qk(q, k, qw, kw, eps, cos, sin)
    # q as prepared
    u = _ulps(q_out.cpu(), eq)
    assert float(u.max()) <= 1.0 and float((u == 0).float().mean()) > 0.98
    # the rows written at position lens[b]
    full = [L + 1 for L in lens]
    if paged:
        gk = ref.paged_gather(kc.cpu().view(torch.uint8) if fp8 else kc.cpu(), bt.cpu(), full)
        gv = ref.paged_gather(vc.cpu().view(torch.uint8) if fp8 else vc.cpu(), bt.cpu(), full)
        gks = ref.paged_gather(ks.cpu(), bt.cpu(), full) if fp8 else None
        gvs = ref.paged_gather(vs.cpu(), bt.cpu(), full) if fp8 else None
    else:
        gk = [(kc.cpu().view(torch.uint8) if fp8 else kc.cpu())[b, :, : full[b]] for b in range(B)]
        gv = [(vc.cpu().view(torch.uint8) if fp8 else vc.cpu())[b, :, : full[b]] for b in range(B)]
        gks = [ks.cpu()[b, :, : full[b]] for b in range(B)] if fp8 else None
        gvs = [vs.cpu()[b, :, : full[b]] for b in range(B)] if fp8 else None
    table = ref.e4m3_decode_table()
    keys, values = [], []
    for b, L in enumerate(lens):
        if fp8:
            kd = table[gk[b].long()] * gks[b][..., None]
            vd = table[gv[b].long()] * gvs[b][..., None]
            want = ek[b, :, 0].float()
            step = want.abs().amax(-1, keepdim=True) / 448 * 32  # one e4m3 step at the top of the row's range
            assert bool(((kd[:, L] - want).abs() <= step + 1e-6).all())
            c, s = ref.fp8_quantize_rows(v[b, :, 0])
            assert torch.equal(gv[b][:, L], c.view(torch.uint8)) and torch.equal(gvs[b][:, L], s)
        else:
            kd, vd = gk[b].float(), gv[b].float()
            uk = _ulps(gk[b][:, L], ek[b, :, 0])
            assert float(uk.max()) <= 1.0
            assert torch.equal(gv[b][:, L].view(torch.int16), v[b, :, 0].view(torch.int16))
        keys.append(kd)
        values.append(vd)
    # attention: over the cache as the device holds it, with q as prepared, and against the full oracle step
    got = out.float().cpu()
    dev_q = q_out.cpu()
    inner = ref.ragged_decode(dev_q.float(), keys, values, D ** -0.5, G).float()
    if fp8:
        assert float((got - inner).abs().max()) < ATOL_FP8
    else:
        torch.testing.assert_close(got, inner, atol=ATOL_16, rtol=RTOL_16)
    # the whole step against the oracle's q and K row (cached rows and V as the device holds them, so that
    # only the preparation is under test here); an fp8 cache holds the oracle's K row as its e4m3 codes
    def stored_row(b):
        if not fp8:
            return ek[b, :, :1].float()
        return ref.fp8_dequantize_rows(*ref.fp8_quantize_rows(ek[b, :, 0]))[:, None]

    ok_keys = [torch.cat([keys[b][:, :L], stored_row(b)], 1) for b, L in enumerate(lens)]
    oracle = ref.ragged_decode(eq.float(), ok_keys, values, D ** -0.5, G).float()
    if fp8:
        assert float((got - oracle).abs().max()) < ATOL_FP8
    else:
        torch.testing.assert_close(got, oracle, atol=ATOL_16, rtol=RTOL_16)


@pytest.mark.parametrize("kv_dtype, page_size", [(None, None), (torch.float8_e4m3fn, 16)])
def test_hf_fused_decode_matches_dynamic_cache_sdpa(dev, kv_dtype, page_size):
    """A 3-layer Qwen3-VL text decoder: prefill, then decode steps whose every layer runs one fused launch
    (norms, rotary embedding, cache update, attention), against the same model on DynamicCache + SDPA."""
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    import aicas_amd.fused_attention as fa
    from aicas_amd import AicasDecodeCache

    cfg = Qwen3VLTextConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=4096)
    torch.manual_seed(0)
    model = Qwen3VLTextModel(cfg).to(dev, torch.bfloat16).eval()
    for m in model.modules():  # non-trivial norm weights
        if m.__class__.__name__ == "Qwen3VLTextRMSNorm":
            with torch.no_grad():
                m.weight.copy_(1 + 0.1 * torch.randn_like(m.weight))
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
        assert fa.install_fused_decode(model) == 3
        calls = {"n": 0}
        real = fa.AicasKVCacheLayer.fused_decode_step

        def counting(self, *a, **k):
            calls["n"] += 1
            return real(self, *a, **k)

        fa.AicasKVCacheLayer.fused_decode_step = counting
        try:
            cache = AicasDecodeCache(num_layers=3, max_cache_len=64, kv_dtype=kv_dtype, page_size=page_size)
            outs = [model(input_ids=prompt, past_key_values=cache, use_cache=True).last_hidden_state[:, -1]]
            for s in range(steps.shape[1]):
                outs.append(model(input_ids=steps[:, s : s + 1], past_key_values=cache,
                                  use_cache=True).last_hidden_state[:, -1])
        finally:
            fa.AicasKVCacheLayer.fused_decode_step = real
            assert fa.uninstall_fused_decode(model) == 3
    assert calls["n"] == steps.shape[1] * 3
    assert cache.get_seq_length() == 37 + steps.shape[1]
    tol = 3e-2 if kv_dtype is None else 8e-2
    for a, b in zip(outs, ref_outs):
        assert float((a.float() - b.float()).norm() / b.float().norm()) < tol


@pytest.mark.parametrize("kind", ["bf16", "fp16", "bf16_fp8"])
def test_fused_qk_early_fetch_is_bitwise_the_ordered_launch(dev, kind):
    """With a lower bound on the positions that keeps every split busy, the q/k step takes the early-fetch kernel
    variant (contiguous caches); output, prepared q, cache rows and lengths equal the ordered launch's bit for bit."""
    qdt = torch.float16 if kind.startswith("fp16") else torch.bfloat16
    fp8 = "fp8" in kind
    B, Hkv, G, D = 3, 8, 2, 128
    Hq = Hkv * G
    lens = [600, 610, 620]
    cap = max(lens) + 1
    plan = ops.decode_plan(ops.FP8_DTYPE if fp8 else qdt, B, Hq, Hkv, D, cap)
    assert -(-(min(lens) + 1) // plan.tokens_per_split) >= plan.num_splits  # early-fetch variant
    g = torch.Generator().manual_seed(5 + len(kind))
    q = (3 * torch.randn((B, Hq, 1, D), generator=g)).to(qdt).to(dev)
    k = (3 * torch.randn((B, Hkv, 1, D), generator=g)).to(qdt).to(dev)
    v = torch.randn((B, Hkv, 1, D), generator=g).to(qdt).to(dev)
    qw = (1 + 0.2 * torch.randn(D, generator=g)).to(qdt).to(dev)
    kw = (1 + 0.2 * torch.randn(D, generator=g)).to(qdt).to(dev)
    cos, sin = (t.to(dev) for t in _rope_rows(B, D, lens, qdt))
    store = ops.FP8_DTYPE if fp8 else qdt
    prefix_k = torch.randn((B, Hkv, max(lens), D), generator=g).to(qdt).to(dev)
    prefix_v = torch.randn((B, Hkv, max(lens), D), generator=g).to(qdt).to(dev)
    results = []
    for bound in (0, min(lens)):
        kc = torch.zeros((B, Hkv, cap, D), dtype=store, device=dev)
        vc = torch.zeros_like(kc)
        ks = torch.zeros((B, Hkv, cap), dtype=torch.float32, device=dev) if fp8 else None
        vs = torch.zeros_like(ks) if fp8 else None
        view = ops.KVCacheView(kc, vc, ks, vs)
        ops.kv_append(view, prefix_k, prefix_v, torch.zeros(B, dtype=torch.int32, device=dev))
        pos = torch.tensor(lens, dtype=torch.int32, device=dev)
        q_out = torch.zeros((B, Hq, 1, D), dtype=qdt, device=dev)
        qk = ops.QKPrologue(q_norm_weight=qw, k_norm_weight=kw, eps=1e-6, cos=cos, sin=sin, q_out=q_out)
        out = ops.decode_attention_append(q, view, k, v, pos, sm_scale=D ** -0.5, max_seq_len=cap,
                                          min_seq_len=bound, seq_lens_out=pos, qk=qk)
        torch.cuda.synchronize()
        results.append([t.cpu() for t in (out, q_out, kc.view(torch.uint8), vc.view(torch.uint8), pos)]
                       + ([ks.cpu(), vs.cpu()] if fp8 else []))
    for a, b in zip(*results):
        assert torch.equal(a, b)
