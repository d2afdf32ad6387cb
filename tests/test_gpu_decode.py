"""Decode attention on the GPU through the C ABI against the CPU oracle.

Tolerances: bf16/fp16 KV max-abs 2e-2 and rel 1e-2 against SDPA over repeat_kv on the same
rounded inputs; fp8 KV 6e-2 against the oracle on the dequantised cache.
"""

import math

import pytest
import torch

from aicas_amd import _lib, ops
from aicas_amd.gqa_decode_attention import gqa_decode_attention
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

ATOL_16 = 2e-2
RTOL_16 = 1e-2
ATOL_FP8 = 6e-2


def _rand(shape, gen, dtype=torch.bfloat16, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(dtype)


def _close16(out, expect):
    torch.testing.assert_close(out.float().cpu(), expect.float(), atol=ATOL_16, rtol=RTOL_16)


def test_reference_decode_case_fp16(dev):
    """The reference's own decode numerics test (test/test_qwen3vl_triton_patch.py:419-446, forward part):
    seed 1, fp16, q [1,4,1,64], k/v [1,2,65,64], scale 64^-0.5, vs SDPA(repeat_kv), atol = rtol = 1e-2."""
    torch.manual_seed(1)
    q = torch.randn(1, 4, 1, 64, device=dev, dtype=torch.float16)
    k = torch.randn(1, 2, 65, 64, device=dev, dtype=torch.float16)
    v = torch.randn(1, 2, 65, 64, device=dev, dtype=torch.float16)
    scale = 64 ** -0.5
    out = gqa_decode_attention(q, k, v, sm_scale=scale, num_key_value_groups=2)
    expect = ref.sdpa_decode(q.cpu().float(), k.cpu().float(), v.cpu().float(), scale, 2)
    torch.testing.assert_close(out.float().cpu(), expect, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_decode_shapes(dev, dtype, D, G):
    gen = torch.Generator().manual_seed(100 + D + G)
    B, Hkv, L = 2, 2, 300
    q = _rand((B, Hkv * G, 1, D), gen, dtype)
    k = _rand((B, Hkv, L, D), gen, dtype)
    v = _rand((B, Hkv, L, D), gen, dtype)
    scale = 1.0 / math.sqrt(D)
    out = gqa_decode_attention(q.to(dev), k.to(dev), v.to(dev), sm_scale=scale, num_key_value_groups=G)
    _close16(out, ref.sdpa_decode(q, k, v, scale, G))
    assert (out.float().cpu() - ref.decode_fp64(q, k, v, scale, G)).abs().max() < ATOL_16


@pytest.mark.parametrize("L", [1, 2, 7, 63, 64, 65, 129, 1000, 4099])
def test_decode_lengths(dev, L):
    gen = torch.Generator().manual_seed(L)
    B, Hkv, G, D = 3, 8, 2, 128
    q = _rand((B, Hkv * G, 1, D), gen)
    k = _rand((B, Hkv, L, D), gen)
    v = _rand((B, Hkv, L, D), gen)
    scale = D ** -0.5
    out = gqa_decode_attention(q.to(dev), k.to(dev), v.to(dev), sm_scale=scale, num_key_value_groups=G)
    _close16(out, ref.sdpa_decode(q, k, v, scale, G))
    if L == 1:
        # one key: the output is that key's V row exactly
        assert torch.equal(out.cpu(), ref.repeat_kv(v, G))


def test_split_count_invariance(dev):
    gen = torch.Generator().manual_seed(5)
    B, Hkv, G, D, L = 2, 8, 2, 128, 3000
    q, k, v = _rand((B, 16, 1, D), gen), _rand((B, Hkv, L, D), gen), _rand((B, Hkv, L, D), gen)
    view = ops.KVCacheView(k.to(dev), v.to(dev))
    outs = []
    for tps in (64, 128, 256, 448, 1024, 4096):
        outs.append(ops.decode_attention(q.to(dev), view, sm_scale=D ** -0.5, tokens_per_split=tps).float().cpu())
    expect = ref.sdpa_decode(q, k, v, D ** -0.5, G)
    for o in outs:
        _close16(o, expect)
        # different split partitions only reorder fp32 sums: at most one bf16 rounding step apart
        assert (o - outs[0]).abs().max() <= 2.0 ** -7 * outs[0].abs().max()


def test_ragged_seq_lens(dev, status):
    gen = torch.Generator().manual_seed(9)
    B, Hkv, G, D, cap = 6, 8, 2, 128, 700
    lens = [0, 1, 64, 333, 512, 700]
    q = _rand((B, Hkv * G, 1, D), gen)
    k = _rand((B, Hkv, cap, D), gen)
    v = _rand((B, Hkv, cap, D), gen)
    view = ops.KVCacheView(k.to(dev), v.to(dev))
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = ops.decode_attention(q.to(dev), view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=cap, status=status)
    torch.cuda.synchronize()
    out = out.float().cpu()
    assert out[0].abs().max() == 0  # empty sequence -> zeros
    expect = ref.ragged_decode(q[1:], [k[b, :, : lens[b]] for b in range(1, B)],
                               [v[b, :, : lens[b]] for b in range(1, B)], D ** -0.5, G)
    torch.testing.assert_close(out[1:], expect.float(), atol=ATOL_16, rtol=RTOL_16)
    assert int(status.item()) == 0


def test_len_beyond_bound_is_clamped_and_reported(dev, status):
    gen = torch.Generator().manual_seed(2)
    B, Hkv, D, cap = 2, 2, 64, 100
    q = _rand((B, 4, 1, D), gen)
    k = _rand((B, Hkv, cap, D), gen)
    v = _rand((B, Hkv, cap, D), gen)
    sl = torch.tensor([100, 5000], dtype=torch.int32, device=dev)
    out = ops.decode_attention(q.to(dev), ops.KVCacheView(k.to(dev), v.to(dev)), sm_scale=0.125,
                               seq_lens=sl, max_seq_len=cap, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.STATUS_LEN_CLAMPED
    _close16(out, ref.sdpa_decode(q, k, v, 0.125, 2))


def test_strided_views_and_outputs(dev):
    """K/V as views into a larger preallocated buffer (the HF cache's returned views) and a strided q."""
    gen = torch.Generator().manual_seed(11)
    B, Hkv, G, D, cap, L = 2, 8, 2, 128, 512, 301
    kbuf = _rand((B, Hkv, cap, D), gen).to(dev)
    vbuf = _rand((B, Hkv, cap, D), gen).to(dev)
    qbig = _rand((B, 1, Hkv * G, D), gen).to(dev)
    q = qbig.transpose(1, 2)  # [B, Hq, 1, D] non-contiguous
    out = gqa_decode_attention(q, kbuf[:, :, :L], vbuf[:, :, :L], sm_scale=D ** -0.5, num_key_value_groups=G)
    expect = ref.sdpa_decode(q.cpu(), kbuf[:, :, :L].cpu(), vbuf[:, :, :L].cpu(), D ** -0.5, G)
    _close16(out, expect)


def test_special_cases(dev):
    D, G = 128, 2
    gen = torch.Generator().manual_seed(3)
    # all keys equal -> uniform weights -> mean of V
    q = _rand((1, 16, 1, D), gen)
    k = _rand((1, 8, 1, D), gen).expand(1, 8, 777, D).contiguous()
    v = _rand((1, 8, 777, D), gen)
    out = gqa_decode_attention(q.to(dev), k.to(dev), v.to(dev), sm_scale=D ** -0.5, num_key_value_groups=G)
    mean_v = ref.repeat_kv(v.float().mean(dim=2, keepdim=True), G)
    torch.testing.assert_close(out.float().cpu(), mean_v, atol=ATOL_16, rtol=RTOL_16)
    # equal queries within a group -> identical outputs for both heads
    q2 = q.clone()
    q2[:, 1::2] = q2[:, 0::2]
    k2 = _rand((1, 8, 2000, D), gen)
    out2 = gqa_decode_attention(q2.to(dev), k2.to(dev), v[:, :, :1].expand(1, 8, 2000, D).contiguous().to(dev),
                                sm_scale=D ** -0.5, num_key_value_groups=G)
    assert torch.equal(out2[:, 0::2].cpu(), out2[:, 1::2].cpu())


def test_planted_logit_across_splits(dev):
    """One dominant key per head (logit >= 10 above the rest) far from split 0: the LSE merge must pick its
    V row. Different split sizes put it in different splits."""
    gen = torch.Generator().manual_seed(4)
    B, Hkv, G, D, L = 1, 8, 2, 128, 20000
    q = _rand((B, 16, 1, D), gen)
    k = _rand((B, Hkv, L, D), gen)
    v = _rand((B, Hkv, L, D), gen)
    from aicas_amd.workloads import plant_keys

    planted = plant_keys(k, q, gen, [L])
    view = ops.KVCacheView(k.to(dev), v.to(dev))
    expect = ref.sdpa_decode(q, k, v, D ** -0.5, G)
    for tps in (128, 1024, 8192):
        out = ops.decode_attention(q.to(dev), view, sm_scale=D ** -0.5, tokens_per_split=tps).float().cpu()
        torch.testing.assert_close(out, expect.float(), atol=ATOL_16, rtol=RTOL_16)
        for (_, j, p, _) in planted:
            # e^-10 * 20000 ~ 0.9 of mass elsewhere at worst; check the planted row dominates
            w = out[0, j * G, 0]
            assert torch.nn.functional.cosine_similarity(w, v[0, j, p].float(), dim=0) > 0.5


@pytest.mark.parametrize("src_scale", [1.0])
def test_paged_fp8_decode(dev, status, src_scale):
    gen = torch.Generator().manual_seed(55)
    B, Hkv, G, D, page = 5, 8, 2, 128, 16
    lens = [1, 16, 17, 900, 2050]
    per_seq = max((L + page - 1) // page for L in lens)
    nblocks = B * per_seq
    bt = torch.randperm(nblocks, generator=gen).to(torch.int32).view(B, per_seq)
    src_k = _rand((nblocks, Hkv, page, D), gen, scale=src_scale)
    src_v = _rand((nblocks, Hkv, page, D), gen, scale=src_scale)
    ck, sk = ref.fp8_quantize_rows(src_k)
    cv, sv = ref.fp8_quantize_rows(src_v)
    q = _rand((B, Hkv * G, 1, D), gen)
    view = ops.KVCacheView(ck.to(dev), cv.to(dev), sk.to(dev), sv.to(dev), bt.to(dev))
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = ops.decode_attention(q.to(dev), view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=max(lens),
                               status=status).float().cpu()
    torch.cuda.synchronize()
    deq_k = ref.fp8_dequantize_rows(ck, sk)
    deq_v = ref.fp8_dequantize_rows(cv, sv)
    ks = ref.paged_gather(deq_k, bt, lens)
    vs = ref.paged_gather(deq_v, bt, lens)
    expect = ref.ragged_decode(q.float(), ks, vs, D ** -0.5, G)
    assert (out - expect).abs().max() < ATOL_FP8
    # Against the unquantised source the fp8 bar holds once the rounding errors of many rows average out
    # (lengths >= 256, the range of the paged fp8 workload). A 1-token sequence returns one V row whose
    # e4m3 rounding alone is up to 2^-4 relative per element, above any fixed absolute bar.
    ks0 = ref.paged_gather(src_k.float(), bt, lens)
    vs0 = ref.paged_gather(src_v.float(), bt, lens)
    full = ref.ragged_decode(q.float(), ks0, vs0, D ** -0.5, G)
    long_rows = [b for b, L in enumerate(lens) if L >= 256]
    assert (out[long_rows] - full[long_rows]).abs().max() < ATOL_FP8
    assert int(status.item()) == 0


def test_paged_bf16_decode(dev):
    gen = torch.Generator().manual_seed(56)
    B, Hkv, G, D, page = 3, 8, 2, 128, 16
    lens = [5, 300, 1111]
    per_seq = max((L + page - 1) // page for L in lens)
    nblocks = B * per_seq + 7
    bt = torch.randperm(nblocks, generator=gen)[: B * per_seq].to(torch.int32).view(B, per_seq)
    pk = _rand((nblocks, Hkv, page, D), gen)
    pv = _rand((nblocks, Hkv, page, D), gen)
    q = _rand((B, Hkv * G, 1, D), gen)
    view = ops.KVCacheView(pk.to(dev), pv.to(dev), block_table=bt.to(dev))
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = ops.decode_attention(q.to(dev), view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=max(lens))
    expect = ref.ragged_decode(q, ref.paged_gather(pk, bt, lens), ref.paged_gather(pv, bt, lens), D ** -0.5, G)
    _close16(out, expect)


def test_invalid_block_ids_are_skipped_and_reported(dev, status):
    B, Hkv, D, page = 1, 2, 64, 16
    pk = torch.randn((4, Hkv, page, D)).to(torch.bfloat16)
    bt = torch.tensor([[0, 99, -3, 1]], dtype=torch.int32)
    view = ops.KVCacheView(pk.to(dev), pk.clone().to(dev), block_table=bt.to(dev))
    q = torch.randn((B, 4, 1, D)).to(torch.bfloat16)
    sl = torch.tensor([64], dtype=torch.int32, device=dev)
    out = ops.decode_attention(q.to(dev), view, sm_scale=0.125, seq_lens=sl, max_seq_len=64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.STATUS_BLOCK_OUT_OF_RANGE
    # only blocks 0 and 1 (tokens 0..15 and 48..63) are visible
    keys = torch.cat([pk[0], pk[1]], dim=1)[None]
    _close16(out, ref.sdpa_decode(q, keys, keys, 0.125, 2))


def test_fp8_code_decode_matches_table(dev):
    """Every e4m3 code through the kernel's hardware conversion: a cache whose row is all 1.0-scaled codes,
    a query that selects one position, so out = code value. Checks the gfx950 fp8 conversion is OCP."""
    D = 16
    table = ref.e4m3_decode_table()
    finite = torch.tensor([c for c in range(256) if not math.isnan(table[c])], dtype=torch.int32)
    B = finite.numel()
    # sequence b holds one token whose every element is code finite[b]; with one key the output is that
    # V row exactly (every e4m3 value is representable in bf16)
    rows = finite.to(torch.uint8).view(B, 1, 1, 1).expand(B, 1, 1, D).contiguous().view(ops.FP8_DTYPE)
    ones = torch.ones((B, 1, 1), dtype=torch.float32)
    view = ops.KVCacheView(rows.to(dev), rows.clone().to(dev), ones.to(dev), ones.clone().to(dev))
    q = torch.zeros((B, 1, 1, D), dtype=torch.bfloat16)
    out = ops.decode_attention(q.to(dev), view, sm_scale=1.0).float().cpu()
    expect = table[finite.long()].view(B, 1, 1, 1).expand(B, 1, 1, D)
    assert torch.equal(out, expect)


@pytest.mark.parametrize("tps", [64, 320])
@pytest.mark.parametrize("lens, bound", [([2250, 2260, 2270, 2299], 2250),  # the true lower bound
                                         ([5, 100, 2270, 2299], 2299)])      # a wrong one: idle splits fetch
def test_early_fetch_variant_is_bitwise_the_ordered_launch(dev, tps, lens, bound):
    """A lower bound that keeps every split of a contiguous cache busy selects the kernel variant that issues its
    first rows before reading the lengths. Its output (and, fused, the cache and lengths) equals the ordered
    launch's bit for bit, whether the bound is right or not: the rows' validity always comes from the lengths."""
    gen = torch.Generator().manual_seed(78)
    B, Hkv, G, D, cap = 4, 8, 2, 128, 2300
    hi = max(lens)
    plan = ops.decode_plan(torch.bfloat16, B, Hkv * G, Hkv, D, hi, 0, tps)
    assert -(-bound // plan.tokens_per_split) >= plan.num_splits  # every split counts as busy: early-fetch variant
    q = _rand((B, Hkv * G, 1, D), gen).to(dev)
    view = ops.KVCacheView(_rand((B, Hkv, cap, D), gen).to(dev), _rand((B, Hkv, cap, D), gen).to(dev))
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    base = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=hi, tokens_per_split=tps)
    early = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=hi, min_seq_len=bound,
                                 tokens_per_split=tps)
    assert torch.equal(base.cpu(), early.cpu())
    kd, vd = view.k.cpu().float(), view.v.cpu().float()
    expect = ref.ragged_decode(q.cpu().float(), [kd[b, :, :lens[b]] for b in range(B)],
                               [vd[b, :, :lens[b]] for b in range(B)], D ** -0.5, G).float()
    torch.testing.assert_close(early.float().cpu(), expect, atol=2e-2, rtol=1e-2)
    kn = _rand((B, Hkv, 1, D), gen).to(dev)
    vn = _rand((B, Hkv, 1, D), gen).to(dev)
    view_b = ops.KVCacheView(view.k.clone(), view.v.clone())
    pos_a, pos_b = sl.clone(), sl.clone()
    fa = ops.decode_attention_append(q, view, kn, vn, pos_a, sm_scale=D ** -0.5, max_seq_len=hi + 1,
                                     seq_lens_out=pos_a, tokens_per_split=tps)
    fb = ops.decode_attention_append(q, view_b, kn, vn, pos_b, sm_scale=D ** -0.5, max_seq_len=hi + 1,
                                     min_seq_len=bound, seq_lens_out=pos_b, tokens_per_split=tps)
    assert torch.equal(fa.cpu(), fb.cpu())
    assert torch.equal(view.k.cpu().view(torch.int16), view_b.k.cpu().view(torch.int16))
    assert torch.equal(view.v.cpu().view(torch.int16), view_b.v.cpu().view(torch.int16))
    assert pos_a.cpu().tolist() == pos_b.cpu().tolist() == [L + 1 for L in lens]


@pytest.mark.parametrize("tps", [0, 64, 320])
def test_min_seq_len_hint_gives_identical_results(dev, tps):
    """A caller-guaranteed lower bound on the lengths only lets the kernel fetch early; results are unchanged."""
    gen = torch.Generator().manual_seed(77)
    B, Hkv, G, D, cap = 4, 8, 2, 128, 2300
    lens = [2100, 2112, 2200, 2299]
    q = _rand((B, Hkv * G, 1, D), gen).to(dev)
    view = ops.KVCacheView(_rand((B, Hkv, cap, D), gen).to(dev), _rand((B, Hkv, cap, D), gen).to(dev))
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    base = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=cap, tokens_per_split=tps)
    hinted = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=cap, min_seq_len=min(lens),
                                  tokens_per_split=tps)
    assert torch.equal(base.cpu(), hinted.cpu())
    kn = _rand((B, Hkv, 1, D), gen).to(dev)
    pos_a = sl.clone()
    view_b = ops.KVCacheView(view.k.clone(), view.v.clone())
    pos_b = sl.clone()
    fa = ops.decode_attention_append(q, view, kn, kn, pos_a, sm_scale=D ** -0.5, max_seq_len=cap, seq_lens_out=pos_a,
                                     tokens_per_split=tps)
    fb = ops.decode_attention_append(q, view_b, kn, kn, pos_b, sm_scale=D ** -0.5, max_seq_len=cap,
                                     min_seq_len=min(lens), seq_lens_out=pos_b, tokens_per_split=tps)
    assert torch.equal(fa.cpu(), fb.cpu())
    assert torch.equal(view.k.cpu().view(torch.int16), view_b.k.cpu().view(torch.int16))


@pytest.mark.parametrize("B, lens, cap", [(8, [2048] * 8, 4096), (1, [32768], 65536), (2, [700, 1300], 8192)])
def test_loose_bound_runs_the_tight_grid(dev, B, lens, cap):
    """With few (batch row, kv head) pairs each sequence takes its split count from its own length, so a launch
    bounded by the cache capacity (a graph captured once for every later step) gives the bits of a launch bounded
    by the exact length: the same splits, merged in the same order."""
    gen = torch.Generator().manual_seed(91)
    Hkv, G, D = 8, 2, 128
    q = _rand((B, Hkv * G, 1, D), gen).to(dev)
    view = ops.KVCacheView(_rand((B, Hkv, cap, D), gen).to(dev), _rand((B, Hkv, cap, D), gen).to(dev))
    kn = _rand((B, Hkv, 1, D), gen).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    tight = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=max(lens))
    loose = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=sl, max_seq_len=cap)
    assert torch.equal(tight.cpu().view(torch.int16), loose.cpu().view(torch.int16))
    outs = []
    for bound, lo in ((max(lens) + 1, min(lens)), (cap, min(lens)), (cap, 0)):
        vw, pos = ops.KVCacheView(view.k.clone(), view.v.clone()), sl.clone()
        outs.append(ops.decode_attention_append(q, vw, kn, kn, pos, sm_scale=D ** -0.5, max_seq_len=bound,
                                                min_seq_len=lo, seq_lens_out=pos).cpu())
        assert pos.cpu().tolist() == [L + 1 for L in lens]
    assert all(torch.equal(o.view(torch.int16), outs[0].view(torch.int16)) for o in outs[1:])
    kd, vd = view.k.cpu().float(), view.v.cpu().float()
    expect = ref.ragged_decode(q.cpu().float(), [kd[b, :, :lens[b]] for b in range(B)],
                               [vd[b, :, :lens[b]] for b in range(B)], D ** -0.5, G).float()
    torch.testing.assert_close(loose.float().cpu(), expect, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("page", [1, 2])
@pytest.mark.parametrize("fused", [False, True])
def test_paged_range_mode(dev, status, fp8, page, fused):
    """Paged rows longer than the kernel's LDS block-id cache (2048 entries: here 1- and 2-token pages with
    lengths up to 5000) are streamed as one static token range per split, each split staging only its range's
    block ids. A randomly permuted block table with one invalid entry (its page is skipped and reported); plain
    decode and the fused append + attend, bf16 and fp8, against the oracle over the gathered pages."""
    gen = torch.Generator().manual_seed(400 + 10 * page + 2 * fp8 + fused)
    B, Hkv, G, D = 3, 8, 2, 128
    lens = [2100 * page + 1, 4999, 1500 * page + 777]
    assert max(-(-L // page) for L in lens) > 2048
    per_seq = [-(-(L + 1) // page) for L in lens]
    nblocks = sum(per_seq) + 7
    perm = torch.randperm(nblocks, generator=gen).to(torch.int32)
    bt = torch.full((B, max(per_seq)), -1, dtype=torch.int32)
    at = 0
    for b, n in enumerate(per_seq):
        bt[b, :n] = perm[at : at + n]
        at += n
    bad_b, bad_page = 1, 1234 // page  # one invalid entry inside sequence 1: its tokens are skipped
    bt[bad_b, bad_page] = -5
    kv_dtype = ops.FP8_DTYPE if fp8 else torch.bfloat16
    src_k = _rand((nblocks, Hkv, page, D), gen)
    src_v = _rand((nblocks, Hkv, page, D), gen)
    if fp8:
        ck, sk = ref.fp8_quantize_rows(src_k)
        cv, sv = ref.fp8_quantize_rows(src_v)
        view = ops.KVCacheView(ck.to(dev), cv.to(dev), sk.to(dev), sv.to(dev), bt.to(dev))
    else:
        view = ops.KVCacheView(src_k.to(dev), src_v.to(dev), block_table=bt.to(dev))
    q = _rand((B, Hkv * G, 1, D), gen).to(dev)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    if fused:
        kn, vn = _rand((B, Hkv, 1, D), gen).to(dev), _rand((B, Hkv, 1, D), gen).to(dev)
        out = ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=D ** -0.5, max_seq_len=max(lens) + 1,
                                          seq_lens_out=pos, status=status)
        full = [L + 1 for L in lens]
    else:
        out = ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=pos, max_seq_len=max(lens), status=status)
        full = list(lens)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.STATUS_BLOCK_OUT_OF_RANGE
    if fused:
        assert pos.cpu().tolist() == full
    # the oracle: every valid page gathered from the pool as the kernel leaves it, the invalid page's tokens
    # dropped, then per-sequence attention
    table = ref.e4m3_decode_table()
    cpu_bt = bt.clamp(min=0)
    ks, vs = [], []
    for b, L in enumerate(full):
        if fp8:
            k = ref.paged_gather(view.k.cpu().view(torch.uint8), cpu_bt[b : b + 1], [L])[0]
            v = ref.paged_gather(view.v.cpu().view(torch.uint8), cpu_bt[b : b + 1], [L])[0]
            k = table[k.long()] * ref.paged_gather(view.k_scale.cpu(), cpu_bt[b : b + 1], [L])[0][..., None]
            v = table[v.long()] * ref.paged_gather(view.v_scale.cpu(), cpu_bt[b : b + 1], [L])[0][..., None]
        else:
            k = ref.paged_gather(view.k.cpu(), cpu_bt[b : b + 1], [L])[0].float()
            v = ref.paged_gather(view.v.cpu(), cpu_bt[b : b + 1], [L])[0].float()
        keep = torch.ones(L, dtype=torch.bool)
        if b == bad_b:
            keep[bad_page * page : (bad_page + 1) * page] = False
        ks.append(k[:, keep])
        vs.append(v[:, keep])
    expect = ref.ragged_decode(q.cpu().float(), ks, vs, D ** -0.5, G, fp64=True)
    err = float((out.double().cpu() - expect).abs().max())
    assert err <= (ATOL_FP8 if fp8 else ATOL_16), err
    if fused and not fp8:
        for b, L in enumerate(lens):  # the appended rows landed in their pages
            blk, row = int(bt[b, L // page]), L % page
            assert torch.equal(view.k[blk, :, row].cpu().view(torch.int16), kn[b, :, 0].cpu().view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B, Hq, Hkv, D, cap, visible", [(1, 16, 8, 128, 1024, 700), (4, 16, 8, 128, 4096, 4096),
                                                         (2, 8, 2, 64, 65, 65), (1, 16, 4, 128, 8192, 8000)])
def test_native_decode_entry(dev, dtype, B, Hq, Hkv, D, cap, visible):
    """decode_q1_gqa_forward, the drop-in for dujunbaoV1's native op: [B, Hq, D] out of a fixed-capacity cache
    attended to its first visible_len tokens, against the oracle; and the reference's argument checks."""
    from aicas_amd import native_ops

    gen = torch.Generator().manual_seed(B * 1000 + cap)
    q = _rand((B, Hq, D), gen, dtype)
    k = _rand((B, Hkv, cap, D), gen, dtype)
    v = _rand((B, Hkv, cap, D), gen, dtype)
    out = native_ops.decode_q1_gqa_forward(q.to(dev), k.to(dev), v.to(dev), visible, D ** -0.5)
    assert out.shape == (B, Hq, D) and out.dtype == dtype
    expect = ref.sdpa_decode(q[:, :, None].float(), k[:, :, :visible].float(), v[:, :, :visible].float(),
                             D ** -0.5, Hq // Hkv)[:, :, 0]
    torch.testing.assert_close(out.float().cpu(), expect, atol=ATOL_16, rtol=1e-2)
    for bad_len in (0, cap + 1):
        with pytest.raises(RuntimeError, match="visible_len"):
            native_ops.decode_q1_gqa_forward(q.to(dev), k.to(dev), v.to(dev), bad_len, D ** -0.5)
    with pytest.raises(RuntimeError, match="contiguous"):
        native_ops.decode_q1_gqa_forward(q.to(dev), k.to(dev).transpose(2, 3), v.to(dev), visible, D ** -0.5)
