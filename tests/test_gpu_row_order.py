"""Ragged batches with many (batch row, kv head) pairs are dispatched in folded length order.

When a launch has more pairs than 3/4 of the compute units, device lengths and at most 256 batch rows, every
workgroup reads all the rows' lengths, ranks them (decreasing length, ties in row order) and takes the row that
its grid slot folds to (slot z < ceil(B/2): rank z; slot ceil(B/2) + i: rank B - 1 - i); the fused append's length
bump then waits for every workgroup of the launch, not only those of the row. The order may change the timing only: the fused launch must still equal the append followed
by the plain decode bit for bit, cover every row (ties and empty sequences included), bump every length by one,
leave the workspace counters at zero and match the oracle. 257 rows take the natural order.
"""

import math

import pytest
import torch

from aicas_amd import ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

H, G, D = 8, 2, 128
COUNTER_BYTES = 512 << 10  # the workspace's counters, ahead of the split partials


def _caches(dev, gen, kind, B, cap):
    """Two identical caches (fused / two-launch copies) holding random rows."""
    if kind == "bf16":
        k = torch.randn((B, H, cap, D), generator=gen).to(torch.bfloat16)
        v = torch.randn((B, H, cap, D), generator=gen).to(torch.bfloat16)
        return [ops.KVCacheView(k.clone().to(dev), v.clone().to(dev)) for _ in range(2)]
    page = 16
    per_seq = math.ceil(cap / page)
    nblocks = B * per_seq + 3
    bt = torch.randperm(nblocks, generator=gen)[: B * per_seq].to(torch.int32).view(B, per_seq)
    ck, sk = ref.fp8_quantize_rows(torch.randn((nblocks, H, page, D), generator=gen).to(torch.bfloat16))
    cv, sv = ref.fp8_quantize_rows(torch.randn((nblocks, H, page, D), generator=gen).to(torch.bfloat16))
    return [ops.KVCacheView(ck.clone().to(dev), cv.clone().to(dev), sk.clone().to(dev), sv.clone().to(dev),
                            bt.to(dev)) for _ in range(2)]


@pytest.mark.parametrize("B, kind", [(40, "bf16"), (40, "fp8_paged"), (256, "bf16"), (257, "bf16")])
def test_ordered_rows_fused_equals_two_launches_and_oracle(dev, status, B, kind):
    gen = torch.Generator().manual_seed(900 + B + (1 if kind != "bf16" else 0))
    cap = 640
    lens = torch.randint(0, 600, (B,), generator=gen).tolist()
    lens[0] = 0
    for i in range(3, B, 7):  # ties: equal lengths rank in row order
        lens[i] = lens[1]
    fused, twol = _caches(dev, gen, kind, B, cap)
    q = torch.randn((B, H * G, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    kn = torch.randn((B, H, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    vn = torch.randn((B, H, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    pos_f = torch.tensor(lens, dtype=torch.int32, device=dev)
    pos_t = pos_f.clone()
    scale = D ** -0.5
    ws = torch.zeros(ops.decode_plan(fused.k.dtype, B, H * G, H, D, cap, 16 if fused.paged else 0).workspace_bytes,
                     dtype=torch.uint8, device=dev)
    out_f = ops.decode_attention_append(q, fused, kn, vn, pos_f, sm_scale=scale, max_seq_len=cap,
                                        seq_lens_out=pos_f, workspace=ws, status=status)
    ops.kv_append(twol, kn, vn, pos_t, pos_t)
    out_t = ops.decode_attention(q, twol, sm_scale=scale, seq_lens=pos_t, max_seq_len=cap, workspace=ws)
    torch.cuda.synchronize()
    new_lens = [L + 1 for L in lens]
    assert pos_f.cpu().tolist() == new_lens
    assert pos_t.cpu().tolist() == new_lens
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
    assert int(status.item()) == 0
    assert torch.equal(fused.k.cpu().view(torch.uint8), twol.k.cpu().view(torch.uint8))
    assert torch.equal(fused.v.cpu().view(torch.uint8), twol.v.cpu().view(torch.uint8))
    assert torch.equal(out_f.cpu().view(torch.int16), out_t.cpu().view(torch.int16))

    if fused.paged:
        deq_k = ref.fp8_dequantize_rows(fused.k.cpu(), fused.k_scale.cpu())
        deq_v = ref.fp8_dequantize_rows(fused.v.cpu(), fused.v_scale.cpu())
        ks = ref.paged_gather(deq_k, fused.block_table.cpu(), new_lens)
        vs = ref.paged_gather(deq_v, fused.block_table.cpu(), new_lens)
        qq = q.cpu().float()
    else:
        ks = [fused.k[b, :, :L].cpu() for b, L in enumerate(new_lens)]
        vs = [fused.v[b, :, :L].cpu() for b, L in enumerate(new_lens)]
        qq = q.cpu()
    expect = ref.ragged_decode(qq, ks, vs, scale, G).float()
    atol = 6e-2 if fused.paged else 2e-2
    torch.testing.assert_close(out_f.float().cpu(), expect, atol=atol, rtol=1e-2)


def test_ordered_rows_replayed_graph_bumps_every_step(dev, status):
    """A captured fused step of a ragged batch replayed several times, the lengths bumped by each replay: after
    every replay each row has grown by one and its output matches the oracle over the rows written so far."""
    gen = torch.Generator().manual_seed(977)
    B, cap, steps = 48, 700, 4
    lens = torch.randint(1, 600, (B,), generator=gen).tolist()
    view, _ = _caches(dev, gen, "bf16", B, cap)
    q = torch.randn((B, H * G, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    kn = torch.randn((B, H, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    vn = torch.randn((B, H, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    ws = torch.zeros(ops.decode_plan(torch.bfloat16, B, H * G, H, D, cap).workspace_bytes, dtype=torch.uint8,
                     device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        warm = pos.clone()  # an eager launch first (it writes the same rows the first replay writes)
        ops.decode_attention_append(q, view, kn, vn, warm, sm_scale=D ** -0.5, max_seq_len=cap, seq_lens_out=warm,
                                    out=out, workspace=ws, status=status)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=D ** -0.5, max_seq_len=cap,
                                        seq_lens_out=pos, out=out, workspace=ws, status=status)
        for step in range(steps):
            graph.replay()
            torch.cuda.synchronize()
            now = [L + step + 1 for L in lens]
            assert pos.cpu().tolist() == now, step
            ks = [view.k[b, :, :L].cpu() for b, L in enumerate(now)]
            vs = [view.v[b, :, :L].cpu() for b, L in enumerate(now)]
            expect = ref.ragged_decode(q.cpu(), ks, vs, D ** -0.5, G).float()
            torch.testing.assert_close(out.float().cpu(), expect, atol=2e-2, rtol=1e-2)
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
    assert int(status.item()) == 0


@pytest.mark.parametrize("seed", range(6))
def test_ordered_rows_random_shapes(dev, status, seed):
    """Seeded random ragged batches that take the row order (25..256 rows of 8 kv heads): bf16, fp16 or paged
    fp8, lengths with ties and empty sequences, the plain decode and the fused launch; the fused launch equals
    the append followed by the plain decode bit for bit, and both match the oracle."""
    gen = torch.Generator().manual_seed(5000 + seed)
    B = int(torch.randint(25, 257, (1,), generator=gen))
    kind = ("bf16", "fp16", "fp8_paged")[seed % 3]
    cap = 512
    lens = torch.randint(0, cap - 8, (B,), generator=gen).tolist()
    for i in range(0, B, 5):
        lens[i] = lens[(i * 7) % B]  # repeated lengths
    lens[-1] = 0
    dt = torch.float16 if kind == "fp16" else torch.bfloat16
    if kind == "fp8_paged":
        fused, twol = _caches(dev, gen, kind, B, cap)
    else:
        k = torch.randn((B, H, cap, D), generator=gen).to(dt)
        v = torch.randn((B, H, cap, D), generator=gen).to(dt)
        fused, twol = [ops.KVCacheView(k.clone().to(dev), v.clone().to(dev)) for _ in range(2)]
    q = torch.randn((B, H * G, 1, D), generator=gen).to(dt).to(dev)
    kn = torch.randn((B, H, 1, D), generator=gen).to(dt).to(dev)
    vn = torch.randn((B, H, 1, D), generator=gen).to(dt).to(dev)
    pos_f = torch.tensor(lens, dtype=torch.int32, device=dev)
    pos_t = pos_f.clone()
    scale = D ** -0.5
    out_f = ops.decode_attention_append(q, fused, kn, vn, pos_f, sm_scale=scale, max_seq_len=cap,
                                        seq_lens_out=pos_f, status=status)
    ops.kv_append(twol, kn, vn, pos_t, pos_t)
    out_t = ops.decode_attention(q, twol, sm_scale=scale, seq_lens=pos_t, max_seq_len=cap, status=status)
    torch.cuda.synchronize()
    new_lens = [L + 1 for L in lens]
    assert pos_f.cpu().tolist() == new_lens and pos_t.cpu().tolist() == new_lens
    assert int(status.item()) == 0
    assert torch.equal(out_f.cpu().view(torch.int16), out_t.cpu().view(torch.int16))
    if fused.paged:
        deq_k = ref.fp8_dequantize_rows(fused.k.cpu(), fused.k_scale.cpu())
        deq_v = ref.fp8_dequantize_rows(fused.v.cpu(), fused.v_scale.cpu())
        ks = ref.paged_gather(deq_k, fused.block_table.cpu(), new_lens)
        vs = ref.paged_gather(deq_v, fused.block_table.cpu(), new_lens)
        qq, atol = q.cpu().float(), 6e-2
    else:
        ks = [fused.k[b, :, :L].cpu() for b, L in enumerate(new_lens)]
        vs = [fused.v[b, :, :L].cpu() for b, L in enumerate(new_lens)]
        qq, atol = q.cpu(), 2e-2
    expect = ref.ragged_decode(qq, ks, vs, scale, G).float()
    torch.testing.assert_close(out_f.float().cpu(), expect, atol=atol, rtol=1e-2)


def test_ordered_rows_few_rows_many_heads(dev, status):
    """Three rows of 96 kv heads (288 pairs, so the row order applies), head_dim 64, lengths 300 / 0 / 5: the
    fused launch against the two-launch path bit for bit and against the oracle."""
    gen = torch.Generator().manual_seed(4242)
    B, Hkv, Gq, Dh, cap = 3, 96, 2, 64, 320
    lens = [300, 0, 5]
    k = torch.randn((B, Hkv, cap, Dh), generator=gen).to(torch.bfloat16)
    v = torch.randn((B, Hkv, cap, Dh), generator=gen).to(torch.bfloat16)
    fused, twol = [ops.KVCacheView(k.clone().to(dev), v.clone().to(dev)) for _ in range(2)]
    q = torch.randn((B, Hkv * Gq, 1, Dh), generator=gen).to(torch.bfloat16).to(dev)
    kn = torch.randn((B, Hkv, 1, Dh), generator=gen).to(torch.bfloat16).to(dev)
    vn = torch.randn((B, Hkv, 1, Dh), generator=gen).to(torch.bfloat16).to(dev)
    pos_f = torch.tensor(lens, dtype=torch.int32, device=dev)
    pos_t = pos_f.clone()
    scale = Dh ** -0.5
    out_f = ops.decode_attention_append(q, fused, kn, vn, pos_f, sm_scale=scale, max_seq_len=cap,
                                        seq_lens_out=pos_f, status=status)
    ops.kv_append(twol, kn, vn, pos_t, pos_t)
    out_t = ops.decode_attention(q, twol, sm_scale=scale, seq_lens=pos_t, max_seq_len=cap, status=status)
    torch.cuda.synchronize()
    new_lens = [L + 1 for L in lens]
    assert pos_f.cpu().tolist() == new_lens and pos_t.cpu().tolist() == new_lens
    assert int(status.item()) == 0
    assert torch.equal(out_f.cpu().view(torch.int16), out_t.cpu().view(torch.int16))
    ks = [fused.k[b, :, :L].cpu() for b, L in enumerate(new_lens)]
    vs = [fused.v[b, :, :L].cpu() for b, L in enumerate(new_lens)]
    expect = ref.ragged_decode(q.cpu(), ks, vs, scale, Gq).float()
    torch.testing.assert_close(out_f.float().cpu(), expect, atol=2e-2, rtol=1e-2)


def test_ordered_rows_replay_soak(dev, status):
    """A correctness soak (not aimed at any known failure) of the launch-wide reader count: a ragged fused step
    (64 rows of 8 kv heads, lengths U{1..400}) captured once and replayed 150 times, lengths bumped by every
    replay; every length has grown by exactly the number of replays, the counters are zero, and the plain decode
    over the final cache, in row order too, replayed 50 times, gives the same bits every time."""
    gen = torch.Generator().manual_seed(808)
    B, cap, n = 64, 600, 150
    lens = torch.randint(1, 400, (B,), generator=gen).tolist()
    view, _ = _caches(dev, gen, "bf16", B, cap)
    q = torch.randn((B, H * G, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    kn = torch.randn((B, H, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    vn = torch.randn((B, H, 1, D), generator=gen).to(torch.bfloat16).to(dev)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    ws = torch.zeros(ops.decode_plan(torch.bfloat16, B, H * G, H, D, cap).workspace_bytes, dtype=torch.uint8,
                     device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        warm = pos.clone()
        ops.decode_attention_append(q, view, kn, vn, warm, sm_scale=D ** -0.5, max_seq_len=cap, seq_lens_out=warm,
                                    out=out, workspace=ws, status=status)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=D ** -0.5, max_seq_len=cap,
                                        seq_lens_out=pos, out=out, workspace=ws, status=status)
        for _ in range(n):
            graph.replay()
        torch.cuda.synchronize()
        assert pos.cpu().tolist() == [L + n for L in lens]
        assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
        assert int(status.item()) == 0
        plain = torch.cuda.CUDAGraph()
        with torch.cuda.graph(plain, stream=stream):
            ops.decode_attention(q, view, sm_scale=D ** -0.5, seq_lens=pos, max_seq_len=cap, out=out, workspace=ws,
                                 status=status)
        hist = torch.empty((50,) + tuple(q.shape), dtype=q.dtype, device=dev)
        for i in range(50):
            plain.replay()
            hist[i].copy_(out)
        torch.cuda.synchronize()
    for i in range(1, 50):
        assert torch.equal(hist[i].view(torch.int16), hist[0].view(torch.int16)), f"replay {i} differs"
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
