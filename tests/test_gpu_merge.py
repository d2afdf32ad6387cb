"""The split merge of the decode kernel: replay determinism, the workspace counters it leaves at zero, and q_out
written in place over q.

A sequence split over several workgroups is merged by the split that arrives last on its (batch row, kv head)
arrival counter: every split publishes its partial (m, l, acc) with agent-scope stores, waits for them to be
acknowledged and counts in; the last one reads all partials and re-arms the counter. The merge order is the
split order, so a replay of the same launch must give the same bits, and every launch must leave the counters
at zero whatever its shape.
"""

import math

import pytest
import torch

from aicas_amd import _lib, ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

COUNTER_BYTES = 512 << 10  # the workspace's counters, ahead of the split partials


def _case(dev, gen, B, Hq, Hkv, D, lens, fp8=False, page=0, dtype=torch.bfloat16):
    cap = max(lens) + 8
    kv_dtype = ops.FP8_DTYPE if fp8 else dtype
    if page:
        per_seq = math.ceil(cap / page)
        nblocks = B * per_seq
        bt = torch.randperm(nblocks, generator=gen, device=dev).to(torch.int32).view(B, per_seq)
        k = torch.zeros((nblocks, Hkv, page, D), dtype=kv_dtype, device=dev)
        scale_shape = (nblocks, Hkv, page)
    else:
        bt = None
        k = torch.zeros((B, Hkv, cap, D), dtype=kv_dtype, device=dev)
        scale_shape = (B, Hkv, cap)
    v = torch.zeros_like(k)
    ks = torch.zeros(scale_shape, dtype=torch.float32, device=dev) if fp8 else None
    vs = torch.zeros_like(ks) if fp8 else None
    view = ops.KVCacheView(k, v, ks, vs, bt)
    rows = lambda n: torch.randn((B, Hkv, n, D), generator=gen, device=dev).to(dtype)  # noqa: E731
    ops.kv_append(view, rows(max(lens)), rows(max(lens)), torch.zeros(B, dtype=torch.int32, device=dev))
    q = torch.randn((B, Hq, 1, D), generator=gen, device=dev).to(dtype)
    return view, q, rows(1), rows(1), torch.tensor(lens, dtype=torch.int32, device=dev)


def _clone(view):
    c = lambda t: None if t is None else t.clone()  # noqa: E731
    return ops.KVCacheView(c(view.k), c(view.v), c(view.k_scale), c(view.v_scale), view.block_table)


def _bits(t):
    return t.contiguous().view(torch.uint8)


def test_counters_zero_across_shapes(dev):
    """One workspace, launches of different shapes and split counts in turn (the fused append with its length bump,
    and the plain decode): the counters are zero after each, and each output matches the oracle."""
    gen = torch.Generator(device=dev).manual_seed(5)
    ws = torch.zeros(8 << 20, dtype=torch.uint8, device=dev)
    shapes = [(8, [2048] * 8, 0), (1, [32768], 0), (4, [100, 5000, 40, 3000], 64), (2, [9000, 17], 0)]
    for i, (B, lens, tps) in enumerate(shapes * 2):
        view, q, kn, vn, pos = _case(dev, gen, B, 16, 8, 128, lens)
        out = ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=128 ** -0.5, max_seq_len=max(lens) + 1,
                                          seq_lens_out=pos, tokens_per_split=tps, workspace=ws)
        torch.cuda.synchronize()
        assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0, (i, B, lens)
        assert pos.cpu().tolist() == [L + 1 for L in lens]
        plain = ops.decode_attention(q, view, sm_scale=128 ** -0.5, seq_lens=pos, max_seq_len=max(lens) + 1,
                                     tokens_per_split=tps, workspace=ws)
        torch.cuda.synchronize()
        assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0, (i, B, lens)
        assert torch.equal(_bits(plain), _bits(out))  # fused append + attend == append, then attend
        b = max(range(B), key=lambda j: lens[j])
        L = lens[b] + 1
        expect = ref.decode_fp64(q[b : b + 1].cpu(), view.k[b, :, :L].cpu()[None], view.v[b, :, :L].cpu()[None],
                                 128 ** -0.5, 2)
        assert (out[b : b + 1].double().cpu() - expect).abs().max().item() <= 2e-2


def test_replay_soak_long_sequence(dev):
    """A correctness soak (not aimed at any known failure): the fused step of one 32768-token sequence (28
    splits per pair) captured once and replayed back to back, the lengths held, so every replay computes the
    same thing; each replay's output must equal the first's bit for bit (stops at the first mismatch)."""
    gen = torch.Generator(device=dev).manual_seed(11)
    view, q, kn, vn, pos = _case(dev, gen, 1, 16, 8, 128, [32768])
    out = torch.empty_like(q)
    ws = torch.zeros(ops.decode_plan(torch.bfloat16, 1, 16, 8, 128, 32769).workspace_bytes, dtype=torch.uint8,
                     device=dev)
    n = 500
    hist = torch.empty((n,) + tuple(q.shape), dtype=q.dtype, device=dev)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=128 ** -0.5, max_seq_len=32769, out=out,
                                    workspace=ws)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=128 ** -0.5, max_seq_len=32769,
                                        out=out, workspace=ws)
        for i in range(n):
            graph.replay()
            hist[i].copy_(out)
        torch.cuda.synchronize()
    ref_bits = _bits(hist[0])
    for i in range(1, n):
        assert torch.equal(_bits(hist[i]), ref_bits), f"replay {i} differs from replay 0"
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
    assert pos.cpu().tolist() == [32768]


def test_q_out_in_place_over_q(dev):
    """With the q/k prologue, q_out may be q itself: the prepared q replaces the projection only once every
    workgroup of its pair has read it, so the output is that of a separate q_out."""
    gen = torch.Generator(device=dev).manual_seed(13)
    B, Hq, Hkv, D, lens = 4, 16, 8, 128, [3000, 2048, 77, 5000]
    view, q, kn, vn, pos = _case(dev, gen, B, Hq, Hkv, D, lens)
    w = lambda: (1 + 0.1 * torch.randn(D, generator=gen, device=dev)).to(torch.bfloat16)  # noqa: E731
    qn, knw = w(), w()
    ang = torch.rand((B, D // 2), generator=gen, device=dev) * 6.0
    ang = torch.cat([ang, ang], -1)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    results = []
    for in_place in (False, True):
        vw, p, qq = _clone(view), pos.clone(), q.clone()
        q_out = qq if in_place else torch.empty_like(qq)
        pro = ops.QKPrologue(q_norm_weight=qn, k_norm_weight=knw, eps=1e-6, cos=cos, sin=sin, q_out=q_out)
        out = ops.decode_attention_append(qq, vw, kn, vn, p, sm_scale=D ** -0.5, max_seq_len=max(lens) + 1,
                                          seq_lens_out=p, qk=pro)
        torch.cuda.synchronize()
        results.append((out, q_out, vw))
    assert torch.equal(_bits(results[0][0]), _bits(results[1][0]))
    assert torch.equal(_bits(results[0][1]), _bits(results[1][1]))
    assert torch.equal(_bits(results[0][2].k), _bits(results[1][2].k))


def test_q_out_partial_overlap_rejected(dev):
    """q_out may be q itself, but any other overlap with q or with k_new is refused before launch."""
    gen = torch.Generator(device=dev).manual_seed(14)
    view, q, kn, vn, pos = _case(dev, gen, 2, 16, 8, 128, [100, 200])
    buf = torch.zeros((2 * 16 * 128 + 8,), dtype=torch.bfloat16, device=dev)
    qq = buf[:-8].view(2, 16, 1, 128)
    qq.copy_(q)
    shifted = buf[8:].view(2, 16, 1, 128)  # q moved by 8 elements: overlaps q without being q
    kbuf = torch.zeros((2 * 16 * 128,), dtype=torch.bfloat16, device=dev)
    kn2 = kbuf[: 2 * 8 * 128].view(2, 8, 1, 128)
    kn2.copy_(kn)
    for qin, kin, q_out in ((qq, kn, shifted), (q, kn2, kbuf.view(2, 16, 1, 128))):
        with pytest.raises(_lib.AicasError) as ei:
            ops.decode_attention_append(qin, view, kin, vn, pos, sm_scale=0.1, max_seq_len=201,
                                        qk=ops.QKPrologue(q_out=q_out))
        assert "overlap" in str(ei.value)
    torch.cuda.synchronize()
    assert pos.cpu().tolist() == [100, 200]


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_merge_paths_every_group_shape(dev, D, G):
    """Split counts from a few to a few hundred for every (G, D): up to 8 splits the last arriver reads one
    (head, d) cell per thread and round (two rounds when a thread holds four cells, G * D = 1024); above 8 it
    reads 16-byte pieces of the partials, 256 * 4 / (G * D) threads per quad of cells, combined through LDS.
    Both match the float64 oracle, and different split counts only reorder fp32 sums."""
    gen = torch.Generator().manual_seed(300 + 10 * G + D)
    B, Hkv, L = 2, 2, 3200
    scale = D ** -0.5
    q = torch.randn((B, Hkv * G, 1, D), generator=gen).to(torch.bfloat16)
    k = torch.randn((B, Hkv, L, D), generator=gen).to(torch.bfloat16)
    v = torch.randn((B, Hkv, L, D), generator=gen).to(torch.bfloat16)
    expect = ref.decode_fp64(q, k, v, scale, G)
    view = ops.KVCacheView(k.to(dev), v.to(dev))
    rows = 2048 // D  # rows one workgroup load covers: split sizes are multiples of it
    outs = {}
    for want in (rows, 128, 192, 384, 448, 640, 1600):
        tps = -(-want // rows) * rows
        plan = ops.decode_plan(torch.bfloat16, B, Hkv * G, Hkv, D, L, 0, tps)
        out = ops.decode_attention(q.to(dev), view, sm_scale=scale, tokens_per_split=tps).float().cpu()
        err = (out - expect).abs().max().item()
        assert err < 2e-2, (plan.num_splits, err)
        outs[plan.num_splits] = out
    counts = sorted(outs)
    assert counts[0] <= 8 < counts[-1], counts
    if G * D == 1024:
        assert any(4 < n <= 8 for n in counts), counts
    base = outs[counts[0]]
    for n in counts[1:]:
        assert (outs[n] - base).abs().max() <= 2.0 ** -7 * base.abs().max(), n


@pytest.mark.parametrize("name, B, lens, tps, fp8, page", [
    ("uniform 4 splits", 8, [2048] * 8, 0, False, 0),
    ("ragged split sizes", 4, [100, 5000, 40, 3000], 64, False, 0),
    ("paged fp8 ragged", 6, [300, 4100, 2000, 17, 6000, 900], 0, True, 16),
])
def test_replay_soak_few_splits(dev, name, B, lens, tps, fp8, page):
    """A correctness soak (not aimed at any known failure) of merges of few splits (the headline's shape among
    them): the plain decode captured once and replayed back to back; every replay's output equals the first's
    bit for bit (stops at the first mismatch), the counters end at zero, and the output matches the oracle."""
    gen = torch.Generator(device=dev).manual_seed(21 + len(lens))
    view, q, kn, vn, pos = _case(dev, gen, B, 16, 8, 128, lens, fp8=fp8, page=page)
    ws = torch.zeros(8 << 20, dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    stream = torch.cuda.Stream(device=dev)
    n = 200
    hist = torch.empty((n,) + tuple(q.shape), dtype=q.dtype, device=dev)
    with torch.cuda.stream(stream):
        ops.decode_attention(q, view, sm_scale=128 ** -0.5, seq_lens=pos, max_seq_len=max(lens), out=out,
                             tokens_per_split=tps, workspace=ws, status=status)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.decode_attention(q, view, sm_scale=128 ** -0.5, seq_lens=pos, max_seq_len=max(lens), out=out,
                                 tokens_per_split=tps, workspace=ws, status=status)
        for i in range(n):
            graph.replay()
            hist[i].copy_(out)
        torch.cuda.synchronize()
    assert int(status.item()) == 0
    first = _bits(hist[0])
    for i in range(1, n):
        assert torch.equal(_bits(hist[i]), first), f"replay {i} differs from replay 0"
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
    b = max(range(B), key=lambda j: lens[j])
    L = lens[b]
    if page:
        bt = view.block_table[b : b + 1].cpu()
        k = ref.paged_gather(view.k.cpu(), bt, [L])[0].float()
        v = ref.paged_gather(view.v.cpu(), bt, [L])[0].float()
        k = k * ref.paged_gather(view.k_scale.cpu()[..., None], bt, [L])[0]
        v = v * ref.paged_gather(view.v_scale.cpu()[..., None], bt, [L])[0]
    else:
        k, v = view.k[b, :, :L].cpu(), view.v[b, :, :L].cpu()
    expect = ref.decode_fp64(q[b : b + 1].cpu(), k[None], v[None], 128 ** -0.5, 2)
    assert (hist[0][b : b + 1].double().cpu() - expect).abs().max().item() <= (6e-2 if fp8 else 2e-2)
