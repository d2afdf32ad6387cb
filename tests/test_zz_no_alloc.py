"""aicas_decode_attention_append_noalloc (the fused append + attend entry point whose split partials live in the
library's static per-device scratch instead of a caller's workspace) against aicas_decode_attention_append on
the same inputs: identical outputs, cache rows and lengths, bit for bit, on consecutive calls whose second is
smaller than the first (the scratch keeps the first call's contents), and a launch too large for the scratch
is refused before anything is enqueued.
"""

import pytest
import torch

from aicas_amd import _lib, ops
from aicas_amd._lib import AicasError

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128
SCALE = D ** -0.5


def _case(dev, gen, B, lens, fp8=False, page=0):
    """A cache holding `lens[b]` random rows per sequence (bf16, or paged fp8 through the append kernel), the
    step's q and new rows, and the lengths."""
    cap = max(lens) + 16
    kv_dtype = ops.FP8_DTYPE if fp8 else torch.bfloat16
    if page:
        per_seq = (cap + page - 1) // page
        nblocks = B * per_seq
        perm = torch.randperm(nblocks, generator=gen, device=dev).to(torch.int32).view(B, per_seq)
        k = torch.zeros((nblocks, HKV, page, D), dtype=kv_dtype, device=dev)
        v = torch.zeros_like(k)
        ks = torch.zeros((nblocks, HKV, page), dtype=torch.float32, device=dev) if fp8 else None
        vs = torch.zeros_like(ks) if fp8 else None
        view = ops.KVCacheView(k, v, ks, vs, perm)
    else:
        k = torch.zeros((B, HKV, cap, D), dtype=kv_dtype, device=dev)
        v = torch.zeros_like(k)
        view = ops.KVCacheView(k, v)
    rows_k = torch.randn((B, HKV, max(lens), D), generator=gen, device=dev).to(torch.bfloat16)
    rows_v = torch.randn((B, HKV, max(lens), D), generator=gen, device=dev).to(torch.bfloat16)
    ops.kv_append(view, rows_k, rows_v, torch.zeros(B, dtype=torch.int32, device=dev))
    q = torch.randn((B, HQ, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn((B, HKV, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    vn = torch.randn((B, HKV, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    return view, q, kn, vn, pos


def _clone(view):
    c = lambda t: None if t is None else t.clone()  # noqa: E731
    return ops.KVCacheView(c(view.k), c(view.v), c(view.k_scale), c(view.v_scale), view.block_table)


def _bits(t):
    return t.contiguous().view(torch.uint8)


def _run_pair(dev, gen, B, lens, **kw):
    view, q, kn, vn, pos = _case(dev, gen, B, lens, **kw)
    view2, pos2 = _clone(view), pos.clone()
    bound, lo = max(lens) + 1, min(lens)
    expect = ops.decode_attention_append(q, view, kn, vn, pos, sm_scale=SCALE, max_seq_len=bound, min_seq_len=lo,
                                         seq_lens_out=pos)
    out = torch.full_like(expect, float("nan"))
    got = ops.decode_attention_append_noalloc(q, view2, kn, vn, pos2, out=out, sm_scale=SCALE, max_seq_len=bound,
                                              min_seq_len=lo, seq_lens_out=pos2)
    torch.cuda.synchronize()
    assert got is out
    assert torch.equal(_bits(out), _bits(expect))
    for a, b in ((view.k, view2.k), (view.v, view2.v), (view.k_scale, view2.k_scale), (view.v_scale, view2.v_scale)):
        if a is not None:
            assert torch.equal(_bits(a), _bits(b))
    assert pos2.cpu().tolist() == pos.cpu().tolist() == [L + 1 for L in lens]


def test_noalloc_matches_workspace_entry_two_calls(dev):
    """First call: B=8, 2048 cached tokens each (four splits per sequence); second, smaller: B=2 with 300 and
    45 cached tokens — its counters and partial slots are those the first call left behind."""
    gen = torch.Generator(device=dev).manual_seed(7)
    _run_pair(dev, gen, 8, [2048] * 8)
    _run_pair(dev, gen, 2, [300, 45])


def test_noalloc_paged_fp8_then_smaller(dev):
    """Paged fp8 (16-token pages, permuted table), ragged, then a smaller contiguous bf16 call."""
    gen = torch.Generator(device=dev).manual_seed(8)
    _run_pair(dev, gen, 16, [int(x) for x in torch.randint(256, 4096, (16,), generator=gen, device=dev)],
              fp8=True, page=16)
    _run_pair(dev, gen, 1, [700])


def test_noalloc_rejects_launch_beyond_scratch(dev):
    """A launch whose workspace exceeds the scratch is refused with ERR_WORKSPACE, and nothing runs."""
    B = 512
    pl = ops.decode_plan(torch.bfloat16, B, HQ, HKV, D, 4096)
    assert pl.workspace_bytes > ops.NOALLOC_SCRATCH_BYTES
    k = torch.zeros((B, HKV, 16, D), dtype=torch.bfloat16, device=dev)
    view = ops.KVCacheView(k, k.clone())
    q = torch.zeros((B, HQ, 1, D), dtype=torch.bfloat16, device=dev)
    kn = torch.zeros((B, HKV, 1, D), dtype=torch.bfloat16, device=dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    out = torch.full_like(q, 3.0)
    with pytest.raises(AicasError) as ei:
        ops.decode_attention_append_noalloc(q, view, kn, kn, pos, out=out, sm_scale=SCALE, max_seq_len=4096,
                                            seq_lens_out=pos)
    assert ei.value.code == _lib.ERR_WORKSPACE
    assert "scratch" in str(ei.value)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all()) and int(pos.abs().sum()) == 0
