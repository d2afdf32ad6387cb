"""The device block pool (aicas_block_alloc / aicas_block_free) on the GPU.

Against the oracle's sequential allocator (reference_path.block_alloc / block_free, pinned in
test_block_pool_oracle.py): after every operation of random alloc / free sequences the block table, the free
count, the free stack and the status word are equal bit for bit — with batches past one 1024-sequence tile, so
that the workgroup scan's carry between tiles is exercised, and with the pool running out. Then a paged cache
layer whose pages come from the pool: prefill, fused decode steps (bf16 and fp8), attention against the oracle
over the pages the table names, and every block back in the pool after reset.
"""

import random

import pytest
import torch

from aicas_amd import ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


def _state(pool):
    return pool.free_blocks.cpu().tolist(), int(pool.free_count.item())


@pytest.mark.parametrize("B, N, W, page", [(5, 40, 8, 4), (1500, 3000, 4, 16), (2100, 2500, 3, 1)])
def test_alloc_free_match_the_oracle(dev, B, N, W, page):
    rng = random.Random(B + N)
    pool = ops.BlockPool(N, dev)
    stack, count = ref.block_pool_init(N)
    assert _state(pool) == (stack, count)
    table = torch.full((B, W), -1, dtype=torch.int32)
    dtable = table.to(dev)
    lens = [0] * B
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    for op in range(12):
        if op % 4 == 3:
            release = [int(rng.random() < 0.4) for _ in range(B)]
            count, st = ref.block_free(stack, count, table, release, lens, N)
            dlens = torch.tensor([0] * B, dtype=torch.int32, device=dev)
            pool.free(dtable, torch.tensor(release, dtype=torch.int32, device=dev), dlens, status=status)
        else:
            n = rng.randint(1, page * 2 + 1)
            pos = [min(lens[b], W * page - 1) for b in range(B)]
            count, st = ref.block_alloc(stack, count, table, pos, n, page)
            pool.alloc(dtable, torch.tensor(pos, dtype=torch.int32, device=dev), n, page, status=status)
            lens = [min(p_ + n, W * page) for p_ in pos]
        torch.cuda.synchronize()
        assert torch.equal(dtable.cpu(), table), op
        got_stack, got_count = _state(pool)
        assert got_count == count, op
        assert got_stack[:count] == stack[:count], op
        assert int(status.item()) == st, op
        status.zero_()


def test_exhaustion_leaves_pages_empty_and_reports(dev):
    pool = ops.BlockPool(3, dev)
    table = torch.full((4, 2), -1, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    pool.alloc(table, torch.zeros(4, dtype=torch.int32, device=dev), 1, 16, status=status)
    torch.cuda.synchronize()
    assert table[:, 0].cpu().tolist() == [0, 1, 2, -1]
    assert int(status.item()) == 8 and pool.available() == 0
    status.zero_()
    pool.free(table, torch.tensor([0, 1, 0, 0], dtype=torch.int32, device=dev), status=status)
    pool.alloc(table, torch.zeros(4, dtype=torch.int32, device=dev), 1, 16, status=status)
    torch.cuda.synchronize()
    # sequence 1's freed block goes back to it (sequence order); sequence 3 still finds the pool empty
    assert table[:, 0].cpu().tolist() == [0, 1, 2, -1] and int(status.item()) == 8 and pool.available() == 0


@pytest.mark.parametrize("kv_dtype", [None, torch.float8_e4m3fn])
def test_paged_layer_with_pool_decodes_like_the_oracle(dev, status, kv_dtype):
    from aicas_amd.kv_cache import AicasKVCacheLayer

    B, H, G, D, page = 3, 4, 2, 64, 16
    lens = [5, 40, 17]
    g = torch.Generator().manual_seed(11)
    layer = AicasKVCacheLayer(max_cache_len=128, kv_dtype=kv_dtype, page_size=page, block_pool=True)
    prefix_k = torch.randn((B, H, max(lens), D), generator=g).to(torch.bfloat16)
    prefix_v = torch.randn((B, H, max(lens), D), generator=g).to(torch.bfloat16)
    layer.load_prefix(prefix_k.to(dev), prefix_v.to(dev), lens)
    assert layer.pool.available() == layer.pool.num_blocks - B * ((max(lens) + page - 1) // page)
    q = torch.randn((B, H * G, 1, D), generator=g).to(torch.bfloat16).to(dev)
    steps = 20
    for s in range(steps):
        kn = torch.randn((B, H, 1, D), generator=g).to(torch.bfloat16).to(dev)
        vn = torch.randn((B, H, 1, D), generator=g).to(torch.bfloat16).to(dev)
        out = layer.fused_decode_step(q, kn, vn, sm_scale=D ** -0.5)
    torch.cuda.synchronize()
    new_lens = [L + steps for L in lens]
    assert layer.seq_lens.cpu().tolist() == new_lens
    bt = layer.block_table.cpu()
    # every page a sequence reached has a distinct block; no page past it has one
    held = [int(e) for e in bt.flatten() if e >= 0]
    assert len(held) == len(set(held))
    for b, L in enumerate(new_lens):
        reach = max((L + page - 1) // page, (max(lens) + page - 1) // page)
        assert (bt[b, :reach] >= 0).all() and (bt[b, reach:] < 0).all()
    if layer.view.is_fp8:
        kd = ref.fp8_dequantize_rows(layer.keys.cpu(), layer.k_scale.cpu())
        vd = ref.fp8_dequantize_rows(layer.values.cpu(), layer.v_scale.cpu())
    else:
        kd, vd = layer.keys.cpu().float(), layer.values.cpu().float()
    ks = ref.paged_gather(kd, bt, new_lens)
    vs = ref.paged_gather(vd, bt, new_lens)
    expect = ref.ragged_decode(q.cpu().float(), ks, vs, D ** -0.5, G).float()
    atol = 6e-2 if layer.view.is_fp8 else 2e-2
    torch.testing.assert_close(out.float().cpu(), expect, atol=atol, rtol=1e-2)
    layer.reset()
    torch.cuda.synchronize()
    assert layer.pool.available() == layer.pool.num_blocks
    assert (layer.block_table.cpu() < 0).all() and layer.seq_lens.cpu().tolist() == [0] * B
