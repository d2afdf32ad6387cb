"""The C ABI's largest launch on the GPU: 65536 (batch row, kv head) pairs, the most one launch may cover.

At that size every split-arrival counter of the workspace is in use, and the batch rows' length-reader counters
sit 8 slots apart instead of one cache line apart. Checked for the fused append + attend entry, with one split
per pair (the planner's choice: many pairs) and with two (every pair's arrival counter counts and re-arms).
"""

import pytest
import torch

from aicas_amd import ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

B, HKV, G, D, CAP = 8192, 8, 2, 128, 32


def _rand(shape, gen):
    return torch.randn(shape, generator=gen).to(torch.bfloat16)


@pytest.mark.parametrize("tps", [0, 16])
def test_max_pairs_fused_append_and_decode(dev, status, tps):
    gen = torch.Generator().manual_seed(65536 + tps)
    lens = torch.randint(0, CAP, (B,), generator=gen, dtype=torch.int32)  # cached tokens before the append
    lens[0], lens[-1] = 0, CAP - 1
    q = _rand((B, HKV * G, 1, D), gen)
    k = _rand((B, HKV, CAP, D), gen)
    v = _rand((B, HKV, CAP, D), gen)
    kn = _rand((B, HKV, 1, D), gen)
    vn = _rand((B, HKV, 1, D), gen)
    view = ops.KVCacheView(k.to(dev), v.to(dev))
    pos = lens.to(dev)
    out = ops.decode_attention_append(q.to(dev), view, kn.to(dev), vn.to(dev), pos, sm_scale=D ** -0.5,
                                      max_seq_len=CAP, seq_lens_out=pos, tokens_per_split=tps, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert torch.equal(pos.cpu(), lens + 1)
    # the new rows land bit for bit at each sequence's length; every other row is untouched
    ref.ragged_append(k, v, kn, vn, lens.tolist())
    assert torch.equal(view.k.cpu(), k) and torch.equal(view.v.cpu(), v)
    # attention over each grown sequence, on a sample of the batch rows (the oracle loops over sequences)
    rows = sorted(set(range(0, B, 61)) | {0, B - 1})
    grown = [int(lens[b]) + 1 for b in rows]
    expect = ref.ragged_decode(q[rows], [k[b, :, :n] for b, n in zip(rows, grown)],
                               [v[b, :, :n] for b, n in zip(rows, grown)], D ** -0.5, G)
    torch.testing.assert_close(out.float().cpu()[rows], expect.float(), atol=2e-2, rtol=1e-2)
