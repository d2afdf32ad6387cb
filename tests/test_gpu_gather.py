"""aicas_kv_gather: a cache in any layout the kernels read, as dense 16-bit rows.

16-bit caches come out bit for bit; fp8 caches as the oracle's dequantisation (code * scale in fp32) rounded once
to the output type, bit for bit; rows past a sequence's length, and rows behind invalid block ids, are zero.
Compared with the oracle's paged_gather / fp8_dequantize_rows on the same cache contents.
"""

import math

import pytest
import torch

from aicas_amd import _lib, ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


def _cache(dev, gen, B, Hkv, D, lens, fp8, page, dtype=torch.bfloat16, cap=None):
    """A cache holding N(0,1) rows (1% outliers of +-8) at each sequence's first lens[b] positions, written by
    the append kernel; returns the view and the source rows."""
    cap = cap or max(lens) + 5
    kv_dtype = ops.FP8_DTYPE if fp8 else dtype
    if page:
        per_seq = math.ceil(cap / page)
        bt = torch.randperm(B * per_seq + 3, generator=gen)[: B * per_seq].to(torch.int32).view(B, per_seq).to(dev)
        shape, nblocks = (B * per_seq + 3, Hkv, page, D), B * per_seq + 3
        sshape = (nblocks, Hkv, page)
    else:
        bt, shape, sshape = None, (B, Hkv, cap, D), (B, Hkv, cap)
    # stale contents past the lengths: 0.5 / -0.5 (fp8: codes 0x30 / 0xb0, +-0.5)
    if fp8:
        k = torch.full(shape, 0x30, dtype=torch.uint8, device=dev).view(kv_dtype)
        v = torch.full(shape, 0xB0, dtype=torch.uint8, device=dev).view(kv_dtype)
    else:
        k = torch.full(shape, 0.5, dtype=kv_dtype, device=dev)
        v = torch.full(shape, -0.5, dtype=kv_dtype, device=dev)
    ks = torch.ones(sshape, dtype=torch.float32, device=dev) if fp8 else None
    vs = torch.ones(sshape, dtype=torch.float32, device=dev) if fp8 else None
    view = ops.KVCacheView(k, v, ks, vs, bt)
    n = max(lens)
    src_k = torch.randn((B, Hkv, n, D), generator=gen)
    src_v = torch.randn((B, Hkv, n, D), generator=gen)
    out_mask = torch.rand((B, Hkv, n, D), generator=gen) < 0.01
    src_k[out_mask] = 8.0
    src_v = src_v.to(dtype)
    src_k = src_k.to(dtype)
    ops.kv_append(view, src_k.to(dev), src_v.to(dev), torch.zeros(B, dtype=torch.int32, device=dev))
    return view, src_k, src_v


def _expected(view, lens, out_len, out_dtype):
    """Dense [B, Hkv, out_len, D] K and V from the cache's contents through the oracle."""
    k, v = view.k.cpu(), view.v.cpu()
    ks = view.k_scale.cpu() if view.k_scale is not None else None
    vs = view.v_scale.cpu() if view.v_scale is not None else None
    bt = view.block_table.cpu() if view.block_table is not None else None
    outs = []
    for pool, scale in ((k, ks), (v, vs)):
        if bt is not None:
            seqs = ref.paged_gather(pool, bt, lens)
            sc = ref.paged_gather(scale[..., None], bt, lens) if scale is not None else None
        else:
            seqs = [pool[b, :, :L] for b, L in enumerate(lens)]
            sc = [scale[b, :, :L, None] for b, L in enumerate(lens)] if scale is not None else None
        dense = torch.zeros((len(lens), pool.shape[1], out_len, pool.shape[-1]), dtype=out_dtype)
        for b, L in enumerate(lens):
            rows = seqs[b]
            if scale is not None:
                rows = ref.fp8_dequantize_rows(rows, sc[b][..., 0]).to(out_dtype)
            dense[b, :, :L] = rows
        outs.append(dense)
    return outs


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("page", [0, 16])
@pytest.mark.parametrize("D", [64, 128])
def test_gather_matches_oracle(dev, fp8, page, D):
    gen = torch.Generator().manual_seed(40 + D + page + fp8)
    lens = [37, 1, 0, 300]
    view, src_k, src_v = _cache(dev, gen, 4, 2, D, lens, fp8, page)
    out_len = 310
    k, v = ops.kv_gather(view, torch.tensor(lens, dtype=torch.int32, device=dev), out_len)
    ek, ev = _expected(view, lens, out_len, torch.bfloat16)
    assert torch.equal(_bits(k.cpu()), _bits(ek)) and torch.equal(_bits(v.cpu()), _bits(ev))
    if not fp8:  # a 16-bit cache gives back the appended rows themselves
        for b, L in enumerate(lens):
            assert torch.equal(_bits(k[b, :, :L].cpu()), _bits(src_k[b, :, :L]))
    else:  # an fp8 one rows within the quantisation's error of them: half an e4m3 step (at most 1/16 of the
        # row's amax) plus the output's bf16 rounding
        for b, L in enumerate(lens):
            amax = src_v[b, :, :L].float().abs().amax(-1, keepdim=True)
            assert ((v[b, :, :L].cpu().float() - src_v[b, :, :L].float()).abs() <= amax * (1 / 16 + 1 / 256)).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gather_output_dtypes(dev, dtype):
    """fp16 caches gather into fp16; fp8 caches into either 16-bit type, each rounded from the fp32 product."""
    gen = torch.Generator().manual_seed(7)
    lens = [50, 129]
    view16, _, _ = _cache(dev, gen, 2, 2, 128, lens, False, 0, dtype=dtype)
    k, _ = ops.kv_gather(view16, torch.tensor(lens, dtype=torch.int32, device=dev), 130)
    assert k.dtype == dtype
    assert torch.equal(_bits(k.cpu()), _bits(_expected(view16, lens, 130, dtype)[0]))
    view8, _, _ = _cache(dev, gen, 2, 2, 128, lens, True, 16)
    k8, v8 = ops.kv_gather(view8, torch.tensor(lens, dtype=torch.int32, device=dev), 130, dtype=dtype)
    ek, ev = _expected(view8, lens, 130, dtype)
    assert torch.equal(_bits(k8.cpu()), _bits(ek)) and torch.equal(_bits(v8.cpu()), _bits(ev))
    with pytest.raises(_lib.AicasError, match="own dtype"):
        other = torch.float16 if dtype == torch.bfloat16 else torch.bfloat16
        ops.kv_gather(view16, torch.tensor(lens, dtype=torch.int32, device=dev), 130, dtype=other)


def test_gather_into_strided_outputs(dev):
    """Outputs may be views with any 8-element-multiple strides (here every other token of a larger buffer)."""
    gen = torch.Generator().manual_seed(8)
    lens = [20, 33]
    view, _, _ = _cache(dev, gen, 2, 2, 64, lens, True, 0)
    big_k = torch.full((2, 2, 80, 64), 7.0, dtype=torch.bfloat16, device=dev)
    big_v = torch.full((2, 2, 80, 64), 7.0, dtype=torch.bfloat16, device=dev)
    k, v = ops.kv_gather(view, torch.tensor(lens, dtype=torch.int32, device=dev), 40,
                         out=(big_k[:, :, ::2], big_v[:, :, ::2]))
    ek, ev = _expected(view, lens, 40, torch.bfloat16)
    assert torch.equal(_bits(big_k[:, :, ::2].cpu()), _bits(ek)) and torch.equal(_bits(big_v[:, :, ::2].cpu()), _bits(ev))
    assert (big_k[:, :, 1::2] == 7.0).all() and (big_v[:, :, 1::2] == 7.0).all()  # untouched between


def test_gather_clamps_and_reports(dev, status):
    """A length beyond the cache is clamped (rows up to the capacity come out) and an invalid block id gives zero
    rows; both are reported in the status word."""
    gen = torch.Generator().manual_seed(9)
    lens = [40, 40]
    view, _, _ = _cache(dev, gen, 2, 2, 128, lens, False, 16, cap=48)
    bt = view.block_table.clone()
    bt[1, 1] = -1
    bad = ops.KVCacheView(view.k, view.v, None, None, bt)
    status.zero_()
    k, v = ops.kv_gather(bad, torch.tensor([40, 40], dtype=torch.int32, device=dev), 40, status=status)
    ek, _ = _expected(view, lens, 40, torch.bfloat16)
    assert torch.equal(_bits(k[0].cpu()), _bits(ek[0]))
    assert (k[1, :, 16:32] == 0).all() and torch.equal(_bits(k[1, :, :16].cpu()), _bits(ek[1, :, :16]))
    assert int(status.item()) & _lib.STATUS_BLOCK_OUT_OF_RANGE
    status.zero_()
    k, _ = ops.kv_gather(view, torch.tensor([100, 40], dtype=torch.int32, device=dev), 60, status=status)
    assert int(status.item()) & _lib.STATUS_LEN_CLAMPED
    full = _expected(view, [48, 40], 60, torch.bfloat16)[0]
    assert torch.equal(_bits(k.cpu()), _bits(full))


def test_gather_poisoned_fp8_rows_come_out_nan(dev, status):
    """A row stored poisoned (a NaN input: scale NaN, zero codes) comes out NaN; its neighbours are untouched."""
    gen = torch.Generator().manual_seed(10)
    view, _, _ = _cache(dev, gen, 1, 2, 64, [8], True, 0)
    row = torch.randn((1, 2, 1, 64), generator=gen).to(torch.bfloat16)
    row[0, 1, 0, 5] = float("nan")
    ops.kv_append(view, row.to(dev), row.to(dev), torch.tensor([8], dtype=torch.int32, device=dev), status=status)
    k, _ = ops.kv_gather(view, torch.tensor([9], dtype=torch.int32, device=dev), 9)
    assert torch.isnan(k[0, 1, 8].float()).all() and not torch.isnan(k[0, 0, 8].float()).any()
    assert not torch.isnan(k[0, :, :8].float()).any()


def test_gather_rejects_overlapping_outputs(dev):
    gen = torch.Generator().manual_seed(11)
    view, _, _ = _cache(dev, gen, 1, 2, 64, [8], False, 0)
    buf = torch.zeros((1, 2, 16, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.AicasError, match="overlap"):
        ops.kv_gather(view, torch.tensor([8], dtype=torch.int32, device=dev), 16, out=(buf, buf))
