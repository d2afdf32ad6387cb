"""KV append on the GPU through the C ABI, bit-exact against the oracle.

Oracle: reference_path.inplace_layer_update / ragged_append (index_copy_ at the current length, which is
bitwise what DynamicLayer.update's torch.cat produces, see test_oracle.py), fp8_quantize_rows for fp8
caches, paged_scatter_rows for paged caches.
"""

import math

import pytest
import torch

from aicas_amd import _lib, ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


def _bits(x: torch.Tensor) -> torch.Tensor:
    return x.view(torch.int16) if x.element_size() == 2 else x.view(torch.uint8)


def _rand(shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("n_new", [1, 3, 37])
def test_append_contiguous_bitexact(dev, status, dtype, D, n_new):
    B, H, cap = 3, 4, 96
    lens = [0, 17, 50]
    cache_k = _rand((B, H, cap, D), 10, dtype)
    cache_v = _rand((B, H, cap, D), 11, dtype)
    k_new = _rand((B, H, n_new, D), 12, dtype)
    v_new = _rand((B, H, n_new, D), 13, dtype)
    exp_k, exp_v = cache_k.clone(), cache_v.clone()
    new_lens = ref.ragged_append(exp_k, exp_v, k_new, v_new, lens)

    gk, gv = cache_k.to(dev), cache_v.to(dev)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    ops.kv_append(ops.KVCacheView(gk, gv), k_new.to(dev), v_new.to(dev), pos, pos, status)
    torch.cuda.synchronize()
    assert torch.equal(_bits(gk.cpu()), _bits(exp_k))
    assert torch.equal(_bits(gv.cpu()), _bits(exp_v))
    assert pos.cpu().tolist() == new_lens
    assert int(status.item()) == 0


def test_append_matches_dynamic_cache_cat(dev):
    """Decode-step append of HF-layout rows (a transposed [B,1,H,D] view, as Qwen3VLTextAttention passes
    them) reproduces DynamicLayer.update's torch.cat bit for bit."""
    B, H, D, L = 2, 8, 128, 40
    prefix_k, prefix_v = _rand((B, H, L, D), 1), _rand((B, H, L, D), 2)
    new_k = _rand((B, 1, H, D), 3).transpose(1, 2)  # [B, H, 1, D], non-contiguous
    new_v = _rand((B, 1, H, D), 4).transpose(1, 2)
    exp_k, exp_v = ref.dynamic_layer_update(prefix_k, prefix_v, new_k, new_v)

    gk = torch.zeros((B, H, 64, D), dtype=torch.bfloat16, device=dev)
    gv = torch.zeros_like(gk)
    gk[:, :, :L] = prefix_k.to(dev)
    gv[:, :, :L] = prefix_v.to(dev)
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    ops.kv_append(ops.KVCacheView(gk, gv), new_k.to(dev), new_v.to(dev), lens, lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(gk[:, :, : L + 1].cpu()), _bits(exp_k))
    assert torch.equal(_bits(gv[:, :, : L + 1].cpu()), _bits(exp_v))
    assert torch.count_nonzero(gk[:, :, L + 1 :]).item() == 0  # canary: rows past the append untouched


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16])
def test_append_fp8_contiguous_bitexact(dev, status, D, src_dtype):
    B, H, cap, n_new = 2, 8, 48, 5
    lens = [3, 40]
    k_new = _rand((B, H, n_new, D), 21, src_dtype)
    v_new = _rand((B, H, n_new, D), 22, src_dtype, scale=3.0)
    # 1% outliers at +-8 and one all-zero row
    k_new[0, 1, 2, 5] = 8.0
    v_new[1, 3, 0, 7] = -8.0
    k_new[1, 2, 1] = 0.0
    gk = torch.zeros((B, H, cap, D), dtype=ops.FP8_DTYPE, device=dev)
    gv = torch.zeros_like(gk)
    ks = torch.full((B, H, cap), -1.0, device=dev)
    vs = torch.full((B, H, cap), -1.0, device=dev)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    ops.kv_append(ops.KVCacheView(gk, gv, ks, vs), k_new.to(dev), v_new.to(dev), pos, pos, status)
    torch.cuda.synchronize()
    ck, sk = ref.fp8_quantize_rows(k_new)
    cv, sv = ref.fp8_quantize_rows(v_new)
    for b, L in enumerate(lens):
        assert torch.equal(gk[b, :, L : L + n_new].cpu().view(torch.uint8), ck[b].view(torch.uint8))
        assert torch.equal(gv[b, :, L : L + n_new].cpu().view(torch.uint8), cv[b].view(torch.uint8))
        assert torch.equal(ks[b, :, L : L + n_new].cpu(), sk[b])
        assert torch.equal(vs[b, :, L : L + n_new].cpu(), sv[b])
        # untouched rows keep their sentinel scale
        assert bool((ks[b, :, :L] == -1.0).all()) and bool((ks[b, :, L + n_new :] == -1.0).all())
    assert pos.cpu().tolist() == [L + n_new for L in lens]
    assert int(status.item()) == 0


@pytest.mark.parametrize("fp8", [False, True])
def test_append_paged_bitexact(dev, status, fp8):
    B, H, D, page, per_seq = 4, 8, 128, 16, 6
    nblocks = B * per_seq + 3
    g = torch.Generator().manual_seed(7)
    bt = torch.randperm(nblocks, generator=g)[: B * per_seq].to(torch.int32).view(B, per_seq)
    lens = [0, 15, 16, 70]
    n_new = 9
    k_new = _rand((B, H, n_new, D), 31)
    v_new = _rand((B, H, n_new, D), 32)
    store = ops.FP8_DTYPE if fp8 else torch.bfloat16
    pk = torch.zeros((nblocks, H, page, D), dtype=store)
    pv = torch.zeros_like(pk)
    sk = torch.zeros((nblocks, H, page)) if fp8 else None
    sv = torch.zeros((nblocks, H, page)) if fp8 else None
    ek, ev = pk.clone(), pv.clone()
    esk = sk.clone() if fp8 else None
    esv = sv.clone() if fp8 else None
    if fp8:
        qk, qsk = ref.fp8_quantize_rows(k_new)
        qv, qsv = ref.fp8_quantize_rows(v_new)
    for b, L in enumerate(lens):
        for j in range(n_new):
            if fp8:
                ref.paged_scatter_rows(ek, bt, b, L + j, qk[b, :, j])
                ref.paged_scatter_rows(ev, bt, b, L + j, qv[b, :, j])
                ref.paged_scatter_rows(esk, bt, b, L + j, qsk[b, :, j])
                ref.paged_scatter_rows(esv, bt, b, L + j, qsv[b, :, j])
            else:
                ref.paged_scatter_rows(ek, bt, b, L + j, k_new[b, :, j])
                ref.paged_scatter_rows(ev, bt, b, L + j, v_new[b, :, j])
    view = ops.KVCacheView(
        pk.to(dev), pv.to(dev), sk.to(dev) if fp8 else None, sv.to(dev) if fp8 else None, bt.to(dev)
    )
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    ops.kv_append(view, k_new.to(dev), v_new.to(dev), pos, pos, status)
    torch.cuda.synchronize()
    assert torch.equal(_bits(view.k.cpu()), _bits(ek))
    assert torch.equal(_bits(view.v.cpu()), _bits(ev))
    if fp8:
        assert torch.equal(view.k_scale.cpu(), esk)
        assert torch.equal(view.v_scale.cpu(), esv)
    assert pos.cpu().tolist() == [L + n_new for L in lens]
    assert int(status.item()) == 0


@pytest.mark.parametrize("n_new, H, page", [(1, 1, 1), (2, 3, 2), (5, 8, 4), (7, 2, 16), (16, 8, 16),
                                             (33, 5, 64), (300, 3, 32), (1000, 1, 128)])
@pytest.mark.parametrize("fp8", [False, True])
def test_append_paged_row_indexing_shapes(dev, status, n_new, H, page, fp8):
    """The append kernel finds each row's head and token by dividing its index by the launch's new-row count (a
    multiplier computed on the host) and its page by a shift: over new-row counts, head counts and page sizes
    whose rows straddle workgroups, heads and pages in every way, every row lands bit for bit where the oracle
    scatters it (bf16, and fp8 codes and scales)."""
    B, D = 3, 64
    g = torch.Generator().manual_seed(1000 * n_new + 10 * H + page)
    lens = [0, 5, 3 * page + 1]
    per_seq = -(-(max(lens) + n_new) // page)
    nblocks = B * per_seq + 2
    bt = torch.randperm(nblocks, generator=g)[: B * per_seq].to(torch.int32).view(B, per_seq)
    k_new = torch.randn((B, H, n_new, D), generator=g).to(torch.bfloat16)
    v_new = torch.randn((B, H, n_new, D), generator=g).to(torch.bfloat16)
    store = ops.FP8_DTYPE if fp8 else torch.bfloat16
    pk = torch.zeros((nblocks, H, page, D), dtype=store)
    pv = torch.zeros_like(pk)
    sk = torch.zeros((nblocks, H, page)) if fp8 else None
    sv = torch.zeros((nblocks, H, page)) if fp8 else None
    ek, ev = pk.clone(), pv.clone()
    esk = sk.clone() if fp8 else None
    esv = sv.clone() if fp8 else None
    kr, vr = (ref.fp8_quantize_rows(k_new), ref.fp8_quantize_rows(v_new)) if fp8 else ((k_new, None), (v_new, None))
    for b, L in enumerate(lens):
        for j in range(n_new):
            ref.paged_scatter_rows(ek, bt, b, L + j, kr[0][b, :, j])
            ref.paged_scatter_rows(ev, bt, b, L + j, vr[0][b, :, j])
            if fp8:
                ref.paged_scatter_rows(esk, bt, b, L + j, kr[1][b, :, j])
                ref.paged_scatter_rows(esv, bt, b, L + j, vr[1][b, :, j])
    view = ops.KVCacheView(pk.to(dev), pv.to(dev), sk.to(dev) if fp8 else None, sv.to(dev) if fp8 else None,
                           bt.to(dev))
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    ops.kv_append(view, k_new.to(dev), v_new.to(dev), pos, pos, status)
    torch.cuda.synchronize()
    assert torch.equal(_bits(view.k.cpu()), _bits(ek))
    assert torch.equal(_bits(view.v.cpu()), _bits(ev))
    if fp8:
        assert torch.equal(view.k_scale.cpu(), esk)
        assert torch.equal(view.v_scale.cpu(), esv)
    assert pos.cpu().tolist() == [L + n_new for L in lens]
    assert int(status.item()) == 0


def test_append_overflow_is_dropped_and_reported(dev, status):
    B, H, D, cap = 2, 2, 64, 8
    gk = torch.zeros((B, H, cap, D), dtype=torch.bfloat16, device=dev)
    gv = torch.zeros_like(gk)
    pos = torch.tensor([6, 2], dtype=torch.int32, device=dev)
    lens_out = torch.zeros(B, dtype=torch.int32, device=dev)
    k_new = torch.ones((B, H, 3, D), dtype=torch.bfloat16, device=dev)
    ops.kv_append(ops.KVCacheView(gk, gv), k_new, k_new, pos, lens_out, status)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.STATUS_APPEND_OVERFLOW
    # sequence 0: rows 6, 7 written, row 8 dropped; sequence 1: rows 2..4 written
    assert gk[0, :, 6:].eq(1).all() and gk[0, :, :6].eq(0).all()
    assert gk[1, :, 2:5].eq(1).all() and gk[1, :, 5:].eq(0).all() and gk[1, :, :2].eq(0).all()
    assert lens_out.cpu().tolist() == [9, 5]
    assert pos.cpu().tolist() == [6, 2]


def test_append_rejects_bad_arguments(dev):
    gk = torch.zeros((1, 2, 8, 64), dtype=torch.bfloat16, device=dev)
    view = ops.KVCacheView(gk, gk.clone())
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.AicasError):
        ops.kv_append(view, torch.zeros((1, 2, 1, 64), dtype=torch.float16, device=dev),
                      torch.zeros((1, 2, 1, 64), dtype=torch.float16, device=dev), pos)
    with pytest.raises(_lib.AicasError):
        ops.kv_append(view, torch.zeros((1, 3, 1, 64), dtype=torch.bfloat16, device=dev),
                      torch.zeros((1, 3, 1, 64), dtype=torch.bfloat16, device=dev), pos)


def test_prefill_sized_append_many_sequences(dev, status):
    """A prompt-sized append (several workgroups per sequence) for more sequences than one block of the
    length-bump launch covers, with the bumped lengths written over the positions."""
    B, H, D, cap, n_new = 300, 2, 16, 640, 300
    g = torch.Generator().manual_seed(41)
    lens = torch.randint(0, cap - n_new, (B,), generator=g).tolist()
    cache_k = _rand((B, H, cap, D), 42)
    cache_v = _rand((B, H, cap, D), 43)
    k_new, v_new = _rand((B, H, n_new, D), 44), _rand((B, H, n_new, D), 45)
    exp_k, exp_v = cache_k.clone(), cache_v.clone()
    new_lens = ref.ragged_append(exp_k, exp_v, k_new, v_new, lens)
    gk, gv = cache_k.to(dev), cache_v.to(dev)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    ops.kv_append(ops.KVCacheView(gk, gv), k_new.to(dev), v_new.to(dev), pos, pos, status)
    torch.cuda.synchronize()
    assert torch.equal(_bits(gk.cpu()), _bits(exp_k))
    assert torch.equal(_bits(gv.cpu()), _bits(exp_v))
    assert pos.cpu().tolist() == new_lens
    assert int(status.item()) == 0


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fused", [False, True])
def test_fp8_non_finite_rows_are_stored_poisoned(dev, status, D, fused):
    """Rows holding NaN, +Inf or -Inf reach an fp8 cache as the oracle stores them (scale NaN, all-zero codes)
    and set AICAS_STATUS_NONFINITE_ROW; finite rows of the same launch are written code for code. Through the
    fused append + attend, the sequence with a poisoned row attends to NaN (as the unquantised reference would),
    the others are unaffected."""
    B, H, G, cap = 4, 4, 2, 64
    lens = [10, 20, 30, 40]
    k_new = _rand((B, H, 1, D), 70 + D, scale=2.0).float()
    v_new = _rand((B, H, 1, D), 71 + D, scale=2.0).float()
    k_new[1, 2, 0, 5] = float("nan")
    k_new[2, 0, 0, 0] = float("inf")
    v_new[2, 3, 0, D - 1] = float("-inf")
    k_new, v_new = k_new.to(torch.bfloat16), v_new.to(torch.bfloat16)
    exp_kc, exp_ks = ref.fp8_quantize_rows(k_new[:, :, 0])
    exp_vc, exp_vs = ref.fp8_quantize_rows(v_new[:, :, 0])
    kc = torch.zeros((B, H, cap, D), dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((B, H, cap), dtype=torch.float32, device=dev)
    vs = torch.zeros_like(ks)
    view = ops.KVCacheView(kc, vc, ks, vs)
    pos = torch.tensor(lens, dtype=torch.int32, device=dev)
    if fused:
        q = _rand((B, H * G, 1, D), 72).to(dev)
        out = ops.decode_attention_append(q, view, k_new.to(dev), v_new.to(dev), pos, sm_scale=D ** -0.5,
                                          max_seq_len=max(lens) + 1, status=status)
    else:
        ops.kv_append(view, k_new.to(dev), v_new.to(dev), pos, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.STATUS_NONFINITE_ROW
    for b, L in enumerate(lens):
        got_k, got_v = kc[b, :, L].cpu().view(torch.uint8), vc[b, :, L].cpu().view(torch.uint8)
        assert torch.equal(got_k, exp_kc[b].view(torch.uint8)) and torch.equal(got_v, exp_vc[b].view(torch.uint8))
        torch.testing.assert_close(ks[b, :, L].cpu(), exp_ks[b], rtol=0, atol=0, equal_nan=True)
        torch.testing.assert_close(vs[b, :, L].cpu(), exp_vs[b], rtol=0, atol=0, equal_nan=True)
    assert math.isnan(float(ks[1, 2, lens[1]])) and math.isnan(float(ks[2, 0, lens[2]]))
    assert math.isnan(float(vs[2, 3, lens[2]])) and not math.isnan(float(ks[0, 0, lens[0]]))
    if fused:
        o = out.float().cpu()
        assert bool(torch.isnan(o[1, 2 * G : 3 * G]).all()) and bool(torch.isnan(o[2, 0:G]).all())
        assert bool(torch.isnan(o[2, 3 * G : 4 * G]).all())  # a poisoned V row turns its heads' outputs NaN
        assert bool(torch.isfinite(o[0]).all()) and bool(torch.isfinite(o[3]).all())
