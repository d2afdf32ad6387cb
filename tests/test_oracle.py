"""Pin the CPU oracle (oracle/reference_path.py) before trusting it as the checker.

The reference ships no golden vectors for this path, so each oracle function is pinned by something a
plausible mistake would fail: brute force in pure Python on tiny inputs, closed forms, exhaustive tables,
an independent scalar implementation, and special cases. None of these retype the oracle's own formula.
"""

import math
import random

import pytest
import torch

from oracle import reference_path as ref


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


# --------------------------------------------------------------------------------------------------- GQA
def test_repeat_kv_head_mapping():
    """q head i reads kv head i // n_rep (HF/reference convention); an i % Hkv mapping would fail here."""
    x = torch.arange(2 * 4 * 3 * 2, dtype=torch.float32).view(2, 4, 3, 2)
    for n_rep in (1, 2, 4):
        y = ref.repeat_kv(x, n_rep)
        assert y.shape == (2, 4 * n_rep, 3, 2)
        for h in range(4 * n_rep):
            assert torch.equal(y[:, h], x[:, h // n_rep])


def _brute_decode(q, k, v, scale, n_rep):
    """softmax(q.k * scale).v with Python floats and math.exp, one (b, head) at a time."""
    B, Hq, _, D = q.shape
    L = k.shape[2]
    out = torch.zeros(B, Hq, 1, D, dtype=torch.float64)
    for b in range(B):
        for h in range(Hq):
            kv = h // n_rep
            logits = []
            for t in range(L):
                logits.append(sum(float(q[b, h, 0, d]) * float(k[b, kv, t, d]) for d in range(D)) * scale)
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            z = sum(w)
            for d in range(D):
                out[b, h, 0, d] = sum(w[t] * float(v[b, kv, t, d]) for t in range(L)) / z
    return out


@pytest.mark.parametrize("L", [1, 3, 8])
@pytest.mark.parametrize("n_rep", [1, 2])
def test_decode_matches_brute_force(L, n_rep):
    B, Hkv, D = 2, 2, 16
    q = _bf16((B, Hkv * n_rep, 1, D), 1 + L)
    k = _bf16((B, Hkv, L, D), 2 + L)
    v = _bf16((B, Hkv, L, D), 3 + L)
    scale = D ** -0.5
    brute = _brute_decode(q, k, v, scale, n_rep)
    assert (ref.decode_fp64(q, k, v, scale, n_rep) - brute).abs().max() < 1e-12
    got = ref.sdpa_decode(q.float(), k.float(), v.float(), scale, n_rep).double()
    assert (got - brute).abs().max() < 1e-5
    # bf16 SDPA (what the reference runs) stays within bf16 rounding of the exact result
    got16 = ref.sdpa_decode(q, k, v, scale, n_rep).double()
    assert (got16 - brute).abs().max() < 2e-2


def test_decode_special_cases():
    D, n_rep = 32, 2
    scale = D ** -0.5
    q = _bf16((1, 4, 1, D), 5)
    # one key: the output is exactly that V row (for every q head of the group)
    k1, v1 = _bf16((1, 2, 1, D), 6), _bf16((1, 2, 1, D), 7)
    assert torch.equal(ref.sdpa_decode(q.float(), k1.float(), v1.float(), scale, n_rep),
                       ref.repeat_kv(v1.float(), n_rep))
    # identical keys: uniform weights, the output is the mean of V
    k = _bf16((1, 2, 1, D), 8).expand(1, 2, 50, D).contiguous()
    v = _bf16((1, 2, 50, D), 9)
    out = ref.sdpa_decode(q.float(), k.float(), v.float(), scale, n_rep)
    torch.testing.assert_close(out, ref.repeat_kv(v.float().mean(dim=2, keepdim=True), n_rep), atol=1e-6, rtol=0)
    # a key whose logit exceeds all others by >= 30: the output is (to e^-30) that key's V row
    kp = _bf16((1, 2, 50, D), 10).float()
    qh = q[0, 0, 0].float()
    kp[0, 0, 17] = qh / qh.norm() * (30.0 + 20.0) / (scale * qh.norm())
    out = ref.sdpa_decode(q.float(), kp, v.float(), scale, n_rep)
    torch.testing.assert_close(out[0, 0, 0], v[0, 0, 17].float(), atol=1e-5, rtol=0)


def test_eager_and_sdpa_restatements_agree():
    """The two reference attention forms (SDPA fallback, eager with fp32 softmax cast to bf16) agree within
    the bf16 bar; neither is the other's retyping (one calls torch's SDPA kernel)."""
    q, k, v = _bf16((2, 16, 1, 128), 11), _bf16((2, 8, 300, 128), 12), _bf16((2, 8, 300, 128), 13)
    a = ref.sdpa_decode(q, k, v, 128 ** -0.5, 2).float()
    b = ref.eager_decode(q, k, v, 128 ** -0.5, 2).float()
    exact = ref.decode_fp64(q, k, v, 128 ** -0.5, 2)
    assert (a - exact).abs().max() < 2e-2
    assert (b - exact).abs().max() < 2e-2


def test_ragged_decode_is_per_sequence():
    q = _bf16((3, 4, 1, 16), 14)
    ks = [_bf16((2, L, 16), 20 + L) for L in (1, 5, 9)]
    vs = [_bf16((2, L, 16), 30 + L) for L in (1, 5, 9)]
    out = ref.ragged_decode(q, ks, vs, 0.25, 2, fp64=True)
    for b in range(3):
        brute = _brute_decode(q[b : b + 1], ks[b][None], vs[b][None], 0.25, 2)
        assert (out[b : b + 1] - brute).abs().max() < 1e-12


# ---------------------------------------------------------------------------------------------- appends
def test_cat_index_copy_and_ragged_append_agree_bitwise():
    B, H, L, D, n = 2, 3, 7, 16, 2
    keys, values = _bf16((B, H, L, D), 40), _bf16((B, H, L, D), 41)
    kn, vn = _bf16((B, H, n, D), 42), _bf16((B, H, n, D), 43)
    ck, cv = ref.dynamic_layer_update(keys, values, kn, vn)
    kb = torch.full((B, H, 16, D), float("nan")).to(torch.bfloat16)
    vb = kb.clone()
    kb[:, :, :L], vb[:, :, :L] = keys, values
    ik, iv = ref.inplace_layer_update(kb, vb, kn, vn, L)
    assert torch.equal(ck.view(torch.int16), ik.view(torch.int16))
    assert torch.equal(cv.view(torch.int16), iv.view(torch.int16))
    assert torch.isnan(kb[:, :, L + n :].float()).all()  # rows past the append untouched
    kb2 = torch.zeros((B, H, 16, D), dtype=torch.bfloat16)
    vb2 = kb2.clone()
    kb2[:, :, :L], vb2[:, :, :L] = keys, values
    assert ref.ragged_append(kb2, vb2, kn, vn, [L, L]) == [L + n, L + n]
    assert torch.equal(kb2[:, :, : L + n].view(torch.int16), ck.view(torch.int16))
    # the very first append of an empty DynamicLayer returns the new rows
    fk, fv = ref.dynamic_layer_update(None, None, kn, vn)
    assert torch.equal(fk, kn) and torch.equal(fv, vn)


def test_paged_scatter_gather_round_trip():
    B, H, D, page = 3, 2, 8, 4
    lens = [1, 4, 11]
    per_seq = 3
    g = torch.Generator().manual_seed(44)
    bt = torch.randperm(B * per_seq + 2, generator=g)[: B * per_seq].to(torch.int32).view(B, per_seq)
    pool = torch.zeros((B * per_seq + 2, H, page, D))
    seqs = [torch.randn((H, L, D), generator=g) for L in lens]
    for b, L in enumerate(lens):
        for t in range(L):
            ref.paged_scatter_rows(pool, bt, b, t, seqs[b][:, t])
    back = ref.paged_gather(pool, bt, lens)
    for b in range(B):
        assert torch.equal(back[b], seqs[b])
    # identity block table == contiguous layout
    ident = torch.arange(B * per_seq, dtype=torch.int32).view(B, per_seq)
    contig = torch.randn((B, H, per_seq * page, D), generator=g)
    pool2 = contig.view(B, H, per_seq, page, D).transpose(1, 2).reshape(B * per_seq, H, page, D)
    for b, s in enumerate(ref.paged_gather(pool2, ident, lens)):
        assert torch.equal(s, contig[b, :, : lens[b]])


# ------------------------------------------------------------------------------------------------ fp8
def test_e4m3_decode_table_closed_form():
    """All 256 codes: torch's float8_e4m3fn cast equals the OCP E4M3 closed form (bias 7, no infinities,
    S.1111.111 = NaN, subnormals m * 2^-9)."""
    table = ref.e4m3_decode_table()
    for code in range(256):
        expect = ref.e4m3_value(code)
        if math.isnan(expect):
            assert math.isnan(float(table[code])), code
        else:
            assert float(table[code]) == expect, code
    assert float(table[0x7E]) == 448.0 and float(table[0x01]) == 2.0 ** -9 and float(table[0x08]) == 2.0 ** -6


@pytest.mark.parametrize("x, code", [
    (448.0, 0x7E), (-448.0, 0xFE), (1.0, 0x38), (1.0625, 0x38), (1.1875, 0x3A), (1.125, 0x39),
    (2.0 ** -9, 0x01), (2.0 ** -10, 0x00), (3 * 2.0 ** -10, 0x02), (-1e-3, 0x81), (2.0 ** -6, 0x08),
    (15 * 2.0 ** -10, 0x08), (0.0, 0x00), (-0.0, 0x80), (440.0, 0x7E), (416.0, 0x7D), (432.0, 0x7E),
])
def test_e4m3_encode_known_answers(x, code):
    """Round-to-nearest-even at mantissa ties (1.0625 -> 1.0, 1.1875 -> 1.25), in the subnormal range
    (2^-10 -> 0, 3*2^-10 -> 2*2^-9) and across the subnormal/normal boundary (15*2^-10 -> 2^-6)."""
    assert ref.e4m3_encode_py(x) == code
    assert int(torch.tensor([x]).to(torch.float8_e4m3fn).view(torch.uint8)) == code


def test_e4m3_python_encoder_matches_torch_cast():
    """An exact-rational scalar encoder agrees with torch's cast on 20000 random values of every magnitude
    in [-448, 448] (torch's cast turns values above 448 into NaN, which is why the quantizer clamps)."""
    rnd = random.Random(45)
    xs = [0.0, -0.0, 448.0, -448.0]
    for _ in range(20000):
        mag = 2.0 ** rnd.uniform(-12, math.log2(448.0))
        xs.append(mag if rnd.random() < 0.5 else -mag)
    codes = torch.tensor(xs, dtype=torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).tolist()
    for x, c in zip(xs, codes):
        assert ref.e4m3_encode_py(x) == c, x
    assert math.isnan(float(torch.tensor([500.0]).to(torch.float8_e4m3fn).float()))


def test_fp8_quantize_rows_properties():
    x = _bf16((5, 64), 46, scale=3.0).float()
    x[1] = 0.0
    x[2, 7] = 8.0
    codes, scale = ref.fp8_quantize_rows(x)
    assert torch.equal(scale, x.abs().amax(dim=-1) / 448.0)
    assert scale[1] == 0 and torch.count_nonzero(codes[1].view(torch.uint8)) == 0
    deq = ref.fp8_dequantize_rows(codes, scale)
    # the row maximum maps to exactly +-448 * scale
    for r in (0, 2, 3, 4):
        i = int(x[r].abs().argmax())
        assert float(deq[r, i]) == pytest.approx(float(x[r, i]), rel=1e-6)
    # elementwise error: half an e4m3 ulp (2^-4 relative) in the normal range, 2^-10 * scale below it
    err = (deq - x).abs()
    bound = torch.maximum(x.abs() * 2.0 ** -4, scale[:, None] * 2.0 ** -10) * 1.0001
    assert bool((err <= bound).all())


def test_fp8_quantize_rows_poisons_non_finite_rows():
    """A row holding NaN or +-Inf (anywhere, any sign) is stored poisoned: scale NaN, every code 0, so that it
    dequantises to NaN everywhere; finite rows in the same call are quantized as on their own."""
    x = _bf16((6, 32), 48, scale=2.0).float()
    finite_rows = x[[0, 5]].clone()
    x[1, 3] = float("nan")
    x[2, 0] = float("inf")
    x[3, 31] = float("-inf")
    x[4, :] = float("nan")
    codes, scale = ref.fp8_quantize_rows(x)
    for r in (1, 2, 3, 4):
        assert math.isnan(float(scale[r]))
        assert torch.count_nonzero(codes[r].view(torch.uint8)) == 0
        assert bool(torch.isnan(ref.fp8_dequantize_rows(codes[r : r + 1], scale[r : r + 1])).all())
    c0, s0 = ref.fp8_quantize_rows(finite_rows)
    assert torch.equal(codes[[0, 5]].view(torch.uint8), c0.view(torch.uint8)) and torch.equal(scale[[0, 5]], s0)
    assert torch.equal(s0, finite_rows.abs().amax(dim=-1) / 448.0)


# ------------------------------------------------------------------------------------------- LSE merge
@pytest.mark.parametrize("splits", [[0, 100], [0, 1, 100], [0, 37, 64, 99, 100], list(range(0, 101, 10))])
def test_lse_merge_equals_single_pass(splits):
    g = torch.Generator().manual_seed(47)
    k = torch.randn((100, 32), generator=g, dtype=torch.float64)
    v = torch.randn((100, 32), generator=g, dtype=torch.float64)
    q = torch.randn(32, generator=g, dtype=torch.float64)
    ms, ls, accs = ref.split_partials(q, k, v, 32 ** -0.5, splits)
    merged = ref.merge_partials(ms, ls, accs)
    single = torch.softmax(k @ q * 32 ** -0.5, dim=0) @ v
    assert (merged - single).abs().max() < 1e-12
    # a planted dominant key in the last split: the merge still returns (almost) its V row
    k2 = k.clone()
    k2[95] = q / q.norm() * (40.0 / (32 ** -0.5 * q.norm()))
    ms, ls, accs = ref.split_partials(q, k2, v, 32 ** -0.5, splits)
    assert (ref.merge_partials(ms, ls, accs) - v[95]).abs().max() < 1e-6


# ------------------------------------------------------------------------- q/k preparation (norm + RoPE)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qk_preparation_matches_transformers_modules(dtype):
    """rms_norm / apply_rope / prepare_qk against the library routines the reference path calls:
    transformers' Qwen3VLTextRMSNorm and apply_rotary_pos_emb, with cos/sin from its Qwen3VLTextRotaryEmbedding
    (interleaved M-RoPE, text positions) — bit for bit."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (
        Qwen3VLTextRMSNorm, Qwen3VLTextRotaryEmbedding, apply_rotary_pos_emb)

    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, D = 3, 16, 8, 128
    cfg = Qwen3VLTextConfig(hidden_size=256, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D)
    qn, kn = Qwen3VLTextRMSNorm(D, eps=1e-6), Qwen3VLTextRMSNorm(D, eps=1e-6)
    with torch.no_grad():
        qn.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
        kn.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
    qn, kn = qn.to(dtype), kn.to(dtype)
    q = (3 * torch.randn((B, 1, Hq, D), generator=g)).to(dtype)
    k = (3 * torch.randn((B, 1, Hkv, D), generator=g)).to(dtype)
    pos = torch.tensor([[5], [1000], [31000]])
    cos, sin = Qwen3VLTextRotaryEmbedding(cfg)(q, pos)
    with torch.no_grad():
        hq, hk = apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
        oq, ok = ref.prepare_qk(q.transpose(1, 2), k.transpose(1, 2), qn.weight, kn.weight, 1e-6, cos, sin)
        assert torch.equal(ref.rms_norm(q, qn.weight, 1e-6), qn(q))
    assert torch.equal(oq, hq) and torch.equal(ok, hk)


def test_rope_is_the_pairwise_rotation():
    """In float64, x * cos + rotate_half(x) * sin with cos/sin = cat(c, c) / cat(s, s) rotates each pair
    (x_j, x_{j+D/2}) by the angle of frequency j, so it keeps every pair's length; angle 0 is the identity."""
    g = torch.Generator().manual_seed(4)
    B, H, D = 2, 3, 64
    x = torch.randn((B, H, 1, D), generator=g, dtype=torch.float64)
    theta = torch.rand((B, 1, D // 2), generator=g, dtype=torch.float64) * 2 * math.pi
    cos, sin = torch.cat([theta.cos()] * 2, -1), torch.cat([theta.sin()] * 2, -1)
    y = ref.apply_rope(x, cos, sin)
    a, b_ = x[..., : D // 2], x[..., D // 2 :]
    t = theta.unsqueeze(1)
    assert torch.allclose(y[..., : D // 2], a * t.cos() - b_ * t.sin(), atol=1e-12)
    assert torch.allclose(y[..., D // 2 :], b_ * t.cos() + a * t.sin(), atol=1e-12)
    assert torch.allclose(y[..., : D // 2] ** 2 + y[..., D // 2 :] ** 2, a ** 2 + b_ ** 2, atol=1e-12)
    zero = torch.zeros_like(theta)
    assert torch.equal(ref.apply_rope(x, torch.cat([zero.cos()] * 2, -1), torch.cat([zero.sin()] * 2, -1)), x)


def test_rms_norm_closed_forms():
    """A constant row c gives weight * c / sqrt(c^2 + eps); with unit weight any row comes out with mean square
    1 / (1 + eps / mean(x^2)); scaling the row does not change it when eps = 0. (The norm is computed in float32
    whatever the input type, as the model's module does, hence float32 tolerances.)"""
    D, eps = 128, 1e-6
    w = torch.linspace(0.5, 1.5, D, dtype=torch.float64)
    for c in (-3.0, 1e-4, 7.5):
        y = ref.rms_norm(torch.full((D,), c, dtype=torch.float64), w, eps)
        assert torch.allclose(y, w * c / math.sqrt(c * c + eps), rtol=1e-6)
    x = torch.randn((5, D), generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    ms = x.pow(2).mean(-1)
    y = ref.rms_norm(x, torch.ones(D, dtype=torch.float64), eps)
    assert torch.allclose(y.pow(2).mean(-1), 1 / (1 + eps / ms), rtol=1e-6)
    assert torch.allclose(ref.rms_norm(37.0 * x, w, 0.0), ref.rms_norm(x, w, 0.0), rtol=1e-6)
