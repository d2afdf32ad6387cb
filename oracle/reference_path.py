"""CPU oracle for the KV-append + q_len=1 GQA decode-attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``aicas_amd``) imports this module; only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it, as the checker or as the
timed CPU baseline.

It restates, in torch on the CPU, the reference path of Frun1na/AICAS:
  * KV append = HF ``DynamicLayer.update`` (``torch.cat`` along the token axis),
    transformers/cache_utils.py:127-146, and the preallocated variant ``InplaceDecodeCacheLayer.update``
    (``index_copy_`` at the current length), dujunbaoV1/evaluation_wrapper.py:84-100;
  * decode attention = ``sdpa_fallback`` (triton_qwen3vl/fallback.py:23-64): SDPA over the
    ``repeat_kv``-expanded cache (fallback.py:7-12), non-causal because q_len == 1
    (transformers/integrations/sdpa_attention.py:120), scale = module.scaling;
  * the eager variant of the KV wrappers (new KV cache/evaluation_wrapper.py:248-265, same math as
    transformers/models/qwen3_vl/modeling_qwen3_vl.py:171-193): fp32 softmax cast back to the query dtype
    before the P.V product;
  * the paged layout (block table of fixed-size pages, new KV cache/evaluation_wrapper.py:143-232) with fp8
    e4m3 (OCP "e4m3fn") rows and one fp32 scale per (token, kv head) in place of the KIVI 2-bit codec, and the
    growth of its page table one page at a time (block_alloc / block_free).

The reference ships no golden vectors for this path, so each function here is pinned in
tests/test_oracle.py against closed forms, brute force and library routines (see the test docstrings).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

FP8_MAX = 448.0


# ---------------------------------------------------------------------------------------------- KV append
def dynamic_layer_update(
    keys: torch.Tensor | None, values: torch.Tensor | None, k_new: torch.Tensor, v_new: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """transformers/cache_utils.py:127-146: the cache grows by concatenation along dim -2."""
    if keys is None:
        keys = torch.tensor([], dtype=k_new.dtype, device=k_new.device)
        values = torch.tensor([], dtype=v_new.dtype, device=v_new.device)
    return torch.cat([keys, k_new], dim=-2), torch.cat([values, v_new], dim=-2)


def inplace_layer_update(
    keys_buf: torch.Tensor, values_buf: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, start: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """dujunbaoV1/evaluation_wrapper.py:84-100 (write_mode "index_copy"): rows go to [start, start+n)."""
    n = k_new.shape[-2]
    positions = torch.arange(start, start + n, device=k_new.device)
    keys_buf.index_copy_(2, positions, k_new)
    values_buf.index_copy_(2, positions, v_new)
    return keys_buf[:, :, : start + n, :], values_buf[:, :, : start + n, :]


def ragged_append(
    keys_buf: torch.Tensor, values_buf: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, lens: list[int]
) -> list[int]:
    """Per-sequence in-place append at each sequence's own length (the ragged form of the above)."""
    n = k_new.shape[-2]
    for b, L in enumerate(lens):
        keys_buf[b, :, L : L + n, :] = k_new[b]
        values_buf[b, :, L : L + n, :] = v_new[b]
    return [L + n for L in lens]


# --------------------------------------------------------------------------------------- decode attention
def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """triton_qwen3vl/fallback.py:7-12: [B, Hkv, L, D] -> [B, Hkv*n_rep, L, D], kv head j serves q heads
    j*n_rep .. j*n_rep+n_rep-1."""
    b, h, L, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None, :, :].expand(b, h, n_rep, L, d).reshape(b, h * n_rep, L, d)


def sdpa_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, n_rep: int) -> torch.Tensor:
    """The oracle proper: triton_qwen3vl/fallback.py:23-64 without HF, i.e. SDPA over repeat_kv with
    is_causal = q_len > 1 and mask is None (False for decode). Returns [B, Hq, 1, D] in q's dtype."""
    is_causal = q.shape[2] > 1
    return F.scaled_dot_product_attention(
        q, repeat_kv(k, n_rep), repeat_kv(v, n_rep), attn_mask=None, dropout_p=0.0, scale=scale, is_causal=is_causal
    )


def eager_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, n_rep: int) -> torch.Tensor:
    """new KV cache/evaluation_wrapper.py:248-265 / modeling_qwen3_vl.py:171-193 (no mask, no dropout)."""
    ks = repeat_kv(k, n_rep)
    vs = repeat_kv(v, n_rep)
    w = torch.matmul(q, ks.transpose(2, 3)) * scale
    w = torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(w, vs)


def decode_fp64(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, n_rep: int) -> torch.Tensor:
    """Closed form softmax(q K^T s) V evaluated in float64 from the same (rounded) inputs."""
    q64, k64, v64 = q.double(), repeat_kv(k, n_rep).double(), repeat_kv(v, n_rep).double()
    w = torch.softmax(torch.matmul(q64, k64.transpose(2, 3)) * scale, dim=-1)
    return torch.matmul(w, v64)


def ragged_decode(
    q: torch.Tensor, k_seqs: list[torch.Tensor], v_seqs: list[torch.Tensor], scale: float, n_rep: int,
    fp64: bool = False,
) -> torch.Tensor:
    """Per-sequence decode over [Hkv, L_b, D] caches of different lengths; returns [B, Hq, 1, D]."""
    outs = []
    for b in range(q.shape[0]):
        fn = decode_fp64 if fp64 else sdpa_decode
        outs.append(fn(q[b : b + 1], k_seqs[b][None], v_seqs[b][None], scale, n_rep))
    return torch.cat(outs, dim=0)


# --------------------------------------------------------------------------------------------- LSE merge
def merge_partials(ms: torch.Tensor, ls: torch.Tensor, accs: torch.Tensor) -> torch.Tensor:
    """Combine split partials (running max m_i and sum l_i in the exp2 domain, unnormalised acc_i [.., D]):
    M = max m_i, l = sum l_i 2^(m_i - M), out = sum acc_i 2^(m_i - M) / l (split axis = 0)."""
    M = ms.max(dim=0).values
    c = torch.exp2(ms - M)
    l = (ls * c).sum(dim=0)
    return (accs * c[..., None]).sum(dim=0) / l[..., None]


def split_partials(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, splits: list[int]):
    """Partials of one query row q [D] over key ranges [splits[i], splits[i+1]) in float64 (exp2 domain)."""
    s = (k.double() @ q.double()) * scale * (1.0 / math.log(2.0))
    ms, ls, accs = [], [], []
    for a, b in zip(splits[:-1], splits[1:]):
        m = s[a:b].max()
        p = torch.exp2(s[a:b] - m)
        ms.append(m)
        ls.append(p.sum())
        accs.append(p @ v[a:b].double())
    return torch.stack(ms), torch.stack(ls), torch.stack(accs)


# ------------------------------------------------------------------------------------------------ fp8 e4m3
def e4m3_value(code: int) -> float:
    """Closed form of the OCP E4M3 (e4m3fn) encoding: bias 7, 3 mantissa bits, no infinities,
    S.1111.111 = NaN, subnormals m * 2^-9."""
    sign = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def e4m3_encode_py(x: float) -> int:
    """Independent scalar encoder (exact rational arithmetic, round half to even, saturating at 448)."""
    if math.isnan(x):
        return 0x7F
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    a = abs(x)
    if a >= FP8_MAX:
        return sign | 0x7E
    from fractions import Fraction

    fa = Fraction(a)
    if fa < Fraction(1, 64):
        m = fa * 512
        r = round(m)  # Python's round is half-to-even on Fractions
        return sign | int(r)
    e = math.floor(math.log2(a))
    # guard against log2 rounding at exact powers of two
    while Fraction(2) ** e > fa:
        e -= 1
    while Fraction(2) ** (e + 1) <= fa:
        e += 1
    mant = (fa / Fraction(2) ** e - 1) * 8
    r = round(mant)
    if r == 8:
        r = 0
        e += 1
    return sign | ((e + 7) << 3) | int(r)


def e4m3_decode_table() -> torch.Tensor:
    """float32 [256]: value of each code, as torch's float8_e4m3fn -> float32 cast gives it."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    return codes.view(torch.float8_e4m3fn).to(torch.float32)


def fp8_quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize-on-write for fp8 caches: rows along the last axis; scale = amax/448 (fp32) per row;
    codes = e4m3(clamp(x / scale, -448, 448)) (torch's cast rounds to nearest even; without the clamp it
    would turn values above 448 into NaN); an all-zero row has scale 0 and zero codes. A row holding any NaN
    or +-Inf is stored poisoned: scale NaN and zero codes, so that it dequantises to NaN everywhere (the
    unquantised row would make every score that touches it non-finite). The fp8 layout replaces the
    reference's KIVI codec (new KV cache/evaluation_wrapper.py:68-140), which defines no such case.
    Returns (codes as torch.float8_e4m3fn, scales float32 of shape x.shape[:-1])."""
    xf = x.float()
    finite = torch.isfinite(xf).all(dim=-1)
    amax = torch.where(finite[..., None], xf, torch.zeros_like(xf)).abs().amax(dim=-1)
    scale = torch.where(finite, amax / FP8_MAX, torch.full_like(amax, float("nan")))
    ok = finite & (scale > 0)
    safe = torch.where(ok, scale, torch.ones_like(scale))
    y = (torch.where(ok[..., None], xf, torch.zeros_like(xf)) / safe[..., None]).clamp(-FP8_MAX, FP8_MAX)
    y = torch.where(ok[..., None], y, torch.zeros_like(y))
    return y.to(torch.float8_e4m3fn), scale


def fp8_dequantize_rows(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return codes.to(torch.float32) * scale[..., None]


# ----------------------------------------------------------------------------------------------- paging
def paged_gather(pool: torch.Tensor, block_table: torch.Tensor, lens: list[int]) -> list[torch.Tensor]:
    """pool [num_blocks, Hkv, page, ...] + block_table [B, max_blocks] -> per-sequence [Hkv, L_b, ...]:
    token t of sequence b is row t % page of block block_table[b, t // page]."""
    page = pool.shape[2]
    out = []
    for b, L in enumerate(lens):
        nb = (L + page - 1) // page
        blocks = pool[block_table[b, :nb].long()]  # [nb, Hkv, page, ...]
        seq = blocks.transpose(0, 1).reshape(pool.shape[1], nb * page, *pool.shape[3:])
        out.append(seq[:, :L])
    return out


# ----------------------------------------------------------------------------------------- block pool
def block_pool_init(num_blocks: int) -> tuple[list[int], int]:
    """A pool with every block free, as a stack whose pops hand out 0, 1, 2, ...: (stack, count)."""
    return [num_blocks - 1 - i for i in range(num_blocks)], num_blocks


def block_alloc(stack: list[int], count: int, table: torch.Tensor, positions: list[int], n_new: int,
                page_size: int) -> tuple[int, int]:
    """Sequential page-table growth: in sequence order, every page that tokens [positions[b], positions[b] + n_new)
    touch and whose entry is negative takes the block on top of the stack — the reference grows its page table
    one page at a time in the same way, appending {"logical_page_id", "block_id"} with the next block id
    (new KV cache/evaluation_wrapper.py:164-190). Pages past the row's width set status 4 (append overflow); an
    empty stack leaves the entry at -1 and sets status 8 (out of blocks). Mutates ``table``; returns
    (new count, status)."""
    status = 0
    width = table.shape[1]
    for b in range(table.shape[0]):
        pos = max(int(positions[b]), 0)
        first, last = pos // page_size, (pos + n_new - 1) // page_size
        if last >= width:
            status |= 4
            last = width - 1
        for pg in range(first, last + 1):
            if int(table[b, pg]) < 0:
                if count > 0:
                    count -= 1
                    table[b, pg] = stack[count]
                else:
                    status |= 8
    return count, status


def block_free(stack: list[int], count: int, table: torch.Tensor, release: list[int], seq_lens: list[int] | None,
               num_blocks: int) -> tuple[int, int]:
    """In sequence order, every released sequence pushes its valid block ids (page order) back onto the stack,
    its row becomes -1 and its length 0 (the reference's reset drops the whole list, new KV
    cache/evaluation_wrapper.py:502-521). Ids outside
    [0, num_blocks) and pushes past a full stack are dropped with status 2. Mutates ``stack``, ``table`` and
    ``seq_lens``; returns (new count, status)."""
    status = 0
    for b in range(table.shape[0]):
        if not release[b]:
            continue
        for pg in range(table.shape[1]):
            e = int(table[b, pg])
            if 0 <= e < num_blocks:
                if count < num_blocks:
                    stack[count] = e
                    count += 1
                else:
                    status |= 2
            elif e >= num_blocks:
                status |= 2
            table[b, pg] = -1
        if seq_lens is not None:
            seq_lens[b] = 0
    return count, status


def paged_scatter_rows(
    pool: torch.Tensor, block_table: torch.Tensor, b: int, t: int, rows: torch.Tensor
) -> None:
    """Write rows [Hkv, ...] of token t of sequence b into the pool."""
    page = pool.shape[2]
    pool[block_table[b, t // page].long(), :, t % page] = rows


# ------------------------------------------------------------------------- q/k preparation (norm + RoPE)
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3VLTextRMSNorm.forward (transformers/models/qwen3_vl/modeling_qwen3_vl.py:391-404): over the last
    axis in float32, x / sqrt(mean(x^2) + eps), cast back to x's dtype, times the weight (in that dtype)."""
    dtype = x.dtype
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    return weight * (xf * torch.rsqrt(var + eps)).to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """modeling_qwen3_vl.py:138-142: (x1, x2) -> (-x2, x1) over the halves of the last axis."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """apply_rotary_pos_emb (modeling_qwen3_vl.py:412-438) for one of q/k: x [B, H, S, D], cos/sin [B, S, D]
    broadcast over the heads; x * cos + rotate_half(x) * sin in x's dtype (each product and the sum rounded)."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return (x * cos) + (rotate_half(x) * sin)


def prepare_qk(q: torch.Tensor, k: torch.Tensor, q_w, k_w, eps: float, cos, sin):
    """What Qwen3VLTextAttention.forward does to the q/k projections before the cache update and the attention
    (modeling_qwen3_vl.py:481-486): q_norm / k_norm, then the rotary embedding. q [B, Hq, S, D], k [B, Hkv, S, D];
    a None weight or cos skips that step."""
    if q_w is not None:
        q = rms_norm(q, q_w, eps)
    if k_w is not None:
        k = rms_norm(k, k_w, eps)
    if cos is not None:
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    return q, k
