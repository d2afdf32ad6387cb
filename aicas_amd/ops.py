"""Tensor-level wrappers around the C ABI: cache descriptors, KV append, decode attention, workspaces.

All work is enqueued on torch's current HIP stream of the tensors' device; nothing here synchronises the
host, so the calls can be captured in a HIP graph (``torch.cuda.CUDAGraph``) once the decode workspace has
been reserved for the largest shape the graph will see.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import AicasError, KVCacheDesc, check

_DTYPE_CODE = {
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float16: _lib.DTYPE_FP16,
    torch.float8_e4m3fn: _lib.DTYPE_FP8_E4M3,
}

FP8_DTYPE = torch.float8_e4m3fn
SUPPORTED_HEAD_DIMS = frozenset({16, 32, 64, 128})
SUPPORTED_GROUP_SIZES = frozenset({1, 2, 4, 8})


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise AicasError(_lib.ERR_UNSUPPORTED, f"dtype {dtype} is not supported") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: torch.Tensor | None) -> None:
    """Every tensor handed to a kernel must live on one GPU: a host pointer would be dereferenced on the
    device. Raised here, before the library is called."""
    devs = {t.device for t in tensors if t is not None}
    for d in devs:
        if d.type != "cuda":
            raise AicasError(_lib.ERR_INVALID, f"tensors must be on a GPU (got {d})")
    if len(devs) > 1:
        raise AicasError(_lib.ERR_INVALID, f"tensors must be on one device (got {sorted(map(str, devs))})")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


@dataclass
class KVCacheView:
    """Where the K/V rows of a cache live, in the form the kernels take (``aicas_kv_cache_t``).

    Contiguous: ``k``/``v`` are ``[B, Hkv, capacity, D]`` (any strides that keep rows 16-byte aligned,
    head_dim stride 1), ``block_table`` is None. Paged: ``k``/``v`` are pools ``[num_blocks, Hkv, page, D]``
    and ``block_table`` is ``[B, max_blocks]`` int32. fp8 caches carry fp32 scales shaped like the rows
    without the head_dim axis.
    """

    k: torch.Tensor
    v: torch.Tensor
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    block_table: torch.Tensor | None = None

    def __post_init__(self) -> None:
        if self.k.shape != self.v.shape or self.k.dtype != self.v.dtype:
            raise AicasError(_lib.ERR_INVALID, "K and V caches must have the same shape and dtype")
        if self.k.dim() != 4:
            raise AicasError(_lib.ERR_INVALID, "K/V caches must be 4-D")
        if self.k.stride(3) != 1 or self.v.stride(3) != 1:
            raise AicasError(_lib.ERR_INVALID, "K/V caches need a unit head_dim stride")
        if self.k.stride() != self.v.stride():
            raise AicasError(_lib.ERR_INVALID, "K and V caches must share strides")
        if self.is_fp8:
            if self.k_scale is None or self.v_scale is None:
                raise AicasError(_lib.ERR_INVALID, "fp8 caches need k_scale and v_scale")
            for s in (self.k_scale, self.v_scale):
                if s.dtype != torch.float32 or s.dim() != 3 or s.stride(2) != 1:
                    raise AicasError(_lib.ERR_INVALID, "fp8 scales must be float32 [blocks, Hkv, rows] with unit row stride")
            if self.k_scale.stride() != self.v_scale.stride():
                raise AicasError(_lib.ERR_INVALID, "k_scale and v_scale must share strides")
        if self.block_table is not None:
            bt = self.block_table
            if bt.dtype != torch.int32 or bt.dim() != 2 or bt.stride(1) != 1:
                raise AicasError(_lib.ERR_INVALID, "block_table must be int32 [B, max_blocks] with unit column stride")
            if bt.shape[1] != bt.stride(0):
                # the kernels take a row's width to be its stride (aicas_kv_cache_t has no width field): a
                # column-sliced table would let a length past the width read the next row's entries
                raise AicasError(_lib.ERR_INVALID, "block_table rows must be contiguous (width == row stride)")

    @property
    def is_fp8(self) -> bool:
        return self.k.dtype == FP8_DTYPE

    @property
    def paged(self) -> bool:
        return self.block_table is not None

    @property
    def num_kv_heads(self) -> int:
        return self.k.shape[1]

    @property
    def head_dim(self) -> int:
        return self.k.shape[3]

    @property
    def page_size(self) -> int:
        return self.k.shape[2]

    @property
    def max_tokens(self) -> int:
        """Tokens one sequence can hold."""
        if self.paged:
            return self.block_table.shape[1] * self.page_size
        return self.k.shape[2]

    @property
    def device(self) -> torch.device:
        return self.k.device

    def desc(self) -> KVCacheDesc:
        _require_gpu(self.k, self.v, self.k_scale, self.v_scale, self.block_table)
        d = KVCacheDesc()
        d.k = self.k.data_ptr()
        d.v = self.v.data_ptr()
        d.k_scale = _ptr(self.k_scale)
        d.v_scale = _ptr(self.v_scale)
        d.stride_blk = self.k.stride(0)
        d.stride_h = self.k.stride(1)
        d.stride_t = self.k.stride(2)
        if self.k_scale is not None:
            d.scale_stride_blk = self.k_scale.stride(0)
            d.scale_stride_h = self.k_scale.stride(1)
        d.page_size = self.k.shape[2]
        d.kv_dtype = dtype_code(self.k.dtype)
        if self.block_table is not None:
            d.block_table = self.block_table.data_ptr()
            d.block_table_stride = self.block_table.stride(0)
            d.num_blocks = self.k.shape[0]
        else:
            d.num_blocks = self.k.shape[0]
        return d


def _check_rows(x: torch.Tensor, name: str) -> None:
    if x.dim() != 4 or x.stride(3) != 1:
        raise AicasError(_lib.ERR_INVALID, f"{name} must be [B, Hkv, n, D] with unit head_dim stride")


def kv_append(
    cache: KVCacheView,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    positions: torch.Tensor,
    seq_lens_out: torch.Tensor | None = None,
    status: torch.Tensor | None = None,
) -> None:
    """Write ``k_new``/``v_new`` ``[B, Hkv, n, D]`` at ``positions[b] .. +n-1`` of each sequence.

    ``seq_lens_out[b] = positions[b] + n`` is stored after the rows (it may be ``positions`` itself).
    fp8 caches quantize on write with one fp32 scale per (token, kv head).
    """
    _check_rows(k_new, "k_new")
    _check_rows(v_new, "v_new")
    if k_new.shape != v_new.shape or k_new.dtype != v_new.dtype:
        raise AicasError(_lib.ERR_INVALID, "k_new and v_new must match")
    B, H, n, D = k_new.shape
    if H != cache.num_kv_heads or D != cache.head_dim:
        raise AicasError(_lib.ERR_INVALID, f"new rows {tuple(k_new.shape)} do not fit cache heads/head_dim")
    if positions.dtype != torch.int32 or positions.numel() < B or not positions.is_contiguous():
        raise AicasError(_lib.ERR_INVALID, "positions must be a contiguous int32 tensor with one entry per sequence")
    if seq_lens_out is not None and (seq_lens_out.dtype != torch.int32 or not seq_lens_out.is_contiguous()):
        raise AicasError(_lib.ERR_INVALID, "seq_lens_out must be a contiguous int32 tensor")
    _require_gpu(cache.k, k_new, v_new, positions, seq_lens_out, status)
    desc = cache.desc()
    check(
        _lib.lib().aicas_kv_append(
            ctypes.byref(desc), dtype_code(k_new.dtype),
            k_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_new.stride(2),
            v_new.data_ptr(), v_new.stride(0), v_new.stride(1), v_new.stride(2),
            positions.data_ptr(), _ptr(seq_lens_out), _ptr(status),
            B, H, D, n, _stream(cache.device),
        )
    )


def kv_gather(
    cache: KVCacheView,
    seq_lens: torch.Tensor,
    out_len: int,
    dtype: torch.dtype | None = None,
    out: tuple[torch.Tensor, torch.Tensor] | None = None,
    status: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The first ``seq_lens[b]`` tokens of every sequence as dense ``[B, Hkv, out_len, D]`` K and V (rows past
    a sequence's length zero): a 16-bit cache copied as it is, an fp8 cache dequantised (code * scale in fp32,
    rounded once to ``dtype``, bf16 by default). What a prefill's attention reads from a paged or fp8 cache
    (new KV cache/evaluation_wrapper.py:198-245, ``_gather_paged_kv_cache``)."""
    if seq_lens.dtype != torch.int32 or not seq_lens.is_contiguous() or seq_lens.dim() != 1:
        raise AicasError(_lib.ERR_INVALID, "seq_lens must be a contiguous 1-D int32 tensor")
    B = seq_lens.numel()
    if cache.block_table is not None and cache.block_table.shape[0] < B:
        raise AicasError(_lib.ERR_INVALID, "the block table has fewer rows than seq_lens")
    if cache.block_table is None and cache.k.shape[0] < B:
        raise AicasError(_lib.ERR_INVALID, "the cache holds fewer sequences than seq_lens")
    if dtype is None:
        dtype = torch.bfloat16 if cache.is_fp8 else cache.k.dtype
    shape = (B, cache.num_kv_heads, int(out_len), cache.head_dim)
    if out is None:
        k_out = torch.empty(shape, dtype=dtype, device=cache.device)
        v_out = torch.empty(shape, dtype=dtype, device=cache.device)
    else:
        k_out, v_out = out
        for t, name in ((k_out, "k_out"), (v_out, "v_out")):
            if tuple(t.shape) != shape or t.dtype != dtype or t.stride(3) != 1:
                raise AicasError(_lib.ERR_INVALID, f"{name} must be {shape} {dtype} with unit head_dim stride")
        if k_out.stride() != v_out.stride():
            raise AicasError(_lib.ERR_INVALID, "k_out and v_out must share strides")
    _require_gpu(cache.k, seq_lens, k_out, v_out, status)
    desc = cache.desc()
    check(
        _lib.lib().aicas_kv_gather(
            ctypes.byref(desc), seq_lens.data_ptr(), B, cache.num_kv_heads, cache.head_dim, dtype_code(dtype),
            k_out.data_ptr(), v_out.data_ptr(), k_out.stride(0), k_out.stride(1), k_out.stride(2), int(out_len),
            _ptr(status), _stream(cache.device),
        )
    )
    return k_out, v_out


class BlockPool:
    """Free block ids of a paged cache's pool, kept on the device (``aicas_block_pool_t``): ``alloc`` gives the
    pages an append is about to touch a block, ``free`` takes a finished sequence's blocks back — both kernels
    on the current stream, so a decode step that needs a new page stays free of host synchronisation (and can be
    captured in a HIP graph). Replaces the reference's Python page table (new KV cache/evaluation_wrapper.py:141-190).
    """

    def __init__(self, num_blocks: int, device: torch.device | str = "cuda"):
        if num_blocks <= 0:
            raise AicasError(_lib.ERR_INVALID, "num_blocks must be positive")
        self.num_blocks = int(num_blocks)
        self.device = torch.device(device)
        self.free_blocks = torch.empty(self.num_blocks, dtype=torch.int32, device=self.device)
        self.free_count = torch.empty(1, dtype=torch.int32, device=self.device)
        _require_gpu(self.free_blocks)
        self.reset()

    def desc(self) -> _lib.BlockPoolDesc:
        return _lib.BlockPoolDesc(self.free_blocks.data_ptr(), self.free_count.data_ptr(), self.num_blocks)

    def reset(self) -> None:
        """Every block free again; pops hand out 0, 1, 2, ..."""
        check(_lib.lib().aicas_block_pool_init(ctypes.byref(self.desc()), _stream(self.device)))

    @staticmethod
    def _check_table(block_table: torch.Tensor) -> None:
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
            raise AicasError(_lib.ERR_INVALID, "block_table must be an int32 [batch, width] tensor with unit column stride")

    def alloc(self, block_table: torch.Tensor, positions: torch.Tensor, n_new: int, page_size: int,
              status: torch.Tensor | None = None) -> None:
        """Give every page that an append of ``n_new`` tokens at ``positions[b]`` touches a block where
        ``block_table`` holds a negative entry (in sequence order, each sequence's pages in page order)."""
        self._check_table(block_table)
        B = block_table.shape[0]
        if positions.dtype != torch.int32 or positions.numel() < B or not positions.is_contiguous():
            raise AicasError(_lib.ERR_INVALID, "positions must be a contiguous int32 tensor with one entry per sequence")
        _require_gpu(self.free_blocks, block_table, positions, status)
        check(_lib.lib().aicas_block_alloc(
            ctypes.byref(self.desc()), block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            positions.data_ptr(), int(n_new), B, int(page_size), _ptr(status), _stream(self.device)))

    def free(self, block_table: torch.Tensor, release: torch.Tensor, seq_lens: torch.Tensor | None = None,
             status: torch.Tensor | None = None) -> None:
        """Return the blocks of every sequence with ``release[b] != 0`` (int32) to the pool; their rows become -1
        and, if given, their ``seq_lens`` 0."""
        self._check_table(block_table)
        B = block_table.shape[0]
        if release.dtype != torch.int32 or release.numel() < B or not release.is_contiguous():
            raise AicasError(_lib.ERR_INVALID, "release must be a contiguous int32 tensor with one entry per sequence")
        if seq_lens is not None and (seq_lens.dtype != torch.int32 or not seq_lens.is_contiguous()):
            raise AicasError(_lib.ERR_INVALID, "seq_lens must be a contiguous int32 tensor")
        _require_gpu(self.free_blocks, block_table, release, seq_lens, status)
        check(_lib.lib().aicas_block_free(
            ctypes.byref(self.desc()), block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            release.data_ptr(), _ptr(seq_lens), B, _ptr(status), _stream(self.device)))

    def available(self) -> int:
        """Free blocks left (reads the device count: synchronises with the stream)."""
        return int(self.free_count.item())


@dataclass(frozen=True)
class DecodePlan:
    """A launch plan (``aicas_decode_plan``): a sequence of L tokens is spread over
    ``min(num_splits, ceil(L / tokens_per_split))`` splits; ``workspace_bytes`` is the workspace the launch needs.
    Pass the same ``tokens_per_split`` argument (0: automatic) to the launch as to the plan: the library plans
    the launch itself from the same inputs."""

    tokens_per_split: int
    num_splits: int
    workspace_bytes: int


def decode_plan(
    kv_dtype: torch.dtype,
    batch: int,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    max_seq_len: int,
    page_size: int = 0,
    tokens_per_split: int = 0,
) -> DecodePlan:
    tps = ctypes.c_int32()
    ns = ctypes.c_int32()
    wb = ctypes.c_size_t()
    check(
        _lib.lib().aicas_decode_plan(
            dtype_code(kv_dtype), batch, num_q_heads, num_kv_heads, head_dim, max_seq_len, page_size,
            tokens_per_split, ctypes.byref(tps), ctypes.byref(ns), ctypes.byref(wb),
        )
    )
    return DecodePlan(tps.value, ns.value, wb.value)


class Workspace:
    """Zero-initialised scratch for split partials and arrival counters, one per (device, stream).

    The kernels leave the counters at zero after every launch, so the buffer is reused as is. It only grows;
    call :meth:`reserve` before capturing a HIP graph so that no allocation happens during capture. A buffer
    that a larger one replaces is kept alive, not freed: a graph captured earlier holds its address and keeps
    writing partials and counters there on every replay, which must never land in memory the allocator has
    handed to another tensor.
    """

    _pool: dict[tuple[int, int], torch.Tensor] = {}
    _retired: list[torch.Tensor] = []

    @classmethod
    def get(cls, device: torch.device, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (idx, torch.cuda.current_stream(device).cuda_stream)
        buf = cls._pool.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 1 << 20)
            if buf is not None:
                size = max(size, 2 * buf.numel())
                cls._retired.append(buf)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            cls._pool[key] = buf
        return buf

    @classmethod
    def reserve(cls, device: torch.device, nbytes: int) -> torch.Tensor:
        return cls.get(device, nbytes)

    @classmethod
    def clear(cls) -> None:
        """Drop every workspace, retired ones included: only when no captured graph still launches on them."""
        cls._pool.clear()
        cls._retired.clear()


def decode_attention(
    q: torch.Tensor,
    cache: KVCacheView,
    *,
    sm_scale: float,
    seq_lens: torch.Tensor | None = None,
    max_seq_len: int | None = None,
    min_seq_len: int = 0,
    out: torch.Tensor | None = None,
    tokens_per_split: int = 0,
    workspace: torch.Tensor | None = None,
    status: torch.Tensor | None = None,
) -> torch.Tensor:
    """q ``[B, Hq, 1, D]`` (or ``[B, Hq, D]``) -> out of the same shape, attending to each sequence's cache.

    ``seq_lens`` (int32 ``[B]``, on device) gives per-sequence lengths; ``max_seq_len`` must bound them.
    ``min_seq_len`` (optional) is a lower bound on the lengths the caller may pass: when it keeps every split of a
    contiguous cache busy, the launch fetches its first rows before reading the lengths. Results never depend on
    it (a wrong bound costs bandwidth only). Without ``seq_lens`` every sequence has ``max_seq_len`` tokens
    (default: the cache capacity).
    """
    squeeze = q.dim() == 3
    q4 = q.unsqueeze(2) if squeeze else q
    if q4.dim() != 4 or q4.shape[2] != 1 or q4.stride(3) != 1:
        raise AicasError(_lib.ERR_INVALID, "q must be [B, Hq, 1, D] with unit head_dim stride")
    B, Hq, _, D = q4.shape
    Hkv = cache.num_kv_heads
    if D != cache.head_dim:
        raise AicasError(_lib.ERR_INVALID, f"q head_dim {D} != cache head_dim {cache.head_dim}")
    if max_seq_len is None:
        max_seq_len = cache.max_tokens
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or seq_lens.numel() < B or not seq_lens.is_contiguous():
            raise AicasError(_lib.ERR_INVALID, "seq_lens must be a contiguous int32 tensor with one entry per sequence")
    _require_gpu(cache.k, q4, seq_lens, out, workspace, status)
    if out is None:
        out = torch.empty((B, Hq, 1, D), dtype=q.dtype, device=q.device)
    out4 = out.unsqueeze(2) if out.dim() == 3 else out
    if out4.shape != (B, Hq, 1, D) or out4.stride(3) != 1 or out4.dtype != q.dtype:
        raise AicasError(_lib.ERR_INVALID, "out must be [B, Hq, 1, D] in q's dtype with unit head_dim stride")
    pl = decode_plan(
        cache.k.dtype, B, Hq, Hkv, D, max_seq_len, cache.page_size if cache.paged else 0, tokens_per_split
    )
    if workspace is None:
        workspace = Workspace.get(cache.device, pl.workspace_bytes)
    desc = cache.desc()
    check(
        _lib.lib().aicas_decode_attention(
            ctypes.byref(desc), dtype_code(q.dtype), q4.data_ptr(), q4.stride(0), q4.stride(1),
            out4.data_ptr(), out4.stride(0), out4.stride(1),
            _ptr(seq_lens), int(max_seq_len) if seq_lens is None else 0, int(min_seq_len), int(max_seq_len), B,
            Hq, Hkv, D, float(sm_scale),
            int(tokens_per_split), workspace.data_ptr(), workspace.numel(), _ptr(status),
            _stream(cache.device),
        )
    )
    return out


@dataclass
class QKPrologue:
    """The model's q/k preparation done inside :func:`decode_attention_append` (``aicas_qk_prologue_t``):
    RMSNorm over head_dim with ``q_norm_weight`` / ``k_norm_weight`` (``[D]``, q's dtype) and ``eps``, then the
    rotary embedding with ``cos`` / ``sin`` rows (``[B, D]`` or ``[B, 1, D]``, q's dtype) — what
    ``Qwen3VLTextAttention.forward`` does to the projections (transformers/models/qwen3_vl/
    modeling_qwen3_vl.py:481-486). Any part may be None. ``q_out`` (``[B, Hq, 1, D]``) receives q as prepared."""

    q_norm_weight: torch.Tensor | None = None
    k_norm_weight: torch.Tensor | None = None
    eps: float = 1e-6
    cos: torch.Tensor | None = None
    sin: torch.Tensor | None = None
    q_out: torch.Tensor | None = None

    def desc(self, B: int, Hq: int, D: int, dtype: torch.dtype) -> _lib.QKPrologueDesc:
        d = _lib.QKPrologueDesc()
        for name in ("q_norm_weight", "k_norm_weight"):
            w = getattr(self, name)
            if w is not None:
                if w.shape != (D,) or w.dtype != dtype or not w.is_contiguous():
                    raise AicasError(_lib.ERR_INVALID, f"{name} must be a contiguous [{D}] tensor in q's dtype")
                setattr(d, name, w.data_ptr())
        d.eps = float(self.eps)
        if (self.cos is None) != (self.sin is None):
            raise AicasError(_lib.ERR_INVALID, "give both cos and sin, or neither")
        if self.cos is not None:
            for name in ("cos", "sin"):
                t = getattr(self, name)
                t2 = t.reshape(t.shape[0], t.shape[-1]) if t.dim() == 3 and t.shape[1] == 1 else t
                if t2.shape != (B, D) or t2.dtype != dtype or t2.stride(1) != 1:
                    raise AicasError(_lib.ERR_INVALID, f"{name} must be [B, D] (or [B, 1, D]) in q's dtype")
                setattr(d, name, t2.data_ptr())
                setattr(d, f"{name}_stride_b", t2.stride(0))
        if self.q_out is not None:
            qo = self.q_out.unsqueeze(2) if self.q_out.dim() == 3 else self.q_out
            if qo.shape != (B, Hq, 1, D) or qo.dtype != dtype or qo.stride(3) != 1:
                raise AicasError(_lib.ERR_INVALID, "q_out must be [B, Hq, 1, D] in q's dtype")
            d.q_out, d.q_out_stride_b, d.q_out_stride_h = qo.data_ptr(), qo.stride(0), qo.stride(1)
        return d

    def tensors(self):
        return [t for t in (self.q_norm_weight, self.k_norm_weight, self.cos, self.sin, self.q_out) if t is not None]


def _append_call(q, cache, k_new, v_new, positions, *, sm_scale, max_seq_len, min_seq_len, seq_lens_out, out,
                 tokens_per_split, status, extra=()):
    """Checks shared by the fused append + attend entry points; returns the output tensor, the plan, the cache
    descriptor and the C-ABI arguments that follow it up to tokens_per_split, and the trailing (status,
    stream)."""
    squeeze = q.dim() == 3
    q4 = q.unsqueeze(2) if squeeze else q
    if q4.dim() != 4 or q4.shape[2] != 1 or q4.stride(3) != 1:
        raise AicasError(_lib.ERR_INVALID, "q must be [B, Hq, 1, D] with unit head_dim stride")
    B, Hq, _, D = q4.shape
    kn = k_new.squeeze(2) if k_new.dim() == 4 else k_new
    vn = v_new.squeeze(2) if v_new.dim() == 4 else v_new
    if kn.shape != (B, cache.num_kv_heads, D) or vn.shape != kn.shape or kn.stride(2) != 1 or vn.stride(2) != 1:
        raise AicasError(_lib.ERR_INVALID, "k_new/v_new must be [B, Hkv, 1, D] with unit head_dim stride")
    if kn.dtype != q.dtype or vn.dtype != q.dtype:
        raise AicasError(_lib.ERR_INVALID, "k_new/v_new must have q's dtype")
    if D != cache.head_dim:
        raise AicasError(_lib.ERR_INVALID, f"q head_dim {D} != cache head_dim {cache.head_dim}")
    if positions.dtype != torch.int32 or positions.numel() < B or not positions.is_contiguous():
        raise AicasError(_lib.ERR_INVALID, "positions must be a contiguous int32 tensor with one entry per sequence")
    if seq_lens_out is not None and (seq_lens_out.dtype != torch.int32 or not seq_lens_out.is_contiguous()):
        raise AicasError(_lib.ERR_INVALID, "seq_lens_out must be a contiguous int32 tensor")
    _require_gpu(cache.k, q4, kn, vn, positions, seq_lens_out, out, status, *extra)
    if out is None:
        out = torch.empty((B, Hq, 1, D), dtype=q.dtype, device=q.device)
    out4 = out.unsqueeze(2) if out.dim() == 3 else out
    if out4.shape != (B, Hq, 1, D) or out4.stride(3) != 1 or out4.dtype != q.dtype:
        raise AicasError(_lib.ERR_INVALID, "out must be [B, Hq, 1, D] in q's dtype with unit head_dim stride")
    pl = decode_plan(
        cache.k.dtype, B, Hq, cache.num_kv_heads, D, max_seq_len, cache.page_size if cache.paged else 0,
        tokens_per_split,
    )
    desc = cache.desc()
    head = (dtype_code(q.dtype), q4.data_ptr(), q4.stride(0), q4.stride(1),
            kn.data_ptr(), kn.stride(0), kn.stride(1), vn.data_ptr(), vn.stride(0), vn.stride(1),
            out4.data_ptr(), out4.stride(0), out4.stride(1),
            positions.data_ptr(), _ptr(seq_lens_out), int(min_seq_len), int(max_seq_len),
            B, Hq, cache.num_kv_heads, D, float(sm_scale), int(tokens_per_split))
    tail = (_ptr(status), _stream(cache.device))
    return out, pl, desc, head, tail


def decode_attention_append(
    q: torch.Tensor,
    cache: KVCacheView,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    positions: torch.Tensor,
    *,
    sm_scale: float,
    max_seq_len: int,
    min_seq_len: int = 0,
    seq_lens_out: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    tokens_per_split: int = 0,
    workspace: torch.Tensor | None = None,
    status: torch.Tensor | None = None,
    qk: QKPrologue | None = None,
) -> torch.Tensor:
    """One decode step in one launch: append ``k_new``/``v_new`` (``[B, Hkv, 1, D]`` or ``[B, Hkv, D]``) at
    ``positions[b]`` and attend over ``positions[b] + 1`` tokens. ``seq_lens_out[b] = positions[b] + 1`` (it
    may be ``positions`` itself). ``max_seq_len`` bounds ``positions[b] + 1``; ``min_seq_len`` (optional) is a
    lower bound on every ``positions[b]``, used as by :func:`decode_attention`. With ``qk``, q and ``k_new`` are
    the projections' outputs and are normalised and rotated as the model does before use
    (``aicas_decode_attention_append_qk``)."""
    extra = (workspace, *(qk.tensors() if qk is not None else ()))
    out, pl, desc, head, tail = _append_call(
        q, cache, k_new, v_new, positions, sm_scale=sm_scale, max_seq_len=max_seq_len, min_seq_len=min_seq_len,
        seq_lens_out=seq_lens_out, out=out, tokens_per_split=tokens_per_split, status=status, extra=extra)
    if workspace is None:
        workspace = Workspace.get(cache.device, pl.workspace_bytes)
    args = (*head, workspace.data_ptr(), workspace.numel(), *tail)
    if qk is None:
        check(_lib.lib().aicas_decode_attention_append(ctypes.byref(desc), *args))
    else:
        B, Hq, D = out.shape[0], out.shape[1], out.shape[-1]
        pro = qk.desc(B, Hq, D, q.dtype)
        check(_lib.lib().aicas_decode_attention_append_qk(ctypes.byref(desc), ctypes.byref(pro), *args))
    return out


# Bytes of the library's static scratch behind aicas_decode_attention_append_noalloc.
NOALLOC_SCRATCH_BYTES = 4 << 20


def decode_attention_append_noalloc(
    q: torch.Tensor,
    cache: KVCacheView,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    positions: torch.Tensor,
    *,
    out: torch.Tensor,
    sm_scale: float,
    max_seq_len: int,
    min_seq_len: int = 0,
    seq_lens_out: torch.Tensor | None = None,
    tokens_per_split: int = 0,
    status: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`decode_attention_append` for callers that cannot allocate: ``out`` must be given, and the split
    partials live in the library's static per-device scratch (``aicas_decode_attention_append_noalloc``), so
    neither this function nor the library allocates device memory. Launches whose workspace would exceed
    ``NOALLOC_SCRATCH_BYTES`` raise ``AicasError`` (ERR_WORKSPACE). Calls that may overlap on one device share
    the scratch and must be serialised by the caller."""
    if out is None:
        raise AicasError(_lib.ERR_INVALID, "decode_attention_append_noalloc needs a preallocated out")
    out, _, desc, head, tail = _append_call(
        q, cache, k_new, v_new, positions, sm_scale=sm_scale, max_seq_len=max_seq_len, min_seq_len=min_seq_len,
        seq_lens_out=seq_lens_out, out=out, tokens_per_split=tokens_per_split, status=status)
    check(_lib.lib().aicas_decode_attention_append_noalloc(ctypes.byref(desc), *head, *tail))
    return out
