"""Preallocated / paged / fp8 KV cache behind HF's Cache API, written by the HIP append kernel.

``AicasKVCacheLayer`` implements transformers' ``CacheLayerMixin`` contract (transformers/cache_utils.py:27-101:
``lazy_initialization(key_states, value_states)``, ``update``, ``get_mask_sizes(query_length)``,
``get_seq_length``, ``get_max_length``) and replaces HF ``DynamicLayer.update``'s ``torch.cat`` of the whole
cache per step (cache_utils.py:127-146) with an in-place append of the new rows, as the reference's
preallocated layers do (dujunbaoV1/evaluation_wrapper.py:54-112 and :124-184). ``AicasDecodeCache`` is the
``Cache`` holding one such layer per decoder layer; its ``update(key_states, value_states, layer_idx, ...)``
is HF's ``Cache.update`` (cache_utils.py:1349-1381).

Storage layouts:
  * contiguous (default): K/V ``[B, Hkv, capacity, D]`` in the states' dtype, or fp8 e4m3 with fp32 scales
    ``[B, Hkv, capacity]`` when ``kv_dtype=torch.float8_e4m3fn``;
  * paged (``page_size=16`` etc.): pools ``[num_blocks, Hkv, page_size, D]`` addressed through an int32
    block table ``[B, ceil(capacity / page_size)]`` (identity allocation unless one is given), in place of the
    reference's Python list page table (new KV cache/evaluation_wrapper.py:143-232).

Per-sequence lengths live on the device (``seq_lens``, int32 [B]); the append kernel bumps them in place,
so a decode step issues no host synchronisation. The host keeps its own copy (``host_lens``) for HF's
mask sizing and for the kernel's length bound.

What ``update`` returns: for a 16-bit contiguous cache, views ``[B, Hkv, L, D]`` of the storage (any HF
attention backend can read them); for fp8 or paged caches, the pools themselves, which only the aicas
decode kernel can read — except for the first prefill, where the fresh rows are returned as they came so
that the prefill attention (SDPA) sees them. Either way the returned key tensor carries the ``_aicas_kv``
descriptor consumed by ``gqa_decode_attention``.
"""

from __future__ import annotations

import math

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from . import ops
from .gqa_decode_attention import AicasKV


class AicasKVCacheLayer(CacheLayerMixin):
    is_compileable = False
    is_sliding = False

    def __init__(
        self,
        max_cache_len: int,
        kv_dtype: torch.dtype | None = None,
        page_size: int | None = None,
        num_blocks: int | None = None,
        block_table: torch.Tensor | None = None,
        block_pool: bool = False,
    ):
        super().__init__()
        if block_pool and (page_size is None or block_table is not None):
            raise ValueError("block_pool needs a paged cache whose block table it owns (page_size, no block_table)")
        if kv_dtype not in (None, torch.bfloat16, torch.float16, ops.FP8_DTYPE):
            raise ValueError(f"unsupported kv_dtype {kv_dtype}")
        if page_size is not None and (page_size <= 0 or page_size & (page_size - 1)):
            raise ValueError("page_size must be a power of two")
        self.max_cache_len = int(max_cache_len)
        self.kv_dtype = kv_dtype
        self.page_size = page_size
        self.num_blocks = num_blocks
        self._given_block_table = block_table
        self.use_block_pool = bool(block_pool)
        self.pool: ops.BlockPool | None = None  # device block allocator (block_pool=True)
        self.k_scale = None
        self.v_scale = None
        self.block_table = None
        self.seq_lens: torch.Tensor | None = None
        self.host_lens: list[int] = []
        self.view: ops.KVCacheView | None = None
        # graph mode: a captured step must stay valid while the lengths grow on the device, so its launches are
        # bounded by this (the capacity) instead of by host_lens, which the capturing runner advances itself
        self.static_bound: int | None = None
        self.static_min = 0  # graph mode: a lower bound on every length for the rest of the capture's life

    # -- CacheLayerMixin -------------------------------------------------------------------------------
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, H, _, D = key_states.shape
        self.dtype, self.device = key_states.dtype, key_states.device
        store = self.kv_dtype or key_states.dtype
        if store != ops.FP8_DTYPE and store != key_states.dtype:
            raise ValueError("a 16-bit cache stores the states' own dtype")
        fp8 = store == ops.FP8_DTYPE
        dev = self.device
        if self.page_size is None:
            shape = (B, H, self.max_cache_len, D)
            self.keys = torch.zeros(shape, dtype=store, device=dev)
            self.values = torch.zeros(shape, dtype=store, device=dev)
            if fp8:
                self.k_scale = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
                self.v_scale = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
        else:
            per_seq = math.ceil(self.max_cache_len / self.page_size)
            if self._given_block_table is not None:
                bt = self._given_block_table.to(device=dev, dtype=torch.int32).contiguous()
                if bt.shape[0] != B:
                    raise ValueError("block_table must have one row per sequence")
                nblocks = self.num_blocks or int(bt.max().item()) + 1
            elif self.use_block_pool:
                # pages get blocks from the device pool as appends reach them
                nblocks = self.num_blocks or B * per_seq
                bt = torch.full((B, per_seq), -1, dtype=torch.int32, device=dev)
                self.pool = ops.BlockPool(nblocks, dev)
            else:
                nblocks = self.num_blocks or B * per_seq
                if nblocks < B * per_seq:
                    raise ValueError("num_blocks too small for the identity block allocation")
                bt = torch.arange(B * per_seq, dtype=torch.int32, device=dev).view(B, per_seq)
            shape = (nblocks, H, self.page_size, D)
            self.keys = torch.zeros(shape, dtype=store, device=dev)
            self.values = torch.zeros(shape, dtype=store, device=dev)
            if fp8:
                self.k_scale = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
                self.v_scale = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
            self.block_table = bt
        self.view = ops.KVCacheView(self.keys, self.values, self.k_scale, self.v_scale, self.block_table)
        self.seq_lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.host_lens = [0] * B
        self.batch = B
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.shape[-2]
        was_empty = max(self.host_lens) == 0
        if max(self.host_lens) + n > self.view.max_tokens:
            raise RuntimeError(
                f"KV cache capacity exceeded: {max(self.host_lens)} + {n} > {self.view.max_tokens} tokens"
            )
        self._reserve(self.seq_lens, n)
        ops.kv_append(self.view, key_states, value_states, self.seq_lens, self.seq_lens)
        self.host_lens = [L + n for L in self.host_lens]
        return self._result(key_states, value_states, n, was_empty)

    def _reserve(self, positions: torch.Tensor, n: int) -> None:
        """With a block pool: blocks for the pages an append of n tokens at positions will touch."""
        if self.pool is not None:
            self.pool.alloc(self.block_table, positions, n, self.page_size)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        if not self.is_initialized:
            return 0
        return max(self.host_lens)

    def get_max_length(self) -> int:
        return self.view.max_tokens if self.view is not None else self.max_cache_len

    def reset(self) -> None:
        if self.is_initialized:
            if self.pool is not None:  # every sequence's blocks back to the pool (rows -1, lengths 0)
                self.pool.free(self.block_table, torch.ones(self.batch, dtype=torch.int32, device=self.device),
                               self.seq_lens)
            self.seq_lens.zero_()
            self.host_lens = [0] * self.batch

    def offload(self):
        raise NotImplementedError("AicasKVCacheLayer keeps its storage on the GPU")

    # Beam search and cache surgery reorder or cut HF's per-layer keys/values tensors; here the kernels read the
    # storage through a descriptor (device lengths, block table, scales) that those edits would leave behind, so
    # they are refused rather than half-applied. The reference turns its custom caches off for num_beams != 1
    # (dujunbaoV1/evaluation_wrapper.py:1670, :2592).
    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        raise NotImplementedError("AicasKVCacheLayer does not support beam search (reorder_cache); use num_beams=1")

    def crop(self, max_length: int) -> None:
        raise NotImplementedError("AicasKVCacheLayer does not support crop")

    def batch_repeat_interleave(self, repeats: int) -> None:
        raise NotImplementedError("AicasKVCacheLayer does not support batch_repeat_interleave")

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        raise NotImplementedError("AicasKVCacheLayer does not support batch_select_indices")

    def prefetch(self):
        return None

    # -- extras ----------------------------------------------------------------------------------------
    def load_prefix(self, keys: torch.Tensor, values: torch.Tensor, lens: list[int] | None = None):
        """Fill the cache from ``[B, Hkv, L, D]`` states (as the reference's GraphDecodeCacheLayer.load_prefix,
        dujunbaoV1/evaluation_wrapper.py:150-156), through the append kernel; ``lens`` (<= L) makes the
        batch ragged: sequence b keeps its first lens[b] rows."""
        if not self.is_initialized:
            self.lazy_initialization(keys, values)
        B, L = keys.shape[0], keys.shape[2]
        lens = [L] * B if lens is None else [int(x) for x in lens]
        if len(lens) != B or max(lens) > L or min(lens) < 0:
            raise ValueError("lens must give 0 <= lens[b] <= L for every sequence")
        if L > self.view.max_tokens:
            raise RuntimeError("prefix longer than the cache capacity")
        zeros = torch.zeros(B, dtype=torch.int32, device=self.device)
        if L > 0:
            self._reserve(zeros, L)
        ops.kv_append(self.view, keys, values, zeros)
        self.seq_lens.copy_(torch.tensor(lens, dtype=torch.int32), non_blocking=False)
        self.host_lens = lens

    def fused_decode_step(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, *, sm_scale: float,
                          qk: ops.QKPrologue | None = None) -> torch.Tensor:
        """One decode step of this layer in one launch: append ``k_new``/``v_new`` (``[B, Hkv, 1, D]``) at every
        sequence's length, bump the lengths on the device, and return the attention of ``q`` (``[B, Hq, 1, D]``)
        over the grown cache. With ``qk``, q and k_new are the projections' outputs, prepared (RMSNorm, rotary
        embedding) inside the launch as the model would."""
        if not self.is_initialized:
            raise RuntimeError("the cache layer is empty: prefill through update() first")
        self._reserve(self.seq_lens, 1)
        if self.static_bound is not None:
            # graph mode: nothing host-side may depend on the step (the runner checks capacity and advances
            # host_lens per replay); a token with no slot left is dropped and reported by the kernel
            return ops.decode_attention_append(q, self.view, k_new, v_new, self.seq_lens, sm_scale=sm_scale,
                                               max_seq_len=self.static_bound, min_seq_len=self.static_min,
                                               seq_lens_out=self.seq_lens, qk=qk)
        if max(self.host_lens) + 1 > self.view.max_tokens:
            raise RuntimeError(f"KV cache capacity exceeded: {max(self.host_lens)} + 1 > {self.view.max_tokens} tokens")
        out = ops.decode_attention_append(
            q, self.view, k_new, v_new, self.seq_lens, sm_scale=sm_scale, max_seq_len=max(self.host_lens) + 1,
            min_seq_len=min(self.host_lens), seq_lens_out=self.seq_lens, qk=qk)
        self.host_lens = [L + 1 for L in self.host_lens]
        return out

    def descriptor(self, workspace: torch.Tensor | None = None) -> AicasKV:
        uniform = len(set(self.host_lens)) == 1
        contiguous16 = self.page_size is None and not self.view.is_fp8
        return AicasKV(
            cache=self.view, seq_lens=self.seq_lens, max_seq_len=max(self.host_lens), batch=self.batch,
            min_seq_len=min(self.host_lens), workspace=workspace, dense=contiguous16 and uniform,
        )

    def _result(self, key_states, value_states, n, was_empty):
        meta = self.descriptor()
        if self.page_size is None and not self.view.is_fp8:
            L = meta.max_seq_len
            k, v = self.keys[:, :, :L, :], self.values[:, :, :L, :]
        elif n > 1 and was_empty:
            return key_states, value_states
        else:
            k, v = self.keys, self.values
        k._aicas_kv = meta
        v._aicas_kv = meta
        return k, v


class AicasDecodeCache(Cache):
    """One :class:`AicasKVCacheLayer` per decoder layer; pass as ``past_key_values`` to ``generate``.
    ``block_pool=True`` (paged caches) hands out pages from a device block pool as appends reach them, instead
    of a fixed identity block table; ``num_blocks`` sizes each layer's pool (default: enough for every sequence
    at full capacity)."""

    def __init__(
        self,
        num_layers: int | None = None,
        max_cache_len: int = 4096,
        kv_dtype: torch.dtype | None = None,
        page_size: int | None = None,
        config=None,
        block_pool: bool = False,
        num_blocks: int | None = None,
    ):
        if num_layers is None:
            if config is None:
                raise ValueError("give num_layers or config")
            text_config = config.get_text_config() if hasattr(config, "get_text_config") else config
            num_layers = text_config.num_hidden_layers
        layers = [
            AicasKVCacheLayer(max_cache_len=max_cache_len, kv_dtype=kv_dtype, page_size=page_size,
                              num_blocks=num_blocks, block_pool=block_pool)
            for _ in range(num_layers)
        ]
        super().__init__(layers=layers)
