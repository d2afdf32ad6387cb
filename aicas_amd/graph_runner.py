"""A decode step of the Qwen3-VL text model captured once as a HIP graph and replayed per generated token.

``AicasGraphDecodeRunner`` is the counterpart of the reference's ``CUDAGraphDecodeRunner``
(dujunbaoV1/evaluation_wrapper.py:210-389) with the same methods — ``load_prefix``, ``prepare_step``,
``maybe_capture``, ``replay`` — and static input / output buffers. What differs is underneath: the cache is an
:class:`~aicas_amd.kv_cache.AicasDecodeCache` whose per-sequence lengths live on the device, and every layer's
attention is one fused launch (q/k RMSNorm, rotary embedding, KV append, attention; :mod:`aicas_amd.fused_attention`)
that reads and bumps those lengths itself. The reference's ``GraphDecodeCache`` (:124-207) instead returns
fixed-size K/V and needs a host-maintained boolean visibility mask over the whole capacity; here nothing
about the length is baked into the graph, so one capture serves every step until the cache is full, for
contiguous, paged and fp8 caches alike.

The captured step is embed_tokens → rotary_emb → every decoder layer → norm → lm_head, as the reference's
``_run_step`` (:272-337) does for its non-native path; the argmax over the vocabulary runs right after each
replay, on the same stream, outside the graph: torch reduces a 152k-wide row across workgroups and zeroes
their semaphores with hipMemsetAsync, and a memset recorded into a graph has produced wrong results on
replays after the first on MI355X (a wrong token then indexes past the embedding table).
"""

from __future__ import annotations

import torch

from .fused_attention import install_fused_decode
from .kv_cache import AicasDecodeCache


class AicasGraphDecodeRunner:
    def __init__(self, language_model, lm_head, max_cache_len: int, batch_size: int = 1,
                 kv_dtype: torch.dtype | None = None, page_size: int | None = None, block_pool: bool = False):
        self.language_model = language_model
        self.lm_head = lm_head
        self.max_cache_len = int(max_cache_len)
        self.batch_size = int(batch_size)
        self.device = lm_head.weight.device
        self.cache = AicasDecodeCache(num_layers=len(language_model.layers), max_cache_len=self.max_cache_len,
                                      kv_dtype=kv_dtype, page_size=page_size, block_pool=block_pool)
        B = self.batch_size
        self.static_input_ids = torch.zeros((B, 1), dtype=torch.long, device=self.device)
        self.static_position_ids = torch.zeros((3, B, 1), dtype=torch.long, device=self.device)
        self.static_next_token = torch.zeros((B, 1), dtype=torch.long, device=self.device)
        self.static_logits: torch.Tensor | None = None  # [B, 1, vocab], written by every replay
        self.graph: torch.cuda.CUDAGraph | None = None
        self.is_captured = False
        self.capture_failed = False
        self._stream: torch.cuda.Stream | None = None

    # -- inputs ----------------------------------------------------------------------------------------
    def _has_compatible_step_shapes(self, input_ids: torch.Tensor, position_ids: torch.Tensor) -> bool:
        if not isinstance(input_ids, torch.Tensor) or tuple(input_ids.shape) != tuple(self.static_input_ids.shape):
            return False
        return isinstance(position_ids, torch.Tensor) and self._position_rows(position_ids) is not None

    def _position_rows(self, position_ids: torch.Tensor) -> torch.Tensor | None:
        """[3, B, 1] temporal/height/width positions from what the model accepts: [B, 1] text positions,
        [3, B, 1], or [4, B, 1] with the text row first (modeling_qwen3_vl.py Qwen3VLTextModel.forward)."""
        B = self.batch_size
        if position_ids.dim() == 2 and tuple(position_ids.shape) == (B, 1):
            return position_ids[None].expand(3, B, 1)
        if position_ids.dim() == 3 and tuple(position_ids.shape[1:]) == (B, 1):
            if position_ids.shape[0] == 3:
                return position_ids
            if position_ids.shape[0] == 4:
                return position_ids[1:]
        return None

    def load_prefix(self, past_key_values, prefix_len: int | None = None) -> bool:
        """Copy a prefill cache (any cache whose ``layers[i].keys`` / ``.values`` are ``[B, Hkv, L, D]``, e.g. HF's
        DynamicCache) into this runner's cache, keeping the first ``prefix_len`` tokens (all of them by default).
        Returns False when the layer count or the batch does not match (as the reference does, :185-207)."""
        layers = getattr(past_key_values, "layers", [])
        if len(layers) != len(self.cache.layers):
            return False
        for src, dst in zip(layers, self.cache.layers):
            keys, values = getattr(src, "keys", None), getattr(src, "values", None)
            if not isinstance(keys, torch.Tensor) or not isinstance(values, torch.Tensor):
                return False
            if keys.shape[0] != self.batch_size:
                return False
            n = keys.shape[2] if prefix_len is None else min(int(prefix_len), keys.shape[2])
            dst.load_prefix(keys[:, :, :n], values[:, :, :n])
        return True

    def prepare_step(self, input_ids: torch.Tensor, position_ids: torch.Tensor, cache_position=None,
                     visible_len=None) -> None:
        """Stage the next step's token ids ``[B, 1]`` and positions. ``cache_position`` and ``visible_len`` are
        accepted for the reference's signature and not needed: the lengths are on the device."""
        rows = self._position_rows(position_ids)
        if rows is None or tuple(input_ids.shape) != tuple(self.static_input_ids.shape):
            raise ValueError("input_ids must be [B, 1] and position_ids [B, 1], [3, B, 1] or [4, B, 1]")
        self.static_input_ids.copy_(input_ids)
        self.static_position_ids.copy_(rows)

    # -- the step --------------------------------------------------------------------------------------
    def _run_step(self) -> None:
        lm = self.language_model
        # token ids bounded on the device: a wrong id gives a wrong token, never a read past the embedding table
        ids = torch.clamp(self.static_input_ids, 0, lm.embed_tokens.num_embeddings - 1)
        hidden = lm.embed_tokens(ids)
        position_embeddings = lm.rotary_emb(hidden, self.static_position_ids)
        for layer in lm.layers:
            hidden = layer(hidden, attention_mask=None, position_ids=None, past_key_values=self.cache,
                           use_cache=True, position_embeddings=position_embeddings)
        hidden = lm.norm(hidden)
        logits = self.lm_head(hidden[:, -1:, :])
        if self.static_logits is None:
            self.static_logits = torch.empty_like(logits)
        self.static_logits.copy_(logits)

    def _pick(self) -> None:
        """Greedy choice from the step's logits (outside any graph)."""
        torch.argmax(self.static_logits[:, -1, :], dim=-1, keepdim=True, out=self.static_next_token)

    def _set_static(self, on: bool) -> None:
        # graph mode: every launch is bounded by the capacity and by the lengths at capture, which the replays
        # only grow (the planner then gives the grid, and the early-fetch kernel variant, of tight bounds)
        for layer in self.cache.layers:
            layer.static_bound = layer.view.max_tokens if on else None
            layer.static_min = min(layer.host_lens) if on else 0

    def maybe_capture(self, past_key_values, prefix_len: int | None, input_ids: torch.Tensor,
                      position_ids: torch.Tensor, cache_position=None, visible_len=None) -> bool:
        """Load the prefix, then run the step a few times eagerly on a side stream (lengths restored afterwards)
        and capture it. Returns False, capturing nothing, when the step shapes or the prefix do not fit this
        runner; any other failure raises."""
        if self.is_captured:
            return True
        if self.capture_failed:
            return False
        if not self._has_compatible_step_shapes(input_ids, position_ids) or not self.load_prefix(
                past_key_values, prefix_len):
            self.capture_failed = True
            return False
        install_fused_decode(self.language_model)
        self._set_static(True)
        self.prepare_step(input_ids, position_ids)
        saved = [(layer.seq_lens.clone(), list(layer.host_lens)) for layer in self.cache.layers]
        side = torch.cuda.Stream(device=self.device)
        self._stream = side  # kept: the workspace the graph uses belongs to this stream
        side.wait_stream(torch.cuda.current_stream())
        with torch.no_grad():
            with torch.cuda.stream(side):
                for _ in range(3):
                    self._run_step()
                    self._pick()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            # the warm-up steps appended rows past the prefix and bumped the lengths: take the lengths back
            # (the rows are overwritten by the real steps)
            for layer, (dev_lens, host_lens) in zip(self.cache.layers, saved):
                layer.seq_lens.copy_(dev_lens)
                layer.host_lens = host_lens
            torch.cuda.synchronize()
            # captured on the warm-up stream, whose workspace (one per stream) the warm-up has already sized
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                self._run_step()
        torch.cuda.synchronize()
        self.graph = graph
        self.is_captured = True
        return True

    def replay(self) -> torch.Tensor:
        """Run the captured step for the staged inputs (every layer appends the step's K/V and bumps its lengths
        on the device), then take the greedy token from its logits. Returns the static ``[B, 1]`` next-token
        buffer (overwritten by the next replay)."""
        if not self.is_captured:
            raise RuntimeError("nothing captured: call maybe_capture first")
        first = self.cache.layers[0]
        if max(first.host_lens) + 1 > first.view.max_tokens:
            raise RuntimeError(f"KV cache capacity exceeded: {max(first.host_lens)} + 1 > {first.view.max_tokens}")
        self.graph.replay()
        self._pick()
        for layer in self.cache.layers:
            layer.host_lens = [L + 1 for L in layer.host_lens]
        return self.static_next_token

    def release(self) -> None:
        """Leave graph mode: later eager calls on ``cache`` bound their launches by the host lengths again."""
        self._set_static(False)
