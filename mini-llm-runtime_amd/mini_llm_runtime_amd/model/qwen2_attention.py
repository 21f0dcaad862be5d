"""Qwen2 attention with the paged KV cache, on the MI355X kernels.

The callers of the paged path in the reference (model/qwen2.py:258-767):
``Qwen2Attention`` and its pieces, with the same module names, construction
order (q_proj, v_proj, k_proj, so a seeded initialisation and a reference
state_dict both carry over), arguments, validation order and messages.

On the cache paths the step before attention is fused: one projection GEMM
over the concatenated [q | k | v] weights and biases, then one
``mlr_qkv_rope_write`` launch that rotates q and k at their positions and
writes k and v into the layer's cache (reference :605-613, :737-746), with
the reference's rounding; then the attention kernel:

- ``forward_decode_batch_with_cache`` validates the step's metadata with one
  host sync, then runs the fused step and the batched decode, replacing the
  write_slots + paged_attention_decode_batch_parallel pair (reference
  :608-621). For bf16 with head_dim 64 or 128 the rotation, the KV write and
  the decode are a single ``mlr_paged_decode_qkv`` launch after the
  projection; the results are the same bit for bit.
- ``forward_prefill_packed_with_cache`` (all prefill requests of a step) runs
  the fused step and one varlen prefill.
- ``forward_prefill_chunk_with_cache`` runs the fused step and the tiled
  chunk prefill (reference :737-767).
- ``forward_prefill_with_cache`` keeps PyTorch projections and rotation,
  writes the prompt's rows and attends over the fresh K/V with the chunk
  kernel at prefix 0, viewing them as a pool of 16-row blocks (the reference
  uses its dense attention here, :427-439).
- ``forward_decode_with_cache`` is the single-request decode (:441-536), on
  the fused step.

``forward`` (no cache) keeps the reference's dense PyTorch attention: it is
not on the paged path.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from ..kernels import paged_attention as kpa
from ..kernels import pre_attention as kpre
from ..runtime.paged_kv_cache import PagedKVCache


class Qwen2RotaryEmbedding(nn.Module):
    """cos/sin of the rotary embedding (reference model/qwen2.py:125-170)."""

    def __init__(self, head_dim: int, theta: float = 1_000_000.0) -> None:
        super().__init__()
        if head_dim <= 0 or head_dim % 2 != 0:
            raise ValueError("head_dim must be a positive even integer")
        if theta <= 0:
            raise ValueError("theta must be greater than 0")
        exponents = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
        self.head_dim = head_dim
        self.theta = theta
        self.register_buffer("inv_freq", 1.0 / (theta ** exponents), persistent=False)

    def forward(self, hidden_states: torch.Tensor,
                position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        if not hidden_states.is_floating_point():
            raise TypeError("hidden_states must be a floating-point tensor")
        if position_ids.ndim == 0:
            raise ValueError("position_ids must have at least one dimension")
        if tuple(hidden_states.shape[:-2]) != tuple(position_ids.shape):
            raise ValueError(
                "position_ids shape must match hidden_states dimensions before "
                f"the head dimensions, got {tuple(position_ids.shape)} and "
                f"{tuple(hidden_states.shape)}")
        if hidden_states.shape[-1] != self.head_dim:
            raise ValueError(
                "hidden_states last dimension must match head_dim "
                f"({self.head_dim}), got {hidden_states.shape[-1]}")
        angles = (position_ids.to(device=hidden_states.device, dtype=torch.float32)
                  .unsqueeze(-1) * self.inv_freq.to(hidden_states.device))
        angles = torch.cat((angles, angles), dim=-1)
        return angles.cos().to(hidden_states.dtype), angles.sin().to(hidden_states.dtype)


def rotate_half(hidden_states: torch.Tensor) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) over the two halves of the last dimension."""
    if hidden_states.shape[-1] % 2 != 0:
        raise ValueError("hidden_states last dimension must be even")
    first, second = hidden_states.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def apply_rotary_pos_emb(query: torch.Tensor, key: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotary embedding of Q and K in [..., heads, head_dim] layout
    (reference model/qwen2.py:183-209)."""
    if query.ndim < 2 or key.ndim < 2:
        raise ValueError("query and key must include head and head_dim dimensions")
    if query.shape[:-2] != key.shape[:-2]:
        raise ValueError("query and key token dimensions must match")
    if query.shape[-1] != key.shape[-1]:
        raise ValueError("query and key head_dim must match")
    expected = query.shape[:-2] + (query.shape[-1],)
    if cos.shape != expected or sin.shape != expected:
        raise ValueError(
            "cos and sin shape must match token dimensions plus head_dim, "
            f"expected {tuple(expected)}")
    cos = cos.to(query.dtype).unsqueeze(-2)
    sin = sin.to(query.dtype).unsqueeze(-2)
    return query * cos + rotate_half(query) * sin, key * cos + rotate_half(key) * sin


class Qwen2QKVProjection(nn.Module):
    """q/k/v projections with bias (reference model/qwen2.py:211-236)."""

    def __init__(self, config) -> None:
        super().__init__()
        self.hidden_size = config.hidden_size
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.hidden_dim = config.head_dim
        # Construction order q, v, k as in the reference: a seeded
        # initialisation then draws the same weights.
        self.q_proj = nn.Linear(config.hidden_size,
                                config.num_attention_heads * config.head_dim)
        self.v_proj = nn.Linear(config.hidden_size,
                                config.num_key_value_heads * config.head_dim)
        self.k_proj = nn.Linear(config.hidden_size,
                                config.num_key_value_heads * config.head_dim)

    def forward(self, hidden_states: torch.Tensor):
        if hidden_states.shape[-1] != self.hidden_size:
            raise ValueError("Unexpect input shape")
        lead = hidden_states.shape[:-1]
        query = self.q_proj(hidden_states).reshape(
            lead + (self.num_attention_heads, self.hidden_dim))
        key = self.k_proj(hidden_states).reshape(
            lead + (self.num_key_value_heads, self.hidden_dim))
        value = self.v_proj(hidden_states).reshape(
            lead + (self.num_key_value_heads, self.hidden_dim))
        return query, key, value


def _raise_first(checks) -> None:
    """Raise the first failing (flag, exception) pair; flags are host bools."""
    for failed, error in checks:
        if failed:
            raise error


class Qwen2Attention(nn.Module):
    def __init__(self, config) -> None:
        super().__init__()
        self.hidden_size = config.hidden_size
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.head_dim = config.head_dim
        self.scale = config.head_dim ** -0.5
        self.qkv_proj = Qwen2QKVProjection(config)
        self.rotary_embedding = Qwen2RotaryEmbedding(head_dim=config.head_dim,
                                                     theta=config.rope_theta)
        self.o_proj = nn.Linear(config.hidden_size, config.hidden_size, bias=False)
        self._qkv_cat_key = None
        self._qkv_cat = None

    # ------------------------------------------------------------------
    # Shared pieces
    # ------------------------------------------------------------------
    @staticmethod
    def _check_hidden(hidden_states: torch.Tensor, shape_text: str,
                      one_request: str | None) -> None:
        if hidden_states.ndim != 3:
            raise ValueError(f"hidden_states must have shape {shape_text}, "
                             f"got {tuple(hidden_states.shape)}")
        if one_request is not None and hidden_states.shape[0] != 1:
            raise ValueError(f"{one_request} currently supports exactly one request, "
                             f"got batch_size={hidden_states.shape[0]}")

    def _check_width_and_positions(self, hidden_states, position_ids, dims_name="sequence"):
        if hidden_states.shape[-1] != self.hidden_size:
            raise ValueError("hidden_states last dimension must match hidden_size "
                             f"({self.hidden_size}), got {hidden_states.shape[-1]}")
        if position_ids.shape != hidden_states.shape[:2]:
            raise ValueError(
                "position_ids shape must match hidden_states batch and "
                f"{dims_name} dimensions {tuple(hidden_states.shape[:2])}, "
                f"got {tuple(position_ids.shape)}")

    def _qkv_rope(self, hidden_states: torch.Tensor, position_ids: torch.Tensor):
        query, key, value = self.qkv_proj(hidden_states)
        cos, sin = self.rotary_embedding(query, position_ids)
        query, key = apply_rotary_pos_emb(query, key, cos, sin)
        return query, key, value

    def _qkv_weights(self) -> tuple[torch.Tensor, torch.Tensor]:
        """[q; k; v] projection weight and bias, concatenated once and rebuilt
        when a projection parameter is replaced or changed in place."""
        proj = self.qkv_proj
        parts = (proj.q_proj.weight, proj.k_proj.weight, proj.v_proj.weight,
                 proj.q_proj.bias, proj.k_proj.bias, proj.v_proj.bias)
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in parts)
        if key != self._qkv_cat_key:
            with torch.no_grad():
                weight = torch.cat(parts[:3], dim=0)
                bias = torch.cat(parts[3:], dim=0)
            self._qkv_cat, self._qkv_cat_key = (weight, bias), key
        return self._qkv_cat

    @staticmethod
    def _check_fused_inputs(hidden_states, position_ids, kv_cache, slot_mapping) -> None:
        """write_slots' type and device checks (runtime/paged_kv_cache.py:
        218-233), which the fused step must keep."""
        if slot_mapping.dtype not in (torch.int32, torch.int64):
            raise TypeError("slot_mapping must use an integer index dtype")
        cache_device = kv_cache.k_cache.device
        if slot_mapping.device != cache_device or hidden_states.device != cache_device:
            raise ValueError("slot_mapping and K/V must be on the KV cache device")

    def _fused_qkv_rope_write(self, hidden_2d: torch.Tensor, positions: torch.Tensor,
                              kv_cache: PagedKVCache, layer_idx: int,
                              slot_mapping: torch.Tensor) -> torch.Tensor:
        """Rotated q [T, Hq, D] of the tokens hidden_2d [T, hidden]; their
        rotated k and v are written to slot_mapping of the layer's cache.
        A cache of another dtype than the model (write_slots converts, as in
        the reference) or a dtype the kernel lacks takes the unfused path."""
        if hidden_2d.dtype != kv_cache.dtype or hidden_2d.dtype not in (
                torch.float32, torch.float16, torch.bfloat16):
            query, key, value = self._qkv_rope(hidden_2d.unsqueeze(0), positions.unsqueeze(0))
            kv_cache.write_slots(slot_mapping=slot_mapping, k=key[0], v=value[0],
                                 layer_idx=layer_idx, validate=False)
            return query[0]
        weight, bias = self._qkv_weights()
        qkv = torch.nn.functional.linear(hidden_2d, weight, bias)
        return kpre.qkv_rope_write(qkv, positions.to(torch.long), self.rotary_embedding.inv_freq,
                                   kv_cache, layer_idx, slot_mapping, self.num_attention_heads)

    # ------------------------------------------------------------------
    # No cache: the reference's dense attention (model/qwen2.py:282-370)
    # ------------------------------------------------------------------
    def forward(self, hidden_states: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must have shape "
                             "[batch_size, seq_len, hidden_size], "
                             f"got {tuple(hidden_states.shape)}")
        self._check_width_and_positions(hidden_states, position_ids)
        query, key, value = self._qkv_rope(hidden_states, position_ids)
        return self.o_proj(self._dense_attention(query, key, value))

    def _dense_attention(self, query, key, value):
        groups = self.num_key_value_groups
        if groups > 1:
            key = torch.repeat_interleave(key, groups, dim=-2)
            value = torch.repeat_interleave(value, groups, dim=-2)
        seq_len = query.shape[1]
        # Right-hand operands of the batched products are made contiguous.
        q = query.transpose(1, 2)
        k = key.transpose(1, 2).transpose(-2, -1).contiguous()
        v = value.transpose(1, 2).contiguous()
        scores = (q @ k) * self.scale
        causal = torch.tril(torch.ones(seq_len, seq_len, dtype=torch.bool, device=q.device))
        scores = scores.masked_fill(~causal, float("-inf"))
        softmax_dtype = (torch.float32 if scores.dtype in (torch.float16, torch.bfloat16)
                         else scores.dtype)
        weights = torch.softmax(scores, dim=-1, dtype=softmax_dtype).to(v.dtype)
        out = (weights @ v).transpose(1, 2)
        return out.reshape(out.shape[0], seq_len, self.hidden_size)

    # ------------------------------------------------------------------
    # Whole-prompt prefill (reference :372-439)
    # ------------------------------------------------------------------
    def forward_prefill_with_cache(self, hidden_states: torch.Tensor,
                                   position_ids: torch.Tensor, kv_cache: PagedKVCache,
                                   layer_idx: int, slot_mapping: torch.Tensor) -> torch.Tensor:
        self._check_hidden(hidden_states, "[1, seq_len, hidden_size]", "prefill with cache")
        self._check_width_and_positions(hidden_states, position_ids)
        if slot_mapping.ndim != 1:
            raise ValueError("slot_mapping must have shape [seq_len], "
                             f"got {tuple(slot_mapping.shape)}")
        if slot_mapping.shape[0] != hidden_states.shape[1]:
            raise ValueError("slot_mapping length must match sequence length "
                             f"({hidden_states.shape[1]}), got {slot_mapping.shape[0]}")
        query, key, value = self._qkv_rope(hidden_states, position_ids)
        kv_cache.write_slots(slot_mapping=slot_mapping, k=key.squeeze(0),
                             v=value.squeeze(0), layer_idx=layer_idx)
        out = self._attend_fresh(query.squeeze(0), key.squeeze(0), value.squeeze(0))
        return self.o_proj(out.reshape(1, -1, self.hidden_size))

    def _attend_fresh(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Causal attention of a whole prompt over its own K/V with the chunk
        kernel: the [S, Hkv, D] rows, padded to whole 16-row blocks, are a pool
        whose block table is 0, 1, 2, ..."""
        seq_len = q.shape[0]
        block = 16
        blocks = -(-seq_len // block)
        pool_k = k.new_zeros((blocks * block,) + tuple(k.shape[1:]))
        pool_v = v.new_zeros((blocks * block,) + tuple(v.shape[1:]))
        pool_k[:seq_len] = k
        pool_v[:seq_len] = v
        pool_k = pool_k.view(blocks, block, *k.shape[1:])
        pool_v = pool_v.view(blocks, block, *v.shape[1:])
        table = torch.arange(blocks, dtype=torch.long, device=q.device).unsqueeze(0)
        qsl = torch.tensor([0, seq_len], dtype=torch.long, device=q.device)
        ctx = torch.tensor([seq_len], dtype=torch.long, device=q.device)
        return kpa.paged_prefill_launch(q.contiguous(), pool_k, pool_v, table, qsl, ctx, seq_len)

    # ------------------------------------------------------------------
    # Single-request decode (reference :441-536)
    # ------------------------------------------------------------------
    def forward_decode_with_cache(self, hidden_states: torch.Tensor, position_ids: torch.Tensor,
                                  kv_cache: PagedKVCache, layer_idx: int,
                                  slot_mapping: torch.Tensor, block_table: list[int],
                                  context_len: int) -> torch.Tensor:
        self._check_hidden(hidden_states, "[1, 1, hidden_size]", "decode with cache")
        if hidden_states.shape[1] != 1:
            raise ValueError("decode with cache requires exactly one input token, "
                             f"got {hidden_states.shape[1]}")
        self._check_width_and_positions(hidden_states, position_ids)
        if slot_mapping.ndim != 1 or slot_mapping.shape[0] != 1:
            raise ValueError("slot_mapping must have shape [1] for decode, "
                             f"got {tuple(slot_mapping.shape)}")
        if context_len <= 0:
            raise ValueError("context_len must be greater than 0")
        position = int(position_ids.item())
        if position != context_len - 1:
            raise ValueError("decode position must equal context_len - 1, "
                             f"got position={position} and context_len={context_len}")
        self._check_fused_inputs(hidden_states, position_ids, kv_cache, slot_mapping)
        kv_cache.check_slots(slot_mapping)
        query = self._fused_qkv_rope_write(hidden_states[0], position_ids[0], kv_cache,
                                           layer_idx, slot_mapping)
        k_layer, v_layer = kv_cache.get_layer_cache(layer_idx)
        out = kpa.paged_attention_decode(q=query[0], k_cache=k_layer, v_cache=v_layer,
                                         block_table=block_table, seq_len=context_len,
                                         block_size=kv_cache.block_size)
        return self.o_proj(out.reshape(1, 1, self.hidden_size))

    # ------------------------------------------------------------------
    # Batched decode (reference :538-622)
    # ------------------------------------------------------------------
    def forward_decode_batch_with_cache(self, hidden_states: torch.Tensor,
                                        position_ids: torch.Tensor, kv_cache: PagedKVCache,
                                        layer_idx: int, slot_mapping: torch.Tensor,
                                        block_tables: torch.Tensor,
                                        context_lens: torch.Tensor, *,
                                        metadata_checked: bool = False) -> torch.Tensor:
        """Decode one token per request; context lengths include this token.

        metadata_checked: these same position, slot, block-table and length
        tensors already passed the device-side metadata checks against this
        cache (the model checks them in its first layer), so they are not
        checked again; the shape, dtype and device checks still run."""
        if hidden_states.ndim != 3 or hidden_states.shape[1:] != (1, self.hidden_size):
            raise ValueError("hidden_states must have shape [B, 1, hidden_size]")
        batch = hidden_states.shape[0]
        if batch == 0:
            raise ValueError("decode batch must not be empty")
        if position_ids.shape != (batch, 1):
            raise ValueError("position_ids must have shape [B, 1]")
        if slot_mapping.shape != (batch,):
            raise ValueError("slot_mapping must have shape [B]")
        if context_lens.shape != (batch,):
            raise ValueError("context_lens must have shape [B]")
        if block_tables.ndim != 2 or block_tables.shape[0] != batch:
            raise ValueError("block_tables must have shape [B, max_num_blocks]")
        for name, tensor in (("position_ids", position_ids), ("slot_mapping", slot_mapping),
                             ("context_lens", context_lens), ("block_tables", block_tables)):
            if tensor.dtype != torch.long:
                raise ValueError(f"{name} must use torch.long dtype")
            if tensor.device != hidden_states.device:
                raise ValueError(f"{name} must be on the hidden_states device")
        if kv_cache.k_cache.device != hidden_states.device:
            raise ValueError("KV cache must be on the hidden_states device")
        if kv_cache.dtype != hidden_states.dtype:
            raise ValueError("KV cache dtype must match hidden_states dtype")
        if not metadata_checked:
            self._check_decode_metadata(kv_cache, position_ids, slot_mapping, block_tables,
                                        context_lens)
        # The metadata checks above are the ones write_slots and the decode
        # would repeat.
        if kpre.qkv_rope_decode_fusable(hidden_states.dtype, kv_cache, self.num_attention_heads):
            # Rotation, KV write and decode in one launch after the projection.
            weight, bias = self._qkv_weights()
            qkv = torch.nn.functional.linear(hidden_states[:, 0], weight, bias)
            out = kpre.qkv_rope_decode(qkv, self.rotary_embedding.inv_freq, kv_cache,
                                       layer_idx, slot_mapping, block_tables, context_lens,
                                       self.num_attention_heads)
            return self.o_proj(out.reshape(batch, 1, self.hidden_size))
        k_layer, v_layer = kv_cache.get_layer_cache(layer_idx)
        query = self._fused_qkv_rope_write(hidden_states[:, 0], position_ids[:, 0], kv_cache,
                                           layer_idx, slot_mapping)
        out = kpa.paged_decode_launch(query, k_layer, v_layer, block_tables, context_lens)
        return self.o_proj(out.reshape(batch, 1, self.hidden_size))

    @staticmethod
    def _check_decode_metadata(kv_cache, position_ids, slot_mapping, block_tables,
                               context_lens) -> None:
        """The reference's checks (:578-602), evaluated on the device in one
        pass with one host sync; the first failing one raises, in the
        reference's order, before anything is written."""
        bs, nblocks = kv_cache.block_size, kv_cache.num_blocks
        width = block_tables.shape[1]
        batch = block_tables.shape[0]
        positions = position_ids[:, 0]
        required = (context_lens + bs - 1) // bs
        columns = torch.arange(width, device=block_tables.device)
        used = columns[None, :] < required[:, None]
        bad_block = used & ((block_tables < 0) | (block_tables >= nblocks))
        # Clamped gather: only meaningful once the checks before it pass.
        col = (positions // bs).clamp(0, width - 1)
        rows = torch.arange(batch, device=block_tables.device)
        expected = block_tables[rows, col] * bs + positions % bs
        ordered = slot_mapping.sort().values
        flags = torch.stack([
            (context_lens <= 0).any(),
            (positions != context_lens - 1).any(),
            (required > width).any(),
            bad_block.any(),
            (slot_mapping != expected).any(),
            (ordered[1:] == ordered[:-1]).any() if batch > 1 else torch.zeros(
                (), dtype=torch.bool, device=slot_mapping.device),
        ]).tolist()
        _raise_first([
            (flags[0], ValueError("context_lens must be greater than 0")),
            (flags[1], ValueError("decode positions must equal context_lens - 1")),
            (flags[2], ValueError("block_tables have insufficient blocks for context_lens")),
            (flags[3], ValueError("block_tables contain an invalid physical block")),
            (flags[4], ValueError("slot_mapping must match block_tables and positions")),
            (flags[5], ValueError("decode requests must use distinct write slots")),
        ])

    # ------------------------------------------------------------------
    # Packed prefill of several requests (no counterpart in the reference's
    # attention; its runner calls forward_prefill_with_cache per request,
    # runtime/model_runner.py:254-266)
    # ------------------------------------------------------------------
    def forward_prefill_packed_with_cache(self, hidden_states: torch.Tensor,
                                          position_ids: torch.Tensor, kv_cache: PagedKVCache,
                                          layer_idx: int, slot_mapping: torch.Tensor,
                                          block_tables: torch.Tensor,
                                          query_start_loc: torch.Tensor,
                                          context_lens: torch.Tensor,
                                          max_query_len: int) -> torch.Tensor:
        """Prefill the packed tokens [T, hidden] of R requests: request r owns
        rows query_start_loc[r]:query_start_loc[r+1], which sit at positions
        context_lens[r] - len_r .. context_lens[r] - 1 and are written to
        slot_mapping before attending causally over the request's cached
        prefix and themselves (one mlr_kv_write, one mlr_paged_prefill).

        The caller has validated the metadata (TinyQwen2Model does, once per
        forward): positions follow the layout above, slots follow the block
        tables and are distinct."""
        if hidden_states.ndim != 2 or hidden_states.shape[1] != self.hidden_size:
            raise ValueError("hidden_states must have shape [num_tokens, hidden_size]")
        if position_ids.shape != hidden_states.shape[:1]:
            raise ValueError("position_ids must have shape [num_tokens]")
        self._check_fused_inputs(hidden_states, position_ids, kv_cache, slot_mapping)
        query = self._fused_qkv_rope_write(hidden_states, position_ids, kv_cache, layer_idx,
                                           slot_mapping)
        k_layer, v_layer = kv_cache.get_layer_cache(layer_idx)
        out = kpa.paged_prefill_launch(query, k_layer, v_layer,
                                       block_tables, query_start_loc, context_lens,
                                       max_query_len)
        return self.o_proj(out.reshape(-1, self.hidden_size))

    # ------------------------------------------------------------------
    # Chunk prefill (reference :624-767)
    # ------------------------------------------------------------------
    def forward_prefill_chunk_with_cache(self, hidden_states: torch.Tensor,
                                         position_ids: torch.Tensor, kv_cache: PagedKVCache,
                                         layer_idx: int, slot_mapping: torch.Tensor,
                                         block_table: list[int], prefix_len: int,
                                         context_len: int, tile_size: int) -> torch.Tensor:
        self._check_hidden(hidden_states, "[1, chunk_len, hidden_size]", "chunk prefill")
        chunk_len = hidden_states.shape[1]
        if chunk_len == 0:
            raise ValueError("chunk_len must be greater than 0")
        self._check_width_and_positions(hidden_states, position_ids, "chunk")
        if position_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("position_ids must use an integer dtype")
        if slot_mapping.ndim != 1 or slot_mapping.shape[0] != chunk_len:
            raise ValueError("slot_mapping must have shape [chunk_len], "
                             f"got {tuple(slot_mapping.shape)}")
        if prefix_len < 0:
            raise ValueError("prefix_len cannot be negative")
        if context_len != prefix_len + chunk_len:
            raise ValueError(
                "context_len must equal prefix_len + chunk_len, "
                f"got prefix_len={prefix_len}, chunk_len={chunk_len}, "
                f"and context_len={context_len}")
        if tile_size <= 0:
            raise ValueError("tile_size must be greater than 0")
        bs = kv_cache.block_size
        required = (context_len + bs - 1) // bs
        table = list(block_table)
        # Positions and slots are compared on the device, one host sync; the
        # table's own checks are host-side, as in the reference (:707-726).
        expected_pos = torch.arange(prefix_len, context_len, dtype=position_ids.dtype,
                                    device=position_ids.device).unsqueeze(0)
        pos_ok = torch.equal(position_ids, expected_pos)
        if not pos_ok:
            raise ValueError("position_ids must contain the contiguous global positions "
                             "from prefix_len through context_len - 1")
        if len(table) < required:
            raise ValueError("block_table does not contain enough blocks for context_len")
        if any(b < 0 or b >= kv_cache.num_blocks for b in table[:required]):
            raise ValueError("block_table contains an out-of-range physical block")
        positions = torch.arange(prefix_len, context_len, dtype=torch.long,
                                 device=slot_mapping.device)
        table_t = torch.as_tensor(table, dtype=torch.long, device=slot_mapping.device)
        expected_slots = table_t[positions // bs] * bs + positions % bs
        if not torch.equal(slot_mapping.to(torch.long), expected_slots):
            raise ValueError("slot_mapping does not match block_table for the chunk positions")
        self._check_fused_inputs(hidden_states, position_ids, kv_cache, slot_mapping)
        # write_slots' value checks (reference runtime/paged_kv_cache.py:235-239,
        # reached from model/qwen2.py:741-746): a table that repeats a block
        # inside the chunk's range passes the checks above but maps two
        # positions to one slot.
        kv_cache.check_slots(slot_mapping)
        query = self._fused_qkv_rope_write(hidden_states[0], position_ids[0], kv_cache,
                                           layer_idx, slot_mapping)
        k_layer, v_layer = kv_cache.get_layer_cache(layer_idx)
        out = kpa.paged_attention_prefill_chunk_tiled(
            q=query, k_cache=k_layer, v_cache=v_layer, block_table=table,
            prefix_len=prefix_len, context_len=context_len, block_size=bs,
            tile_size=tile_size)
        return self.o_proj(out.reshape(1, chunk_len, self.hidden_size))
