"""Qwen2 causal LM around the MI355X paged attention (reference
model/qwen2.py:14-123, 768-1240).

The modules, their names and construction order follow the reference, so a
reference state_dict loads unchanged and a seeded construction draws the same
random weights: ``TinyQwen2ForCausalLM`` = ``TinyQwen2Model`` (embed_tokens,
layers of ``Qwen2DecoderLayer``, norm) + lm_head (tied to the embedding when
the config says so). Each layer is pre-norm attention + pre-norm SwiGLU MLP
with residuals; RMSNorm keeps FP32 statistics for half-precision inputs.

On a HIP device each RMSNorm, the residual add before the post-attention
norm together with that norm, and the MLP's silu(gate) * up are one launch
each (kernels/layer_ops.py), with the gate and up projections as one GEMM;
the roundings are those of the PyTorch operations they replace.

The attention is ``Qwen2Attention`` on the HIP kernels. Besides the
reference's entry points, the model has ``forward_prefill_packed_with_cache``:
the prompts (or prompt chunks) of several requests in one packed forward,
which the runner uses for every prefill of a step.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels import layer_ops as kops
from ..runtime.paged_kv_cache import PagedKVCache
from .qwen2_attention import Qwen2Attention, _raise_first


@dataclass(frozen=True)
class TinyQwen2Config:
    vocab_size: int = 128
    hidden_size: int = 64
    intermediate_size: int = 128
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    max_position_embeddings: int = 128
    rope_theta: float = 1_000_000.0
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = False
    bos_token_id: int | None = None
    eos_token_id: int | None = None

    @classmethod
    def from_dict(cls, config_dict: dict[str, Any]) -> "TinyQwen2Config":
        """Build from a HF-style config dict, ignoring keys it does not know."""
        known = {f.name for f in fields(cls)}
        return cls(**{k: v for k, v in config_dict.items() if k in known})

    def __post_init__(self) -> None:
        for name in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                     "num_attention_heads", "num_key_value_heads",
                     "max_position_embeddings"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be greater than 0")
        if self.rope_theta <= 0:
            raise ValueError("rope_theta must be greater than 0")
        if self.rms_norm_eps <= 0:
            raise ValueError("rms_norm_eps must be greater than 0")
        if self.hidden_size % self.num_attention_heads != 0:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        if self.num_attention_heads % self.num_key_value_heads != 0:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        if self.head_dim % 2 != 0:
            raise ValueError("head_dim must be even for rotary embeddings")

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


class Qwen2RMSNorm(nn.Module):
    """x / sqrt(mean(x^2) + eps) * weight; statistics in FP32 for FP16/BF16
    inputs, and the product taken in the input dtype (reference :88-123)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        if hidden_size <= 0:
            raise ValueError("hidden_size must be greater than 0")
        if eps <= 0:
            raise ValueError("eps must be greater than 0")
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.shape[-1] != self.weight.shape[0]:
            raise ValueError("hidden_states last dimension must match hidden_size "
                             f"({self.weight.shape[0]}), got {hidden_states.shape[-1]}")
        dtype = hidden_states.dtype
        if kops.supported(hidden_states):
            # One launch (mlr_rms_norm), the same roundings as below.
            return kops.rms_norm(hidden_states, self.weight.to(dtype), self.variance_epsilon)
        stats = torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype
        x = hidden_states.to(stats)
        normalized = x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True)
                                     + self.variance_epsilon)
        return self.weight.to(dtype) * normalized.to(dtype)

    def forward_with_residual(self, hidden_states: torch.Tensor,
                              residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(self(residual + hidden_states), residual + hidden_states): the
        decoder layer's residual add and the norm after it, in one launch on a
        HIP device."""
        if hidden_states.shape != residual.shape:
            raise ValueError("hidden_states and residual must have the same shape")
        if hidden_states.shape[-1] != self.weight.shape[0]:
            raise ValueError("hidden_states last dimension must match hidden_size "
                             f"({self.weight.shape[0]}), got {hidden_states.shape[-1]}")
        dtype = hidden_states.dtype
        if (kops.supported(hidden_states) and residual.dtype == dtype
                and residual.device == hidden_states.device):
            return kops.rms_norm(hidden_states, self.weight.to(dtype), self.variance_epsilon,
                                 residual=residual)
        total = residual + hidden_states
        return self(total), total


class Qwen2MLP(nn.Module):
    """down(silu(gate(x)) * up(x)) (reference :768-792)."""

    def __init__(self, config: TinyQwen2Config) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)
        self._gate_up = None
        self._gate_up_key = None

    def _gate_up_weight(self) -> torch.Tensor:
        """[gate; up] weight, concatenated once and rebuilt when either
        parameter is replaced or changed in place."""
        parts = (self.gate_proj.weight, self.up_proj.weight)
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in parts)
        if key != self._gate_up_key:
            with torch.no_grad():
                self._gate_up = torch.cat(parts, dim=0)
            self._gate_up_key = key
        return self._gate_up

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if kops.supported(hidden_states):
            # One GEMM for both projections, then one launch for
            # silu(gate) * up (mlr_silu_mul, the same roundings as below).
            gate_up = F.linear(hidden_states, self._gate_up_weight())
            return self.down_proj(kops.silu_mul(gate_up))
        return self.down_proj(F.silu(self.gate_proj(hidden_states)) * self.up_proj(hidden_states))


class Qwen2DecoderLayer(nn.Module):
    """Pre-norm attention and MLP blocks with residuals (reference :794-940)."""

    def __init__(self, config: TinyQwen2Config) -> None:
        super().__init__()
        self.self_attn = Qwen2Attention(config)
        self.mlp = Qwen2MLP(config)
        self.input_layernorm = Qwen2RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = Qwen2RMSNorm(config.hidden_size,
                                                     eps=config.rms_norm_eps)

    def _block_parts(self, residual: torch.Tensor, delta: torch.Tensor | None, attend):
        """The layer on the input residual + delta (delta None: the input is
        residual), returned as (residual', delta') whose sum is the layer's
        output. Each residual add rides in the launch of the norm after it
        (Qwen2RMSNorm.forward_with_residual), with the bits of a separate add
        followed by the norm."""
        if delta is None:
            normed = self.input_layernorm(residual)
        else:
            normed, residual = self.input_layernorm.forward_with_residual(delta, residual)
        normed, residual = self.post_attention_layernorm.forward_with_residual(
            attend(normed), residual)
        return residual, self.mlp(normed)

    def _block(self, hidden_states: torch.Tensor, attend) -> torch.Tensor:
        residual, delta = self._block_parts(hidden_states, None, attend)
        return residual + delta

    def forward(self, hidden_states: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
        return self._block(hidden_states, lambda h: self.self_attn(h, position_ids))

    def forward_prefill_with_cache(self, hidden_states, position_ids, kv_cache, layer_idx,
                                   slot_mapping) -> torch.Tensor:
        return self._block(hidden_states, lambda h: self.self_attn.forward_prefill_with_cache(
            hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
            layer_idx=layer_idx, slot_mapping=slot_mapping))

    def forward_decode_with_cache(self, hidden_states, position_ids, kv_cache, layer_idx,
                                  slot_mapping, block_table, context_len) -> torch.Tensor:
        return self._block(hidden_states, lambda h: self.self_attn.forward_decode_with_cache(
            hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
            layer_idx=layer_idx, slot_mapping=slot_mapping, block_table=block_table,
            context_len=context_len))

    def forward_decode_batch_with_cache(self, hidden_states, position_ids, kv_cache,
                                        layer_idx, slot_mapping, block_tables,
                                        context_lens, *,
                                        metadata_checked: bool = False) -> torch.Tensor:
        return self._block(
            hidden_states, lambda h: self.self_attn.forward_decode_batch_with_cache(
                hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
                layer_idx=layer_idx, slot_mapping=slot_mapping, block_tables=block_tables,
                context_lens=context_lens, metadata_checked=metadata_checked))

    def forward_prefill_packed_with_cache(self, hidden_states, position_ids, kv_cache,
                                          layer_idx, slot_mapping, block_tables,
                                          query_start_loc, context_lens,
                                          max_query_len) -> torch.Tensor:
        return self._block(
            hidden_states, lambda h: self.self_attn.forward_prefill_packed_with_cache(
                hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
                layer_idx=layer_idx, slot_mapping=slot_mapping, block_tables=block_tables,
                query_start_loc=query_start_loc, context_lens=context_lens,
                max_query_len=max_query_len))


class TinyQwen2Model(nn.Module):
    """Embedding, decoder layers and the final norm (reference :943-1167)."""

    def __init__(self, config: TinyQwen2Config) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(
            [Qwen2DecoderLayer(config) for _ in range(config.num_hidden_layers)])
        self.norm = Qwen2RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    # Shared argument checks -------------------------------------------------
    @staticmethod
    def _check_ids(input_ids: torch.Tensor) -> None:
        if input_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("input_ids must have dtype torch.int32 or torch.int64, "
                            f"got {input_ids.dtype}")

    def _check_cache(self, kv_cache: PagedKVCache) -> None:
        if kv_cache.num_layers != len(self.layers):
            raise ValueError("KV cache num_layers must match model layers "
                             f"({len(self.layers)}), got {kv_cache.num_layers}")
        if kv_cache.num_kv_heads != self.config.num_key_value_heads:
            raise ValueError("KV cache num_kv_heads must match model num_key_value_heads "
                             f"({self.config.num_key_value_heads}), "
                             f"got {kv_cache.num_kv_heads}")
        if kv_cache.head_dim != self.config.head_dim:
            raise ValueError("KV cache head_dim must match model head_dim "
                             f"({self.config.head_dim}), got {kv_cache.head_dim}")

    def _run(self, input_ids: torch.Tensor, attend_of) -> torch.Tensor:
        """Embedding, the layers and the final norm; attend_of(layer, i) is
        layer i's attention on its normed input. Between layers the hidden
        state travels as (residual, delta), whose sum it is: the add of a
        layer's MLP output rides in the next norm's launch, with the bits of a
        separate add (Qwen2DecoderLayer._block_parts)."""
        residual, delta = self.embed_tokens(input_ids), None
        for layer_idx, layer in enumerate(self.layers):
            residual, delta = layer._block_parts(residual, delta, attend_of(layer, layer_idx))
        if delta is None:
            return self.norm(residual)
        return self.norm.forward_with_residual(delta, residual)[0]

    # Entry points -----------------------------------------------------------
    def forward(self, input_ids: torch.Tensor,
                position_ids: torch.Tensor | None = None) -> torch.Tensor:
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch_size, seq_len], "
                             f"got {tuple(input_ids.shape)}")
        self._check_ids(input_ids)
        batch_size, seq_len = input_ids.shape
        if seq_len == 0:
            raise ValueError("input_ids sequence length must be greater than 0")
        if position_ids is None:
            position_ids = torch.arange(seq_len, dtype=torch.long,
                                        device=input_ids.device).expand(batch_size, -1)
        elif position_ids.shape != input_ids.shape:
            raise ValueError("position_ids shape must match input_ids shape "
                             f"{tuple(input_ids.shape)}, got {tuple(position_ids.shape)}")
        return self._run(input_ids, lambda layer, i: lambda h: layer.self_attn(h, position_ids))

    def forward_prefill_with_cache(self, input_ids, position_ids, kv_cache,
                                   slot_mapping) -> torch.Tensor:
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [1, seq_len], "
                             f"got {tuple(input_ids.shape)}")
        if input_ids.shape[0] != 1:
            raise ValueError("prefill with cache currently supports exactly one request, "
                             f"got batch_size={input_ids.shape[0]}")
        if input_ids.shape[1] == 0:
            raise ValueError("input_ids sequence length must be greater than 0")
        self._check_ids(input_ids)
        if position_ids.shape != input_ids.shape:
            raise ValueError("position_ids shape must match input_ids shape "
                             f"{tuple(input_ids.shape)}, got {tuple(position_ids.shape)}")
        if slot_mapping.ndim != 1:
            raise ValueError("slot_mapping must have shape [seq_len], "
                             f"got {tuple(slot_mapping.shape)}")
        if slot_mapping.shape[0] != input_ids.shape[1]:
            raise ValueError("slot_mapping length must match sequence length "
                             f"({input_ids.shape[1]}), got {slot_mapping.shape[0]}")
        self._check_cache(kv_cache)
        return self._run(input_ids, lambda layer, i: lambda h:
                         layer.self_attn.forward_prefill_with_cache(
                             hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
                             layer_idx=i, slot_mapping=slot_mapping))

    def forward_decode_with_cache(self, input_ids, position_ids, kv_cache, slot_mapping,
                                  block_table, context_len) -> torch.Tensor:
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [1, 1] for decode, "
                             f"got {tuple(input_ids.shape)}")
        if tuple(input_ids.shape) != (1, 1):
            raise ValueError("decode with cache requires exactly one request and one token, "
                             f"got {tuple(input_ids.shape)}")
        self._check_ids(input_ids)
        if position_ids.shape != input_ids.shape:
            raise ValueError("position_ids shape must match input_ids shape "
                             f"{tuple(input_ids.shape)}, got {tuple(position_ids.shape)}")
        if slot_mapping.ndim != 1 or slot_mapping.shape[0] != 1:
            raise ValueError("slot_mapping must have shape [1] for decode, "
                             f"got {tuple(slot_mapping.shape)}")
        if context_len <= 0:
            raise ValueError("context_len must be greater than 0")
        position = int(position_ids.item())
        if position != context_len - 1:
            raise ValueError("decode position must equal context_len - 1, "
                             f"got position={position} and context_len={context_len}")
        if len(block_table) < -(-context_len // kv_cache.block_size):
            raise ValueError("block_table does not contain enough blocks for context_len")
        self._check_cache(kv_cache)
        return self._run(input_ids, lambda layer, i: lambda h:
                         layer.self_attn.forward_decode_with_cache(
                             hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
                             layer_idx=i, slot_mapping=slot_mapping, block_table=block_table,
                             context_len=context_len))

    def forward_decode_batch_with_cache(self, input_ids, position_ids, kv_cache, slot_mapping,
                                        block_tables, context_lens, *,
                                        metadata_checked: bool = False) -> torch.Tensor:
        """[B, 1] token ids -> [B, 1, hidden_size].

        metadata_checked: the caller already ran the device-side metadata
        checks on these position, slot, block-table and length tensors against
        this cache (Qwen2Attention._check_decode_metadata), so no layer runs
        them and the call makes no host sync; the HIP-graph decode
        (runtime/step_graphs.py) checks before it copies its inputs in."""
        if input_ids.ndim != 2 or input_ids.shape[1] != 1:
            raise ValueError("input_ids must have shape [B, 1] for decode")
        if input_ids.shape[0] == 0:
            raise ValueError("decode batch must not be empty")
        if input_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("input_ids must have dtype torch.int32 or torch.int64")
        if position_ids.shape != input_ids.shape:
            raise ValueError("position_ids shape must match input_ids shape")
        if input_ids.device != self.embed_tokens.weight.device:
            raise ValueError("input_ids and model must be on the same device")
        if kv_cache.num_layers != len(self.layers):
            raise ValueError("KV cache num_layers must match model layers")
        if kv_cache.num_kv_heads != self.config.num_key_value_heads:
            raise ValueError("KV cache num_kv_heads must match model num_key_value_heads")
        if kv_cache.head_dim != self.config.head_dim:
            raise ValueError("KV cache head_dim must match model head_dim")
        # Every layer gets the same metadata tensors: the first layer checks
        # them (one host sync, before any cache write) and the others do not
        # repeat the checks.
        return self._run(input_ids, lambda layer, i: lambda h:
                         layer.self_attn.forward_decode_batch_with_cache(
                             hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
                             layer_idx=i, slot_mapping=slot_mapping, block_tables=block_tables,
                             context_lens=context_lens,
                             metadata_checked=metadata_checked or i > 0))

    def forward_prefill_packed_with_cache(self, input_ids: torch.Tensor,
                                          position_ids: torch.Tensor,
                                          kv_cache: PagedKVCache,
                                          slot_mapping: torch.Tensor,
                                          block_tables: torch.Tensor,
                                          query_start_loc: torch.Tensor,
                                          context_lens: torch.Tensor,
                                          max_query_len: int, *,
                                          metadata_checked: bool = False) -> torch.Tensor:
        """Packed prefill of R requests: [T] token ids -> [T, hidden_size].

        Request r owns tokens query_start_loc[r]:query_start_loc[r+1]
        (non-empty), at positions context_lens[r] - len_r .. context_lens[r] - 1
        of its block table (a whole prompt when the prefix is 0, else a chunk
        after a cached prefix). The metadata is checked once here, on the
        device with one host sync, before any layer writes the cache.

        metadata_checked: the caller already ran these checks
        (check_prefill_packed_inputs) on these tensors, so the call makes no
        host sync; the HIP-graph prefill (runtime/step_graphs.py) does."""
        if not metadata_checked:
            self.check_prefill_packed_inputs(input_ids, position_ids, kv_cache, slot_mapping,
                                             block_tables, query_start_loc, context_lens,
                                             max_query_len)
        return self._run(input_ids, lambda layer, i: lambda h:
                         layer.self_attn.forward_prefill_packed_with_cache(
                             hidden_states=h, position_ids=position_ids, kv_cache=kv_cache,
                             layer_idx=i, slot_mapping=slot_mapping, block_tables=block_tables,
                             query_start_loc=query_start_loc, context_lens=context_lens,
                             max_query_len=max_query_len))

    def check_prefill_packed_inputs(self, input_ids, position_ids, kv_cache, slot_mapping,
                                    block_tables, query_start_loc, context_lens,
                                    max_query_len) -> None:
        """The checks of forward_prefill_packed_with_cache: shapes, dtypes,
        devices and the cache first, then the metadata on the device (one host
        sync); raises before anything is written."""
        if input_ids.ndim != 1 or input_ids.shape[0] == 0:
            raise ValueError("input_ids must have shape [num_tokens] with num_tokens > 0")
        self._check_ids(input_ids)
        for name, tensor in (("position_ids", position_ids), ("slot_mapping", slot_mapping)):
            if tensor.shape != input_ids.shape:
                raise ValueError(f"{name} must have the shape of input_ids")
        num_requests = context_lens.shape[0]
        if context_lens.ndim != 1 or num_requests == 0:
            raise ValueError("context_lens must have shape [num_requests]")
        if query_start_loc.shape != (num_requests + 1,):
            raise ValueError("query_start_loc must have num_requests + 1 entries")
        if block_tables.ndim != 2 or block_tables.shape[0] != num_requests:
            raise ValueError("block_tables must have shape [num_requests, max_num_blocks]")
        for name, tensor in (("position_ids", position_ids), ("slot_mapping", slot_mapping),
                             ("block_tables", block_tables),
                             ("query_start_loc", query_start_loc),
                             ("context_lens", context_lens)):
            if tensor.dtype != torch.long:
                raise ValueError(f"{name} must use torch.long dtype")
            if tensor.device != input_ids.device:
                raise ValueError(f"{name} must be on the same device as input_ids")
        self._check_cache(kv_cache)
        self._check_packed_metadata(kv_cache, position_ids, slot_mapping, block_tables,
                                    query_start_loc, context_lens, max_query_len,
                                    input_ids.shape[0])

    @staticmethod
    def _check_packed_metadata(kv_cache, position_ids, slot_mapping, block_tables,
                               query_start_loc, context_lens, max_query_len,
                               num_tokens) -> None:
        bs, width = kv_cache.block_size, block_tables.shape[1]
        device = position_ids.device
        lens = query_start_loc[1:] - query_start_loc[:-1]
        # Request of each packed row: how many request ends lie at or before
        # it. A binary search stays in bounds whatever query_start_loc holds,
        # so a malformed one reaches its own check below instead of a
        # size mismatch inside a device kernel.
        owner = torch.searchsorted(
            query_start_loc[1:].contiguous(), torch.arange(num_tokens, device=device),
            right=True).clamp_(max=context_lens.shape[0] - 1)
        first = (context_lens - lens)[owner]
        offset = torch.arange(num_tokens, device=device) - query_start_loc[:-1][owner]
        required = (context_lens + bs - 1) // bs
        used = torch.arange(width, device=device)[None, :] < required[:, None]
        col = (position_ids // bs).clamp(0, max(width - 1, 0))
        expected = block_tables[owner, col] * bs + position_ids % bs
        ordered = slot_mapping.sort().values
        flags = torch.stack([
            query_start_loc[0] != 0,
            (lens <= 0).any(),
            query_start_loc[-1] != num_tokens,
            (lens > max_query_len).any(),
            (context_lens < lens).any(),
            (required > width).any(),
            (used & ((block_tables < 0) | (block_tables >= kv_cache.num_blocks))).any(),
            (position_ids != first + offset).any(),
            (slot_mapping != expected).any(),
            (ordered[1:] == ordered[:-1]).any(),
        ]).tolist()
        _raise_first([
            (flags[0], ValueError("query_start_loc must start at 0")),
            (flags[1], ValueError("query_start_loc must be strictly increasing")),
            (flags[2], ValueError("query_start_loc must end at the packed token count")),
            (flags[3], ValueError("max_query_len is smaller than a request's token count")),
            (flags[4], ValueError("context_lens must cover each request's tokens")),
            (flags[5], ValueError("block_tables have insufficient blocks for context_lens")),
            (flags[6], ValueError("block_tables contain an invalid physical block")),
            (flags[7], ValueError("position_ids must run from context_len - num_tokens "
                                  "to context_len - 1 for each request")),
            (flags[8], ValueError("slot_mapping must match block_tables and positions")),
            (flags[9], ValueError("packed tokens must use distinct write slots")),
        ])


class TinyQwen2ForCausalLM(nn.Module):
    """Backbone + lm_head (reference :1170-1240)."""

    def __init__(self, config: TinyQwen2Config) -> None:
        super().__init__()
        self.model = TinyQwen2Model(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids, position_ids=None) -> torch.Tensor:
        return self.lm_head(self.model(input_ids, position_ids))

    def logits(self, hidden_states: torch.Tensor, out: torch.Tensor | None = None
               ) -> torch.Tensor:
        """lm_head(hidden_states) for [N, hidden_size] rows. With `out`
        (a contiguous [N, vocab_size] tensor, e.g. a row range of a larger
        logits buffer) the GEMM writes its result there directly instead of
        into a new tensor that the caller would then copy: the same product
        as the module's forward (lm_head has no bias). The GEMM library may
        pick its kernel by the operands' address alignment, so `out` is
        written directly only when it is 256-byte aligned like a new
        allocation; otherwise the product goes to a new tensor and is copied."""
        if out is None:
            return self.lm_head(hidden_states)
        if (out.shape != (hidden_states.shape[0], self.lm_head.out_features)
                or not out.is_contiguous()):
            raise ValueError("out must be a contiguous [N, vocab_size] tensor")
        if out.data_ptr() % 256:
            return out.copy_(self.lm_head(hidden_states))
        return torch.mm(hidden_states, self.lm_head.weight.t(), out=out)

    def forward_prefill_with_cache(self, input_ids, position_ids, kv_cache,
                                   slot_mapping) -> torch.Tensor:
        return self.lm_head(self.model.forward_prefill_with_cache(
            input_ids=input_ids, position_ids=position_ids, kv_cache=kv_cache,
            slot_mapping=slot_mapping))

    def forward_decode_with_cache(self, input_ids, position_ids, kv_cache, slot_mapping,
                                  block_table, context_len) -> torch.Tensor:
        return self.lm_head(self.model.forward_decode_with_cache(
            input_ids=input_ids, position_ids=position_ids, kv_cache=kv_cache,
            slot_mapping=slot_mapping, block_table=block_table, context_len=context_len))

    def forward_decode_batch_with_cache(self, input_ids, position_ids, kv_cache, slot_mapping,
                                        block_tables, context_lens, *,
                                        metadata_checked: bool = False) -> torch.Tensor:
        """[B, 1] -> [B, 1, vocab_size] logits."""
        return self.lm_head(self.model.forward_decode_batch_with_cache(
            input_ids=input_ids, position_ids=position_ids, kv_cache=kv_cache,
            slot_mapping=slot_mapping, block_tables=block_tables, context_lens=context_lens,
            metadata_checked=metadata_checked))

    def forward_prefill_packed_with_cache(self, input_ids, position_ids, kv_cache,
                                          slot_mapping, block_tables, query_start_loc,
                                          context_lens, max_query_len, *,
                                          metadata_checked: bool = False) -> torch.Tensor:
        """[T] -> [T, vocab_size] logits for the packed prefill tokens."""
        return self.lm_head(self.model.forward_prefill_packed_with_cache(
            input_ids, position_ids, kv_cache, slot_mapping, block_tables, query_start_loc,
            context_lens, max_query_len, metadata_checked=metadata_checked))
