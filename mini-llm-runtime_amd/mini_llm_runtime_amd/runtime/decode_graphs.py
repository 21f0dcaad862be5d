"""The batched decode step of a causal LM replayed from HIP graphs.

The reference runs every decode step eagerly
(runtime/model_runner.py:execute_model_batch ->
TinyQwen2ForCausalLM.forward_decode_batch_with_cache, model/qwen2.py), so a
step costs the host time of issuing each layer's kernels: embedding, then per
layer RMSNorms, the QKV GEMM, the fused rotation + KV write + paged decode,
the output projection, the MLP and the residual adds, then the final norm and
the LM head, several hundred launches for a 24-layer model. At small batches
that host time is the whole step.

``DecodeGraphs`` records that step once per batch size into a HIP graph
(``torch.cuda.CUDAGraph``) over static input buffers and replays it. A call:

1. checks shapes, dtypes and devices, then the step's metadata against the
   cache with the model's own device-side checks
   (``Qwen2Attention._check_decode_metadata``: one host sync, the reference's
   messages and order, before anything is written);
2. copies token ids, positions, slots, context lengths and the block table
   into the batch size's static buffers on the current stream; the block
   table is right-padded with -1 to the fixed width ``max_blocks_per_seq``,
   so every replay's decode launch has the grid it was recorded with (the
   padded columns lie past every context and are never read);
3. replays the graph on the current stream.

The first call of a batch size records its graph: one eager step on the
runner's own stream (it sizes the decode workspace cached for that stream and
the model's concatenated QKV weights), then the capture on that stream with
the layers' metadata checks off (they were done in step 1). Nothing in the
recorded step allocates outside the graph's private pool or clears memory with
a memset: the decode workspace is returned to zero by the kernels themselves.

``record(batch_sizes)`` records graphs ahead of serving, as a server does at
start-up, so that no serving step pays for a recording: the dummy step of a
batch size puts row j at position j % block_size of a block the runner holds
(a context of j % block_size + 1 tokens), so every row writes its own slot and
nothing outside those blocks. The blocks come from the cache's allocator, as
a sequence of the runner's own, and go back with ``release()``.

The returned logits are the graph's static output, valid until the next call
with the same batch size. Graphs hold the weights and the cache as they were
recorded: replace a weight or the cache and call ``reset()``. Replays must not
overlap (one stream at a time): the graphs of one runner share its decode
workspace. A block table wider than ``max_blocks_per_seq`` runs the same step
eagerly (counted in ``eager_calls``).
"""

from __future__ import annotations

import torch

from ..model.qwen2_attention import Qwen2Attention
from .paged_kv_cache import PagedKVCache


class _Recorded:
    """Static inputs of one batch size and, once recorded, its graph."""

    def __init__(self, batch: int, width: int, device: torch.device) -> None:
        self.input_ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.position_ids = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.slot_mapping = torch.zeros(batch, dtype=torch.long, device=device)
        self.block_tables = torch.full((batch, width), -1, dtype=torch.long, device=device)
        self.context_lens = torch.ones(batch, dtype=torch.long, device=device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None

    def load(self, input_ids, position_ids, slot_mapping, block_tables, context_lens) -> None:
        width = block_tables.shape[1]
        self.input_ids.copy_(input_ids)
        self.position_ids.copy_(position_ids)
        self.slot_mapping.copy_(slot_mapping)
        self.context_lens.copy_(context_lens)
        self.block_tables[:, :width].copy_(block_tables)
        if width < self.block_tables.shape[1]:
            self.block_tables[:, width:].fill_(-1)


class DecodeGraphs:
    """HIP-graph replay of ``model.forward_decode_batch_with_cache`` on one
    paged KV cache (see the module docstring).

    model: a TinyQwen2ForCausalLM on a HIP device, in eval mode.
    kv_cache: the PagedKVCache the steps read and write.
    max_blocks_per_seq: the block-table width every graph is recorded with;
        the longest context a replay serves is max_blocks_per_seq * block_size.
    """

    def __init__(self, model, kv_cache: PagedKVCache, max_blocks_per_seq: int) -> None:
        device = kv_cache.device
        if device.type != "cuda":
            raise ValueError("DecodeGraphs needs the KV cache on a HIP device")
        if model.lm_head.weight.device != device:
            raise ValueError("model and KV cache must be on the same device")
        config = model.model.config
        if kv_cache.num_layers != config.num_hidden_layers:
            raise ValueError("KV cache num_layers must match model layers")
        if kv_cache.num_kv_heads != config.num_key_value_heads:
            raise ValueError("KV cache num_kv_heads must match model num_key_value_heads")
        if kv_cache.head_dim != config.head_dim:
            raise ValueError("KV cache head_dim must match model head_dim")
        if kv_cache.dtype != model.lm_head.weight.dtype:
            raise ValueError("KV cache dtype must match the model's dtype")
        if int(max_blocks_per_seq) <= 0:
            raise ValueError("max_blocks_per_seq must be > 0")
        self.model = model
        self.kv_cache = kv_cache
        self.width = int(max_blocks_per_seq)
        self.device = device
        self.stream = torch.cuda.Stream(device)  # default priority
        self._recorded: dict[int, _Recorded] = {}
        self._scratch_key = ("decode_graphs", id(self))
        self.captures = 0
        self.replays = 0
        self.eager_calls = 0

    def reset(self) -> None:
        """Drop every recorded graph (after a weight or the cache changed)."""
        self._recorded.clear()

    def record(self, batch_sizes) -> None:
        """Record the graphs of `batch_sizes` (those not recorded yet) on
        dummy steps over the runner's own blocks (see the module docstring)."""
        sizes = sorted({int(b) for b in batch_sizes})
        if not sizes or sizes[0] <= 0:
            raise ValueError("batch sizes must be > 0")
        sizes = [b for b in sizes if b not in self._recorded]
        if not sizes:
            return
        cache, bs = self.kv_cache, self.kv_cache.block_size
        if self._scratch_key not in cache.block_tables:
            cache.add_sequence(self._scratch_key)
        if not cache.reserve_tokens(self._scratch_key, sizes[-1]):
            raise RuntimeError("KV cache has no free blocks for the dummy decode rows")
        blocks = torch.tensor(cache.block_tables[self._scratch_key], dtype=torch.long)
        cache.k_cache[:, blocks.to(self.device)] = 0
        cache.v_cache[:, blocks.to(self.device)] = 0
        for batch in sizes:
            rows = torch.arange(batch)
            offsets = rows % bs
            tables = blocks[rows // bs][:, None]
            r = _Recorded(batch, self.width, self.device)
            r.load(torch.zeros(batch, 1, dtype=torch.long), offsets[:, None],
                   tables[:, 0] * bs + offsets, tables, offsets + 1)
            self._record(r)
            self._recorded[batch] = r

    def release(self) -> None:
        """Drop every recorded graph and return the dummy rows' blocks."""
        self.reset()
        if self._scratch_key in self.kv_cache.block_tables:
            self.kv_cache.free_sequence(self._scratch_key)

    def _check(self, input_ids, position_ids, slot_mapping, block_tables, context_lens) -> int:
        if input_ids.ndim != 2 or input_ids.shape[1] != 1:
            raise ValueError("input_ids must have shape [B, 1] for decode")
        batch = input_ids.shape[0]
        if batch == 0:
            raise ValueError("decode batch must not be empty")
        if input_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("input_ids must have dtype torch.int32 or torch.int64")
        if position_ids.shape != (batch, 1):
            raise ValueError("position_ids must have shape [B, 1]")
        if slot_mapping.shape != (batch,):
            raise ValueError("slot_mapping must have shape [B]")
        if context_lens.shape != (batch,):
            raise ValueError("context_lens must have shape [B]")
        if block_tables.ndim != 2 or block_tables.shape[0] != batch or block_tables.shape[1] == 0:
            raise ValueError("block_tables must have shape [B, max_num_blocks]")
        for name, tensor in (("input_ids", input_ids), ("position_ids", position_ids),
                             ("slot_mapping", slot_mapping), ("context_lens", context_lens),
                             ("block_tables", block_tables)):
            if tensor.device != self.device:
                raise ValueError(f"{name} must be on the KV cache's device")
            if name != "input_ids" and tensor.dtype != torch.long:
                raise ValueError(f"{name} must use torch.long dtype")
        return batch

    def _step(self, r: _Recorded) -> torch.Tensor:
        return self.model.forward_decode_batch_with_cache(
            r.input_ids, r.position_ids, self.kv_cache, r.slot_mapping, r.block_tables,
            r.context_lens, metadata_checked=True)

    def _record(self, r: _Recorded) -> None:
        current = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(current)
        with torch.cuda.stream(self.stream):
            self._step(r)  # eager: sizes this stream's decode workspace
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            r.logits = self._step(r)
        current.wait_stream(self.stream)
        r.graph = graph
        self.captures += 1

    def __call__(self, input_ids: torch.Tensor, position_ids: torch.Tensor,
                 slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                 context_lens: torch.Tensor) -> torch.Tensor:
        """[B, 1] token ids -> [B, 1, vocab_size] logits (the graph's output
        buffer, valid until the next call with this batch size)."""
        batch = self._check(input_ids, position_ids, slot_mapping, block_tables, context_lens)
        if block_tables.shape[1] > self.width:
            self.eager_calls += 1
            return self.model.forward_decode_batch_with_cache(
                input_ids, position_ids, self.kv_cache, slot_mapping, block_tables,
                context_lens)
        Qwen2Attention._check_decode_metadata(self.kv_cache, position_ids, slot_mapping,
                                              block_tables, context_lens)
        r = self._recorded.get(batch)
        if r is None:
            r = _Recorded(batch, self.width, self.device)
            r.load(input_ids, position_ids, slot_mapping, block_tables, context_lens)
            self._record(r)
            self._recorded[batch] = r
        else:
            r.load(input_ids, position_ids, slot_mapping, block_tables, context_lens)
        r.graph.replay()
        self.replays += 1
        return r.logits
