"""Continuous-batching scheduler (reference runtime/scheduler.py:1-162).

Policy, per ``schedule()`` call, under a token budget and a seat limit:

1. Running requests decode first, in admission order, one token each. A
   request whose next token needs a KV block the pool cannot supply sits the
   step out (it keeps its seat).
2. Then waiting requests are admitted first-come first-served while the
   budget and the seats last. Admission is all or nothing: the whole prompt is
   scheduled and its blocks reserved, or admission stops (no skipping ahead).

``update_after_model`` applies the sampled tokens and retires finished
requests, returning their blocks to the pool (prefills first, then decodes,
each in table order: the allocator reuses the last freed block first).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from .paged_kv_cache import PagedKVCache
from .request import Request, RequestStatus


@dataclass
class SchedulerOutput:
    prefill_requests: list[Request] = field(default_factory=list)
    decode_requests: list[Request] = field(default_factory=list)
    num_scheduled_tokens: dict[str, int] = field(default_factory=dict)

    def __post_init__(self) -> None:
        seen: set[str] = set()
        for kind, requests in (("prefill_requests", self.prefill_requests),
                               ("decode_requests", self.decode_requests)):
            for request in requests:
                if request.request_id in seen:
                    raise ValueError(f"Duplicate request {request.request_id} in {kind}")
                seen.add(request.request_id)
        counted = set(self.num_scheduled_tokens)
        if counted != seen:
            raise ValueError(
                "Mismatch between scheduled requests and num_scheduled_tokens keys. "
                f"Scheduled request IDs: {seen}, num_scheduled_tokens keys: {counted}")
        for request_id, count in self.num_scheduled_tokens.items():
            if count <= 0:
                raise ValueError(f"Number of scheduled tokens for request {request_id} "
                                 f"must be positive, got {count}")

    @property
    def scheduled_requests(self) -> list[Request]:
        return self.prefill_requests + self.decode_requests

    @property
    def total_num_scheduled_tokens(self) -> int:
        return sum(self.num_scheduled_tokens.values())

    @property
    def is_empty(self) -> bool:
        return not self.prefill_requests and not self.decode_requests


class Scheduler:
    def __init__(self, max_num_batched_tokens: int, max_num_seqs: int,
                 kv_cache: PagedKVCache | None = None) -> None:
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_seqs = max_num_seqs
        self.waiting: deque[Request] = deque()
        self.running: list[Request] = []
        self.request_ids: set[str] = set()
        if kv_cache is None:
            # A bookkeeping-only pool, as the reference builds (:69-76).
            kv_cache = PagedKVCache(num_layers=1, num_blocks=max_num_batched_tokens,
                                    block_size=max_num_batched_tokens, num_kv_heads=1,
                                    head_dim=1)
        self.kv_cache = kv_cache

    def add_request(self, request: Request) -> None:
        if request.request_id in self.request_ids:
            raise ValueError(f"Request {request.request_id} is already in the scheduler.")
        if request.status is not RequestStatus.WAITING:
            raise ValueError(f"Request {request.request_id} must be in WAITING status to be "
                             "added to the scheduler.")
        self.kv_cache.add_sequence(request.request_id)
        request.block_table = self.kv_cache.block_tables[request.request_id]
        self.waiting.append(request)
        self.request_ids.add(request.request_id)

    def schedule(self) -> SchedulerOutput:
        decode: list[Request] = []
        prefill: list[Request] = []
        counts: dict[str, int] = {}
        budget = self.max_num_batched_tokens

        for request in self.running:
            if budget <= 0:
                break
            # Every running request is DECODING here: admission happens after
            # this loop and update_after_model moves PREFILLING to DECODING.
            if not self.kv_cache.reserve_tokens(request.request_id,
                                                request.num_computed_tokens + 1):
                continue
            decode.append(request)
            counts[request.request_id] = 1
            budget -= 1

        seats = len(self.running)
        while self.waiting and budget > 0 and seats < self.max_num_seqs:
            head = self.waiting[0]
            if head.status is not RequestStatus.WAITING:
                raise ValueError(f"Request {head.request_id} must be in WAITING status to be "
                                 "scheduled.")
            if head.prompt_len > budget:
                break
            if not self.kv_cache.reserve_tokens(head.request_id, head.prompt_len):
                break
            self.waiting.popleft()
            head.start_prefill()
            prefill.append(head)
            counts[head.request_id] = head.prompt_len
            budget -= head.prompt_len
            seats += 1
            self.running.append(head)

        return SchedulerOutput(prefill_requests=prefill, decode_requests=decode,
                               num_scheduled_tokens=counts)

    def update_after_model(self, scheduler_output: SchedulerOutput,
                           sampled_token_ids: dict[str, int],
                           reached_eos_request_ids: set[str] | None = None) -> list[Request]:
        eos = reached_eos_request_ids or set()
        finished: list[Request] = []
        for request in scheduler_output.scheduled_requests:
            rid = request.request_id
            request.update_after_model(
                num_new_computed_tokens=scheduler_output.num_scheduled_tokens[rid],
                sampled_token_id=sampled_token_ids[rid],
                reached_eos=rid in eos)
            if request.is_finished:
                finished.append(request)
                self.running.remove(request)
                self.request_ids.remove(rid)
                self.kv_cache.free_sequence(rid)
        return finished
