"""One generation request and its lifecycle (reference runtime/request.py:1-87).

States: WAITING -> PREFILLING (admitted by the scheduler) -> DECODING (after
the prompt's forward) -> FINISHED (EOS sampled or max_new_tokens reached).
``num_computed_tokens`` counts tokens whose K/V are in the cache; the last
sampled token is the pending input of the next decode step.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum


class RequestStatus(Enum):
    WAITING = "WAITING"
    PREFILLING = "PREFILLING"
    DECODING = "DECODING"
    FINISHED = "FINISHED"


class FinishReason(Enum):
    LENGTH = "LENGTH"
    EOS = "EOS"
    CANCELLED = "CANCELLED"
    ERROR = "ERROR"


@dataclass
class Request:
    request_id: str
    prompt_token_ids: list[int]
    max_new_tokens: int
    arrival_time: float

    output_token_ids: list[int] = field(default_factory=list)
    status: RequestStatus = RequestStatus.WAITING
    num_computed_tokens: int = 0
    # The scheduler aliases this to the KV cache's table for the request, so
    # blocks the cache reserves appear here without a copy.
    block_table: list[int] = field(default_factory=list)
    finish_reason: FinishReason | None = None

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def num_output_tokens(self) -> int:
        return len(self.output_token_ids)

    @property
    def num_all_tokens(self) -> int:
        return self.prompt_len + self.num_output_tokens

    @property
    def pending_token_id(self) -> int | None:
        """The last sampled token: the input of the next decode step."""
        return self.output_token_ids[-1] if self.output_token_ids else None

    @property
    def is_finished(self) -> bool:
        return self.status is RequestStatus.FINISHED

    def start_prefill(self) -> None:
        if self.status is not RequestStatus.WAITING:
            raise RuntimeError(
                f"Cannot start prefill for request {self.request_id} in status "
                f"{self.status}. Expected status: {RequestStatus.WAITING}")
        self.status = RequestStatus.PREFILLING

    def update_after_model(self, *, num_new_computed_tokens: int,
                           sampled_token_id: int | None,
                           reached_eos: bool = False) -> None:
        """Account one forward pass: its tokens are now cached, its sample is
        the newest output, and the request finishes on EOS or at its length
        limit (EOS takes precedence)."""
        if self.status not in (RequestStatus.PREFILLING, RequestStatus.DECODING):
            raise RuntimeError(
                f"Cannot update request {self.request_id} after model in status "
                f"{self.status}. Expected status: {RequestStatus.PREFILLING} or "
                f"{RequestStatus.DECODING}")
        self.num_computed_tokens += num_new_computed_tokens
        if sampled_token_id is not None:
            self.output_token_ids.append(sampled_token_id)
        if reached_eos:
            self.status, self.finish_reason = RequestStatus.FINISHED, FinishReason.EOS
        elif self.num_output_tokens >= self.max_new_tokens:
            self.status, self.finish_reason = RequestStatus.FINISHED, FinishReason.LENGTH
        else:
            self.status = RequestStatus.DECODING
