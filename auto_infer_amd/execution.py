"""The per-step input contract of the packing path.

Mirrors the fields the reference's packing code reads from its immutable
step snapshot (auto_infer/engine/execution.py:137-191 ``RequestView`` /
``BatchPlan``; auto_infer/engine/scheduler.py:9-14 ``ScheduledRequest``).
The packers in ``auto_infer_amd.packing`` only use this duck-typed surface,
so the reference's own ``BatchPlan`` objects are accepted unchanged.
"""
from dataclasses import dataclass, field
from types import MappingProxyType
from typing import Mapping


@dataclass(frozen=True)
class ScheduledRequest:
    request_id: str
    num_tokens_to_compute: int
    is_prefill: bool
    block_ids: tuple = ()


@dataclass(frozen=True)
class RequestView:
    request_id: str
    all_token_ids: tuple
    num_computed_tokens: int
    num_prompt_tokens: int
    num_prefill_tokens: int
    spec_draft: tuple = ()

    @property
    def num_tokens(self) -> int:
        return len(self.all_token_ids)


@dataclass(frozen=True)
class BatchPlan:
    scheduled: tuple
    requests: Mapping[str, RequestView]
    block_tables: Mapping[str, tuple]
    num_batched_tokens: int = 0

    @classmethod
    def make(cls, scheduled, requests, block_tables):
        scheduled = tuple(scheduled)
        return cls(scheduled, MappingProxyType(dict(requests)),
                   MappingProxyType({k: tuple(v) for k, v in block_tables.items()}),
                   sum(s.num_tokens_to_compute for s in scheduled))

    def get_request(self, request_id: str) -> RequestView:
        return self.requests[request_id]
