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


@dataclass(frozen=True)
class DeviceTokenRef:
    """One row of a retained sampled-token tensor (reference
    auto_infer/engine/execution.py:60-65): ``owner.tokens[row]``."""
    owner: "DeviceTokenBatch"
    row: int


@dataclass(frozen=True)
class DeviceTokenBatch:
    """A step's sampled tokens, kept on the device, with the request order
    they were sampled in (reference execution.py:68-100).  The splices in
    ``auto_infer_amd.packing`` read ``tokens`` (int64, 1-D) and
    ``ref.row`` only, so the reference's own objects work unchanged."""
    tokens: object
    order: tuple
    row_by_request: Mapping[str, int]

    @classmethod
    def from_output(cls, tokens, order):
        order = tuple(order)
        if tokens.ndim != 1 or tokens.shape[0] != len(order):
            raise ValueError("sampled tokens and request order must have equal length")
        return cls.from_rows(tokens, order, range(len(order)))

    @classmethod
    def from_rows(cls, tokens, order, rows):
        order, rows = tuple(order), tuple(rows)
        if tokens.ndim != 1 or len(rows) != len(order):
            raise ValueError("sampled rows and request order must have equal length")
        if any(r < 0 or r >= tokens.shape[0] for r in rows):
            raise ValueError("sampled token row is out of bounds")
        by_rid = dict(zip(order, rows))
        if len(by_rid) != len(order):
            raise ValueError("sampled request order contains duplicate IDs")
        return cls(tokens, order, MappingProxyType(by_rid))

    def refs(self):
        return {rid: DeviceTokenRef(self, row) for rid, row in self.row_by_request.items()}
