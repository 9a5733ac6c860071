"""Torch-CPU restatement of the MTP verify compaction.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``confirmed_layout`` -- auto_infer/spec_decode/layout.py:17-43: each
  request's 1 + accepted confirmed rows, packed in request order.
* ``target_compact`` -- the accept/compact block of
  GraphMtpRunner._target_body, auto_infer/worker/graph_mtp_runner.py:
  224-248, op for op.
"""
import torch


def confirmed_layout(accepted, draft_depth):
    """layout.py:17-43; returns (source_rows, query_lengths,
    cumulative_query_lengths, final_rows, active_tokens)."""
    counts = tuple(int(v) for v in accepted)
    if any(not 0 <= v <= draft_depth for v in counts):
        raise ValueError(f"MTP accepted counts must be between 0 and {draft_depth}")
    width = draft_depth + 1
    source, cumulative, final, active = [], [], [], 0
    for row, v in enumerate(counts):
        source.extend(range(width * row, width * row + v + 1))
        active += v + 1
        cumulative.append(active)
        final.append(active - 1)
    return tuple(source), tuple(1 + v for v in counts), tuple(cumulative), tuple(final), active


def target_compact(preds, drafts, active_mask, hidden, positions, slots, scratch_positions,
                   scratch_slots):
    """graph_mtp_runner.py:224-248 on CPU tensors.  Returns (accepted,
    compact_hidden, compact_tokens, compact_positions, compact_slots)."""
    g, width = preds.shape
    accepted = torch.cumprod((drafts == preds[:, :-1]).to(torch.int32), 1).sum(1)
    accepted = accepted * active_mask
    lengths = active_mask * (1 + accepted)
    starts = lengths.cumsum(0) - lengths
    dest = torch.arange(g * width)
    owner = ((dest[:, None] >= starts[None, :]).sum(1) - 1).clamp_min(0)
    offset = dest - starts[owner]
    source = (width * owner + offset).clamp(0, g * width - 1)
    valid = dest < lengths.sum()
    hid = torch.where(valid[:, None], hidden[source], torch.zeros_like(hidden))
    flat = preds.reshape(-1)
    tokens = torch.where(valid, flat[source], torch.zeros_like(dest))
    pos = torch.where(valid, positions[source], scratch_positions)
    slot = torch.where(valid, slots[source], scratch_slots)
    return accepted.to(torch.int64), hid, tokens, pos, slot
