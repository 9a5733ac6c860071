"""Numpy restatement of the reference's BatchPlan -> device-metadata packing.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference builds its attention metadata on the host with numpy/python
loops; these functions restate that algorithm with plain loops so they can
be read against the cited lines.  Every function takes a *plan* with the
reference's duck-typed surface (``plan.scheduled`` items with
``request_id`` / ``num_tokens_to_compute`` / ``is_prefill``,
``plan.get_request(rid)`` with ``all_token_ids`` / ``num_computed_tokens`` /
``num_prompt_tokens`` / ``num_prefill_tokens`` / ``spec_draft``, and
``plan.block_tables[rid]``), exactly what the reference's own tests fake.
"""
import numpy as np

INT32_MIN = np.iinfo(np.int32).min


def slot_mapping(block_table, positions, block_size):
    """``bt[pos // bs] * bs + pos % bs`` -- auto_infer/engine/token_layout.py:1-4."""
    return block_table[positions // block_size] * block_size + positions % block_size


def build(plan, block_size):
    """Eager runner packing -- auto_infer/worker/model_runner.py:111-188.

    Returns the values the reference's ``_build`` puts into ForwardContext
    plus its two side outputs:
    token_ids int64 (T,), positions int64 (T,), slot_mapping int32 (T,),
    block_table int32 (B, max_blocks) zero padded, cu_seqlens_q (list,
    cumulative, no leading 0), seqlens_kv (list, start + n per request),
    is_decode, sample_idx {rid: last flat row}, decode_splice [(row, rid)]
    for rows whose position is >= the prompt length.
    """
    tokens, positions, slots, rows = [], [], [], []
    cu_q, kv = [], []
    sample_idx, decode_splice = {}, []
    all_decode = True
    qacc = 0
    for sr in plan.scheduled:                              # :126-138
        req = plan.get_request(sr.request_id)
        n = sr.num_tokens_to_compute
        start = req.num_computed_tokens
        bt = list(plan.block_tables[sr.request_id])
        draft = list(getattr(req, "spec_draft", ()) or ())
        if draft and not sr.is_prefill:                    # :149-151 spec decode row
            ids = [req.all_token_ids[start]] + draft
        else:
            ids = [req.all_token_ids[p] for p in range(start, start + n)]
        for j in range(n):                                 # :146-166
            pos = start + j
            if pos >= req.num_prompt_tokens:
                decode_splice.append((len(tokens), sr.request_id))
            else:
                all_decode = False
            tokens.append(int(ids[j]))
            positions.append(pos)
            slots.append(bt[pos // block_size] * block_size + pos % block_size)
        qacc += n
        cu_q.append(qacc)
        kv.append(start + n)
        sample_idx[sr.request_id] = qacc - 1
        rows.append(bt)
    width = max((len(r) for r in rows), default=0)
    table = np.zeros((len(rows), width), dtype=np.int32)   # :143 zero padded
    for r, bt in enumerate(rows):
        table[r, :len(bt)] = bt
    return dict(
        token_ids=np.asarray(tokens, dtype=np.int64),
        positions=np.asarray(positions, dtype=np.int64),
        slot_mapping=np.asarray(slots, dtype=np.int32),
        block_table=table,
        cu_seqlens_q=cu_q,
        seqlens_kv=kv,
        is_decode=all_decode,
        sample_idx=sample_idx,
        decode_splice=decode_splice,
    )


class DirtyRows:
    """Shadow-compare block-table upload -- auto_infer/worker/staging.py:20-48.

    The shadow starts at INT32_MIN everywhere (decode_input_stager.py:70-71),
    so the first stage copies every row.  ``upload`` returns (rows, elements)
    copied, counting contiguous dirty spans row by row.
    """

    def __init__(self, shape):
        self.shadow = np.full(shape, INT32_MIN, dtype=np.int32)
        self.rows = 0
        self.elements = 0

    def upload(self, current, active_rows=None):
        dirty = np.any(current != self.shadow, axis=1)
        if active_rows is not None:
            dirty[active_rows:] = False
        copied = 0
        for r in range(current.shape[0]):
            if dirty[r]:
                self.shadow[r] = current[r]
                copied += 1
        self.rows += copied
        self.elements += copied * current.shape[1]
        return copied, copied * current.shape[1]


def decode_stage(plan, *, gear, max_blocks, block_size, scratch0, dirty=None,
                 scheduled=None):
    """Fixed-gear decode packing -- auto_infer/worker/decode_input_stager.py:74-123.

    Live row r: token all_token_ids[pos], pos = num_computed_tokens, slot by
    slot_mapping, block-table row, kv length pos + 1.  Padding rows
    (:100-106): block scratch0 + row, slot block * bs, bt[row, 0] = block,
    kv length 1, token 0, position 0.
    """
    scheduled = plan.scheduled if scheduled is None else scheduled
    if len(scheduled) > gear:
        raise ValueError(f"decode batch {len(scheduled)} exceeds gear {gear}")
    tid = np.zeros(gear, dtype=np.int64)
    pos = np.zeros(gear, dtype=np.int64)
    slots = np.zeros(gear, dtype=np.int32)
    bt = np.zeros((gear, max_blocks), dtype=np.int32)
    active = np.zeros(gear, dtype=bool)
    kv, order = [], []
    for row, item in enumerate(scheduled):
        req = plan.get_request(item.request_id)
        p = req.num_computed_tokens
        blocks = plan.block_tables[item.request_id]
        tid[row] = req.all_token_ids[p]
        pos[row] = p
        slots[row] = blocks[p // block_size] * block_size + p % block_size
        bt[row, :len(blocks)] = blocks
        active[row] = True
        kv.append(p + 1)
        order.append(item.request_id)
    for row in range(len(scheduled), gear):
        block = scratch0 + row
        slots[row] = block * block_size
        bt[row, 0] = block
        kv.append(1)
    copied = dirty.upload(bt) if dirty is not None else None
    return dict(token_ids=tid, positions=pos, slots=slots, block_table=bt,
                kv_lengths=kv, order=order, active_token_mask=active,
                copied=copied)


def spec_decode_stage(plan, *, gear, max_blocks, block_size, scratch0,
                      draft_depth, dirty=None, scheduled=None):
    """MTP-verify packing -- auto_infer/worker/decode_input_stager.py:304-373.

    query_width = draft_depth + 1 rows per request: tokens (last, *drafts),
    positions pos + offset, slots per position, kv length pos + width;
    padding request rows use scratch block scratch0 + row with positions
    arange(width) and slots block * bs + arange(width).
    """
    width = draft_depth + 1
    scheduled = plan.scheduled if scheduled is None else scheduled
    if len(scheduled) > gear:
        raise ValueError(
            f"spec decode batch {len(scheduled)} exceeds gear {gear}")
    n = gear * width
    tid = np.zeros(n, dtype=np.int64)
    pos = np.zeros(n, dtype=np.int64)
    slots = np.zeros(n, dtype=np.int32)
    drafts = np.zeros((gear, draft_depth), dtype=np.int64)
    bt = np.zeros((gear, max_blocks), dtype=np.int32)
    active = np.zeros(gear, dtype=np.int32)
    kv, order = [], []
    for row, item in enumerate(scheduled):
        rid = item.request_id
        req = plan.get_request(rid)
        p = req.num_computed_tokens
        blocks = plan.block_tables[rid]
        if len(req.spec_draft) != draft_depth:
            raise ValueError(
                f"request {rid} has {len(req.spec_draft)} drafts; "
                f"expected {draft_depth}")
        start = row * width
        tid[start:start + width] = (req.all_token_ids[p], *req.spec_draft)
        drafts[row] = req.spec_draft
        active[row] = 1
        for off in range(width):
            q = p + off
            pos[start + off] = q
            slots[start + off] = blocks[q // block_size] * block_size + q % block_size
        bt[row, :len(blocks)] = blocks
        kv.append(p + width)
        order.append(rid)
    for row in range(len(scheduled), gear):
        block = scratch0 + row
        start = row * width
        pos[start:start + width] = np.arange(width)
        slots[start:start + width] = block * block_size + np.arange(width)
        bt[row, 0] = block
        kv.append(width)
    copied = dirty.upload(bt) if dirty is not None else None
    return dict(token_ids=tid, positions=pos, slots=slots, block_table=bt,
                drafts=drafts, active_mask=active, kv_lengths=kv, order=order,
                copied=copied)


def continuation_stage(plan, scheduled, accepted, steps, *, gear, max_blocks,
                       block_size, scratch0, dirty=None):
    """Recurrent MTP continuation packing -- decode_input_stager.py:217-251.

    For each step s: live row position = num_computed + accepted + s, slot by
    slot_mapping, kv length position + 1; padding rows use scratch0 + row
    with position s and slot block * bs + s, kv length s + 1.
    """
    if len(scheduled) > gear or len(accepted) != len(scheduled):
        raise ValueError("continuation metadata does not match graph gear")
    bt = np.zeros((gear, max_blocks), dtype=np.int32)
    pos = np.zeros((len(steps), gear), dtype=np.int64)
    slots = np.zeros((len(steps), gear), dtype=np.int32)
    kv_by_step = []
    for si, step in enumerate(steps):
        kv = []
        for row, (item, acc) in enumerate(zip(scheduled, accepted)):
            req = plan.get_request(item.request_id)
            p = req.num_computed_tokens + acc + step
            blocks = plan.block_tables[item.request_id]
            pos[si, row] = p
            slots[si, row] = blocks[p // block_size] * block_size + p % block_size
            bt[row, :len(blocks)] = blocks
            kv.append(p + 1)
        for row in range(len(scheduled), gear):
            block = scratch0 + row
            pos[si, row] = step
            slots[si, row] = block * block_size + step
            bt[row, 0] = block
            kv.append(step + 1)
        kv_by_step.append(kv)
    copied = dirty.upload(bt) if dirty is not None else None
    return dict(positions=pos, slots=slots, block_table=bt,
                kv_by_step=kv_by_step, copied=copied)


def prefill_stage(plan, *, query_gear, sequence_gear, max_blocks, block_size,
                  scratch0, dirty=None):
    """Flattened-token prefill/mixed packing -- prefill_input_stager.py:72-162.

    Rows are packed request after request; cumulative query lengths; kv
    length start + n; sample rows only for requests whose chunk completes the
    prefill (start + n >= num_prefill_tokens).  Unused token-gear slack
    becomes one padding pseudo-sequence on scratch blocks scratch0 + k
    (:122-139) with kv length equal to the padding length.
    """
    scheduled = plan.scheduled
    real = sum(item.num_tokens_to_compute for item in scheduled)
    nseq = len(scheduled)
    if real > query_gear or nseq > sequence_gear:
        raise ValueError(
            f"batch ({real} tokens, {nseq} sequences) "
            f"exceeds prefill gear ({query_gear}, {sequence_gear})")
    if not scheduled:
        raise ValueError("prefill staging requires at least one sequence")
    tid = np.zeros(query_gear, dtype=np.int64)
    pos = np.zeros(query_gear, dtype=np.int64)
    slots = np.zeros(query_gear, dtype=np.int32)
    bt = np.zeros((sequence_gear, max_blocks), dtype=np.int32)
    sample_rows = np.zeros(sequence_gear, dtype=np.int64)
    active = np.zeros(query_gear, dtype=bool)
    active[:real] = True
    cu, kv, sample_order, splice_order, splice_rows = [], [], [], [], []
    q = 0
    for srow, item in enumerate(scheduled):
        rid = item.request_id
        req = plan.get_request(rid)
        start = req.num_computed_tokens
        blocks = plan.block_tables[rid]
        bt[srow, :len(blocks)] = blocks
        for off in range(item.num_tokens_to_compute):
            p = start + off
            tid[q] = req.all_token_ids[p]
            pos[q] = p
            slots[q] = blocks[p // block_size] * block_size + p % block_size
            q += 1
        cu.append(q)
        kv.append(start + item.num_tokens_to_compute)
        splice_order.append(rid)
        splice_rows.append(q - 1)
        if start + item.num_tokens_to_compute >= req.num_prefill_tokens:
            sample_rows[len(sample_order)] = q - 1
            sample_order.append(rid)
    padding = query_gear - real
    if padding:
        nblk = (padding + block_size - 1) // block_size
        for c in range(nblk):
            bt[nseq, c] = scratch0 + c
        for off in range(padding):
            block = scratch0 + off // block_size
            pos[q] = off
            slots[q] = block * block_size + off % block_size
            q += 1
        cu.append(query_gear)
        kv.append(padding)
    attn_seqs = nseq + int(bool(padding))
    copied = dirty.upload(bt, active_rows=attn_seqs) if dirty is not None else None
    return dict(token_ids=tid, positions=pos, slots=slots,
                block_table=bt[:attn_seqs], sample_rows=sample_rows,
                cumulative_query_lengths=cu, kv_lengths=kv,
                sample_order=sample_order, splice_order=splice_order,
                splice_rows=splice_rows, query_tokens=query_gear,
                real_query_tokens=real, sequence_count=nseq,
                active_token_mask=active, copied=copied)
