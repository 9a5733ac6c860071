"""Packing of a BatchPlan into device attention metadata, on the GPU.

Host side of the ``aia_pack_rows`` kernel.  The reference packs every step
on the host (numpy loops + H2D copies of every buffer): the eager runner's
``_build`` (auto_infer/worker/model_runner.py:111-188) and the fixed-gear
stagers (worker/decode_input_stager.py:74-123, :304-373,
worker/prefill_input_stager.py:72-162).  Here the per-request state lives
on the device in a ``DeviceRequestTable`` (block ids and token ids per
request slot); a step uploads only what changed since the last step (new
blocks, new tokens, drafts) plus one 8-int descriptor per row, in ONE
host-to-device copy, and the kernel writes token_ids, positions,
slot_mapping, the zero-padded block table, cu_seqlens_q, seqlens_kv and
the sample rows.

The classes keep the reference's names, constructor arguments, outputs and
error messages (``DecodeInputStager``, ``SpecDecodeInputStager``,
``PrefillInputStager`` and ``DeviceBatchPacker.build`` for ``_build``).
Their ``copied_block_rows`` / ``copied_block_elements`` counters keep the
reference's meaning (worker/staging.py:30-48: gear block-table rows whose
contents changed since the last stage, times the row width); what this
design actually uploads (new block ids only) is counted by the shared
``DeviceRequestTable.uploaded_block_rows`` / ``uploaded_block_elements``.
"""
import types
from dataclasses import dataclass

import numpy as np

import torch

from auto_infer_amd import _native
from auto_infer_amd.attention.base import ForwardContext

try:        # native per-request host loop (auto_infer_amd/csrc/hostpack.cpp)
    from auto_infer_amd import _hostpack
except ImportError:
    _hostpack = None
from auto_infer_amd.ops import _check_device_tensor, _ptr, _stream

_ROW_INTS = 8
_HIP_ERROR = -1000      # _hostpack.upload_pack: statuses at or below are HIP runtime errors
# the current stream's raw handle without building a Stream object (about 2 us
# less per step than torch.cuda.current_stream); the public call where absent
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_PLAIN_MAPPINGS = (types.MappingProxyType, dict)


class DeviceRequestTable:
    """Per-request block ids and token ids, resident on the device.

    ``block_pool`` int32 [slots, max_blocks], ``token_pool`` int64
    [slots, max_len].  Slots are assigned on first sight of a request id and
    recycled least-recently-used when the table is full (or on
    ``release``).  Growth reallocates (amortised, like the reference's
    ``_ensure_capacity``, model_runner.py:99-109).
    """

    def __init__(self, device, max_slots=64, max_blocks=64, max_len=4096):
        self.device = torch.device(device)
        self.block_pool = torch.zeros(max_slots, max_blocks, dtype=torch.int32, device=self.device)
        self.token_pool = torch.zeros(max_slots, max_len, dtype=torch.int64, device=self.device)
        self._slot = {}           # rid -> slot
        self._blocks = {}         # rid -> tuple of synced block ids
        self._ntok = {}           # rid -> number of synced leading token ids
        self._last_use = {}       # rid -> step counter
        self._free = list(range(max_slots - 1, -1, -1))
        self._step = 0
        self._cap_blocks, self._cap_tokens = max_blocks, max_len
        # (token row width, token pool address, block row width, block pool
        # address) for the pack launch, refreshed when the pools grow
        self.pool_args = None
        self.uploaded_block_rows = 0
        self.uploaded_block_elements = 0

    # -- capacity ---------------------------------------------------------
    def _grow(self, slots=None, blocks=None, tokens=None):
        s0, b0 = self.block_pool.shape
        t0 = self.token_pool.shape[1]
        s1 = max(s0, slots or 0)
        b1 = max(b0, blocks or 0)
        t1 = max(t0, tokens or 0)
        if (s1, b1) != (s0, b0):
            bp = torch.zeros(s1, b1, dtype=torch.int32, device=self.device)
            bp[:s0, :b0] = self.block_pool
            self.block_pool = bp
        if (s1, t1) != (s0, t0):
            tp = torch.zeros(s1, t1, dtype=torch.int64, device=self.device)
            tp[:s0, :t0] = self.token_pool
            self.token_pool = tp
        if s1 > s0:
            self._free = list(range(s1 - 1, s0 - 1, -1)) + self._free
        self._cap_blocks, self._cap_tokens = b1, t1
        self.pool_args = None

    def release(self, rid):
        slot = self._slot.pop(rid, None)
        if slot is not None:
            self._free.append(slot)
        self._blocks.pop(rid, None)
        self._ntok.pop(rid, None)
        self._last_use.pop(rid, None)

    def _slot_for(self, rid, live):
        slot = self._slot.get(rid)
        if slot is None:
            if not self._free:
                idle = [r for r in self._slot if r not in live]
                if idle:
                    self.release(min(idle, key=lambda r: self._last_use[r]))
                else:
                    n = self.block_pool.shape[0]
                    self._grow(slots=2 * n)
            slot = self._free.pop()
            self._slot[rid] = slot
        self._last_use[rid] = self._step
        return slot

    # -- per-step sync ----------------------------------------------------
    def begin_step(self):
        self._step += 1
        return _Updates()

    def sync(self, upd, rid, req, blocks, upto, live, drafts=()):
        """Make slot rows hold ``blocks`` and token ids [0, upto) of the
        request (drafts written right after position upto - 1 - len(drafts)
        + 1, i.e. at the query positions they occupy); returns the slot."""
        slot = self._slot.get(rid)
        if slot is None:
            slot = self._slot_for(rid, live)
        else:
            self._last_use[rid] = self._step
        nb = len(blocks)
        if nb > self._cap_blocks:
            self._grow(blocks=max(nb, 2 * self._cap_blocks))
        if upto > self._cap_tokens:
            self._grow(tokens=max(upto, 2 * self._cap_tokens))
        prev = self._blocks.get(rid)
        if prev is not None and len(prev) == nb and prev == blocks:
            first = nb                                    # steady state: nothing new
        elif prev is not None and len(prev) <= nb and tuple(blocks[:len(prev)]) == prev:
            first = len(prev)
        else:
            first = 0
        if first < nb:
            upd.blk_slot.extend([slot] * (nb - first))
            upd.blk_idx.extend(range(first, nb))
            upd.blk_val.extend(blocks[first:nb])
            self.uploaded_block_rows += 1
            self.uploaded_block_elements += nb - first
            self._blocks[rid] = tuple(blocks)
        elif prev is None:
            self._blocks[rid] = tuple(blocks)
        ids = req.all_token_ids
        have = self._ntok.get(rid, 0)
        real_hi = min(upto - len(drafts), len(ids))
        if real_hi > have:
            upd.tok_slot.extend([slot] * (real_hi - have))
            upd.tok_idx.extend(range(have, real_hi))
            upd.tok_val.extend(ids[have:real_hi])
            self._ntok[rid] = real_hi
        if drafts:
            base = upto - len(drafts)
            upd.tok_slot.extend([slot] * len(drafts))
            upd.tok_idx.extend(range(base, base + len(drafts)))
            upd.tok_val.extend(drafts)
            # drafted positions are not real tokens: resync them later
            self._ntok[rid] = min(self._ntok.get(rid, 0), upto - len(drafts))
        return slot


class _Updates:
    """One step's changes: pool entries as (slot, column, value) -- flattened
    only at upload time, after any pool growth -- and the row descriptors."""

    def __init__(self):
        self.tok_slot, self.tok_idx, self.tok_val = [], [], []
        self.blk_slot, self.blk_idx, self.blk_val = [], [], []
        self.rows = []

    def row(self, slot, start, n, nblocks, base, q_off, zero_tokens, sample_slot):
        self.rows.append((slot, start, n, nblocks, base, q_off, zero_tokens, sample_slot))


def _stage_py(upd, h, token_width, block_width, offs):
    """Writes one step's uploads into the uint8 host array h at offs (token
    pool index / value int64, block pool index int64 / value int32, row
    descriptors int32): the specification of ``_hostpack.stage``."""
    nt, nb, nr = len(upd.tok_idx), len(upd.blk_idx), len(upd.rows)
    if nt:
        h[offs[0]:offs[0] + nt * 8].view(np.int64)[:] = (
            np.asarray(upd.tok_slot, dtype=np.int64) * token_width +
            np.asarray(upd.tok_idx, dtype=np.int64))
        h[offs[1]:offs[1] + nt * 8].view(np.int64)[:] = upd.tok_val
    if nb:
        h[offs[2]:offs[2] + nb * 8].view(np.int64)[:] = (
            np.asarray(upd.blk_slot, dtype=np.int64) * block_width +
            np.asarray(upd.blk_idx, dtype=np.int64))
        h[offs[3]:offs[3] + nb * 4].view(np.int32)[:] = upd.blk_val
    if nr:
        h[offs[4]:offs[4] + nr * _ROW_INTS * 4].view(np.int32)[:] = np.asarray(
            upd.rows, dtype=np.int32).reshape(-1)


class _Uploader:
    """Pinned host staging -> one device buffer per step.  Two host buffers
    alternate; before one is rewritten, the copy that last read it is waited
    for (an event), so a step never overwrites bytes still in flight."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.device_index = (self.device.index if self.device.index is not None
                             else torch.cuda.current_device() if self.device.type == "cuda" else -1)
        self._host = [None, None]
        self._event = [None, None]
        self._used = [False, False]
        self._dev = None
        self._turn = 0
        self._views = {}           # (turn, bytes) -> (device slice, host slice)
        self.inline_addr = 0       # aia_pack_rows_inline, looked up on first use

    def reserve(self, upd):
        """Offsets and buffers of this step's upload, for the native upload
        (``_hostpack.upload_pack``): (host address, device address, offsets,
        total bytes, raw event to wait for or 0, raw event to record)."""
        nt, nb, nr = len(upd.tok_idx), len(upd.blk_idx), len(upd.rows)
        offs, total = [], 0
        for sz in (nt * 8, nt * 8, nb * 8, nb * 4, nr * _ROW_INTS * 4):
            offs.append(total)
            total += (sz + 15) & ~15
        total = max(total, 16)
        i = self._turn
        self._turn ^= 1
        host = self._host[i]
        if host is None or host.numel() < total:
            if self._used[i]:
                self._event[i].synchronize()      # the old buffer may still be read
            host = torch.empty(max(total * 2, 4096), dtype=torch.uint8, pin_memory=True)
            self._host[i] = host
            self._views.clear()
        if self._dev is None or self._dev.numel() < total:
            self._dev = torch.empty(max(total * 2, 4096), dtype=torch.uint8, device=self.device)
            self._views.clear()
        if self._event[i] is None:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))   # creates the runtime event
            self._event[i] = ev
        wait = self._event[i].cuda_event if self._used[i] else 0
        self._used[i] = True
        return host.data_ptr(), self._dev.data_ptr(), offs, total, wait, self._event[i].cuda_event

    def upload(self, upd, token_width, block_width, stream=None):
        nt, nb, nr = len(upd.tok_idx), len(upd.blk_idx), len(upd.rows)
        sizes = [nt * 8, nt * 8, nb * 8, nb * 4, nr * _ROW_INTS * 4]
        offs, total = [], 0
        for s in sizes:
            offs.append(total)
            total += (s + 15) & ~15
        total = max(total, 16)
        i = self._turn
        self._turn ^= 1
        if self._used[i]:
            self._event[i].synchronize()
        host = self._host[i]
        if host is None or host.numel() < total:
            cap = max(total * 2, 4096)
            host = torch.empty(cap, dtype=torch.uint8, pin_memory=self.device.type == "cuda")
            self._host[i] = host
            self._views.clear()
        if self._dev is None or self._dev.numel() < total:
            self._dev = torch.empty(max(total * 2, 4096), dtype=torch.uint8, device=self.device)
            self._views.clear()
        if _hostpack is not None:
            _hostpack.stage(upd, host.data_ptr(), token_width, block_width, *offs, _ROW_INTS)
        else:
            _stage_py(upd, host.numpy(), token_width, block_width, offs)
        views = self._views.get((i, total))
        if views is None:
            views = self._views[(i, total)] = (self._dev[:total], host[:total])
        views[0].copy_(views[1], non_blocking=True)
        if self.device.type == "cuda":
            if self._event[i] is None:
                self._event[i] = torch.cuda.Event()
            self._event[i].record(stream or torch.cuda.current_stream(self.device))
            self._used[i] = True
        base = self._dev.data_ptr()
        return [base + o for o in offs]


@dataclass
class PackedStep:
    """Device outputs of one pack (views of persistent buffers)."""
    token_ids: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    block_table: torch.Tensor
    cu_seqlens_q: torch.Tensor     # (rows + 1,) int32 with leading 0
    seqlens_kv: torch.Tensor       # (rows,) int32
    last_rows: torch.Tensor        # (rows,) int64


# Steps whose updates and row descriptors fit AIA_PACK_INLINE_BYTES go out in
# the pack launch's arguments (aia_pack_rows_inline); the rest through the
# staging copy.  (Tests switch the inline path off to cover the other.)
_USE_INLINE = True
_INLINE_TOO_LARGE = 1      # _hostpack.pack_inline: the step does not fit, nothing launched


def _launch(table, uploader, upd, *, block_size, bt_width, token_ids, positions, slot_mapping,
            block_table, cu, kv, last_rows, sample_rows=None, sample_count=0, stream=None,
            out_ptrs=None):
    """Pack one step on the device.  ``out_ptrs`` may carry the output
    tensors' device addresses (token_ids, positions, slot_mapping,
    block_table, cu, kv, last_rows) when the caller keeps them."""
    cap = sample_rows.numel() if sample_rows is not None else 0
    if _USE_INLINE and _hostpack is not None and uploader.device.type == "cuda":
        # small step: updates and rows travel in the launch's arguments, no
        # staging copy (aia_pack_rows_inline); the native call stages them
        # and says so (returns 1, nothing launched) when they do not fit
        sp = (stream.cuda_stream if stream is not None
              else _raw_stream(uploader.device_index) if _raw_stream is not None
              else torch.cuda.current_stream(uploader.device).cuda_stream)
        o = out_ptrs or (token_ids.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(),
                         block_table.data_ptr(), cu.data_ptr(), kv.data_ptr(),
                         last_rows.data_ptr())
        pa = table.pool_args
        if pa is None:
            tp, bp = table.token_pool, table.block_pool
            pa = table.pool_args = (tp.shape[1], tp.data_ptr(), bp.shape[1], bp.data_ptr())
        tw, tpa, bw, bpa = pa
        fn = uploader.inline_addr
        if not fn:
            fn = uploader.inline_addr = _native.address("aia_pack_rows_inline")
        rc = _hostpack.pack_inline(
            upd, fn, sp, tw, bw, _ROW_INTS,
            tpa, tw, bpa, bw, block_size, bt_width, o[0], o[1], o[2], o[3],
            o[4], o[5], o[6], sample_rows.data_ptr() if sample_rows is not None else 0,
            sample_count, cap)
        if rc != _INLINE_TOO_LARGE:
            _native.check(rc, "aia_pack_rows_inline")
            return
    if _hostpack is not None and uploader.device.type == "cuda":
        # one native call: event wait, staging, copy, event record, pack launch
        sp = (stream.cuda_stream if stream is not None
              else _raw_stream(uploader.device_index) if _raw_stream is not None
              else torch.cuda.current_stream(uploader.device).cuda_stream)
        host, dev, offs, total, wait, rec = uploader.reserve(upd)
        rc = _hostpack.upload_pack(
            upd, _native.address("aia_pack_rows"), host, dev, wait, rec, sp,
            table.token_pool.shape[1], table.block_pool.shape[1], total, *offs, _ROW_INTS,
            table.token_pool.data_ptr(), table.token_pool.shape[1], table.block_pool.data_ptr(),
            table.block_pool.shape[1], block_size, bt_width, token_ids.data_ptr(),
            positions.data_ptr(), slot_mapping.data_ptr(), block_table.data_ptr(), cu.data_ptr(),
            kv.data_ptr(), last_rows.data_ptr(),
            sample_rows.data_ptr() if sample_rows is not None else 0, sample_count, cap)
        if rc <= _HIP_ERROR:
            raise RuntimeError(f"aia_pack_rows upload: HIP runtime error {_HIP_ERROR - rc}")
        _native.check(rc, "aia_pack_rows")
        return
    if stream is None:
        stream = torch.cuda.current_stream(table.device)
    ptrs = uploader.upload(upd, table.token_pool.shape[1], table.block_pool.shape[1], stream)
    nt, nb, nr = len(upd.tok_idx), len(upd.blk_idx), len(upd.rows)
    _native.call(
        "aia_pack_rows", ptrs[0], ptrs[1], nt, ptrs[2], ptrs[3], nb,
        _ptr(table.token_pool), table.token_pool.shape[1], _ptr(table.block_pool),
        table.block_pool.shape[1], ptrs[4], nr, block_size, bt_width, _ptr(token_ids),
        _ptr(positions), _ptr(slot_mapping), _ptr(block_table), _ptr(cu), _ptr(kv),
        _ptr(last_rows), _ptr(sample_rows), sample_count, cap, stream.cuda_stream)


def _check_blocks(rid, blocks, end, block_size):
    if end > len(blocks) * block_size:
        raise ValueError(f"request {rid}: {len(blocks)} blocks cannot hold position {end - 1}")


def build_rows_py(table, scheduled, get_request, tables, bs, upd, live):
    """Per-request loop of ``DeviceBatchPacker.build`` (the reference's
    model_runner.py:126-166 minus the device work): sync each request into
    the device table, queue its row descriptor, and collect cu_seqlens_q,
    seqlens_kv, sample_idx and decode_splice.  The native extension
    ``_hostpack.build_rows`` runs the same loop; this is its specification.
    Returns (cu, kv, sample_idx, decode_splice, all_decode, tokens, width)."""
    cu, kv = [], []
    sample_idx, decode_splice = {}, []
    all_decode = True
    qacc, width = 0, 0
    sync, rows = table.sync, upd.rows
    for sr in scheduled:
        rid = sr.request_id
        req = get_request(rid)
        n = sr.num_tokens_to_compute
        start = req.num_computed_tokens
        blocks = tables[rid]
        nb = len(blocks)
        end = start + n
        if end > nb * bs:
            _check_blocks(rid, blocks, end, bs)
        draft = getattr(req, "spec_draft", ())
        drafts = tuple(draft) if (draft and not sr.is_prefill) else ()
        slot = sync(upd, rid, req, blocks, end, live, drafts)
        rows.append((slot, start, n, nb, 0, qacc, 0, -1))
        npr = req.num_prompt_tokens
        if end > npr:                                      # positions >= prompt length
            for li in range(max(npr - start, 0), n):
                decode_splice.append((qacc + li, rid))
        if start < npr:
            all_decode = False
        qacc += n
        cu.append(qacc)
        kv.append(end)
        sample_idx[rid] = qacc - 1
        if nb > width:
            width = nb
    return cu, kv, sample_idx, decode_splice, all_decode, qacc, width


class DeviceBatchPacker:
    """GPU version of the eager runner's per-step packing (``_build``,
    model_runner.py:111-188): persistent grow-only device buffers, one
    upload, one kernel; returns ``(ForwardContext, sample_idx,
    decode_splice)`` like the reference, with the context's tensors as views
    of the persistent buffers and the host lists ``cu_seqlens_q`` /
    ``seqlens_kv`` it carries.  The device copies of those lists (and the
    leading-0 cumulative form the attention kernels read) are attached as
    ``ctx.aia_cu_seqlens_q`` / ``ctx.aia_seqlens_kv``."""

    def __init__(self, block_size, device, table=None, max_num_batched_tokens=256,
                 max_num_seqs=64, max_blocks=64):
        self.block_size = block_size
        self.device = torch.device(device)
        self.table = table or DeviceRequestTable(self.device)
        self._uploader = _Uploader(self.device)
        self._tokens = self._seqs = self._blocks = 0
        self._alloc(max_num_batched_tokens, max_num_seqs, max_blocks)

    def _alloc(self, n_tokens, n_seqs, n_blocks):
        n_tokens, n_seqs = max(n_tokens, self._tokens), max(n_seqs, self._seqs)
        n_blocks = max(n_blocks, self._blocks)
        dev = self.device
        self.token_ids_buf = torch.zeros(n_tokens, dtype=torch.int64, device=dev)
        self.positions_buf = torch.zeros(n_tokens, dtype=torch.int64, device=dev)
        self.slot_mapping_buf = torch.zeros(n_tokens, dtype=torch.int32, device=dev)
        self.block_table_buf = torch.zeros(n_seqs * n_blocks, dtype=torch.int32, device=dev)
        self.cu_buf = torch.zeros(n_seqs + 1, dtype=torch.int32, device=dev)
        self.kv_buf = torch.zeros(n_seqs, dtype=torch.int32, device=dev)
        self.last_buf = torch.zeros(n_seqs, dtype=torch.int64, device=dev)
        self._tokens, self._seqs, self._blocks = n_tokens, n_seqs, n_blocks
        self._views = {}           # (T, B, width) -> output views

    def build(self, plan, attn_backend=None, kv_caches=None, attn_mask=None):
        bs = self.block_size
        table = self.table
        upd = table.begin_step()
        scheduled = plan.scheduled
        if _hostpack is not None:     # builds the live set itself, only if a slot is needed
            # a BatchPlan's get_request is a lookup in its request mapping
            # (execution.py:54-55 in the reference): the native loop reads the
            # mapping directly then
            reqs = getattr(plan, "requests", None)
            lookup = reqs if type(reqs) in _PLAIN_MAPPINGS else plan.get_request
            cu, kv, sample_idx, decode_splice, all_decode, qacc, width = _hostpack.build_rows(
                table, scheduled, lookup, plan.block_tables, bs, upd, None)
        else:
            cu, kv, sample_idx, decode_splice, all_decode, qacc, width = build_rows_py(
                table, scheduled, plan.get_request, plan.block_tables, bs, upd,
                {sr.request_id for sr in scheduled})
        T, B = qacc, len(plan.scheduled)
        if T > self._tokens or B > self._seqs or width > self._blocks:
            self._alloc(T * 2 if T > self._tokens else T, B * 2 if B > self._seqs else B,
                        width * 2 if width > self._blocks else width)
        views = self._views.get((T, B, width))
        if views is None:      # steady decode steps repeat their shape
            bt = self.block_table_buf[:B * width].view(B, width)
            views = self._views[(T, B, width)] = (
                self.token_ids_buf[:T], self.positions_buf[:T], self.slot_mapping_buf[:T], bt,
                self.cu_buf[:B + 1], self.kv_buf[:B],
                tuple(t.data_ptr() for t in (self.token_ids_buf, self.positions_buf,
                                             self.slot_mapping_buf, bt, self.cu_buf,
                                             self.kv_buf, self.last_buf)))
        bt = views[3]
        _launch(self.table, self._uploader, upd, block_size=bs, bt_width=width,
                token_ids=self.token_ids_buf, positions=self.positions_buf,
                slot_mapping=self.slot_mapping_buf, block_table=bt, cu=self.cu_buf,
                kv=self.kv_buf, last_rows=self.last_buf, out_ptrs=views[6])
        ctx = ForwardContext(
            token_ids=views[0], positions=views[1], slot_mapping=views[2], block_table=bt,
            cu_seqlens_q=cu, seqlens_kv=kv, attn_mask=attn_mask, attn_backend=attn_backend,
            kv_caches=kv_caches, is_decode=all_decode)
        ctx.aia_cu_seqlens_q = views[4]
        ctx.aia_seqlens_kv = views[5]
        # every slot this packer writes is block_table[pos // bs] * bs + pos % bs
        # of its row's block table, so the attention kernel may do the KV write
        ctx.aia_slots_from_block_table = True
        return ctx, sample_idx, decode_splice


# ------------------------------------------------------- device token splice

@dataclass(frozen=True)
class PreparedTokenSplice:
    """A splice planned by ``prepare_splice`` (reference
    decode_input_stager.py:27-31): either one aligned owner (``fast_owner``,
    its first ``fast_count`` tokens) or ``count`` (source address, row)
    pairs already on the device in ``pairs``.  ``groups`` holds the owning
    batches, which keeps their token tensors alive until the splice runs."""
    groups: tuple
    fast_owner: object = None
    fast_count: int = 0
    pairs: torch.Tensor = None
    count: int = 0


def _token_address(tokens, row):
    if tokens.dtype != torch.int64 or tokens.dim() != 1 or not tokens.is_cuda:
        raise ValueError("sampled tokens must be a 1-D int64 GPU tensor")
    if not 0 <= row < tokens.shape[0]:
        raise ValueError("sampled token row is out of bounds")
    return tokens.data_ptr() + row * tokens.stride(0) * 8


class _PairUploader:
    """(source address, target row) pairs -> a persistent device buffer,
    through pinned memory.  The host buffer is rewritten only after the copy
    that last read it has finished."""

    def __init__(self, device, cap):
        self.device = torch.device(device)
        self._cap = 0
        self._grow(max(int(cap), 16))
        self._event = None

    def _grow(self, cap):
        self._host = torch.empty(cap, 2, dtype=torch.int64, pin_memory=True)
        self._dev = torch.empty(cap, 2, dtype=torch.int64, device=self.device)
        self._cap = cap

    def upload(self, pairs):
        n = len(pairs)
        if self._event is not None:
            self._event.synchronize()
        if n > self._cap:
            self._grow(2 * n)
        self._host.numpy()[:n] = pairs
        dev = self._dev[:n]
        dev.copy_(self._host[:n], non_blocking=True)
        self._event = torch.cuda.Event()
        self._event.record(torch.cuda.current_stream(self.device))
        return dev


_default_pairs = {}


def splice_device_tokens(target, target_rows, request_order, refs, *, uploader=None):
    """``target[target_rows[i]] = refs[request_order[i]].owner.tokens[row]``
    for every request that has a ref, in one kernel launch whatever the
    number of owning tensors (reference worker/staging.py:51-70 issues an
    index_select + index_copy_ per owner).  ``target``: 1-D int64 on the
    GPU."""
    _check_device_tensor(target, "target", torch.int64)
    if target.dim() != 1 or not target.is_contiguous():
        raise ValueError("target must be a contiguous 1-D tensor")
    pairs, owners = [], []
    for row, rid in zip(target_rows, request_order):
        ref = refs.get(rid)
        if ref is None:
            continue
        pairs.append((_token_address(ref.owner.tokens, ref.row), int(row)))
        owners.append(ref.owner)
    if not pairs:
        return
    if uploader is None:
        uploader = _default_pairs.get(target.device)
        if uploader is None:
            uploader = _default_pairs[target.device] = _PairUploader(target.device, 64)
    dev = uploader.upload(pairs)
    _native.call("aia_splice_tokens", _ptr(dev), len(pairs), _ptr(target), target.numel(),
                 _stream(target.device))
    for o in owners:          # the kernel reads them on this stream
        o.tokens.record_stream(torch.cuda.current_stream(target.device))


# ---------------------------------------------------------------- stagers

@dataclass(frozen=True)
class StagedDecodeInput:
    token_ids: torch.Tensor
    positions: torch.Tensor
    slots: torch.Tensor
    block_table: torch.Tensor
    kv_lengths: list
    order: list
    cu_seqlens_q: torch.Tensor = None
    seqlens_kv: torch.Tensor = None

    def data_ptrs(self):
        return (self.token_ids.data_ptr(), self.positions.data_ptr(),
                self.slots.data_ptr(), self.block_table.data_ptr())


def _contig(t, name, dtype):
    _check_device_tensor(t, name, dtype)
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _row_key(ids):
    """The contents of a zero-padded block-table row, as a comparable key
    (trailing zeros dropped: [5] and [5, 0] fill a row identically)."""
    ids = tuple(ids)
    n = len(ids)
    while n and ids[n - 1] == 0:
        n -= 1
    return ids[:n]


class _BlockRowLedger:
    """The reference's dirty-row accounting of a gear block table
    (worker/staging.py:20-48, used by decode_input_stager.py:115-119,
    :246-250, :365-369 and prefill_input_stager.py:151-155): a row counts as
    copied when its contents differ from what the last copy left, every row
    the first time (the shadow starts at INT32_MIN); elements = rows x row
    width.  Rows from ``active`` on are neither compared nor recorded.
    Only keys are kept: the kernel writes the device rows either way."""

    def __init__(self, rows, width):
        self._shadow = [None] * rows
        self._width = width

    def account(self, keys, active=None):
        n = len(keys) if active is None else min(active, len(keys))
        copied = 0
        for r in range(n):
            if keys[r] != self._shadow[r]:
                self._shadow[r] = keys[r]
                copied += 1
        return copied, copied * self._width


class _GearStager:
    def __init__(self, device, table, rows, width):
        self.table = table or DeviceRequestTable(device)
        self._uploader = _Uploader(device)
        self._cu = torch.zeros(rows + 1, dtype=torch.int32, device=device)
        self._kv = torch.zeros(rows, dtype=torch.int32, device=device)
        self._last = torch.zeros(rows, dtype=torch.int64, device=device)
        self._ledger = _BlockRowLedger(rows, width)
        self.copied_block_rows = 0
        self.copied_block_elements = 0

    def _count(self, keys, active=None):
        rows, elems = self._ledger.account(keys, active)
        self.copied_block_rows += rows
        self.copied_block_elements += elems


class DecodeInputStager(_GearStager):
    """Fixed-address decode gear (reference decode_input_stager.py:35-123):
    live row = (token at num_computed_tokens, that position, its slot, the
    request's block row, kv length pos + 1); padding rows use scratch block
    scratch0 + row, slot block * bs, token 0, position 0, kv length 1."""

    def __init__(self, *, tid, positions, slots, block_table, block_size, scratch0,
                 active_token_mask=None, table=None):
        _contig(tid, "tid", torch.int64)
        _contig(positions, "positions", torch.int64)
        _contig(slots, "slots", torch.int32)
        _contig(block_table, "block_table", torch.int32)
        self.tid, self.positions, self.slots, self.block_table = tid, positions, slots, block_table
        self.active_token_mask = active_token_mask
        if active_token_mask is not None and (active_token_mask.dtype is not torch.bool or
                                              tuple(active_token_mask.shape) != (tid.shape[0],)):
            raise ValueError("decode active-token mask must be gear-shaped bool")
        self.block_size = block_size
        self.scratch0 = scratch0
        self.gear = tid.shape[0]
        self.max_blocks = block_table.shape[1]
        super().__init__(tid.device, table, self.gear, self.max_blocks)
        self._splice_pairs = _PairUploader(tid.device, self.gear)

    def stage(self, plan, scheduled=None):
        scheduled = plan.scheduled if scheduled is None else scheduled
        if len(scheduled) > self.gear:
            raise ValueError(f"decode batch {len(scheduled)} exceeds gear {self.gear}")
        upd = self.table.begin_step()
        live = {item.request_id for item in scheduled}
        kv, order, keys = [], [], []
        for row, item in enumerate(scheduled):
            rid = item.request_id
            req = plan.get_request(rid)
            pos = req.num_computed_tokens
            blocks = plan.block_tables[rid]
            if len(blocks) > self.max_blocks:
                raise ValueError(f"request {rid} has {len(blocks)} blocks > {self.max_blocks}")
            _check_blocks(rid, blocks, pos + 1, self.block_size)
            slot = self.table.sync(upd, rid, req, blocks, pos + 1, live)
            upd.row(slot, pos, 1, len(blocks), 0, row, 0, -1)
            kv.append(pos + 1)
            order.append(rid)
            keys.append(_row_key(blocks))
        for row in range(len(scheduled), self.gear):
            upd.row(-1, 0, 1, 1, self.scratch0 + row, row, 1, -1)
            kv.append(1)
            keys.append(_row_key((self.scratch0 + row,)))
        _launch(self.table, self._uploader, upd, block_size=self.block_size,
                bt_width=self.max_blocks, token_ids=self.tid, positions=self.positions,
                slot_mapping=self.slots, block_table=self.block_table, cu=self._cu,
                kv=self._kv, last_rows=self._last)
        if self.active_token_mask is not None:
            self.active_token_mask[:len(scheduled)].fill_(True)
            self.active_token_mask[len(scheduled):].fill_(False)
        self._count(keys)
        return StagedDecodeInput(self.tid, self.positions, self.slots, self.block_table, kv,
                                 order, self._cu, self._kv)

    # -- device token splice (decode_input_stager.py:125-170) -------------
    def prepare_splice(self, refs, request_order):
        """Plan the move of retained sampled tokens into ``tid`` rows: row i
        takes ``refs[request_order[i]]`` when present.  One owner whose rows
        0..n-1 line up with rows 0..n-1 becomes a plain copy; anything else
        becomes (source address, row) pairs uploaded now, for one splice
        launch in ``apply_splice``."""
        owners, dst, src = [], [], []
        for i, rid in enumerate(request_order):
            ref = refs.get(rid)
            if ref is None:
                continue
            if all(o is not ref.owner for o in owners):
                owners.append(ref.owner)
            dst.append(i)
            src.append(ref)
        if len(owners) == 1 and dst == list(range(len(dst))) and \
                [r.row for r in src] == dst:
            return PreparedTokenSplice((), owners[0], len(dst))
        pairs = [(_token_address(r.owner.tokens, r.row), d) for r, d in zip(src, dst)]
        buf = self._splice_pairs.upload(pairs) if pairs else None
        return PreparedTokenSplice(tuple(owners), None, 0, buf, len(pairs))

    def apply_splice(self, prepared):
        if prepared.fast_owner is not None:
            n = prepared.fast_count
            self.tid[:n].copy_(prepared.fast_owner.tokens[:n])
            return
        if prepared.count:
            _native.call("aia_splice_tokens", _ptr(prepared.pairs), prepared.count,
                         _ptr(self.tid), self.tid.numel(), _stream(self.tid.device))

    def splice(self, refs, request_order):
        self.apply_splice(self.prepare_splice(refs, request_order))


class SpecDecodeInputStager(_GearStager):
    """MTP-verify gear (reference decode_input_stager.py:257-373): query_width
    = draft_depth + 1 rows per request with tokens (last, *drafts),
    positions pos + offset, kv length pos + width; padding request rows on
    scratch block scratch0 + row with positions 0..width-1."""

    def __init__(self, *, tid, positions, slots, block_table, drafts, block_size, scratch0,
                 geometry=None, draft_depth=None, active_mask=None, active_token_mask=None,
                 table=None):
        if draft_depth is None:
            draft_depth = geometry.draft_depth
        self.draft_depth = draft_depth
        self.query_width = draft_depth + 1
        _contig(tid, "tid", torch.int64)
        _contig(positions, "positions", torch.int64)
        _contig(slots, "slots", torch.int32)
        _contig(block_table, "block_table", torch.int32)
        self.tid, self.positions, self.slots, self.block_table = tid, positions, slots, block_table
        self.drafts = drafts
        self.active_mask = active_mask
        self.active_token_mask = active_token_mask
        self.block_size = block_size
        self.scratch0 = scratch0
        self.gear, self.max_blocks = block_table.shape
        if tid.numel() != self.gear * self.query_width:
            raise ValueError("spec decode token buffer must match the configured query width")
        if active_mask is not None and tuple(active_mask.shape) != (self.gear,):
            raise ValueError("spec active mask must have one row per request")
        super().__init__(tid.device, table, self.gear, self.max_blocks)
        self._draft_host = torch.zeros(tuple(drafts.shape), dtype=torch.int64,
                                       pin_memory=tid.is_cuda)
        self._draft_event = None

    def stage(self, plan, scheduled=None):
        scheduled = plan.scheduled if scheduled is None else scheduled
        if len(scheduled) > self.gear:
            raise ValueError(f"spec decode batch {len(scheduled)} exceeds gear {self.gear}")
        upd = self.table.begin_step()
        live = {item.request_id for item in scheduled}
        w = self.query_width
        kv, order, keys = [], [], []
        if self._draft_event is not None:
            self._draft_event.synchronize()
        dh = self._draft_host.numpy()
        dh.fill(0)
        for row, item in enumerate(scheduled):
            rid = item.request_id
            req = plan.get_request(rid)
            pos = req.num_computed_tokens
            blocks = plan.block_tables[rid]
            if len(req.spec_draft) != self.draft_depth:
                raise ValueError(f"request {rid} has {len(req.spec_draft)} drafts; "
                                 f"expected {self.draft_depth}")
            _check_blocks(rid, blocks, pos + w, self.block_size)
            slot = self.table.sync(upd, rid, req, blocks, pos + w, live, tuple(req.spec_draft))
            upd.row(slot, pos, w, len(blocks), 0, row * w, 0, -1)
            dh[row] = req.spec_draft
            kv.append(pos + w)
            order.append(rid)
            keys.append(_row_key(blocks))
        for row in range(len(scheduled), self.gear):
            upd.row(-1, 0, w, 1, self.scratch0 + row, row * w, 1, -1)
            kv.append(w)
            keys.append(_row_key((self.scratch0 + row,)))
        _launch(self.table, self._uploader, upd, block_size=self.block_size,
                bt_width=self.max_blocks, token_ids=self.tid, positions=self.positions,
                slot_mapping=self.slots, block_table=self.block_table, cu=self._cu,
                kv=self._kv, last_rows=self._last)
        self.drafts.copy_(self._draft_host, non_blocking=True)
        if self.drafts.is_cuda:
            self._draft_event = torch.cuda.Event()
            self._draft_event.record(torch.cuda.current_stream(self.drafts.device))
        if self.active_mask is not None:
            self.active_mask[:len(scheduled)].fill_(1)
            self.active_mask[len(scheduled):].fill_(0)
        if self.active_token_mask is not None:
            self.active_token_mask[:len(scheduled) * w].fill_(True)
            self.active_token_mask[len(scheduled) * w:].fill_(False)
        self._count(keys)
        return StagedDecodeInput(self.tid, self.positions, self.slots, self.block_table, kv,
                                 order, self._cu, self._kv)


@dataclass(frozen=True)
class StagedPrefillInput:
    token_ids: torch.Tensor
    positions: torch.Tensor
    slots: torch.Tensor
    block_table: torch.Tensor
    sample_rows: torch.Tensor
    cumulative_query_lengths: list
    kv_lengths: list
    sample_order: list
    splice_order: list
    splice_rows: list
    query_tokens: int
    real_query_tokens: int
    sequence_count: int
    cu_seqlens_q: torch.Tensor = None
    seqlens_kv: torch.Tensor = None

    def data_ptrs(self):
        return (self.token_ids.data_ptr(), self.positions.data_ptr(), self.slots.data_ptr(),
                self.block_table.data_ptr(), self.sample_rows.data_ptr())


class PrefillInputStager(_GearStager):
    """Flattened-token prefill/mixed gear (reference prefill_input_stager.py:
    35-162): rows packed request after request, cumulative query lengths,
    kv length start + n, sample rows for requests whose chunk completes the
    prefill, and one padding pseudo-sequence on scratch blocks scratch0 + k
    covering the token-gear slack."""

    def __init__(self, *, token_ids, positions, slots, block_table, sample_rows, block_size,
                 scratch0, active_token_mask=None, table=None):
        _contig(token_ids, "token_ids", torch.int64)
        _contig(positions, "positions", torch.int64)
        _contig(slots, "slots", torch.int32)
        _contig(block_table, "block_table", torch.int32)
        _contig(sample_rows, "sample_rows", torch.int64)
        self.token_ids, self.positions, self.slots = token_ids, positions, slots
        self.block_table, self.sample_rows = block_table, sample_rows
        self.active_token_mask = active_token_mask
        if active_token_mask is not None and (active_token_mask.dtype is not torch.bool or
                                              tuple(active_token_mask.shape) !=
                                              (token_ids.shape[0],)):
            raise ValueError("prefill active-token mask must be gear-shaped bool")
        self.block_size = block_size
        self.scratch0 = scratch0
        self.query_gear = token_ids.shape[0]
        self.sequence_gear = sample_rows.shape[0]
        self.max_blocks = block_table.shape[1]
        super().__init__(token_ids.device, table, block_table.shape[0], self.max_blocks)
        self._splice_pairs = _PairUploader(token_ids.device, self.query_gear)

    def stage(self, plan):
        scheduled = plan.scheduled
        real = sum(item.num_tokens_to_compute for item in scheduled)
        nseq = len(scheduled)
        if real > self.query_gear or nseq > self.sequence_gear:
            raise ValueError(
                f"batch ({real} tokens, {nseq} sequences) "
                f"exceeds prefill gear ({self.query_gear}, {self.sequence_gear})")
        if not scheduled:
            raise ValueError("prefill staging requires at least one sequence")
        upd = self.table.begin_step()
        live = {item.request_id for item in scheduled}
        cu, kv, sample_order, splice_order, splice_rows = [], [], [], [], []
        keys = []
        q = 0
        for item in scheduled:
            rid = item.request_id
            req = plan.get_request(rid)
            start = req.num_computed_tokens
            n = item.num_tokens_to_compute
            blocks = plan.block_tables[rid]
            _check_blocks(rid, blocks, start + n, self.block_size)
            slot = self.table.sync(upd, rid, req, blocks, start + n, live)
            sample = -1
            if start + n >= req.num_prefill_tokens:
                sample = len(sample_order)
                sample_order.append(rid)
            upd.row(slot, start, n, len(blocks), 0, q, 0, sample)
            q += n
            cu.append(q)
            kv.append(start + n)
            splice_order.append(rid)
            splice_rows.append(q - 1)
            keys.append(_row_key(blocks))
        padding = self.query_gear - real
        if padding:
            nblk = (padding + self.block_size - 1) // self.block_size
            upd.row(-1, 0, padding, nblk, self.scratch0, q, 1, -1)
            keys.append(_row_key(range(self.scratch0, self.scratch0 + nblk)))
            cu.append(self.query_gear)
            kv.append(padding)
        rows = nseq + int(bool(padding))
        if rows > self.block_table.shape[0]:
            raise ValueError(f"batch ({real} tokens, {nseq} sequences) "
                             f"exceeds prefill gear ({self.query_gear}, {self.sequence_gear})")
        _launch(self.table, self._uploader, upd, block_size=self.block_size,
                bt_width=self.max_blocks, token_ids=self.token_ids, positions=self.positions,
                slot_mapping=self.slots, block_table=self.block_table, cu=self._cu,
                kv=self._kv, last_rows=self._last, sample_rows=self.sample_rows,
                sample_count=len(sample_order))
        # rows past the attention sequences keep zeros (reference fills them)
        if rows < self.block_table.shape[0]:
            self.block_table[rows:].zero_()
        if self.active_token_mask is not None:
            self.active_token_mask[:real].fill_(True)
            self.active_token_mask[real:].fill_(False)
        self._count(keys, active=rows)
        return StagedPrefillInput(
            self.token_ids, self.positions, self.slots, self.block_table[:rows],
            self.sample_rows, cu, kv, sample_order, splice_order, splice_rows,
            self.query_gear, real, nseq, self._cu[:rows + 1], self._kv[:rows])

    def splice(self, refs, request_order, target_rows):
        """Retained sampled tokens into ``token_ids`` rows (reference
        prefill_input_stager.py:164-166)."""
        splice_device_tokens(self.token_ids, target_rows, request_order, refs,
                             uploader=self._splice_pairs)


@dataclass(frozen=True)
class StagedContinuationInput:
    kv_lengths: list


class ContinuationInputStager:
    """Recurrent MTP continuation gear (reference decode_input_stager.py:
    178-251): for draft step s, live row position = num_computed_tokens +
    accepted + s, its slot, kv length position + 1, and the request's block
    row; padding rows use scratch block scratch0 + row with position s, slot
    block * bs + s and kv length s + 1.  ``positions`` / ``slots`` are
    (gear,) for one step or (steps, gear) for ``stage_all``.  All steps'
    rows are packed by one kernel from the device request table."""

    def __init__(self, *, positions, slots, block_table, block_size, scratch0, table=None):
        _contig(positions, "positions", torch.int64)
        _contig(slots, "slots", torch.int32)
        _contig(block_table, "block_table", torch.int32)
        self.positions, self.slots, self.block_table = positions, slots, block_table
        self.block_size = block_size
        self.scratch0 = scratch0
        self.gear, self.max_blocks = block_table.shape
        self._batched_steps = positions.dim() == 2
        self.steps = positions.shape[0] if self._batched_steps else 1
        if slots.shape != positions.shape:
            raise ValueError("continuation positions and slots must match")
        if positions.shape[-1] != self.gear:
            raise ValueError("continuation positions must have one column per gear row")
        dev = positions.device
        self.table = table or DeviceRequestTable(dev)
        self._uploader = _Uploader(dev)
        n = self.steps * self.gear
        # outputs the continuation does not use (token ids, per-step block
        # rows, query offsets) land in private buffers
        self._tid = torch.zeros(n, dtype=torch.int64, device=dev)
        self._bt_all = torch.zeros(n, self.max_blocks, dtype=torch.int32, device=dev)
        self._cu = torch.zeros(n + 1, dtype=torch.int32, device=dev)
        self._kv = torch.zeros(n, dtype=torch.int32, device=dev)
        self._last = torch.zeros(n, dtype=torch.int64, device=dev)
        self._ledger = _BlockRowLedger(self.gear, self.max_blocks)
        self.copied_block_rows = 0
        self.copied_block_elements = 0

    def stage(self, plan, scheduled, accepted, step):
        if self._batched_steps:
            raise ValueError("use stage_all for a multi-step continuation gear")
        return StagedContinuationInput(self._stage_all(plan, scheduled, accepted, (step,))[0])

    def stage_all(self, plan, scheduled, accepted):
        return self._stage_all(plan, scheduled, accepted, range(1, self.steps + 1))

    def _stage_all(self, plan, scheduled, accepted, steps):
        if len(scheduled) > self.gear or len(accepted) != len(scheduled):
            raise ValueError("continuation metadata does not match graph gear")
        steps = list(steps)
        upd = self.table.begin_step()
        live = {item.request_id for item in scheduled}
        bs, g = self.block_size, self.gear
        slots, keys = [], []
        for item, acc in zip(scheduled, accepted):
            rid = item.request_id
            req = plan.get_request(rid)
            blocks = plan.block_tables[rid]
            if len(blocks) > self.max_blocks:
                raise ValueError(f"request {rid} has {len(blocks)} blocks > {self.max_blocks}")
            _check_blocks(rid, blocks, req.num_computed_tokens + acc + max(steps) + 1, bs)
            # blocks only: the continuation reads no token ids
            slots.append(self.table.sync(upd, rid, req, blocks, 0, live))
            keys.append(_row_key(blocks))
        for row in range(len(scheduled), g):
            keys.append(_row_key((self.scratch0 + row,)))
        kv_by_step = []
        for si, step in enumerate(steps):
            kv = []
            for row, (item, acc) in enumerate(zip(scheduled, accepted)):
                req = plan.get_request(item.request_id)
                pos = req.num_computed_tokens + acc + step
                upd.row(slots[row], pos, 1, len(plan.block_tables[item.request_id]), 0,
                        si * g + row, 1, -1)
                kv.append(pos + 1)
            for row in range(len(scheduled), g):
                upd.row(-1, step, 1, 1, self.scratch0 + row, si * g + row, 1, -1)
                kv.append(step + 1)
            kv_by_step.append(kv)
        _launch(self.table, self._uploader, upd, block_size=bs, bt_width=self.max_blocks,
                token_ids=self._tid, positions=self.positions, slot_mapping=self.slots,
                block_table=self._bt_all, cu=self._cu, kv=self._kv, last_rows=self._last)
        self.block_table.copy_(self._bt_all[:g])
        rows, elems = self._ledger.account(keys)
        self.copied_block_rows += rows
        self.copied_block_elements += elems
        return kv_by_step
