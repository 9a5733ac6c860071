"""Per-step device metadata shared by every layer of a step.

The reference hands the attention op host lists (``ctx.cu_seqlens_q``
cumulative ends, ``ctx.seqlens_kv`` per request; forward_context.py:14-15)
and a device block table.  Our kernels read device int32 copies and a
split-K plan; both depend only on the step, so they are built once per
``ForwardContext`` (on first use, or by the GPU packer which attaches them
as ``ctx.aia_cu_seqlens_q`` / ``ctx.aia_seqlens_kv``) and cached on it.
Every context's plan owns its workspace, so steps in flight on different
streams do not share scratch memory.

Device metadata attached by a packer is not checked on the host.  Query
lengths that do not add up to the step's token count make the planner plan
nothing (status -1); the attention call then fills its output with NaN.
With ``AIA_CHECK_PLAN=1`` in the environment, ``step_plan`` also reads the
status back after planning (one device synchronisation per step) and raises
the ValueError of the reference's stager contract
(prefill_input_stager.py:77-81).
"""
import os

import torch

from auto_infer_amd import ops


def step_plan(ctx, num_q_heads, num_kv_heads, head_dim_v, block_size):
    plans = getattr(ctx, "_aia_plans", None)
    if plans is None:
        plans = {}
        ctx._aia_plans = plans
    key = (num_q_heads, num_kv_heads, head_dim_v, block_size)
    plan = plans.get(key)
    if plan is not None:
        return plan
    bt = ctx.block_table
    cu = getattr(ctx, "aia_cu_seqlens_q", None)
    kv = getattr(ctx, "aia_seqlens_kv", None)
    if cu is None or kv is None:
        dev = bt.device
        ops.check_lists(ctx.cu_seqlens_q, ctx.seqlens_kv, bt.shape[1] * block_size)
        cu = torch.tensor([0, *ctx.cu_seqlens_q], dtype=torch.int32).to(dev)
        kv = torch.tensor(list(ctx.seqlens_kv), dtype=torch.int32).to(dev)
        ctx.aia_cu_seqlens_q, ctx.aia_seqlens_kv = cu, kv
        owned = [cu, kv]
    else:
        owned = []
    T = int(ctx.cu_seqlens_q[-1]) if len(ctx.cu_seqlens_q) else 0
    if bt.dtype != torch.int32:
        bt = bt.to(torch.int32)
        owned.append(bt)
    # each context (one step in flight) gets its own workspace from the
    # caching allocator: two steps on two streams never share one, and the
    # plan records every stream it is used on, so the memory is not handed
    # out again while a step on another stream still reads it
    plan = ops.AttentionPlan(bt, cu, kv, T, num_q_heads, num_kv_heads, head_dim_v, block_size,
                             owned=owned)
    if not owned and os.environ.get("AIA_CHECK_PLAN", "0") == "1" and \
            not torch.cuda.is_current_stream_capturing():
        plan.status()
    plans[key] = plan
    return plan
