"""Helpers that turn the JSON golden fixtures into plan objects."""
import json
import os

from auto_infer_amd.execution import BatchPlan, RequestView, ScheduledRequest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        return json.load(f)


def make_plan(requests, scheduled):
    views = {
        rid: RequestView(rid, tuple(r["tokens"]), r["computed"], r["prompt"],
                         r["prefill"], tuple(r["draft"]))
        for rid, r in requests.items()}
    items = [ScheduledRequest(rid, n, bool(p), tuple(requests[rid]["blocks"]))
             for rid, n, p in scheduled]
    return BatchPlan.make(items, views,
                          {rid: r["blocks"] for rid, r in requests.items()})
