"""Write the packing golden vectors as JSON fixtures.

Every expected value below is transcribed from a literal assertion in the
reference's own host tests (file:line given per case), or -- for the eager
``_build`` cases of tests/test_input_buffers.py, whose reference test
compares against an inline re-implementation instead of literals -- worked
out by hand from the inputs with ``slot = bt[pos // bs] * bs + pos % bs``
and written here literally.  Nothing in this file imports or runs the
reference.

Plan encoding: ``requests`` maps rid -> {tokens, computed, prompt, prefill,
draft, blocks}; ``scheduled`` lists [rid, num_tokens_to_compute, is_prefill].
Run: ``python tests/golden/make_fixtures.py`` (rewrites the JSON files).
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def req(tokens, computed, blocks, prompt=None, prefill=None, draft=()):
    tokens = list(tokens)
    prompt = len(tokens) if prompt is None else prompt
    return dict(tokens=tokens, computed=computed, blocks=list(blocks),
                prompt=prompt, prefill=prompt if prefill is None else prefill,
                draft=list(draft))


def runner_req(rid, prompt_len, num_output=0, computed=0, blocks=(), draft=()):
    """tests/test_input_buffers.py:56-67 make_req: prompt 1000 + rid*100 + i,
    outputs 9000 + rid*10 + i."""
    prompt = [1000 + rid * 100 + i for i in range(prompt_len)]
    out = [9000 + rid * 10 + i for i in range(num_output)]
    return req(prompt + out, computed, blocks, prompt=prompt_len, draft=draft)


# ---------------------------------------------------------------- decode
DEC_A = req(range(20), 5, [7, 8, 9], draft=[99])
DEC_B = req(range(20, 40), 1, [3], draft=[99])

decode = {
    "source": "tests/test_decode_input_stager.py:9-50 (fixtures), :72-85, :88-98, :101-110, :140-205",
    "stager": dict(gear=4, max_blocks=4, block_size=4, scratch0=100),
    "cases": [
        {   # :72-85 live and padding rows
            "name": "live_and_padding_rows",
            "requests": {"a": DEC_A, "b": DEC_B},
            "scheduled": [["a", 1, False], ["b", 1, False]],
            "expect": dict(order=["a", "b"], kv_lengths=[6, 2, 1, 1],
                           token_ids=[5, 21, 0, 0], positions=[5, 1, 0, 0],
                           slots=[33, 13, 408, 412],
                           block_table=[[7, 8, 9, 0], [3, 0, 0, 0],
                                        [102, 0, 0, 0], [103, 0, 0, 0]],
                           active_token_mask=[True, True, False, False]),
        },
    ],
    # :101-110 a row that turns into padding is copied exactly once more;
    # :62-69 an unchanged step copies nothing.
    "dirty_sequence": [
        {"requests": {"a": DEC_A, "b": DEC_B},
         "scheduled": [["a", 1, False], ["b", 1, False]], "copied_rows": 4},
        {"requests": {"a": dict(DEC_A, computed=6), "b": DEC_B},
         "scheduled": [["a", 1, False], ["b", 1, False]], "copied_rows": 0},
        {"requests": {"a": dict(DEC_A, computed=6)},
         "scheduled": [["a", 1, False]], "copied_rows": 1,
         "row1": [101, 0, 0, 0], "active_token_mask": [True, False, False, False]},
    ],
}

spec = {
    "source": "tests/test_decode_input_stager.py:140-186",
    "cases": [
        {   # :140-169 depth 1, gear 4
            "name": "two_token_rows",
            "stager": dict(gear=4, max_blocks=4, block_size=4, scratch0=100,
                           draft_depth=1),
            "requests": {"a": DEC_A, "b": DEC_B},
            "scheduled": [["a", 2, False], ["b", 2, False]],
            "expect": dict(order=["a", "b"], kv_lengths=[7, 3, 2, 2],
                           token_ids=[5, 99, 21, 99, 0, 0, 0, 0],
                           positions=[5, 6, 1, 2, 0, 1, 0, 1],
                           slots=[33, 34, 13, 14, 408, 409, 412, 413],
                           active_mask=[1, 1, 0, 0]),
            "second": {"requests": {"a": dict(DEC_A, computed=6), "b": DEC_B},
                       "extra_copied_rows": 0},
        },
        {   # :171-186 depth 3, gear 2
            "name": "multi_step_rows",
            "stager": dict(gear=2, max_blocks=4, block_size=4, scratch0=100,
                           draft_depth=3),
            "requests": {"a": req(range(20), 5, [7, 8, 9], draft=[90, 91, 92])},
            "scheduled": [["a", 4, False]],
            "expect": dict(token_ids=[5, 90, 91, 92, 0, 0, 0, 0],
                           positions=[5, 6, 7, 8, 0, 1, 2, 3],
                           drafts=[[90, 91, 92], [0, 0, 0]]),
        },
    ],
}

continuation = {
    "source": "tests/test_decode_input_stager.py:208-269",
    "stager": dict(gear=2, max_blocks=4, block_size=4, scratch0=100),
    "reuse": {  # :208-229
        "requests": {"a": req(range(20), 5, [7, 8, 9], draft=[90, 91])},
        "steps": [{"accepted": [1], "step": 1, "kv_lengths": [8, 2]},
                  {"accepted": [2], "step": 2, "kv_lengths": [10, 3],
                   "positions": [9, 2], "slots": [37, 406], "extra_copied_rows": 0}],
    },
    "two_dirty": {  # :232-253
        "first": {"a": req(range(20), 5, [7, 8, 9], draft=[90, 91]),
                  "b": req(range(20, 40), 1, [3], draft=[80, 81])},
        "second_blocks": {"a": [7, 8, 10], "b": [4]},
        "accepted": [1, 1], "step": 1,
        "extra_copied_rows": 2, "extra_copied_elements": 8,
    },
    "stage_all": {  # :256-269 two steps in one copy
        "requests": {"a": req(range(20), 5, [7, 8, 9], draft=[90, 91, 92])},
        "accepted": [1], "steps": [1, 2],
        "kv_by_step": [[8, 2], [9, 3]], "positions": [[7, 1], [8, 2]],
    },
}

prefill = {
    "source": "tests/test_prefill_input_stager.py:39-197",
    "cases": [
        {   # :39-61
            "name": "exact_shape_tnd",
            "stager": dict(query_gear=6, sequence_gear=2, max_blocks=4,
                           block_size=4, scratch0=100),
            "requests": {"a": req([10, 11, 12, 13], 0, [5], prefill=4),
                         "b": req([20, 21, 22], 1, [7], prefill=3)},
            "scheduled": [["a", 4, True], ["b", 2, True]],
            "expect": dict(query_tokens=6, token_ids=[10, 11, 12, 13, 21, 22],
                           positions=[0, 1, 2, 3, 1, 2],
                           slots=[20, 21, 22, 23, 29, 30],
                           cumulative_query_lengths=[4, 6], kv_lengths=[4, 3],
                           sample_order=["a", "b"], sample_rows_head=[3, 5],
                           splice_order=["a", "b"], splice_rows=[3, 5],
                           bt00=5, bt10=7),
        },
        {   # :77-97
            "name": "pads_to_token_gear",
            "stager": dict(query_gear=8, sequence_gear=8, max_blocks=4,
                           block_size=4, scratch0=100),
            "requests": {"a": req([10, 11, 12], 0, [5]),
                         "b": req([20, 21], 0, [7])},
            "scheduled": [["a", 3, True], ["b", 2, True]],
            "expect": dict(real_query_tokens=5, query_tokens=8,
                           sequence_count=2, block_table_rows=3,
                           sample_rows_head=[2, 4],
                           cumulative_query_lengths=[3, 5, 8],
                           kv_lengths=[3, 2, 3], sample_order=["a", "b"],
                           padding_slot_min=400,
                           active_token_mask=[True] * 5 + [False] * 3),
        },
        {   # :134-143
            "name": "scratch_fills_block_table",
            "stager": dict(query_gear=8, sequence_gear=8, max_blocks=4,
                           block_size=4, scratch0=100),
            "requests": {"a": req([1, 2, 3], 0, [9])},
            "scheduled": [["a", 3, True]],
            "expect": dict(bt00=9, bt10=100, bt11=101, padding_slot_min=400),
        },
        {   # :146-165
            "name": "padding_inside_scratch_near_limit",
            "stager": dict(query_gear=8, sequence_gear=8, max_blocks=32,
                           block_size=16, scratch0=100),
            "requests": {"a": req(range(497), 496, range(32), prefill=497)},
            "scheduled": [["a", 1, True]],
            "expect": dict(padding_block_range=[100, 108],
                           cumulative_query_lengths=[1, 8], kv_lengths=[497, 7],
                           block_table_rows=2),
        },
        {   # :168-179
            "name": "incomplete_chunk_does_not_sample",
            "stager": dict(query_gear=8, sequence_gear=8, max_blocks=4,
                           block_size=4, scratch0=100),
            "requests": {"a": req(range(10), 0, [9], prefill=10)},
            "scheduled": [["a", 3, True]],
            "expect": dict(real_query_tokens=3,
                           cumulative_query_lengths=[3, 8], kv_lengths=[3, 5],
                           sample_order=[], sample_rows=[0] * 8,
                           block_table_rows=2),
        },
    ],
    "overflow": {  # :182-197
        "stager": dict(query_gear=4, sequence_gear=1, max_blocks=4,
                       block_size=4, scratch0=100),
        "plans": [
            {"requests": {"a": req(range(5), 0, [1, 2])},
             "scheduled": [["a", 5, True]]},
            {"requests": {"a": req([1], 0, [1]), "b": req([2], 0, [2])},
             "scheduled": [["a", 1, True], ["b", 1, True]]},
        ],
        "message": "exceeds prefill gear",
    },
}

# Eager ``_build``: reference test tests/test_input_buffers.py:153-285 (inputs);
# expected values worked out by hand (bs = 4).
build = {
    "source": "tests/test_input_buffers.py:153-285 (inputs); "
              "tests/test_graph_decode_runner.py:272-305 (marshal literals)",
    "block_size": 4,
    "cases": [
        {
            "name": "pure_decode",   # :153-164
            "requests": {str(r): runner_req(r, 5, 1, 5, [10 + 2 * r, 11 + 2 * r])
                         for r in range(3)},
            "scheduled": [["0", 1, False], ["1", 1, False], ["2", 1, False]],
            "expect": dict(token_ids=[9000, 9010, 9020], positions=[5, 5, 5],
                           slot_mapping=[45, 53, 61],
                           block_table=[[10, 11], [12, 13], [14, 15]],
                           cu_seqlens_q=[1, 2, 3], seqlens_kv=[6, 6, 6],
                           is_decode=True,
                           sample_idx={"0": 0, "1": 1, "2": 2},
                           decode_splice=[[0, "0"], [1, "1"], [2, "2"]]),
        },
        {
            "name": "mixed_prefill_decode",   # :167-182
            "requests": {"0": runner_req(0, 5, 1, 5, [10, 11]),
                         "1": runner_req(1, 4, 0, 0, [20])},
            "scheduled": [["0", 1, False], ["1", 4, True]],
            "expect": dict(token_ids=[9000, 1100, 1101, 1102, 1103],
                           positions=[5, 0, 1, 2, 3],
                           slot_mapping=[45, 80, 81, 82, 83],
                           block_table=[[10, 11], [20, 0]],
                           cu_seqlens_q=[1, 5], seqlens_kv=[6, 4],
                           is_decode=False, sample_idx={"0": 0, "1": 4},
                           decode_splice=[[0, "0"]]),
        },
        {
            "name": "chunked_prefill",   # :185-194
            "requests": {"0": runner_req(0, 10, 0, 4, [30, 31, 32])},
            "scheduled": [["0", 3, True]],
            "expect": dict(token_ids=[1004, 1005, 1006], positions=[4, 5, 6],
                           slot_mapping=[124, 125, 126],
                           block_table=[[30, 31, 32]], cu_seqlens_q=[3],
                           seqlens_kv=[7], is_decode=False,
                           sample_idx={"0": 2}, decode_splice=[]),
        },
        {
            "name": "prefix_cache_hit",   # :197-209
            "requests": {"0": runner_req(0, 8, 0, 5, [40, 41])},
            "scheduled": [["0", 3, True]],
            "expect": dict(token_ids=[1005, 1006, 1007], positions=[5, 6, 7],
                           slot_mapping=[165, 166, 167],
                           block_table=[[40, 41]], cu_seqlens_q=[3],
                           seqlens_kv=[8], is_decode=False,
                           sample_idx={"0": 2}, decode_splice=[]),
        },
        {
            "name": "spec_multi_token_drafts",   # :231-245 (token literal from :245)
            "requests": {"0": runner_req(0, 3, 1, 3, [10, 11], draft=[7, 8, 9])},
            "scheduled": [["0", 4, False]],
            "expect": dict(token_ids=[9000, 7, 8, 9], positions=[3, 4, 5, 6],
                           slot_mapping=[43, 44, 45, 46],
                           block_table=[[10, 11]], cu_seqlens_q=[4],
                           seqlens_kv=[7], is_decode=True,
                           sample_idx={"0": 3},
                           decode_splice=[[0, "0"], [1, "0"], [2, "0"], [3, "0"]]),
        },
        {
            "name": "auto_grow_two_prefills",   # :265-285
            "requests": {"0": runner_req(0, 20, 0, 0, range(5)),
                         "1": runner_req(1, 8, 0, 0, [20, 21])},
            "scheduled": [["0", 20, True], ["1", 8, True]],
            "expect": dict(token_ids=list(range(1000, 1020)) + list(range(1100, 1108)),
                           positions=list(range(20)) + list(range(8)),
                           slot_mapping=list(range(20)) + list(range(80, 88)),
                           block_table=[[0, 1, 2, 3, 4], [20, 21, 0, 0, 0]],
                           cu_seqlens_q=[20, 28], seqlens_kv=[20, 8],
                           is_decode=False, sample_idx={"0": 19, "1": 27},
                           decode_splice=[]),
        },
        {
            "name": "marshal_single_request",   # graph runner :272-285 literals
            "requests": {"a": req([10, 11, 12, 13, 14], 0, [0, 1])},
            "scheduled": [["a", 3, True]],
            "expect": dict(token_ids=[10, 11, 12], positions=[0, 1, 2],
                           slot_mapping=[0, 1, 2], block_table=[[0, 1]],
                           cu_seqlens_q=[3], seqlens_kv=[3],
                           sample_idx={"a": 2}),
        },
        {
            "name": "marshal_two_requests",   # graph runner :288-305 literals
            "requests": {"a": req(range(10), 2, [5]),
                         "b": req(range(10, 20), 0, [6, 7])},
            "scheduled": [["a", 2, True], ["b", 1, True]],
            "expect": dict(token_ids=[2, 3, 10], positions=[2, 3, 0],
                           cu_seqlens_q=[2, 3], seqlens_kv=[4, 1],
                           sample_idx={"a": 1, "b": 2},
                           block_table=[[5, 0], [6, 7]]),
        },
    ],
}


def main():
    for name, obj in [("decode_stager", decode), ("spec_decode_stager", spec),
                      ("continuation_stager", continuation),
                      ("prefill_stager", prefill), ("build", build)]:
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(obj, f, indent=1, sort_keys=True)
            f.write("\n")


if __name__ == "__main__":
    main()
