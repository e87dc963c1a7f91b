"""Writes known_answers.json: the literal known-answer cases of the reference's
own tests for this path (S/ = projects/gl-sdm/src/gl_sdm/, P/ = projects/gl-sdm/).

Nothing is imported from the reference; each case restates the inputs and
expected outputs that the cited test spells out, as data.
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    "route_highest_zero_scores": {
        "source": "P/tests/test_chunk_memory.py:54-58",
        "scores_shape": [1, 5, 2, 8], "scores_fill": 0.0, "width": 4, "tie": "highest",
        "expect_index_row": [12, 13, 14, 15], "expect_weight": 0.25,
    },
    "route_lowest_zero_scores": {
        "source": "P/tests/test_global_memory.py:134-142 (router.route with zeroed q: 2 heads, half 4)",
        "scores_shape": [2, 2, 8], "scores_fill": 0.0, "width": 4, "tie": "lowest",
        "expect_index_row": [0, 1, 2, 3], "expect_weight": 0.25,
    },
    "route_lowest_signed_zero": {
        "source": "P/tests/test_native_memory.py:27-45 (row 0 zeroed, element 0 = -0.0)",
        "cases": [[4, 2], [3, 5], [8, 64], [64, 8]], "tie": "lowest",
        "expect": "index[0, 0] == arange(count); indices strictly ascending",
    },
    "commit_stable_collisions": {
        "source": "P/tests/test_native_memory.py:95-104",
        "rows": 4, "addresses": [0, 3, 0, 0, 3], "deltas": [1e8, 0.125, -1e8, 1.0, 0.25],
        "expect": [1.0, 0.0, 0.0, 0.375],
    },
    "commit_keyed_arrival_order": {
        "source": "P/tests/test_chunk_memory.py:43-51",
        "rows": 4, "addresses": [3, 3, 3], "deltas": [1e8, -1e8, 0.125], "keys": [30, 31, 32],
        "permutation": [2, 0, 1], "expect_row3": 0.125,
    },
    "commit_unrelated_addresses": {
        "source": "P/tests/test_global_memory.py:69-73",
        "rows": 4, "addresses": [0, 3], "deltas": [1e8, 0.125], "expect_row3": 0.125,
    },
}

if __name__ == "__main__":
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(CASES, f, indent=1, sort_keys=True)
        f.write("\n")
