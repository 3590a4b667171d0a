"""Writes the known-answer fixtures under tests/golden/.

The reference holds no stored golden vectors; its pins for this path are the
small hand-written examples in tests/test_batch_and_fork_unit.py.  This script
restates those examples (and hand-worked fork cases of the build's fork
contract) as data: every expected value below is worked out by hand from the
rule it names, not produced by the oracle.

    python tests/golden/make_kats.py
"""

from __future__ import annotations

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def fork_cases():
    # Each: parent [R, W]; suffix_bt [R*W, 1] (row id = beam id); suffix_len [R*W].
    # Rule: a parent's lowest-index child keeps the parent's row in place; other
    # children take childless parents' rows, k-th child (ascending) <-> k-th
    # childless parent (ascending); every child gets its parent's length.
    return [
        dict(name="identity", parent=[[0, 1, 2, 3]], suffix_bt=[[10], [11], [12], [13]],
             suffix_len=[1, 2, 3, 4],
             new_bt=[[10], [11], [12], [13]], new_len=[1, 2, 3, 4], cow=[]),
        dict(name="reversal", parent=[[3, 2, 1, 0]], suffix_bt=[[10], [11], [12], [13]],
             suffix_len=[1, 2, 3, 4],
             new_bt=[[13], [12], [11], [10]], new_len=[4, 3, 2, 1], cow=[]),
        dict(name="all_same_parent", parent=[[1, 1, 1, 1]], suffix_bt=[[10], [11], [12], [13]],
             suffix_len=[1, 2, 3, 4],
             # child 0 keeps row 11; children 1,2,3 take rows of childless 0,2,3
             new_bt=[[11], [10], [12], [13]], new_len=[2, 2, 2, 2], cow=[1, 2, 3]),
        dict(name="mixed", parent=[[2, 2, 0, 3]], suffix_bt=[[10], [11], [12], [13]],
             suffix_len=[5, 6, 7, 8],
             # parents 0 (child 2), 2 (children 0, 1), 3 (child 3); childless 1
             new_bt=[[12], [11], [10], [13]], new_len=[7, 7, 5, 8], cow=[1]),
        # the reference's abort-set example (test_batch_and_fork_unit.py:1070-1080):
        # five beams, selection uses parents 0, 2, 4 -> beams 1 and 3 are aborted.
        # With five children [0, 0, 2, 2, 4] the aborted rows are the ones recycled.
        dict(name="abort_set", parent=[[0, 0, 2, 2, 4]], suffix_bt=[[10], [11], [12], [13], [14]],
             suffix_len=[1, 1, 1, 1, 1],
             new_bt=[[10], [11], [12], [13], [14]], new_len=[1, 1, 1, 1, 1], cow=[1, 3],
             recycled_rows_of=[1, 3]),
        dict(name="two_requests", parent=[[1, 1], [0, 0]], suffix_bt=[[10], [11], [20], [21]],
             suffix_len=[3, 4, 5, 6],
             # request 0: child 0 keeps 11, child 1 takes 10; request 1: child 0 keeps 20, child 1 takes 21
             new_bt=[[11], [10], [20], [21]], new_len=[4, 4, 5, 5], cow=[1, 3]),
    ]


def prune_cases():
    # Restated from tests/test_batch_and_fork_unit.py.
    return dict(
        # 5.15 (:1163-1176): flat candidate index -> (parent beam, token)
        fork_info=dict(logprobs_num=3, all_beams_token_id=[50, 51, 52, 60, 61, 62],
                       selected=[[-0.5, 3], [-1.0, 0], [-1.5, 4]],
                       expected=[[1, 60], [0, 50], [1, 61]]),
        # 5.13 (:1109-1143): the EOS candidate leaves the pool with its score
        eos_split=dict(eos_token_id=2, logprobs_num=3, all_beams_token_id=[50, 51, 2, 60, 61, 62],
                       all_beams_logprob=[-1.0, -1.5, -0.5, -2.0, -2.5, -3.0],
                       completed_beam=0, completed_score=-0.5),
        # 5.19 (:1229-1248): best beams are the top-k by score, descending
        final_sort=dict(scores=[-5.0, -1.0, -3.0, -0.5, -2.0], k=3, expected=[-0.5, -1.0, -2.0]),
    )


def main():
    with open(os.path.join(HERE, "fork_kats.json"), "w") as f:
        json.dump({"fork": fork_cases()}, f, indent=1)
        f.write("\n")
    with open(os.path.join(HERE, "prune_kats.json"), "w") as f:
        json.dump(prune_cases(), f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
