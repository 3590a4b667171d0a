"""Pins of the fork / append oracle (oracle/fork.py), CPU only.

The reference rebuilds each child's suffix as ``parent suffix ++ chosen token``
every step (vllm_gr/entrypoints/openai/serving_engine.py:113-120,
vllm_gr/v1/engine/core.py:108-112); the build forks resident KV instead.
Checked here: the content rule through the paged gather, the table
invariants (per-request permutation, single ownership, lowest-index child
inherits in place, childless parents' rows reused once each), hand-worked
known answers from tests/golden/fork_kats.json (including the reference's
abort-set example, tests/test_batch_and_fork_unit.py:1070-1080), and the
slot arithmetic of the append / reshape_and_cache role
(vllm_gr/v1/attention/backends/beam_attn.py:77-85, 727-732).
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import attention as oa
from oracle import fork as of

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "fork_kats.json")


def _tables(R, W, S, bs, seed, max_len=None):
    rng = np.random.default_rng(seed)
    N = R * W
    NB = N * S + 5
    rows = rng.permutation(NB)[:N * S].reshape(N, S)
    cap = S * bs
    lens = rng.integers(0, (max_len or cap - 1) + 1, size=N)
    parent = rng.integers(0, W, size=(R, W))
    return parent, rows, lens, NB


def test_fork_table_invariants():
    R, W, S, bs = 3, 16, 2, 4
    for seed in range(20):
        parent, bt, ln, _ = _tables(R, W, S, bs, seed)
        new_bt, new_len, src, cow = of.fork_tables(parent, bt, ln)
        for r in range(R):
            rows_old = sorted(map(tuple, bt[r * W:(r + 1) * W]))
            rows_new = sorted(map(tuple, new_bt[r * W:(r + 1) * W]))
            assert rows_old == rows_new  # per-request permutation, no allocator
            par = parent[r]
            kids = {p: [c for c in range(W) if par[c] == p] for p in range(W)}
            childless = [p for p in range(W) if not kids[p]]
            cow_children = [c for c in range(W) if kids[par[c]][0] != c]
            assert len(childless) == len(cow_children)
            for c in range(W):
                n = r * W + c
                assert src[n] == r * W + par[c]
                assert new_len[n] == ln[r * W + par[c]]
                if kids[par[c]][0] == c:  # lowest-index child inherits in place
                    assert not cow[n]
                    np.testing.assert_array_equal(new_bt[n], bt[r * W + par[c]])
            # copy-on-write children take childless parents' rows, matched by rank
            for c, p in zip(cow_children, childless):
                assert cow[r * W + c]
                np.testing.assert_array_equal(new_bt[r * W + c], bt[r * W + p])
        # single ownership over the whole batch
        assert len(set(map(tuple, new_bt))) == R * W


def test_fork_append_content_rule():
    """Each child's materialised suffix is its parent's followed by the new token;
    tokens outside every live suffix are untouched."""
    R, W, S, bs, Hkv, D = 2, 8, 3, 4, 2, 3
    for seed in range(10):
        parent, bt, ln, NB = _tables(R, W, S, bs, 100 + seed, max_len=S * bs - 1)
        rng = np.random.default_rng(seed)
        kc = rng.integers(0, 1 << 16, size=(NB, bs, Hkv, D)).astype(np.uint16)
        vc = rng.integers(0, 1 << 16, size=(NB, bs, Hkv, D)).astype(np.uint16)
        kn = rng.integers(0, 1 << 16, size=(R * W, Hkv, D)).astype(np.uint16)
        vn = rng.integers(0, 1 << 16, size=(R * W, Hkv, D)).astype(np.uint16)
        new_bt, new_len, kc2, vc2 = of.fork_append(parent, bt, ln, kc, vc, kn, vn, block_size=bs)
        live = np.zeros((NB, bs), bool)
        for n in range(R * W):
            p = (n // W) * W + parent[n // W][n % W]
            L = int(ln[p])
            assert new_len[n] == L + 1
            old_k = oa.gather_tokens(kc, bt[p], np.arange(L), bs)
            old_v = oa.gather_tokens(vc, bt[p], np.arange(L), bs)
            got_k = oa.gather_tokens(kc2, new_bt[n], np.arange(L + 1), bs)
            got_v = oa.gather_tokens(vc2, new_bt[n], np.arange(L + 1), bs)
            np.testing.assert_array_equal(got_k[:L], old_k)
            np.testing.assert_array_equal(got_v[:L], old_v)
            np.testing.assert_array_equal(got_k[L], kn[n])
            np.testing.assert_array_equal(got_v[L], vn[n])
            for j in range(L + 1):
                live[new_bt[n][j // bs], j % bs] = True
        np.testing.assert_array_equal(kc2[~live], kc[~live])
        np.testing.assert_array_equal(vc2[~live], vc[~live])


def test_fork_detects_planted_mistake():
    """Giving copy-on-write children the childless rows in descending order
    (a plausible slip) breaks the rank-matching check above."""
    parent = np.array([[2, 2, 2, 0]])
    bt = np.arange(4).reshape(4, 1)
    ln = np.array([1, 2, 3, 4])
    new_bt, _, _, cow = of.fork_tables(parent, bt, ln)
    # childless parents 1, 3 (ascending) -> cow children 1, 2 (ascending)
    assert list(new_bt[:, 0]) == [2, 1, 3, 0]
    assert list(new_bt[:, 0]) != [2, 3, 1, 0]


def _golden():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.mark.parametrize("case", _golden()["fork"], ids=lambda c: c["name"])
def test_fork_known_answers(case):
    parent = np.array(case["parent"])
    bt = np.array(case["suffix_bt"])
    ln = np.array(case["suffix_len"])
    new_bt, new_len, _, cow = of.fork_tables(parent, bt, ln)
    assert new_bt.tolist() == case["new_bt"]
    assert new_len.tolist() == case["new_len"]
    assert np.nonzero(cow)[0].tolist() == case["cow"]
    if "recycled_rows_of" in case:
        # the reference's abort set: parents that no child selected
        # (tests/test_batch_and_fork_unit.py:1070-1080) are exactly the rows recycled
        par = set(int(p) for p in parent.reshape(-1))
        W = parent.shape[1]
        assert sorted(p for p in range(W) if p not in par) == case["recycled_rows_of"]


def test_fork_rejects_bad_parent():
    with pytest.raises(ValueError):
        of.fork_tables(np.array([[0, 4, 1, 2]]), np.arange(4).reshape(4, 1), np.zeros(4, int))


def test_append_round_trip_and_full():
    rng = np.random.default_rng(3)
    bs, S, N = 4, 2, 5
    bt = rng.permutation(20)[:N * S].reshape(N, S)
    ln = np.array([0, 3, 4, 7, 5])
    kc = rng.standard_normal((20, bs, 1, 2))
    vc = rng.standard_normal((20, bs, 1, 2))
    kn = rng.standard_normal((N, 1, 2))
    vn = rng.standard_normal((N, 1, 2))
    new_len, kc2, vc2 = of.append_tokens(bt, ln, kc, vc, kn, vn, block_size=bs)
    assert new_len.tolist() == [1, 4, 5, 8, 6]
    for n in range(N):
        got = oa.gather_tokens(kc2, bt[n], np.array([ln[n]]), bs)
        np.testing.assert_array_equal(got[0], kn[n])
        got = oa.gather_tokens(vc2, bt[n], np.array([ln[n]]), bs)
        np.testing.assert_array_equal(got[0], vn[n])
    with pytest.raises(ValueError):
        of.append_tokens(bt, np.array([0, 0, 0, 8, 0]), kc, vc, kn, vn, block_size=bs)


def test_reshape_and_cache_slots():
    """slot = block * block_size + offset; -1 skips the token."""
    rng = np.random.default_rng(5)
    kc = np.zeros((6, 4, 2, 3))
    vc = np.zeros((6, 4, 2, 3))
    key = rng.standard_normal((4, 2, 3))
    val = rng.standard_normal((4, 2, 3))
    slots = np.array([5, -1, 0, 23])
    kc2, vc2 = of.reshape_and_cache(key, val, kc, vc, slots)
    np.testing.assert_array_equal(kc2[1, 1], key[0])
    np.testing.assert_array_equal(kc2[0, 0], key[2])
    np.testing.assert_array_equal(vc2[5, 3], val[3])
    assert np.count_nonzero(kc2) == 3 * 6
