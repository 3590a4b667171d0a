"""Pins of the mega-request routing oracle (oracle/metadata.py), CPU only.

* The builder's lists on hand-worked cases (every expected value below was
  worked out by hand from the rules at beam_attn.py:255-413, not by running
  the oracle): W=3 beams, shared prefix P=20, block 16, t=2 tokens per beam,
  with the cache hit at 16 (complete step; a chunk budget that cuts beam 1
  and skips beam 2), a standard-routed uncached prefix (cache hit 0, P=40),
  and a batch mixing a plain request with a mega one.
* The cascade over those lists against the reference test's own
  position-based reference (restated as ``dense_by_position``) on its
  scenario grid, against a brute-force loop on a tiny case, and invariant
  to where the cache hit ends for a complete step.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest

from oracle import metadata as om


def _mega(prefix_len, cache_len, W, t):
    return {"is_mega_decode": True, "prefix_len": prefix_len, "cache_len": cache_len, "mega_beam_width": W,
            "mega_decode_steps": t}


def test_lists_complete_step():
    # rows: tail 4 + 3 beams x 2 = 10; beam 0 takes the tail and its 2 tokens
    md = om.build(1, ["a"], {"a": _mega(20, 16, 3, 2)}, [0, 10], 16)
    assert md["std_indices"] == []
    assert md["mega_prefix_indices"] == list(range(10))
    assert md["mega_prefix_q_lens"] == [10] and md["mega_prefix_seq_lens"] == [16]
    assert md["mega_suffix_q_lens"] == [6, 2, 2]
    assert md["mega_suffix_seq_lens"] == [6, 6, 6]
    assert md["mega_suffix_slot_mapping_out"] == [0, 1, 2, 3, 4, 5] + [0, 1, 2, 3, 6, 7] + [0, 1, 2, 3, 8, 9]


def test_lists_chunk_budget():
    # 7 rows: beam 0 takes 6, beam 1 gets 1 of its 2, beam 2 none
    md = om.build(1, ["a"], {"a": _mega(20, 16, 3, 2)}, [0, 7], 16)
    assert md["mega_prefix_q_lens"] == [7]
    assert md["mega_suffix_q_lens"] == [6, 1]
    assert md["mega_suffix_seq_lens"] == [6, 5]
    assert md["mega_suffix_slot_mapping_out"] == [0, 1, 2, 3, 4, 5] + [0, 1, 2, 3, 6]


def test_lists_standard_routed_prefix():
    # P=40, nothing cached: delta 40 >= 2*16 -> rows 0..39 go to the standard
    # path over 40 keys, the mega part starts at row 40 with cache_len 40
    mega = {"a": _mega(40, 0, 2, 1)}
    md = om.build(1, ["a"], mega, [0, 42], 16)
    assert md["std_indices"] == list(range(40))
    assert md["std_q_lens"] == [40] and md["std_kv_lens"] == [40] and md["std_req_idxs"] == [0]
    assert md["mega_prefix_indices"] == [40, 41]
    assert md["mega_prefix_seq_lens"] == [40]
    assert md["mega_suffix_q_lens"] == [1, 1] and md["mega_suffix_seq_lens"] == [1, 1]
    assert md["mega_suffix_slot_mapping_out"] == [0, 1]
    assert mega["a"]["cache_len"] == 40  # written back, as the reference does
    # fewer rows than the uncached prefix: everything is standard, no mega rows
    md = om.build(1, ["a"], {"a": _mega(40, 0, 2, 1)}, [0, 30], 16)
    assert md["std_q_lens"] == [30] and md["std_kv_lens"] == [30] and md["mega_prefix_indices"] == []
    # an uncached tail below two blocks stays with beam 0
    md = om.build(1, ["a"], {"a": _mega(40, 16, 2, 1)}, [0, 26], 16)
    assert md["std_indices"] == [] and md["mega_suffix_q_lens"] == [25, 1]
    assert md["mega_suffix_seq_lens"] == [25, 25]


def test_lists_mixed_batch():
    # request 0 plain (3 rows), request 1 mega (P=20, C=16, W=3, t=2; 10 rows)
    md = om.build(2, ["p", "m"], {"m": _mega(20, 16, 3, 2)}, [0, 3, 13], 16)
    assert md["std_indices"] == [0, 1, 2] and md["std_kv_lens"] == [None] and md["std_req_idxs"] == [0]
    assert md["mega_prefix_indices"] == list(range(3, 13))
    assert md["mega_prefix_bt_reqs"] == [1]
    assert md["mega_suffix_slot_mapping_out"][:6] == [0, 1, 2, 3, 4, 5]
    with pytest.raises(AssertionError, match="prefix_len: 20, cache_len: 24"):
        om.build(1, ["a"], {"a": _mega(20, 24, 3, 2)}, [0, 6], 16)


def _brute(q, keys, vals, scale, softcap=0.0):
    """One row, scalar loops."""
    s = []
    for k in keys:
        x = scale * sum(a * b for a, b in zip(q, k))
        if softcap:
            x = softcap * math.tanh(x / softcap)
        s.append(x)
    m = max(s)
    w = [math.exp(x - m) for x in s]
    tot = sum(w)
    return [sum(wi * v[d] for wi, v in zip(w, vals)) / tot for d in range(len(q))]


def test_dense_and_cascade_brute_force_tiny():
    inp = om.prepare_inputs(1, 3, 2, 1, 4, 2, 22, 16, 2, seed=3)  # P=20, C=16, 3 beams x 2 rows
    md = om.build(1, ["a"], {"a": _mega(20, 16, 3, 2)}, [0, 6], 16)
    got = om.cascade(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_tables"], inp["seq_lens"],
                     inp["slot_mapping"], md, scale=inp["scale"], block_size=16)
    dense = om.dense_by_position(inp)
    k = inp["key_cache"].reshape(-1, 1, 4)
    v = inp["value_cache"].reshape(-1, 1, 4)
    # rows: beam 0 takes 6 (tail 4 at positions 16..19 + its 2 at 20, 21): all 6 rows
    for row in range(6):
        pos = list(range(16 + row + 1))  # row at position 16 + row sees 0 .. itself
        for h in range(2):
            want = _brute(inp["query"][row, h], k[pos, 0], v[pos, 0], inp["scale"])
            np.testing.assert_allclose(got[row, h], want, atol=1e-12)
            np.testing.assert_allclose(dense[row, h], want, atol=1e-12)


@pytest.mark.parametrize("case", [(8, 32, 8), (8, 8, 8), (4, 64, 4), (4, 16, 4), (1, 16, 4), (1, 128, 1),
                                  (4, 32, 7)])
@pytest.mark.parametrize("bs,heads,softcap", [(16, (4, 4), 0.0), (32, (8, 2), 50.0), (16, (16, 2), 0.0)])
def test_cascade_equals_dense_on_reference_grid(case, bs, heads, softcap):
    """The reference test's CASES (test_cascade_beam_flash_attn.py:37-65), two
    requests x 4 beams, head size 16: the cascade over the builder's lists
    equals the test's own position-based reference when the cache hit is the
    whole prefix blocks (what the scheduler reports)."""
    qs, kv, sfx = case
    inp = om.prepare_inputs(2, 4, heads[0], heads[1], 16, qs, kv, bs, sfx, seed=kv + qs)
    chunk = 4 * qs
    mega = {f"r{i}": _mega(inp["shared_tokens_len"], inp["cache_len"], 4, sfx) for i in range(2)}
    md = om.build(2, ["r0", "r1"], mega, [0, chunk, 2 * chunk], bs)
    got = om.cascade(inp["query"], inp["key_cache"], inp["value_cache"], inp["block_tables"], inp["seq_lens"],
                     inp["slot_mapping"], md, scale=inp["scale"], softcap=softcap, block_size=bs)
    want = om.dense_by_position(inp, softcap)
    np.testing.assert_allclose(got, want, atol=1e-12)


def test_cascade_invariant_to_cache_hit():
    """A complete step (every beam's rows present) gives each beam the same
    attention whatever part of the prefix was already cached: P=40, hits 32,
    16 (tail 24 computed by beam 0) and 0 (standard-routed), with the rows
    laid out from the hit as vLLM's slot mapping does."""
    P, W, t, bs, Hq, Hkv, D = 40, 3, 2, 16, 4, 2, 8
    rng = np.random.default_rng(5)
    nblk = (P + W * t + bs - 1) // bs
    kc = rng.standard_normal((nblk, bs, Hkv, D))
    vc = rng.standard_normal((nblk, bs, Hkv, D))
    bt = rng.permutation(nblk).astype(np.int32)[None]
    qbeams = rng.standard_normal((W * t, Hq, D))
    base = None
    for C in (32, 16, 0):
        n = P - C + W * t
        q = np.concatenate([rng.standard_normal((P - C, Hq, D)), qbeams])  # tail rows, then the beams'
        pos = C + np.arange(n)
        slot = bt[0].astype(np.int64)[pos // bs] * bs + pos % bs
        md = om.build(1, ["a"], {"a": _mega(P, C, W, t)}, [0, n], bs)
        got = om.cascade(q, kc, vc, bt, np.array([P + W * t]), slot, md, scale=0.3, block_size=bs)[P - C:]
        if base is None:
            base = got
        else:
            np.testing.assert_allclose(got, base, atol=1e-12)
