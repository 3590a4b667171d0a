"""Catalog of valid semantic-ID sequences (vllm_gr/entrypoints/openai/
serving_models.py:18-49) and the catalog-masked pruning oracle, on the CPU.

* ``Catalog.load`` / ``valid``: the reference's own cases
  (tests/test_catalog.py:29-65 -- expected sets copied as data);
* the device layout (``to_device`` CSR, breadth-first node ids): walking any
  prefix through the CSR arrays gives the trie's valid set and node id;
* the masked C oracle (stage-1 candidates outside the beam's valid set leave
  the pool, serving_engine.py:504-506) against the plain float64
  restatement with per-beam valid sets."""

from __future__ import annotations

import json
import os
import tempfile
import types

import numpy as np
import pytest
import torch

from oracle import prune as op
from vllm_gr_amd.entrypoints.catalog import Catalog

REF_CATALOG = [["1", "2", "3", "4", "5"], ["1", "2", "3", "6", "7"], ["8", "9", "10", "11", "12"]]


def _tok():
    def convert(seq):
        return [int(x) for x in seq] if isinstance(seq, list) else int(seq)
    return types.SimpleNamespace(convert_tokens_to_ids=convert)


def test_catalog_reference_cases():
    with tempfile.NamedTemporaryFile("w", suffix=".json", delete=False) as f:
        json.dump(REF_CATALOG, f)
        path = f.name
    try:
        c = Catalog(_tok())
        c.load(path)
    finally:
        os.remove(path)
    assert c.valid([]) == {1, 8}
    assert c.valid([1, 2, 3]) == {4, 6}
    assert c.valid([1, 2, 3, 4]) == {5}
    assert c.valid([1, 2, 3, 4, 5]) == set()
    assert c.valid([99]) == set()
    assert c.valid([1, 99]) == set()
    with pytest.raises(ValueError, match="not found"):
        Catalog(_tok()).load("/nonexistent/catalog.json")


def _csr_walk(t, prefix):
    starts, toks, kids = (x.tolist() for x in (t.node_start, t.child_token, t.child_node))
    node = 0
    for tok in prefix:
        ch = dict(zip(toks[starts[node]:starts[node + 1]], kids[starts[node]:starts[node + 1]]))
        if tok not in ch:
            return -1, set()
        node = ch[tok]
    return node, set(toks[starts[node]:starts[node + 1]])


def test_catalog_device_layout_matches_trie():
    rng = np.random.default_rng(3)
    c = Catalog()
    seqs = [rng.integers(0, 40, size=3).tolist() for _ in range(200)]
    for s in seqs:
        c.add(s)
    t = c.to_device("cpu")
    st = t.node_start.tolist()
    toks = t.child_token.tolist()
    assert st[0] == 0 and st[-1] == t.num_edges and t.num_nodes == len(st) - 1
    for n in range(t.num_nodes):  # children ascending, ids breadth-first
        ch = toks[st[n]:st[n + 1]]
        assert ch == sorted(set(ch))
    assert sorted(t.child_node.tolist()) == list(range(1, t.num_nodes))
    probes = [[]] + [s[:i] for s in seqs[:50] for i in range(1, 4)] + [[41], [seqs[0][0], 99]]
    for p in probes:
        node, valid = _csr_walk(t, p)
        assert valid == c.valid(p)
        assert node == c.node_of(p)


def test_masked_oracle_matches_float64_restatement():
    rng = np.random.default_rng(5)
    R, W, V, k = 3, 6, 64, 6
    logits = (rng.standard_normal((R, W, V)) * 3).astype(np.float32)
    cum = rng.uniform(-20, 0, (R, W)).astype(np.float32)
    valid = [[set(rng.choice(V, size=int(rng.integers(0, 20)), replace=False).tolist()) for _ in range(W)]
             for _ in range(R)]
    allowed = np.zeros((R, W, V), bool)
    for r in range(R):
        for b in range(W):
            allowed[r, b, list(valid[r][b])] = True
    got = op.prune_topk(logits, cum, k, eos_token_id=7, allowed=allowed)
    ref = op.prune_topk_float64(logits, cum, k, eos_token_id=7, valid_sets=valid)
    for r in range(R):
        fin = np.isfinite(ref["score"][r])
        assert np.array_equal(got["parent"][r][fin], ref["parent"][r][fin])
        assert np.array_equal(got["token"][r][fin], ref["token"][r][fin])
        assert np.allclose(got["score64"][r][fin], ref["score"][r][fin], atol=1e-6)
        assert np.all(got["parent"][r][~fin] == -1)
    # a beam whose valid set is everything equals the unmasked prune
    full = op.prune_topk(logits, cum, k, eos_token_id=7, allowed=np.ones((R, W, V), bool))
    plain = op.prune_topk(logits, cum, k, eos_token_id=7)
    assert all(np.array_equal(full[x], plain[x]) for x in ("parent", "token", "score"))
