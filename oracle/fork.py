"""CPU oracle for beam KV fork + append.  TEST INFRASTRUCTURE ONLY.

The reference never keeps a beam's suffix KV across steps: every decode step
it rebuilds each child's suffix as ``parent suffix ++ new token``
(``vllm_gr/entrypoints/openai/serving_engine.py:113-120``: child tokens are
``all_beams[new_idx].tokens[prefix_len:]``, i.e. the selected parent's
tokens plus the chosen token; ``vllm_gr/v1/engine/core.py:108-112`` packs them)
and recomputes their KV.  The build keeps that KV resident in paged blocks
and forks it instead.  The fork contract (no reference counterpart; the
child-content rule is the reference's):

For request ``r`` with beams ``n = r*W + b`` and ``parent[r, c]`` in ``[0, W)``:

* a parent ``p`` with at least one child hands its block-table row to its
  **lowest-index child**, in place;
* every other child (a copy-on-write child) takes the row of a parent with no
  children **of the same request**, matched by rank: the k-th copy-on-write
  child in ascending ``c`` gets the row of the k-th childless parent in
  ascending ``p``.  The counts always match, so each request's set of rows is
  permuted and no allocator is needed;
* a copy-on-write child receives a copy of the parent's ``suffix_len[p]``
  valid tokens (K and V, all KV heads) into its new row;
* ``new_suffix_len[c] = suffix_len[p]``; with an append, the child's new K/V
  token is written at logical position ``new_suffix_len[c]`` of its row and
  the length grows by one (the ``reshape_and_cache_flash`` role,
  ``vllm_gr/v1/attention/backends/beam_attn.py:727-732``).

Functions and how each is pinned (tests/test_oracle_fork.py):

* ``fork_tables`` -- pinned by the invariants: per-request row multiset is a
  permutation, no row is owned by two beams, every child's materialised
  suffix equals its parent's, childless parents' rows are each reused exactly
  once; plus hand-worked known answers (all-same-parent, identity,
  reversal).
* ``fork_append`` -- pinned by: each child's gathered suffix (via
  ``attention.gather_tokens``) equals ``parent suffix ++ new token``; tokens
  outside every live suffix are untouched.
* ``append_tokens`` / ``reshape_and_cache`` -- slot arithmetic
  ``slot = block * block_size + offset`` (``beam_attn.py:77-85``); pinned by
  a round trip through ``gather_tokens``.
"""

from __future__ import annotations

import numpy as np


def fork_tables(parent: np.ndarray, suffix_bt: np.ndarray, suffix_len: np.ndarray):
    """New block-table rows and lengths after a fork (before any append).

    ``parent``: ``[R, W]`` int; ``suffix_bt``: ``[R*W, S]``; ``suffix_len``:
    ``[R*W]``.  Returns ``(new_bt, new_len, src_row)`` where ``src_row[n]`` is
    the beam whose *old* row supplies child ``n``'s tokens (its parent) and
    ``cow[n]`` says whether a copy is needed.
    """
    parent = np.asarray(parent, dtype=np.int64)
    R, W = parent.shape
    suffix_bt = np.asarray(suffix_bt)
    suffix_len = np.asarray(suffix_len)
    new_bt = np.empty_like(suffix_bt)
    new_len = np.empty_like(suffix_len)
    src = np.empty(R * W, dtype=np.int64)
    cow = np.zeros(R * W, dtype=bool)
    for r in range(R):
        par = parent[r]
        if par.min() < 0 or par.max() >= W:
            raise ValueError(f"parent index out of range in request {r}")
        first_child = {}
        for c in range(W):
            first_child.setdefault(int(par[c]), c)
        childless = [p for p in range(W) if p not in first_child]
        cow_children = [c for c in range(W) if first_child[int(par[c])] != c]
        assert len(childless) == len(cow_children)
        for c in range(W):
            n = r * W + c
            p = r * W + int(par[c])
            src[n] = p
            new_len[n] = suffix_len[p]
        for c in range(W):
            if first_child[int(par[c])] == c:
                new_bt[r * W + c] = suffix_bt[r * W + int(par[c])]
        for c, p_free in zip(cow_children, childless):
            new_bt[r * W + c] = suffix_bt[r * W + p_free]
            cow[r * W + c] = True
    return new_bt, new_len, src, cow


def _write_token(cache, row, pos, block_size, values):
    cache[int(row[pos // block_size]), pos % block_size] = values


def fork_append(parent, suffix_bt, suffix_len, k_cache, v_cache, k_new=None, v_new=None,
                *, block_size):
    """Fork (and optionally append one token per beam) on copies of the caches.

    ``k_cache``/``v_cache``: ``[num_blocks, block_size, Hkv, D]`` (any dtype;
    copied bit for bit).  ``k_new``/``v_new``: ``[R*W, Hkv, D]`` or None.
    Returns ``(new_bt, new_len, k_cache', v_cache')``.
    """
    new_bt, new_len, src, cow = fork_tables(parent, suffix_bt, suffix_len)
    kc = np.array(k_cache, copy=True)
    vc = np.array(v_cache, copy=True)
    old_bt = np.asarray(suffix_bt)
    for n in np.nonzero(cow)[0]:
        p = src[n]
        for j in range(int(new_len[n])):
            b_src, o = int(old_bt[p][j // block_size]), j % block_size
            b_dst = int(new_bt[n][j // block_size])
            kc[b_dst, o] = k_cache[b_src, o]
            vc[b_dst, o] = v_cache[b_src, o]
    new_len = np.array(new_len, copy=True)
    if k_new is not None:
        cap = new_bt.shape[1] * block_size
        for n in range(new_bt.shape[0]):
            pos = int(new_len[n])
            if pos >= cap:
                raise ValueError(f"beam {n}: suffix full ({pos} >= {cap})")
            _write_token(kc, new_bt[n], pos, block_size, k_new[n])
            _write_token(vc, new_bt[n], pos, block_size, v_new[n])
            new_len[n] = pos + 1
    return new_bt, new_len, kc, vc


def append_tokens(suffix_bt, suffix_len, k_cache, v_cache, k_new, v_new, *, block_size):
    """Append one token per beam at ``suffix_len[n]`` (no fork)."""
    kc = np.array(k_cache, copy=True)
    vc = np.array(v_cache, copy=True)
    new_len = np.array(suffix_len, copy=True)
    cap = np.asarray(suffix_bt).shape[1] * block_size
    for n in range(len(new_len)):
        pos = int(new_len[n])
        if pos >= cap:
            raise ValueError(f"beam {n}: suffix full ({pos} >= {cap})")
        _write_token(kc, suffix_bt[n], pos, block_size, k_new[n])
        _write_token(vc, suffix_bt[n], pos, block_size, v_new[n])
        new_len[n] = pos + 1
    return new_len, kc, vc


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping):
    """Scatter ``key/value [T, Hkv, D]`` to flat slots (``-1`` = skip), the
    role of vLLM's ``reshape_and_cache_flash`` (``beam_attn.py:727-732``)."""
    kc = np.array(k_cache, copy=True)
    vc = np.array(v_cache, copy=True)
    bs = kc.shape[1]
    for t, s in enumerate(np.asarray(slot_mapping, dtype=np.int64)):
        if s < 0:
            continue
        kc[s // bs, s % bs] = key[t]
        vc[s // bs, s % bs] = value[t]
    return kc, vc
