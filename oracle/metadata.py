"""CPU oracle of the reference's mega-request routing and cascade.  TEST INFRASTRUCTURE ONLY.

The reference's scheduler packs a beam-search step into one "mega" request:
``prefill ++ concat(beam tokens)`` (``vllm_gr/v1/engine/core.py:108-112``),
with ``{is_mega_decode, mega_beam_width, mega_decode_steps, prefix_len,
cache_len}`` in ``MEGA_DATA_VAR`` (``vllm_gr/v1/engine/engine_core_patch.py:258-271``;
``cache_len`` = the tokens already in the cache, i.e. the prefix-cache hit,
capped at whole prefix blocks by ``patch_get_computed_blocks``, :245-252).
Row ``k`` of such a request's scheduled tokens is the token at logical
position ``cache_len + k`` of its block-table row (vLLM's slot mapping).

Functions and how each is pinned (tests/test_oracle_metadata.py):

* ``segment_requests`` / ``build_std_mappings`` / ``build_mega_mappings`` /
  ``build`` -- the metadata lists of ``BeamAttentionMetadataBuilder``
  (``vllm_gr/v1/attention/backends/beam_attn.py:255-290``, ``:292-314``,
  ``:316-413``, ``:480-559``): the ``delta >= 2 * block_size`` standard-path
  routing of an uncached prefix (:273-282, including its write-back of
  ``cache_len`` into the request's dict), beam 0 computing the uncached
  prefix tail that every other beam's suffix shares (:354-391), and the
  chunk budget that leaves later beams partially run or skipped (:351-366).
  Pinned by hand-worked cases (W=3, P=20, block 16, t=2: complete, budget-cut
  and standard-routed; a mixed batch).
* ``cascade`` -- ``BeamAttentionImpl.cascade_attention`` over those lists in
  float64 (``beam_attn.py:629-701``): the standard requests' causal pass over
  their block-table rows, the non-causal prefix pass of every mega row over
  ``cache_len`` keys, the causal suffix pass over the KV gathered through
  ``slot_mapping[mega_prefix_indices][mega_suffix_slot_mapping_out]``
  (``extract_suffix_kv``, :62-117) and the LSE merge (``merge_attn_states``).
  Pinned against ``dense_by_position`` (below) on the reference test's grid,
  against brute force on a tiny case, and by the invariance of a complete
  step's output to where the cache hit ends.
* ``prepare_inputs`` / ``dense_by_position`` -- the reference kernel test's
  inputs and its own reference (``tests/kernels/attention/
  test_cascade_beam_flash_attn.py:92-188``, ``:191-319``): every beam's KV
  materialised by logical position (prefix, shared tail, the beam's own
  tokens) and one causal varlen pass.  ``dense_by_position`` is checked by
  brute force on a tiny case.
"""

from __future__ import annotations

import numpy as np


# ---- the builder's routing (beam_attn.py:255-413) ----------------------------

def segment_requests(num_reqs, req_ids, mega_data, q_starts, block_size):
    """``_segment_requests`` (beam_attn.py:255-290).  Mutates the request's
    dict as the reference does (``mdata["cache_len"] = cache_len`` after a
    standard-routed prefix, :280)."""
    std_reqs, mega_idx, plens, widths, steps, clens, qoffs = [], [], [], [], [], [], []
    for i in range(num_reqs):
        rid = req_ids[i] if i < len(req_ids) else None
        md = mega_data.get(rid, {}) if rid else {}
        if md.get("is_mega_decode", False):
            mega_idx.append(i)
            prefix_len, cache_len = md["prefix_len"], md["cache_len"]
            delta = prefix_len - cache_len
            q_off = 0
            if delta > 0 and delta >= 2 * block_size:
                q_len = q_starts[i + 1] - q_starts[i]
                std_q = min(delta, q_len)
                std_kv = cache_len + std_q
                cache_len += std_q
                md["cache_len"] = cache_len
                std_reqs.append((i, std_q, std_kv))
                q_off = std_q
            plens.append(prefix_len)
            widths.append(md["mega_beam_width"])
            steps.append(md["mega_decode_steps"])
            clens.append(cache_len)
            qoffs.append(q_off)
        else:
            std_reqs.append((i, None, None))
    return std_reqs, mega_idx, plens, widths, steps, clens, qoffs


def build_std_mappings(std_reqs, q_starts):
    """``_build_std_mappings`` (beam_attn.py:292-314)."""
    idx, qls, kvls, reqs = [], [], [], []
    for i, std_q, std_kv in std_reqs:
        q0, q1 = q_starts[i], q_starts[i + 1]
        ql = q1 - q0 if std_q is None else std_q
        if ql == 0:
            continue
        idx.extend(range(q0, q0 + ql))
        qls.append(ql)
        kvls.append(std_kv)
        reqs.append(i)
    return idx, qls, kvls, reqs


def build_mega_mappings(mega_idx, plens, widths, steps, clens, qoffs, q_starts):
    """``_build_mega_mappings`` (beam_attn.py:316-413).  Returns the prefix
    rows, prefix group q lengths and seq lengths, the per-beam suffix q and
    seq lengths, the block-table row (request index) of each prefix group and
    the suffix slot map (indices into the mega rows' slot mapping)."""
    pidx, pql, psl, sql, ssl, pbt_req, smap = [], [], [], [], [], [], []
    out_slot = 0
    for i, P, w, t, C, qo in zip(mega_idx, plens, widths, steps, clens, qoffs):
        q_start = q_starts[i] + qo
        q_len = q_starts[i + 1] - q_start
        if w == 0 or t == 0 or q_len <= 0:
            continue
        q_curr = q_start
        budget = q_len
        groups = []
        tail = P - C
        assert tail >= 0, f"prefix_len: {P}, cache_len: {C}"
        shared = list(range(out_slot, out_slot + tail))
        for b in range(w):
            if budget <= 0:
                break
            if b == 0:
                unc = min(budget, tail + t)
                slen = unc
            else:
                unc = min(budget, t)
                slen = tail + unc
            if unc <= 0:
                continue
            if groups:
                groups[-1][1] += unc
            else:
                groups.append([q_curr, unc, C])
            if b == 0:
                smap.extend(range(out_slot, out_slot + unc))
            else:
                smap.extend(shared)
                smap.extend(range(out_slot, out_slot + unc))
            sql.append(unc)
            ssl.append(slen)
            q_curr += unc
            budget -= unc
            out_slot += unc
        for g0, gl, gc in groups:
            pidx.extend(range(g0, g0 + gl))
            pql.append(gl)
            psl.append(gc)
            pbt_req.append(i)
    return pidx, pql, psl, sql, ssl, pbt_req, smap


def build(num_reqs, req_ids, mega_data, q_starts, block_size):
    """The lists ``BeamAttentionMetadataBuilder.build`` turns into tensors
    (beam_attn.py:480-559), as a dict."""
    std_reqs, *mega = segment_requests(num_reqs, req_ids, mega_data, q_starts, block_size)
    std_idx, std_ql, std_kvl, std_req = build_std_mappings(std_reqs, q_starts)
    pidx, pql, psl, sql, ssl, pbt_req, smap = build_mega_mappings(*mega, q_starts)
    return dict(std_indices=std_idx, std_q_lens=std_ql, std_kv_lens=std_kvl, std_req_idxs=std_req,
                mega_prefix_indices=pidx, mega_prefix_q_lens=pql, mega_prefix_seq_lens=psl,
                mega_suffix_q_lens=sql, mega_suffix_seq_lens=ssl, mega_prefix_bt_reqs=pbt_req,
                mega_suffix_slot_mapping_out=smap)


# ---- the cascade over those lists (beam_attn.py:629-701) --------------------

def _attend(q, k, v, scale, softcap, causal):
    """Float64 attention of ``q [M, Hq, D]`` over ``k, v [S, Hkv, D]``
    (bottom-right causal when ``causal``); returns ``(out [M, Hq, D], lse
    [M, Hq])``, 0 and -inf for a row without keys."""
    M, Hq, D = q.shape
    S, Hkv = k.shape[0], k.shape[1]
    G = Hq // Hkv
    out = np.zeros((M, Hq, D))
    lse = np.full((M, Hq), -np.inf)
    if S == 0 or M == 0:
        return out, lse
    kk = np.repeat(k, G, axis=1)
    vv = np.repeat(v, G, axis=1)
    s = np.einsum("mhd,shd->hms", q, kk) * scale
    if softcap and softcap > 0:
        s = softcap * np.tanh(s / softcap)
    if causal:
        vis = np.arange(S)[None, :] <= (S - M + np.arange(M))[:, None]
        s = np.where(vis[None], s, -np.inf)
    m = s.max(axis=2, keepdims=True)
    ok = np.isfinite(m)
    m = np.where(ok, m, 0.0)
    e = np.exp(s - m)
    den = e.sum(axis=2, keepdims=True)
    o = np.einsum("hms,shd->mhd", e / np.where(den > 0, den, 1.0), vv)
    out = np.where(ok.transpose(1, 0, 2), o, 0.0)
    lse = np.where(ok[..., 0], (m + np.log(np.where(den > 0, den, 1.0)))[..., 0], -np.inf).T
    return out, lse


def _paged(cache, bt_row, n, block_size):
    pos = np.arange(n)
    return cache[np.asarray(bt_row, np.int64)[pos // block_size], pos % block_size]


def cascade(query, k_cache, v_cache, block_table, seq_lens, slot_mapping, md, *, scale, softcap=0.0,
            block_size, output=None):
    """Float64 ``cascade_attention`` (beam_attn.py:629-701) over the lists of
    :func:`build`.  ``query [T, Hq, D]``; caches ``[NB, bs, Hkv, D]``;
    ``block_table [R, nb]``; ``seq_lens [R]`` (the common metadata's);
    ``slot_mapping [T]`` flat slots.  Rows the metadata does not route keep
    ``output``'s values (zeros by default)."""
    q = np.asarray(query, np.float64)
    kc = np.asarray(k_cache, np.float64)
    vc = np.asarray(v_cache, np.float64)
    out = np.zeros_like(q) if output is None else np.array(output, np.float64)
    # standard requests: causal over their block-table rows (:643-654)
    r0 = 0
    for j, (i, ql) in enumerate(zip(md["std_req_idxs"], md["std_q_lens"])):
        rows = md["std_indices"][r0:r0 + ql]
        r0 += ql
        kvl = md["std_kv_lens"][j]
        kvl = int(seq_lens[i]) if kvl is None else kvl
        o, _ = _attend(q[rows], _paged(kc, block_table[i], kvl, block_size),
                       _paged(vc, block_table[i], kvl, block_size), scale, softcap, True)
        out[rows] = o
    pidx = md["mega_prefix_indices"]
    if not pidx:
        return out
    mq = q[pidx]
    # prefix pass: non-causal over cache_len keys of the request's row (:656-678)
    po = np.zeros_like(mq)
    plse = np.full(mq.shape[:2], -np.inf)
    r0 = 0
    for gl, gc, i in zip(md["mega_prefix_q_lens"], md["mega_prefix_seq_lens"], md["mega_prefix_bt_reqs"]):
        o, l = _attend(mq[r0:r0 + gl], _paged(kc, block_table[i], gc, block_size),
                       _paged(vc, block_table[i], gc, block_size), scale, softcap, False)
        po[r0:r0 + gl], plse[r0:r0 + gl] = o, l
        r0 += gl
    # suffix: KV of the mega rows' own slots, gathered by the slot map (:679-684)
    slots = np.asarray(slot_mapping, np.int64)[np.asarray(pidx, np.int64)][
        np.asarray(md["mega_suffix_slot_mapping_out"], np.int64)]
    nbk = kc.shape[0] * kc.shape[1]
    ck = kc.reshape(nbk, *kc.shape[2:])[slots]
    cv = vc.reshape(nbk, *vc.shape[2:])[slots]
    if len(slots) == 0:
        out[pidx] = po
        return out
    so = np.zeros_like(mq)
    slse = np.full(mq.shape[:2], -np.inf)
    r0 = k0 = 0
    for sq, sk in zip(md["mega_suffix_q_lens"], md["mega_suffix_seq_lens"]):
        o, l = _attend(mq[r0:r0 + sq], ck[k0:k0 + sk], cv[k0:k0 + sk], scale, softcap, True)
        so[r0:r0 + sq], slse[r0:r0 + sq] = o, l
        r0 += sq
        k0 += sk
    # merge_attn_states (:697-699)
    m = np.maximum(plse, slse)
    m = np.where(np.isfinite(m), m, 0.0)
    wp = np.exp(plse - m)
    ws = np.exp(slse - m)
    den = wp + ws
    merged = (po * wp[..., None] + so * ws[..., None]) / np.where(den > 0, den, 1.0)[..., None]
    out[pidx] = merged
    return out


# ---- the reference kernel test's inputs and its dense reference -------------

def prepare_inputs(batch_size, beam_width, num_heads, num_kv_heads, head_size, q_seq_len, kv_seq_len,
                   block_size, suffix_kv_len, seed=0, cache_len=None):
    """The inputs of ``prepare_inputs`` (test_cascade_beam_flash_attn.py:92-188),
    drawn with numpy (float64 N(0,1) x 1/sqrt(head_size)): per request a
    contiguous run of blocks holding ``shared + W * suffix`` tokens, W *
    ``q_seq_len`` query rows, and the slot mapping of rows written from
    ``cache_len`` (default: the whole prefix blocks, ``floor(shared / bs) *
    bs`` as the test computes it; it is the cache hit the scheduler reports).
    Returns a dict (numpy arrays + the scalars)."""
    rng = np.random.default_rng(seed)
    R, W = batch_size, beam_width
    scale = 1.0 / head_size ** 0.5
    shared = kv_seq_len - suffix_kv_len
    mega = shared + W * suffix_kv_len
    bpr = (mega + block_size - 1) // block_size
    q = rng.standard_normal((R * W * q_seq_len, num_heads, head_size)) * scale
    k = rng.standard_normal((R * bpr, block_size, num_kv_heads, head_size)) * scale
    v = rng.standard_normal((R * bpr, block_size, num_kv_heads, head_size)) * scale
    bt = np.arange(R * bpr, dtype=np.int32).reshape(R, bpr)
    chunk = W * q_seq_len
    C = (shared // block_size) * block_size if cache_len is None else cache_len
    assert 0 <= C <= shared
    write = min(shared - C + W * suffix_kv_len, chunk)
    slot = np.full(R * chunk, -1, np.int64)  # rows past the request's tokens: no slot
    for i in range(R):
        phys = (bt[i].astype(np.int64)[:, None] * block_size + np.arange(block_size)).reshape(-1)
        slot[i * chunk:i * chunk + write] = phys[C:C + write]
    return dict(query=q, key_cache=k, value_cache=v, block_tables=bt, seq_lens=np.full(R, mega, np.int32),
                slot_mapping=slot, scale=scale, num_reqs=R, beam_width=W, q_seq_len=q_seq_len,
                shared_tokens_len=shared, suffix_kv_len=suffix_kv_len, block_size=block_size,
                cache_len=C, max_seq_len=mega)


def dense_by_position(inp, softcap=0.0):
    """``run_reference_attention`` (test_cascade_beam_flash_attn.py:191-319) in
    float64: per beam, prefix ``[0, cache_len)``, the shared tail and the
    beam's own tokens by logical position, one causal varlen pass; unused
    rows zero.  The reference packs the rows of all requests back to back
    from row 0; here request i's rows start at its own first query row
    (``i * W * q_seq_len``), the row the cascade path reads -- the two agree
    whenever every request uses its whole chunk, as on the reference test's
    grid."""
    q = inp["query"]
    out = np.zeros_like(q)
    bs, W, t = inp["block_size"], inp["beam_width"], inp["suffix_kv_len"]
    P = inp["shared_tokens_len"]
    C = inp["cache_len"]
    for i in range(inp["num_reqs"]):
        row = i * W * inp["q_seq_len"]
        kseq = _paged(inp["key_cache"], inp["block_tables"][i], int(inp["seq_lens"][i]), bs)
        vseq = _paged(inp["value_cache"], inp["block_tables"][i], int(inp["seq_lens"][i]), bs)
        budget = inp["q_seq_len"] * W
        delta = max(0, C - P)
        for b in range(W):
            if budget <= 0:
                break
            if P >= C:
                tail = P - C
                if b == 0:
                    unc = min(budget, tail + t)
                    pos = np.concatenate([np.arange(C), C + np.arange(unc)])
                else:
                    unc = min(budget, t)
                    pos = np.concatenate([np.arange(P), P + b * t + np.arange(unc)])
            else:
                past = max(0, min(t, delta - b * t))
                unc = min(budget, t - past)
                if unc <= 0:
                    continue
                pos = np.concatenate([np.arange(P), P + b * t + np.arange(past + unc)])
            if unc <= 0:
                continue
            o, _ = _attend(q[row:row + unc], kseq[pos], vseq[pos], inp["scale"], softcap, True)
            out[row:row + unc] = o
            row += unc
            budget -= unc
    return out
