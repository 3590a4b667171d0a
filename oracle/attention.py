"""Float64 CPU oracle for BeamAttention decode.  TEST INFRASTRUCTURE ONLY.

Model of one decode step (the build's data layout; the paged cache keeps the
reference's ``[num_blocks, block_size, num_kv_heads, head_dim]`` per-K/V shape,
``vllm_gr/v1/attention/backends/beam_attn.py:784-785``):

* request ``r`` owns a shared prefix of ``prefix_len[r]`` tokens, addressed by
  block-table row ``prefix_bt[r]``;
* its beams are ``beam_start[r] .. beam_start[r+1]-1``; beam ``n`` owns a
  private suffix of ``suffix_len[n]`` tokens; suffix token ``j`` sits at
  logical position ``suffix_start[n] + j`` of block-table row ``suffix_bt[n]``;
* each beam carries ``T`` query tokens (rows ``n*T .. n*T+T-1`` of ``q``);
  query ``i`` sees the whole prefix and suffix tokens ``j <= L - T + i``
  (bottom-right causal, the flash-attention convention used for the suffix
  pass at ``beam_attn.py:686-695``);
* GQA: query head ``h`` reads KV head ``h // (Hq // Hkv)``
  (``beam_attn.py:612``);
* scores are ``scale * q.k``, optionally soft-capped as
  ``softcap * tanh(score / softcap)`` (``beam_attn.py:607-609``);
* an empty row (no visible key) yields output 0 and LSE ``-inf``.

Functions and how each is pinned (tests/test_oracle_attention.py):

* ``beam_attention_dense`` -- per-beam materialised KV then explicit softmax,
  restating ``run_reference_attention``
  (``tests/kernels/attention/test_cascade_beam_flash_attn.py:191-319``).
  Pinned by a brute-force scalar loop on tiny shapes, by scipy
  ``logsumexp``/``softmax`` on random rows, by the closed form for identical
  keys (output = V row) and by the invariants block-permutation, beam
  independence and the W=1 / P=0 reductions.
* ``beam_attention_cascade`` -- prefix pass (non-causal, LSE) + suffix pass
  (causal, LSE) + LSE merge, restating ``cascade_attention``
  (``beam_attn.py:629-701``) and ``merge_attn_states``.  Pinned against
  ``beam_attention_dense`` (must agree to 1e-12; with sinks too, and with a
  window covering every key).  Its window / ALiBi / sinks arguments restate
  the reference's per-pass semantics (flash-attention's bottom-right
  alignment in each pass), pinned by a scalar loop written from the
  documented formulas; ``tests/test_oracle_options.py`` measures how far
  they depart from this build's absolute-position semantics.
* ``gather_tokens`` -- paged gather, restating the index arithmetic of
  ``paged_kv_to_contig_suffix_kernel`` (``beam_attn.py:62-92``).  Pinned by
  a block-permutation test.
* The optional features of ``beam_attention_dense`` (``window``, ``causal``,
  ``sinks``, ``alibi_slopes``: the ``window_size`` / ``causal`` /
  ``s_aux`` / ``alibi_slopes`` arguments the reference hands to
  flash_attn_varlen_func, ``beam_attn.py:597-625``, ``:643-695``).  A key or
  query position is its index in the row's ``[prefix ; suffix]`` sequence,
  a query sitting at its own token's.  Pinned by a brute-force scalar loop,
  by the window = the unwindowed oracle over the truncated key set, and by
  the sink closed forms ``lse' = logaddexp(lse, sink)`` and
  ``out' = out * exp(lse - lse')``.
"""

from __future__ import annotations

import numpy as np


def gather_tokens(cache: np.ndarray, bt_row: np.ndarray, positions: np.ndarray,
                  block_size: int) -> np.ndarray:
    """Rows ``cache[bt_row[p // bs], p % bs]`` for each logical position p.

    ``cache`` is ``[num_blocks, block_size, Hkv, D]``; returns ``[len, Hkv, D]``
    (``beam_attn.py:77-85``: slot = block * block_size + offset).
    """
    positions = np.asarray(positions, dtype=np.int64)
    if positions.size == 0:
        return np.zeros((0,) + cache.shape[2:], dtype=cache.dtype)
    blocks = np.asarray(bt_row, dtype=np.int64)[positions // block_size]
    return cache[blocks, positions % block_size]


def _softcap(s: np.ndarray, softcap: float) -> np.ndarray:
    if softcap and softcap > 0:
        return softcap * np.tanh(s / softcap)
    return s


def _beam_kv(k_cache, v_cache, prefix_bt, prefix_len, suffix_bt, suffix_len,
             suffix_start, r, n, block_size):
    P = int(prefix_len[r])
    L = int(suffix_len[n])
    s0 = 0 if suffix_start is None else int(suffix_start[n])
    pre_pos = np.arange(P)
    suf_pos = s0 + np.arange(L)
    kp = gather_tokens(k_cache, prefix_bt[r], pre_pos, block_size).astype(np.float64)
    vp = gather_tokens(v_cache, prefix_bt[r], pre_pos, block_size).astype(np.float64)
    ks = gather_tokens(k_cache, suffix_bt[n], suf_pos, block_size).astype(np.float64)
    vs = gather_tokens(v_cache, suffix_bt[n], suf_pos, block_size).astype(np.float64)
    return kp, vp, ks, vs


def _softmax_rows(s: np.ndarray, visible: np.ndarray, V: np.ndarray):
    """Masked softmax-weighted sum.  ``s``: ``[rows, S]`` scores, ``visible``:
    ``[rows, S]`` bool, ``V``: ``[S, D]``.  Returns ``(out [rows, D], lse [rows])``;
    rows with no visible key give 0 and ``-inf``."""
    s = np.where(visible, s, -np.inf)
    m = s.max(axis=1, initial=-np.inf)
    empty = np.isneginf(m)
    m_safe = np.where(empty, 0.0, m)
    e = np.where(visible, np.exp(s - m_safe[:, None]), 0.0)
    l = e.sum(axis=1)
    l_safe = np.where(empty, 1.0, l)
    out = (e @ V) / l_safe[:, None]
    out[empty] = 0.0
    lse = np.where(empty, -np.inf, m_safe + np.log(l_safe))
    return out, lse


def _attend_group(qg: np.ndarray, K: np.ndarray, V: np.ndarray, visible: np.ndarray,
                  scale: float, softcap: float, bias: np.ndarray | None = None,
                  sink: np.ndarray | None = None):
    """Query rows ``qg [rows, D]`` of one KV head against ``K, V [S, D]``;
    ``bias [rows, S]`` is added after the soft cap, ``sink [rows]`` joins
    each row's softmax as a logit without a value."""
    s = _softcap(scale * (qg @ K.T), softcap)
    if bias is not None:
        s = s + bias
    out, lse = _softmax_rows(s, visible, V)
    if sink is not None:
        new = np.logaddexp(lse, sink)
        out = out * np.exp(lse - new)[:, None]
        lse = new
    return out, lse


def beam_attention_dense(q, k_cache, v_cache, prefix_bt, prefix_len, beam_start,
                         suffix_bt, suffix_len, suffix_start=None, *, q_per_beam=1,
                         scale, softcap=0.0, block_size, window=(-1, -1), causal=True,
                         sinks=None, alibi_slopes=None):
    """Dense per-beam attention in float64.

    Mirrors ``run_reference_attention`` (``test_cascade_beam_flash_attn.py:191-319``):
    each beam's ``[prefix ; suffix]`` KV is materialised (``:281-282``) and the
    beam's query tokens attend causally, bottom-right aligned (``:301-315``).
    Options (flash_attn_varlen_func's, ``beam_attn.py:643-695``): key kpos is
    visible to query qpos only if ``qpos - window[0] <= kpos`` (window[0] >=
    0) and ``kpos <= qpos + window[1]`` (window[1] >= 0); ``causal=False``
    lets every query see all ``P + L`` keys (the one-beam prefill form of
    the encoder types); ``alibi_slopes[h]`` adds ``-slope * |qpos - kpos|``
    after the soft cap; ``sinks[h]`` joins head h's softmax as a logit
    without a value.

    ``q``: ``[N*T, Hq, D]``.  Returns ``(out [N*T, Hq, D] float64, lse [N*T, Hq])``.
    """
    q = np.asarray(q, dtype=np.float64)
    T = int(q_per_beam)
    NT, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    out = np.zeros((NT, Hq, D), dtype=np.float64)
    lse = np.full((NT, Hq), -np.inf, dtype=np.float64)
    for r in range(len(prefix_len)):
        for n in range(int(beam_start[r]), int(beam_start[r + 1])):
            kp, vp, ks, vs = _beam_kv(k_cache, v_cache, prefix_bt, prefix_len, suffix_bt,
                                      suffix_len, suffix_start, r, n, block_size)
            P, L = kp.shape[0], ks.shape[0]
            K = np.concatenate([kp, ks], axis=0)
            V = np.concatenate([vp, vs], axis=0)
            # visible[i, j] for query token i: whole prefix, suffix j <= L - T + i
            vis_t = np.concatenate(
                [np.ones((T, P), bool), np.arange(L)[None, :] <= (L - T + np.arange(T))[:, None]],
                axis=1)
            if not causal:
                vis_t = np.ones((T, P + L), bool)
            qpos = P + L - T + np.arange(T)  # query token i sits at its own token's position
            kpos = np.arange(P + L)
            if window[0] >= 0:
                vis_t &= kpos[None, :] >= (qpos - window[0])[:, None]
            if window[1] >= 0:
                vis_t &= kpos[None, :] <= (qpos + window[1])[:, None]
            dist = np.abs(qpos[:, None] - kpos[None, :]).astype(np.float64)  # [T, P+L]
            for hk in range(Hkv):
                qg = q[n * T:(n + 1) * T, hk * G:(hk + 1) * G].reshape(T * G, D)
                vis = np.repeat(vis_t, G, axis=0)
                heads = np.tile(np.arange(hk * G, (hk + 1) * G), T)  # row (i, g) -> head hk*G + g
                bias = None
                if alibi_slopes is not None:
                    bias = -np.asarray(alibi_slopes, np.float64)[heads][:, None] * np.repeat(dist, G, axis=0)
                sink = None if sinks is None else np.asarray(sinks, np.float64)[heads]
                o, l = _attend_group(qg, K[:, hk], V[:, hk], vis, scale, softcap, bias, sink)
                out[n * T:(n + 1) * T, hk * G:(hk + 1) * G] = o.reshape(T, G, D)
                lse[n * T:(n + 1) * T, hk * G:(hk + 1) * G] = l.reshape(T, G)
    return out, lse


def _fa_window(Lq: int, Lk: int, window, causal: bool):
    """One flash-attention pass's visibility ``[Lq, Lk]`` and ALiBi distances
    under its bottom-right alignment: query row i sits at ``i + Lk - Lq``."""
    qpos = np.arange(Lq) + Lk - Lq
    kpos = np.arange(Lk)
    vis = np.ones((Lq, Lk), bool)
    if causal:
        vis &= kpos[None, :] <= qpos[:, None]
    if window[0] >= 0:
        vis &= kpos[None, :] >= (qpos - window[0])[:, None]
    if window[1] >= 0:
        vis &= kpos[None, :] <= (qpos + window[1])[:, None]
    return vis, np.abs(qpos[:, None] - kpos[None, :]).astype(np.float64)


def merge_states(out_a, lse_a, out_b, lse_b):
    """LSE merge of two partial attention states (the role of vLLM's
    ``merge_attn_states`` at ``beam_attn.py:697-699``): both inputs are
    normalised partial outputs with their log-sum-exp; an empty side has LSE
    ``-inf`` and contributes nothing."""
    lse_a = np.asarray(lse_a, dtype=np.float64)
    lse_b = np.asarray(lse_b, dtype=np.float64)
    m = np.maximum(lse_a, lse_b)
    both_empty = np.isneginf(m)
    m_safe = np.where(both_empty, 0.0, m)
    wa = np.where(np.isneginf(lse_a), 0.0, np.exp(lse_a - m_safe))
    wb = np.where(np.isneginf(lse_b), 0.0, np.exp(lse_b - m_safe))
    tot = wa + wb
    tot_safe = np.where(tot == 0, 1.0, tot)
    out = (wa[..., None] * out_a + wb[..., None] * out_b) / tot_safe[..., None]
    out = np.where(both_empty[..., None], 0.0, out)
    lse = np.where(both_empty, -np.inf, m_safe + np.log(tot_safe))
    return out, lse


def beam_attention_cascade(q, k_cache, v_cache, prefix_bt, prefix_len, beam_start,
                           suffix_bt, suffix_len, suffix_start=None, *, q_per_beam=1,
                           scale, softcap=0.0, block_size, window=(-1, -1), sinks=None,
                           alibi_slopes=None):
    """Cascade form of the same step in float64 (``beam_attn.py:629-701``).

    (i) all query rows of a request attend the shared prefix non-causally, as
    one group, and return their LSE (``:656-678``; all beams of a request form
    one prefix group, ``:381-384``); (ii) each beam's rows attend the beam's
    suffix causally, bottom-right aligned (``:686-695``); (iii) the two
    states are merged by LSE (``:697-699``).

    The options follow the reference's per-pass arguments literally, with
    flash-attention's documented conventions for a pass of ``Lq`` query rows
    against ``Lk`` keys: query row i sits at ``i + Lk - Lq``; the window keeps
    keys ``j`` in ``[i + Lk - Lq - left, i + Lk - Lq + right]`` (a negative
    bound is unbounded); ALiBi adds ``-slope * |i + Lk - Lq - j|``.  In the
    prefix pass the request's W * T stacked rows are one sequence (row i =
    beam-major token index), with ``s_aux`` (the sinks, ``:676``) joining its
    softmax; in the suffix pass each beam's T rows face its L keys, with no
    sinks.  These are the reference's semantics, which this build departs
    from for windows and ALiBi (it places every query at its own token's
    absolute position, as ``beam_attention_dense`` does); with no window and
    no ALiBi the two agree.
    """
    q = np.asarray(q, dtype=np.float64)
    T = int(q_per_beam)
    NT, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    o_pre = np.zeros((NT, Hq, D))
    l_pre = np.full((NT, Hq), -np.inf)
    o_suf = np.zeros((NT, Hq, D))
    l_suf = np.full((NT, Hq), -np.inf)
    for r in range(len(prefix_len)):
        n0, n1 = int(beam_start[r]), int(beam_start[r + 1])
        if n1 <= n0:
            continue
        P = int(prefix_len[r])
        kp = gather_tokens(k_cache, prefix_bt[r], np.arange(P), block_size).astype(np.float64)
        vp = gather_tokens(v_cache, prefix_bt[r], np.arange(P), block_size).astype(np.float64)
        rows = slice(n0 * T, n1 * T)
        Lq = (n1 - n0) * T
        vis_p, dist_p = _fa_window(Lq, P, window, causal=False)
        for hk in range(Hkv):
            qg = q[rows, hk * G:(hk + 1) * G].reshape(-1, D)  # row (i, g): stacked row i, head hk*G + g
            heads = np.tile(np.arange(hk * G, (hk + 1) * G), Lq)
            bias = None
            if alibi_slopes is not None:
                bias = -np.asarray(alibi_slopes, np.float64)[heads][:, None] * np.repeat(dist_p, G, axis=0)
            sink = None if sinks is None else np.asarray(sinks, np.float64)[heads]
            o, l = _attend_group(qg, kp[:, hk], vp[:, hk], np.repeat(vis_p, G, axis=0),
                                 scale, softcap, bias, sink)
            o_pre[rows, hk * G:(hk + 1) * G] = o.reshape(-1, G, D)
            l_pre[rows, hk * G:(hk + 1) * G] = l.reshape(-1, G)
        for n in range(n0, n1):
            L = int(suffix_len[n])
            s0 = 0 if suffix_start is None else int(suffix_start[n])
            ks = gather_tokens(k_cache, suffix_bt[n], s0 + np.arange(L), block_size).astype(np.float64)
            vs = gather_tokens(v_cache, suffix_bt[n], s0 + np.arange(L), block_size).astype(np.float64)
            vis_t, dist_s = _fa_window(T, L, window, causal=True)
            for hk in range(Hkv):
                qg = q[n * T:(n + 1) * T, hk * G:(hk + 1) * G].reshape(T * G, D)
                heads = np.tile(np.arange(hk * G, (hk + 1) * G), T)
                bias = None
                if alibi_slopes is not None:
                    bias = -np.asarray(alibi_slopes, np.float64)[heads][:, None] * np.repeat(dist_s, G, axis=0)
                o, l = _attend_group(qg, ks[:, hk], vs[:, hk], np.repeat(vis_t, G, axis=0),
                                     scale, softcap, bias)
                o_suf[n * T:(n + 1) * T, hk * G:(hk + 1) * G] = o.reshape(T, G, D)
                l_suf[n * T:(n + 1) * T, hk * G:(hk + 1) * G] = l.reshape(T, G)
    return merge_states(o_pre, l_pre, o_suf, l_suf)
