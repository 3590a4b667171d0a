"""Pins of the oracle's optional attention features (CPU only).

The window, non-causal mode, ALiBi and sinks of
``oracle.attention.beam_attention_dense`` (the reference hands them to every
flash_attn_varlen_func call: window_size, causal, alibi_slopes, s_aux;
vllm_gr/v1/attention/backends/beam_attn.py:597-625, :643-695) are checked
against
* a brute-force scalar loop on a tiny batch with every feature on at once;
* the same attention without the feature built another way: a left window
  as keys whose scores are driven to -inf through K; a sink as one more key
  whose score equals the sink and whose value is zero;
* reductions: slope 0 = no ALiBi, causal=False = causal for the last query.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import attention as oa

BS = 4


def _layout(P, Ls, T, Hkv, D, seed, extra=2):
    """One request, len(Ls) beams: prefix blocks, then each beam's own blocks."""
    rng = np.random.default_rng(seed)
    npb = -(-P // BS)
    nsb = [-(-L // BS) for L in Ls]
    NB = npb + sum(nsb) + extra
    perm = rng.permutation(NB)
    kc = rng.standard_normal((NB, BS, Hkv, D))
    vc = rng.standard_normal((NB, BS, Hkv, D))
    pbt = np.full((1, max(npb, 1)), -1, np.int64)
    pbt[0, :npb] = perm[:npb]
    sbt = np.full((len(Ls), max(max(nsb), 1)), -1, np.int64)
    o = npb
    for i, n in enumerate(nsb):
        sbt[i, :n] = perm[o:o + n]
        o += n
    return kc, vc, pbt, sbt, rng


def _brute(q, kc, vc, pbt, sbt, P, Ls, T, scale, softcap, window, causal, sinks, alibi):
    N = len(Ls)
    Hq, D = q.shape[1], q.shape[2]
    Hkv = kc.shape[2]
    G = Hq // Hkv
    out = np.zeros(q.shape)
    lse = np.full(q.shape[:2], -math.inf)
    for n in range(N):
        L = Ls[n]
        keys = [(pbt[0][j // BS], j % BS) for j in range(P)] + [(sbt[n][j // BS], j % BS) for j in range(L)]
        for i in range(T):
            qpos = P + L - T + i
            for h in range(Hq):
                hk = h // G
                qv = q[n * T + i, h]
                sc, vals = [], []
                for kpos, (b, off) in enumerate(keys):
                    vis = kpos < P or not causal or (kpos - P) <= L - T + i
                    if window[0] >= 0 and kpos < qpos - window[0]:
                        vis = False
                    if window[1] >= 0 and kpos > qpos + window[1]:
                        vis = False
                    if not vis:
                        continue
                    x = scale * sum(qv[d] * kc[b, off, hk, d] for d in range(D))
                    if softcap:
                        x = softcap * math.tanh(x / softcap)
                    if alibi is not None:
                        x -= alibi[h] * abs(qpos - kpos)
                    sc.append(x)
                    vals.append(vc[b, off, hk])
                if sinks is not None:
                    sc.append(sinks[h])
                    vals.append(np.zeros(D))
                if not sc:
                    continue
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                tot = sum(w)
                out[n * T + i, h] = sum(wi * v for wi, v in zip(w, vals)) / tot
                lse[n * T + i, h] = m + math.log(tot)
    return out, lse


def _oracle(q, kc, vc, pbt, sbt, P, Ls, T, scale, **kw):
    N = len(Ls)
    return oa.beam_attention_dense(q, kc, vc, pbt, np.array([P]), np.array([0, N]), sbt, np.array(Ls),
                                   q_per_beam=T, scale=scale, block_size=BS, **kw)


@pytest.mark.parametrize("window,causal", [((3, -1), True), ((-1, -1), False), ((2, 1), False), ((0, 0), False)])
@pytest.mark.parametrize("softcap", [0.0, 5.0])
def test_brute_force_all_features(window, causal, softcap):
    P, Ls, T, Hq, Hkv, D = 6, [3, 4], 2, 4, 2, 3
    kc, vc, pbt, sbt, rng = _layout(P, Ls, T, Hkv, D, seed=len(Ls) + int(softcap))
    q = rng.standard_normal((len(Ls) * T, Hq, D))
    sinks = rng.standard_normal(Hq)
    alibi = np.abs(rng.standard_normal(Hq)) * 0.3
    want = _brute(q, kc, vc, pbt, sbt, P, Ls, T, 0.7, softcap, window, causal, sinks, alibi)
    got = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, 0.7, softcap=softcap, window=window, causal=causal,
                  sinks=sinks, alibi_slopes=alibi)
    np.testing.assert_allclose(got[0], want[0], atol=1e-12)
    np.testing.assert_allclose(got[1], want[1], atol=1e-12)


def test_left_window_equals_keys_masked_through_scores():
    """One query row (T = 1, G = 1): the keys left of the window are given
    K = -c * q, so their scores fall to about -1e6 and their weight to 0."""
    P, Ls, W = 11, [5], 4
    kc, vc, pbt, sbt, rng = _layout(P, Ls, 1, 1, 8, seed=3)
    q = rng.standard_normal((1, 1, 8))
    got = _oracle(q, kc, vc, pbt, sbt, P, Ls, 1, 0.5, window=(W, -1))
    qpos = P + Ls[0] - 1
    kc2 = kc.copy()
    keys = [(pbt[0][j // BS], j % BS) for j in range(P)] + [(sbt[0][j // BS], j % BS) for j in range(Ls[0])]
    for kpos, (b, off) in enumerate(keys):
        if kpos < qpos - W:
            kc2[b, off, 0] = -1e6 * q[0, 0] / float(q[0, 0] @ q[0, 0])
    want = _oracle(q, kc2, vc, pbt, sbt, P, Ls, 1, 0.5)
    np.testing.assert_allclose(got[0], want[0], atol=1e-12)
    np.testing.assert_allclose(got[1], want[1], atol=1e-9)


def test_sink_equals_an_extra_zero_value_key():
    """One query row: a sink s acts as one more prefix key whose score is s
    (K = s / (scale |q|^2) * q) and whose value is zero."""
    P, Ls = 7, [3]
    kc, vc, pbt, sbt, rng = _layout(P + 1, Ls, 1, 1, 5, seed=4)
    q = rng.standard_normal((1, 1, 5))
    sink, scale = 1.3, 0.4
    # the extra key is prefix position 0 of a layout one token longer; its
    # window-free effect must match the sink on the layout without it
    b0, o0 = pbt[0][0], 0
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[b0, o0, 0] = sink / (scale * float(q[0, 0] @ q[0, 0])) * q[0, 0]
    vc2[b0, o0, 0] = 0.0
    want = _oracle(q, kc2, vc2, pbt, sbt, P + 1, Ls, 1, scale)
    # the same keys without position 0: shift the prefix by one position
    pos = np.arange(1, P + 1)
    kp = kc[pbt[0][pos // BS], pos % BS]
    vp = vc[pbt[0][pos // BS], pos % BS]
    ks = kc[sbt[0][np.arange(3) // BS], np.arange(3) % BS]
    vs = vc[sbt[0][np.arange(3) // BS], np.arange(3) % BS]
    K, V = np.concatenate([kp, ks])[:, 0], np.concatenate([vp, vs])[:, 0]
    got = oa._attend_group(q[0], K, V, np.ones((1, P + 3), bool), scale, 0.0, None, np.array([sink]))
    np.testing.assert_allclose(got[0], want[0][0], atol=1e-12)
    np.testing.assert_allclose(got[1], want[1][0], atol=1e-12)


def test_reductions():
    P, Ls, T, Hq, Hkv, D = 9, [2, 5, 0], 2, 4, 2, 6
    kc, vc, pbt, sbt, rng = _layout(P, Ls, T, Hkv, D, seed=5)
    q = rng.standard_normal((len(Ls) * T, Hq, D))
    base = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, 0.3)
    zero_alibi = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, 0.3, alibi_slopes=np.zeros(Hq))
    np.testing.assert_allclose(zero_alibi[0], base[0], atol=1e-12)
    # the last query token of every beam sees every key either way
    nc = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, 0.3, causal=False)
    last = np.arange(len(Ls)) * T + T - 1
    np.testing.assert_allclose(nc[0][last], base[0][last], atol=1e-12)
    # an unbounded window is no window
    w = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, 0.3, window=(P + 20, -1))
    np.testing.assert_allclose(w[0], base[0], atol=1e-12)


# ---- the reference's per-pass option semantics, and the departure from them ----

def _brute_reference_cascade(q, kc, vc, pbt, sbt, P, Ls, T, scale, window, sinks, alibi):
    """The reference's cascade with options, written from flash-attention's
    documented conventions as scalar loops: a pass of Lq rows against Lk keys
    puts row i at i + Lk - Lq; the prefix pass stacks the request's beams'
    rows (beam-major) non-causally with the sinks; each beam's suffix pass is
    causal; the two states merge by LSE (beam_attn.py:656-699)."""
    N = len(Ls)
    Hq, D = q.shape[1], q.shape[2]
    Hkv = kc.shape[2]
    G = Hq // Hkv
    out = np.zeros(q.shape)
    lse = np.full(q.shape[:2], -math.inf)

    def attend(qv, keys, qpos, causal, hk, h, sink):
        sc, vals = [], []
        for kpos, (b, off) in enumerate(keys):
            if causal and kpos > qpos:
                continue
            if window[0] >= 0 and kpos < qpos - window[0]:
                continue
            if window[1] >= 0 and kpos > qpos + window[1]:
                continue
            x = scale * sum(qv[d] * kc[b, off, hk, d] for d in range(D))
            if alibi is not None:
                x -= alibi[h] * abs(qpos - kpos)
            sc.append(x)
            vals.append(vc[b, off, hk])
        if sink is not None:
            sc.append(sink)
            vals.append(np.zeros(D))
        if not sc:
            return np.zeros(D), -math.inf
        m = max(sc)
        w = [math.exp(x - m) for x in sc]
        return sum(wi * v for wi, v in zip(w, vals)) / sum(w), m + math.log(sum(w))

    pkeys = [(pbt[0][j // BS], j % BS) for j in range(P)]
    Lq = N * T
    for n in range(N):
        skeys = [(sbt[n][j // BS], j % BS) for j in range(Ls[n])]
        for i in range(T):
            row = n * T + i
            for h in range(Hq):
                hk = h // G
                o1, l1 = attend(q[row, h], pkeys, row + P - Lq, False, hk, h, None if sinks is None else sinks[h])
                o2, l2 = attend(q[row, h], skeys, i + Ls[n] - T, True, hk, h, None)
                m = max(l1, l2)
                if m == -math.inf:
                    continue
                w1, w2 = math.exp(l1 - m), math.exp(l2 - m)
                out[row, h] = (w1 * o1 + w2 * o2) / (w1 + w2)
                lse[row, h] = m + math.log(w1 + w2)
    return out, lse


def _cascade(q, kc, vc, pbt, sbt, P, Ls, T, scale, **kw):
    N = len(Ls)
    return oa.beam_attention_cascade(q, kc, vc, pbt, np.array([P]), np.array([0, N]), sbt, np.array(Ls),
                                     q_per_beam=T, scale=scale, block_size=BS, **kw)


@pytest.mark.parametrize("window", [(-1, -1), (3, -1), (5, 0), (2, 2)])
@pytest.mark.parametrize("extras", [False, True])
def test_reference_cascade_options_vs_scalar_loop(window, extras):
    """The oracle's restatement of the reference's per-pass options equals the
    scalar loop written from flash-attention's documented formulas."""
    P, Ls, T, Hq, Hkv, D = 7, [3, 5, 2], 2, 4, 2, 3
    kc, vc, pbt, sbt, rng = _layout(P, Ls, T, Hkv, D, seed=11 + window[0])
    q = rng.standard_normal((len(Ls) * T, Hq, D))
    sinks = rng.standard_normal(Hq) if extras else None
    alibi = rng.uniform(0.05, 0.5, Hq) if extras else None
    got = _cascade(q, kc, vc, pbt, sbt, P, Ls, T, 0.5, window=window, sinks=sinks, alibi_slopes=alibi)
    want = _brute_reference_cascade(q, kc, vc, pbt, sbt, P, Ls, T, 0.5, window, sinks, alibi)
    np.testing.assert_allclose(got[0], want[0], atol=1e-12)
    np.testing.assert_allclose(got[1], want[1], atol=1e-12)


def test_reference_cascade_agrees_without_window_or_alibi():
    """Sinks alone, or a window that covers every key: the reference's
    per-pass semantics and this build's absolute positions give the same
    attention (the sink joins the prefix pass once, as it joins the whole
    softmax once)."""
    P, Ls, T, Hq, Hkv, D = 9, [4, 2, 6], 2, 4, 2, 3
    kc, vc, pbt, sbt, rng = _layout(P, Ls, T, Hkv, D, seed=5)
    q = rng.standard_normal((len(Ls) * T, Hq, D))
    sinks = rng.standard_normal(Hq)
    for kw in (dict(sinks=sinks), dict(window=(P + 10, -1)), dict(window=(P + 10, P + 10), sinks=sinks)):
        ref = _cascade(q, kc, vc, pbt, sbt, P, Ls, T, 0.5, **kw)
        ours = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, 0.5, **kw)
        np.testing.assert_allclose(ref[0], ours[0], atol=1e-12)
        np.testing.assert_allclose(ref[1], ours[1], atol=1e-12)


def test_reference_cascade_window_alibi_departure_measured():
    """Departure, measured: with a sliding window or ALiBi the reference's
    prefix pass places a request's stacked beam rows at P - W*T + i, not at
    each query's own position P + L - T + t, so its attention differs from
    this build's.  On a W = 8, T = 1, P = 64 request with suffixes of 1-4
    tokens, a left window of 16 changes every row, and ALiBi (slopes
    2^(-8h/H)) changes them by a measurable amount; the printed maxima are
    the size of the departure."""
    P, Ls, T, Hq, Hkv, D = 64, [1, 2, 3, 4, 1, 2, 3, 4], 1, 4, 2, 8
    kc, vc, pbt, sbt, rng = _layout(P, Ls, T, Hkv, D, seed=23)
    q = rng.standard_normal((len(Ls) * T, Hq, D))
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)])
    for name, kw in (("window 16", dict(window=(16, -1))), ("alibi", dict(alibi_slopes=slopes))):
        ref_o, ref_l = _cascade(q, kc, vc, pbt, sbt, P, Ls, T, D ** -0.5, **kw)
        our_o, our_l = _oracle(q, kc, vc, pbt, sbt, P, Ls, T, D ** -0.5, **kw)
        d_o, d_l = np.abs(ref_o - our_o).max(), np.abs(ref_l - our_l).max()
        print(f"{name}: max |out difference| {d_o:.3g}, max |lse difference| {d_l:.3g}")
        assert d_o > 1e-3 and d_l > 1e-3
