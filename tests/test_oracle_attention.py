"""Pins of the float64 BeamAttention oracle (oracle/attention.py), CPU only.

Each check is independent of the oracle's own formula: a scalar brute-force
loop, scipy's logsumexp/softmax, closed forms (identical keys, softcap), and
invariants the reference's cascade relies on (block-permutation, beam
independence, GQA head mapping, the W=1 / P=0 reductions, cascade == dense
over the reference's scenario grid, tests/kernels/attention/
test_cascade_beam_flash_attn.py:33-65).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.special

from oracle import attention as oa


def _case(R=2, W=3, P=5, L=(0, 3), Hq=4, Hkv=2, D=4, bs=2, T=1, seed=0, suffix_start=False):
    """Random paged inputs: distinct physical blocks for every prefix/suffix row."""
    rng = np.random.default_rng(seed)
    N = R * W
    npb = (P + bs - 1) // bs
    lens = rng.integers(L[0], L[1] + 1, size=N)
    lens = np.maximum(lens, T) if T > 1 else lens
    s0 = rng.integers(0, 3, size=N) if suffix_start else np.zeros(N, np.int64)
    nsb = int(((lens + s0).max() + bs - 1) // bs) if N else 1
    nsb = max(nsb, 1)
    NB = R * npb + N * nsb + 3
    perm = rng.permutation(NB)
    prefix_bt = perm[:R * npb].reshape(R, npb) if npb else np.zeros((R, 0), np.int64)
    suffix_bt = perm[R * npb:R * npb + N * nsb].reshape(N, nsb)
    k_cache = rng.standard_normal((NB, bs, Hkv, D))
    v_cache = rng.standard_normal((NB, bs, Hkv, D))
    q = rng.standard_normal((N * T, Hq, D))
    beam_start = np.arange(R + 1) * W
    return dict(q=q, k_cache=k_cache, v_cache=v_cache, prefix_bt=prefix_bt,
                prefix_len=np.full(R, P), beam_start=beam_start, suffix_bt=suffix_bt,
                suffix_len=lens, suffix_start=s0 if suffix_start else None, T=T, bs=bs)


def _run(fn, c, scale=0.5, softcap=0.0):
    return fn(c["q"], c["k_cache"], c["v_cache"], c["prefix_bt"], c["prefix_len"], c["beam_start"],
              c["suffix_bt"], c["suffix_len"], c["suffix_start"], q_per_beam=c["T"], scale=scale,
              softcap=softcap, block_size=c["bs"])


def _brute(c, scale, softcap=0.0, head_map=None):
    """Scalar loops with math.exp: the decode step written from its definition."""
    q, kc, vc, bs, T = c["q"], c["k_cache"], c["v_cache"], c["bs"], c["T"]
    NT, Hq, D = q.shape
    Hkv = kc.shape[2]
    G = Hq // Hkv
    head_map = head_map or (lambda h: h // G)
    out = np.zeros((NT, Hq, D))
    lse = np.full((NT, Hq), -np.inf)
    for r in range(len(c["prefix_len"])):
        P = int(c["prefix_len"][r])
        for n in range(int(c["beam_start"][r]), int(c["beam_start"][r + 1])):
            L = int(c["suffix_len"][n])
            s0 = 0 if c["suffix_start"] is None else int(c["suffix_start"][n])
            toks = [(int(c["prefix_bt"][r][p // bs]), p % bs) for p in range(P)]
            toks += [(int(c["suffix_bt"][n][(s0 + j) // bs]), (s0 + j) % bs) for j in range(L)]
            for i in range(T):
                nvis = P + (L - T + i + 1)
                for h in range(Hq):
                    hk = head_map(h)
                    sc = []
                    for (blk, off) in toks[:max(nvis, 0)]:
                        s = scale * sum(q[n * T + i, h, d] * kc[blk, off, hk, d] for d in range(D))
                        if softcap:
                            s = softcap * math.tanh(s / softcap)
                        sc.append(s)
                    if not sc:
                        continue
                    m = max(sc)
                    w = [math.exp(s - m) for s in sc]
                    tot = sum(w)
                    lse[n * T + i, h] = m + math.log(tot)
                    for d in range(D):
                        out[n * T + i, h, d] = sum(wj * vc[blk, off, hk, d]
                                                   for wj, (blk, off) in zip(w, toks)) / tot
    return out, lse


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("suffix_start", [False, True])
def test_dense_matches_brute_force(T, suffix_start):
    c = _case(T=T, suffix_start=suffix_start, seed=T + 2 * suffix_start)
    want_o, want_l = _brute(c, 0.5)
    got_o, got_l = _run(oa.beam_attention_dense, c)
    np.testing.assert_allclose(got_o, want_o, rtol=0, atol=1e-12)
    np.testing.assert_array_equal(np.isneginf(got_l), np.isneginf(want_l))
    fin = np.isfinite(want_l)
    np.testing.assert_allclose(got_l[fin], want_l[fin], rtol=0, atol=1e-12)


def test_brute_force_detects_wrong_head_mapping():
    """A plausible GQA mistake (h % Hkv instead of h // G) changes the answer,
    so the brute-force comparison above would catch it."""
    c = _case(Hq=4, Hkv=2, seed=7, L=(1, 3))
    good, _ = _brute(c, 0.5)
    bad, _ = _brute(c, 0.5, head_map=lambda h: h % 2)
    assert np.abs(good - bad).max() > 1e-3


def test_softcap_matches_brute_force():
    c = _case(seed=3, L=(1, 3))
    want_o, want_l = _brute(c, 2.0, softcap=1.5)
    got_o, got_l = _run(oa.beam_attention_dense, c, scale=2.0, softcap=1.5)
    np.testing.assert_allclose(got_o, want_o, atol=1e-12)
    np.testing.assert_allclose(got_l, want_l, atol=1e-12)
    # softcap changes the result (scores are large enough to saturate tanh)
    plain, _ = _run(oa.beam_attention_dense, c, scale=2.0)
    assert np.abs(plain - got_o).max() > 1e-3


def test_dense_matches_scipy():
    """One query row per beam: out = softmax(scale*K q) @ V, lse = logsumexp."""
    c = _case(R=3, W=4, P=37, L=(0, 9), Hq=8, Hkv=2, D=16, bs=16, seed=11)
    out, lse = _run(oa.beam_attention_dense, c, scale=0.25)
    G = 4
    for r in range(3):
        for n in range(r * 4, r * 4 + 4):
            pos_p = np.arange(37)
            L = int(c["suffix_len"][n])
            kp = c["k_cache"][c["prefix_bt"][r][pos_p // 16], pos_p % 16]
            vp = c["v_cache"][c["prefix_bt"][r][pos_p // 16], pos_p % 16]
            pos_s = np.arange(L)
            ks = c["k_cache"][c["suffix_bt"][n][pos_s // 16], pos_s % 16]
            vs = c["v_cache"][c["suffix_bt"][n][pos_s // 16], pos_s % 16]
            K = np.concatenate([kp, ks])
            V = np.concatenate([vp, vs])
            for h in range(8):
                s = 0.25 * K[:, h // G] @ c["q"][n, h]
                np.testing.assert_allclose(lse[n, h], scipy.special.logsumexp(s), atol=1e-12)
                np.testing.assert_allclose(out[n, h], scipy.special.softmax(s) @ V[:, h // G], atol=1e-12)


def test_identical_keys_closed_form():
    """All keys equal: weights are uniform, out = mean of V, lse = s + log(n)."""
    c = _case(R=1, W=3, P=6, L=(1, 4), Hq=2, Hkv=1, D=4, bs=4, seed=5)
    c["k_cache"][:] = np.array([0.3, -1.0, 0.5, 2.0])[None, None, None, :]
    out, lse = _run(oa.beam_attention_dense, c, scale=0.7)
    for n in range(3):
        L = int(c["suffix_len"][n])
        pos = np.arange(L)
        vs = c["v_cache"][c["suffix_bt"][n][pos // 4], pos % 4, 0]
        pp = np.arange(6)
        vp = c["v_cache"][c["prefix_bt"][0][pp // 4], pp % 4, 0]
        V = np.concatenate([vp, vs])
        for h in range(2):
            s = 0.7 * float(c["q"][n, h] @ np.array([0.3, -1.0, 0.5, 2.0]))
            np.testing.assert_allclose(out[n, h], V.mean(axis=0), atol=1e-12)
            np.testing.assert_allclose(lse[n, h], s + math.log(len(V)), atol=1e-12)


def test_block_permutation_invariance():
    c = _case(R=2, W=3, P=9, L=(1, 5), bs=2, seed=9)
    base, base_l = _run(oa.beam_attention_dense, c)
    rng = np.random.default_rng(1)
    NB = c["k_cache"].shape[0]
    perm = rng.permutation(NB)  # physical block b moves to perm[b]
    d = dict(c)
    d["k_cache"] = np.empty_like(c["k_cache"])
    d["v_cache"] = np.empty_like(c["v_cache"])
    d["k_cache"][perm] = c["k_cache"]
    d["v_cache"][perm] = c["v_cache"]
    d["prefix_bt"] = perm[c["prefix_bt"]]
    d["suffix_bt"] = perm[c["suffix_bt"]]
    got, got_l = _run(oa.beam_attention_dense, d)
    np.testing.assert_array_equal(got, base)
    np.testing.assert_array_equal(got_l, base_l)


def test_beam_independence():
    c = _case(R=1, W=4, P=8, L=(2, 4), bs=4, seed=13)
    base, _ = _run(oa.beam_attention_dense, c)
    d = dict(c)
    d["k_cache"] = c["k_cache"].copy()
    blk = c["suffix_bt"][2][0]
    d["k_cache"][blk] += 1.0  # perturb beam 2's own suffix only
    got, _ = _run(oa.beam_attention_dense, d)
    for n in range(4):
        if n == 2:
            assert np.abs(got[n] - base[n]).max() > 1e-6
        else:
            np.testing.assert_array_equal(got[n], base[n])


def test_gqa_head_mapping():
    """Query heads h*G .. h*G+G-1 see KV head h and nothing else."""
    c = _case(R=1, W=2, P=7, L=(1, 3), Hq=6, Hkv=3, D=4, bs=4, seed=17)
    full, _ = _run(oa.beam_attention_dense, c)
    for hk in range(3):
        d = dict(c)
        d["k_cache"] = c["k_cache"][:, :, hk:hk + 1].copy()
        d["v_cache"] = c["v_cache"][:, :, hk:hk + 1].copy()
        d["q"] = c["q"][:, 2 * hk:2 * hk + 2].copy()
        part, _ = _run(oa.beam_attention_dense, d)
        np.testing.assert_allclose(full[:, 2 * hk:2 * hk + 2], part, atol=1e-14)


def _sdpa(q, K, V, scale):
    s = scale * K @ q
    w = np.exp(s - s.max())
    return (w / w.sum()) @ V


def test_no_prefix_is_plain_paged_decode():
    """P = 0 (the reference's "No Shared Prefix" scenario): ordinary paged decode per beam."""
    c = _case(R=1, W=3, P=0, L=(1, 6), Hq=2, Hkv=2, D=4, bs=4, seed=19)
    out, _ = _run(oa.beam_attention_dense, c, scale=0.3)
    for n in range(3):
        pos = np.arange(int(c["suffix_len"][n]))
        K = c["k_cache"][c["suffix_bt"][n][pos // 4], pos % 4]
        V = c["v_cache"][c["suffix_bt"][n][pos // 4], pos % 4]
        for h in range(2):
            np.testing.assert_allclose(out[n, h], _sdpa(c["q"][n, h], K[:, h], V[:, h], 0.3), atol=1e-12)


def test_single_beam_is_plain_paged_decode():
    """W = 1: prefix ++ suffix is one ordinary sequence."""
    c = _case(R=2, W=1, P=11, L=(2, 5), Hq=2, Hkv=1, D=4, bs=4, seed=23)
    out, _ = _run(oa.beam_attention_dense, c, scale=0.3)
    for r in range(2):
        pp = np.arange(11)
        ps = np.arange(int(c["suffix_len"][r]))
        K = np.concatenate([c["k_cache"][c["prefix_bt"][r][pp // 4], pp % 4],
                            c["k_cache"][c["suffix_bt"][r][ps // 4], ps % 4]])
        V = np.concatenate([c["v_cache"][c["prefix_bt"][r][pp // 4], pp % 4],
                            c["v_cache"][c["suffix_bt"][r][ps // 4], ps % 4]])
        for h in range(2):
            np.testing.assert_allclose(out[r, h], _sdpa(c["q"][r, h], K[:, 0], V[:, 0], 0.3), atol=1e-12)


def test_empty_rows():
    """No visible key at all (P = 0, L = 0): output 0, lse -inf."""
    c = _case(R=1, W=2, P=0, L=(0, 0), seed=29)
    out, lse = _run(oa.beam_attention_dense, c)
    assert np.all(out == 0) and np.all(np.isneginf(lse))
    out_c, lse_c = _run(oa.beam_attention_cascade, c)
    assert np.all(out_c == 0) and np.all(np.isneginf(lse_c))


# The reference's scenario grid: (beam width, shared prefix, suffix tokens)
# from test_cascade_beam_flash_attn.py:38-64, with its head pairs (:33) and
# block sizes (:35); D reduced to 16 so the float64 loops stay fast.
CASES = [(8, 32, 8), (8, 8, 8), (4, 64, 4), (4, 16, 4), (1, 16, 4), (1, 128, 1), (4, 32, 7)]


@pytest.mark.parametrize("W,P,L", CASES)
@pytest.mark.parametrize("heads", [(4, 4), (8, 2), (16, 2)])
@pytest.mark.parametrize("bs", [16, 32])
def test_cascade_equals_dense(W, P, L, heads, bs):
    Hq, Hkv = heads
    for T in (1, min(L, 3)):
        c = _case(R=2, W=W, P=P, L=(L, L), Hq=Hq, Hkv=Hkv, D=16, bs=bs, T=T, seed=W * 1000 + P + L)
        d_o, d_l = _run(oa.beam_attention_dense, c, scale=16 ** -0.5)
        c_o, c_l = _run(oa.beam_attention_cascade, c, scale=16 ** -0.5)
        np.testing.assert_allclose(c_o, d_o, rtol=0, atol=1e-12)
        np.testing.assert_allclose(c_l, d_l, rtol=0, atol=1e-12)


def test_merge_states_closed_form():
    """Merging two halves of one softmax reproduces the whole (and -inf sides drop out)."""
    rng = np.random.default_rng(31)
    s = rng.standard_normal(10)
    V = rng.standard_normal((10, 3))
    a, b = slice(0, 4), slice(4, 10)
    oa_, la = scipy.special.softmax(s[a]) @ V[a], scipy.special.logsumexp(s[a])
    ob_, lb = scipy.special.softmax(s[b]) @ V[b], scipy.special.logsumexp(s[b])
    o, l = oa.merge_states(oa_[None], np.array([la]), ob_[None], np.array([lb]))
    np.testing.assert_allclose(o[0], scipy.special.softmax(s) @ V, atol=1e-14)
    np.testing.assert_allclose(l[0], scipy.special.logsumexp(s), atol=1e-14)
    o2, l2 = oa.merge_states(oa_[None], np.array([la]), np.zeros((1, 3)), np.array([-np.inf]))
    np.testing.assert_allclose(o2[0], oa_, atol=1e-15)
    assert l2[0] == la


def test_cpu_baseline_matches_oracle():
    """The float32 torch cascade timed as the CPU baseline computes the same step (1e-5)."""
    import torch

    from oracle.cpu_baseline import cascade_decode_fp32
    c = _case(R=2, W=8, P=40, L=(1, 8), Hq=8, Hkv=2, D=32, bs=16, seed=37)
    want, _ = _run(oa.beam_attention_cascade, c, scale=32 ** -0.5)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    got = cascade_decode_fp32(t(c["q"]).float(), t(c["k_cache"]).float(), t(c["v_cache"]).float(),
                              t(c["prefix_bt"]).int(), t(c["prefix_len"]).int(), t(c["beam_start"]).int(),
                              t(c["suffix_bt"]).int(), t(c["suffix_len"]).int(), scale=32 ** -0.5,
                              block_size=16)
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=1e-5)
