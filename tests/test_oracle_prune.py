"""Pins of the pruning oracle (oracle/prune.py + oracle/prune_ref.c), CPU only.

* exp2_neg / log_f64 against Python's float64 ``2.0 ** t`` and ``math.log``;
* row statistics against scipy's float64 logsumexp;
* prune_topk against the plain float64 restatement of the reference's
  arithmetic (serving_engine.py:511, 538-539, 566-567) and against the
  one-stage global top-k (the reference's per-beam top-K then global top-W
  structure loses nothing);
* the reference's known answers (tests/test_batch_and_fork_unit.py:1109-1176,
  1229-1248), restated in tests/golden/prune_kats.json;
* all-equal logits (lowest flat index wins ties);
* when oracle/_ref was built from the reference's sources, the reference's
  own MinHeapTuple.push_candidates_striped (vllm_gr/csrc/minheap.cpp:75-114)
  on tie-free data.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import scipy.special

from oracle import prune as op

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "prune_kats.json")


@pytest.fixture(scope="module", autouse=True)
def _built():
    op.build()


def _ulp32(x):
    return np.spacing(np.float32(abs(x)))


def test_exp2_neg_accuracy():
    ts = np.concatenate([np.linspace(-126, 0, 20001), -np.random.default_rng(0).random(5000) * 126,
                         [0.0, -0.5, -1.0, -1e-7, -124.999, -125.5, -126.0],
                         # arguments just below an integer (the row maximum's own term is one)
                         [-2.0 ** -25, -2.0 ** -30, -1e-20, -3.0 - 2.0 ** -23]]).astype(np.float32)
    worst = 0.0
    for t in ts:
        got = op.exp2_neg(float(t))
        want = 2.0 ** float(t)
        worst = max(worst, abs(got - want) / float(_ulp32(want)))
    assert worst <= 4.0, worst
    # below -126 the argument is raised to -126: the result stays normal, 2^-126
    assert op.exp2_neg(-1e30) == 2.0 ** -126 and op.exp2_neg(float("-inf")) == 2.0 ** -126
    assert op.exp2_neg(-126.5) == 2.0 ** -126 and op.exp2_neg(float("nan")) == 2.0 ** -126
    assert op.exp2_neg(0.0) == 1.0


def test_log_f64_accuracy():
    rng = np.random.default_rng(1)
    xs = np.concatenate([1.0 + rng.random(3000) * 10, np.exp(rng.random(3000) * 9), [1.0, 2.0, 8192.0,
                         math.sqrt(2), math.sqrt(0.5) * 2]])
    for s in xs:
        got = op.log_f64(float(s))
        want = math.log(float(s))
        assert abs(got - want) <= 2 * np.spacing(max(abs(want), 1e-300)), (s, got, want)
    assert op.log_f64(1.0) == 0.0


def test_row_stats_vs_scipy():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((6, 4096)) * 3).astype(np.float32)
    cum = (rng.random(6) * -20).astype(np.float32)
    m, S, lse, c = op.row_stats(x, cum)
    want = scipy.special.logsumexp(x.astype(np.float64), axis=1)
    np.testing.assert_allclose(lse, want, rtol=0, atol=1e-6)
    np.testing.assert_array_equal(m, x.max(axis=1))
    np.testing.assert_allclose(c, cum.astype(np.float64) - lse, rtol=0, atol=0)


def _rand(R, W, V, seed, sigma=3.0):
    rng = np.random.default_rng(seed)
    return ((rng.standard_normal((R, W, V)) * sigma).astype(np.float32),
            (rng.random((R, W)) * -20).astype(np.float32))


@pytest.mark.parametrize("R,W,V,k,eos", [(3, 8, 64, 8, -1), (2, 16, 256, 16, 5), (1, 4, 4096, 4, -1),
                                          (2, 32, 128, 32, 0)])
def test_prune_vs_float64_restatement(R, W, V, k, eos):
    x, cum = _rand(R, W, V, seed=R * W + V)
    got = op.prune_topk(x, cum, k, eos)
    ref = op.prune_topk_float64(x, cum, k, eos)
    for r in range(R):
        s = ref["score"][r]
        gaps = np.abs(np.diff(s))
        if np.all(gaps > 1e-9):
            np.testing.assert_array_equal(got["parent"][r], ref["parent"][r])
            np.testing.assert_array_equal(got["token"][r], ref["token"][r])
        np.testing.assert_allclose(got["score64"][r], s, rtol=0, atol=1e-6)
        np.testing.assert_array_equal(got["score"][r], got["score64"][r].astype(np.float32))


def test_two_stage_equals_global_topk():
    """Per-beam top-k, then top-k of the union == top-k over all W x V."""
    x, cum = _rand(2, 8, 200, seed=11)
    two = op.prune_topk_float64(x, cum, 8)
    x64 = x.astype(np.float64)
    logp = x64 - scipy.special.logsumexp(x64, axis=2, keepdims=True)
    for r in range(2):
        s = (cum[r].astype(np.float64)[:, None] + logp[r]).reshape(-1)
        flat = np.lexsort((np.arange(s.size), -s))[:8]
        np.testing.assert_array_equal(two["parent"][r], flat // 200)
        np.testing.assert_array_equal(two["token"][r], flat % 200)


def _kats():
    with open(GOLDEN) as f:
        return json.load(f)


def _logits_with(V, W, tops):
    """Beam b gets logits ``tops[b] = {token: logit}``, all else -40."""
    x = np.full((1, W, V), -40.0, np.float32)
    for b, d in enumerate(tops):
        for t, v in d.items():
            x[0, b, t] = v
    return x


def _cum_for(x, beam, token, score):
    """cum[beam] such that score(beam, token) == score (to fp32 rounding of cum)."""
    lse = scipy.special.logsumexp(x[0, beam].astype(np.float64))
    return np.float32(score - (x[0, beam, token] - lse))


def test_kat_fork_info():
    """Selected flat candidates map to (parent beam, token) (:1163-1176)."""
    kat = _kats()["fork_info"]
    K = kat["logprobs_num"]
    toks = kat["all_beams_token_id"]
    assert [[idx // K, toks[idx]] for _, idx in kat["selected"]] == kat["expected"]
    # the same selection produced by the fused pruning: beam 0 offers 50, 51, 52 and beam 1
    # offers 60, 61, 62; scores make (1,60) > (0,50) > (1,61) > the rest
    V = 64
    x = _logits_with(V, 2, [{50: 2.0, 51: 0.5, 52: 0.0}, {60: 2.0, 61: 1.0, 62: -1.0}])
    cum = np.array([[_cum_for(x, 0, 50, -1.0), _cum_for(x, 1, 60, -0.5)]], np.float32)
    got = op.prune_topk(x, cum, 3)
    assert [[int(p), int(t)] for p, t in zip(got["parent"][0], got["token"][0])] == kat["expected"]
    np.testing.assert_allclose(got["score"][0], [s for s, _ in kat["selected"]], atol=1e-5)


def test_kat_eos_split():
    """The EOS candidate leaves the pool with its score (:1109-1143)."""
    kat = _kats()["eos_split"]
    V, eos = 64, kat["eos_token_id"]
    lp = kat["all_beams_logprob"]
    toks = kat["all_beams_token_id"]
    K = kat["logprobs_num"]
    # logits reproduce each beam's candidate scores relative to its best one
    tops = []
    for b in range(2):
        sc = lp[b * K:(b + 1) * K]
        best = max(sc)
        tops.append({toks[b * K + j]: float(sc[j] - best) for j in range(K)})
    x = _logits_with(V, 2, tops)
    cum = np.array([[_cum_for(x, b, toks[b * K + int(np.argmax(lp[b * K:(b + 1) * K]))],
                              max(lp[b * K:(b + 1) * K])) for b in range(2)]], np.float32)
    got = op.prune_topk(x, cum, 3, eos)
    b = kat["completed_beam"]
    assert abs(float(got["eos_score"][0, b]) - kat["completed_score"]) < 1e-5
    assert np.isneginf(got["eos_score"][0, 1 - b])
    # the remaining pool: (0,50) -1.0, (0,51) -1.5, (1,60) -2.0
    assert got["token"][0].tolist() == [50, 51, 60]
    assert got["parent"][0].tolist() == [0, 0, 1]
    assert eos not in got["token"][0].tolist()


def test_kat_final_sort():
    """Best beams are the top-k by score, descending (:1229-1248)."""
    kat = _kats()["final_sort"]
    sc = kat["scores"]
    W, V = len(sc), 16
    x = _logits_with(V, W, [{3: 0.0} for _ in range(W)])
    cum = np.array([[_cum_for(x, b, 3, sc[b]) for b in range(W)]], np.float32)
    got = op.prune_topk(x, cum, kat["k"])
    np.testing.assert_allclose(got["score"][0], kat["expected"], atol=1e-5)
    assert got["parent"][0].tolist() == [3, 1, 4]


def test_all_equal_lowest_flat_index_wins():
    x = np.zeros((2, 4, 32), np.float32)
    cum = np.zeros((2, 4), np.float32)
    got = op.prune_topk(x, cum, 6)
    for r in range(2):
        assert got["parent"][r].tolist() == [0] * 6
        assert got["token"][r].tolist() == list(range(6))
    # equal logits but distinct cum: beams rank by cum, tokens ascend inside a beam
    cum = np.array([[-3, -1, -2, -4]] * 2, np.float32)
    got = op.prune_topk(x, cum, 6)
    assert got["parent"][0].tolist() == [1] * 6
    got = op.prune_topk(x, cum, 40)
    assert got["parent"][0].tolist() == [1] * 32 + [2] * 8
    assert got["token"][0].tolist() == list(range(32)) + list(range(8))


def test_unfilled_slots():
    """k larger than the surviving pool: trailing slots are (-1, -1, -inf)."""
    x = np.zeros((1, 1, 8), np.float32)
    got = op.prune_topk(x, np.zeros((1, 1), np.float32), 8, eos_token_id=0)
    assert got["token"][0].tolist() == list(range(1, 8)) + [-1]
    assert got["parent"][0, -1] == -1 and np.isneginf(got["score"][0, -1])


def test_reference_minheap_cross_check():
    """The reference's own bounded top-k over per-beam sorted candidates
    (compiled from vllm_gr/csrc/minheap.cpp by oracle/Makefile) selects the
    same candidates on tie-free data."""
    mh = op.ref_minheap_module()
    if mh is None:
        pytest.skip("oracle/_ref not built (reference sources not mounted when building)")
    R, W, V, k = 2, 16, 512, 16
    x, cum = _rand(R, W, V, seed=21)
    got = op.prune_topk(x, cum, k)
    ref64 = op.prune_topk_float64(x, cum, k)
    x64 = x.astype(np.float64)
    logp = x64 - scipy.special.logsumexp(x64, axis=2, keepdims=True)
    for r in range(R):
        scores, toks = [], []
        for b in range(W):
            order = np.lexsort((np.arange(V), -x[r, b]))[:k]
            scores.extend((cum[r, b] + logp[r, b, order]).astype(np.float32))
            toks.extend(order.astype(np.int64))
        heap = mh.MinHeapTuple(k)
        heap.push_candidates_striped(np.array(scores, np.float32), np.array(toks, np.int64), k, -1)
        sel = sorted(heap.items(), key=lambda t: -t[0])
        assert len(sel) == k
        pairs = [(idx // k, int(toks[idx])) for _, idx in sel]
        if np.all(np.abs(np.diff(ref64["score"][r])) > 1e-5):
            assert pairs == list(zip(got["parent"][r].tolist(), got["token"][r].tolist()))


def test_candidate_lists_vs_log_softmax():
    """Each beam's top-k list before EOS removal: the tokens of a stable
    (logit desc, token asc) sort, their logprobs equal to scipy's float64
    log_softmax within float32 rounding; EOS stays in the list."""
    rng = np.random.default_rng(7)
    R, W, V, k = 3, 5, 96, 6
    x = (rng.standard_normal((R, W, V)) * 3).astype(np.float32)
    x[0, 1, 10:20] = x[0, 1, 10]  # a run of ties inside the top-k
    x[0, 1, 10] += 9.0
    x[2, 3] = -np.inf  # a row without any finite logit
    cum = rng.uniform(-20, 0, (R, W))
    eos = int(np.argmax(x[1, 2]))  # the top candidate of one beam
    got = op.prune_topk(x, cum, k, eos, candidates=True)
    ls = scipy.special.log_softmax(x.astype(np.float64), axis=2)
    for r in range(R):
        for b in range(W):
            order = np.lexsort((np.arange(V), -x[r, b].astype(np.float64)))[:k]
            assert got["cand_token"][r, b].tolist() == order.tolist()
            if r == 2 and b == 3:
                assert np.all(np.isneginf(got["cand_logprob"][r, b]))
                continue
            np.testing.assert_allclose(got["cand_logprob"][r, b], ls[r, b, order], atol=2e-6, rtol=0)
    assert eos == got["cand_token"][1, 2, 0]


def test_float64_cum_matches_float64_restatement():
    """float64 scores between steps: the selected sets equal the plain float64
    restatement's wherever its gaps exceed 2e-6, the scores agree to 1e-6 (the
    float32 exp-sum of the build contract bounds the difference), and
    cumulative scores that are exact float32 values give the float32 path's
    bits."""
    rng = np.random.default_rng(8)
    R, W, V, k = 4, 8, 200, 8
    x = (rng.standard_normal((R, W, V)) * 3).astype(np.float32)
    cum = rng.uniform(-20, 0, (R, W))  # not float32 values
    got = op.prune_topk(x, cum, k)
    want = op.prune_topk_float64(x, cum, k)
    for r in range(R):
        s = np.sort(want["score"][r])[::-1]
        if np.all(np.abs(np.diff(s)) > 2e-6):
            assert set(zip(got["parent"][r], got["token"][r])) == set(zip(want["parent"][r], want["token"][r]))
    np.testing.assert_allclose(got["score64"], want["score"], atol=1e-6, rtol=0)
    c32 = cum.astype(np.float32)
    a, b = op.prune_topk(x, c32, k), op.prune_topk(x, c32.astype(np.float64), k)
    assert np.array_equal(a["score64"].view(np.int64), b["score64"].view(np.int64))
    assert np.array_equal(a["parent"], b["parent"]) and np.array_equal(a["token"], b["token"])


def test_float64_cum_planted_flip():
    """Two beams with identical logits whose scores differ by 2^-30: float64
    carrying ranks the second beam first, the float32 rounding of the same
    scores ties them and the lowest flat index (the first beam) wins."""
    x = np.tile(np.linspace(-1, 1, 8, dtype=np.float32), (1, 2, 1))
    c = -10.0 + 2.0 ** -30
    cum64 = np.array([[-10.0, c]])
    assert np.float32(c) == np.float32(-10.0)
    got64 = op.prune_topk(x, cum64, 1)
    got32 = op.prune_topk(x, cum64.astype(np.float32), 1)
    assert (got64["parent"][0, 0], got64["token"][0, 0]) == (1, 7)
    assert (got32["parent"][0, 0], got32["token"][0, 0]) == (0, 7)
    assert got64["score64"][0, 0] - got32["score64"][0, 0] == 2.0 ** -30


def test_topk_float64_global_matches_two_stage():
    """The vectorised float64 selection equals the per-beam-then-union one."""
    for seed, (R, W, V, k) in enumerate([(3, 16, 300, 16), (2, 5, 64, 7), (1, 1, 40, 3)]):
        x, cum = _rand(R, W, V, seed=100 + seed)
        g = op.topk_float64_global(x, cum, k)
        two = op.prune_topk_float64(x, cum, k)
        np.testing.assert_array_equal(g["parent"], two["parent"])
        np.testing.assert_array_equal(g["token"], two["token"])
        np.testing.assert_allclose(g["score"], two["score"], rtol=0, atol=1e-12)


def test_prune_full_size_vs_float64_mathematics():
    """At the full 64 x 128 x 8192 pruning (logits N(0, 3^2), cum U(-20, 0)),
    the C restatement selects what float64 mathematics selects, in the same
    order, for every request whose 128th/129th float64 gap exceeds 1e-6 (all
    of them at seed 0), with scores within 1e-6."""
    from vllm_gr_amd import workloads
    wl = workloads.prune_beam128(seed=0)
    x, cum = wl.logits.numpy(), wl.cum.numpy()
    ref = op.topk_float64_global(x, cum, wl.k)
    got = op.prune_topk(x, cum, wl.k)
    firm = ref["gap"] > 1e-6
    print(f"requests with a 128th/129th gap <= 1e-6: {int((~firm).sum())} of {len(firm)}")
    assert firm.sum() >= len(firm) - 2
    for r in np.nonzero(firm)[0]:
        np.testing.assert_array_equal(got["parent"][r], ref["parent"][r])
        np.testing.assert_array_equal(got["token"][r], ref["token"][r])
    np.testing.assert_allclose(got["score64"], ref["score"], rtol=0, atol=1e-6)


def test_f64_scores_vs_float32_logprob_scores():
    """Departure, measured: the float64 path scores a candidate as
    ``cum + (x - lse)`` in float64 (one rounding); the reference adds vLLM's
    float32 logprob to a Python float, ``cum + float64(float32(x - lse))``
    (serving_engine.py:511; llm.py's ``cum_logprob + lp``).  The two differ by
    up to one float32 ulp of the logprob.  At the full 64 x 128 x 8192 size
    (seed 0) they select the same (parent, token) lists in the same order for
    every request."""
    from vllm_gr_amd import workloads
    wl = workloads.prune_beam128(seed=0)
    x, cum = wl.logits.numpy(), wl.cum.numpy().astype(np.float64)
    k = wl.k
    got = op.prune_topk(x, cum, k)
    R, W, V = x.shape
    differ = 0
    for r in range(R):
        m = x[r].max(1, keepdims=True)
        lse32 = (m + np.log(np.exp(x[r] - m).sum(1, keepdims=True, dtype=np.float32))).astype(np.float32)
        lp32 = (x[r] - lse32).astype(np.float32)  # the sampler's float32 logprobs
        s = (cum[r][:, None] + lp32.astype(np.float64)).reshape(-1)
        part = np.argpartition(-s, k)[:k]
        part = part[np.lexsort((part, -s[part]))]
        differ += not np.array_equal(part, got["parent"][r] * V + got["token"][r])
    print(f"requests whose selection differs between the two score forms: {differ} of {R}")
    assert differ == 0
