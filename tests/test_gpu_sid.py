"""End-to-end semantic-ID beam decode on the GPU (prefill once, then per
step decode -> prune -> fork through the HIP kernels) against the CPU oracle
of the reference's recompute-every-beam loop (oracle/sid_beam.py).

* float32 models (generic decode kernel): the beams -- tokens and cumulative
  logprobs -- equal the oracle's (scores to 1e-4); every seed is checked to
  leave each step's selection boundary at least 1e-3 from a tie, so a
  mismatch is a defect, not rounding.  Ragged prompts over several blocks,
  forks at every step, EOS completion and begin/end tokens are covered.
* a bf16 model at head_dim 128 (the MFMA decode kernel): each returned
  beam's cumulative logprob equals the oracle's recomputation of that
  beam's tokens within a bf16 tolerance.
* the 28-layer, 2048-hidden decoder at 4 prompts x 2048 tokens x 128 beams:
  the beam path's scores against a from-scratch prefill of a few beams'
  whole token lists on the same GPU (resident-suffix decode with forks vs
  recompute, the self-consistency the reference's cascade test checks,
  tests/kernels/attention/test_cascade_beam_flash_attn.py:474-478), and
  against the oracle's float64 model (prompt-cached restatement run on the
  GPU): every beam's score by teacher forcing, and the returned set against
  a float64 beam search's own final boundary and beams.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import prune as op
from oracle import sid_beam as so
from vllm_gr_amd.entrypoints.beam_search import BeamSearchParams
from vllm_gr_amd.entrypoints.llm import LLM
from vllm_gr_amd.v1.sid_decoder import SID_DECODER_1P7B, DecoderConfig, init_weights
from vllm_gr_amd.v1.sid_runner import blocks_needed

pytestmark = pytest.mark.gpu

F32 = DecoderConfig(num_layers=2, hidden=64, num_heads=4, num_kv_heads=2, head_dim=32, ffn=96, vocab=96,
                    init_std=0.25, dtype=torch.float32)
BF16_128 = DecoderConfig(num_layers=2, hidden=256, num_heads=4, num_kv_heads=2, head_dim=128, ffn=512,
                         vocab=512, init_std=0.05, dtype=torch.bfloat16)


def _prompts(seed, lens, vocab):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (n,), generator=g).tolist() for n in lens]


def _llm(cfg, w, R, P, W, steps, eos=None):
    nb = blocks_needed(R, P, W, steps, 16) + 8
    print(f"[sid] cfg layers={cfg.num_layers} hidden={cfg.hidden} D={cfg.head_dim} dtype={cfg.dtype} "
          f"R={R} P<={P} W={W} steps={steps} blocks={nb}", flush=True)
    return LLM(cfg, weights={k: v.cuda() for k, v in w.items()}, num_blocks=nb, eos_token_id=eos)


def _assert_logprobs(got_seqs, ref_seqs, tol):
    """Every output beam's per-step logprob lists equal the oracle's: the same
    tokens at each position and logprobs within ``tol``."""
    ref = {tuple(s.tokens): s.logprobs for s in ref_seqs}
    for s in got_seqs:
        want = ref[tuple(s.tokens)]
        assert len(s.logprobs) == len(want)
        for i, (wt, wl) in enumerate(want):
            run = s.logprobs.position(i)
            assert dict(zip(wt, range(len(wt)))).keys() == {t for t, _, _ in run}
            got = {t: lp for t, lp, _ in run}
            for t, lp in zip(wt, wl):
                assert abs(got[t] - lp) <= tol, (s.tokens, i, t, got[t], lp)


def _min_margin(trace, W):
    gaps = [c[W - 1] - c[W] for c in trace if len(c) > W]
    return min(gaps) if gaps else float("inf")


@pytest.mark.parametrize("seed,lens,W,max_tokens", [
    (1, [23, 40, 17], 8, 4),     # three forks across ragged multi-block prompts
    (2, [5], 16, 5),             # short prompt: the suffix is a large share of attention
    (3, [33, 16, 64, 1], 4, 3),
])
def test_sid_beam_search_f32_matches_oracle(seed, lens, W, max_tokens):
    w = init_weights(F32, seed)
    prompts = _prompts(seed, lens, F32.vocab)
    trace = []
    ref = so.beam_search(so.decoder_next_logprobs(so.weights_f64(w), F32), prompts, W, max_tokens,
                         trace=trace)
    assert _min_margin(trace, W) > 1e-3, "seed leaves a near tie at a selection boundary"
    llm = _llm(F32, w, len(lens), max(lens), W, max_tokens)
    out = llm.beam_search([{"prompt_token_ids": p} for p in prompts], BeamSearchParams(W, max_tokens))
    for o, r in zip(out, ref):
        got = {tuple(s.tokens): s.cum_logprob for s in o.sequences}
        exp = {tuple(s.tokens): s.cum_logprob for s in r}
        assert set(got) == set(exp)
        for k in exp:
            assert abs(got[k] - exp[k]) < 1e-4, (k, got[k], exp[k])
        sc = [s.cum_logprob for s in o.sequences]
        assert sc == sorted(sc, reverse=True)
        _assert_logprobs(o.sequences, r, 1e-4)
    t = llm.last_times
    assert t.prefill_ms > 0 and len(t.step_ms) == max_tokens - 1


@pytest.mark.parametrize("seed,lens,W,max_tokens,eos", [(21, [19, 40], 8, 5, None), (22, [30, 7, 12], 16, 4, 3)])
def test_sid_beam_search_replayed_logits_exact(seed, lens, W, max_tokens, eos):
    """No tie-margin filter: the oracle's beam-search loop (the reference's
    llm.py:118-292 restated) runs over the GPU's own logits of every step,
    with the prune contract's log_softmax, so every selection -- near ties
    included -- must come out the same.  Beams, EOS completions, float64
    cumulative scores (to 1e-12: the two sides associate the float64 sum
    differently) and per-step logprob lists (tokens exact, values to 1e-6)
    agree."""
    w = init_weights(F32, seed)
    prompts = _prompts(seed, lens, F32.vocab)
    llm = _llm(F32, w, len(lens), max(lens), W, max_tokens, eos=eos)
    rec = []
    llm.logits_hook = lambda step, logits, hist: rec.append((logits.clone(), hist.clone()))
    out = llm.beam_search(prompts, BeamSearchParams(W, max_tokens))
    rows = {}
    for lg, h in rec:
        lg, h = lg.cpu().numpy(), h.cpu().numpy()
        for r in range(lg.shape[0]):
            for b in range(lg.shape[1]):
                rows[tuple(prompts[r] + h[r, b].tolist())] = lg[r, b]

    def next_logprobs(tokens):
        x = rows[tuple(tokens)]
        _, _, lse, _ = op.row_stats(x[None], np.zeros(1))
        return x.astype(np.float64) - lse[0]

    ref = so.beam_search(next_logprobs, prompts, W, max_tokens, eos_token_id=eos)
    for o, r in zip(out, ref):
        assert [s.tokens for s in o.sequences] == [s.tokens for s in r]
        for a, b in zip(o.sequences, r):
            assert abs(a.cum_logprob - b.cum_logprob) <= 1e-12, (a.tokens, a.cum_logprob, b.cum_logprob)
            assert (a.finish_reason == "stop") == (b.finish_reason == "stop")
            for i, (wt, wl) in enumerate(b.logprobs):
                run = a.logprobs.position(i)
                assert [t for t, _, _ in run] == wt
                assert max(abs(lp - v) for (_, lp, _), v in zip(run, wl)) <= 1e-6
    if eos is not None:
        assert any(s.finish_reason == "stop" for o in out for s in o.sequences)


def test_sid_beam_search_f32_eos_begin_end():
    seed, lens, W = 4, [12, 30], 8
    w = init_weights(F32, seed)
    prompts = _prompts(seed, lens, F32.vocab)
    begin, end = 7, 9
    f = so.decoder_next_logprobs(so.weights_f64(w), F32)
    # EOS = the first prompt's most likely first token, so EOS completes at step 0
    eos = int(np.argmax(f(prompts[0] + [begin])))
    trace = []
    ref = so.beam_search(f, prompts, W, 5, eos_token_id=eos, begin_token=begin, end_token=end, trace=trace)
    assert _min_margin(trace, W) > 1e-3
    assert any(s.finish_reason == "stop" for s in ref[0])
    llm = _llm(F32, w, len(lens), max(lens) + 1, W, 5, eos=eos)
    out = llm.beam_search(prompts, BeamSearchParams(W, 5, begin_token=begin, end_token=end))
    for o, r in zip(out, ref):
        got = {tuple(s.tokens): (s.cum_logprob, s.finish_reason) for s in o.sequences}
        exp = {tuple(s.tokens): (s.cum_logprob, s.finish_reason) for s in r}
        assert set(got) == set(exp)
        for k in exp:
            assert abs(got[k][0] - exp[k][0]) < 1e-4 and (got[k][1] == "stop") == (exp[k][1] == "stop")
        _assert_logprobs(o.sequences, r, 1e-4)


def test_sid_beam_search_f32_catalog():
    """A catalog of 3-token semantic IDs restricts every beam to valid
    continuations of its generated tokens: same beams as the oracle with the
    catalog rule, every output a catalog entry."""
    from vllm_gr_amd.entrypoints.catalog import Catalog
    seed, lens, W = 10, [14, 27], 8
    w = init_weights(F32, seed)
    prompts = _prompts(seed, lens, F32.vocab)
    rng = np.random.default_rng(seed)
    cat = Catalog()
    sids = set()  # about half the vocabulary valid at each level (57,600 IDs)
    for a in rng.choice(F32.vocab, 48, replace=False):
        for b in rng.choice(F32.vocab, 40, replace=False):
            for c in rng.choice(F32.vocab, 30, replace=False):
                sids.add((int(a), int(b), int(c)))
    for sid in sids:
        cat.add(sid)
    f = so.decoder_next_logprobs(so.weights_f64(w), F32)
    trace = []
    ref = so.beam_search(f, prompts, W, 3, trace=trace, valid_fn=cat.valid)
    assert _min_margin(trace, W) > 1e-3
    llm = _llm(F32, w, len(lens), max(lens), W, 3)
    llm.catalog = cat
    out = llm.beam_search(prompts, BeamSearchParams(W, 3))
    for o, r, p in zip(out, ref, prompts):
        got = {tuple(s.tokens): s.cum_logprob for s in o.sequences}
        exp = {tuple(s.tokens): s.cum_logprob for s in r if math.isfinite(s.cum_logprob)}
        assert set(got) == set(exp) and len(got) > 0
        for kk in exp:
            assert abs(got[kk] - exp[kk]) < 1e-4
            assert kk[len(p):] in sids


def test_sid_beam_search_bf16_mfma_rescored():
    seed, lens, W, steps = 5, [70, 129], 16, 4
    w = init_weights(BF16_128, seed)
    prompts = _prompts(seed, lens, BF16_128.vocab)
    llm = _llm(BF16_128, w, len(lens), max(lens), W, steps)
    out = llm.beam_search(prompts, BeamSearchParams(W, steps))
    w64 = so.weights_f64(w)
    for o, p in zip(out, prompts):
        assert len(o.sequences) == W
        # rescore a spread of the returned beams with the float64 recompute
        for s in o.sequences[::5]:
            lg = torch.log_softmax(so.decoder_logits(w64, BF16_128, s.tokens[:-1]), dim=-1)
            cum = sum(float(lg[len(p) - 1 + j, t]) for j, t in enumerate(s.tokens[len(p):]))
            assert abs(cum - s.cum_logprob) < 0.05 * steps, (s.tokens[len(p):], cum, s.cum_logprob)


@pytest.mark.parametrize("cfg", [F32, BF16_128], ids=["f32", "bf16_mfma"])
def test_sid_graph_replays_match_eager(cfg):
    """Decode steps replayed from captured graphs give the eager run's beams
    and scores; several replays, with eager batches and host syncs between
    them, all agree."""
    seed, lens, W, steps = 7, [19, 44], 8, 4
    w = init_weights(cfg, seed)
    prompts = _prompts(seed, lens, cfg.vocab)
    nb = blocks_needed(len(lens), max(lens), W, steps, 16) + 8
    wd = {k: v.cuda() for k, v in w.items()}
    eager = LLM(cfg, weights=wd, num_blocks=nb, use_graphs=False)
    graphed = LLM(cfg, weights=wd, num_blocks=nb, use_graphs=True)
    params = BeamSearchParams(W, steps)
    ref = eager.beam_search(prompts, params)
    for i in range(3):
        got = graphed.beam_search(prompts, params)  # first call captures, later ones replay
        torch.cuda.synchronize()
        for o, r in zip(got, ref):
            assert [s.tokens for s in o.sequences] == [s.tokens for s in r.sequences], i
            assert np.allclose([s.cum_logprob for s in o.sequences], [s.cum_logprob for s in r.sequences],
                               rtol=0, atol=1e-5), i
        eager.beam_search(prompts, params)
    assert len(graphed.runner._graphs) == 1


def test_sid_beam_search_full_size_self_consistent():
    """4 x 2048-token prompts, 128 beams, 3 SID tokens through the 28-layer
    decoder; two returned beams per request rescored by prefilling their
    whole token lists as plain requests (no beams, no resident suffix)."""
    cfg, R, P, W, steps = SID_DECODER_1P7B, 4, 2048, 128, 3
    llm = LLM(cfg, seed=0, num_blocks=blocks_needed(R, P, W, steps, 16) + 64)
    print(f"[sid] full size R={R} P={P} W={W} steps={steps}", flush=True)
    prompts = _prompts(6, [P] * R, cfg.vocab)
    out = llm.beam_search(prompts, BeamSearchParams(W, steps))
    t = llm.last_times
    print(f"[sid] prefill {t.prefill_ms:.2f} ms, steps {[round(x, 3) for x in t.step_ms]} ms, "
          f"wall {t.wall_ms:.1f} ms", flush=True)
    for o, p in zip(out, prompts):
        sc = [s.cum_logprob for s in o.sequences]
        assert len(sc) == W and sc == sorted(sc, reverse=True) and math.isfinite(sc[-1])
    seqs = [s for o in out for s in (o.sequences[0], o.sequences[W - 1])]
    # recompute: prefill prompt + generated[:-1] as plain requests, sum the chosen tokens' logprobs
    runner = llm.runner
    toks = [s.tokens[:-1] for s in seqs]
    logits_rows = []
    for j in range(steps):
        ctx = [t[:P + j] for t in toks]
        lg, _, _, blocks = runner.prefill(ctx, [f"re-{i}" for i in range(len(ctx))])
        runner.pool.release([b for bl in blocks for b in bl])
        logits_rows.append(torch.log_softmax(lg, dim=-1).cpu())
    for i, s in enumerate(seqs):
        cum = sum(float(logits_rows[j][i, s.tokens[P + j]]) for j in range(steps))
        assert abs(cum - s.cum_logprob) < 0.05 * steps, (i, cum, s.cum_logprob)


def _f64_beam_boundary(w64, cfg, cache, W, steps):
    """A float64 beam search from the cached prompt (no EOS: candidates are
    cum + logprob over every (beam, token), the best W kept per step --
    the reference's loop, llm.py:203-261, where each beam's own top-W
    candidates hold every member of the global top W).  Returns the final
    cumulative scores (descending) and the token lists of the final beams."""
    lp = torch.log_softmax(cache.last_logits, dim=-1)
    cum, tok = torch.topk(lp, W)
    beams = [[int(t)] for t in tok]
    for _ in range(steps - 1):
        lg = so.decoder_suffix_logits(w64, cfg, cache, beams)[:, -1]
        cand = cum[:, None] + torch.log_softmax(lg, dim=-1)
        cum, flat = torch.topk(cand.reshape(-1), W)
        V = lg.shape[-1]
        beams = [beams[int(f) // V] + [int(f) % V] for f in flat]
    return cum, beams


def test_sid_beam_search_full_size_vs_float64():
    """The 28-layer decoder at 4 prompts x 2048 tokens x 128 beams x 3 SID
    tokens against an independent float64 restatement of the same model
    (oracle/sid_beam.py's prompt-cached forward, run on the GPU as the
    checker, with the bf16 weights upcast exactly):

    * every returned beam's cumulative logprob equals the float64 model's
      score of its tokens (teacher forcing) within a bf16 tolerance;
    * every returned beam scores, in float64, at least the float64 beam
      search's 128th final score minus that tolerance -- the returned set is
      the best 128 up to bf16 rounding -- and most returned beams are the
      float64 search's own beams."""
    cfg, R, P, W, steps = SID_DECODER_1P7B, 4, 2048, 128, 3
    llm = LLM(cfg, seed=0, num_blocks=blocks_needed(R, P, W, steps, 16) + 64)
    print(f"[sid] full size vs float64 R={R} P={P} W={W} steps={steps}", flush=True)
    prompts = _prompts(11, [P] * R, cfg.vocab)
    out = llm.beam_search(prompts, BeamSearchParams(W, steps))
    w64 = {k: v.detach().to(torch.float64) for k, v in llm.model.w.items()}
    worst_score, worst_margin, overlaps = 0.0, float("inf"), []
    for r, (o, p) in enumerate(zip(out, prompts)):
        cache = so.decoder_prompt(w64, cfg, p)
        lp0 = torch.log_softmax(cache.last_logits, dim=-1)
        lpb = torch.log_softmax(so.decoder_suffix_logits(w64, cfg, cache, [s.tokens[P:P + steps - 1]
                                                                         for s in o.sequences]), dim=-1)
        f64 = torch.stack([lp0[s.tokens[P]] + sum(lpb[b, j, s.tokens[P + 1 + j]] for j in range(steps - 1))
                           for b, s in enumerate(o.sequences)]).cpu().numpy()
        got = np.array([s.cum_logprob for s in o.sequences])
        ref_cum, ref_beams = _f64_beam_boundary(w64, cfg, cache, W, steps)
        boundary = float(ref_cum[-1])
        ref_set = {tuple(b) for b in ref_beams}
        ov = sum(tuple(s.tokens[P:]) in ref_set for s in o.sequences)
        worst_score = max(worst_score, float(np.abs(f64 - got).max()))
        worst_margin = min(worst_margin, float(f64.min() - boundary))
        overlaps.append(ov)
        print(f"[sid] request {r}: max |score - float64| {np.abs(f64 - got).max():.4f}, "
              f"min float64 score - float64 boundary {f64.min() - boundary:+.4f}, "
              f"beams shared with the float64 search {ov}/{W}", flush=True)
        del cache, lpb
    # bf16 activations through 28 layers against float64: measured at most
    # 0.19 nats over three steps and -0.12 below the boundary, 112-118 of 128
    # beams shared (4 requests); the bounds keep about a 2x margin
    TOL = 0.4
    assert worst_score < TOL, worst_score
    assert worst_margin > -TOL, worst_margin
    assert min(overlaps) >= 3 * W // 4, overlaps
