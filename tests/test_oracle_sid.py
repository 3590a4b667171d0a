"""The end-to-end oracle (oracle/sid_beam.py) pinned, and the host logic of
the semantic-ID beam decode (block pool, output assembly, batch tables in
the metadata builder) on the CPU.

* decoder: float64 logits against transformers' Qwen3ForCausalLM loaded with
  the same weights (random norm weights, so each norm's placement counts);
* beam search: against brute-force enumeration when the beam keeps every
  sequence, a hand-computed planted case (pruning, ties to the lower token),
  an EOS case (a beam whose top-W holds EOS contributes W-1 candidates;
  length penalty excludes the EOS, llm.py:226-254 and :75-79) and the
  begin/end token accounting (llm.py:130-151, 275-280)."""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import sid_beam as so
from vllm_gr_amd.entrypoints import llm as llm_mod
from vllm_gr_amd.v1.attention.backends import beam_attn as ba
from vllm_gr_amd.v1.beam_kv import BeamKVTable
from vllm_gr_amd.v1.sid_decoder import DecoderConfig, init_weights
from vllm_gr_amd.v1.sid_runner import BlockPool, blocks_needed

TINY = DecoderConfig(num_layers=2, hidden=32, num_heads=4, num_kv_heads=2, head_dim=16, ffn=48,
                     vocab=64, init_std=0.3, dtype=torch.float32)


def _random_norms(w, seed):
    g = torch.Generator().manual_seed(seed)
    for k in list(w):
        if k.endswith("norm"):
            w[k] = 0.5 + torch.rand(w[k].shape, generator=g, dtype=torch.float32)
    return w


def _hf_state_dict(w, cfg):
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["final_norm"],
          "lm_head.weight": w["lm_head"]}
    for i in range(cfg.num_layers):
        p, hp = f"layers.{i}.", f"model.layers.{i}."
        q, k, v = w[p + "qkv"].split([cfg.q_size, cfg.kv_size, cfg.kv_size])
        g, u = w[p + "gate_up"].split([cfg.ffn, cfg.ffn])
        sd.update({hp + "self_attn.q_proj.weight": q, hp + "self_attn.k_proj.weight": k,
                   hp + "self_attn.v_proj.weight": v, hp + "self_attn.o_proj.weight": w[p + "o"],
                   hp + "self_attn.q_norm.weight": w[p + "q_norm"],
                   hp + "self_attn.k_norm.weight": w[p + "k_norm"],
                   hp + "mlp.gate_proj.weight": g, hp + "mlp.up_proj.weight": u,
                   hp + "mlp.down_proj.weight": w[p + "down"],
                   hp + "input_layernorm.weight": w[p + "input_norm"],
                   hp + "post_attention_layernorm.weight": w[p + "post_norm"]})
    return {k: v.to(torch.float64) for k, v in sd.items()}


@pytest.mark.parametrize("tie", [True, False])
def test_decoder_matches_transformers_qwen3(tie):
    tr = pytest.importorskip("transformers")
    cfg = DecoderConfig(**{**TINY.__dict__, "tie_embeddings": tie})
    w = _random_norms(init_weights(cfg, seed=3), seed=5)
    if tie:
        w["lm_head"] = w["embed"]
    hc = tr.Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.ffn,
                        num_hidden_layers=cfg.num_layers, num_attention_heads=cfg.num_heads,
                        num_key_value_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                        rms_norm_eps=cfg.rms_eps, tie_word_embeddings=tie, attention_bias=False,
                        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta})
    hc._attn_implementation = "eager"
    m = tr.Qwen3ForCausalLM(hc).to(torch.float64).eval()
    missing, unexpected = m.load_state_dict(_hf_state_dict(w, cfg), strict=False)
    assert not unexpected and all(k == "lm_head.weight" for k in missing)
    tokens = torch.randint(0, cfg.vocab, (37,), generator=torch.Generator().manual_seed(7)).tolist()
    with torch.no_grad():
        ref = m(input_ids=torch.tensor([tokens])).logits[0]
    got = so.decoder_logits(so.weights_f64(w), cfg, tokens)
    # transformers forms the rotary angles in float32 (inv_freq and position
    # products), which bounds the agreement near 1e-6; a wrong pairing, head
    # mapping or norm placement moves logits by O(1)
    assert torch.allclose(got, ref, rtol=0, atol=2e-5), (got - ref).abs().max()


def _table_logprobs(table: dict, vocab: int, prompt_len: int):
    """next_logprobs from a dict {generated-token tuple: probabilities}."""
    def f(tokens):
        return np.log(np.asarray(table[tuple(tokens[prompt_len:])], dtype=np.float64))
    return f


def _hash_logprobs(vocab: int, seed: int):
    def f(tokens):
        rng = np.random.default_rng([seed] + list(tokens))
        x = rng.normal(0, 2, vocab)
        return x - np.log(np.exp(x - x.max()).sum()) - x.max()
    return f


@pytest.mark.parametrize("V,steps", [(3, 2), (3, 3), (4, 2)])
def test_beam_search_exhaustive_matches_enumeration(V, steps):
    """With beam_width = V**steps nothing is pruned: the result is every
    sequence, best first (score = sum of logprobs / length)."""
    W = V ** steps
    prompt = [1, 2]
    f = _hash_logprobs(V, seed=11)
    got = so.beam_search(f, [prompt], W, steps)[0]
    allseq = []
    for gen in itertools.product(range(V), repeat=steps):
        toks, cum = list(prompt), 0.0
        for t in gen:
            cum += f(toks)[t]
            toks.append(t)
        allseq.append((cum / len(toks), toks, cum))
    allseq.sort(key=lambda s: -s[0])
    assert [s.tokens for s in got] == [s[1] for s in allseq]
    assert np.allclose([s.cum_logprob for s in got], [s[2] for s in allseq], atol=1e-12)


def test_beam_search_planted_pruning_and_ties():
    P = [5, 6, 7]
    table = {(): [.5, .4, .1], (0,): [.3, .3, .4], (1,): [.9, .05, .05],
             (1, 0): [.6, .3, .1], (0, 2): [.2, .7, .1]}
    got = so.beam_search(_table_logprobs(table, 3, len(P)), [P], 2, 3)[0]
    # step 1: (1,0)=.36, (0,2)=.2 beat (0,0)=.15 (the .3/.3 tie within beam (0,) goes to token 0)
    # step 2: (1,0,0)=.216, (0,2,1)=.14
    assert [s.tokens for s in got] == [P + [1, 0, 0], P + [0, 2, 1]]
    assert np.allclose([s.cum_logprob for s in got], [math.log(.216), math.log(.14)])


def test_beam_search_eos_and_length_penalty():
    P = [9, 9]
    eos = 3
    table = {(): [.4, .1, .1, .4], (0,): [.5, .2, .2, .1]}
    got = so.beam_search(_table_logprobs(table, 4, len(P)), [P], 2, 2, eos_token_id=eos)[0]
    # step 0: top-2 of the prompt = token 0 and EOS (tie .4, lower token first) -> EOS completes,
    # one live beam.  step 1: (0,0)=.2, (0,1)=.08 (the .2/.2 tie goes to token 1).
    # scores: (0,0) log(.2)/4 = -0.402 > [eos] log(.4)/2 = -0.458 > (0,1) log(.08)/4
    assert [s.tokens for s in got] == [P + [0, 0], P + [eos]]
    assert got[1].finish_reason == "stop"
    assert math.isclose(got[1].cum_logprob, math.log(.4))


def test_beam_search_catalog_mask_after_top_w():
    """The catalog masks a beam's candidates after its top-W (serving_engine.py:
    504-506): a valid token outside the beam's top-W is not a candidate."""
    P = [3]
    table = {(): [.5, .3, .15, .05], (0,): [.7, .2, .05, .05], (3,): [.1, .2, .3, .4]}
    valid = {(): {0, 3}, (0,): {1, 3}, (3,): {0}}
    got = so.beam_search(_table_logprobs(table, 4, len(P)), [P], 2, 2,
                         valid_fn=lambda g: valid.get(tuple(g), set()))[0]
    # step 0: top-2 = {0 (.5), 1 (.3)}; 3 is valid but outside the top-2, 1 is invalid -> beam [0]
    # step 1 from (0,): top-2 = {0 (.7), 1 (.2)}; only 1 is valid -> [0, 1] = .5 * .2
    assert [s.tokens for s in got] == [P + [0, 1]]
    assert math.isclose(got[0].cum_logprob, math.log(.1))


def test_beam_search_begin_end_tokens():
    P = [1]
    f = _hash_logprobs(5, seed=2)
    got = so.beam_search(f, [P], 2, 3, begin_token=4, end_token=0)[0]
    # 3 tokens = begin + 1 generated + end
    assert all(len(s.tokens) == 4 and s.tokens[:2] == [1, 4] and s.tokens[-1] == 0 for s in got)
    lp = f([1, 4])
    best = np.lexsort((np.arange(5), -lp))[:2]
    assert [s.tokens[2] for s in got] == best.tolist()


# ---------------------------------------------------------------- host logic


def test_block_pool():
    p = BlockPool(8)
    a = p.allocate(3)
    assert a == [0, 1, 2] and p.num_free == 5
    b = p.allocate(5)
    with pytest.raises(RuntimeError):
        p.allocate(1)
    p.release(a)
    assert p.allocate(2) == [0, 1]
    with pytest.raises(ValueError):
        p.release([8])
    assert blocks_needed(4, 2048, 128, 2, 16) == 4 * (128 + 128)
    assert blocks_needed(1, 17, 2, 0, 16) == 2 + 2


def test_outputs_assembly():
    """EOS sequences from every step, live beams with the end token, slots
    no candidate filled dropped, sorted by the length-penalised score."""
    ninf = float("-inf")
    toks = [[7, 7]]
    hist = [[[1, 2], [3, 4], [0, 0]]]
    score = [[-1.0, -3.0, ninf]]
    finished = [([[-0.5]], [[[]]]), ([[ninf, -2.5, ninf]], [[[1], [3], [5]]])]
    # step 0: the prompt's top-3 list; step 1: each of the three beams' lists
    parents = [[[0, 0, 0]], [[0, 1, -1]]]
    c0 = ([[[1, 3, 5]]], [[[-0.1, -0.2, -0.3]]])
    c1 = ([[[2, 9, 4], [4, 9, 6], [7, 8, 6]]], [[[-1.0, -1.1, -1.2], [-2.0, -2.1, -2.2], [-3.0, -3.1, -3.2]]])
    out = llm_mod.LLM._outputs(toks, hist, score, finished, 2, 9, None, 8, 1.0, 3, parents, [c0, c1])[0].sequences
    # scores: [7,7,9] -0.5/2; [7,7,3,9] -2.5/3; [7,7,1,2,8] -1/5; [7,7,3,4,8] -3/5
    assert [s.tokens for s in out] == [[7, 7, 1, 2, 8], [7, 7, 9], [7, 7, 3, 4, 8]]
    assert [s.finish_reason for s in out] == ["length", "stop", "length"]
    # logprob lists rebuilt along the parents (worked by hand): each step's
    # entry is the parent's whole list, ranks 1..3; the end token closes the
    # live beams, not the EOS one
    pos = lambda s: [s.logprobs.position(i) for i in range(len(s.logprobs))]
    l0 = [(1, -0.1, 1), (3, -0.2, 2), (5, -0.3, 3)]
    end = [(8, 0.0, None)]
    assert pos(out[0]) == [l0, [(2, -1.0, 1), (9, -1.1, 2), (4, -1.2, 3)], end]
    assert pos(out[1]) == [l0]
    assert pos(out[2]) == [l0, [(4, -2.0, 1), (9, -2.1, 2), (6, -2.2, 3)], end]
    out0 = llm_mod.LLM._outputs(toks, [[[]]], [[0.0]], [], 0, None, 5, 6, 1.0, 2, [], [])[0].sequences
    assert [s.tokens for s in out0] == [[7, 7, 6]]
    assert pos(out0[0]) == [[(5, 0.0, None)], [(6, 0.0, None)]]


def _mega_side(tables_of_reqs, W):
    rids = [f"r{i}" for i in range(len(tables_of_reqs))]
    md = {rid: {"is_mega_decode": True, "mega_beam_width": W, "mega_decode_steps": 1, "prefix_len": 32,
                "cache_len": 32, "beam_kv": t} for rid, t in zip(rids, tables_of_reqs)}
    return {"mega_data": md, "req_ids": rids}


def _common(R, W, bt):
    N = R * W
    qsl = torch.arange(0, N + 1, W, dtype=torch.int32)
    seq = torch.full((R,), 33, dtype=torch.int32)
    return ba.CommonAttentionMetadata(qsl, qsl, seq, seq, R, N, 1, 33, bt,
                                      torch.zeros(N, dtype=torch.int64))


def test_builder_batch_table_one_group():
    R, W = 3, 4
    pbt = torch.arange(R * 2, dtype=torch.int32).view(R, 2)
    table = BeamKVTable(pbt, torch.full((R,), 32), W, torch.arange(100, 100 + R * W, dtype=torch.int32)[:, None],
                        block_size=16)
    builder = ba.BeamAttentionMetadataBuilder(type("S", (), {"block_size": 16})(), [], None, "cpu")
    tok = ba.MEGA_DATA_VAR.set(_mega_side([table] * R, W))
    try:
        md = builder.build(0, _common(R, W, pbt))
    finally:
        ba.MEGA_DATA_VAR.reset(tok)
    assert len(md.groups) == 1
    g = md.groups[0]
    assert g.token_index is None and g.max_beams == W
    assert g.beam_start.tolist() == [0, 4, 8, 12]
    assert torch.equal(g.prefix_bt, pbt) and torch.equal(g.suffix_bt, table.suffix_bt)
    assert g.suffix_len.tolist() == [1] * (R * W)
    assert md.slot_mapping.tolist() == [(100 + n) * 16 for n in range(R * W)]


def test_builder_batch_table_count_mismatch():
    R, W = 3, 2
    pbt = torch.zeros(R, 2, dtype=torch.int32)
    table = BeamKVTable(pbt, torch.full((R,), 32), W, torch.zeros(R * W, 1, dtype=torch.int32), block_size=16)
    builder = ba.BeamAttentionMetadataBuilder(type("S", (), {"block_size": 16})(), [], None, "cpu")
    other = BeamKVTable(pbt[:1], torch.full((1,), 32), W, torch.zeros(W, 1, dtype=torch.int32), block_size=16)
    for names in ([table, table, other], [table, other, table]):
        tok = ba.MEGA_DATA_VAR.set(_mega_side(names, W))
        try:
            with pytest.raises(ValueError, match="consecutive requests"):
                builder.build(0, _common(R, W, pbt))
        finally:
            ba.MEGA_DATA_VAR.reset(tok)


@pytest.mark.parametrize("cfg_seed", [0, 1])
def test_prompt_cache_suffix_logits_match_full_forward(cfg_seed):
    """decoder_prompt + decoder_suffix_logits equal decoder_logits over each
    whole token list (the prompt's last row and every suffix row)."""
    cfg = DecoderConfig(num_layers=3, hidden=48, num_heads=6, num_kv_heads=2, head_dim=8, ffn=64, vocab=80,
                        init_std=0.3, dtype=torch.float32)
    w = so.weights_f64(_random_norms(init_weights(cfg, cfg_seed), cfg_seed))
    g = torch.Generator().manual_seed(cfg_seed)
    prompt = torch.randint(0, cfg.vocab, (23,), generator=g).tolist()
    sufs = torch.randint(0, cfg.vocab, (5, 3), generator=g).tolist()
    cache = so.decoder_prompt(w, cfg, prompt)
    got = so.decoder_suffix_logits(w, cfg, cache, sufs)
    assert got.shape == (5, 3, cfg.vocab)
    for b, suf in enumerate(sufs):
        full = so.decoder_logits(w, cfg, prompt + suf)
        assert torch.allclose(cache.last_logits, full[len(prompt) - 1], rtol=0, atol=1e-10)
        assert torch.allclose(got[b], full[len(prompt):], rtol=0, atol=1e-10)


def test_prompt_cache_suffix_reads_the_cached_prompt():
    """The suffix rows depend on the cached prompt's keys and values: a cache
    built from a prompt that differs in its first token moves them, by far
    more than the 1e-10 agreement above."""
    cfg = DecoderConfig(num_layers=2, hidden=48, num_heads=6, num_kv_heads=2, head_dim=8, ffn=64, vocab=80,
                        init_std=0.3, dtype=torch.float32)
    w = so.weights_f64(_random_norms(init_weights(cfg, 3), 3))
    prompt = list(range(10, 27))
    other = [11] + prompt[1:]
    sufs = [[5, 6]]
    full = so.decoder_logits(w, cfg, prompt + sufs[0])[len(prompt):]
    good = so.decoder_suffix_logits(w, cfg, so.decoder_prompt(w, cfg, prompt), sufs)[0]
    bad = so.decoder_suffix_logits(w, cfg, so.decoder_prompt(w, cfg, other), sufs)[0]
    assert torch.allclose(good, full, rtol=0, atol=1e-10)
    assert (bad - full).abs().max() > 1e-3
