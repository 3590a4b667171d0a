"""CPU oracle of the end-to-end semantic-ID beam decode.  TEST INFRASTRUCTURE ONLY.

Three pieces, all float64:

* ``decoder_logits(weights, cfg, tokens)`` -- the Qwen-style decoder's full
  forward over one token sequence at positions 0..n-1 (causal attention,
  query head j reading KV head j // (Hq / Hkv)), logits of every position.
  The reference recomputes every beam this way each step
  (vllm_gr/entrypoints/llm.py:183-199: each beam's whole token list becomes a
  new one-token request).  Pinned against transformers' ``Qwen3ForCausalLM``
  loaded with the same weights (tests/test_oracle_sid.py).
* ``decoder_prompt`` / ``decoder_suffix_logits`` -- the same forward split
  at the prompt: the prompt's per-layer keys and values computed once, then
  the logits after every token of many suffixes that share it (teacher
  forcing of whole beams).  Same arithmetic, float64, on whatever device the
  weights sit (the full-size model's checks run it on the GPU, as a checker).
  Pinned against ``decoder_logits`` over each whole list
  (tests/test_oracle_sid.py).
* ``beam_search(next_logprobs, prompts, ...)`` -- the reference's offline
  beam-search loop (llm.py:118-292) over a callable that returns a token
  list's next-token log-probabilities: the begin token appended to each
  prompt and the steps reduced by the begin/end tokens (:130-151), each
  beam's top ``beam_width`` logprobs (:100-108, deduplicated :208-212),
  candidate score = cumulative logprob + logprob (:214-217), EOS candidates
  completed with their score and excluded (:226-254), the top
  ``beam_width`` of the union (:256-261), then the end token appended to live
  beams and the best ``beam_width`` of completed + live by vLLM's beam-search
  score (:273-292).  The reference's ``np.argpartition`` leaves the order of
  equal scores open; here ties go to the lower (beam, token), the order of
  the flat index ``beam * vocab + token``.  Each sequence also carries its
  per-step logprob lists (llm.py:115-118, :203-220, :283-288): the begin
  token, the parent's top ``beam_width`` (token, logprob) list of every
  step, the end token.  Pinned against brute-force
  enumeration where the beam keeps every sequence, against a hand-computed
  planted case and against an EOS case (tests/test_oracle_sid.py).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch


def weights_f64(weights: dict) -> dict:
    return {k: v.detach().to("cpu", torch.float64) for k, v in weights.items()}


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c, s = cos[:, None], sin[:, None]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


def decoder_logits(w: dict, cfg, tokens) -> torch.Tensor:
    """``w``: float64 weights (``weights_f64``); returns float64 ``[n, V]``
    (the arithmetic follows the weights' dtype)."""
    n, D = len(tokens), cfg.head_dim
    Hq, Hkv = cfg.num_heads, cfg.num_kv_heads
    G = Hq // Hkv
    ids = torch.as_tensor(list(tokens), dtype=torch.int64)
    x = w["embed"][ids]
    half = D // 2
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(half, dtype=torch.float64) * 2.0 / D))
    ang = torch.arange(n, dtype=torch.float64)[:, None] * inv[None]
    cos, sin = ang.cos().to(x.dtype), ang.sin().to(x.dtype)
    mask = torch.triu(torch.ones(n, n, dtype=torch.bool), diagonal=1)
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        h = _rms(x, w[p + "input_norm"], cfg.rms_eps)
        qkv = h @ w[p + "qkv"].T
        q = qkv[:, :Hq * D].reshape(n, Hq, D)
        k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(n, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D:].reshape(n, Hkv, D)
        q = _rope(_rms(q, w[p + "q_norm"], cfg.rms_eps), cos, sin)
        k = _rope(_rms(k, w[p + "k_norm"], cfg.rms_eps), cos, sin)
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
        s = torch.einsum("thd,shd->hts", q, k) / math.sqrt(D)
        s = s.masked_fill(mask[None], float("-inf"))
        a = torch.softmax(s, dim=-1)
        o = torch.einsum("hts,shd->thd", a, v).reshape(n, Hq * D)
        x = x + o @ w[p + "o"].T
        h = _rms(x, w[p + "post_norm"], cfg.rms_eps)
        gu = h @ w[p + "gate_up"].T
        g, u = gu[:, :cfg.ffn], gu[:, cfg.ffn:]
        x = x + (torch.nn.functional.silu(g) * u) @ w[p + "down"].T
    x = _rms(x, w["final_norm"], cfg.rms_eps)
    return x @ w["lm_head"].T


def _rope_table(cfg, n: int, device, dtype):
    D = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(D // 2, dtype=torch.float64, device=device) * 2.0 / D))
    ang = torch.arange(n, dtype=torch.float64, device=device)[:, None] * inv[None]
    return ang.cos().to(dtype), ang.sin().to(dtype)


def _attend(q, k, v, mask):
    """q [.., Hq, t, D], k / v [.., Hq, s, D] (contiguous), mask [t, s] or
    [.., 1, t, s] (True = hidden): softmax(q k^T / sqrt D) v."""
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
    s = s.masked_fill(mask, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


@dataclass
class PromptCache:
    """decoder_prompt's output: each layer's rotated keys and values of the
    prompt (float64, [Hkv, P, D]) and the prompt's last-position logits."""
    keys: list
    values: list
    last_logits: torch.Tensor
    length: int


def decoder_prompt(w: dict, cfg, prompt) -> PromptCache:
    """The forward of ``decoder_logits`` over ``prompt`` alone, keeping every
    layer's keys and values for ``decoder_suffix_logits``.  Runs on the
    weights' device (a GPU makes the 28-layer, 2048-token forward take
    seconds instead of minutes); the arithmetic is decoder_logits' step for
    step (matmul in place of einsum)."""
    dev, dt = w["embed"].device, w["embed"].dtype
    n, D, Hq, Hkv = len(prompt), cfg.head_dim, cfg.num_heads, cfg.num_kv_heads
    G = Hq // Hkv
    x = w["embed"][torch.as_tensor(list(prompt), dtype=torch.int64, device=dev)]
    cos, sin = _rope_table(cfg, n, dev, dt)
    mask = torch.triu(torch.ones(n, n, dtype=torch.bool, device=dev), diagonal=1)
    keys, values = [], []
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        qkv = _rms(x, w[p + "input_norm"], cfg.rms_eps) @ w[p + "qkv"].T
        q = qkv[:, :Hq * D].reshape(n, Hq, D)
        k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(n, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D:].reshape(n, Hkv, D)
        q = _rope(_rms(q, w[p + "q_norm"], cfg.rms_eps), cos, sin)
        k = _rope(_rms(k, w[p + "k_norm"], cfg.rms_eps), cos, sin)
        kh, vh = k.transpose(0, 1).contiguous(), v.transpose(0, 1).contiguous()  # [Hkv, n, D]
        keys.append(kh)
        values.append(vh)
        o = _attend(q.transpose(0, 1).contiguous(), kh.repeat_interleave(G, dim=0),
                    vh.repeat_interleave(G, dim=0), mask)  # [Hq, n, D]
        x = x + o.transpose(0, 1).reshape(n, Hq * D) @ w[p + "o"].T
        gu = _rms(x, w[p + "post_norm"], cfg.rms_eps) @ w[p + "gate_up"].T
        x = x + (torch.nn.functional.silu(gu[:, :cfg.ffn]) * gu[:, cfg.ffn:]) @ w[p + "down"].T
    last = _rms(x[-1:], w["final_norm"], cfg.rms_eps) @ w["lm_head"].T
    return PromptCache(keys, values, last[0], n)


def decoder_suffix_logits(w: dict, cfg, cache: PromptCache, suffixes) -> torch.Tensor:
    """Logits after each token of ``suffixes`` ([B, S] token lists, equal S)
    appended to the cached prompt: row [b, j] equals
    ``decoder_logits(prompt + suffixes[b])[P + j]``.  Suffix token j sits at
    position P + j and attends to every prompt key and to its own suffix's
    tokens 0..j -- the causal attention decoder_logits computes over the
    whole list.  Returns float64 [B, S, V] on the weights' device."""
    dev, dt = w["embed"].device, w["embed"].dtype
    B, S = len(suffixes), len(suffixes[0])
    P, D, Hq, Hkv = cache.length, cfg.head_dim, cfg.num_heads, cfg.num_kv_heads
    G = Hq // Hkv
    x = w["embed"][torch.as_tensor(suffixes, dtype=torch.int64, device=dev).reshape(B, S)]  # [B, S, H]
    cos, sin = _rope_table(cfg, P + S, dev, dt)
    cos, sin = cos[P:], sin[P:]
    # suffix query j sees the P prompt keys and suffix keys 0..j
    mask = torch.zeros(S, P + S, dtype=torch.bool, device=dev)
    mask[:, P:] = torch.triu(torch.ones(S, S, dtype=torch.bool, device=dev), diagonal=1)
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        qkv = _rms(x, w[p + "input_norm"], cfg.rms_eps) @ w[p + "qkv"].T  # [B, S, .]
        q = qkv[..., :Hq * D].reshape(B, S, Hq, D)
        k = qkv[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D)
        v = qkv[..., (Hq + Hkv) * D:].reshape(B, S, Hkv, D)
        q = _rope(_rms(q, w[p + "q_norm"], cfg.rms_eps), cos, sin)
        k = _rope(_rms(k, w[p + "k_norm"], cfg.rms_eps), cos, sin)
        # scores against the shared prompt keys (broadcast over the suffixes)
        # and against the suffix's own keys, one softmax over both
        kp = cache.keys[i].repeat_interleave(G, dim=0)  # [Hq, P, D]
        vp = cache.values[i].repeat_interleave(G, dim=0)
        qh = q.transpose(1, 2).contiguous()  # [B, Hq, S, D]
        ks = k.transpose(1, 2).repeat_interleave(G, dim=1).contiguous()
        vs = v.transpose(1, 2).repeat_interleave(G, dim=1).contiguous()
        sc = torch.cat((torch.matmul(qh, kp.transpose(-1, -2).contiguous()),
                        torch.matmul(qh, ks.transpose(-1, -2).contiguous())), dim=-1) / math.sqrt(D)
        a = torch.softmax(sc.masked_fill(mask, float("-inf")), dim=-1)  # [B, Hq, S, P + S]
        o = torch.matmul(a[..., :P].contiguous(), vp) + torch.matmul(a[..., P:].contiguous(), vs)
        x = x + o.transpose(1, 2).reshape(B, S, Hq * D) @ w[p + "o"].T
        gu = _rms(x, w[p + "post_norm"], cfg.rms_eps) @ w[p + "gate_up"].T
        x = x + (torch.nn.functional.silu(gu[..., :cfg.ffn]) * gu[..., cfg.ffn:]) @ w[p + "down"].T
    return _rms(x, w["final_norm"], cfg.rms_eps) @ w["lm_head"].T


def decoder_next_logprobs(w: dict, cfg):
    """``tokens -> log_softmax(last-position logits)`` (float64 numpy)."""
    def f(tokens):
        lg = decoder_logits(w, cfg, tokens)[-1]
        return torch.log_softmax(lg, dim=-1).numpy()
    return f


@dataclass
class Seq:
    tokens: list
    cum_logprob: float
    finish_reason: str | None = None
    # per generated position: (token ids, logprobs) -- the begin token (0.0),
    # each step's parent top-W list, the end token (0.0) on a non-EOS beam
    # (vllm_gr/entrypoints/llm.py:115-118, :203-220, :283-288)
    logprobs: list = field(default_factory=list)


@dataclass
class _Instance:
    beams: list
    completed: list = field(default_factory=list)


def beam_score(tokens, cum, eos, length_penalty) -> float:
    """vLLM's get_beam_search_score (the sort key of llm.py:75-79)."""
    n = len(tokens)
    if eos is not None and n and tokens[-1] == eos:
        n -= 1
    return cum / (n ** length_penalty)


def beam_search(next_logprobs, prompts, beam_width: int, max_tokens: int, eos_token_id=None,
                length_penalty: float = 1.0, begin_token=None, end_token=None, trace=None, valid_fn=None):
    """Returns, per prompt, the list of :class:`Seq` the reference outputs.
    ``trace`` (a list) receives, per step and prompt, the sorted scores of
    the candidates left after the EOS split, and per prompt the sorted
    final scores of completed + live sequences -- the gap between entries
    ``beam_width - 1`` and ``beam_width`` of each is how close that cut came
    to a different selection.  ``valid_fn(generated_tokens) -> set`` is the
    catalog (serving_engine.py:381-394): a beam's candidates outside the set
    are masked to -inf after its top-W (:504-506); such a candidate is never
    kept as a beam here (the reference keeps -inf beams when fewer than W
    valid ones exist)."""
    W = beam_width
    insts, plen = [], []
    for p in prompts:
        toks = list(p) + ([begin_token] if begin_token is not None else [])
        first = [([begin_token], [0.0])] if begin_token is not None else []
        insts.append(_Instance([Seq(toks, 0.0, logprobs=first)]))
        plen.append(len(toks))
    pre_calc = (begin_token is not None) + (end_token is not None)
    for _ in range(max(0, max_tokens - pre_calc)):
        for ii, inst in enumerate(insts):
            cand = []  # (score, beam index, token)
            step_lists = []  # per beam: its top-W (tokens, logprobs)
            for bi, beam in enumerate(inst.beams):
                lp = np.asarray(next_logprobs(beam.tokens), dtype=np.float64)
                V = lp.shape[0]
                top = np.lexsort((np.arange(V), -lp))[:W]  # (logprob desc, token asc)
                step_lists.append(([int(t) for t in top], [float(lp[t]) for t in top]))
                ok = None if valid_fn is None else valid_fn(beam.tokens[plen[ii]:])
                for t in top:
                    if ok is not None and int(t) not in ok:
                        continue
                    cand.append((beam.cum_logprob + float(lp[t]), bi, int(t)))
            keep = []
            for sc, bi, t in cand:
                if eos_token_id is not None and t == eos_token_id:
                    inst.completed.append(Seq(inst.beams[bi].tokens + [t], sc, "stop",
                                              inst.beams[bi].logprobs + [step_lists[bi]]))
                else:
                    keep.append((sc, bi, t))
            keep.sort(key=lambda c: (-c[0], c[1], c[2]))
            if trace is not None:
                trace.append([c[0] for c in keep])
            inst.beams = [Seq(inst.beams[bi].tokens + [t], sc, None, inst.beams[bi].logprobs + [step_lists[bi]])
                          for sc, bi, t in keep[:W]]
    out = []
    for inst in insts:
        if end_token is not None:
            for b in inst.beams:
                b.tokens.append(end_token)
                b.logprobs = b.logprobs + [([end_token], [0.0])]
        allseq = inst.completed + inst.beams
        key = lambda s: beam_score(s.tokens, s.cum_logprob, eos_token_id, length_penalty)
        allseq = sorted(allseq, key=key, reverse=True)
        if trace is not None:
            trace.append([key(s) for s in allseq])
        out.append(allseq[:W])
    return out
