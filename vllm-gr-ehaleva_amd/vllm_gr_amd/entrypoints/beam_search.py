"""One beam-search step on the device: prune, then fork.

Mirrors the per-step arithmetic of the reference's beam search
(vllm_gr/entrypoints/openai/serving_engine.py:457-592, offline twin
vllm_gr/entrypoints/llm.py:201-280):

* candidate score = cumulative logprob + log_softmax(logits) of the token
  (:511); the reference asks the sampler for each beam's top W candidates
  and takes the top W of their union (:566-567) -- the fused kernel takes
  the top W over beams x vocab directly, which selects the same set (any
  global top-W candidate is within its beam's top W), ties to the lowest
  flat index ``beam * vocab + token``;
* EOS candidates leave the pool and finish with their score (:541-562);
* ``fork_info`` lists (parent beam, token) per new beam in score order
  (:588-590); parents no child selected are the reference's pruned / abort
  set (:141-142);
* the new beams' suffix KV is forked on the device (BeamKVTable.fork) instead
  of being rebuilt from tokens.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import ops
from ..tracing import roctx_range


@dataclass
class BeamSearchParams:
    """Beam-search parameters (vLLM's BeamSearchParams plus the reference's
    ``begin_token`` / ``end_token``, vllm_gr/sampling_params.py:14-15)."""
    beam_width: int
    max_tokens: int
    ignore_eos: bool = False
    temperature: float = 0.0
    length_penalty: float = 1.0
    include_stop_str_in_output: bool = False
    begin_token: str | None = None
    end_token: str | None = None


@dataclass
class PruneResult:
    parent: torch.Tensor     # [R, W] int32: beam (within the request) each new beam extends
    token: torch.Tensor      # [R, W] int32
    score: torch.Tensor      # [R, W] new cumulative logprob (cum's dtype), descending per request
    eos_score: torch.Tensor  # [R, W_old] score of a beam's EOS candidate (-inf if none)
    node: torch.Tensor | None = None  # [R, W] int32: each new beam's catalog trie node (with a catalog)
    # with candidates=True: each old beam's top-W list before EOS / catalog removal
    cand_token: torch.Tensor | None = None    # [R, W_old, W] int32
    cand_logprob: torch.Tensor | None = None  # [R, W_old, W] float32 (logit - lse)


def prune_step(logits: torch.Tensor, cum_logprob: torch.Tensor, beam_width: int,
               eos_token_id: int | None = None, *, workspace: torch.Tensor | None = None,
               catalog=None, beam_node: torch.Tensor | None = None, candidates: bool = False,
               status: torch.Tensor | None = None) -> PruneResult:
    """Fused log_softmax + cumulative logprob + top-``beam_width`` over
    beams x vocab per request.  ``logits [R, W, V]`` float32, ``cum [R, W]``
    float64 (the reference's Python-float scores, serving_engine.py:511,
    :538-539; the result's scores are float64 too) or float32.
    With ``catalog`` (device trie) and ``beam_node [R, W]``, each beam's
    candidates outside its valid continuations leave the pool (the catalog
    mask of serving_engine.py:381-394, 504-506) and the result carries the
    new beams' trie nodes.  ``candidates`` (float64 ``cum`` only) also
    returns every old beam's top-``beam_width`` (token, logprob) list, the
    per-step logprobs of the reference's beam search
    (vllm_gr/entrypoints/llm.py:203-220).  ``status``: a device status
    word (``ops.new_status``) the kernels OR table errors into."""
    eos = -1 if eos_token_id is None else int(eos_token_id)
    with roctx_range("beam_prune_topk"):
        out = list(ops.beam_prune_topk(logits, cum_logprob, beam_width, eos, workspace=workspace,
                                       catalog=catalog, beam_node=beam_node, candidates=candidates,
                                       status=status))
    ct = cl = None
    if candidates:
        ct, cl = out[-2], out[-1]
        del out[-2:]
    node = out[4] if catalog is not None else None
    return PruneResult(out[0], out[1], out[2], out[3], node, ct, cl)


def fork_info(res: PruneResult) -> list[list[tuple[int, int]]]:
    """Per request, the (parent beam, token) of each new beam in score order
    (serving_engine.py:588-590).  Synchronises with the device."""
    par = res.parent.cpu().tolist()
    tok = res.token.cpu().tolist()
    return [[(p, t) for p, t in zip(pr, tr) if p >= 0] for pr, tr in zip(par, tok)]


def pruned_parents(res: PruneResult, beam_width: int) -> list[list[int]]:
    """Per request, the beams no new beam descends from (the abort set of
    serving_engine.py:141-142).  Synchronises with the device."""
    out = []
    for pr in res.parent.cpu().tolist():
        used = set(p for p in pr if p >= 0)
        out.append([b for b in range(beam_width) if b not in used])
    return out


def beam_search_step(table, logits: torch.Tensor, cum_logprob: torch.Tensor, kv_caches,
                     eos_token_id: int | None = None, status: torch.Tensor | None = None, *,
                     catalog=None, beam_node: torch.Tensor | None = None, candidates: bool = False):
    """Prune the candidates of every beam and fork the beams' resident KV.

    ``table``: the batch's :class:`~vllm_gr_amd.v1.beam_kv.BeamKVTable`;
    ``logits [R, W, V]`` are the last decode step's logits rows (one per
    beam), ``cum_logprob [R, W]`` the beams' scores.  Returns the
    :class:`PruneResult`; its ``token`` are the next step's query tokens and
    its ``score`` the new cumulative logprobs (float64 when ``cum_logprob``
    is).  Unfilled slots (fewer live
    candidates than beams) keep their parent's KV."""
    W = table.beam_width
    res = prune_step(logits, cum_logprob, W, eos_token_id, catalog=catalog, beam_node=beam_node,
                     candidates=candidates, status=status)
    parent = torch.where(res.parent >= 0, res.parent,
                         torch.arange(W, device=res.parent.device, dtype=res.parent.dtype)[None])
    with roctx_range("beam_kv_fork"):
        table.fork(parent, kv_caches, status=status)
    return res
