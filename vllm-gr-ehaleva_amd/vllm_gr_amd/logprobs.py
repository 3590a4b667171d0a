"""Per-step logprob lists of beam search (vllm_gr/logprobs.py).

:class:`FlatLogprobs` holds the fields of vLLM's ``FlatLogprobs`` that the
reference fills: one entry per generated position, each a run of
``(token_id, logprob, rank, decoded_token)`` in ``[start_indices[i],
end_indices[i])`` of the flat lists.  ``append_fast`` appends one position
(vllm_gr/logprobs.py:10-31).

A beam's lists are the reference's (vllm_gr/entrypoints/llm.py:115-118,
:203-220, :283-288 with vllm_gr/logprobs.py:56-85): the begin token with
logprob 0.0 when one is set, then for every step the top ``beam_width``
candidates of the beam's parent at that step (token ids by logprob
descending, their logprobs, ranks 1..beam_width, no decoded text), then the
end token with 0.0 for a beam that did not finish on EOS.  Here the
candidate lists come from the fused prune kernel (each beam's top-k by
logit, ties to the lower token id) and are rebuilt along the parent
indices once, after the last step, instead of through per-beam parent
pointers.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class FlatLogprobs:
    start_indices: list[int] = field(default_factory=list)
    end_indices: list[int] = field(default_factory=list)
    token_ids: list[int] = field(default_factory=list)
    logprobs: list[float] = field(default_factory=list)
    ranks: list[int | None] = field(default_factory=list)
    decoded_tokens: list[str | None] = field(default_factory=list)

    def append_fast(self, token_ids, logprobs, ranks, decoded_tokens) -> None:
        """One position's run (vllm_gr/logprobs.py:10-31)."""
        n = len(token_ids)
        self.start_indices.append(len(self.logprobs))
        self.token_ids.extend(token_ids)
        self.logprobs.extend(logprobs)
        self.ranks.extend(list(ranks)[:n])
        self.decoded_tokens.extend(list(decoded_tokens)[:n])
        self.end_indices.append(len(self.logprobs))

    def __len__(self) -> int:
        return len(self.start_indices)

    def position(self, i: int) -> list[tuple[int, float, int | None]]:
        """``(token_id, logprob, rank)`` of position ``i``."""
        s, e = self.start_indices[i], self.end_indices[i]
        return list(zip(self.token_ids[s:e], self.logprobs[s:e], self.ranks[s:e]))


def step_lists(cand_token, cand_logprob):
    """Per-step host lists: ``cand_token / cand_logprob [R, W_old, K]`` as
    nested Python lists (one device-to-host copy each)."""
    return cand_token.cpu().tolist(), cand_logprob.cpu().tolist()


def rebuild(r: int, parent: int, last_step: int, parents: list, cands: list, begin: int | None,
            end: int | None) -> FlatLogprobs:
    """The lists of a beam of request ``r`` whose parent at step
    ``last_step`` is ``parent`` (a live beam after the last step, or a beam
    that finished on EOS at ``last_step`` from beam ``parent``).
    ``parents[s][r][j]``: the parent, at step ``s``, of beam ``j`` of that
    step's output; ``cands[s]``: the host ``(tokens, logprobs)`` of
    :func:`step_lists` for step ``s``."""
    runs = []
    p = parent
    for s in range(last_step, -1, -1):
        runs.append((cands[s][0][r][p], cands[s][1][r][p]))
        if s > 0:
            p = parents[s - 1][r][p]
    lp = FlatLogprobs()
    if begin is not None:
        lp.append_fast([begin], [0.0], [None], [None])
    for toks, lps in reversed(runs):
        k = len(toks)
        lp.append_fast(toks, lps, list(range(1, k + 1)), [None] * k)
    if end is not None:
        lp.append_fast([end], [0.0], [None], [None])
    return lp
