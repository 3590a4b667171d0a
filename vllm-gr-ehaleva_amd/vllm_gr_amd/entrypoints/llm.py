"""Offline semantic-ID beam search over the resident-KV path.

Mirrors ``LLM.beam_search`` of the reference (vllm_gr/entrypoints/llm.py:31-280):
same parameters (beam width, max tokens, ignore_eos, length penalty, the
``begin_token`` / ``end_token`` pair), the same per-step candidate rule (each
beam's top ``beam_width`` tokens by logprob, candidate score = cumulative
logprob + logprob, EOS candidates finish with their score and leave the
pool, the top ``beam_width`` of the union become the new beams, :201-271) and
the same output (per prompt the best ``beam_width`` of finished + live
sequences by vLLM's beam-search score, :273-292).

What differs is how a step is computed.  The reference re-submits every
beam's whole token list as a new one-token request each step (:183-199).
Here a batch of prompts is prefilled once, then each step decodes exactly one
token per beam against the shared prompt prefix and the beam's resident
suffix (gr_beam_attn_decode), prunes on the device (gr_beam_prune_topk) and
forks the beams' suffix KV (gr_beam_kv_fork) -- no host round trip between
steps.  There is no tokenizer: ``begin_token`` / ``end_token`` of the
:class:`BeamSearchParams` are token ids, or strings looked up in the
``special_tokens`` map given to :class:`LLM` (an unknown one is ignored with
a warning, as at llm.py:60-74), and ``text`` stays None.
"""

from __future__ import annotations

import logging
import time
from dataclasses import dataclass, field

import torch

from .. import logprobs as lpm
from .. import ops
from ..tracing import roctx_range
from ..v1.beam_kv import BeamKVTable
from ..v1.sid_decoder import SID_DECODER_1P7B, DecoderConfig, SidDecoder, init_weights
from ..v1.sid_runner import SidModelRunner
from . import beam_search as bsm
from .beam_search import BeamSearchParams

logger = logging.getLogger(__name__)


@dataclass
class BeamSearchSequence:
    """vLLM's BeamSearchSequence, the fields the offline path fills."""
    tokens: list[int]
    cum_logprob: float = 0.0
    finish_reason: str | None = None
    stop_reason: int | None = None
    text: str | None = None
    logprobs: lpm.FlatLogprobs | None = None


@dataclass
class BeamSearchOutput:
    sequences: list[BeamSearchSequence]


@dataclass
class StepTimes:
    """Device time of each phase of the last batch, milliseconds (HIP
    events on the current stream), and the host wall time of the whole
    batch including the final copy of the results."""
    prefill_ms: float = 0.0
    step_ms: list[float] = field(default_factory=list)
    total_ms: float = 0.0
    wall_ms: float = 0.0


def beam_search_score(tokens: list[int], cum_logprob: float, eos_token_id: int | None,
                      length_penalty: float) -> float:
    """vLLM's beam-search sort key: ``cum_logprob / len ** length_penalty``,
    the length excluding a final EOS (llm.py:75-79)."""
    n = len(tokens)
    if eos_token_id is not None and n and tokens[-1] == eos_token_id:
        n -= 1
    return cum_logprob / (n ** length_penalty)


class LLM:
    """A random-init Qwen-style decoder served through the beam path.

    ``weights`` (from :func:`init_weights`) default to ``init_weights(cfg,
    seed, device)``.  ``num_blocks`` KV-cache blocks of ``block_size``
    tokens are allocated per layer up front; a batch needs
    :func:`~vllm_gr_amd.v1.sid_runner.blocks_needed` of them.  With
    ``use_graphs`` each decode step shape is captured once and replayed.
    With a :class:`~vllm_gr_amd.entrypoints.catalog.Catalog`, every beam's
    candidates are restricted to the catalog's valid continuations of its
    generated tokens; a candidate the catalog rules out never becomes a beam
    (the reference keeps it as a -inf-score beam, serving_engine.py:504-506,
    which only reaches the output when fewer than beam_width valid sequences
    exist)."""

    def __init__(self, cfg: DecoderConfig = SID_DECODER_1P7B, *, seed: int = 0, device="cuda",
                 num_blocks: int = 4096, block_size: int = 16, eos_token_id: int | None = None,
                 special_tokens: dict[str, int] | None = None, weights: dict | None = None,
                 max_position: int = 32768, use_graphs: bool = True, catalog=None, logprobs: bool = True):
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError("the beam path runs on a HIP device (torch 'cuda')")
        if weights is None:
            weights = init_weights(cfg, seed, dev)
        self.cfg = cfg
        self.model = SidDecoder(cfg, weights, max_position=max_position)
        self.runner = SidModelRunner(self.model, num_blocks, block_size, use_graphs=use_graphs)
        self.eos_token_id = eos_token_id
        self.special_tokens = dict(special_tokens or {})
        # the catalog of valid semantic IDs (serving_models.py:52-65 loads it per server)
        self.catalog = catalog
        self._catalog_dev = None
        self.last_times = StepTimes()
        self._batch = 0
        # rebuild every output beam's per-step logprob lists (the reference always does,
        # vllm_gr/entrypoints/llm.py:283-288)
        self.logprobs = logprobs
        # observer of every step's logits: hook(step, logits [R, W, V] float32,
        # the beams' generated tokens [R, W, step] int32), called on the
        # stream before the step's pruning reads the logits
        self.logits_hook = None

    def _token_id(self, tok, what: str) -> int | None:
        if tok is None:
            return None
        tid = tok if isinstance(tok, int) else self.special_tokens.get(tok)
        if tid is None or not 0 <= tid < self.cfg.vocab:
            logger.warning("%s must be a valid token in the vocabulary, got token %s", what, tok)
            return None
        return int(tid)

    def beam_search(self, prompts, params: BeamSearchParams) -> list[BeamSearchOutput]:
        """``prompts``: token-id lists or ``{"prompt_token_ids": [...]}``
        dicts.  Returns one :class:`BeamSearchOutput` per prompt."""
        W = int(params.beam_width)
        if W < 1:
            raise ValueError("beam_width must be >= 1")
        toks = [list(p["prompt_token_ids"]) if isinstance(p, dict) else list(p) for p in prompts]
        if not toks:
            return []
        begin = self._token_id(params.begin_token, "begin_token")
        end = self._token_id(params.end_token, "end_token")
        if begin is not None:
            toks = [t + [begin] for t in toks]
        pre_calc = (begin is not None) + (end is not None)
        steps = max(0, int(params.max_tokens) - pre_calc)
        eos = None if params.ignore_eos else self.eos_token_id
        if W > self.cfg.vocab:
            raise ValueError("beam_width must not exceed the vocabulary")
        for t in toks:
            if any(not 0 <= x < self.cfg.vocab for x in t):
                raise ValueError("prompt token id outside the vocabulary")

        R, dev, bs = len(toks), self.model.device, self.runner.block_size
        self._batch += 1
        rids = [f"beam-{self._batch}-{r}" for r in range(R)]
        lens = [len(t) for t in toks]
        times = StepTimes()
        t_wall = time.perf_counter()
        stream = torch.cuda.current_stream(dev)
        ev = [torch.cuda.Event(enable_timing=True)]
        ev[0].record(stream)

        cat = None
        if self.catalog is not None:
            if self._catalog_dev is None:
                self._catalog_dev = self.catalog.to_device(dev)
            cat = self._catalog_dev
        hist = torch.empty(R, W, 0, dtype=torch.int32, device=dev)
        # beam scores stay float64 from step to step (serving_engine.py:511, :538-539)
        score = torch.zeros(R, W, dtype=torch.float64, device=dev)
        finished: list[tuple[torch.Tensor, torch.Tensor]] = []  # (eos_score [R, W_old], hist_old)
        parents: list[torch.Tensor] = []  # per step: each new beam's parent [R, W]
        cands: list[tuple[torch.Tensor, torch.Tensor]] = []  # per step: old beams' top-W lists
        lp = self.logprobs
        # one device status word for the batch's launches (the builder's, which the
        # attention and cache-write kernels already use), checked at the batch's sync
        status = self.runner.builder.status
        status.zero_()
        blocks: list[int] = []
        try:
            if steps > 0:
                sbt = None
                if steps > 1:  # the beams' suffix blocks (host-to-device copy before any kernel)
                    per_beam = -(-(steps - 1) // bs)
                    sblocks = self.runner.pool.allocate(R * W * per_beam)
                    blocks += sblocks
                    sbt = torch.tensor(sblocks, dtype=torch.int32).view(R * W, per_beam).to(dev)
                with roctx_range("LLM.beam_search prefill"):
                    logits, prefix_bt, prefix_len, pblocks = self.runner.prefill(toks, rids)
                blocks += [b for bl in pblocks for b in bl]
                ev.append(torch.cuda.Event(enable_timing=True))
                ev[-1].record(stream)
                # the prompt is the one beam of every request (llm.py:118-146), at the trie's root
                node0 = None if cat is None else torch.zeros(R, 1, dtype=torch.int32, device=dev)
                if self.logits_hook is not None:
                    self.logits_hook(0, logits[:, None], torch.empty(R, 1, 0, dtype=torch.int32, device=dev))
                res = bsm.prune_step(logits[:, None], torch.zeros(R, 1, dtype=torch.float64, device=dev), W, eos,
                                     catalog=cat, beam_node=node0, candidates=lp, status=status)
                finished.append((res.eos_score, torch.empty(R, 1, 0, dtype=torch.int32, device=dev)))
                parents.append(res.parent)
                if lp:
                    cands.append((res.cand_token, res.cand_logprob))
                hist = res.token[..., None]
                score = res.score
                table = None if sbt is None else BeamKVTable(prefix_bt, prefix_len, W, sbt, block_size=bs)
                for s in range(1, steps):
                    tok = res.token.clamp(min=0).view(-1).to(torch.int64)
                    with roctx_range(f"LLM.beam_search decode step {s}"):
                        logits = self.runner.decode(table, tok, rids, lens, step=s - 1)
                    table.advance()
                    if self.logits_hook is not None:
                        self.logits_hook(s, logits, hist)
                    node = res.node
                    if s + 1 < steps:
                        res = bsm.beam_search_step(table, logits, score, self.runner.kv_caches, eos, status,
                                                   catalog=cat, beam_node=node, candidates=lp)
                    else:
                        res = bsm.prune_step(logits, score, W, eos, catalog=cat, beam_node=node, candidates=lp,
                                             status=status)
                    finished.append((res.eos_score, hist))
                    parents.append(res.parent)
                    if lp:
                        cands.append((res.cand_token, res.cand_logprob))
                    par = res.parent.clamp(min=0).to(torch.int64)
                    hist = torch.cat((hist.gather(1, par[..., None].expand(-1, -1, hist.shape[2])),
                                      res.token[..., None]), dim=2)
                    score = res.score
                    ev.append(torch.cuda.Event(enable_timing=True))
                    ev[-1].record(stream)
            hist_h, score_h = hist.cpu().tolist(), score.cpu().tolist()
            fin_h = [(e.cpu().tolist(), h.cpu().tolist()) for e, h in finished]
            par_h = [p.cpu().tolist() for p in parents]
            cand_h = [lpm.step_lists(t, l) for t, l in cands] if lp else None
            ops.check_status(status)  # the copies above synchronised: raises on a flagged table entry
        finally:
            self.runner.pool.release(blocks)
        times.wall_ms = (time.perf_counter() - t_wall) * 1e3
        if len(ev) > 1:
            times.prefill_ms = ev[0].elapsed_time(ev[1])
            times.step_ms = [a.elapsed_time(b) for a, b in zip(ev[1:-1], ev[2:])]
            times.total_ms = ev[0].elapsed_time(ev[-1])
        self.last_times = times
        return self._outputs(toks, hist_h, score_h, fin_h, steps, eos, begin, end, params.length_penalty, W,
                             par_h, cand_h)

    @staticmethod
    def _outputs(toks, hist, score, finished, steps, eos, begin, end, length_penalty, W, parents, cands):
        outs = []
        for r, prompt in enumerate(toks):
            # (sequence, parent at its last step, that step) per candidate output
            done = []
            for s, (eos_sc, hist_old) in enumerate(finished):
                for b, sc in enumerate(eos_sc[r]):
                    if sc != float("-inf"):
                        done.append((BeamSearchSequence(prompt + hist_old[r][b] + [eos], sc,
                                                        finish_reason="stop", stop_reason=eos), b, s))
            live = []
            tail = [] if end is None else [end]
            if steps == 0:
                live.append((BeamSearchSequence(prompt + tail, 0.0, finish_reason="length"), None, -1))
            else:
                for b in range(W):
                    if score[r][b] == float("-inf"):
                        continue  # a slot no candidate filled
                    live.append((BeamSearchSequence(prompt + hist[r][b] + tail, score[r][b],
                                                    finish_reason="length"), parents[-1][r][b], steps - 1))
            allseq = done + live
            allseq.sort(key=lambda x: beam_search_score(x[0].tokens, x[0].cum_logprob, eos, length_penalty),
                        reverse=True)
            best = allseq[:W]
            if cands is not None:
                # the best beams' lists, rebuilt along the parent indices (llm.py:283-288)
                for seq, p, s in best:
                    if s < 0:
                        seq.logprobs = lpm.rebuild(r, 0, -1, parents, cands, begin, end)
                    else:
                        stop = seq.finish_reason == "stop"
                        seq.logprobs = lpm.rebuild(r, p, s, parents, cands, begin, None if stop else end)
            outs.append(BeamSearchOutput([seq for seq, _, _ in best]))
        return outs
