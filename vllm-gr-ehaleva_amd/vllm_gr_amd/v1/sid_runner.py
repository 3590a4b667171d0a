"""Model runner of the end-to-end semantic-ID beam decode: KV-cache blocks,
per-forward backend metadata and the decoder's forward.

It plays the part of vLLM's GPU model runner for one batch of beam-search
requests: the prompts go through the backend's standard path once (varlen
causal attention, gr_paged_attn_prefill), then every step runs one query
token per beam through the mega-decode path over the batch's
:class:`BeamKVTable`.  Host-to-device copies are issued before the forward
they feed (a copy from pageable host memory waits for the stream), so a
whole batch is enqueued without a host round trip.  The side channel is
the reference's ``MEGA_DATA_VAR`` (engine_core_patch.py:544-554) with the
``beam_kv`` key the backend adds.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .attention.backends.beam_attn import (MEGA_DATA_VAR, BeamAttentionBackend,
                                           BeamAttentionMetadataBuilder, CommonAttentionMetadata)
from .beam_kv import BeamKVTable
from .sid_decoder import SidDecoder


class BlockPool:
    """Host free list of KV-cache block ids; allocation hands out the lowest
    free ids first."""

    def __init__(self, num_blocks: int):
        self.num_blocks = int(num_blocks)
        self._free = list(range(self.num_blocks - 1, -1, -1))

    @property
    def num_free(self) -> int:
        return len(self._free)

    def allocate(self, n: int) -> list[int]:
        if n > len(self._free):
            raise RuntimeError(f"KV cache out of blocks: need {n}, {len(self._free)} free")
        out = [self._free.pop() for _ in range(n)]
        return out

    def release(self, ids) -> None:
        ids = list(ids)
        if any(not 0 <= b < self.num_blocks for b in ids):
            raise ValueError("block id outside the pool")
        self._free.extend(sorted(ids, reverse=True))
        self._free.sort(reverse=True)


@dataclass(frozen=True)
class _KVSpec:
    block_size: int


def blocks_needed(num_reqs: int, prompt_len: int, beam_width: int, new_tokens: int, block_size: int) -> int:
    """Blocks one batch holds: each prompt's blocks plus each beam's suffix
    blocks for ``new_tokens`` resident tokens."""
    per_prompt = -(-prompt_len // block_size)
    per_beam = max(1, -(-new_tokens // block_size))
    return num_reqs * (per_prompt + beam_width * per_beam)


class _DecodeGraph:
    """The decode forward of one batch shape captured as a HIP graph.

    It owns a static :class:`BeamKVTable` and token buffer; capturing runs the
    metadata builder and the decoder once, so the builder's device work
    (positions, slot mapping, attention suffix lengths) is recorded too and
    replays from whatever the static table holds.  A replay copies the live
    table and tokens in (six small device copies) and returns the captured
    logits buffer, valid until the next replay."""

    def __init__(self, runner: "SidModelRunner", table: BeamKVTable, tokens: torch.Tensor, req_ids, prompt_lens,
                 step: int):
        self.table = BeamKVTable(table.prefix_bt.clone(), table.prefix_len.clone(), table.beam_width,
                                 table.suffix_bt.clone(), table.suffix_len.clone(), block_size=table.block_size)
        self.tokens = tokens.clone()
        args = (self.table, self.tokens, list(req_ids), list(prompt_lens), step)
        side = torch.cuda.Stream(device=runner.device)  # warm-up off the main stream, as capture expects
        side.wait_stream(torch.cuda.current_stream(runner.device))
        with torch.cuda.stream(side):
            runner._decode_eager(*args)
        torch.cuda.current_stream(runner.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = runner._decode_eager(*args)

    def replay(self, table: BeamKVTable, tokens: torch.Tensor) -> torch.Tensor:
        st = self.table
        st.prefix_bt.copy_(table.prefix_bt)
        st.prefix_len.copy_(table.prefix_len)
        st.beam_start.copy_(table.beam_start)
        st.suffix_bt.copy_(table.suffix_bt)
        st.suffix_len.copy_(table.suffix_len)
        self.tokens.copy_(tokens)
        self.graph.replay()
        return self.logits


class SidModelRunner:
    """Owns one ``[2, num_blocks, block_size, Hkv, D]`` cache per layer.

    With ``use_graphs`` the decode forward of each batch shape (requests,
    beams, table widths, longest prompt) runs eagerly once and is then
    captured; later steps of that shape replay the graph."""

    def __init__(self, model: SidDecoder, num_blocks: int, block_size: int = 16, use_graphs: bool = True):
        cfg = model.cfg
        if block_size % 16 != 0:
            raise ValueError("block_size must be a multiple of 16")
        self.model = model
        self.block_size = block_size
        self.device = model.device
        shape = BeamAttentionBackend.get_kv_cache_shape(num_blocks, block_size, cfg.num_kv_heads,
                                                        cfg.head_dim)
        self.kv_caches = [torch.zeros(shape, dtype=cfg.dtype, device=self.device)
                          for _ in range(cfg.num_layers)]
        self.builder = BeamAttentionMetadataBuilder(_KVSpec(block_size), model.layer_names, None,
                                                    self.device)
        self.pool = BlockPool(num_blocks)
        self.use_graphs = use_graphs
        self._graphs: dict = {}

    def _forward(self, ids, positions, m: CommonAttentionMetadata, side: dict):
        token = MEGA_DATA_VAR.set(side)
        try:
            md = self.builder.build(0, m)
        finally:
            MEGA_DATA_VAR.reset(token)
        return self.model.forward(ids, positions, md, self.kv_caches)

    def prefill(self, prompts: list[list[int]], req_ids: list[str]):
        """Prompts through the standard path, each into fresh blocks.
        Returns ``(logits [R, V] float32 of each prompt's last token,
        prefix_bt [R, blocks] int32, prefix_len [R] int32, blocks per
        request)``."""
        bs = self.block_size
        lens = [len(p) for p in prompts]
        if min(lens) < 1:
            raise ValueError("empty prompt")
        if max(lens) > self.model.rope.max_pos:
            raise ValueError(f"prompt longer than the rotary table ({self.model.rope.max_pos})")
        nbs = [-(-n // bs) for n in lens]
        flat = self.pool.allocate(sum(nbs))
        try:
            return self._prefill(prompts, req_ids, lens, nbs, flat)
        except BaseException:
            self.pool.release(flat)
            raise

    def _prefill(self, prompts, req_ids, lens, nbs, flat):
        bs, dev = self.block_size, self.device
        offs = [0]
        for n in nbs:
            offs.append(offs[-1] + n)
        blocks = [flat[offs[r]:offs[r + 1]] for r in range(len(nbs))]
        R, width = len(prompts), max(nbs)
        bt = torch.zeros(R, width, dtype=torch.int32)
        for r, b in enumerate(blocks):
            bt[r, :len(b)] = torch.tensor(b, dtype=torch.int32)
        pos = torch.cat([torch.arange(n) for n in lens])
        req = torch.cat([torch.full((n,), r) for r, n in enumerate(lens)])
        slots = bt[req, pos // bs].to(torch.int64) * bs + pos % bs
        qsl = torch.tensor([0] + lens, dtype=torch.int64).cumsum(0).to(torch.int32)
        seq = torch.tensor(lens, dtype=torch.int32)
        m = CommonAttentionMetadata(
            query_start_loc=qsl.to(dev), query_start_loc_cpu=qsl, seq_lens=seq.to(dev), seq_lens_cpu=seq,
            num_reqs=R, num_actual_tokens=int(qsl[-1]), max_query_len=max(lens), max_seq_len=max(lens),
            block_table_tensor=bt.to(dev), slot_mapping=slots.to(dev))
        ids = torch.tensor([t for p in prompts for t in p], dtype=torch.int64).to(dev)
        # every host-to-device copy precedes the forward: none waits for it
        last = (qsl[1:].to(torch.int64) - 1).to(dev)
        hidden = self._forward(ids, pos.to(dev), m, {"mega_data": {}, "req_ids": list(req_ids)})
        logits = self.model.compute_logits(hidden.index_select(0, last))
        return logits, m.block_table_tensor, m.seq_lens, blocks

    def decode(self, table: BeamKVTable, tokens: torch.Tensor, req_ids: list[str],
               prompt_lens: list[int], step: int) -> torch.Tensor:
        """One query token per beam (``tokens [R*W]``, beam-major) at
        position ``prefix_len + suffix_len``; its K/V goes to the beam's next
        suffix slot.  ``step`` = tokens already resident per beam (host
        copy of ``table.suffix_len``, equal for every beam).  Returns logits
        ``[R, W, V]`` float32."""
        R, W = table.num_reqs, table.beam_width
        if max(prompt_lens) + step >= self.model.rope.max_pos:
            raise ValueError(f"position beyond the rotary table ({self.model.rope.max_pos})")
        if step >= table.suffix_capacity:
            raise ValueError("beam suffix blocks are full")
        if tokens.shape != (R * W,):
            raise ValueError("tokens must hold one query token per beam")
        if not self.use_graphs:
            return self._decode_eager(table, tokens, req_ids, prompt_lens, step)
        key = (R, W, table.prefix_bt.shape[1], table.suffix_bt.shape[1], max(prompt_lens))
        g = self._graphs.get(key)
        if g is None:
            out = self._decode_eager(table, tokens, req_ids, prompt_lens, step)
            self._graphs[key] = _DecodeGraph(self, table, tokens, req_ids, prompt_lens, step)
            return out
        return g.replay(table, tokens)

    def _decode_eager(self, table: BeamKVTable, tokens: torch.Tensor, req_ids, prompt_lens, step: int):
        R, W = table.num_reqs, table.beam_width
        N = R * W
        qsl = torch.arange(0, N + 1, W, dtype=torch.int32)
        seq = torch.tensor([p + step + 1 for p in prompt_lens], dtype=torch.int32)
        # device copies come from device tensors: a host-to-device copy here would
        # wait for the previous step's kernels
        m = CommonAttentionMetadata(
            query_start_loc=table.beam_start, query_start_loc_cpu=qsl,
            seq_lens=table.prefix_len + (step + 1), seq_lens_cpu=seq,
            num_reqs=R, num_actual_tokens=N, max_query_len=1, max_seq_len=int(seq.max()),
            block_table_tensor=table.prefix_bt, slot_mapping=table.slot_mapping())
        side = {"req_ids": list(req_ids), "mega_data": {
            rid: {"is_mega_decode": True, "mega_beam_width": W, "mega_decode_steps": step + 1,
                  "prefix_len": p, "cache_len": p, "beam_kv": table}
            for rid, p in zip(req_ids, prompt_lens)}}
        hidden = self._forward(tokens, table.positions(), m, side)
        return self.model.compute_logits(hidden).view(R, W, -1)
