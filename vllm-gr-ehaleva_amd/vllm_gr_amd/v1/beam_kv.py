"""Resident per-beam suffix KV state of a batch of beam-search requests.

The reference keeps no per-beam KV between steps: every step it rebuilds each
child's suffix as ``parent suffix ++ chosen token``
(vllm_gr/entrypoints/openai/serving_engine.py:113-120,
vllm_gr/v1/engine/core.py:108-112) and recomputes those W*t tokens through
every layer.  Here each beam's tokens after the shared prompt prefix stay in
private paged blocks of the engine's KV cache; a step only appends the newest
token per beam, and a fork permutes / copies block-table rows on the device
(``gr_beam_kv_fork``).

Layout (device, int32): ``prefix_bt [R, prefix_blocks]`` and
``prefix_len [R]`` address each request's shared prompt prefix;
``beam_start [R+1]`` gives request r the beams ``beam_start[r] ..
beam_start[r+1]-1``; ``suffix_bt [N, suffix_blocks]`` and ``suffix_len [N]``
hold each beam's private tokens.  Positions follow the reference: the j-th
suffix token of a beam sits at position ``prefix_len + j``
(vllm_gr/v1/engine/engine_core_patch.py:362-365).
"""

from __future__ import annotations

import torch

from .. import ops


class BeamKVTable:
    """Block tables and lengths of R requests x W beams (all on one device)."""

    def __init__(self, prefix_bt: torch.Tensor, prefix_len: torch.Tensor, beam_width: int,
                 suffix_bt: torch.Tensor, suffix_len: torch.Tensor | None = None, *, block_size: int):
        if prefix_bt.dim() != 2 or prefix_len.dim() != 1 or prefix_bt.shape[0] != prefix_len.numel():
            raise ValueError("prefix_bt must be [R, blocks] and prefix_len [R]")
        R = prefix_len.numel()
        N = R * beam_width
        if suffix_bt.dim() != 2 or suffix_bt.shape[0] != N:
            raise ValueError(f"suffix_bt must be [{N}, blocks] (R * beam_width rows)")
        dev = prefix_bt.device
        self.block_size = int(block_size)
        self.beam_width = int(beam_width)
        self.prefix_bt = prefix_bt.to(torch.int32).contiguous()
        self.prefix_len = prefix_len.to(device=dev, dtype=torch.int32).contiguous()
        self.beam_start = torch.arange(0, N + 1, beam_width, dtype=torch.int32, device=dev)
        self.suffix_bt = suffix_bt.to(torch.int32).contiguous()
        self.suffix_len = (torch.zeros(N, dtype=torch.int32, device=dev) if suffix_len is None
                           else suffix_len.to(device=dev, dtype=torch.int32).contiguous())
        # the fork writes out of place: a second table set to alternate with
        self._spare_bt = torch.empty_like(self.suffix_bt)
        self._spare_len = torch.empty_like(self.suffix_len)
        self._beam_req = torch.arange(R, device=dev, dtype=torch.int64).repeat_interleave(beam_width)

    @property
    def num_reqs(self) -> int:
        return self.prefix_len.numel()

    @property
    def num_beams(self) -> int:
        return self.suffix_len.numel()

    @property
    def suffix_capacity(self) -> int:
        return self.suffix_bt.shape[1] * self.block_size

    def positions(self) -> torch.Tensor:
        """RoPE position of each beam's next token: ``prefix_len + suffix_len``
        (engine_core_patch.py:362-365).  int64 ``[N]``."""
        return (self.prefix_len.to(torch.int64)[self._beam_req] + self.suffix_len.to(torch.int64))

    def slot_mapping(self) -> torch.Tensor:
        """Cache slot of each beam's next token (``block * block_size + offset``
        at suffix position ``suffix_len``), the ``slot_mapping`` that
        ``reshape_and_cache`` writes the step's K/V through.  int64 ``[N]``;
        -1 (nothing written) for a beam whose suffix blocks are full -- its
        attention length then exceeds the table and the decode kernel reports
        it in the status word."""
        L = self.suffix_len.to(torch.int64)
        bs = self.block_size
        col = torch.clamp(L // bs, max=self.suffix_bt.shape[1] - 1)
        blk = self.suffix_bt.to(torch.int64).gather(1, col[:, None])[:, 0]
        return torch.where(L < self.suffix_capacity, blk * bs + L % bs, torch.full_like(L, -1))

    def attention_suffix_len(self) -> torch.Tensor:
        """Suffix lengths the step's attention sees: the resident tokens plus
        the token being decoded (its K/V is written before attention)."""
        return self.suffix_len + 1

    def advance(self) -> None:
        """After a decode step (every layer done): the new token is resident."""
        self.suffix_len += 1

    def fork(self, parent: torch.Tensor, kv_caches, status: torch.Tensor | None = None) -> None:
        """Children take their parents' suffixes (``parent [R, W]`` beam index
        within the request): the lowest-index child of a parent keeps its row,
        other children copy into rows of parents that have no child, in every
        layer's cache.  ``kv_caches``: iterable of ``[2, num_blocks,
        block_size, Hkv, D]`` tensors (one per layer)."""
        if parent.shape != (self.num_reqs, self.beam_width):
            raise ValueError(f"parent must be [{self.num_reqs}, {self.beam_width}]")
        parent = parent.to(torch.int32).contiguous()
        caches = list(kv_caches)
        if not caches:
            raise ValueError("fork needs at least one KV cache")
        # one launch for every layer: the tables are worked out once, each
        # workgroup copies its share of the copy-on-write tokens in all layers
        ops.beam_kv_fork_layers(parent, self.suffix_bt, self.suffix_len, caches,
                                bt_out=self._spare_bt, len_out=self._spare_len, status=status)
        self.suffix_bt, self._spare_bt = self._spare_bt, self.suffix_bt
        self.suffix_len, self._spare_len = self._spare_len, self.suffix_len
