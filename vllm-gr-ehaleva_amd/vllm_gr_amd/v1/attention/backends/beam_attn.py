"""BeamAttention backend: the attention-backend plugin surface of
vllm_gr/v1/attention/backends/beam_attn.py, over the gfx950 kernels.

Kept from the reference (same names, argument meaning and error behaviour):

* ``MEGA_DATA_VAR`` (beam_attn.py:60): a ContextVar holding
  ``{"mega_data": {req_id: {...}}, "req_ids": [...]}`` per forward, with the
  per-request keys ``is_mega_decode``, ``mega_beam_width``,
  ``mega_decode_steps``, ``prefix_len``, ``cache_len``
  (engine_core_patch.py:544-554).  One key is added here: ``beam_kv``, the
  request's :class:`~vllm_gr_amd.v1.beam_kv.BeamKVTable` (the reference has no
  resident per-beam KV, so it needs none).
* ``BeamAttentionMetadataBuilder.build(common_prefix_len,
  common_attn_metadata, fast_build)`` (:480-485) and ``update_block_table``
  (:561-570).
* ``BeamAttentionImpl.__init__`` (:579-627) and ``forward(layer, query, key,
  value, kv_cache, attn_metadata, output, output_scale, output_block_scale)``
  (:703-755): output buffer required, output quantization rejected with
  NotImplementedError, zero-fill without metadata, K/V append through the
  slot mapping, then attention.
* ``BeamAttentionBackend`` static surface (:758-846): name ``CUSTOM``,
  fp16/bf16, block size a multiple of 16, KV shape ``(2, NB, bs, Hkv, D)``,
  NHD/HND stride orders, head size %8 and <= 256, ``supports_combination``
  returning a reason string or None; the four attention types (:771-773).
* the optional features of ``BeamAttentionImpl`` (:597-625): ALiBi slopes,
  the sliding window ((w-1, 0), or (w-1, w-1) for ENCODER_ONLY) and the
  sinks reach every kernel launch (``gr_attn_options``), and a non-causal
  batch (the encoder types) runs its standard rows over every key of their
  sequence.  An fp8 cache (``kv_cache_dtype`` "fp8" / "fp8_e4m3", stored as
  float8_e4m3fn, :734-737, :801-804) is written as e4m3(x / scale) with the
  layer's ``_k_scale`` / ``_v_scale`` and read as e4m3 * scale.

Two mega-request layouts are accepted:

* the reference's own (``MEGA_DATA_VAR`` exactly as engine_core_patch.py:258-271
  emits it): ``prefill ++ concat(beam tokens)`` scheduled as one request
  (core.py:108-112), row k at logical position ``cache_len + k`` of its
  block-table row.  The builder applies the reference's routing
  (beam_attn.py:255-413): an uncached prefix of at least two blocks goes to
  the standard path (and ``cache_len`` is written back, :280), beam 0
  computes the uncached prefix tail every other beam's suffix shares, and the
  chunk budget leaves later beams partially run or skipped.  It maps that
  routing onto the kernels by position: the standard rows and beam 0's rows
  continue one causal prefill of the request (``gr_paged_attn_prefill``: a
  row at position p sees keys 0..p, which is the cascade's cached prefix +
  causal suffix), and every other beam is a decode beam whose prefix is the
  whole shared prompt (cached part + the tail written this step) and whose
  suffix is its own tokens at positions ``prefix_len + b * t + j``
  (``gr_beam_attn_decode`` with ``q_per_beam`` = its row count, bottom-right
  causal);
* the resident layout of this build (the request's dict carries
  ``beam_kv``, its :class:`~vllm_gr_amd.v1.beam_kv.BeamKVTable`): each beam
  attends its resident suffix with one new query token, and the mega
  requests of a batch are one ``gr_beam_attn_decode`` launch instead of
  recomputing W*t tokens (no prefix/suffix/merge passes, :656-701).

The standard requests (prefill chunks, plain decodes) are one
``gr_paged_attn_prefill`` launch: varlen causal attention over their
block-table rows, the ``flash_attn_varlen_func`` call of the standard path
(:643-654).
"""

from __future__ import annotations

import contextvars
import copy
import os
from dataclasses import dataclass, field
from enum import Enum

import torch

from vllm_gr_amd import ops
from vllm_gr_amd.tracing import roctx_range

MEGA_DATA_VAR = contextvars.ContextVar("mega_data", default=None)


FP8_KV_DTYPES = ("fp8", "fp8_e4m3")


class AttentionCGSupport(Enum):
    """How far a metadata builder's batches can be captured in a device
    graph: the levels of vLLM's ``AttentionCGSupport`` (vllm==0.14,
    ``vllm/v1/attention/backend.py``), by the same names and values."""
    ALWAYS = 3
    UNIFORM_BATCH = 2
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    NEVER = 0


_KV_CACHE_LAYOUT_OVERRIDE: str | None = None


def set_kv_cache_layout(cache_layout: str | None) -> None:
    """Set the engine's KV-cache layout ("NHD" / "HND"; None clears it), the
    role of vLLM's ``set_kv_cache_layout`` (a KV connector's choice)."""
    global _KV_CACHE_LAYOUT_OVERRIDE
    _KV_CACHE_LAYOUT_OVERRIDE = cache_layout


def get_kv_cache_layout() -> str:
    """The KV-cache layout the engine configured, read as vLLM's
    ``get_kv_cache_layout`` (``beam_attn.py:789`` calls it) reads it: the layout
    set by :func:`set_kv_cache_layout`, else ``$VLLM_KV_CACHE_LAYOUT``, else
    ``"NHD"``.  Inside a vLLM install the engine's own function is used, so one
    knob drives both the engine's allocation and this backend's stride order."""
    try:
        from vllm.v1.attention.backends.utils import get_kv_cache_layout as engine_layout
    except ImportError:
        engine_layout = None
    if engine_layout is not None:
        return engine_layout()
    if _KV_CACHE_LAYOUT_OVERRIDE is not None:
        return _KV_CACHE_LAYOUT_OVERRIDE
    return os.environ.get("VLLM_KV_CACHE_LAYOUT") or "NHD"


def _batch_invariant() -> bool:
    """vLLM's ``vllm_is_batch_invariant()``: ``$VLLM_BATCH_INVARIANT`` set to a
    non-zero integer.  The kernels here are batch invariant either way (a
    row's reduction order never depends on the batch); the flag is carried
    for the engine's bookkeeping."""
    try:
        return int(os.environ.get("VLLM_BATCH_INVARIANT", "0")) != 0
    except ValueError:
        return False


class AttentionType(str, Enum):
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"
    ENCODER_DECODER = "encoder_decoder"


@dataclass(frozen=True)
class MultipleOf:
    """Kernel block-size constraint (``MultipleOf(16)`` at beam_attn.py:764-765)."""
    base: int


@dataclass
class CommonAttentionMetadata:
    """The per-batch fields of vLLM's CommonAttentionMetadata the builder reads."""
    query_start_loc: torch.Tensor        # [num_reqs+1] int32 (device)
    query_start_loc_cpu: torch.Tensor    # [num_reqs+1] int32 (host)
    seq_lens: torch.Tensor               # [num_reqs] int32 (device)
    seq_lens_cpu: torch.Tensor           # [num_reqs] int32 (host)
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor     # [num_reqs, max_blocks] int32 (device)
    slot_mapping: torch.Tensor           # [num_actual_tokens] int64 (device)
    causal: bool = True


@dataclass
class DecodeGroup:
    """One ``gr_beam_attn_decode`` launch: every beam carries ``q_per_beam``
    query rows; ``token_index`` maps its rows to batch token positions (None
    when they are the batch's tokens in order)."""
    token_index: torch.Tensor | None
    prefix_bt: torch.Tensor
    prefix_len: torch.Tensor
    beam_start: torch.Tensor
    suffix_bt: torch.Tensor
    suffix_len: torch.Tensor
    suffix_start: torch.Tensor | None
    q_per_beam: int
    max_beams: int
    max_prefix_len: int = 0  # host hint for the split decode (0 = unknown)


@dataclass
class PrefillGroup:
    """One ``gr_paged_attn_prefill`` launch over the standard requests:
    request i's queries are rows ``query_start[i] .. query_start[i+1]-1`` of
    the gathered query (``token_index`` maps them to batch positions; None
    when they are the batch's tokens in order) and it sees ``seq_len[i]``
    keys of ``block_table`` row i, causally."""
    token_index: torch.Tensor | None
    block_table: torch.Tensor
    query_start: torch.Tensor
    seq_len: torch.Tensor
    max_query_len: int


@dataclass
class BeamAttentionMetadata:
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    causal: bool = True
    groups: list[DecodeGroup] = field(default_factory=list)
    prefill: PrefillGroup | None = None
    mega_req_idxs: list[int] = field(default_factory=list)
    std_req_idxs: list[int] = field(default_factory=list)
    # the builder's device status word: every launch of the forward ORs the
    # error bits of out-of-range table entries into it (ops.check_status reads it)
    status: torch.Tensor | None = None


class BeamAttentionMetadataBuilder:
    """Routes each request of a batch to a decode group (beam_attn.py:163-570).

    ``_cudagraph_support`` is ``UNIFORM_BATCH`` as in the reference
    (:164), and here it holds: a batch of resident-layout mega requests
    routes to one decode group whose device tables the caller owns, so its
    forward is captured once per batch shape and replayed
    (``vllm_gr_amd.v1.sid_runner``).  The engine configuration the reference
    reads in ``__init__`` (:167-200) is kept under the same names; the
    ahead-of-time FlashAttention schedule (``aot_schedule``,
    ``max_num_splits``) stays off, since the kernels here choose their own
    split."""

    _cudagraph_support = AttentionCGSupport.UNIFORM_BATCH
    supports_update_block_table: bool = True

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device: torch.device):
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = torch.device(device)
        self.block_size = int(kv_cache_spec.block_size)
        self.kv_cache_dtype = getattr(kv_cache_spec, "dtype", None)
        cfg = lambda name: getattr(vllm_config, name, None)
        self.model_config = cfg("model_config")
        self.parallel_config = cfg("parallel_config")
        self.cache_config = cfg("cache_config")
        self.compilation_config = cfg("compilation_config")
        mc, pc = self.model_config, self.parallel_config
        self.num_heads_q = mc.get_num_attention_heads(pc) if mc is not None else None
        self.num_heads_kv = mc.get_num_kv_heads(pc) if mc is not None else None
        self.headdim = mc.get_head_size() if mc is not None else None
        self.max_num_splits = 0
        self.aot_schedule = False
        cc = self.compilation_config
        mode = getattr(cc, "cudagraph_mode", None)
        self.use_full_cuda_graph = bool(mode is not None and mode.has_full_cudagraphs())
        self.max_cudagraph_size = getattr(cc, "max_cudagraph_capture_size", None)
        self.scheduler_metadata = None
        self.aot_sliding_window: tuple[int, int] | None = None
        # one status word for every batch this builder routes: sticky until
        # the caller clears it (ops.check_status after a synchronisation)
        self.status = ops.new_status(self.device)

    def build(self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata,
              fast_build: bool = False) -> BeamAttentionMetadata:
        # one roctx range per build, where the reference has its NVTX range (beam_attn.py:486, :526)
        with roctx_range("BeamAttentionMetadataBuilder.build"):
            return self._build(common_prefix_len, common_attn_metadata)

    def _build(self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata) -> BeamAttentionMetadata:
        m = common_attn_metadata
        info = MEGA_DATA_VAR.get()
        mega_data = info["mega_data"] if info else {}
        req_ids = info["req_ids"] if info else []
        q_starts = m.query_start_loc_cpu.tolist()
        seq_lens = m.seq_lens_cpu.tolist()
        bs = self.block_size
        dev = self.device
        slot_mapping = m.slot_mapping

        mega, ref_mega, std = [], [], []
        for i in range(m.num_reqs):
            rid = req_ids[i] if i < len(req_ids) else None
            md = mega_data.get(rid, {}) if rid is not None else {}
            if not md.get("is_mega_decode", False):
                std.append((i, md))
            elif "beam_kv" in md:
                mega.append((i, md))
            else:
                ref_mega.append((i, md))

        groups: list[DecodeGroup] = []
        # ---- mega-decode requests: one query token per beam over the resident suffix.
        # A table may hold several requests: then exactly that many consecutive batch
        # requests name it, its i-th request being the i-th of them, and their query
        # rows are contiguous, so the table's tensors are used whole.
        if mega:
            runs: list[tuple[object, list[tuple[int, dict]]]] = []
            for i, md in mega:
                table = md["beam_kv"]
                if runs and runs[-1][0] is table and runs[-1][1][-1][0] == i - 1:
                    runs[-1][1].append((i, md))
                else:
                    runs.append((table, [(i, md)]))
            rows, pbt, plen, sbt, slen, widths, slots = [], [], [], [], [], [], []
            max_prefix = max(int(md["prefix_len"]) for _, md in mega)
            for table, members in runs:
                W = table.beam_width
                if len(members) != table.num_reqs:
                    raise ValueError(
                        f"request {req_ids[members[0][0]]}: its beam_kv table holds {table.num_reqs} "
                        f"requests but {len(members)} consecutive requests name it")
                for i, md in members:
                    if int(md["mega_beam_width"]) != W:
                        raise ValueError(f"request {req_ids[i]}: beam_kv must hold requests of "
                                         f"{int(md['mega_beam_width'])} beams")
                    if int(md["cache_len"]) < int(md["prefix_len"]):
                        raise NotImplementedError(
                            "mega decode needs the whole prompt prefix cached (prefill it through the "
                            "standard path first)")
                    if q_starts[i + 1] - q_starts[i] != W:
                        raise ValueError(f"request {req_ids[i]}: expected {W} query tokens (one per "
                                         f"beam), got {q_starts[i + 1] - q_starts[i]}")
                q0, q1 = q_starts[members[0][0]], q_starts[members[-1][0] + 1]
                rows.append((q0, q1))
                pbt.append(table.prefix_bt)
                plen.append(table.prefix_len)
                sbt.append(table.suffix_bt)
                slen.append(table.attention_suffix_len())
                widths.extend([W] * table.num_reqs)
                slots.append((q0, q1, table.slot_mapping()))
            if len(runs) == 1 and rows[0] == (0, m.num_actual_tokens):
                # one table covering the batch: its tensors as they are (no host copies)
                slot_mapping = slots[0][2]
                table = runs[0][0]
                groups.append(DecodeGroup(
                    token_index=None, prefix_bt=table.prefix_bt, prefix_len=table.prefix_len,
                    beam_start=table.beam_start, suffix_bt=table.suffix_bt, suffix_len=slen[0],
                    suffix_start=None, q_per_beam=1, max_beams=table.beam_width, max_prefix_len=max_prefix))
            else:
                slot_mapping = slot_mapping.clone()
                for q0, q1, s in slots:
                    slot_mapping[q0:q1] = s
                groups.append(self._group(rows, m.num_actual_tokens, pbt, plen, widths, sbt, slen, None, 1))
                groups[-1].max_prefix_len = max_prefix

        # ---- the reference's mega layout: causal prefill rows + decode beams
        causal = [(q_starts[i], q_starts[i + 1], i, seq_lens[i]) for i, _ in std]
        if ref_mega:
            causal += self._route_reference_mega(ref_mega, q_starts, m, groups)

        # ---- standard requests (and beam-0 / standard-routed mega rows): one
        # varlen causal launch over their own rows
        prefill = None
        causal = [c for c in causal if c[1] > c[0]]
        if causal:
            rows = [(q0, q1) for q0, q1, _, _ in causal]
            qlens = [q1 - q0 for q0, q1 in rows]
            reqs = [i for _, _, i, _ in causal]
            if not ref_mega and reqs == list(range(m.num_reqs)):  # the batch's own tensors serve as they are
                bt, qs, sl = m.block_table_tensor, m.query_start_loc, m.seq_lens
            else:
                idx = torch.tensor(reqs, dtype=torch.int64).to(dev)
                bt = m.block_table_tensor.index_select(0, idx)
                qs = torch.tensor([0] + qlens, dtype=torch.int64).cumsum(0).to(torch.int32).to(dev)
                sl = torch.tensor([c[3] for c in causal], dtype=torch.int32).to(dev)
            prefill = PrefillGroup(
                token_index=self._token_index(rows, m.num_actual_tokens),
                block_table=bt.to(torch.int32).contiguous(), query_start=qs.to(torch.int32).contiguous(),
                seq_len=sl.to(torch.int32).contiguous(), max_query_len=max(qlens))
        return BeamAttentionMetadata(
            num_actual_tokens=m.num_actual_tokens, max_query_len=m.max_query_len,
            query_start_loc=m.query_start_loc, max_seq_len=m.max_seq_len, seq_lens=m.seq_lens,
            block_table=m.block_table_tensor, slot_mapping=slot_mapping, causal=m.causal,
            groups=groups, prefill=prefill, mega_req_idxs=sorted(i for i, _ in mega + ref_mega),
            std_req_idxs=[i for i, _ in std], status=self.status)

    def _route_reference_mega(self, reqs, q_starts, m, groups) -> list[tuple[int, int, int, int]]:
        """Route the reference-layout mega requests (beam_attn.py:255-413):
        returns their causal-prefill row ranges ``(q0, q1, request, seq_len)``
        and appends their decode beams to ``groups``, one group per query
        count (full beams take ``mega_decode_steps`` rows; the chunk budget
        leaves at most one partial beam per request)."""
        bs, dev = self.block_size, self.device
        causal = []
        beams: dict[int, list[tuple[int, int, int, int]]] = {}  # rows -> [(request, prefix, pos0, row0)]
        for i, md in reqs:
            P, C = int(md["prefix_len"]), int(md["cache_len"])
            W, t = int(md["mega_beam_width"]), int(md["mega_decode_steps"])
            q0, q1 = q_starts[i], q_starts[i + 1]
            # an uncached prefix of two blocks or more: the standard path over
            # its rows (:273-282); the reference writes the new hit back
            std_q = 0
            if P - C > 0 and P - C >= 2 * bs:
                std_q = min(P - C, q1 - q0)
                C += std_q
                md["cache_len"] = C
            start = q0 + std_q
            budget = q1 - start
            b0 = 0
            if W > 0 and t > 0 and budget > 0:
                tail = P - C
                assert tail >= 0, f"prefix_len: {P}, cache_len: {C}"
                # beam 0: the shared tail and its own tokens, continuing the
                # causal prefill at position C (:368-372)
                b0 = min(budget, tail + t)
                budget -= b0
                row = start + b0
                for b in range(1, W):
                    if budget <= 0:
                        break
                    n = min(budget, t)  # the last beam may be cut by the chunk budget (:351-366)
                    beams.setdefault(n, []).append((i, P, P + b * t, row))
                    row += n
                    budget -= n
            if std_q + b0 > 0:
                causal.append((q0, start + b0, i, C + b0))
        for n, members in sorted(beams.items(), reverse=True):
            groups.append(self._reference_beam_group(members, n, m, bs, dev))
        return causal

    def _reference_beam_group(self, members, n, m, bs, dev) -> DecodeGroup:
        """Decode beams of the reference layout with ``n`` query rows each:
        prefix = the request's first ``prefix_len`` tokens; suffix = the
        beam's own ``n`` tokens at logical positions ``pos0 ..`` of the same
        block-table row, given to the kernel as a window of that row."""
        reqs = []
        for i, P, _, _ in members:
            if not reqs or reqs[-1][0] != i:
                reqs.append((i, P))
        widths = [sum(1 for mi in members if mi[0] == i) for i, _ in reqs]
        req_of_beam = torch.tensor([mi[0] for mi in members], dtype=torch.int64)
        pos0 = torch.tensor([mi[2] for mi in members], dtype=torch.int64)
        first = pos0 // bs
        cap = int(((pos0 % bs + n + bs - 1) // bs).max())
        nb = m.block_table_tensor.shape[1]
        win = (first[:, None] + torch.arange(cap)[None]).clamp(max=nb - 1)
        bt = m.block_table_tensor
        suffix_bt = bt[req_of_beam.to(dev)[:, None], win.to(dev)].to(torch.int32).contiguous()
        rows = [(r0, r0 + n) for _, _, _, r0 in members]
        idx = torch.tensor([i for i, _ in reqs], dtype=torch.int64).to(dev)
        return DecodeGroup(
            token_index=self._token_index(rows, m.num_actual_tokens),
            prefix_bt=bt.index_select(0, idx).to(torch.int32).contiguous(),
            prefix_len=torch.tensor([P for _, P in reqs], dtype=torch.int32).to(dev),
            beam_start=torch.tensor([0] + widths, dtype=torch.int64).cumsum(0).to(torch.int32).to(dev),
            suffix_bt=suffix_bt,
            suffix_len=torch.full((len(members),), n, dtype=torch.int32).to(dev),
            suffix_start=(pos0 % bs).to(torch.int32).to(dev), q_per_beam=n, max_beams=max(widths),
            max_prefix_len=max(P for _, P in reqs))

    def _token_index(self, rows, ntok) -> torch.Tensor | None:
        """Batch positions of token ranges ``(q0, q1)``; None when they are
        the batch's tokens in order."""
        pos, in_order = 0, True
        for q0, q1 in rows:
            in_order &= q0 == pos
            pos = q1
        if in_order and pos == ntok:
            return None
        return torch.cat([torch.arange(q0, q1) for q0, q1 in rows]).to(self.device)

    def _group(self, rows, ntok, pbt, plen, widths, sbt, slen, sstart, T) -> DecodeGroup:
        """``rows``: the group's batch token ranges ``(q0, q1)`` in beam order."""
        dev = self.device
        pw = max(t.shape[1] for t in pbt)
        sw = max(t.shape[1] for t in sbt)
        pad = lambda ts, w: torch.cat([torch.nn.functional.pad(t, (0, w - t.shape[1]), value=-1) for t in ts])
        beam_start = torch.tensor([0] + widths, dtype=torch.int64).cumsum(0).to(torch.int32).to(dev)
        return DecodeGroup(
            token_index=self._token_index(rows, ntok), prefix_bt=pad(pbt, pw).contiguous(),
            prefix_len=torch.cat(plen).contiguous(), beam_start=beam_start,
            suffix_bt=pad(sbt, sw).contiguous(), suffix_len=torch.cat(slen).to(torch.int32).contiguous(),
            suffix_start=None if sstart is None else torch.cat(sstart).contiguous(), q_per_beam=T,
            max_beams=max(widths))

    def update_block_table(self, metadata: BeamAttentionMetadata, blk_table: torch.Tensor,
                           slot_mapping: torch.Tensor) -> BeamAttentionMetadata:
        new = copy.copy(metadata)
        new.block_table = blk_table
        new.slot_mapping = slot_mapping
        return new


class BeamAttentionImpl:
    """``AttentionImpl`` of the backend (beam_attn.py:575-755).

    ``supports_quant_query_input`` is true as in the reference (:626): with an
    fp8 cache vLLM then hands ``forward`` an e4m3 query, which is widened to
    the output dtype times the layer's ``_q_scale`` before the launch (the
    kernels take fp16/bf16 queries).  ``vllm_flash_attn_version`` is None:
    no FlashAttention build is involved."""

    can_return_lse_for_decode: bool = True

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: list[float] | None, sliding_window: int | None, kv_cache_dtype: str,
                 logits_soft_cap: float | None = None, attn_type: str = AttentionType.DECODER,
                 kv_sharing_target_layer_name: str | None = None,
                 running_sinks: torch.Tensor | None = None) -> None:
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        if num_heads % num_kv_heads != 0:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        self.num_queries_per_kv = num_heads // num_kv_heads
        # ALiBi slopes, the sliding window as (left, right) and the sinks as the
        # reference keeps them (beam_attn.py:597-625); they reach every kernel
        # launch through gr_attn_options
        self.alibi_slopes = None if alibi_slopes is None else torch.tensor(alibi_slopes, dtype=torch.float32)
        if sliding_window is None:
            self.sliding_window = (-1, -1)
        elif attn_type == AttentionType.ENCODER_ONLY:
            self.sliding_window = (sliding_window - 1, sliding_window - 1)
        else:
            self.sliding_window = (sliding_window - 1, 0)
        if kv_cache_dtype not in ("auto", None) + FP8_KV_DTYPES:
            raise NotImplementedError(f"BeamAttention does not support kv_cache_dtype={kv_cache_dtype}.")
        # an fp8 e4m3 cache (beam_attn.py:734-737): written with the layer's
        # _k_scale / _v_scale (reshape_and_cache_flash, :727-732), read back
        # scaled by them
        self.kv_fp8 = kv_cache_dtype in FP8_KV_DTYPES
        self._scales: dict = {}
        self.sinks = running_sinks
        if self.sinks is not None:
            assert self.sinks.shape[0] == num_heads, (
                "Sinks must have the same number of heads as the number of heads in the layer")
        self._dev_opts: dict = {}
        self.kv_cache_dtype = kv_cache_dtype
        self.logits_soft_cap = float(logits_soft_cap or 0.0)
        self.attn_type = attn_type
        self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
        self.vllm_flash_attn_version = None
        self.batch_invariant_enabled = _batch_invariant()
        self.supports_quant_query_input = True
        self.use_cascade = True

    def _kv_scales(self, layer, device):
        """The layer's (_k_scale, _v_scale) as one-element float32 device
        tensors (vLLM keeps them as tensors; floats and a missing layer are
        accepted, 1.0 by default); None for a cache that is not fp8."""
        if not self.kv_fp8:
            return None, None
        out = []
        for name in ("_k_scale", "_v_scale"):
            v = getattr(layer, name, None) if layer is not None else None
            if isinstance(v, torch.Tensor) and v.device == device and v.dtype == torch.float32 and v.numel() == 1:
                out.append(v.reshape(1))
                continue
            val = 1.0 if v is None else float(v)
            key = (name, device, val)
            t = self._scales.get(key)
            if t is None:
                t = self._scales[key] = torch.tensor([val], dtype=torch.float32, device=device)
            out.append(t)
        return out[0], out[1]

    def _options(self, device) -> dict:
        """The optional features as kernel arguments on ``device`` (float32
        copies of the sinks and slopes, made once per device)."""
        opts = self._dev_opts.get(device)
        if opts is None:
            opts = dict(sinks=None if self.sinks is None else
                        self.sinks.detach().to(device=device, dtype=torch.float32).contiguous(),
                        alibi_slopes=None if self.alibi_slopes is None else self.alibi_slopes.to(device))
            self._dev_opts[device] = opts
        return opts

    def forward(self, layer, query: torch.Tensor, key: torch.Tensor | None, value: torch.Tensor | None,
                kv_cache: torch.Tensor, attn_metadata: BeamAttentionMetadata | None,
                output: torch.Tensor | None = None, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None) -> torch.Tensor:
        with roctx_range("BeamAttentionImpl.forward"):
            return self._forward(layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                                 output_block_scale)

    def _forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                 output_block_scale) -> torch.Tensor:
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("fused output quantization is not yet supported for BeamAttentionImpl")
        if attn_metadata is None:
            return output.fill_(0)
        k_cache, v_cache = ops.split_kv_cache(kv_cache)
        n = attn_metadata.num_actual_tokens
        k_sc, v_sc = self._kv_scales(layer, query.device)
        if self.kv_sharing_target_layer_name is None and key is not None and value is not None:
            ops.reshape_and_cache(key[:n], value[:n], k_cache, v_cache, attn_metadata.slot_mapping,
                                  status=attn_metadata.status, k_scale=k_sc, v_scale=v_sc)
        if query.dtype == torch.float8_e4m3fn:
            # a query vLLM quantized for the fp8 cache (supports_quant_query_input)
            q_scale = getattr(layer, "_q_scale", None) if layer is not None else None
            query = query.to(output.dtype)
            if q_scale is not None:
                query = query * (q_scale.to(device=query.device, dtype=torch.float32).to(output.dtype)
                                 if isinstance(q_scale, torch.Tensor) else float(q_scale))
        opts = self._options(query.device)
        BeamAttentionImpl.cascade_attention(
            output=output, query=query, key_cache=k_cache, value_cache=v_cache, attn_metadata=attn_metadata,
            sliding_window_size=list(self.sliding_window), scale=self.scale,
            logits_soft_cap=self.logits_soft_cap, vllm_flash_attn_version=self.vllm_flash_attn_version,
            s_aux=opts["sinks"], alibi_slopes=opts["alibi_slopes"], k_scale=k_sc, v_scale=v_sc)
        return output

    @staticmethod
    def cascade_attention(output: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                          value_cache: torch.Tensor, attn_metadata: BeamAttentionMetadata,
                          sliding_window_size, scale: float, logits_soft_cap: float,
                          vllm_flash_attn_version=None, s_aux: torch.Tensor | None = None,
                          alibi_slopes: torch.Tensor | None = None, *, k_scale: torch.Tensor | None = None,
                          v_scale: torch.Tensor | None = None) -> None:
        """The attention of ``forward`` after the cache write
        (beam_attn.py:629-701, same arguments): every decode group is one
        ``gr_beam_attn_decode`` launch (prefix, suffix and their merge in
        one kernel) and the standard rows one ``gr_paged_attn_prefill``
        launch, written into ``output`` in place.  ``sliding_window_size`` is
        the impl's ``(left, right)`` window ((-1, -1) = none), applied by
        absolute key position; ``s_aux`` are the sinks; an fp8 cache is read
        as e4m3 times ``k_scale`` / ``v_scale`` (one-element float32 device
        tensors).  ``vllm_flash_attn_version`` is accepted and unused."""
        dev = query.device
        n = attn_metadata.num_actual_tokens
        sinks = None if s_aux is None else s_aux.detach().to(device=dev, dtype=torch.float32).contiguous()
        slopes = None if alibi_slopes is None else alibi_slopes.to(device=dev, dtype=torch.float32).contiguous()
        left, right = (-1, -1) if sliding_window_size is None else (int(sliding_window_size[0]),
                                                                     int(sliding_window_size[1]))
        window = (left, right) if left >= 0 or right >= 0 else None
        # decode attention is causal over the beam's own tokens: its window has no right bound
        dec_window = None if window is None else (window[0], -1)
        for g in attn_metadata.groups:
            q = query[:n] if g.token_index is None else query.index_select(0, g.token_index)
            out = output[:n] if g.token_index is None else None
            res = ops.beam_attn_decode(q, key_cache, value_cache, g.prefix_bt, g.prefix_len, g.beam_start,
                                       g.suffix_bt, g.suffix_len, g.suffix_start, q_per_beam=g.q_per_beam,
                                       scale=scale, softcap=logits_soft_cap,
                                       max_beams_per_req=g.max_beams, out=out, max_prefix_len=g.max_prefix_len,
                                       window=dec_window, sinks=sinks, alibi_slopes=slopes,
                                       status=attn_metadata.status, k_scale=k_scale, v_scale=v_scale)
            if g.token_index is not None:
                output.index_copy_(0, g.token_index, res)
        p = attn_metadata.prefill
        if p is not None:
            q = query[:n] if p.token_index is None else query.index_select(0, p.token_index)
            out = output[:n] if p.token_index is None else None
            causal = attn_metadata.causal
            win = window
            if win is not None and causal:
                win = (win[0], -1)
            res = ops.paged_attn_prefill(q, key_cache, value_cache, p.block_table, p.query_start, p.seq_len,
                                         max_query_len=p.max_query_len, scale=scale,
                                         softcap=logits_soft_cap, out=out, causal=causal, window=win,
                                         sinks=sinks, alibi_slopes=slopes,
                                         status=attn_metadata.status, k_scale=k_scale, v_scale=v_scale)
            if p.token_index is not None:
                output.index_copy_(0, p.token_index, res)


class BeamAttentionBackend:
    """Static surface registered as the ``CUSTOM`` backend (beam_attn.py:758-846)."""

    accept_output_buffer = True
    supported_dtypes = [torch.float16, torch.bfloat16]

    @staticmethod
    def get_supported_kernel_block_sizes() -> list:
        return [MultipleOf(16)]

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type in (AttentionType.DECODER, AttentionType.ENCODER, AttentionType.ENCODER_ONLY,
                             AttentionType.ENCODER_DECODER)

    @staticmethod
    def get_impl_cls() -> type[BeamAttentionImpl]:
        return BeamAttentionImpl

    @staticmethod
    def get_builder_cls() -> type[BeamAttentionMetadataBuilder]:
        return BeamAttentionMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple[int, ...]:
        return (2, num_blocks, block_size, num_kv_heads, head_size)

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple[int, ...]:
        # the layout the engine configured (get_kv_cache_layout); the kernels
        # take block/token/head strides, so both layouts run as is
        cache_layout = get_kv_cache_layout()
        if cache_layout == "NHD":
            return (2, 0, 1, 3, 4, 5) if include_num_layers_dimension else (0, 1, 2, 3, 4)
        if cache_layout == "HND":
            return (2, 4, 0, 1, 3, 5) if include_num_layers_dimension else (0, 1, 3, 2, 4)
        raise ValueError(f"Unknown cache layout format {cache_layout}.")

    @staticmethod
    def get_fp8_dtype_for_flashattn(kv_cache_dtype: str) -> torch.dtype:
        """The storage dtype of an fp8 cache (beam_attn.py:800-804): e4m3 only."""
        if kv_cache_dtype in FP8_KV_DTYPES:
            return torch.float8_e4m3fn
        raise ValueError(f"Unrecognized FP8 dtype: {kv_cache_dtype}")

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        return head_size % 8 == 0 and head_size <= 256

    @classmethod
    def supports_kv_cache_dtype(cls, kv_cache_dtype: str | None) -> bool:
        return kv_cache_dtype is None or kv_cache_dtype == "auto" or kv_cache_dtype in FP8_KV_DTYPES

    @classmethod
    def supports_sink(cls) -> bool:
        return True  # sinks join every row's softmax (gr_attn_options)

    @classmethod
    def supports_compute_capability(cls, capability) -> bool:
        """gfx950 (MI355X): the kernels are built for that target only."""
        return str(capability).startswith("gfx950")

    @classmethod
    def supports_combination(cls, head_size, dtype, kv_cache_dtype, block_size, use_mla, has_sink,
                             use_sparse, device_capability) -> str | None:
        if dtype not in cls.supported_dtypes:
            return f"Unsupported dtype {dtype}."
        if not cls.supports_head_size(head_size):
            return f"Unsupported head_size={head_size}."
        if not cls.supports_kv_cache_dtype(kv_cache_dtype):
            return f"Unsupported kv_cache_dtype={kv_cache_dtype}."
        if block_size is not None and block_size % 16 != 0:
            return f"block_size={block_size} not multiple of 16."
        if not cls.supports_compute_capability(device_capability):
            return "Requires gfx950 (MI355X)."
        if has_sink and not cls.supports_sink():
            return "No attention sink support."
        if use_mla:
            return "No MLA support."
        if use_sparse:
            return "No sparse support."
        return None
