"""Host logic of the backend mirror (CPU only, no kernel launch): the static
backend contract (vllm_gr/v1/attention/backends/beam_attn.py:758-846), the
impl's argument checks (:579-627, :715-723), the metadata builder's routing
of mega-decode and standard requests, the resident beam table's position /
slot arithmetic (engine_core_patch.py:362-365; slot = block * bs + offset,
beam_attn.py:77-85) and the beam-search step's fork_info / abort set
(serving_engine.py:141-142, 588-590; tests/test_batch_and_fork_unit.py
5.10 and 5.15)."""

from __future__ import annotations

import types

import pytest
import torch

from vllm_gr_amd.entrypoints import beam_search as bsm
from vllm_gr_amd.v1.attention.backends import beam_attn as ba
from vllm_gr_amd.v1.beam_kv import BeamKVTable

B = ba.BeamAttentionBackend


def test_backend_static_contract():
    assert B.get_name() == "CUSTOM"
    assert B.accept_output_buffer is True
    assert B.get_supported_kernel_block_sizes() == [ba.MultipleOf(16)]
    assert B.get_kv_cache_shape(10, 16, 8, 128) == (2, 10, 16, 8, 128)
    assert B.get_kv_cache_stride_order() == (0, 1, 2, 3, 4)
    assert B.get_kv_cache_stride_order(True) == (2, 0, 1, 3, 4, 5)
    assert B.get_impl_cls() is ba.BeamAttentionImpl
    assert B.get_builder_cls() is ba.BeamAttentionMetadataBuilder
    for hs, ok in ((8, True), (128, True), (256, True), (12, False), (264, False)):
        assert B.supports_head_size(hs) is ok


def test_stride_order_follows_engine_layout(monkeypatch):
    """get_kv_cache_stride_order reads the layout the engine configured
    (beam_attn.py:787-798): the override, else $VLLM_KV_CACHE_LAYOUT."""
    monkeypatch.delenv("VLLM_KV_CACHE_LAYOUT", raising=False)
    assert ba.get_kv_cache_layout() == "NHD"
    monkeypatch.setenv("VLLM_KV_CACHE_LAYOUT", "HND")
    assert B.get_kv_cache_stride_order() == (0, 1, 3, 2, 4)
    assert B.get_kv_cache_stride_order(True) == (2, 4, 0, 1, 3, 5)
    try:
        ba.set_kv_cache_layout("NHD")  # the override wins over the environment
        assert B.get_kv_cache_stride_order() == (0, 1, 2, 3, 4)
        ba.set_kv_cache_layout("XYZ")
        with pytest.raises(ValueError, match="Unknown cache layout"):
            B.get_kv_cache_stride_order()
    finally:
        ba.set_kv_cache_layout(None)
    assert B.get_kv_cache_stride_order() == (0, 1, 3, 2, 4)


def test_fp8_dtype_and_graph_support():
    assert B.get_fp8_dtype_for_flashattn("fp8") is torch.float8_e4m3fn
    assert B.get_fp8_dtype_for_flashattn("fp8_e4m3") is torch.float8_e4m3fn
    with pytest.raises(ValueError, match="Unrecognized FP8 dtype"):
        B.get_fp8_dtype_for_flashattn("fp8_e5m2")
    assert ba.BeamAttentionMetadataBuilder._cudagraph_support is ba.AttentionCGSupport.UNIFORM_BATCH
    assert ba.AttentionCGSupport.UNIFORM_BATCH.value == 2


def test_plugin_members_match_reference():
    """Every member the reference's backend, impl and builder classes define
    (tests/golden/plugin_members.json, read from beam_attn.py's text with the
    line of each) exists on the classes here, class members on the class and
    __init__ members on an instance."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "plugin_members.json")) as f:
        ref = json.load(f)["classes"]
    impl = ba.BeamAttentionImpl(num_heads=32, head_size=128, scale=0.1, num_kv_heads=8, alibi_slopes=None,
                                sliding_window=None, kv_cache_dtype="auto")
    cfg = types.SimpleNamespace(
        model_config=types.SimpleNamespace(get_num_attention_heads=lambda pc: 32,
                                           get_num_kv_heads=lambda pc: 8, get_head_size=lambda: 128),
        parallel_config=None, cache_config=None,
        compilation_config=types.SimpleNamespace(
            cudagraph_mode=types.SimpleNamespace(has_full_cudagraphs=lambda: True),
            max_cudagraph_capture_size=512))
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=16, dtype=torch.bfloat16),
                                              ["l0"], cfg, "cpu")
    assert (builder.num_heads_q, builder.num_heads_kv, builder.headdim) == (32, 8, 128)
    assert builder.use_full_cuda_graph and builder.max_cudagraph_size == 512
    assert builder.kv_cache_dtype is torch.bfloat16 and builder.max_num_splits == 0
    here = {"BeamAttentionBackend": (B, B), "BeamAttentionImpl": (ba.BeamAttentionImpl, impl),
            "BeamAttentionMetadataBuilder": (ba.BeamAttentionMetadataBuilder, builder)}
    missing = []
    for name, kinds in ref.items():
        cls, inst = here[name]
        missing += [f"{name}.{m} (beam_attn.py:{ln})" for m, ln in kinds["class"].items() if not hasattr(cls, m)]
        missing += [f"{name}().{m} (beam_attn.py:{ln})" for m, ln in kinds["instance"].items()
                    if not hasattr(inst, m)]
    assert not missing, missing
    assert impl.supports_quant_query_input and impl.use_cascade
    assert callable(ba.BeamAttentionImpl.cascade_attention)


def test_layer_set_cache_holds_no_tensor():
    """The fork's per-cache-list pointer cache keeps addresses only: dropping
    the caches frees them, and the dead entry is evicted on the next lookup."""
    import gc
    import weakref
    from vllm_gr_amd import ops
    caches = [torch.zeros(2, 4, 16, 2, 8, dtype=torch.bfloat16) for _ in range(3)]
    ls = ops._layer_set(caches)
    assert ls.n == 3 and ls.shape == (4, 16, 2, 8)
    refs = [weakref.ref(c) for c in caches]
    del caches, ls
    gc.collect()
    assert all(r() is None for r in refs)
    other = [torch.zeros(2, 4, 16, 2, 8, dtype=torch.bfloat16)]
    ops._layer_set(other)
    assert all(entry.alive() for entry in ops._LAYER_SETS.values())


def test_supports_combination_sinks_accepted():
    args = dict(head_size=128, dtype=torch.bfloat16, kv_cache_dtype="auto", block_size=16, use_mla=False,
                has_sink=True, use_sparse=False, device_capability="gfx950:sramecc+:xnack-")
    assert B.supports_sink() and B.supports_combination(**args) is None


@pytest.mark.parametrize("kw,reason", [
    (dict(dtype=torch.float32), "Unsupported dtype"),
    (dict(head_size=264), "Unsupported head_size"),
    (dict(kv_cache_dtype="fp8_e5m2"), "Unsupported kv_cache_dtype"),
    (dict(block_size=8), "not multiple of 16"),
    (dict(device_capability="gfx942"), "gfx950"),
    (dict(use_mla=True), "MLA"),
    (dict(use_sparse=True), "sparse"),
])
def test_supports_combination_reasons(kw, reason):
    args = dict(head_size=128, dtype=torch.bfloat16, kv_cache_dtype="auto", block_size=16, use_mla=False,
                has_sink=False, use_sparse=False, device_capability="gfx950:sramecc+:xnack-")
    assert B.supports_combination(**args) is None
    args.update(kw)
    assert reason in B.supports_combination(**args)


def test_impl_rejects_unsupported_features():
    mk = lambda **kw: ba.BeamAttentionImpl(**{**dict(num_heads=32, head_size=128, scale=0.1, num_kv_heads=8,
                                                      alibi_slopes=None, sliding_window=None,
                                                      kv_cache_dtype="auto"), **kw})
    impl = mk()
    assert impl.num_queries_per_kv == 4 and impl.logits_soft_cap == 0.0
    # fp8 e4m3 caches are accepted (beam_attn.py:617-618, :801-804); e5m2 is
    # not (the reference's get_fp8_dtype_for_flashattn knows only e4m3)
    assert mk(kv_cache_dtype="fp8").kv_fp8 and mk(kv_cache_dtype="fp8_e4m3").kv_fp8 and not impl.kv_fp8
    assert B.supports_kv_cache_dtype("fp8") and B.supports_kv_cache_dtype("fp8_e4m3")
    assert not B.supports_kv_cache_dtype("fp8_e5m2")
    with pytest.raises(NotImplementedError):
        mk(kv_cache_dtype="fp8_e5m2")
    with pytest.raises(AssertionError, match="Sinks must have the same number of heads"):
        mk(running_sinks=torch.zeros(31))
    # the reference's window convention (beam_attn.py:600-605)
    assert mk(sliding_window=128).sliding_window == (127, 0)
    assert mk(sliding_window=128, attn_type=ba.AttentionType.ENCODER_ONLY).sliding_window == (127, 127)
    assert mk().sliding_window == (-1, -1)
    assert mk(alibi_slopes=[0.1] * 32).alibi_slopes.dtype == torch.float32
    assert mk(running_sinks=torch.zeros(32)).sinks.shape == (32,)
    for t in ba.AttentionType:
        assert ba.BeamAttentionBackend.supports_attn_type(t)
    assert not ba.BeamAttentionBackend.supports_attn_type("mamba")
    q = torch.zeros(4, 32, 128)
    kv = torch.zeros(2, 4, 16, 8, 128)
    with pytest.raises(AssertionError):
        impl.forward(None, q, None, None, kv, None, output=None)
    with pytest.raises(NotImplementedError):
        impl.forward(None, q, None, None, kv, None, output=torch.ones_like(q), output_scale=torch.ones(1))
    out = torch.ones_like(q)
    assert torch.equal(impl.forward(None, q, None, None, kv, None, output=out), torch.zeros_like(q))


def _table(W=3, P=20, bs=16, lens=(0, 5, 16)):
    prefix_bt = torch.tensor([[7, 3]], dtype=torch.int32)
    suffix_bt = torch.tensor([[10, 11], [12, 13], [14, 15]], dtype=torch.int32)[:W]
    return BeamKVTable(prefix_bt, torch.tensor([P]), W, suffix_bt,
                       torch.tensor(lens, dtype=torch.int32), block_size=bs)


def test_beam_table_positions_and_slots():
    t = _table()
    # beam b's j-th suffix token sits at prefix_len + j (engine_core_patch.py:362-365)
    assert t.positions().tolist() == [20, 25, 36]
    # next token slot: suffix position L -> block suffix_bt[n][L // 16], offset L % 16
    assert t.slot_mapping().tolist() == [10 * 16 + 0, 12 * 16 + 5, 15 * 16 + 0]
    assert t.attention_suffix_len().tolist() == [1, 6, 17]
    t.advance()
    assert t.suffix_len.tolist() == [1, 6, 17]
    full = _table(lens=(31, 32, 0))
    assert full.slot_mapping().tolist() == [11 * 16 + 15, -1, 14 * 16]


def _common(q_lens, seq_lens, bt, bs=16):
    qs = torch.tensor([0] + list(q_lens)).cumsum(0).to(torch.int32)
    n = int(qs[-1])
    slots = torch.arange(1000, 1000 + n, dtype=torch.int64)
    return ba.CommonAttentionMetadata(
        query_start_loc=qs, query_start_loc_cpu=qs, seq_lens=torch.tensor(seq_lens, dtype=torch.int32),
        seq_lens_cpu=torch.tensor(seq_lens, dtype=torch.int32), num_reqs=len(q_lens), num_actual_tokens=n,
        max_query_len=max(q_lens), max_seq_len=max(seq_lens), block_table_tensor=bt, slot_mapping=slots)


def test_builder_routes_mega_and_standard_requests():
    table = _table()
    bt = torch.tensor([[7, 3, 0, 0], [20, 21, 22, 23], [30, 31, 32, 33]], dtype=torch.int32)
    # request "a": mega decode, 3 beams; "b": standard decode; "c": standard prefill of 5 tokens
    m = _common([3, 1, 5], [20, 40, 45], bt)
    info = {"req_ids": ["a", "b", "c"],
            "mega_data": {"a": dict(is_mega_decode=True, mega_beam_width=3, mega_decode_steps=2, prefix_len=20,
                                    cache_len=20, beam_kv=table)}}
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=16), ["l0"], None, "cpu")
    tok = ba.MEGA_DATA_VAR.set(info)
    try:
        md = builder.build(0, m)
    finally:
        ba.MEGA_DATA_VAR.reset(tok)
    assert md.mega_req_idxs == [0] and md.std_req_idxs == [1, 2]
    # mega rows write their K/V into each beam's private block; other rows keep vLLM's slots
    assert md.slot_mapping[:3].tolist() == table.slot_mapping().tolist()
    assert md.slot_mapping[3:].tolist() == list(range(1003, 1009))
    (g_mega,) = md.groups
    assert g_mega.q_per_beam == 1 and g_mega.token_index.tolist() == [0, 1, 2]
    assert g_mega.beam_start.tolist() == [0, 3] and g_mega.prefix_len.tolist() == [20]
    assert g_mega.suffix_len.tolist() == [1, 6, 17]
    # standard decode (1 new token of 40) and prefill chunk (5 new of 45): one varlen causal
    # launch over their own block-table rows (flash_attn_varlen_func, beam_attn.py:643-654)
    p = md.prefill
    assert p.token_index.tolist() == [3, 4, 5, 6, 7, 8]
    assert p.query_start.tolist() == [0, 1, 6] and p.seq_len.tolist() == [40, 45]
    assert p.block_table.tolist() == bt[1:].tolist() and p.max_query_len == 5


def test_builder_standard_only_batch_uses_batch_tensors():
    bt = torch.tensor([[1, 2, 0], [3, 4, 5]], dtype=torch.int32)
    m = _common([17, 40], [17, 40], bt)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=16), ["l0"], None, "cpu")
    md = builder.build(0, m)
    assert md.groups == [] and md.prefill.token_index is None and md.prefill.max_query_len == 40
    assert md.prefill.block_table is m.block_table_tensor and md.prefill.seq_len is m.seq_lens
    assert md.prefill.query_start is m.query_start_loc


def test_builder_rejects_inconsistent_mega_request():
    table = _table()
    bt = torch.zeros(1, 4, dtype=torch.int32)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=16), ["l0"], None, "cpu")
    for md_over, q, exc in ((dict(), 2, ValueError), (dict(cache_len=10), 3, NotImplementedError)):
        md = dict(is_mega_decode=True, mega_beam_width=3, mega_decode_steps=1, prefix_len=20, cache_len=20,
                  beam_kv=table)
        md.update(md_over)
        tok = ba.MEGA_DATA_VAR.set({"req_ids": ["a"], "mega_data": {"a": md}})
        try:
            with pytest.raises(exc):
                builder.build(0, _common([q], [20], bt))
        finally:
            ba.MEGA_DATA_VAR.reset(tok)


def test_fork_info_and_abort_set():
    # tests/test_batch_and_fork_unit.py 5.15: selection (1, 60), (0, 50), (1, 61)
    res = bsm.PruneResult(parent=torch.tensor([[1, 0, 1]], dtype=torch.int32),
                          token=torch.tensor([[60, 50, 61]], dtype=torch.int32),
                          score=torch.tensor([[-0.5, -1.0, -1.5]]), eos_score=torch.full((1, 3), -float("inf")))
    assert bsm.fork_info(res) == [[(1, 60), (0, 50), (1, 61)]]
    assert bsm.pruned_parents(res, 3) == [[2]]
    # 5.10: parents 0, 2, 4 of five selected -> beams 1 and 3 aborted
    res5 = bsm.PruneResult(parent=torch.tensor([[0, 2, 4, 0, 2]], dtype=torch.int32),
                           token=torch.zeros(1, 5, dtype=torch.int32), score=torch.zeros(1, 5),
                           eos_score=torch.zeros(1, 5))
    assert bsm.pruned_parents(res5, 5) == [[1, 3]]


def _ref_build(q_lens, seq_lens, bt, mega, bs=16):
    """Build with the reference's own mega dicts (no beam_kv)."""
    m = _common(q_lens, seq_lens, bt, bs)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=bs), ["l0"], None, "cpu")
    rids = [f"r{i}" for i in range(len(q_lens))]
    tok = ba.MEGA_DATA_VAR.set({"req_ids": rids, "mega_data": {rids[i]: d for i, d in mega.items()}})
    try:
        return builder.build(0, m)
    finally:
        ba.MEGA_DATA_VAR.reset(tok)


def _ref_mega(P, C, W, t):
    return dict(is_mega_decode=True, mega_beam_width=W, mega_decode_steps=t, prefix_len=P, cache_len=C)


def test_builder_reference_layout_complete_step():
    """W=3, P=20, block 16, t=2, cache hit 16 (worked by hand): rows 0..5 are
    beam 0 (the tail at positions 16..19 and its tokens at 20, 21) -> one
    causal prefill row range over 22 keys; beams 1 and 2 (rows 6..7 and 8..9,
    own tokens at positions 22.. and 24..) -> a decode group with the whole
    20-token prompt as prefix and 2 query rows each."""
    bt = torch.tensor([[5, 9, 4, 0]], dtype=torch.int32)
    md = _ref_build([10], [26], bt, {0: _ref_mega(20, 16, 3, 2)})
    p = md.prefill
    assert p.token_index.tolist() == list(range(6)) and p.seq_len.tolist() == [22]
    assert p.query_start.tolist() == [0, 6] and p.block_table.tolist() == bt.tolist()
    (g,) = md.groups
    assert g.q_per_beam == 2 and g.token_index.tolist() == [6, 7, 8, 9]
    assert g.prefix_len.tolist() == [20] and g.beam_start.tolist() == [0, 2]
    assert g.prefix_bt.tolist() == bt.tolist()
    # positions 22 and 24 live in logical block 1 (physical 9) at offsets 6 and 8
    assert g.suffix_bt.tolist() == [[9], [9]] and g.suffix_start.tolist() == [6, 8]
    assert g.suffix_len.tolist() == [2, 2]
    assert md.slot_mapping is not None and md.mega_req_idxs == [0]


def test_builder_reference_layout_budget_and_standard_routing():
    bt = torch.tensor([[5, 9, 4, 0], [1, 2, 3, 6]], dtype=torch.int32)
    # request 0: 7 rows -> beam 0 takes 6, beam 1 only 1 of its 2, beam 2 none;
    # request 1: P=40 with nothing cached -> rows 0..39 standard over 40 keys,
    # beam 0's 1 token continues that prefill, beam 1 decodes at position 41
    mega = {0: _ref_mega(20, 16, 3, 2), 1: _ref_mega(40, 0, 2, 1)}
    md = _ref_build([7, 42], [26, 42], bt, mega)
    assert mega[1]["cache_len"] == 40  # written back (beam_attn.py:280)
    p = md.prefill
    assert p.token_index.tolist() == list(range(6)) + list(range(7, 48))
    assert p.query_start.tolist() == [0, 6, 47] and p.seq_len.tolist() == [22, 41]
    assert p.block_table.tolist() == bt.tolist()
    (g,) = md.groups  # both decode beams have one row: one group
    assert g.q_per_beam == 1 and g.token_index.tolist() == [6, 48]
    assert g.prefix_len.tolist() == [20, 40] and g.beam_start.tolist() == [0, 1, 2]
    assert g.suffix_start.tolist() == [22 % 16, 41 % 16] and g.suffix_bt[:, 0].tolist() == [9, 3]
    # a full beam and a budget-cut one make two groups (2 rows, 1 row)
    md = _ref_build([9], [26], bt[:1], {0: _ref_mega(20, 16, 3, 2)})
    assert [g.q_per_beam for g in md.groups] == [2, 1]
    assert md.groups[0].token_index.tolist() == [6, 7] and md.groups[1].token_index.tolist() == [8]
    # the reference's assertion for a cache hit past the prefix
    with pytest.raises(AssertionError, match="prefix_len: 20, cache_len: 24"):
        _ref_build([6], [26], bt[:1], {0: _ref_mega(20, 24, 3, 2)})
