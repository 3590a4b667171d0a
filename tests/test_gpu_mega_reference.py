"""BeamAttentionImpl.forward on the reference's own mega-request layout.

The batch is what the reference's scheduler and runner hand the backend: one
request per beam-search session holding ``prefill tail ++ concat(beam
tokens)`` (vllm_gr/v1/engine/core.py:108-112), ``MEGA_DATA_VAR`` with the
keys engine_core_patch.py:258-271 emits (``cache_len`` = the prefix-cache
hit), vLLM's slot mapping (row k at logical position cache_len + k) and the
new tokens' K/V passed to forward, which must write them into the cache
before attending (the cache holds zeros at those slots beforehand).

The inputs follow the reference kernel test (tests/kernels/attention/
test_cascade_beam_flash_attn.py:33-65, :92-188) over its CASES x NUM_HEADS x
HEAD_SIZES x BLOCK_SIZES x soft cap grid (dtype, batch 1/4 and beam width
16/32 rotate over the grid); the expected output is the float64 restatement
of the reference's routing and cascade (oracle/metadata.py: the builder's
lists, the cached-prefix pass, the slot-mapped suffix pass, the LSE merge),
compared at the reference test's tolerance, 1e-2.  More cases cover a cache
hit below the whole prefix blocks (standard-routed prefix), a chunk budget
that cuts and skips beams, and a batch mixing standard requests with mega
ones.
"""

from __future__ import annotations

import itertools
import types

import numpy as np
import pytest
import torch

from oracle import metadata as om
from vllm_gr_amd.v1.attention.backends import beam_attn as ba

pytestmark = pytest.mark.gpu

CASES = [(8, 32, 8), (8, 8, 8), (4, 64, 4), (4, 16, 4), (1, 16, 4), (1, 128, 1), (4, 32, 7)]
NUM_HEADS = [(4, 4), (8, 2), (16, 2)]
HEAD_SIZES = [128, 256]
BLOCK_SIZES = [16, 32]
SOFTCAPS = [None, 50.0]
GRID = list(itertools.product(CASES, NUM_HEADS, HEAD_SIZES, BLOCK_SIZES, SOFTCAPS))
TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _run(inp, mega, q_starts, dtype, softcap, device, std_rows=None):
    """forward over the batch; returns (output, expected)."""
    dt = TORCH_DT[dtype]
    R = len(q_starts) - 1
    Hq, D = inp["query"].shape[1], inp["query"].shape[2]
    Hkv = inp["key_cache"].shape[2]
    bs = inp["block_size"]
    # the caches as the device will hold them (rounded), and the new rows' K/V
    kc = torch.from_numpy(inp["key_cache"]).to(dt)
    vc = torch.from_numpy(inp["value_cache"]).to(dt)
    slot = torch.from_numpy(inp["slot_mapping"])
    ok = slot >= 0
    key = torch.zeros((len(slot), Hkv, D), dtype=dt)
    val = torch.zeros((len(slot), Hkv, D), dtype=dt)
    key[ok] = kc.view(-1, Hkv, D)[slot[ok]]
    val[ok] = vc.view(-1, Hkv, D)[slot[ok]]
    kv = torch.stack([kc, vc]).to(device)
    kv.view(2, -1, Hkv, D)[:, slot[ok].to(device)] = 0  # forward must write them before attending
    q = torch.from_numpy(inp["query"]).to(dt)
    seq = torch.from_numpy(np.asarray(inp["seq_lens"], np.int32))
    qs = torch.tensor(q_starts, dtype=torch.int32)
    bt = torch.from_numpy(inp["block_tables"])
    m = ba.CommonAttentionMetadata(
        query_start_loc=qs.to(device), query_start_loc_cpu=qs, seq_lens=seq.to(device), seq_lens_cpu=seq,
        num_reqs=R, num_actual_tokens=len(slot), max_query_len=int((qs[1:] - qs[:-1]).max()),
        max_seq_len=int(seq.max()), block_table_tensor=bt.to(device), slot_mapping=slot.to(device))
    rids = [f"req_{i}" for i in range(R)]
    info = {"req_ids": rids, "mega_data": {rids[i]: dict(d) for i, d in mega.items()}}
    oracle_info = {rids[i]: dict(d) for i, d in mega.items()}
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=bs), ["l0"], None, device)
    tok = ba.MEGA_DATA_VAR.set(info)
    try:
        md = builder.build(0, m)
    finally:
        ba.MEGA_DATA_VAR.reset(tok)
    impl = ba.BeamAttentionImpl(num_heads=Hq, head_size=D, scale=inp["scale"], num_kv_heads=Hkv,
                                alibi_slopes=None, sliding_window=None, kv_cache_dtype="auto",
                                logits_soft_cap=softcap)
    out = torch.zeros((len(slot), Hq, D), dtype=dt, device=device)
    impl.forward(types.SimpleNamespace(), q.to(device), key.to(device), val.to(device), kv, md, output=out)
    torch.cuda.synchronize()
    lists = om.build(R, rids, oracle_info, q_starts, bs)
    want = om.cascade(q.to(torch.float64).numpy(), kc.to(torch.float64).numpy(), vc.to(torch.float64).numpy(),
                      inp["block_tables"], inp["seq_lens"], inp["slot_mapping"], lists, scale=inp["scale"],
                      softcap=softcap or 0.0, block_size=bs)
    return out.to(torch.float64).cpu().numpy(), want


@pytest.mark.parametrize("idx", range(len(GRID)), ids=lambda i: "-".join(map(str, GRID[i])).replace(" ", ""))
def test_forward_reference_grid(device, idx):
    (qs, kvl, sfx), (Hq, Hkv), D, bs, softcap = GRID[idx]
    dtype = ("bf16", "fp16")[idx % 2]
    batch = (1, 4)[(idx // 2) % 2]
    W = (16, 32)[(idx // 4) % 2]
    print(f"[mega-ref] case={qs, kvl, sfx} heads={Hq, Hkv} D={D} bs={bs} softcap={softcap} {dtype} "
          f"batch={batch} W={W}", flush=True)
    inp = om.prepare_inputs(batch, W, Hq, Hkv, D, qs, kvl, bs, sfx, seed=idx)
    chunk = W * qs
    mega = {i: dict(is_mega_decode=True, prefix_len=inp["shared_tokens_len"], mega_beam_width=W,
                    mega_decode_steps=sfx, cache_len=inp["cache_len"]) for i in range(batch)}
    got, want = _run(inp, mega, [i * chunk for i in range(batch + 1)], dtype, softcap, device)
    err = float(np.abs(got - want).max())
    assert err <= 1e-2, err


@pytest.mark.parametrize("P,C,W,t,rows,D", [
    (40, 0, 4, 2, 48, 128),      # 40 uncached prompt tokens: standard path, then the beams
    (40, 0, 4, 2, 30, 128),      # the budget ends inside the standard-routed prefix
    (100, 16, 8, 3, 108, 128),   # tail 84 standard-routed, beam 0 takes its 3 tokens, 7 beams decode
    (37, 32, 6, 4, 20, 128),     # budget: beam 0 (5 + 4), beams 1, 2 full, beam 3 cut at 3, 4-5 skipped
    (64, 64, 5, 2, 10, 256),     # the prompt fully cached: beam 0 has only its own tokens
])
def test_forward_reference_cache_hits_and_budgets(device, P, C, W, t, rows, D):
    print(f"[mega-ref] P={P} C={C} W={W} t={t} rows={rows} D={D}", flush=True)
    bs = 16
    inp = om.prepare_inputs(2, W, 8, 2, D, 1, P + t, bs, t, seed=P + C + rows, cache_len=C)
    # two requests of `rows` scheduled tokens each, written from position C
    R = 2
    nb = inp["block_tables"].shape[1]
    slot = np.full(R * rows, -1, np.int64)
    q = np.random.default_rng(rows).standard_normal((R * rows, 8, D)) * D ** -0.5
    for i in range(R):
        pos = C + np.arange(rows)
        keep = pos < nb * bs
        phys = inp["block_tables"][i].astype(np.int64)[pos[keep] // bs] * bs + pos[keep] % bs
        slot[i * rows:i * rows + keep.sum()] = phys
    inp = dict(inp, query=q, slot_mapping=slot)
    mega = {i: dict(is_mega_decode=True, prefix_len=P, mega_beam_width=W, mega_decode_steps=t, cache_len=C)
            for i in range(R)}
    got, want = _run(inp, mega, [0, rows, 2 * rows], "bf16", None, device)
    assert float(np.abs(got - want).max()) <= 1e-2


def test_forward_reference_mixed_with_standard(device):
    """A standard prefill chunk, a mega request and a standard decode in one
    batch (the builder's std + mega segmentation, beam_attn.py:264-290)."""
    bs, D, W, t, P = 16, 128, 8, 2, 50
    inp = om.prepare_inputs(3, W, 8, 4, D, 3, P + t, bs, t, seed=9)
    nb = inp["block_tables"].shape[1]
    C = 48
    rows = [7, P - C + W * t, 1]
    seq = [30, nb * bs, 45]
    starts = np.concatenate([[0], np.cumsum(rows)]).tolist()
    slot = np.full(starts[-1], -1, np.int64)
    for i, (n, s) in enumerate(zip(rows, seq)):
        first = C if i == 1 else s - n
        pos = first + np.arange(n)
        slot[starts[i]:starts[i + 1]] = inp["block_tables"][i].astype(np.int64)[pos // bs] * bs + pos % bs
    q = np.random.default_rng(3).standard_normal((starts[-1], 8, D)) * D ** -0.5
    inp = dict(inp, query=q, slot_mapping=slot, seq_lens=np.array(seq, np.int32))
    mega = {1: dict(is_mega_decode=True, prefix_len=P, mega_beam_width=W, mega_decode_steps=t, cache_len=C)}
    got, want = _run(inp, mega, starts, "bf16", None, device)
    assert float(np.abs(got - want).max()) <= 1e-2
