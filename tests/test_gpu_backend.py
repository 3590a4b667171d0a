"""The backend mirror end to end on the GPU: BeamAttentionImpl.forward over a
builder-made batch (mega-decode requests with resident beam suffixes,
standard decode and prefill requests) against the float64 oracle, and a
multi-step beam search (decode -> prune -> fork) whose resident suffix KV must
equal, bit for bit, each surviving beam's lineage (the reference's content
rule: child = parent suffix ++ chosen token, serving_engine.py:113-120)."""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from oracle import attention as oa
from vllm_gr_amd.entrypoints import beam_search as bsm
from vllm_gr_amd.v1.attention.backends import beam_attn as ba
from vllm_gr_amd.v1.beam_kv import BeamKVTable

pytestmark = pytest.mark.gpu

BS = 16


def _impl(Hq, Hkv, D):
    return ba.BeamAttentionImpl(num_heads=Hq, head_size=D, scale=D ** -0.5, num_kv_heads=Hkv,
                                alibi_slopes=None, sliding_window=None, kv_cache_dtype="auto")


def _common(q_lens, seq_lens, bt, dev, slots=None):
    qs = torch.tensor([0] + list(q_lens)).cumsum(0).to(torch.int32)
    n = int(qs[-1])
    if slots is None:
        slots = torch.full((n,), -1, dtype=torch.int64)
    return ba.CommonAttentionMetadata(
        query_start_loc=qs.to(dev), query_start_loc_cpu=qs, seq_lens=torch.tensor(seq_lens, dtype=torch.int32,
                                                                                 device=dev),
        seq_lens_cpu=torch.tensor(seq_lens, dtype=torch.int32), num_reqs=len(q_lens), num_actual_tokens=n,
        max_query_len=max(q_lens), max_seq_len=max(seq_lens), block_table_tensor=bt.to(dev),
        slot_mapping=slots.to(dev))


def _build(builder, md_info, common):
    tok = ba.MEGA_DATA_VAR.set(md_info)
    try:
        return builder.build(0, common)
    finally:
        ba.MEGA_DATA_VAR.reset(tok)


def test_forward_mega_decode(device):
    g = torch.Generator().manual_seed(0)
    R, W, P, Hq, Hkv, D = 2, 8, 100, 16, 4, 128
    N = R * W
    pb = (P + BS - 1) // BS
    NB = R * pb + N + 4
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    kv = torch.randn((2, NB, BS, Hkv, D), generator=g).to(torch.bfloat16)
    prefix_bt = perm[:R * pb].reshape(R, pb)
    suffix_bt = perm[R * pb:R * pb + N].reshape(N, 1)
    L = torch.randint(0, 11, (N,), generator=g).to(torch.int32)
    q = torch.randn((N, Hq, D), generator=g).to(torch.bfloat16)
    k_new = torch.randn((N, Hkv, D), generator=g).to(torch.bfloat16)
    v_new = torch.randn((N, Hkv, D), generator=g).to(torch.bfloat16)

    kv_d = kv.to(device)
    tables = [BeamKVTable(prefix_bt[r:r + 1].to(device), torch.tensor([P]), W, suffix_bt[r * W:(r + 1) * W].to(device),
                          L[r * W:(r + 1) * W].to(device), block_size=BS) for r in range(R)]
    info = {"req_ids": ["r0", "r1"], "mega_data": {
        f"r{r}": dict(is_mega_decode=True, mega_beam_width=W, mega_decode_steps=3, prefix_len=P, cache_len=P,
                      beam_kv=tables[r]) for r in range(R)}}
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=BS), ["l0"], None, device)
    md = _build(builder, info, _common([W] * R, [P + 1] * R, torch.zeros(R, 1, dtype=torch.int32), device))
    out = torch.empty_like(q, device=device)
    _impl(Hq, Hkv, D).forward(None, q.to(device), k_new.to(device), v_new.to(device), kv_d, md, output=out)
    torch.cuda.synchronize()

    # expected cache: the new token at suffix position L of each beam
    kv_ref = kv.clone()
    for n in range(N):
        blk, off = int(suffix_bt[n, 0]), int(L[n])
        kv_ref[0, blk, off] = k_new[n]
        kv_ref[1, blk, off] = v_new[n]
    bits = lambda t: t.cpu().contiguous().view(torch.int16)
    assert torch.equal(bits(kv_d), bits(kv_ref))
    kv64 = kv_ref.to(torch.float64).numpy()
    ref, _ = oa.beam_attention_cascade(q.to(torch.float64).numpy(), kv64[0], kv64[1], prefix_bt.numpy(),
                                       np.full(R, P), np.arange(0, N + 1, W), suffix_bt.numpy(),
                                       (L + 1).numpy(), scale=D ** -0.5, block_size=BS)
    err = np.abs(out.cpu().to(torch.float64).numpy() - ref).max()
    assert err <= 2e-2, err


def test_forward_standard_requests(device):
    """A decode request and a 5-token prefill chunk (no beams) through the same kernel."""
    g = torch.Generator().manual_seed(1)
    Hq, Hkv, D = 8, 2, 128
    NB = 16
    kv = torch.randn((2, NB, BS, Hkv, D), generator=g).to(torch.bfloat16)
    bt = torch.tensor([[3, 7, 1, 0], [9, 2, 12, 5]], dtype=torch.int32)
    seq = [40, 45]  # request 0 decodes its 40th token, request 1 prefills tokens 40..44
    q_lens = [1, 5]
    n = sum(q_lens)
    q = torch.randn((n, Hq, D), generator=g).to(torch.bfloat16)
    k_new = torch.randn((n, Hkv, D), generator=g).to(torch.bfloat16)
    v_new = torch.randn((n, Hkv, D), generator=g).to(torch.bfloat16)
    slots = []
    for r, (S, ql) in enumerate(zip(seq, q_lens)):
        for pos in range(S - ql, S):
            slots.append(int(bt[r, pos // BS]) * BS + pos % BS)
    slots = torch.tensor(slots, dtype=torch.int64)
    kv_d = kv.to(device)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=BS), ["l0"], None, device)
    md = _build(builder, None, _common(q_lens, seq, bt, device, slots))
    out = torch.empty((n, Hq, D), dtype=torch.bfloat16, device=device)
    _impl(Hq, Hkv, D).forward(None, q.to(device), k_new.to(device), v_new.to(device), kv_d, md, output=out)
    torch.cuda.synchronize()
    kv_ref = kv.clone()
    for t, s in enumerate(slots.tolist()):
        kv_ref[0, s // BS, s % BS] = k_new[t]
        kv_ref[1, s // BS, s % BS] = v_new[t]
    kv64 = kv_ref.to(torch.float64).numpy()
    q64 = q.to(torch.float64).numpy()
    row = 0
    for r, (S, ql) in enumerate(zip(seq, q_lens)):
        # one beam: prefix = cached tokens, suffix = the new tokens (bottom-right causal)
        ref, _ = oa.beam_attention_dense(q64[row:row + ql], kv64[0], kv64[1], bt[r:r + 1].numpy(),
                                         np.array([S - ql]), np.array([0, 1]), bt[r:r + 1].numpy(),
                                         np.array([ql]), np.array([S - ql]), q_per_beam=ql, scale=D ** -0.5,
                                         block_size=BS)
        err = np.abs(out[row:row + ql].cpu().to(torch.float64).numpy() - ref).max()
        assert err <= 2e-2, (r, err)
        row += ql


def test_beam_search_loop_keeps_lineage(device):
    """Five decode -> prune -> fork steps: each surviving beam's resident suffix
    K/V is exactly the K/V its ancestors appended, in order."""
    g = torch.Generator().manual_seed(2)
    W, P, Hq, Hkv, D, V = 8, 64, 8, 2, 128, 64
    steps = 5
    pb = P // BS
    NB = pb + W + 3
    kv = torch.zeros((2, NB, BS, Hkv, D), dtype=torch.bfloat16)
    kv[:, :pb] = torch.randn((2, pb, BS, Hkv, D), generator=g).to(torch.bfloat16)
    kv_d = kv.to(device)
    table = BeamKVTable(torch.arange(pb, dtype=torch.int32)[None].to(device), torch.tensor([P]), W,
                        torch.arange(pb, pb + W, dtype=torch.int32)[:, None].to(device), block_size=BS)
    impl = _impl(Hq, Hkv, D)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=BS), ["l0"], None, device)
    hist_k = [[] for _ in range(W)]
    hist_v = [[] for _ in range(W)]
    cum = torch.zeros((1, W), dtype=torch.float32, device=device)
    for step in range(steps):
        q = torch.randn((W, Hq, D), generator=g).to(torch.bfloat16)
        k_new = torch.randn((W, Hkv, D), generator=g).to(torch.bfloat16)
        v_new = torch.randn((W, Hkv, D), generator=g).to(torch.bfloat16)
        info = {"req_ids": ["r"], "mega_data": {"r": dict(is_mega_decode=True, mega_beam_width=W,
                                                          mega_decode_steps=step + 1, prefix_len=P, cache_len=P,
                                                          beam_kv=table)}}
        md = _build(builder, info, _common([W], [P + step + 1], torch.zeros(1, 1, dtype=torch.int32), device))
        out = torch.empty((W, Hq, D), dtype=torch.bfloat16, device=device)
        impl.forward(None, q.to(device), k_new.to(device), v_new.to(device), kv_d, md, output=out)
        table.advance()
        for n in range(W):
            hist_k[n].append(k_new[n])
            hist_v[n].append(v_new[n])
        logits = (torch.randn((1, W, V), generator=g) * 3).to(device)
        res = bsm.beam_search_step(table, logits, cum, [kv_d])
        cum = res.score.contiguous()
        parent = res.parent.cpu()[0].tolist()
        hist_k = [list(hist_k[p]) for p in parent]
        hist_v = [list(hist_v[p]) for p in parent]
    torch.cuda.synchronize()
    assert table.suffix_len.cpu().tolist() == [steps] * W
    kvh = kv_d.cpu()
    sbt = table.suffix_bt.cpu()
    for n in range(W):
        for j in range(steps):
            blk = int(sbt[n, j // BS])
            assert torch.equal(kvh[0, blk, j % BS].view(torch.int16), hist_k[n][j].view(torch.int16))
            assert torch.equal(kvh[1, blk, j % BS].view(torch.int16), hist_v[n][j].view(torch.int16))
    # every beam owns distinct blocks
    assert len(set(sbt[:, 0].tolist())) == W


def test_forward_reports_bad_block_through_metadata_status(device):
    """The builder's status word reaches every launch of the forward: a block
    id past the cache in a request's table leaves the result finite (the
    kernels read that block as zeros) and is reported by ops.check_status;
    a clean batch leaves the word at zero."""
    from vllm_gr_amd import ops
    g = torch.Generator().manual_seed(2)
    Hq, Hkv, D = 8, 2, 128
    NB = 16
    kv = torch.randn((2, NB, BS, Hkv, D), generator=g).to(torch.bfloat16).to(device)
    bt = torch.tensor([[3, 7, 1, 0], [9, 2, 12, 5]], dtype=torch.int32)
    seq, q_lens = [40, 45], [1, 5]
    n = sum(q_lens)
    slots = torch.tensor([int(bt[r, p // BS]) * BS + p % BS for r, (S, ql) in enumerate(zip(seq, q_lens))
                          for p in range(S - ql, S)], dtype=torch.int64)
    q = torch.randn((n, Hq, D), generator=g).to(torch.bfloat16).to(device)
    k_new = torch.randn((n, Hkv, D), generator=g).to(torch.bfloat16).to(device)
    v_new = torch.randn((n, Hkv, D), generator=g).to(torch.bfloat16).to(device)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=BS), ["l0"], None, device)
    out = torch.empty((n, Hq, D), dtype=torch.bfloat16, device=device)
    md = _build(builder, None, _common(q_lens, seq, bt, device, slots))
    assert md.status is builder.status
    _impl(Hq, Hkv, D).forward(None, q, k_new, v_new, kv, md, output=out)
    ops.check_status(md.status)  # clean batch: no bits
    bad = bt.clone()
    bad[0, 1] = NB + 5  # request 0's cached positions 16..31 (no new token is written there)
    md = _build(builder, None, _common(q_lens, seq, bad, device, slots))
    _impl(Hq, Hkv, D).forward(None, q, k_new, v_new, kv, md, output=out)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    with pytest.raises(ValueError, match="block id out of range"):
        ops.check_status(md.status)
    builder.status.zero_()
