"""Varlen causal attention of standard requests (gr_paged_attn_prefill) on
the GPU vs the float64 oracle.

Each request is checked as the oracle's one-beam case: prefix = its ctx
cached tokens, suffix = its ql new tokens at positions ctx .. ctx+ql-1 of
the same block-table row, queries bottom-right causal -- the
flash_attn_varlen_func(causal=True, block_table) call of the reference's
standard path (vllm_gr/v1/attention/backends/beam_attn.py:643-654).
Tolerances: bf16 <= 2e-2 max abs on N(0,1) inputs (outputs of order 0.1-1),
float32 <= 1e-5.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from vllm_gr_amd import ops

pytestmark = pytest.mark.gpu

BS = 16


def _case(qlens, ctxs, Hq, Hkv, D, dtype, seed, extra_blocks=3):
    g = torch.Generator().manual_seed(seed)
    seqs = [c + q for c, q in zip(ctxs, qlens)]
    nbs = [max(1, -(-s // BS)) for s in seqs]
    width = max(nbs) + extra_blocks
    NB = sum(nbs) + 7
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    bt = torch.full((len(qlens), width), -1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(nbs):
        bt[r, :n] = perm[o:o + n]
        o += n
    kv = torch.randn((2, NB, BS, Hkv, D), generator=g).to(dtype)
    NT = sum(qlens)
    q = torch.randn((NT, Hq, D), generator=g).to(dtype)
    qs = torch.tensor([0] + list(qlens)).cumsum(0).to(torch.int32)
    return q, kv, bt, qs, torch.tensor(seqs, dtype=torch.int32)


def _oracle(q, kv, bt, qs, seqs, scale, softcap=0.0):
    q64 = q.to(torch.float64).numpy()
    kv64 = kv.to(torch.float64).numpy()
    out = np.zeros(q64.shape)
    lse = np.full(q64.shape[:2], -np.inf)
    for r in range(len(seqs)):
        q0, q1 = int(qs[r]), int(qs[r + 1])
        ql, S = q1 - q0, int(seqs[r])
        if ql == 0:
            continue
        row = bt[r:r + 1].numpy()
        o, l = oa.beam_attention_dense(q64[q0:q1], kv64[0], kv64[1], row, np.array([S - ql]), np.array([0, 1]),
                                       row, np.array([ql]), np.array([S - ql]), q_per_beam=ql, scale=scale,
                                       softcap=softcap, block_size=BS)
        out[q0:q1], lse[q0:q1] = o, l
    return out, lse


def _run(device, q, kv, bt, qs, seqs, scale, softcap=0.0, kernel="auto", max_ql=None):
    print(f"[prefill] R={len(seqs)} tokens={q.shape[0]} heads={q.shape[1]}/{kv.shape[3]} D={q.shape[2]} "
          f"{q.dtype} max_ql={max_ql} kernel={kernel}", flush=True)
    kv_d = kv.to(device)
    out = torch.full_like(q, 7.0, device=device)
    lse = torch.empty(q.shape[:2], dtype=torch.float32, device=device)
    status = ops.new_status(device)
    mql = max_ql if max_ql is not None else int((qs[1:] - qs[:-1]).max())
    ops.set_decode_kernel(kernel)
    try:
        ops.paged_attn_prefill(q.to(device), kv_d[0], kv_d[1], bt.to(device), qs.to(device), seqs.to(device),
                               max_query_len=mql, scale=scale, softcap=softcap, out=out, lse=lse,
                               status=status)
        torch.cuda.synchronize()
    finally:
        ops.set_decode_kernel("auto")
    return out.cpu().to(torch.float64).numpy(), lse.cpu().to(torch.float64).numpy(), status


QLENS = [1, 5, 64, 129, 300]
CTXS = [0, 17, 100, 3, 250]


@pytest.mark.parametrize("heads", [(16, 8), (32, 8), (8, 8), (12, 4)])
def test_prefill_mfma_bf16(device, heads):
    Hq, Hkv = heads
    q, kv, bt, qs, seqs = _case(QLENS, CTXS, Hq, Hkv, 128, torch.bfloat16, seed=Hq + Hkv)
    out, lse, st = _run(device, q, kv, bt, qs, seqs, 128 ** -0.5)
    ops.check_status(st)
    ref, ref_lse = _oracle(q, kv, bt, qs, seqs, 128 ** -0.5)
    assert np.abs(out - ref).max() <= 2e-2
    assert np.abs(lse - ref_lse).max() <= 2e-2


@pytest.mark.parametrize("heads,dtype", [((16, 8), torch.bfloat16), ((8, 2), torch.float16), ((6, 6), torch.bfloat16),
                                         ((9, 3), torch.bfloat16)])
def test_prefill_head_dim_64(device, heads, dtype):
    """head_dim 64: an even KV head count runs on the matrix-core kernel as
    pairs of adjacent KV heads read as 128-dim heads (each query row's half
    of Q zero in the other half, only its own half written); an odd count
    takes the generic kernel.  Against the float64 oracle, and the generic
    kernel's output."""
    Hq, Hkv = heads
    q, kv, bt, qs, seqs = _case(QLENS, CTXS, Hq, Hkv, 64, dtype, seed=Hq * 3 + Hkv)
    out, lse, st = _run(device, q, kv, bt, qs, seqs, 64 ** -0.5)
    ops.check_status(st)
    ref, ref_lse = _oracle(q, kv, bt, qs, seqs, 64 ** -0.5)
    assert np.abs(out - ref).max() <= 2e-2
    assert np.abs(lse - ref_lse).max() <= 2e-2
    gen, _, st = _run(device, q, kv, bt, qs, seqs, 64 ** -0.5, kernel="generic")
    ops.check_status(st)
    assert np.abs(out - gen).max() <= 2e-2


def test_prefill_long_prompt_one_request(device):
    """The 2048-token prompt of the end-to-end decode (16 query / 8 KV heads)."""
    q, kv, bt, qs, seqs = _case([2048], [0], 16, 8, 128, torch.bfloat16, seed=11)
    out, lse, st = _run(device, q, kv, bt, qs, seqs, 128 ** -0.5)
    ops.check_status(st)
    ref, _ = _oracle(q, kv, bt, qs, seqs, 128 ** -0.5)
    assert np.abs(out - ref).max() <= 2e-2


@pytest.mark.parametrize("D,dtype,tol", [(128, torch.bfloat16, 2e-2), (64, torch.float32, 1e-5),
                                         (256, torch.float16, 2e-2)])
def test_prefill_generic(device, D, dtype, tol):
    q, kv, bt, qs, seqs = _case(QLENS, CTXS, 8, 2, D, dtype, seed=D)
    out, lse, st = _run(device, q, kv, bt, qs, seqs, D ** -0.5, kernel="generic")
    ops.check_status(st)
    ref, ref_lse = _oracle(q, kv, bt, qs, seqs, D ** -0.5)
    assert np.abs(out - ref).max() <= tol
    assert np.abs(lse - ref_lse).max() <= max(tol, 1e-5)


@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_prefill_softcap_empty_request_and_loose_bound(device, kernel):
    """Soft cap, a request with no queries between others, and a
    max_query_len above every request's count (the grid's extra tiles exit)."""
    qlens, ctxs = [40, 0, 77], [9, 30, 0]
    q, kv, bt, qs, seqs = _case(qlens, ctxs, 16, 4, 128, torch.bfloat16, seed=5)
    out, lse, st = _run(device, q, kv, bt, qs, seqs, 128 ** -0.5, softcap=20.0, kernel=kernel, max_ql=300)
    ops.check_status(st)
    ref, _ = _oracle(q, kv, bt, qs, seqs, 128 ** -0.5, softcap=20.0)
    assert np.abs(out - ref).max() <= 2e-2


@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_prefill_flags_inconsistent_request(device, kernel):
    """A request whose sequence is shorter than its queries is flagged and
    skipped (its rows untouched); the others are still exact."""
    qlens, ctxs = [20, 30, 10], [5, 0, 40]
    q, kv, bt, qs, seqs = _case(qlens, ctxs, 16, 8, 128, torch.bfloat16, seed=6)
    bad = seqs.clone()
    bad[1] = 12  # 30 queries, 12 keys
    out, lse, st = _run(device, q, kv, bt, qs, bad, 128 ** -0.5, kernel=kernel)
    assert int(st.item()) & 2  # GR_DEV_BAD_LENGTH
    ref, _ = _oracle(q, kv, bt, qs, seqs, 128 ** -0.5)
    for r in (0, 2):
        q0, q1 = int(qs[r]), int(qs[r + 1])
        assert np.abs(out[q0:q1] - ref[q0:q1]).max() <= 2e-2
    assert np.all(out[int(qs[1]):int(qs[2])] == 7.0)


@pytest.mark.parametrize("pos,dtype", [(20, torch.bfloat16), (300, torch.bfloat16), (700, torch.bfloat16),
                                       (1010, torch.bfloat16), (1030, torch.bfloat16), (300, torch.float16)])
def test_prefill_dominant_key(device, pos, dtype):
    """A key planted to dominate one query row far beyond the lazy rescale
    margin: in the first tile, in the pipelined tiles (the workgroup's exact
    recomputation; 1010 is in the last of them for that row's workgroup) and
    on the causal edge (1030, one of the request's own new tokens), and in
    fp16, whose P operand bounds the lazy-rescale margin at 2^15: every row
    matches the oracle, the planted row's LSE included."""
    ctx, ql = 1000, 64
    q, kv, bt, qs, seqs = _case([ql], [ctx], 16, 4, 128, dtype, seed=23)
    qi, h = 40, 5  # query token 40 (sees keys 0 .. ctx + 40), query head 5 (KV head 1)
    qv = q[qi, h].float()
    blk = int(bt[0, pos // BS])
    kv[0, blk, pos % BS, h // 4] = (qv / qv.norm() * 60.0).to(dtype)
    out, lse, status = _run(device, q, kv, bt, qs, seqs, 128 ** -0.5)
    ops.check_status(status)
    ref, ref_lse = _oracle(q, kv, bt, qs, seqs, 128 ** -0.5)
    assert ref_lse[qi, h] > 50.0
    assert np.abs(out - ref).max() <= 2e-2
    assert np.abs(lse - ref_lse).max() <= 2e-2
