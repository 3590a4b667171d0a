"""fp8 e4m3 KV caches on the GPU (kv_cache_dtype "fp8" / "fp8_e4m3" of the
reference, vllm_gr/v1/attention/backends/beam_attn.py:617-618, :727-737).

* the quantising cache write (gr_reshape_and_cache_fp8) equals the oracle's
  e4m3(clamp(x / scale, -448, 448)) byte for byte (oracle/fp8.py, pinned
  against torch's float8_e4m3fn);
* decode and prefill over fp8 caches equal the float64 oracle over the
  dequantised caches (e4m3 * scale) within the bf16/fp16 output tolerance
  2e-2: the matrix-core kernel (bytes staged in LDS and widened to bf16 /
  fp16 tiles, K scale folded into the softmax constant, V scale into the
  output) at short and long prefixes, split and unsplit, with the decode
  options, through lean and row-by-row tile loads and the exact
  recomputation; the generic kernel on the short case;
* the fork moves fp8 bytes exactly as oracle.fork does;
* BeamAttentionImpl.forward with an fp8 cache and the layer's scales.
"""

import types

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import fork as of
from oracle import fp8
from vllm_gr_amd import ops, workloads

pytestmark = pytest.mark.gpu

BS = 16


def _codes(shape, scale, g):
    """e4m3 codes of N(0, 1) values / scale (no NaN codes)."""
    x = torch.randn(shape, generator=g).numpy().astype(np.float32)
    return torch.from_numpy(fp8.quantize(x, scale))


def _deq(codes, scale):
    return fp8.decode(codes.numpy()) * scale


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("scales", [None, (0.37, 2.5)])
@pytest.mark.parametrize("view", [torch.uint8, torch.float8_e4m3fn])
def test_reshape_and_cache_fp8_bit_exact(device, src_dtype, scales, view):
    print(f"[fp8] cache write {src_dtype} scales={scales} view={view}", flush=True)
    g = torch.Generator().manual_seed(3)
    T, Hkv, D, NB = 37, 4, 128, 12
    key = (torch.randn((T, Hkv, D), generator=g) * 40).to(src_dtype)
    value = (torch.randn((T, Hkv, D), generator=g) * 40).to(src_dtype)
    key[0, 0, :4] = torch.tensor([1e6, -1e6, 0.0, -0.0]).to(src_dtype)  # saturation and signed zero
    slots = torch.randperm(NB * BS, generator=g)[:T].to(torch.int64)
    slots[5] = -1  # skipped
    kv = torch.full((2, NB, BS, Hkv, D), 0x55, dtype=torch.uint8)
    kv_d = kv.to(device).view(view)
    ks = vs = None
    if scales:
        ks = torch.tensor([scales[0]], dtype=torch.float32, device=device)
        vs = torch.tensor([scales[1]], dtype=torch.float32, device=device)
    st = ops.new_status(device)
    ops.reshape_and_cache(key.to(device), value.to(device), kv_d[0], kv_d[1], slots.to(device), status=st,
                          k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    ops.check_status(st)
    want = kv.clone().numpy()
    sk, sv = (1.0, 1.0) if scales is None else scales
    kf, vf = key.float().numpy(), value.float().numpy()
    for t, s in enumerate(slots.tolist()):
        if s < 0:
            continue
        want[0, s // BS, s % BS] = fp8.quantize(kf[t], sk)
        want[1, s // BS, s % BS] = fp8.quantize(vf[t], sv)
    got = kv_d.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype,T", [(torch.bfloat16, 1), (torch.float16, 2), (torch.bfloat16, 3)])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.05, 0.02)])
@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_decode_fp8_cache(device, dtype, T, scales, kernel):
    print(f"[fp8] decode {dtype} T={T} scales={scales} kernel={kernel}", flush=True)
    wl = workloads.make_decode(R=3, W=5, P=140, L=(T, T + 9), Hq=8, Hkv=2, D=128, dtype=dtype,
                               input_scale=1.0, seed=11 + T, q_per_beam=T)
    g = torch.Generator().manual_seed(5 + T)
    sk, sv = scales
    kc = _codes(wl.kv_cache.shape[1:], sk, g)
    vc = _codes(wl.kv_cache.shape[1:], sv, g)
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    st = ops.new_status(device)
    ops.set_decode_kernel(kernel)
    try:
        ops.beam_attn_decode(d.q, kc.to(device), vc.to(device), d.prefix_bt, d.prefix_len, d.beam_start,
                             d.suffix_bt, d.suffix_len, q_per_beam=T, scale=d.scale, out=out, lse=lse, status=st,
                             k_scale=torch.tensor([sk], device=device), v_scale=torch.tensor([sv], device=device))
        torch.cuda.synchronize()
    finally:
        ops.set_decode_kernel("auto")
    ops.check_status(st)
    ro, rl = oa.beam_attention_dense(wl.q.to(torch.float64).numpy(), _deq(kc, sk), _deq(vc, sv),
                                     wl.prefix_bt.numpy(), wl.prefix_len.numpy(), wl.beam_start.numpy(),
                                     wl.suffix_bt.numpy(), wl.suffix_len.numpy(), q_per_beam=T, scale=wl.scale,
                                     block_size=wl.block_size)
    assert np.abs(out.cpu().double().numpy() - ro).max() <= 2e-2
    assert np.abs(lse.cpu().double().numpy() - rl).max() <= 2e-2


def _long_fp8_case(dtype, bs, seed, sk=0.05, sv=0.02):
    wl = workloads.make_decode(R=3, W=24, P=1000, L=(1, 8), Hq=16, Hkv=4, D=128, block_size=bs, dtype=dtype,
                               input_scale=1.0, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    return wl, _codes(wl.kv_cache.shape[1:], sk, g), _codes(wl.kv_cache.shape[1:], sv, g)


def _run_fp8_decode(wl, kc, vc, sk, sv, device, split, **kw):
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    st = ops.new_status(device)
    kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    ops.beam_attn_decode(d.q, kc.to(device).view(torch.float8_e4m3fn), vc.to(device).view(torch.float8_e4m3fn),
                         d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt, d.suffix_len, scale=d.scale, out=out,
                         lse=lse, status=st, split=split, max_prefix_len=int(wl.prefix_len.max()) if split else None,
                         k_scale=torch.tensor([sk], device=device), v_scale=torch.tensor([sv], device=device), **kw)
    torch.cuda.synchronize()
    ops.check_status(st)
    return out.cpu().double().numpy(), lse.cpu().double().numpy()


def _fp8_oracle(wl, kc, vc, sk, sv, **kw):
    kw = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    return oa.beam_attention_dense(wl.q.to(torch.float64).numpy(), _deq(kc, sk), _deq(vc, sv),
                                   wl.prefix_bt.numpy(), wl.prefix_len.numpy(), wl.beam_start.numpy(),
                                   wl.suffix_bt.numpy(), wl.suffix_len.numpy(), scale=wl.scale,
                                   block_size=wl.block_size, **kw)


@pytest.mark.parametrize("opts", [False, True])
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("dtype,bs", [(torch.bfloat16, 16), (torch.float16, 16), (torch.bfloat16, 4)])
def test_decode_fp8_long_prefix(device, dtype, bs, split, opts):
    """Sixteen 64-key prefix tiles per request on the matrix-core decode: the
    fp8 staging ring through the pipelined loop, with lean tile loads (block
    size 16) and row-by-row loads through the staged block table (block size
    4); with a left window, sinks and ALiBi (the option variant) or none."""
    print(f"[fp8] long decode {dtype} bs={bs} split={split} opts={opts}", flush=True)
    sk, sv = 0.05, 0.02
    wl, kc, vc = _long_fp8_case(dtype, bs, seed=61 + bs)
    kw = {}
    if opts:
        kw = dict(window=(400, -1), sinks=torch.randn(16, generator=torch.Generator().manual_seed(2)) * 3,
                  alibi_slopes=torch.tensor([2.0 ** (-8.0 * (h + 1) / 16) for h in range(16)]))
    out, lse = _run_fp8_decode(wl, kc, vc, sk, sv, device, split, **kw)
    ro, rl = _fp8_oracle(wl, kc, vc, sk, sv, **kw)
    assert np.abs(out - ro).max() <= 2e-2
    assert np.abs(lse - rl).max() <= 2e-2


@pytest.mark.parametrize("dtype,pos", [(torch.bfloat16, 200), (torch.float16, 930)])
def test_decode_fp8_dominant_key(device, dtype, pos):
    """A K row planted (in fp8) to dominate one query row far beyond the lazy
    softmax margin: the workgroup's exact recomputation stages and widens the
    fp8 tiles one at a time."""
    sk, sv = 0.05, 0.02
    wl, kc, vc = _long_fp8_case(dtype, 16, seed=71)
    n, h = int(wl.beam_start[1]) + 3, 2  # request 1's beam 3, query head 2 (KV head 0)
    q = wl.q[n, h].double()
    blk = int(wl.prefix_bt[1, pos // wl.block_size])
    kc[blk, pos % wl.block_size, 0] = torch.from_numpy(fp8.quantize((q / q.norm() * 60.0).float().numpy(), sk))
    print(f"[fp8] dominant key {dtype} pos={pos}", flush=True)
    out, lse = _run_fp8_decode(wl, kc, vc, sk, sv, device, False)
    ro, rl = _fp8_oracle(wl, kc, vc, sk, sv)
    assert rl[n, h] > 50.0
    assert np.abs(out - ro).max() <= 2e-2
    assert np.abs(lse - rl).max() <= 2e-2


@pytest.mark.parametrize("causal,qlens,ctxs,dtype", [
    (True, [1, 30, 70], [0, 20, 50], torch.bfloat16), (False, [1, 30, 70], [0, 20, 50], torch.bfloat16),
    # long causal prompts: the matrix-core prefill's pipelined fp8 loop, cached context included
    (True, [500, 260, 3], [0, 300, 900], torch.bfloat16), (True, [500, 260, 3], [0, 300, 900], torch.float16)])
def test_prefill_fp8_cache(device, causal, qlens, ctxs, dtype):
    print(f"[fp8] prefill causal={causal} qlens={qlens} {dtype}", flush=True)
    g = torch.Generator().manual_seed(8 + qlens[0])
    Hq, Hkv, D = 8, 4, 128
    seqs = [c + q for c, q in zip(ctxs, qlens)]
    nbs = [-(-s // BS) for s in seqs]
    NB = sum(nbs) + 3
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    bt = torch.full((3, max(nbs) + 1), -1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(nbs):
        bt[r, :n] = perm[o:o + n]
        o += n
    kc, vc = _codes((NB, BS, Hkv, D), 0.1, g), _codes((NB, BS, Hkv, D), 0.08, g)
    q = torch.randn((sum(qlens), Hq, D), generator=g).to(dtype)
    qs = torch.tensor([0] + qlens).cumsum(0).to(torch.int32)
    sq = torch.tensor(seqs, dtype=torch.int32)
    out = torch.empty_like(q, device=device)
    st = ops.new_status(device)
    ops.paged_attn_prefill(q.to(device), kc.to(device).view(torch.float8_e4m3fn), vc.to(device).view(torch.float8_e4m3fn),
                           bt.to(device), qs.to(device), sq.to(device), max_query_len=max(qlens), scale=D ** -0.5,
                           out=out, status=st, causal=causal, k_scale=torch.tensor([0.1], device=device),
                           v_scale=torch.tensor([0.08], device=device))
    torch.cuda.synchronize()
    ops.check_status(st)
    k64, v64 = _deq(kc, 0.1), _deq(vc, 0.08)
    q64 = q.double().numpy()
    for r in range(3):
        q0, q1 = int(qs[r]), int(qs[r + 1])
        ql, S = q1 - q0, seqs[r]
        row = bt[r:r + 1].numpy()
        ref, _ = oa.beam_attention_dense(q64[q0:q1], k64, v64, row, np.array([S - ql]), np.array([0, 1]), row,
                                         np.array([ql]), np.array([S - ql]), q_per_beam=ql, scale=D ** -0.5,
                                         block_size=BS, causal=causal)
        assert np.abs(out[q0:q1].cpu().double().numpy() - ref).max() <= 2e-2, r


def test_fork_fp8_cache_bit_exact(device):
    print("[fp8] fork", flush=True)
    g = torch.Generator().manual_seed(9)
    R, W, S, Hkv, D = 3, 16, 2, 4, 128
    N = R * W
    NB = N * S + 4
    bt = torch.randperm(NB, generator=g)[:N * S].view(N, S).to(torch.int32)
    lens = torch.randint(0, S * BS - 1, (N,), generator=g).to(torch.int32)
    parent = torch.randint(0, W, (R, W), generator=g).to(torch.int32)
    parent[0] = torch.randint(0, 3, (W,), generator=g)
    kv = torch.randint(0, 256, (2, NB, BS, Hkv, D), generator=g).to(torch.uint8)
    kn = torch.randint(0, 256, (N, Hkv, D), generator=g).to(torch.uint8)
    vn = torch.randint(0, 256, (N, Hkv, D), generator=g).to(torch.uint8)
    kv_d = kv.to(device)
    st = ops.new_status(device)
    bt_o, len_o = ops.beam_kv_fork(parent.to(device), bt.to(device), lens.to(device), kv_d[0], kv_d[1],
                                   kn.to(device), vn.to(device), status=st)
    torch.cuda.synchronize()
    ops.check_status(st)
    wb, wl_, wk, wv = of.fork_append(parent.numpy(), bt.numpy(), lens.numpy(), kv[0].numpy(), kv[1].numpy(),
                                     kn.numpy(), vn.numpy(), block_size=BS)
    assert np.array_equal(bt_o.cpu().numpy(), wb) and np.array_equal(len_o.cpu().numpy(), wl_)
    assert np.array_equal(kv_d[0].cpu().numpy(), wk) and np.array_equal(kv_d[1].cpu().numpy(), wv)


def test_backend_forward_fp8(device):
    """BeamAttentionImpl(kv_cache_dtype="fp8") writes the new tokens with the
    layer's _k_scale / _v_scale and attends over the dequantised cache."""
    from vllm_gr_amd.v1.attention.backends import beam_attn as ba
    print("[fp8] backend forward", flush=True)
    g = torch.Generator().manual_seed(10)
    Hq, Hkv, D, NB = 8, 2, 128, 16
    sk, sv = 0.07, 0.05
    kv = torch.stack([_codes((NB, BS, Hkv, D), sk, g), _codes((NB, BS, Hkv, D), sv, g)])
    bt = torch.tensor([[3, 7, 1, 0], [9, 2, 12, 5]], dtype=torch.int32)
    seq, q_lens = [40, 45], [1, 5]
    n = sum(q_lens)
    slots = torch.tensor([int(bt[r, p // BS]) * BS + p % BS for r, (S, ql) in enumerate(zip(seq, q_lens))
                          for p in range(S - ql, S)], dtype=torch.int64)
    q = torch.randn((n, Hq, D), generator=g).to(torch.bfloat16)
    k_new = torch.randn((n, Hkv, D), generator=g).to(torch.bfloat16)
    v_new = torch.randn((n, Hkv, D), generator=g).to(torch.bfloat16)
    impl = ba.BeamAttentionImpl(num_heads=Hq, head_size=D, scale=D ** -0.5, num_kv_heads=Hkv, alibi_slopes=None,
                                sliding_window=None, kv_cache_dtype="fp8")
    layer = types.SimpleNamespace(_k_scale=torch.tensor([sk], device=device), _v_scale=sv)
    qs = torch.tensor([0] + q_lens).cumsum(0).to(torch.int32)
    m = ba.CommonAttentionMetadata(
        query_start_loc=qs.to(device), query_start_loc_cpu=qs, seq_lens=torch.tensor(seq, dtype=torch.int32,
                                                                                     device=device),
        seq_lens_cpu=torch.tensor(seq, dtype=torch.int32), num_reqs=2, num_actual_tokens=n, max_query_len=5,
        max_seq_len=45, block_table_tensor=bt.to(device), slot_mapping=slots.to(device))
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=BS), ["l0"], None, device)
    md = builder.build(0, m)
    kv_d = kv.to(device)
    out = torch.empty((n, Hq, D), dtype=torch.bfloat16, device=device)
    impl.forward(layer, q.to(device), k_new.to(device), v_new.to(device), kv_d, md, output=out)
    torch.cuda.synchronize()
    ops.check_status(md.status)
    ref_kv = kv.clone()
    for t, s in enumerate(slots.tolist()):
        ref_kv[0, s // BS, s % BS] = torch.from_numpy(fp8.quantize(k_new[t].float().numpy(), sk))
        ref_kv[1, s // BS, s % BS] = torch.from_numpy(fp8.quantize(v_new[t].float().numpy(), sv))
    assert torch.equal(kv_d.cpu(), ref_kv)
    k64, v64 = _deq(ref_kv[0], sk), _deq(ref_kv[1], sv)
    row = 0
    for r, (S, ql) in enumerate(zip(seq, q_lens)):
        ref, _ = oa.beam_attention_dense(q[row:row + ql].double().numpy(), k64, v64, bt[r:r + 1].numpy(),
                                         np.array([S - ql]), np.array([0, 1]), bt[r:r + 1].numpy(), np.array([ql]),
                                         np.array([S - ql]), q_per_beam=ql, scale=D ** -0.5, block_size=BS)
        assert np.abs(out[row:row + ql].cpu().double().numpy() - ref).max() <= 2e-2, r
        row += ql
