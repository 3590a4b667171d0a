"""Seeded random-shape sweeps of every kernel against the oracles, all through
the C ABI: shapes the hand-picked tests do not reach (odd GQA ratios, block
size 32, empty prefixes and suffixes, two query tokens per beam, the split
decode on and off, ragged prefill batches, fork tables of several blocks,
wide prune rows), and decodes over random dtypes, fp8 caches and attention
options.  Tolerances as elsewhere: bf16 attention <= 2e-2 on N(0,1)
inputs, fork and prune bit for bit."""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import fork as of
from oracle import fp8
from oracle import prune as op
from vllm_gr_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _pick(rng, xs):
    return xs[int(rng.integers(0, len(xs)))]


@pytest.mark.parametrize("seed", range(12))
def test_random_decode(device, seed):
    rng = np.random.default_rng(1000 + seed)
    Hkv = _pick(rng, [1, 2, 4, 8])
    G = _pick(rng, [1, 2, 3, 4, 8])
    R = int(rng.integers(1, 4))
    W = int(rng.integers(1, 40))
    P = int(_pick(rng, [0, 17, 64, 300, 1000]))
    T = _pick(rng, [1, 1, 2])
    L = (T, T + int(rng.integers(0, 12)))
    bs = _pick(rng, [16, 32])
    cap = float(_pick(rng, [0.0, 0.0, 30.0]))
    split = bool(rng.integers(0, 2))
    wl = workloads.make_decode(R=R, W=W, P=P, L=L, Hq=Hkv * G, Hkv=Hkv, D=128, block_size=bs,
                               dtype=torch.bfloat16, input_scale=1.0, seed=seed, q_per_beam=T, softcap=cap)
    print(f"[random] decode R={R} W={W} P={P} T={T} L={L} Hkv={Hkv} G={G} bs={bs} cap={cap} split={split}",
          flush=True)
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    status = ops.new_status(device)
    ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt,
                         d.suffix_len, q_per_beam=T, scale=d.scale, softcap=cap, max_beams_per_req=d.max_beams,
                         out=out, lse=lse, status=status, split=split, max_prefix_len=P)
    torch.cuda.synchronize()
    ops.check_status(status)
    kv = wl.kv_cache.to(torch.float64).numpy()
    ref, ref_lse = oa.beam_attention_cascade(
        wl.q.to(torch.float64).numpy(), kv[0], kv[1], wl.prefix_bt.numpy(), wl.prefix_len.numpy(),
        wl.beam_start.numpy(), wl.suffix_bt.numpy(), wl.suffix_len.numpy(), q_per_beam=T, scale=wl.scale,
        softcap=cap, block_size=bs)
    got = out.cpu().to(torch.float64).numpy()
    assert np.abs(got - ref).max() <= 2e-2
    fin = np.isfinite(ref_lse)
    assert (np.isfinite(lse.cpu().numpy()) == fin).all()
    assert np.abs(lse.cpu().numpy()[fin] - ref_lse[fin]).max(initial=0.0) <= 2e-2


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_variants(device, seed):
    """Random decodes over the space the shape sweep above keeps fixed: bf16
    and fp16, head dim 128 or 64 (head pairs on the matrix-core kernel for an
    even KV head count, the generic kernel for an odd one), fp8 e4m3 caches
    with random scales, a left window, sinks and ALiBi in any combination,
    soft cap, split or not -- against the dense float64 oracle with the same
    options (within 2e-2, LSE finiteness equal)."""
    rng = np.random.default_rng(7000 + seed)
    Hkv = _pick(rng, [1, 2, 4, 8])
    G = _pick(rng, [1, 2, 4, 8])
    Hq = Hkv * G
    R = int(rng.integers(1, 4))
    W = int(rng.integers(1, 33))
    P = int(_pick(rng, [0, 33, 64, 300, 1000]))
    T = _pick(rng, [1, 1, 2])
    L = (T, T + int(rng.integers(0, 12)))
    bs = _pick(rng, [16, 32])
    dtype = _pick(rng, [torch.bfloat16, torch.float16])
    kv8 = bool(rng.integers(0, 3) == 0)
    cap = float(_pick(rng, [0.0, 0.0, 0.0, 30.0]))
    split = bool(rng.integers(0, 2))
    D = int(_pick(rng, [128, 128, 64]))
    g = torch.Generator().manual_seed(seed)
    kw = {}
    if rng.integers(0, 2):
        kw["window"] = (int(_pick(rng, [2, 40, 70, 300, 999])), -1)
    if rng.integers(0, 2):
        kw["sinks"] = torch.randn(Hq, generator=g) * 2
    if rng.integers(0, 2):
        kw["alibi_slopes"] = torch.rand(Hq, generator=g) * 0.05
    print(f"[random] decode variant R={R} W={W} P={P} T={T} L={L} Hkv={Hkv} G={G} D={D} bs={bs} {dtype} kv8={kv8} "
          f"cap={cap} split={split} options={sorted(kw)} window={kw.get('window')}", flush=True)
    wl = workloads.make_decode(R=R, W=W, P=P, L=L, Hq=Hq, Hkv=Hkv, D=D, block_size=bs, dtype=dtype,
                               input_scale=1.0, seed=seed, q_per_beam=T, softcap=cap)
    d = wl.to(device)
    if kv8:
        sk, sv = 0.05 * (1 + rng.random()), 0.02 * (1 + rng.random())
        codes = [torch.from_numpy(fp8.quantize(torch.randn(wl.kv_cache.shape[1:], generator=g).numpy()
                                               .astype(np.float32), s_)) for s_ in (sk, sv)]
        kd, vd = (c.to(device).view(torch.float8_e4m3fn) for c in codes)
        extra = dict(k_scale=torch.tensor([sk], device=device), v_scale=torch.tensor([sv], device=device))
        k64, v64 = fp8.decode(codes[0].numpy()) * sk, fp8.decode(codes[1].numpy()) * sv
    else:
        kd, vd, extra = d.k_cache, d.v_cache, {}
        kv = wl.kv_cache.to(torch.float64).numpy()
        k64, v64 = kv[0], kv[1]
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    status = ops.new_status(device)
    gkw = {k_: (v_.to(device) if isinstance(v_, torch.Tensor) else v_) for k_, v_ in kw.items()}
    ops.beam_attn_decode(d.q, kd, vd, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt, d.suffix_len,
                         q_per_beam=T, scale=d.scale, softcap=cap, max_beams_per_req=d.max_beams, out=out, lse=lse,
                         status=status, split=split, max_prefix_len=P if split else None, **gkw, **extra)
    torch.cuda.synchronize()
    ops.check_status(status)
    okw = {k_: (v_.numpy() if isinstance(v_, torch.Tensor) else v_) for k_, v_ in kw.items()}
    ref, ref_lse = oa.beam_attention_dense(wl.q.to(torch.float64).numpy(), k64, v64, wl.prefix_bt.numpy(),
                                           wl.prefix_len.numpy(), wl.beam_start.numpy(), wl.suffix_bt.numpy(),
                                           wl.suffix_len.numpy(), q_per_beam=T, scale=wl.scale, softcap=cap,
                                           block_size=bs, **okw)
    got, got_lse = out.cpu().double().numpy(), lse.cpu().double().numpy()
    assert np.abs(got - ref).max() <= 2e-2
    fin = np.isfinite(ref_lse)
    assert (np.isfinite(got_lse) == fin).all()
    assert np.abs(got_lse[fin] - ref_lse[fin]).max(initial=0.0) <= 2e-2


@pytest.mark.parametrize("seed", range(8))
def test_random_prefill(device, seed):
    rng = np.random.default_rng(2000 + seed)
    Hkv = _pick(rng, [1, 2, 8])
    G = _pick(rng, [1, 2, 4])
    R = int(rng.integers(1, 6))
    qlens = [int(_pick(rng, [0, 1, 7, 64, 65, 200])) for _ in range(R)]
    ctxs = [int(_pick(rng, [0, 5, 128, 333])) for _ in range(R)]
    if sum(qlens) == 0:
        qlens[0] = 3
    g = torch.Generator().manual_seed(seed)
    BS = 16
    seqs = [c + q for c, q in zip(ctxs, qlens)]
    nbs = [max(1, -(-s // BS)) for s in seqs]
    NB = sum(nbs) + 3
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    bt = torch.full((R, max(nbs) + 1), -1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(nbs):
        bt[r, :n] = perm[o:o + n]
        o += n
    kv = torch.randn((2, NB, BS, Hkv, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((sum(qlens), Hkv * G, 128), generator=g).to(torch.bfloat16)
    qs = torch.tensor([0] + qlens).cumsum(0).to(torch.int32)
    print(f"[random] prefill R={R} qlens={qlens} ctxs={ctxs} Hkv={Hkv} G={G}", flush=True)
    kvd = kv.to(device)
    out = torch.empty_like(q, device=device)
    status = ops.new_status(device)
    ops.paged_attn_prefill(q.to(device), kvd[0], kvd[1], bt.to(device), qs.to(device),
                           torch.tensor(seqs, dtype=torch.int32).to(device), max_query_len=max(qlens),
                           scale=128 ** -0.5, out=out, status=status)
    torch.cuda.synchronize()
    ops.check_status(status)
    kv64 = kv.to(torch.float64).numpy()
    q64 = q.to(torch.float64).numpy()
    got = out.cpu().to(torch.float64).numpy()
    for r in range(R):
        q0, q1 = int(qs[r]), int(qs[r + 1])
        if q1 == q0:
            continue
        row = bt[r:r + 1].numpy()
        ref, _ = oa.beam_attention_dense(q64[q0:q1], kv64[0], kv64[1], row, np.array([ctxs[r]]), np.array([0, 1]),
                                         row, np.array([qlens[r]]), np.array([ctxs[r]]), q_per_beam=qlens[r],
                                         scale=128 ** -0.5, block_size=BS)
        assert np.abs(got[q0:q1] - ref).max() <= 2e-2, r


@pytest.mark.parametrize("seed", range(8))
def test_random_fork(device, seed):
    rng = np.random.default_rng(3000 + seed)
    R = int(rng.integers(1, 5))
    W = int(_pick(rng, [1, 3, 16, 64, 128, 200]))
    S = int(_pick(rng, [1, 2, 5]))
    lo = int(rng.integers(0, 16 * S))
    L_old = (lo, int(rng.integers(lo, 16 * S)))
    Hkv = _pick(rng, [1, 2, 8])
    print(f"[random] fork R={R} W={W} S={S} L_old={L_old} Hkv={Hkv}", flush=True)
    fw = workloads.make_fork(R=R, W=W, Hkv=Hkv, D=128, S=S, L_old=L_old, seed=seed)
    fd = fw.to(device)
    status = ops.new_status(device)
    append = bool(rng.integers(0, 2)) and L_old[1] < 16 * S
    bt, ln = ops.beam_kv_fork(fd.parent, fd.suffix_bt, fd.suffix_len, fd.kv_cache[0], fd.kv_cache[1],
                              fd.k_new if append else None, fd.v_new if append else None, status=status)
    torch.cuda.synchronize()
    ops.check_status(status)
    bits = lambda t: t.cpu().contiguous().view(torch.int16).numpy()
    want = of.fork_append(fw.parent.numpy(), fw.suffix_bt.numpy(), fw.suffix_len.numpy(), bits(fw.kv_cache[0]),
                          bits(fw.kv_cache[1]), bits(fw.k_new) if append else None,
                          bits(fw.v_new) if append else None, block_size=fw.block_size)
    assert np.array_equal(bt.cpu().numpy(), want[0]) and np.array_equal(ln.cpu().numpy(), want[1])
    assert np.array_equal(bits(fd.kv_cache[0]), want[2]) and np.array_equal(bits(fd.kv_cache[1]), want[3])


@pytest.mark.parametrize("seed", range(8))
def test_random_prune(device, seed):
    rng = np.random.default_rng(4000 + seed)
    R = int(rng.integers(1, 5))
    W = int(_pick(rng, [1, 4, 32, 128]))
    V = int(_pick(rng, [64, 1000, 8192, 12000]))
    k = int(min(V, _pick(rng, [1, 8, W, 200])))
    eos = int(_pick(rng, [-1, 0, V - 1]))
    print(f"[random] prune R={R} W={W} V={V} k={k} eos={eos}", flush=True)
    pw = workloads.make_prune(R=R, W=W, V=V, k=k, seed=seed)
    pd = pw.to(device)
    parent, token, score, eos_score = ops.beam_prune_topk(pd.logits, pd.cum, k, eos)
    torch.cuda.synchronize()
    want = op.prune_topk(pw.logits.numpy(), pw.cum.numpy(), k, eos)
    assert np.array_equal(parent.cpu().numpy(), want["parent"])
    assert np.array_equal(token.cpu().numpy(), want["token"])
    assert np.array_equal(score.cpu().numpy().view(np.int32), want["score"].view(np.int32))
    assert np.array_equal(eos_score.cpu().numpy().view(np.int32), want["eos_score"].reshape(R, W).view(np.int32))
