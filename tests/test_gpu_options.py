"""The optional attention features (gr_attn_options: sliding window, sinks,
ALiBi, non-causal prefill) on the GPU vs the float64 oracle.

The reference hands window_size / causal / alibi_slopes / s_aux to every
flash_attn_varlen_func call of its cascade and standard path
(vllm_gr/v1/attention/backends/beam_attn.py:597-625, :643-695); the oracle
(oracle.attention.beam_attention_dense) states them per key position and is
pinned in tests/test_oracle_options.py.  Decode runs gr_beam_attn_decode_opt,
prefill gr_paged_attn_prefill_opt (windows and sinks of bf16/fp16 head-dim-128
decodes, and sinks of such prefills, on the matrix-core kernel; the rest on
the generic kernel).
Tolerances: float32 1e-5, bf16/fp16 2e-2 on N(0,1) inputs.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from vllm_gr_amd import ops, workloads

pytestmark = pytest.mark.gpu

BS = 16


def _decode_case(dtype, D, T, seed):
    return workloads.make_decode(R=2, W=6, P=150, L=(T, T + 9), Hq=8, Hkv=2, D=D, dtype=dtype,
                                 input_scale=1.0, seed=seed, q_per_beam=T)


def _decode_gpu(wl, device, **kw):
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    st = ops.new_status(device)
    ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt,
                         d.suffix_len, q_per_beam=d.q_per_beam, scale=d.scale, softcap=d.softcap,
                         out=out, lse=lse, status=st, **kw)
    torch.cuda.synchronize()
    ops.check_status(st)
    return out.cpu().to(torch.float64).numpy(), lse.cpu().to(torch.float64).numpy()


def _decode_oracle(wl, **kw):
    kv = wl.kv_cache.to(torch.float64).numpy()
    return oa.beam_attention_dense(wl.q.to(torch.float64).numpy(), kv[0], kv[1], wl.prefix_bt.numpy(),
                                   wl.prefix_len.numpy(), wl.beam_start.numpy(), wl.suffix_bt.numpy(),
                                   wl.suffix_len.numpy(), q_per_beam=wl.q_per_beam, scale=wl.scale,
                                   softcap=wl.softcap, block_size=wl.block_size, **kw)


def _close(got, want, atol):
    (o, l), (ro, rl) = got, want
    assert np.abs(o - ro).max() <= atol, np.abs(o - ro).max()
    fin = np.isfinite(rl)
    assert (np.isfinite(l) == fin).all()
    assert np.abs(l[fin] - rl[fin]).max() <= max(atol, 1e-4)


FEATURES = {
    "window": lambda Hq, g: dict(window=(40, -1)),
    "window_tiny": lambda Hq, g: dict(window=(2, -1)),
    "sinks": lambda Hq, g: dict(sinks=torch.randn(Hq, generator=g) * 2),
    "alibi": lambda Hq, g: dict(alibi_slopes=torch.rand(Hq, generator=g) * 0.1),
    "all": lambda Hq, g: dict(window=(60, -1), sinks=torch.randn(Hq, generator=g),
                              alibi_slopes=torch.rand(Hq, generator=g) * 0.05),
}


def _split(kw, device):
    gpu = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    orc = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    return gpu, orc


@pytest.mark.parametrize("feature", list(FEATURES))
@pytest.mark.parametrize("dtype,D,T", [(torch.bfloat16, 128, 1), (torch.float16, 128, 3),
                                       (torch.float32, 64, 2), (torch.bfloat16, 256, 1)])
def test_decode_options(device, feature, dtype, D, T):
    print(f"[options] decode {feature} {dtype} D={D} T={T}", flush=True)
    wl = _decode_case(dtype, D, T, seed=D + T)
    kw = FEATURES[feature](8, torch.Generator().manual_seed(T))
    gpu_kw, orc_kw = _split(kw, device)
    _close(_decode_gpu(wl, device, **gpu_kw), _decode_oracle(wl, **orc_kw),
           1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("kw", [dict(window=(300, -1)), dict(window=(999, -1)), dict(window=(3, -1)),
                                dict(window=(70, -1)), dict(sinks=True), dict(window=(250, -1), sinks=True),
                                dict(alibi=True), dict(window=(400, -1), alibi=True, sinks=True)])
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_options_long_prefix(device, kw, split, dtype):
    """Windows, sinks and ALiBi on the matrix-core decode at a long prefix (many
    pipelined tiles, the window's edge tiles masked, the rest on the fast
    loop; split and unsplit): suffix lengths differ between requests, so the
    window edge falls at different keys per row."""
    print(f"[options] long decode {kw} split={split} {dtype}", flush=True)
    wl = workloads.make_decode(R=3, W=24, P=1000, L=(1, 8), Hq=16, Hkv=4, D=128, dtype=dtype,
                               input_scale=1.0, seed=77)
    kw = dict(kw)
    if kw.get("sinks"):
        kw["sinks"] = torch.randn(16, generator=torch.Generator().manual_seed(5)) * 3
    if kw.pop("alibi", False):  # the usual geometric slopes 2^(-8 h / H), h = 1 .. 16
        kw["alibi_slopes"] = torch.tensor([2.0 ** (-8.0 * (h + 1) / 16) for h in range(16)])
    gpu_kw, orc_kw = _split(kw, device)
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    st = ops.new_status(device)
    ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt,
                         d.suffix_len, scale=d.scale, out=out, lse=lse, status=st, split=split,
                         max_prefix_len=1000 if split else None, **gpu_kw)
    torch.cuda.synchronize()
    ops.check_status(st)
    got = (out.cpu().to(torch.float64).numpy(), lse.cpu().to(torch.float64).numpy())
    _close(got, _decode_oracle(wl, **orc_kw), 2e-2)


def test_decode_window_with_softcap(device):
    wl = workloads.make_decode(R=2, W=4, P=90, L=(1, 5), Hq=8, Hkv=2, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=9, softcap=7.0)
    _close(_decode_gpu(wl, device, window=(30, -1)), _decode_oracle(wl, window=(30, -1)), 2e-2)


def test_decode_rejects_non_causal(device):
    wl = _decode_case(torch.bfloat16, 128, 1, seed=1).to(device)
    with pytest.raises(ValueError, match="invalid argument"):
        ops._C.check("gr_beam_attn_decode_opt", _raw_decode_opt(wl, device, causal=0))


def _raw_decode_opt(d, device, causal):
    opt = ops._C.AttnOptions(-1, -1, causal, None, None)
    out = torch.empty_like(d.q)
    import ctypes
    return ops._C.lib().gr_beam_attn_decode_opt(
        out.data_ptr(), out.stride(0), d.q.data_ptr(), d.q.stride(0), d.k_cache.data_ptr(), d.v_cache.data_ptr(),
        d.k_cache.shape[0], *ops._cache_strides(d.k_cache, d.v_cache), d.prefix_bt.data_ptr(),
        d.prefix_bt.shape[1], d.prefix_len.data_ptr(), d.beam_start.data_ptr(), d.suffix_bt.data_ptr(),
        d.suffix_bt.shape[1], d.suffix_len.data_ptr(), None, d.prefix_len.numel(), 6, d.suffix_len.numel(),
        d.q_per_beam, 8, 2, 128, BS, ops._dtype_code(d.q), float(d.scale), 0.0, None, None, 0, None, 0,
        ctypes.byref(opt), ops._stream(device))


def _prefill_case(qlens, ctxs, Hq, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    seqs = [c + q for c, q in zip(ctxs, qlens)]
    nbs = [max(1, -(-s // BS)) for s in seqs]
    width = max(nbs) + 2
    NB = sum(nbs) + 5
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    bt = torch.full((len(qlens), width), -1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(nbs):
        bt[r, :n] = perm[o:o + n]
        o += n
    kv = torch.randn((2, NB, BS, Hkv, D), generator=g).to(dtype)
    q = torch.randn((sum(qlens), Hq, D), generator=g).to(dtype)
    qs = torch.tensor([0] + list(qlens)).cumsum(0).to(torch.int32)
    return q, kv, bt, qs, torch.tensor(seqs, dtype=torch.int32), g


def _prefill_oracle(q, kv, bt, qs, seqs, scale, **kw):
    q64, kv64 = q.to(torch.float64).numpy(), kv.to(torch.float64).numpy()
    out, lse = np.zeros(q64.shape), np.full(q64.shape[:2], -np.inf)
    for r in range(len(seqs)):
        q0, q1 = int(qs[r]), int(qs[r + 1])
        ql, S = q1 - q0, int(seqs[r])
        if ql == 0:
            continue
        row = bt[r:r + 1].numpy()
        out[q0:q1], lse[q0:q1] = oa.beam_attention_dense(
            q64[q0:q1], kv64[0], kv64[1], row, np.array([S - ql]), np.array([0, 1]), row, np.array([ql]),
            np.array([S - ql]), q_per_beam=ql, scale=scale, block_size=BS, **kw)
    return out, lse


@pytest.mark.parametrize("causal,window", [(True, (50, -1)), (False, (-1, -1)), (False, (30, 30)),
                                           (False, (20, 0)), (True, (-1, -1))])
@pytest.mark.parametrize("extras", [False, True, "sinks"])
def test_prefill_options(device, causal, window, extras):
    """extras: sinks and ALiBi, or sinks alone (a causal prefill with sinks
    alone runs on the matrix-core kernel)."""
    print(f"[options] prefill causal={causal} window={window} extras={extras}", flush=True)
    q, kv, bt, qs, seqs, g = _prefill_case([1, 37, 120], [0, 25, 64], 8, 4, 128, torch.bfloat16,
                                           seed=int(causal) + window[0] + 3 * bool(extras))
    kw = dict(window=window)
    if extras == "sinks":
        kw.update(sinks=torch.randn(8, generator=g) * 2)
    elif extras:
        kw.update(sinks=torch.randn(8, generator=g), alibi_slopes=torch.rand(8, generator=g) * 0.05)
    gpu_kw, orc_kw = _split(kw, device)
    kv_d = kv.to(device)
    out = torch.empty_like(q, device=device)
    lse = torch.empty(q.shape[:2], dtype=torch.float32, device=device)
    st = ops.new_status(device)
    ops.paged_attn_prefill(q.to(device), kv_d[0], kv_d[1], bt.to(device), qs.to(device), seqs.to(device),
                           max_query_len=120, scale=128 ** -0.5, out=out, lse=lse, status=st, causal=causal,
                           **gpu_kw)
    torch.cuda.synchronize()
    ops.check_status(st)
    want = _prefill_oracle(q, kv, bt, qs, seqs, 128 ** -0.5, causal=causal, **orc_kw)
    _close((out.cpu().to(torch.float64).numpy(), lse.cpu().to(torch.float64).numpy()), want, 2e-2)


@pytest.mark.parametrize("attn_type", ["encoder_only", "decoder"])
def test_backend_forward_with_options(device, attn_type):
    """BeamAttentionImpl.forward with the reference's constructor arguments
    (sliding_window, alibi_slopes, running_sinks; beam_attn.py:579-627) on a
    standard batch; ENCODER_ONLY metadata is non-causal with a two-sided
    window (w-1, w-1), the decoder one causal with (w-1, 0)."""
    import types
    from vllm_gr_amd.v1.attention.backends import beam_attn as ba
    print(f"[options] backend forward {attn_type}", flush=True)
    Hq, Hkv, D, w = 8, 4, 128, 24
    qlens, ctxs = [9, 40, 1], [0, 30, 55]
    q, kv, bt, qs, seqs, g = _prefill_case(qlens, ctxs, Hq, Hkv, D, torch.bfloat16, seed=21)
    sinks = torch.randn(Hq, generator=g)
    slopes = (torch.rand(Hq, generator=g) * 0.05).tolist()
    causal = attn_type == "decoder"
    impl = ba.BeamAttentionImpl(num_heads=Hq, head_size=D, scale=D ** -0.5, num_kv_heads=Hkv,
                                alibi_slopes=slopes, sliding_window=w, kv_cache_dtype="auto",
                                attn_type=ba.AttentionType(attn_type), running_sinks=sinks.to(device))
    NT = q.shape[0]
    slot = torch.full((NT,), -1, dtype=torch.int64)  # the cache already holds every token
    m = ba.CommonAttentionMetadata(
        query_start_loc=qs.to(device), query_start_loc_cpu=qs, seq_lens=seqs.to(device), seq_lens_cpu=seqs,
        num_reqs=len(qlens), num_actual_tokens=NT, max_query_len=max(qlens), max_seq_len=int(seqs.max()),
        block_table_tensor=bt.to(device), slot_mapping=slot.to(device), causal=causal)
    builder = ba.BeamAttentionMetadataBuilder(types.SimpleNamespace(block_size=BS), ["l0"], None, device)
    tok = ba.MEGA_DATA_VAR.set({"req_ids": [f"r{i}" for i in range(len(qlens))], "mega_data": {}})
    try:
        md = builder.build(0, m)
    finally:
        ba.MEGA_DATA_VAR.reset(tok)
    out = torch.zeros((NT, Hq, D), dtype=torch.bfloat16, device=device)
    impl.forward(types.SimpleNamespace(), q.to(device), None, None, kv.to(device), md, output=out)
    torch.cuda.synchronize()
    want, _ = _prefill_oracle(q, kv, bt, qs, seqs, D ** -0.5, causal=causal,
                              window=(w - 1, -1 if causal else w - 1), sinks=sinks.numpy(),
                              alibi_slopes=np.array(slopes))
    assert np.abs(out.cpu().to(torch.float64).numpy() - want).max() <= 2e-2
