"""BeamAttention decode on the GPU vs the float64 oracle.

Tolerances: float32 path <= 1e-5 max abs error vs the
float64 oracle; bf16/fp16 <= 2e-2 max abs error.  Because N(0,1)/sqrt(128)
inputs make every output tiny (|o| ~ 1e-2), bf16 cases are also checked
relative to the output scale (<= 2e-2 * max|ref|) and on unscaled N(0,1)
inputs where |o| ~ 0.1-1 and 2e-2 is a real bound.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from vllm_gr_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _host(t):
    return t.detach().cpu().to(torch.float64).numpy()


def run_gpu(wl, device, kernel="auto", split=True, max_prefix_len=None):
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty((d.q.shape[0], d.q.shape[1]), dtype=torch.float32, device=device)
    status = ops.new_status(device)
    ops.set_decode_kernel(kernel)
    try:
        ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start,
                             d.suffix_bt, d.suffix_len, q_per_beam=d.q_per_beam, scale=d.scale,
                             softcap=d.softcap, max_beams_per_req=d.max_beams, out=out, lse=lse,
                             status=status, split=split, max_prefix_len=max_prefix_len)
        torch.cuda.synchronize()
    finally:
        ops.set_decode_kernel("auto")
    ops.check_status(status)
    return _host(out), lse.cpu().numpy().astype(np.float64)


def run_oracle(wl):
    kv = wl.kv_cache.to(torch.float64).numpy()
    return oa.beam_attention_cascade(
        _host(wl.q), kv[0], kv[1], wl.prefix_bt.numpy(), wl.prefix_len.numpy(), wl.beam_start.numpy(),
        wl.suffix_bt.numpy(), wl.suffix_len.numpy(), q_per_beam=wl.q_per_beam, scale=wl.scale,
        softcap=wl.softcap, block_size=wl.block_size)


def _check(out, lse, ref, ref_lse, atol, rel=None):
    err = np.abs(out - ref).max()
    assert err <= atol, f"max abs err {err:.3e} > {atol}"
    if rel is not None:
        scale = np.abs(ref).max()
        assert err <= rel * scale, f"max abs err {err:.3e} > {rel} * max|ref| ({scale:.3e})"
    fin = np.isfinite(ref_lse)
    assert (np.isfinite(lse) == fin).all(), "LSE finiteness differs"
    lerr = np.abs(lse[fin] - ref_lse[fin]).max() if fin.any() else 0.0
    assert lerr <= max(atol, 1e-4), f"LSE err {lerr:.3e}"


def test_decode_small_fp32(device):
    """1 req x 32 beams, P=512, L=4, 16/4 heads, fp32: <= 1e-5 vs float64."""
    wl = workloads.decode_small_fp32(seed=0)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_decode_unscaled_tail_tile(device, dtype, kernel):
    """Prefix not a multiple of the 64-key tile, ragged suffixes, N(0,1) inputs."""
    wl = workloads.make_decode(R=2, W=16, P=300, L=(1, 8), Hq=32, Hkv=8, D=128, dtype=dtype,
                               input_scale=1.0, seed=1)
    out, lse = run_gpu(wl, device, kernel)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


@pytest.mark.parametrize("heads", [(4, 4), (8, 2), (16, 2), (32, 8)])
@pytest.mark.parametrize("T", [1, 3])
def test_decode_gqa_and_multi_query(device, heads, T):
    """Reference grid heads (test_cascade_beam_flash_attn.py:33) and q_per_beam > 1
    (bottom-right causal suffix)."""
    Hq, Hkv = heads
    wl = workloads.make_decode(R=3, W=8, P=200, L=(T, T + 5), Hq=Hq, Hkv=Hkv, D=128,
                               dtype=torch.bfloat16, input_scale=1.0, seed=2 + T, q_per_beam=T)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


@pytest.mark.parametrize("D", [64, 256])
def test_decode_other_head_dims_generic(device, D):
    """head_size 64 and 256 (reference HEAD_SIZES include 256) run the generic kernel."""
    wl = workloads.make_decode(R=2, W=4, P=100, L=(1, 6), Hq=8, Hkv=2, D=D, dtype=torch.bfloat16,
                               input_scale=1.0, seed=7)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


def test_decode_softcap(device):
    wl = workloads.make_decode(R=2, W=8, P=130, L=(2, 6), Hq=16, Hkv=4, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=9, softcap=50.0)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


def test_decode_block32(device):
    wl = workloads.make_decode(R=2, W=8, P=100, L=(1, 20), Hq=16, Hkv=4, D=128, block_size=32,
                               dtype=torch.bfloat16, input_scale=1.0, seed=11)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


@pytest.mark.parametrize("P,L", [(0, 5), (64, 0), (0, 0)])
def test_decode_empty_sides(device, P, L):
    """No shared prefix (reference case (8, 8, 8)), no suffix, and nothing at all."""
    wl = workloads.make_decode(R=2, W=8, P=P, L=L, Hq=16, Hkv=4, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=13)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)
    if P == 0 and L == 0:
        assert (out == 0).all() and np.isneginf(lse).all()


def test_decode_beam128_full(device):
    """8 requests x 128 beams x 2048 prefix, bf16, Q/K/V ~ N(0,1)/sqrt(128)."""
    wl = workloads.decode_beam128(seed=0)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2, rel=2e-2)


def test_decode_beam128_unscaled(device):
    """Same shape with N(0,1) inputs: peaked softmax, so a key/row mix-up cannot hide
    behind near-uniform attention weights."""
    wl = workloads.make_decode(R=8, W=128, P=2048, L=(1, 8), Hq=32, Hkv=8, D=128,
                               dtype=torch.bfloat16, input_scale=1.0, seed=1)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


def test_decode_mfma_matches_generic(device):
    wl = workloads.make_decode(R=4, W=64, P=1000, L=(1, 8), Hq=32, Hkv=8, D=128,
                               dtype=torch.bfloat16, input_scale=1.0, seed=21)
    a, la = run_gpu(wl, device, "auto")
    b, lb = run_gpu(wl, device, "generic")
    assert np.abs(a - b).max() <= 2e-2
    assert np.abs(la - lb).max() <= 1e-3


def test_decode_uneven_beams_per_request(device):
    """Requests with different beam counts in one launch (beam_start ragged)."""
    wl = workloads.make_decode(R=3, W=40, P=150, L=(1, 4), Hq=16, Hkv=4, D=128,
                               dtype=torch.bfloat16, input_scale=1.0, seed=23)
    wl.beam_start = torch.tensor([0, 40, 47, 120], dtype=torch.int32)
    wl.max_beams = 73
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


def test_decode_deterministic(device):
    wl = workloads.make_decode(R=2, W=32, P=500, L=(1, 8), Hq=32, Hkv=8, D=128,
                               dtype=torch.bfloat16, seed=5)
    a, _ = run_gpu(wl, device)
    b, _ = run_gpu(wl, device)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("kernel", ["auto", "generic"])
@pytest.mark.parametrize("P", [64, 700])
def test_decode_bad_block_flagged(device, kernel, P):
    """An out-of-range prefix block id is reported and never dereferenced.
    The matrix-core kernel reads its keys as zero rows (its output equals the
    oracle's over a cache whose block there is all zeros, in a one-tile range
    and in a pipelined one); the generic kernel leaves them out of the
    softmax (finite output).  Either way the request's status is an error."""
    wl = workloads.make_decode(R=1, W=4, P=P, L=2, Hq=8, Hkv=2, D=128, dtype=torch.bfloat16, seed=3,
                               input_scale=1.0)
    nb = wl.kv_cache.shape[1]
    wl.prefix_bt[0, 1] = nb + 7
    with pytest.raises(ValueError, match="block id out of range"):
        run_gpu(wl, device, kernel=kernel)
    d = wl.to(device)
    out = torch.empty_like(d.q)
    status = ops.new_status(device)
    ops.set_decode_kernel(kernel)
    try:
        ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt,
                             d.suffix_len, scale=d.scale, max_beams_per_req=d.max_beams, out=out, status=status)
        torch.cuda.synchronize()
    finally:
        ops.set_decode_kernel("auto")
    assert int(status.item()) & ops._C.GR_DEV_BAD_BLOCK
    got = _host(out)
    assert np.isfinite(got).all()
    if kernel != "generic":
        zero = wl.kv_cache.new_zeros((2, 1) + tuple(wl.kv_cache.shape[2:]))
        wl.kv_cache = torch.cat([wl.kv_cache, zero], dim=1)  # block nb: all zeros
        wl.prefix_bt[0, 1] = nb
        ref, _ = run_oracle(wl)
        err = np.abs(got - ref).max()
        assert err <= 2e-2, f"max abs err {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Hq,Hkv,T,split", [(32, 8, 1, False), (8, 2, 2, True), (4, 4, 1, True), (16, 2, 1, False),
                                            (6, 3, 1, False)])
def test_decode_head_dim_64(device, dtype, Hq, Hkv, T, split):
    """head_dim 64: an even KV head count runs on the matrix-core kernel as
    pairs of adjacent KV heads read as 128-dim heads (each query row's Q fills
    its own head's half, only that half of its output is written; never
    split); an odd count (6/3) takes the generic kernel.  Against the float64
    oracle, and the generic kernel's output."""
    wl = workloads.make_decode(R=2, W=16, P=300, L=(T, T + 5), Hq=Hq, Hkv=Hkv, D=64, dtype=dtype, input_scale=1.0,
                               seed=Hq + Hkv + T, q_per_beam=T)
    out, lse = run_gpu(wl, device, split=split, max_prefix_len=300 if split else None)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, 2e-2)
    gen, _ = run_gpu(wl, device, kernel="generic")
    assert np.abs(out - gen).max() <= 2e-2


@pytest.mark.parametrize("opt", ["window", "sinks_alibi"])
def test_decode_head_dim_64_options(device, opt):
    """head_dim 64 head pairs with the option variant: a left window, or
    sinks and ALiBi (indexed by the real query head)."""
    wl = workloads.make_decode(R=2, W=8, P=400, L=(1, 6), Hq=16, Hkv=4, D=64, dtype=torch.bfloat16,
                               input_scale=1.0, seed=5)
    g = torch.Generator().manual_seed(7)
    kw = dict(window=(90, -1)) if opt == "window" else dict(sinks=torch.randn(16, generator=g),
                                                              alibi_slopes=torch.rand(16, generator=g) * 0.05)
    d = wl.to(device)
    out = torch.empty_like(d.q)
    lse = torch.empty(d.q.shape[:2], dtype=torch.float32, device=device)
    status = ops.new_status(device)
    ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt,
                         d.suffix_len, scale=d.scale, max_beams_per_req=d.max_beams, out=out, lse=lse,
                         status=status, **{k_: (v_.to(device) if isinstance(v_, torch.Tensor) else v_)
                                           for k_, v_ in kw.items()})
    torch.cuda.synchronize()
    ops.check_status(status)
    kv = wl.kv_cache.to(torch.float64).numpy()
    ref, ref_lse = oa.beam_attention_dense(_host(wl.q), kv[0], kv[1], wl.prefix_bt.numpy(), wl.prefix_len.numpy(),
                                           wl.beam_start.numpy(), wl.suffix_bt.numpy(), wl.suffix_len.numpy(),
                                           scale=wl.scale, block_size=wl.block_size,
                                           **{k_: (v_.numpy() if isinstance(v_, torch.Tensor) else v_)
                                              for k_, v_ in kw.items()})
    _check(_host(out), lse.cpu().numpy().astype(np.float64), ref, ref_lse, 2e-2)


@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_decode_understated_max_beams_flagged(device, kernel):
    """A request with more beams than max_beams_per_req says would leave rows
    that no workgroup computes: the request is reported instead."""
    wl = workloads.make_decode(R=2, W=6, P=100, L=2, Hq=8, Hkv=2, D=128, dtype=torch.bfloat16, seed=4,
                               input_scale=1.0)
    d = wl.to(device)
    out = torch.zeros_like(d.q)
    status = ops.new_status(device)
    ops.set_decode_kernel(kernel)
    try:
        ops.beam_attn_decode(d.q, d.k_cache, d.v_cache, d.prefix_bt, d.prefix_len, d.beam_start, d.suffix_bt,
                             d.suffix_len, scale=d.scale, max_beams_per_req=d.max_beams - 1, out=out,
                             status=status, split=False)
        torch.cuda.synchronize()
    finally:
        ops.set_decode_kernel("auto")
    assert int(status.item()) & ops._C.GR_DEV_BAD_LENGTH


def test_decode_late_dominant_key(device):
    """A key far above every earlier score of its row, late in the prefix (its
    weight relative to the running reference exceeds 2^60), must move the
    softmax reference and rescale the accumulated output."""
    wl = workloads.make_decode(R=1, W=4, P=1000, L=3, Hq=8, Hkv=2, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=29)
    q = wl.q[1, 0].float()
    pos = 900
    blk = int(wl.prefix_bt[0, pos // wl.block_size])
    wl.kv_cache[0, blk, pos % wl.block_size, 0] = (q / q.norm() * 100.0).to(torch.bfloat16)
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    assert ref_lse[1, 0] > 60.0  # the planted key dominates that row by far
    _check(out, lse, ref, ref_lse, atol=2e-2)


def test_decode_prefix_beyond_staged_window(device):
    """A prefix longer than the 2048 block ids the matrix-core kernel stages in
    LDS (33,000 tokens at block size 16): the staged window moves mid-prefix."""
    wl = workloads.make_decode(R=1, W=2, P=33000, L=(1, 8), Hq=8, Hkv=2, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=31, pool_factor=1.0)
    assert wl.prefix_bt.shape[1] > 2048
    out, lse = run_gpu(wl, device)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2, rel=5e-2)


@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_decode_long_suffix(device, kernel):
    """Suffixes spanning several blocks (37 and 60 tokens at block size 16):
    block ids past the ones staged per beam are read from the table."""
    wl = workloads.make_decode(R=2, W=8, P=200, L=[37, 60], Hq=16, Hkv=4, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=37)
    assert wl.suffix_bt.shape[1] == 4
    out, lse = run_gpu(wl, device, kernel)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)


@pytest.mark.parametrize("R,W,P,hint,dtype,softcap", [
    (1, 128, 2048, 2048, torch.bfloat16, 0.0),   # one request x 128 beams: 8 splits of 4 tiles
    (1, 128, 2048, 0, torch.bfloat16, 0.0),      # no hint: 8 splits
    (2, 32, 1000, 1000, torch.float16, 0.0),     # splits of uneven tile counts
    (1, 16, 100, 0, torch.bfloat16, 0.0),        # 16 splits over 2 tiles: most splits empty
    (3, 8, 300, 0, torch.bfloat16, 30.0),        # soft cap, 11 splits over 5 tiles
])
def test_decode_split_prefix(device, R, W, P, hint, dtype, softcap):
    """Small batches spread each row tile's prefix over several workgroups and
    merge the partials by LSE in a second kernel: same result as the oracle
    and as the unsplit kernel; a repeated call is bit-identical."""
    from vllm_gr_amd import _C
    assert _C.lib().gr_beam_attn_decode_workspace_size(R, W, 1, 32, 8, 128, hint) > 0
    wl = workloads.make_decode(R=R, W=W, P=P, L=(1, 8), Hq=32, Hkv=8, D=128, dtype=dtype, input_scale=1.0,
                               seed=R * 7 + W, softcap=softcap)
    print(f"[decode] split R={R} W={W} P={P} hint={hint} {dtype} softcap={softcap}", flush=True)
    out, lse = run_gpu(wl, device, split=True, max_prefix_len=hint)
    ref, ref_lse = run_oracle(wl)
    _check(out, lse, ref, ref_lse, atol=2e-2)
    whole, whole_lse = run_gpu(wl, device, split=False)
    assert np.abs(out - whole).max() <= 1e-2 and np.abs(lse - whole_lse).max() <= 1e-4
    again, again_lse = run_gpu(wl, device, split=True, max_prefix_len=hint)
    assert np.array_equal(out, again) and np.array_equal(lse, again_lse)


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("pos", [5, 70, 200, 470, 520])
def test_decode_dominant_key(device, split, pos):
    """One prefix key planted to dominate one row by far more than the
    kernels' lazy-rescale margin, in the first tile, the pipelined tiles, the
    second-to-last and the last tile (P = 530: nine 64-key tiles), with and
    without the split prefix: the exact path gives the oracle's result for
    every row."""
    wl = workloads.make_decode(R=2, W=32, P=530, L=(1, 6), Hq=32, Hkv=8, D=128, dtype=torch.bfloat16,
                               input_scale=1.0, seed=41)
    r, b, h = 1, 3, 2  # request 1's beam 3, query head 2 (KV head 0)
    n = int(wl.beam_start[r]) + b
    q = wl.q[n, h].float()
    blk = int(wl.prefix_bt[r, pos // wl.block_size])
    wl.kv_cache[0, blk, pos % wl.block_size, 0] = (q / q.norm() * 60.0).to(torch.bfloat16)
    print(f"[decode] dominant key pos={pos} split={split}", flush=True)
    out, lse = run_gpu(wl, device, split=split, max_prefix_len=530 if split else None)
    ref, ref_lse = run_oracle(wl)
    assert ref_lse[n, h] > 50.0
    _check(out, lse, ref, ref_lse, atol=2e-2)


@pytest.mark.parametrize("dtype,softcap", [(torch.float16, 0.0), (torch.bfloat16, 30.0), (torch.float16, 30.0)])
def test_decode_dominant_key_fp16_softcap(device, dtype, softcap):
    """The exact recomputation in the fp16 and soft-capped instantiations: a
    key in a pipelined tile dominates one row (with a soft cap of 30 the
    score range is still 2 * 30 * log2(e) ~ 86 log2 units, above the 60 of
    the lazy-rescale margin)."""
    wl = workloads.make_decode(R=2, W=32, P=530, L=(1, 6), Hq=32, Hkv=8, D=128, dtype=dtype,
                               input_scale=1.0, seed=43, softcap=softcap)
    r, b, h = 0, 7, 1
    n = int(wl.beam_start[r]) + b
    q = wl.q[n, h].float()
    pos = 200
    blk = int(wl.prefix_bt[r, pos // wl.block_size])
    wl.kv_cache[0, blk, pos % wl.block_size, 0] = (q / q.norm() * 60.0).to(dtype)
    print(f"[decode] dominant key {dtype} softcap={softcap}", flush=True)
    out, lse = run_gpu(wl, device, split=False)
    ref, ref_lse = run_oracle(wl)
    assert ref_lse[n, h] > (25.0 if softcap else 50.0)
    _check(out, lse, ref, ref_lse, atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kernel,split", [("auto", False), ("auto", True), ("generic", False)])
def test_decode_large_scores(device, dtype, kernel, split):
    """Q/K/V ~ N(0, 16): scores spread over tens of log2 units, so many rows
    leave the lazy softmax reference in the prefix loop, the last tiles and
    the suffix.  Outputs are compared relative to their scale (V ~ N(0, 16));
    no inf or NaN anywhere."""
    wl = workloads.make_decode(R=2, W=16, P=700, L=(1, 8), Hq=32, Hkv=8, D=128, dtype=dtype, input_scale=4.0,
                               seed=47)
    print(f"[decode] large scores {dtype} kernel={kernel} split={split}", flush=True)
    out, lse = run_gpu(wl, device, kernel, split=split, max_prefix_len=700 if split else None)
    ref, ref_lse = run_oracle(wl)
    assert np.isfinite(out).all()
    _check(out, lse, ref, ref_lse, atol=0.2, rel=2e-2)
