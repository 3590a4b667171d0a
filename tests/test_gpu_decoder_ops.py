"""Fused decoder stages (include/gr_decoder.h) on the GPU vs float64.

* gr_rms_norm: the written-back residual equals torch's rounded x + residual
  bit for bit; the output is within one rounding of the float64 norm
  (bf16 <= 2^-8 relative to the row scale, float32 <= 1e-6);
* gr_qk_norm_rope_cache: rotated queries and cached keys against the float64
  per-head RMSNorm + rotate-half rotation of the oracle (oracle/sid_beam.py),
  values copied bit for bit, untouched slots unchanged, skipped tokens
  (slot -1) write nothing, an out-of-table position is flagged;
* gr_silu_mul against float64 silu(g) * u.
"""

import math

import numpy as np
import pytest
import torch

from oracle import sid_beam as so
from vllm_gr_amd import ops
from vllm_gr_amd.v1.sid_decoder import RotaryEmbedding

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -10, torch.float32: 1e-6}


def _rel_err(got, ref):
    got = got.double().cpu()
    scale = ref.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    return float(((got - ref).abs() / scale).max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("H", [2048, 100, 1000, 5000])  # 1, 1 partial, 4 partial vectors per thread
@pytest.mark.parametrize("with_res", [False, True])
def test_rms_norm(device, dtype, H, with_res):
    g = torch.Generator().manual_seed(H + with_res)
    T = 37
    # x as a strided view (rows of a wider buffer) to cover the row-stride path
    xbuf = torch.randn(T, H + 16, generator=g).to(dtype)
    x = xbuf[:, :H]
    r = torch.randn(T, H, generator=g).to(dtype) if with_res else None
    w = (torch.rand(H, generator=g) + 0.5).to(dtype)
    xd, wd = xbuf.to(device)[:, :H], w.to(device)
    rd = r.to(device) if with_res else None
    print(f"[ops] rms_norm {dtype} H={H} residual={with_res}", flush=True)
    out = ops.rms_norm(xd, wd, 1e-6, residual=rd)
    torch.cuda.synchronize()
    y = (x.float() + r.float()).to(dtype) if with_res else x
    if with_res:
        assert torch.equal(rd.cpu(), y)
    yd = y.double()
    ref = yd * torch.rsqrt(yd.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert _rel_err(out, ref) <= TOL[dtype] * 1.01


@pytest.mark.parametrize("dtype,D,heads,T", [(torch.bfloat16, 128, (16, 8), 53), (torch.float32, 32, (4, 2), 53),
                                             (torch.float16, 256, (4, 4), 53), (torch.bfloat16, 64, (6, 2), 53),
                                             (torch.bfloat16, 40, (3, 1), 53),  # 40: the scalar form
                                             # four tokens per workgroup, a partial last group
                                             (torch.bfloat16, 128, (16, 8), 2051), (torch.float32, 64, (4, 1), 1025)])
def test_qk_norm_rope_cache(device, dtype, D, heads, T):
    Hq, Hkv = heads
    g = torch.Generator().manual_seed(D + Hq)
    BS, maxpos = 16, 40000
    NB = T // BS + 9
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g).to(dtype)
    qn = (torch.rand(D, generator=g) + 0.5).to(dtype)
    kn = (torch.rand(D, generator=g) + 0.5).to(dtype)
    pos = torch.randint(0, maxpos, (T,), generator=g)
    pos[:3] = torch.tensor([0, 1, maxpos - 1])
    slots = torch.randperm(NB * BS, generator=g)[:T].to(torch.int64)
    slots[5] = -1  # skipped token
    kv0 = torch.randn(2, NB, BS, Hkv, D, generator=g).to(dtype)
    rope = RotaryEmbedding(D, 1.0e6, maxpos, device)
    kv = kv0.to(device)
    status = ops.new_status(device)
    print(f"[ops] qk_norm_rope_cache {dtype} D={D} heads={heads} T={T}", flush=True)
    q = ops.qk_norm_rope_cache(qkv.to(device), pos.to(device), rope.cos, rope.sin, qn.to(device), kn.to(device),
                               kv[0], kv[1], slots.to(device), num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                               eps=1e-6, status=status)
    torch.cuda.synchronize()
    ops.check_status(status)
    # float64 reference
    x = qkv.double()
    half = D // 2
    inv = 1.0 / (1.0e6 ** (torch.arange(half, dtype=torch.float64) * 2.0 / D))
    ang = pos.double()[:, None] * inv[None]
    qr = so._rope(so._rms(x[:, :Hq * D].view(T, Hq, D), qn.double(), 1e-6), ang.cos(), ang.sin())
    kr = so._rope(so._rms(x[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D), kn.double(), 1e-6), ang.cos(), ang.sin())
    v = qkv[:, (Hq + Hkv) * D:].view(T, Hkv, D)
    # the rotary tables are float32: their rounding adds ~1e-7 relative
    tol = TOL[dtype] * 1.01 + 1e-6
    assert _rel_err(q, qr) <= tol
    kvh = kv.cpu()
    want = kv0.clone()
    for t in range(T):
        s = int(slots[t])
        if s < 0:
            continue
        blk, off = divmod(s, BS)
        assert _rel_err(kvh[0, blk, off], kr[t]) <= tol
        want[0, blk, off] = kvh[0, blk, off]
        want[1, blk, off] = v[t]
    assert torch.equal(kvh, want)  # values exact, nothing else touched


def test_qk_norm_rope_flags_position_beyond_table(device):
    D, Hq, Hkv, T = 32, 2, 1, 4
    rope = RotaryEmbedding(D, 1.0e6, 16, device)
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, device=device)
    pos = torch.tensor([0, 3, 16, 2], device=device)
    status = ops.new_status(device)
    kv = torch.zeros(2, 2, 16, Hkv, D, device=device)
    out = torch.full((T, Hq, D), 5.0, device=device)
    ops.qk_norm_rope_cache(qkv, pos, rope.cos, rope.sin, None, None, kv[0], kv[1],
                           torch.tensor([0, 1, 2, 3], device=device), num_q_heads=Hq, num_kv_heads=Hkv,
                           head_dim=D, eps=1e-6, q_out=out, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & 2
    assert torch.all(out[2] == 5.0) and torch.all(kv[:, 0, 2] == 0)
    assert not torch.all(out[1] == 5.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("F", [6144, 10])
def test_silu_mul(device, dtype, F):
    g = torch.Generator().manual_seed(F)
    x = (3 * torch.randn(29, 2 * F, generator=g)).to(dtype)
    print(f"[ops] silu_mul {dtype} F={F}", flush=True)
    out = ops.silu_mul(x.to(device))
    torch.cuda.synchronize()
    xd = x.double()
    gte, up = xd[:, :F], xd[:, F:]
    ref = gte / (1 + torch.exp(-gte)) * up
    err = (out.double().cpu() - ref).abs() / ref.abs().clamp_min(1e-3)
    assert float(err.max()) <= (2.0 ** -8 if dtype == torch.bfloat16 else 1e-5)
