"""Beam KV fork/append on the GPU vs the CPU oracle: bit-exact tables and cache."""

import numpy as np
import pytest
import torch

from oracle import fork as of
from vllm_gr_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _bits(t):
    """Raw bit pattern of a cache tensor (bit-exact comparisons)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy()
    return t.view(torch.int32).numpy()


def run_fork(wl, device, append=True):
    d = wl.to(device)
    status = ops.new_status(device)
    kc, vc = d.kv_cache[0], d.kv_cache[1]
    bt, ln = ops.beam_kv_fork(d.parent, d.suffix_bt, d.suffix_len, kc, vc,
                              d.k_new if append else None, d.v_new if append else None, status=status)
    torch.cuda.synchronize()
    ops.check_status(status)
    return bt.cpu().numpy(), ln.cpu().numpy(), _bits(d.kv_cache[0]), _bits(d.kv_cache[1])


def run_oracle(wl, append=True):
    kc, vc = _bits(wl.kv_cache[0]), _bits(wl.kv_cache[1])
    kn = _bits(wl.k_new) if append else None
    vn = _bits(wl.v_new) if append else None
    return of.fork_append(wl.parent.numpy(), wl.suffix_bt.numpy(), wl.suffix_len.numpy(), kc, vc, kn, vn,
                          block_size=wl.block_size)


def _assert_same(got, want):
    for g, w, name in zip(got, want, ("block table", "lengths", "K cache", "V cache")):
        assert np.array_equal(g, w), f"{name} differs"


def test_fork_beam128_full(device):
    """16 requests x 128 beams, 8 KV heads x 128, bf16: tables and cache bit-exact."""
    wl = workloads.fork_beam128(seed=0)
    _assert_same(run_fork(wl, device), run_oracle(wl))


@pytest.mark.parametrize("append", [True, False])
@pytest.mark.parametrize("S,L", [(1, (1, 15)), (3, (10, 40))])
def test_fork_multi_block_rows(device, append, S, L):
    wl = workloads.make_fork(R=5, W=24, Hkv=4, D=128, S=S, L_old=L, seed=4)
    _assert_same(run_fork(wl, device, append), run_oracle(wl, append))


@pytest.mark.parametrize("kind", ["identity", "all_same", "reverse", "two_parents"])
def test_fork_structured_parents(device, kind):
    wl = workloads.make_fork(R=3, W=16, Hkv=2, D=64, L_old=(3, 9), seed=6)
    W = 16
    base = torch.arange(W, dtype=torch.int32)
    par = {"identity": base, "all_same": torch.full((W,), 5, dtype=torch.int32),
           "reverse": base.flip(0), "two_parents": (base % 2) * 7}[kind]
    wl.parent = par.repeat(3, 1).contiguous()
    _assert_same(run_fork(wl, device), run_oracle(wl))


def test_fork_fp32_cache(device):
    wl = workloads.make_fork(R=2, W=8, Hkv=2, D=32, dtype=torch.float32, seed=8)
    _assert_same(run_fork(wl, device), run_oracle(wl))


def test_append_only(device):
    wl = workloads.make_fork(R=2, W=16, Hkv=8, D=128, S=2, L_old=(0, 20), seed=10)
    d = wl.to(device)
    ln = d.suffix_len.clone()
    ops.beam_kv_append(d.k_new, d.v_new, d.kv_cache[0], d.kv_cache[1], d.suffix_bt, ln)
    torch.cuda.synchronize()
    want_len, kc, vc = of.append_tokens(wl.suffix_bt.numpy(), wl.suffix_len.numpy(), _bits(wl.kv_cache[0]),
                                        _bits(wl.kv_cache[1]), _bits(wl.k_new), _bits(wl.v_new),
                                        block_size=wl.block_size)
    assert np.array_equal(ln.cpu().numpy(), want_len)
    assert np.array_equal(_bits(d.kv_cache[0]), kc) and np.array_equal(_bits(d.kv_cache[1]), vc)


def test_reshape_and_cache_slots(device):
    g = torch.Generator().manual_seed(3)
    kv = torch.randn((2, 40, 16, 4, 128), generator=g).to(torch.bfloat16)
    key = torch.randn((50, 4, 128), generator=g).to(torch.bfloat16)
    val = torch.randn((50, 4, 128), generator=g).to(torch.bfloat16)
    slots = torch.randperm(40 * 16, generator=g)[:50].to(torch.int64)
    slots[7] = -1
    d_kv = kv.to(device)
    ops.reshape_and_cache(key.to(device), val.to(device), d_kv[0], d_kv[1], slots.to(device))
    torch.cuda.synchronize()
    kc, vc = of.reshape_and_cache(_bits(key), _bits(val), _bits(kv[0]), _bits(kv[1]), slots.numpy())
    assert np.array_equal(_bits(d_kv[0]), kc) and np.array_equal(_bits(d_kv[1]), vc)


def test_fork_bad_parent_flagged(device):
    wl = workloads.make_fork(R=2, W=8, Hkv=2, D=64, seed=12)
    wl.parent[1, 3] = 99
    with pytest.raises(ValueError, match="parent index out of range"):
        run_fork(wl, device)


def test_append_full_row_flagged(device):
    wl = workloads.make_fork(R=1, W=4, Hkv=2, D=64, S=1, L_old=(16, 16), seed=14)
    with pytest.raises(ValueError, match="suffix full"):
        run_fork(wl, device)


@pytest.mark.parametrize("W,S,Hkv,L", [
    (128, 12, 2, (100, 180)),  # request table too big to stage whole: each child's two rows staged
    (4, 300, 2, (200, 600)),   # rows longer than the row staging: block ids read from the table
    (300, 1, 2, (1, 15)),      # more children than threads per workgroup
    (16, 2, 3, (1, 30)),       # a token's vectors (3 heads x 16) do not divide the workgroup
])
def test_fork_table_sizes(device, W, S, Hkv, L):
    wl = workloads.make_fork(R=2, W=W, Hkv=Hkv, D=128, S=S, L_old=L, seed=W + S)
    _assert_same(run_fork(wl, device), run_oracle(wl))


def _layer_caches(wl, n_layers, seed):
    """The workload's cache plus n_layers - 1 more of the same geometry, each with its own contents."""
    g = torch.Generator().manual_seed(seed)
    out = [wl.kv_cache]
    for _ in range(n_layers - 1):
        out.append(torch.randn(wl.kv_cache.shape, generator=g, dtype=torch.float32).to(wl.kv_cache.dtype))
    return out


@pytest.mark.parametrize("n_layers,W,S,L", [
    (3, 16, 1, (1, 15)),
    (35, 8, 2, (3, 30)),  # more layers than one launch takes: two launches
    (28, 128, 1, (1, 15)),
    (2, 300, 1, (1, 15)),  # more children than threads per workgroup
])
def test_fork_layers_matches_oracle(device, n_layers, W, S, L):
    """One multi-layer launch equals the oracle's fork of each layer's cache, bit for bit."""
    wl = workloads.make_fork(R=2, W=W, Hkv=2, D=128, S=S, L_old=L, seed=n_layers + W)
    host = _layer_caches(wl, n_layers, seed=W)
    dev = [kv.to(device) for kv in host]
    d = wl.to(device)
    status = ops.new_status(device)
    bt, ln = ops.beam_kv_fork_layers(d.parent, d.suffix_bt, d.suffix_len, dev, status=status)
    torch.cuda.synchronize()
    ops.check_status(status)
    for layer, (kv_h, kv_d) in enumerate(zip(host, dev)):
        want = of.fork_append(wl.parent.numpy(), wl.suffix_bt.numpy(), wl.suffix_len.numpy(), _bits(kv_h[0]),
                              _bits(kv_h[1]), None, None, block_size=wl.block_size)
        if layer == 0:
            assert np.array_equal(bt.cpu().numpy(), want[0]) and np.array_equal(ln.cpu().numpy(), want[1])
        assert np.array_equal(_bits(kv_d[0]), want[2]), f"layer {layer} K cache differs"
        assert np.array_equal(_bits(kv_d[1]), want[3]), f"layer {layer} V cache differs"


def test_fork_layers_bad_parent_flagged(device):
    wl = workloads.make_fork(R=2, W=8, Hkv=2, D=64, seed=21)
    wl.parent[0, 5] = -3
    d = wl.to(device)
    caches = [kv.to(device) for kv in _layer_caches(wl, 4, seed=3)]
    status = ops.new_status(device)
    bt, ln = ops.beam_kv_fork_layers(d.parent, d.suffix_bt, d.suffix_len, caches, status=status)
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="parent index out of range"):
        ops.check_status(status)
    # the request with the bad parent keeps its tables; the other forks
    assert np.array_equal(bt.cpu().numpy()[:8], wl.suffix_bt.numpy()[:8])


def test_fork_layers_rejects_mixed_geometry(device):
    wl = workloads.make_fork(R=1, W=4, Hkv=2, D=64, seed=22)
    d = wl.to(device)
    other = torch.zeros((2, wl.kv_cache.shape[1] + 1) + tuple(wl.kv_cache.shape[2:]), dtype=wl.kv_cache.dtype,
                        device=device)
    with pytest.raises(ValueError, match="same shape"):
        ops.beam_kv_fork_layers(d.parent, d.suffix_bt, d.suffix_len, [d.kv_cache, other])
