"""Host logic of the synthetic workloads (CPU only): seeded determinism, the
paged-pool layout (distinct physical blocks, pool = ceil(1.25 x used)), and
the algorithmic byte / flop counts the benchmark reports, checked against
their closed forms for the 8 x 128-beam, 2048-prefix decode step."""

from __future__ import annotations

import torch

from vllm_gr_amd import workloads


def test_decode_beam128_layout_and_counts():
    wl = workloads.decode_beam128(seed=0)
    R, W, P, Hq, Hkv, D = 8, 128, 2048, 32, 8, 128
    N = R * W
    assert wl.q.shape == (N, Hq, D) and wl.q.dtype == torch.bfloat16
    assert wl.kv_cache.shape == (2, 2560, 16, Hkv, D)  # ceil(1.25 * (8*128 + 1024*1)) blocks
    assert wl.prefix_bt.shape == (R, P // 16) and wl.suffix_bt.shape == (N, 1)
    ids = torch.cat([wl.prefix_bt.reshape(-1), wl.suffix_bt.reshape(-1)])
    assert ids.unique().numel() == ids.numel() and int(ids.min()) >= 0 and int(ids.max()) < 2560
    # one suffix length per request, drawn from 1..8
    L = wl.suffix_len.reshape(R, W)
    assert torch.all(L == L[:, :1]) and int(L.min()) >= 1 and int(L.max()) <= 8
    mean_L = float(wl.suffix_len.float().mean())
    tables = 4 * (R * 128 + R + (R + 1) + N + N)
    want = 67_108_864 + round(4_194_304 * mean_L) + 16_777_216 + tables
    assert wl.algorithmic_bytes() == want
    assert wl.flops() == 4 * Hq * D * N * (P + mean_L)


def test_decode_workload_is_seeded():
    a = workloads.make_decode(R=2, W=4, P=40, L=(1, 5), Hq=4, Hkv=2, D=16, seed=3)
    b = workloads.make_decode(R=2, W=4, P=40, L=(1, 5), Hq=4, Hkv=2, D=16, seed=3)
    c = workloads.make_decode(R=2, W=4, P=40, L=(1, 5), Hq=4, Hkv=2, D=16, seed=4)
    assert torch.equal(a.q, b.q) and torch.equal(a.prefix_bt, b.prefix_bt)
    assert not torch.equal(a.q, c.q)


def test_multi_token_flops_are_causal():
    """T query tokens per beam: token i sees P + (L - T + i + 1) keys."""
    wl = workloads.make_decode(R=1, W=2, P=10, L=4, Hq=2, Hkv=1, D=8, q_per_beam=3, seed=0)
    keys = 2 * sum(10 + (4 - 3 + i + 1) for i in range(3))
    assert wl.flops() == 4 * keys * 2 * 8


def test_fork_and_prune_workloads():
    fw = workloads.fork_beam128(seed=0)
    assert fw.parent.shape == (16, 128) and int(fw.parent.max()) < 128
    assert fw.suffix_bt.shape == (2048, 1)
    assert fw.algorithmic_bytes() > 2 * 2 * 2048 * 8 * 128 * 2  # at least the appends
    pw = workloads.prune_beam128(seed=0)
    assert pw.logits.shape == (64, 128, 8192) and pw.k == 128
    assert pw.algorithmic_bytes() == 268_435_456 + 32_768 + 98_304
