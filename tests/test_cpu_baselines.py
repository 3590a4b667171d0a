"""The host-core baselines that bench.py times (oracle/cpu_baseline.py) give
the oracle's results: the torch fork equals oracle.fork.fork_append bit for
bit; the torch prune selects the oracle's (parent, token) set on tie-free
data, with scores to float32 logprob precision."""

import numpy as np
import pytest
import torch

from oracle import cpu_baseline as cb
from oracle import fork as of
from oracle import prune as op


@pytest.mark.parametrize("seed,R,W,S,bs", [(0, 3, 8, 4, 4), (1, 2, 16, 3, 8), (2, 1, 1, 2, 4), (3, 4, 6, 5, 2)])
def test_fork_torch_equals_oracle(seed, R, W, S, bs):
    rng = np.random.default_rng(seed)
    Hkv, D = 2, 8
    N = R * W
    NB = N * S + 3
    perm = rng.permutation(NB)[: N * S].reshape(N, S).astype(np.int32)
    lens = rng.integers(0, S * bs, size=N).astype(np.int32)   # room for the appended token
    parent = rng.integers(0, W, size=(R, W)).astype(np.int32)
    parent[0, :] = rng.integers(0, max(1, W // 3), size=W)    # many children of few parents
    kc = rng.integers(-2**15, 2**15, size=(NB, bs, Hkv, D)).astype(np.int16)
    vc = rng.integers(-2**15, 2**15, size=(NB, bs, Hkv, D)).astype(np.int16)
    kn = rng.integers(-2**15, 2**15, size=(N, Hkv, D)).astype(np.int16)
    vn = rng.integers(-2**15, 2**15, size=(N, Hkv, D)).astype(np.int16)
    want_bt, want_len, want_k, want_v = of.fork_append(parent, perm, lens, kc, vc, kn, vn, block_size=bs)
    tk, tv = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    bt, ln = cb.fork_append_torch(torch.from_numpy(parent), torch.from_numpy(perm), torch.from_numpy(lens),
                                  tk, tv, torch.from_numpy(kn), torch.from_numpy(vn), block_size=bs)
    np.testing.assert_array_equal(bt.numpy(), want_bt)
    np.testing.assert_array_equal(ln.numpy(), want_len)
    np.testing.assert_array_equal(tk.numpy(), want_k)
    np.testing.assert_array_equal(tv.numpy(), want_v)


@pytest.mark.parametrize("seed,R,W,V", [(0, 2, 4, 64), (1, 3, 8, 500), (2, 1, 16, 2048)])
def test_prune_torch_equals_oracle(seed, R, W, V):
    rng = np.random.default_rng(seed)
    x = rng.permutation(R * W * V).reshape(R, W, V).astype(np.float32) / (R * W * V) * 20.0  # distinct
    cum = (-rng.random((R, W)) * 3).astype(np.float32)
    res = op.prune_topk(x, cum, W)
    parent, token, score = cb.prune_topk_torch(torch.from_numpy(x), torch.from_numpy(cum), W)
    for r in range(R):
        want = {(int(p), int(t)) for p, t in zip(res["parent"][r], res["token"][r])}
        got = {(int(p), int(t)) for p, t in zip(parent[r], token[r])}
        assert got == want
    np.testing.assert_allclose(np.sort(score.numpy(), axis=1), np.sort(res["score64"], axis=1),
                               rtol=0, atol=1e-4)
