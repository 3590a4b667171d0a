"""Fused beam pruning on the GPU vs the bit-exact CPU oracle."""

import numpy as np
import pytest
import torch

from oracle import prune as op
from vllm_gr_amd import ops, workloads

pytestmark = pytest.mark.gpu


def run_gpu(wl, device, eos=-1):
    d = wl.to(device)
    parent, token, score, eos_score = ops.beam_prune_topk(d.logits, d.cum, wl.k, eos)
    torch.cuda.synchronize()
    return parent.cpu().numpy(), token.cpu().numpy(), score.cpu().numpy(), eos_score.cpu().numpy()


def _assert_exact(got, want):
    p, t, s, e = got
    assert np.array_equal(p, want["parent"]), "parent beams differ"
    assert np.array_equal(t, want["token"]), "tokens differ"
    assert np.array_equal(s.view(np.int32), want["score"].view(np.int32)), "scores differ (bits)"
    assert np.array_equal(e.view(np.int32), want["eos_score"].view(np.int32)), "eos scores differ"


def test_prune_beam128_full(device):
    """logits [64, 128, 8192] ~ N(0, 3^2), cum ~ U(-20, 0), top-128: bit-exact."""
    wl = workloads.prune_beam128(seed=0)
    _assert_exact(run_gpu(wl, device), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), wl.k))


def test_prune_beam128_vs_float64_mathematics(device):
    """The kernel itself against plain float64 mathematics at the full
    64 x 128 x 8192 size (log_softmax + cum + top-128 over beams x vocab,
    serving_engine.py:511,538-567): the same (parent, token) selections, in
    order, for every request whose float64 128th/129th gap exceeds 1e-6
    (printed: none is excluded at seed 0), scores within 1e-5."""
    wl = workloads.prune_beam128(seed=0)
    ref = op.topk_float64_global(wl.logits.numpy(), wl.cum.numpy(), wl.k)
    p, t, s, _ = run_gpu(wl, device)
    firm = ref["gap"] > 1e-6
    print(f"requests with a 128th/129th gap <= 1e-6: {int((~firm).sum())} of {len(firm)}", flush=True)
    assert firm.sum() >= len(firm) - 2
    for r in np.nonzero(firm)[0]:
        assert np.array_equal(p[r], ref["parent"][r]) and np.array_equal(t[r], ref["token"][r]), f"request {r}"
    np.testing.assert_allclose(s.astype(np.float64), ref["score"], rtol=0, atol=1e-5)


@pytest.mark.parametrize("R,W,V,k", [(3, 16, 512, 16), (2, 4, 12288, 32), (1, 1, 64, 8), (2, 300, 256, 100),
                                     (2, 4, 2048, 300)])
def test_prune_shapes(device, R, W, V, k):
    wl = workloads.make_prune(R=R, W=W, V=V, k=k, seed=R + W + V)
    _assert_exact(run_gpu(wl, device), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), k))


@pytest.mark.parametrize("V", [8192, 12288])
def test_prune_one_wave_holds_most_survivors(device, V):
    """200 large logits per row among the elements one wave of the row's
    workgroup reads (token % 1024 in [0, 256) or [768, 1024)): that wave has
    ~235 of the row's ~350 keys above the selection bound, so the direct rank
    runs with eight targets per lane and one wave's survivors filling most of
    the list.  Bit-exact."""
    wl = workloads.make_prune(R=2, W=16, V=V, k=128, seed=5)
    g = np.random.default_rng(5)
    lg = wl.logits.numpy()
    tok = np.arange(V) % 1024
    for r in range(2):
        for b in range(16):
            base = 0 if b % 2 == 0 else 768
            pick = g.choice(np.nonzero((tok >= base) & (tok < base + 256))[0], 200, replace=False)
            lg[r, b, pick] = 10 + g.random(200).astype(np.float32)
    _assert_exact(run_gpu(wl, device), op.prune_topk(lg, wl.cum.numpy(), 128))


def test_prune_all_equal_logits(device):
    """Every score ties: the lowest flat indices (beam 0, tokens 0..k-1) win."""
    wl = workloads.make_prune(R=2, W=8, V=1024, k=8, seed=1)
    wl.logits.zero_()
    wl.cum.zero_()
    got = run_gpu(wl, device)
    _assert_exact(got, op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), 8))
    assert (got[0] == 0).all() and (got[1] == np.arange(8)).all()


def test_prune_quantised_ties(device):
    """Logits on a coarse grid: many exact ties inside and across rows."""
    wl = workloads.make_prune(R=3, W=32, V=2048, k=32, seed=2)
    wl.logits.copy_(torch.round(wl.logits))
    wl.cum.copy_(torch.round(wl.cum))
    _assert_exact(run_gpu(wl, device), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), 32))


def test_prune_with_eos(device):
    wl = workloads.make_prune(R=4, W=16, V=1024, k=16, seed=3)
    eos = 17
    wl.logits[:, :, eos] += 8.0  # EOS lands in many rows' top-k
    _assert_exact(run_gpu(wl, device, eos), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), 16, eos))


def test_prune_masked_logits(device):
    """-inf logits (masked tokens) and a fully masked beam."""
    wl = workloads.make_prune(R=2, W=8, V=512, k=8, seed=4)
    wl.logits[0, :, 100:] = float("-inf")
    wl.logits[1, 3, :] = float("-inf")
    _assert_exact(run_gpu(wl, device), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), 8))


def test_prune_dead_rows(device):
    """-inf cumulative scores (slots no candidate filled): every score of such
    a row ties at -inf, so its candidate list (logit order) is not in flat
    order.  Groups of 32 rows holding one are selected by radix select and
    counting, the others by merging sorted lists, in the same launch."""
    wl = workloads.make_prune(R=4, W=128, V=1024, k=128, seed=7)
    wl.cum[1, 40:] = float("-inf")  # three of request 1's four row groups
    wl.cum[2, 1:] = float("-inf")   # one live row: exactly k finite candidates
    wl.cum[3, :] = float("-inf")    # none finite: the lowest flat indices win
    _assert_exact(run_gpu(wl, device), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), 128))


def test_prune_rounding_collapse(device):
    """Cumulative scores near -1e15 (float64 ulp 0.125): c + x rounds distinct
    logits of a row to one score, whose ties go by token, not by the row's
    logit order -- every group takes the radix-select path, with many ties."""
    wl = workloads.make_prune(R=2, W=128, V=1024, k=128, seed=8)
    g = torch.Generator().manual_seed(8)
    wl.cum.copy_(torch.full_like(wl.cum, -1e15) - torch.randint(0, 4, wl.cum.shape, generator=g).float() * 2.0 ** 27)
    _assert_exact(run_gpu(wl, device), op.prune_topk(wl.logits.numpy(), wl.cum.numpy(), 128))


def test_prune_catalog_matches_oracle(device):
    """Catalog-constrained pruning: each beam's top-k candidates outside its
    trie node's children leave the pool (serving_engine.py:504-506), bit for
    bit against the masked C oracle; node_out is each new beam's trie node."""
    from vllm_gr_amd.entrypoints.catalog import Catalog
    rng = np.random.default_rng(11)
    R, W, V, k, eos = 4, 32, 8192, 32, 5
    cat = Catalog()
    seqs = [rng.integers(0, V, size=3).tolist() for _ in range(3000)]
    seqs += [[s[0], eos] for s in seqs[:40]]  # EOS valid after some first tokens
    for s in seqs:
        cat.add(s)
    # beam prefixes: root, inside the trie, dead (-1) and complete (no children)
    prefixes = []
    for r in range(R):
        row = []
        for b in range(W):
            s = seqs[int(rng.integers(0, len(seqs)))]
            kind = b % 5
            # kind 1: a first token that has EOS among its children
            row.append([] if kind == 0 else seqs[int(rng.integers(0, 40))][:1] if kind == 1 else s[:2]
                       if kind == 2 else [V - 1, V - 2] if kind == 3 else s[:3])
        prefixes.append(row)
    node = torch.tensor([[cat.node_of(p) for p in row] for row in prefixes], dtype=torch.int32)
    allowed = np.zeros((R, W, V), bool)
    for r in range(R):
        for b in range(W):
            allowed[r, b, list(cat.valid(prefixes[r][b]))] = True
    logits = torch.from_numpy((rng.standard_normal((R, W, V)) * 3).astype(np.float32))
    # make the valid tokens competitive so the beams' top-k hold several of them
    logits += torch.from_numpy(allowed.astype(np.float32) * 6.0)
    cum = torch.from_numpy(rng.uniform(-20, 0, (R, W)).astype(np.float32))
    status = ops.new_status(device)
    print(f"[prune] catalog R={R} W={W} V={V} k={k} nodes={cat.to_device('cpu').num_nodes}", flush=True)
    parent, token, score, eos_score, node_out = ops.beam_prune_topk(
        logits.to(device), cum.to(device), k, eos, catalog=cat.to_device(device), beam_node=node.to(device),
        status=status)
    torch.cuda.synchronize()
    ops.check_status(status)
    want = op.prune_topk(logits.numpy(), cum.numpy(), k, eos, allowed=allowed)
    assert np.array_equal(parent.cpu().numpy(), want["parent"])
    assert np.array_equal(token.cpu().numpy(), want["token"])
    assert np.array_equal(score.cpu().numpy().view(np.int32), want["score"].view(np.int32))
    assert np.array_equal(eos_score.cpu().numpy().view(np.int32), want["eos_score"].reshape(R, W).view(np.int32))
    assert (want["parent"] >= 0).sum() > R * k // 2 and np.isfinite(want["eos_score"]).any()
    no = node_out.cpu().numpy()
    for r in range(R):
        for j in range(k):
            p, t = int(want["parent"][r, j]), int(want["token"][r, j])
            assert no[r, j] == (cat.node_of(prefixes[r][p] + [t]) if p >= 0 else -1)


def _assert_exact64(got, want, R, W):
    p, t, s, e = got
    assert np.array_equal(p, want["parent"]), "parent beams differ"
    assert np.array_equal(t, want["token"]), "tokens differ"
    assert np.array_equal(s.view(np.int64), want["score64"].view(np.int64)), "float64 scores differ (bits)"
    assert np.array_equal(e.view(np.int64), want["eos_score64"].reshape(R, W).view(np.int64)), "eos scores differ"


@pytest.mark.parametrize("R,W,V,k,eos", [(64, 128, 8192, 128, -1), (3, 16, 512, 16, 7), (2, 300, 256, 100, 3)])
def test_prune_f64_matches_oracle(device, R, W, V, k, eos):
    """gr_beam_prune_topk_f64: float64 cumulative scores in, float64 scores out
    (the reference's Python-float beam scores, serving_engine.py:511, 538-539),
    and every beam's top-k (token, logprob) list: all bit-exact against the C
    oracle, at the full pruning workload and smaller shapes."""
    wl = workloads.make_prune(R=R, W=W, V=V, k=k, seed=5 + R)
    if eos >= 0:
        wl.logits[:, :, eos] += 6.0
    cum = torch.from_numpy(np.random.default_rng(R + W).uniform(-20, 0, (R, W)))  # float64, not float32 values
    print(f"[prune] f64 R={R} W={W} V={V} k={k} eos={eos}", flush=True)
    parent, token, score, eos_score, ct, cl = ops.beam_prune_topk(wl.logits.to(device), cum.to(device), k, eos,
                                                                  candidates=True)
    torch.cuda.synchronize()
    assert score.dtype == torch.float64 and eos_score.dtype == torch.float64
    want = op.prune_topk(wl.logits.numpy(), cum.numpy(), k, eos, candidates=True)
    _assert_exact64((parent.cpu().numpy(), token.cpu().numpy(), score.cpu().numpy(), eos_score.cpu().numpy()),
                    want, R, W)
    assert np.array_equal(ct.cpu().numpy(), want["cand_token"])
    assert np.array_equal(cl.cpu().numpy().view(np.int32), want["cand_logprob"].view(np.int32))


def test_prune_f64_catalog(device):
    """The float64 entry point in catalog mode equals the masked oracle."""
    from vllm_gr_amd.entrypoints.catalog import Catalog
    rng = np.random.default_rng(12)
    R, W, V, k = 2, 16, 1024, 16
    cat = Catalog()
    seqs = [rng.integers(0, V, size=3).tolist() for _ in range(500)]
    for s in seqs:
        cat.add(s)
    prefixes = [[[] if b % 3 == 0 else seqs[int(rng.integers(0, len(seqs)))][:1 + b % 2] for b in range(W)]
                for _ in range(R)]
    node = torch.tensor([[cat.node_of(p) for p in row] for row in prefixes], dtype=torch.int32)
    allowed = np.zeros((R, W, V), bool)
    for r in range(R):
        for b in range(W):
            allowed[r, b, list(cat.valid(prefixes[r][b]))] = True
    logits = torch.from_numpy((rng.standard_normal((R, W, V)) * 3 + allowed * 6.0).astype(np.float32))
    cum = torch.from_numpy(rng.uniform(-20, 0, (R, W)))
    parent, token, score, eos_score, node_out = ops.beam_prune_topk(
        logits.to(device), cum.to(device), k, -1, catalog=cat.to_device(device), beam_node=node.to(device))
    torch.cuda.synchronize()
    want = op.prune_topk(logits.numpy(), cum.numpy(), k, -1, allowed=allowed)
    _assert_exact64((parent.cpu().numpy(), token.cpu().numpy(), score.cpu().numpy(), eos_score.cpu().numpy()),
                    want, R, W)
    no = node_out.cpu().numpy()
    for r in range(R):
        for j in range(k):
            p, t = int(want["parent"][r, j]), int(want["token"][r, j])
            assert no[r, j] == (cat.node_of(prefixes[r][p] + [t]) if p >= 0 else -1)


def test_prune_f64_planted_flip(device):
    """Identical logits rows, scores 2^-30 apart: the float64 path selects the
    second beam, float32 carrying of the same scores ties them and selects the
    first (lowest flat index) -- a selection that carrying scores in float32
    between steps would flip."""
    x = torch.linspace(-1, 1, 8, dtype=torch.float32).repeat(1, 2, 1).contiguous()
    cum64 = torch.tensor([[-10.0, -10.0 + 2.0 ** -30]], dtype=torch.float64)
    p64, t64, s64, _ = ops.beam_prune_topk(x.to(device), cum64.to(device), 1)
    p32, t32, s32, _ = ops.beam_prune_topk(x.to(device), cum64.to(torch.float32).to(device), 1)
    torch.cuda.synchronize()
    assert (int(p64[0, 0]), int(t64[0, 0])) == (1, 7)
    assert (int(p32[0, 0]), int(t32[0, 0])) == (0, 7)
    want = op.prune_topk(x.numpy(), cum64.numpy(), 1)
    assert float(s64[0, 0]) == float(want["score64"][0, 0])
