"""gr_beam_prune_topk_noalloc: the pruning entry point on the library's static
per-GPU scratch, through the C-ABI, against gr_beam_prune_topk (the same
kernels on a caller workspace) -- bit for bit, on two calls in a row, the
second smaller, so the second call runs over the first call's leftovers in
the shared scratch."""

import numpy as np
import pytest
import torch

from vllm_gr_amd import _C, ops, workloads

pytestmark = pytest.mark.gpu


def _outs(R, W, k, device):
    return (torch.empty((R, k), dtype=torch.int32, device=device),
            torch.empty((R, k), dtype=torch.int32, device=device),
            torch.empty((R, k), dtype=torch.float32, device=device),
            torch.empty((R, W), dtype=torch.float32, device=device))


def _bits(t):
    return t.cpu().contiguous().view(torch.int32).numpy()


@pytest.mark.parametrize("shapes", [[(64, 128, 8192, 128, -1), (3, 16, 512, 16, 7)],
                                    [(8, 128, 8192, 128, 5), (2, 8, 1024, 8, -1)]])
def test_noalloc_matches_workspace_entry(device, shapes):
    for i, (R, W, V, k, eos) in enumerate(shapes):
        wl = workloads.make_prune(R=R, W=W, V=V, k=k, seed=31 + i)
        if eos >= 0:
            wl.logits[:, :, eos] += 6.0
        d = wl.to(device)
        print(f"[noalloc] call {i}: R={R} W={W} V={V} k={k} eos={eos}", flush=True)
        got = ops.beam_prune_topk_noalloc(d.logits, d.cum, k, eos, out=_outs(R, W, k, device))
        want = ops.beam_prune_topk(d.logits, d.cum, k, eos)
        torch.cuda.synchronize()
        for g, w in zip(got, want):
            assert np.array_equal(_bits(g), _bits(w))


def test_noalloc_rejects_oversized_call(device):
    """A call whose workspace exceeds the static scratch is refused before any
    launch, with the library's GR_ERR_WORKSPACE."""
    R, W, V, k = 16, 512, 1024, 512
    assert ops.prune_workspace_bytes(R, W, V, k) > _C.GR_PRUNE_SCRATCH_BYTES
    x = torch.empty((R, W, V), dtype=torch.float32, device=device)
    c = torch.empty((R, W), dtype=torch.float32, device=device)
    with pytest.raises(ValueError, match="static"):
        ops.beam_prune_topk_noalloc(x, c, k, out=_outs(R, W, k, device))
    outs = _outs(R, W, k, device)
    code = _C.lib().gr_beam_prune_topk_noalloc(x.data_ptr(), V, c.data_ptr(), R, W, V, k, -1,
                                               *[t.data_ptr() for t in outs], None)
    assert code == _C.GR_ERR_WORKSPACE
