"""CPU baseline for BeamAttention decode.  TEST INFRASTRUCTURE ONLY (timed by
``bench.py``'s ``cpu_baseline`` leg, never part of the product path).

The reference's own Python cannot run without vLLM, so the baseline is the
torch float32 restatement of the reference algorithm on the host cores: the
cascade of ``vllm_gr/v1/attention/backends/beam_attn.py:629-701`` -- a
non-causal prefix pass over all beams of a request as one group with its LSE
(``:656-678``), a per-beam suffix pass with LSE (``:686-695``), and the LSE
merge (``:697-699``); the paged prefix/suffix KV is gathered by block table
first, as the reference's Triton gather does for the suffix (``:62-117``).
Decode shape: one query token per beam.
"""

from __future__ import annotations

import torch


def _gather(cache: torch.Tensor, row: torch.Tensor, n: int, bs: int) -> torch.Tensor:
    pos = torch.arange(n)
    return cache[row.long()[pos // bs], pos % bs]


def cascade_decode_fp32(q, k_cache, v_cache, prefix_bt, prefix_len, beam_start, suffix_bt, suffix_len,
                        *, scale: float, block_size: int, requests=None) -> torch.Tensor:
    """q ``[N, Hq, D]``; caches ``[num_blocks, block_size, Hkv, D]`` (CPU).
    Returns float32 ``[N, Hq, D]`` for the beams of ``requests`` (default all)."""
    N, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    out = torch.zeros((N, Hq, D), dtype=torch.float32)
    reqs = range(len(prefix_len)) if requests is None else requests
    for r in reqs:
        n0, n1 = int(beam_start[r]), int(beam_start[r + 1])
        Wr = n1 - n0
        P = int(prefix_len[r])
        kp = _gather(k_cache, prefix_bt[r], P, block_size).float().permute(1, 2, 0)  # [Hkv, D, P]
        vp = _gather(v_cache, prefix_bt[r], P, block_size).float().permute(1, 0, 2)  # [Hkv, P, D]
        qr = q[n0:n1].float().reshape(Wr, Hkv, G, D).permute(1, 0, 2, 3).reshape(Hkv, Wr * G, D)
        s = torch.bmm(qr, kp) * scale                                                  # [Hkv, Wr*G, P]
        lse_p = torch.logsumexp(s, dim=-1)
        o_p = torch.bmm(torch.softmax(s, dim=-1), vp)                                  # [Hkv, Wr*G, D]
        # suffix pass, padded to the longest suffix of the request with a mask
        lens = suffix_len[n0:n1].long()
        Lmax = int(lens.max()) if Wr else 0
        if Lmax > 0:
            pos = torch.arange(Lmax)
            blk = suffix_bt[n0:n1].long().gather(1, (pos // block_size).expand(Wr, -1).clamp_max(
                suffix_bt.shape[1] - 1))
            ks = k_cache[blk, pos % block_size].float()                               # [Wr, Lmax, Hkv, D]
            vs = v_cache[blk, pos % block_size].float()
            qb = q[n0:n1].float().reshape(Wr, Hkv, G, D)
            ss = torch.einsum("bhgd,blhd->bhgl", qb, ks) * scale
            mask = pos[None, :] < lens[:, None]                                        # [Wr, Lmax]
            ss = ss.masked_fill(~mask[:, None, None, :], float("-inf"))
            lse_s = torch.logsumexp(ss, dim=-1)                                        # [Wr, Hkv, G]
            o_s = torch.einsum("bhgl,blhd->bhgd", torch.softmax(ss, dim=-1).nan_to_num(0.0), vs)
            lse_s = lse_s.permute(1, 0, 2).reshape(Hkv, Wr * G)
            o_s = o_s.permute(1, 0, 2, 3).reshape(Hkv, Wr * G, D)
        else:
            lse_s = torch.full((Hkv, Wr * G), float("-inf"))
            o_s = torch.zeros_like(o_p)
        m = torch.maximum(lse_p, lse_s)
        wa = torch.exp(lse_p - m)
        wb = torch.exp(lse_s - m)
        o = (wa[..., None] * o_p + wb[..., None] * o_s) / (wa + wb)[..., None]
        out[n0:n1] = o.reshape(Hkv, Wr, G, D).permute(1, 0, 2, 3).reshape(Wr, Hq, D)
    return out


def fork_append_torch(parent, suffix_bt, suffix_len, k_cache, v_cache, k_new, v_new, *, block_size):
    """Beam KV fork + append as torch index operations on the host cores (the
    CPU baseline of the device fork).  Same contract as ``oracle.fork``'s
    ``fork_append`` (the reference's content rule, child suffix = parent
    suffix ++ new token, ``vllm_gr/entrypoints/openai/serving_engine.py:113-120``),
    vectorised: the owner / copy-on-write assignment as tensor ops, then one
    gather-scatter of every copy-on-write token's K and V rows by slot and one
    scatter of the appended tokens.  Updates the caches in place and returns
    ``(new_bt, new_len)``."""
    parent = parent.long()
    R, W = parent.shape
    NB, bs = k_cache.shape[0], block_size
    cols = torch.arange(W).expand(R, W)
    first = torch.full((R, W), W, dtype=torch.long).scatter_reduce(1, parent, cols, "amin")
    owner = first.gather(1, parent) == cols                           # child inherits the row in place
    free = first == W                                                 # childless parents
    # k-th copy-on-write child <- k-th childless parent (stable sorts put them first, in order)
    cow_c = torch.argsort((owner).to(torch.int8), dim=1, stable=True)
    free_p = torch.argsort((~free).to(torch.int8), dim=1, stable=True)
    src_row = torch.where(owner, parent, torch.zeros_like(parent))
    src_row.scatter_(1, cow_c, torch.where(~owner.gather(1, cow_c), free_p, src_row.gather(1, cow_c)))
    base = (torch.arange(R) * W)[:, None]
    new_bt = suffix_bt[(base + src_row).reshape(-1)]
    par_flat = (base + parent).reshape(-1)
    new_len = suffix_len[par_flat].clone()
    # copy-on-write tokens: slots of the parent's row -> slots of the child's new row
    cow = (~owner).reshape(-1).nonzero().squeeze(1)
    n_tok = new_len[cow].long()
    child = torch.repeat_interleave(cow, n_tok)
    pos = torch.arange(int(n_tok.sum())) - torch.repeat_interleave(torch.cumsum(n_tok, 0) - n_tok, n_tok)
    src_slot = suffix_bt[par_flat[child], pos // bs].long() * bs + pos % bs
    dst_slot = new_bt[child, pos // bs].long() * bs + pos % bs
    for cache, new in ((k_cache, k_new), (v_cache, v_new)):
        flat = cache.view(NB * bs, -1)
        flat[dst_slot] = flat[src_slot]
        L = new_len.long()
        app = new_bt[torch.arange(R * W), L // bs].long() * bs + L % bs
        flat[app] = new.reshape(R * W, -1)
    return new_bt, new_len + 1


def prune_topk_torch(logits, cum, k):
    """Beam pruning in the reference's formulation on the host cores (the CPU
    baseline of the fused prune): the sampler's float32 ``log_softmax`` and
    per-beam top-k logprobs (``serving_engine.py:300-308``), then per request
    the top-k of ``cum + logprob`` over all beams' candidates
    (``serving_engine.py:511-567``).  Returns ``(parent, token, score)``
    ``[R, k]`` for ``logits [R, W, V]`` and ``cum [R, W]``; ties are left in
    torch's order."""
    R, W, V = logits.shape
    lp, tok = torch.log_softmax(logits, dim=-1).topk(k, dim=-1)          # [R, W, k]
    score = (cum.double().reshape(R, W, 1) + lp.double()).reshape(R, W * k)
    best, idx = score.topk(k, dim=-1)
    return idx // k, tok.reshape(R, W * k).gather(1, idx), best
