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
