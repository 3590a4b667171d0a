"""Seeded synthetic workloads for the beam path (inputs only; no compute).

Every tensor is drawn on the CPU from one ``torch.Generator`` seeded by the
caller, in a fixed order, then copied to the target device, so a GPU run and
a CPU check see bit-identical inputs.

Named shapes:

* ``decode_small_fp32``: 1 request x 32 beams, shared prefix 512, suffix 4,
  16 query / 4 KV heads, head_dim 128, block 16, float32, N(0,1) inputs.
* ``decode_beam128``: 8 requests x 128 beams, shared prefix 2048, suffix
  length per request uniform in [1, 8], 32 query / 8 KV heads, head_dim 128,
  block 16, bf16, N(0,1)/sqrt(128) inputs, block pool 1.25x the blocks in
  use, every table a slice of one random permutation of the pool.
* ``fork_beam128``: 16 requests x 128 beams, parent uniform over the
  request's beams, one 16-token suffix block per beam, old suffix length per
  request uniform in [1, 15], 8 KV heads x 128, bf16 new tokens N(0,1).
* ``prune_beam128``: logits [64, 128, 8192] float32 N(0, 3^2) (sigma = 3),
  cumulative logprobs [64, 128] uniform in (-20, 0).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, fields

import torch


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


@dataclass
class DecodeWorkload:
    q: torch.Tensor            # [N*T, Hq, D]
    kv_cache: torch.Tensor     # [2, num_blocks, block_size, Hkv, D]
    prefix_bt: torch.Tensor    # [R, prefix_blocks] int32
    prefix_len: torch.Tensor   # [R] int32
    beam_start: torch.Tensor   # [R+1] int32
    suffix_bt: torch.Tensor    # [N, suffix_blocks] int32
    suffix_len: torch.Tensor   # [N] int32
    q_per_beam: int
    scale: float
    softcap: float
    block_size: int
    max_beams: int

    def to(self, device) -> "DecodeWorkload":
        kw = {}
        for f in fields(self):
            v = getattr(self, f.name)
            kw[f.name] = v.to(device) if isinstance(v, torch.Tensor) else v
        return DecodeWorkload(**kw)

    @property
    def k_cache(self):
        return self.kv_cache[0]

    @property
    def v_cache(self):
        return self.kv_cache[1]

    def algorithmic_bytes(self) -> int:
        """Bytes one decode step must move at minimum: each request's prefix
        K/V once, each beam's suffix K/V, Q read, O written, the tables."""
        es = self.q.element_size()
        Hkv, D = self.kv_cache.shape[3], self.kv_cache.shape[4]
        kv_tok = 2 * Hkv * D * es
        pre = int(self.prefix_len.sum()) * kv_tok
        suf = int(self.suffix_len.sum()) * kv_tok
        qo = 2 * self.q.numel() * es
        tables = 4 * (self.prefix_bt.numel() + self.prefix_len.numel() + self.beam_start.numel()
                      + self.suffix_bt.numel() + self.suffix_len.numel())
        return pre + suf + qo + tables

    def flops(self) -> int:
        """2 flops per multiply-add, QK^T and PV, over every visible key."""
        T = self.q_per_beam
        NT, Hq, D = self.q.shape
        keys = 0
        bs = self.beam_start.tolist()
        P = self.prefix_len.tolist()
        L = self.suffix_len.tolist()
        for r in range(len(P)):
            for n in range(bs[r], bs[r + 1]):
                for i in range(T):
                    keys += P[r] + max(0, min(L[n], L[n] - T + i + 1))
        return 4 * keys * Hq * D


def make_decode(*, R: int, W: int, P: int, L, Hq: int, Hkv: int, D: int, block_size: int = 16,
                dtype=torch.bfloat16, input_scale: float = 1.0, seed: int = 0, q_per_beam: int = 1,
                pool_factor: float = 1.25, softcap: float = 0.0,
                suffix_blocks: int | None = None) -> DecodeWorkload:
    """Random decode step.  ``L``: an int (all beams), ``(lo, hi)`` (one draw
    per request, inclusive), or a list with one length per request."""
    g = _gen(seed)
    N = R * W
    T = q_per_beam
    if isinstance(L, int):
        lens_r = [L] * R
    elif isinstance(L, tuple):
        lens_r = torch.randint(L[0], L[1] + 1, (R,), generator=g).tolist()
    else:
        lens_r = list(L)
    sb = suffix_blocks or max(1, math.ceil(max(lens_r + [1]) / block_size))
    pb = max(1, math.ceil(P / block_size))
    used = R * pb + N * sb
    pool = max(used, math.ceil(pool_factor * used))
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    prefix_bt = perm[:R * pb].reshape(R, pb).clone()
    suffix_bt = perm[R * pb:R * pb + N * sb].reshape(N, sb).clone()
    q = torch.randn((N * T, Hq, D), generator=g, dtype=torch.float32) * input_scale
    kv = torch.randn((2, pool, block_size, Hkv, D), generator=g, dtype=torch.float32) * input_scale
    prefix_len = torch.full((R,), P, dtype=torch.int32)
    beam_start = torch.arange(0, N + 1, W, dtype=torch.int32)
    suffix_len = torch.tensor([lens_r[n // W] for n in range(N)], dtype=torch.int32)
    return DecodeWorkload(q=q.to(dtype), kv_cache=kv.to(dtype), prefix_bt=prefix_bt, prefix_len=prefix_len,
                          beam_start=beam_start, suffix_bt=suffix_bt, suffix_len=suffix_len,
                          q_per_beam=T, scale=1.0 / math.sqrt(D), softcap=softcap,
                          block_size=block_size, max_beams=W)


def decode_small_fp32(seed: int = 0) -> DecodeWorkload:
    return make_decode(R=1, W=32, P=512, L=4, Hq=16, Hkv=4, D=128, dtype=torch.float32,
                       input_scale=1.0, seed=seed, pool_factor=1.0)


def decode_beam128(seed: int = 0) -> DecodeWorkload:
    return make_decode(R=8, W=128, P=2048, L=(1, 8), Hq=32, Hkv=8, D=128, dtype=torch.bfloat16,
                       input_scale=1.0 / math.sqrt(128), seed=seed)


def decode_sid_step(seed: int = 0) -> DecodeWorkload:
    """One layer's attention in a decode step of the semantic-ID beam search:
    4 requests x 128 beams over 2048-token prompts, 16 q / 8 kv heads, each
    beam's 1-3 generated tokens as its suffix."""
    return make_decode(R=4, W=128, P=2048, L=(1, 3), Hq=16, Hkv=8, D=128, dtype=torch.bfloat16,
                       input_scale=1.0 / math.sqrt(128), seed=seed)


@dataclass
class ForkWorkload:
    parent: torch.Tensor      # [R, W] int32
    suffix_bt: torch.Tensor   # [R*W, S] int32
    suffix_len: torch.Tensor  # [R*W] int32
    kv_cache: torch.Tensor    # [2, num_blocks, block_size, Hkv, D]
    k_new: torch.Tensor       # [R*W, Hkv, D]
    v_new: torch.Tensor
    block_size: int

    def to(self, device) -> "ForkWorkload":
        kw = {}
        for f in fields(self):
            v = getattr(self, f.name)
            kw[f.name] = v.to(device) if isinstance(v, torch.Tensor) else v
        return ForkWorkload(**kw)

    def algorithmic_bytes(self) -> int:
        """Tables in/out, parents, every copy-on-write token copied (read +
        write, K and V) and the appended token (read + write, K and V)."""
        R, W = self.parent.shape
        Hkv, D = self.kv_cache.shape[3], self.kv_cache.shape[4]
        tok = Hkv * D * self.kv_cache.element_size()
        cow_tokens = 0
        par = self.parent.tolist()
        lens = self.suffix_len.tolist()
        for r in range(R):
            seen = set()
            for c in range(W):
                p = par[r][c]
                if p in seen:
                    cow_tokens += lens[r * W + p]
                seen.add(p)
        tables = 4 * (self.parent.numel() + 2 * self.suffix_bt.numel() + 2 * self.suffix_len.numel())
        return tables + 2 * 2 * cow_tokens * tok + 2 * 2 * R * W * tok


def make_fork(*, R: int, W: int, Hkv: int, D: int, block_size: int = 16, S: int = 1,
              L_old=(1, 15), dtype=torch.bfloat16, seed: int = 0, pool_factor: float = 1.25) -> ForkWorkload:
    g = _gen(seed)
    N = R * W
    parent = torch.randint(0, W, (R, W), generator=g, dtype=torch.int32)
    lens_r = torch.randint(L_old[0], L_old[1] + 1, (R,), generator=g).tolist()
    pool = math.ceil(pool_factor * N * S)
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    suffix_bt = perm[:N * S].reshape(N, S).clone()
    suffix_len = torch.tensor([lens_r[n // W] for n in range(N)], dtype=torch.int32)
    kv = torch.randn((2, pool, block_size, Hkv, D), generator=g, dtype=torch.float32)
    k_new = torch.randn((N, Hkv, D), generator=g, dtype=torch.float32)
    v_new = torch.randn((N, Hkv, D), generator=g, dtype=torch.float32)
    return ForkWorkload(parent=parent, suffix_bt=suffix_bt, suffix_len=suffix_len, kv_cache=kv.to(dtype),
                        k_new=k_new.to(dtype), v_new=v_new.to(dtype), block_size=block_size)


def fork_beam128(seed: int = 0) -> ForkWorkload:
    return make_fork(R=16, W=128, Hkv=8, D=128, seed=seed)


@dataclass
class PruneWorkload:
    logits: torch.Tensor  # [R, W, V] float32
    cum: torch.Tensor     # [R, W] float32
    k: int

    def to(self, device) -> "PruneWorkload":
        return PruneWorkload(self.logits.to(device), self.cum.to(device), self.k)

    def algorithmic_bytes(self) -> int:
        R, W, V = self.logits.shape
        return 4 * R * W * V + 4 * R * W + 3 * 4 * R * self.k


def make_prune(*, R: int, W: int, V: int, k: int | None = None, sigma: float = 3.0,
               seed: int = 0) -> PruneWorkload:
    g = _gen(seed)
    logits = torch.randn((R, W, V), generator=g, dtype=torch.float32) * sigma
    cum = torch.rand((R, W), generator=g, dtype=torch.float32) * -20.0
    return PruneWorkload(logits=logits, cum=cum, k=k or W)


def prune_beam128(seed: int = 0) -> PruneWorkload:
    return make_prune(R=64, W=128, V=8192, seed=seed)
