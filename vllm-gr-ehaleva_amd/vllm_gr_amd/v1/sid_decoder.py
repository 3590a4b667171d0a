"""Random-init Qwen-style decoder for end-to-end semantic-ID beam decode.

The reference serves a Qwen3 checkpoint through vLLM's model executor
(vllm==0.14, not vendored; the semantic-ID tasks use Qwen3 chat templates,
benchmarks/open_one_rec/tasks/recommendation/config.py:19).  This is the
same architecture, sized by a :class:`DecoderConfig`, with weights drawn
from N(0, std) -- there are no checkpoints here:

* token embedding, tied to the lm_head by default;
* per layer: RMSNorm, q/k/v projections (no bias), per-head RMSNorm of q and
  k, rotary embedding with rotate-half pairing (theta 1e6) at the positions
  the caller gives, attention through the BeamAttention backend, o
  projection, residual add; RMSNorm, SwiGLU MLP (silu(gate) * up, down),
  residual add;
* final RMSNorm; logits = lm_head rows in float32.

GEMMs are ``torch.nn.functional.linear`` (hipBLASLt on ROCm).  The
elementwise stages are fused HIP kernels (include/gr_decoder.h): residual add
+ RMSNorm, per-head q/k RMSNorm + rotary + K/V cache write through the slot
mapping, and the SiLU-gated product.  Attention is
:class:`BeamAttentionImpl.forward`, the call vLLM's Attention layer makes
(beam_attn.py:703-755), with the K/V already written (key/value None).
Positions follow the reference's rule (a beam's j-th suffix token sits at prefix_len + j,
engine_core_patch.py:362-365); logits are taken for one row per beam, the
beam's newest token (:367-369).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .. import ops
from .attention.backends.beam_attn import BeamAttentionImpl


@dataclass(frozen=True)
class DecoderConfig:
    num_layers: int = 28
    hidden: int = 2048
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 6144
    vocab: int = 8192
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6
    tie_embeddings: bool = True
    init_std: float = 0.02
    dtype: torch.dtype = torch.bfloat16

    @property
    def q_size(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    def num_params(self) -> int:
        H, L = self.hidden, self.num_layers
        per_layer = (H * (self.q_size + 2 * self.kv_size) + self.q_size * H + 3 * H * self.ffn
                     + 2 * H + 2 * self.head_dim)
        emb = self.vocab * H * (1 if self.tie_embeddings else 2)
        return L * per_layer + emb + H


#: the 28-layer, 2048-hidden, 16/8-head, 6144-FFN, 8192-token decoder
SID_DECODER_1P7B = DecoderConfig()


def init_weights(cfg: DecoderConfig, seed: int, device="cpu") -> dict[str, torch.Tensor]:
    """Weights in nn.Linear layout ``[out, in]``, drawn from one generator on
    ``device`` in a fixed order (embedding, then per layer qkv, o, gate_up,
    down), N(0, init_std) in float32 rounded to ``cfg.dtype``; norm weights
    are ones.  The same seed and device give the same weights."""
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def normal(*shape):
        w = torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)
        return w.mul_(cfg.init_std).to(cfg.dtype)

    ones = lambda n: torch.ones(n, device=dev, dtype=cfg.dtype)
    H = cfg.hidden
    w = {"embed": normal(cfg.vocab, H)}
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        w[p + "qkv"] = normal(cfg.q_size + 2 * cfg.kv_size, H)
        w[p + "o"] = normal(H, cfg.q_size)
        w[p + "gate_up"] = normal(2 * cfg.ffn, H)
        w[p + "down"] = normal(H, cfg.ffn)
        w[p + "input_norm"] = ones(H)
        w[p + "post_norm"] = ones(H)
        w[p + "q_norm"] = ones(cfg.head_dim)
        w[p + "k_norm"] = ones(cfg.head_dim)
    w["final_norm"] = ones(H)
    w["lm_head"] = w["embed"] if cfg.tie_embeddings else normal(cfg.vocab, H)
    return w


class RotaryEmbedding:
    """Tables of the rotate-half rotary embedding: pair (i, i + D/2) turns by
    ``pos * theta^(-2i/D)``; cos/sin ``[max_pos, D/2]`` evaluated in float64
    and stored as float32 on the device (read by gr_qk_norm_rope_cache)."""

    def __init__(self, head_dim: int, theta: float, max_pos: int, device):
        half = head_dim // 2
        inv = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float64) * 2.0 / head_dim))
        ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None]
        self.cos = ang.cos().float().to(device)
        self.sin = ang.sin().float().to(device)
        self.max_pos = max_pos


class SidDecoder:
    """The decoder's forward over a flat batch of tokens.

    ``forward(input_ids, positions, attn_metadata, kv_caches)`` runs every
    layer; ``kv_caches[i]`` is layer i's ``[2, num_blocks, block_size, Hkv,
    D]`` cache and ``attn_metadata`` the backend metadata of the batch (its
    slot mapping says where each token's K/V is written).  Positions lie
    below ``max_position`` (the rotary table's length; the kernel flags and
    skips a token beyond it).  Returns the final normalised hidden states
    ``[T, hidden]``; :meth:`compute_logits` maps selected rows to float32
    logits."""

    def __init__(self, cfg: DecoderConfig, weights: dict[str, torch.Tensor], *, max_position: int = 32768):
        self.cfg = cfg
        self.w = weights
        dev = weights["embed"].device
        self.rope = RotaryEmbedding(cfg.head_dim, cfg.rope_theta, max_position, dev)
        self.layer_names = [f"model.layers.{i}.self_attn.attn" for i in range(cfg.num_layers)]
        self.attn = [BeamAttentionImpl(cfg.num_heads, cfg.head_dim, 1.0 / math.sqrt(cfg.head_dim),
                                       cfg.num_kv_heads, None, None, "auto")
                     for _ in range(cfg.num_layers)]

    @property
    def device(self) -> torch.device:
        return self.w["embed"].device

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, attn_metadata,
                kv_caches) -> torch.Tensor:
        cfg, w, eps = self.cfg, self.w, self.cfg.rms_eps
        T = input_ids.shape[0]
        slots = attn_metadata.slot_mapping if attn_metadata is not None else None
        status = attn_metadata.status if attn_metadata is not None else None
        h = w["embed"][input_ids]  # the residual stream
        x = ops.rms_norm(h, w["layers.0.input_norm"], eps)
        mlp = None
        for i in range(cfg.num_layers):
            p = f"layers.{i}."
            if i:
                x = ops.rms_norm(mlp, w[p + "input_norm"], eps, residual=h, out=x)
            qkv = F.linear(x, w[p + "qkv"])
            k_cache, v_cache = ops.split_kv_cache(kv_caches[i])
            q = ops.qk_norm_rope_cache(qkv, positions, self.rope.cos, self.rope.sin, w[p + "q_norm"],
                                       w[p + "k_norm"], k_cache, v_cache, slots, num_q_heads=cfg.num_heads,
                                       num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim, eps=eps,
                                       status=status)
            attn = torch.empty_like(q)
            self.attn[i].forward(None, q, None, None, kv_caches[i], attn_metadata, output=attn)
            x = ops.rms_norm(F.linear(attn.view(T, cfg.q_size), w[p + "o"]), w[p + "post_norm"], eps,
                             residual=h, out=x)
            mlp = F.linear(ops.silu_mul(F.linear(x, w[p + "gate_up"])), w[p + "down"])
        return ops.rms_norm(mlp, w["final_norm"], eps, residual=h)

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden, self.w["lm_head"]).float()
