"""ctypes binding of libgr_beam.so (declared in include/gr_beam.h and
include/gr_decoder.h).

The library is the product: there is no Python or CPU fallback.  Loading
fails loudly with an ImportError-like RuntimeError when the shared object is
missing, and every entry point's status code is turned into an exception.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libgr_beam.so")

GR_OK = 0
GR_ERR_INVALID_ARG = 1
GR_ERR_UNSUPPORTED = 2
GR_ERR_LAUNCH = 3
GR_ERR_WORKSPACE = 4

GR_DEV_BAD_BLOCK = 1
GR_DEV_BAD_LENGTH = 2
GR_DEV_BAD_PARENT = 4
GR_DEV_SUFFIX_FULL = 8
GR_DEV_BAD_NODE = 16

GR_PRUNE_SCRATCH_BYTES = 16 << 20  # static scratch of gr_beam_prune_topk_noalloc

GR_DTYPE_F32 = 0
GR_DTYPE_F16 = 1
GR_DTYPE_BF16 = 2
GR_DTYPE_FP8_E4M3 = 3  # KV-cache element type only

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t


class AttnOptions(ctypes.Structure):
    """gr_attn_options (include/gr_beam.h)."""
    _fields_ = [("window_left", ctypes.c_int), ("window_right", ctypes.c_int), ("causal", ctypes.c_int),
                ("sinks", ctypes.c_void_p), ("alibi_slopes", ctypes.c_void_p),
                ("kv_dtype", ctypes.c_int), ("k_scale", ctypes.c_void_p), ("v_scale", ctypes.c_void_p)]


# name -> (restype, argtypes); mirrors include/gr_beam.h and include/gr_decoder.h one to one
SIGNATURES = {
    "gr_status_string": (ctypes.c_char_p, [_I]),
    "gr_version": (_I, []),
    "gr_set_decode_kernel": (_I, [_I]),
    "gr_beam_attn_decode": (_I, [
        _P, _L, _P, _L,                 # out, out_tok_stride, q, q_tok_stride
        _P, _P, _L,                     # k_cache, v_cache, num_blocks
        _L, _L, _L,                     # kv block/tok/head strides
        _P, _I, _P,                     # prefix_bt, prefix_bt_stride, prefix_len
        _P,                             # beam_start
        _P, _I, _P, _P,                 # suffix_bt, stride, suffix_len, suffix_start
        _I, _I, _I, _I,                 # num_reqs, max_beams_per_req, num_beams, q_per_beam
        _I, _I, _I, _I, _I,             # Hq, Hkv, head_dim, block_size, dtype
        _F, _F, _P, _P, _P,             # scale, softcap, lse_out, dev_status, stream
    ]),
    "gr_beam_attn_decode_workspace_size": (_SZ, [_I, _I, _I, _I, _I, _I, _I]),
    "gr_beam_attn_decode_ws": (_I, [
        _P, _L, _P, _L, _P, _P, _L, _L, _L, _L, _P, _I, _P, _P, _P, _I, _P, _P,
        _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _F, _P, _P,
        _I, _P, _SZ, _P,                # max_prefix_len, workspace, workspace_bytes, stream
    ]),
    "gr_beam_attn_decode_opt": (_I, [
        _P, _L, _P, _L, _P, _P, _L, _L, _L, _L, _P, _I, _P, _P, _P, _I, _P, _P,
        _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _F, _P, _P,
        _I, _P, _SZ,                    # max_prefix_len, workspace, workspace_bytes
        _P, _P,                         # options (gr_attn_options*), stream
    ]),
    "gr_paged_attn_prefill_opt": (_I, [
        _P, _L, _P, _L, _P, _P, _L, _L, _L, _L, _P, _I, _P, _P, _I, _I, _I,
        _I, _I, _I, _I, _I, _F, _F, _P, _P,
        _P, _P,                         # options (gr_attn_options*), stream
    ]),
    "gr_paged_attn_prefill": (_I, [
        _P, _L, _P, _L,                 # out, out_tok_stride, q, q_tok_stride
        _P, _P, _L,                     # k_cache, v_cache, num_blocks
        _L, _L, _L,                     # kv block/tok/head strides
        _P, _I, _P, _P,                 # block_table, bt_stride, query_start, seq_len
        _I, _I, _I,                     # num_reqs, num_tokens, max_query_len
        _I, _I, _I, _I, _I,             # Hq, Hkv, head_dim, block_size, dtype
        _F, _F, _P, _P, _P,             # scale, softcap, lse_out, dev_status, stream
    ]),
    "gr_rms_norm": (_I, [_P, _L, _P, _L, _P, _L, _P, _I, _I, _F, _I, _P]),
    "gr_qk_norm_rope_cache": (_I, [
        _P, _L, _P, _L, _P,             # q_out, q_out_stride, qkv, qkv_stride, positions
        _P, _P, _L, _P, _P,             # cos, sin, table_len, q_norm, k_norm
        _P, _P, _L, _L, _L, _L,         # k_cache, v_cache, num_blocks, kv strides
        _P, _I, _I,                     # slot_mapping, block_size, num_tokens
        _I, _I, _I, _F, _I, _P, _P,     # Hq, Hkv, head_dim, eps, dtype, dev_status, stream
    ]),
    "gr_silu_mul": (_I, [_P, _L, _P, _L, _I, _I, _I, _P]),
    "gr_reshape_and_cache": (_I, [
        _P, _L, _P, _L, _P, _P, _L, _L, _L, _L, _P, _I, _I, _I, _I, _I, _P, _P,
    ]),
    "gr_reshape_and_cache_fp8": (_I, [
        _P, _L, _P, _L, _P, _P, _L, _L, _L, _L, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P,
    ]),
    "gr_beam_kv_fork": (_I, [
        _P, _I, _I, _P, _P, _P, _P, _I,
        _P, _P, _L, _L, _L, _L,
        _P, _P, _L, _I, _I, _I, _I, _P, _P,
    ]),
    "gr_beam_kv_fork_layers": (_I, [
        _P, _I, _I, _P, _P, _P, _P, _I, _I,   # parent, R, W, bt_in, len_in, bt_out, len_out, bt_stride, layers
        _P, _P, _L, _L, _L, _L,               # k_caches, v_caches (host pointer arrays), num_blocks, strides
        _I, _I, _I, _I, _P, _P,               # heads, head_dim, block_size, dtype, dev_status, stream
    ]),
    "gr_beam_kv_append": (_I, [
        _P, _P, _L, _P, _P, _L, _L, _L, _L, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P,
    ]),
    "gr_beam_prune_workspace_size": (_SZ, [_I, _I, _I, _I]),
    "gr_beam_prune_topk_catalog": (_I, [
        _P, _L, _P, _I, _I, _I, _I, _I,    # logits, stride, cum, R, W, V, k, eos
        _P, _P, _P, _P, _I, _I,            # beam_node, node_start, child_token, child_node, nodes, edges
        _P, _P, _P, _P, _P,                # parent, token, score, eos_score, node_out
        _P, _SZ, _P, _P,                   # workspace, bytes, dev_status, stream
    ]),
    "gr_beam_prune_topk": (_I, [
        _P, _L, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _SZ, _P,
    ]),
    "gr_beam_prune_topk_noalloc": (_I, [
        _P, _L, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P,
    ]),
    "gr_beam_prune_topk_f64": (_I, [
        _P, _L, _P, _I, _I, _I, _I, _I,    # logits, stride, cum (float64), R, W, V, k, eos
        _P, _P, _P, _P, _I, _I,            # beam_node (nullable), node_start, child_token, child_node, nodes, edges
        _P, _P, _P, _P, _P,                # parent, token, score, eos_score (float64), node_out
        _P, _P,                            # cand_token, cand_logprob (nullable)
        _P, _SZ, _P, _P,                   # workspace, bytes, dev_status, stream
    ]),
}

_lib = None


class GrError(RuntimeError):
    """A library call returned a non-OK status."""

    def __init__(self, fn: str, code: int):
        self.code = code
        super().__init__(f"{fn}: {status_string(code)} (status {code})")


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libgr_beam.so not found at {LIB_PATH}; build it with "
                "`python vllm-gr-ehaleva_amd/build.py` (there is no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def status_string(code: int) -> str:
    return lib().gr_status_string(code).decode()


def check(fn: str, code: int) -> None:
    if code == GR_ERR_INVALID_ARG:
        raise ValueError(f"{fn}: {status_string(code)}")
    if code == GR_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{fn}: {status_string(code)}")
    if code != GR_OK:
        raise GrError(fn, code)
