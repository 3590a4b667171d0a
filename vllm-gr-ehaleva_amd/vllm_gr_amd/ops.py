"""torch-tensor entry points over the C ABI (include/gr_beam.h,
include/gr_decoder.h).

Each function validates shapes/devices on the host, allocates outputs with
the torch caching allocator when the caller passes none, and launches on
``torch.cuda.current_stream()``.  Nothing here computes on the CPU: without
the HIP library every call raises.
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from . import _C

_DTYPES = {torch.float32: _C.GR_DTYPE_F32, torch.float16: _C.GR_DTYPE_F16,
           torch.bfloat16: _C.GR_DTYPE_BF16}
# KV-cache element types: an fp8 e4m3 cache as float8_e4m3fn, or as the raw
# bytes (uint8) the engine allocates it as
_FP8_CACHE = (torch.float8_e4m3fn, torch.uint8)


def is_fp8_cache(t: torch.Tensor) -> bool:
    return t.dtype in _FP8_CACHE


def _cache_dtype_code(t: torch.Tensor) -> int:
    return _C.GR_DTYPE_FP8_E4M3 if is_fp8_cache(t) else _dtype_code(t)


def _scale_arg(name: str, t: torch.Tensor | None, dev) -> int | None:
    if t is not None and (t.device != dev or t.dtype != torch.float32 or t.numel() != 1):
        raise ValueError(f"{name} must be a one-element float32 tensor on the cache's device")
    return _ptr(t)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise NotImplementedError(f"unsupported dtype {t.dtype}") from None


def _need_cuda(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("all tensors must be on a HIP device (torch 'cuda')")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def _need_i32(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor")


def _cache_strides(k_cache: torch.Tensor, v_cache: torch.Tensor):
    """(num_blocks, block_size, Hkv, D) views -> element strides."""
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache / v_cache must be matching [num_blocks, block_size, Hkv, D] views")
    if k_cache.stride(3) != 1:
        raise ValueError("head_dim must be contiguous in the KV cache")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache / v_cache dtype mismatch")
    return k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)


def split_kv_cache(kv_cache: torch.Tensor):
    """``kv_cache [2, num_blocks, block_size, Hkv, D]`` -> (k_cache, v_cache),
    the ``kv_cache.unbind(0)`` of ``beam_attn.py:725``."""
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2:
        raise ValueError("kv_cache must be [2, num_blocks, block_size, num_kv_heads, head_dim]")
    return kv_cache[0], kv_cache[1]


def new_status(device) -> torch.Tensor:
    """Device status word the kernels OR error bits into."""
    return torch.zeros(1, dtype=torch.int32, device=device)


def check_status(status: torch.Tensor) -> None:
    """Raise if a kernel flagged an out-of-range table entry (synchronises)."""
    bits = int(status.item())
    if bits:
        names = [n for b, n in ((_C.GR_DEV_BAD_BLOCK, "block id out of range"),
                                (_C.GR_DEV_BAD_LENGTH, "length beyond table capacity"),
                                (_C.GR_DEV_BAD_PARENT, "parent index out of range"),
                                (_C.GR_DEV_SUFFIX_FULL, "suffix full"),
                                (_C.GR_DEV_BAD_NODE, "catalog node out of range")) if bits & b]
        raise ValueError("device tables rejected: " + ", ".join(names))


def set_decode_kernel(which: str) -> None:
    """'auto' (the matrix-core kernel where supported) or 'generic'."""
    code = {"auto": 0, "generic": 1}[which]
    _C.check("gr_set_decode_kernel", _C.lib().gr_set_decode_kernel(code))


def beam_attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     prefix_bt: torch.Tensor, prefix_len: torch.Tensor, beam_start: torch.Tensor,
                     suffix_bt: torch.Tensor, suffix_len: torch.Tensor,
                     suffix_start: torch.Tensor | None = None, *, q_per_beam: int = 1,
                     scale: float, softcap: float = 0.0, max_beams_per_req: int | None = None,
                     out: torch.Tensor | None = None, lse: torch.Tensor | None = None,
                     status: torch.Tensor | None = None, max_prefix_len: int | None = None,
                     split: bool = True, window: tuple[int, int] | None = None,
                     sinks: torch.Tensor | None = None,
                     alibi_slopes: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
                     v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """BeamAttention decode step; see ``gr_beam_attn_decode`` / ``_ws`` / ``_opt``
    in gr_beam.h.  ``window`` (left, right), ``sinks`` and ``alibi_slopes``
    are the optional features of ``gr_attn_options``; an fp8 e4m3 cache
    (float8_e4m3fn or uint8) is read as ``e4m3 * k_scale`` / ``* v_scale``
    (one-element float32 device tensors, None for 1.0).

    ``q``: ``[num_beams*q_per_beam, Hq, D]`` (token stride free, heads and dims
    contiguous).  Returns ``out`` (same shape/dtype as ``q``).  With ``split``
    a small batch spreads each tile's prefix over several workgroups (a
    per-device workspace is kept for it); ``max_prefix_len`` (host hint) is
    the longest prefix, 0 or None when unknown."""
    dev = _need_cuda(q, k_cache, v_cache, prefix_bt, prefix_len, beam_start, suffix_bt, suffix_len,
                     suffix_start, out, lse, status)
    if q.dim() != 3 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("q must be [tokens, Hq, D] with heads and dims contiguous")
    for name, t in (("prefix_bt", prefix_bt), ("prefix_len", prefix_len), ("beam_start", beam_start),
                    ("suffix_bt", suffix_bt), ("suffix_len", suffix_len)):
        _need_i32(name, t)
    if suffix_start is not None:
        _need_i32("suffix_start", suffix_start)
    kv8 = is_fp8_cache(k_cache)
    if q.dtype != k_cache.dtype and not kv8:
        raise ValueError("q and KV cache dtype must match")
    NT, Hq, D = q.shape
    NB, bs, Hkv, Dk = k_cache.shape
    if Dk != D:
        raise ValueError("head_dim mismatch between q and KV cache")
    R = prefix_len.numel()
    if prefix_bt.dim() != 2 or prefix_bt.shape[0] != R or beam_start.numel() != R + 1:
        raise ValueError("prefix_bt must be [R, blocks], beam_start [R+1]")
    N = suffix_len.numel()
    if suffix_bt.dim() != 2 or suffix_bt.shape[0] != N or NT != N * q_per_beam:
        raise ValueError("suffix_bt must be [N, blocks] and q must hold N*q_per_beam rows")
    if suffix_start is not None and suffix_start.numel() != N:
        raise ValueError("suffix_start must have one entry per beam")
    if max_beams_per_req is None:
        max_beams_per_req = int((beam_start[1:] - beam_start[:-1]).max().item()) if R else 0
    bstr, tstr, hstr = _cache_strides(k_cache, v_cache)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1 or out.stride(1) != D:
        raise ValueError("out must match q's shape/dtype with heads and dims contiguous")
    if lse is not None and (lse.shape != (NT, Hq) or lse.dtype != torch.float32 or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous float32 [tokens, Hq] tensor")
    args = (out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0),
            k_cache.data_ptr(), v_cache.data_ptr(), NB, bstr, tstr, hstr,
            prefix_bt.data_ptr(), prefix_bt.shape[1], prefix_len.data_ptr(), beam_start.data_ptr(),
            suffix_bt.data_ptr(), suffix_bt.shape[1], suffix_len.data_ptr(), _ptr(suffix_start),
            R, max_beams_per_req, N, q_per_beam, Hq, Hkv, D, bs, _dtype_code(q),
            float(scale), float(softcap or 0.0), _ptr(lse), _ptr(status))
    hint = int(max_prefix_len or 0)
    opt = _attn_options(dev, Hq, window, True, sinks, alibi_slopes, kv8, k_scale, v_scale)
    ws_bytes = (_C.lib().gr_beam_attn_decode_workspace_size(R, max_beams_per_req, q_per_beam, Hq, Hkv, D, hint)
                if split and R else 0)
    if opt is not None:
        # windows and sinks run on the matrix-core kernel, split like a plain
        # decode; without split, a prefix hint below one split's minimum (256
        # keys) plans none
        ws = _split_workspace(dev, ws_bytes) if ws_bytes else None
        code = _C.lib().gr_beam_attn_decode_opt(*args, hint if split else 1, _ptr(ws), ws_bytes,
                                                ctypes.byref(opt), _stream(dev))
        _C.check("gr_beam_attn_decode_opt", code)
        return out
    if ws_bytes:
        ws = _split_workspace(dev, ws_bytes)
        code = _C.lib().gr_beam_attn_decode_ws(*args, hint, ws.data_ptr(), ws_bytes, _stream(dev))
        _C.check("gr_beam_attn_decode_ws", code)
    else:
        code = _C.lib().gr_beam_attn_decode(*args, _stream(dev))
        _C.check("gr_beam_attn_decode", code)
    return out


def _attn_options(dev, Hq: int, window, causal: bool, sinks, alibi_slopes, kv8: bool = False, k_scale=None,
                  v_scale=None):
    """The gr_attn_options struct for the optional features, or None when
    none is set.  ``window`` = (left, right), -1 = unbounded; ``sinks`` /
    ``alibi_slopes``: float32 [Hq] device tensors; ``kv8``: an fp8 e4m3
    cache with its scales."""
    left, right = (-1, -1) if window is None else (int(window[0]), int(window[1]))
    if left < -1 or right < -1:
        raise ValueError("window bounds must be >= -1")
    for name, t in (("sinks", sinks), ("alibi_slopes", alibi_slopes)):
        if t is not None and (t.device != dev or t.dtype != torch.float32 or t.shape != (Hq,)
                              or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous float32 [Hq] tensor on the query's device")
    ks, vs = _scale_arg("k_scale", k_scale, dev), _scale_arg("v_scale", v_scale, dev)
    if left < 0 and right < 0 and causal and sinks is None and alibi_slopes is None and not kv8:
        return None
    return _C.AttnOptions(left, right, 1 if causal else 0, _ptr(sinks), _ptr(alibi_slopes),
                          _C.GR_DTYPE_FP8_E4M3 if kv8 else -1, ks if kv8 else None, vs if kv8 else None)


_SPLIT_WS: dict = {}
_SPLIT_WS_RETIRED: list = []


def _split_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device workspace of the split decode (partials only, no initial
    contents); launches on one stream share it in order.  A workspace that is
    outgrown stays allocated: a captured graph may still name it."""
    ws = _SPLIT_WS.get(dev)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _SPLIT_WS_RETIRED.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _SPLIT_WS[dev] = ws
    return ws


def paged_attn_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       block_table: torch.Tensor, query_start: torch.Tensor, seq_len: torch.Tensor, *,
                       max_query_len: int, scale: float, softcap: float = 0.0,
                       out: torch.Tensor | None = None, lse: torch.Tensor | None = None,
                       status: torch.Tensor | None = None, causal: bool = True,
                       window: tuple[int, int] | None = None, sinks: torch.Tensor | None = None,
                       alibi_slopes: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
                       v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Varlen attention of standard requests over the paged cache (causal, or
    over every key of the sequence with ``causal=False``); see
    ``gr_paged_attn_prefill`` / ``_opt`` in gr_beam.h.  ``q``: ``[num_tokens, Hq, D]``,
    ``block_table [R, blocks]``, ``query_start [R+1]``, ``seq_len [R]`` int32.
    ``max_query_len`` must bound every request's query count (it sizes the
    grid; a request above it is flagged and skipped)."""
    dev = _need_cuda(q, k_cache, v_cache, block_table, query_start, seq_len, out, lse, status)
    if q.dim() != 3 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("q must be [tokens, Hq, D] with heads and dims contiguous")
    for name, t in (("block_table", block_table), ("query_start", query_start), ("seq_len", seq_len)):
        _need_i32(name, t)
    kv8 = is_fp8_cache(k_cache)
    if q.dtype != k_cache.dtype and not kv8:
        raise ValueError("q and KV cache dtype must match")
    NT, Hq, D = q.shape
    NB, bs, Hkv, Dk = k_cache.shape
    if Dk != D:
        raise ValueError("head_dim mismatch between q and KV cache")
    R = seq_len.numel()
    if block_table.dim() != 2 or block_table.shape[0] != R or query_start.numel() != R + 1:
        raise ValueError("block_table must be [R, blocks] and query_start [R+1]")
    bstr, tstr, hstr = _cache_strides(k_cache, v_cache)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1 or out.stride(1) != D:
        raise ValueError("out must match q's shape/dtype with heads and dims contiguous")
    if lse is not None and (lse.shape != (NT, Hq) or lse.dtype != torch.float32 or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous float32 [tokens, Hq] tensor")
    args = (out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0),
            k_cache.data_ptr(), v_cache.data_ptr(), NB, bstr, tstr, hstr,
            block_table.data_ptr(), block_table.shape[1], query_start.data_ptr(), seq_len.data_ptr(),
            R, NT, int(max_query_len), Hq, Hkv, D, bs, _dtype_code(q), float(scale), float(softcap or 0.0),
            _ptr(lse), _ptr(status))
    opt = _attn_options(dev, Hq, window, causal, sinks, alibi_slopes, kv8, k_scale, v_scale)
    if opt is not None:
        code = _C.lib().gr_paged_attn_prefill_opt(*args, ctypes.byref(opt), _stream(dev))
        _C.check("gr_paged_attn_prefill_opt", code)
    else:
        code = _C.lib().gr_paged_attn_prefill(*args, _stream(dev))
        _C.check("gr_paged_attn_prefill", code)
    return out


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                      status: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
                      v_scale: torch.Tensor | None = None) -> None:
    """Scatter ``key/value [T, Hkv, D]`` into the paged cache by slot (the
    ``reshape_and_cache_flash`` role, ``beam_attn.py:727-732``).  Into an fp8
    e4m3 cache each element is stored as e4m3(clamp(x / scale, -448, 448))
    (``k_scale`` / ``v_scale``: one-element float32 tensors, None for 1.0)."""
    dev = _need_cuda(key, value, k_cache, v_cache, slot_mapping, status)
    if slot_mapping.dtype != torch.int64 or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be a contiguous int64 tensor")
    T, Hkv, D = key.shape
    if value.shape != key.shape or key.stride(2) != 1 or key.stride(1) != D or value.stride(2) != 1 \
            or value.stride(1) != D:
        raise ValueError("key/value must be [T, Hkv, D] with heads and dims contiguous")
    if slot_mapping.numel() < T:
        raise ValueError("slot_mapping shorter than the number of tokens")
    NB, bs, Hk, Dk = k_cache.shape
    kv8 = is_fp8_cache(k_cache)
    if (Hk, Dk) != (Hkv, D) or value.dtype != key.dtype or (key.dtype != k_cache.dtype and not kv8):
        raise ValueError("key/value do not match the KV cache")
    bstr, tstr, hstr = _cache_strides(k_cache, v_cache)
    if kv8:
        code = _C.lib().gr_reshape_and_cache_fp8(
            key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(),
            v_cache.data_ptr(), NB, bstr, tstr, hstr, slot_mapping.data_ptr(), T, Hkv, D, bs,
            _dtype_code(key), _scale_arg("k_scale", k_scale, dev), _scale_arg("v_scale", v_scale, dev),
            _ptr(status), _stream(dev))
        _C.check("gr_reshape_and_cache_fp8", code)
        return
    code = _C.lib().gr_reshape_and_cache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(),
        v_cache.data_ptr(), NB, bstr, tstr, hstr, slot_mapping.data_ptr(), T, Hkv, D, bs,
        _dtype_code(key), _ptr(status), _stream(dev))
    _C.check("gr_reshape_and_cache", code)


class _LayerSet:
    """Validated per-layer K/V base pointers of one list of caches (every
    layer one geometry), as the host pointer arrays gr_beam_kv_fork_layers
    takes.  It holds addresses and geometry only, never the tensors: a cache
    list that is dropped is freed, and an entry whose caches died is evicted
    on the next lookup (``alive``)."""

    def __init__(self, kv_caches):
        pairs = [split_kv_cache(kv) if isinstance(kv, torch.Tensor) else tuple(kv) for kv in kv_caches]
        k0, v0 = pairs[0]
        self.strides = _cache_strides(k0, v0)
        for k, v in pairs:
            if k.shape != k0.shape or v.shape != k0.shape or k.dtype != k0.dtype or v.dtype != k0.dtype:
                raise ValueError("every layer's cache must have the same shape and dtype")
            if _cache_strides(k, v) != self.strides or k.device != k0.device or v.device != k0.device:
                raise ValueError("every layer's cache must have the same strides and device")
        self.shape = tuple(k0.shape)
        self.device = k0.device
        self.n = len(pairs)
        self.dtype_code = _cache_dtype_code(k0)
        self._k = (ctypes.c_void_p * self.n)(*[k.data_ptr() for k, _ in pairs])
        self._v = (ctypes.c_void_p * self.n)(*[v.data_ptr() for _, v in pairs])
        self.k_ptrs = ctypes.cast(self._k, ctypes.c_void_p)
        self.v_ptrs = ctypes.cast(self._v, ctypes.c_void_p)
        # weak references to the caller's tensors: the entry is valid while they live
        self._refs = [weakref.ref(t) for kv in kv_caches for t in ((kv,) if isinstance(kv, torch.Tensor) else kv)]

    def alive(self) -> bool:
        return all(r() is not None for r in self._refs)


_LAYER_SETS: dict = {}


def _layer_set(kv_caches) -> _LayerSet:
    """The _LayerSet of a list of caches, built once per distinct list (keyed
    by every cache's address, shape, strides and dtype).  Entries hold no
    tensor: those whose caches were freed are dropped here."""
    def sig(kv):
        t = kv if isinstance(kv, torch.Tensor) else kv[0]
        return (t.data_ptr(), tuple(t.shape), t.stride(), t.dtype, isinstance(kv, torch.Tensor),
                None if isinstance(kv, torch.Tensor) else kv[1].data_ptr())
    for k in [k for k, ls in _LAYER_SETS.items() if not ls.alive()]:
        del _LAYER_SETS[k]
    key = tuple(sig(kv) for kv in kv_caches)
    ls = _LAYER_SETS.get(key)
    if ls is None:
        ls = _LayerSet(list(kv_caches))
        if len(_LAYER_SETS) >= 8:
            _LAYER_SETS.pop(next(iter(_LAYER_SETS)))
        _LAYER_SETS[key] = ls
    return ls


def beam_kv_fork_layers(parent: torch.Tensor, bt_in: torch.Tensor, len_in: torch.Tensor, kv_caches, *,
                        bt_out: torch.Tensor | None = None, len_out: torch.Tensor | None = None,
                        status: torch.Tensor | None = None):
    """``beam_kv_fork`` of every layer's cache in one launch (no appended
    token).  ``kv_caches``: a list of per-layer ``[2, NB, bs, Hkv, D]`` caches
    (or of (k_cache, v_cache) pairs) with one geometry.  Returns (bt_out,
    len_out)."""
    kv_caches = list(kv_caches)
    if not kv_caches:
        raise ValueError("kv_caches is empty")
    ls = _layer_set(kv_caches)
    dev = _need_cuda(parent, bt_in, len_in, kv_caches[0] if isinstance(kv_caches[0], torch.Tensor)
                     else kv_caches[0][0], bt_out, len_out, status)
    _need_i32("parent", parent)
    _need_i32("bt_in", bt_in)
    _need_i32("len_in", len_in)
    if parent.dim() != 2:
        raise ValueError("parent must be [R, W]")
    R, W = parent.shape
    if bt_in.dim() != 2 or bt_in.shape[0] != R * W or len_in.numel() != R * W:
        raise ValueError("bt_in must be [R*W, blocks] and len_in [R*W]")
    NB, bs, Hkv, D = ls.shape
    if bt_out is None:
        bt_out = torch.empty_like(bt_in)
    if len_out is None:
        len_out = torch.empty_like(len_in)
    _need_i32("bt_out", bt_out)
    _need_i32("len_out", len_out)
    if bt_out.shape != bt_in.shape or len_out.shape != len_in.shape:
        raise ValueError("output tables must match the input tables' shapes")
    code = _C.lib().gr_beam_kv_fork_layers(
        parent.data_ptr(), R, W, bt_in.data_ptr(), len_in.data_ptr(), bt_out.data_ptr(), len_out.data_ptr(),
        bt_in.shape[1], ls.n, ls.k_ptrs, ls.v_ptrs, NB, *ls.strides, Hkv, D, bs, ls.dtype_code, _ptr(status),
        _stream(dev))
    _C.check("gr_beam_kv_fork_layers", code)
    return bt_out, len_out


def beam_kv_fork(parent: torch.Tensor, bt_in: torch.Tensor, len_in: torch.Tensor,
                 k_cache: torch.Tensor, v_cache: torch.Tensor, k_new: torch.Tensor | None = None,
                 v_new: torch.Tensor | None = None, *, bt_out: torch.Tensor | None = None,
                 len_out: torch.Tensor | None = None, status: torch.Tensor | None = None):
    """Fork each request's beams by ``parent [R, W]`` (copy-on-write suffix
    rows) and optionally append one token per child.  Returns (bt_out, len_out)."""
    dev = _need_cuda(parent, bt_in, len_in, k_cache, v_cache, k_new, v_new, bt_out, len_out, status)
    _need_i32("parent", parent)
    _need_i32("bt_in", bt_in)
    _need_i32("len_in", len_in)
    if parent.dim() != 2:
        raise ValueError("parent must be [R, W]")
    R, W = parent.shape
    if bt_in.dim() != 2 or bt_in.shape[0] != R * W or len_in.numel() != R * W:
        raise ValueError("bt_in must be [R*W, blocks] and len_in [R*W]")
    NB, bs, Hkv, D = k_cache.shape
    bstr, tstr, hstr = _cache_strides(k_cache, v_cache)
    if bt_out is None:
        bt_out = torch.empty_like(bt_in)
    if len_out is None:
        len_out = torch.empty_like(len_in)
    _need_i32("bt_out", bt_out)
    _need_i32("len_out", len_out)
    if bt_out.shape != bt_in.shape or len_out.shape != len_in.shape:
        raise ValueError("output tables must match the input tables' shapes")
    new_stride = 0
    if k_new is not None or v_new is not None:
        if k_new is None or v_new is None or k_new.shape != (R * W, Hkv, D) or v_new.shape != k_new.shape:
            raise ValueError("k_new/v_new must both be [R*W, Hkv, D]")
        if k_new.dtype != k_cache.dtype or v_new.dtype != k_cache.dtype:
            raise ValueError("k_new/v_new dtype must match the cache")
        if k_new.stride(2) != 1 or k_new.stride(1) != D or v_new.stride() != k_new.stride():
            raise ValueError("k_new/v_new must have heads and dims contiguous and equal strides")
        new_stride = k_new.stride(0)
    code = _C.lib().gr_beam_kv_fork(
        parent.data_ptr(), R, W, bt_in.data_ptr(), len_in.data_ptr(), bt_out.data_ptr(),
        len_out.data_ptr(), bt_in.shape[1], k_cache.data_ptr(), v_cache.data_ptr(), NB, bstr, tstr,
        hstr, _ptr(k_new), _ptr(v_new), new_stride, Hkv, D, bs, _cache_dtype_code(k_cache), _ptr(status),
        _stream(dev))
    _C.check("gr_beam_kv_fork", code)
    return bt_out, len_out


def beam_kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                   v_cache: torch.Tensor, suffix_bt: torch.Tensor, suffix_len: torch.Tensor,
                   status: torch.Tensor | None = None) -> None:
    """Append one token per beam at ``suffix_len[n]``; ``suffix_len`` += 1 in place."""
    dev = _need_cuda(k_new, v_new, k_cache, v_cache, suffix_bt, suffix_len, status)
    _need_i32("suffix_bt", suffix_bt)
    _need_i32("suffix_len", suffix_len)
    N = suffix_len.numel()
    NB, bs, Hkv, D = k_cache.shape
    if k_new.shape != (N, Hkv, D) or v_new.shape != k_new.shape or suffix_bt.shape[0] != N:
        raise ValueError("k_new/v_new must be [N, Hkv, D] with N = len(suffix_len) = suffix_bt rows")
    if k_new.stride(2) != 1 or k_new.stride(1) != D or v_new.stride() != k_new.stride():
        raise ValueError("k_new/v_new must have heads and dims contiguous and equal strides")
    bstr, tstr, hstr = _cache_strides(k_cache, v_cache)
    code = _C.lib().gr_beam_kv_append(
        k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
        NB, bstr, tstr, hstr, suffix_bt.data_ptr(), suffix_bt.shape[1], suffix_len.data_ptr(), N,
        Hkv, D, bs, _cache_dtype_code(k_cache), _ptr(status), _stream(dev))
    _C.check("gr_beam_kv_append", code)


def prune_workspace_bytes(num_reqs: int, beam_width: int, vocab: int, k: int) -> int:
    return int(_C.lib().gr_beam_prune_workspace_size(num_reqs, beam_width, vocab, k))


def beam_prune_topk(logits: torch.Tensor, cum: torch.Tensor, k: int, eos_token_id: int = -1, *,
                    workspace: torch.Tensor | None = None, out=None, catalog=None,
                    beam_node: torch.Tensor | None = None, node_out: torch.Tensor | None = None,
                    status: torch.Tensor | None = None, candidates: bool = False):
    """Fused log_softmax + cum + top-k over beams x vocab per request.

    ``logits``: ``[R, W, V]`` float32 (vocab contiguous), ``cum``: ``[R, W]``
    float32 or float64.  Returns ``(parent [R,k] int32, token [R,k] int32,
    score [R,k], eos_score [R,W])``, the scores in ``cum``'s dtype: a float64
    ``cum`` runs gr_beam_prune_topk_f64, which carries the beam scores in
    float64 as the reference does between steps (serving_engine.py:511,
    :538-539).  With ``catalog`` (a
    :class:`~vllm_gr_amd.entrypoints.catalog.CatalogTensors`) and ``beam_node
    [R, W]`` int32, candidates outside each beam's trie node are dropped and
    ``node_out [R, k]`` is appended to the result.  ``candidates=True``
    (float64 ``cum`` only) appends each beam's top-k list before EOS/catalog
    removal: ``cand_token [R, W, k]`` int32 and ``cand_logprob [R, W, k]``
    float32 (logit - lse), the per-step logprob lists of the reference's
    beam search (vllm_gr/logprobs.py:34-85)."""
    dev = _need_cuda(logits, cum, workspace, beam_node, node_out, status)
    if logits.dim() != 3 or logits.dtype != torch.float32 or logits.stride(2) != 1 \
            or logits.stride(0) != logits.shape[1] * logits.stride(1):
        raise ValueError("logits must be float32 [R, W, V] with rows at a uniform stride")
    R, W, V = logits.shape
    f64 = cum.dtype == torch.float64
    if cum.shape != (R, W) or cum.dtype not in (torch.float32, torch.float64) or not cum.is_contiguous():
        raise ValueError("cum must be a contiguous float32 or float64 [R, W] tensor")
    if candidates and not f64:
        raise ValueError("candidates=True needs a float64 cum (gr_beam_prune_topk_f64)")
    need = prune_workspace_bytes(R, W, V, k)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    sdt = cum.dtype
    if out is None:
        parent = torch.empty((R, k), dtype=torch.int32, device=dev)
        token = torch.empty((R, k), dtype=torch.int32, device=dev)
        score = torch.empty((R, k), dtype=sdt, device=dev)
        eos_score = torch.empty((R, W), dtype=sdt, device=dev)
    else:
        parent, token, score, eos_score = out
        if score.dtype != sdt or eos_score.dtype != sdt:
            raise ValueError("score / eos_score must have cum's dtype")
    ws_bytes = workspace.numel() * workspace.element_size()
    if catalog is not None:
        _need_cuda(catalog.node_start, catalog.child_token, catalog.child_node)
        for name, t in (("node_start", catalog.node_start), ("child_token", catalog.child_token),
                        ("child_node", catalog.child_node)):
            _need_i32(name, t)
        if beam_node is None or beam_node.shape != (R, W):
            raise ValueError("beam_node must be an int32 [R, W] tensor")
        _need_i32("beam_node", beam_node)
        if node_out is None:
            node_out = torch.empty((R, k), dtype=torch.int32, device=dev)
        if node_out.shape != (R, k):
            raise ValueError("node_out must be [R, k]")
        _need_i32("node_out", node_out)
        trie = (beam_node.data_ptr(), catalog.node_start.data_ptr(),
                _ptr(catalog.child_token if catalog.num_edges else None),
                _ptr(catalog.child_node if catalog.num_edges else None), catalog.num_nodes, catalog.num_edges)
    if f64:
        cand_tok = cand_lp = None
        if candidates:
            cand_tok = torch.empty((R, W, k), dtype=torch.int32, device=dev)
            cand_lp = torch.empty((R, W, k), dtype=torch.float32, device=dev)
        if catalog is None:
            trie = (None, None, None, None, 0, 0)
        code = _C.lib().gr_beam_prune_topk_f64(
            logits.data_ptr(), logits.stride(1), cum.data_ptr(), R, W, V, int(k), int(eos_token_id), *trie,
            parent.data_ptr(), token.data_ptr(), score.data_ptr(), eos_score.data_ptr(), _ptr(node_out),
            _ptr(cand_tok), _ptr(cand_lp), workspace.data_ptr(), ws_bytes, _ptr(status), _stream(dev))
        _C.check("gr_beam_prune_topk_f64", code)
        res = (parent, token, score, eos_score) + ((node_out,) if catalog is not None else ())
        return res + ((cand_tok, cand_lp) if candidates else ())
    if catalog is None:
        code = _C.lib().gr_beam_prune_topk(
            logits.data_ptr(), logits.stride(1), cum.data_ptr(), R, W, V, int(k), int(eos_token_id),
            parent.data_ptr(), token.data_ptr(), score.data_ptr(), eos_score.data_ptr(),
            workspace.data_ptr(), ws_bytes, _stream(dev))
        _C.check("gr_beam_prune_topk", code)
        return parent, token, score, eos_score
    code = _C.lib().gr_beam_prune_topk_catalog(
        logits.data_ptr(), logits.stride(1), cum.data_ptr(), R, W, V, int(k), int(eos_token_id), *trie,
        parent.data_ptr(), token.data_ptr(), score.data_ptr(), eos_score.data_ptr(), node_out.data_ptr(),
        workspace.data_ptr(), ws_bytes, _ptr(status), _stream(dev))
    _C.check("gr_beam_prune_topk_catalog", code)
    return parent, token, score, eos_score, node_out


def beam_prune_topk_noalloc(logits: torch.Tensor, cum: torch.Tensor, k: int, eos_token_id: int = -1, *,
                            out):
    """``beam_prune_topk`` (float32 scores, no catalog) through
    gr_beam_prune_topk_noalloc: the library's static per-GPU scratch replaces
    the workspace, so the call allocates nothing -- ``out`` = ``(parent [R,k]
    int32, token [R,k] int32, score [R,k] float32, eos_score [R,W] float32)``
    must be given.  Calls that may overlap on one GPU race on the scratch."""
    dev = _need_cuda(logits, cum, *out)
    if logits.dim() != 3 or logits.dtype != torch.float32 or logits.stride(2) != 1 \
            or logits.stride(0) != logits.shape[1] * logits.stride(1):
        raise ValueError("logits must be float32 [R, W, V] with rows at a uniform stride")
    R, W, V = logits.shape
    if cum.shape != (R, W) or cum.dtype != torch.float32 or not cum.is_contiguous():
        raise ValueError("cum must be a contiguous float32 [R, W] tensor")
    parent, token, score, eos_score = out
    if parent.shape != (R, k) or token.shape != (R, k) or score.shape != (R, k) or eos_score.shape != (R, W):
        raise ValueError("out must be (parent [R,k], token [R,k], score [R,k], eos_score [R,W])")
    need = prune_workspace_bytes(R, W, V, k)
    if need > _C.GR_PRUNE_SCRATCH_BYTES:
        raise ValueError(f"gr_beam_prune_topk_noalloc: this call needs {need} bytes of scratch; the static "
                         f"scratch holds {_C.GR_PRUNE_SCRATCH_BYTES} (use beam_prune_topk with a workspace)")
    code = _C.lib().gr_beam_prune_topk_noalloc(
        logits.data_ptr(), logits.stride(1), cum.data_ptr(), R, W, V, int(k), int(eos_token_id),
        parent.data_ptr(), token.data_ptr(), score.data_ptr(), eos_score.data_ptr(), _stream(dev))
    _C.check("gr_beam_prune_topk_noalloc", code)
    return parent, token, score, eos_score


# ---- fused decoder stages (include/gr_decoder.h) ---------------------------


def _rows(name: str, t: torch.Tensor) -> None:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a [tokens, features] tensor with contiguous features")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """``out = RMSNorm(x [+ residual]) * weight``; with ``residual`` the sum is
    also written back into it (vLLM's fused_add_rms_norm).  ``x [T, H]``."""
    dev = _need_cuda(x, weight, residual, out)
    _rows("x", x)
    T, H = x.shape
    if weight.shape != (H,) or not weight.is_contiguous() or weight.dtype != x.dtype:
        raise ValueError("weight must be a contiguous [hidden] tensor of x's dtype")
    if residual is not None:
        _rows("residual", residual)
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match x")
    if out is None:
        out = torch.empty((T, H), dtype=x.dtype, device=x.device)
    _rows("out", out)
    if out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("out must match x")
    code = _C.lib().gr_rms_norm(out.data_ptr(), out.stride(0), x.data_ptr(), x.stride(0), _ptr(residual),
                                0 if residual is None else residual.stride(0), weight.data_ptr(), T, H,
                                float(eps), _dtype_code(x), _stream(dev))
    _C.check("gr_rms_norm", code)
    return out


def qk_norm_rope_cache(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       q_norm: torch.Tensor | None, k_norm: torch.Tensor | None, k_cache: torch.Tensor | None,
                       v_cache: torch.Tensor | None, slot_mapping: torch.Tensor | None, *, num_q_heads: int,
                       num_kv_heads: int, head_dim: int, eps: float, q_out: torch.Tensor | None = None,
                       status: torch.Tensor | None = None) -> torch.Tensor:
    """Per-head q/k RMSNorm + rotate-half rotary at ``positions`` (int64)
    with the ``cos``/``sin`` tables ``[max_pos, head_dim/2]`` float32;
    rotated keys and the values are written to the cache at ``slot_mapping``.
    ``qkv [T, (Hq + 2 Hkv) * D]``.  Returns the rotated queries ``[T, Hq, D]``."""
    dev = _need_cuda(qkv, positions, cos, sin, q_norm, k_norm, k_cache, v_cache, slot_mapping, q_out, status)
    _rows("qkv", qkv)
    T = qkv.shape[0]
    Hq, Hkv, D = num_q_heads, num_kv_heads, head_dim
    if qkv.shape[1] != (Hq + 2 * Hkv) * D:
        raise ValueError("qkv must hold Hq + 2*Hkv heads of head_dim per token")
    if positions.dtype != torch.int64 or not positions.is_contiguous() or positions.numel() != T:
        raise ValueError("positions must be a contiguous int64 [tokens] tensor")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.dim() != 2 or t.shape[1] != D // 2:
            raise ValueError(f"{name} must be a contiguous float32 [max_pos, head_dim/2] table")
    if cos.shape != sin.shape:
        raise ValueError("cos and sin tables differ in shape")
    for name, t in (("q_norm", q_norm), ("k_norm", k_norm)):
        if t is not None and (t.shape != (D,) or not t.is_contiguous() or t.dtype != qkv.dtype):
            raise ValueError(f"{name} must be a contiguous [head_dim] tensor of qkv's dtype")
    NB = bstr = tstr = hstr = bs = 0
    if slot_mapping is not None:
        if slot_mapping.dtype != torch.int64 or not slot_mapping.is_contiguous() or slot_mapping.numel() < T:
            raise ValueError("slot_mapping must be a contiguous int64 tensor covering the tokens")
        if k_cache is None or v_cache is None or k_cache.dtype != qkv.dtype:
            raise ValueError("the KV cache (of qkv's dtype) is needed with a slot mapping")
        NB, bs, Hc, Dc = k_cache.shape
        if (Hc, Dc) != (Hkv, D):
            raise ValueError("KV cache heads / head_dim do not match")
        bstr, tstr, hstr = _cache_strides(k_cache, v_cache)
    if q_out is None:
        q_out = torch.empty((T, Hq, D), dtype=qkv.dtype, device=qkv.device)
    if q_out.shape != (T, Hq, D) or q_out.dtype != qkv.dtype or q_out.stride(2) != 1 or q_out.stride(1) != D:
        raise ValueError("q_out must be [tokens, Hq, D] with heads and dims contiguous")
    code = _C.lib().gr_qk_norm_rope_cache(
        q_out.data_ptr(), q_out.stride(0), qkv.data_ptr(), qkv.stride(0), positions.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0], _ptr(q_norm), _ptr(k_norm),
        _ptr(k_cache), _ptr(v_cache), NB, bstr, tstr, hstr, _ptr(slot_mapping), bs or 1, T, Hq, Hkv, D,
        float(eps), _dtype_code(qkv), _ptr(status), _stream(dev))
    _C.check("gr_qk_norm_rope_cache", code)
    return q_out


def silu_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(x[:, :F]) * x[:, F:]`` for ``x [T, 2F]`` (vLLM's silu_and_mul)."""
    dev = _need_cuda(x, out)
    _rows("x", x)
    T, F2 = x.shape
    if F2 % 2:
        raise ValueError("x must hold gate and up halves")
    F = F2 // 2
    if out is None:
        out = torch.empty((T, F), dtype=x.dtype, device=x.device)
    _rows("out", out)
    if out.shape != (T, F) or out.dtype != x.dtype:
        raise ValueError("out must be [tokens, F] of x's dtype")
    code = _C.lib().gr_silu_mul(out.data_ptr(), out.stride(0), x.data_ptr(), x.stride(0), T, F,
                                _dtype_code(x), _stream(dev))
    _C.check("gr_silu_mul", code)
    return out
