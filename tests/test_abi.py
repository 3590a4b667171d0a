"""The C-ABI library without a GPU: it loads, exports every function
include/*.h declare, the ctypes table mirrors the header, and the
argument checks that run before any HIP call reject bad input with the
documented status codes.  No compute call is made here."""

from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def _header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(gr_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_entry_points():
    names = _header_functions()
    for n in ("gr_beam_attn_decode", "gr_beam_kv_fork", "gr_beam_kv_append", "gr_reshape_and_cache",
              "gr_beam_prune_topk", "gr_beam_prune_workspace_size", "gr_status_string", "gr_version",
              "gr_paged_attn_prefill", "gr_rms_norm", "gr_qk_norm_rope_cache", "gr_silu_mul"):
        assert n in names


def test_library_exports_every_header_symbol(built_lib):
    for n in _header_functions():
        assert hasattr(built_lib, n), f"{n} declared in include/ but not exported"


def test_ctypes_table_mirrors_header(built_lib):
    from vllm_gr_amd import _C
    assert sorted(_C.SIGNATURES) == _header_functions()


def test_version_and_status_strings(built_lib):
    from vllm_gr_amd import _C
    assert built_lib.gr_version() == 100
    for code in range(5):
        assert isinstance(built_lib.gr_status_string(code), bytes)
    assert built_lib.gr_status_string(0) != built_lib.gr_status_string(1)
    with pytest.raises(_C.GrError):
        _C.check("gr_x", _C.GR_ERR_LAUNCH)
    with pytest.raises(ValueError):
        _C.check("gr_x", _C.GR_ERR_INVALID_ARG)
    with pytest.raises(NotImplementedError):
        _C.check("gr_x", _C.GR_ERR_UNSUPPORTED)


_BAD = 0x10  # a non-null pointer value that is never dereferenced: the checks reject first


def _decode(lib, **over):
    args = dict(out=_BAD, out_tok_stride=4096, q=_BAD, q_tok_stride=4096, k=_BAD, v=_BAD, nb=10,
                bstr=16 * 8 * 128, tstr=8 * 128, hstr=128, pbt=_BAD, pbt_stride=4, plen=_BAD,
                bstart=_BAD, sbt=_BAD, sbt_stride=1, slen=_BAD, sstart=None, R=1, maxb=4, N=4, T=1,
                Hq=32, Hkv=8, D=128, bs=16, dtype=2, scale=0.1, softcap=0.0, lse=None, status=None,
                stream=None)
    args.update(over)
    return lib.gr_beam_attn_decode(*args.values())


def test_decode_argument_checks(built_lib):
    from vllm_gr_amd import _C
    lib = built_lib
    assert _decode(lib, N=0) == _C.GR_OK  # nothing to do, no launch
    assert _decode(lib, Hq=30) == _C.GR_ERR_INVALID_ARG  # Hq % Hkv
    assert _decode(lib, D=12) == _C.GR_ERR_INVALID_ARG
    assert _decode(lib, D=264) == _C.GR_ERR_UNSUPPORTED  # head_size <= 256 (beam_attn.py:807-808)
    assert _decode(lib, dtype=7) == _C.GR_ERR_INVALID_ARG
    assert _decode(lib, softcap=-1.0) == _C.GR_ERR_INVALID_ARG
    assert _decode(lib, q=None) == _C.GR_ERR_INVALID_ARG
    assert _decode(lib, q_tok_stride=100) == _C.GR_ERR_INVALID_ARG
    assert _decode(lib, T=0) == _C.GR_ERR_INVALID_ARG
    assert lib.gr_set_decode_kernel(5) == _C.GR_ERR_INVALID_ARG
    assert lib.gr_set_decode_kernel(2) == _C.GR_ERR_INVALID_ARG


def test_fork_append_prune_argument_checks(built_lib):
    from vllm_gr_amd import _C
    lib = built_lib
    geom = [_BAD, _BAD, 10, 16 * 8 * 128, 8 * 128, 128]
    # fork: tables must be written out of place; beam_width >= 1
    assert lib.gr_beam_kv_fork(_BAD, 1, 4, _BAD, _BAD, _BAD, _BAD, 1, *geom, None, None, 0, 8, 128, 16, 2,
                               None, None) == _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_kv_fork(_BAD, 1, 0, 0x20, 0x30, 0x40, 0x50, 1, *geom, None, None, 0, 8, 128, 16, 2,
                               None, None) == _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_kv_fork(_BAD, 0, 4, 0x20, 0x30, 0x40, 0x50, 1, *geom, None, None, 0, 8, 128, 16, 2,
                               None, None) == _C.GR_OK
    # multi-layer fork: at least one layer, pointer arrays present, every layer's cache 16-byte aligned
    import ctypes
    ptrs = (ctypes.c_void_p * 2)(0x1000, 0x2000)
    bad = (ctypes.c_void_p * 2)(0x1000, 0x2008)
    lgeom = [10, 16 * 8 * 128, 8 * 128, 128]
    args = (_BAD, 1, 4, 0x20, 0x30, 0x40, 0x50, 1)
    assert lib.gr_beam_kv_fork_layers(*args, 0, ptrs, ptrs, *lgeom, 8, 128, 16, 2, None, None) == \
        _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_kv_fork_layers(*args, 2, None, ptrs, *lgeom, 8, 128, 16, 2, None, None) == \
        _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_kv_fork_layers(*args, 2, ptrs, bad, *lgeom, 8, 128, 16, 2, None, None) == \
        _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_kv_fork_layers(_BAD, 0, 4, 0x20, 0x30, 0x40, 0x50, 1, 2, ptrs, ptrs, *lgeom, 8, 128, 16, 2,
                                      None, None) == _C.GR_OK
    # append: misaligned cache pointer
    assert lib.gr_beam_kv_append(0x20, 0x30, 1024, 0x11, 0x20, 10, 16 * 8 * 128, 8 * 128, 128, _BAD, 1, _BAD,
                                 4, 8, 128, 16, 2, None, None) == _C.GR_ERR_INVALID_ARG
    # reshape_and_cache: negative token count
    assert lib.gr_reshape_and_cache(_BAD, 1024, _BAD, 1024, *geom, _BAD, -1, 8, 128, 16, 2, None,
                                    None) == _C.GR_ERR_INVALID_ARG
    # prune: vocab must be a multiple of 4, k <= vocab, workspace large enough
    ws = lib.gr_beam_prune_workspace_size(2, 8, 64, 8)
    assert ws > 0
    assert lib.gr_beam_prune_topk(0x100, 64, _BAD, 2, 8, 62, 8, -1, _BAD, _BAD, _BAD, None, 0x1000, ws,
                                  None) == _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_prune_topk(0x100, 64, _BAD, 2, 8, 64, 65, -1, _BAD, _BAD, _BAD, None, 0x1000, ws,
                                  None) == _C.GR_ERR_INVALID_ARG
    assert lib.gr_beam_prune_topk(0x100, 64, _BAD, 2, 8, 64, 8, -1, _BAD, _BAD, _BAD, None, 0x1000, ws - 1,
                                  None) == _C.GR_ERR_WORKSPACE


def test_python_wrapper_rejects_host_tensors(built_lib):
    """The torch entry points never compute on the CPU: host tensors are an error."""
    from vllm_gr_amd import ops
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    kc = torch.zeros(10, 16, 8, 128, dtype=torch.bfloat16)
    i32 = lambda *s: torch.zeros(*s, dtype=torch.int32)
    with pytest.raises(ValueError):
        ops.beam_attn_decode(q, kc, kc, i32(1, 4), i32(1), i32(2), i32(4, 1), i32(4), scale=0.1)
    with pytest.raises(ValueError):
        ops.beam_prune_topk(torch.zeros(1, 4, 64), torch.zeros(1, 4), 4)
    with pytest.raises(ValueError):
        ops.split_kv_cache(torch.zeros(3, 2, 2, 2, 8))


def test_split_decode_workspace_plan_and_check(built_lib):
    """The split plan: a 1-request x 128-beam decode splits (workspace > 0), the
    8-request one fills the GPU unsplit (0), and the _ws entry point rejects a
    missing workspace before any HIP call (pointer values are never used)."""
    ws = built_lib.gr_beam_attn_decode_workspace_size
    assert ws(1, 128, 1, 32, 8, 128, 2048) > 0
    assert ws(8, 128, 1, 32, 8, 128, 2048) == 0
    assert ws(1, 128, 1, 32, 8, 64, 2048) == 0  # generic kernel: no split
    assert ws(1, 128, 1, 32, 8, 128, 200) == 0  # under 4 tiles per split
    P = 0x1000  # aligned, non-null, never dereferenced
    code = built_lib.gr_beam_attn_decode_ws(
        P, 4096, P, 4096, P, P, 100, 16 * 8 * 128, 8 * 128, 128, P, 128, P, P, P, 1, P, None,
        1, 128, 128, 1, 32, 8, 128, 16, 2, 0.088, 0.0, None, None, 2048, None, 0, None)
    assert code == 4  # GR_ERR_WORKSPACE
