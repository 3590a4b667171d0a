"""CPU oracle for fused beam pruning.  TEST INFRASTRUCTURE ONLY.

``prune_topk`` calls the C restatement in ``prune_ref.c`` (bit-exact build
contract: fixed-order fp32 exp-sum, fp64 log, fp64 score, stage-1 order
``(logit desc, token asc)``, stage-2 order ``(score desc, flat asc)``).

Functions and how each is pinned (tests/test_oracle_prune.py):

* ``exp2_neg`` / ``log_f64`` -- against ``2.0**t`` and ``math.log`` on
  dense grids and random inputs (<= 4 ulp and <= 2 ulp).
* ``row_stats`` -- lse against ``scipy.special.logsumexp`` in float64
  (<= 1e-6 absolute: the fp32 sum bounds it).
* ``prune_topk`` -- against ``prune_topk_float64`` (plain numpy float64 of
  the reference arithmetic, ``serving_engine.py:511,538-539,566-567``) on
  random data: identical index sets wherever the float64 gap exceeds 1e-9;
  against the one-stage global top-k (the two-stage structure of the
  reference loses nothing, ``serving_engine.py:492-567``); against the
  reference's KATs (``tests/test_batch_and_fork_unit.py:1109-1176``,
  ``:1229-1248``); against all-equal logits (lowest flat index wins); and,
  when ``oracle/_ref`` was built from the reference sources, against the
  reference's own ``MinHeapTuple.push_candidates_striped``
  (``vllm_gr/csrc/minheap.cpp:75-114``) on tie-free data; and, at the full
  64 x 128 x 8192 size, against ``topk_float64_global`` (vectorised float64
  mathematics, checked itself against ``prune_topk_float64`` on small cases):
  the same selections wherever the float64 128th/129th gap exceeds 1e-6.
"""

from __future__ import annotations

import ctypes
import glob
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "liboracle_prune.so")
_lib = None


def build() -> None:
    """Compile the C restatement (and ``_ref`` when the reference is mounted)."""
    targets = ["all"]
    if os.path.isdir("/root/reference/vllm_gr"):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", _HERE] + targets, check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_exp2_neg.restype = ctypes.c_float
        lib.oracle_exp2_neg.argtypes = [ctypes.c_float]
        lib.oracle_log_f64.restype = ctypes.c_double
        lib.oracle_log_f64.argtypes = [ctypes.c_double]
        P = ctypes.c_void_p
        lib.oracle_prune_row_stats.restype = None
        lib.oracle_prune_row_stats.argtypes = [P, P, ctypes.c_int, ctypes.c_int, P, P, P, P]
        lib.oracle_prune_topk.restype = ctypes.c_int
        lib.oracle_prune_topk.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P, P]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def exp2_neg(t: float) -> float:
    return float(_load().oracle_exp2_neg(float(t)))


def log_f64(s: float) -> float:
    return float(_load().oracle_log_f64(float(s)))


def _cum64(cum) -> np.ndarray:
    """The cumulative scores as float64: a float32 array enters exactly."""
    c = np.asarray(cum)
    return c.astype(np.float64) if c.dtype != np.float64 else c


def row_stats(logits: np.ndarray, cum: np.ndarray):
    """Per-row (max, fp32 exp-sum, lse, cum - lse) under the build contract."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = x.reshape(-1, x.shape[-1]).shape
    c_in = np.ascontiguousarray(np.broadcast_to(_cum64(cum).reshape(-1), (rows,)))
    m = np.empty(rows, np.float32)
    S = np.empty(rows, np.float32)
    lse = np.empty(rows, np.float64)
    c = np.empty(rows, np.float64)
    _load().oracle_prune_row_stats(_ptr(x), _ptr(c_in), rows, V, _ptr(m), _ptr(S), _ptr(lse), _ptr(c))
    return m, S, lse, c


def prune_topk(logits: np.ndarray, cum: np.ndarray, k: int, eos_token_id: int = -1, allowed=None,
               candidates: bool = False):
    """Bit-exact oracle.  ``logits [R, W, V]`` fp32, ``cum [R, W]`` fp32 or
    fp64 (a float32 score enters as its exact float64 value); ``allowed [R,
    W, V]`` bool (optional): the catalog mask applied to each beam's top-k
    candidates.

    Returns dict with ``parent, token [R, k]`` int32, ``score [R, k]`` fp32,
    ``score64 [R, k]`` fp64, ``eos_score [R, W]`` fp32 and ``eos_score64``
    fp64; with ``candidates``, also ``cand_token [R, W, k1]`` int32 and
    ``cand_logprob [R, W, k1]`` fp32 (each beam's top-k1 before EOS/catalog
    removal, logprob = x - lse).
    """
    x = np.ascontiguousarray(logits, dtype=np.float32)
    R, W, V = x.shape
    cm = np.ascontiguousarray(_cum64(cum).reshape(R, W))
    k1 = min(k, V)
    parent = np.empty((R, k), np.int32)
    token = np.empty((R, k), np.int32)
    score = np.empty((R, k), np.float32)
    score64 = np.empty((R, k), np.float64)
    eos_score64 = np.empty((R, W), np.float64)
    ct = np.empty((R, W, k1), np.int32) if candidates else None
    cl = np.empty((R, W, k1), np.float32) if candidates else None
    al = None if allowed is None else np.ascontiguousarray(allowed, dtype=np.uint8).reshape(R, W, V)
    rc = _load().oracle_prune_topk(_ptr(x), _ptr(cm), R, W, V, int(k), int(eos_token_id),
                                   _ptr(parent), _ptr(token), _ptr(score), _ptr(score64),
                                   _ptr(eos_score64), None if al is None else _ptr(al),
                                   None if ct is None else _ptr(ct), None if cl is None else _ptr(cl))
    if rc != 0:
        raise ValueError("oracle_prune_topk: bad arguments")
    out = dict(parent=parent, token=token, score=score, score64=score64,
               eos_score=eos_score64.astype(np.float32), eos_score64=eos_score64)
    if candidates:
        out.update(cand_token=ct, cand_logprob=cl)
    return out


def prune_topk_float64(logits: np.ndarray, cum: np.ndarray, k: int, eos_token_id: int = -1, valid_sets=None):
    """Plain numpy float64 restatement of the reference's pruning arithmetic.

    Per beam: ``log_softmax`` then the beam's top-k candidates
    (``serving_engine.py:300-308`` asks the sampler for ``logprobs=W``);
    ``score = cum + logprob`` (``:511``) in float64 (``:538-539``); EOS
    candidates leave the pool (``:541-562``); top-k over the union
    (``:566-567``), sorted by (score desc, flat asc).  ``valid_sets`` (one
    set of tokens per beam, ``[R][W]``): the catalog's valid continuations;
    the beam's other candidates become -inf (``:504-506``) and, being
    -inf, are never selected here.
    """
    x = np.asarray(logits, dtype=np.float64)
    R, W, V = x.shape
    m = x.max(axis=2, keepdims=True)
    lse = m + np.log(np.exp(x - m).sum(axis=2, keepdims=True))
    logp = x - lse
    out_parent = np.full((R, k), -1, np.int64)
    out_token = np.full((R, k), -1, np.int64)
    out_score = np.full((R, k), -np.inf)
    for r in range(R):
        cand_s, cand_f = [], []
        for b in range(W):
            order = np.lexsort((np.arange(V), -x[r, b]))[:min(k, V)]
            for v in order:
                if valid_sets is not None and int(v) not in valid_sets[r][b]:
                    continue
                if v == eos_token_id:
                    continue
                cand_s.append(float(cum[r][b]) + logp[r, b, v])
                cand_f.append(b * V + int(v))
        cand_s = np.array(cand_s)
        cand_f = np.array(cand_f, dtype=np.int64)
        sel = np.lexsort((cand_f, -cand_s))[:k]
        out_parent[r, :len(sel)] = cand_f[sel] // V
        out_token[r, :len(sel)] = cand_f[sel] % V
        out_score[r, :len(sel)] = cand_s[sel]
    return dict(parent=out_parent, token=out_token, score=out_score)


def topk_float64_global(logits: np.ndarray, cum: np.ndarray, k: int):
    """Plain float64 mathematics of the pruning at any size, vectorised:
    ``score = cum + log_softmax(logits)`` in float64, then per request the
    top-k of all W x V candidates by (score desc, flat index asc) -- the
    global selection the reference's two stages compute
    (``serving_engine.py:511,538-539,566-567``; a global top-k element is
    within its beam's top-k).  Returns ``parent``, ``token``, ``score``
    (float64, ``[R, k]``) and ``gap`` (``[R]``): the k-th score minus the
    (k+1)-th, the margin by which the selected set is determined."""
    x = np.asarray(logits, dtype=np.float32)
    R, W, V = x.shape
    parent = np.empty((R, k), np.int64)
    token = np.empty((R, k), np.int64)
    score = np.empty((R, k))
    gap = np.empty(R)
    cum64 = np.asarray(cum, dtype=np.float64).reshape(R, W)
    for r in range(R):  # one request at a time: W x V float64 scores
        x64 = x[r].astype(np.float64)
        m = x64.max(axis=1, keepdims=True)
        lse = m + np.log(np.exp(x64 - m).sum(axis=1, keepdims=True))
        s = ((x64 - lse) + cum64[r][:, None]).reshape(-1)
        n = min(k + 1, s.size)
        part = np.argpartition(-s, n - 1)[:n]
        o = np.lexsort((part, -s[part]))
        part = part[o]
        parent[r] = part[:k] // V
        token[r] = part[:k] % V
        score[r] = s[part[:k]]
        gap[r] = s[part[k - 1]] - s[part[k]] if n > k else np.inf
    return dict(parent=parent, token=token, score=score, gap=gap)


def ref_minheap_module():
    """The reference's own ``minheap_cpp`` built under ``oracle/_ref`` by
    ``make -C oracle ref`` from ``vllm_gr/csrc/minheap.cpp``; None if absent."""
    hits = glob.glob(os.path.join(_HERE, "_ref", "minheap_cpp*.so"))
    if not hits:
        return None
    import importlib.util
    spec = importlib.util.spec_from_file_location("minheap_cpp", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod
