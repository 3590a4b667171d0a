"""fp8 e4m3 conversions of an fp8 KV cache.  TEST INFRASTRUCTURE ONLY.

The reference keeps an fp8 cache as ``float8_e4m3fn`` (OCP e4m3: sign, 4
exponent bits with bias 7, 3 mantissa bits, no infinities, 0x7F / 0xFF NaN,
largest finite 448; ``vllm_gr/v1/attention/backends/beam_attn.py:734-737,
801-804``), written by ``reshape_and_cache_flash`` with the layer's
``_k_scale`` / ``_v_scale`` (``:727-732``): element = e4m3(clamp(x / scale,
-448, 448)), rounded to nearest even.

Functions and how each is pinned (tests/test_oracle_fp8.py):

* ``decode(codes)`` -- the value of each byte; against torch's
  ``float8_e4m3fn`` for all 256 codes.
* ``quantize(x, scale)`` -- the byte of each float32 ``x / scale`` (float32
  division), NaN -> 0x7F; against torch's clamp + ``float8_e4m3fn`` cast on
  dense ranges, every representable value and every midpoint between two
  (ties), the subnormal range, saturation and signed zeros.
"""

from __future__ import annotations

import numpy as np


def decode(codes) -> np.ndarray:
    """float64 value of each e4m3 byte."""
    b = np.asarray(codes).astype(np.uint8)
    s = (b >> 7) & 1
    e = ((b >> 3) & 15).astype(np.int64)
    m = (b & 7).astype(np.float64)
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(s == 1, -v, v)


def quantize(x, scale: float = 1.0) -> np.ndarray:
    """e4m3 byte of float32(x) / float32(scale), clamped to +-448, nearest
    even; NaN -> 0x7F.  With e = max(floor(log2 |y|), -6) the quantum is
    2^(e - 3) and the code ((e + 7) << 3) + rint(|y| / quantum) - 8."""
    y = np.asarray(x, dtype=np.float32) / np.float32(scale)
    nan = np.isnan(y)
    a = np.minimum(np.abs(np.where(nan, np.float32(0), y)), np.float32(448.0)).astype(np.float64)
    _, ex = np.frexp(np.where(a > 0, a, 1.0))          # a = mant * 2^ex, mant in [0.5, 1)
    e = np.maximum(ex.astype(np.int64) - 1, -6)
    q = np.rint(a * np.exp2(3 - e))                     # exact scaling; rint ties to even
    code = np.where(a > 0, (e + 7) * 8 + q.astype(np.int64) - 8, 0)
    code = code | np.where(np.signbit(y), 0x80, 0)
    return np.where(nan, 0x7F, code).astype(np.uint8)
