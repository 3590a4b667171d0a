"""The fp8 e4m3 oracle (oracle/fp8.py) against torch's float8_e4m3fn, an
independent implementation of the same format."""

import numpy as np
import torch

from oracle import fp8


def _torch_q(y: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.asarray(y, dtype=np.float32)).clamp(-448.0, 448.0)
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = fp8.decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert fp8.decode(np.uint8(0x7E)) == 448.0 and fp8.decode(np.uint8(0x01)) == 2.0 ** -9


def test_quantize_matches_torch():
    rng = np.random.default_rng(0)
    vals = fp8.decode(np.arange(256, dtype=np.uint8))
    fin = np.sort(np.unique(vals[np.isfinite(vals)]))
    mids = (fin[:-1] + fin[1:]) / 2                    # every tie between neighbours
    xs = np.concatenate([
        np.linspace(-500, 500, 200001), rng.standard_normal(100000) * 3, rng.standard_normal(20000) * 1e-2,
        np.linspace(-2.0 ** -5, 2.0 ** -5, 40001),     # the subnormal range and its edge
        fin, mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf),
        [0.0, -0.0, 448.0, -448.0, 449.0, 464.0, 1e30, -1e30, np.inf, -np.inf]]).astype(np.float32)
    got = fp8.quantize(xs)
    assert np.array_equal(got, _torch_q(xs))
    # every representable value survives the round trip
    assert np.array_equal(fp8.decode(fp8.quantize(fin)), fin)


def test_quantize_with_scale_and_nan():
    rng = np.random.default_rng(1)
    xs = (rng.standard_normal(50000) * 40).astype(np.float32)
    for s in (0.37, 2.5, 1.0):
        y = xs / np.float32(s)                          # the same float32 division as the kernel
        assert np.array_equal(fp8.quantize(xs, s), _torch_q(y))
    assert fp8.quantize(np.float32(np.nan)) == 0x7F and fp8.quantize(np.float32(-np.nan)) == 0x7F
