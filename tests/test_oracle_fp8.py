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


def test_unscaled_read_departure_measured():
    """Departure, measured: the reference writes an fp8 cache with the
    layer's scales but its flash-attention calls pass no descale
    (beam_attn.py:646-695), so it attends over e4m3 codes = x / scale; this
    build reads e4m3 * scale.  At scale 1.0 the two are the same attention;
    at K / V scales 0.05 / 0.02 the reference's reading is far from the
    attention over the cached values."""
    from oracle import attention as oa
    rng = np.random.default_rng(7)
    NB, BS, Hkv, D, P, W = 12, 16, 2, 32, 100, 4
    x_k = rng.standard_normal((NB, BS, Hkv, D))
    x_v = rng.standard_normal((NB, BS, Hkv, D))
    q = rng.standard_normal((W, 4, D))
    pbt = rng.permutation(NB)[None, :7]
    sbt = np.array([[7], [8], [9], [10]])
    args = dict(prefix_bt=pbt, prefix_len=np.array([P]), beam_start=np.array([0, W]), suffix_bt=sbt,
                suffix_len=np.array([1, 2, 3, 1]), scale=D ** -0.5, block_size=BS)
    for sk, sv, same in ((1.0, 1.0, True), (0.05, 0.02, False)):
        ck, cv = fp8.decode(fp8.quantize(x_k, sk)), fp8.decode(fp8.quantize(x_v, sv))
        ours = oa.beam_attention_dense(q, ck * sk, cv * sv, **args)[0]
        ref = oa.beam_attention_dense(q, ck, cv, **args)[0]
        diff = np.abs(ours - ref).max()
        print(f"scales {sk}/{sv}: max |out difference| {diff:.3g}")
        assert (diff == 0.0) if same else diff > 1.0
