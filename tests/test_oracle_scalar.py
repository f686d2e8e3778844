"""Pins the oracle's scalar arithmetic (CPU only): fp16 conversion, nearest_int, exp/log and the activations, the
pairwise sum, against numpy, libm in float64, the reference's own conversion (stored vectors and, where the
reference tree is present, the compiled reference), and known answers."""
import math

import numpy as np
import pytest

from golden_data import golden


def test_half_to_float_exhaustive(orc):
    """All 65536 fp16 patterns against numpy's float16 (gemvq_ref.h:16-30)."""
    o = orc.orc()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([o.orc_half_to_float(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_rne(orc):
    """float -> fp16 round to nearest even against numpy on random bit patterns, all rounding ties around 1 and in
    the subnormal range, overflow to infinity (gemvq_ref.h:32-52)."""
    o = orc.orc()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 60000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    halfway = (np.arange(0x3C00, 0x3D00, dtype=np.uint16).view(np.float16).astype(np.float64) +
               2.0**-11).astype(np.float32)  # exactly between two halves in [1, 1.25)
    sub = (np.arange(1, 200, dtype=np.float64) * 2.0**-25).astype(np.float32)  # ties in the subnormal range
    edge = np.array([65504.0, 65519.0, 65520.0, 65536.0, 1e30, -65520.0, 2.0**-25, 2.0**-26, 0.0, -0.0], np.float32)
    xs = np.concatenate([x, halfway, sub, -sub, edge])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([o.orc_float_to_half(float(v)) for v in xs], np.uint16)
    assert np.array_equal(got, want)


def test_fp16_matches_reference_vectors(orc):
    o = orc.orc()
    g = golden()
    got = np.array([o.orc_float_to_half(float(v)) for v in g["f2h_in"]], np.uint16)
    assert np.array_equal(got, g["f2h_out"])


def test_nearest_int(orc):
    """Round half to even for |v| < 2^22 (gemvq_ref.h:54-60): random values, exact halves, reference vectors."""
    o = orc.orc()
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.uniform(-300, 300, 5000), np.arange(-50, 50) + 0.5]).astype(np.float32)
    got = np.array([o.orc_nearest_int(float(t)) for t in v])
    assert np.array_equal(got, np.rint(v.astype(np.float64)).astype(np.int64))
    g = golden()
    assert [o.orc_nearest_int(float(t)) for t in g["nearest_in"]] == list(g["nearest_out"])


def ulp_err(got: np.ndarray, exact: np.ndarray) -> np.ndarray:
    """|got - exact| in units of the FP32 spacing at the exact value."""
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - exact) / ulp


def test_expf_within_two_ulp(orc):
    """The oracle's own exp (Cody-Waite + Taylor to degree 7) against float64 exp over the whole normal range."""
    o = orc.orc()
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-87, 88.7, 40000), rng.uniform(-1, 1, 10000), [0.0, -0.0, 1.0, -1.0, 88.7]])
    x = x.astype(np.float32)
    got = np.array([o.orc_expf(float(t)) for t in x], np.float32)
    err = ulp_err(got, np.exp(x.astype(np.float64)))
    assert err.max() <= 2.0, (x[err.argmax()], err.max())
    assert np.mean(err <= 1.0) > 0.99
    assert o.orc_expf(0.0) == 1.0
    assert o.orc_expf(-100.0) == 0.0 and math.isinf(o.orc_expf(89.0))


def test_logf_within_two_ulp(orc):
    o = orc.orc()
    rng = np.random.default_rng(4)
    x = np.concatenate([10.0 ** rng.uniform(-37, 38, 30000), rng.uniform(0.5, 2.0, 20000), [1.0, 2.0, 0.5]])
    x = x.astype(np.float32)
    got = np.array([o.orc_logf(float(t)) for t in x], np.float32)
    exact = np.log(x.astype(np.float64))
    nz = exact != 0
    err = ulp_err(got[nz], exact[nz])
    assert err.max() <= 2.0, (x[nz][err.argmax()], err.max())
    assert o.orc_logf(1.0) == 0.0
    assert math.isinf(o.orc_logf(0.0)) and math.isnan(o.orc_logf(-1.0))


def test_activations_against_float64(orc):
    """SiLU x / (1 + e^-x), sigmoid 1 / (1 + e^-x), softplus (x > 20 ? x : log(1 + e^x)) (gemvq_ref.h:332-342)."""
    o = orc.orc()
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-30, 30, 6000), [20.0, 20.000002, 19.999998, 0.0, -87.0]]).astype(np.float32)
    xd = x.astype(np.float64)
    silu = np.array([o.orc_silu(float(t)) for t in x])
    sig = np.array([o.orc_sigmoid(float(t)) for t in x])
    sp = np.array([o.orc_softplus(float(t)) for t in x])
    np.testing.assert_allclose(silu, xd / (1 + np.exp(-xd)), rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(sig, 1 / (1 + np.exp(-xd)), rtol=2e-6, atol=1e-30)
    sp_want = np.where(xd > 20, xd, np.log1p(np.exp(xd)))
    # log(1 + e^x) is formed in FP32 (as ggml does, not log1p): 1 + e^x carries an absolute error up to 2^-24
    np.testing.assert_allclose(sp, sp_want, rtol=2e-6, atol=1.2e-7)
    assert o.orc_softplus(20.5) == np.float32(20.5)  # the threshold passes x through unchanged


def test_pair_sum_known_answers(orc):
    """The canonical sum is the adjacent-pair tree: ((a0 + a1) + (a2 + a3)). In FP32 these inputs tell it apart
    from the sequential sum (1) and from the strided pairing (a0 + a2) + (a1 + a3) (2)."""
    assert orc.pair_sum(np.array([1e8, 1, -1e8, 1], np.float32)) == 0.0
    # zero padding to the next power of two: 5 values are summed as a tree over 8
    assert orc.pair_sum(np.array([1e8, 1, -1e8, 1, 7], np.float32)) == 7.0
    assert orc.pair_sum(np.array([], np.float32)) == 0.0
    rng = np.random.default_rng(6)
    for n in (1, 2, 3, 127, 128, 4096):
        a = rng.standard_normal(n).astype(np.float32)
        assert abs(orc.pair_sum(a) - a.astype(np.float64).sum()) <= 1e-6 * max(1.0, np.abs(a).sum())


def test_scalar_matches_compiled_reference(orc):
    """Where the reference tree is present, its own conversions agree with the oracle on random inputs."""
    if not orc.ref_available():
        pytest.skip("reference library not built (needs the reference tree)")
    o, r = orc.orc(), orc.ref()
    rng = np.random.default_rng(7)
    x = rng.standard_normal(20000).astype(np.float32) * np.float32(300)
    assert all(o.orc_float_to_half(float(v)) == r.refshim_float_to_half(float(v)) for v in x)
    assert all(o.orc_nearest_int(float(v)) == r.refshim_nearest_int(float(v)) for v in x[:5000])
    for b in range(0, 65536, 7):
        a, c = o.orc_half_to_float(b), r.refshim_half_to_float(b)
        assert a == c or (math.isnan(a) and math.isnan(c))
