"""Pins the oracle's activation quantizers and GEMVs (CPU only).

- Q8_0 / Q8_K quantizers: numpy brute force of the closed forms (roundf half away from zero, nearest_int half to
  even, first maximum on ties), the special blocks, and the reference's own outputs (stored vectors).
- Block sums: exact integers from an independent numpy decoding of the GGUF blocks (tests/ggml_blocks.py), on
  synthetic matrices and on random block bytes (every bit pattern of the quants and K-quant scales).
- Canonical row values: the exact rational closed form of the fixed-point sum, floor(term * 2^40) per block
  evaluated with Python integers, rounded to FP32 once; and the float64 value within 1e-5 rel / 1e-6 abs.
- Reference path: the oracle's sequential FP32 restatement reproduces the reference's own gemvq_ref.h outputs bit
  for bit (stored vectors; the compiled reference when present), and the canonical path stays within the
  reference's tolerance of it (gemvq_ref.h:267-272).
"""
from fractions import Fraction

import numpy as np
import pytest

import ggml_blocks as B
from golden_data import golden

FORMATS = [(B.Q4_0, 32), (B.Q4_1, 32), (B.Q8_0, 32), (B.Q5_K, 256), (B.Q6_K, 256)]


# ---------------------------------------------------------------------------------------------------------------
def test_q8_0_closed_form(orc, gq):
    x = gq.normal(0, 1, 4096)
    x[:32] = 0.0  # all-zero block: d = 0, q = 0
    x[32:64] = (np.arange(32) - 16).astype(np.float32) + np.float32(0.5)  # evenly spaced values
    x[64:96] = np.float32(0.0)
    x[64], x[65], x[66] = 127.0, 2.5, -2.5  # amax 127: scale 1, x * 1 is an exact half: roundf goes away from 0
    x[96:128] = np.float32(127 * 70000.0)  # amax / 127 beyond the fp16 range: d = inf, id finite
    q, d = orc.quantize_q8_0(x)
    qw, dw = B.quantize_q8_0(x)
    assert np.array_equal(q, qw) and np.array_equal(d, dw)
    assert q[65] == 3 and q[66] == -3 and d[0] == 0 and np.all(q[:32] == 0)
    assert d[3] == 0x7C00


def test_q8_K_closed_form_and_reference_vectors(orc, gq):
    x = gq.normal(0, 2, 2048)
    x[256:512] = 0.0
    x[512:768] *= np.float32(0.1)
    x[515], x[519] = 5.0, -5.0  # first maximum wins: iscale = -127 / 5 (the last would flip every sign)
    x[768:1024] = (np.arange(256) % 9 - 4).astype(np.float32) * np.float32(0.5)
    x[768] = -127.0  # iscale = 1: exact halves round to even
    q, d, bs = orc.quantize_q8_K(x)
    qw, dw, bsw = B.quantize_q8_K(x)
    assert np.array_equal(q, qw) and np.array_equal(d.view(np.uint32), dw.view(np.uint32))
    assert np.array_equal(bs, bsw)
    assert np.all(q[256:512] == 0) and d[1] == 0
    assert q[515] == -127 and q[519] == 127
    # -1.5, -0.5, 0.5, 1.5 -> -2, 0, 0, 2 (half to even; roundf would give -2, -1, 1, 2)
    assert [q[769], q[771], q[773], q[775]] == [-2, 0, 0, 2]
    g = golden()
    q2, d2, _ = orc.quantize_q8_K(g["q8k_x"])
    assert np.array_equal(q2, g["q8k_q"]) and np.array_equal(d2.view(np.uint32), g["q8k_d"].view(np.uint32))


# ---------------------------------------------------------------------------------------------------------------
def random_blocks(t: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Random block bytes with finite fp16 scales: every quant and scale bit pattern."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // B.BLOCK_ELEMS[t]
    blk = rng.integers(0, 256, (nb, B.BLOCK_BYTES[t]), dtype=np.uint8)
    halves = lambda lo, hi: rng.uniform(lo, hi, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)  # noqa: E731
    if t == B.Q4_1:
        blk[:, 0:2] = halves(0.0, 0.005)
        blk[:, 2:4] = halves(-0.04, 0.0)
    elif t in (B.Q4_0, B.Q8_0):
        blk[:, 0:2] = halves(-0.01, 0.01)
    elif t == B.Q5_K:
        blk[:, 0:2] = halves(-0.002, 0.002)
        blk[:, 2:4] = halves(-0.002, 0.002)
    else:
        blk[:, 208:210] = halves(-0.002, 0.002)
    return blk.ravel()


def f32_round(acc: int) -> float:
    """An integer rounded to FP32, round to nearest even (exact integer arithmetic, no double rounding)."""
    s = -1 if acc < 0 else 1
    a = abs(acc)
    n = a.bit_length()
    if n > 24:
        sh = n - 24
        qv, rem = a >> sh, a & ((1 << sh) - 1)
        half = 1 << (sh - 1)
        if rem > half or (rem == half and (qv & 1)):
            qv += 1
        a = qv << sh
    return float(np.float32(s * a))


def canonical_rows(t: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int):
    """(exact fixed-point rows as FP32, float64 values, block sums) from the independent decoders: each block term
    floor(sum * d_w * d_x * 2^40) with exact rationals (FP32 subnormal activation scales count as zero)."""
    def frac(v) -> Fraction:
        v = float(v)
        if v != 0 and abs(v) < 1.1754943508222875e-38:
            return Fraction(0)
        return Fraction(v)

    TWO40 = 1 << 40
    if t == B.Q4_1:  # floor(sumi d_w d_x 2^40) + floor(m_w s_x 2^40) per block
        xq, xd, xs = B.quantize_q8_1(x)
        sums = B.block_sums(t, w, xq, rows, cols).reshape(rows, -1)
        blk = B.blocks(t, w, rows, cols)
        dw = blk[..., 0:2].copy().view(np.float16)[..., 0]
        mw = blk[..., 2:4].copy().view(np.float16)[..., 0]
        dx, sx = xd.view(np.float16), xs.view(np.float16)
        out, f64 = [], []
        for r in range(rows):
            acc, v = 0, 0.0
            for b in range(sums.shape[1]):
                t1 = sums[r, b] * frac(dw[r, b]) * frac(dx[b])
                t2 = frac(mw[r, b]) * frac(sx[b])
                acc += (t1 * TWO40).__floor__() + (t2 * TWO40).__floor__()
                v += float(t1 + t2)
            out.append(f32_round(acc) / TWO40)
            f64.append(v)
        return np.array(out, np.float32), np.array(f64), sums.ravel()
    if t in (B.Q4_0, B.Q8_0):
        xq, xd = B.quantize_q8_0(x)
        sums = B.block_sums(t, w, xq, rows, cols).reshape(rows, -1)
        dw = B.blocks(t, w, rows, cols)[..., 0:2].copy().view(np.float16)[..., 0]
        dx = xd.view(np.float16)
        out, f64 = [], []
        for r in range(rows):
            acc, v = 0, 0.0
            for b in range(sums.shape[1]):
                term = sums[r, b] * frac(dw[r, b]) * frac(dx[b])
                acc += (term * TWO40).__floor__()
                v += float(term)
            out.append(f32_round(acc) / TWO40)
            f64.append(v)
        return np.array(out, np.float32), np.array(f64), sums.ravel()
    xq, xd, xbs = B.quantize_q8_K(x)
    sm = B.block_sums(t, w, xq, rows, cols, xbs).reshape(rows, -1, 2)
    blk = B.blocks(t, w, rows, cols)
    if t == B.Q5_K:
        d = blk[..., 0:2].copy().view(np.float16)[..., 0]
        dmin = blk[..., 2:4].copy().view(np.float16)[..., 0]
    else:
        d = blk[..., 208:210].copy().view(np.float16)[..., 0]
        dmin = np.zeros_like(d)
    out, f64 = [], []
    for r in range(rows):
        acc, v = 0, 0.0
        for b in range(sm.shape[1]):
            ts = sm[r, b, 0] * frac(d[r, b]) * frac(xd[b])
            tm = sm[r, b, 1] * frac(dmin[r, b]) * frac(xd[b])
            acc += (ts * TWO40).__floor__() - (tm * TWO40).__floor__()
            v += float(ts - tm)
        out.append(f32_round(acc) / TWO40)
        f64.append(v)
    return np.array(out, np.float32), np.array(f64), sm.ravel()


@pytest.mark.parametrize("t,blk", FORMATS)
@pytest.mark.parametrize("source", ["synthetic", "random-bytes"])
def test_fx_gemv_exact_closed_form(orc, gq, t, blk, source):
    rows, cols = 12, 1024
    w = gq.matrix(t, rows, cols, 3, 200 + t) if source == "synthetic" else random_blocks(t, rows, cols, 300 + t)
    x = gq.normal(3, 7, cols)
    y, bs, _ = orc.fx_gemv(t, w, x, rows, cols, blocksums=True)
    want_y, f64, want_bs = canonical_rows(t, w, x, rows, cols)
    assert np.array_equal(bs.astype(np.int64), want_bs.astype(np.int64)), "block sums"
    assert np.array_equal(y.view(np.uint32), want_y.view(np.uint32)), "fixed-point row values"
    assert np.all(np.abs(y - f64) <= 1e-6 + 1e-5 * np.abs(f64))
    # the reference's sequential FP32 path within its own tolerance of the canonical result
    yr, mag = orc.ref_gemv(t, w, x, rows, cols)
    assert all(orc.orc().orc_ref_within_tolerance(float(a), float(b), float(m)) for a, b, m in zip(y, yr, mag))


def test_q8_1_closed_form(orc, gq):
    x = gq.normal(0, 3, 2048)
    x[:32] = 0.0
    q, d, s_ = orc.quantize_q8_1(x)
    qw, dw, sw = B.quantize_q8_1(x)
    assert np.array_equal(q, qw) and np.array_equal(d, dw) and np.array_equal(s_, sw)
    assert d[0] == 0 and s_[0] == 0


def q6_K_unit_block(idx: int, qv: int) -> np.ndarray:
    """One Q6_K super-block: d = 1, every group scale 1, every weight 0 except weight idx = qv."""
    blk = np.zeros(210, np.uint8)
    blk[128:192] = 0xAA  # every 2-bit high field = 2: stored 32, weight 0
    blk[192:208] = 1
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    n, l = divmod(idx, 128)
    part, li = divmod(l, 32)
    s = qv + 32
    lo, hi = s & 15, s >> 4
    li_ql = 64 * n + li + (32 if part in (1, 3) else 0)
    if part in (0, 1):
        blk[li_ql] = (blk[li_ql] & 0xF0) | lo
    else:
        blk[li_ql] = (blk[li_ql] & 0x0F) | (lo << 4)
    qh = 128 + 32 * n + li
    shift = 2 * part
    blk[qh] = (int(blk[qh]) & ~(3 << shift) & 0xFF) | (hi << shift)
    return blk


def q5_K_unit_block(idx: int, qv: int, mins: int) -> np.ndarray:
    """One Q5_K super-block: d = dmin = 1, every sub-block scale 1 and min `mins`, weights 0 except idx = qv."""
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([1.0], np.float16).view(np.uint8)
    blk[4:8] = 1  # scales of sub-blocks 0..3
    blk[8:12] = mins  # mins of sub-blocks 0..3
    blk[12:16] = 1 | (mins << 4)  # scale and min of sub-blocks 4..7
    j, r = divmod(idx, 64)
    hi_nib = r >= 32
    byte = 48 + 32 * j + (r % 32)
    blk[byte] = (qv & 15) << 4 if hi_nib else (qv & 15)
    blk[16 + (r % 32)] |= ((qv >> 4) & 1) << (2 * j + (1 if hi_nib else 0))
    return blk


@pytest.mark.parametrize("idx", [0, 77, 200, 255])
def test_k_quant_known_answers(orc, idx):
    """Hand-built super-blocks against x = e_idx: Q8_K gives q = -127, d = -1/127, so y = weight(idx) (to FP32
    rounding of d) and the block sums are exact known integers."""
    x = np.zeros(256, np.float32)
    x[idx] = 1.0
    w6 = q6_K_unit_block(idx, 5)
    assert np.array_equal(B.q6_K(w6, 1, 256)[0][0], np.where(np.arange(256) == idx, 5, 0))
    y, bs, _ = orc.fx_gemv(B.Q6_K, w6, x, 1, 256, blocksums=True)
    assert list(bs) == [5 * -127, 0] and abs(y[0] - 5.0) <= 1e-6
    for mins in (0, 1):
        w5 = q5_K_unit_block(idx, 21, mins)
        y, bs, _ = orc.fx_gemv(B.Q5_K, w5, x, 1, 256, blocksums=True)
        assert list(bs) == [21 * -127, mins * -127]
        assert abs(y[0] - (21.0 - mins)) <= 1e-5
        np.testing.assert_allclose(B.dequantize(B.Q5_K, w5, 1, 256)[0][idx], 21.0 - mins)


# ---------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("t", [2, 3, 8, 13, 14])
def test_ref_gemv_reproduces_reference_vectors(orc, t):
    """The oracle's sequential FP32 path against the reference's own outputs, bit for bit (incl. Q4_1)."""
    g = golden()
    w, x = g[f"gemv{t}_w"], g["gemv_x"]
    y, mag = orc.ref_gemv(t, w, x, 16, 512)
    assert np.array_equal(y.view(np.uint32), g[f"gemv{t}_y"].view(np.uint32))
    assert np.array_equal(mag, g[f"gemv{t}_mag"])
    yf = orc.fx_gemv(t, w, x, 16, 512)  # the canonical path within the reference tolerance of the reference
    o = orc.orc()
    assert all(o.orc_ref_within_tolerance(float(a), float(b), float(m))
               for a, b, m in zip(yf, g[f"gemv{t}_y"], g[f"gemv{t}_mag"]))


@pytest.mark.parametrize("t,blk", FORMATS)
def test_ref_gemv_matches_compiled_reference(orc, gq, t, blk):
    if not orc.ref_available():
        pytest.skip("reference library not built (needs the reference tree)")
    rows, cols = 64, 2048
    w = gq.matrix(t, rows, cols, 4, 50 + t)
    x = gq.normal(4, 9, cols)
    y, mag = orc.ref_gemv(t, w, x, rows, cols)
    yr = np.empty(rows, np.float32)
    mr = np.empty(rows, np.float64)
    orc.ref().refshim_gemv(w.ctypes.data, x.ctypes.data, rows, cols, t, yr.ctypes.data, mr.ctypes.data)
    assert np.array_equal(y.view(np.uint32), yr.view(np.uint32)) and np.array_equal(mag, mr)
