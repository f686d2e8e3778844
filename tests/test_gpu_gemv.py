"""GEMV parity on the GPU through the C ABI: bit-exact against the oracle's fixed-point arithmetic (the reference
kernel's, fpga/src/gemvqw_engine.h:352-445), per-block integer sums bit-exact, and within the reference's own
tolerance (fpga/src/gemvq_ref.h:267-272) of its sequential FP32 CPU path."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 0


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.nonzero(bits(got) != bits(want))[0]
    assert bad.size == 0, f"{what}: {bad.size} of {want.size} differ, first {bad[:5]} got {got[bad[:5]]} want {want[bad[:5]]}"


def run_gemv(gq, t, rows, cols, w, x, blocksums=False):
    act = ((cols + 15) // 16 * 16) + ((rows + 15) // 16 * 16) + 64
    with gq.Context(act_floats=act, weight_bytes=w.size + 4096) as ctx:
        off = ctx.upload(t, rows, cols, w)
        x_off, y_off = 0, (cols + 15) // 16 * 16
        ctx.write(x_off, x)
        dbg = None
        if blocksums:
            nbs = rows * (cols // 256 * 2 if t in (gq.Q5_K, gq.Q6_K) else cols // 32)
            dbg = np.zeros(nbs, np.int32)
            ctx.debug_blocksums(dbg)
        assert ctx.run(gq.gemv(t, rows, cols, off, x_off, y_off)) == 0, ctx.error()
        y = ctx.read(y_off, rows)
    return (y, dbg) if blocksums else y


@pytest.mark.parametrize("t,rows,cols", [
    (2, 64, 256), (2, 100, 2560), (2, 33, 4096), (2, 64, 12288), (2, 16, 16384), (2, 17, 9728),
    (3, 64, 256), (3, 100, 4096), (3, 17, 12288),
    (8, 64, 256), (8, 100, 2560), (8, 40, 9728), (8, 31, 4096),
    (13, 64, 256), (13, 50, 4096), (13, 20, 12288),
    (14, 64, 256), (14, 50, 4096), (14, 20, 12288), (14, 7, 16384),
    # Q4_0 / Q4_1 / Q8_0 rows of an odd number of 32-column blocks (one block, three, five, 81, 129)
    (2, 37, 32), (3, 9, 96), (8, 70, 160), (2, 33, 2592), (8, 5, 4128), (3, 21, 800),
])
def test_gemv_formats_bitexact(gq, orc, t, rows, cols):
    w = gq.matrix(t, rows, cols, SEED, 1 + t, std=0.02)
    x = gq.normal(SEED, 100 + t, cols)
    y, dbg = run_gemv(gq, t, rows, cols, w, x, blocksums=True)
    yo, bso, _ = orc.fx_gemv(t, w, x, rows, cols, blocksums=True)
    assert np.array_equal(dbg, bso), f"block sums differ at {np.nonzero(dbg != bso)[0][:5]}"
    assert_bits(y, yo, f"type {t} {rows}x{cols}")
    yr, mag = orc.ref_gemv(t, w, x, rows, cols)
    ok = [orc.orc().orc_ref_within_tolerance(float(a), float(b), float(m)) for a, b, m in zip(y, yr, mag)]
    assert all(ok)


def test_c1_q4_0_gemv(gq, orc):
    """C1: Q4_0 [9728 x 2560] x Q8_0, seed 0."""
    rows, cols = 9728, 2560
    w = gq.matrix(gq.Q4_0, rows, cols, SEED, 1, std=0.02)
    x = gq.normal(SEED, 2, cols)
    y, dbg = run_gemv(gq, gq.Q4_0, rows, cols, w, x, blocksums=True)
    yo, bso, _ = orc.fx_gemv(gq.Q4_0, w, x, rows, cols, blocksums=True)
    assert np.array_equal(dbg, bso)
    assert_bits(y, yo, "C1")
    yr, mag = orc.ref_gemv(gq.Q4_0, w, x, rows, cols)
    err = np.abs(y.astype(np.float64) - yr)
    assert np.all(err <= 1e-6 + 1e-5 * np.abs(yr) + 1e-6 * mag)


def test_gemv_edge_inputs(gq, orc):
    """Zero blocks, a zero vector, exact halves in the activation quantizer, negative scales."""
    rows, cols = 64, 512
    w = gq.matrix(gq.Q4_0, rows, cols, SEED, 7, std=0.02)
    x = gq.normal(SEED, 8, cols)
    x[:32] = 0.0                      # all-zero activation block: d = 0, q = 0
    x[32:64] = np.arange(32) - 15.5   # amax 16.5: many x / d land near .5
    x[64] = 127.0 * 3                 # d = 3 exactly: x / d integral
    y = run_gemv(gq, gq.Q4_0, rows, cols, w, x)
    assert_bits(y, orc.fx_gemv(gq.Q4_0, w, x, rows, cols), "edge")
    y0 = run_gemv(gq, gq.Q4_0, rows, cols, w, np.zeros(cols, np.float32))
    assert np.all(bits(y0) == 0)
    # Q8_0 weights with negative fp16 scales (the sign goes through the fixed-point term)
    w8 = gq.matrix(gq.Q8_0, rows, cols, SEED, 9, std=0.02).reshape(rows, -1).copy()
    w8.reshape(rows, cols // 32, 34)[:, ::3, 1] |= 0x80  # flip the sign bit of every third block scale
    w8 = w8.ravel()
    y8 = run_gemv(gq, gq.Q8_0, rows, cols, w8, x)
    assert_bits(y8, orc.fx_gemv(gq.Q8_0, w8, x, rows, cols), "negative scales")


@pytest.mark.parametrize("t", [2, 3, 8, 13, 14])
def test_gemv_against_reference_vectors(gq, t):
    """The GPU GEMV on the stored inputs against the reference's own CPU results (tests/golden), within the
    reference tolerance |got - ref| <= 1e-6 + 1e-5 |ref| + 1e-6 sum |block terms| (gemvq_ref.h:267-272)."""
    from golden_data import golden

    g = golden()
    y = run_gemv(gq, t, 16, 512, g[f"gemv{t}_w"], g["gemv_x"])
    ref, mag = g[f"gemv{t}_y"].astype(np.float64), g[f"gemv{t}_mag"]
    assert np.all(np.abs(y - ref) <= 1e-6 + 1e-5 * np.abs(ref) + 1e-6 * mag)


@pytest.mark.parametrize("t,rows,cols", [(14, 151936, 4096), (13, 12288, 4096)])
def test_c3_k_quant_full_shapes(gq, orc, t, rows, cols):
    """C3 at its real shapes: the Q6_K output head [151936 x 4096] and a Q5_K projection [12288 x 4096] against
    Q8_K activations. Every row's result and block sums are checked against the oracle on a sample of rows (rows are
    independent), and those rows against the reference's sequential path within its tolerance."""
    w = gq.matrix(t, rows, cols, SEED, 30 + t, std=0.02)
    x = gq.normal(SEED, 40 + t, cols)
    y, dbg = run_gemv(gq, t, rows, cols, w, x, blocksums=True)
    rb = gq.row_bytes(t, cols)
    sample = np.arange(0, rows, 37)
    ws = w.reshape(rows, rb)[sample].ravel()
    yo, bso, _ = orc.fx_gemv(t, ws, x, len(sample), cols, blocksums=True)
    assert_bits(y[sample], yo, f"C3 type {t}")
    assert np.array_equal(dbg.reshape(rows, -1)[sample].ravel(), bso)
    yr, mag = orc.ref_gemv(t, ws, x, len(sample), cols)
    assert np.all(np.abs(y[sample].astype(np.float64) - yr) <= 1e-6 + 1e-5 * np.abs(yr) + 1e-6 * mag)
