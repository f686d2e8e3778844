"""The GEMM command for 2-4 tokens, which runs as one small-token GEMV launch (every workgroup quantizes the token rows
in its prologue, each lane keeps its activation blocks of every token in registers, and each weight row is
streamed once for all tokens). Every token's output row must equal, bit for bit, the oracle's single-token GEMV of
that row and the GPU's own GEMV command on it. Covered: Q4_0 and Q8_0; 2, 3 and 4 tokens; 512 to 12288 columns
(fewer blocks than lanes, one to six blocks per lane); row counts that are not a multiple of the 8 slices; strided
rows; the SwiGLU pair, residual ADD and SiLU epilogs; the folded per-token norm (with weight, L2 without); block
terms past 2^53 LSB; the routing (one launch here, the quantization and MFMA launches for Q4_1, for 3 tokens of 12288
columns and for an output over the input rows). Q5_K and Q6_K (no MFMA form) run any token count in launches of up
to 4 tokens (2 above 4096 columns), each reading the weights once."""
import numpy as np
import pytest

from test_gpu_ops import assert_bits

pytestmark = pytest.mark.gpu


@pytest.fixture()
def ctx(gq):
    c = gq.Context(act_floats=1 << 21, weight_bytes=1 << 28)
    yield c
    c.close()


def up16(n: int) -> int:
    return (n + 15) // 16 * 16


@pytest.mark.parametrize("fmt", [2, 8])
@pytest.mark.parametrize("rows,cols,ntok", [(1000, 1024, 2), (1000, 1024, 4), (64, 512, 3), (4096, 4096, 2),
                                            (333, 4096, 3), (2000, 4096, 4), (300, 6144, 2), (512, 12288, 2)])
def test_tok_rows_equal_single_token_gemv(gq, orc, ctx, fmt, rows, cols, ntok):
    xs, ys = cols + 16, up16(rows) + 32  # strided token rows
    w = gq.matrix(fmt, rows, cols, 3, 10 + fmt, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(3, 11, ntok * xs) * 2.0
    X, Y, Y1 = 0, up16(ntok * xs), up16(ntok * xs) + up16(ntok * ys)
    ctx.write(X, x)
    print(f"[gemm tok] fmt {fmt} rows {rows} cols {cols} tokens {ntok}", flush=True)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, xs, ys)) == 0, ctx.error()
    assert ctx.launch_count() == 1  # no separate quantization launch
    y = ctx.read(Y, ntok * ys).reshape(ntok, ys)[:, :rows]
    for t in range(ntok):
        want = orc.fx_gemv(fmt, w, x[t * xs:t * xs + cols], rows, cols)
        assert_bits(y[t], want, f"token {t}")
        assert ctx.run(gq.gemv(fmt, rows, cols, off, X + t * xs, Y1)) == 0, ctx.error()
        assert_bits(ctx.read(Y1, rows), y[t], f"GEMV command, token {t}")


@pytest.mark.parametrize("fmt,ntok", [(2, 2), (2, 3), (2, 4), (8, 2), (8, 4)])
def test_tok_epilogs_and_norm(gq, orc, ctx, fmt, ntok):
    rows, cols, eps = 2000, 4096, 1e-6
    wg, wu = gq.matrix(fmt, rows, cols, 4, 20, std=0.02), gq.matrix(fmt, rows, cols, 4, 21, std=0.02)
    og, ou = ctx.upload(fmt, rows, cols, wg), ctx.upload(fmt, rows, cols, wu)
    x = gq.normal(4, 22, ntok * cols) * 3.0
    nw = gq.uniform(4, 23, cols, 0.5, 1.5)
    res = gq.normal(4, 24, ntok * rows)
    X, NW, RES, Y, YG = 0, 1 << 16, 1 << 17, 1 << 18, 1 << 19
    ctx.write(X, x)
    ctx.write(NW, nw)
    ctx.write(RES, res)
    rows_of = lambda a: [a[t * cols:(t + 1) * cols] for t in range(ntok)]
    xn = [orc.rownorm(r, nw, cols, 1, eps) for r in rows_of(x)]
    xl2 = [orc.rownorm(r, None, cols, 1, eps, gq.NORM_L2 | gq.NORM_NO_WEIGHT) for r in rows_of(x)]
    g = [orc.fx_gemv(fmt, wg, r, rows, cols) for r in xn]
    u = [orc.fx_gemv(fmt, wu, r, rows, cols) for r in xn]
    norm = dict(norm_w=NW, eps=eps, norm_flags=gq.NORM_DEFER)
    print(f"[gemm tok] epilogs fmt {fmt} tokens {ntok}", flush=True)
    cmd = (gq.gemm(fmt, rows, cols, og, X, YG, ntok, cols, rows, gq.GEMV_SWIGLU, **norm) +
           gq.gemm(fmt, rows, cols, ou, X, Y, ntok, cols, rows, **norm))
    assert ctx.run(cmd) == 0, ctx.error()
    assert ctx.launch_count() == 1
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.silu_mul(g[t], u[t]), f"swiglu token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, og, X, Y, ntok, cols, rows, gq.GEMV_ADD, RES, rows, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], g[t] + res[t * rows:(t + 1) * rows], f"add token {t}")
    # the residual is the output itself (y = y + W x, rows of each token in place)
    ctx.write(Y, res)
    assert ctx.run(gq.gemm(fmt, rows, cols, og, X, Y, ntok, cols, rows, gq.GEMV_ADD, Y, rows, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], g[t] + res[t * rows:(t + 1) * rows], f"in-place add token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, ou, X, Y, ntok, cols, rows, gq.GEMV_SILU, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.unary(u[t], 1), f"silu token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, og, X, Y, ntok, cols, rows, eps=eps,
                           norm_flags=gq.NORM_DEFER | gq.NORM_L2 | gq.NORM_NO_WEIGHT)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.fx_gemv(fmt, wg, xl2[t], rows, cols), f"l2 token {t}")


@pytest.mark.parametrize("fmt,ntok", [(2, 3), (8, 4), (2, 2)])
def test_tok_huge_activations_exact(gq, orc, ctx, fmt, ntok):
    """Outliers of 3e5 in some tokens' rows drive block terms to 2^54 LSB: those waves sum their terms in two FP64
    parts, and every token row still equals the oracle's exact int64 sums."""
    rows, cols = 300, 4096
    w = gq.matrix(fmt, rows, cols, 6, 40 + fmt, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(6, 41, ntok * cols)
    for t in range(0, ntok, 2):
        x[t * cols + np.array([5, 1000, 2047, 4095])] = np.array([1, -1, 1, -1], np.float32) * 3e5
    X, Y = 0, ntok * cols
    ctx.write(X, x)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, 512)) == 0, ctx.error()
    assert ctx.launch_count() == 1
    y = ctx.read(Y, ntok * 512).reshape(ntok, 512)[:, :rows]
    for t in range(ntok):
        want = orc.fx_gemv(fmt, w, x[t * cols:(t + 1) * cols], rows, cols)
        assert_bits(y[t], want, f"token {t}")
        if t % 2 == 0:
            assert np.abs(want).max() > 1e3  # the outlier blocks dominate these rows


def test_tok_routing(gq, orc, ctx):
    """Q4_1 weights, 3 tokens of 12288 columns and an output over the input rows keep the quantization launch and
    the MFMA batched GEMV (two launches); their rows are the same bits."""
    for fmt, rows, cols, ntok, over in ((3, 512, 4096, 2, False), (2, 256, 12288, 3, False), (2, 512, 512, 4, True)):
        w = gq.matrix(fmt, rows, cols, 9, 80 + fmt, std=0.02)
        off = ctx.upload(fmt, rows, cols, w)
        x = gq.normal(9, 81, ntok * cols)
        X = 0
        Y = X if over else up16(ntok * cols)
        ctx.write(X, x)
        print(f"[gemm tok] routing fmt {fmt} cols {cols} tokens {ntok} over {over}", flush=True)
        assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, rows)) == 0, ctx.error()
        assert ctx.launch_count() == 2
        y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
        for t in range(ntok):
            assert_bits(y[t], orc.fx_gemv(fmt, w, x[t * cols:(t + 1) * cols], rows, cols), f"fmt {fmt} token {t}")


@pytest.mark.parametrize("fmt", [13, 14])
@pytest.mark.parametrize("rows,cols,ntok", [(1000, 4096, 1), (333, 4096, 4), (1000, 4096, 9), (700, 12288, 3),
                                            (256, 2048, 6)])
def test_tok_k_quant_rows(gq, orc, ctx, fmt, rows, cols, ntok):
    xs, ys = cols + 16, up16(rows) + 16
    w = gq.matrix(fmt, rows, cols, 5, 30 + fmt, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(5, 31, ntok * xs) * 2.0
    X, Y, Y1 = 0, up16(ntok * xs), up16(ntok * xs) + up16(ntok * ys)
    ctx.write(X, x)
    print(f"[gemm tok] k-quant fmt {fmt} rows {rows} cols {cols} tokens {ntok}", flush=True)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, xs, ys)) == 0, ctx.error()
    per = 4 if cols <= 4096 else 2
    assert ctx.launch_count() == (ntok + per - 1) // per
    y = ctx.read(Y, ntok * ys).reshape(ntok, ys)[:, :rows]
    for t in range(ntok):
        want = orc.fx_gemv(fmt, w, x[t * xs:t * xs + cols], rows, cols)
        assert_bits(y[t], want, f"token {t}")
        if t in (0, ntok - 1):
            assert ctx.run(gq.gemv(fmt, rows, cols, off, X + t * xs, Y1)) == 0, ctx.error()
            assert_bits(ctx.read(Y1, rows), y[t], f"GEMV command, token {t}")


@pytest.mark.parametrize("ntok", [3, 6])
def test_tok_k_quant_norm_and_epilogs(gq, orc, ctx, ntok):
    fmt, rows, cols, eps = 14, 1504, 4096, 1e-6
    w = gq.matrix(fmt, rows, cols, 6, 50, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(6, 51, ntok * cols) * 3.0
    nw = gq.uniform(6, 52, cols, 0.5, 1.5)
    res = gq.normal(6, 53, ntok * rows)
    X, NW, RES, Y = 0, 1 << 16, 1 << 17, 1 << 18
    ctx.write(X, x)
    ctx.write(NW, nw)
    ctx.write(RES, res)
    xn = [orc.rownorm(x[t * cols:(t + 1) * cols], nw, cols, 1, eps) for t in range(ntok)]
    v = [orc.fx_gemv(fmt, w, r, rows, cols) for r in xn]
    norm = dict(norm_w=NW, eps=eps, norm_flags=gq.NORM_DEFER)
    print(f"[gemm tok] k-quant norm and epilogs, tokens {ntok}", flush=True)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, rows, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], v[t], f"norm token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, rows, gq.GEMV_ADD, RES, rows, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], v[t] + res[t * rows:(t + 1) * rows], f"add token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, rows, gq.GEMV_SILU, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.unary(v[t], 1), f"silu token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, rows, eps=eps,
                           norm_flags=gq.NORM_DEFER | gq.NORM_L2 | gq.NORM_NO_WEIGHT)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        xl2 = orc.rownorm(x[t * cols:(t + 1) * cols], None, cols, 1, eps, gq.NORM_L2 | gq.NORM_NO_WEIGHT)
        assert_bits(y[t], orc.fx_gemv(fmt, w, xl2, rows, cols), f"l2 token {t}")
