"""The batched GEMV (GEMM command) on the GPU through the C ABI. Every token's output row must equal, bit for bit, the
oracle's single-token GEMV of that token's row and the GPU's own GEMV command on it: the same activation quantizer,
the same exact block terms, the same epilogs, only the block sums come from int8 MFMAs. Covered: Q4_0, Q4_1 and Q8_0;
1, 5, 16, 17, 20 and 32 tokens (one and two token tiles, padding tokens; 2-4 tokens run as a small-token GEMV,
tests/test_gpu_gemm_tok.py); row counts that are not a multiple of the
16-row tile; 2560, 4096 and 12288 columns; strided rows; the SwiGLU pair, residual ADD and SiLU epilogs; the folded
per-token RMS norm (with and without weight, L2); output rows over the input rows; invalid commands."""
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


@pytest.mark.parametrize("fmt", [2, 3, 8])
@pytest.mark.parametrize("rows,cols,ntok", [(1000, 2560, 1), (1000, 2560, 5), (4096, 4096, 16), (333, 4096, 17),
                                            (512, 12288, 32), (8200, 4096, 20)])
def test_gemm_rows_equal_single_token_gemv(gq, orc, ctx, fmt, rows, cols, ntok):
    xs, ys = cols + 16, up16(rows) + 32  # strided token rows
    w = gq.matrix(fmt, rows, cols, 3, 10 + fmt, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(3, 11, ntok * xs) * 2.0
    X, Y, Y1 = 0, up16(ntok * xs), up16(ntok * xs) + up16(ntok * ys)
    ctx.write(X, x)
    print(f"[gemm] fmt {fmt} rows {rows} cols {cols} tokens {ntok}", flush=True)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, xs, ys)) == 0, ctx.error()
    assert ctx.launch_count() == 2  # the activation quantization, then the weight pass
    y = ctx.read(Y, ntok * ys).reshape(ntok, ys)[:, :rows]
    for t in range(ntok):
        want = orc.fx_gemv(fmt, w, x[t * xs:t * xs + cols], rows, cols)
        assert_bits(y[t], want, f"token {t}")
    for t in sorted({0, ntok // 2, ntok - 1}):  # the single-token GEMV command on the same row
        assert ctx.run(gq.gemv(fmt, rows, cols, off, X + t * xs, Y1)) == 0, ctx.error()
        assert_bits(ctx.read(Y1, rows), y[t], f"GEMV command, token {t}")


@pytest.mark.parametrize("fmt", [2, 3, 8])
@pytest.mark.parametrize("xscale", [3e-3, 1e-5])
def test_tiny_scales_floor_every_term(gq, orc, ctx, fmt, xscale):
    """Small activations: d_w * d_x * 2^40 falls below 2^21, so the scaled block products have fractional parts and
    the floor of every term decides low bits of the sum (at 1e-5 the fp16 activation scales are subnormal). Every
    token row of the GEMM and the GEMV command equal the oracle bit for bit."""
    rows, cols, ntok = 300, 4096, 17
    w = gq.matrix(fmt, rows, cols, 7, 50 + fmt, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(7, 51, ntok * cols) * np.float32(xscale)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.median(amax / 127.0) * 0.01 < 2.0 ** -19  # typical d_x * d_w below 2^-19
    X, Y, Y1 = 0, ntok * cols, ntok * cols + ntok * 512
    ctx.write(X, x)
    print(f"[gemm] tiny scales fmt {fmt} x scale {xscale}", flush=True)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, 512)) == 0, ctx.error()
    y = ctx.read(Y, ntok * 512).reshape(ntok, 512)[:, :rows]
    for t in range(ntok):
        want = orc.fx_gemv(fmt, w, x[t * cols:(t + 1) * cols], rows, cols)
        assert np.count_nonzero(want) > rows // 2
        assert_bits(y[t], want, f"GEMM token {t}")
        if t in (0, ntok - 1):
            assert ctx.run(gq.gemv(fmt, rows, cols, off, X + t * cols, Y1)) == 0, ctx.error()
            assert_bits(ctx.read(Y1, rows), want, f"GEMV, token {t}")


@pytest.mark.parametrize("fmt,outlier", [(2, 3e5), (8, 3e5), (3, 2e4)])
def test_huge_activations_exact(gq, orc, ctx, fmt, outlier):
    """Activations with outliers (block scales up to 2362): block terms reach 2^54 LSB, beyond the 2^53 LSB inside
    which the kernels' FP64 partial sums are exact. The GEMV command and the GEMM's every token row still equal the
    oracle's exact int64 sums bit for bit at FP32 (a partial sum can lose a few LSB of 2^-40, which moves the FP32
    result only at a rounding boundary). (Q4_1 keeps its Q8_1 sums, fp16(sum * d), finite: outliers of 2e4.)"""
    rows, cols, ntok = 300, 4096, 20
    w = gq.matrix(fmt, rows, cols, 6, 40 + fmt, std=0.02)
    off = ctx.upload(fmt, rows, cols, w)
    x = gq.normal(6, 41, ntok * cols)
    for t in range(0, ntok, 3):  # some tokens carry outliers, of both signs, in several blocks
        x[t * cols + np.array([5, 1000, 2047, 4095])] = np.array([1, -1, 1, -1], np.float32) * outlier
    X, Y, Y1 = 0, ntok * cols, ntok * cols + ntok * 512
    ctx.write(X, x)
    assert ctx.run(gq.gemm(fmt, rows, cols, off, X, Y, ntok, cols, 512)) == 0, ctx.error()
    y = ctx.read(Y, ntok * 512).reshape(ntok, 512)[:, :rows]
    for t in range(ntok):
        want = orc.fx_gemv(fmt, w, x[t * cols:(t + 1) * cols], rows, cols)
        assert_bits(y[t], want, f"GEMM token {t}")
        if t % 3 == 0:
            assert ctx.run(gq.gemv(fmt, rows, cols, off, X + t * cols, Y1)) == 0, ctx.error()
            assert_bits(ctx.read(Y1, rows), want, f"GEMV, token {t}")
            assert np.abs(want).max() > outlier / 300.0  # the outlier blocks dominate these rows


def _q4_0_block(d_bits: int, nibbles) -> bytes:
    """One Q4_0 block: fp16 d, then byte j holding element j (low nibble) and element j + 16 (high nibble)."""
    q = np.asarray(nibbles, np.uint8)
    return int(d_bits).to_bytes(2, "little") + bytes((q[:16] | (q[16:] << 4)).tolist())


def test_fp64_partial_past_2_53_is_exact(gq, orc, ctx):
    """Rows whose FP64 partial sums would drop low bits: a block term of -260096 * 2^40 LSB and a term of 3 LSB in one
    partial (row 0: one GEMV lane, blocks 0 and 64; row 1: one GEMM wave's round, blocks 0 and 2), cancelled by
    +260096 * 2^40 in another partial. In FP64 the 3 is lost (the ulp at 2^58 is 64) and the row would be 0; the
    kernels see the matrix's term bound and the activation's scales reach 2^53 LSB and sum those terms in int64, so
    the row is 3 * 2^-40, the oracle's exact sum. Other rows are random."""
    rows, cols = 64, 4096
    nb = cols // 32
    big_neg, big_pos, tiny, zero = 0x3400, 0xB400, 0x0001, 0x0000  # fp16: 0.25, -0.25, 2^-24, 0
    all8, plus1 = [0] * 32, [8] * 32  # all8: every weight -8; plus1: +1 at element 1, 0 elsewhere
    plus1[1] = 9
    w = bytearray(gq.matrix(gq.Q4_0, rows, cols, 7, 60, std=0.02).tobytes())
    row_bytes = nb * 18

    def set_row(r, blocks):
        for b in range(nb):
            d, q = blocks.get(b, (zero, [8] * 32))
            w[r * row_bytes + b * 18:r * row_bytes + (b + 1) * 18] = _q4_0_block(d, q)

    set_row(0, {0: (big_neg, all8), 1: (big_pos, all8), 64: (tiny, plus1)})
    set_row(1, {0: (big_neg, all8), 2: (tiny, plus1), 4: (big_pos, all8)})
    w = np.frombuffer(bytes(w), np.uint8)
    x = np.zeros(cols, np.float32)
    for b in (0, 1, 4):  # d_x = 4064 / 127 = 32, every quant 127
        x[32 * b:32 * b + 32] = 4064.0
    for b in (2, 64):  # d_x = 2^-16, quants 127 and 3
        x[32 * b] = 127 * 2.0 ** -16
        x[32 * b + 1] = 3 * 2.0 ** -16
    want = orc.fx_gemv(gq.Q4_0, w, x, rows, cols)
    assert want[0] == want[1] == np.float32(3 * 2.0 ** -40)
    off = ctx.upload(gq.Q4_0, rows, cols, w)
    X, Y = 0, 8192
    xt = np.concatenate([x, gq.normal(7, 61, cols)])  # a second token for the GEMM
    ctx.write(X, xt)
    assert ctx.run(gq.gemv(gq.Q4_0, rows, cols, off, X, Y)) == 0, ctx.error()
    assert_bits(ctx.read(Y, rows), want, "GEMV")
    assert ctx.run(gq.gemm(gq.Q4_0, rows, cols, off, X, Y, 2, cols, 64)) == 0, ctx.error()
    y = ctx.read(Y, 2 * 64).reshape(2, 64)
    assert_bits(y[0], want, "GEMM token 0")
    assert_bits(y[1], orc.fx_gemv(gq.Q4_0, w, xt[cols:], rows, cols), "GEMM token 1")


@pytest.mark.parametrize("fmt", [2, 3, 8])
def test_gemm_epilogs_and_norm(gq, orc, ctx, fmt):
    rows, cols, ntok, eps = 2000, 4096, 9, 1e-6
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
    # SwiGLU pair on the normalized rows
    cmd = (gq.gemm(fmt, rows, cols, og, X, YG, ntok, cols, rows, gq.GEMV_SWIGLU, **norm) +
           gq.gemm(fmt, rows, cols, ou, X, Y, ntok, cols, rows, **norm))
    assert ctx.run(cmd) == 0, ctx.error()
    assert ctx.launch_count() == 2
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.silu_mul(g[t], u[t]), f"swiglu token {t}")
    # residual ADD and SiLU on the same normalized rows
    assert ctx.run(gq.gemm(fmt, rows, cols, og, X, Y, ntok, cols, rows, gq.GEMV_ADD, RES, rows, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], g[t] + res[t * rows:(t + 1) * rows], f"add token {t}")
    assert ctx.run(gq.gemm(fmt, rows, cols, ou, X, Y, ntok, cols, rows, gq.GEMV_SILU, **norm)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.unary(u[t], 1), f"silu token {t}")
    # the L2 norm without weight
    assert ctx.run(gq.gemm(fmt, rows, cols, og, X, Y, ntok, cols, rows, eps=eps,
                           norm_flags=gq.NORM_DEFER | gq.NORM_L2 | gq.NORM_NO_WEIGHT)) == 0, ctx.error()
    y = ctx.read(Y, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.fx_gemv(fmt, wg, xl2[t], rows, cols), f"l2 token {t}")
    # the same as a deferred RMSNORM + GEMV command per token
    for t in (0, ntok - 1):
        c = gq.rmsnorm(cols, X + t * cols, NW, YG, eps, flags=gq.NORM_DEFER) + gq.gemv(fmt, rows, cols, og, YG, YG + 8192)
        assert ctx.run(c) == 0, ctx.error()
        assert_bits(ctx.read(YG + 8192, rows), g[t], f"deferred norm GEMV token {t}")


def test_gemm_output_over_input(gq, orc, ctx):
    """Output rows written over the input rows (the quantization reads every row first)."""
    rows, cols, ntok = 512, 512, 7
    w = gq.matrix(2, rows, cols, 5, 30)
    off = ctx.upload(2, rows, cols, w)
    x = gq.normal(5, 31, ntok * cols)
    ctx.write(0, x)
    assert ctx.run(gq.gemm(2, rows, cols, off, 0, 0, ntok, cols, rows)) == 0, ctx.error()
    y = ctx.read(0, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y[t], orc.fx_gemv(2, w, x[t * cols:(t + 1) * cols], rows, cols), f"token {t}")


def test_gemm_invalid_commands_rejected(gq, ctx):
    w = gq.matrix(2, 64, 1024, 6, 40)
    off = ctx.upload(2, 64, 1024, w)
    wk = gq.matrix(14, 64, 1024, 6, 41)
    ok = ctx.upload(14, 64, 1024, wk)
    good = gq.gemm(2, 64, 1024, off, 0, 65536, 4, 1024, 64)
    assert ctx.run(good) == 0, ctx.error()
    bad = [
        gq.gemm(14, 64, 1024, ok, 0, 65536, 4, 1024, 64, gq.GEMV_SWIGLU),         # K-quant SwiGLU pair
        gq.gemm(14, 64, 1024, ok, 0, 0, 4, 1024, 64),                             # K-quant output over its rows
        gq.gemm(2, 64, 1024, off, 0, 65536, 0, 1024, 64),                         # no tokens
        gq.gemm(2, 64, 1024, off, 0, 65536, gq.GEMM_MAX_TOK + 1, 1024, 64),       # too many tokens
        gq.gemm(2, 64, 1024, off, 0, 65536, 4, 1000, 64),                         # stride below cols
        gq.gemm(2, 64, 1024, off, 0, 65536, 4, 1024, 48),                         # output stride below rows
        gq.gemm(2, 64, 1024, off, 0, ctx.act_floats - 64, 4, 1024, 64),          # output out of range
        gq.gemm(2, 64, 1024, off, 0, 65536, 4, 1024, 64, gq.GEMV_CONV),           # unsupported epilog
        gq.gemm(2, 64, 1024, off, 0, 65536, 4, 1024, 64, gq.GEMV_SWIGLU),         # SwiGLU without its u
        gq.gemm(2, 64, 1024, off + 1, 0, 65536, 4, 1024, 64),                     # unknown weight
        gq.gemm(2, 64, 1024, off, 0, 65536, 4, 1024, 64, gq.GEMV_ADD, 3, 64),     # misaligned residual
    ]
    for i, c in enumerate(bad):
        assert ctx.run(good + c) == 3, (i, ctx.error())  # nothing runs; the first bad command is slot 3


def test_gemm_reuses_quantized_rows_until_overwritten(gq, orc, ctx):
    """Consecutive GEMMs on the same rows and norm quantize them once; a GEMM whose output overwrites those rows
    makes the next one quantize again (its result is that of the new rows)."""
    rows, cols, ntok = 512, 512, 6
    w1, w2 = gq.matrix(2, rows, cols, 7, 50), gq.matrix(8, rows, cols, 7, 51)
    o1, o2 = ctx.upload(2, rows, cols, w1), ctx.upload(8, rows, cols, w2)
    x = gq.normal(7, 52, ntok * cols)
    X, Y1, Y2 = 0, 8192, 16384
    ctx.write(X, x)
    assert ctx.run(gq.gemm(2, rows, cols, o1, X, Y1, ntok, cols, rows) +
                   gq.gemm(8, rows, cols, o2, X, Y2, ntok, cols, rows)) == 0, ctx.error()
    assert ctx.launch_count() == 3  # one quantization, two weight passes
    xr = [x[t * cols:(t + 1) * cols] for t in range(ntok)]
    y1 = ctx.read(Y1, ntok * rows).reshape(ntok, rows)
    y2 = ctx.read(Y2, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        assert_bits(y1[t], orc.fx_gemv(2, w1, xr[t], rows, cols), f"first GEMM token {t}")
        assert_bits(y2[t], orc.fx_gemv(8, w2, xr[t], rows, cols), f"second GEMM token {t}")
    # the first GEMM now writes over x (rows == cols): the second must see the new rows
    ctx.write(X, x)
    assert ctx.run(gq.gemm(2, rows, cols, o1, X, X, ntok, cols, rows) +
                   gq.gemm(8, rows, cols, o2, X, Y2, ntok, cols, rows)) == 0, ctx.error()
    assert ctx.launch_count() == 4
    y2 = ctx.read(Y2, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        xn = orc.fx_gemv(2, w1, xr[t], rows, cols)
        assert_bits(y2[t], orc.fx_gemv(8, w2, xn, rows, cols), f"after overwrite token {t}")


@pytest.mark.parametrize("ntok", [3, 20])
def test_gemm_group_of_members(gq, orc, ctx, ntok):
    """Consecutive GEMMs of one format on the same quantized rows run as one launch (up to four members, each with its
    own rows, output and epilog; rows that are not whole 16-row tiles); an output that overlaps an earlier member's
    output or feeds its residual starts a new launch, so the commands' order still decides the result. With 3 tokens
    the groups are small-token GEMV launches, which quantize the rows themselves (no quantization launch)."""
    q = 0 if ntok <= 4 else 1  # the quantization launch of the MFMA path
    cols, eps = 1024, 1e-6
    shapes = [(100, gq.GEMV_SILU), (33, 0), (512, gq.GEMV_ADD), (16, 0), (48, 0)]
    ws = [gq.matrix(2, r, cols, 8, 60 + j, std=0.02) for j, (r, _) in enumerate(shapes)]
    offs = [ctx.upload(2, r, cols, w) for (r, _), w in zip(shapes, ws)]
    x = gq.normal(8, 70, ntok * cols) * 2.0
    nw = gq.uniform(8, 71, cols, 0.5, 1.5)
    res = gq.normal(8, 72, ntok * 512)
    X, NW, RES = 0, 1 << 16, 1 << 17
    Y = [(1 << 18) + j * (1 << 15) for j in range(len(shapes))]
    ctx.write(X, x)
    ctx.write(NW, nw)
    ctx.write(RES, res)
    norm = dict(norm_w=NW, eps=eps, norm_flags=gq.NORM_DEFER)

    def cmd(j, y, ys=None):
        r, e = shapes[j]
        ys = up16(r) if ys is None else ys
        if e == gq.GEMV_ADD:
            return gq.gemm(2, r, cols, offs[j], X, y, ntok, cols, ys, e, RES, 512, **norm)
        return gq.gemm(2, r, cols, offs[j], X, y, ntok, cols, ys, e, **norm)

    xn = [orc.rownorm(x[t * cols:(t + 1) * cols], nw, cols, 1, eps) for t in range(ntok)]

    def want(j, t):
        r, e = shapes[j]
        v = orc.fx_gemv(2, ws[j], xn[t], r, cols)
        if e == gq.GEMV_SILU:
            return orc.unary(v, 1)
        if e == gq.GEMV_ADD:
            return v + res[t * 512:t * 512 + r]
        return v

    assert ctx.run(sum((cmd(j, Y[j]) for j in range(5)), [])) == 0, ctx.error()
    assert ctx.launch_count() == q + 2  # (the quantization,) a group of four, then the fifth member's own launch
    for j, (r, _) in enumerate(shapes):
        got = ctx.read(Y[j], ntok * up16(r)).reshape(ntok, up16(r))[:, :r]
        for t in range(ntok):
            assert_bits(got[t], want(j, t), f"member {j} token {t}")
    # the second output overlaps the first's (rows 48..80 of every token): two launches, the later command's values
    # win where they overlap
    assert ctx.run(cmd(0, Y[0]) + cmd(1, Y[0] + 48, ys=112)) == 0, ctx.error()
    assert ctx.launch_count() == q + 2
    got = ctx.read(Y[0], ntok * 112).reshape(ntok, 112)[:, :100]
    for t in range(ntok):
        first = want(0, t)
        assert_bits(got[t, :48], first[:48], f"overlap: rows before, token {t}")
        assert_bits(got[t, 48:81], want(1, t), f"overlap: the later command's rows, token {t}")
        assert_bits(got[t, 81:], first[81:], f"overlap: rows after, token {t}")
    # a member whose residual is an earlier member's output (rows 0..15 of every token): a new launch that adds the
    # new values
    assert ctx.run(cmd(3, RES, ys=512) + cmd(2, Y[2])) == 0, ctx.error()
    assert ctx.launch_count() == q + 2
    got = ctx.read(Y[2], ntok * 512).reshape(ntok, 512)
    for t in range(ntok):
        r16 = want(3, t)
        res_t = res[t * 512:t * 512 + 512].copy()
        res_t[:16] = r16
        assert_bits(got[t], orc.fx_gemv(2, ws[2], xn[t], 512, cols) + res_t, f"residual after member, token {t}")


# An activation block whose Q8_1 sum s = fp16(sum(q) * d) falls on an fp16 tie: the FP32 product sum * d is exactly
# halfway between two fp16 values (6.986328125, sum 160), so it must round to even (0x46fc); rounding the exact
# product once instead (a multiply fused into the conversion) gives 0x46fd.
TIE_BLOCK = [3205777222,1076638343,1070347095,1067654670,3217158963,3226446569,1061787943,1076228752,1066425760,3220559183,1019700895,1043250633,3213579224,1083621115,3201029249,1060894146,3219640152,3206132165,1052879561,1085371367,3231080033,3228257810,3216771732,3210901803,3208034114,1058367542,1068577287,3187710123,1073944164,3212800904,1075424494,1076089562]


def test_q4_1_sum_on_fp16_tie(gq, orc, ctx):
    rows, cols, ntok = 64, 512, 3
    blk = np.array(TIE_BLOCK, np.uint32).view(np.float32)
    x = np.zeros(ntok * cols, np.float32)
    for t in range(ntok):
        x[t * cols + 32 * (5 + t):t * cols + 32 * (6 + t)] = blk
    q = np.zeros(32, np.int8)
    d16, s16 = np.zeros(1, np.uint16), np.zeros(1, np.uint16)
    orc.orc().orc_quantize_q8_1(blk.ctypes.data, 32, q.ctypes.data, d16.ctypes.data, s16.ctypes.data)
    assert int(q.astype(np.int32).sum()) == 160 and s16[0] == 0x46fc  # the oracle rounds the tie to even
    w = gq.matrix(3, rows, cols, 8, 60, std=0.02)
    off = ctx.upload(3, rows, cols, w)
    ctx.write(0, x)
    assert ctx.run(gq.gemm(3, rows, cols, off, 0, 8192, ntok, cols, rows)) == 0, ctx.error()
    y = ctx.read(8192, ntok * rows).reshape(ntok, rows)
    for t in range(ntok):
        want = orc.fx_gemv(3, w, x[t * cols:(t + 1) * cols], rows, cols)
        assert_bits(y[t], want, f"GEMM token {t}")
        assert ctx.run(gq.gemv(3, rows, cols, off, t * cols, 16384)) == 0, ctx.error()
        assert_bits(ctx.read(16384, rows), want, f"GEMV token {t}")
