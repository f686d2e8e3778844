"""The reference-arithmetic mode (gemvq_set_arith(GEMVQ_ARITH_REFERENCE)) on the GPU through the C ABI, bit for bit
against the oracle's restatement of the reference's CPU path (fpga/src/gemvq_ref.h: sequential FP32 GEMV rows,
double sums of squares, sequential DeltaNet dots), with the correctly rounded exp / log in place of libm's."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS = 1e-6


def assert_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size}/{want.size} differ; first {bad[:4]}: got {got[bad[:4]]} want {want[bad[:4]]}"


@pytest.fixture()
def ctx(gq):
    c = gq.Context(act_floats=1 << 20, weight_bytes=1 << 27, state_rows=64 * 128)
    c.set_arith(gq.ARITH_REFERENCE)
    yield c
    c.close()


@pytest.mark.parametrize("fn", [0, 1])
def test_correctly_rounded_math_on_every_input(gq, orc, ctx, fn):
    """The device's exp (0) / log (1) on all 2^32 binary32 inputs: block hashes equal the oracle's."""
    print(f"[ref] crmath hash fn {fn}", flush=True)
    assert np.array_equal(ctx.crmath_hash(fn), orc.crmath_hash(fn))


@pytest.mark.parametrize("t,rows,cols", [
    (2, 300, 2560), (2, 64, 12288), (2, 129, 512), (8, 257, 2560), (8, 40, 16384), (3, 200, 4096),
    (14, 301, 4096), (14, 33, 12288), (13, 130, 4096), (13, 50, 2048),
    (2, 37, 96), (8, 70, 2592), (3, 11, 160), (8, 9, 32),  # odd numbers of 32-column blocks
    (14, 36000, 4096),  # Q6_K rows enough for several batches per wave (each requested before the one before is added)
])
def test_gemv_rows(gq, orc, ctx, t, rows, cols):
    """GEMV rows in every weight format equal gemvq_ref.h's sequential FP32 rows (orc_ref_gemv, itself pinned to
    the compiled reference by the golden vectors), bit for bit; activations of varied scale."""
    w = gq.matrix(t, rows, cols, seed=3, stream=t, std=0.02)
    x = gq.normal(3, 100 + t, cols) * np.float32(3.0)
    off = ctx.upload(t, rows, cols, w)
    ctx.write(0, x)
    assert ctx.run(gq.gemv(t, rows, cols, off, 0, 32768)) == 0, ctx.error()
    assert_bits(ctx.read(32768, rows), orc.ref_gemv(t, w, x, rows, cols)[0], f"type {t}")


def test_deferred_norm_and_epilogs(gq, orc, ctx):
    """The deferred RMS norm folded into a GEMV group (its scale from the reference's double sum), and the SwiGLU,
    ADD, SiLU, CONV and ARGMAX epilogs in the reference's arithmetic."""
    E, F, R = 2048, 1536, 512
    x = gq.normal(4, 1, E)
    nw = gq.uniform(4, 2, E, 0.5, 1.5)
    res = gq.normal(4, 3, R)
    cst = gq.normal(4, 4, 3 * R)
    cw = gq.normal(4, 5, 4 * R, std=0.5)
    wg, wu, wa, wc, ws = (gq.matrix(2, rows, E, seed=4, stream=10 + i, std=0.02) for i, rows in enumerate((F, F, R, R, R)))
    og, ou, oa, oc, os_ = (ctx.upload(2, r, E, w) for r, w in ((F, wg), (F, wu), (R, wa), (R, wc), (R, ws)))
    O = dict(x=0, nw=4096, xn=8192, res=12288, cst=16384, cw=20480, g=24576, a=28672, a2=32768, c=36864, c2=40960,
             s=45056, cnew=49152, key=53248)
    for k, v in (("x", x), ("nw", nw), ("res", res), ("cst", cst), ("cw", cw)):
        ctx.write(O[k], v)
    cmds = [gq.rmsnorm(E, O["x"], O["nw"], O["xn"], EPS, flags=gq.NORM_DEFER),
            gq.gemv(2, F, E, og, O["xn"], 0, gq.GEMV_SWIGLU), gq.gemv(2, F, E, ou, O["xn"], O["g"]),
            gq.gemv(2, R, E, oa, O["xn"], O["a"], gq.GEMV_ADD) + gq.add(R, O["a"], O["res"], O["a2"]),
            gq.gemv(2, R, E, oc, O["xn"], O["c"], gq.GEMV_CONV) + gq.conv(R, O["c"], O["cw"], O["c2"], O["cst"], O["cnew"]),
            gq.gemv(2, R, E, os_, O["xn"], O["s"], gq.GEMV_SILU)]
    assert ctx.run([w for c in cmds for w in c]) == 0, ctx.error()
    xn = orc.ref_rownorm(x, nw, E, 1, EPS)
    g, u, a, c, s = (orc.ref_gemv(2, w, xn, r, E)[0] for w, r in ((wg, F), (wu, F), (wa, R), (wc, R), (ws, R)))
    assert_bits(ctx.read(O["g"], F), orc.ref_silu_mul_cr(g, u), "SwiGLU")
    assert_bits(ctx.read(O["a2"], R), a + res, "ADD")
    y, ns = orc.ref_conv_cr(cst, c, cw)
    assert_bits(ctx.read(O["c2"], R), y, "CONV")
    assert_bits(ctx.read(O["cnew"], 3 * R), ns, "CONV state")
    assert_bits(ctx.read(O["s"], R), orc.ref_unary_cr(s, 1), "SiLU")
    # the head's form: a Q6_K GEMV with the ARGMAX epilog on a normed row
    wh = gq.matrix(14, 3000, 4096, seed=4, stream=20, std=0.02)
    oh = ctx.upload(14, 3000, 4096, wh)
    xh = gq.normal(4, 21, 4096)
    ctx.write(O["x"], xh)
    ctx.write(O["nw"], np.ones(4096, np.float32))
    ctx.write(O["key"], np.zeros(2, np.float32))
    cmds = [gq.rmsnorm(4096, O["x"], O["nw"], O["xn"], EPS, flags=gq.NORM_DEFER),
            gq.gemv(14, 3000, 4096, oh, O["xn"], 60000, gq.GEMV_ARGMAX) + gq.argmax(3000, 60000, O["key"])]
    assert ctx.run([w for c in cmds for w in c]) == 0, ctx.error()
    lg = orc.ref_gemv(14, wh, orc.ref_rownorm(xh, np.ones(4096, np.float32), 4096, 1, EPS), 3000, 4096)[0]
    assert_bits(ctx.read(60000, 3000), lg, "head")
    key = ctx.read(O["key"], 2, np.uint32)
    assert 0xFFFFFFFF - int(key[0]) == int(np.argmax(lg))


@pytest.mark.parametrize("n,rows,flags", [(4096, 1, 0), (128, 32, 0), (128, 16, 1 | 2), (256, 20, 0), (1024, 3, 2)])
def test_rmsnorm_rows(gq, orc, ctx, n, rows, flags):
    x = gq.normal(5, n, n * rows) * np.float32(2.0)
    w = gq.uniform(5, n + 1, n, 0.5, 1.5)
    ctx.write(0, x)
    ctx.write(1 << 18, w)
    assert ctx.run(gq.rmsnorm(n, 0, 1 << 18, 1 << 19, EPS, rows=rows, flags=flags)) == 0, ctx.error()
    assert_bits(ctx.read(1 << 19, n * rows), orc.ref_rownorm(x, w, n, rows, EPS, flags), f"flags {flags}")


def test_rmsnorm_sum_on_a_rounding_boundary(gq, orc, ctx):
    """Squares whose exact sum / n is halfway between two floats (1 + 2^-24): the tree sum cannot decide the
    rounding, so the kernel adds the squares in order, as the reference does (ties to even: 1.0)."""
    n = 4096
    x = np.ones(n, np.float32)
    x[1234] = np.float32(1.0 + 2.0 ** -13)  # its FP32 square is 1 + 2^-12
    assert np.float32(x[1234] * x[1234]) == np.float32(1.0 + 2.0 ** -12)
    w = gq.uniform(5, 7, n, 0.5, 1.5)
    ctx.write(0, x)
    ctx.write(1 << 18, w)
    for flags in (0, 2):
        assert ctx.run(gq.rmsnorm(n, 0, 1 << 18, 1 << 19, EPS, flags=flags)) == 0, ctx.error()
        assert_bits(ctx.read(1 << 19, n), orc.ref_rownorm(x, w, n, 1, EPS, flags), f"flags {flags}")
    # folded into a GEMV's prologue as well
    wq = gq.matrix(2, 256, n, seed=5, stream=8, std=0.02)
    off = ctx.upload(2, 256, n, wq)
    cmds = gq.rmsnorm(n, 0, 1 << 18, 1 << 19, EPS, flags=gq.NORM_DEFER) + gq.gemv(2, 256, n, off, 1 << 19, 1 << 17)
    assert ctx.run(cmds) == 0, ctx.error()
    assert_bits(ctx.read(1 << 17, 256), orc.ref_gemv(2, wq, orc.ref_rownorm(x, w, n, 1, EPS), 256, n)[0], "GEMV")


def test_elementwise(gq, orc, ctx):
    n = 4096
    g = gq.normal(6, 1, n) * np.float32(6.0)
    g[:8] = [0.0, -0.0, 20.0, 20.5, -90.0, 89.0, 1e-30, -1e-30]
    u = gq.normal(6, 2, n)
    ctx.write(0, g)
    ctx.write(8192, u)
    assert ctx.run(gq.silu_mul(n, 0, 8192, 16384)) == 0
    assert_bits(ctx.read(16384, n), orc.ref_silu_mul_cr(g, u), "SILU_MUL")
    assert ctx.run(gq.silu_mul(n, 0, 8192, 16384, sigmoid=True)) == 0
    assert_bits(ctx.read(16384, n), orc.ref_unary_cr(g, 2) * u, "SILU_MUL sigmoid")
    for kind in (1, 2, 3):
        assert ctx.run(gq.unary(n, 0, kind, 16384)) == 0
        assert_bits(ctx.read(16384, n), orc.ref_unary_cr(g, kind), f"UNARY {kind}")


def test_conv_tokens(gq, orc, ctx):
    ch, ntok = 1024, 3
    st = gq.normal(7, 1, 3 * ch)
    w = gq.normal(7, 2, 4 * ch, std=0.5)
    x = gq.normal(7, 3, ntok * ch)
    ctx.write(0, st)
    ctx.write(4096, w)
    ctx.write(8192, x)
    c = gq.conv(ch, 8192, 4096, 16384, 0, 0)
    c[7] |= ntok << 16
    assert ctx.run(c) == 0, ctx.error()
    s = st
    for t in range(ntok):
        y, s = orc.ref_conv_cr(s, x[t * ch:(t + 1) * ch], w)
        assert_bits(ctx.read(16384 + t * ch, ch), y, f"token {t}")
    assert_bits(ctx.read(0, 3 * ch), s, "state")


SCALE = np.float32(1.0) / np.sqrt(np.float32(128))  # the DeltaNet scale as the decoders form it, 1.0f / sqrtf(128)


def _gdn_reference(orc, state, q, k, v, ar, br, dt, a, z, wn, hv, hk, z_silu):
    """ggml's graph around the reference step (qwen35_oracle.c's reference mode): L2 norms, gates, the step, the
    gated RMS norm."""
    S = 128
    qn = orc.ref_rownorm(q, None, S, hk, EPS, 3)
    kn = orc.ref_rownorm(k, None, S, hk, EPS, 3)
    g = orc.ref_unary_cr(ar + dt, 3) * a
    be = orc.ref_unary_cr(br, 2)
    y, st = orc.ref_gdn_cr(state, qn, kn, v, g, be, hv, hk, SCALE)
    yt = orc.ref_rownorm(y, wn, S, hv, EPS, 0)
    return yt * (z if z_silu else orc.ref_unary_cr(z, 1)), st


def boundary_row(n, i):
    """Ones but element i, whose FP32 square is 1 + n 2^-24: the row's sum of squares, n + n 2^-24, lies halfway
    between two floats, and so does its mean over n, 1 + 2^-24 (n a power of two up to 256): no tree sum with an
    error bound decides either rounding, the in-order sum does (ties to even)."""
    x = np.ones(n, np.float32)
    x[i] = np.float32(1.0 + 2.0 ** (-25 + int(np.log2(n))))
    assert np.float32(x[i] * x[i]) == np.float32(1.0 + n * 2.0 ** -24)
    return x


@pytest.mark.parametrize("hv,hk,ntok,z_silu,edge", [(32, 16, 1, True, False), (16, 4, 1, False, False),
                                                    (32, 16, 3, True, False), (16, 4, 2, True, True)])
def test_gdn_layer_step(gq, orc, ctx, hv, hk, ntok, z_silu, edge):
    """The DeltaNet GDN command as the model uses it (L2 q/k, gates from the raw projections, gated output norm),
    for one token and for several in order; edge: the first token's q and k rows of key head 0 with sums of squares
    on a rounding boundary."""
    S = 128
    st0 = gq.normal(8, 1, hv * S * S, std=0.1)
    qkv = gq.normal(8, 2, ntok * (2 * hk + hv) * S)
    if edge:
        qkv[:S] = boundary_row(S, 5)
        qkv[hk * S:hk * S + S] = boundary_row(S, 77)
        assert np.float32(np.sum((qkv[:S] * qkv[:S]).astype(np.float64))) == np.float32(128.0)  # the tie, to even
    ab = gq.normal(8, 3, ntok * 2 * 64)
    dt = gq.normal(8, 4, hv)
    a = -np.abs(gq.normal(8, 5, hv))
    z = gq.normal(8, 6, ntok * hv * S)
    wn = gq.uniform(8, 7, S, 0.5, 1.5)
    ctx.state_write(0, st0)
    ch = (2 * hk + hv) * S
    O = dict(qkv=0, ab=1 << 17, dt=(1 << 17) + 8192, a=(1 << 17) + 8320, z=1 << 18, wn=(1 << 18) + 65536, y=1 << 19)
    for key, val in (("qkv", qkv), ("ab", ab), ("dt", dt), ("a", a), ("z", z), ("wn", wn)):
        ctx.write(O[key], val)
    flags = gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES | (gq.GDN_Z_SILU if z_silu else 0)
    c = gq.gdn(hv, hk, O["qkv"], O["qkv"] + hk * S, O["qkv"] + 2 * hk * S, O["ab"] + 64, O["ab"], O["y"], 0, 0,
               float(SCALE), flags, EPS, EPS, O["wn"], O["z"], O["dt"], O["a"])
    c[16 + 2], c[16 + 3], c[16 + 4] = ntok, ch, 128  # tokens, q / k / v row stride, g / beta row stride
    assert ctx.run(c) == 0, ctx.error()
    st = st0
    for t in range(ntok):
        row = qkv[t * ch:(t + 1) * ch]
        y, st = _gdn_reference(orc, st, row[:hk * S], row[hk * S:2 * hk * S], row[2 * hk * S:], ab[t * 128 + 64:t * 128 + 64 + hv],
                               ab[t * 128:t * 128 + hv], dt, a, z[t * hv * S:(t + 1) * hv * S], wn, hv, hk, z_silu)
        assert_bits(ctx.read(O["y"] + t * hv * S, hv * S), y, f"token {t}")
    assert_bits(ctx.state_read(0, hv * S), st, "state")


@pytest.mark.parametrize("nh,nkv,hd,nrot,npos,edge", [
    (16, 4, 256, 64, 70, False), (6, 2, 128, 128, 3, False),
    (8, 2, 64, 64, 300, False), (4, 1, 32, 32, 20, False), (2, 2, 16, 16, 9, False),  # values staged in 256-position chunks
    (16, 4, 256, 64, 4, True), (6, 2, 128, 128, 3, True),
])
def test_attention(gq, orc, ctx, nh, nkv, hd, nrot, npos, edge):
    """Attention token by token (q / k RMS norm, RoPE, fp16 cache, softmax, sigmoid gate) against the reference
    decoder's attention (the reference's norms, ggml's CPU softmax with double sums); edge: q head 0 and KV head 0
    rows whose mean squares lie on a rounding boundary at every position."""
    n_ctx = 128 if npos <= 128 else 320
    kv = ctx.kv_create(n_ctx, nkv, hd)
    qn = gq.uniform(9, 1, hd, 0.5, 1.5)
    kn = gq.uniform(9, 2, hd, 0.5, 1.5)
    table = np.concatenate([orc.rope_cache(p, nrot, 1e7) for p in range(n_ctx)])
    O = dict(qg=0, k=16384, v=20480, qn=24576, kn=25088, pos=25600, y=26624, cs=32768)
    ctx.write(O["qn"], qn)
    ctx.write(O["kn"], kn)
    ctx.write(O["cs"], table)
    kc = np.zeros((n_ctx, nkv, hd), np.uint16)
    vc = np.zeros((n_ctx, nkv, hd), np.uint16)
    for pos in range(npos):
        qg = gq.normal(9, 100 + pos, 2 * nh * hd)
        k = gq.normal(9, 300 + pos, nkv * hd)
        v = gq.normal(9, 500 + pos, nkv * hd)
        if edge:
            qg[:hd] = boundary_row(hd, 3 + pos)
            k[:hd] = boundary_row(hd, 2 * pos + 1)
        ctx.write(O["qg"], qg)
        ctx.write(O["k"], k)
        ctx.write(O["v"], v)
        ctx.write(O["pos"], np.array([pos], np.int32))
        c = gq.attn(nh, nkv, O["qg"], kv, O["y"], hd, nrot, O["pos"], O["k"], O["v"], 1 / 16, EPS, O["qn"], O["kn"],
                    O["cs"], gate=O["qg"] + hd)
        assert ctx.run(c) == 0, ctx.error()
        cs = table[pos * nrot:(pos + 1) * nrot]
        q = qg.reshape(nh, 2 * hd)[:, :hd].ravel()
        qh = orc.rope(orc.ref_rownorm(q, qn, hd, nh, EPS), cs, nrot, hd, nh)
        kh = orc.rope(orc.ref_rownorm(k, kn, hd, nkv, EPS), cs, nrot, hd, nkv)
        kc[pos] = orc.f2h(kh).reshape(nkv, hd)
        vc[pos] = orc.f2h(v).reshape(nkv, hd)
        if pos in (0, 1, npos - 1, 63, 64, 255, 256, 257):
            att = orc.ref_attn_cr(qh, kc, vc, nh, nkv, hd, pos + 1, 1 / 16)
            gate = qg.reshape(nh, 2 * hd)[:, hd:].ravel()
            assert_bits(ctx.read(O["y"], nh * hd), orc.ref_unary_cr(gate, 2) * att, f"attention at {pos}")
    k_dev, v_dev = ctx.kv_read(kv, 0, npos, nkv * hd)
    assert np.array_equal(k_dev, kc[:npos].ravel()) and np.array_equal(v_dev, vc[:npos].ravel())


@pytest.mark.parametrize("ntok,over", [(3, False), (8, False), (5, True)])
def test_gemm_runs_as_token_gemvs(gq, orc, ctx, ntok, over):
    """A GEMM command in the reference arithmetic: each token row as the GEMV command on it (the per-token norm
    folded, SwiGLU pair and residual epilogs), bit for bit; with `over`, the down projection's outputs are written
    over its own token rows (which the batched command reads before it writes)."""
    E, F = 1024, 2048
    wg, wu, wd = gq.matrix(2, F, E, seed=10, stream=1), gq.matrix(2, F, E, seed=10, stream=2), gq.matrix(2, E, F, seed=10, stream=3)
    og, ou, od = ctx.upload(2, F, E, wg), ctx.upload(2, F, E, wu), ctx.upload(2, E, F, wd)
    x = gq.normal(10, 4, ntok * E)
    nw = gq.uniform(10, 5, E, 0.5, 1.5)
    O = dict(x=0, nw=65536, h=1 << 17, d=1 << 18)
    ctx.write(O["x"], x)
    ctx.write(O["nw"], nw)
    hout = O["h"] if over else O["d"]
    cmds = (gq.gemm(2, F, E, og, O["x"], O["h"], ntok, E, F, gq.GEMV_SWIGLU, norm_w=O["nw"], eps=EPS, norm_flags=gq.NORM_DEFER) +
            gq.gemm(2, F, E, ou, O["x"], O["h"], ntok, E, F, norm_w=O["nw"], eps=EPS, norm_flags=gq.NORM_DEFER) +
            gq.gemm(2, E, F, od, O["h"], hout, ntok, F, E, gq.GEMV_ADD, res_off=O["x"], res_stride=E))
    assert ctx.run(cmds) == 0, ctx.error()
    for t in range(ntok):
        xt = x[t * E:(t + 1) * E]
        xn = orc.ref_rownorm(xt, nw, E, 1, EPS)
        h = orc.ref_silu_mul_cr(orc.ref_gemv(2, wg, xn, F, E)[0], orc.ref_gemv(2, wu, xn, F, E)[0])
        if not over:
            assert_bits(ctx.read(O["h"] + t * F, F), h, f"SwiGLU token {t}")
        assert_bits(ctx.read(hout + t * E, E), orc.ref_gemv(2, wd, h, E, F)[0] + xt, f"down token {t}")


@pytest.fixture(scope="module")
def q35():
    import qwen35

    return qwen35


@pytest.mark.parametrize("wtype,n_layer,n_prompt,n_gen", [(2, 4, 8, 24), (8, 8, 40, 12)])
def test_tiny_model_matches_reference_decoder(gq, orc, q35, wtype, n_layer, n_prompt, n_gen):
    """Greedy decode in the reference arithmetic: tokens, last logits and hidden state identical to the oracle's
    reference-arithmetic decoder."""
    cfg = q35.tiny(n_layer=n_layer, wtype=wtype)
    blob = q35.generate(cfg, seed=0)
    prompt = q35.prompt_ids(cfg, n_prompt)
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data, mode=orc.MODE_REFERENCE)
    lo = np.empty(cfg.n_vocab, np.float32)
    want = om.generate_fast(prompt, n_gen, lo)
    with q35.Model(blob) as m:
        m.set_arith(gq.ARITH_REFERENCE)
        got = m.generate(prompt, n_gen)
        lg, hd = m.logits(), m.hidden()
    assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}"
    assert_bits(lg, lo, "logits")
    assert_bits(hd, om.hidden(), "hidden")


def test_full_width_prefill_and_decode_match_reference_decoder(gq, orc, q35):
    """C5 widths with 4 layers: the batched prefill (its GEMMs token by token in this arithmetic) and the decode
    steps after it give the reference decoder's tokens and logits."""
    cfg = q35.Config(n_layer=4, n_ctx=96)
    blob = q35.generate(cfg, seed=2)
    prompt = q35.prompt_ids(cfg, 40, seed=2)
    n_gen = 10
    om = orc.Model(q35.config_c(cfg), blob.table, blob.n, blob.data, mode=orc.MODE_REFERENCE)
    lo = np.empty(cfg.n_vocab, np.float32)
    want = om.generate_fast(prompt, n_gen, lo)
    with q35.Model(blob) as m:
        m.set_arith(gq.ARITH_REFERENCE)
        m.reset(prompt)
        assert m.prefill(len(prompt) - 1)
        m.step(n_gen)
        got, lg = m.tokens(len(prompt) + n_gen), m.logits()
    assert np.array_equal(got, want), f"first mismatch at {np.nonzero(got != want)[0][:3]}"
    assert_bits(lg, lo, "logits")
