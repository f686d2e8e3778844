"""Every opcode and fused epilog on the GPU through the C ABI, bit-exact against the oracle (the canonical
arithmetic), plus the reference CPU path's tolerances where the reference defines them."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def assert_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size}/{want.size} differ; first {bad[:4]}: got {got[bad[:4]]} want {want[bad[:4]]}"


@pytest.fixture()
def ctx(gq):
    c = gq.Context(act_floats=1 << 20, weight_bytes=1 << 27, state_rows=64 * 128)
    yield c
    c.close()


def test_features(gq, ctx):
    assert ctx.run([]) == 0
    f = ctx.read(0, 2, np.uint32)
    assert f[0] >> 16 == 0x6B51 and f[1] >> 16 == 0x6B52
    # the format bits a planner checks before it offloads a type (ggml-xrt.cpp:341-375): Q5_K 1, Q6_K 2, Q4_1 4
    assert f[0] & 7 == 7
    assert tuple(int(v) for v in f) == ctx.features()


def test_rmsnorm_rows_strided_l2(gq, orc, ctx):
    n, rows = 4096, 1
    x = gq.normal(0, 11, 16384) * 3
    w = gq.uniform(0, 12, 16384, 0.5, 1.5)
    ctx.write(0, x)
    ctx.write(16384, w)
    for n, rows, flags, stride in [(4096, 1, 0, 0), (2560, 1, 0, 0), (12288, 1, 0, 0), (128, 16, 0, 0),
                                   (256, 8, 0, 2 * 256), (128, 32, gq.NORM_L2 | gq.NORM_NO_WEIGHT, 0),
                                   (16384, 1, gq.NORM_NO_WEIGHT, 0)]:
        cmd = gq.rmsnorm(n, 0, 16384, 32768, 1e-6, rows=rows, flags=flags, stride_words=stride // 16)
        assert ctx.run(cmd) == 0, ctx.error()
        y = ctx.read(32768, n * rows)
        want = orc.rownorm(x, None if flags & gq.NORM_NO_WEIGHT else w[:n], n, rows, 1e-6, flags, stride)
        assert_bits(y, want, f"rmsnorm n={n} rows={rows} flags={flags}")
        if flags == 0 and stride == 0:  # the reference CPU path (double sums) within its element-wise tolerance
            ref = np.empty(n * rows, np.float32)
            orc.orc().orc_ref_rownorm(x.ctypes.data, w.ctypes.data, n, rows, 1e-6, 0, ref.ctypes.data)
            assert np.all(np.abs(y - ref) <= 1e-6 + 2e-5 * np.abs(ref))


def test_elementwise(gq, orc, ctx):
    n = 4096
    a = gq.normal(0, 21, n) * 4
    b = gq.normal(0, 22, n)
    a[:8] = [0.0, -0.0, 20.0, 20.5, -87.5, 88.0, -20.0, 1e-3]
    ctx.write(0, a)
    ctx.write(n, b)
    checks = [
        (gq.add(n, 0, n, 2 * n), a + b),
        (gq.mul(n, 0, n, 2 * n), a * b),
        (gq.silu_mul(n, 0, n, 2 * n), orc.silu_mul(a, b)),
        (gq.silu_mul(n, 0, n, 2 * n, sigmoid=True), orc.silu_mul(a, b, sigmoid=True)),
        (gq.unary(n, 0, gq.UNARY_SILU, 2 * n), orc.unary(a, 1)),
        (gq.unary(n, 0, gq.UNARY_SIGMOID, 2 * n), orc.unary(a, 2)),
        (gq.unary(n, 0, gq.UNARY_SOFTPLUS, 2 * n), orc.unary(a, 3)),
        (gq.unary(n, 0, gq.UNARY_COPY, 2 * n), a),
        (gq.fill(n, 2 * n, 0.25), np.full(n, 0.25, np.float32)),
    ]
    for c, want in checks:
        assert ctx.run(c) == 0, ctx.error()
        assert_bits(ctx.read(2 * n, n), want, f"op {c[0]} flags {c[5]}")
    # strided rows: 16 rows of 128 every 256 floats
    assert ctx.run(gq.unary(2048, 0, gq.UNARY_SIGMOID, 2 * n, row=128, stride=256)) == 0
    strided = a.reshape(16, 256)[:, :128].ravel()
    assert_bits(ctx.read(2 * n, 2048), orc.unary(strided, 2), "strided unary")
    assert ctx.run(gq.silu_mul(2048, 0, n, 2 * n, sigmoid=True, row=128, stride=256)) == 0
    assert_bits(ctx.read(2 * n, 2048), orc.silu_mul(strided, b[:2048], sigmoid=True), "strided silu_mul")


def test_conv_and_rope(gq, orc, ctx):
    ch = 8192
    st = gq.normal(0, 31, 3 * ch)
    x = gq.normal(0, 32, ch)
    w = gq.normal(0, 33, 4 * ch) * 0.5
    ctx.write(0, x)
    ctx.write(ch, w)
    ctx.write(5 * ch, st)
    assert ctx.run(gq.conv(ch, 0, ch, 8 * ch, 5 * ch, 5 * ch, silu=True)) == 0, ctx.error()
    y, ns = orc.conv(st, x, w, silu=True)
    assert_bits(ctx.read(8 * ch, ch), y, "conv y")
    assert_bits(ctx.read(5 * ch, 3 * ch), ns, "conv state (in place)")
    # RoPE NEOX on 20 heads of 256, first 64 dims, cache from the position table
    ne0, rows, nd = 256, 20, 64
    xr = gq.normal(0, 34, ne0 * rows)
    table = np.concatenate([orc.rope_cache(p, nd, 1e7) for p in range(40)])
    ctx.write(0, xr)
    ctx.write(1 << 14, table)
    ctx.write(1 << 15, np.array([37], np.int32))
    assert ctx.run(gq.rope(nd, 0, 1 << 14, 1 << 16, ne0, rows, pos_off=1 << 15)) == 0, ctx.error()
    assert_bits(ctx.read(1 << 16, ne0 * rows), orc.rope(xr, table[37 * nd:38 * nd], nd, ne0, rows), "rope")


@pytest.mark.parametrize("flags,hv,hk", [(0, 4, 2), (2 | 4 | 8, 32, 16), (2 | 8, 8, 8), (4, 2, 1)])
def test_gdn_step(gq, orc, ctx, flags, hv, hk):
    S = 128
    q = gq.normal(1, 41, hk * S)
    k = gq.normal(1, 42, hk * S)
    if not flags & 2:  # unnormalized q/k: keep the state bounded as the model would
        q /= np.linalg.norm(q.reshape(hk, S), axis=1).repeat(S)
        k /= np.linalg.norm(k.reshape(hk, S), axis=1).repeat(S)
    v = gq.normal(1, 43, hv * S)
    g = gq.normal(1, 44, hv) if flags & 8 else -np.log1p(np.exp(gq.normal(1, 44, hv))).astype(np.float32)
    beta = gq.normal(1, 45, hv) if flags & 8 else (1 / (1 + np.exp(-gq.normal(1, 45, hv)))).astype(np.float32)
    dt, a = gq.normal(1, 46, hv), -np.abs(gq.normal(1, 47, hv))
    z = gq.normal(1, 48, hv * S)
    w = gq.uniform(1, 49, S, 0.5, 1.5)
    state = gq.normal(1, 50, hv * S * S) * 0.1
    offs = dict(q=0, k=4096, v=8192, g=16384, beta=16384 + 64, y=20480, w=24576, z=24576 + 128, dt=32768, a=32768 + 64)
    for name, arr in dict(q=q, k=k, v=v, g=g, beta=beta, w=w, z=z, dt=dt, a=a).items():
        ctx.write(offs[name], arr)
    ctx.state_write(128, state)
    c = gq.gdn(hv, hk, offs["q"], offs["k"], offs["v"], offs["g"], offs["beta"], offs["y"], 128, 128,
               1 / np.sqrt(S), flags, 1e-6, 1e-6, offs["w"], offs["z"], offs["dt"], offs["a"])
    assert ctx.run(c) == 0, ctx.error()
    y_want, st_want = orc.gdn(state, q, k, v, g, beta, hv, hk, float(1 / np.sqrt(S)), flags, dt, a, z, w)
    assert_bits(ctx.read(offs["y"], hv * S), y_want, "gdn y")
    assert_bits(ctx.state_read(128, hv * 128), st_want, "gdn state")
    if flags == 0:  # the reference CPU step (gemvq_ref.h:363-397) within its rounding-aware tolerance
        st_ref = state.copy()
        y_ref = np.empty(hv * S, np.float32)
        ymag = np.empty(hv * S)
        orc.orc().orc_ref_gdn(st_ref.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, g.ctypes.data,
                              beta.ctypes.data, hv, hk, float(1 / np.sqrt(S)), y_ref.ctypes.data, ymag.ctypes.data, None)
        assert np.all(np.abs(y_want - y_ref) <= 1e-6 + 4e-6 * ymag)


@pytest.mark.parametrize("hv,hk,wtype,z_silu", [(32, 16, 2, True), (32, 16, 2, False), (8, 2, 8, False)])
def test_gdn_gated_norm_folded_into_gemv(gq, orc, ctx, hv, hk, wtype, z_silu):
    """A GDN with the gated output norm followed by a GEMV that reads its output: the norm runs in the GEMV's
    activation prologue (no separate launch). Results equal the unfused sequence and the oracle, bit for bit, and the
    gated output is still written to the GDN's y."""
    S, R = 128, 96
    cols = hv * S
    flags = gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES | (gq.GDN_Z_SILU if z_silu else 0)
    q, k, v = gq.normal(5, 1, hk * S), gq.normal(5, 2, hk * S), gq.normal(5, 3, hv * S)
    g, beta, dt, a = gq.normal(5, 4, hv), gq.normal(5, 5, hv), gq.normal(5, 6, hv), -np.abs(gq.normal(5, 7, hv))
    z, w = gq.normal(5, 8, cols), gq.uniform(5, 9, S, 0.5, 1.5)
    if z_silu:  # the gate already activated (a SiLU epilog upstream): z holds silu(z)
        z = orc.unary(z, 1)
    state = gq.normal(5, 10, hv * S * S) * 0.1
    res = gq.normal(5, 11, R)
    W = gq.matrix(wtype, R, cols, 5, 12)
    off = ctx.upload(wtype, R, cols, W)
    O = dict(q=0, k=4096, v=8192, g=12288, beta=12352, dt=12416, a=12480, y=16384, w=24576, z=28672, res=36864,
             out=37376, dummy=38400)
    for name, arr in dict(q=q, k=k, v=v, g=g, beta=beta, dt=dt, a=a, w=w, z=z).items():
        ctx.write(O[name], arr)
    gdn = gq.gdn(hv, hk, O["q"], O["k"], O["v"], O["g"], O["beta"], O["y"], 256, 256, 1 / np.sqrt(S), flags,
                 1e-6, 1e-6, O["w"], O["z"], O["dt"], O["a"])
    gemv = gq.gemv(wtype, R, cols, off, O["y"], O["out"], gq.GEMV_ADD) + gq.add(R, O["out"], O["res"], O["res"])
    results = []
    for fused in (True, False):
        ctx.state_write(256, state)
        ctx.write(O["res"], res)
        ctx.write(O["y"], np.zeros(cols, np.float32))
        cmds = gdn + (gemv if fused else gq.fill(16, O["dummy"], 0.0) + gemv)
        assert ctx.run(cmds) == 0, ctx.error()
        assert ctx.launch_count() == (2 if fused else 4)  # folded: no separate gated-norm launch
        results.append((ctx.read(O["res"], R), ctx.read(O["y"], cols), ctx.state_read(256, hv * 128)))
    y_want, st_want = orc.gdn(state, q, k, v, g, beta, hv, hk, float(1 / np.sqrt(S)), flags, dt, a, z, w)
    out_want = orc.fx_gemv(wtype, W, y_want, R, cols) + res
    for (o, y, st), what in zip(results, ("folded", "separate")):
        assert_bits(y, y_want, f"{what}: gated y")
        assert_bits(st, st_want, f"{what}: state")
        assert_bits(o, out_want, f"{what}: GEMV + residual")


@pytest.mark.parametrize("hv,hk,wtype,z_silu,ntok,seqs", [
    (32, 16, 2, False, 2, False),  # small-token GEMV
    (32, 16, 8, True, 4, True),
    (16, 4, 2, False, 9, False),  # quantization launch + MFMA GEMM
    (8, 2, 8, True, 20, True),
])
def test_gdn_tokens_gated_norm_then_gemm(gq, orc, hv, hk, wtype, z_silu, ntok, seqs):
    """A GDN of several tokens (one sequence in order, or one token of each of several sequences decoded in
    lockstep, each on its own state rows) with gates, L2 q/k and the gated output norm over every token's heads,
    followed by a GEMM + residual on its output rows: the gated rows, the state rows and the GEMM outputs equal the
    oracle's tokens run one by one, bit for bit."""
    S, R = 128, 160
    cols = hv * S
    flags = (gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES | (gq.GDN_Z_SILU if z_silu else 0) |
             (gq.GDN_SEQS if seqs else 0))
    sq, sg = up16_(cols), up16_(hv)
    q, k, v = gq.normal(6, 1, ntok * sq), gq.normal(6, 2, ntok * sq), gq.normal(6, 3, ntok * sq)
    g, beta = gq.normal(6, 4, ntok * sg), gq.normal(6, 5, ntok * sg)
    dt, a = gq.normal(6, 6, hv), -np.abs(gq.normal(6, 7, hv))
    z, w = gq.normal(6, 8, ntok * cols), gq.uniform(6, 9, S, 0.5, 1.5)
    if z_silu:
        z = orc.unary(z, 1)
    n_st = hv * S * (ntok if seqs else 1)
    state = gq.normal(6, 10, n_st * S) * 0.1
    res = gq.normal(6, 11, ntok * R)
    W = gq.matrix(wtype, R, cols, 6, 12)
    O, at = {}, 0
    for name, size in dict(q=ntok * sq, k=ntok * sq, v=ntok * sq, g=ntok * sg, beta=ntok * sg, dt=hv, a=hv,
                           y=ntok * cols, w=S, z=ntok * cols, res=ntok * R, out=ntok * R).items():
        O[name], at = at, at + up16_(size)
    ctx = gq.Context(act_floats=up16_(at), weight_bytes=1 << 26, state_rows=n_st)
    try:
        off = ctx.upload(wtype, R, cols, W)
        for name, arr in dict(q=q, k=k, v=v, g=g, beta=beta, dt=dt, a=a, w=w, z=z, res=res).items():
            ctx.write(O[name], arr)
        ctx.state_write(0, state)
        gdn = gq.gdn(hv, hk, O["q"], O["k"], O["v"], O["g"], O["beta"], O["y"], 0, 0, 1 / np.sqrt(S), flags,
                     1e-6, 1e-6, O["w"], O["z"], O["dt"], O["a"])
        gdn[16 + 2:16 + 5] = [ntok, sq, sg]  # gates slot: n_tok, q / k / v row stride, g / beta row stride
        gemm = gq.gemm(wtype, R, cols, off, O["y"], O["out"], ntok, cols, R, gq.GEMV_ADD, O["res"], R)
        print(f"[gdn gemm] hv {hv} fmt {wtype} tokens {ntok} seqs {seqs}", flush=True)
        assert ctx.run(gdn + gemm) == 0, ctx.error()
        st = state.copy()
        y_want, out_want = [], []
        for t in range(ntok):
            qkv = [x[t * sq:t * sq + n] for x, n in ((q, hk * S), (k, hk * S), (v, cols))]
            gb = [x[t * sg:t * sg + hv] for x in (g, beta)]
            rows = slice(t * hv * S * S, (t + 1) * hv * S * S) if seqs else slice(None)
            y_t, st[rows] = orc.gdn(st[rows], *qkv, *gb, hv, hk, float(1 / np.sqrt(S)), flags & ~gq.GDN_SEQS,
                                    dt, a, z[t * cols:(t + 1) * cols], w)
            y_want.append(y_t)
            out_want.append(orc.fx_gemv(wtype, W, y_t, R, cols) + res[t * R:(t + 1) * R])
        assert_bits(ctx.read(O["y"], ntok * cols), np.concatenate(y_want), "gated rows")
        assert_bits(ctx.state_read(0, n_st), st, "state")
        assert_bits(ctx.read(O["out"], ntok * R), np.concatenate(out_want), "GEMM + residual")
    finally:
        ctx.close()


def up16_(n: int) -> int:
    return (n + 15) // 16 * 16


@pytest.mark.parametrize("nh,nkv,hd,nrot,n_ctx,npos,checks", [
    (16, 4, 256, 64, 200, 130, (0, 1, 63, 64, 65, 127, 128, 129)),  # Qwen3.5 shape, crosses two chunk boundaries
    (6, 2, 128, 128, 1100, 1041, (1023, 1024, 1040)),  # 17 chunks
    (6, 2, 128, 128, 2200, 2113, (2047, 2048, 2112)),  # 34 chunks: two load rounds in the combine
    (4, 4, 64, 16, 80, 70, (5, 69)),  # one q head per KV head
    (24, 4, 128, 64, 200, 130, (64, 129)),  # 6 q heads per KV head
    (16, 4, 256, 64, 4096, 4096, (2048, 4095)),  # the whole of a 4096-position cache, one token at a time
])
def test_attention(gq, orc, ctx, nh, nkv, hd, nrot, n_ctx, npos, checks):
    kv = ctx.kv_create(n_ctx, nkv, hd)
    qn = gq.uniform(2, 51, hd, 0.5, 1.5)
    kn = gq.uniform(2, 52, hd, 0.5, 1.5)
    table = np.concatenate([orc.rope_cache(p, nrot, 1e7) for p in range(n_ctx)])
    O = dict(qg=0, k=8192, v=9216, qn=10240, kn=10496, pos=10752, y=10768, cs=16384)  # cs: n_ctx * nrot floats
    ctx.write(O["qn"], qn)
    ctx.write(O["kn"], kn)
    ctx.write(O["cs"], table)
    kc = np.zeros((n_ctx, nkv, hd), np.uint16)
    vc = np.zeros((n_ctx, nkv, hd), np.uint16)
    for pos in range(npos):
        qg = gq.normal(3, 1000 + pos, 2 * nh * hd)
        k = gq.normal(3, 5000 + pos, nkv * hd)
        v = gq.normal(3, 9000 + pos, nkv * hd)
        ctx.write(O["qg"], qg)
        ctx.write(O["k"], k)
        ctx.write(O["v"], v)
        ctx.write(O["pos"], np.array([pos], np.int32))
        c = gq.attn(nh, nkv, O["qg"], kv, O["y"], hd, nrot, O["pos"], O["k"], O["v"], 1 / 16, 1e-6, O["qn"],
                    O["kn"], O["cs"], gate=O["qg"] + hd)
        assert ctx.run(c) == 0, ctx.error()
        cs = table[pos * nrot:(pos + 1) * nrot]
        qh = orc.rope(orc.rownorm(qg, qn, hd, nh, 1e-6, 0, 2 * hd), cs, nrot, hd, nh)
        kh = orc.rope(orc.rownorm(k, kn, hd, nkv, 1e-6), cs, nrot, hd, nkv)
        kc[pos] = orc.f2h(kh).reshape(nkv, hd)
        vc[pos] = orc.f2h(v).reshape(nkv, hd)
        if pos in checks:
            att = orc.attn(qh, kc, vc, nh, nkv, hd, pos + 1, 1 / 16)
            gate = qg.reshape(nh, 2 * hd)[:, hd:].ravel()
            want = orc.silu_mul(gate, att, sigmoid=True)
            assert_bits(ctx.read(O["y"], nh * hd), want, f"attention at pos {pos}")
    k_dev, v_dev = ctx.kv_read(kv, 0, npos, nkv * hd)
    assert np.array_equal(k_dev, kc[:npos].ravel()) and np.array_equal(v_dev, vc[:npos].ravel())


@pytest.mark.parametrize("nh,nkv,hd,nrot,n_ctx,p0,ntok", [
    (16, 4, 256, 64, 200, 50, 32),  # Qwen3.5 shape, the batch crosses a chunk boundary
    (16, 4, 256, 64, 200, 0, 5),    # from an empty cache
    (16, 4, 256, 64, 200, 190, 16),  # the last six positions are past the capacity (not stored, no output)
    (6, 2, 128, 128, 1100, 1020, 7),  # 17 chunks
    (6, 2, 128, 128, 2200, 2100, 7),  # 34 chunks: two load rounds in the combine
    (16, 4, 256, 64, 4096, 4064, 32),  # a batch ending at the last position of a 4096-position cache
    (32, 4, 64, 32, 300, 250, 9),  # 8 q heads per KV head
])
def test_attention_tokens(gq, orc, ctx, nh, nkv, hd, nrot, n_ctx, p0, ntok):
    """One ATTN command over n_tok tokens (positions act[pos] + t, packed rows) against n_tok one-token commands on
    a second KV buffer with the same history: outputs and caches bit for bit, and the oracle for the last stored
    token."""
    kv_one, kv_batch = ctx.kv_create(n_ctx, nkv, hd), ctx.kv_create(n_ctx, nkv, hd)
    qrow, kvrow, arow = 2 * nh * hd, nkv * hd, nh * hd
    O = dict(q=0, k=262144, v=294912, qn=327680, kn=327936, pos=328192, y=328704, y2=460800, cs=600064)
    qn = gq.uniform(2, 61, hd, 0.5, 1.5)
    kn = gq.uniform(2, 62, hd, 0.5, 1.5)
    table = np.concatenate([orc.rope_cache(p, nrot, 1e7) for p in range(n_ctx)])
    ctx.write(O["qn"], qn)
    ctx.write(O["kn"], kn)
    ctx.write(O["cs"], table)

    def one(kv, t, y):  # the one-token command of packed token t (its position in pos slot t)
        return gq.attn(nh, nkv, O["q"] + t * qrow, kv, y, hd, nrot, O["pos"] + 16 * t, O["k"] + t * kvrow,
                       O["v"] + t * kvrow, 1 / 16, 1e-6, O["qn"], O["kn"], O["cs"], gate=O["q"] + t * qrow + hd)

    def tokens(first, n, seed):  # packed q + gate, k, v rows and the position slots of n tokens
        qg, k, v = gq.normal(4, seed, n * qrow), gq.normal(4, seed + 1, n * kvrow), gq.normal(4, seed + 2, n * kvrow)
        ctx.write(O["q"], qg)
        ctx.write(O["k"], k)
        ctx.write(O["v"], v)
        slots = np.zeros(16 * 32, np.int32)
        slots[0:16 * n:16] = np.arange(first, first + n)
        ctx.write(O["pos"], slots)
        return qg

    for b0 in range(0, p0, 32):  # the same history in both buffers
        n = min(32, p0 - b0)
        tokens(b0, n, 100 + b0)
        assert ctx.run(sum((one(kv, t, O["y"]) for t in range(n) for kv in (kv_one, kv_batch)), [])) == 0, ctx.error()
    qg = tokens(p0, ntok, 7)
    sentinel = np.full(ntok * arow, -7.25, np.float32)
    ctx.write(O["y"], sentinel)
    ctx.write(O["y2"], sentinel)
    assert ctx.run(sum((one(kv_one, t, O["y"] + t * arow) for t in range(ntok)), [])) == 0, ctx.error()
    batch = gq.attn(nh, nkv, O["q"], kv_batch, O["y2"], hd, nrot, O["pos"], O["k"], O["v"], 1 / 16, 1e-6, O["qn"],
                    O["kn"], O["cs"], gate=O["q"] + hd, n_tok=ntok)
    assert ctx.run(batch) == 0, ctx.error()
    y_one, y_batch = ctx.read(O["y"], ntok * arow), ctx.read(O["y2"], ntok * arow)
    assert_bits(y_batch, y_one, "batched vs one-token outputs")
    npos = min(n_ctx, p0 + ntok)
    k1, v1 = ctx.kv_read(kv_one, 0, npos, kvrow)
    k2, v2 = ctx.kv_read(kv_batch, 0, npos, kvrow)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    stored = npos - p0
    assert np.all(y_batch[stored * arow:] == -7.25) and not np.any(y_batch[:stored * arow] == -7.25)
    t, pos = stored - 1, npos - 1  # the oracle for the last stored token
    q_t = qg[t * qrow:(t + 1) * qrow]
    qh = orc.rope(orc.rownorm(q_t, qn, hd, nh, 1e-6, 0, 2 * hd), table[pos * nrot:(pos + 1) * nrot], nrot, hd, nh)
    att = orc.attn(qh, k2.reshape(npos, nkv, hd), v2.reshape(npos, nkv, hd), nh, nkv, hd, pos + 1, 1 / 16)
    want = orc.silu_mul(q_t.reshape(nh, 2 * hd)[:, hd:].ravel(), att, sigmoid=True)
    assert_bits(y_batch[t * arow:(t + 1) * arow], want, "oracle, last stored token")
    too_many = gq.attn(nh, nkv, O["q"], kv_batch, O["y2"], hd, nrot, O["pos"], O["k"], O["v"], 1 / 16, 1e-6,
                       O["qn"], O["kn"], O["cs"], gate=O["q"] + hd, n_tok=33)
    assert ctx.run(too_many) == 1


@pytest.mark.parametrize("t", [2, 14])
def test_gemv_epilogs_on_streamed_rows(gq, orc, t):
    """Members long enough that each wave streams several chunks of rows (50000 rows: more than the resident waves
    hold at once; a wave's range is not a whole number of chunks): plain + ARGMAX, residual ADD, SiLU, CONV (in-place
    state) and the SwiGLU pair, each against the oracle bit for bit."""
    R, K = 50000, 256
    c = gq.Context(act_floats=1 << 20, weight_bytes=1 << 26, state_rows=0)
    try:
        x = gq.normal(0, 81, K)
        w1 = gq.matrix(t, R, K, 0, 82)
        w2 = gq.matrix(t, R, K, 0, 83)
        o1, o2 = c.upload(t, R, K, w1), c.upload(t, R, K, w2)
        X, RES, Y, Y2, KEY, CW, ST = 0, 1024, 65536, 131072, 196608, 262144, 524288
        c.write(X, x)
        res = gq.normal(0, 84, R)
        c.write(RES, res)
        y1 = orc.fx_gemv(t, w1, x, R, K)
        y2 = orc.fx_gemv(t, w2, x, R, K)
        c.write(KEY, np.zeros(4, np.float32))
        assert c.run(gq.gemv(t, R, K, o1, X, Y, gq.GEMV_ARGMAX) + gq.argmax(R, Y, KEY)) == 0, c.error()
        assert_bits(c.read(Y, R), y1, "plain")
        assert 0xFFFFFFFF - int(c.read(KEY, 2, np.uint32)[0]) == int(np.argmax(y1))
        assert c.run(gq.gemv(t, R, K, o1, X, Y2, gq.GEMV_ADD) + gq.add(R, Y2, RES, Y2)) == 0, c.error()
        assert_bits(c.read(Y2, R), y1 + res, "add")
        assert c.run(gq.gemv(t, R, K, o2, X, Y, gq.GEMV_SILU)) == 0, c.error()
        assert_bits(c.read(Y, R), orc.unary(y2, 1), "silu")
        assert c.run(gq.gemv(t, R, K, o1, X, Y, gq.GEMV_SWIGLU) + gq.gemv(t, R, K, o2, X, Y)) == 0, c.error()
        assert_bits(c.read(Y, R), orc.silu_mul(y1, y2), "swiglu")
        if t == 2:
            st = gq.normal(0, 85, 3 * R)
            kw = gq.normal(0, 86, 4 * R)
            c.write(CW, kw)
            c.write(ST, st)
            assert c.run(gq.gemv(t, R, K, o2, X, Y2, gq.GEMV_CONV) + gq.conv(R, Y2, CW, Y, ST, ST)) == 0, c.error()
            yc, ns = orc.conv(st, y2, kw)
            assert_bits(c.read(Y, R), yc, "conv")
            assert_bits(c.read(ST, 3 * R), ns, "conv state")
    finally:
        c.close()


def test_gemv_fused_epilogs(gq, orc, ctx):
    """SwiGLU pair, residual ADD, CONV, ARGMAX epilogs and the deferred norm fold (gemvqc16.h:31-51)."""
    E, F = 2560, 9728
    eps = 1e-6
    x = gq.normal(0, 61, E)
    r = gq.normal(0, 62, E)
    nw = gq.uniform(0, 63, E, 0.5, 1.5)
    wg = gq.matrix(gq.Q8_0, F, E, 0, 64)
    wu = gq.matrix(gq.Q8_0, F, E, 0, 65)
    wd = gq.matrix(gq.Q8_0, E, F, 0, 66)
    og, ou, od = (ctx.upload(gq.Q8_0, a, b, w) for a, b, w in ((F, E, wg), (F, E, wu), (E, F, wd)))
    X, R, NW, XN, ACT, T, Y = 0, 4096, 8192, 12288, 16384, 32768, 36864
    ctx.write(X, x)
    ctx.write(R, r)
    ctx.write(NW, nw)
    cmds = (gq.rmsnorm(E, X, NW, XN, eps, flags=gq.NORM_DEFER) + gq.gemv(gq.Q8_0, F, E, og, XN, ACT, gq.GEMV_SWIGLU) +
            gq.gemv(gq.Q8_0, F, E, ou, XN, ACT) + gq.gemv(gq.Q8_0, E, F, od, ACT, T, gq.GEMV_ADD) + gq.add(E, T, R, Y))
    assert ctx.run(cmds) == 0, ctx.error()
    assert ctx.launch_count() == 2
    xn = orc.rownorm(x, nw, E, 1, eps)
    g = orc.fx_gemv(gq.Q8_0, wg, xn, F, E)
    u = orc.fx_gemv(gq.Q8_0, wu, xn, F, E)
    act = orc.silu_mul(g, u)
    assert_bits(ctx.read(ACT, F), act, "swiglu")
    want = orc.fx_gemv(gq.Q8_0, wd, act, E, F) + r
    assert_bits(ctx.read(Y, E), want, "down + residual")
    # conv epilog on a Q4_0 GEMV, in-place state
    ch, K = 512, 256
    wc = gq.matrix(gq.Q4_0, ch, K, 0, 67)
    oc = ctx.upload(gq.Q4_0, ch, K, wc)
    xc = gq.normal(0, 68, K)
    st = gq.normal(0, 69, 3 * ch)
    kw = gq.normal(0, 70, 4 * ch)
    ctx.write(X, xc)
    ctx.write(40960, kw)
    ctx.write(49152, st)
    cmds = gq.gemv(gq.Q4_0, ch, K, oc, X, T, gq.GEMV_CONV) + gq.conv(ch, T, 40960, Y, 49152, 49152)
    assert ctx.run(cmds) == 0, ctx.error()
    yc, ns = orc.conv(st, orc.fx_gemv(gq.Q4_0, wc, xc, ch, K), kw)
    assert_bits(ctx.read(Y, ch), yc, "conv epilog")
    assert_bits(ctx.read(49152, 3 * ch), ns, "conv epilog state")
    # argmax epilog on a Q6_K head with an L2 deferred norm (no weight); ties resolve to the first index
    V, D = 3000, 512
    wh = gq.matrix(gq.Q6_K, V, D, 0, 71)
    oh = ctx.upload(gq.Q6_K, V, D, wh)
    xh = gq.normal(0, 72, D)
    ctx.write(X, xh)
    ctx.write(65536, np.zeros(16, np.float32))
    cmds = (gq.rmsnorm(D, X, 0, XN, 1e-6, flags=gq.NORM_DEFER | gq.NORM_L2 | gq.NORM_NO_WEIGHT) +
            gq.gemv(gq.Q6_K, V, D, oh, XN, ACT, gq.GEMV_ARGMAX) + gq.argmax(V, ACT, 65536))
    assert ctx.run(cmds) == 0, ctx.error()
    logits = orc.fx_gemv(gq.Q6_K, wh, orc.rownorm(xh, None, D, 1, 1e-6, 3), V, D)
    assert_bits(ctx.read(ACT, V), logits, "head logits")
    key = ctx.read(65536, 2, np.uint32)
    assert 0xFFFFFFFF - int(key[0]) == int(np.argmax(logits))
    # SiLU epilog (a UNARY SiLU folded into the GEMV) on a group member next to a plain one
    zs = gq.matrix(gq.Q4_0, 384, K, 0, 73)
    oz = ctx.upload(gq.Q4_0, 384, K, zs)
    cmds = gq.gemv(gq.Q4_0, ch, K, oc, X, T) + gq.gemv(gq.Q4_0, 384, K, oz, X, Y, gq.GEMV_SILU)
    ctx.write(X, xc)
    assert ctx.run(cmds) == 0, ctx.error()
    assert ctx.launch_count() == 1
    assert_bits(ctx.read(T, ch), orc.fx_gemv(gq.Q4_0, wc, xc, ch, K), "plain member")
    assert_bits(ctx.read(Y, 384), orc.unary(orc.fx_gemv(gq.Q4_0, zs, xc, 384, K), 1), "silu epilog")


def test_get_rows_and_next_token(gq, orc, ctx):
    V, D = 1000, 1024
    w = gq.matrix(gq.Q6_K, V, D, 0, 81)
    o = ctx.upload(gq.Q6_K, V, D, w)
    ctx.write(0, np.array([777], np.int32))
    assert ctx.run(gq.get_rows(gq.Q6_K, V, D, o, 0, 1024)) == 0, ctx.error()
    rb = gq.row_bytes(gq.Q6_K, D)
    assert_bits(ctx.read(1024, D), orc.dequant_row_q6_K(w[777 * rb:778 * rb], D), "get_rows Q6_K")
    # a block of tokens: ids 16 floats apart, rows packed; an id out of range leaves its row untouched
    ids = [3, 999, 0, 512, -1, 777, 41]
    slots = np.zeros(16 * len(ids), np.int32)
    slots[::16] = ids
    ctx.write(8192, slots)
    ctx.write(16384, np.full(len(ids) * D, -3.5, np.float32))
    assert ctx.run(gq.get_rows(gq.Q6_K, V, D, o, 8192, 16384, n_tok=len(ids))) == 0, ctx.error()
    got = ctx.read(16384, len(ids) * D).reshape(len(ids), D)
    for t, i in enumerate(ids):
        want = orc.dequant_row_q6_K(w[i * rb:(i + 1) * rb], D) if i >= 0 else np.full(D, -3.5, np.float32)
        assert_bits(got[t], want, f"get_rows token {t} (id {i})")
    assert ctx.run(gq.get_rows(gq.Q6_K, V, D, o, 8192, 16384, n_tok=33)) == 1
    # NEXT_TOKEN: prompt phase then the argmax key
    KEY, TOK, POS, PR, OUT = 4096, 4112, 4128, 4144, 4400
    ctx.write(PR, np.array([5, 6, 7], np.int32))
    ctx.write(POS, np.array([0], np.int32))
    ctx.write(KEY, np.array([0, 0], np.uint32))
    c = gq.next_token(KEY, TOK, POS, PR, 3, OUT)
    assert ctx.run(c) == 0
    assert ctx.read(TOK, 1, np.int32)[0] == 6 and ctx.read(POS, 1, np.int32)[0] == 1
    ctx.write(POS, np.array([2], np.int32))
    key_lo = 0xFFFFFFFF - 42
    ctx.write(KEY, np.array([key_lo, 0x80000000], np.uint32))
    assert ctx.run(c) == 0
    assert ctx.read(TOK, 1, np.int32)[0] == 42 and ctx.read(OUT + 3, 1, np.int32)[0] == 42
    assert tuple(ctx.read(KEY, 2, np.uint32)) == (0, 0)


def test_invalid_commands_rejected(gq, ctx):
    """Validation returns the 1-based index of the first bad command and runs nothing (gemvqc16.cpp:455-466)."""
    good = gq.fill(16, 0, 1.0)
    assert ctx.run(good + gq.cmd(99)) == 2
    assert ctx.run(good + good + gq.gemv(gq.Q4_0, 16, 256, 123456, 0, 256)) == 3  # unknown weight
    assert ctx.run(gq.add(16, 3, 0, 32)) == 1                                      # misaligned offset
    assert ctx.run(gq.add(16, 0, 0, ctx.act_floats)) == 1                          # out of range
    assert ctx.run(gq.gdn(64, 3, 0, 0, 0, 0, 0, 0, 0, 0, 1.0)) == 1                # hv not a multiple of hk


def test_c4_gated_deltanet_layer(gq, orc):
    """C4: one Gated DeltaNet layer at hidden 4096 as the decoder issues it: deferred RMS norm, the {qkv + CONV, z +
    SiLU, beta, alpha} Q4_0 GEMV group, the GDN step with L2 q/k, gates and the gated norm (folded into ssm_out's
    prologue), ssm_out Q4_0 [4096 x 4096] + residual. State N(0, 0.1^2), conv cache N(0, 1), gate logits N(0, 1)."""
    E, Hk, Hv, S = 4096, 16, 32, 128
    ch = 2 * Hk * S + Hv * S
    eps = 1e-6
    x, nw = gq.normal(7, 1, E), gq.uniform(7, 2, E, 0.5, 1.5)
    Wqkv, Wz = gq.matrix(2, ch, E, 7, 3), gq.matrix(2, Hv * S, E, 7, 4)
    Wb, Wa, Wo = gq.matrix(2, Hv, E, 7, 5), gq.matrix(2, Hv, E, 7, 6), gq.matrix(2, E, Hv * S, 7, 7)
    cw, cst = gq.normal(7, 8, 4 * ch, std=0.5), gq.normal(7, 9, 3 * ch)
    dt, a, sw = gq.normal(7, 10, Hv), -np.abs(gq.normal(7, 11, Hv)), gq.uniform(7, 12, S, 0.5, 1.5)
    state = gq.normal(7, 13, Hv * S * S) * 0.1
    ctx = gq.Context(act_floats=1 << 17, weight_bytes=48 << 20, state_rows=Hv * 128)
    oq, oz, ob, oa, oo = (ctx.upload(2, r, c, w) for r, c, w in
                          ((ch, E, Wqkv), (Hv * S, E, Wz), (Hv, E, Wb), (Hv, E, Wa), (E, Hv * S, Wo)))
    O = dict(x=0, nw=4096, xn=8192, qkv=12288, cqkv=20480, z=28672, ba=32768, y=32832, cw=40960, cst=73728,
             dt=98304, a=98368, sw=98432, out=98560)
    for k_, v_ in dict(x=x, nw=nw, cw=cw, cst=cst, dt=dt, a=a, sw=sw).items():
        ctx.write(O[k_], v_)
    ctx.state_write(0, state)
    flags = gq.GDN_L2_QK | gq.GDN_GATED | gq.GDN_GATES | gq.GDN_Z_SILU
    cmds = (gq.rmsnorm(E, O["x"], O["nw"], O["xn"], eps, flags=gq.NORM_DEFER) +
            gq.gemv(2, ch, E, oq, O["xn"], O["qkv"], gq.GEMV_CONV) +
            gq.conv(ch, O["qkv"], O["cw"], O["cqkv"], O["cst"], O["cst"]) +
            gq.gemv(2, Hv * S, E, oz, O["xn"], O["z"], gq.GEMV_SILU) +
            gq.gemv(2, Hv, E, ob, O["xn"], O["ba"]) + gq.gemv(2, Hv, E, oa, O["xn"], O["ba"] + 32) +
            gq.gdn(Hv, Hk, O["cqkv"], O["cqkv"] + Hk * S, O["cqkv"] + 2 * Hk * S, O["ba"] + 32, O["ba"], O["y"], 0, 0,
                   1 / np.sqrt(S), flags, eps, eps, O["sw"], O["z"], O["dt"], O["a"]) +
            gq.gemv(2, E, Hv * S, oo, O["y"], O["out"], gq.GEMV_ADD) + gq.add(E, O["out"], O["x"], O["x"]))
    assert ctx.run(cmds) == 0, ctx.error()
    assert ctx.launch_count() == 3  # group (norm folded), GDN, ssm_out (gated norm folded)
    xn = orc.rownorm(x, nw, E, 1, eps)
    yc, ns = orc.conv(cst, orc.fx_gemv(2, Wqkv, xn, ch, E), cw)
    z = orc.unary(orc.fx_gemv(2, Wz, xn, Hv * S, E), 1)
    b, al = orc.fx_gemv(2, Wb, xn, Hv, E), orc.fx_gemv(2, Wa, xn, Hv, E)
    y, st = orc.gdn(state, yc[:Hk * S], yc[Hk * S:2 * Hk * S], yc[2 * Hk * S:], al, b, Hv, Hk, float(1 / np.sqrt(S)),
                    flags, dt, a, z, sw)
    assert_bits(ctx.read(O["cst"], 3 * ch), ns, "conv state")
    assert_bits(ctx.read(O["cqkv"], ch), yc, "conv output")
    assert_bits(ctx.read(O["z"], Hv * S), z, "silu(z)")
    assert_bits(ctx.state_read(0, Hv * 128), st, "DeltaNet state")
    assert_bits(ctx.read(O["y"], Hv * S), y, "gated output")
    assert_bits(ctx.read(O["x"], E), orc.fx_gemv(2, Wo, y, E, Hv * S) + x, "layer output")
    ctx.close()
