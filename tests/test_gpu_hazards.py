"""Command lists whose commands overlap in the activation buffer: the fused launches give, bit for bit, what the
commands run one by one give (the reference kernel's semantics, gemvqc16.h:26-51)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROWS, COLS = 512, 1024


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def env(gq):
    w = [gq.matrix(gq.Q4_0, ROWS, COLS, seed=11, stream=s, std=0.02) for s in range(4)]
    x = gq.normal(11, 10, COLS)
    r = gq.normal(11, 11, 4096)
    nw = gq.uniform(11, 12, COLS, 0.5, 1.5)
    ctx = gq.Context(act_floats=1 << 16, weight_bytes=1 << 24)
    offs = [ctx.upload(gq.Q4_0, ROWS, COLS, wi) for wi in w]
    yield gq, ctx, offs, x, r, nw
    ctx.close()


def run_state(ctx, x, r, nw, cmds, one_by_one):
    """Fresh activation contents, then the list (as one list or command by command); the whole buffer back."""
    ctx.write(0, np.zeros(1 << 16, np.float32))
    ctx.write(0, x)
    ctx.write(4096, r)
    ctx.write(8192, nw)
    if one_by_one:
        for c in cmds:
            assert ctx.run(c) == 0, ctx.error()
    else:
        assert ctx.run([w for c in cmds for w in c]) == 0, ctx.error()
    return ctx.read(0, 1 << 16)


def check(env, cmds, launches=None):
    gq, ctx, offs, x, r, nw = env
    fused = run_state(ctx, x, r, nw, cmds, False)
    n = ctx.launch_count()
    single = run_state(ctx, x, r, nw, cmds, True)
    assert np.array_equal(bits(fused), bits(single))
    if launches is not None:
        assert n == launches
    return fused


def test_member_output_is_a_later_members_residual(env):
    """GEMV A writes the residual of GEMV B (same x): B must read A's output, so B starts a new launch."""
    gq, ctx, offs, *_ = env
    A = gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 0, 4096)
    B = gq.gemv(gq.Q4_0, ROWS, COLS, offs[1], 0, 12288, gq.GEMV_ADD) + gq.add(ROWS, 12288, 4096, 16384)
    check(env, [A, B], launches=2)


def test_member_overwrites_an_earlier_members_residual(env):
    """GEMV A reads residual r (ADD epilog); GEMV B then writes over r: A must read the old r."""
    gq, ctx, offs, *_ = env
    A = gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 0, 12288, gq.GEMV_ADD) + gq.add(ROWS, 12288, 4096, 16384)
    B = gq.gemv(gq.Q4_0, ROWS, COLS, offs[1], 0, 4096 + 256)
    check(env, [A, B], launches=2)


def test_members_writing_the_same_rows(env):
    """Two members storing into overlapping rows: the later one's values win, as one by one."""
    gq, ctx, offs, *_ = env
    A = gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 0, 12288)
    B = gq.gemv(gq.Q4_0, ROWS, COLS, offs[1], 0, 12288 + 128)
    check(env, [A, B], launches=2)


def test_independent_members_still_share_a_launch(env):
    gq, ctx, offs, *_ = env
    A = gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 0, 12288)
    B = gq.gemv(gq.Q4_0, ROWS, COLS, offs[1], 0, 12288 + ROWS)
    C = gq.gemv(gq.Q4_0, ROWS, COLS, offs[2], 0, 16384, gq.GEMV_ADD) + gq.add(ROWS, 16384, 4096, 20480)
    check(env, [A, B, C], launches=1)


def test_gemv_output_over_its_own_input(env):
    """y overlapping x: every row is computed from the x before the launch."""
    gq, ctx, offs, x, *_ = env
    A = gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 0, 256)
    out = check(env, [A])
    ctx.write(0, x)
    assert ctx.run(gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 0, 32768)) == 0
    assert np.array_equal(bits(out[256:256 + ROWS]), bits(ctx.read(32768, ROWS)))


def test_deferred_norm_then_its_row_is_overwritten(env):
    """A deferred RMSNORM fixes its normalized row when it runs (gemvqc16.h:46-51); an ADD that then writes over
    the norm's input does not change what the following GEMVs on the norm read. Expected: the same list with the
    norm stored (not deferred) and the GEMVs reading the stored row."""
    gq, ctx, offs, x, r, nw = env
    deferred = [gq.rmsnorm(COLS, 0, 8192, 12288, 1e-6, flags=gq.NORM_DEFER),
                gq.add(COLS, 0, 4096, 0),
                gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 12288, 20480),
                gq.gemv(gq.Q4_0, ROWS, COLS, offs[1], 12288, 20480 + ROWS)]
    stored = [gq.rmsnorm(COLS, 0, 8192, 12288, 1e-6)] + deferred[1:]
    a = run_state(ctx, x, r, nw, deferred, False)
    b = run_state(ctx, x, r, nw, stored, True)
    assert np.array_equal(bits(a[20480:20480 + 2 * ROWS]), bits(b[20480:20480 + 2 * ROWS]))
    assert np.array_equal(bits(a[:COLS]), bits(b[:COLS]))  # the ADD ran


def test_deferred_norm_weight_overwritten_by_a_member(env):
    """A GEMV on the deferred norm whose output overwrites the norm's weight: its own launch and the next GEMV on
    the norm read the row as it was when the norm ran."""
    gq, ctx, offs, x, r, nw = env
    deferred = [gq.rmsnorm(COLS, 0, 8192, 12288, 1e-6, flags=gq.NORM_DEFER),
                gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 12288, 8192),
                gq.gemv(gq.Q4_0, ROWS, COLS, offs[1], 12288, 20480)]
    stored = [gq.rmsnorm(COLS, 0, 8192, 12288, 1e-6)] + deferred[1:]
    a = run_state(ctx, x, r, nw, deferred, False)
    b = run_state(ctx, x, r, nw, stored, True)
    assert np.array_equal(bits(a[8192:8192 + ROWS]), bits(b[8192:8192 + ROWS]))
    assert np.array_equal(bits(a[20480:20480 + ROWS]), bits(b[20480:20480 + ROWS]))


def test_deferred_norm_row_overwritten_by_a_merged_gemm(env):
    """A deferred RMSNORM, then two batched GEMVs on the same token rows that share one launch, the second writing
    over the norm's input row, then a GEMV on the norm. The merged launch is the one that overwrites the row, so
    the norm's row must be fixed before it: the GEMV reads the row as it was when the norm ran. Expected: the norm
    stored (not deferred) and the commands run one by one."""
    gq, ctx, offs, x, r, nw = env
    ntok = 8  # the MFMA batched GEMV (more than 4 tokens), whose launches merge consecutive GEMMs on the same rows
    rows_x = gq.normal(11, 13, ntok * COLS)
    deferred = [gq.rmsnorm(COLS, 0, 8192, 12288, 1e-6, flags=gq.NORM_DEFER),
                gq.gemm(gq.Q4_0, ROWS, COLS, offs[2], 32768, 40960, ntok, COLS, ROWS),
                gq.gemm(gq.Q4_0, ROWS, COLS, offs[3], 32768, 0, ntok, COLS, ROWS),
                gq.gemv(gq.Q4_0, ROWS, COLS, offs[0], 12288, 20480)]
    stored = [gq.rmsnorm(COLS, 0, 8192, 12288, 1e-6)] + deferred[1:]

    def state(cmds, one_by_one):
        ctx.write(0, np.zeros(1 << 16, np.float32))
        ctx.write(0, x)
        ctx.write(8192, nw)
        ctx.write(32768, rows_x)
        if one_by_one:
            for c in cmds:
                assert ctx.run(c) == 0, ctx.error()
        else:
            assert ctx.run([w for c in cmds for w in c]) == 0, ctx.error()
        return ctx.read(0, 1 << 16)

    a = state(deferred, False)
    assert ctx.launch_count() == 4  # quantization, the norm's snapshot, the two GEMMs as one launch, the GEMV
    b = state(stored, True)
    assert np.array_equal(bits(a[20480:20480 + ROWS]), bits(b[20480:20480 + ROWS]))
    assert np.array_equal(bits(a[:ntok * ROWS]), bits(b[:ntok * ROWS]))  # the second GEMM's output
    assert np.array_equal(bits(a[40960:40960 + ntok * ROWS]), bits(b[40960:40960 + ntok * ROWS]))
