"""Failure handling at the boundary (the reference's bounded kernel wait, ggml-xrt.cpp:69-78 and 1258-1264, and its
runtime_valid latch, ggml-xrt.cpp:2761-2770), forced from the host: a wait bound far shorter than work that runs
normally to its end. The timed-out wait returns GEMVQ_ETIMEDOUT and latches the context: later device calls return
GEMVQ_EUNUSABLE with the first failure kept in the message; destroying it waits for the outstanding work; a new
context works."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_timed_out_wait_latches_the_context(gq, orc):
    rows, cols = 8192, 16384  # 75.5 MB of Q4_0: tens of microseconds per GEMV
    w = gq.matrix(gq.Q4_0, rows, cols, seed=0, stream=7, std=0.02)
    x = gq.normal(0, 8, cols)
    ctx = gq.Context(act_floats=1 << 16, weight_bytes=1 << 27)
    off = ctx.upload(gq.Q4_0, rows, cols, w)
    ctx.write(0, x)
    one = gq.gemv(gq.Q4_0, rows, cols, off, 0, cols)
    g = ctx.graph(one * 200)  # one replay: milliseconds of device work behind a single host launch
    assert ctx.usable()
    ctx.set_wait_timeout(1)
    print("[failure] 5 replays of 200 GEMVs of 75.5 MB against a 1 ms wait", flush=True)
    ctx.replay(g, 5)
    st = ctx.lib.gemvq_sync(ctx.h)
    assert st == gq.ETIMEDOUT, st
    assert not ctx.usable()
    assert "did not finish within 1 ms" in ctx.error()
    words = (gq.C.c_uint32 * 8)(*one)
    for call in (lambda: ctx.lib.gemvq_sync(ctx.h), lambda: ctx.lib.gemvq_graph_replay(ctx.h, g, 1),
                 lambda: ctx.lib.gemvq_run(ctx.h, words, 1)):
        assert call() == gq.EUNUSABLE
    assert "unusable" in ctx.error() and "did not finish" in ctx.error()
    ctx.close()  # waits for the replays, which end normally
    r2, c2s = 512, 2560
    w2 = gq.matrix(gq.Q4_0, r2, c2s, seed=0, stream=1, std=0.02)
    x2 = gq.normal(0, 2, c2s)
    with gq.Context(act_floats=1 << 16, weight_bytes=1 << 22) as c2:
        off2 = c2.upload(gq.Q4_0, r2, c2s, w2)
        c2.write(0, x2)
        assert c2.run(gq.gemv(gq.Q4_0, r2, c2s, off2, 0, c2s)) == 0
        y = c2.read(c2s, r2)
        ref = orc.fx_gemv(gq.Q4_0, w2, x2, r2, c2s)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
        assert c2.usable()


def test_host_read_after_long_work_is_bounded(gq):
    """A read of the activation buffer behind work that outlasts the wait bound returns GEMVQ_ETIMEDOUT (the copy
    waits, bounded, for the queued work before it is issued) and latches the context."""
    rows, cols = 8192, 16384
    w = gq.matrix(gq.Q4_0, rows, cols, seed=0, stream=7, std=0.02)
    x = gq.normal(0, 8, cols)
    ctx = gq.Context(act_floats=1 << 16, weight_bytes=1 << 27)
    off = ctx.upload(gq.Q4_0, rows, cols, w)
    ctx.write(0, x)
    g = ctx.graph(gq.gemv(gq.Q4_0, rows, cols, off, 0, cols) * 200)
    ctx.set_wait_timeout(1)
    print("[failure] act read behind 5 replays of 200 GEMVs of 75.5 MB against a 1 ms wait", flush=True)
    ctx.replay(g, 5)
    dst = np.zeros(16, np.float32)
    st = ctx.lib.gemvq_act_read(ctx.h, 0, dst.ctypes.data_as(gq.C.c_void_p), 16)
    assert st == gq.ETIMEDOUT, st
    assert not ctx.usable()
    assert "act read" in ctx.error()
    ctx.close()  # waits for the replays, which end normally
