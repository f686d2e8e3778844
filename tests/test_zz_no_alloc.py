"""gemvq_gemm_static (the allocation-free batched GEMV) against the GEMM command of a context, bit for bit, on two
calls in a row (the second smaller), and its argument checks. The caller's device buffers come from hipMalloc of the
HIP runtime the library itself links (a second runtime in the process, such as the one a torch wheel bundles, may
not initialise once the first holds the device)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _fn(gq):
    lib = gq.hip_lib()
    f = lib.gemvq_gemm_static
    f.restype = C.c_int
    f.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    return f


class Hip:
    """hipMalloc / hipMemcpy / hipFree of the runtime the library is linked against (already loaded with it)."""

    H2D, D2H = 1, 2

    def __init__(self, gq):
        gq.hip_lib()
        self.rt = C.CDLL("libamdhip64.so.7", mode=C.RTLD_GLOBAL)
        for name, args in (("hipMalloc", [C.POINTER(C.c_void_p), C.c_size_t]), ("hipFree", [C.c_void_p]),
                           ("hipMemcpy", [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]),
                           ("hipDeviceSynchronize", []), ("hipSetDevice", [C.c_int])):
            fn = getattr(self.rt, name)
            fn.restype = C.c_int
            fn.argtypes = args
        assert self.rt.hipSetDevice(0) == 0
        self.held = []

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), C.c_size_t(max(nbytes, 256))) == 0
        self.held.append(p.value)
        return p.value

    def upload(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        assert self.rt.hipMemcpy(p, a.ctypes.data, a.nbytes, self.H2D) == 0
        return p

    def download(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        assert self.rt.hipMemcpy(out.ctypes.data, p, out.nbytes, self.D2H) == 0
        return out

    def close(self):
        self.rt.hipDeviceSynchronize()
        for p in self.held:
            self.rt.hipFree(p)
        self.held = []


@pytest.fixture
def hip(gq):
    h = Hip(gq)
    yield h
    h.close()


def _gemm_command(gq, t, rows, cols, w, x, n_tok, ys):
    """The existing entry point: a GEMM command on a context holding the same matrix and rows."""
    with gq.Context(act_floats=1 << 20, weight_bytes=1 << 26) as ctx:
        off = ctx.upload(t, rows, cols, w)
        ctx.write(0, x)
        y0 = (n_tok * cols + 15) // 16 * 16
        assert ctx.run(gq.gemm(t, rows, cols, off, 0, y0, n_tok, cols, ys)) == 0, ctx.error()
        return ctx.read(y0, n_tok * ys).reshape(n_tok, ys)[:, :rows]


@pytest.mark.parametrize("t", [2, 3, 8])
def test_static_gemm_matches_gemm_command(gq, hip, t):
    f = _fn(gq)
    for rows, cols, n_tok, seed in ((1000, 4096, 29, 1), (300, 1024, 5, 2)):  # the second call smaller
        w = gq.matrix(t, rows, cols, seed=seed, stream=20 + t, std=0.02)
        x = gq.normal(seed, 30 + t, n_tok * cols).reshape(n_tok, cols)
        ys = (rows + 15) // 16 * 16
        print(f"[static gemm] type {t} rows {rows} cols {cols} tokens {n_tok}", flush=True)
        dw = hip.upload(gq.repack(t, rows, cols, w))
        dx = hip.upload(x.astype(np.float32))
        dy = hip.upload(np.full((n_tok, ys), np.nan, np.float32))
        st = f(t, rows, cols, dw, dx, n_tok, cols, dy, ys, None)  # the null stream
        assert st == 0
        assert hip.rt.hipDeviceSynchronize() == 0
        got = hip.download(dy, (n_tok, ys), np.float32)[:, :rows]
        want = _gemm_command(gq, t, rows, cols, w, x, n_tok, ys)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_static_gemm_rejects_bad_arguments(gq, hip):
    f = _fn(gq)
    w = hip.upload(np.zeros(1 << 20, np.uint8))
    x = hip.upload(np.zeros(33 * 1024, np.float32))
    y = hip.upload(np.zeros(33 * 1024, np.float32))
    ok = (2, 64, 1024, w, x, 4, 1024, y, 64, None)
    bad = [
        dict(n_tok=33),                      # beyond the scratch's 32 token rows
        dict(n_tok=0),
        dict(cols=1000),                     # not a multiple of 512
        dict(cols=16896),                    # beyond GEMVQ_MAX_COLS
        dict(t=14),                          # no batched GEMV for Q6_K
        dict(x=x + 4),                       # misaligned
        dict(w=w + 64),
        dict(xs=1000),
        dict(ys=40),
    ]
    names = ["t", "rows", "cols", "w", "x", "n_tok", "xs", "y", "ys", "stream"]
    for b in bad:
        args = list(ok)
        for k, v in b.items():
            args[names.index(k)] = v
        assert f(*args) == gq.EINVAL, b
    assert f(*ok) == 0  # and the valid call still runs
    assert hip.rt.hipDeviceSynchronize() == 0
