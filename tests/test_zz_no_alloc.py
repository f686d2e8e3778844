"""gemvq_gemm_static (the allocation-free batched GEMV) against the GEMM command of a context, bit for bit, on two
calls in a row (the second smaller), and its argument checks. Device buffers come from torch, not the library."""
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


def _gemm_command(gq, t, rows, cols, w, x, n_tok, ys):
    """The existing entry point: a GEMM command on a context holding the same matrix and rows."""
    with gq.Context(act_floats=1 << 20, weight_bytes=1 << 26) as ctx:
        off = ctx.upload(t, rows, cols, w)
        ctx.write(0, x)
        y0 = (n_tok * cols + 15) // 16 * 16
        assert ctx.run(gq.gemm(t, rows, cols, off, 0, y0, n_tok, cols, ys)) == 0, ctx.error()
        return ctx.read(y0, n_tok * ys).reshape(n_tok, ys)[:, :rows]


@pytest.mark.parametrize("t", [2, 3, 8])
def test_static_gemm_matches_gemm_command(gq, t):
    import torch

    f = _fn(gq)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for rows, cols, n_tok, seed in ((1000, 4096, 29, 1), (300, 1024, 5, 2)):  # the second call smaller
        w = gq.matrix(t, rows, cols, seed=seed, stream=20 + t, std=0.02)
        x = gq.normal(seed, 30 + t, n_tok * cols).reshape(n_tok, cols)
        ys = (rows + 15) // 16 * 16
        print(f"[static gemm] type {t} rows {rows} cols {cols} tokens {n_tok}", flush=True)
        dw = torch.from_numpy(gq.repack(t, rows, cols, w)).cuda()
        dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        dy = torch.full((n_tok, ys), float("nan"), dtype=torch.float32, device="cuda")
        st = f(t, rows, cols, dw.data_ptr(), dx.data_ptr(), n_tok, cols, dy.data_ptr(), ys, stream)
        assert st == 0
        torch.cuda.synchronize()
        got = dy.cpu().numpy()[:, :rows]
        want = _gemm_command(gq, t, rows, cols, w, x, n_tok, ys)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_static_gemm_rejects_bad_arguments(gq):
    import torch

    f = _fn(gq)
    w = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(33 * 1024, dtype=torch.float32, device="cuda")
    y = torch.zeros(33 * 1024, dtype=torch.float32, device="cuda")
    ok = (2, 64, 1024, w.data_ptr(), x.data_ptr(), 4, 1024, y.data_ptr(), 64, None)
    bad = [
        dict(n_tok=33),                      # beyond the scratch's 32 token rows
        dict(n_tok=0),
        dict(cols=1000),                     # not a multiple of 512
        dict(cols=16896),                    # beyond GEMVQ_MAX_COLS
        dict(t=14),                          # no batched GEMV for Q6_K
        dict(x=x.data_ptr() + 4),            # misaligned
        dict(w=w.data_ptr() + 64),
        dict(xs=1000),
        dict(ys=40),
    ]
    names = ["t", "rows", "cols", "w", "x", "n_tok", "xs", "y", "ys", "stream"]
    for b in bad:
        args = list(ok)
        for k, v in b.items():
            args[names.index(k)] = v
        assert f(*args) == gq.EINVAL, b
    torch.cuda.synchronize()
