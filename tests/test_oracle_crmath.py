"""The correctly rounded exp and log of the reference-arithmetic mode (oracle orc_crmath.c; the library's
gq_refmath.h), checked on every binary32 input: against an 80-bit evaluation (quad precision near rounding
boundaries), and the library's host build against the oracle's. The reference's CPU path calls the host libm
(gemvq_ref.h:298-342, 367); how many inputs glibc's expf / logf round differently is counted and printed."""
import ctypes as C

import numpy as np
import pytest


@pytest.mark.parametrize("fn,name", [(0, "exp"), (1, "log")])
def test_correctly_rounded_on_every_input(orc, fn, name):
    r = orc.crmath_check(fn)
    print(f"[crmath] {name}: {r}")
    assert r["misrounded"] == 0
    assert r["inputs"] > 2_000_000_000


def test_known_values(orc):
    o = orc.orc()
    bits = lambda v: int(np.float32(v).view(np.uint32))
    assert o.orc_cr_expf(0.0) == 1.0 and o.orc_cr_logf(1.0) == 0.0
    assert bits(o.orc_cr_expf(1.0)) == 0x402DF854  # e rounded to binary32
    assert bits(o.orc_cr_logf(2.0)) == 0x3F317218  # ln 2
    assert o.orc_cr_expf(-1e9) == 0.0 and o.orc_cr_expf(1e9) == np.inf and o.orc_cr_expf(89.0) == np.inf
    assert o.orc_cr_logf(0.0) == -np.inf and np.isnan(o.orc_cr_logf(-1.0)) and np.isnan(o.orc_cr_expf(np.nan))
    assert bits(o.orc_cr_expf(-103.97208)) in (1, 0)  # the bottom of the subnormals
    assert o.orc_cr_expf(88.72283935546875) == np.float32(3.4028235e38) or np.isinf(o.orc_cr_expf(88.72283935546875))


@pytest.mark.parametrize("fn,name", [(0, "gemvq_cr_expf"), (1, "gemvq_cr_logf")])
def test_library_host_build_equals_oracle(gq, orc, fn, name):
    """The library's exp / log (the code the kernels evaluate) compiled for the host, on every input."""
    ptr = C.cast(getattr(gq.hip_lib(), name), C.c_void_p).value
    assert orc.crmath_compare(fn, ptr) == 0
