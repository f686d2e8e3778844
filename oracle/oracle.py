"""ctypes bindings of the CPU oracle (liborc_gemvq.so) and of the reference's own CPU path compiled into
_ref/libgemvq_ref.so. TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product path."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_PATH = os.path.join(HERE, "liborc_gemvq.so")
REF_PATH = os.path.join(HERE, "_ref", "libgemvq_ref.so")
REF_SRC = "/root/reference/fpga/src"

Q4_0, Q4_1, Q8_0, Q5_K, Q6_K = 2, 3, 8, 13, 14
F = np.float32


def build(ref: bool = True) -> None:
    """Compiles the oracle; also the reference's own gemvq_ref.h into _ref/ when the reference tree is present."""
    subprocess.run(["make", "-B", "-C", HERE, "liborc_gemvq.so"], check=True, capture_output=True)
    if ref and os.path.isdir(REF_SRC):
        subprocess.run(["make", "-B", "-C", HERE, "ref"], check=True, capture_output=True)


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _fn(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_orc = None
_ref = None


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        lib = C.CDLL(ORC_PATH)
        vp, i, fl = C.c_void_p, C.c_int, C.c_float
        _fn(lib, "orc_half_to_float", fl, C.c_uint16)
        _fn(lib, "orc_float_to_half", C.c_uint16, fl)
        _fn(lib, "orc_nearest_int", i, fl)
        for n in ("orc_expf", "orc_logf", "orc_silu", "orc_sigmoid", "orc_softplus"):
            _fn(lib, n, fl, fl)
        _fn(lib, "orc_pair_sum", fl, vp, i)
        _fn(lib, "orc_row_bytes", C.c_size_t, i, i)
        _fn(lib, "orc_quantize_q8_0", None, vp, i, vp, vp)
        _fn(lib, "orc_quantize_q8_K", None, vp, i, vp, vp, vp)
        _fn(lib, "orc_quantize_q8_1", None, vp, i, vp, vp, vp)
        _fn(lib, "orc_ref_gemv", None, i, vp, vp, i, i, vp, vp)
        _fn(lib, "orc_ref_within_tolerance", i, fl, fl, C.c_double)
        _fn(lib, "orc_fx_gemv", None, i, vp, vp, i, i, vp, vp, vp)
        _fn(lib, "orc_fx_gemv_q", None, i, vp, vp, vp, vp, vp, i, i, vp, vp, vp)
        _fn(lib, "orc_fixed_to_float", fl, C.c_int64)
        _fn(lib, "orc_ref_rmsnorm", None, vp, vp, i, fl, vp)
        _fn(lib, "orc_ref_rownorm", None, vp, vp, i, i, fl, i, vp)
        _fn(lib, "orc_norm_scale", fl, vp, i, fl, i)
        _fn(lib, "orc_rownorm", None, vp, vp, i, i, i, fl, i, vp)
        _fn(lib, "orc_silu_mul", None, vp, vp, i, i, vp)
        _fn(lib, "orc_unary", None, vp, i, i, vp)
        _fn(lib, "orc_ref_unary", None, vp, i, i, vp)
        _fn(lib, "orc_conv", None, vp, vp, vp, i, i, vp, vp)
        _fn(lib, "orc_ref_conv", None, vp, vp, vp, i, i, vp, vp)
        _fn(lib, "orc_rope", None, vp, vp, i, i, i, vp)
        _fn(lib, "orc_ref_gdn", None, vp, vp, vp, vp, vp, vp, i, i, fl, vp, vp, vp)
        _fn(lib, "orc_gdn", None, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i, i, fl, fl, fl, i, vp)
        _fn(lib, "orc_attn", None, vp, vp, vp, i, i, i, i, fl, vp)
        _fn(lib, "orc_dequant_row_q6_K", None, vp, i, vp)
        _fn(lib, "orc_argmax", i, vp, i)
        _fn(lib, "orc_rope_cache", None, i, i, fl, vp)
        _fn(lib, "orc_model_create", vp, vp, vp, i, vp, i)
        _fn(lib, "orc_model_decode", i, vp, i, i, vp)
        _fn(lib, "orc_model_hidden", C.POINTER(fl), vp)
        _fn(lib, "orc_model_destroy", None, vp)
        _fn(lib, "orc_model_set_mode", i, vp, i)
        _fn(lib, "orc_model_set_fault", i, vp, i)
        _fn(lib, "orc_model_set_trace", i, vp, vp)
        _fn(lib, "orc_model_reset", i, vp)
        _fn(lib, "orc_model_prefill", i, vp, vp, i, i)
        _fn(lib, "orc_model_generate", i, vp, vp, i, i, vp, vp)
        _fn(lib, "orc_fast_gemv", None, i, i, vp, vp, i, i, vp)
        _fn(lib, "orc_fast_gemv_mt", None, i, i, vp, vp, i, i, vp, i)
        _fn(lib, "orc_fast_simd", i)
        _fn(lib, "orc_fast_set_simd", i, i)
        _fn(lib, "orc_gdn_mt", None, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i, i, fl, fl, fl, i, vp, i)
        _fn(lib, "orc_attn_mt", None, vp, vp, vp, i, i, i, i, fl, vp, i)
        _fn(lib, "orc_ref_attn", None, vp, vp, vp, i, i, i, i, fl, vp)
        for n in ("orc_cr_expf", "orc_cr_logf"):
            _fn(lib, n, fl, fl)
        u64p = C.POINTER(C.c_uint64)
        _fn(lib, "orc_crmath_check", None, i, i, u64p)
        _fn(lib, "orc_crmath_compare", C.c_uint64, i, vp, i)
        _fn(lib, "orc_crmath_hash", None, i, u64p, i)
        _fn(lib, "orc_ref_unary_cr", None, vp, i, i, vp)
        _fn(lib, "orc_ref_conv_cr", None, vp, vp, vp, i, i, vp, vp)
        _fn(lib, "orc_ref_silu_mul_cr", None, vp, vp, i, vp)
        _fn(lib, "orc_ref_gdn_cr_mt", None, vp, vp, vp, vp, vp, vp, i, i, fl, vp, i)
        _fn(lib, "orc_ref_attn_cr_mt", None, vp, vp, vp, i, i, i, i, fl, vp, i)
        _orc = lib
    return _orc


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> C.CDLL:
    """The reference's gemvq_ref.h itself, compiled from the reference tree (see Makefile target `ref`)."""
    global _ref
    if _ref is None:
        lib = C.CDLL(REF_PATH)
        vp, u, fl = C.c_void_p, C.c_uint, C.c_float
        _fn(lib, "refshim_half_to_float", fl, C.c_uint16)
        _fn(lib, "refshim_float_to_half", C.c_uint16, fl)
        _fn(lib, "refshim_nearest_int", C.c_int, fl)
        _fn(lib, "refshim_quantize_q8_k", None, vp, u, vp, vp)
        _fn(lib, "refshim_gemv", None, vp, vp, u, u, u, vp, vp)
        _fn(lib, "refshim_within_tolerance", C.c_int, fl, fl, C.c_double)
        _fn(lib, "refshim_within_elementwise", C.c_int, fl, fl)
        _fn(lib, "refshim_within_swiglu", C.c_int, fl, fl, C.c_double, fl, C.c_double)
        _fn(lib, "refshim_rmsnorm", None, vp, vp, u, fl, vp)
        _fn(lib, "refshim_rownorm", None, vp, vp, u, u, fl, u, vp)
        _fn(lib, "refshim_silu_mul", None, vp, vp, u, vp)
        _fn(lib, "refshim_unary", None, vp, u, u, vp)
        _fn(lib, "refshim_conv", None, vp, vp, vp, u, C.c_int, vp, vp)
        _fn(lib, "refshim_gdn", None, vp, vp, vp, vp, vp, vp, u, u, fl, vp, vp, vp)
        _ref = lib
    return _ref


# ---- convenience wrappers (numpy in, numpy out) ----
def row_bytes(t: int, cols: int) -> int:
    return int(orc().orc_row_bytes(t, cols))


def quantize_q8_0(x: np.ndarray):
    x = np.ascontiguousarray(x, F)
    q = np.empty(x.size, np.int8)
    d = np.empty(x.size // 32, np.uint16)
    orc().orc_quantize_q8_0(_p(x), x.size, _p(q), _p(d))
    return q, d


def quantize_q8_1(x: np.ndarray):
    x = np.ascontiguousarray(x, F)
    q = np.empty(x.size, np.int8)
    d = np.empty(x.size // 32, np.uint16)
    s_ = np.empty(x.size // 32, np.uint16)
    orc().orc_quantize_q8_1(_p(x), x.size, _p(q), _p(d), _p(s_))
    return q, d, s_


def quantize_q8_K(x: np.ndarray):
    x = np.ascontiguousarray(x, F)
    q = np.empty(x.size, np.int8)
    d = np.empty(x.size // 256, F)
    bs = np.empty(x.size // 16, np.int16)
    orc().orc_quantize_q8_K(_p(x), x.size, _p(q), _p(d), _p(bs))
    return q, d, bs


def ref_gemv(t: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int):
    x = np.ascontiguousarray(x, F)
    y = np.empty(rows, F)
    mag = np.empty(rows, np.float64)
    orc().orc_ref_gemv(t, _p(w), _p(x), rows, cols, _p(y), _p(mag))
    return y, mag


def fx_gemv(t: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, blocksums: bool = False):
    x = np.ascontiguousarray(x, F)
    y = np.empty(rows, F)
    acc = np.empty(rows, np.int64)
    nbs = rows * (cols // 256 * 2 if t in (Q5_K, Q6_K) else cols // 32)
    bs = np.empty(nbs, np.int32) if blocksums else None
    orc().orc_fx_gemv(t, _p(w), _p(x), rows, cols, _p(y), _p(bs), _p(acc))
    return (y, bs, acc) if blocksums else y


SIMD_AVX2, SIMD_AVX512_VNNI = 0, 1


def simd_levels() -> list[int]:
    """The fast rows' SIMD levels this host runs (AVX2 always; AVX-512 VNNI where the CPU has it)."""
    L = orc()
    prev = L.orc_fast_simd()
    top = L.orc_fast_set_simd(SIMD_AVX512_VNNI)
    L.orc_fast_set_simd(prev)
    return list(range(top + 1))


def set_simd(level: int) -> int:
    return orc().orc_fast_set_simd(level)


def fast_gemv(mode: int, t: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, threads: int = 1) -> np.ndarray:
    """The decoder's SIMD rows: mode 0 canonical (= fx_gemv), 1 reference (= ref_gemv); rows split over threads."""
    x = np.ascontiguousarray(x, F)
    y = np.empty(rows, F)
    wp = _p(np.ascontiguousarray(w, np.uint8))
    if threads > 1:
        orc().orc_fast_gemv_mt(mode, t, wp, _p(x), rows, cols, _p(y), threads)
    else:
        orc().orc_fast_gemv(mode, t, wp, _p(x), rows, cols, _p(y))
    return y


def norm_scale(x: np.ndarray, eps: float, l2: bool = False) -> float:
    x = np.ascontiguousarray(x, F)
    return float(orc().orc_norm_scale(_p(x), x.size, eps, 1 if l2 else 0))


def rownorm(x: np.ndarray, w: np.ndarray | None, n: int, rows: int, eps: float, flags: int = 0, stride: int = 0):
    x = np.ascontiguousarray(x, F)
    w = np.ascontiguousarray(w, F) if w is not None else np.zeros(n, F)
    y = np.empty(n * rows, F)
    orc().orc_rownorm(_p(x), _p(w), n, rows, stride, eps, flags, _p(y))
    return y


def ref_rownorm(x: np.ndarray, w: np.ndarray | None, n: int, rows: int, eps: float, flags: int = 0):
    """The reference's row norm (gemvq_ref.h:309-324): the FP32 squares summed in double in order; packed rows."""
    x = np.ascontiguousarray(x, F)
    w = np.ascontiguousarray(w, F) if w is not None else np.zeros(n, F)
    y = np.empty(n * rows, F)
    orc().orc_ref_rownorm(_p(x), _p(w), n, rows, eps, flags, _p(y))
    return y


def pair_sum(a: np.ndarray) -> float:
    a = np.ascontiguousarray(a, F)
    return float(orc().orc_pair_sum(_p(a), a.size))


def silu_mul(g, u, sigmoid=False):
    g = np.ascontiguousarray(g, F)
    u = np.ascontiguousarray(u, F)
    y = np.empty(g.size, F)
    orc().orc_silu_mul(_p(g), _p(u), g.size, 1 if sigmoid else 0, _p(y))
    return y


def unary(x, kind):
    x = np.ascontiguousarray(x, F)
    y = np.empty(x.size, F)
    orc().orc_unary(_p(x), x.size, kind, _p(y))
    return y


def conv(state, x, w, silu=True):
    state, x, w = (np.ascontiguousarray(a, F) for a in (state, x, w))
    y = np.empty(x.size, F)
    ns = np.empty(state.size, F)
    orc().orc_conv(_p(state), _p(x), _p(w), x.size, 1 if silu else 0, _p(y), _p(ns))
    return y, ns


def rope(x, cs, n_dims, ne0, rows):
    x, cs = np.ascontiguousarray(x, F), np.ascontiguousarray(cs, F)
    y = np.empty(x.size, F)
    orc().orc_rope(_p(x), _p(cs), n_dims, ne0, rows, _p(y))
    return y


def rope_cache(pos: int, n_dims: int, base: float) -> np.ndarray:
    cs = np.empty(n_dims, F)
    orc().orc_rope_cache(pos, n_dims, base, _p(cs))
    return cs


def gdn(state, q, k, v, graw, braw, hv, hk, scale, flags=0, dt=None, a=None, z=None, w=None, l2_eps=1e-6, rms_eps=1e-6):
    st = np.ascontiguousarray(state, F).copy()
    args = [np.ascontiguousarray(t, F) if t is not None else None for t in (q, k, v, graw, braw, dt, a, z, w)]
    y = np.empty(hv * 128, F)
    orc().orc_gdn(_p(st), *[_p(t) for t in args], hv, hk, scale, l2_eps, rms_eps, flags, _p(y))
    return y, st


def attn(q, kc, vc, nh, nkvh, hd, n_kv, scale, threads: int = 1, reference: bool = False):
    q = np.ascontiguousarray(q, F)
    out = np.empty(nh * hd, F)
    kc, vc = np.ascontiguousarray(kc, np.uint16), np.ascontiguousarray(vc, np.uint16)
    if reference:
        orc().orc_ref_attn(_p(q), _p(kc), _p(vc), nh, nkvh, hd, n_kv, scale, _p(out))
    else:
        orc().orc_attn_mt(_p(q), _p(kc), _p(vc), nh, nkvh, hd, n_kv, scale, _p(out), threads)
    return out


def crmath_check(fn: int, threads: int = 0) -> dict:
    """Exhaustive check of the correctly rounded exp (fn 0) / log (fn 1) over every binary32 input."""
    out = (C.c_uint64 * 4)()
    orc().orc_crmath_check(fn, threads or min(16, os.cpu_count() or 1), out)
    return {"misrounded": int(out[0]), "libm_differs": int(out[1]), "quad_decided": int(out[2]), "inputs": int(out[3])}


def crmath_compare(fn: int, func_ptr: int, threads: int = 0) -> int:
    """Inputs (of all 2^32) where the float(float) function at func_ptr differs from the oracle's exp / log."""
    return int(orc().orc_crmath_compare(fn, func_ptr, threads or min(16, os.cpu_count() or 1)))


def crmath_hash(fn: int, threads: int = 0) -> np.ndarray:
    out = np.zeros(4096, np.uint64)
    orc().orc_crmath_hash(fn, out.ctypes.data_as(C.POINTER(C.c_uint64)), threads or min(16, os.cpu_count() or 1))
    return out


def ref_unary_cr(x, kind):
    x = np.ascontiguousarray(x, F)
    y = np.empty_like(x)
    orc().orc_ref_unary_cr(_p(x), x.size, kind, _p(y))
    return y


def ref_silu_mul_cr(g, u):
    g, u = np.ascontiguousarray(g, F), np.ascontiguousarray(u, F)
    y = np.empty_like(g)
    orc().orc_ref_silu_mul_cr(_p(g), _p(u), g.size, _p(y))
    return y


def ref_conv_cr(state, x, w, silu=True):
    state, x, w = (np.ascontiguousarray(t, F) for t in (state, x, w))
    y = np.empty(x.size, F)
    ns = np.empty(3 * x.size, F)
    orc().orc_ref_conv_cr(_p(state), _p(x), _p(w), x.size, 1 if silu else 0, _p(y), _p(ns))
    return y, ns


def ref_gdn_cr(state, q, k, v, g, beta, hv, hk, scale, threads: int = 1):
    """The reference DeltaNet step (gemvq_ref.h:360-397) with the correctly rounded exp: g is the log decay, beta
    the gate. Returns y and the new state."""
    st = np.ascontiguousarray(state, F).copy()
    args = [np.ascontiguousarray(t, F) for t in (q, k, v, g, beta)]
    y = np.empty(hv * 128, F)
    orc().orc_ref_gdn_cr_mt(_p(st), *[_p(t) for t in args], hv, hk, scale, _p(y), threads)
    return y, st


def ref_attn_cr(q, kc, vc, nh, nkvh, hd, n_kv, scale, threads: int = 1):
    q = np.ascontiguousarray(q, F)
    out = np.empty(nh * hd, F)
    kc, vc = np.ascontiguousarray(kc, np.uint16), np.ascontiguousarray(vc, np.uint16)
    orc().orc_ref_attn_cr_mt(_p(q), _p(kc), _p(vc), nh, nkvh, hd, n_kv, scale, _p(out), threads)
    return out


def dequant_row_q6_K(row: np.ndarray, cols: int) -> np.ndarray:
    y = np.empty(cols, F)
    orc().orc_dequant_row_q6_K(_p(np.ascontiguousarray(row, np.uint8)), cols, _p(y))
    return y


def f2h(x: np.ndarray) -> np.ndarray:
    o = orc()
    return np.array([o.orc_float_to_half(float(v)) for v in np.asarray(x, F).ravel()], np.uint16)


MODE_CANONICAL, MODE_REFERENCE, MODE_REFERENCE_LIBM = 0, 1, 2
FAULT_ATTN_RESIDUAL, FAULT_QGATE_SWAP, FAULT_GATES_SWAP, FAULT_FFN_SWAP, FAULT_ROPE_K, FAULT_SSM_RESIDUAL = range(1, 7)


class Model:
    """The oracle decoder (qwen35_oracle.c) on the same tensor table and blob as the GPU model."""

    def __init__(self, cfg_c, table, n: int, data: np.ndarray, threads: int = 0, mode: int = MODE_CANONICAL):
        self.lib = orc()
        self.data = data  # keep the blob alive
        self.n_vocab = cfg_c.n_vocab
        self.n_embd = cfg_c.n_embd
        threads = threads or min(16, os.cpu_count() or 1)
        self.h = self.lib.orc_model_create(C.byref(cfg_c), table, n, data.ctypes.data, threads)
        if not self.h:
            raise RuntimeError("orc_model_create failed")
        self.set_mode(mode)

    def set_mode(self, mode: int) -> None:
        if self.lib.orc_model_set_mode(self.h, mode):
            raise ValueError(f"mode {mode}")

    def set_fault(self, fault: int) -> None:
        """Plants a wiring mistake (ORC_FAULT_*) in this decoder: only for tests of the independent checks."""
        if self.lib.orc_model_set_fault(self.h, fault):
            raise ValueError(f"fault {fault}")

    def reset(self) -> None:
        self.lib.orc_model_reset(self.h)

    def trace(self, n_layer: int) -> np.ndarray:
        """Turns on the residual-stream trace; the returned array [(n_layer + 1), n_embd] is filled by every later
        decode (the stream before layer 0 and after each layer)."""
        self._trace = np.zeros((n_layer + 1, self.n_embd), F)
        self.lib.orc_model_set_trace(self.h, _p(self._trace))
        return self._trace

    def prefill(self, tokens: np.ndarray, pos0: int) -> None:
        t = np.ascontiguousarray(tokens, np.int32)
        if self.lib.orc_model_prefill(self.h, _p(t), t.size, int(pos0)):
            raise RuntimeError("orc_model_prefill failed")

    def generate_fast(self, prompt: np.ndarray, n_gen: int, logits: np.ndarray | None = None) -> np.ndarray:
        """Greedy decode from a reset state: the prompt prefilled in chunks (all but its last token), then n_gen
        decode steps; returns all ids, and the last step's logits in `logits`."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(p.size + n_gen, np.int32)
        if self.lib.orc_model_generate(self.h, _p(p), p.size, int(n_gen), _p(out), _p(logits) if logits is not None else None):
            raise RuntimeError("orc_model_generate failed")
        return out

    def decode(self, token: int, pos: int, logits: np.ndarray | None = None) -> int:
        r = self.lib.orc_model_decode(self.h, int(token), int(pos), _p(logits) if logits is not None else None)
        if r < 0:
            raise RuntimeError("orc_model_decode failed")
        return r

    def hidden(self) -> np.ndarray:
        p = self.lib.orc_model_hidden(self.h)
        return np.ctypeslib.as_array(p, shape=(self.n_embd,)).copy()

    def generate(self, prompt: np.ndarray, n_gen: int) -> np.ndarray:
        toks = [int(t) for t in prompt]
        cur = toks[0]
        for pos in range(len(prompt) - 1 + n_gen):
            nxt = self.decode(cur, pos)
            cur = toks[pos + 1] if pos + 1 < len(prompt) else nxt
            if pos + 1 >= len(prompt):
                toks.append(nxt)
        return np.array(toks, np.int32)

    def close(self):
        if self.h:
            self.lib.orc_model_set_trace(self.h, None)
            self.lib.orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
