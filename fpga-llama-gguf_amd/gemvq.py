"""Python host side of the MI355X decode backend: ctypes bindings over the C ABI (include/gemvq_hip.h,
include/gemvq_synth.h) and builders for the command-list words.

The command words mirror the reference kernel's command list (fpga/src/gemvqc16.h:24-135); `Context.run` returns
the same status convention as gemvqc16 (0, the 1-based index of the first invalid command, or a negative error).
The GPU path has no fallback: without the built libgemvq_hip.so or a HIP device, loading fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
HIP_LIB_PATH = os.path.join(PKG, "libgemvq_hip.so")
SYNTH_LIB_PATH = os.path.join(PKG, "libgemvq_synth.so")

# ggml type ids
Q4_0, Q4_1, Q8_0, Q5_K, Q6_K = 2, 3, 8, 13, 14
# opcodes (gemvqc16.h:100-111 plus the opcodes of this backend)
OP_GEMV, OP_RMSNORM, OP_ADD, OP_SILU_MUL, OP_MUL, OP_UNARY, OP_GDN, OP_CONV, OP_STATE_LOAD, OP_ROPE, OP_TRACE = range(1, 12)
OP_ATTN, OP_GET_ROWS, OP_ARGMAX, OP_NEXT_TOKEN, OP_FILL, OP_GEMM = 12, 13, 14, 15, 16, 17
GEMM_MAX_TOK = 32
GEMV_SWIGLU, GEMV_CONV, GEMV_ADD, GEMV_ARGMAX, GEMV_SILU = 0x100, 0x200, 0x400, 0x800, 0x1000
GDN_WITH_GEMV, GDN_L2_QK, GDN_GATED, GDN_GATES, GDN_WITH_OUT, GDN_Z_SILU, GDN_SEQS = 1, 2, 4, 8, 16, 32, 64
NORM_L2, NORM_NO_WEIGHT, NORM_DEFER = 1, 2, 4
SILU_MUL_SIGMOID = 1
UNARY_SILU, UNARY_SIGMOID, UNARY_SOFTPLUS, UNARY_COPY = 1, 2, 3, 4
EINVAL, ETIMEDOUT, EUNUSABLE = -10000, -10001, -10002
ARITH_CANONICAL, ARITH_REFERENCE = 0, 1
MAX_CMDS = 4096


def fbits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def row_bytes(t: int, cols: int) -> int:
    return {Q4_0: cols // 32 * 18, Q4_1: cols // 32 * 20, Q8_0: cols // 32 * 34, Q5_K: cols // 256 * 176,
            Q6_K: cols // 256 * 210}[t]


# ---------------------------------------------------------------------------------------------------------------
# command builders (8 words each)
def cmd(*words: int) -> list[int]:
    w = [int(x) & 0xFFFFFFFF for x in words]
    assert len(w) <= 8
    return w + [0] * (8 - len(w))


def gemv(fmt: int, rows: int, cols: int, w_off: int, x_off: int, y_off: int, flags: int = 0) -> list[int]:
    return cmd(OP_GEMV, fmt | flags, rows, cols, w_off & 0xFFFFFFFF, w_off >> 32, x_off, y_off)


def rmsnorm(n: int, x_off: int, w_off: int, y_off: int, eps: float, rows: int = 1, flags: int = 0,
            stride_words: int = 0) -> list[int]:
    return cmd(OP_RMSNORM, n, x_off, w_off, y_off, fbits(eps), rows, flags | (stride_words << 8))


def add(n: int, a: int, b: int, y: int) -> list[int]:
    return cmd(OP_ADD, n, a, b, y)


def mul(n: int, a: int, b: int, y: int) -> list[int]:
    return cmd(OP_MUL, n, a, b, y)


def silu_mul(n: int, g: int, u: int, y: int, sigmoid: bool = False, row: int = 0, stride: int = 0) -> list[int]:
    return cmd(OP_SILU_MUL, n, g, u, y, SILU_MUL_SIGMOID if sigmoid else 0, row, stride)


def unary(n: int, x: int, kind: int, y: int, row: int = 0, stride: int = 0) -> list[int]:
    return cmd(OP_UNARY, n, x, kind, y, row, stride)


def conv(ch: int, x: int, w: int, y: int, s_src: int, s_dst: int, silu: bool = True) -> list[int]:
    return cmd(OP_CONV, ch, x, w, y, s_src, s_dst, 1 if silu else 0)


def rope(n_dims: int, x: int, cs: int, y: int, ne0: int, rows: int, pos_off: int = 0) -> list[int]:
    return cmd(OP_ROPE, n_dims, x, cs, y, ne0, rows, pos_off)


def gdn(hv: int, hk: int, q: int, k: int, v: int, g: int, beta: int, y: int, src_row: int, dst_row: int,
        scale: float, flags: int = 0, l2_eps: float = 1e-6, rms_eps: float = 1e-6, w: int = 0, z: int = 0,
        dt: int = 0, a: int = 0) -> list[int]:
    out = cmd(OP_GDN, hv | (hk << 16), q, k, v, g, beta, y)
    out += cmd(src_row, dst_row, fbits(scale), flags, fbits(l2_eps), fbits(rms_eps), w, z)
    if flags & GDN_GATES:
        out += cmd(dt, a)
    return out


def attn(n_head: int, n_head_kv: int, q: int, kv: int, y: int, head_dim: int, n_rot: int, pos_off: int,
         k: int, v: int, scale: float, eps: float, qn: int, kn: int, cs: int, gate: int | None = None,
         n_tok: int = 1) -> list[int]:
    """n_tok > 1: tokens at positions act[pos_off] + t with packed rows (q / gate, k, v and y of token t follow
    those of token t - 1)."""
    flags = (1 if gate is not None else 0) | ((n_tok << 16) if n_tok > 1 else 0)
    out = cmd(OP_ATTN, n_head | (n_head_kv << 16), q, kv, y, head_dim | (n_rot << 16), pos_off, flags)
    out += cmd(k, v, fbits(scale), fbits(eps), qn, kn, cs, gate or 0)
    return out


def get_rows(fmt: int, rows: int, cols: int, w_off: int, id_off: int, y_off: int, n_tok: int = 1) -> list[int]:
    """n_tok > 1: token t's id at act[id_off + 16 t], its row at y_off + t * cols."""
    return cmd(OP_GET_ROWS, fmt | ((n_tok << 16) if n_tok > 1 else 0), rows, cols, w_off & 0xFFFFFFFF, w_off >> 32,
               id_off, y_off)


def argmax(n: int, x: int, key: int) -> list[int]:
    return cmd(OP_ARGMAX, n, x, key)


def next_token(key: int, tok: int, pos: int, prompt: int, n_prompt: int, out: int) -> list[int]:
    return cmd(OP_NEXT_TOKEN, key, tok, pos, prompt, n_prompt, out)


def fill(n: int, y: int, value: float) -> list[int]:
    return cmd(OP_FILL, n, y, fbits(value))


def gemm(fmt: int, rows: int, cols: int, w_off: int, x_off: int, y_off: int, n_tok: int, x_stride: int,
         y_stride: int, flags: int = 0, res_off: int = 0, res_stride: int = 0, norm_w: int = 0, eps: float = 0.0,
         norm_flags: int = 0) -> list[int]:
    """Batched GEMV over n_tok token rows (x_stride / y_stride floats apart); norm_flags NORM_DEFER folds a per-token
    RMS norm (weight at norm_w unless NORM_NO_WEIGHT) into the activation quantization."""
    out = cmd(OP_GEMM, fmt | flags, rows, cols, w_off & 0xFFFFFFFF, w_off >> 32, x_off, y_off)
    out += cmd(n_tok, x_stride, y_stride, res_off, res_stride, norm_w, fbits(eps), norm_flags)
    return out


# ---------------------------------------------------------------------------------------------------------------
_hip = None
_synth = None


class LaunchStat(C.Structure):  # gemvq_launch_stat
    _fields_ = [("name", C.c_char * 40), ("first_cmd", C.c_int32), ("n_cmds", C.c_int32), ("bytes", C.c_uint64),
                ("us", C.c_double)]


def _c_fn(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


def hip_lib() -> C.CDLL:
    """Loads libgemvq_hip.so (raises if it has not been built)."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB_PATH):
            raise RuntimeError(f"{HIP_LIB_PATH} is missing: build it first (python __graft_entry__.py or build.py)")
        lib = C.CDLL(HIP_LIB_PATH)
        vp, u64p = C.c_void_p, C.POINTER(C.c_uint64)
        _c_fn(lib, "gemvq_ctx_create", vp, C.c_int, C.c_size_t, C.c_size_t, C.c_size_t)
        _c_fn(lib, "gemvq_ctx_destroy", None, vp)
        _c_fn(lib, "gemvq_last_error", C.c_char_p, vp)
        _c_fn(lib, "gemvq_features", None, vp, C.POINTER(C.c_uint32))
        _c_fn(lib, "gemvq_upload_weight", C.c_int, vp, C.c_int, C.c_int, C.c_int, vp, u64p)
        _c_fn(lib, "gemvq_weight_bytes_used", C.c_uint64, vp)
        _c_fn(lib, "gemvq_repack", C.c_int, C.c_int, C.c_int, C.c_int, vp, vp)
        _c_fn(lib, "gemvq_unpack", C.c_int, C.c_int, C.c_int, C.c_int, vp, vp)
        _c_fn(lib, "gemvq_act_write", C.c_int, vp, C.c_size_t, vp, C.c_size_t)
        _c_fn(lib, "gemvq_act_read", C.c_int, vp, C.c_size_t, vp, C.c_size_t)
        _c_fn(lib, "gemvq_state_write", C.c_int, vp, C.c_size_t, vp, C.c_size_t)
        _c_fn(lib, "gemvq_state_read", C.c_int, vp, C.c_size_t, vp, C.c_size_t)
        _c_fn(lib, "gemvq_state_clear", C.c_int, vp)
        _c_fn(lib, "gemvq_kv_create", C.c_int, vp, C.c_int, C.c_int, C.c_int)
        _c_fn(lib, "gemvq_kv_read", C.c_int, vp, C.c_int, C.c_int, C.c_int, vp, vp)
        _c_fn(lib, "gemvq_kv_clear", C.c_int, vp)
        _c_fn(lib, "gemvq_run", C.c_int, vp, C.POINTER(C.c_uint32), C.c_uint)
        _c_fn(lib, "gemvq_graph_create", C.c_int, vp, C.POINTER(C.c_uint32), C.c_uint, C.POINTER(C.c_int))
        _c_fn(lib, "gemvq_graph_replay", C.c_int, vp, C.c_int, C.c_int)
        _c_fn(lib, "gemvq_graph_destroy", C.c_int, vp, C.c_int)
        _c_fn(lib, "gemvq_sync", C.c_int, vp)
        _c_fn(lib, "gemvq_set_wait_timeout", C.c_int, vp, C.c_uint)
        _c_fn(lib, "gemvq_usable", C.c_int, vp)
        _c_fn(lib, "gemvq_last_launch_count", C.c_int, vp)
        _c_fn(lib, "gemvq_debug_blocksums", C.c_int, vp, vp, C.c_size_t)
        _c_fn(lib, "gemvq_graph_time", C.c_int, vp, C.c_int, C.c_int, C.POINTER(C.c_double))
        _c_fn(lib, "gemvq_set_arith", C.c_int, vp, C.c_int)
        _c_fn(lib, "gemvq_profile", C.c_int, vp, C.POINTER(C.c_uint32), C.c_uint, C.c_int, C.c_void_p, C.c_int)
        _c_fn(lib, "gemvq_arith", C.c_int, vp)
        _c_fn(lib, "gemvq_cr_expf", C.c_float, C.c_float)
        _c_fn(lib, "gemvq_cr_logf", C.c_float, C.c_float)
        _c_fn(lib, "gemvq_crmath_hash", C.c_int, vp, C.c_int, u64p)
        _hip = lib
    return _hip


def synth_lib() -> C.CDLL:
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB_PATH):
            raise RuntimeError(f"{SYNTH_LIB_PATH} is missing: build it first")
        lib = C.CDLL(SYNTH_LIB_PATH)
        vp = C.c_void_p
        _c_fn(lib, "gqs_u64", C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64)
        _c_fn(lib, "gqs_normal", None, C.c_uint64, C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, vp)
        _c_fn(lib, "gqs_uniform", None, C.c_uint64, C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, vp)
        _c_fn(lib, "gqs_quantize", C.c_size_t, C.c_int, vp, C.c_int64, C.c_int64, vp)
        _c_fn(lib, "gqs_row_bytes", C.c_size_t, C.c_int, C.c_int64)
        _c_fn(lib, "gqs_matrix", C.c_size_t, C.c_int, C.c_int64, C.c_int64, C.c_uint64, C.c_uint64, C.c_float,
              C.c_float, vp, C.c_int)
        _synth = lib
    return _synth


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------------------------------------------------------
# synthetic data
def normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    synth_lib().gqs_normal(seed, stream, first, n, mean, std, _ptr(out))
    return out


def uniform(seed: int, stream: int, n: int, lo: float, hi: float, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    synth_lib().gqs_uniform(seed, stream, first, n, lo, hi, _ptr(out))
    return out


def quantize(t: int, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == rows * cols
    out = np.empty(rows * row_bytes(t, cols), dtype=np.uint8)
    if synth_lib().gqs_quantize(t, _ptr(x), rows, cols, _ptr(out)) != out.size:
        raise ValueError("quantize: unsupported type or shape")
    return out


def matrix(t: int, rows: int, cols: int, seed: int, stream: int, std: float = 0.02, mean: float = 0.0,
           threads: int = 0) -> np.ndarray:
    """rows x cols from N(mean, std^2) quantized to type t (GGUF bytes), generated in parallel."""
    threads = threads or min(16, os.cpu_count() or 1)
    out = np.empty(rows * row_bytes(t, cols), dtype=np.uint8)
    if synth_lib().gqs_matrix(t, rows, cols, seed, stream, mean, std, _ptr(out), threads) != out.size:
        raise ValueError("matrix: unsupported type or shape")
    return out


def repack(t: int, rows: int, cols: int, gguf: np.ndarray) -> np.ndarray:
    out = np.empty_like(gguf)
    if hip_lib().gemvq_repack(t, rows, cols, _ptr(gguf), _ptr(out)) != 0:
        raise ValueError("repack: bad type or shape")
    return out


def unpack(t: int, rows: int, cols: int, packed: np.ndarray) -> np.ndarray:
    out = np.empty_like(packed)
    if hip_lib().gemvq_unpack(t, rows, cols, _ptr(packed), _ptr(out)) != 0:
        raise ValueError("unpack: bad type or shape")
    return out


# ---------------------------------------------------------------------------------------------------------------
class GemvqError(RuntimeError):
    pass


class Context:
    """One device context: activation buffer (floats), weight arena, GDN state rows, KV buffers, graphs."""

    def __init__(self, act_floats: int = 1 << 22, weight_bytes: int = 1 << 28, state_rows: int = 0, device: int = 0):
        self.lib = hip_lib()
        self.h = self.lib.gemvq_ctx_create(device, act_floats, weight_bytes, state_rows)
        if not self.h:
            raise GemvqError(self.lib.gemvq_last_error(None).decode())
        self.act_floats = act_floats

    def close(self) -> None:
        if self.h:
            self.lib.gemvq_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def error(self) -> str:
        return self.lib.gemvq_last_error(self.h).decode()

    def _check(self, st: int, what: str) -> int:
        if st < 0:
            raise GemvqError(f"{what}: status {st}: {self.error()}")
        return st

    def features(self) -> tuple[int, int]:
        out = (C.c_uint32 * 2)()
        self.lib.gemvq_features(self.h, out)
        return int(out[0]), int(out[1])

    def upload(self, t: int, rows: int, cols: int, gguf: np.ndarray) -> int:
        gguf = np.ascontiguousarray(gguf, dtype=np.uint8)
        assert gguf.size == rows * row_bytes(t, cols)
        off = C.c_uint64()
        self._check(self.lib.gemvq_upload_weight(self.h, t, rows, cols, _ptr(gguf), C.byref(off)), "upload")
        return int(off.value)

    def write(self, off: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        assert data.dtype.itemsize == 4
        self._check(self.lib.gemvq_act_write(self.h, off, _ptr(data), data.size), "act write")

    def read(self, off: int, n: int, dtype=np.float32) -> np.ndarray:
        out = np.empty(n, dtype=dtype)
        self._check(self.lib.gemvq_act_read(self.h, off, _ptr(out), n), "act read")
        return out

    def state_write(self, row: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, dtype=np.float32)
        assert data.size % 128 == 0
        self._check(self.lib.gemvq_state_write(self.h, row, _ptr(data), data.size // 128), "state write")

    def state_read(self, row: int, rows: int) -> np.ndarray:
        out = np.empty(rows * 128, dtype=np.float32)
        self._check(self.lib.gemvq_state_read(self.h, row, _ptr(out), rows), "state read")
        return out

    def kv_create(self, n_ctx: int, n_head_kv: int, head_dim: int) -> int:
        return self._check(self.lib.gemvq_kv_create(self.h, n_ctx, n_head_kv, head_dim), "kv create")

    def kv_read(self, kv: int, pos0: int, npos: int, row: int) -> tuple[np.ndarray, np.ndarray]:
        k = np.empty(npos * row, dtype=np.uint16)
        v = np.empty(npos * row, dtype=np.uint16)
        self._check(self.lib.gemvq_kv_read(self.h, kv, pos0, npos, _ptr(k), _ptr(v)), "kv read")
        return k, v

    @staticmethod
    def _words(cmds) -> tuple[np.ndarray, int]:
        w = np.ascontiguousarray(np.asarray(cmds, dtype=np.uint64).astype(np.uint32).ravel())
        assert w.size % 8 == 0
        return w, w.size // 8

    def run(self, cmds) -> int:
        """Runs a command list; returns 0 or the 1-based index of the first invalid command; raises on errors."""
        w, n = self._words(cmds)
        return self._check(self.lib.gemvq_run(self.h, w.ctypes.data_as(C.POINTER(C.c_uint32)), n), "run")

    def graph(self, cmds) -> int:
        w, n = self._words(cmds)
        g = C.c_int(-1)
        st = self.lib.gemvq_graph_create(self.h, w.ctypes.data_as(C.POINTER(C.c_uint32)), n, C.byref(g))
        if st != 0:
            raise GemvqError(f"graph create: status {st}: {self.error()}")
        return g.value

    def replay(self, g: int, times: int = 1) -> None:
        self._check(self.lib.gemvq_graph_replay(self.h, g, times), "replay")

    def graph_time_us(self, g: int, times: int) -> float:
        us = C.c_double()
        self._check(self.lib.gemvq_graph_time(self.h, g, times, C.byref(us)), "graph time")
        return us.value

    def sync(self) -> None:
        self._check(self.lib.gemvq_sync(self.h), "sync")

    def set_wait_timeout(self, ms: int) -> None:
        """Bound of every wait for the device (a timed-out wait makes the context unusable)."""
        self._check(self.lib.gemvq_set_wait_timeout(self.h, ms), "wait timeout")

    def usable(self) -> bool:
        return bool(self.lib.gemvq_usable(self.h))

    def launch_count(self) -> int:
        return self.lib.gemvq_last_launch_count(self.h)

    def set_arith(self, arith: int) -> None:
        """Arithmetic of the lists compiled from now on: ARITH_CANONICAL (default) or ARITH_REFERENCE (the reference's
        CPU arithmetic, gemvq_hip.h)."""
        self._check(self.lib.gemvq_set_arith(self.h, arith), "set arith")

    def arith(self) -> int:
        return self.lib.gemvq_arith(self.h)

    def profile(self, cmds, reps: int = 1) -> list[dict]:
        """The launches the list compiles to, each timed on the stream with HIP events (gemvq_profile: the median
        over reps repetitions of the list): name, first command, HBM bytes (algorithmic), microseconds."""
        w, n = self._words(cmds)
        out = (LaunchStat * 4096)()
        got = self.lib.gemvq_profile(self.h, w.ctypes.data_as(C.POINTER(C.c_uint32)), n, reps, out, 4096)
        if got < 0:
            raise GemvqError(f"profile: {got}: {self.error()}")
        return [dict(name=out[i].name.decode(), first=out[i].first_cmd, bytes=int(out[i].bytes), us=out[i].us)
                for i in range(got)]

    def crmath_hash(self, fn: int) -> np.ndarray:
        """The device's correctly rounded exp (fn 0) or log (fn 1) over every binary32 input, as 4096 block hashes."""
        out = np.zeros(4096, dtype=np.uint64)
        self._check(self.lib.gemvq_crmath_hash(self.h, fn, out.ctypes.data_as(C.POINTER(C.c_uint64))), "crmath hash")
        return out

    def debug_blocksums(self, out: np.ndarray) -> None:
        assert out.dtype == np.int32 and out.flags["C_CONTIGUOUS"]
        self._check(self.lib.gemvq_debug_blocksums(self.h, _ptr(out), out.size), "debug blocksums")
