"""The ggml-shaped graph IR of include/gemvq_ggml.h from Python: tensors with ggml's fields, graph builders named as
ggml's constructors (ggml_mul_mat, ggml_rms_norm, ggml_view_2d, ...), and the backend's C ABI (plan, compute,
recurrent-state and KV buffers). Host tensors own numpy buffers; weights point into a model blob."""
from __future__ import annotations

import ctypes as C

import numpy as np

import gemvq as gq

F32, F16, Q4_0, Q4_1, Q8_0, Q5_K, Q6_K, I32, I64 = 0, 1, 2, 3, 8, 13, 14, 26, 27
(OP_NONE, OP_ADD, OP_MUL, OP_SCALE, OP_RMS_NORM, OP_L2_NORM, OP_MUL_MAT, OP_CPY, OP_CONT, OP_RESHAPE, OP_VIEW,
 OP_PERMUTE, OP_TRANSPOSE, OP_GET_ROWS, OP_SET_ROWS, OP_CONCAT, OP_ROPE, OP_FLASH_ATTN_EXT, OP_SSM_CONV,
 OP_GATED_DELTA_NET, OP_UNARY, OP_GLU, OP_SOFT_MAX) = range(23)
UNARY_SILU, UNARY_SIGMOID, UNARY_SOFTPLUS = 1, 2, 3
GLU_SWIGLU = 1
ROPE_NEOX = 2
FLAG_INPUT, FLAG_OUTPUT, FLAG_SPLIT_OUTPUT = 1, 2, 1 << 8
BUF_HOST, BUF_WEIGHTS, BUF_RS, BUF_KV = 0, 1, 2, 3
STATUS_SUCCESS, STATUS_FAILED, STATUS_ALLOC_FAILED = 0, -1, -2

_BLOCK = {F32: (1, 4), F16: (1, 2), I32: (1, 4), I64: (1, 8), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34),
          Q5_K: (256, 176), Q6_K: (256, 210)}


class Tensor(C.Structure):
    pass


Tensor._fields_ = [("type", C.c_int32), ("op", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4),
                   ("op_params", C.c_int32 * 16), ("flags", C.c_int32), ("buffer", C.c_int32),
                   ("src", C.POINTER(Tensor) * 10), ("view_src", C.POINTER(Tensor)), ("view_offs", C.c_size_t),
                   ("data", C.c_void_p), ("name", C.c_char * 64)]


class CGraph(C.Structure):
    _fields_ = [("n_nodes", C.c_int), ("nodes", C.POINTER(C.POINTER(Tensor)))]


class Params(C.Structure):
    _fields_ = [("device", C.c_int), ("act_floats", C.c_size_t), ("weight_bytes", C.c_size_t),
                ("state_rows", C.c_size_t), ("dry", C.c_int)]


def _fbits(x: float) -> int:
    return int(np.array([x], np.float32).view(np.int32)[0])


def nelements(t: Tensor) -> int:
    return int(t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3])


class Graph:
    """Tensors and the forward order of one graph (ggml_build_forward_expand: sources before their readers)."""

    def __init__(self):
        self.tensors: list[Tensor] = []
        self.keep: list[object] = []  # host buffers
        self.nodes: list[Tensor] = []
        self._in: set[int] = set()

    # ---- tensors ----
    def _make(self, type_: int, ne, name: str = "", op: int = OP_NONE) -> Tensor:
        t = Tensor()
        ne = list(ne) + [1] * (4 - len(ne))
        blk, size = _BLOCK[type_]
        t.type, t.op = type_, op
        for d in range(4):
            t.ne[d] = ne[d]
        t.nb[0] = size
        t.nb[1] = size * (ne[0] // blk)
        t.nb[2] = t.nb[1] * ne[1]
        t.nb[3] = t.nb[2] * ne[2]
        t.name = name.encode()[:63]
        self.tensors.append(t)
        return t

    def new(self, type_: int, ne, name: str = "", flags: int = 0, op: int = OP_NONE) -> Tensor:
        """A tensor with its own host buffer."""
        t = self._make(type_, ne, name, op)
        n = int(np.prod([x for x in ne])) * _BLOCK[type_][1] // _BLOCK[type_][0]
        buf = np.zeros(max(n, 16) + 64, np.uint8)
        off = (-buf.ctypes.data) % 64
        self.keep.append(buf)
        t.data = buf.ctypes.data + off
        t.flags = flags
        return t

    def at(self, type_: int, ne, data: int, name: str = "", buffer: int = BUF_HOST) -> Tensor:
        """A tensor over existing memory (weights in a blob, a state or KV buffer)."""
        t = self._make(type_, ne, name)
        t.data = data
        t.buffer = buffer
        return t

    def host(self, t: Tensor, dtype=np.float32) -> np.ndarray:
        return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(np.ctypeslib.as_ctypes_type(dtype))), (nelements(t),))

    def _op(self, op: int, type_: int, ne, srcs, name: str = "", params=()) -> Tensor:
        t = self.new(type_, ne, name, op=op)
        for i, s in enumerate(srcs):
            if s is not None:
                t.src[i] = C.pointer(s)
        for i, p in enumerate(params):
            t.op_params[i] = p
        return t

    def _view(self, op: int, a: Tensor, ne, nb, offs: int, name: str = "") -> Tensor:
        t = self._make(a.type, ne, name or a.name.decode() + " (view)", op)
        for d in range(4):
            t.nb[d] = nb[d]
        root = a
        offs_total = offs
        if a.view_src:
            root = a.view_src.contents
            offs_total += a.view_offs
        t.view_src = C.pointer(root)
        t.view_offs = offs_total
        t.data = a.data + offs
        t.buffer = root.buffer
        t.src[0] = C.pointer(a)
        return t

    # ---- ggml constructors ----
    def view(self, a: Tensor, ne, nb1: int = 0, nb2: int = 0, offs: int = 0, name: str = "") -> Tensor:
        ne = list(ne) + [1] * (4 - len(ne))
        es = _BLOCK[a.type][1]
        nb = [es, nb1 or es * ne[0], 0, 0]
        nb[2] = nb2 or nb[1] * ne[1]
        nb[3] = nb[2] * ne[2]
        return self._view(OP_VIEW, a, ne, nb, offs, name)

    def reshape(self, a: Tensor, ne, name: str = "") -> Tensor:
        ne = list(ne) + [1] * (4 - len(ne))
        es = _BLOCK[a.type][1]
        nb = [es, es * ne[0], es * ne[0] * ne[1], es * ne[0] * ne[1] * ne[2]]
        return self._view(OP_RESHAPE, a, ne, nb, 0, name)

    def transpose(self, a: Tensor) -> Tensor:
        ne = [a.ne[1], a.ne[0], a.ne[2], a.ne[3]]
        nb = [a.nb[1], a.nb[0], a.nb[2], a.nb[3]]
        return self._view(OP_TRANSPOSE, a, ne, nb, 0)

    def permute(self, a: Tensor, axes) -> Tensor:
        ne, nb = [0] * 4, [0] * 4
        for i, ax in enumerate(axes):
            ne[ax], nb[ax] = a.ne[i], a.nb[i]
        return self._view(OP_PERMUTE, a, ne, nb, 0)

    def mul_mat(self, w: Tensor, x: Tensor, name: str = "") -> Tensor:
        return self._op(OP_MUL_MAT, F32, [w.ne[1], x.ne[1]], [w, x], name)

    def rms_norm(self, x: Tensor, eps: float, name: str = "") -> Tensor:
        return self._op(OP_RMS_NORM, F32, list(x.ne), [x], name, [_fbits(eps)])

    def l2_norm(self, x: Tensor, eps: float, name: str = "") -> Tensor:
        return self._op(OP_L2_NORM, F32, list(x.ne), [x], name, [_fbits(eps)])

    def mul(self, a: Tensor, b: Tensor, name: str = "") -> Tensor:
        return self._op(OP_MUL, F32, list(a.ne), [a, b], name)

    def add(self, a: Tensor, b: Tensor, name: str = "") -> Tensor:
        return self._op(OP_ADD, F32, list(a.ne), [a, b], name)

    def unary(self, a: Tensor, kind: int, name: str = "") -> Tensor:
        return self._op(OP_UNARY, F32, list(a.ne), [a], name, [kind])

    def swiglu(self, a: Tensor, b: Tensor, name: str = "") -> Tensor:
        return self._op(OP_GLU, F32, list(a.ne), [a, b], name, [GLU_SWIGLU, 0])

    def cont(self, a: Tensor, name: str = "") -> Tensor:
        return self._op(OP_CONT, F32, list(a.ne), [a], name)

    def get_rows(self, a: Tensor, ids: Tensor, name: str = "") -> Tensor:
        return self._op(OP_GET_ROWS, F32, [a.ne[0], ids.ne[0]], [a, ids], name)

    def concat(self, a: Tensor, b: Tensor, dim: int = 0, name: str = "") -> Tensor:
        ne = list(a.ne)
        ne[dim] += b.ne[dim]
        return self._op(OP_CONCAT, F32, ne, [a, b], name, [dim])

    def ssm_conv(self, sx: Tensor, c: Tensor, name: str = "") -> Tensor:
        return self._op(OP_SSM_CONV, F32, [c.ne[1], sx.ne[0] - c.ne[0] + 1, sx.ne[2]], [sx, c], name)

    def gated_delta_net(self, q, k, v, g, beta, state, name: str = "") -> Tensor:
        hv, S = v.ne[1], v.ne[0]
        return self._op(OP_GATED_DELTA_NET, F32, [hv * S + hv * S * S], [q, k, v, g, beta, state], name, [1])

    def cpy(self, a: Tensor, b: Tensor, name: str = "") -> Tensor:
        t = self._view(OP_CPY, b, list(b.ne), list(b.nb), 0, name)
        t.src[0] = C.pointer(a)
        t.src[1] = C.pointer(b)
        return t

    def set_rows(self, dst: Tensor, src: Tensor, idx: Tensor, name: str = "") -> Tensor:
        t = self._view(OP_SET_ROWS, dst, list(dst.ne), list(dst.nb), 0, name)
        t.src[0] = C.pointer(dst)
        t.src[1] = C.pointer(src)
        t.src[2] = C.pointer(idx)
        return t

    def rope(self, x: Tensor, pos: Tensor, n_dims: int, mode: int, freq_base: float, name: str = "") -> Tensor:
        p = [0, n_dims, mode, 0, 0, _fbits(freq_base), _fbits(1.0), _fbits(0.0), _fbits(1.0), _fbits(32.0), _fbits(1.0)]
        return self._op(OP_ROPE, F32, list(x.ne), [x, pos], name, p)

    def flash_attn_ext(self, q, k, v, mask, scale: float, name: str = "") -> Tensor:
        # ggml's result: [head_dim, n_head, n_tokens] (permuted back)
        return self._op(OP_FLASH_ATTN_EXT, F32, [q.ne[0], q.ne[2], q.ne[1]], [q, k, v, mask], name,
                        [_fbits(scale), _fbits(0.0), _fbits(0.0)])

    def soft_max(self, a: Tensor, name: str = "") -> Tensor:
        return self._op(OP_SOFT_MAX, F32, list(a.ne), [a], name)

    # ---- order ----
    def expand(self, t: Tensor) -> None:
        """ggml_build_forward_expand: t after its sources, src[0] first (leafs are not nodes)."""
        stack = [[t, 0]]
        while stack:
            x, i = stack[-1]
            if C.addressof(x) in self._in:
                stack.pop()
                continue
            while i < 10:
                if x.src[i] and C.addressof(x.src[i].contents) not in self._in:
                    stack[-1][1] = i + 1
                    stack.append([x.src[i].contents, 0])
                    break
                i += 1
            else:
                stack.pop()
                self._in.add(C.addressof(x))
                if x.op != OP_NONE:
                    self.nodes.append(x)

    def cgraph(self, nodes: list[Tensor] | None = None) -> CGraph:
        nodes = self.nodes if nodes is None else nodes
        arr = (C.POINTER(Tensor) * len(nodes))(*[C.pointer(x) for x in nodes])
        self.keep.append(arr)
        return CGraph(len(nodes), arr)


_fns = False


def lib():
    global _fns
    L = gq.hip_lib()
    if not _fns:
        vp, P = C.c_void_p, C.POINTER
        gq._c_fn(L, "gqg_backend_init", vp, P(Params))
        gq._c_fn(L, "gqg_backend_free", None, vp)
        gq._c_fn(L, "gqg_backend_error", C.c_char_p, vp)
        gq._c_fn(L, "gqg_supports_op", C.c_int, vp, P(Tensor))
        gq._c_fn(L, "gqg_graph_compute", C.c_int, vp, P(CGraph))
        gq._c_fn(L, "gqg_graph_plan", C.c_int, vp, P(CGraph), P(C.c_uint32), C.c_size_t)
        gq._c_fn(L, "gqg_plan_stats", None, vp, P(C.c_uint64))
        gq._c_fn(L, "gqg_graph_io", C.c_int, vp, P(CGraph), P(vp), P(vp), C.c_size_t, P(C.c_int))
        gq._c_fn(L, "gqg_rs_buffer_alloc", vp, vp, C.c_size_t)
        gq._c_fn(L, "gqg_kv_buffer_alloc", vp, vp, C.c_size_t)
        gq._c_fn(L, "gqg_buffer_base", vp, vp)
        gq._c_fn(L, "gqg_buffer_init_tensor", C.c_int, vp, P(Tensor))
        gq._c_fn(L, "gqg_buffer_set", C.c_int, vp, P(Tensor), vp, C.c_size_t, C.c_size_t)
        gq._c_fn(L, "gqg_buffer_get", C.c_int, vp, P(Tensor), vp, C.c_size_t, C.c_size_t)
        gq._c_fn(L, "gqg_buffer_clear", C.c_int, vp, C.c_uint8)
        gq._c_fn(L, "gqg_buffer_free", None, vp)
        gq._c_fn(L, "gqg_backend_get_reg", vp)
        _fns = True
    return L


class Backend:
    """A gqg_backend (dry: plans only, no device)."""

    def __init__(self, act_floats: int, weight_bytes: int, state_rows: int, dry: bool = False, device: int = 0):
        self.L = lib()
        self.h = self.L.gqg_backend_init(C.byref(Params(device, act_floats, weight_bytes, state_rows, int(dry))))
        if not self.h:
            raise RuntimeError("gqg_backend_init failed (one backend per process)")
        self.buffers: list[int] = []

    def close(self):
        if self.h:
            self.L.gqg_backend_free(self.h)  # buffers still held are detached, then freed here
            self.h = None
        for b in self.buffers:
            self.L.gqg_buffer_free(b)
        self.buffers = []

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def error(self) -> str:
        return self.L.gqg_backend_error(self.h).decode()

    def supports(self, t: Tensor) -> bool:
        return bool(self.L.gqg_supports_op(self.h, C.byref(t)))

    def plan(self, g: CGraph, cap_cmds: int = 1 << 16) -> np.ndarray:
        """The command words the split compiles to (one plan lookup)."""
        w = np.zeros(cap_cmds * 8, np.uint32)
        n = self.L.gqg_graph_plan(self.h, C.byref(g), w.ctypes.data_as(C.POINTER(C.c_uint32)), w.size)
        if n < 0:
            raise RuntimeError(f"plan: {self.error()}")
        if n > cap_cmds:
            raise RuntimeError(f"plan: {n} commands exceed {cap_cmds}")
        return w[:n * 8].reshape(n, 8).copy()

    def compute(self, g: CGraph) -> int:
        return self.L.gqg_graph_compute(self.h, C.byref(g))

    def io(self, g: CGraph, cap: int = 256) -> tuple[list[int], list[int]]:
        """The host data addresses the split's plan copies in and copies back."""
        ins, outs = (C.c_void_p * cap)(), (C.c_void_p * cap)()
        counts = (C.c_int * 2)()
        if self.L.gqg_graph_io(self.h, C.byref(g), ins, outs, cap, counts) != 0:
            raise RuntimeError(f"io: {self.error()}")
        return [ins[i] for i in range(min(counts[0], cap))], [outs[i] for i in range(min(counts[1], cap))]

    def stats(self) -> tuple[int, int]:
        out = (C.c_uint64 * 2)()
        self.L.gqg_plan_stats(self.h, out)
        return int(out[0]), int(out[1])

    def buffer(self, size: int, kind: int) -> int:
        b = (self.L.gqg_rs_buffer_alloc if kind == BUF_RS else self.L.gqg_kv_buffer_alloc)(self.h, size)
        if not b:
            raise RuntimeError("buffer alloc failed")
        self.buffers.append(b)
        return b

    def free_buffer(self, b: int) -> None:
        if b in self.buffers:
            self.buffers.remove(b)
            self.L.gqg_buffer_free(b)
