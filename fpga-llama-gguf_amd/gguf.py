"""GGUF model files: the reader of include/gemvq_gguf.h (ctypes), a writer for synthetic models, the inverse of
ggml's CPU_REPACK Q4_0x8 layout, and the Qwen3.5 configuration a file implies.

The reference gets its weights from llama.cpp's GGUF loader and, for Q4_0 tensors held in the CPU_REPACK buffer
type, turns them back into GGUF rows before its own repack (ggml-xrt.cpp:675-710). `open_model` gives the decode
driver of qwen35.py the same source: the tensors stay in the read-only mapping of the file, and the table handed to
gemvq_qwen35_create points into it. Metadata keys follow llama.cpp's `<arch>.<key>` convention; every dimension
that a tensor's shape fixes is taken from the shape, and metadata only supplies what shapes cannot (eps, RoPE base
and dimensions, context length).
"""
from __future__ import annotations

import ctypes as C
import os
import re
import struct

import numpy as np

import gemvq as gq
import qwen35 as qw

F32, F16 = 0, 1
# bytes per block and elements per block of the ggml types this reader sizes
TYPE_SIZE = {0: (4, 1), 1: (2, 1), 2: (18, 32), 3: (20, 32), 6: (22, 32), 7: (24, 32), 8: (34, 32), 10: (84, 256),
             11: (110, 256), 12: (144, 256), 13: (176, 256), 14: (210, 256), 24: (1, 1), 25: (2, 1), 26: (4, 1),
             30: (2, 1)}

_fns = False


def _lib() -> C.CDLL:
    global _fns
    lib = gq.hip_lib()
    if not _fns:
        vp = C.c_void_p
        gq._c_fn(lib, "gemvq_gguf_open", vp, C.c_char_p)
        gq._c_fn(lib, "gemvq_gguf_close", None, vp)
        gq._c_fn(lib, "gemvq_gguf_last_error", C.c_char_p)
        gq._c_fn(lib, "gemvq_gguf_version", C.c_int, vp)
        gq._c_fn(lib, "gemvq_gguf_n_tensors", C.c_int, vp)
        gq._c_fn(lib, "gemvq_gguf_tensor", C.c_int, vp, C.c_int, C.c_char_p, C.c_size_t, C.POINTER(C.c_int),
                 C.POINTER(C.c_int64), C.POINTER(C.c_void_p), C.POINTER(C.c_uint64))
        gq._c_fn(lib, "gemvq_gguf_file_offset", C.c_int64, vp, C.c_int)
        gq._c_fn(lib, "gemvq_gguf_find", C.c_int, vp, C.c_char_p)
        gq._c_fn(lib, "gemvq_gguf_get_f64", C.c_int, vp, C.c_char_p, C.POINTER(C.c_double))
        gq._c_fn(lib, "gemvq_gguf_get_str", C.c_char_p, vp, C.c_char_p)
        gq._c_fn(lib, "gemvq_unrepack_q4_0x8", C.c_int, C.c_int, C.c_int, vp, vp)
        _fns = True
    return lib


class GGUFError(RuntimeError):
    pass


class Tensor:
    __slots__ = ("name", "type", "ne", "offset", "nbytes")

    def __init__(self, name: str, type_: int, ne: tuple[int, ...], offset: int, nbytes: int):
        self.name, self.type, self.ne, self.offset, self.nbytes = name, type_, ne, offset, nbytes

    def __repr__(self) -> str:
        return f"Tensor({self.name!r}, type={self.type}, ne={self.ne}, offset={self.offset}, nbytes={self.nbytes})"


class GGUF:
    """A parsed, memory-mapped GGUF file. `data` is the whole file as a read-only uint8 array; tensor offsets are
    absolute file offsets into it."""

    def __init__(self, path: str):
        self.lib = _lib()
        self.path = path
        self.h = self.lib.gemvq_gguf_open(os.fsencode(path))
        if not self.h:
            raise GGUFError(self.lib.gemvq_gguf_last_error().decode())
        self.version = self.lib.gemvq_gguf_version(self.h)
        self.tensors: list[Tensor] = []
        name = C.create_string_buffer(256)
        t, ne, ptr, nb = C.c_int(), (C.c_int64 * 4)(), C.c_void_p(), C.c_uint64()
        base = None
        for i in range(self.lib.gemvq_gguf_n_tensors(self.h)):
            self.lib.gemvq_gguf_tensor(self.h, i, name, len(name), C.byref(t), ne, C.byref(ptr), C.byref(nb))
            off = self.lib.gemvq_gguf_file_offset(self.h, i)
            base = (ptr.value or 0) - off
            self.tensors.append(Tensor(name.value.decode(), t.value, tuple(int(x) for x in ne), off, nb.value))
        size = os.path.getsize(path)
        if base is None:  # no tensors: the mapping is not needed
            self.data = np.zeros(0, np.uint8)
        else:
            self.data = np.ctypeslib.as_array((C.c_uint8 * size).from_address(base))
            self.data.flags.writeable = False
        self.by_name = {x.name: x for x in self.tensors}

    def close(self) -> None:
        if getattr(self, "h", None):
            self.data = None
            self.lib.gemvq_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def get(self, key: str, default=None):
        """A metadata value: float for numeric types, str for strings, `default` when absent (arrays are skipped)."""
        v = C.c_double()
        if self.lib.gemvq_gguf_get_f64(self.h, key.encode(), C.byref(v)) == 0:
            return v.value
        s = self.lib.gemvq_gguf_get_str(self.h, key.encode())
        return default if s is None else s.decode()

    def tensor(self, name: str) -> np.ndarray:
        x = self.by_name[name]
        return self.data[x.offset:x.offset + x.nbytes]


# ---------------------------------------------------------------------------------------------------------------
# writer (the GGUF v3 layout; used to put synthetic models into files)
_KV_U32, _KV_F32, _KV_STR, _KV_U64 = 4, 6, 8, 10


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, value) -> bytes:
    if isinstance(value, str):
        return _s(key) + struct.pack("<I", _KV_STR) + _s(value)
    if isinstance(value, float):
        return _s(key) + struct.pack("<If", _KV_F32, value)
    return _s(key) + struct.pack("<II", _KV_U32, int(value))


def write(path: str, kv: dict, tensors: list[tuple[str, int, tuple[int, ...], np.ndarray]], alignment: int = 32) -> None:
    """Writes a GGUF v3 file: `kv` maps keys to int (u32), float (f32) or str values; `tensors` lists
    (name, ggml type, ne (ne0 first), bytes)."""
    kv = dict(kv)
    kv.setdefault("general.alignment", alignment)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv)))
    for k, v in kv.items():
        head += _kv(k, v)
    off = 0
    offsets = []
    for name, t, ne, data in tensors:
        bb, be = TYPE_SIZE[t]
        n = int(np.prod(ne))
        assert ne[0] % be == 0 and data.nbytes == n // be * bb, name
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", t, off)
        offsets.append(off)
        off = (off + data.nbytes + alignment - 1) // alignment * alignment
    start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (start - len(head)))
        pos = 0
        for (name, t, ne, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(np.ascontiguousarray(data).view(np.uint8).tobytes())
            pos = o + data.nbytes
        f.write(b"\0" * (off - pos))


def config_kv(cfg: qw.Config, arch: str = "qwen35") -> dict:
    """The llama.cpp metadata of a Qwen3.5-shaped model."""
    return {"general.architecture": arch, "general.name": "synthetic",
            f"{arch}.block_count": cfg.n_layer, f"{arch}.context_length": 262144,
            f"{arch}.embedding_length": cfg.n_embd, f"{arch}.feed_forward_length": cfg.n_ff,
            f"{arch}.attention.head_count": cfg.n_head, f"{arch}.attention.head_count_kv": cfg.n_head_kv,
            f"{arch}.attention.key_length": cfg.head_dim, f"{arch}.attention.value_length": cfg.head_dim,
            f"{arch}.attention.layer_norm_rms_epsilon": float(cfg.eps),
            f"{arch}.rope.dimension_count": cfg.n_rot, f"{arch}.rope.freq_base": float(cfg.rope_base),
            f"{arch}.ssm.conv_kernel": cfg.ssm_conv, f"{arch}.ssm.state_size": cfg.ssm_head_dim,
            f"{arch}.ssm.group_count": cfg.ssm_k_heads, f"{arch}.ssm.time_step_rank": cfg.ssm_v_heads,
            f"{arch}.ssm.inner_size": cfg.ssm_v_heads * cfg.ssm_head_dim,
            f"{arch}.full_attention_interval": cfg.attn_interval}


def write_model(path: str, blob: qw.Blob, arch: str = "qwen35") -> None:
    """A synthetic model blob as a GGUF file (2-D tensors for matrices, 1-D for vectors)."""
    tensors = []
    for d in blob.table:
        ne = (d.ne0,) if d.ne1 == 1 else (d.ne0, d.ne1)
        tensors.append((d.name.decode(), d.type, ne, blob.data[d.offset:d.offset + d.nbytes]))
    write(path, config_kv(blob.cfg, arch), tensors)


# ---------------------------------------------------------------------------------------------------------------
# Qwen3.5 from a file
_BLK = re.compile(r"^blk\.(\d+)\.")


def config_from(g: GGUF, n_ctx: int = 640) -> qw.Config:
    """The decode configuration of a Qwen3.5-shaped GGUF. Dimensions come from tensor shapes; eps, RoPE base and
    RoPE dimensions from metadata (defaults 1e-6, 1e7, head_dim / 4)."""
    arch = g.get("general.architecture", "qwen35")
    ne = {t.name: t.ne for t in g.tensors}

    def need(name: str):
        if name not in ne:
            raise GGUFError(f"{g.path}: tensor {name} is missing")
        return ne[name]

    layers = sorted({int(m.group(1)) for t in g.tensors if (m := _BLK.match(t.name))})
    if not layers or layers != list(range(len(layers))):
        raise GGUFError(f"{g.path}: layers are not numbered 0..n-1")
    attn = [il for il in layers if f"blk.{il}.attn_q.weight" in ne]
    if not attn:
        raise GGUFError(f"{g.path}: no full-attention layer")
    interval = attn[0] + 1
    if attn != [il for il in layers if (il + 1) % interval == 0]:
        raise GGUFError(f"{g.path}: full-attention layers are not every {interval}th layer")
    n_embd, n_vocab = need("token_embd.weight")[:2]
    a, s = attn[0], next(il for il in layers if il not in attn)
    head_dim = need(f"blk.{a}.attn_q_norm.weight")[0]
    n_head = need(f"blk.{a}.attn_q.weight")[1] // (2 * head_dim)
    n_head_kv = need(f"blk.{a}.attn_k.weight")[1] // head_dim
    S = need(f"blk.{s}.ssm_norm.weight")[0]
    hv = need(f"blk.{s}.ssm_a")[0]
    conv_k, conv_ch = need(f"blk.{s}.ssm_conv1d.weight")[:2]
    hk = (conv_ch - hv * S) // (2 * S)
    if 2 * hk * S + hv * S != conv_ch:
        raise GGUFError(f"{g.path}: ssm_conv1d channels {conv_ch} do not split into q, k (2 x {S} x hk) and v")
    mtype = g.by_name[f"blk.{s}.ffn_gate.weight"].type
    etype = g.by_name["output.weight" if "output.weight" in ne else "token_embd.weight"].type
    return qw.Config(n_layer=len(layers), n_embd=n_embd, n_ff=need(f"blk.{s}.ffn_gate.weight")[1], n_vocab=n_vocab,
                     n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim,
                     n_rot=int(g.get(f"{arch}.rope.dimension_count", head_dim // 4)), ssm_k_heads=hk,
                     ssm_v_heads=hv, ssm_head_dim=S, ssm_conv=conv_k, attn_interval=interval, n_ctx=n_ctx,
                     eps=float(g.get(f"{arch}.attention.layer_norm_rms_epsilon", 1e-6)),
                     rope_base=float(g.get(f"{arch}.rope.freq_base", 1e7)), wtype=mtype, etype=etype)


def open_model(path: str, n_ctx: int = 640) -> qw.Blob:
    """A Qwen3.5 GGUF as a model blob for qwen35.Model: the table points into the file's mapping, which the blob
    keeps open. A file without output.weight (tied embeddings) uses token_embd.weight for the head. Vectors must be
    F32 (the decode path reads norms, conv kernels and gates as fp32)."""
    g = GGUF(path)
    try:
        cfg = config_from(g, n_ctx)
        names = [n for n, *_ in qw.tensor_specs(cfg)]
        table = (qw.TensorDesc * len(names))()
        for i, n in enumerate(names):
            t = g.by_name.get(n) or (g.by_name["token_embd.weight"] if n == "output.weight" else None)
            if t is None:
                raise GGUFError(f"{path}: tensor {n} is missing")
            if len(t.ne) > 2 and any(d != 1 for d in t.ne[2:]):
                raise GGUFError(f"{path}: tensor {n} has more than 2 dimensions")
            ne0, ne1 = t.ne[0], t.ne[1] if len(t.ne) > 1 else 1
            if t.type == F16:
                raise GGUFError(f"{path}: tensor {n} is F16; the decode path takes F32 vectors")
            table[i] = qw.TensorDesc(n.encode(), t.type, ne0, ne1, 0, t.offset, t.nbytes)
    except Exception:
        g.close()
        raise
    return qw.Blob(cfg, table, g.data, len(names), owner=g)


def unrepack_q4_0x8(rows: int, cols: int, x8: np.ndarray) -> np.ndarray:
    """block_q4_0x8 data (CPU_REPACK) -> GGUF Q4_0 rows (ggml-xrt.cpp:675-710); lossless."""
    x8 = np.ascontiguousarray(x8, np.uint8)
    if rows % 8 or cols % 32 or x8.nbytes != rows * cols // 32 * 18:
        raise ValueError(f"unrepack_q4_0x8: bad shape {rows}x{cols} for {x8.nbytes} bytes")
    out = np.empty(rows * cols // 32 * 18, np.uint8)
    if _lib().gemvq_unrepack_q4_0x8(rows, cols, x8.ctypes.data, out.ctypes.data):
        raise ValueError("unrepack_q4_0x8 failed")
    return out
