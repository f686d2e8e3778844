"""Synthetic Qwen3.5-shaped hybrid model and its decode driver (Python side of include/gemvq_qwen35.h).

The 9B shape: 32 layers in a 3:1 pattern of Gated DeltaNet to full attention (8 attention layers, GQA 16 query /
4 KV heads, head dim 256, partial RoPE over 64 dims with theta 1e7), hidden 4096, SwiGLU FFN 12288, vocab 151936;
DeltaNet: 16 key heads and 32 value heads of dim 128, conv kernel 4 over the 8192 qkv channels. Layer matrices are
N(0, 0.02^2) quantized to Q4_0 (or another type), embedding and head Q6_K, norms fp32 ones. The remaining fp32
vectors, which the shape does not fix, are: conv kernel N(0, 0.5^2), dt bias 0 and a = -1 (A_log = 0), so
decay = exp(-softplus(alpha)). Tensor names follow GGUF / llama.cpp's qwen35 conventions.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os

import numpy as np

import gemvq as gq

F32 = 0


@dataclasses.dataclass
class Config:
    n_layer: int = 32
    n_embd: int = 4096
    n_ff: int = 12288
    n_vocab: int = 151936
    n_head: int = 16
    n_head_kv: int = 4
    head_dim: int = 256
    n_rot: int = 64
    ssm_k_heads: int = 16
    ssm_v_heads: int = 32
    ssm_head_dim: int = 128
    ssm_conv: int = 4
    attn_interval: int = 4
    n_ctx: int = 640
    eps: float = 1e-6
    rope_base: float = 1e7
    wtype: int = gq.Q4_0       # layer matrices
    etype: int = gq.Q6_K       # embedding and output head

    def is_attn(self, il: int) -> bool:
        return (il + 1) % self.attn_interval == 0

    @property
    def conv_ch(self) -> int:
        return 2 * self.ssm_k_heads * self.ssm_head_dim + self.ssm_v_heads * self.ssm_head_dim


QWEN35_9B = Config()


def tiny(n_layer: int = 4, n_embd: int = 256, n_ff: int = 512, n_vocab: int = 1024, n_ctx: int = 96,
         wtype: int = gq.Q4_0) -> Config:
    """The same structure at test sizes (GDN heads keep dim 128, attention keeps GQA 4:1)."""
    return Config(n_layer=n_layer, n_embd=n_embd, n_ff=n_ff, n_vocab=n_vocab, n_head=4, n_head_kv=1, head_dim=128,
                  n_rot=32, ssm_k_heads=1, ssm_v_heads=2, ssm_head_dim=128, n_ctx=n_ctx, wtype=wtype)


class ConfigC(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layer", "n_embd", "n_ff", "n_vocab", "n_head", "n_head_kv", "head_dim",
                                         "n_rot", "ssm_k_heads", "ssm_v_heads", "ssm_head_dim", "ssm_conv",
                                         "attn_interval", "n_ctx")] + [("eps", C.c_float), ("rope_base", C.c_float)]


class TensorDesc(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("type", C.c_int32), ("ne0", C.c_int32), ("ne1", C.c_int32),
                ("pad", C.c_int32), ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


def config_c(cfg: Config) -> ConfigC:
    return ConfigC(*[getattr(cfg, f[0]) for f in ConfigC._fields_])


def tensor_specs(cfg: Config, types: dict[str, int] | None = None) -> list[tuple[str, int, int, int, str]]:
    """(name, type, ne0 = cols, ne1 = rows, init) for every tensor; init is 'w', 'ones', 'zeros', 'neg1', 'conv'.
    `types` overrides the ggml type of named matrices (a real "Q4_0" Qwen3.5 file holds some Q4_1 ffn_down)."""
    E, S = cfg.n_embd, cfg.ssm_head_dim
    specs = [("token_embd.weight", cfg.etype, E, cfg.n_vocab, "w")]
    for il in range(cfg.n_layer):
        p = f"blk.{il}."
        specs.append((p + "attn_norm.weight", F32, E, 1, "ones"))
        if cfg.is_attn(il):
            hd = cfg.head_dim
            specs += [(p + "attn_q.weight", cfg.wtype, E, 2 * cfg.n_head * hd, "w"),
                      (p + "attn_k.weight", cfg.wtype, E, cfg.n_head_kv * hd, "w"),
                      (p + "attn_v.weight", cfg.wtype, E, cfg.n_head_kv * hd, "w"),
                      (p + "attn_q_norm.weight", F32, hd, 1, "ones"),
                      (p + "attn_k_norm.weight", F32, hd, 1, "ones"),
                      (p + "attn_output.weight", cfg.wtype, cfg.n_head * hd, E, "w")]
        else:
            hv = cfg.ssm_v_heads
            specs += [(p + "attn_qkv.weight", cfg.wtype, E, cfg.conv_ch, "w"),
                      (p + "attn_gate.weight", cfg.wtype, E, hv * S, "w"),
                      (p + "ssm_beta.weight", cfg.wtype, E, hv, "w"),
                      (p + "ssm_alpha.weight", cfg.wtype, E, hv, "w"),
                      (p + "ssm_conv1d.weight", F32, cfg.ssm_conv, cfg.conv_ch, "conv"),
                      (p + "ssm_dt.bias", F32, hv, 1, "zeros"),
                      (p + "ssm_a", F32, hv, 1, "neg1"),
                      (p + "ssm_norm.weight", F32, S, 1, "ones"),
                      (p + "ssm_out.weight", cfg.wtype, hv * S, E, "w")]
        specs += [(p + "post_attention_norm.weight", F32, E, 1, "ones"),
                  (p + "ffn_gate.weight", cfg.wtype, E, cfg.n_ff, "w"),
                  (p + "ffn_up.weight", cfg.wtype, E, cfg.n_ff, "w"),
                  (p + "ffn_down.weight", cfg.wtype, cfg.n_ff, E, "w")]
    specs += [("output_norm.weight", F32, E, 1, "ones"), ("output.weight", cfg.etype, E, cfg.n_vocab, "w")]
    if types:
        unknown = set(types) - {n for n, t, *_ in specs if t != F32}
        if unknown:
            raise KeyError(f"type overrides for tensors that are not matrices: {sorted(unknown)}")
        specs = [(n, types.get(n, t), a, b, i) for n, t, a, b, i in specs]
    return specs


def tensor_bytes(t: int, ne0: int, ne1: int) -> int:
    return ne0 * ne1 * 4 if t == F32 else ne1 * gq.row_bytes(t, ne0)


def weight_bytes(cfg: Config) -> int:
    """GGUF bytes of the quantized matrices one token reads (layer matrices and the head; not the embedding)."""
    return sum(tensor_bytes(t, a, b) for n, t, a, b, _ in tensor_specs(cfg)
               if t != F32 and n != "token_embd.weight")


@dataclasses.dataclass
class Blob:
    cfg: Config
    table: C.Array
    data: np.ndarray
    n: int
    owner: object = None  # what keeps `data` alive (the GGUF mapping of a model read from a file)

    def tensor(self, name: str) -> np.ndarray:
        for d in self.table:
            if d.name.decode() == name:
                return self.data[d.offset:d.offset + d.nbytes]
        raise KeyError(name)


def generate(cfg: Config, seed: int = 0, threads: int = 0, types: dict[str, int] | None = None) -> Blob:
    """All tensors of the model from `seed`: tensor i uses RNG stream 1000 + i."""
    specs = tensor_specs(cfg, types)
    table = (TensorDesc * len(specs))()
    off = 0
    for i, (name, t, ne0, ne1, _) in enumerate(specs):
        nb = tensor_bytes(t, ne0, ne1)
        table[i] = TensorDesc(name.encode(), t, ne0, ne1, 0, off, nb)
        off += (nb + 255) // 256 * 256
    data = np.zeros(off, np.uint8)
    for i, (name, t, ne0, ne1, init) in enumerate(specs):
        d = table[i]
        view = data[d.offset:d.offset + d.nbytes]
        if t != F32:
            view[:] = gq.matrix(t, ne1, ne0, seed, 1000 + i, std=0.02, threads=threads)
        else:
            n = ne0 * ne1
            if init == "ones":
                v = np.ones(n, np.float32)
            elif init == "zeros":
                v = np.zeros(n, np.float32)
            elif init == "neg1":
                v = -np.ones(n, np.float32)
            else:
                v = gq.normal(seed, 1000 + i, n, 0.0, 0.5)
            view[:] = v.view(np.uint8)
    return Blob(cfg, table, data, len(specs))


def prompt_ids(cfg: Config, n: int, seed: int = 0) -> np.ndarray:
    """n token ids uniform over the vocabulary (RNG stream 7)."""
    synth = gq.synth_lib()
    return np.array([synth.gqs_u64(seed, 7, i) % cfg.n_vocab for i in range(n)], np.int32)


_fns = False


def _lib():
    global _fns
    lib = gq.hip_lib()
    if not _fns:
        vp = C.c_void_p
        gq._c_fn(lib, "gemvq_qwen35_sizes", C.c_int, vp, vp, C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t),
                 C.POINTER(C.c_size_t))
        gq._c_fn(lib, "gemvq_qwen35_create", vp, vp, vp, vp, C.c_int, vp)
        gq._c_fn(lib, "gemvq_qwen35_destroy", None, vp)
        gq._c_fn(lib, "gemvq_qwen35_reset", C.c_int, vp, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_step", C.c_int, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_prefill", C.c_int, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_tokens", C.c_int, vp, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_logits", C.c_int, vp, vp)
        gq._c_fn(lib, "gemvq_qwen35_hidden", C.c_int, vp, vp)
        gq._c_fn(lib, "gemvq_qwen35_commands", C.c_int, vp, vp, C.c_size_t)
        gq._c_fn(lib, "gemvq_qwen35_graph", C.c_int, vp)
        gq._c_fn(lib, "gemvq_qwen35_set_arith", C.c_int, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_batch_sizes", C.c_int, vp, vp, C.c_int, C.c_int, C.POINTER(C.c_size_t),
                 C.POINTER(C.c_size_t), C.POINTER(C.c_size_t))
        gq._c_fn(lib, "gemvq_qwen35_batch_create", vp, vp, vp, vp, C.c_int, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_batch_reset", C.c_int, vp, vp, vp)
        gq._c_fn(lib, "gemvq_qwen35_batch_tokens", C.c_int, vp, C.c_int, vp, C.c_int)
        gq._c_fn(lib, "gemvq_qwen35_batch_logits", C.c_int, vp, C.c_int, vp)
        _fns = True
    return lib


class Model:
    """The model on the GPU: one context sized for it, the weights uploaded, the per-token command list built (its
    graph is captured by the first `step`)."""

    def __init__(self, blob: Blob, device: int = 0):
        self.lib = _lib()
        self.cfg = blob.cfg
        self.cc = config_c(blob.cfg)
        act, wb, st = C.c_size_t(), C.c_size_t(), C.c_size_t()
        if self.lib.gemvq_qwen35_sizes(C.byref(self.cc), blob.table, blob.n, C.byref(act), C.byref(wb), C.byref(st)):
            raise gq.GemvqError("qwen35 sizes")
        self.ctx = gq.Context(act_floats=act.value, weight_bytes=wb.value, state_rows=st.value, device=device)
        self.h = self.lib.gemvq_qwen35_create(self.ctx.h, C.byref(self.cc), blob.table, blob.n, blob.data.ctypes.data)
        if not self.h:
            raise gq.GemvqError("qwen35 create: " + self.ctx.error())

    def close(self):
        if getattr(self, "h", None):
            self.lib.gemvq_qwen35_destroy(self.h)
            self.h = None
        if getattr(self, "ctx", None):
            self.ctx.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _ok(self, st, what):
        if st:
            raise gq.GemvqError(f"{what}: status {st}: {self.ctx.error()}")

    def reset(self, prompt: np.ndarray) -> None:
        p = np.ascontiguousarray(prompt, np.int32)
        self._ok(self.lib.gemvq_qwen35_reset(self.h, p.ctypes.data, p.size), "reset")

    def step(self, n: int = 1) -> None:
        self._ok(self.lib.gemvq_qwen35_step(self.h, n), "step")

    def prefill(self, n: int) -> bool:
        """Runs the next n prompt positions batched (GEMM commands); False (nothing run) when the model's
        projections have no batched form, in which case `step(n)` does the same work."""
        st = self.lib.gemvq_qwen35_prefill(self.h, n)
        if st == gq.EINVAL and any(w in self.ctx.error() for w in ("no batched GEMV", "multiples of 512")):
            return False
        self._ok(st, "prefill")
        return True

    def sync(self) -> None:
        self.ctx.sync()

    def step_direct(self, n: int = 1) -> None:
        """n decode steps as plain stream launches of the same command list (no graph; each step synchronizes)."""
        cmds = self.commands()
        for _ in range(n):
            st = self.ctx.run(cmds)
            if st:
                raise gq.GemvqError(f"step_direct: command {st}: {self.ctx.error()}")

    def tokens(self, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self._ok(self.lib.gemvq_qwen35_tokens(self.h, out.ctypes.data, n), "tokens")
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.n_vocab, np.float32)
        self._ok(self.lib.gemvq_qwen35_logits(self.h, out.ctypes.data), "logits")
        return out

    def hidden(self) -> np.ndarray:
        out = np.empty(self.cfg.n_embd, np.float32)
        self._ok(self.lib.gemvq_qwen35_hidden(self.h, out.ctypes.data), "hidden")
        return out

    def commands(self) -> np.ndarray:
        n = self.lib.gemvq_qwen35_commands(self.h, None, 0)
        out = np.empty(n * 8, np.uint32)
        self.lib.gemvq_qwen35_commands(self.h, out.ctypes.data, out.size)
        return out.reshape(n, 8)

    def graph(self) -> int:
        return self.lib.gemvq_qwen35_graph(self.h)

    def set_arith(self, arith: int) -> None:
        """gq.ARITH_REFERENCE: the following steps and prefills in the reference's CPU arithmetic (gemvq_hip.h)."""
        self._ok(self.lib.gemvq_qwen35_set_arith(self.h, arith), "set arith")

    def generate(self, prompt: np.ndarray, n_gen: int) -> np.ndarray:
        """Greedy decode: the prompt token by token, then n_gen generated tokens; returns all ids."""
        self.reset(prompt)
        self.step(len(prompt) - 1 + n_gen)
        return self.tokens(len(prompt) + n_gen)


class BatchModel:
    """n_seq sequences decoded in lockstep on the GPU (include/gemvq_qwen35.h gemvq_qwen35_batch_*): one step
    advances every sequence by one position, the layer projections reading each weight row once for all of them."""

    def __init__(self, blob: Blob, n_seq: int, device: int = 0):
        self.lib = _lib()
        self.cfg = blob.cfg
        self.n_seq = n_seq
        self.cc = config_c(blob.cfg)
        act, wb, st = C.c_size_t(), C.c_size_t(), C.c_size_t()
        if self.lib.gemvq_qwen35_batch_sizes(C.byref(self.cc), blob.table, blob.n, n_seq, C.byref(act), C.byref(wb),
                                             C.byref(st)):
            raise gq.GemvqError("qwen35 batch sizes")
        self.ctx = gq.Context(act_floats=act.value, weight_bytes=wb.value, state_rows=st.value, device=device)
        self.h = self.lib.gemvq_qwen35_batch_create(self.ctx.h, C.byref(self.cc), blob.table, blob.n,
                                                    blob.data.ctypes.data, n_seq)
        if not self.h:
            raise gq.GemvqError("qwen35 batch create: " + self.ctx.error())

    def close(self):
        if getattr(self, "h", None):
            self.lib.gemvq_qwen35_destroy(self.h)
            self.h = None
        if getattr(self, "ctx", None):
            self.ctx.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _ok(self, st, what):
        if st:
            raise gq.GemvqError(f"{what}: status {st}: {self.ctx.error()}")

    def reset(self, prompts: list) -> None:
        """One prompt (1..n_ctx ids) per sequence."""
        assert len(prompts) == self.n_seq
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompts]), np.int32)
        offs = np.zeros(self.n_seq + 1, np.int32)
        offs[1:] = np.cumsum([len(p) for p in prompts])
        self._ok(self.lib.gemvq_qwen35_batch_reset(self.h, flat.ctypes.data, offs.ctypes.data), "batch reset")

    def step(self, n: int = 1) -> None:
        self._ok(self.lib.gemvq_qwen35_step(self.h, n), "batch step")

    def set_arith(self, arith: int) -> None:
        """gq.ARITH_REFERENCE: the following steps in the reference's CPU arithmetic (gemvq_qwen35_set_arith)."""
        self._ok(self.lib.gemvq_qwen35_set_arith(self.h, arith), "batch set arith")

    def sync(self) -> None:
        self.ctx.sync()

    def tokens(self, seq: int, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self._ok(self.lib.gemvq_qwen35_batch_tokens(self.h, seq, out.ctypes.data, n), "batch tokens")
        return out

    def logits(self, seq: int) -> np.ndarray:
        out = np.empty(self.cfg.n_vocab, np.float32)
        self._ok(self.lib.gemvq_qwen35_batch_logits(self.h, seq, out.ctypes.data), "batch logits")
        return out

    def commands(self) -> np.ndarray:
        n = self.lib.gemvq_qwen35_commands(self.h, None, 0)
        out = np.empty(n * 8, np.uint32)
        self.lib.gemvq_qwen35_commands(self.h, out.ctypes.data, out.size)
        return out.reshape(n, 8)

    def graph(self) -> int:
        return self.lib.gemvq_qwen35_graph(self.h)
