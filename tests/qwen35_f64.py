"""Independent float64 restatement of the synthetic Qwen3.5-shaped hybrid decoder, for pinning the oracle decoder.

Written from the model's definition (llama.cpp's qwen35 graph as the reference offloads it,
llama.cpp/patches/0006-qwen35-graph-order.patch, with the op semantics of fpga/src/gemvq_ref.h and the gate and norm
compositions of ggml-xrt.cpp:1944-1992), not from the oracle's C code: weights are dequantized to float64 by the
numpy block decoders of ggml_blocks.py and every operation runs in float64 with numpy's exp and log. What the model
itself rounds is kept: each quantized matrix product quantizes its activation, taken as FP32, with ggml's FP32
quantizer (Q8_0 for Q4_0 / Q4_1 / Q8_0 weights, Q8_K for the K-quant head; ggml_blocks.quantize_q8_0 / _q8_K, whose
FP32 steps decide exact ties such as an element at half its block's maximum, which quantized embeddings produce),
and attention reads an F16 KV cache with an fp16 query (the F16 vec_dot type). The oracle's canonical arithmetic (fixed-point block terms, FP32 pairwise trees, its own exp/log)
then differs from this only by FP32 rounding, plus the Q8 quantization decisions those roundings flip.

Per layer (DeltaNet layers i with (i + 1) % attn_interval != 0, attention layers otherwise):
  x = rmsnorm(h) * attn_norm
  DeltaNet:  qkv = W_qkv x; z = W_gate x; b = W_beta x; a = W_alpha x
             c = silu(causal depthwise conv1d over [state (3), qkv] with kernel [ch][4]); state shifts by one
             q, k = L2-normalized key heads of c (q: c[0 : hk*S], k: c[hk*S : 2 hk*S]), v = c[2 hk*S :]
             beta = sigmoid(b); g = softplus(a + dt) * A; for value head h (key head h % hk), row j of its state:
               s_j = s_j * exp(g_h); delta = (v_j - s_j . k) * beta_h; s_j += k * delta; y_j = (s_j . q) / sqrt(S)
             y = silu(z) * (rmsnorm_per_head(y) * ssm_norm); h = h + W_ssm_out y
  attention: [q | gate] per head interleaved = W_q x; k = W_k x; v = W_v x
             q, k = rmsnorm per head * q_norm / k_norm, NEOX RoPE on the first n_rot dims; K, V appended as fp16
             o_h = softmax(fp16(q_h) . K_kv / sqrt(hd)) V_kv (kv head h // (n_head / n_head_kv))
             h = h + W_o (sigmoid(gate) * o)
  FFN:       x = rmsnorm(h) * post_norm; h = h + W_down (silu(W_gate x) * W_up x)
logits = W_out (rmsnorm(h) * output_norm).
"""
from __future__ import annotations

import numpy as np

import ggml_blocks as gb

F32 = 0


def _f16(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def q8_0_values(x: np.ndarray) -> np.ndarray:
    """The activation a Q8_0 matrix product sees: ggml's FP32 Q8_0 quantization of x, dequantized exactly."""
    q, d = gb.quantize_q8_0(np.asarray(x, np.float64).astype(np.float32))
    return q.astype(np.float64) * gb.half(d).repeat(32)


def q8_K_values(x: np.ndarray) -> np.ndarray:
    """The activation a K-quant matrix product sees: ggml's FP32 Q8_K quantization of x, dequantized exactly."""
    q, d, _ = gb.quantize_q8_K(np.asarray(x, np.float64).astype(np.float32))
    return q.astype(np.float64) * d.astype(np.float64).repeat(256)


def rmsnorm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    y = x / np.sqrt(np.mean(x * x) + eps)
    return y * w if w is not None else y


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


class F64Decoder:
    def __init__(self, blob, quantize_activations: bool = True):
        cfg = blob.cfg
        self.cfg = cfg
        self.qa = quantize_activations
        self.w: dict[str, np.ndarray] = {}
        self.types: dict[str, int] = {}
        for d in blob.table:
            name = d.name.decode()
            raw = blob.data[d.offset:d.offset + d.nbytes]
            self.types[name] = d.type
            if d.type == F32:
                self.w[name] = raw.view(np.float32).astype(np.float64)
            elif name == "token_embd.weight":
                self.emb = (raw, d.type, d.ne1, d.ne0)
            elif d.type == gb.Q4_1:  # value = d q + m: the q part and the per-block m kept apart (see mm)
                q, dd, mm = gb.q4_1(raw, d.ne1, d.ne0)
                self.w[name] = (q.reshape(d.ne1, -1, 32) * dd[..., None]).reshape(d.ne1, d.ne0)
                self.w[name + ":m"] = mm
            else:
                self.w[name] = gb.dequantize(d.type, raw, d.ne1, d.ne0).reshape(d.ne1, d.ne0)
        S, hk, hv = cfg.ssm_head_dim, cfg.ssm_k_heads, cfg.ssm_v_heads
        self.conv = {il: np.zeros((cfg.conv_ch, 3)) for il in range(cfg.n_layer) if not cfg.is_attn(il)}
        self.ssm = {il: np.zeros((hv, S, S)) for il in range(cfg.n_layer) if not cfg.is_attn(il)}
        self.kc = {il: np.zeros((cfg.n_ctx, cfg.n_head_kv, cfg.head_dim)) for il in range(cfg.n_layer) if cfg.is_attn(il)}
        self.vc = {il: np.zeros((cfg.n_ctx, cfg.n_head_kv, cfg.head_dim)) for il in range(cfg.n_layer) if cfg.is_attn(il)}
        self.h = None

    def mm(self, name: str, x: np.ndarray) -> np.ndarray:
        t = self.types[name]
        if t == gb.Q4_1:
            # ggml's Q4_1 x Q8_1: d_w d_x sum(q_w q_x) + m_w s_x per block, s_x = fp16(sum(q_x) * d_x) (FP32 d_x)
            q, dbits, sbits = gb.quantize_q8_1(np.asarray(x, np.float64).astype(np.float32))
            xv = q.astype(np.float64) * gb.half(dbits).repeat(32)
            return self.w[name] @ xv + self.w[name + ":m"] @ gb.half(sbits)
        if self.qa:
            x = q8_K_values(x) if t in (gb.Q5_K, gb.Q6_K) else q8_0_values(x)
        return self.w[name] @ x

    def embed(self, tok: int) -> np.ndarray:
        raw, t, rows, cols = self.emb
        rb = len(raw) // rows
        return gb.dequantize(t, raw[tok * rb:(tok + 1) * rb], 1, cols).ravel()

    def rope(self, x: np.ndarray, pos: int) -> np.ndarray:
        """NEOX rotation of pairs (i, i + n_rot / 2), theta_i = pos * base^(-2 i / n_rot)."""
        c = self.cfg
        half = c.n_rot // 2
        th = pos * c.rope_base ** (-2.0 * np.arange(half) / c.n_rot)
        cs, sn = np.cos(th), np.sin(th)
        y = x.copy()
        x0, x1 = x[..., :half], x[..., half:c.n_rot]
        y[..., :half] = x0 * cs - x1 * sn
        y[..., half:c.n_rot] = x0 * sn + x1 * cs
        return y

    def layer(self, il: int, h: np.ndarray, pos: int) -> np.ndarray:
        """The residual stream after layer il given the stream h before it (the layer's states advance)."""
        c = self.cfg
        S, hk, hv, hd = c.ssm_head_dim, c.ssm_k_heads, c.ssm_v_heads, c.head_dim
        p = f"blk.{il}."
        h = np.asarray(h, np.float64)
        x = rmsnorm(h, self.w[p + "attn_norm.weight"], c.eps)
        if c.is_attn(il):
            qg = self.mm(p + "attn_q.weight", x).reshape(c.n_head, 2, hd)
            k = self.mm(p + "attn_k.weight", x).reshape(c.n_head_kv, hd)
            v = self.mm(p + "attn_v.weight", x).reshape(c.n_head_kv, hd)
            q = np.stack([rmsnorm(qg[i, 0], self.w[p + "attn_q_norm.weight"], c.eps) for i in range(c.n_head)])
            k = np.stack([rmsnorm(k[i], self.w[p + "attn_k_norm.weight"], c.eps) for i in range(c.n_head_kv)])
            q, k = self.rope(q, pos), self.rope(k, pos)
            self.kc[il][pos] = _f16(k)
            self.vc[il][pos] = _f16(v)
            grp = c.n_head // c.n_head_kv
            o = np.empty((c.n_head, hd))
            for i in range(c.n_head):
                K, V = self.kc[il][:pos + 1, i // grp], self.vc[il][:pos + 1, i // grp]
                sc = (K @ _f16(q[i])) / np.sqrt(hd)
                e = np.exp(sc - sc.max())
                o[i] = (e / e.sum()) @ V
            o = sigmoid(qg[:, 1]) * o
            h = h + self.mm(p + "attn_output.weight", o.ravel())
        else:
            qkv = self.mm(p + "attn_qkv.weight", x)
            z = self.mm(p + "attn_gate.weight", x)
            b = self.mm(p + "ssm_beta.weight", x)
            a = self.mm(p + "ssm_alpha.weight", x)
            kw = self.w[p + "ssm_conv1d.weight"].reshape(c.conv_ch, 4)
            win = np.concatenate([self.conv[il], qkv[:, None]], axis=1)
            cy = silu((win * kw).sum(axis=1))
            self.conv[il] = win[:, 1:]
            qh = cy[:hk * S].reshape(hk, S)
            kh = cy[hk * S:2 * hk * S].reshape(hk, S)
            vh = cy[2 * hk * S:].reshape(hv, S)
            qh = qh / np.maximum(np.linalg.norm(qh, axis=1, keepdims=True), c.eps)
            kh = kh / np.maximum(np.linalg.norm(kh, axis=1, keepdims=True), c.eps)
            beta = sigmoid(b)
            g = softplus(a + self.w[p + "ssm_dt.bias"]) * self.w[p + "ssm_a"]
            st = self.ssm[il]
            y = np.empty((hv, S))
            for i in range(hv):
                qq, kk = qh[i % hk], kh[i % hk]
                st[i] *= np.exp(g[i])
                delta = (vh[i] - st[i] @ kk) * beta[i]
                st[i] += delta[:, None] * kk[None, :]
                y[i] = (st[i] @ qq) / np.sqrt(S)
            zs = silu(z).reshape(hv, S)
            yn = np.stack([rmsnorm(y[i], self.w[p + "ssm_norm.weight"], c.eps) for i in range(hv)]) * zs
            h = h + self.mm(p + "ssm_out.weight", yn.ravel())
        x = rmsnorm(h, self.w[p + "post_attention_norm.weight"], c.eps)
        f = silu(self.mm(p + "ffn_gate.weight", x)) * self.mm(p + "ffn_up.weight", x)
        return h + self.mm(p + "ffn_down.weight", f)

    def head(self, h: np.ndarray) -> np.ndarray:
        return self.mm("output.weight", rmsnorm(np.asarray(h, np.float64), self.w["output_norm.weight"], self.cfg.eps))

    def decode(self, tok: int, pos: int) -> np.ndarray:
        """One token through the whole model on this decoder's own residual stream; returns the logits."""
        h = self.embed(tok)
        for il in range(self.cfg.n_layer):
            h = self.layer(il, h, pos)
        self.h = h
        return self.head(h)
