"""One decode token of the Qwen3.5 hybrid as a ggml graph in the IR of include/gemvq_ggml.h, shaped as llama.cpp's
qwen35 graph is with the reference's graph-order patch (llama.cpp/patches/0006: a layer's input projections right
after its norm) and as the reference's planner expects its DeltaNet chain (ggml-xrt.cpp:1819-2060: conv window from
a recurrent-state GET_ROWS, CONCAT, SSM_CONV, SILU and the CPY of the new window; L2 norms, gates, GATED_DELTA_NET
on state rows and the CPY of the new state; the gated norm MUL(MUL(RMS_NORM(y), w), SILU(z))). Attention is the
flash-attention form: q/k RMS norms, NEOX RoPE, SET_ROWS of k and v into the cache, FLASH_ATTN_EXT, and the
sigmoid gate from the interleaved q projection.

The graph is built once and reused for every token (llama.cpp's graph reuse): a step writes the token id, its
position and the KV row into the input tensors and computes the graph."""
from __future__ import annotations

import ctypes as C

import numpy as np

import ggml_ir as ir
import qwen35


class Qwen35Graph:
    def __init__(self, blob: qwen35.Blob, backend: ir.Backend, seq: int = 0):
        cfg = blob.cfg
        self.cfg, self.backend = cfg, backend
        G = self.G = ir.Graph()
        L = backend.L
        E, S, hv, hk = cfg.n_embd, cfg.ssm_head_dim, cfg.ssm_v_heads, cfg.ssm_k_heads
        ch, hd, nh, nkv = cfg.conv_ch, cfg.head_dim, cfg.n_head, cfg.n_head_kv
        eps = cfg.eps
        base = blob.data.ctypes.data
        self.W = {}
        for d in blob.table:
            name = d.name.decode()
            self.W[name] = G.at(d.type, [d.ne0, d.ne1] if d.ne1 > 1 else [d.ne0], base + d.offset, name, ir.BUF_WEIGHTS)
        W = self.W
        # inputs (one token of one sequence)
        self.tok = G.new(ir.I32, [1], "inp_tokens", ir.FLAG_INPUT)
        self.pos = G.new(ir.I32, [1], "inp_pos", ir.FLAG_INPUT)
        self.kv_idx = G.new(ir.I64, [1], "kv_idxs", ir.FLAG_INPUT)
        self.s_ids = G.new(ir.I32, [1], "inp_s_ids", ir.FLAG_INPUT)
        G.host(self.s_ids, np.int32)[0] = seq
        self.mask = G.new(ir.F32, [cfg.n_ctx, 1], "kq_mask", ir.FLAG_INPUT)
        # recurrent states (conv windows, DeltaNet states) in a state buffer, KV caches in a KV buffer
        gdn_layers = [il for il in range(cfg.n_layer) if not cfg.is_attn(il)]
        att_layers = [il for il in range(cfg.n_layer) if cfg.is_attn(il)]
        r_bytes, s_bytes = 3 * ch * 4, S * S * hv * 4
        r_pad = (r_bytes + 511) // 512 * 512
        self.rs = backend.buffer(len(gdn_layers) * (r_pad + s_bytes), ir.BUF_RS)
        rs_base = L.gqg_buffer_base(self.rs)
        self.r_cache, self.s_cache = {}, {}
        off = 0
        for il in gdn_layers:  # the states first, in layer order (state rows follow the layer order)
            t = G.at(ir.F32, [S * S * hv], rs_base + off, f"cache_s_l{il}")
            self._init(t)
            self.s_cache[il] = t
            off += s_bytes
        for il in gdn_layers:
            t = G.at(ir.F32, [3 * ch], rs_base + off, f"cache_r_l{il}")
            self._init(t)
            self.r_cache[il] = t
            off += r_pad
        kv_row = hd * nkv * 2
        self.kvb = backend.buffer(len(att_layers) * 2 * kv_row * cfg.n_ctx, ir.BUF_KV)
        kv_base = L.gqg_buffer_base(self.kvb)
        self.k_cache, self.v_cache = {}, {}
        off = 0
        for il in att_layers:
            for which, dst in (("k", self.k_cache), ("v", self.v_cache)):
                t = G.at(ir.F16, [hd * nkv, cfg.n_ctx], kv_base + off, f"cache_{which}_l{il}")
                self._init(t)
                dst[il] = t
                off += kv_row * cfg.n_ctx

        inp = G.get_rows(W["token_embd.weight"], self.tok, "inp_embd")
        for il in range(cfg.n_layer):
            p = f"blk.{il}."
            cur = G.mul(G.rms_norm(inp, eps, f"norm-{il}"), W[p + "attn_norm.weight"], f"attn_norm-{il}")
            if cfg.is_attn(il):
                qf = G.mul_mat(W[p + "attn_q.weight"], cur, f"Qcur_full-{il}")
                kc = G.mul_mat(W[p + "attn_k.weight"], cur, f"Kcur-{il}")
                vc = G.mul_mat(W[p + "attn_v.weight"], cur, f"Vcur-{il}")
                for t in (qf, kc, vc):
                    G.expand(t)
                q = G.view(qf, [hd, nh, 1], nb1=2 * hd * 4, nb2=2 * hd * nh * 4, offs=0, name=f"Qcur-{il}")
                gate = G.view(qf, [hd, nh, 1], nb1=2 * hd * 4, nb2=2 * hd * nh * 4, offs=hd * 4, name=f"gate-{il}")
                q = G.mul(G.rms_norm(q, eps), W[p + "attn_q_norm.weight"], f"Qcur_normed-{il}")
                k = G.mul(G.rms_norm(G.reshape(kc, [hd, nkv, 1]), eps), W[p + "attn_k_norm.weight"], f"Kcur_normed-{il}")
                v = G.reshape(vc, [hd, nkv, 1])
                q = G.rope(q, self.pos, cfg.n_rot, ir.ROPE_NEOX, cfg.rope_base, f"Qcur_rope-{il}")
                k = G.rope(k, self.pos, cfg.n_rot, ir.ROPE_NEOX, cfg.rope_base, f"Kcur_rope-{il}")
                G.expand(G.set_rows(self.k_cache[il], G.reshape(k, [hd * nkv, 1]), self.kv_idx, f"k_store-{il}"))
                G.expand(G.set_rows(self.v_cache[il], G.reshape(v, [hd * nkv, 1]), self.kv_idx, f"v_store-{il}"))
                kv = G.view(self.k_cache[il], [hd, cfg.n_ctx, nkv], nb1=kv_row, nb2=hd * 2, name=f"k-{il}")
                vv = G.view(self.v_cache[il], [hd, cfg.n_ctx, nkv], nb1=kv_row, nb2=hd * 2, name=f"v-{il}")
                scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
                fa = G.flash_attn_ext(G.permute(q, (0, 2, 1, 3)), kv, vv, self.mask, scale, f"fattn-{il}")
                att = G.mul(G.reshape(fa, [hd * nh]), G.unary(G.cont(gate), ir.UNARY_SIGMOID), f"attn_gated-{il}")
                cur = G.mul_mat(W[p + "attn_output.weight"], att, f"attn_out-{il}")
            else:
                qkv = G.mul_mat(W[p + "attn_qkv.weight"], cur, f"qkv_mixed-{il}")
                z = G.mul_mat(W[p + "attn_gate.weight"], cur, f"z-{il}")
                beta = G.mul_mat(W[p + "ssm_beta.weight"], cur, f"beta-{il}")
                alpha = G.mul_mat(W[p + "ssm_alpha.weight"], cur, f"alpha-{il}")
                for t in (qkv, z, beta, alpha):
                    G.expand(t)
                beta = G.unary(G.reshape(beta, [1, hv]), ir.UNARY_SIGMOID, f"beta_sigmoid-{il}")
                gdec = G.mul(G.unary(G.add(G.reshape(alpha, [hv]), W[p + "ssm_dt.bias"]), ir.UNARY_SOFTPLUS),
                             W[p + "ssm_a"], f"gate-{il}")
                rows = G.get_rows(G.reshape(self.r_cache[il], [3 * ch, 1]), self.s_ids, f"conv_states-{il}")
                cx = G.concat(G.reshape(rows, [3, ch]), G.transpose(G.reshape(qkv, [ch, 1])), 0, f"conv_input-{il}")
                G.expand(G.cpy(G.view(cx, [3, ch], nb1=4 * 4, offs=4), self.r_cache[il], f"conv_state_store-{il}"))
                conv = G.unary(G.ssm_conv(cx, W[p + "ssm_conv1d.weight"], f"conv-{il}"), ir.UNARY_SILU, f"conv_silu-{il}")
                q = G.l2_norm(G.view(conv, [S, hk], offs=0), eps, f"q_l2-{il}")
                k = G.l2_norm(G.view(conv, [S, hk], offs=hk * S * 4), eps, f"k_l2-{il}")
                v = G.view(conv, [S, hv], offs=2 * hk * S * 4, name=f"v_conv-{il}")
                st = G.reshape(G.get_rows(G.reshape(self.s_cache[il], [S * S * hv, 1]), self.s_ids, f"ssm_states-{il}"),
                               [S, S, hv])
                out = G.gated_delta_net(q, k, v, gdec, beta, st, f"gdn-{il}")
                G.expand(G.cpy(G.view(out, [S * S * hv], offs=hv * S * 4), self.s_cache[il], f"ssm_state_store-{il}"))
                y = G.view(out, [S, hv], offs=0, name=f"gdn_y-{il}")
                gated = G.mul(G.mul(G.rms_norm(y, eps), W[p + "ssm_norm.weight"]), G.unary(z, ir.UNARY_SILU),
                              f"gated_norm-{il}")
                cur = G.mul_mat(W[p + "ssm_out.weight"], G.reshape(gated, [hv * S]), f"ssm_out-{il}")
            h = G.add(cur, inp, f"attn_residual-{il}")
            cur = G.mul(G.rms_norm(h, eps), W[p + "post_attention_norm.weight"], f"ffn_norm-{il}")
            ffn = G.swiglu(G.mul_mat(W[p + "ffn_gate.weight"], cur, f"ffn_gate-{il}"),
                           G.mul_mat(W[p + "ffn_up.weight"], cur, f"ffn_up-{il}"), f"ffn_swiglu-{il}")
            inp = G.add(G.mul_mat(W[p + "ffn_down.weight"], ffn, f"ffn_down-{il}"), h, f"l_out-{il}")
            G.expand(inp)
        self.hidden_t = inp
        norm = G.mul(G.rms_norm(inp, eps), W["output_norm.weight"], "result_norm")
        self.logits_t = G.mul_mat(W["output.weight"], norm, "result_output")
        self.logits_t.flags |= ir.FLAG_OUTPUT
        G.expand(self.logits_t)
        self.cgraph = G.cgraph()

    def layer_splits(self) -> list[ir.CGraph]:
        """The token's nodes as one split per layer (the embedding rows with layer 0, the output norm and head after
        the last layer), the way ggml's scheduler cuts a graph into splits: a tensor that a later split reads is
        flagged GGML_TENSOR_FLAG_SPLIT_OUTPUT (the reference's scheduler patch 0002), so its split copies it back to
        the host and the later split copies it in. Returns the splits' graphs, in order."""
        nodes, cfg = self.G.nodes, self.cfg
        names = [t.name.decode() for t in nodes]
        starts = [0] + [names.index(f"norm-{il}") for il in range(1, cfg.n_layer)]
        starts.append(names.index(f"l_out-{cfg.n_layer - 1}") + 1)
        bounds = list(zip(starts, starts[1:] + [len(nodes)]))
        split_of = {}
        for k, (a, b) in enumerate(bounds):
            for t in nodes[a:b]:
                split_of[C.addressof(t)] = k
        root = lambda t: t.view_src.contents if t.view_src else t
        for k, (a, b) in enumerate(bounds):
            for t in nodes[a:b]:
                for i in range(10):
                    if not t.src[i]:
                        continue
                    r = root(t.src[i].contents)
                    kr = split_of.get(C.addressof(r))
                    if kr is not None and kr < k:
                        r.flags |= ir.FLAG_SPLIT_OUTPUT
        self.splits = [self.G.cgraph(nodes[a:b]) for a, b in bounds]
        return self.splits

    def step_splits(self, tok: int, pos: int) -> np.ndarray:
        """One token through the backend split by split (layer_splits); returns the logits."""
        self.set_token(tok, pos)
        for k, g in enumerate(self.splits):
            st = self.backend.compute(g)
            if st != 0:
                raise RuntimeError(f"graph_compute of split {k}: {st}: {self.backend.error()}")
        return self.G.host(self.logits_t).copy()

    def _init(self, t: ir.Tensor) -> None:
        buf = self.rs if t.name.startswith(b"cache_s") or t.name.startswith(b"cache_r") else self.kvb
        if self.backend.L.gqg_buffer_init_tensor(buf, C.byref(t)) != 0:
            raise RuntimeError(f"init_tensor {t.name}: {self.backend.error()}")

    def set_token(self, tok: int, pos: int) -> None:
        self.G.host(self.tok, np.int32)[0] = tok
        self.G.host(self.pos, np.int32)[0] = pos
        self.G.host(self.kv_idx, np.int64)[0] = pos
        m = self.G.host(self.mask)
        m[:] = -np.inf
        m[:pos + 1] = 0.0

    def step(self, tok: int, pos: int) -> np.ndarray:
        """One token through the backend; returns the logits."""
        self.set_token(tok, pos)
        st = self.backend.compute(self.cgraph)
        if st != 0:
            raise RuntimeError(f"graph_compute: {st}: {self.backend.error()}")
        return self.G.host(self.logits_t).copy()

    def words(self) -> np.ndarray:
        return self.backend.plan(self.cgraph)

    def close(self) -> None:
        for b in (getattr(self, "rs", None), getattr(self, "kvb", None)):
            if b:
                self.backend.free_buffer(b)
        self.rs = self.kvb = None
