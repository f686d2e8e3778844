// Per-token command list of a Qwen3.5-shaped hybrid decoder, captured once as a hipGraph (include/gemvq_qwen35.h).
//
// Layer order follows llama.cpp's qwen35 graph as the reference offloads it (llama.cpp/patches/0006: all input
// projections of a layer right after its norm) in the fused forms of the reference kernel (fpga/src/gemvqc16.h):
//   DeltaNet layer: deferred RMSNORM -> GEMV group {qkv + CONV epilog, z + SiLU epilog, beta, alpha} -> GDN (L2
//                   q/k, gates, gated output norm on silu(z)) -> ssm_out GEMV + residual ADD epilog (the runtime
//                   applies the gated norm in that GEMV's activation prologue; GDN_WITH_OUT, the step and ssm_out in
//                   one launch, is not asked for: in graph replays it is slower than the two launches)
//   attention layer: deferred RMSNORM -> GEMV group {q+gate, k, v} -> ATTN (q/k norm, RoPE, KV append, softmax,
//                   sigmoid gate) -> attn_output GEMV + ADD
//   both: deferred RMSNORM -> {ffn_gate, ffn_up} SwiGLU pair -> ffn_down GEMV + ADD
// then the output norm, the head GEMV with the ARGMAX epilog and NEXT_TOKEN.
#include "gemvq_qwen35.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {

constexpr int F32 = 0, T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q5_K = 13, T_Q6_K = 14;  // ggml type ids

uint32_t fb(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

size_t up16(size_t n) { return (n + 15) / 16 * 16; }

struct T {
    const gemvq_tensor_desc * d = nullptr;
    uint64_t w_off = 0;     // quantized: weight arena offset
    uint32_t act_off = 0;   // F32: activation buffer offset
};

}  // namespace

struct gemvq_qwen35 {
    gemvq_ctx * ctx = nullptr;
    gemvq_qw_config c{};
    std::vector<gemvq_tensor_desc> descs;  // copy of the caller's table
    std::map<std::string, T> t;
    std::vector<uint32_t> cmds;
    int graph = -1;
    int chunk_graph = -1;  // the prefill's full-chunk command list (positions and ids come from the act slots)
    std::vector<int> kv;  // per layer (attention layers only)
    // activation layout
    uint32_t tok = 16, pos = 32, key = 48;
    uint32_t h = 0, xn = 0, qkv = 0, cqkv = 0, z = 0, ba = 0, y = 0, tmp = 0, qg = 0, kk = 0, vv = 0, att = 0, ffn = 0,
             logits = 0, rope = 0, prompt = 0, out = 0;
    std::vector<uint32_t> conv_state;  // per layer
    size_t act_floats = 0;
    // batched prefill: rows of up to GEMVQ_GEMM_MAX_TOK prompt tokens (token ids and positions one per 16 floats)
    bool can_batch = false;
    std::string batch_why;
    uint32_t bh = 0, bqkv = 0, bcqkv = 0, bz = 0, bbeta = 0, balpha = 0, by = 0, bqg = 0, bk = 0, bv = 0, batt = 0,
             bffn = 0, bid = 0, bpos = 0;
    std::vector<int32_t> prompt_ids;
    // lockstep decode of n_seq sequences (gemvq_qwen35_batch_create): per sequence, 16 floats apart, its key
    // (skey), position (spos) and prompt length (slen); its prompt, token ids and logits in regions of n_ctx
    // (n_vocab) floats; its conv windows, DeltaNet state rows and KV region follow those of the sequence before
    int n_seq = 1;
    uint32_t skey = 0, spos = 0, slen = 0, sprompt = 0, sout = 0, slogits = 0;
};

namespace {

const gemvq_tensor_desc * find(const gemvq_tensor_desc * tab, int n, const std::string & name) {
    for (int i = 0; i < n; ++i)
        if (name == tab[i].name) return &tab[i];
    return nullptr;
}

bool is_attn(const gemvq_qw_config & c, int il) { return (il + 1) % c.attn_interval == 0; }

int conv_ch(const gemvq_qw_config & c) { return 2 * c.ssm_k_heads * c.ssm_head_dim + c.ssm_v_heads * c.ssm_head_dim; }

// Layout of the activation buffer; returns the number of floats.
size_t layout(gemvq_qwen35 & m, const gemvq_tensor_desc * tab, int n) {
    const gemvq_qw_config & c = m.c;
    size_t off = 64;
    auto take = [&](size_t floats) {
        const size_t o = off;
        off += up16(floats);
        return uint32_t(o);
    };
    for (int i = 0; i < n; ++i) {
        if (tab[i].type != F32) continue;
        T & x = m.t[tab[i].name];
        x.d = &tab[i];
        x.act_off = take(size_t(tab[i].ne0) * size_t(tab[i].ne1 > 0 ? tab[i].ne1 : 1));
    }
    const int ch = conv_ch(c), S = c.ssm_head_dim, hv = c.ssm_v_heads;
    const size_t ns = size_t(m.n_seq);
    m.conv_state.assign(c.n_layer, 0);
    for (int il = 0; il < c.n_layer; ++il)
        if (!is_attn(c, il)) m.conv_state[il] = take(size_t(ch) * 3 * ns);
    m.rope = take(size_t(c.n_ctx) * c.n_rot);
    m.prompt = take(size_t(c.n_ctx));
    m.out = take(size_t(c.n_ctx) + 16);
    m.h = take(c.n_embd);
    m.xn = take(std::max(c.n_embd, c.n_ff));
    m.qkv = take(ch);
    m.cqkv = take(ch);
    m.z = take(size_t(hv) * S);
    m.ba = take(2 * up16(hv));
    m.y = take(size_t(hv) * S);
    m.tmp = take(c.n_embd);
    m.qg = take(size_t(2) * c.n_head * c.head_dim);
    m.kk = take(size_t(c.n_head_kv) * c.head_dim);
    m.vv = take(size_t(c.n_head_kv) * c.head_dim);
    m.att = take(size_t(c.n_head) * c.head_dim);
    m.ffn = take(c.n_ff);
    m.logits = take(c.n_vocab);
    const size_t B = GEMVQ_GEMM_MAX_TOK;
    m.bh = take(B * c.n_embd);
    m.bqkv = take(B * ch);
    m.bcqkv = take(B * ch);
    m.bz = take(B * hv * S);
    m.bbeta = take(B * up16(hv));
    m.balpha = take(B * up16(hv));
    m.by = take(B * hv * S);
    m.bqg = take(B * 2 * c.n_head * c.head_dim);
    m.bk = take(B * c.n_head_kv * c.head_dim);
    m.bv = take(B * c.n_head_kv * c.head_dim);
    m.batt = take(B * c.n_head * c.head_dim);
    m.bffn = take(B * c.n_ff);
    m.bid = take(B * 16);
    m.bpos = take(16);
    if (m.n_seq > 1) {
        m.skey = take(ns * 16);
        m.spos = take(ns * 16);
        m.slen = take(ns * 16);
        m.sprompt = take(ns * size_t(c.n_ctx));
        m.sout = take(ns * size_t(c.n_ctx));
        m.slogits = take(ns * size_t(c.n_vocab));
    }
    return off;
}

struct Emit {
    std::vector<uint32_t> & w;
    void cmd(std::initializer_list<uint32_t> words) {
        size_t k = 0;
        for (uint32_t v : words) {
            w.push_back(v);
            ++k;
        }
        for (; k < GEMVQ_CMD_WORDS; ++k) w.push_back(0);
    }
    void gemv(const T & t, uint32_t x, uint32_t y, uint32_t flags = 0) {
        cmd({GEMVQ_OP_GEMV, uint32_t(t.d->type) | flags, uint32_t(t.d->ne1), uint32_t(t.d->ne0), uint32_t(t.w_off),
             uint32_t(t.w_off >> 32), x, y});
    }
    // batched GEMV over ntok rows; norm: the per-token RMS norm folded into its quantization
    void gemm(const T & t, uint32_t x, uint32_t xs, uint32_t y, uint32_t ys, uint32_t ntok, uint32_t flags = 0,
              uint32_t res = 0, uint32_t rs = 0, const T * norm = nullptr, float eps = 0.0f) {
        cmd({GEMVQ_OP_GEMM, uint32_t(t.d->type) | flags, uint32_t(t.d->ne1), uint32_t(t.d->ne0), uint32_t(t.w_off),
             uint32_t(t.w_off >> 32), x, y});
        cmd({ntok, xs, ys, res, rs, norm ? norm->act_off : 0u, fb(eps), norm ? GEMVQ_NORM_DEFER : 0u});
    }
};

// The projections a batched prefill runs as GEMM commands: Q4_0 / Q4_1 / Q8_0 with columns a multiple of 512.
bool batchable(const gemvq_qwen35 & m, std::string & why) {
    const gemvq_qw_config & c = m.c;
    if (c.n_embd % 512 || c.n_ff % 512 || (c.ssm_v_heads * c.ssm_head_dim) % 512 || (c.n_head * c.head_dim) % 512) {
        why = "widths are not multiples of 512";
        return false;
    }
    for (const auto & kv : m.t) {
        const std::string & n = kv.first;
        if (n.rfind("blk.", 0) != 0 || !kv.second.d || kv.second.d->type == F32) continue;
        if (n.find("ssm_conv1d") != std::string::npos) continue;
        const int t = kv.second.d->type;
        if ((t != T_Q4_0 && t != T_Q4_1 && t != T_Q8_0) || kv.second.d->ne0 % 512) {
            why = "tensor " + n + " has no batched GEMV (Q4_0 / Q4_1 / Q8_0, columns a multiple of 512)";
            return false;
        }
    }
    return true;
}

// Prompt positions p0 .. p0 + ntok - 1 through every layer (no head): the projections as GEMM commands over the
// token rows, the conv and the DeltaNet step over the tokens in order, attention token by token (each token's
// keys and values are in the cache before the next token reads them). The results equal ntok decode steps bit for
// bit, except that no logits are computed.
bool build_chunk(const gemvq_qwen35 & m, uint32_t ntok, std::vector<uint32_t> & w) {
    const gemvq_qw_config & c = m.c;
    Emit e{w};
    auto W = [&](const std::string & name) { return &m.t.at(name); };
    const float eps = c.eps;
    const uint32_t E = uint32_t(c.n_embd), S = uint32_t(c.ssm_head_dim), hv = uint32_t(c.ssm_v_heads),
                   hk = uint32_t(c.ssm_k_heads), ch = uint32_t(conv_ch(c)), F = uint32_t(c.n_ff);
    const uint32_t hd = uint32_t(c.head_dim), qrow = 2 * uint32_t(c.n_head) * hd, kvrow = uint32_t(c.n_head_kv) * hd,
                   arow = uint32_t(c.n_head) * hd, hvs = hv * S, gb = uint32_t(up16(hv));
    const T * emb = W("token_embd.weight");
    e.cmd({GEMVQ_OP_GET_ROWS, uint32_t(emb->d->type) | (ntok << 16), uint32_t(emb->d->ne1), uint32_t(emb->d->ne0),
           uint32_t(emb->w_off), uint32_t(emb->w_off >> 32), m.bid, m.bh});  // the chunk's ids, 16 floats apart
    int slot = 0;
    for (int il = 0; il < c.n_layer; ++il) {
        const std::string p = "blk." + std::to_string(il) + ".";
        const T * an = W(p + "attn_norm.weight");
        const T * pn = W(p + "post_attention_norm.weight");
        if (is_attn(c, il)) {
            e.gemm(*W(p + "attn_q.weight"), m.bh, E, m.bqg, qrow, ntok, 0, 0, 0, an, eps);
            e.gemm(*W(p + "attn_k.weight"), m.bh, E, m.bk, kvrow, ntok, 0, 0, 0, an, eps);
            e.gemm(*W(p + "attn_v.weight"), m.bh, E, m.bv, kvrow, ntok, 0, 0, 0, an, eps);
            // the chunk's tokens at positions act[bpos] + i, packed rows (q + gate, k, v, output)
            e.cmd({GEMVQ_OP_ATTN, uint32_t(c.n_head) | (uint32_t(c.n_head_kv) << 16), m.bqg, uint32_t(m.kv[il]), m.batt,
                   hd | (uint32_t(c.n_rot) << 16), m.bpos, 1u | (ntok << 16)});
            e.cmd({m.bk, m.bv, fb(1.0f / std::sqrt(float(c.head_dim))), fb(eps), W(p + "attn_q_norm.weight")->act_off,
                   W(p + "attn_k_norm.weight")->act_off, m.rope, m.bqg + hd});
            e.gemm(*W(p + "attn_output.weight"), m.batt, arow, m.bh, E, ntok, GEMVQ_GEMV_ADD, m.bh, E);
        } else {
            // the four projections of the normed rows back to back (one quantization), then the conv
            e.gemm(*W(p + "attn_qkv.weight"), m.bh, E, m.bqkv, ch, ntok, 0, 0, 0, an, eps);
            e.gemm(*W(p + "attn_gate.weight"), m.bh, E, m.bz, hvs, ntok, GEMVQ_GEMV_SILU, 0, 0, an, eps);
            e.gemm(*W(p + "ssm_beta.weight"), m.bh, E, m.bbeta, gb, ntok, 0, 0, 0, an, eps);
            e.gemm(*W(p + "ssm_alpha.weight"), m.bh, E, m.balpha, gb, ntok, 0, 0, 0, an, eps);
            e.cmd({GEMVQ_OP_CONV, ch, m.bqkv, W(p + "ssm_conv1d.weight")->act_off, m.bcqkv, m.conv_state[il],
                   m.conv_state[il], 1u | (ntok << 16)});
            const uint32_t row = uint32_t(slot) * hv * 128u;
            const uint32_t flags = GEMVQ_GDN_L2_QK | GEMVQ_GDN_GATED | GEMVQ_GDN_GATES | GEMVQ_GDN_Z_SILU;
            e.cmd({GEMVQ_OP_GDN, hv | (hk << 16), m.bcqkv, m.bcqkv + hk * S, m.bcqkv + 2 * hk * S, m.balpha, m.bbeta, m.by});
            e.cmd({row, row, fb(1.0f / std::sqrt(float(S))), flags, fb(eps), fb(eps), W(p + "ssm_norm.weight")->act_off,
                   m.bz});
            e.cmd({W(p + "ssm_dt.bias")->act_off, W(p + "ssm_a")->act_off, ntok, ch, gb});
            e.gemm(*W(p + "ssm_out.weight"), m.by, hvs, m.bh, E, ntok, GEMVQ_GEMV_ADD, m.bh, E);
            ++slot;
        }
        e.gemm(*W(p + "ffn_gate.weight"), m.bh, E, m.bffn, F, ntok, GEMVQ_GEMV_SWIGLU, 0, 0, pn, eps);
        e.gemm(*W(p + "ffn_up.weight"), m.bh, E, m.bffn, F, ntok, 0, 0, 0, pn, eps);
        e.gemm(*W(p + "ffn_down.weight"), m.bffn, F, m.bh, E, ntok, GEMVQ_GEMV_ADD, m.bh, E);
    }
    return true;
}

// One lockstep step of n_seq sequences, token t of sequence t: the chunk's GEMM projections over the n_seq token
// rows; CONV, the DeltaNet step and attention in their sequences forms (each token on its own sequence's conv
// window, state rows, KV region and position); the output norm and head per sequence; the argmax of every
// sequence's logits and NEXT_TOKEN over all of them (the prompt token while one is left, else the argmax). Each
// sequence's ids, logits, states and cache are those of a single-sequence decode of its prompt, bit for bit.
bool build_batch(gemvq_qwen35 & m, std::string & err) {
    const gemvq_qw_config & c = m.c;
    const uint32_t B = uint32_t(m.n_seq);
    std::vector<uint32_t> & w = m.cmds;
    if (!build_chunk(m, B, w)) return false;
    // the chunk list is one sequence's tokens in order; turn its CONV, GDN and ATTN into their sequences forms
    const uint32_t hv = uint32_t(c.ssm_v_heads);
    int slot = 0;
    for (size_t i = 0; i < w.size(); i += GEMVQ_CMD_WORDS) {
        uint32_t * k = &w[i];
        if (k[0] == GEMVQ_OP_CONV) {
            k[7] |= GEMVQ_CONV_SEQS;
        } else if (k[0] == GEMVQ_OP_GDN) {
            uint32_t * k2 = k + GEMVQ_CMD_WORDS;
            const uint32_t row = uint32_t(slot++) * B * hv * 128u;  // the layer's rows of all sequences
            k2[0] = k2[1] = row;
            k2[3] |= GEMVQ_GDN_SEQS;
            i += 2 * GEMVQ_CMD_WORDS;
        } else if (k[0] == GEMVQ_OP_ATTN) {
            k[6] = m.spos;
            k[7] |= GEMVQ_ATTN_SEQS;
            i += GEMVQ_CMD_WORDS;
        } else if (k[0] == GEMVQ_OP_GEMM) {
            i += GEMVQ_CMD_WORDS;
        }
    }
    Emit e{w};
    const T & onorm = m.t.at("output_norm.weight");
    const T & head = m.t.at("output.weight");
    const uint32_t E = uint32_t(c.n_embd), V = uint32_t(c.n_vocab);
    const int ht = head.d->type;
    if ((ht == T_Q4_0 || ht == T_Q4_1 || ht == T_Q8_0 || ((ht == T_Q5_K || ht == T_Q6_K) && head.d->ne0 <= 12288)) &&
        head.d->ne0 % 512 == 0) {
        e.gemm(head, m.bh, E, m.slogits, V, B, 0, 0, 0, &onorm, c.eps);
    } else {  // no batched form of the head's type: each sequence's row normed and multiplied on its own
        for (uint32_t t = 0; t < B; ++t) {
            e.cmd({GEMVQ_OP_RMSNORM, E, m.bh + t * E, onorm.act_off, m.xn, fb(c.eps), 1, GEMVQ_NORM_DEFER});
            e.gemv(head, m.xn, m.slogits + t * V);
        }
    }
    e.cmd({GEMVQ_OP_ARGMAX, V, m.slogits, m.skey, B, V});
    e.cmd({GEMVQ_OP_NEXT_TOKEN, m.skey, m.bid, m.spos, m.sprompt, m.slen, m.sout, B | (uint32_t(c.n_ctx) << 8)});
    (void)err;
    return true;
}

bool build_commands(gemvq_qwen35 & m, std::string & err) {
    const gemvq_qw_config & c = m.c;
    Emit e{m.cmds};
    auto W = [&](const std::string & name) -> const T * {
        auto it = m.t.find(name);
        if (it == m.t.end() || !it->second.d) {
            err = "missing tensor " + name;
            return nullptr;
        }
        return &it->second;
    };
    const float eps = c.eps;
    const int E = c.n_embd, S = c.ssm_head_dim, hv = c.ssm_v_heads, hk = c.ssm_k_heads, ch = conv_ch(c);
    const T * emb = W("token_embd.weight");
    const T * onorm = W("output_norm.weight");
    const T * head = W("output.weight");
    if (!emb || !onorm || !head) return false;
    e.cmd({GEMVQ_OP_GET_ROWS, uint32_t(emb->d->type), uint32_t(emb->d->ne1), uint32_t(emb->d->ne0),
           uint32_t(emb->w_off), uint32_t(emb->w_off >> 32), m.tok, m.h});
    for (int il = 0; il < c.n_layer; ++il) {
        const std::string p = "blk." + std::to_string(il) + ".";
        const T * an = W(p + "attn_norm.weight");
        const T * pn = W(p + "post_attention_norm.weight");
        const T * fg = W(p + "ffn_gate.weight");
        const T * fu = W(p + "ffn_up.weight");
        const T * fd = W(p + "ffn_down.weight");
        if (!an || !pn || !fg || !fu || !fd) return false;
        e.cmd({GEMVQ_OP_RMSNORM, uint32_t(E), m.h, an->act_off, m.xn, fb(eps), 1, GEMVQ_NORM_DEFER});
        if (is_attn(c, il)) {
            const T * wq = W(p + "attn_q.weight");
            const T * wk = W(p + "attn_k.weight");
            const T * wv = W(p + "attn_v.weight");
            const T * qn = W(p + "attn_q_norm.weight");
            const T * kn = W(p + "attn_k_norm.weight");
            const T * wo = W(p + "attn_output.weight");
            if (!wq || !wk || !wv || !qn || !kn || !wo) return false;
            e.gemv(*wq, m.xn, m.qg);
            e.gemv(*wk, m.xn, m.kk);
            e.gemv(*wv, m.xn, m.vv);
            const uint32_t hd = uint32_t(c.head_dim);
            e.cmd({GEMVQ_OP_ATTN, uint32_t(c.n_head) | (uint32_t(c.n_head_kv) << 16), m.qg, uint32_t(m.kv[il]), m.att,
                   hd | (uint32_t(c.n_rot) << 16), m.pos, 1u});
            e.cmd({m.kk, m.vv, fb(1.0f / std::sqrt(float(c.head_dim))), fb(eps), qn->act_off, kn->act_off, m.rope,
                   m.qg + hd});
            e.gemv(*wo, m.att, m.tmp, GEMVQ_GEMV_ADD);
            e.cmd({GEMVQ_OP_ADD, uint32_t(E), m.tmp, m.h, m.h});
        } else {
            const T * wqkv = W(p + "attn_qkv.weight");
            const T * wz = W(p + "attn_gate.weight");
            const T * wb = W(p + "ssm_beta.weight");
            const T * wa = W(p + "ssm_alpha.weight");
            const T * cw = W(p + "ssm_conv1d.weight");
            const T * dt = W(p + "ssm_dt.bias");
            const T * a = W(p + "ssm_a");
            const T * sn = W(p + "ssm_norm.weight");
            const T * so = W(p + "ssm_out.weight");
            if (!wqkv || !wz || !wb || !wa || !cw || !dt || !a || !sn || !so) return false;
            const uint32_t ba2 = m.ba + uint32_t(up16(hv));
            e.gemv(*wqkv, m.xn, m.qkv, GEMVQ_GEMV_CONV);
            e.cmd({GEMVQ_OP_CONV, uint32_t(ch), m.qkv, cw->act_off, m.cqkv, m.conv_state[il], m.conv_state[il], 1u});
            e.gemv(*wz, m.xn, m.z, GEMVQ_GEMV_SILU);  // the gate's SiLU, once per element
            e.gemv(*wb, m.xn, m.ba);
            e.gemv(*wa, m.xn, ba2);
            // state rows of this layer: layer slot * hv * 128
            int slot = 0;
            for (int j = 0; j < il; ++j) slot += !is_attn(c, j);
            const uint32_t row = uint32_t(slot) * uint32_t(hv) * 128u;
            const uint32_t flags = GEMVQ_GDN_L2_QK | GEMVQ_GDN_GATED | GEMVQ_GDN_GATES | GEMVQ_GDN_Z_SILU;
            e.cmd({GEMVQ_OP_GDN, uint32_t(hv) | (uint32_t(hk) << 16), m.cqkv, m.cqkv + uint32_t(hk * S),
                   m.cqkv + uint32_t(2 * hk * S), ba2, m.ba, m.y});
            e.cmd({row, row, fb(1.0f / std::sqrt(float(S))), flags, fb(eps), fb(eps), sn->act_off, m.z});
            e.cmd({dt->act_off, a->act_off});
            e.gemv(*so, m.y, m.tmp, GEMVQ_GEMV_ADD);
            e.cmd({GEMVQ_OP_ADD, uint32_t(E), m.tmp, m.h, m.h});
        }
        e.cmd({GEMVQ_OP_RMSNORM, uint32_t(E), m.h, pn->act_off, m.xn, fb(eps), 1, GEMVQ_NORM_DEFER});
        e.gemv(*fg, m.xn, m.ffn, GEMVQ_GEMV_SWIGLU);
        e.gemv(*fu, m.xn, m.ffn);
        e.gemv(*fd, m.ffn, m.tmp, GEMVQ_GEMV_ADD);
        e.cmd({GEMVQ_OP_ADD, uint32_t(E), m.tmp, m.h, m.h});
    }
    e.cmd({GEMVQ_OP_RMSNORM, uint32_t(E), m.h, onorm->act_off, m.xn, fb(eps), 1, GEMVQ_NORM_DEFER});
    e.gemv(*head, m.xn, m.logits, GEMVQ_GEMV_ARGMAX);
    e.cmd({GEMVQ_OP_ARGMAX, uint32_t(head->d->ne1), m.logits, m.key});
    e.cmd({GEMVQ_OP_NEXT_TOKEN, m.key, m.tok, m.pos, m.prompt, 0u, m.out});
    return true;
}

}  // namespace

extern "C" void gq_set_error(gemvq_ctx * ctx, const char * what);  // gq_runtime.hip

namespace {
int set_err(gemvq_ctx * ctx, const std::string & what) {
    gq_set_error(ctx, what.c_str());
    return GEMVQ_EINVAL;
}
}  // namespace

extern "C" {

int gemvq_qwen35_sizes(const gemvq_qw_config * cfg, const gemvq_tensor_desc * tab, int n, size_t * act_floats,
                       size_t * weight_bytes, size_t * state_rows) {
    return gemvq_qwen35_batch_sizes(cfg, tab, n, 1, act_floats, weight_bytes, state_rows);
}

int gemvq_qwen35_batch_sizes(const gemvq_qw_config * cfg, const gemvq_tensor_desc * tab, int n, int n_seq,
                             size_t * act_floats, size_t * weight_bytes, size_t * state_rows) {
    if (!cfg || !tab || n <= 0 || n_seq < 1 || n_seq > int(GEMVQ_GEMM_MAX_TOK)) return GEMVQ_EINVAL;
    gemvq_qwen35 m;
    m.c = *cfg;
    m.n_seq = n_seq;
    const size_t act = layout(m, tab, n);
    size_t wb = 0;
    for (int i = 0; i < n; ++i)
        if (tab[i].type != F32) wb += (tab[i].nbytes + 255) / 256 * 256;
    int gdn_layers = 0;
    for (int il = 0; il < cfg->n_layer; ++il) gdn_layers += !is_attn(*cfg, il);
    if (act_floats) *act_floats = act;
    if (weight_bytes) *weight_bytes = wb + 4096;
    if (state_rows) *state_rows = size_t(gdn_layers) * cfg->ssm_v_heads * 128 * size_t(n_seq);
    return 0;
}

gemvq_qwen35 * gemvq_qwen35_create(gemvq_ctx * ctx, const gemvq_qw_config * cfg, const gemvq_tensor_desc * tab,
                                   int n, const uint8_t * blob) {
    return gemvq_qwen35_batch_create(ctx, cfg, tab, n, blob, 1);
}

gemvq_qwen35 * gemvq_qwen35_batch_create(gemvq_ctx * ctx, const gemvq_qw_config * cfg, const gemvq_tensor_desc * tab,
                                         int n, const uint8_t * blob, int n_seq) {
    if (!ctx || !cfg || !tab || !blob || n <= 0) return nullptr;
    if (n_seq < 1 || n_seq > int(GEMVQ_GEMM_MAX_TOK)) {
        set_err(ctx, "gemvq_qwen35_batch_create: 1 to GEMVQ_GEMM_MAX_TOK sequences");
        return nullptr;
    }
    auto * m = new gemvq_qwen35();
    m->ctx = ctx;
    m->c = *cfg;
    m->n_seq = n_seq;
    const gemvq_qw_config & c = m->c;
    if (c.n_rot % 2 || c.n_rot > c.head_dim || c.ssm_head_dim != 128 || c.attn_interval <= 0 || c.n_ctx <= 0) {
        set_err(ctx, "gemvq_qwen35_create: unsupported configuration");
        delete m;
        return nullptr;
    }
    m->descs.assign(tab, tab + n);
    m->act_floats = layout(*m, m->descs.data(), n);
    for (int i = 0; i < n; ++i) {
        T & x = m->t[tab[i].name];
        x.d = &m->descs[i];
        if (tab[i].type == F32) {
            if (gemvq_act_write(ctx, x.act_off, blob + tab[i].offset, size_t(tab[i].ne0) * std::max(1, tab[i].ne1))) {
                delete m;
                return nullptr;
            }
        } else if (gemvq_upload_weight(ctx, tab[i].type, tab[i].ne1, tab[i].ne0, blob + tab[i].offset, &x.w_off)) {
            delete m;
            return nullptr;
        }
    }
    m->kv.assign(c.n_layer, -1);
    for (int il = 0; il < c.n_layer; ++il) {
        if (!is_attn(c, il)) continue;
        m->kv[il] = gemvq_kv_create(ctx, c.n_ctx * n_seq, c.n_head_kv, c.head_dim);  // one region per sequence
        if (m->kv[il] < 0) {
            delete m;
            return nullptr;
        }
    }
    // ggml's rope cache for every position (theta advanced by theta *= base^(-2 / n_rot), ggml-xrt.cpp:875-946
    // with ext_factor 0): cos and sin of pair i at 2i, 2i + 1
    std::vector<float> rope(size_t(c.n_ctx) * c.n_rot);
    const float theta_scale = std::pow(c.rope_base, -2.0f / float(c.n_rot));
    for (int p = 0; p < c.n_ctx; ++p) {
        float theta = float(p);
        for (int i0 = 0; i0 < c.n_rot; i0 += 2) {
            rope[size_t(p) * c.n_rot + i0] = std::cos(theta);
            rope[size_t(p) * c.n_rot + i0 + 1] = std::sin(theta);
            theta *= theta_scale;
        }
    }
    std::string err;
    m->can_batch = batchable(*m, m->batch_why);
    if (n_seq > 1 && !m->can_batch) {
        set_err(ctx, "gemvq_qwen35_batch_create: " + m->batch_why);
        delete m;
        return nullptr;
    }
    if (gemvq_act_write(ctx, m->rope, rope.data(), rope.size()) ||
        !(n_seq > 1 ? build_batch(*m, err) : build_commands(*m, err))) {
        if (!err.empty()) set_err(ctx, err);
        delete m;
        return nullptr;
    }
    return m;  // the per-token graph is captured by the first gemvq_qwen35_step
}

void gemvq_qwen35_destroy(gemvq_qwen35 * m) {
    if (!m) return;
    if (m->graph >= 0) gemvq_graph_destroy(m->ctx, m->graph);
    if (m->chunk_graph >= 0) gemvq_graph_destroy(m->ctx, m->chunk_graph);
    delete m;
}

int gemvq_qwen35_reset(gemvq_qwen35 * m, const int32_t * prompt, int n) {
    if (!m || !prompt || n < 1 || n > m->c.n_ctx || m->n_seq > 1) return GEMVQ_EINVAL;
    gemvq_ctx * ctx = m->ctx;
    int st = gemvq_sync(ctx);
    if (!st) st = gemvq_state_clear(ctx);
    if (!st) st = gemvq_kv_clear(ctx);
    const int ch = conv_ch(m->c);
    std::vector<float> zeros(size_t(ch) * 3, 0.0f);
    for (int il = 0; il < m->c.n_layer && !st; ++il)
        if (!is_attn(m->c, il)) st = gemvq_act_write(ctx, m->conv_state[il], zeros.data(), zeros.size());
    std::vector<int32_t> p(size_t(m->c.n_ctx), 0);
    std::memcpy(p.data(), prompt, size_t(n) * 4);
    if (!st) st = gemvq_act_write(ctx, m->prompt, p.data(), p.size());
    std::vector<int32_t> o(size_t(m->c.n_ctx) + 16, -1);
    o[0] = prompt[0];
    if (!st) st = gemvq_act_write(ctx, m->out, o.data(), o.size());
    const int32_t scal[48] = {};
    if (!st) st = gemvq_act_write(ctx, 16, scal, 48);
    if (!st) st = gemvq_act_write(ctx, m->tok, &prompt[0], 1);
    if (st) return st;
    m->prompt_ids.assign(prompt, prompt + n);
    // NEXT_TOKEN reads the prompt length from its command; the graph is captured again when it changes
    const size_t last = m->cmds.size() - GEMVQ_CMD_WORDS;
    if (m->cmds[last + 5] != uint32_t(n)) {
        m->cmds[last + 5] = uint32_t(n);
        if (m->graph >= 0) gemvq_graph_destroy(ctx, m->graph);
        m->graph = -1;
    }
    return st;
}

int gemvq_qwen35_prefill(gemvq_qwen35 * m, int n) {
    if (!m || n < 0 || m->n_seq > 1) return GEMVQ_EINVAL;
    gemvq_ctx * ctx = m->ctx;
    if (n == 0) return 0;
    if (!m->can_batch) return set_err(ctx, "gemvq_qwen35_prefill: " + m->batch_why);
    int32_t pos = 0;
    int st = gemvq_sync(ctx);
    if (!st) st = gemvq_act_read(ctx, m->pos, &pos, 1);
    if (st) return st;
    const int np = int(m->prompt_ids.size());
    if (pos < 0 || pos + n > np - 1) return set_err(ctx, "gemvq_qwen35_prefill: positions past the last prompt token but one");
    std::vector<uint32_t> w;
    for (int p0 = pos; p0 < pos + n && !st;) {
        const int nt = std::min<int>(GEMVQ_GEMM_MAX_TOK, pos + n - p0);
        std::vector<int32_t> slots(size_t(16) * GEMVQ_GEMM_MAX_TOK, 0);  // ids, one per 16 floats
        for (int i = 0; i < nt; ++i) slots[size_t(16) * i] = m->prompt_ids[size_t(p0 + i)];
        st = gemvq_act_write(ctx, m->bid, slots.data(), slots.size());
        if (!st) st = gemvq_act_write(ctx, m->bpos, &p0, 1);  // the chunk's first position
        if (!st && nt == int(GEMVQ_GEMM_MAX_TOK)) {
            // full chunks replay one captured list: it reads the chunk's ids and first position from the slots
            // just written (the write waits for the previous replay; the replay follows it on the same stream)
            if (m->chunk_graph < 0) {
                w.clear();
                build_chunk(*m, GEMVQ_GEMM_MAX_TOK, w);
                st = gemvq_graph_create(ctx, w.data(), unsigned(w.size() / GEMVQ_CMD_WORDS), &m->chunk_graph);
            }
            if (!st) st = gemvq_graph_replay(ctx, m->chunk_graph, 1);
        } else if (!st) {
            w.clear();
            build_chunk(*m, uint32_t(nt), w);
            st = gemvq_run(ctx, w.data(), unsigned(w.size() / GEMVQ_CMD_WORDS));
        }
        p0 += nt;
    }
    if (!st) st = gemvq_sync(ctx);
    if (st) return st;
    // what the steps' NEXT_TOKEN would have left: the next prompt token at the next position, the ids so far
    const int32_t end = pos + n, tok = m->prompt_ids[size_t(end)];
    st = gemvq_act_write(ctx, m->pos, &end, 1);
    if (!st) st = gemvq_act_write(ctx, m->tok, &tok, 1);
    if (!st) st = gemvq_act_write(ctx, m->out + size_t(pos) + 1, m->prompt_ids.data() + pos + 1, size_t(n));
    return st;
}

int gemvq_qwen35_step(gemvq_qwen35 * m, int n) {
    if (!m) return GEMVQ_EINVAL;
    if (m->graph < 0) {
        const int st = gemvq_graph_create(m->ctx, m->cmds.data(), unsigned(m->cmds.size() / GEMVQ_CMD_WORDS), &m->graph);
        if (st) return st;
    }
    return gemvq_graph_replay(m->ctx, m->graph, n);
}

int gemvq_qwen35_tokens(gemvq_qwen35 * m, int32_t * out, int n) {
    if (!m || !out || n < 0 || n > m->c.n_ctx || m->n_seq > 1) return GEMVQ_EINVAL;
    return gemvq_act_read(m->ctx, m->out, out, size_t(n));
}

int gemvq_qwen35_logits(gemvq_qwen35 * m, float * out) {
    if (!m || !out || m->n_seq > 1) return GEMVQ_EINVAL;
    return gemvq_act_read(m->ctx, m->logits, out, size_t(m->c.n_vocab));
}

int gemvq_qwen35_hidden(gemvq_qwen35 * m, float * out) {
    if (!m || !out || m->n_seq > 1) return GEMVQ_EINVAL;
    return gemvq_act_read(m->ctx, m->h, out, size_t(m->c.n_embd));
}

int gemvq_qwen35_batch_reset(gemvq_qwen35 * m, const int32_t * prompts, const int32_t * offsets) {
    if (!m || !prompts || !offsets || m->n_seq < 2) return GEMVQ_EINVAL;
    const gemvq_qw_config & c = m->c;
    const int ns = m->n_seq, cap = c.n_ctx;
    for (int s = 0; s < ns; ++s)
        if (offsets[s + 1] - offsets[s] < 1 || offsets[s + 1] - offsets[s] > cap) return GEMVQ_EINVAL;
    gemvq_ctx * ctx = m->ctx;
    int st = gemvq_sync(ctx);
    if (!st) st = gemvq_state_clear(ctx);
    if (!st) st = gemvq_kv_clear(ctx);
    std::vector<float> zeros(size_t(conv_ch(c)) * 3 * ns, 0.0f);
    for (int il = 0; il < c.n_layer && !st; ++il)
        if (!is_attn(c, il)) st = gemvq_act_write(ctx, m->conv_state[il], zeros.data(), zeros.size());
    std::vector<int32_t> pr(size_t(ns) * cap, 0), out(size_t(ns) * cap, -1), slots(size_t(ns) * 16, 0),
        len(size_t(ns) * 16, 0), ids(size_t(GEMVQ_GEMM_MAX_TOK) * 16, 0);
    for (int s = 0; s < ns; ++s) {
        const int n = offsets[s + 1] - offsets[s];
        std::memcpy(&pr[size_t(s) * cap], prompts + offsets[s], size_t(n) * 4);
        out[size_t(s) * cap] = prompts[offsets[s]];
        len[size_t(s) * 16] = n;
        ids[size_t(s) * 16] = prompts[offsets[s]];
    }
    if (!st) st = gemvq_act_write(ctx, m->sprompt, pr.data(), pr.size());
    if (!st) st = gemvq_act_write(ctx, m->sout, out.data(), out.size());
    if (!st) st = gemvq_act_write(ctx, m->slen, len.data(), len.size());
    if (!st) st = gemvq_act_write(ctx, m->spos, slots.data(), slots.size());  // every position 0
    if (!st) st = gemvq_act_write(ctx, m->skey, slots.data(), slots.size());
    if (!st) st = gemvq_act_write(ctx, m->bid, ids.data(), ids.size());
    return st;
}

int gemvq_qwen35_batch_tokens(gemvq_qwen35 * m, int seq, int32_t * out, int n) {
    if (!m || !out || m->n_seq < 2 || seq < 0 || seq >= m->n_seq || n < 0 || n > m->c.n_ctx) return GEMVQ_EINVAL;
    return gemvq_act_read(m->ctx, m->sout + size_t(seq) * m->c.n_ctx, out, size_t(n));
}

int gemvq_qwen35_batch_logits(gemvq_qwen35 * m, int seq, float * out) {
    if (!m || !out || m->n_seq < 2 || seq < 0 || seq >= m->n_seq) return GEMVQ_EINVAL;
    return gemvq_act_read(m->ctx, m->slogits + size_t(seq) * m->c.n_vocab, out, size_t(m->c.n_vocab));
}

int gemvq_qwen35_commands(gemvq_qwen35 * m, uint32_t * words, size_t n_words) {
    if (!m) return GEMVQ_EINVAL;
    if (words && n_words >= m->cmds.size()) std::memcpy(words, m->cmds.data(), m->cmds.size() * 4);
    return int(m->cmds.size() / GEMVQ_CMD_WORDS);
}

int gemvq_qwen35_graph(gemvq_qwen35 * m) { return m ? m->graph : -1; }

int gemvq_qwen35_set_arith(gemvq_qwen35 * m, int arith) {
    if (!m) return GEMVQ_EINVAL;
    const int st = gemvq_set_arith(m->ctx, arith);
    if (st) return st;
    // the captured graphs hold the kernels of the arithmetic they were compiled in: capture again on next use
    if (m->graph >= 0) gemvq_graph_destroy(m->ctx, m->graph);
    if (m->chunk_graph >= 0) gemvq_graph_destroy(m->ctx, m->chunk_graph);
    m->graph = m->chunk_graph = -1;
    return 0;
}

}  // extern "C"

extern "C" int gemvq_qwen35_dry_commands(const gemvq_qw_config * cfg, const gemvq_tensor_desc * tab, int n,
                                         uint32_t * words, size_t n_words) {
    if (!cfg || !tab || n <= 0) return GEMVQ_EINVAL;
    gemvq_qwen35 m;
    m.c = *cfg;
    m.descs.assign(tab, tab + n);
    layout(m, m.descs.data(), n);
    uint64_t used = 0;  // gemvq_upload_weight's placement: each matrix at the next 256-byte boundary, in table order
    for (int i = 0; i < n; ++i) {
        T & x = m.t[tab[i].name];
        x.d = &m.descs[i];
        if (tab[i].type == F32) continue;
        x.w_off = (used + 255) & ~uint64_t(255);
        used = x.w_off + tab[i].nbytes;
    }
    m.kv.assign(cfg->n_layer, -1);
    int kv = 0;
    for (int il = 0; il < cfg->n_layer; ++il)
        if (is_attn(*cfg, il)) m.kv[il] = kv++;
    std::string err;
    if (!build_commands(m, err)) return GEMVQ_EINVAL;
    if (words && n_words >= m.cmds.size()) std::memcpy(words, m.cmds.data(), m.cmds.size() * 4);
    return int(m.cmds.size() / GEMVQ_CMD_WORDS);
}
