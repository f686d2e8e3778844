// ggml-facing backend (include/gemvq_ggml.h): a split of a ggml-shaped graph compiled into one gemvq command list
// (the reference's xrt_qc_build_plan + xrt_qc_graph_compute_gdn, ggml-xrt.cpp:1813-2745), cached with its captured
// hipGraph under the split's exact identity, and run with its inputs copied in and its outputs copied back.
//
// Act buffer layout of a backend: [0, 64) unused, [64, trans_end) the transient region (the inputs and outputs of
// the split being run; every plan starts from 64, splits run one after another), [trans_end, act_floats) the
// resident region (F32 weights, conv states, rope tables, position slots), filled from the top of the transient
// region upward as first uses come.
#include "gemvq_ggml.h"
#include "gemvq_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <sys/mman.h>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

constexpr int HEAD = 128;  // DeltaNet head size (state rows of 128 floats)

size_t up16(size_t n) { return (n + 15) / 16 * 16; }

uint32_t fbits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

float pf(const gqg_tensor * t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], 4);
    return f;
}

int64_t nel(const gqg_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

bool is_view(const gqg_tensor * t) {
    return t->op == GQG_OP_VIEW || t->op == GQG_OP_RESHAPE || t->op == GQG_OP_PERMUTE || t->op == GQG_OP_TRANSPOSE ||
           t->op == GQG_OP_NONE;
}

const gqg_tensor * root_of(const gqg_tensor * t) {
    while (t && t->view_src) t = t->view_src;
    return t;
}

bool contiguous(const gqg_tensor * t) {
    size_t s = 4;
    for (int d = 0; d < GQG_MAX_DIMS; ++d) {
        if (t->ne[d] > 1 && t->nb[d] != s) return false;
        s *= size_t(t->ne[d]);
    }
    return true;
}

// One token row of F32: a contiguous vector (ggml's [n, 1, 1, 1] after any reshape).
bool token_row(const gqg_tensor * t) { return t->type == GQG_TYPE_F32 && contiguous(t); }

// Strided F32 rows: ne0 floats each, rows nb1 bytes apart (a multiple of 64 bytes), one dimension of rows.
bool strided_rows(const gqg_tensor * t) {
    return t->type == GQG_TYPE_F32 && t->nb[0] == 4 && t->ne[2] == 1 && t->ne[3] == 1 && t->nb[1] % 64 == 0 &&
           t->nb[1] >= size_t(t->ne[0]) * 4 && t->ne[0] % 16 == 0;
}

bool quant_type(int t) {
    return t == GQG_TYPE_Q4_0 || t == GQG_TYPE_Q4_1 || t == GQG_TYPE_Q8_0 || t == GQG_TYPE_Q5_K || t == GQG_TYPE_Q6_K;
}

size_t row_bytes(int type, int64_t cols) {
    switch (type) {
    case GQG_TYPE_Q4_0: return size_t(cols / 32) * 18;
    case GQG_TYPE_Q4_1: return size_t(cols / 32) * 20;
    case GQG_TYPE_Q8_0: return size_t(cols / 32) * 34;
    case GQG_TYPE_Q5_K: return size_t(cols / 256) * 176;
    case GQG_TYPE_Q6_K: return size_t(cols / 256) * 210;
    default: return 0;
    }
}

bool is_weight(const gqg_tensor * t) {
    const gqg_tensor * r = root_of(t);
    return r && r->buffer == GQG_BUF_WEIGHTS;
}

bool f32_weight(const gqg_tensor * t) { return is_weight(t) && t->type == GQG_TYPE_F32 && contiguous(t); }

int unary_kind(const gqg_tensor * t) {  // command UNARY kind: 1 SiLU, 2 sigmoid, 3 softplus
    if (t->op != GQG_OP_UNARY) return 0;
    const int u = t->op_params[0];
    return u == GQG_UNARY_SILU ? 1 : u == GQG_UNARY_SIGMOID ? 2 : u == GQG_UNARY_SOFTPLUS ? 3 : 0;
}

bool in_buf(const gqg_tensor * t, int buf) {
    const gqg_tensor * r = root_of(t);
    return r && r->buffer == buf;
}

// GET_ROWS of one row (the sequence's) from a recurrent-state tensor (through views).
const gqg_tensor * rs_rows(const gqg_tensor * t) {
    while (t && is_view(t) && t->op != GQG_OP_NONE) t = t->src[0];
    return t && t->op == GQG_OP_GET_ROWS && in_buf(t->src[0], GQG_BUF_RS) && nel(t->src[1]) == 1 ? t : nullptr;
}

struct Status {
    int code = GQG_STATUS_SUCCESS;
    std::string what;
};

}  // namespace

struct gqg_buffer {
    gqg_backend * owner = nullptr;
    int kind = GQG_BUF_RS;
    uint8_t * base = nullptr;
    size_t size = 0;
    struct Entry {
        size_t off = 0, bytes = 0;
        bool state = false;  // RS: on state rows (else resident act floats)
        size_t dev = 0;      // first state row, or act offset
        int kv = -1;         // KV: the device cache
        bool v = false;      // KV: the value half
    };
    std::vector<Entry> tensors;
    const Entry * find(const void * p) const {
        const auto * b = static_cast<const uint8_t *>(p);
        if (b < base || b >= base + size) return nullptr;
        const size_t off = size_t(b - base);
        for (const auto & e : tensors)
            if (off >= e.off && off < e.off + e.bytes) return &e;
        return nullptr;
    }
};

struct gqg_backend {
    gqg_params p{};
    gemvq_ctx * ctx = nullptr;
    bool valid = true;
    std::string err;
    uint64_t w_used = 0;  // dry: the arena's bump pointer (gemvq_upload_weight's rule)
    std::map<std::vector<uint64_t>, uint64_t> weights;
    std::unordered_map<const void *, uint32_t> consts;   // F32 weight data -> resident act offset
    std::map<std::vector<uint64_t>, uint32_t> tables;    // rope table identity -> resident act offset
    size_t trans_end = 0, res_used = 0;
    size_t state_rows_used = 0;
    std::vector<gqg_buffer *> buffers;
    struct KvPair { int kv = -1; int64_t n_ctx = 0, row = 0; };
    std::map<std::string, KvPair> kv_layers;  // layer suffix -> device cache
    struct Io { const void * host; uint32_t off; size_t floats; };
    struct Plan {
        std::vector<uint64_t> sig;  // the split's structural signature (signature_of) and its hash
        uint64_t hash = 0;
        std::vector<uint32_t> words;
        std::vector<Io> in, out;  // host data copied in before, results copied back after the run
        std::vector<std::pair<const int64_t *, const int32_t *>> pos_checks;  // KV row == position
        int graph = -1;
    };
    std::vector<std::unique_ptr<Plan>> plans;
    uint64_t built = 0, reused = 0;

    bool dry() const { return p.dry != 0; }
};

namespace {

gqg_backend * g_active = nullptr;  // one backend per process (ggml-xrt.cpp:381-387)

int fail(gqg_backend * b, const std::string & what, int code = GQG_STATUS_FAILED) {
    if (b) b->err = what;
    return code;
}

// ---- device-side resources (dry backends only assign offsets) ----

bool upload_weight(gqg_backend * b, const gqg_tensor * t, uint64_t & off, std::string & err) {
    const gqg_tensor * r = root_of(t);
    std::vector<uint64_t> key = {uint64_t(reinterpret_cast<uintptr_t>(r)), uint64_t(reinterpret_cast<uintptr_t>(t->data)),
                                 uint64_t(t->type)};
    for (int d = 0; d < GQG_MAX_DIMS; ++d) {
        key.push_back(uint64_t(t->ne[d]));
        key.push_back(uint64_t(t->nb[d]));
    }
    const auto it = b->weights.find(key);
    if (it != b->weights.end()) {
        off = it->second;
        return true;
    }
    const int cols = int(t->ne[0]), rows = int(t->ne[1]);
    if (!quant_type(t->type) || t->ne[2] != 1 || t->ne[3] != 1 || t->nb[1] != row_bytes(t->type, cols)) {
        err = std::string("weight ") + t->name + ": not a packed quantized matrix";
        return false;
    }
    if (b->dry()) {
        off = (b->w_used + 255) & ~uint64_t(255);
        b->w_used = off + row_bytes(t->type, cols) * uint64_t(rows);
        if (b->w_used > b->p.weight_bytes) {
            err = "weight arena full";
            return false;
        }
    } else if (gemvq_upload_weight(b->ctx, t->type, rows, cols, t->data, &off)) {
        err = std::string("weight ") + t->name + ": " + gemvq_last_error(b->ctx);
        return false;
    }
    b->weights[key] = off;
    return true;
}

bool take_resident(gqg_backend * b, size_t floats, uint32_t & off, std::string & err) {
    const size_t at = b->trans_end + b->res_used;
    if (at + up16(floats) > b->p.act_floats) {
        err = "resident act region full";
        return false;
    }
    b->res_used += up16(floats);
    off = uint32_t(at);
    return true;
}

bool act_write(gqg_backend * b, uint32_t off, const void * src, size_t floats, std::string & err) {
    if (b->dry() || floats == 0) return true;
    if (gemvq_act_write(b->ctx, off, src, floats)) {
        err = gemvq_last_error(b->ctx);
        return false;
    }
    return true;
}

bool const_of(gqg_backend * b, const gqg_tensor * t, uint32_t & off, std::string & err) {
    const auto it = b->consts.find(t->data);
    if (it != b->consts.end()) {
        off = it->second;
        return true;
    }
    const size_t n = size_t(nel(t));
    if (!take_resident(b, n, off, err) || !act_write(b, off, t->data, n, err)) return false;
    b->consts[t->data] = off;
    return true;
}

// ggml's rope cache for every position of a cache of n_ctx (theta advanced by theta *= base^(-2 / n_dims)): cos
// and sin of pair i at 2i, 2i + 1 (the arithmetic of the model builder's table, so both paths read equal tables).
bool rope_table(gqg_backend * b, int n_dims, float base, int64_t n_ctx, uint32_t & off, std::string & err) {
    const std::vector<uint64_t> key = {uint64_t(n_dims), uint64_t(fbits(base)), uint64_t(n_ctx)};
    const auto it = b->tables.find(key);
    if (it != b->tables.end()) {
        off = it->second;
        return true;
    }
    std::vector<float> t(size_t(n_ctx) * n_dims);
    const float theta_scale = std::pow(base, -2.0f / float(n_dims));
    for (int64_t p = 0; p < n_ctx; ++p) {
        float theta = float(p);
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            t[size_t(p) * n_dims + i0] = std::cos(theta);
            t[size_t(p) * n_dims + i0 + 1] = std::sin(theta);
            theta *= theta_scale;
        }
    }
    if (!take_resident(b, t.size(), off, err) || !act_write(b, off, t.data(), t.size(), err)) return false;
    b->tables[key] = off;
    return true;
}

// ---- the fusion plan of a split ----
//
// A reader index of the split (for every data root, the non-view nodes that read it, through which operand), then
// one pass over the nodes from the last to the first. Each fused form is anchored at the node that consumes its
// chain: the conv's SSM_CONV, the DeltaNet step, the attention, the GLU of a SwiGLU pair, a GEMV (for the ADD that
// reads it), a norm (for the GEMVs that read it). Walking backwards, every consumer has settled what it absorbs
// before its producers are visited, so a GEMV or a norm decides its own fusion against the final set of absorbed
// nodes. The conditions are the ones the reference kernel's fused forms need (gemvqc16.h; the reference's planner
// decides the same forms, ggml-xrt.cpp:1813-2110).

bool unfused_output(const gqg_tensor * t) { return (t->flags & (GQG_FLAG_OUTPUT | GQG_FLAG_SPLIT_OUTPUT)) == 0; }

// Through views to the computing node.
const gqg_tensor * through_views(const gqg_tensor * t) {
    while (t && is_view(t) && t->op != GQG_OP_NONE && t->src[0]) t = t->src[0];
    return t;
}

struct ReaderIndex {
    struct Read {
        const gqg_tensor * node;  // the reading node
        int slot;                 // its operand index
        const gqg_tensor * via;   // the operand as the node names it (the root or a view of it)
    };
    std::unordered_map<const gqg_tensor *, std::vector<Read>> reads;  // data root -> its reads, in node order
    std::unordered_map<const gqg_tensor *, int> nodes_reading;        // data root -> distinct nodes reading it
    std::unordered_map<const gqg_tensor *, int> at;                   // node -> position in the split

    void build(const gqg_cgraph * g) {
        for (int i = 0; i < g->n_nodes; ++i) at[g->nodes[i]] = i;
        for (int i = 0; i < g->n_nodes; ++i) {
            const gqg_tensor * m = g->nodes[i];
            if (is_view(m)) continue;
            for (int k = 0; k < GQG_MAX_SRC; ++k) {
                if (!m->src[k]) continue;
                const gqg_tensor * r = root_of(m->src[k]);
                auto & v = reads[r];
                bool seen = false;
                for (const Read & x : v) seen = seen || x.node == m;
                if (!seen) ++nodes_reading[r];
                v.push_back({m, k, m->src[k]});
            }
        }
    }
    int readers(const gqg_tensor * r) const {
        const auto it = nodes_reading.find(r);
        return it == nodes_reading.end() ? 0 : it->second;
    }
    // the node that alone reads root r, when r is no graph or split output (its value is then needed only there)
    const gqg_tensor * sole(const gqg_tensor * r) const {
        if (readers(r) != 1 || !unfused_output(r)) return nullptr;
        return reads.at(r).front().node;
    }
    // the first read of root r that pred accepts
    template <typename P>
    const Read * first(const gqg_tensor * r, P pred) const {
        const auto it = reads.find(r);
        if (it == reads.end()) return nullptr;
        for (const Read & x : it->second)
            if (pred(x)) return &x;
        return nullptr;
    }
    bool in_split(const gqg_tensor * t) const { return at.count(t) != 0; }
};

// The one-token conv chain (gemvqc16.cpp:161-190, 244-281): the state's window row, CONCAT with the input, SSM_CONV,
// and the CPY of the new window back into the state.
struct ConvChain {
    const gqg_tensor * state_rows = nullptr, * window = nullptr, * store = nullptr, * conv = nullptr, * input = nullptr;
};
// The DeltaNet step with what the GDN command folds into it (gemvqc16.h:60-81, gemvqc_gdn.h).
struct DeltaStep {
    const gqg_tensor * state_rows = nullptr, * store = nullptr;
    bool l2 = false;
    float l2_eps = 0.0f, rms_eps = 0.0f;
    const gqg_tensor * gated = nullptr, * norm_w = nullptr, * gate = nullptr;  // gated norm output, its weight, z
    bool gate_silu = false;                                                      // gate holds silu(z)
    const gqg_tensor * alpha = nullptr, * beta = nullptr, * dt = nullptr, * a = nullptr;  // raw gates
};
// One-token gated attention: the q (+ gate) / k / v projections, the norms, RoPE, the cache stores and the output.
struct AttnChain {
    const gqg_tensor * q_proj = nullptr, * k_proj = nullptr, * v_proj = nullptr, * q_norm_w = nullptr,
                     * k_norm_w = nullptr, * fa = nullptr, * k_store = nullptr, * v_store = nullptr, * pos = nullptr,
                     * k_row = nullptr;
    float eps = 0.0f, scale = 0.0f, base = 0.0f;
    int n_rot = 0, n_head = 0, n_head_kv = 0, head_dim = 0;
    std::string layer;
};

struct FusionPlan {
    ReaderIndex ix;
    std::unordered_set<const gqg_tensor *> absorbed;  // nodes computed inside another node's command
    std::unordered_map<const gqg_tensor *, ConvChain> conv_by_silu;            // the SiLU closing a conv chain
    std::unordered_map<const gqg_tensor *, const gqg_tensor *> conv_input_gemv;  // GEMV -> SiLU of the conv it feeds
    std::unordered_map<const gqg_tensor *, DeltaStep> steps;                     // GATED_DELTA_NET nodes
    std::unordered_map<const gqg_tensor *, const gqg_tensor *> silu_written;     // GEMV -> the SiLU it writes
    std::unordered_map<const gqg_tensor *, std::pair<const gqg_tensor *, const gqg_tensor *>> glu_pairs;  // GLU -> g, u
    std::unordered_set<const gqg_tensor *> add_epilog;   // GEMVs whose one reader, an ADD, becomes their epilog
    std::unordered_set<const gqg_tensor *> adds_taken;   // those ADDs
    std::unordered_set<const gqg_tensor *> deferred;     // norm rows read only by GEMVs (never written)
    std::unordered_map<const gqg_tensor *, AttnChain> attn_by_gate;  // the gate MUL closing an attention
    int readers(const gqg_tensor * t) const { return ix.readers(t); }
    void absorb(std::initializer_list<const gqg_tensor *> ts) { absorbed.insert(ts); }
};

bool match_conv(FusionPlan & F, const gqg_tensor * c, std::string & err) {
    ConvChain cc;
    cc.conv = c;
    cc.window = c->src[0];
    const bool concat = cc.window && cc.window->op == GQG_OP_CONCAT;
    if (concat) {
        cc.state_rows = rs_rows(cc.window->src[0]);
        cc.input = cc.window->src[1];
        // the new window: the last three columns of the concatenation (a view one float in) copied into the state
        const auto * st = F.ix.first(cc.window, [](const ReaderIndex::Read & r) {
            return r.node->op == GQG_OP_CPY && r.slot == 0 && r.via->view_offs == 4 && in_buf(r.node->src[1], GQG_BUF_RS);
        });
        cc.store = st ? st->node : nullptr;
    }
    const auto * sr = F.ix.first(c, [c](const ReaderIndex::Read & r) { return unary_kind(r.node) == 1 && r.node->src[0] == c; });
    const gqg_tensor * silu = sr ? sr->node : nullptr;
    if (!concat || !cc.state_rows || !cc.store || !silu || !f32_weight(c->src[1]) || c->ne[0] % 16 ||
        cc.window->ne[0] != 4 || cc.window->ne[1] != c->ne[0]) {
        err = std::string("conv ") + c->name + ": not the state-window CONCAT, SSM_CONV, SiLU and state CPY of one token";
        return false;
    }
    F.conv_by_silu[silu] = cc;
    F.absorb({cc.state_rows, cc.window, cc.store, c});
    // its input straight from a GEMV of this split that nothing else reads: the CONV becomes that GEMV's epilog
    const gqg_tensor * x = root_of(cc.input);
    if (x->op == GQG_OP_MUL_MAT && F.ix.in_split(x) && F.ix.sole(x) && x->ne[0] == c->ne[0]) F.conv_input_gemv[x] = silu;
    return true;
}

// The gated output norm after the step: RMS_NORM over rows of 128 of the step's output -> MUL by a 128-float weight ->
// MUL by SILU(z), each read by the next alone; the step read by that norm and its state CPY only.
void match_gated_norm(FusionPlan & F, const gqg_tensor * node, DeltaStep & p) {
    const gqg_tensor * v = node->src[2];
    const auto * nr = F.ix.first(node, [&](const ReaderIndex::Read & r) {
        const gqg_tensor * m = r.node;
        return m->op == GQG_OP_RMS_NORM && r.slot == 0 && r.via->view_offs == 0 && m->ne[0] == HEAD && nel(m) == nel(v);
    });
    const gqg_tensor * norm = nr ? nr->node : nullptr;
    if (!norm || F.readers(node) != 2) return;
    const gqg_tensor * mw = F.ix.sole(norm);
    if (!mw || mw->op != GQG_OP_MUL || mw->src[0] != norm) return;
    const gqg_tensor * mz = F.ix.sole(mw);
    if (!mz || mz->op != GQG_OP_MUL || mz->src[0] != mw) return;
    const gqg_tensor * w = mw->src[1], * sl = mz->src[1];
    if (!f32_weight(w) || nel(w) != HEAD || unary_kind(sl) != 1 || F.ix.sole(sl) != mz || nel(sl) != nel(mz) ||
        nel(mz) != nel(norm) || !contiguous(sl->src[0]) || !contiguous(mz))
        return;
    p.gated = mz;
    p.norm_w = w;
    p.rms_eps = pf(norm, 0);
    F.absorb({norm, mw, mz, sl});
    // z = silu(GEMV output) where that GEMV feeds the SiLU alone: the GEMV writes silu(z) (its SiLU epilog) once
    const gqg_tensor * zg = root_of(sl->src[0]);
    if (zg->op == GQG_OP_MUL_MAT && F.ix.in_split(zg) && F.ix.sole(zg) && sl->src[0]->data == zg->data && nel(zg) == nel(sl)) {
        F.silu_written[zg] = sl;
        p.gate = sl;
        p.gate_silu = true;
    } else {
        p.gate = sl->src[0];
    }
}

// The gates: SIGMOID(beta raw) and MUL(SOFTPLUS(ADD(alpha raw, dt)), a), every link read by the next alone, dt and a
// weights of one float per value head.
void match_gates(FusionPlan & F, const gqg_tensor * node, DeltaStep & p) {
    const int64_t hv = node->src[2]->ne[1];
    const gqg_tensor * sig = root_of(node->src[4]), * mul = root_of(node->src[3]);
    const auto head_weight = [hv](const gqg_tensor * x) { return x && f32_weight(x) && nel(x) == hv; };
    const auto head_row = [hv](const gqg_tensor * x) { return x->type == GQG_TYPE_F32 && contiguous(x) && nel(x) == hv; };
    if (unary_kind(sig) != 2 || F.ix.sole(sig) != node || mul->op != GQG_OP_MUL || F.ix.sole(mul) != node ||
        !head_row(sig->src[0]))
        return;
    const bool sp_first = mul->src[0]->op == GQG_OP_UNARY;
    const gqg_tensor * sp = mul->src[sp_first ? 0 : 1], * a = mul->src[sp_first ? 1 : 0];
    if (unary_kind(sp) != 3 || F.ix.sole(sp) != mul || !head_weight(a)) return;
    const gqg_tensor * add = sp->src[0];
    if (add->op != GQG_OP_ADD || F.ix.sole(add) != sp) return;
    const bool dt_second = head_weight(add->src[1]);
    const gqg_tensor * dt = add->src[dt_second ? 1 : 0], * alpha = add->src[dt_second ? 0 : 1];
    if (!head_weight(dt) || !head_row(alpha)) return;
    p.beta = sig->src[0];
    p.alpha = alpha;
    p.dt = dt;
    p.a = a;
    F.absorb({sig, mul, sp, add});
}

bool match_step(FusionPlan & F, const gqg_tensor * node, std::string & err) {
    DeltaStep p;
    p.state_rows = rs_rows(node->src[5]);
    const size_t y_bytes = size_t(node->src[2]->ne[1]) * HEAD * 4;  // the new state follows the outputs
    const auto * st = F.ix.first(node, [y_bytes](const ReaderIndex::Read & r) {
        return r.node->op == GQG_OP_CPY && r.slot == 0 && r.via->view_offs == y_bytes && in_buf(r.node->src[1], GQG_BUF_RS);
    });
    p.store = st ? st->node : nullptr;
    if (!p.state_rows || !p.store) {
        err = std::string("DeltaNet step ") + node->name + ": no state row read from, or new state copied to, a state buffer";
        return false;
    }
    F.absorb({p.state_rows, p.store});
    const gqg_tensor * q = node->src[0], * k = node->src[1];
    if (q->op == GQG_OP_L2_NORM && k->op == GQG_OP_L2_NORM && F.ix.sole(q) == node && F.ix.sole(k) == node &&
        contiguous(q->src[0]) && contiguous(k->src[0]) && q->op_params[0] == k->op_params[0]) {
        p.l2 = true;
        p.l2_eps = pf(q, 0);
        F.absorb({q, k});
    }
    match_gated_norm(F, node, p);
    match_gates(F, node, p);
    F.steps[node] = p;
    return true;
}

// ROPE(MUL(RMS_NORM(rows), weight)) -> the rows, the weight and the norm's eps
bool rope_of_norm(const gqg_tensor * rope, const gqg_tensor *& rows, const gqg_tensor *& w, float & eps) {
    if (!rope || rope->op != GQG_OP_ROPE) return false;
    const gqg_tensor * mw = rope->src[0];
    if (!mw || mw->op != GQG_OP_MUL || !mw->src[0] || mw->src[0]->op != GQG_OP_RMS_NORM || !f32_weight(mw->src[1]))
        return false;
    rows = mw->src[0]->src[0];
    w = mw->src[1];
    eps = pf(mw->src[0], 0);
    return true;
}

bool match_attention(FusionPlan & F, const gqg_tensor * fa, std::string & err) {
    AttnChain at;
    at.fa = fa;
    at.scale = pf(fa, 0);
    const gqg_tensor * kc = root_of(fa->src[1]), * vc = root_of(fa->src[2]);
    const gqg_tensor * qrope = through_views(fa->src[0]);
    const gqg_tensor * qrows = nullptr, * krows = nullptr;
    float qeps = 0.0f, keps = 0.0f;
    const auto store_into = [&](const gqg_tensor * cache) {
        const auto * r = F.ix.first(cache, [cache](const ReaderIndex::Read & x) {
            return x.node->op == GQG_OP_SET_ROWS && x.slot == 0 && root_of(x.node->src[0]) == cache;
        });
        return r ? r->node : nullptr;
    };
    bool ok = in_buf(kc, GQG_BUF_KV) && in_buf(vc, GQG_BUF_KV) && rope_of_norm(qrope, qrows, at.q_norm_w, qeps);
    if (ok) {
        at.k_store = store_into(kc);
        at.v_store = store_into(vc);
    }
    const gqg_tensor * krope = ok && at.k_store ? through_views(at.k_store->src[1]) : nullptr;
    ok = ok && at.v_store && rope_of_norm(krope, krows, at.k_norm_w, keps) && qeps == keps;
    if (ok) {
        at.eps = qeps;
        at.q_proj = root_of(qrows);
        at.k_proj = root_of(krows);
        at.v_proj = root_of(at.v_store->src[1]);
        at.head_dim = int(qrows->ne[0]);
        at.n_head = int(qrows->ne[1]);
        at.n_head_kv = int(krows->ne[1] > 1 ? krows->ne[1] : nel(krows) / at.head_dim);
        at.n_rot = qrope->op_params[1];
        at.base = pf(qrope, 5);
        at.pos = qrope->src[1];
        at.k_row = at.k_store->src[2];
        const bool neox = qrope->op_params[2] == GQG_ROPE_TYPE_NEOX && krope->op_params[2] == GQG_ROPE_TYPE_NEOX;
        const bool same_rope = krope->op_params[1] == at.n_rot && pf(krope, 5) == at.base && krope->src[1] == at.pos;
        const bool plain_rope = pf(qrope, 6) == 1.0f && pf(qrope, 7) == 0.0f && pf(qrope, 8) == 1.0f;  // no YaRN
        const bool q_gate_rows = qrows->view_offs == 0 && qrows->nb[0] == 4 && qrows->nb[1] == size_t(2 * at.head_dim) * 4 &&
                                 nel(at.q_proj) == int64_t(2) * at.head_dim * at.n_head;
        ok = at.q_proj->op == GQG_OP_MUL_MAT && at.k_proj->op == GQG_OP_MUL_MAT && at.v_proj->op == GQG_OP_MUL_MAT &&
             nel(at.v_proj) == nel(at.k_proj) && q_gate_rows && neox && same_rope && plain_rope &&
             at.pos->type == GQG_TYPE_I32 && nel(at.pos) == 1 && at.k_row->type == GQG_TYPE_I64 && nel(at.k_row) == 1 &&
             at.v_store->src[2] == at.k_row;
    }
    // the output gate: MUL(the output, SIGMOID(CONT(the gate rows of q, head_dim floats in))), the output read there alone
    const auto * gr = ok ? F.ix.first(fa, [fa](const ReaderIndex::Read & r) {
        return r.node->op == GQG_OP_MUL && root_of(r.node->src[0]) == fa;
    }) : nullptr;
    const gqg_tensor * gmul = gr ? gr->node : nullptr;
    const gqg_tensor * sig = gmul ? gmul->src[1] : nullptr;
    const gqg_tensor * grow = sig && unary_kind(sig) == 2 && sig->src[0]->op == GQG_OP_CONT ? sig->src[0]->src[0] : nullptr;
    ok = ok && gmul && grow && root_of(grow) == at.q_proj && grow->view_offs == size_t(at.head_dim) * 4 &&
         grow->nb[1] == size_t(2 * at.head_dim) * 4 && nel(gmul) == int64_t(at.n_head) * at.head_dim &&
         F.readers(fa) == 1 && unfused_output(fa);
    if (!ok) {
        err = std::string("attention ") + fa->name + ": not the one-token gated attention of a KV buffer of this backend";
        return false;
    }
    const std::string cname = root_of(at.k_store->src[0])->name;  // cache_k_l<N>: the layer is what follows cache_k_
    at.layer = cname.size() > 7 ? cname.substr(7) : cname;
    F.attn_by_gate[gmul] = at;
    F.absorb({qrope, qrope->src[0], qrope->src[0]->src[0], krope, krope->src[0], krope->src[0]->src[0], at.k_store,
              at.v_store, fa, sig, sig->src[0]});
    return true;
}

// GLU(g, u) of two GEMVs on the same row, each read by the GLU alone: a SwiGLU pair (gemvqc16.cpp:224-243).
void match_glu(FusionPlan & F, const gqg_tensor * m) {
    if (m->op_params[0] != GQG_GLU_SWIGLU || m->op_params[1] != 0) return;
    const gqg_tensor * g = m->src[0], * u = m->src[1];
    const auto lone_gemv = [&](const gqg_tensor * x) {
        return x && x->op == GQG_OP_MUL_MAT && F.ix.in_split(x) && F.ix.sole(x) == m;
    };
    if (!lone_gemv(g) || !lone_gemv(u) || g->src[1]->data != u->src[1]->data || g->src[0]->ne[0] != u->src[0]->ne[0] ||
        g->ne[0] != u->ne[0] || g->ne[0] != m->ne[0] || g->src[0]->type != u->src[0]->type)
        return;
    F.glu_pairs[m] = {g, u};
    F.absorb({g, u});
}

// A GEMV read only by an ADD of its own length, whose other operand exists before the GEMV runs: the ADD becomes the
// GEMV's epilog (gemvqc16.cpp:282-301). The GEMV's place in the row must be the ADD operand itself.
void match_add_epilog(FusionPlan & F, const gqg_tensor * m) {
    if (F.silu_written.count(m) || F.conv_input_gemv.count(m)) return;
    const gqg_tensor * add = F.ix.sole(m);
    if (!add || add->op != GQG_OP_ADD || F.absorbed.count(add) || F.adds_taken.count(add)) return;
    if (nel(m) != nel(add) || m->ne[0] < 256 || m->ne[0] % 16) return;
    for (int s = 0; s < 2; ++s) {
        if (root_of(add->src[s]) != m || add->src[s]->data != m->data) continue;
        const gqg_tensor * other = root_of(add->src[1 - s]);
        if (other == m || (F.ix.in_split(other) && F.ix.at.at(other) > F.ix.at.at(m))) return;
        F.add_epilog.insert(m);
        F.adds_taken.insert(add);
        return;
    }
}

// A norm row (RMS_NORM, or the MUL by its weight) that only GEMVs of this split read, as their activation: the
// deferred RMSNORM (gemvqc16.h:46-51), folded into their quantization and never written.
void match_deferred(FusionPlan & F, const gqg_tensor * r) {
    if (!unfused_output(r) || nel(r) != r->ne[0] || r->ne[0] % 16 || r->ne[0] > 16384) return;
    const auto it = F.ix.reads.find(r);
    if (it == F.ix.reads.end() || it->second.empty()) return;
    for (const auto & x : it->second)
        if (x.node->op != GQG_OP_MUL_MAT || x.slot != 1) return;
    F.deferred.insert(r);
}

bool plan_fusions(const gqg_cgraph * g, FusionPlan & F, std::string & err) {
    F.ix.build(g);
    for (int i = g->n_nodes - 1; i >= 0; --i) {
        const gqg_tensor * t = g->nodes[i];
        if (is_view(t) || F.absorbed.count(t)) continue;
        switch (t->op) {
        case GQG_OP_SSM_CONV:
            if (!match_conv(F, t, err)) return false;
            break;
        case GQG_OP_GATED_DELTA_NET:
            if (!match_step(F, t, err)) return false;
            break;
        case GQG_OP_FLASH_ATTN_EXT:
            if (!match_attention(F, t, err)) return false;
            break;
        case GQG_OP_GLU: match_glu(F, t); break;
        case GQG_OP_MUL_MAT: match_add_epilog(F, t); break;
        case GQG_OP_RMS_NORM:
        case GQG_OP_MUL: match_deferred(F, t); break;
        default: break;
        }
    }
    return true;
}

// ---- the plan cache key: a structural signature of the split ----
// Every node contributes its operation, types, flags, buffer, shape, strides, parameters, data address and view
// offset, and for each operand (and its view source) a reference: the producing node's position in the split, or an
// entry of a table of the tensors read from outside the split (weights, inputs, states), each described once with
// the same fields, its name and its own address (weights are uploaded once per tensor). A state GET_ROWS adds the
// row it selects (the command's state rows depend on it). Plans are found by a 64-bit mix of the signature and
// confirmed by comparing it whole.
struct Signature {
    std::vector<uint64_t> words;
    uint64_t hash = 0;
};

uint64_t mix64(uint64_t h) {  // a finalizer with full avalanche (the SplitMix64 one)
    h ^= h >> 30;
    h *= 0xbf58476d1ce4e5b9ull;
    h ^= h >> 27;
    h *= 0x94d049bb133111ebull;
    return h ^ (h >> 31);
}

struct SignatureBuilder {
    const ReaderIndex & ix;
    std::vector<uint64_t> & w;
    std::unordered_map<const gqg_tensor *, uint64_t> outside;
    std::vector<const gqg_tensor *> outside_order;

    uint64_t ref(const gqg_tensor * t) {
        if (!t) return 0;
        const auto n = ix.at.find(t);
        if (n != ix.at.end()) return (1ull << 62) | uint64_t(n->second);
        const auto o = outside.find(t);
        if (o != outside.end()) return o->second;
        const uint64_t id = (2ull << 62) | uint64_t(outside.size());
        outside[t] = id;
        outside_order.push_back(t);
        return id;
    }
    void fields(const gqg_tensor * t) {
        w.push_back(uint64_t(uint32_t(t->op)) | uint64_t(uint32_t(t->type)) << 16 | uint64_t(uint32_t(t->buffer)) << 32 |
                    uint64_t(uint32_t(t->flags) & 0xffffu) << 48);
        for (int d = 0; d < GQG_MAX_DIMS; ++d) w.push_back(uint64_t(t->ne[d]) ^ (uint64_t(t->nb[d]) << 40) ^ (uint64_t(t->nb[d]) >> 24));
        for (int k = 0; k < GQG_MAX_OP_PARAMS; k += 2)
            w.push_back(uint64_t(uint32_t(t->op_params[k])) | uint64_t(uint32_t(t->op_params[k + 1])) << 32);
        w.push_back(uint64_t(reinterpret_cast<uintptr_t>(t->data)));
        w.push_back(uint64_t(t->view_offs));
        w.push_back(ref(t->view_src));
    }
};

void signature_of(const gqg_cgraph * g, const ReaderIndex & ix, Signature & s) {
    s.words.clear();
    SignatureBuilder b{ix, s.words, {}, {}};
    s.words.push_back(uint64_t(g->n_nodes));
    for (int i = 0; i < g->n_nodes; ++i) {
        const gqg_tensor * t = g->nodes[i];
        b.fields(t);
        for (int k = 0; k < GQG_MAX_SRC; ++k) s.words.push_back(b.ref(t->src[k]));
        if (t->op == GQG_OP_GET_ROWS && in_buf(t->src[0], GQG_BUF_RS) && t->src[1]->data)
            s.words.push_back(uint64_t(uint32_t(*static_cast<const int32_t *>(t->src[1]->data))));
    }
    // the outside tensors, in order of first reference (describing one may add its view source)
    for (size_t i = 0; i < b.outside_order.size(); ++i) {
        const gqg_tensor * t = b.outside_order[i];
        s.words.push_back(uint64_t(reinterpret_cast<uintptr_t>(t)));
        b.fields(t);
        uint64_t nh = 0xcbf29ce484222325ull;  // FNV-1a of the name
        for (const char * c = t->name; *c && c < t->name + sizeof(t->name); ++c) nh = (nh ^ uint8_t(*c)) * 0x100000001b3ull;
        s.words.push_back(nh);
    }
    uint64_t h = 0x9e3779b97f4a7c15ull;
    for (uint64_t v : s.words) h = mix64(h ^ v);
    s.hash = h;
}

// ---- emission ----

struct Emitter {
    gqg_backend * b;
    const gqg_cgraph * g;
    const FusionPlan & F;
    gqg_backend::Plan & P;
    std::string err;
    size_t used = 64;  // transient region bump pointer
    struct Region { const uint8_t * lo; size_t bytes; uint32_t off; };
    std::vector<Region> outs, ins;  // produced roots; host inputs
    std::unordered_map<const gqg_tensor *, size_t> add_at, conv_at;  // GEMV command word (ADD / CONV epilog)
    std::unordered_map<const gqg_tensor *, size_t> deferred_at;
    const gqg_tensor * last_deferred = nullptr;
    std::unordered_set<const gqg_tensor *> fused_silu, fused_sigmoid;  // UNARY nodes emitted with the MUL after them

    void push(std::initializer_list<uint32_t> w) {
        size_t k = 0;
        for (uint32_t v : w) {
            P.words.push_back(v);
            ++k;
        }
        for (; k < GEMVQ_CMD_WORDS; ++k) P.words.push_back(0);
    }
    void insert_after(size_t at, const uint32_t (&cmd)[GEMVQ_CMD_WORDS]) {
        const size_t pos = at + GEMVQ_CMD_WORDS;
        P.words.insert(P.words.begin() + long(pos), cmd, cmd + GEMVQ_CMD_WORDS);
        for (auto * m : {&add_at, &conv_at, &deferred_at})
            for (auto & e : *m)
                if (e.second >= pos) e.second += GEMVQ_CMD_WORDS;
    }
    void undefer(const gqg_tensor * t) {
        const auto it = deferred_at.find(t);
        if (it == deferred_at.end()) return;
        P.words[it->second + 7] &= ~GEMVQ_NORM_DEFER;
        deferred_at.erase(it);
        if (last_deferred == t) last_deferred = nullptr;
    }
    bool take(size_t floats, uint32_t & off) {
        if (used + up16(floats) > b->trans_end) {
            err = "transient act region full";
            return false;
        }
        off = uint32_t(used);
        used += up16(floats);
        return true;
    }
    // act offset of the output of node t (its data root gets a fresh region)
    bool output(const gqg_tensor * t, uint32_t & off) {
        const gqg_tensor * r = root_of(t);
        for (const auto & o : outs)
            if (o.lo == r->data) {
                off = o.off + uint32_t((static_cast<const uint8_t *>(t->data) - o.lo) / 4);
                return true;
            }
        const size_t bytes = size_t(nel(r)) * 4;
        if (!take(bytes / 4, off)) return false;
        outs.push_back({static_cast<const uint8_t *>(r->data), bytes, off});
        if (!unfused_output(r)) P.out.push_back({r->data, off, bytes / 4});
        off += uint32_t((static_cast<const uint8_t *>(t->data) - static_cast<const uint8_t *>(r->data)) / 4);
        return true;
    }
    // act offset of an operand: a produced result, a resident F32 weight, a state buffer row, or a host input
    bool operand(const gqg_tensor * t, size_t floats, uint32_t & off) {
        const gqg_tensor * r = root_of(t);
        const auto * lo = static_cast<const uint8_t *>(t->data);
        const auto aligned = [&](size_t within) {
            if (within % 64) {
                err = std::string("operand ") + t->name + " is not 16-float aligned";
                return false;
            }
            return true;
        };
        for (const auto & o : outs)
            if (lo >= o.lo && lo + floats * 4 <= o.lo + o.bytes) {
                if (!aligned(size_t(lo - o.lo))) return false;
                off = o.off + uint32_t((lo - o.lo) / 4);
                return true;
            }
        if (r->buffer == GQG_BUF_WEIGHTS && r->type == GQG_TYPE_F32) {
            uint32_t base;
            if (!const_of(b, r, base, err)) return false;
            const size_t within = size_t(lo - static_cast<const uint8_t *>(r->data));
            if (!aligned(within)) return false;
            off = base + uint32_t(within / 4);
            return true;
        }
        if (r->buffer == GQG_BUF_RS) {
            err = std::string("state tensor ") + t->name + " read outside a conv or GDN step";
            return false;
        }
        for (const auto & in : ins)
            if (lo >= in.lo && lo + floats * 4 <= in.lo + in.bytes) {
                off = in.off + uint32_t((lo - in.lo) / 4);
                return true;
            }
        if (!take(floats, off)) return false;
        ins.push_back({lo, floats * 4, off});
        P.in.push_back({lo, off, floats});
        return true;
    }
    // the state rows or resident offset of an RS tensor range
    bool rs_at(const gqg_tensor * t, const void * data, bool & state, size_t & dev) {
        for (gqg_buffer * buf : b->buffers) {
            if (buf->kind != GQG_BUF_RS) continue;
            const gqg_buffer::Entry * e = buf->find(data);
            if (!e) continue;
            const size_t within = size_t(static_cast<const uint8_t *>(data) - buf->base) - e->off;
            state = e->state;
            if (state) {
                if (within % 512) break;
                dev = e->dev + within / 512;
            } else {
                if (within % 64) break;
                dev = e->dev + within / 4;
            }
            return true;
        }
        err = std::string("state tensor ") + t->name + " is not placed in a state buffer of this backend";
        return false;
    }
    // host data of the one sequence id a state GET_ROWS selects
    const void * state_row(const gqg_tensor * gr) {
        const int32_t id = gr->src[1]->data ? *static_cast<const int32_t *>(gr->src[1]->data) : 0;
        return static_cast<const uint8_t *>(gr->src[0]->data) + size_t(id) * gr->src[0]->nb[1];
    }

    bool gemv(const gqg_tensor * m, uint32_t x, uint32_t y, uint32_t flags) {
        uint64_t w;
        if (!upload_weight(b, m->src[0], w, err)) return false;
        push({GEMVQ_OP_GEMV, uint32_t(m->src[0]->type) | flags, uint32_t(m->src[0]->ne[1]), uint32_t(m->src[0]->ne[0]),
              uint32_t(w), uint32_t(w >> 32), x, y});
        return true;
    }

    bool run() {
        const int n = g->n_nodes;
        for (int i = 0; i < n; ++i) {
            const gqg_tensor * node = g->nodes[i];
            if (is_view(node) || F.absorbed.count(node) || nel(node) == 0) continue;
            const size_t ne = size_t(nel(node));
            const gqg_tensor * a = node->src[0], * bsrc = node->src[1];
            const gqg_tensor * next = i + 1 < n ? g->nodes[i + 1] : nullptr;
            switch (node->op) {
            case GQG_OP_MUL_MAT: {
                if (!quant_type(a->type) || !token_row(bsrc) || nel(bsrc) != a->ne[0]) {
                    err = std::string("MUL_MAT ") + node->name + ": not a quantized GEMV on one row";
                    return false;
                }
                if (root_of(bsrc) != last_deferred) undefer(root_of(bsrc));
                uint32_t x, y;
                if (!operand(bsrc, size_t(a->ne[0]), x)) return false;
                const auto se = F.silu_written.find(node);
                if (!output(se != F.silu_written.end() ? se->second : node, y)) return false;
                if (F.add_epilog.count(node)) add_at[node] = P.words.size();
                if (F.conv_input_gemv.count(node)) conv_at[node] = P.words.size();
                if (!gemv(node, x, y, se != F.silu_written.end() ? GEMVQ_GEMV_SILU : 0u)) return false;
                break;
            }
            case GQG_OP_RMS_NORM:
            case GQG_OP_L2_NORM:
            case GQG_OP_MUL: {
                const gqg_tensor * norm = node->op == GQG_OP_MUL ? a : node;
                const bool weight_mul = node->op == GQG_OP_MUL && a->op == GQG_OP_RMS_NORM && i > 0 && g->nodes[i - 1] == a &&
                                        F.readers(a) == 1 && nel(bsrc) == node->ne[0] && f32_weight(bsrc);
                if (node->op == GQG_OP_RMS_NORM && next && next->op == GQG_OP_MUL && next->src[0] == node &&
                    F.readers(node) == 1 && nel(next->src[1]) == node->ne[0] && f32_weight(next->src[1]))
                    break;  // emitted with the weight MUL
                if (node->op != GQG_OP_MUL || weight_mul) {
                    const uint32_t row = uint32_t(norm->ne[0]), rows = uint32_t(ne / row);
                    const gqg_tensor * nx = norm->src[0];
                    const bool strided = !token_row(nx);
                    if (strided && !strided_rows(nx)) {
                        err = std::string("norm ") + node->name + ": rows neither packed nor strided by 64 bytes";
                        return false;
                    }
                    const uint32_t stride_words = strided ? uint32_t(nx->nb[1] / 64) : 0u;
                    uint32_t x, w = 0, y;
                    const size_t span = strided ? size_t(nx->nb[1] / 4) * (rows - 1) + row : ne;
                    if (!operand(nx, span, x) || (weight_mul && !operand(bsrc, row, w)) || !output(node, y)) return false;
                    const uint32_t flags = (norm->op == GQG_OP_L2_NORM ? GEMVQ_NORM_L2 : 0u) |
                                           (weight_mul ? 0u : GEMVQ_NORM_NO_WEIGHT);
                    const bool defer = rows == 1 && !strided && F.deferred.count(node);
                    if (defer) {
                        deferred_at[node] = P.words.size();
                        last_deferred = node;
                    }
                    push({GEMVQ_OP_RMSNORM, row, x, w, y, fbits(pf(norm, 0)), rows,
                          flags | (defer ? GEMVQ_NORM_DEFER : 0u) | (stride_words << 8)});
                    break;
                }
                if (nel(bsrc) != nel(node)) {
                    err = std::string("broadcast MUL ") + node->name + " is not the weight of the preceding norm";
                    return false;
                }
                const auto at = F.attn_by_gate.find(node);
                if (at != F.attn_by_gate.end()) {
                    if (!attention(node, at->second)) return false;
                    break;
                }
                const bool silu = fused_silu.count(bsrc) != 0, sig = fused_sigmoid.count(bsrc) != 0;
                const gqg_tensor * gsrc = silu || sig ? bsrc->src[0] : bsrc;
                uint32_t go, xo, y;
                if (!operand(gsrc, ne, go) || !operand(a, ne, xo) || !output(node, y)) return false;
                if (silu) push({GEMVQ_OP_SILU_MUL, uint32_t(ne), go, xo, y});
                else if (sig) push({GEMVQ_OP_SILU_MUL, uint32_t(ne), go, xo, y, GEMVQ_SILU_MUL_SIGMOID});
                else push({GEMVQ_OP_MUL, uint32_t(ne), xo, go, y});
                break;
            }
            case GQG_OP_ADD:
            case GQG_OP_GLU: {
                const auto sw = F.glu_pairs.find(node);
                if (sw != F.glu_pairs.end()) {
                    const gqg_tensor * gt = sw->second.first, * ut = sw->second.second, * x = gt->src[1];
                    if (!quant_type(gt->src[0]->type) || !token_row(x)) {
                        err = std::string("SwiGLU pair ") + node->name + ": not quantized GEMVs on one row";
                        return false;
                    }
                    if (root_of(x) != last_deferred) undefer(root_of(x));
                    uint32_t xo, y;
                    if (!operand(x, size_t(gt->src[0]->ne[0]), xo) || !output(node, y)) return false;
                    if (!gemv(gt, xo, y, GEMVQ_GEMV_SWIGLU) || !gemv(ut, xo, y, 0)) return false;
                    break;
                }
                if (node->op == GQG_OP_GLU) {
                    err = std::string("GLU ") + node->name + " is not a SwiGLU pair of GEMVs";
                    return false;
                }
                if (!token_row(a) || !token_row(bsrc) || nel(a) != nel(bsrc)) {
                    err = std::string("ADD ") + node->name + ": operands are not rows of its length";
                    return false;
                }
                uint32_t ao, bo, y;
                if (!operand(a, ne, ao) || !operand(bsrc, ne, bo) || !output(node, y)) return false;
                bool fused = false;
                for (int s = 0; s < 2 && !fused; ++s) {
                    const auto it = add_at.find(root_of(node->src[s]));
                    if (it == add_at.end() || P.words[it->second + 7] != (s ? bo : ao)) continue;
                    const size_t at = it->second;
                    add_at.erase(it);
                    P.words[at + 1] |= GEMVQ_GEMV_ADD;
                    const uint32_t cmd[GEMVQ_CMD_WORDS] = {GEMVQ_OP_ADD, uint32_t(ne), ao, bo, y, 0, 0, 0};
                    insert_after(at, cmd);
                    fused = true;
                }
                if (!fused) push({GEMVQ_OP_ADD, uint32_t(ne), ao, bo, y});
                break;
            }
            case GQG_OP_UNARY: {
                const auto cv = F.conv_by_silu.find(node);
                if (cv != F.conv_by_silu.end()) {
                    if (!conv(node, cv->second)) return false;
                    break;
                }
                const int kind = unary_kind(node);
                if (!kind || !token_row(node)) {
                    err = std::string("UNARY ") + node->name + ": unsupported";
                    return false;
                }
                if ((kind == 1 || kind == 2) && next && next->op == GQG_OP_MUL && next->src[1] == node &&
                    next->src[0] != node && F.readers(node) == 1 && nel(next) == nel(node) && token_row(a)) {
                    (kind == 1 ? fused_silu : fused_sigmoid).insert(node);  // emitted with the MUL
                    break;
                }
                const gqg_tensor * x = a->op == GQG_OP_CONT && strided_rows(a->src[0]) && F.readers(a) == 1 ? a->src[0] : a;
                const bool strided = x != a;
                if (!strided && !token_row(x)) {
                    err = std::string("UNARY ") + node->name + ": input rows";
                    return false;
                }
                const uint32_t row = strided ? uint32_t(x->ne[0]) : 0u, stride = strided ? uint32_t(x->nb[1] / 4) : 0u;
                uint32_t xo, y;
                const size_t span = strided ? size_t(stride) * (ne / row - 1) + row : ne;
                if (!operand(x, span, xo) || !output(node, y)) return false;
                push({GEMVQ_OP_UNARY, uint32_t(ne), xo, uint32_t(kind), y, row, stride});
                break;
            }
            case GQG_OP_CONT: {
                if (!strided_rows(a)) {
                    err = std::string("CONT ") + node->name + ": not strided rows";
                    return false;
                }
                const uint32_t row = uint32_t(a->ne[0]), stride = uint32_t(a->nb[1] / 4);
                uint32_t xo, y;
                if (!operand(a, size_t(stride) * (ne / row - 1) + row, xo) || !output(node, y)) return false;
                push({GEMVQ_OP_UNARY, uint32_t(ne), xo, 4u, y, row, stride});
                break;
            }
            case GQG_OP_GATED_DELTA_NET:
                if (!gdn(node, F.steps.at(node))) return false;
                break;
            case GQG_OP_GET_ROWS: {
                const gqg_tensor * w = a, * ids = bsrc;
                if (!quant_type(w->type) && w->type != GQG_TYPE_F32) {
                    err = std::string("GET_ROWS ") + node->name + ": type";
                    return false;
                }
                if (!quant_type(w->type) || ids->type != GQG_TYPE_I32 || nel(ids) != 1 || !is_weight(w)) {
                    err = std::string("GET_ROWS ") + node->name + ": one row of a quantized weight by an I32 id";
                    return false;
                }
                uint64_t wo;
                uint32_t io, y;
                if (!upload_weight(b, w, wo, err) || !operand(ids, 1, io) || !output(node, y)) return false;
                push({GEMVQ_OP_GET_ROWS, uint32_t(w->type), uint32_t(w->ne[1]), uint32_t(w->ne[0]), uint32_t(wo),
                      uint32_t(wo >> 32), io, y});
                break;
            }
            default:
                err = std::string("node ") + node->name + " (op " + std::to_string(node->op) + ") has no command";
                return false;
            }
        }
        // deferred norms whose rows a graph output or split output asks for are written after all
        std::vector<const gqg_tensor *> needed;
        for (const auto & d : deferred_at)
            if (!unfused_output(d.first)) needed.push_back(d.first);
        for (const auto * t : needed) undefer(t);
        return true;
    }

    bool conv(const gqg_tensor * silu, const ConvChain & cv) {
        const uint32_t ch = uint32_t(cv.conv->ne[0]);
        bool st;
        size_t s_src, s_dst;
        if (!rs_at(cv.state_rows, state_row(cv.state_rows), st, s_src) || !rs_at(cv.store->src[1], cv.store->src[1]->data, st, s_dst))
            return false;
        uint32_t xo, wo, y;
        if (!operand(cv.input, ch, xo) || !operand(cv.conv->src[1], size_t(ch) * 4, wo) || !output(silu, y)) return false;
        const uint32_t cmd[GEMVQ_CMD_WORDS] = {GEMVQ_OP_CONV, ch, xo, wo, y, uint32_t(s_src), uint32_t(s_dst), 1u};
        const auto it = conv_at.find(root_of(cv.input));
        if (it != conv_at.end() && P.words[it->second + 7] == xo) {
            P.words[it->second + 1] |= GEMVQ_GEMV_CONV;  // the CONV right behind the GEMV of its input
            insert_after(it->second, cmd);
            conv_at.erase(it);
        } else {
            P.words.insert(P.words.end(), cmd, cmd + GEMVQ_CMD_WORDS);
        }
        return true;
    }

    bool gdn(const gqg_tensor * node, const DeltaStep & p) {
        const gqg_tensor * q = node->src[0], * k = node->src[1], * v = node->src[2];
        const uint32_t hv = uint32_t(v->ne[1]), hk = uint32_t(q->ne[1]);
        bool st_src, st_dst;
        size_t src_row, dst_row;
        if (!rs_at(p.state_rows, state_row(p.state_rows), st_src, src_row) || !rs_at(p.store->src[1], p.store->src[1]->data, st_dst, dst_row))
            return false;
        if (!st_src || !st_dst) {
            err = std::string("GDN state of ") + node->name + " is not on state rows";
            return false;
        }
        const gqg_tensor * qi = p.l2 ? q->src[0] : q, * ki = p.l2 ? k->src[0] : k;
        const bool gates = p.alpha != nullptr;
        const gqg_tensor * gi = gates ? p.alpha : node->src[3], * bi = gates ? p.beta : node->src[4];
        uint32_t qo, ko, vo, go, bo, wo = 0, zo = 0, dto = 0, ao = 0, y;
        if (!operand(qi, size_t(hk) * HEAD, qo) || !operand(ki, size_t(hk) * HEAD, ko) || !operand(v, size_t(hv) * HEAD, vo) ||
            !operand(gi, hv, go) || !operand(bi, hv, bo))
            return false;
        if (p.gated && (!operand(p.norm_w, HEAD, wo) || !operand(p.gate, size_t(hv) * HEAD, zo))) return false;
        if (gates && (!operand(p.dt, hv, dto) || !operand(p.a, hv, ao))) return false;
        if (!output(p.gated ? p.gated : node, y)) return false;
        const uint32_t flags = (p.l2 ? GEMVQ_GDN_L2_QK : 0u) | (p.gated ? GEMVQ_GDN_GATED : 0u) | (gates ? GEMVQ_GDN_GATES : 0u) |
                               (p.gate_silu ? GEMVQ_GDN_Z_SILU : 0u);
        // GEMVQ_GDN_WITH_OUT, which the reference sets for the ssm_out GEMV right behind the step
        // (ggml-xrt.cpp:2259-2270), is left clear: on this GPU the fused launch is slower in graph replays than the
        // step and the gated GEMV as two launches
        push({GEMVQ_OP_GDN, hv | (hk << 16), qo, ko, vo, go, bo, y});
        push({uint32_t(src_row), uint32_t(dst_row), fbits(1.0f / std::sqrt(float(HEAD))), flags, fbits(p.l2_eps),
              fbits(p.rms_eps), wo, zo});
        if (gates) push({dto, ao});
        return true;
    }

    bool attention(const gqg_tensor * mul, const AttnChain & at) {
        // the layer's device KV cache: created on first use with the cache's size
        auto & kvp = b->kv_layers[at.layer];
        const int64_t n_ctx = root_of(at.fa->src[1])->ne[1];
        if (kvp.kv < 0) {
            if (b->dry()) {
                kvp.kv = int(b->kv_layers.size()) - 1;
            } else {
                kvp.kv = gemvq_kv_create(b->ctx, int(n_ctx), at.n_head_kv, at.head_dim);
                if (kvp.kv < 0) {
                    err = gemvq_last_error(b->ctx);
                    return false;
                }
            }
            kvp.n_ctx = n_ctx;
        }
        uint32_t qo, ko, vo, qno, kno, po, cs, y;
        if (!operand(at.q_proj, size_t(2) * at.head_dim * at.n_head, qo) ||
            !operand(at.k_proj, size_t(at.n_head_kv) * at.head_dim, ko) ||
            !operand(at.v_proj, size_t(at.n_head_kv) * at.head_dim, vo) || !operand(at.q_norm_w, at.head_dim, qno) ||
            !operand(at.k_norm_w, at.head_dim, kno) || !operand(at.pos, 1, po) ||
            !rope_table(b, at.n_rot, at.base, kvp.n_ctx, cs, err) || !output(mul, y))
            return false;
        P.pos_checks.push_back({static_cast<const int64_t *>(at.k_row->data), static_cast<const int32_t *>(at.pos->data)});
        push({GEMVQ_OP_ATTN, uint32_t(at.n_head) | (uint32_t(at.n_head_kv) << 16), qo, uint32_t(kvp.kv), y,
              uint32_t(at.head_dim) | (uint32_t(at.n_rot) << 16), po, 1u});
        push({ko, vo, fbits(at.scale), fbits(at.eps), qno, kno, cs, qo + uint32_t(at.head_dim)});
        return true;
    }
};

int supports(const gqg_tensor * op) {
    const gqg_tensor * a = op->src[0], * b = op->src[1];
    switch (op->op) {
    case GQG_OP_NONE:
    case GQG_OP_VIEW:
    case GQG_OP_RESHAPE:
    case GQG_OP_PERMUTE:
    case GQG_OP_TRANSPOSE:
        return 1;
    case GQG_OP_MUL_MAT:
        return quant_type(a->type) && b->type == GQG_TYPE_F32 && nel(b) == a->ne[0] && a->ne[0] <= 16384 &&
               a->ne[2] == 1 && a->ne[3] == 1;
    case GQG_OP_GET_ROWS:
        return (quant_type(a->type) && b->type == GQG_TYPE_I32 && nel(b) == 1) ||
               (in_buf(a, GQG_BUF_RS) && a->type == GQG_TYPE_F32 && b->type == GQG_TYPE_I32);
    case GQG_OP_CPY:
        return in_buf(b, GQG_BUF_RS) && a->type == GQG_TYPE_F32;
    case GQG_OP_SET_ROWS:
        return in_buf(a, GQG_BUF_KV);
    case GQG_OP_RMS_NORM:
    case GQG_OP_L2_NORM:
        return token_row(op) && (token_row(a) || strided_rows(a)) && op->ne[0] % 16 == 0;
    case GQG_OP_MUL:
        return token_row(op) && (token_row(a) || a->op == GQG_OP_RESHAPE) && b->type == GQG_TYPE_F32 &&
               contiguous(b) && (nel(b) == nel(op) || (nel(b) == op->ne[0] && op->ne[0] % 16 == 0));
    case GQG_OP_ADD:
        return token_row(op) && token_row(a) && token_row(b) && nel(a) == nel(b);
    case GQG_OP_UNARY:
        return unary_kind(op) != 0 && token_row(op);
    case GQG_OP_GLU:
        return op->op_params[0] == GQG_GLU_SWIGLU && op->op_params[1] == 0 && token_row(op);
    case GQG_OP_CONT:
        return token_row(op) && strided_rows(a) && nel(op) == nel(a);
    case GQG_OP_CONCAT:
        return op->op_params[0] == 0 && op->type == GQG_TYPE_F32 && op->ne[0] == 4 && op->ne[1] % 16 == 0 &&
               a->ne[0] == 3 && b->ne[0] == 1 && rs_rows(a);
    case GQG_OP_SSM_CONV:
        return a->ne[0] == 4 && b->ne[0] == 4 && b->type == GQG_TYPE_F32 && op->ne[0] % 16 == 0 && op->ne[0] <= 16384 &&
               op->ne[1] == 1 && a->op == GQG_OP_CONCAT;
    case GQG_OP_GATED_DELTA_NET: {
        const gqg_tensor * q = op->src[0], * k = op->src[1], * v = op->src[2];
        const auto rows_ok = [](const gqg_tensor * t) {
            return t->type == GQG_TYPE_F32 && t->ne[0] == HEAD && t->ne[2] == 1 && t->ne[3] == 1 && t->nb[0] == 4 &&
                   t->nb[1] == HEAD * 4;
        };
        const int64_t hv = v->ne[1], hk = q->ne[1];
        return rows_ok(q) && rows_ok(k) && rows_ok(v) && k->ne[1] == hk && hk > 0 && hv <= 64 && hv % hk == 0 &&
               nel(op->src[3]) == hv && nel(op->src[4]) == hv && rs_rows(op->src[5]) != nullptr;
    }
    case GQG_OP_ROPE:
        return op->op_params[2] == GQG_ROPE_TYPE_NEOX && b && b->type == GQG_TYPE_I32 && op->ne[0] % 16 == 0 &&
               op->op_params[1] % 2 == 0 && op->op_params[1] <= op->ne[0];
    case GQG_OP_FLASH_ATTN_EXT:
        return in_buf(op->src[1], GQG_BUF_KV) && in_buf(op->src[2], GQG_BUF_KV) && op->src[0]->ne[0] <= 256 &&
               op->src[0]->ne[0] % 16 == 0;
    default:
        return 0;
    }
}

bool build(gqg_backend * b, const gqg_cgraph * g, gqg_backend::Plan & P, std::string & err) {
    for (int i = 0; i < g->n_nodes; ++i)
        if (!supports(g->nodes[i])) {
            err = std::string("node ") + g->nodes[i]->name + " is not supported";
            return false;
        }
    FusionPlan F;
    if (!plan_fusions(g, F, err)) return false;
    Emitter E{b, g, F, P};
    if (!E.run()) {
        err = E.err;
        return false;
    }
    if (P.words.empty()) {
        err = "the split has no command";
        return false;
    }
    return true;
}

gqg_backend::Plan * get_plan(gqg_backend * b, const gqg_cgraph * g, std::string & err) {
    ReaderIndex ix;
    for (int i = 0; i < g->n_nodes; ++i) ix.at[g->nodes[i]] = i;
    Signature sig;
    signature_of(g, ix, sig);
    for (auto & p : b->plans)
        if (p->hash == sig.hash && p->sig == sig.words) {
            ++b->reused;
            return p.get();
        }
    auto P = std::make_unique<gqg_backend::Plan>();
    if (!build(b, g, *P, err)) return nullptr;
    P->sig = std::move(sig.words);
    P->hash = sig.hash;
    ++b->built;
    if (b->plans.size() >= 64) {  // a decode token has a few splits; bound the cache
        for (auto & p : b->plans)
            if (p->graph >= 0 && b->ctx) gemvq_graph_destroy(b->ctx, p->graph);
        b->plans.clear();
    }
    b->plans.push_back(std::move(P));
    return b->plans.back().get();
}

}  // namespace

extern "C" {

gqg_backend * gqg_backend_init(const gqg_params * params) {
    if (!params || params->act_floats < 4096 || g_active) return nullptr;
    auto * b = new gqg_backend();
    b->p = *params;
    b->trans_end = params->act_floats / 2 / 16 * 16;
    if (!b->dry()) {
        b->ctx = gemvq_ctx_create(params->device, params->act_floats, params->weight_bytes, params->state_rows);
        if (!b->ctx) {
            delete b;
            return nullptr;
        }
    }
    g_active = b;
    return b;
}

void gqg_backend_free(gqg_backend * b) {
    if (!b) return;
    for (gqg_buffer * buf : b->buffers) buf->owner = nullptr;  // detached: only gqg_buffer_free works on them now
    if (b->ctx) gemvq_ctx_destroy(b->ctx);
    if (g_active == b) g_active = nullptr;
    delete b;
}

const char * gqg_backend_error(const gqg_backend * b) { return b ? b->err.c_str() : "no backend"; }

int gqg_supports_op(const gqg_backend * b, const gqg_tensor * op) { return b && op && supports(op); }

int gqg_graph_plan(gqg_backend * b, gqg_cgraph * g, uint32_t * words, size_t cap) {
    if (!b || !g || g->n_nodes <= 0) return fail(b, "gqg_graph_plan: arguments");
    std::string err;
    gqg_backend::Plan * P = get_plan(b, g, err);
    if (!P) return fail(b, err);
    if (words && cap >= P->words.size()) std::memcpy(words, P->words.data(), P->words.size() * 4);
    return int(P->words.size() / GEMVQ_CMD_WORDS);
}

int gqg_graph_compute(gqg_backend * b, gqg_cgraph * g) {
    if (!b) return GQG_STATUS_FAILED;
    if (!b->valid) return fail(b, "backend invalidated by an earlier failure");
    if (!g || g->n_nodes <= 0) return GQG_STATUS_SUCCESS;
    if (b->dry()) return fail(b, "a dry backend only plans");
    std::string err;
    gqg_backend::Plan * P = get_plan(b, g, err);
    bool ok = P != nullptr;
    for (size_t i = 0; ok && i < P->pos_checks.size(); ++i) {
        const auto & pc = P->pos_checks[i];
        if (int64_t(*pc.second) != *pc.first) {  // the cache row a one-token attention writes is its position
            err = "attention: the KV row stored is not the token's position";
            ok = false;
        }
    }
    for (size_t i = 0; ok && i < P->in.size(); ++i)
        ok = act_write(b, P->in[i].off, P->in[i].host, P->in[i].floats, err);
    if (ok && P->graph < 0 &&
        gemvq_graph_create(b->ctx, P->words.data(), unsigned(P->words.size() / GEMVQ_CMD_WORDS), &P->graph)) {
        err = gemvq_last_error(b->ctx);
        ok = false;
    }
    if (ok && (gemvq_graph_replay(b->ctx, P->graph, 1) || gemvq_sync(b->ctx))) {
        err = gemvq_last_error(b->ctx);
        ok = false;
    }
    for (size_t i = 0; ok && i < P->out.size(); ++i)
        if (gemvq_act_read(b->ctx, P->out[i].off, const_cast<void *>(P->out[i].host), P->out[i].floats)) {
            err = gemvq_last_error(b->ctx);
            ok = false;
        }
    if (ok) return GQG_STATUS_SUCCESS;
    b->valid = false;  // a failed list leaves the device state unknown (ggml-xrt.cpp:2761-2770)
    return fail(b, err);
}

int gqg_graph_io(gqg_backend * b, gqg_cgraph * g, const void ** ins, const void ** outs, size_t cap, int counts[2]) {
    if (!b || !g || g->n_nodes <= 0 || !counts) return fail(b, "gqg_graph_io: arguments");
    std::string err;
    gqg_backend::Plan * P = get_plan(b, g, err);
    if (!P) return fail(b, err);
    counts[0] = int(P->in.size());
    counts[1] = int(P->out.size());
    for (size_t i = 0; ins && i < P->in.size() && i < cap; ++i) ins[i] = P->in[i].host;
    for (size_t i = 0; outs && i < P->out.size() && i < cap; ++i) outs[i] = P->out[i].host;
    return 0;
}

void gqg_plan_stats(const gqg_backend * b, uint64_t out[2]) {
    out[0] = b ? b->built : 0;
    out[1] = b ? b->reused : 0;
}

static gqg_buffer * buffer_alloc(gqg_backend * b, size_t size, int kind) {
    if (!b) return nullptr;
    const size_t reserved = std::max<size_t>(size, 1);
    void * base = mmap(nullptr, reserved, PROT_NONE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (base == MAP_FAILED) return nullptr;
    auto * buf = new gqg_buffer();
    buf->owner = b;
    buf->kind = kind;
    buf->base = static_cast<uint8_t *>(base);
    buf->size = reserved;
    b->buffers.push_back(buf);
    return buf;
}

gqg_buffer * gqg_rs_buffer_alloc(gqg_backend * b, size_t size) { return buffer_alloc(b, size, GQG_BUF_RS); }
gqg_buffer * gqg_kv_buffer_alloc(gqg_backend * b, size_t size) { return buffer_alloc(b, size, GQG_BUF_KV); }
void * gqg_buffer_base(const gqg_buffer * buf) { return buf ? buf->base : nullptr; }

int gqg_buffer_init_tensor(gqg_buffer * buf, gqg_tensor * t) {
    if (!buf || !t || !buf->owner) return GQG_STATUS_FAILED;
    if (t->view_src) return GQG_STATUS_SUCCESS;
    gqg_backend * b = buf->owner;
    const auto * p = static_cast<const uint8_t *>(t->data);
    const size_t bytes = size_t(nel(t)) * (t->type == GQG_TYPE_F16 ? 2 : 4);
    if (p < buf->base || p + bytes > buf->base + buf->size) return fail(b, "tensor outside its buffer");
    t->buffer = buf->kind;
    gqg_buffer::Entry e;
    e.off = size_t(p - buf->base);
    e.bytes = bytes;
    if (buf->kind == GQG_BUF_KV) {  // placed when an attention first reads it
        buf->tensors.push_back(e);
        return GQG_STATUS_SUCCESS;
    }
    e.state = std::strncmp(t->name, "cache_s_l", 9) == 0;
    if (e.state) {
        const size_t rows = (bytes + 511) / 512;
        if (b->state_rows_used + rows > b->p.state_rows) return fail(b, std::string("state rows full at ") + t->name, GQG_STATUS_ALLOC_FAILED);
        e.dev = b->state_rows_used;
        b->state_rows_used += rows;
    } else {
        uint32_t off;
        std::string err;
        if (!take_resident(b, bytes / 4, off, err)) return fail(b, err + " at " + t->name, GQG_STATUS_ALLOC_FAILED);
        e.dev = off;
    }
    buf->tensors.push_back(e);
    return GQG_STATUS_SUCCESS;
}

static int buffer_io(gqg_buffer * buf, const gqg_tensor * t, void * data, size_t offset, size_t size, bool to_dev) {
    if (!buf || !t || !buf->owner) return GQG_STATUS_FAILED;
    gqg_backend * b = buf->owner;
    if (buf->kind != GQG_BUF_RS) return fail(b, "KV buffers are written by attention commands only");
    const gqg_buffer::Entry * e = buf->find(static_cast<const uint8_t *>(t->data) + offset);
    if (!e) return fail(b, std::string("tensor not placed: ") + t->name);
    const size_t within = size_t(static_cast<const uint8_t *>(t->data) + offset - buf->base) - e->off;
    if (within + size > e->bytes || within % 4 || size % 4) return fail(b, "state access out of range");
    if (b->dry() || size == 0) return GQG_STATUS_SUCCESS;
    int st;
    if (e->state) {
        if (within % 512 || size % 512) return fail(b, "state rows are accessed whole (512 bytes)");
        st = to_dev ? gemvq_state_write(b->ctx, e->dev + within / 512, static_cast<const float *>(data), size / 512)
                    : gemvq_state_read(b->ctx, e->dev + within / 512, static_cast<float *>(data), size / 512);
    } else {
        st = to_dev ? gemvq_act_write(b->ctx, e->dev + within / 4, data, size / 4)
                    : gemvq_act_read(b->ctx, e->dev + within / 4, data, size / 4);
    }
    return st ? fail(b, gemvq_last_error(b->ctx)) : GQG_STATUS_SUCCESS;
}

int gqg_buffer_set(gqg_buffer * buf, const gqg_tensor * t, const void * data, size_t offset, size_t size) {
    return buffer_io(buf, t, const_cast<void *>(data), offset, size, true);
}

int gqg_buffer_get(gqg_buffer * buf, const gqg_tensor * t, void * data, size_t offset, size_t size) {
    return buffer_io(buf, t, data, offset, size, false);
}

int gqg_buffer_clear(gqg_buffer * buf, uint8_t value) {
    if (!buf || !buf->owner) return GQG_STATUS_FAILED;
    gqg_backend * b = buf->owner;
    if (b->dry()) return GQG_STATUS_SUCCESS;
    if (buf->kind == GQG_BUF_KV) {
        if (value) return fail(b, "KV buffers clear to zero only");
        return gemvq_kv_clear(b->ctx) ? fail(b, gemvq_last_error(b->ctx)) : GQG_STATUS_SUCCESS;
    }
    for (const auto & e : buf->tensors) {
        std::vector<uint8_t> fill(e.bytes, value);
        const int st = e.state ? gemvq_state_write(b->ctx, e.dev, reinterpret_cast<const float *>(fill.data()), e.bytes / 512)
                               : gemvq_act_write(b->ctx, e.dev, fill.data(), e.bytes / 4);
        if (st) return fail(b, gemvq_last_error(b->ctx));
    }
    return GQG_STATUS_SUCCESS;
}

void gqg_buffer_free(gqg_buffer * buf) {
    if (!buf) return;
    if (gqg_backend * b = buf->owner) {
        auto & v = b->buffers;
        v.erase(std::remove(v.begin(), v.end(), buf), v.end());
    }
    munmap(buf->base, buf->size);
    delete buf;
}

static const char * reg_description(void) { return "AMD Instinct MI355X (gfx950), gemvq command lists"; }

static void reg_memory(size_t * free_bytes, size_t * total_bytes) {
    size_t f = 0, t = 0;
    gemvq_device_memory(0, &f, &t);
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
}

const gqg_backend_reg * gqg_backend_get_reg(void) {
    static const gqg_backend_reg reg = {
        "GEMVQ", reg_description, reg_memory, 2, gqg_backend_init, gqg_backend_free, gqg_supports_op, gqg_supports_op,
        gqg_graph_compute, gqg_rs_buffer_alloc, gqg_kv_buffer_alloc,
    };
    return &reg;
}

}  // extern "C"
