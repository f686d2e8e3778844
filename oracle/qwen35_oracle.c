/* CPU oracle of the synthetic Qwen3.5-shaped hybrid decoder: TEST INFRASTRUCTURE ONLY (see qwen35_oracle.h).
 *
 * A chunk of T tokens runs layer by layer: every projection reads each weight row once for all T tokens (the
 * per-token arithmetic is that of one token, so a chunk equals T decode steps bit for bit), the conv, DeltaNet step
 * and attention run token by token in order. Two arithmetics:
 *   ORC_MODE_CANONICAL  the arithmetic the GPU reproduces bit for bit (gemvq_oracle.c's canonical ops);
 *   ORC_MODE_REFERENCE  the reference's CPU arithmetic: gemvq_ref.h's sequential FP32 GEMV rows, sums of squares in
 *                       double (gemvq_ref.h:94-358), composed as ggml's graph composes them (ggml-xrt.cpp:1944-1992:
 *                       L2_NORM of q and k, SIGMOID(beta), MUL(SOFTPLUS(ADD(alpha, dt)), a), RMS_NORM rows of 128 ->
 *                       MUL weight -> MUL SILU(z)); attention as orc_ref_attn; exp and log correctly rounded
 *                       (orc_crmath.c), the functions the GPU's reference-arithmetic mode evaluates;
 *   ORC_MODE_REFERENCE_LIBM  the same with the host libm's expf / logf, as the compiled reference path calls them. */
#include "qwen35_oracle.h"
#include "gemvq_oracle.h"
#include "orc_fast.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    int type, rows, cols;
    const void * data;
} orc_t;

typedef struct {
    int attn;
    orc_t attn_norm, post_norm;
    /* DeltaNet */
    orc_t qkv, z, beta, alpha, conv1d, dt, a, ssm_norm, ssm_out;
    /* attention */
    orc_t wq, wk, wv, q_norm, k_norm, wo;
    /* FFN */
    orc_t gate, up, down;
} orc_layer;

enum { CHUNK = 32 };

typedef struct {
    orc_qw_config c;
    int n_threads, mode, fault;
    float * trace;         /* non-NULL: the residual stream of the last token of a chunk before layer 0 and after
                            * every layer, (n_layer + 1) x n_embd floats */
    orc_t tok_embd, output_norm, output;
    orc_layer * layers;
    float ** conv_state;   /* per DeltaNet layer [ch][3] */
    float ** ssm_state;    /* per DeltaNet layer [hv][128][128] */
    uint16_t ** kcache;    /* per attention layer [n_ctx][n_head_kv][head_dim] fp16 */
    uint16_t ** vcache;
    int big;               /* the widest per-token vector */
    /* per-token rows of a chunk: [CHUNK][big] each */
    float * h, * xn, * b1, * b2, * b3, * b4, * logits;
} orc_model;

static int find(const orc_tensor_desc * t, int n, const uint8_t * blob, const char * name, orc_t * out) {
    for (int i = 0; i < n; ++i) {
        if (strncmp(t[i].name, name, sizeof(t[i].name)) == 0) {
            out->type = t[i].type;
            out->cols = t[i].ne0;
            out->rows = t[i].ne1;
            out->data = blob + t[i].offset;
            return 1;
        }
    }
    fprintf(stderr, "orc_model_create: missing tensor %s\n", name);
    return 0;
}

void orc_rope_cache(int pos, int n_dims, float base, float * cs) {
    const float theta_scale = powf(base, -2.0f / (float)n_dims);
    float theta = (float)pos;
    for (int i0 = 0; i0 < n_dims; i0 += 2) {
        cs[i0] = cosf(theta);
        cs[i0 + 1] = sinf(theta);
        theta *= theta_scale;
    }
}

static int conv_channels(const orc_qw_config * c) { return 2 * c->ssm_k_heads * c->ssm_head_dim + c->ssm_v_heads * c->ssm_head_dim; }

void * orc_model_create(const orc_qw_config * cfg, const orc_tensor_desc * table, int nt, const uint8_t * blob,
                        int n_threads) {
    orc_model * m = (orc_model *)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    m->n_threads = n_threads > 0 ? n_threads : 1;
    int ok = find(table, nt, blob, "token_embd.weight", &m->tok_embd) &&
             find(table, nt, blob, "output_norm.weight", &m->output_norm) &&
             find(table, nt, blob, "output.weight", &m->output);
    m->layers = (orc_layer *)calloc((size_t)cfg->n_layer, sizeof(orc_layer));
    m->conv_state = (float **)calloc((size_t)cfg->n_layer, sizeof(float *));
    m->ssm_state = (float **)calloc((size_t)cfg->n_layer, sizeof(float *));
    m->kcache = (uint16_t **)calloc((size_t)cfg->n_layer, sizeof(uint16_t *));
    m->vcache = (uint16_t **)calloc((size_t)cfg->n_layer, sizeof(uint16_t *));
    const int ch = conv_channels(cfg);
    char nm[64];
#define F(field, fmt) (snprintf(nm, sizeof nm, fmt, il), find(table, nt, blob, nm, &L->field))
    for (int il = 0; il < cfg->n_layer && ok; ++il) {
        orc_layer * L = &m->layers[il];
        L->attn = (il + 1) % cfg->attn_interval == 0;
        ok = F(attn_norm, "blk.%d.attn_norm.weight") && F(post_norm, "blk.%d.post_attention_norm.weight") &&
             F(gate, "blk.%d.ffn_gate.weight") && F(up, "blk.%d.ffn_up.weight") && F(down, "blk.%d.ffn_down.weight");
        if (!ok) break;
        if (L->attn) {
            ok = F(wq, "blk.%d.attn_q.weight") && F(wk, "blk.%d.attn_k.weight") && F(wv, "blk.%d.attn_v.weight") &&
                 F(q_norm, "blk.%d.attn_q_norm.weight") && F(k_norm, "blk.%d.attn_k_norm.weight") &&
                 F(wo, "blk.%d.attn_output.weight");
            const size_t kv = (size_t)cfg->n_ctx * cfg->n_head_kv * cfg->head_dim;
            m->kcache[il] = (uint16_t *)calloc(kv, sizeof(uint16_t));
            m->vcache[il] = (uint16_t *)calloc(kv, sizeof(uint16_t));
        } else {
            ok = F(qkv, "blk.%d.attn_qkv.weight") && F(z, "blk.%d.attn_gate.weight") &&
                 F(beta, "blk.%d.ssm_beta.weight") && F(alpha, "blk.%d.ssm_alpha.weight") &&
                 F(conv1d, "blk.%d.ssm_conv1d.weight") && F(dt, "blk.%d.ssm_dt.bias") && F(a, "blk.%d.ssm_a") &&
                 F(ssm_norm, "blk.%d.ssm_norm.weight") && F(ssm_out, "blk.%d.ssm_out.weight");
            m->conv_state[il] = (float *)calloc((size_t)ch * 3, sizeof(float));
            m->ssm_state[il] = (float *)calloc((size_t)cfg->ssm_v_heads * cfg->ssm_head_dim * cfg->ssm_head_dim,
                                               sizeof(float));
        }
    }
#undef F
    int big = cfg->n_ff > cfg->n_embd ? cfg->n_ff : cfg->n_embd;
    if (2 * cfg->n_head * cfg->head_dim > big) big = 2 * cfg->n_head * cfg->head_dim;
    if (ch > big) big = ch;
    big = (big + 63) / 64 * 64;
    m->big = big;
    const size_t rowsz = (size_t)CHUNK * (size_t)big;
    m->h = (float *)calloc(rowsz, sizeof(float));
    m->xn = (float *)calloc(rowsz, sizeof(float));
    m->b1 = (float *)calloc(rowsz, sizeof(float));
    m->b2 = (float *)calloc(rowsz, sizeof(float));
    m->b3 = (float *)calloc(rowsz, sizeof(float));
    m->b4 = (float *)calloc(rowsz, sizeof(float));
    m->logits = (float *)calloc((size_t)cfg->n_vocab, sizeof(float));
    if (!ok) {
        orc_model_destroy(m);
        return NULL;
    }
    return m;
}

void orc_model_destroy(void * mp) {
    orc_model * m = (orc_model *)mp;
    if (!m) return;
    for (int il = 0; il < m->c.n_layer; ++il) {
        free(m->conv_state[il]);
        free(m->ssm_state[il]);
        free(m->kcache[il]);
        free(m->vcache[il]);
    }
    free(m->conv_state); free(m->ssm_state); free(m->kcache); free(m->vcache);
    free(m->layers);
    free(m->h); free(m->xn); free(m->b1); free(m->b2); free(m->b3); free(m->b4); free(m->logits);
    free(m);
}

int orc_model_set_mode(void * mp, int mode) {
    orc_model * m = (orc_model *)mp;
    if (!m || (mode != ORC_MODE_CANONICAL && mode != ORC_MODE_REFERENCE && mode != ORC_MODE_REFERENCE_LIBM)) return -1;
    m->mode = mode;
    return 0;
}

int orc_model_set_fault(void * mp, int fault) {
    orc_model * m = (orc_model *)mp;
    if (!m || fault < 0 || fault > ORC_FAULT_LAST) return -1;
    m->fault = fault;
    return 0;
}

int orc_model_set_trace(void * mp, float * out) {
    orc_model * m = (orc_model *)mp;
    if (!m) return -1;
    m->trace = out;
    return 0;
}

int orc_model_reset(void * mp) {
    orc_model * m = (orc_model *)mp;
    if (!m) return -1;
    const orc_qw_config * c = &m->c;
    const int ch = conv_channels(c);
    for (int il = 0; il < c->n_layer; ++il) {
        if (m->conv_state[il]) memset(m->conv_state[il], 0, sizeof(float) * (size_t)ch * 3);
        if (m->ssm_state[il])
            memset(m->ssm_state[il], 0, sizeof(float) * (size_t)c->ssm_v_heads * c->ssm_head_dim * c->ssm_head_dim);
        if (m->kcache[il]) {
            const size_t kv = (size_t)c->n_ctx * c->n_head_kv * c->head_dim;
            memset(m->kcache[il], 0, kv * sizeof(uint16_t));
            memset(m->vcache[il], 0, kv * sizeof(uint16_t));
        }
    }
    return 0;
}

/* Y[t] = W X[t] for T token rows (X rows xs floats apart, Y rows ys floats apart): every weight row is read once for
 * all tokens; rows split over the threads (a row's result does not depend on the split). */
static void gemm(orc_model * m, const orc_t * w, const float * X, int xs, int T, float * Y, int ys) {
    const int rows = w->rows, cols = w->cols, fmt = w->type;
    const int fmode = m->mode == ORC_MODE_CANONICAL ? 0 : 1;  /* orc_fast: 0 canonical rows, 1 sequential FP32 rows */
    if (fmode && !orc_fast_supported(fmt)) {
        for (int t = 0; t < T; ++t) orc_ref_gemv(fmt, (const uint8_t *)w->data, X + (size_t)t * xs, rows, cols, Y + (size_t)t * ys, NULL);
        return;
    }
    orc_act acts[CHUNK];
    const orc_act * ap[CHUNK];
    for (int t = 0; t < T; ++t) {
        orc_act_init(&acts[t], fmt, X + (size_t)t * xs, cols);
        ap[t] = &acts[t];
    }
    const int chunk = 16;
    const int nchunks = (rows + chunk - 1) / chunk;
#pragma omp parallel for schedule(dynamic, 4) num_threads(m->n_threads)
    for (int cidx = 0; cidx < nchunks; ++cidx) {
        const int r0 = cidx * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
        float tmp[CHUNK * 16];
        orc_fast_rows_multi(fmode, fmt, (const uint8_t *)w->data, ap, T, r0, r1, tmp, 16);
        for (int t = 0; t < T; ++t) memcpy(Y + (size_t)t * ys + r0, tmp + 16 * t, sizeof(float) * (size_t)(r1 - r0));
    }
    for (int t = 0; t < T; ++t) orc_act_free(&acts[t]);
}

/* RMS norm of one row with weight (canonical pairwise tree, or ggml's double sum of float squares). */
static void rmsnorm(const orc_model * m, const float * x, const orc_t * w, int n, float * y) {
    if (m->mode != ORC_MODE_CANONICAL) orc_ref_rownorm(x, (const float *)w->data, n, 1, m->c.eps, 0, y);
    else orc_rownorm(x, (const float *)w->data, n, 1, 0, m->c.eps, 0, y);
}

static float unary1(const orc_model * m, float v, int kind) {
    float y;
    if (m->mode == ORC_MODE_REFERENCE) orc_ref_unary_cr(&v, 1, kind, &y);
    else if (m->mode == ORC_MODE_REFERENCE_LIBM) orc_ref_unary(&v, 1, kind, &y);
    else orc_unary(&v, 1, kind, &y);
    return y;
}

/* One attention layer over T tokens (positions pos0 ..): q (+ gate interleaved per head) / k / v projections of the
 * normed rows, per token q/k norm, RoPE, KV append, attention over positions 0..pos, the sigmoid output gate, then
 * the output projection and the residual add. */
static void attn_layer(orc_model * m, int il, int T, int pos0) {
    const orc_qw_config * c = &m->c;
    orc_layer * L = &m->layers[il];
    const int E = c->n_embd, hd = c->head_dim, nh = c->n_head, nkv = c->n_head_kv, B = m->big;
    const int ref = m->mode != ORC_MODE_CANONICAL, cr = m->mode == ORC_MODE_REFERENCE;
    float * qg = m->b1, * kk = m->b2, * vv = m->b3;
    gemm(m, &L->wq, m->xn, B, T, qg, B);
    gemm(m, &L->wk, m->xn, B, T, kk, B);
    gemm(m, &L->wv, m->xn, B, T, vv, B);
    float * qn = (float *)malloc(sizeof(float) * (size_t)nh * hd);
    float * tmp = (float *)malloc(sizeof(float) * (size_t)hd * (nh > nkv ? nh : nkv));
    float * kr = (float *)malloc(sizeof(float) * (size_t)nkv * hd);
    float * att = (float *)malloc(sizeof(float) * (size_t)nh * hd);
    float * cs = (float *)malloc(sizeof(float) * (size_t)c->n_rot);
    float * xo = m->b4;
    for (int t = 0; t < T; ++t) {
        const int pos = pos0 + t;
        const float * q = qg + (size_t)t * B, * kt = kk + (size_t)t * B, * vt = vv + (size_t)t * B;
        const int qoff = m->fault == ORC_FAULT_QGATE_SWAP ? hd : 0, goff = hd - qoff;
        orc_rope_cache(pos, c->n_rot, c->rope_base, cs);
        if (ref) {
            float * qrow = (float *)malloc(sizeof(float) * (size_t)nh * hd);
            for (int h = 0; h < nh; ++h) memcpy(qrow + h * hd, q + (size_t)h * 2 * hd + qoff, sizeof(float) * hd);
            orc_ref_rownorm(qrow, (const float *)L->q_norm.data, hd, nh, c->eps, 0, tmp);
            free(qrow);
        } else {
            orc_rownorm(q + qoff, (const float *)L->q_norm.data, hd, nh, 2 * hd, c->eps, 0, tmp);
        }
        orc_rope(tmp, cs, c->n_rot, hd, nh, qn);
        if (ref) orc_ref_rownorm(kt, (const float *)L->k_norm.data, hd, nkv, c->eps, 0, tmp);
        else orc_rownorm(kt, (const float *)L->k_norm.data, hd, nkv, 0, c->eps, 0, tmp);
        if (m->fault == ORC_FAULT_ROPE_K) memcpy(kr, tmp, sizeof(float) * (size_t)nkv * hd);
        else orc_rope(tmp, cs, c->n_rot, hd, nkv, kr);
        uint16_t * kc = m->kcache[il] + (size_t)pos * nkv * hd, * vc = m->vcache[il] + (size_t)pos * nkv * hd;
        for (int i = 0; i < nkv * hd; ++i) {
            kc[i] = orc_float_to_half(kr[i]);
            vc[i] = orc_float_to_half(vt[i]);
        }
        const float scale = 1.0f / sqrtf((float)hd);
        if (cr) orc_ref_attn_cr_mt(qn, m->kcache[il], m->vcache[il], nh, nkv, hd, pos + 1, scale, att, m->n_threads);
        else if (ref) orc_ref_attn_mt(qn, m->kcache[il], m->vcache[il], nh, nkv, hd, pos + 1, scale, att, m->n_threads);
        else orc_attn_mt(qn, m->kcache[il], m->vcache[il], nh, nkv, hd, pos + 1, scale, att, m->n_threads);
        /* output gate: sigmoid(gate) * att */
        float * o = xo + (size_t)t * B;
        for (int h = 0; h < nh; ++h)
            for (int d = 0; d < hd; ++d) {
                const float g = q[(size_t)h * 2 * hd + goff + d];
                o[h * hd + d] = ref ? unary1(m, g, 2) * att[h * hd + d] : (1.0f / (1.0f + orc_expf(-g))) * att[h * hd + d];
            }
    }
    free(qn); free(tmp); free(kr); free(att); free(cs);
    float * y = m->b1;
    gemm(m, &L->wo, xo, B, T, y, B);
    for (int t = 0; t < T; ++t) {
        float * h = m->h + (size_t)t * B;
        const float * yt = y + (size_t)t * B;
        for (int i = 0; i < E; ++i) h[i] = m->fault == ORC_FAULT_ATTN_RESIDUAL ? yt[i] : yt[i] + h[i];
    }
}

/* One Gated DeltaNet layer over T tokens: qkv / z / beta / alpha projections, then per token the causal conv, the
 * step with L2-normed q/k and the gates, the gated output norm; then ssm_out and the residual add. */
static void gdn_layer(orc_model * m, int il, int T) {
    const orc_qw_config * c = &m->c;
    orc_layer * L = &m->layers[il];
    const int E = c->n_embd, S = c->ssm_head_dim, hk = c->ssm_k_heads, hv = c->ssm_v_heads, B = m->big;
    const int ch = conv_channels(c);
    const int ref = m->mode != ORC_MODE_CANONICAL, cr = m->mode == ORC_MODE_REFERENCE;
    float * qkv = m->b1, * z = m->b2, * ba = m->b3;  /* ba row: beta [hv] then alpha at + 64 */
    gemm(m, &L->qkv, m->xn, B, T, qkv, B);
    gemm(m, &L->z, m->xn, B, T, z, B);
    gemm(m, &L->beta, m->xn, B, T, ba, B);
    gemm(m, &L->alpha, m->xn, B, T, ba + (hv + 63) / 64 * 64, B);
    float * cy = (float *)malloc(sizeof(float) * (size_t)ch);
    float * ns = (float *)malloc(sizeof(float) * (size_t)ch * 3);
    float * y = m->b4;
    const float * dt = (const float *)L->dt.data, * av = (const float *)L->a.data, * wn = (const float *)L->ssm_norm.data;
    for (int t = 0; t < T; ++t) {
        const float * bt = ba + (size_t)t * B, * at = bt + (hv + 63) / 64 * 64;
        const float * braw = m->fault == ORC_FAULT_GATES_SWAP ? at : bt, * araw = m->fault == ORC_FAULT_GATES_SWAP ? bt : at;
        float * yt = y + (size_t)t * B;
        if (cr) {
            orc_ref_conv_cr(m->conv_state[il], qkv + (size_t)t * B, (const float *)L->conv1d.data, ch, 1, cy, ns);
        } else if (ref) {
            orc_ref_conv(m->conv_state[il], qkv + (size_t)t * B, (const float *)L->conv1d.data, ch, 1, cy, ns);
        } else {
            orc_conv(m->conv_state[il], qkv + (size_t)t * B, (const float *)L->conv1d.data, ch, 1, cy, ns);
        }
        memcpy(m->conv_state[il], ns, sizeof(float) * (size_t)ch * 3);
        if (ref) {
            /* ggml's graph: L2_NORM(q), L2_NORM(k), SIGMOID(beta), MUL(SOFTPLUS(ADD(alpha, dt)), a), the step,
             * RMS_NORM rows of 128 -> MUL weight -> MUL SILU(z) */
            float * qn = (float *)malloc(sizeof(float) * (size_t)hk * S), * kn = (float *)malloc(sizeof(float) * (size_t)hk * S);
            orc_ref_rownorm(cy, NULL, S, hk, c->eps, 3, qn);
            orc_ref_rownorm(cy + hk * S, NULL, S, hk, c->eps, 3, kn);
            float * g = (float *)malloc(sizeof(float) * (size_t)hv), * be = (float *)malloc(sizeof(float) * (size_t)hv);
            for (int h = 0; h < hv; ++h) {
                be[h] = unary1(m, braw[h], 2);
                g[h] = unary1(m, araw[h] + dt[h], 3) * av[h];
            }
            float * yr = (float *)malloc(sizeof(float) * (size_t)hv * S);
            if (cr)
                orc_ref_gdn_cr_mt(m->ssm_state[il], qn, kn, cy + 2 * hk * S, g, be, hv, hk, 1.0f / sqrtf((float)S), yr,
                                  m->n_threads);
            else
                orc_ref_gdn_mt(m->ssm_state[il], qn, kn, cy + 2 * hk * S, g, be, hv, hk, 1.0f / sqrtf((float)S), yr, NULL,
                               NULL, m->n_threads);
            orc_ref_rownorm(yr, wn, S, hv, c->eps, 0, yt);
            for (int i = 0; i < hv * S; ++i) yt[i] = yt[i] * unary1(m, z[(size_t)t * B + i], 1);
            free(qn); free(kn); free(g); free(be); free(yr);
        } else {
            orc_gdn_mt(m->ssm_state[il], cy, cy + hk * S, cy + 2 * hk * S, araw, braw, dt, av, z + (size_t)t * B, wn, hv, hk,
                       1.0f / sqrtf((float)S), c->eps, c->eps, 2 | 4 | 8, yt, m->n_threads);
        }
    }
    free(cy); free(ns);
    float * o = m->b1;
    gemm(m, &L->ssm_out, y, B, T, o, B);
    for (int t = 0; t < T; ++t) {
        float * h = m->h + (size_t)t * B;
        const float * ot = o + (size_t)t * B;
        for (int i = 0; i < E; ++i) h[i] = m->fault == ORC_FAULT_SSM_RESIDUAL ? ot[i] : ot[i] + h[i];
    }
}

/* T tokens at positions pos0 .. pos0 + T - 1 through every layer; the logits of the last token when asked. */
static int run_chunk(orc_model * m, const int32_t * tok, int T, int pos0, int logits) {
    const orc_qw_config * c = &m->c;
    const int E = c->n_embd, B = m->big;
    if (T < 1 || T > CHUNK || pos0 < 0 || pos0 + T > c->n_ctx) return -1;
    for (int t = 0; t < T; ++t) {
        if (tok[t] < 0 || tok[t] >= c->n_vocab) return -1;
        orc_dequant_row_q6_K((const uint8_t *)m->tok_embd.data + orc_row_bytes(ORC_Q6_K, E) * (size_t)tok[t], E,
                             m->h + (size_t)t * B);
    }
    if (m->trace) memcpy(m->trace, m->h + (size_t)(T - 1) * B, sizeof(float) * (size_t)E);
    for (int il = 0; il < c->n_layer; ++il) {
        orc_layer * L = &m->layers[il];
        for (int t = 0; t < T; ++t) rmsnorm(m, m->h + (size_t)t * B, &L->attn_norm, E, m->xn + (size_t)t * B);
        if (L->attn) attn_layer(m, il, T, pos0);
        else gdn_layer(m, il, T);
        /* FFN: post norm, gate/up, SwiGLU, down + residual */
        for (int t = 0; t < T; ++t) rmsnorm(m, m->h + (size_t)t * B, &L->post_norm, E, m->xn + (size_t)t * B);
        const orc_t * gw = m->fault == ORC_FAULT_FFN_SWAP ? &L->up : &L->gate, * uw = m->fault == ORC_FAULT_FFN_SWAP ? &L->gate : &L->up;
        gemm(m, gw, m->xn, B, T, m->b1, B);
        gemm(m, uw, m->xn, B, T, m->b2, B);
        for (int t = 0; t < T; ++t) {
            float * g = m->b1 + (size_t)t * B, * u = m->b2 + (size_t)t * B, * o = m->b3 + (size_t)t * B;
            if (m->mode == ORC_MODE_REFERENCE) {
                orc_ref_silu_mul_cr(g, u, c->n_ff, o);  /* gemvq_ref.h:303-307 */
            } else if (m->mode == ORC_MODE_REFERENCE_LIBM) {
                for (int i = 0; i < c->n_ff; ++i) o[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
            } else {
                orc_silu_mul(g, u, c->n_ff, 0, o);
            }
        }
        gemm(m, &L->down, m->b3, B, T, m->b1, B);
        for (int t = 0; t < T; ++t) {
            float * h = m->h + (size_t)t * B;
            const float * d = m->b1 + (size_t)t * B;
            for (int i = 0; i < E; ++i) h[i] = d[i] + h[i];
        }
        if (m->trace) memcpy(m->trace + (size_t)(il + 1) * E, m->h + (size_t)(T - 1) * B, sizeof(float) * (size_t)E);
    }
    if (!logits) return 0;
    const float * hl = m->h + (size_t)(T - 1) * B;
    rmsnorm(m, hl, &m->output_norm, E, m->xn);
    gemm(m, &m->output, m->xn, B, 1, m->logits, c->n_vocab);
    return orc_argmax(m->logits, c->n_vocab);
}

int orc_model_decode(void * mp, int token, int pos, float * logits) {
    orc_model * m = (orc_model *)mp;
    if (!m) return -1;
    const int32_t t = token;
    const int r = run_chunk(m, &t, 1, pos, 1);
    if (r >= 0 && logits) memcpy(logits, m->logits, sizeof(float) * (size_t)m->c.n_vocab);
    return r;
}

int orc_model_prefill(void * mp, const int32_t * tokens, int n, int pos0) {
    orc_model * m = (orc_model *)mp;
    if (!m || n < 0 || !tokens) return -1;
    for (int i = 0; i < n; i += CHUNK) {
        const int T = n - i < CHUNK ? n - i : CHUNK;
        if (run_chunk(m, tokens + i, T, pos0 + i, 0) < 0) return -1;
    }
    return 0;
}

int orc_model_generate(void * mp, const int32_t * prompt, int n_prompt, int n_gen, int32_t * out, float * last_logits) {
    orc_model * m = (orc_model *)mp;
    if (!m || !prompt || !out || n_prompt < 1 || n_gen < 0 || n_prompt + n_gen > m->c.n_ctx) return -1;
    memcpy(out, prompt, sizeof(int32_t) * (size_t)n_prompt);
    if (orc_model_prefill(m, prompt, n_prompt - 1, 0) < 0) return -1;
    for (int i = 0; i < n_gen; ++i) {
        const int pos = n_prompt - 1 + i;
        const int nxt = orc_model_decode(m, out[pos], pos, i == n_gen - 1 ? last_logits : NULL);
        if (nxt < 0) return -1;
        out[pos + 1] = nxt;
    }
    return 0;
}

const float * orc_model_hidden(void * mp) {
    orc_model * m = (orc_model *)mp;
    return m->h;  /* the last decode's token row is row 0 */
}
