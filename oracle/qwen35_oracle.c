/* CPU oracle of the synthetic Qwen3.5-shaped hybrid decoder: TEST INFRASTRUCTURE ONLY (see qwen35_oracle.h). */
#include "qwen35_oracle.h"
#include "gemvq_oracle.h"

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

typedef struct {
    orc_qw_config c;
    int n_threads;
    orc_t tok_embd, output_norm, output;
    orc_layer * layers;
    /* recurrent state and KV cache */
    float ** conv_state;   /* per DeltaNet layer [ch][3] */
    float ** ssm_state;    /* per DeltaNet layer [hv][128][128] */
    uint16_t ** kcache;    /* per attention layer [n_ctx][n_head_kv][head_dim] fp16 */
    uint16_t ** vcache;
    /* scratch */
    float * h, * xn, * buf, * buf2, * buf3, * logits;
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
    const int ch = 2 * cfg->ssm_k_heads * cfg->ssm_head_dim + cfg->ssm_v_heads * cfg->ssm_head_dim;
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
    m->h = (float *)calloc((size_t)cfg->n_embd, sizeof(float));
    m->xn = (float *)calloc((size_t)big, sizeof(float));
    m->buf = (float *)calloc((size_t)big, sizeof(float));
    m->buf2 = (float *)calloc((size_t)big, sizeof(float));
    m->buf3 = (float *)calloc((size_t)big, sizeof(float));
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
    free(m->h); free(m->xn); free(m->buf); free(m->buf2); free(m->buf3); free(m->logits);
    free(m);
}

/* y = W x in the canonical fixed-point arithmetic, rows split over threads (row results do not depend on it). */
static void gemv(orc_model * m, const orc_t * w, const float * x, float * y) {
    const int rows = w->rows, cols = w->cols, fmt = w->type;
    const int k = fmt == ORC_Q5_K || fmt == ORC_Q6_K;
    int8_t * q = (int8_t *)malloc((size_t)cols);
    uint16_t * d16 = NULL;
    float * d32 = NULL;
    int16_t * bs = NULL;
    if (k) {
        d32 = (float *)malloc(sizeof(float) * (size_t)(cols / 256));
        bs = (int16_t *)malloc(sizeof(int16_t) * (size_t)(cols / 16));
        orc_quantize_q8_K(x, cols, q, d32, bs);
    } else if (fmt == ORC_Q4_1) { /* Q8_1: the fp16 s bits travel in bs */
        d16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(cols / 32));
        bs = (int16_t *)malloc(sizeof(int16_t) * (size_t)(cols / 32));
        orc_quantize_q8_1(x, cols, q, d16, (uint16_t *)bs);
    } else {
        d16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(cols / 32));
        orc_quantize_q8_0(x, cols, q, d16);
    }
    const size_t rb = orc_row_bytes(fmt, cols);
    const int chunk = 64;
    const int nchunks = (rows + chunk - 1) / chunk;
#pragma omp parallel for schedule(dynamic, 4) num_threads(m->n_threads)
    for (int c = 0; c < nchunks; ++c) {
        const int r0 = c * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
        orc_fx_gemv_q(fmt, (const uint8_t *)w->data + (size_t)r0 * rb, q, d16, d32, bs, r1 - r0, cols, y + r0, NULL,
                      NULL);
    }
    free(q); free(d16); free(d32); free(bs);
}

static void rmsnorm(const float * x, const orc_t * w, int n, float eps, float * y) {
    orc_rownorm(x, (const float *)w->data, n, 1, 0, eps, 0, y);
}

int orc_model_decode(void * mp, int token, int pos, float * logits) {
    orc_model * m = (orc_model *)mp;
    const orc_qw_config * c = &m->c;
    if (!m || token < 0 || token >= c->n_vocab || pos < 0 || pos >= c->n_ctx) return -1;
    const int E = c->n_embd, hd = c->head_dim, nh = c->n_head, nkv = c->n_head_kv;
    const int S = c->ssm_head_dim, hk = c->ssm_k_heads, hv = c->ssm_v_heads;
    const int ch = 2 * hk * S + hv * S;
    /* embedding: one Q6_K row dequantized */
    orc_dequant_row_q6_K((const uint8_t *)m->tok_embd.data + orc_row_bytes(ORC_Q6_K, E) * (size_t)token, E, m->h);
    float * cs = (float *)malloc(sizeof(float) * (size_t)c->n_rot);
    orc_rope_cache(pos, c->n_rot, c->rope_base, cs);
    for (int il = 0; il < c->n_layer; ++il) {
        orc_layer * L = &m->layers[il];
        rmsnorm(m->h, &L->attn_norm, E, c->eps, m->xn);
        if (L->attn) {
            /* q (+ gate interleaved per head: [q 0..hd), gate hd..2hd)), k, v */
            float * qg = m->buf, * kv = m->buf2;
            gemv(m, &L->wq, m->xn, qg);
            gemv(m, &L->wk, m->xn, kv);
            gemv(m, &L->wv, m->xn, kv + nkv * hd);
            float * qn = m->buf3;   /* [nh][hd] normed + roped q */
            float * tmp = (float *)malloc(sizeof(float) * (size_t)hd * (nh > nkv ? nh : nkv));
            orc_rownorm(qg, (const float *)L->q_norm.data, hd, nh, 2 * hd, c->eps, 0, tmp);
            orc_rope(tmp, cs, c->n_rot, hd, nh, qn);
            orc_rownorm(kv, (const float *)L->k_norm.data, hd, nkv, 0, c->eps, 0, tmp);
            float * kr = (float *)malloc(sizeof(float) * (size_t)nkv * hd);
            orc_rope(tmp, cs, c->n_rot, hd, nkv, kr);
            uint16_t * kc = m->kcache[il] + (size_t)pos * nkv * hd, * vc = m->vcache[il] + (size_t)pos * nkv * hd;
            for (int i = 0; i < nkv * hd; ++i) {
                kc[i] = orc_float_to_half(kr[i]);
                vc[i] = orc_float_to_half(kv[nkv * hd + i]);
            }
            float * att = (float *)malloc(sizeof(float) * (size_t)nh * hd);
            orc_attn(qn, m->kcache[il], m->vcache[il], nh, nkv, hd, pos + 1, 1.0f / sqrtf((float)hd), att);
            /* output gate: sigmoid(gate) * att (SILU_MUL with the sigmoid flag) */
            float * gate = (float *)malloc(sizeof(float) * (size_t)nh * hd);
            for (int h = 0; h < nh; ++h) memcpy(gate + h * hd, qg + (size_t)h * 2 * hd + hd, sizeof(float) * hd);
            orc_silu_mul(gate, att, nh * hd, 1, m->xn);
            gemv(m, &L->wo, m->xn, m->buf);
            for (int i = 0; i < E; ++i) m->h[i] = m->buf[i] + m->h[i];
            free(tmp); free(kr); free(att); free(gate);
        } else {
            float * qkv = m->buf, * z = m->buf2, * ba = m->buf3;
            gemv(m, &L->qkv, m->xn, qkv);
            gemv(m, &L->z, m->xn, z);
            gemv(m, &L->beta, m->xn, ba);
            gemv(m, &L->alpha, m->xn, ba + hv);
            float * cy = (float *)malloc(sizeof(float) * (size_t)ch);
            float * ns = (float *)malloc(sizeof(float) * (size_t)ch * 3);
            orc_conv(m->conv_state[il], qkv, (const float *)L->conv1d.data, ch, 1, cy, ns);
            memcpy(m->conv_state[il], ns, sizeof(float) * (size_t)ch * 3);
            float * y = (float *)malloc(sizeof(float) * (size_t)hv * S);
            orc_gdn(m->ssm_state[il], cy, cy + hk * S, cy + 2 * hk * S, ba + hv, ba, (const float *)L->dt.data,
                    (const float *)L->a.data, z, (const float *)L->ssm_norm.data, hv, hk, 1.0f / sqrtf((float)S),
                    c->eps, c->eps, 2 | 4 | 8, y);
            gemv(m, &L->ssm_out, y, m->xn);
            for (int i = 0; i < E; ++i) m->h[i] = m->xn[i] + m->h[i];
            free(cy); free(ns); free(y);
        }
        /* FFN: post norm, gate/up, SwiGLU, down + residual */
        rmsnorm(m->h, &L->post_norm, E, c->eps, m->xn);
        gemv(m, &L->gate, m->xn, m->buf);
        gemv(m, &L->up, m->xn, m->buf2);
        orc_silu_mul(m->buf, m->buf2, c->n_ff, 0, m->buf3);
        gemv(m, &L->down, m->buf3, m->buf);
        for (int i = 0; i < E; ++i) m->h[i] = m->buf[i] + m->h[i];
    }
    free(cs);
    rmsnorm(m->h, &m->output_norm, E, c->eps, m->xn);
    gemv(m, &m->output, m->xn, m->logits);
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)c->n_vocab);
    return orc_argmax(m->logits, c->n_vocab);
}

const float * orc_model_hidden(void * mp) { return ((orc_model *)mp)->h; }
