/* cpvo_model.c — CPU restatement of the qwen35 verify round and the fused
 * speculative loop.  Test infrastructure only (see cpvo.h).
 *
 * Follows crates/codpiece-model/src/qwen35.rs for an all-attention model
 * (full_attention_interval = 1): build_inner :2445-2786, build_attn_block
 * :3000-3198, the LM head and argmax :2788-2821, the fused MTP chain
 * :2840-2962, step_fused_cached's position / mask / window rules :1693-1948;
 * and crates/codpiece-cli/src/main.rs:643-931 (cmd_fused) for the loop. */
#include "cpvo.h"
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct { int type; uint8_t* data; int64_t ne0, ne1; } wt_t;

/* a planted mistake (cpvo.h), 0 in every normal use */
static int g_fault = 0;
void cpvo_set_fault(int code) { g_fault = code; }
/* attention in binary64 (cpvo_attn_f64) instead of the exact chunked contract */
static int g_attn_f64 = 0;
void cpvo_set_attn_f64(int on) { g_attn_f64 = on; }
/* mul_mat on the unquantized f32 activation rows, summed in binary64 */
static int g_smooth = 0;
void cpvo_set_smooth(int on) { g_smooth = on; }
/* threads of the round's GEMMs and attention */
static int g_threads = 8;
void cpvo_set_threads(int n)
{
    g_threads = n > 0 ? n : 1;
    omp_set_num_threads(g_threads);
}

typedef struct {
    wt_t wq, wk, wv, wo, gate, up, down;
    float *attn_norm, *post_norm, *q_norm, *k_norm;
} layer_t;

struct cpvo_model {
    cpvo_hparams hp;
    layer_t* L;
    int nl_total;
    wt_t tok_embd, output, eh_proj, mtp_embed, mtp_head;
    float *output_norm, *enorm, *hnorm, *mtp_head_norm;
};

struct cpvo_session {
    cpvo_model* m;
    int64_t n_ctx, mtp_ctx, n_past, mtp_past;
    uint16_t** kc;
    uint16_t** vc;
    float* rope;
    /* attention injection: when set, each attention call's output is checked
     * against the injected one (2e-5 + 2e-4|ref| per element) and replaced by it */
    const float* inj;
    int64_t inj_cap, inj_off;
    double inj_ratio;
};

cpvo_model* cpvo_model_create(const cpvo_hparams* hp)
{
    cpvo_model* m = calloc(1, sizeof *m);
    m->hp = *hp;
    m->nl_total = hp->n_layer + (hp->has_mtp ? 1 : 0);
    m->L = calloc((size_t)m->nl_total, sizeof(layer_t));
    return m;
}

static void wt_free(wt_t* w) { free(w->data); }

void cpvo_model_free(cpvo_model* m)
{
    if (!m) return;
    for (int i = 0; i < m->nl_total; i++) {
        layer_t* L = &m->L[i];
        wt_free(&L->wq); wt_free(&L->wk); wt_free(&L->wv); wt_free(&L->wo);
        wt_free(&L->gate); wt_free(&L->up); wt_free(&L->down);
        free(L->attn_norm); free(L->post_norm); free(L->q_norm); free(L->k_norm);
    }
    free(m->L);
    wt_free(&m->tok_embd); wt_free(&m->output); wt_free(&m->eh_proj);
    wt_free(&m->mtp_embed); wt_free(&m->mtp_head);
    free(m->output_norm); free(m->enorm); free(m->hnorm); free(m->mtp_head_norm);
    free(m);
}

int cpvo_model_set(cpvo_model* m, const char* name, int type, const void* data, int64_t ne0, int64_t ne1)
{
    const int64_t rb = cpvo_row_bytes(type, ne0);
    if (rb < 0) return -1;
    const size_t bytes = (size_t)(rb * ne1);
    wt_t w = {type, malloc(bytes), ne0, ne1};
    memcpy(w.data, data, bytes);
    float* f = (float*)w.data;
    int il = -1;
    char rest[128] = {0};
    const int blk = sscanf(name, "blk.%d.%127s", &il, rest) == 2;
#define NORM(dst) do { if (type != CPVO_F32 || ne1 != 1) { free(w.data); return -1; } (dst) = f; return 0; } while (0)
#define LIN(dst) do { (dst) = w; return 0; } while (0)
    if (!strcmp(name, "token_embd.weight")) LIN(m->tok_embd);
    if (!strcmp(name, "output.weight")) LIN(m->output);
    if (!strcmp(name, "output_norm.weight")) NORM(m->output_norm);
    if (!blk || il < 0 || il >= m->nl_total) { free(w.data); return -1; }
    layer_t* L = &m->L[il];
    if (!strcmp(rest, "attn_norm.weight")) NORM(L->attn_norm);
    if (!strcmp(rest, "post_attention_norm.weight")) NORM(L->post_norm);
    if (!strcmp(rest, "attn_q_norm.weight")) NORM(L->q_norm);
    if (!strcmp(rest, "attn_k_norm.weight")) NORM(L->k_norm);
    if (!strcmp(rest, "attn_q.weight")) LIN(L->wq);
    if (!strcmp(rest, "attn_k.weight")) LIN(L->wk);
    if (!strcmp(rest, "attn_v.weight")) LIN(L->wv);
    if (!strcmp(rest, "attn_output.weight")) LIN(L->wo);
    if (!strcmp(rest, "ffn_gate.weight")) LIN(L->gate);
    if (!strcmp(rest, "ffn_up.weight")) LIN(L->up);
    if (!strcmp(rest, "ffn_down.weight")) LIN(L->down);
    if (il == m->hp.n_layer) {
        if (!strcmp(rest, "nextn.eh_proj.weight")) LIN(m->eh_proj);
        if (!strcmp(rest, "nextn.enorm.weight")) NORM(m->enorm);
        if (!strcmp(rest, "nextn.hnorm.weight")) NORM(m->hnorm);
        if (!strcmp(rest, "nextn.embed_tokens.weight")) LIN(m->mtp_embed);
        if (!strcmp(rest, "nextn.shared_head_norm.weight")) NORM(m->mtp_head_norm);
        if (!strcmp(rest, "nextn.shared_head_head.weight")) LIN(m->mtp_head);
    }
#undef NORM
#undef LIN
    free(w.data);
    return -1;
}

/* resolved tensors: output tied to the embedding when absent (qwen35.rs:2789),
 * nextn extras falling back to the trunk's (mtp_graph.rs:60-75) */
static const wt_t* head_w(const cpvo_model* m) { return m->output.data ? &m->output : &m->tok_embd; }
static const wt_t* mtp_embed_w(const cpvo_model* m) { return m->mtp_embed.data ? &m->mtp_embed : &m->tok_embd; }
static const wt_t* mtp_head_w(const cpvo_model* m) { return m->mtp_head.data ? &m->mtp_head : head_w(m); }
static const float* mtp_head_norm(const cpvo_model* m) { return m->mtp_head_norm ? m->mtp_head_norm : m->output_norm; }

cpvo_session* cpvo_session_create(cpvo_model* m, int64_t n_ctx)
{
    cpvo_session* s = calloc(1, sizeof *s);
    s->m = m;
    s->n_ctx = n_ctx;
    s->mtp_ctx = n_ctx < 16384 ? n_ctx : 16384;
    const cpvo_hparams* hp = &m->hp;
    const int64_t row = (int64_t)hp->n_head_kv * hp->head_dim;
    s->kc = calloc((size_t)m->nl_total, sizeof(uint16_t*));
    s->vc = calloc((size_t)m->nl_total, sizeof(uint16_t*));
    for (int i = 0; i < m->nl_total; i++) {
        const int64_t rows = i == hp->n_layer ? s->mtp_ctx : n_ctx;
        s->kc[i] = calloc((size_t)(rows * row), 2);
        s->vc[i] = calloc((size_t)(rows * row), 2);
    }
    if (hp->n_rot > 0) {
        s->rope = malloc(sizeof(float) * (size_t)((n_ctx + 2) * hp->n_rot));
        cpvo_rope_table_sections((int)(n_ctx + 2), hp->n_rot, hp->freq_base, hp->rope_sections, s->rope);
    }
    return s;
}

void cpvo_session_free(cpvo_session* s)
{
    if (!s) return;
    for (int i = 0; i < s->m->nl_total; i++) { free(s->kc[i]); free(s->vc[i]); }
    free(s->kc); free(s->vc); free(s->rope); free(s);
}

void cpvo_session_set_pos(cpvo_session* s, int64_t n_past, int64_t mtp_past) { s->n_past = n_past; s->mtp_past = mtp_past; }

void cpvo_session_set_attn_inject(cpvo_session* s, const float* att, int64_t n_floats)
{
    s->inj = att;
    s->inj_cap = n_floats;
    s->inj_off = 0;
    s->inj_ratio = 0.0;
}

double cpvo_session_inject_ratio(const cpvo_session* s) { return s->inj_ratio; }
void cpvo_session_get_pos(const cpvo_session* s, int64_t* n_past, int64_t* mtp_past)
{
    *n_past = s->n_past;
    *mtp_past = s->mtp_past;
}

static void mm(const wt_t* w, const float* x, int T, float* y)
{
    if (!g_smooth) {
        cpvo_qgemm(w->type, w->data, w->ne1, w->ne0, x, T, y, g_threads);
        return;
    }
    const int64_t K = w->ne0, rb = cpvo_row_bytes(w->type, K);
    #pragma omp parallel for num_threads(g_threads)
    for (int64_t n = 0; n < w->ne1; n++) {
        float* wr = malloc(sizeof(float) * (size_t)K);
        cpvo_dequantize(w->type, w->data + n * rb, K, wr);
        for (int t = 0; t < T; t++) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; k++) acc += (double)wr[k] * (double)x[(int64_t)t * K + k];
            y[(int64_t)t * w->ne1 + n] = (float)acc;
        }
        free(wr);
    }
}

static void rms_rows(const float* x, int T, int n, int64_t xs, const float* w, float eps, float* y, int64_t ys)
{
    for (int t = 0; t < T; t++) cpvo_rms_norm(x + t * xs, n, eps, w, y + t * ys);
}

/* one attention block + FFN block of layer L on x (in place) */
static void block(cpvo_session* s, const layer_t* L, float* x, int T, int64_t rope_pos0, int64_t kv_row0,
                  int64_t attn_past, uint16_t* kc, uint16_t* vc, int write)
{
    const cpvo_hparams* hp = &s->m->hp;
    const int E = hp->n_embd, hd = hp->head_dim, H = hp->n_head, Hkv = hp->n_head_kv, F = hp->n_ff;
    float* xn = malloc(sizeof(float) * (size_t)T * E);
    float* qg = malloc(sizeof(float) * (size_t)T * 2 * H * hd);
    float* kk = malloc(sizeof(float) * (size_t)T * Hkv * hd);
    float* vv = malloc(sizeof(float) * (size_t)T * Hkv * hd);
    float* q = malloc(sizeof(float) * (size_t)T * H * hd);
    float* att = malloc(sizeof(float) * (size_t)T * H * hd);
    float* o = malloc(sizeof(float) * (size_t)T * E);
    float* up = malloc(sizeof(float) * (size_t)T * F);
    float* gt = malloc(sizeof(float) * (size_t)T * F);
    float tmp[128];
    rms_rows(x, T, E, E, L->attn_norm, hp->rms_eps, xn, E);
    mm(&L->wq, xn, T, qg);
    mm(&L->wk, xn, T, kk);
    mm(&L->wv, xn, T, vv);
    for (int t = 0; t < T; t++) {
        const float* cs = s->rope ? s->rope + (rope_pos0 + t) * hp->n_rot : NULL;
        for (int h = 0; h < H; h++) {
            /* Q is the first hd of each head's 2*hd slot; the gate the second (:3029-3045) */
            cpvo_rms_norm(qg + ((int64_t)t * H + h) * 2 * hd + (g_fault == 1 ? hd : 0), hd, hp->rms_eps, L->q_norm,
                          tmp);
            if (cs) cpvo_rope_neox(tmp, hp->n_rot, cs);
            memcpy(q + ((int64_t)t * H + h) * hd, tmp, sizeof(float) * (size_t)hd);
        }
        for (int kh = 0; kh < Hkv; kh++) {
            cpvo_rms_norm(kk + ((int64_t)t * Hkv + kh) * hd, hd, hp->rms_eps, L->k_norm, tmp);
            if (cs) cpvo_rope_neox(tmp, hp->n_rot, cs);
            if (write) {
                const int64_t r = (kv_row0 + t) * Hkv * hd + (int64_t)kh * hd;
                for (int i = 0; i < hd; i++) {
                    kc[r + i] = cpvo_fp32_to_fp16(tmp[i]);
                    vc[r + i] = cpvo_fp32_to_fp16(vv[((int64_t)t * Hkv + kh) * hd + i]);
                }
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    (g_attn_f64 ? cpvo_attn_f64 : cpvo_attn)(q, kc, vc, attn_past, NULL, T, H, Hkv, hd, scale, att);
    if (s->inj) {
        const int64_t n = (int64_t)T * H * hd;
        if (s->inj_off + n <= s->inj_cap) {
            const float* src = s->inj + s->inj_off;
            for (int64_t i = 0; i < n; i++) {
                const double tol = 2e-5 + 2e-4 * fabs((double)att[i]);
                const double r = fabs((double)src[i] - (double)att[i]) / tol;
                if (!(r <= s->inj_ratio)) s->inj_ratio = r;   /* NaN propagates */
                att[i] = src[i];
            }
        } else {
            s->inj_ratio = INFINITY;
        }
        s->inj_off += n;
    }
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++)
            for (int i = 0; i < hd; i++) {
                const float g = qg[((int64_t)t * H + h) * 2 * hd + (g_fault == 1 ? 0 : hd) + i];
                const float sig = 1.0f / (1.0f + cpvo_expf(-g));
                if (g_fault != 2) att[((int64_t)t * H + h) * hd + i] *= sig;
            }
    mm(&L->wo, att, T, o);
    if (g_fault == 2 && H * hd == E)
        for (int t = 0; t < T; t++)
            for (int i = 0; i < H * hd; i++) {
                const float g = qg[((int64_t)t * H + i / hd) * 2 * hd + hd + i % hd];
                o[(int64_t)t * E + i] *= 1.0f / (1.0f + cpvo_expf(-g));
            }
    for (int64_t e = 0; e < (int64_t)T * E; e++) x[e] = o[e] + x[e];
    if (g_fault == 5) memcpy(xn, x, sizeof(float) * (size_t)T * E);
    else rms_rows(x, T, E, E, L->post_norm, hp->rms_eps, xn, E);
    mm(&L->up, xn, T, up);
    mm(&L->gate, xn, T, gt);
    for (int64_t e = 0; e < (int64_t)T * F; e++) {
        const float g = gt[e];
        const float si = g / (1.0f + cpvo_expf(-g));
        gt[e] = si * up[e];
    }
    mm(&L->down, gt, T, o);
    for (int64_t e = 0; e < (int64_t)T * E; e++) x[e] = o[e] + x[e];
    free(xn); free(qg); free(kk); free(vv); free(q); free(att); free(o); free(up); free(gt);
}

static void embed(const wt_t* w, const int32_t* tok, int T, float* x)
{
    const int64_t rb = cpvo_row_bytes(w->type, w->ne0);
    for (int t = 0; t < T; t++) cpvo_dequantize(w->type, w->data + (int64_t)tok[t] * rb, w->ne0, x + (int64_t)t * w->ne0);
}

int cpvo_prefill(cpvo_session* s, const int32_t* tok, int T)
{
    const cpvo_model* m = s->m;
    if (s->n_past + T > s->n_ctx) return -1;
    float* x = malloc(sizeof(float) * (size_t)T * m->hp.n_embd);
    embed(&m->tok_embd, tok, T, x);
    for (int il = 0; il < m->hp.n_layer; il++)
        block(s, &m->L[il], x, T, s->n_past, s->n_past, s->n_past, s->kc[il], s->vc[il], 1);
    s->n_past += T;
    free(x);
    return 0;
}

static float peak(const float* l, int64_t V)
{
    float mx = -INFINITY;
    for (int64_t i = 0; i < V; i++) mx = fmaxf(mx, l[i]);
    double sum = 0.0;
    for (int64_t i = 0; i < V; i++) sum += (double)cpvo_expf(l[i] - mx);
    return 1.0f * (float)(1.0 / sum);
}

/* The draft head over a shortlist (MtpTail::n_cand, qwen35.rs:208-216): each
 * link's logits are the head's rows `cands` (get_rows then mul_mat,
 * :2925-2931; the same values as the full head's columns, rows being
 * independent), its argmax and softmax peak are over those n_cand logits, the
 * reported draft is cands[argmax] (:1904-1910) and, as in the graph, the next
 * link embeds the argmax itself (`tok_src = ids`, :2958). */
int cpvo_verify_step_cands(cpvo_session* s, const int32_t* tok, int T, int depth, const float* noise,
                           const int32_t* cands, int n_cand, int32_t* preds, int32_t* chain, float* conf,
                           float* logits_out, float* hidden_out);

int cpvo_verify_step(cpvo_session* s, const int32_t* tok, int T, int depth, const float* noise, int32_t* preds,
                     int32_t* chain, float* conf, float* logits_out, float* hidden_out)
{
    return cpvo_verify_step_cands(s, tok, T, depth, noise, NULL, 0, preds, chain, conf, logits_out, hidden_out);
}

int cpvo_verify_step_cands(cpvo_session* s, const int32_t* tok, int T, int depth, const float* noise,
                           const int32_t* cands, int n_cand, int32_t* preds, int32_t* chain, float* conf,
                           float* logits_out, float* hidden_out)
{
    const cpvo_model* m = s->m;
    const cpvo_hparams* hp = &m->hp;
    const int64_t E = hp->n_embd, V = hp->n_vocab;
    if (s->n_past + T > s->n_ctx) return -1;
    if (s->mtp_past + T > s->mtp_ctx) s->mtp_past = 0;
    float* x = malloc(sizeof(float) * (size_t)(T * E));
    float* h = malloc(sizeof(float) * (size_t)(T * E));
    float* logits = malloc(sizeof(float) * (size_t)(T * V));
    embed(&m->tok_embd, tok, T, x);
    for (int il = 0; il < hp->n_layer; il++)
        block(s, &m->L[il], x, T, s->n_past, s->n_past, s->n_past, s->kc[il], s->vc[il], 1);
    rms_rows(x, T, (int)E, E, m->output_norm, hp->rms_eps, h, E);
    mm(head_w(m), h, T, logits);
    for (int t = 0; t < T; t++) {
        if (noise) {
            int32_t bi = 0;
            float bv = -INFINITY;
            for (int64_t i = 0; i < V; i++) {
                const float v = logits[t * V + i] + noise[t * V + i];
                if (v > bv) { bv = v; bi = (int32_t)i; }
            }
            preds[t] = bi;
        } else {
            preds[t] = cpvo_argmax(logits + t * V, V);
        }
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)(T * V));
    if (hidden_out) memcpy(hidden_out, h, sizeof(float) * (size_t)(T * E));
    if (depth > 0) {
        const layer_t* ML = &m->L[hp->n_layer];
        float* hsrc = malloc(sizeof(float) * (size_t)(T * E));
        float* e = malloc(sizeof(float) * (size_t)(T * E));
        float* cat = malloc(sizeof(float) * (size_t)(T * 2 * E));
        float* d = malloc(sizeof(float) * (size_t)(T * E));
        int32_t* tsrc = malloc(sizeof(int32_t) * (size_t)T);
        memcpy(hsrc, h, sizeof(float) * (size_t)(T * E));
        memcpy(tsrc, preds, sizeof(int32_t) * (size_t)T);
        for (int step = 0; step < depth; step++) {
            embed(mtp_embed_w(m), tsrc, T, e);
            const int64_t eo = g_fault == 3 ? E : 0;
            rms_rows(e, T, (int)E, E, g_fault == 6 ? m->hnorm : m->enorm, hp->rms_eps, cat + eo, 2 * E);
            rms_rows(hsrc, T, (int)E, E, g_fault == 6 ? m->enorm : m->hnorm, hp->rms_eps, cat + E - eo, 2 * E);
            mm(&m->eh_proj, cat, T, d);
            block(s, ML, d, T, s->n_past + 1, s->mtp_past, s->mtp_past, s->kc[hp->n_layer], s->vc[hp->n_layer],
                  step == 0);
            rms_rows(d, T, (int)E, E, mtp_head_norm(m), hp->rms_eps, hsrc, E);
            mm(mtp_head_w(m), hsrc, T, logits);
            if (g_fault == 4) memcpy(hsrc, d, sizeof(float) * (size_t)(T * E));
            for (int t = 0; t < T; t++) {
                if (cands && n_cand > 0) {
                    float* lc = malloc(sizeof(float) * (size_t)n_cand);
                    for (int j = 0; j < n_cand; j++) lc[j] = logits[t * V + cands[j]];
                    const int32_t idx = cpvo_argmax(lc, n_cand);
                    chain[step * T + t] = cands[idx];
                    if (conf) conf[step * T + t] = peak(lc, n_cand);
                    tsrc[t] = idx;
                    free(lc);
                } else {
                    chain[step * T + t] = cpvo_argmax(logits + t * V, V);
                    if (conf) conf[step * T + t] = peak(logits + t * V, V);
                    tsrc[t] = chain[step * T + t];
                }
            }
        }
        free(hsrc); free(e); free(cat); free(d); free(tsrc);
    }
    s->n_past += T;
    free(x); free(h); free(logits);
    return 0;
}

/* Qwen35::mtp_draft (qwen35.rs:2086-2192) on the graph of build_mtp_impl
 * (mtp_graph.rs:123-249): the link of the round's chain for one row, except
 * that its K/V row is written at mtp_past (row_ids, :2177-2181), it attends
 * rows 0..mtp_past (the mask, :2163-2174), its rope position is the caller's
 * `pos` (:2161), and mtp_past advances by 1 (:2189). */
int cpvo_mtp_draft(cpvo_session* s, const float* hidden, int32_t token, int64_t pos, float* logits_out,
                   float* hidden_out)
{
    const cpvo_model* m = s->m;
    const cpvo_hparams* hp = &m->hp;
    const int64_t E = hp->n_embd;
    if (!hp->has_mtp || s->mtp_past + 1 > s->mtp_ctx || pos < 0 || pos > s->n_ctx + 1) return -1;
    if (token < 0 || token >= hp->n_vocab) return -1;
    float* e = malloc(sizeof(float) * (size_t)E);
    float* cat = malloc(sizeof(float) * (size_t)(2 * E));
    float* d = malloc(sizeof(float) * (size_t)E);
    embed(mtp_embed_w(m), &token, 1, e);
    const int64_t eo = g_fault == 3 ? E : 0;
    rms_rows(e, 1, (int)E, E, g_fault == 6 ? m->hnorm : m->enorm, hp->rms_eps, cat + eo, 2 * E);
    rms_rows(hidden, 1, (int)E, E, g_fault == 6 ? m->enorm : m->hnorm, hp->rms_eps, cat + E - eo, 2 * E);
    mm(&m->eh_proj, cat, 1, d);
    block(s, &m->L[hp->n_layer], d, 1, pos, s->mtp_past, s->mtp_past, s->kc[hp->n_layer], s->vc[hp->n_layer], 1);
    rms_rows(d, 1, (int)E, E, mtp_head_norm(m), hp->rms_eps, hidden_out, E);
    mm(mtp_head_w(m), hidden_out, 1, logits_out);
    if (g_fault == 4) memcpy(hidden_out, d, sizeof(float) * (size_t)E);
    s->mtp_past += 1;
    free(e); free(cat); free(d);
    return 0;
}

/* cmd_fused (crates/codpiece-cli/src/main.rs:643-931) at a fixed depth, no
 * EOS (the seeded model has no tokenizer): bulk prefill through the trunk,
 * the last `tail` prompt tokens through a round, then rounds of
 * [last] + drafts with greedy acceptance and KV rewind.  committed must hold
 * n_gen tokens; stats = {accepted, proposed, rounds}. */
int cpvo_fused_generate(cpvo_session* s, const int32_t* prompt, int n_prompt, int n_gen, int depth, int tail,
                        int bulk, int32_t* committed, int64_t* stats)
{
    const cpvo_hparams* hp = &s->m->hp;
    const int split = n_prompt > tail ? n_prompt - tail : 0;
    for (int c = 0; c < split; c += bulk)
        if (cpvo_prefill(s, prompt + c, split - c < bulk ? split - c : bulk)) return -1;
    const int T0 = n_prompt - split;
    int32_t* preds = malloc(sizeof(int32_t) * (size_t)(T0 > depth + 1 ? T0 : depth + 1));
    int32_t* chain = malloc(sizeof(int32_t) * (size_t)((depth ? depth : 1) * (T0 > depth + 1 ? T0 : depth + 1)));
    if (cpvo_verify_step(s, prompt + split, T0, depth, NULL, preds, chain, NULL, NULL, NULL)) return -1;
    s->mtp_past += T0;
    int n = 0;
    committed[n++] = preds[T0 - 1];
    int32_t drafts[16];
    int nd = depth;
    for (int l = 0; l < depth; l++) drafts[l] = chain[l * T0 + T0 - 1];
    int64_t accepted = 0, proposed = 0, rounds = 0;
    while (n < n_gen) {
        int32_t batch[17];
        batch[0] = committed[n - 1];
        for (int i = 0; i < nd; i++) batch[1 + i] = drafts[i];
        const int T = nd + 1;
        if (cpvo_verify_step(s, batch, T, depth, NULL, preds, chain, NULL, NULL, NULL)) return -1;
        rounds++;
        proposed += nd;
        int keep = 0;
        while (keep < nd && preds[keep] == drafts[keep]) keep++;
        accepted += keep;
        int done = 0;
        for (int i = 0; i < keep; i++) {
            committed[n++] = drafts[i];
            if (n >= n_gen) { done = 1; break; }
        }
        if (done) break;
        committed[n++] = preds[keep];
        for (int l = 0; l < depth; l++) drafts[l] = chain[l * T + keep];
        nd = depth;
        const int over = T - (keep + 1);
        s->mtp_past += keep + 1;
        if (over > 0) s->n_past -= over;
    }
    (void)hp;
    stats[0] = accepted;
    stats[1] = proposed;
    stats[2] = rounds;
    free(preds);
    free(chain);
    return n;
}
