/* cpvo_sample.c — restatement of crates/codpiece-sample/src/lib.rs and of the
 * acceptance loop in crates/codpiece-server/src/engine.rs:2326-2461.
 * Test infrastructure only (see cpvo.h).  Build with -ffp-contract=off.
 *
 * Float semantics follow the Rust source exactly: f32 throughout, sums are
 * sequential folds in candidate order, Rust never fuses a*b+c, f32::max is
 * fmaxf, f32::exp is libm expf (cpvo_expf equals it on every input),
 * f32::ln is libm logf. */
#include "cpvo.h"
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct { int32_t id; float logit; float p; } cand_t;

/* cmp_desc (lib.rs:453-459): logit descending, ties by id ascending */
static int cmp_desc(const void* pa, const void* pb)
{
    const cand_t* a = (const cand_t*)pa;
    const cand_t* b = (const cand_t*)pb;
    if (a->logit > b->logit) return -1;
    if (a->logit < b->logit) return 1;
    return (a->id > b->id) - (a->id < b->id);
}

/* softmax (lib.rs:461-471) */
static void softmax(cand_t* c, int n)
{
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, c[i].logit);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        c[i].p = cpvo_expf(c[i].logit - mx);
        sum += c[i].p;
    }
    for (int i = 0; i < n; i++) c[i].p /= sum;
}

static int penalties_on(const cpvo_sampler_params* p)
{
    return !(p->penalty_repeat == 1.0f && p->penalty_freq == 0.0f && p->penalty_present == 0.0f);
}

/* Sampler::build (lib.rs:229-376).  Returns the candidate count; c must hold V. */
static int build(const cpvo_sampler_params* p, const float* logits, int V, const int32_t* hist,
                 int n_hist, cand_t* c, float* pen)
{
    /* penalties (:233-266): pen[] is a dense copy of the logits with the
     * penalised entries replaced, which is what logit_of() returns */
    const float* lg = logits;
    if (penalties_on(p) && n_hist > 0) {
        memcpy(pen, logits, sizeof(float) * (size_t)V);
        for (int a = 0; a < n_hist; a++) {
            const int32_t tok = hist[a];
            if (tok < 0 || tok >= V) continue;
            int first = 1, count = 0;
            for (int b = 0; b < n_hist; b++) {
                if (hist[b] == tok) {
                    if (b < a) first = 0;
                    count++;
                }
            }
            if (!first) continue;
            float l = logits[tok];
            if (l <= 0.0f) l *= p->penalty_repeat;
            else l /= p->penalty_repeat;
            const float sub = (float)count * p->penalty_freq;
            l -= sub + p->penalty_present;
            pen[tok] = l;
        }
        lg = pen;
    }

    int n = 0;
    if (p->top_k > 0 && p->top_k < V) {                                   /* :272-280 */
        for (int i = 0; i < V; i++) c[i] = (cand_t){i, lg[i], 0.0f};
        int k = p->top_k > p->min_keep ? p->top_k : p->min_keep;
        if (k > V) k = V;
        qsort(c, (size_t)V, sizeof(cand_t), cmp_desc);
        n = k;
    } else if (p->min_p > 0.0f) {                                         /* :281-295 */
        float mx = -INFINITY;
        for (int i = 0; i < V; i++) mx = fmaxf(mx, lg[i]);
        const float floor_l = mx + logf(p->min_p);
        for (int i = 0; i < V; i++)
            if (lg[i] >= floor_l) c[n++] = (cand_t){i, lg[i], 0.0f};
        qsort(c, (size_t)n, sizeof(cand_t), cmp_desc);
    } else if (p->top_p < 1.0f) {                                         /* :296-316 */
        for (int i = 0; i < V; i++) c[i] = (cand_t){i, lg[i], 0.0f};
        softmax(c, V);
        /* select_nth_unstable + sum over the probe: the probe's summation
         * order is implementation-defined in Rust; it is taken here in the
         * sorted (cmp_desc) order, which is what the cut below also uses. */
        qsort(c, (size_t)V, sizeof(cand_t), cmp_desc);
        int probe = 1024 < V ? 1024 : V;
        for (;;) {
            float covered = 0.0f;
            for (int i = 0; i < probe; i++) covered += c[i].p;
            if (covered >= p->top_p || probe >= V) break;
            probe = probe * 8 < V ? probe * 8 : V;
        }
        n = probe;
    } else {                                                              /* :317-322 */
        for (int i = 0; i < V; i++) c[i] = (cand_t){i, lg[i], 0.0f};
        n = V;
    }

    if (p->temp <= 0.0f) {                                                /* :324-337 */
        int best = 0;
        for (int i = 1; i < n; i++)
            if (c[i].logit > c[best].logit) best = i;
        c[0] = c[best];
        c[0].p = 1.0f;
        return 1;
    }

    if (p->top_p < 1.0f && n > 1) {                                       /* :343-358 */
        if (p->top_k > 0 || p->min_p > 0.0f) softmax(c, n);
        float cum = 0.0f;
        int last = n;
        for (int i = 0; i < n; i++) {
            cum += c[i].p;
            if (cum >= p->top_p && i + 1 >= p->min_keep) {
                last = i + 1;
                break;
            }
        }
        n = last;
    }
    if (p->min_p > 0.0f && p->top_k > 0 && n > 1) {                      /* :360-369 */
        const float floor_l = c[0].logit + logf(p->min_p);
        int keep = 1;
        while (keep < n && (c[keep].logit >= floor_l || keep < p->min_keep)) keep++;
        n = keep;
    }
    for (int i = 0; i < n; i++) c[i].logit /= p->temp;                   /* :371-374 */
    softmax(c, n);
    return n;
}

int cpvo_distribution(const cpvo_sampler_params* p, const float* logits, int V, const int32_t* hist,
                      int n_hist, int32_t* ids, float* probs, float* tlogit)
{
    cand_t* c = malloc(sizeof(cand_t) * (size_t)V);
    float* pen = malloc(sizeof(float) * (size_t)V);
    const int n = build(p, logits, V, hist, n_hist, c, pen);
    for (int i = 0; i < n; i++) {
        ids[i] = c[i].id;
        probs[i] = c[i].p;
        if (tlogit) tlogit[i] = c[i].logit;
    }
    free(c);
    free(pen);
    return n;
}

float cpvo_dist_prob_of(const int32_t* ids, const float* probs, int n, int32_t token)
{
    for (int i = 0; i < n; i++)
        if (ids[i] == token) return probs[i];
    return 0.0f;
}

int32_t cpvo_dist_draw(const int32_t* ids, const float* probs, int n, float r)      /* :395-404 */
{
    float cum = 0.0f;
    for (int i = 0; i < n; i++) {
        cum += probs[i];
        if (r < cum) return ids[i];
    }
    return ids[n - 1];
}

int32_t cpvo_dist_draw_excluding(const int32_t* ids, const float* probs, int n, int32_t token,
                                 float r)                                            /* :408-436 */
{
    float total = 0.0f;
    for (int i = 0; i < n; i++)
        if (ids[i] != token) total += probs[i];
    if (total <= 0.0f) return cpvo_dist_draw(ids, probs, n, r);
    const float target = r * total;
    float cum = 0.0f;
    for (int i = 0; i < n; i++) {
        if (ids[i] == token) continue;
        cum += probs[i];
        if (target < cum) return ids[i];
    }
    for (int i = n - 1; i >= 0; i--)
        if (ids[i] != token) return ids[i];
    return ids[n - 1];
}

float cpvo_dist_peak(const float* probs, int n)                                       /* :440-442 */
{
    float m = 0.0f;
    for (int i = 0; i < n; i++) m = fmaxf(m, probs[i]);
    return m;
}

int32_t cpvo_sample_coupled(const cpvo_sampler_params* p, const float* logits, int V,
                            const int32_t* hist, int n_hist, const float* noise_t)  /* :197-216 */
{
    cand_t* c = malloc(sizeof(cand_t) * (size_t)V);
    float* pen = malloc(sizeof(float) * (size_t)V);
    const int n = build(p, logits, V, hist, n_hist, c, pen);
    const float inv_t = 1.0f / fmaxf(p->temp, FLT_MIN);
    float best = -INFINITY;
    int32_t id = n > 0 ? c[0].id : 0;
    for (int i = 0; i < n; i++) {
        const float nz = noise_t[c[i].id] * inv_t;
        const float v = c[i].logit + nz;
        if (v > best) {
            best = v;
            id = c[i].id;
        }
    }
    free(c);
    free(pen);
    return id;
}

/* ggml_argmax / qwen35::argmax (qwen35.rs:3659-3669): first maximum */
int32_t cpvo_argmax(const float* x, int64_t n)
{
    int64_t bi = 0;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (x[i] > bv) { bv = x[i]; bi = i; }
    return (int32_t)bi;
}

float cpvo_softmax_peak_seq(const float* l, int64_t n)      /* engine.rs:2598-2606 */
{
    float m = -INFINITY;
    for (int64_t i = 0; i < n; i++) m = fmaxf(m, l[i]);
    float lse = 0.0f;
    for (int64_t i = 0; i < n; i++) lse += cpvo_expf(l[i] - m);
    return 1.0f / lse;
}

static int32_t argmax_plus(const float* x, const float* nz, int V)
{
    int32_t bi = 0;
    float bv = -INFINITY;
    for (int i = 0; i < V; i++) {
        const float v = x[i] + nz[i];
        if (v > bv) { bv = v; bi = i; }
    }
    return bi;
}

static int coupling_is_exact(const cpvo_sampler_params* p)                         /* :70-78 */
{
    return p->temp > 0.0f && p->top_k == 0 && p->top_p >= 1.0f && p->min_p <= 0.0f &&
           p->penalty_repeat == 1.0f && p->penalty_freq == 0.0f && p->penalty_present == 0.0f;
}

/* the penalty window: Sampler::accept keeps the last penalty_last_n tokens */
typedef struct { int32_t* t; int n, cap; } window_t;

static void window_push(window_t* w, int32_t tok)
{
    if (w->cap <= 0) return;
    if (w->n == w->cap) {
        memmove(w->t, w->t + 1, sizeof(int32_t) * (size_t)(w->n - 1));
        w->n--;
    }
    w->t[w->n++] = tok;
}

/* residual draw of the general rule: r(y) = max(0, p(y) - q(y)) over the
 * target's candidates in the target's order */
static int32_t draw_residual(const int32_t* pid, const float* pp, int pn, const float* qdense, float r)
{
    float total = 0.0f;
    for (int i = 0; i < pn; i++) {
        const float d = pp[i] - qdense[pid[i]];
        total += d > 0.0f ? d : 0.0f;
    }
    if (total <= 0.0f) return cpvo_dist_draw(pid, pp, pn, r);
    const float target = r * total;
    float cum = 0.0f;
    for (int i = 0; i < pn; i++) {
        const float d = pp[i] - qdense[pid[i]];
        cum += d > 0.0f ? d : 0.0f;
        if (target < cum) return pid[i];
    }
    for (int i = pn - 1; i >= 0; i--)
        if (pp[i] - qdense[pid[i]] > 0.0f) return pid[i];
    return pid[pn - 1];
}

int cpvo_spec_accept(const float* p_logits, const float* q_logits, const int32_t* draft, int B,
                     int k, int V, const cpvo_sampler_params* p, int mode, const float* u,
                     const float* noise_t, const int32_t* hist, int hist_len, int32_t* out_tok,
                     int32_t* out_n)
{
    int32_t* pid = malloc(sizeof(int32_t) * (size_t)V);
    float* pp = malloc(sizeof(float) * (size_t)V);
    int32_t* qid = malloc(sizeof(int32_t) * (size_t)V);
    float* qp = malloc(sizeof(float) * (size_t)V);
    float* qdense = calloc((size_t)V, sizeof(float));
    const int cap = p->penalty_last_n;
    int32_t* wbuf = malloc(sizeof(int32_t) * (size_t)(cap > 0 ? cap : 1));
    const int plain = coupling_is_exact(p);

    for (int b = 0; b < B; b++) {
        window_t win = {wbuf, 0, cap};
        for (int a = 0; a < hist_len; a++)
            if (hist && hist[(int64_t)b * hist_len + a] >= 0) window_push(&win, hist[(int64_t)b * hist_len + a]);
        const float* pl = p_logits + (int64_t)b * (k + 1) * V;
        const int32_t* dr = draft + (int64_t)b * k;
        int n_keep = 0, have_rep = 0;
        int32_t rep = 0;
        for (int j = 0; j < k; j++) {
            const float* lj = pl + (int64_t)j * V;
            int keep;
            if (mode == CPVO_ACCEPT_GREEDY) {
                keep = cpvo_argmax(lj, V) == dr[j];
            } else if (mode == CPVO_ACCEPT_GUMBEL) {
                const float* nj = noise_t + ((int64_t)b * (k + 1) + j) * V;
                const int32_t commit = plain ? argmax_plus(lj, nj, V)
                                             : cpvo_sample_coupled(p, lj, V, win.t, win.n, nj);
                keep = dr[j] == commit;
                if (!keep) { rep = commit; have_rep = 1; }
            } else {
                const float u0 = u[((int64_t)b * (k + 1) + j) * 2 + 0];
                const float u1 = u[((int64_t)b * (k + 1) + j) * 2 + 1];
                const int pn = cpvo_distribution(p, lj, V, win.t, win.n, pid, pp, NULL);
                const float px = cpvo_dist_prob_of(pid, pp, pn, dr[j]);
                if (!q_logits) {
                    keep = u0 < px;
                    if (!keep) { rep = cpvo_dist_draw_excluding(pid, pp, pn, dr[j], u1); have_rep = 1; }
                } else {
                    const float* qj = q_logits + ((int64_t)b * k + j) * V;
                    const int qn = cpvo_distribution(p, qj, V, win.t, win.n, qid, qp, NULL);
                    const float qx = cpvo_dist_prob_of(qid, qp, qn, dr[j]);
                    keep = u0 * qx < px;
                    if (!keep) {
                        for (int i = 0; i < qn; i++) qdense[qid[i]] = qp[i];
                        rep = draw_residual(pid, pp, pn, qdense, u1);
                        for (int i = 0; i < qn; i++) qdense[qid[i]] = 0.0f;
                        have_rep = 1;
                    }
                }
            }
            if (!keep) break;
            out_tok[(int64_t)b * (k + 1) + n_keep] = dr[j];
            n_keep++;
            window_push(&win, dr[j]);
        }
        int32_t next;
        const float* ln = pl + (int64_t)n_keep * V;
        if (have_rep) {
            next = rep;
        } else if (mode == CPVO_ACCEPT_GREEDY) {
            next = cpvo_argmax(ln, V);
        } else if (mode == CPVO_ACCEPT_GUMBEL) {
            const float* nn = noise_t + ((int64_t)b * (k + 1) + n_keep) * V;
            next = plain ? argmax_plus(ln, nn, V) : cpvo_sample_coupled(p, ln, V, win.t, win.n, nn);
        } else {
            const int pn = cpvo_distribution(p, ln, V, win.t, win.n, pid, pp, NULL);
            next = cpvo_dist_draw(pid, pp, pn, u[((int64_t)b * (k + 1) + n_keep) * 2 + 0]);
        }
        out_tok[(int64_t)b * (k + 1) + n_keep] = next;
        out_n[b] = n_keep;
    }
    free(pid); free(pp); free(qid); free(qp); free(qdense); free(wbuf);
    return 0;
}

int cpvo_spec_accept_rng(const float* p_logits, const int32_t* draft, int k, int V,
                         const cpvo_sampler_params* p, uint64_t rng[4], const int32_t* hist,
                         int n_hist, int32_t* out_tok, float* u_used)
{
    int32_t* pid = malloc(sizeof(int32_t) * (size_t)V);
    float* pp = malloc(sizeof(float) * (size_t)V);
    const int cap = p->penalty_last_n;
    int32_t* wbuf = malloc(sizeof(int32_t) * (size_t)(cap > 0 ? cap : 1));
    window_t win = {wbuf, 0, cap};
    for (int a = 0; a < n_hist; a++) window_push(&win, hist[a]);
    for (int i = 0; i < 2 * (k + 1); i++) u_used[i] = NAN;
    int n_keep = 0, have_rep = 0;
    int32_t rep = 0;
    for (int j = 0; j < k; j++) {
        const float* lj = p_logits + (int64_t)j * V;
        const int pn = cpvo_distribution(p, lj, V, win.t, win.n, pid, pp, NULL);
        const float roll = cpvo_rng_next_f32(rng);
        u_used[2 * j] = roll;
        if (!(roll < cpvo_dist_prob_of(pid, pp, pn, draft[j]))) {
            const float r = cpvo_rng_next_f32(rng);
            u_used[2 * j + 1] = r;
            rep = cpvo_dist_draw_excluding(pid, pp, pn, draft[j], r);
            have_rep = 1;
            break;
        }
        out_tok[n_keep++] = draft[j];
        window_push(&win, draft[j]);
    }
    if (have_rep) {
        out_tok[n_keep] = rep;
    } else {
        const int pn = cpvo_distribution(p, p_logits + (int64_t)n_keep * V, V, win.t, win.n, pid, pp, NULL);
        const float r = cpvo_rng_next_f32(rng);
        u_used[2 * n_keep] = r;
        out_tok[n_keep] = cpvo_dist_draw(pid, pp, pn, r);
    }
    free(pid); free(pp); free(wbuf);
    return n_keep;
}
