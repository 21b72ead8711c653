/* cpvo_glue.c — rms_norm, RoPE and masked GQA attention.
 * Test infrastructure only (see cpvo.h).  Build with -ffp-contract=off. */
#include "cpvo.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <limits.h>

static int ceil_log2_i(int64_t v)
{
    int b = 0;
    while (((int64_t)1 << b) < v) b++;
    return b;
}

/* ggml_rms_norm + ggml_mul(weight), as built at qwen35.rs:2534-2537,3025-3028.
 * ggml sums the f32 squares in a double accumulator, then
 *   mean = (float)(sum / n); scale = 1.0f / sqrtf(mean + eps); y = x * scale
 * and the following ggml_mul multiplies by the weight in f32.  The sum here
 * is exact rather than sequential: each f32 square goes into an int64 window
 * 2^-(62 - ceil(log2(n+1))) below the largest possible square, so the result
 * is the same for any summation order and equals ggml's double sum rounded
 * to f32 except within ~2^-40 of a tie. */
void cpvo_rms_norm(const float* x, int64_t n, float eps, const float* w, float* y)
{
    float amax = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    double sum = 0.0;
    if (amax > 0.0f) {
        int e;
        frexpf(amax, &e);
        const int g = 2 * e - (62 - ceil_log2_i(n + 1));
        int64_t S = 0;
        for (int64_t i = 0; i < n; i++) {
            const float sq = x[i] * x[i];
            S += (int64_t)floor(ldexp((double)sq, -g));
        }
        sum = ldexp((double)S, g);
    }
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) {
        float v = x[i] * scale;
        y[i] = w ? v * w[i] : v;
    }
}

/* ggml's rope cache for IMROPE (ggml_rope_multi, mode GGML_ROPE_TYPE_IMROPE,
 * qwen35.rs:3053-3062) with text positions: the t/h/w streams all carry pos
 * and the fourth stream 0 (fill_inputs, qwen35.rs:3542-3548).  Per pair i the
 * interleaved section rule picks a stream; theta follows ggml's recurrence
 * theta_{i+1} = theta_i * theta_scale in f32 with theta_scale =
 * powf(freq_base, -2/n_rot); freq_scale = 1, ext_factor = 0, attn_factor = 1
 * make rope_yarn return (cosf(theta), sinf(theta)).  sections == NULL means
 * every pair uses pos (plain NEOX rope). */
static void rope_row(int64_t pos, int n_rot, float theta_scale, const int32_t* sections, float* cs)
{
    float th_t = (float)pos, th_h = (float)pos, th_w = (float)pos, th_e = 0.0f;
    int sect_dims = 0;
    if (sections) sect_dims = sections[0] + sections[1] + sections[2] + sections[3];
    for (int i = 0; i < n_rot / 2; i++) {
        float theta = th_t;
        if (sections && sect_dims > 0) {
            int s = i % sect_dims;
            if (s % 3 == 1 && s < 3 * sections[1]) theta = th_h;
            else if (s % 3 == 2 && s < 3 * sections[2]) theta = th_w;
            else if (s % 3 == 0 && s < 3 * sections[0]) theta = th_t;
            else theta = th_e;
        }
        cs[2 * i + 0] = cosf(theta);
        cs[2 * i + 1] = sinf(theta);
        th_t *= theta_scale;
        th_h *= theta_scale;
        th_w *= theta_scale;
        th_e *= theta_scale;
    }
}

void cpvo_rope_table(int n_pos, int n_rot, float freq_base, float* cs)
{
    const float theta_scale = powf(freq_base, -2.0f / (float)n_rot);
    for (int p = 0; p < n_pos; p++) rope_row(p, n_rot, theta_scale, NULL, cs + (int64_t)p * n_rot);
}

void cpvo_rope_table_sections(int n_pos, int n_rot, float freq_base, const int32_t* sections,
                              float* cs)
{
    const float theta_scale = powf(freq_base, -2.0f / (float)n_rot);
    for (int p = 0; p < n_pos; p++) rope_row(p, n_rot, theta_scale, sections, cs + (int64_t)p * n_rot);
}

/* NEOX pair rotation (x[i], x[i + n_rot/2]), products rounded before the
 * add/sub; dims past n_rot are left as they are. */
void cpvo_rope_neox(float* x, int n_rot, const float* cs)
{
    const int h = n_rot / 2;
    for (int i = 0; i < h; i++) {
        const float c = cs[2 * i], s = cs[2 * i + 1];
        const float x0 = x[i], x1 = x[i + h];
        const float a = x0 * c, b = x1 * s, d = x0 * s, e = x1 * c;
        x[i] = a - b;
        x[i + h] = d + e;
    }
}

/* ggml_flash_attn_ext with an f16 mask (qwen35.rs:3182-3187).  ggml's CPU
 * kernel converts Q to f16 before the dot with the f16 cache; that rounding
 * is kept.  Everything after it is evaluated in binary64, which makes this
 * the closed-form reference the GPU kernel is held to within a tolerance. */
static float f16_tab[65536];
static int f16_tab_ready;

static void f16_tab_init(void)
{
    if (f16_tab_ready) return;
#pragma omp critical(cpvo_f16_tab)
    if (!f16_tab_ready) {
        for (int i = 0; i < 65536; i++) f16_tab[i] = cpvo_fp16_to_fp32((uint16_t)i);
        f16_tab_ready = 1;
    }
}

void cpvo_attn_f64(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t n_past,
               const int32_t* parent, int T, int H, int Hkv, int D, float scale, float* out)
{
    const int g = H / Hkv;
    const int64_t row = (int64_t)Hkv * D;
    const int64_t nmax = n_past + T;
    f16_tab_init();
    /* each (t, h) row is independent: the result does not depend on the thread count */
#pragma omp parallel
    {
        double* s = malloc(sizeof(double) * (size_t)nmax);
        char* vis = malloc((size_t)T);
        double* qd = malloc(sizeof(double) * (size_t)D);
        double* o = malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic)
        for (int th = 0; th < T * H; th++) {
            const int t = th / H, h = th % H;
            memset(vis, 0, (size_t)T);
            for (int a = t; a >= 0; a = parent ? parent[a] : a - 1) vis[a] = 1;
            const int kh = h / g;
            for (int d = 0; d < D; d++)
                qd[d] = (double)f16_tab[cpvo_fp32_to_fp16(q[((int64_t)t * H + h) * D + d])];
            double mx = -INFINITY;
            for (int64_t r = 0; r < nmax; r++) {
                if (r >= n_past && !vis[r - n_past]) { s[r] = -INFINITY; continue; }
                const uint16_t* kr = kc + r * row + (int64_t)kh * D;
                double acc = 0.0;
                for (int d = 0; d < D; d++) acc += qd[d] * (double)f16_tab[kr[d]];
                s[r] = acc * (double)scale;
                if (s[r] > mx) mx = s[r];
            }
            double z = 0.0;
            for (int d = 0; d < D; d++) o[d] = 0.0;
            for (int64_t r = 0; r < nmax; r++) {
                if (s[r] == -INFINITY) continue;
                const double p = exp(s[r] - mx);
                z += p;
                const uint16_t* vr = vc + r * row + (int64_t)kh * D;
                for (int d = 0; d < D; d++) o[d] += p * (double)f16_tab[vr[d]];
            }
            for (int d = 0; d < D; d++) out[((int64_t)t * H + h) * D + d] = (float)(o[d] / z);
        }
        free(s); free(vis); free(qd); free(o);
    }
}

/* The exact-window attention contract (what the device computes, bit for
 * bit, in any launch configuration).  The reference's default attention is
 * ggml_flash_attn_ext with prec F32 (qwen35.rs:534, 3182-3187), whose CPU
 * kernel rounds q to f16 (the f16 cache's vec_dot_type), keeps a running
 * max, weights V by expf(s - max) and divides by the sum of the weights at
 * the end, summing in an order set by its SIMD width (and, for an f16 cache,
 * accumulating V in f16).  This restatement keeps the f16 q and the deferred
 * normalisation and fixes every sum, chunk by chunk:
 *  1. q16 = f16(q).  Per query head, Eq = frexp exponent of max|q16|,
 *     qf = rint(q16 * 2^(14 - Eq)) (|qf| <= 2^14).  Per cache row j and KV
 *     head, Ek = exponent of max|k16|, kf = rint(k16 * 2^(14 - Ek)).  The
 *     score is s_j = (float)(sum_d qf*kf * 2^(Eq + Ek - 28)), the integer sum
 *     exact (|sum| < 2^36); an all-zero q head or k row scores 0.
 *     w_j = s_j * scale (f32).
 *  2. Chunks of CPVO_ATTN_CHUNK consecutive cache rows (absolute row index).
 *     For each chunk c with a visible row: m_c = max of its visible w;
 *     e_j = expf(w_j - m_c) (the glibc expf restatement); its weight in
 *     fixed point p_j = rint(e_j * 2^CPVO_ATTN_PBITS) (an integer in
 *     [0, 2^22]); every f16 cache value v in fixed point at one scale for the
 *     whole cache, vq = rint(v * 2^CPVO_ATTN_VBITS) (|vq| < 2^30, exact for
 *     |v| >= 2^-4, within 2^-15 below); the integer sums over its visible
 *     rows S_c[d] = sum p_j vq_jd (exact in int64, |S| < 2^59) and
 *     Z_c = sum p_j; P_c[d] = (float)S_c[d] * 2^-(PBITS + VBITS) (one
 *     rounding: (float) of the integer, then an exact scaling).
 *  3. M = max m_c; f_c = expf(m_c - M); over the chunks in increasing order
 *     Zt = Zt + (Z_c * 2^-PBITS) * f_c in binary64 from 0, and
 *     O[d] = fmaf(P_c[d], f_c, O[d]) in f32 from +0; out[d] = O[d] * (float)(1 / Zt).
 * Every sum of step 2 is an exact integer sum, so the same bits come out of
 * any order: the device forms it on the int8 MFMA (p and vq as signed 8-bit
 * limbs), from a cache that stores vq's limbs.
 * The f64 attention above is the accuracy reference this is tested against. */
int64_t cpvo_attn_vq(uint16_t h)
{
    return (int64_t)rintf(ldexpf(f16_tab[h], CPVO_ATTN_VBITS));
}

static int64_t ipow_exp(const uint16_t* h, int n)
{
    float mx = 0.0f;
    for (int i = 0; i < n; i++) {
        const float a = fabsf(f16_tab[h[i]]);
        if (a > mx) mx = a;
    }
    int e = INT_MIN;
    if (mx > 0.0f) frexpf(mx, &e);
    return e;
}

void cpvo_attn(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t n_past,
               const int32_t* parent, int T, int H, int Hkv, int D, float scale, float* out)
{
    const int g = H / Hkv;
    const int64_t row = (int64_t)Hkv * D;
    const int64_t nmax = n_past + T;
    const int64_t nchunk = (nmax + CPVO_ATTN_CHUNK - 1) / CPVO_ATTN_CHUNK;
    f16_tab_init();
#pragma omp parallel
    {
        float* w = malloc(sizeof(float) * (size_t)nmax);
        char* vis = malloc((size_t)T);
        uint16_t* q16 = malloc(sizeof(uint16_t) * (size_t)D);
        int64_t* qf = malloc(sizeof(int64_t) * (size_t)D);
        float* P = malloc(sizeof(float) * (size_t)nchunk * D);
        float* mc = malloc(sizeof(float) * (size_t)nchunk);
        int64_t* Zc = malloc(sizeof(int64_t) * (size_t)nchunk);
        int64_t* S = malloc(sizeof(int64_t) * (size_t)D);
#pragma omp for schedule(dynamic)
        for (int th = 0; th < T * H; th++) {
            const int t = th / H, h = th % H, kh = h / g;
            memset(vis, 0, (size_t)T);
            for (int a = t; a >= 0; a = parent ? parent[a] : a - 1) vis[a] = 1;
            for (int d = 0; d < D; d++) q16[d] = cpvo_fp32_to_fp16(q[((int64_t)t * H + h) * D + d]);
            const int64_t eq = ipow_exp(q16, D);
            for (int d = 0; d < D; d++)
                qf[d] = eq == INT_MIN ? 0 : (int64_t)rint(ldexp((double)f16_tab[q16[d]], 14 - (int)eq));
            /* 1: scores, scaled; -inf marks an invisible row */
            for (int64_t r = 0; r < nmax; r++) {
                if (r >= n_past && !vis[r - n_past]) { w[r] = -INFINITY; continue; }
                const uint16_t* kr = kc + r * row + (int64_t)kh * D;
                const int64_t ek = ipow_exp(kr, D);
                float s = 0.0f;
                if (eq != INT_MIN && ek != INT_MIN) {
                    int64_t S = 0;
                    for (int d = 0; d < D; d++)
                        S += qf[d] * (int64_t)rint(ldexp((double)f16_tab[kr[d]], 14 - (int)ek));
                    s = (float)ldexp((double)S, (int)(eq + ek) - 28);
                }
                w[r] = s * scale;
            }
            /* 2: per chunk */
            float M = -INFINITY;
            for (int64_t c = 0; c < nchunk; c++) {
                const int64_t r0 = c * CPVO_ATTN_CHUNK;
                const int64_t r1 = r0 + CPVO_ATTN_CHUNK < nmax ? r0 + CPVO_ATTN_CHUNK : nmax;
                float m = -INFINITY;
                for (int64_t r = r0; r < r1; r++) if (w[r] > m) m = w[r];
                mc[c] = m;
                Zc[c] = 0;
                for (int d = 0; d < D; d++) P[c * D + d] = 0.0f;
                if (m == -INFINITY) continue;
                if (m > M) M = m;
                for (int d = 0; d < D; d++) S[d] = 0;
                for (int64_t r = r0; r < r1; r++) {
                    if (w[r] == -INFINITY) continue;
                    const int64_t p = (int64_t)rintf(ldexpf(cpvo_expf(w[r] - m), CPVO_ATTN_PBITS));
                    Zc[c] += p;
                    const uint16_t* vr = vc + r * row + (int64_t)kh * D;
                    for (int d = 0; d < D; d++) S[d] += p * cpvo_attn_vq(vr[d]);
                }
                for (int d = 0; d < D; d++) P[c * D + d] = ldexpf((float)S[d], -(CPVO_ATTN_PBITS + CPVO_ATTN_VBITS));
            }
            /* 3: fold the chunks in order, normalise once */
            float* o = out + ((int64_t)t * H + h) * D;
            double Zt = 0.0;
            for (int d = 0; d < D; d++) o[d] = 0.0f;
            for (int64_t c = 0; c < nchunk; c++) {
                if (mc[c] == -INFINITY) continue;
                const float f = cpvo_expf(mc[c] - M);
                Zt = Zt + ldexp((double)Zc[c], -CPVO_ATTN_PBITS) * (double)f;
                for (int d = 0; d < D; d++) o[d] = fmaf(P[c * D + d], f, o[d]);
            }
            const float inv = (float)(1.0 / Zt);
            for (int d = 0; d < D; d++) o[d] = o[d] * inv;
        }
        free(w); free(vis); free(q16); free(qf); free(P); free(mc); free(Zc); free(S);
    }
}
