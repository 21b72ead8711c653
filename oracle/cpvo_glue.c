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

void cpvo_attn(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t n_past,
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
