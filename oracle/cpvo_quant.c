/* cpvo_quant.c — ggml block formats and the quantized GEMM contract.
 * Test infrastructure only (see cpvo.h).  Build with -ffp-contract=off.
 *
 * Block formats follow ggml's published layouts (GGUF type ids and sizes are
 * pinned by crates/codpiece-gguf/src/lib.rs:173-185,545-550).  The call sites
 * are ggml_mul_mat in crates/codpiece-model/src/qwen35.rs:2779-2782,2797,
 * 3029,3047,3051,3197 and ggml_get_rows at :2545,2794. */
#include "cpvo.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <limits.h>

int64_t cpvo_type_block(int type)
{
    switch (type) {
    case CPVO_F32: case CPVO_F16: return 1;
    case CPVO_Q8_0: return 32;
    case CPVO_Q4_K: case CPVO_Q6_K: case CPVO_Q8_K: return 256;
    default: return -1;
    }
}

int64_t cpvo_type_size(int type)
{
    switch (type) {
    case CPVO_F32: return 4;
    case CPVO_F16: return 2;
    case CPVO_Q8_0: return 34;
    case CPVO_Q4_K: return 144;
    case CPVO_Q6_K: return 210;
    case CPVO_Q8_K: return 292;
    default: return -1;
    }
}

int64_t cpvo_row_bytes(int type, int64_t k)
{
    int64_t b = cpvo_type_block(type);
    if (b <= 0 || k % b) return -1;
    return k / b * cpvo_type_size(type);
}

static inline int nearest_int(float x) { return (int)rintf(x); }

/* ---- Q8_0: quantize_row_q8_0_ref (d = amax/127, q = roundf(x/d)) -------- */
void cpvo_quantize_q8_0(const float* x, int64_t n, cpvo_block_q8_0* y)
{
    for (int64_t i = 0; i < n / 32; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = fabsf(x[i * 32 + j]);
            amax = v > amax ? v : amax;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = cpvo_fp32_to_fp16(d);
        for (int j = 0; j < 32; j++) y[i].qs[j] = (int8_t)roundf(x[i * 32 + j] * id);
    }
}

/* ---- Q8_K: quantize_row_q8_K_ref (iscale = -127/max, the signed element of
 * largest magnitude, first occurrence; q = nearest_int; d = 1/iscale) ----- */
void cpvo_quantize_q8_K(const float* x, int64_t n, cpvo_block_q8_K* y)
{
    for (int64_t i = 0; i < n / 256; i++) {
        const float* xb = x + i * 256;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 256; j++) {
            float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(y[i]));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < 256; j++) {
            int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[j * 16 + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* ---- Q4_K ---------------------------------------------------------------- */
static inline void scale_min_k4(int j, const uint8_t* q, int* sc, int* m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* A valid Q4_K encoder: per 32-sub-block min/max fit, 6-bit scales and mins
 * relative to the super-block maxima, 4-bit codes.  ggml's own encoder adds an
 * iterative search (make_qkx2_quants); parity only needs both sides to read
 * the same bytes, so that search is not restated. */
static void quantize_q4_K(const float* x, int64_t n, cpvo_block_q4_K* y)
{
    for (int64_t i = 0; i < n / 256; i++) {
        const float* xb = x + i * 256;
        float scales[8], mins[8], max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            float mn = xb[j * 32], mx = xb[j * 32];
            for (int l = 1; l < 32; l++) {
                float v = xb[j * 32 + l];
                mn = v < mn ? v : mn;
                mx = v > mx ? v : mx;
            }
            if (mn > 0.0f) mn = 0.0f;
            scales[j] = (mx - mn) / 15.0f;
            mins[j] = -mn;
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            int a = nearest_int(inv_scale * scales[j]), b = nearest_int(inv_min * mins[j]);
            ls[j] = (uint8_t)(a > 63 ? 63 : a);
            lm[j] = (uint8_t)(b > 63 ? 63 : b);
        }
        memset(y[i].scales, 0, 12);
        for (int j = 0; j < 8; j++) {
            if (j < 4) {
                y[i].scales[j] = ls[j];
                y[i].scales[j + 4] = lm[j];
            } else {
                y[i].scales[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
                y[i].scales[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
                y[i].scales[j] |= (uint8_t)((lm[j] >> 4) << 6);
            }
        }
        y[i].d = cpvo_fp32_to_fp16(max_scale / 63.0f);
        y[i].dmin = cpvo_fp32_to_fp16(max_min / 63.0f);
        uint8_t L[256];
        for (int j = 0; j < 8; j++) {
            int sc, m;
            scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = cpvo_fp16_to_fp32(y[i].d) * (float)sc;
            const float dm = cpvo_fp16_to_fp32(y[i].dmin) * (float)m;
            for (int l = 0; l < 32; l++) {
                int v = d != 0.0f ? nearest_int((xb[j * 32 + l] + dm) / d) : 0;
                L[j * 32 + l] = (uint8_t)(v < 0 ? 0 : v > 15 ? 15 : v);
            }
        }
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++)
                y[i].qs[c * 32 + l] = (uint8_t)(L[c * 64 + l] | (L[c * 64 + l + 32] << 4));
    }
}

/* integer view of one Q4_K super-block: codes in element order, 6-bit
 * scales and mins per 32-sub-block */
static void unpack_q4_K(const cpvo_block_q4_K* b, int8_t q[256], int sc[8], int m[8])
{
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            q[c * 64 + l] = (int8_t)(b->qs[c * 32 + l] & 0xF);
            q[c * 64 + l + 32] = (int8_t)(b->qs[c * 32 + l] >> 4);
        }
    for (int j = 0; j < 8; j++) scale_min_k4(j, b->scales, &sc[j], &m[j]);
}

/* dequantize_row_q4_K: y = (d*sc)*q - (dmin*m), f32, no fused multiply-add */
static void dequant_q4_K(const cpvo_block_q4_K* x, int64_t n, float* y)
{
    for (int64_t i = 0; i < n / 256; i++) {
        int8_t q[256];
        int sc[8], m[8];
        unpack_q4_K(&x[i], q, sc, m);
        const float d = cpvo_fp16_to_fp32(x[i].d), mn = cpvo_fp16_to_fp32(x[i].dmin);
        for (int j = 0; j < 8; j++) {
            const float d1 = d * (float)sc[j], m1 = mn * (float)m[j];
            for (int l = 0; l < 32; l++) y[i * 256 + j * 32 + l] = d1 * (float)q[j * 32 + l] - m1;
        }
    }
}

/* ---- Q6_K ---------------------------------------------------------------- */
/* A valid Q6_K encoder: per 16-group signed-max scale, int8 group scales
 * relative to the super-block's largest (iscale = -128/max, as ggml), 6-bit
 * codes.  ggml's make_qx_quants refinement is not restated (see Q4_K). */
static void quantize_q6_K(const float* x, int64_t n, cpvo_block_q6_K* y)
{
    for (int64_t i = 0; i < n / 256; i++) {
        const float* xb = x + i * 256;
        float scales[16], max_scale = 0.0f, max_abs = 0.0f;
        for (int g = 0; g < 16; g++) {
            float amax = 0.0f, mx = 0.0f;
            for (int l = 0; l < 16; l++) {
                float v = xb[g * 16 + l];
                if (fabsf(v) > amax) { amax = fabsf(v); mx = v; }
            }
            scales[g] = amax > 0.0f ? -mx / 32.0f : 0.0f;
            if (fabsf(scales[g]) > max_abs) { max_abs = fabsf(scales[g]); max_scale = scales[g]; }
        }
        memset(&y[i], 0, sizeof(y[i]));
        uint8_t L[256];
        if (max_abs == 0.0f) {
            memset(L, 32, sizeof L);
        } else {
            const float iscale = -128.0f / max_scale;
            y[i].d = cpvo_fp32_to_fp16(1.0f / iscale);
            for (int g = 0; g < 16; g++) {
                int v = nearest_int(iscale * scales[g]);
                y[i].scales[g] = (int8_t)(v > 127 ? 127 : v < -128 ? -128 : v);
            }
            for (int g = 0; g < 16; g++) {
                const float d = cpvo_fp16_to_fp32(y[i].d) * (float)y[i].scales[g];
                for (int l = 0; l < 16; l++) {
                    int v = d != 0.0f ? nearest_int(xb[g * 16 + l] / d) : 0;
                    v = v < -32 ? -32 : v > 31 ? 31 : v;
                    L[g * 16 + l] = (uint8_t)(v + 32);
                }
            }
        }
        for (int h = 0; h < 2; h++) {
            uint8_t* ql = y[i].ql + h * 64;
            uint8_t* qh = y[i].qh + h * 32;
            const uint8_t* Lh = L + h * 128;
            for (int l = 0; l < 32; l++) {
                ql[l] = (uint8_t)((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
                ql[l + 32] = (uint8_t)((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
                qh[l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) |
                                  ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6));
            }
        }
    }
}

/* signed 6-bit codes in element order */
static void unpack_q6_K(const cpvo_block_q6_K* b, int8_t q[256])
{
    for (int h = 0; h < 2; h++) {
        const uint8_t* ql = b->ql + h * 64;
        const uint8_t* qh = b->qh + h * 32;
        int8_t* o = q + h * 128;
        for (int l = 0; l < 32; l++) {
            o[l] = (int8_t)(((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
            o[l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
            o[l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            o[l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
        }
    }
}

/* dequantize_row_q6_K: y = (d*sc)*q, f32, evaluated left to right */
static void dequant_q6_K(const cpvo_block_q6_K* x, int64_t n, float* y)
{
    for (int64_t i = 0; i < n / 256; i++) {
        int8_t q[256];
        unpack_q6_K(&x[i], q);
        const float d = cpvo_fp16_to_fp32(x[i].d);
        for (int e = 0; e < 256; e++) y[i * 256 + e] = d * (float)x[i].scales[e / 16] * (float)q[e];
    }
}

int cpvo_quantize(int type, const float* x, int64_t n, void* out)
{
    if (cpvo_row_bytes(type, n) < 0) return -1;
    switch (type) {
    case CPVO_F32: memcpy(out, x, (size_t)n * 4); return 0;
    case CPVO_F16: cpvo_fp32_to_fp16_n(x, n, (uint16_t*)out); return 0;
    case CPVO_Q8_0: cpvo_quantize_q8_0(x, n, (cpvo_block_q8_0*)out); return 0;
    case CPVO_Q4_K: quantize_q4_K(x, n, (cpvo_block_q4_K*)out); return 0;
    case CPVO_Q6_K: quantize_q6_K(x, n, (cpvo_block_q6_K*)out); return 0;
    case CPVO_Q8_K: cpvo_quantize_q8_K(x, n, (cpvo_block_q8_K*)out); return 0;
    default: return -1;
    }
}

int cpvo_dequantize(int type, const void* q, int64_t n, float* y)
{
    if (cpvo_row_bytes(type, n) < 0) return -1;
    switch (type) {
    case CPVO_F32: memcpy(y, q, (size_t)n * 4); return 0;
    case CPVO_F16: cpvo_fp16_to_fp32_n((const uint16_t*)q, n, y); return 0;
    case CPVO_Q8_0: {
        const cpvo_block_q8_0* b = (const cpvo_block_q8_0*)q;
        for (int64_t i = 0; i < n / 32; i++) {
            const float d = cpvo_fp16_to_fp32(b[i].d);
            for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)b[i].qs[j] * d;
        }
        return 0;
    }
    case CPVO_Q4_K: dequant_q4_K((const cpvo_block_q4_K*)q, n, y); return 0;
    case CPVO_Q6_K: dequant_q6_K((const cpvo_block_q6_K*)q, n, y); return 0;
    case CPVO_Q8_K: {
        const cpvo_block_q8_K* b = (const cpvo_block_q8_K*)q;
        for (int64_t i = 0; i < n / 256; i++)
            for (int j = 0; j < 256; j++) y[i * 256 + j] = b[i].d * (float)b[i].qs[j];
        return 0;
    }
    default: return -1;
    }
}

/* ---- quantized GEMM: the exact-window contract ---------------------------
 *
 * ggml's CPU mul_mat quantizes each activation row to vec_dot_type (Q8_0 for
 * Q8_0 weights, Q8_K for K-quants) and sums per-block integer dots scaled by
 * the block scales.  That much is fixed by the formats.  The order in which
 * ggml then adds the per-block f32 products differs between its generic, AVX2
 * and CUDA builds, so no single ggml order exists to follow.  This contract
 * removes order from the result instead:
 *
 *   for each output (m, n) and each unit u along K (a Q8_0 block of 32, a
 *   K-quant super-block of 256):
 *     isum_u   exact integer   (Q8_0: sum q_w q_a;  Q4_K: sum_j sc_j dot_j;
 *                               Q6_K: sum_g sc_g dot_g)
 *     imin_u   exact integer   (Q4_K only: sum_j m_j * bsum_j)
 *     A_u    = (double)d_w * (double)d_a * 2^-g          exact in binary64
 *     S     += rint(A_u * (double)isum_u)                an integer
 *              (Q4_K: S -= rint(B_u * (double)imin_u),
 *               B_u = (double)dmin_w * (double)d_a * 2^-g)
 *   y = (float)(S * 2^g)
 *
 * The window g = Ew(n) + Ea(m) - W, with Ew / Ea the frexp exponents of the
 * largest weight-row / activation-row scale magnitude and
 * W = 52 - isum_bits - ceil(log2(terms + 1)), bounds |S| < 2^53: S is an
 * integer exactly representable in binary64, so it can be accumulated in
 * int64 or in double, in any order and split any way over lanes, waves or
 * workgroups, with the same result.  The grid sits ~2^-45 below the largest
 * possible term; for real data y is the correctly rounded quantized dot
 * product except within ~2^-10 ulp of a rounding tie. */
static int isum_bits(int type) { return type == CPVO_Q8_0 ? 20 : type == CPVO_Q4_K ? 25 : 28; }

static int64_t n_terms(int type, int64_t K)
{
    return type == CPVO_Q8_0 ? K / 32 : type == CPVO_Q4_K ? 2 * (K / 256) : K / 256;
}

static int ceil_log2(int64_t v)
{
    int b = 0;
    while (((int64_t)1 << b) < v) b++;
    return b;
}

int cpvo_qgemm_window(int type, int64_t K)
{
    return 52 - isum_bits(type) - ceil_log2(n_terms(type, K) + 1);
}

#define CPVO_E_EMPTY INT_MIN
static int exp_of(float v)
{
    if (!(v > 0.0f)) return CPVO_E_EMPTY;
    int e;
    frexpf(v, &e);
    return e;
}

static inline int64_t fx_round(double t) { return (int64_t)rint(t); }

static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int n)
{
    int32_t s = 0;
    for (int i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

int cpvo_qgemm(int type, const void* w, int64_t N, int64_t K, const float* x, int64_t M,
               float* y, int n_threads)
{
    if (type != CPVO_Q8_0 && type != CPVO_Q4_K && type != CPVO_Q6_K) return -1;
    if (cpvo_row_bytes(type, K) < 0) return -1;
    const int W = cpvo_qgemm_window(type, K);
    const int64_t rb = cpvo_row_bytes(type, K);
    const int64_t nb = K / cpvo_type_block(type);
    if (n_threads <= 0) n_threads = 1;

    if (type == CPVO_Q8_0) {
        cpvo_block_q8_0* xa = malloc(sizeof(cpvo_block_q8_0) * (size_t)(M * nb));
        int* Ea = malloc(sizeof(int) * (size_t)M);
        float* dta = malloc(sizeof(float) * (size_t)(M * nb));
        for (int64_t m = 0; m < M; m++) {
            cpvo_quantize_q8_0(x + m * K, K, xa + m * nb);
            float mx = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                dta[m * nb + b] = cpvo_fp16_to_fp32(xa[m * nb + b].d);
                float v = fabsf(dta[m * nb + b]);
                mx = v > mx ? v : mx;
            }
            Ea[m] = exp_of(mx);
        }
        #pragma omp parallel for num_threads(n_threads) schedule(dynamic, 16)
        for (int64_t n = 0; n < N; n++) {
            const cpvo_block_q8_0* wr = (const cpvo_block_q8_0*)((const uint8_t*)w + n * rb);
            float mx = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                float v = fabsf(cpvo_fp16_to_fp32(wr[b].d));
                mx = v > mx ? v : mx;
            }
            const int Ew = exp_of(mx);
            for (int64_t m = 0; m < M; m++) {
                if (Ew == CPVO_E_EMPTY || Ea[m] == CPVO_E_EMPTY) { y[m * N + n] = 0.0f; continue; }
                const int g = Ew + Ea[m] - W;
                int64_t S = 0;
                for (int64_t b = 0; b < nb; b++) {
                    const int32_t isum = dot_i8(wr[b].qs, xa[m * nb + b].qs, 32);
                    double A = ldexp((double)cpvo_fp16_to_fp32(wr[b].d) * (double)dta[m * nb + b], -g);
                    S += fx_round(A * (double)isum);
                }
                y[m * N + n] = (float)ldexp((double)S, g);
            }
        }
        free(xa); free(Ea); free(dta);
        return 0;
    }

    /* K-quants: activations in Q8_K */
    cpvo_block_q8_K* xa = malloc(sizeof(cpvo_block_q8_K) * (size_t)(M * nb));
    int* Ea = malloc(sizeof(int) * (size_t)M);
    for (int64_t m = 0; m < M; m++) {
        cpvo_quantize_q8_K(x + m * K, K, xa + m * nb);
        float mx = 0.0f;
        for (int64_t b = 0; b < nb; b++) {
            float v = fabsf(xa[m * nb + b].d);
            mx = v > mx ? v : mx;
        }
        Ea[m] = exp_of(mx);
    }
    #pragma omp parallel for num_threads(n_threads) schedule(dynamic, 16)
    for (int64_t n = 0; n < N; n++) {
        const uint8_t* wr = (const uint8_t*)w + n * rb;
        int8_t q[256];
        float mx = 0.0f;
        for (int64_t b = 0; b < nb; b++) {
            if (type == CPVO_Q4_K) {
                const cpvo_block_q4_K* bl = (const cpvo_block_q4_K*)wr + b;
                float v1 = fabsf(cpvo_fp16_to_fp32(bl->d)), v2 = fabsf(cpvo_fp16_to_fp32(bl->dmin));
                mx = v1 > mx ? v1 : mx;
                mx = v2 > mx ? v2 : mx;
            } else {
                const cpvo_block_q6_K* bl = (const cpvo_block_q6_K*)wr + b;
                float v = fabsf(cpvo_fp16_to_fp32(bl->d));
                mx = v > mx ? v : mx;
            }
        }
        const int Ew = exp_of(mx);
        int64_t S[64];
        int gm[64];
        for (int64_t m0 = 0; m0 < M; m0 += 64) {
            const int64_t mc = M - m0 < 64 ? M - m0 : 64;
            for (int64_t mm = 0; mm < mc; mm++) {
                S[mm] = 0;
                gm[mm] = (Ew == CPVO_E_EMPTY || Ea[m0 + mm] == CPVO_E_EMPTY) ? 0 : Ew + Ea[m0 + mm] - W;
            }
            for (int64_t b = 0; b < nb; b++) {
                if (type == CPVO_Q4_K) {
                    const cpvo_block_q4_K* bl = (const cpvo_block_q4_K*)wr + b;
                    int sc[8], mn[8];
                    unpack_q4_K(bl, q, sc, mn);
                    const double dw = cpvo_fp16_to_fp32(bl->d), dmn = cpvo_fp16_to_fp32(bl->dmin);
                    for (int64_t mm = 0; mm < mc; mm++) {
                        const cpvo_block_q8_K* a = &xa[(m0 + mm) * nb + b];
                        int32_t isum = 0, imin = 0;
                        for (int j = 0; j < 8; j++) {
                            isum += sc[j] * dot_i8(q + j * 32, a->qs + j * 32, 32);
                            imin += mn[j] * (a->bsums[2 * j] + a->bsums[2 * j + 1]);
                        }
                        const double A = ldexp(dw * (double)a->d, -gm[mm]);
                        const double Bm = ldexp(dmn * (double)a->d, -gm[mm]);
                        S[mm] += fx_round(A * (double)isum);
                        S[mm] -= fx_round(Bm * (double)imin);
                    }
                } else {
                    const cpvo_block_q6_K* bl = (const cpvo_block_q6_K*)wr + b;
                    unpack_q6_K(bl, q);
                    const double dw = cpvo_fp16_to_fp32(bl->d);
                    for (int64_t mm = 0; mm < mc; mm++) {
                        const cpvo_block_q8_K* a = &xa[(m0 + mm) * nb + b];
                        int32_t isum = 0;
                        for (int g = 0; g < 16; g++)
                            isum += (int32_t)bl->scales[g] * dot_i8(q + g * 16, a->qs + g * 16, 16);
                        const double A = ldexp(dw * (double)a->d, -gm[mm]);
                        S[mm] += fx_round(A * (double)isum);
                    }
                }
            }
            for (int64_t mm = 0; mm < mc; mm++) {
                const int64_t m = m0 + mm;
                if (Ew == CPVO_E_EMPTY || Ea[m] == CPVO_E_EMPTY) y[m * N + n] = 0.0f;
                else y[m * N + n] = (float)ldexp((double)S[mm], gm[mm]);
            }
        }
    }
    free(xa); free(Ea);
    return 0;
}

void cpvo_mul_mat_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M, float* y)
{
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float s = 0.0f;
            for (int64_t k = 0; k < K; k++) s += w[n * K + k] * x[m * K + k];
            y[m * N + n] = s;
        }
}

/* the same quantized product with every weight and activation value formed
 * in binary64 and summed in binary64 (no f32 rounding anywhere) */
int cpvo_qgemm_f64(int type, const void* w, int64_t N, int64_t K, const float* x, int64_t M,
                   double* y, int n_threads)
{
    if (type != CPVO_Q8_0 && type != CPVO_Q4_K && type != CPVO_Q6_K) return -1;
    if (cpvo_row_bytes(type, K) < 0) return -1;
    const int64_t rb = cpvo_row_bytes(type, K);
    double* xa = malloc(sizeof(double) * (size_t)(M * K));
    for (int64_t m = 0; m < M; m++) {
        if (type == CPVO_Q8_0) {
            cpvo_block_q8_0* t = malloc(sizeof(cpvo_block_q8_0) * (size_t)(K / 32));
            cpvo_quantize_q8_0(x + m * K, K, t);
            for (int64_t k = 0; k < K; k++)
                xa[m * K + k] = (double)cpvo_fp16_to_fp32(t[k / 32].d) * t[k / 32].qs[k % 32];
            free(t);
        } else {
            cpvo_block_q8_K* t = malloc(sizeof(cpvo_block_q8_K) * (size_t)(K / 256));
            cpvo_quantize_q8_K(x + m * K, K, t);
            for (int64_t k = 0; k < K; k++) xa[m * K + k] = (double)t[k / 256].d * t[k / 256].qs[k % 256];
            free(t);
        }
    }
    if (n_threads <= 0) n_threads = 1;
    #pragma omp parallel for num_threads(n_threads)
    for (int64_t n = 0; n < N; n++) {
        double* wv = malloc(sizeof(double) * (size_t)K);
        const uint8_t* wr = (const uint8_t*)w + n * rb;
        for (int64_t b = 0; b < K / cpvo_type_block(type); b++) {
            if (type == CPVO_Q8_0) {
                const cpvo_block_q8_0* bl = (const cpvo_block_q8_0*)wr + b;
                for (int j = 0; j < 32; j++) wv[b * 32 + j] = (double)cpvo_fp16_to_fp32(bl->d) * bl->qs[j];
            } else if (type == CPVO_Q4_K) {
                const cpvo_block_q4_K* bl = (const cpvo_block_q4_K*)wr + b;
                int8_t q[256];
                int sc[8], mn[8];
                unpack_q4_K(bl, q, sc, mn);
                for (int e = 0; e < 256; e++)
                    wv[b * 256 + e] = (double)cpvo_fp16_to_fp32(bl->d) * sc[e / 32] * q[e] -
                                      (double)cpvo_fp16_to_fp32(bl->dmin) * mn[e / 32];
            } else {
                const cpvo_block_q6_K* bl = (const cpvo_block_q6_K*)wr + b;
                int8_t q[256];
                unpack_q6_K(bl, q);
                for (int e = 0; e < 256; e++)
                    wv[b * 256 + e] = (double)cpvo_fp16_to_fp32(bl->d) * bl->scales[e / 16] * q[e];
            }
        }
        for (int64_t m = 0; m < M; m++) {
            double s = 0.0;
            for (int64_t k = 0; k < K; k++) s += wv[k] * xa[m * K + k];
            y[m * N + n] = s;
        }
        free(wv);
    }
    free(xa);
    return 0;
}
