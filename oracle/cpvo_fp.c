/* cpvo_fp.c — scalar contracts of the oracle: fp16, exp, Philox, xoshiro.
 * Test infrastructure only (see cpvo.h).  Build with -ffp-contract=off. */
#include "cpvo.h"
#include <math.h>
#include <string.h>

/* IEEE binary32 -> binary16, round to nearest even (GGML_FP32_TO_FP16). */
uint16_t cpvo_fp32_to_fp16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                                           /* fp16 normal */
        uint32_t mant = ax & 0x7fffffu;
        uint32_t h = (((ax >> 23) - 112u) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;                      /* < 2^-25 -> 0 */
    uint32_t e = ax >> 23;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;                                         /* 14..24 */
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float cpvo_fp16_to_fp32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    uint32_t x;
    if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (mant << 13);
    } else if (exp == 0u) {
        float v = ldexpf((float)mant, -24);
        return sign ? -v : v;
    } else {
        x = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void cpvo_fp32_to_fp16_n(const float* x, int64_t n, uint16_t* y)
{
    for (int64_t i = 0; i < n; i++) y[i] = cpvo_fp32_to_fp16(x[i]);
}

void cpvo_fp16_to_fp32_n(const uint16_t* x, int64_t n, float* y)
{
    for (int64_t i = 0; i < n; i++) y[i] = cpvo_fp16_to_fp32(x[i]);
}

/* expf restated from the table-driven algorithm glibc (>= 2.27) ships, which
 * it takes from ARM's optimized-routines: k = round(x * 32/ln2), r = the
 * remainder, e^x = 2^(k/32) * p(r) with a 32-entry table of 2^(i/32) (stored
 * minus i<<47 so the exponent can be added as an integer) and a cubic p with
 * the published minimax coefficients, everything in binary64 with the fused
 * multiply-adds glibc's FMA build uses, then one rounding to f32.  The
 * reference's Rust f32::exp calls libm expf; cpvo_expf_vs_libm checks the two
 * agree on every f32 input (tests/test_oracle_fp.py); the table entries are
 * the correctly rounded doubles of 2^(i/32), which that test regenerates. */
static const uint64_t CPVO_EXP2_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

float cpvo_expf(float x)
{
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = CPVO_EXP2_TAB[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

void cpvo_exp_table(uint64_t out[32])
{
    memcpy(out, CPVO_EXP2_TAB, sizeof CPVO_EXP2_TAB);
}

void cpvo_expf_n(const float* x, int64_t n, float* y)
{
    for (int64_t i = 0; i < n; i++) y[i] = cpvo_expf(x[i]);
}

int64_t cpvo_expf_vs_libm(float lo, float hi, int64_t stride)
{
    /* walk the float bit patterns between lo and hi (same sign or spanning 0) */
    int64_t bad = 0;
    uint32_t ulo, uhi;
    if (stride < 1) stride = 1;
    /* negative half: bit patterns of -|x| grow with |x| */
    if (lo < 0.0f) {
        float a = hi < 0.0f ? -hi : 0.0f, b = -lo;
        memcpy(&ulo, &a, 4);
        memcpy(&uhi, &b, 4);
        #pragma omp parallel for reduction(+:bad) schedule(static)
        for (int64_t u = ulo; u <= (int64_t)uhi; u += stride) {
            uint32_t bits = (uint32_t)u | 0x80000000u;
            float x;
            memcpy(&x, &bits, 4);
            float a1 = cpvo_expf(x), a2 = expf(x);
            if (memcmp(&a1, &a2, 4) != 0) bad++;
        }
    }
    if (hi >= 0.0f) {
        float a = lo > 0.0f ? lo : 0.0f, b = hi;
        memcpy(&ulo, &a, 4);
        memcpy(&uhi, &b, 4);
        #pragma omp parallel for reduction(+:bad) schedule(static)
        for (int64_t u = ulo; u <= (int64_t)uhi; u += stride) {
            uint32_t bits = (uint32_t)u;
            float x;
            memcpy(&x, &bits, 4);
            float a1 = cpvo_expf(x), a2 = expf(x);
            if (memcmp(&a1, &a2, 4) != 0) bad++;
        }
    }
    return bad;
}

/* ---- Philox4x64-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers:
 * as easy as 1, 2, 3", SC'11).  Round function and constants are the paper's;
 * numpy.random.Philox implements the same generator. */
static inline void mulhilo64(uint64_t a, uint64_t b, uint64_t* hi, uint64_t* lo)
{
    unsigned __int128 p = (unsigned __int128)a * b;
    *hi = (uint64_t)(p >> 64);
    *lo = (uint64_t)p;
}

void cpvo_philox4x64(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4])
{
    uint64_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint64_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; round++) {
        uint64_t hi0, lo0, hi1, lo1;
        mulhilo64(0xD2E7470EE14C6C93ull, c0, &hi0, &lo0);
        mulhilo64(0xCA5A826395121157ull, c2, &hi1, &lo1);
        uint64_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B97F4A7C15ull;
        k1 += 0xBB67AE8584CAA73Bull;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float cpvo_u01(uint64_t x)
{
    return (float)(x >> 40) / (float)(1u << 24);
}

void cpvo_philox_uniforms(uint64_t seed, uint64_t round, int B, int k, float* u)
{
    uint64_t key[2] = {seed, 0};
    for (int b = 0; b < B; b++)
        for (int j = 0; j <= k; j++)
            for (int r = 0; r < 2; r++) {
                uint64_t ctr[4] = {(uint64_t)b, (uint64_t)j, (uint64_t)r, round}, out[4];
                cpvo_philox4x64(ctr, key, out);
                u[((int64_t)b * (k + 1) + j) * 2 + r] = cpvo_u01(out[0]);
            }
}

/* ---- xoshiro256++ via splitmix64 (crates/codpiece-sample/src/lib.rs:98-130) */
void cpvo_rng_seed(uint64_t seed, uint64_t s[4])
{
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    for (int i = 0; i < 4; i++) {
        z += 0x9E3779B97F4A7C15ull;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        s[i] = x ^ (x >> 31);
    }
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t cpvo_rng_next_u64(uint64_t s[4])
{
    uint64_t r = rotl64(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return r;
}

float cpvo_rng_next_f32(uint64_t s[4])
{
    return cpvo_u01(cpvo_rng_next_u64(s));
}
