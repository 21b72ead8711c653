// qgemm.hip — fused dequant skinny GEMM for Q4_K / Q6_K / Q8_0 weights.
//
// y[m][n] = x[m][:] . dequant(w[n][:]) for m <= 16 activation rows, the
// ggml_mul_mat of the verify step (crates/codpiece-model/src/qwen35.rs:
// 2779-2782,2797,3029,3047,3051,3197).
//
// Numerics (the exact-window contract, identical to the CPU oracle):
//  * x is quantized per row as ggml's CPU vec_dot_type: Q8_K (f32 scale per
//    256, codes rint(-127/max * x)) for K-quants, Q8_0 (fp16 scale per 32,
//    codes roundf(x / (amax/127))) for Q8_0.
//  * per unit (256-element super-block, or 32-element Q8_0 block) the integer
//    dot is exact (v_dot4_i32_i8), its term A * isum is formed in binary64
//    (A = d_w * d_a * 2^-g is exact) and rounded to an integer; the integers
//    are summed in binary64, exactly because the window g keeps every partial
//    sum below 2^53.  Any split of the K loop gives the same bits.
//
// Mapping.  Weights are repacked in tiles of 64 rows: a wave works on one
// tile at a time, lane = row, and reads each 256-element unit of its row as
// 16-byte pieces, so every load instruction of the wave is one contiguous
// KiB (api.hip).  The integer dots run on the 16-block 4x4x4 int8 MFMA:
// block b of lanes 4b..4b+3 multiplies 4 activation rows (A, from LDS) by the
// 4 weight rows of its lanes (B), so each lane receives the dots of its own
// row with 4 activation rows; a launch takes up to 8 rows (2 row groups).  The
// per-unit scale work and the binary64 rounding then run lane-locally, with
// no cross-lane traffic.  The grid is persistent (one workgroup per CU): the
// (tile, unit) items are dealt out evenly to the workgroups and within each
// to its waves in consecutive runs, so K is split wherever a run starts or
// ends.  A workgroup stages only the activation units its items touch.  The
// partial sums are exact integers below 2^53 and add in any order: the waves
// add theirs into per-tile sums in LDS, and each workgroup then writes a tile
// it covers whole and adds (f64 atomics) a tile it shares into an accumulator
// that a small finalize kernel (or the fused consumer of a kept result) turns
// into y and leaves zeroed for the next launch (no device-scope fence in the
// GEMM: on gfx950 one would write back a whole L2 per workgroup).
#include <math.h>

#include <mutex>

#include "cpv_internal.h"

namespace {

__device__ __forceinline__ float h2f(uint32_t h) { return cpv_h2f((uint16_t)h); }

__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }

// ---------------------------------------------------------------- activations
// Q8_K per 256-element unit: signed element of largest magnitude (first
// occurrence), iscale = -127/max, q = min(127, rint(iscale * x)), d = 1/iscale,
// plus 32- and 16-element code sums.  One block of 256 threads per (unit, row).
__global__ __launch_bounds__(256) void quant_q8k_kernel(const float* __restrict__ x, int64_t K, int U,
                                                        int8_t* __restrict__ qa, float* __restrict__ da,
                                                        int32_t* __restrict__ bs32, int32_t* __restrict__ bs16)
{
    const int u = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int64_t e = (int64_t)u * 256 + t;
    const float v = e < K ? x[(int64_t)m * K + e] : 0.0f;
    __shared__ float sx[256];
    __shared__ float s_ax[4];
    __shared__ int s_ix[4];
    sx[t] = v;
    float ax = fabsf(v), sv = v;
    int ix = t;
    cpv_wave_amax(ax, ix, sv);
    if ((t & 63) == 0) { s_ax[t >> 6] = ax; s_ix[t >> 6] = ix; }
    __syncthreads();
    float amax = s_ax[0];
    int imax = s_ix[0];
    for (int w = 1; w < 4; w++)
        if (s_ax[w] > amax || (s_ax[w] == amax && s_ix[w] < imax)) { amax = s_ax[w]; imax = s_ix[w]; }
    int q = 0;
    float d = 0.0f;
    if (amax > 0.0f) {
        const float iscale = -127.0f / sx[imax];
        const int vq = (int)rintf(iscale * v);
        q = vq < 127 ? vq : 127;
        d = 1.0f / iscale;
    }
    const int64_t Kp = (int64_t)U * 256;
    qa[(int64_t)m * Kp + e] = (int8_t)q;
    const int s16 = cpv_group_reduce<16>(q, cpv_op_add());
    const int s32 = s16 + __shfl_xor(s16, 16);
    if ((t & 15) == 0) bs16[((int64_t)m * U + u) * 16 + (t >> 4)] = s16;
    if ((t & 31) == 0) bs32[((int64_t)m * U + u) * 8 + (t >> 5)] = s32;
    if (t == 0) da[(int64_t)m * U + u] = d;
}

// Q8_0 per 32-element block: d = amax/127, q = roundf(x * (1/d)), d stored as
// fp16 (its f32 value kept).  256 threads = 8 blocks of one 256-unit.
__global__ __launch_bounds__(256) void quant_q80_kernel(const float* __restrict__ x, int64_t K, int U,
                                                        int8_t* __restrict__ qa, float* __restrict__ da)
{
    const int u = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int64_t e = (int64_t)u * 256 + t;
    const float v = e < K ? x[(int64_t)m * K + e] : 0.0f;
    float amax = fabsf(v);
    amax = cpv_group_reduce<16>(amax, cpv_op_max());
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)roundf(v * id);
    const int64_t Kp = (int64_t)U * 256;
    qa[(int64_t)m * Kp + e] = (int8_t)q;
    if ((t & 31) == 0) da[((int64_t)m * U + u) * 8 + (t >> 5)] = cpv_h2f(cpv_f2h(d));
}

// ---------------------------------------------------------------- GEMM
typedef int v4i __attribute__((ext_vector_type(4)));

template <int TYPE>
struct Fmt {
    // 16-byte pieces per (row, unit) in the repacked tile, activation scales
    // per unit, activation code sums per unit
    static constexpr int PIECES = TYPE == CPV_Q4_K ? 9 : TYPE == CPV_Q6_K ? 13 : 17;
    static constexpr int DA = TYPE == CPV_Q8_0 ? 8 : 1;
    static constexpr int BS = TYPE == CPV_Q4_K ? 8 : TYPE == CPV_Q6_K ? 16 : 0;
};

struct GemmArgs {
    const uint8_t* w;      // repacked weight: [tile][unit][piece][lane][16 B] (+ Q6_K d region)
    const int32_t* ew;     // [n_pad] row exponents
    const int8_t* qa;      // [Mtot][U*256] activation codes
    const float* da;       // [Mtot][U*DA]
    const int32_t* bs;     // [Mtot][U*BS]
    double* gsum;          // [rows][n_pad] accumulator (absolute activation rows), zero between uses
    int64_t n_pad;
    int items;             // tiles * U (tile-major)
    int iq, ir;            // items / grid and items % grid: workgroup b takes iq items, one more if b < ir
    double rU;             // 1.0 / U
    int U, M, m0, win;
    int nu_max, nt_max;    // most units / tiles one workgroup's items touch
};

// q = a / d and *r = a % d for 0 <= a < 2^31 and 0 < d < 2^31, with rd the
// binary64 1.0 / d: the estimate is off by at most one, then corrected (no
// integer division, which the scalar unit would run for every wave)
__device__ __forceinline__ int divmod_pos(int a, int d, double rd, int* r)
{
    int q = (int)((double)a * rd);
    int rr = a - q * d;
    if (rr < 0) { q--; rr += d; }
    else if (rr >= d) { q++; rr -= d; }
    *r = rr;
    return q;
}
// the same for 0 <= a < 2^23 and 0 < d < 2^23, with rf an f32 estimate of 1 / d
__device__ __forceinline__ int divmod_small(int a, int d, float rf, int* r)
{
    int q = (int)((float)a * rf);
    int rr = a - q * d;
    if (rr < 0) { q--; rr += d; }
    else if (rr >= d) { q++; rr -= d; }
    *r = rr;
    return q;
}

// waves per workgroup (one workgroup per CU; 12 waves, where registers
// allow 3 per SIMD, measured slower).  Q8_0 above 8 rows: one wave per SIMD,
// the whole register file per wave (its 17-piece items do not fit two).
template <int TYPE, int MC>
constexpr int gemm_waves() { return MC > 8 && TYPE == CPV_Q8_0 ? 4 : 8; }

__device__ __forceinline__ v4i mfma4(int a, int b, v4i c)
{
    return __builtin_amdgcn_mfma_i32_4x4x4i8(a, b, c, 0, 0, 0);
}

// LDS of one workgroup: its nu activation units for M rows (rows of nu*256
// + 16 bytes: 4 rows, 4 bank groups), their scales and code sums, the
// binary64 sums of its nt tiles, and 16 bytes that take the staging writes of
// lanes with nothing to stage (so that the writes need no branch)
template <int TYPE>
__host__ __device__ inline size_t gemm_lds(int M, int nu, int nt)
{
    using F = Fmt<TYPE>;
    const size_t codes = (size_t)M * ((size_t)nu * 256 + 16);
    const size_t da = (size_t)M * nu * F::DA * 4;
    const size_t bs = (size_t)M * nu * F::BS * 4;
    const size_t acc = (size_t)nt * M * 64 * 8;
    return ((codes + 15) & ~(size_t)15) + ((da + 15) & ~(size_t)15) + ((bs + 15) & ~(size_t)15) + acc + 16;
}

// One (tile, unit) item: the unit's integer dots for all MC rows and its
// binary64 terms, added to S.  pcu: the lane's pieces of the unit.
template <int TYPE, int MC>
__device__ __forceinline__ void gemm_unit(const v4i* pcu, uint16_t d6, int er, int u, int M, int U,
                                          const uint8_t* const* arow, const int* mrow, const double* sm,
                                          const float* s_da, const int32_t* s_bs, double* S)
{
    constexpr int RG = (MC + 3) / 4;
    if constexpr (TYPE == CPV_Q4_K) {
        const uint32_t h0 = (uint32_t)pcu[8][0], hy = (uint32_t)pcu[8][1], hz = (uint32_t)pcu[8][2],
                       hw = (uint32_t)pcu[8][3];
        const double dws = ldexp((double)h2f(h0 & 0xffffu), -er);
        const double dms = ldexp((double)h2f(h0 >> 16), -er);
        const uint32_t sc_lo = hy & 0x3f3f3f3fu, mn_lo = hz & 0x3f3f3f3fu;
        const uint32_t sc_hi = (hw & 0x0f0f0f0fu) | (((hy >> 6) & 0x03030303u) << 4);
        const uint32_t mn_hi = ((hw >> 4) & 0x0f0f0f0fu) | (((hz >> 6) & 0x03030303u) << 4);
        int isum[MC], imin[MC];
#pragma unroll
        for (int m = 0; m < MC; m++) {
            // imin = sum_j m_j * (code sum of sub-block j); 6-bit mins times |sums| <= 32*127
            const v4i b0 = *(const v4i*)(s_bs + (mrow[m] * U + u) * 8);
            const v4i b1 = *(const v4i*)(s_bs + (mrow[m] * U + u) * 8 + 4);
            imin[m] = __mul24(byte_of(mn_lo, 0), b0[0]) + __mul24(byte_of(mn_lo, 1), b0[1]) +
                      __mul24(byte_of(mn_lo, 2), b0[2]) + __mul24(byte_of(mn_lo, 3), b0[3]) +
                      __mul24(byte_of(mn_hi, 0), b1[0]) + __mul24(byte_of(mn_hi, 1), b1[1]) +
                      __mul24(byte_of(mn_hi, 2), b1[2]) + __mul24(byte_of(mn_hi, 3), b1[3]);
            isum[m] = 0;
        }
#pragma unroll
        for (int pr = 0; pr < 4; pr++) {
            // sub-blocks 2pr (low nibbles) and 2pr+1 (high nibbles) of qs dwords 8pr..8pr+7: two chains
            v4i De[RG], Do[RG];
#pragma unroll
            for (int r = 0; r < RG; r++) { De[r] = v4i{0, 0, 0, 0}; Do[r] = v4i{0, 0, 0, 0}; }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                v4i Ae[RG], Ao[RG];
#pragma unroll
                for (int r = 0; r < RG; r++) {
                    Ae[r] = *(const v4i*)(arow[r] + u * 256 + pr * 64 + h * 16);
                    Ao[r] = *(const v4i*)(arow[r] + u * 256 + pr * 64 + 32 + h * 16);
                }
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t wv = (uint32_t)pcu[pr * 2 + h][d];
                    const int be = (int)(wv & 0x0f0f0f0fu), bo = (int)((wv >> 4) & 0x0f0f0f0fu);
#pragma unroll
                    for (int r = 0; r < RG; r++) {
                        De[r] = mfma4(Ae[r][d], be, De[r]);
                        Do[r] = mfma4(Ao[r][d], bo, Do[r]);
                    }
                }
            }
            const uint32_t scw = pr < 2 ? sc_lo : sc_hi;
            const int sce = byte_of(scw, (2 * pr) & 3), sco = byte_of(scw, (2 * pr + 1) & 3);
#pragma unroll
            for (int m = 0; m < MC; m++)   // 6-bit scales times |dots| <= 32*15*127: 24-bit products
                isum[m] += __mul24(sce, De[m >> 2][m & 3]) + __mul24(sco, Do[m >> 2][m & 3]);
        }
#pragma unroll
        for (int m = 0; m < MC; m++) {
            const double da = (double)s_da[mrow[m] * U + u] * sm[m];
            S[m] += rint(dws * da * (double)isum[m]) - rint(dms * da * (double)imin[m]);
        }
    } else if constexpr (TYPE == CPV_Q6_K) {
        const double dws = ldexp((double)h2f(d6), -er);
        // isum = sum_g sc_g * (dot_g - 32 * codesum_g); below 8 rows as
        // sum_g sc_g * dot_g less 32 sum_g sc_g * codesum_g, the code-sum term
        // first (the same integer: |terms| < 2^29; at 8 rows the registers
        // for it would spill)
        constexpr bool HOIST = MC < 8;
        int isum[MC];
#pragma unroll
        for (int m = 0; m < MC; m++) {
            isum[m] = 0;
            if constexpr (!HOIST) continue;
            const v4i* bs = (const v4i*)(s_bs + (mrow[m] * U + u) * 16);
            int t = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const v4i b = bs[q];
                const uint32_t scw = (uint32_t)pcu[12][q];
#pragma unroll
                for (int e = 0; e < 4; e++) t += __mul24((int)(int8_t)byte_of(scw, e), b[e]);
            }
            isum[m] = -32 * t;
        }
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
#pragma unroll
            for (int quad = 0; quad < 4; quad++) {
                // 32 elements hf*128 + quad*32 ..: groups g0 = 2(hf*4 + quad) and g0 + 1, two chains
                const int g0 = (hf * 4 + quad) * 2;
                v4i A0[RG], A1[RG], D0[RG], D1[RG];
#pragma unroll
                for (int r = 0; r < RG; r++) {
                    A0[r] = *(const v4i*)(arow[r] + u * 256 + g0 * 16);
                    A1[r] = *(const v4i*)(arow[r] + u * 256 + g0 * 16 + 16);
                    D0[r] = v4i{0, 0, 0, 0};
                    D1[r] = v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t l0 = (uint32_t)pcu[hf * 4 + (quad & 1) * 2][d];
                    const uint32_t l1 = (uint32_t)pcu[hf * 4 + (quad & 1) * 2 + 1][d];
                    const uint32_t q0 = (uint32_t)pcu[8 + hf * 2][d], q1 = (uint32_t)pcu[8 + hf * 2 + 1][d];
                    const uint32_t lo0 = quad < 2 ? (l0 & 0x0f0f0f0fu) : ((l0 >> 4) & 0x0f0f0f0fu);
                    const uint32_t lo1 = quad < 2 ? (l1 & 0x0f0f0f0fu) : ((l1 >> 4) & 0x0f0f0f0fu);
                    const int b0 = (int)(lo0 | (((q0 >> (2 * quad)) & 0x03030303u) << 4));
                    const int b1 = (int)(lo1 | (((q1 >> (2 * quad)) & 0x03030303u) << 4));
#pragma unroll
                    for (int r = 0; r < RG; r++) {
                        D0[r] = mfma4(A0[r][d], b0, D0[r]);
                        D1[r] = mfma4(A1[r][d], b1, D1[r]);
                    }
                }
                const int sc0 = (int)(int8_t)byte_of((uint32_t)pcu[12][g0 >> 2], g0 & 3);
                const int sc1 = (int)(int8_t)byte_of((uint32_t)pcu[12][(g0 + 1) >> 2], (g0 + 1) & 3);
#pragma unroll
                for (int m = 0; m < MC; m++) {
                    // int8 scales times |dot| and |dot - 32 * code sum| < 2^18: 24-bit products
                    if constexpr (HOIST) {
                        isum[m] += __mul24(sc0, D0[m >> 2][m & 3]) + __mul24(sc1, D1[m >> 2][m & 3]);
                    } else {
                        const int32_t* bs = s_bs + (mrow[m] * U + u) * 16 + g0;
                        isum[m] += __mul24(sc0, D0[m >> 2][m & 3] - 32 * bs[0]) +
                                   __mul24(sc1, D1[m >> 2][m & 3] - 32 * bs[1]);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MC; m++) S[m] += rint(dws * ((double)s_da[mrow[m] * U + u] * sm[m]) * (double)isum[m]);
    } else {
        const uint32_t dw[4] = {(uint32_t)pcu[16][0], (uint32_t)pcu[16][1], (uint32_t)pcu[16][2],
                                (uint32_t)pcu[16][3]};
#pragma unroll
        for (int b2 = 0; b2 < 4; b2++) {
            // blocks 2 b2 and 2 b2 + 1: two chains
            v4i D0[RG], D1[RG];
#pragma unroll
            for (int r = 0; r < RG; r++) { D0[r] = v4i{0, 0, 0, 0}; D1[r] = v4i{0, 0, 0, 0}; }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                v4i A0[RG], A1[RG];
#pragma unroll
                for (int r = 0; r < RG; r++) {
                    A0[r] = *(const v4i*)(arow[r] + u * 256 + b2 * 64 + h * 16);
                    A1[r] = *(const v4i*)(arow[r] + u * 256 + b2 * 64 + 32 + h * 16);
                }
#pragma unroll
                for (int d = 0; d < 4; d++)
#pragma unroll
                    for (int r = 0; r < RG; r++) {
                        D0[r] = mfma4(A0[r][d], pcu[b2 * 4 + h][d], D0[r]);
                        D1[r] = mfma4(A1[r][d], pcu[b2 * 4 + 2 + h][d], D1[r]);
                    }
            }
            const double dw0 = ldexp((double)h2f(dw[b2] & 0xffffu), -er);
            const double dw1 = ldexp((double)h2f(dw[b2] >> 16), -er);
#pragma unroll
            for (int m = 0; m < MC; m++) {
                const float* dam = s_da + (mrow[m] * U + u) * 8 + 2 * b2;
                S[m] += rint(dw0 * ((double)dam[0] * sm[m]) * (double)D0[m >> 2][m & 3]) +
                        rint(dw1 * ((double)dam[1] * sm[m]) * (double)D1[m >> 2][m & 3]);
            }
        }
    }
    (void)M;
}

// Persistent streaming GEMM: one workgroup of GEMM_WAVES waves per CU stages
// the activation units of its items in LDS; then each wave walks its own run
// of consecutive (tile, unit) items with the next item's weights in flight
// while it computes the current one, and keeps the partial sums of its
// current tile in registers, adding them to the tile's sums in LDS whenever
// the tile changes and at the end.  MC: a compile-time bound on the
// activation rows (rows M..MC-1 repeat row M-1 and are never stored), so every
// loop over rows unrolls without branches.
template <int TYPE, int MC>
__global__ __launch_bounds__((64 * gemm_waves<TYPE, MC>())) void qgemm_kernel(GemmArgs a)
{
    using F = Fmt<TYPE>;
    constexpr int GEMM_WAVES = gemm_waves<TYPE, MC>();
    constexpr int RG = (MC + 3) / 4;           // 4-row groups of the MFMA
    constexpr int NT = 64 * GEMM_WAVES;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ea[16];
    // (the wave index read as a scalar: the run's bounds and positions stay in SGPRs)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, U = a.U;
    const int64_t Kp = (int64_t)U * 256;

    // this workgroup's items [I0, I1), their units us, us+1, ... (mod U) and tiles t0..
    const int b = blockIdx.x;
    const int I0 = b * a.iq + (b < a.ir ? b : a.ir), I1 = I0 + a.iq + (b < a.ir ? 1 : 0);
    int us, ul;
    const int t0 = divmod_pos(I0, U, a.rU, &us), nu = I1 - I0 < U ? I1 - I0 : U;
    const int nt = I1 > I0 ? divmod_pos(I1 - 1, U, a.rU, &ul) - t0 + 1 : 0;
    const int cstride = nu * 256 + 16;         // LDS bytes per activation row (+16: 4 rows, 4 bank groups)
    uint8_t* s_codes = smem;
    float* s_da = (float*)(smem + ((M * cstride + 15) & ~15));
    int32_t* s_bs = (int32_t*)((uint8_t*)s_da + ((M * nu * F::DA * 4 + 15) & ~15));
    double* s_acc = (double*)((uint8_t*)s_bs + ((M * nu * F::BS * 4 + 15) & ~15));   // [nt][M][64]
    uint8_t* s_trash = (uint8_t*)(s_acc + nt * M * 64);

    // this wave's run
    const int n = I1 - I0;
    const int i0 = I0 + wave * n / GEMM_WAVES, i1 = I0 + (wave + 1) * n / GEMM_WAVES;
    const uint16_t* d6base = (const uint16_t*)(a.w + (a.n_pad / 64) * (int64_t)U * 13 * 1024);
    // an item with its tile and unit; step() moves to the next item of the run
    // and stays on its last (a wave without items walks item 0)
    struct Pos { int it, tile, u; };
    const int ilast = i0 < i1 ? i1 - 1 : 0;
    auto step = [&](Pos p) {
        if (p.it < ilast) {
            p.it++;
            if (++p.u == U) { p.u = 0; p.tile++; }
        }
        return p;
    };
    auto load = [&](const Pos& p, v4i* pcu, uint16_t& d6, int& er) {
        const v4i* src = (const v4i*)(a.w + (int64_t)p.it * F::PIECES * 1024 + lane * 16);
#pragma unroll
        for (int q = 0; q < F::PIECES; q++) {
            // the LM head (Q6_K, 641 MB, read once per launch) streams past the
            // caches: 138 -> 119 us; the Q4_K projections measured no change
            if constexpr (TYPE == CPV_Q6_K) pcu[q] = __builtin_nontemporal_load(src + q * 64);
            else pcu[q] = src[q * 64];
        }
        if (TYPE == CPV_Q6_K) d6 = d6base[(int64_t)p.it * 64 + lane];
        er = a.ew[p.tile * 64 + lane];
    };
    // ---- staging: the first batch of activation loads goes out before any
    // weight load, so that it is not queued behind them; the LDS writes then
    // wait for these loads only
    constexpr int BC = 4, BD = 2, BB = 4;      // per thread: code pieces, scales, code sums
    const int ncode = M * nu * 16, nda = M * nu * F::DA, nbs = M * nu * F::BS;
    constexpr int BS = F::BS > 0 ? F::BS : 1;   // (code sums are not staged without them)
    const float rc = __builtin_amdgcn_rcpf((float)(nu * 16)), rd = __builtin_amdgcn_rcpf((float)(nu * F::DA)),
                rb = __builtin_amdgcn_rcpf((float)(nu * BS));
    auto code_src = [&](int i) {
        int c;
        const int m = divmod_small(i, nu * 16, rc, &c), j = c >> 4;
        const int u = us + j < U ? us + j : us + j - U;
        return (const v4i*)(a.qa + (int64_t)(a.m0 + m) * Kp + u * 256 + (c & 15) * 16);
    };
    auto code_dst = [&](int i) {
        int c;
        const int m = divmod_small(i, nu * 16, rc, &c);
        return (v4i*)(s_codes + m * cstride + c * 16);
    };
    auto da_src = [&](int i) {
        int c;
        const int m = divmod_small(i, nu * F::DA, rd, &c), j = c / F::DA;
        const int u = us + j < U ? us + j : us + j - U;
        return a.da + ((int64_t)(a.m0 + m) * U + u) * F::DA + (c - j * F::DA);
    };
    auto bs_src = [&](int i) {
        int c;
        const int m = divmod_small(i, nu * BS, rb, &c), j = c / BS;
        const int u = us + j < U ? us + j : us + j - U;
        return a.bs + ((int64_t)(a.m0 + m) * U + u) * BS + (c - j * BS);
    };
    v4i cv[BC];
    float dv[BD];
    int32_t bv[BB];
#pragma unroll
    for (int q = 0; q < BC; q++) cv[q] = *code_src(tid + q * NT < ncode ? tid + q * NT : 0);
#pragma unroll
    for (int q = 0; q < BD; q++) dv[q] = *da_src(tid + q * NT < nda ? tid + q * NT : 0);
    if constexpr (F::BS > 0)
#pragma unroll
        for (int q = 0; q < BB; q++) bv[q] = *bs_src(tid + q * NT < nbs ? tid + q * NT : 0);
    // Ea(m): the exponent of the row's largest |scale|, one wave per row (first two loads per lane here)
    const int m_ea = wave < M ? wave : 0, nrow = U * F::DA;
    const float* dr = a.da + (int64_t)(a.m0 + m_ea) * nrow;
    float ev0 = dr[lane < nrow ? lane : 0], ev1 = dr[lane + 64 < nrow ? lane + 64 : 0];

    // then the weights: Q4_K and Q8_0 start with one item in flight and ask
    // for the next when the current one has arrived (a launch's first
    // requests then sit behind fewer bytes); Q6_K's longer units keep two in
    // flight from the start below 4 rows and at 8 (the head: 104 us at one
    // row either way; 4-7 rows lean, 118 -> 110 us at 5; 8 rows two in
    // flight, 184 against 243 us)
    constexpr bool LEAN = TYPE != CPV_Q6_K || (MC >= 4 && MC < 8);
    v4i bufA[F::PIECES], bufB[F::PIECES];
    uint16_t dA = 0, dB = 0;
    int eA = 0, eB = 0;
    // (unconditional: a wave without items, or with one, reloads a valid item;
    // branches here would make the compiler wait for every load at the join)
    Pos cur;
    cur.it = i0 < i1 ? i0 : 0;
    cur.tile = divmod_pos(cur.it, U, a.rU, &cur.u);
    Pos nl = step(cur);
    load(cur, bufA, dA, eA);
    if constexpr (!LEAN) {
        load(nl, bufB, dB, eB);
        nl = step(nl);
    }

#pragma unroll
    for (int q = 0; q < BC; q++) {
        const int i = tid + q * NT;
        *(i < ncode ? code_dst(i) : (v4i*)s_trash) = cv[q];
    }
#pragma unroll
    for (int q = 0; q < BD; q++) {
        const int i = tid + q * NT;
        *(i < nda ? s_da + i : (float*)s_trash) = dv[q];
    }
    if constexpr (F::BS > 0)
#pragma unroll
        for (int q = 0; q < BB; q++) {
            const int i = tid + q * NT;
            *(i < nbs ? s_bs + i : (int32_t*)s_trash) = bv[q];
        }
    for (int i = tid + BC * NT; i < ncode; i += NT) *code_dst(i) = *code_src(i);
    for (int i = tid + BD * NT; i < nda; i += NT) s_da[i] = *da_src(i);
    if constexpr (F::BS > 0)
        for (int i = tid + BB * NT; i < nbs; i += NT) s_bs[i] = *bs_src(i);
    for (int i = tid; i < nt * M * 64; i += NT) s_acc[i] = 0.0;
    // (rows past the waves, when there are more rows than waves, in further passes)
    for (int r = wave; r < M; r += GEMM_WAVES) {
        const float* drr = a.da + (int64_t)(a.m0 + r) * nrow;
        float mx = 0.0f;
        int ib = lane;
        if (r == wave) {
            mx = fmaxf(lane < nrow ? fabsf(ev0) : 0.0f, lane + 64 < nrow ? fabsf(ev1) : 0.0f);
            ib = lane + 128;
        }
        for (int i = ib; i < nrow; i += 64) mx = fmaxf(mx, fabsf(drr[i]));
        mx = cpv_wave_reduce(mx, cpv_op_max());
        if (lane == 0) {
            int e = CPV_E_EMPTY;
            if (mx > 0.0f) frexpf(mx, &e);
            s_ea[r] = e;
        }
    }
    __syncthreads();

    if (i0 < i1) {
        // per row: the MFMA feed of this lane (row group r takes row 4r + lane%4) and 2^(win - Ea)
        const uint8_t* arow[RG];
#pragma unroll
        for (int r = 0; r < RG; r++) {
            const int m = 4 * r + (lane & 3);
            arow[r] = s_codes + (m < M ? m : M - 1) * cstride;
        }
        // 2^(win - Ea) of each row; above 8 rows built from its bits out of the
        // wave-uniform exponent (the same value), so that it stays in scalar
        // registers (win - Ea + 1023 lies in [1, 2046] for every f32 Ea)
        int mrow[MC];
        double sm[MC];
#pragma unroll
        for (int m = 0; m < MC; m++) {
            mrow[m] = m < M ? m : M - 1;
            if constexpr (MC > 8) {
                const int e = __builtin_amdgcn_readfirstlane(s_ea[mrow[m]]);
                const uint64_t bits = e == CPV_E_EMPTY ? 0ull : (uint64_t)(1023 + a.win - e) << 52;
                sm[m] = __builtin_bit_cast(double, bits);
            } else {
                const int e = s_ea[mrow[m]];
                sm[m] = e == CPV_E_EMPTY ? 0.0 : ldexp(1.0, a.win - e);
            }
        }

        double S[MC];
#pragma unroll
        for (int m = 0; m < MC; m++) S[m] = 0.0;
        int tile = cur.tile;
        auto flush = [&]() {
            // partial sums of this tile's units into its LDS sums: exact, in any order
            double* acc = s_acc + ((tile - t0) * M) * 64 + lane;
#pragma unroll
            for (int m = 0; m < MC; m++)
                if (m < M) {
                    __hip_atomic_fetch_add(acc + m * 64, S[m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    S[m] = 0.0;
                }
        };
        // the item's unit as an LDS slot
        auto slot = [&](int u) { return u >= us ? u - us : u - us + U; };
        // one item for all rows: above 8 rows, in passes of 8 over the same
        // weight registers (each pass's working set alone fits the register file)
        auto unit = [&](const v4i* buf, uint16_t d6, int er, int su) {
            if constexpr (MC <= 8) {
                gemm_unit<TYPE, MC>(buf, d6, er, su, M, nu, arow, mrow, sm, s_da, s_bs, S);
            } else {
#pragma unroll
                for (int h = 0; h < MC / 8; h++) {
                    gemm_unit<TYPE, 8>(buf, d6, er, su, M, nu, arow + 2 * h, mrow + 8 * h, sm + 8 * h, s_da, s_bs,
                                       S + 8 * h);
                    asm volatile("" ::: "memory");   // (keeps the passes apart in the schedule)
                }
            }
        };
        for (int it = i0; it < i1; it += 2) {
            if (cur.tile != tile) { flush(); tile = cur.tile; }
            if constexpr (LEAN) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                load(nl, bufB, dB, eB);
                nl = step(nl);
                unit(bufA, dA, eA, slot(cur.u));
            } else {
                unit(bufA, dA, eA, slot(cur.u));
                load(nl, bufA, dA, eA);
                nl = step(nl);
            }
            if (it + 1 >= i1) break;
            cur = step(cur);
            if (cur.tile != tile) { flush(); tile = cur.tile; }
            if constexpr (LEAN) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                load(nl, bufA, dA, eA);
                nl = step(nl);
                unit(bufB, dB, eB, slot(cur.u));
            } else {
                unit(bufB, dB, eB, slot(cur.u));
                load(nl, bufB, dB, eB);
                nl = step(nl);
            }
            cur = step(cur);
        }
        flush();
    }
    __syncthreads();
    // the tile sums: stored where this workgroup covers the whole tile, else added
    const float rM = __builtin_amdgcn_rcpf((float)M);
    for (int i = tid; i < nt * M * 64; i += NT) {
        int m;
        const int t = divmod_small(i >> 6, M, rM, &m), l = i & 63;
        const int tile = t0 + t;
        double* g = a.gsum + (int64_t)(a.m0 + m) * a.n_pad + (int64_t)tile * 64 + l;
        if (tile * U >= I0 && (tile + 1) * U <= I1) *g = s_acc[i];
        else unsafeAtomicAdd(g, s_acc[i]);
    }
}

// ---------------------------------------------------------------- Q4_K, 9-16 rows
// The items, staging, tile sums and accumulator of qgemm_kernel for Q4_K
// weights and 9 to 16 activation rows, with the integer dots on
// v_mfma_i32_16x16x32_i8: one MFMA per (16-row block rb of the tile,
// 32-element sub-block s of the unit) takes all 16 activation rows at once,
// 32 MFMAs per item where the 4x4x4 shape needs 256 (the same layout as
// qgemm_wide_kernel: A row and B column = lane % 16, codes 8 (lane / 16) ..
// + 7 of the sub-block per lane, D rows 4 (lane / 16) + i of column lane %
// 16).  Lane (c, g) = (lane % 16, lane / 16) thus holds the dots of
// activation rows 4g..4g+3 with weight rows 16 rb + c, rb = 0..3: it decodes
// the scales of those four weight rows (their headers come from the lanes
// that loaded them) and runs the sub-block scale products, the min term
// (packed 8-bit dot products against the split code sums) and the binary64
// terms of its 16 (activation row, weight row) pairs in place.  The terms are
// those of gemm_unit, so the accumulator entries are the same bits.
constexpr int R16 = 16;   // activation rows of one launch (rows M..15 repeat row M-1 and are never stored)

__host__ __device__ inline size_t q4k16_lds(int M, int nu, int nt)
{
    const size_t codes = (size_t)M * ((size_t)nu * 256 + 16);
    const size_t aux = (size_t)nu * R16 * (16 + 8);   // [unit][row] packed code sums, then [unit][row] f64 scales
    const size_t acc = (size_t)nt * M * 64 * 8;
    return ((codes + 15) & ~(size_t)15) + aux + acc + 16;
}

__global__ __launch_bounds__(512) void qgemm_q4k16_kernel(GemmArgs a)
{
    constexpr int NW = 8, NT = 64 * NW;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ea[R16];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, g4 = lane >> 4;
    const int M = a.M, U = a.U;
    const int64_t Kp = (int64_t)U * 256;

    const int b = blockIdx.x;
    const int I0 = b * a.iq + (b < a.ir ? b : a.ir), I1 = I0 + a.iq + (b < a.ir ? 1 : 0);
    int us, ul;
    const int t0 = divmod_pos(I0, U, a.rU, &us), nu = I1 - I0 < U ? I1 - I0 : U;
    const int nt = I1 > I0 ? divmod_pos(I1 - 1, U, a.rU, &ul) - t0 + 1 : 0;
    const int cstride = nu * 256 + 16;
    uint8_t* s_codes = smem;
    int4* s_bsp = (int4*)(smem + ((M * cstride + 15) & ~15));        // [nu][R16]
    double* s_dam = (double*)(s_bsp + nu * R16);                      // [nu][R16]
    double* s_acc = s_dam + nu * R16;                                  // [nt][M][64]
    uint8_t* s_trash = (uint8_t*)(s_acc + nt * M * 64);

    const int n = I1 - I0;
    const int i0 = I0 + wave * n / NW, i1 = I0 + (wave + 1) * n / NW;
    struct Pos { int it, tile, u; };
    const int ilast = i0 < i1 ? i1 - 1 : 0;
    auto step = [&](Pos p) {
        if (p.it < ilast) {
            p.it++;
            if (++p.u == U) { p.u = 0; p.tile++; }
        }
        return p;
    };
    // an item's weights in the MFMA's layout: per (rb, chunk pr) the 8 qs
    // bytes 32 pr + 8 g .. of row 16 rb + c (the low nibbles are sub-block
    // 2 pr, the high ones 2 pr + 1); and the header and exponent of row `lane`
    struct Buf { uint2 w[16]; uint4 h; int er; };
    auto load = [&](const Pos& p, Buf& B) {
        const uint8_t* slab = a.w + (int64_t)p.it * 9 * 1024;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int rb = q >> 2, pr = q & 3;
            // (non-temporal: 95 -> 92 us per layer at 16 rows)
            const unsigned long long wq = __builtin_nontemporal_load(
                (const unsigned long long*)(slab + (2 * pr + (g4 >> 1)) * 1024 + (16 * rb + c16) * 16 + 8 * (g4 & 1)));
            B.w[q] = make_uint2((uint32_t)wq, (uint32_t)(wq >> 32));
        }
        B.h = *(const uint4*)(slab + 8 * 1024 + lane * 16);
        B.er = a.ew[p.tile * 64 + lane];
    };

    // ---- staging, as in qgemm_kernel: activation codes (rows of nu * 256 +
    // 16 bytes), then per (unit, row) the code sums packed for the min term and
    // the scale times 2^(win - Ea) in binary64 (the product gemm_unit forms)
    constexpr int BC = 4;
    const int ncode = M * nu * 16, naux = nu * M;
    const float rc = __builtin_amdgcn_rcpf((float)(nu * 16)), rm = __builtin_amdgcn_rcpf((float)M);
    auto code_src = [&](int i) {
        int c;
        const int m = divmod_small(i, nu * 16, rc, &c), j = c >> 4;
        const int u = us + j < U ? us + j : us + j - U;
        return (const v4i*)(a.qa + (int64_t)(a.m0 + m) * Kp + u * 256 + (c & 15) * 16);
    };
    auto code_dst = [&](int i) {
        int c;
        const int m = divmod_small(i, nu * 16, rc, &c);
        return (v4i*)(s_codes + m * cstride + c * 16);
    };
    // aux entry e = (unit slot j, row m): e = j * M + m
    auto aux_unit = [&](int e, int* m) {
        const int j = divmod_small(e, M, rm, m);
        return us + j < U ? us + j : us + j - U;
    };
    v4i cv[BC];
#pragma unroll
    for (int q = 0; q < BC; q++) cv[q] = *code_src(tid + q * NT < ncode ? tid + q * NT : 0);
    int am;
    const int au = aux_unit(tid < naux ? tid : 0, &am);
    const int32_t* bsrc = a.bs + ((int64_t)(a.m0 + am) * U + au) * 8;
    const v4i bs0 = *(const v4i*)bsrc, bs1 = *(const v4i*)(bsrc + 4);
    const float dav = a.da[(int64_t)(a.m0 + am) * U + au];
    const int m_ea = wave < M ? wave : 0;
    const float* dr = a.da + (int64_t)(a.m0 + m_ea) * U;
    float ev0 = dr[lane < U ? lane : 0], ev1 = dr[lane + 64 < U ? lane + 64 : 0];

    // the first item's weights (one in flight; the next is asked for when it has arrived)
    Buf bufA, bufB;
    Pos cur;
    cur.it = i0 < i1 ? i0 : 0;
    cur.tile = divmod_pos(cur.it, U, a.rU, &cur.u);
    Pos nl = step(cur);
    load(cur, bufA);

#pragma unroll
    for (int q = 0; q < BC; q++) {
        const int i = tid + q * NT;
        *(i < ncode ? code_dst(i) : (v4i*)s_trash) = cv[q];
    }
    for (int i = tid + BC * NT; i < ncode; i += NT) *code_dst(i) = *code_src(i);
    for (int i = tid; i < nt * M * 64; i += NT) s_acc[i] = 0.0;
    for (int r = wave; r < M; r += NW) {
        const float* drr = a.da + (int64_t)(a.m0 + r) * U;
        float mx = 0.0f;
        int ib = lane;
        if (r == wave) {
            mx = fmaxf(lane < U ? fabsf(ev0) : 0.0f, lane + 64 < U ? fabsf(ev1) : 0.0f);
            ib = lane + 128;
        }
        for (int i = ib; i < U; i += 64) mx = fmaxf(mx, fabsf(drr[i]));
        mx = cpv_wave_reduce(mx, cpv_op_max());
        if (lane == 0) {
            int e = CPV_E_EMPTY;
            if (mx > 0.0f) frexpf(mx, &e);
            s_ea[r] = e;
        }
    }
    __syncthreads();
    {
        // a code sum s (|s| <= 32 * 127) as 64 bh + bl, bh = s >> 6 and bl in
        // [0, 63]: both fit a signed byte, as do the 6-bit mins, so
        // imin = 64 dot(mn, bh) + dot(mn, bl) over packed bytes
        auto packb = [](int x0, int x1, int x2, int x3) {
            return (int)(((uint32_t)x0 & 255u) | (((uint32_t)x1 & 255u) << 8) | (((uint32_t)x2 & 255u) << 16) |
                         ((uint32_t)x3 << 24));
        };
        auto put = [&](int e, v4i b0, v4i b1, float dv) {
            int m;
            const int j = divmod_small(e, M, rm, &m);
            s_bsp[j * R16 + m] = int4{packb(b0[0] >> 6, b0[1] >> 6, b0[2] >> 6, b0[3] >> 6),
                                      packb(b1[0] >> 6, b1[1] >> 6, b1[2] >> 6, b1[3] >> 6),
                                      packb(b0[0] & 63, b0[1] & 63, b0[2] & 63, b0[3] & 63),
                                      packb(b1[0] & 63, b1[1] & 63, b1[2] & 63, b1[3] & 63)};
            const int ex = s_ea[m];
            s_dam[j * R16 + m] = ex == CPV_E_EMPTY ? 0.0 : (double)dv * ldexp(1.0, a.win - ex);
        };
        if (tid < naux) put(tid, bs0, bs1, dav);
        for (int e = tid + NT; e < naux; e += NT) {   // (more than NT entries: long rows)
            int m;
            const int u = aux_unit(e, &m);
            const int32_t* src = a.bs + ((int64_t)(a.m0 + m) * U + u) * 8;
            put(e, *(const v4i*)src, *(const v4i*)(src + 4), a.da[(int64_t)(a.m0 + m) * U + u]);
        }
    }
    __syncthreads();

    if (i0 < i1) {
        double S[4][4];   // [rb][i]: activation row 4 g + i, weight row 16 rb + c
#pragma unroll
        for (int rb = 0; rb < 4; rb++)
#pragma unroll
            for (int i = 0; i < 4; i++) S[rb][i] = 0.0;
        int tile = cur.tile;
        auto flush = [&]() {
            double* acc = s_acc + ((tile - t0) * M) * 64 + c16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 4 * g4 + i;
                if (m < M) {
#pragma unroll
                    for (int rb = 0; rb < 4; rb++)
                        __hip_atomic_fetch_add(acc + m * 64 + 16 * rb, S[rb][i], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
                }
#pragma unroll
                for (int rb = 0; rb < 4; rb++) S[rb][i] = 0.0;
            }
        };
        auto slot = [&](int u) { return u >= us ? u - us : u - us + U; };
        // the A operand's row (rows past M repeat row M - 1) and the lane's
        // activation rows for the aux reads
        const uint8_t* arow = s_codes + (c16 < M ? c16 : M - 1) * cstride + 8 * g4;
        int mrow[4];
#pragma unroll
        for (int i = 0; i < 4; i++) mrow[i] = 4 * g4 + i < M ? 4 * g4 + i : M - 1;
        auto unit = [&](const Buf& B, int j) {
            // the headers of weight rows 16 rb + c from lanes 16 rb + c
            uint32_t sc[4][2], mn[4][2];
            double dws[4], dms[4];
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const int src = (16 * rb + c16) * 4;
                const uint32_t hx = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)B.h.x);
                const uint32_t hy = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)B.h.y);
                const uint32_t hz = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)B.h.z);
                const uint32_t hw = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)B.h.w);
                const int er = __builtin_amdgcn_ds_bpermute(src, B.er);
                dws[rb] = ldexp((double)h2f(hx & 0xffffu), -er);
                dms[rb] = ldexp((double)h2f(hx >> 16), -er);
                sc[rb][0] = hy & 0x3f3f3f3fu;
                mn[rb][0] = hz & 0x3f3f3f3fu;
                sc[rb][1] = (hw & 0x0f0f0f0fu) | (((hy >> 6) & 0x03030303u) << 4);
                mn[rb][1] = ((hw >> 4) & 0x0f0f0f0fu) | (((hz >> 6) & 0x03030303u) << 4);
            }
            int isum[4][4];
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int i = 0; i < 4; i++) isum[rb][i] = 0;
            const uint8_t* ab = arow + j * 256;
#pragma unroll
            for (int pr = 0; pr < 4; pr++) {
                const int64_t A0 = *(const int64_t*)(ab + 64 * pr), A1 = *(const int64_t*)(ab + 64 * pr + 32);
#pragma unroll
                for (int rb = 0; rb < 4; rb++) {
                    const uint2 w = B.w[rb * 4 + pr];
                    const int64_t blo = (int64_t)(((uint64_t)(w.y & 0x0f0f0f0fu) << 32) | (w.x & 0x0f0f0f0fu));
                    const int64_t bhi =
                        (int64_t)(((uint64_t)((w.y >> 4) & 0x0f0f0f0fu) << 32) | ((w.x >> 4) & 0x0f0f0f0fu));
                    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A0, blo, v4i{0, 0, 0, 0}, 0, 0, 0);
                    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A1, bhi, v4i{0, 0, 0, 0}, 0, 0, 0);
                    const uint32_t scw = sc[rb][pr >> 1];
                    const int sce = byte_of(scw, (2 * pr) & 3), sco = byte_of(scw, (2 * pr + 1) & 3);
#pragma unroll
                    for (int i = 0; i < 4; i++)   // 6-bit scales times |dots| <= 32*15*127: 24-bit products
                        isum[rb][i] += __mul24(sce, D0[i]) + __mul24(sco, D1[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int4 p = s_bsp[j * R16 + mrow[i]];
                const double da = s_dam[j * R16 + mrow[i]];
#pragma unroll
                for (int rb = 0; rb < 4; rb++) {
                    const int hi = __builtin_amdgcn_sdot4((int)mn[rb][1], p.y,
                                                          __builtin_amdgcn_sdot4((int)mn[rb][0], p.x, 0, false), false);
                    const int lo = __builtin_amdgcn_sdot4((int)mn[rb][1], p.w,
                                                          __builtin_amdgcn_sdot4((int)mn[rb][0], p.z, 0, false), false);
                    const int imin = hi * 64 + lo;
                    S[rb][i] += rint(dws[rb] * da * (double)isum[rb][i]) - rint(dms[rb] * da * (double)imin);
                }
            }
        };
        for (int it = i0; it < i1; it += 2) {
            if (cur.tile != tile) { flush(); tile = cur.tile; }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            load(nl, bufB);
            nl = step(nl);
            unit(bufA, slot(cur.u));
            if (it + 1 >= i1) break;
            cur = step(cur);
            if (cur.tile != tile) { flush(); tile = cur.tile; }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            load(nl, bufA);
            nl = step(nl);
            unit(bufB, slot(cur.u));
            cur = step(cur);
        }
        flush();
    }
    __syncthreads();
    const float rM = __builtin_amdgcn_rcpf((float)M);
    for (int i = tid; i < nt * M * 64; i += NT) {
        int m;
        const int t = divmod_small(i >> 6, M, rM, &m), l = i & 63;
        const int tile = t0 + t;
        double* g = a.gsum + (int64_t)(a.m0 + m) * a.n_pad + (int64_t)tile * 64 + l;
        if (tile * U >= I0 && (tile + 1) * U <= I1) *g = s_acc[i];
        else unsafeAtomicAdd(g, s_acc[i]);
    }
}

// y = the accumulated split-K sums scaled by 2^(Ew + Ea - win); leaves the
// accumulator zero.  One block per 256 outputs of one activation row; Ea(m)
// is recomputed from the row's scales.
__global__ __launch_bounds__(256) void qgemm_finalize_kernel(double* __restrict__ gsum, int64_t n_pad,
                                                             const int32_t* __restrict__ ew,
                                                             const float* __restrict__ da, int nda, int m0,
                                                             int win, float* __restrict__ y, int64_t N)
{
    const int m = blockIdx.y, tid = threadIdx.x;
    __shared__ float s_mx[4];
    float mx = 0.0f;
    for (int i = tid; i < nda; i += 256) mx = fmaxf(mx, fabsf(da[(int64_t)(m0 + m) * nda + i]));
    mx = cpv_wave_reduce(mx, cpv_op_max());
    if ((tid & 63) == 0) s_mx[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3]));
    int ea = CPV_E_EMPTY;
    if (mx > 0.0f) frexpf(mx, &ea);
    const int64_t n = (int64_t)blockIdx.x * 256 + tid;
    if (n >= N) return;
    double* g = gsum + (int64_t)(m0 + m) * n_pad + n;
    const double tot = *g;
    *g = 0.0;
    const int e = ew[n];
    y[(int64_t)(m0 + m) * N + n] = (e == CPV_E_EMPTY || ea == CPV_E_EMPTY) ? 0.0f : (float)ldexp(tot, e + ea - win);
}

template <int TYPE, int MC>
cpv_status launch_mc(cpv_ctx* ctx, const GemmArgs& a, float* y, int64_t N, int64_t k, double wbytes)
{
    // Q4_K above 8 rows: the 16x16x32 kernel
    constexpr bool R16K = TYPE == CPV_Q4_K && MC == R16;
    const size_t lds = R16K ? q4k16_lds(a.M, a.nu_max, a.nt_max) : gemm_lds<TYPE>(a.M, a.nu_max, a.nt_max);
    const unsigned grid = (unsigned)ctx->cu_count;
    auto go = [=]() {
        if constexpr (R16K) qgemm_q4k16_kernel<<<grid, 512, lds, ctx->stream>>>(a);
        else qgemm_kernel<TYPE, MC><<<grid, 64 * gemm_waves<TYPE, MC>(), lds, ctx->stream>>>(a);
        if (y)   // else the sums stay in the accumulator for a fused consumer
            qgemm_finalize_kernel<<<dim3((unsigned)((N + 255) / 256), (unsigned)a.M), 256, 0, ctx->stream>>>(
                a.gsum, a.n_pad, a.ew, a.da, a.U * Fmt<TYPE>::DA, a.m0, a.win, y, N);
    };
    const int ev = cpv_prof_mark(ctx);
    go();
    CPV_HIP(ctx, hipGetLastError());
    if (ev >= 0) {  // algorithmic bytes: the weight, f32 activations in, f32 outputs
        const int cls = TYPE == CPV_Q4_K ? CPV_PROF_Q4_K : TYPE == CPV_Q6_K ? CPV_PROF_Q6_K : CPV_PROF_Q8_0;
        const double bytes = wbytes + 4.0 * a.M * (double)k + 4.0 * a.M * (double)N;
        cpv_prof_add(ctx, ev, cls, bytes);
        cpv_prof_keep(ctx, cls, bytes, go);
    }
    return CPV_OK;
}

template <int TYPE>
cpv_status launch_type(cpv_ctx* ctx, const GemmArgs& a, float* y, int64_t N, int64_t k, double wbytes)
{
    // the smallest instantiated row bound >= M
    if (a.M <= 1) return launch_mc<TYPE, 1>(ctx, a, y, N, k, wbytes);
    if (a.M <= 2) return launch_mc<TYPE, 2>(ctx, a, y, N, k, wbytes);
    if (a.M <= 4) return launch_mc<TYPE, 4>(ctx, a, y, N, k, wbytes);
    if (a.M <= 5) return launch_mc<TYPE, 5>(ctx, a, y, N, k, wbytes);
    if constexpr (TYPE == CPV_Q6_K) return launch_mc<TYPE, 8>(ctx, a, y, N, k, wbytes);
    else {
        if (a.M <= 8) return launch_mc<TYPE, 8>(ctx, a, y, N, k, wbytes);
        return launch_mc<TYPE, 16>(ctx, a, y, N, k, wbytes);
    }
}

template <int TYPE>
size_t lds_of(int M, int nu, int nt)
{
    if (TYPE == CPV_Q4_K && M > 8) return q4k16_lds(M, nu, nt);
    return gemm_lds<TYPE>(M, nu, nt);
}

static int isum_bits(int type) { return type == CPV_Q8_0 ? 20 : type == CPV_Q4_K ? 25 : 28; }

// the split-K accumulator [rows][n_pad]: zeroed once when (re)allocated, left
// zero by every finalize and by every fused consumer of a kept result
static cpv_status gemm_accumulator(cpv_ctx* ctx, int64_t rows, int64_t n_pad, double** gsum)
{
    const size_t need = (size_t)rows * n_pad * sizeof(double);
    if (need > ctx->gsum_bytes) {
        if (cpv_capturing(ctx)) return cpv_refuse_growth(ctx, "GEMM accumulator", need);
        CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->gsum) (void)hipFree(ctx->gsum);
        ctx->gsum = nullptr;
        ctx->gsum_bytes = 0;
        const size_t bs = need > ((size_t)16 << 20) ? need : ((size_t)16 << 20);
        CPV_HIP(ctx, hipMalloc((void**)&ctx->gsum, bs));
        CPV_HIP(ctx, hipMemsetAsync(ctx->gsum, 0, bs, ctx->stream));
        ctx->gsum_bytes = bs;
        ctx->ws_gen++;
    }
    *gsum = ctx->gsum;
    return CPV_OK;
}

}  // namespace

int cpv_qgemm_window(int type, int64_t k)
{
    const int64_t terms = type == CPV_Q8_0 ? k / 32 : type == CPV_Q4_K ? 2 * (k / 256) : k / 256;
    int b = 0;
    while (((int64_t)1 << b) < terms + 1) b++;
    return 52 - isum_bits(type) - b;
}

static int act_units(int64_t k) { return (int)((k + 255) / 256); }

size_t cpv_act_bytes(int type, int64_t k, int64_t m)
{
    const int64_t U = act_units(k);
    const bool kq = type != CPV_Q8_0;
    const size_t qa_b = ((size_t)m * U * 256 + 255) & ~(size_t)255;
    const size_t da_b = ((size_t)m * U * (kq ? 1 : 8) * 4 + 255) & ~(size_t)255;
    const size_t bs_b = kq ? (size_t)m * U * (8 + 16) * 4 : 0;
    return qa_b + da_b + bs_b;
}

void cpv_act_layout(int type, int64_t m, int64_t k, void* buf, cpv_act* out)
{
    const int U = act_units(k);
    const bool kq = type != CPV_Q8_0;
    const size_t qa_b = ((size_t)m * U * 256 + 255) & ~(size_t)255;
    const size_t da_b = ((size_t)m * U * (kq ? 1 : 8) * 4 + 255) & ~(size_t)255;
    out->qa = (int8_t*)buf;
    out->da = (float*)((uint8_t*)buf + qa_b);
    out->bs32 = (int32_t*)((uint8_t*)buf + qa_b + da_b);
    out->bs16 = out->bs32 + (size_t)m * U * 8;
    out->m = m;
    out->k = k;
    out->U = U;
    out->kq = kq;
}

cpv_status cpv_quant_act(cpv_ctx* ctx, int type, const float* x, int64_t m, int64_t k, void* buf, cpv_act* out)
{
    const int U = act_units(k);
    const bool kq = type != CPV_Q8_0;
    const size_t qa_b = ((size_t)m * U * 256 + 255) & ~(size_t)255;
    const size_t da_b = ((size_t)m * U * (kq ? 1 : 8) * 4 + 255) & ~(size_t)255;
    int8_t* qa = (int8_t*)buf;
    float* da = (float*)((uint8_t*)buf + qa_b);
    int32_t* bs32 = (int32_t*)((uint8_t*)buf + qa_b + da_b);
    int32_t* bs16 = bs32 + (size_t)m * U * 8;
    out->qa = qa;
    out->da = da;
    out->bs32 = bs32;
    out->bs16 = bs16;
    out->m = m;
    out->k = k;
    out->U = U;
    out->kq = kq;
    dim3 qgrid((unsigned)U, (unsigned)m);
    if (kq) quant_q8k_kernel<<<qgrid, 256, 0, ctx->stream>>>(x, k, U, qa, da, bs32, bs16);
    else quant_q80_kernel<<<qgrid, 256, 0, ctx->stream>>>(x, k, U, qa, da);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

// the GEMM of quantized activations into the split-K accumulator gsum
// ([act->m][w->n_pad] f64, zero on entry and, when y is given, on return)
static cpv_status qgemm_into(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, float* y, double* gsum)
{
    const bool kq = w->type != CPV_Q8_0;
    if (kq != act->kq || act->k != w->k || act->U != (int)w->units)
        return cpv_fail(ctx, CPV_EINVAL, "qgemm: activation format does not match the weight");
    const int U = act->U;
    const int64_t m = act->m;
    const int64_t tiles = w->n_pad / 64;
    GemmArgs a;
    a.w = (const uint8_t*)w->data;
    a.ew = w->ew;
    a.qa = act->qa;
    a.da = act->da;
    a.bs = w->type == CPV_Q4_K ? act->bs32 : act->bs16;
    a.n_pad = w->n_pad;
    a.U = U;
    if (tiles * U > INT32_MAX / 2)
        return cpv_fail(ctx, CPV_EUNSUPPORTED, "qgemm: %lld tiles of %d units", (long long)tiles, U);
    a.items = (int)(tiles * U);
    a.iq = a.items / ctx->cu_count;
    a.ir = a.items % ctx->cu_count;
    a.rU = 1.0 / U;
    a.win = cpv_qgemm_window(w->type, w->k);
    {
        // one workgroup's items: at most ceil(items / CUs), spanning at most that
        // many units and one tile more than they fill
        const int per = (a.items + ctx->cu_count - 1) / ctx->cu_count;
        a.nu_max = per < U ? per : U;
        a.nt_max = (per + U - 1) / U + 1;
    }
    a.gsum = gsum;
    cpv_status st = CPV_OK;
    const double wb = (double)w->n * (double)(w->k / cpv_type_block(w->type)) * (double)cpv_type_size(w->type);
    auto lds = [&](int M) {
        return w->type == CPV_Q4_K   ? lds_of<CPV_Q4_K>(M, a.nu_max, a.nt_max)
               : w->type == CPV_Q6_K ? lds_of<CPV_Q6_K>(M, a.nu_max, a.nt_max)
                                     : lds_of<CPV_Q8_0>(M, a.nu_max, a.nt_max);
    };
    if (cpv_qgemm_wide_ok(w, m)) {
        if ((st = cpv_qgemm_wide(ctx, w, act, a.gsum, a.win)) != CPV_OK) return st;
        if (y)
            qgemm_finalize_kernel<<<dim3((unsigned)((w->n + 255) / 256), (unsigned)m), 256, 0, ctx->stream>>>(
                a.gsum, a.n_pad, a.ew, a.da, kq ? U : 8 * U, 0, a.win, y, w->n);
        CPV_HIP(ctx, hipGetLastError());
        return CPV_OK;
    }
    const size_t lds_cap = ctx->lds_max - 1024;
    for (int64_t m0 = 0; m0 < m;) {
        // rows per launch: up to 16 (Q6_K: 8, whose 16-row pass measured slower
        // than two 8-row ones: 397 vs 333 us for the 151,936-row head; above 8
        // rows Q6_K and Q8_0 take the wide kernels), as many as LDS holds
        const int cap = w->type == CPV_Q6_K ? 8 : 16;
        int M = (int)((m - m0) < cap ? (m - m0) : cap);
        while (M > 1 && lds(M) > lds_cap) M--;
        if (lds(M) > lds_cap)
            return cpv_fail(ctx, CPV_EUNSUPPORTED, "qgemm: k=%lld needs more LDS than a CU has", (long long)w->k);
        a.m0 = (int)m0;
        a.M = M;
        cpv_status s2 = w->type == CPV_Q4_K ? launch_type<CPV_Q4_K>(ctx, a, y, w->n, w->k, wb)
                      : w->type == CPV_Q6_K ? launch_type<CPV_Q6_K>(ctx, a, y, w->n, w->k, wb)
                                            : launch_type<CPV_Q8_0>(ctx, a, y, w->n, w->k, wb);
        if (s2 != CPV_OK) return s2;
        m0 += M;
    }
    return CPV_OK;
}

cpv_status cpv_qgemm_act(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, float* y)
{
    double* gsum = nullptr;
    cpv_status st = gemm_accumulator(ctx, act->m, w->n_pad, &gsum);
    if (st != CPV_OK) return st;
    return qgemm_into(ctx, w, act, y, gsum);
}

cpv_status cpv_qgemm_keep(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, cpv_gout* out)
{
    cpv_status st = cpv_qgemm_act(ctx, w, act, nullptr);
    if (st != CPV_OK) return st;
    out->acc = ctx->gsum;
    out->n_pad = w->n_pad;
    out->n = w->n;
    out->ew = w->ew;
    out->da = act->da;
    out->nda = act->U * (act->kq ? 1 : 8);
    out->win = cpv_qgemm_window(w->type, w->k);
    return CPV_OK;
}

cpv_status cpv_qgemm_launch(cpv_ctx* ctx, const cpv_weight* w, const float* x, int64_t m, float* y)
{
    void* ws = nullptr;
    cpv_status st = cpv_workspace(ctx, cpv_act_bytes(w->type, w->k, m), &ws);
    if (st != CPV_OK) return st;
    cpv_act act;
    st = cpv_quant_act(ctx, w->type, x, m, w->k, ws, &act);
    if (st != CPV_OK) return st;
    return cpv_qgemm_act(ctx, w, &act, y);
}

extern "C" cpv_status cpv_qgemm(cpv_ctx* ctx, const cpv_weight* w, const float* x_dev, int64_t m, float* y_dev)
{
    if (!ctx || !w || !x_dev || !y_dev) return cpv_fail(ctx, CPV_EINVAL, "qgemm: null argument");
    if (m < 1 || m > 256) return cpv_fail(ctx, CPV_EINVAL, "qgemm: m=%lld outside [1, 256]", (long long)m);
    if (w->ctx != ctx) return cpv_fail(ctx, CPV_EINVAL, "qgemm: weight belongs to another context");
    return cpv_qgemm_launch(ctx, w, x_dev, m, y_dev);
}

// ---------------------------------------------------------------- without allocation
// cpv_qgemm_noalloc keeps its quantized activations and its split-K
// accumulator in one file-scope device array instead of the context's
// workspace.  Each GPU holds its own copy until the process ends.  Host code
// must not use the array's name as an address (on the host it is a stand-in,
// not device memory): cpv_noalloc_setup looks up each device's address once,
// with that device current, and every launch takes that pointer.
namespace {

constexpr size_t NOALLOC_ACT_BYTES = (size_t)2 << 20;    // quantized activations (Q8_K / Q8_0 layout)
constexpr size_t NOALLOC_ACC_BYTES = (size_t)8 << 20;    // [m][n_pad] f64 accumulator
constexpr int NOALLOC_MAX_ROWS = 16;
constexpr int NOALLOC_MAX_DEVICES = 64;

static __device__ __align__(256) uint8_t scratch[NOALLOC_ACT_BYTES + NOALLOC_ACC_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

__global__ __launch_bounds__(256) void zero_f64_kernel(double* __restrict__ p, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.0;
}

}  // namespace

cpv_status cpv_noalloc_setup(cpv_ctx* ctx)
{
    if (ctx->device < 0 || ctx->device >= NOALLOC_MAX_DEVICES)
        return cpv_fail(ctx, CPV_EUNSUPPORTED, "noalloc: device %d beyond the scratch table", ctx->device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[ctx->device]) {
        // the caller (cpv_init) has made ctx->device current
        void* p = nullptr;
        CPV_HIP(ctx, hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_ptr[ctx->device] = p;
    }
    ctx->scratch = g_scratch_ptr[ctx->device];
    return CPV_OK;
}

extern "C" cpv_status cpv_qgemm_noalloc(cpv_ctx* ctx, const cpv_weight* w, const float* x_dev, int64_t m,
                                        float* y_dev)
{
    if (!ctx || !w || !x_dev || !y_dev) return cpv_fail(ctx, CPV_EINVAL, "qgemm_noalloc: null argument");
    if (w->ctx != ctx) return cpv_fail(ctx, CPV_EINVAL, "qgemm_noalloc: weight belongs to another context");
    if (!ctx->scratch) return cpv_fail(ctx, CPV_EDEVICE, "qgemm_noalloc: no scratch address for this device");
    if (m < 1 || m > NOALLOC_MAX_ROWS)
        return cpv_fail(ctx, CPV_EINVAL, "qgemm_noalloc: m=%lld outside [1, %d]", (long long)m, NOALLOC_MAX_ROWS);
    const size_t act_b = cpv_act_bytes(w->type, w->k, m);
    const size_t acc_b = (size_t)m * (size_t)w->n_pad * sizeof(double);
    if (act_b > NOALLOC_ACT_BYTES)
        return cpv_fail(ctx, CPV_EINVAL, "qgemm_noalloc: k=%lld at m=%lld needs %zu activation bytes, above %zu",
                        (long long)w->k, (long long)m, act_b, NOALLOC_ACT_BYTES);
    if (acc_b > NOALLOC_ACC_BYTES)
        return cpv_fail(ctx, CPV_EINVAL, "qgemm_noalloc: %lld rows at m=%lld need %zu accumulator bytes, above %zu",
                        (long long)w->n, (long long)m, acc_b, NOALLOC_ACC_BYTES);
    uint8_t* base = (uint8_t*)ctx->scratch;
    double* acc = (double*)(base + NOALLOC_ACT_BYTES);
    // the previous call on this device left the accumulator zero unless it
    // failed part-way; clear it with a kernel (no memset node, so the call can
    // be captured into a graph)
    const int64_t n_acc = m * w->n_pad;
    const int64_t zb = (n_acc + 255) / 256;
    zero_f64_kernel<<<(unsigned)(zb < 1024 ? zb : 1024), 256, 0, ctx->stream>>>(acc, n_acc);
    CPV_HIP(ctx, hipGetLastError());
    // no kernel timing here: it creates events and keeps launches
    const bool prof = ctx->prof;
    ctx->prof = false;
    cpv_act act;
    cpv_status st = cpv_quant_act(ctx, w->type, x_dev, m, w->k, base, &act);
    if (st == CPV_OK) st = qgemm_into(ctx, w, &act, y_dev, acc);
    ctx->prof = prof;
    return st;
}
