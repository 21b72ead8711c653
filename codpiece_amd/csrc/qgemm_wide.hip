// qgemm_wide.hip — the GEMMs for many activation rows (prompt prefill): Q4_K
// first, then Q8_0 and Q6_K (below) on the same mapping.
//
// The prefill pushes a chunk of the prompt through the trunk as one batch of
// rows (engine.rs:1922-1953, step_greedy -> run_general, qwen35.rs:1125-1302),
// so every ggml_mul_mat there has tens to hundreds of activation rows.  The
// numbers are exactly those of the skinny kernel (qgemm.hip): for activation
// row m, weight row n and 256-element unit u,
//     isum = sum_j sc_j * dot_j      imin = sum_j mn_j * (codes of sub-block j)
//     term = rint(dws * da * isum) - rint(dms * da * imin)        (binary64)
// and the terms of all units are summed exactly into the same accumulator
// entry, so the finalize kernel and the fused consumers of a kept result are
// shared and the outputs are bit-identical to the skinny path's.
//
// Mapping.  A workgroup of 4 waves owns one 64-row weight tile and 64
// activation rows (and, when the grid would be small, one slice of K).  Wave w
// takes weight rows 16w..16w+15 against all 64 activation rows: four 16 x 16
// output blocks.  Per unit and 32-element sub-block j it runs two 16x16x32
// int8 MFMAs per block, one against the sub-block's 4-bit codes (the dots,
// scaled by sc_j on the VALU) and one against mn_j in every byte, which sums
// to imin directly (sum over k of a_k * mn_j(k)).  The activation codes of one
// unit are staged in LDS for all four waves, double-buffered, while the next
// unit's codes and weights are in flight.  The lane layout of the MFMA (A row
// and B column = lane % 16, 8 consecutive k per lane >> 4, C rows 4 (lane >>
// 4) + i of column lane % 16) puts one weight row in each lane, so its scales
// are decoded once per unit.
#include <math.h>

#include "cpv_internal.h"

namespace {

constexpr int WBM = 64;                 // activation rows per workgroup
constexpr int WT = 256;                 // threads per workgroup (4 waves)
constexpr int WROW = 256 + 16;          // LDS bytes per staged activation row (+16 spreads the banks)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

struct WideArgs {
    const uint8_t* w;      // repacked Q4_K tiles: [tile][unit][9 pieces][64 rows][16 B]
    const int32_t* ew;     // [n_pad] row exponents
    const int8_t* qa;      // [rows][U*256] activation codes
    const float* da;       // [rows][U] activation scales
    double* gsum;          // [rows][n_pad], zero on entry
    int64_t n_pad;
    int U, M, m0, win;
    int tiles, mblocks, ksplit, upk;   // grid = tiles * mblocks * ksplit; upk units per K slice
};

__device__ __forceinline__ int64_t pack2(uint32_t lo, uint32_t hi)
{
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ v4i mfma16(int64_t a, int64_t b, v4i c)
{
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int byte_at(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }

// NMT: 16-row blocks of the 64 that hold rows (fewer when M <= 48)
template <int NMT>
__global__ __launch_bounds__(WT) __attribute__((amdgpu_waves_per_eu(3))) void qgemm_wide_kernel(WideArgs a)
{
    __shared__ __align__(16) uint8_t s_codes[2][16 * NMT][WROW];
    __shared__ double s_dad[2][16 * NMT + 1];   // da * 2^(win - Ea) per staged row (+ a dump slot)
    __shared__ double s_sm[WBM];        // 2^(win - Ea(m)), 0 for an all-zero row

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int U = a.U, M = a.M;
    const int64_t Kp = (int64_t)U * 256;

    // workgroup -> (tile, K slice, row block).  Consecutive workgroups go to
    // different XCDs, so the order is laid out per XCD: the row blocks of one
    // tile (which read the same weights) run side by side on one XCD's L2.
    const int nb = gridDim.x, b0 = blockIdx.x;
    const int L = (nb & 7) == 0 ? (b0 & 7) * (nb >> 3) + (b0 >> 3) : b0;
    const int mb = L % a.mblocks, r0 = L / a.mblocks;
    const int ks = r0 % a.ksplit, tile = r0 / a.ksplit;
    const int u0 = ks * a.upk, u1 = min(U, u0 + a.upk);
    const int rbase = mb * WBM;

    // Ea(m) per row of the block: the exponent of the row's largest |scale|
    for (int r = wave; r < WBM; r += WT / 64) {
        const int mr = a.m0 + min(rbase + r, M - 1);
        float mx = 0.0f;
        for (int u = lane; u < U; u += 64) mx = fmaxf(mx, fabsf(a.da[(int64_t)mr * U + u]));
        mx = cpv_wave_reduce(mx, cpv_op_max());
        if (lane == 0) {
            int e = CPV_E_EMPTY;
            if (mx > 0.0f) frexpf(mx, &e);
            s_sm[r] = e == CPV_E_EMPTY ? 0.0 : ldexp(1.0, a.win - e);
        }
    }

    // staging of one unit: 64 rows x 16 pieces of 16 B, 4 per thread, and the row scales
    // (32-bit offsets from the block's first row: rows * Kp stays below 2^31)
    const int8_t* qbase = a.qa + (int64_t)(a.m0 + rbase) * Kp;
    int soff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int p = tid + q * WT, r = p >> 4;
        soff[q] = (min(rbase + r, M - 1) - rbase) * (int)Kp + (p & 15) * 16;
    }
    const float* sda = a.da + (int64_t)(a.m0 + min(rbase + (tid & 63), M - 1)) * U;
    auto stage_load = [&](int u, v4i* cv, float& dv) {
#pragma unroll
        for (int q = 0; q < NMT; q++) cv[q] = *(const v4i*)(qbase + soff[q] + u * 256);
        dv = sda[u];
    };
    auto stage_store = [&](int buf, const v4i* cv, float dv) {
#pragma unroll
        for (int q = 0; q < NMT; q++) {
            const int p = tid + q * WT;
            *(v4i*)&s_codes[buf][p >> 4][(p & 15) * 16] = cv[q];
        }
        // (threads past the rows write the dump slot: no branch around the store)
        const int sr = tid < 16 * NMT ? tid : 16 * NMT;
        s_dad[buf][sr] = (double)dv * s_sm[tid & (WBM - 1)];
    };

    // this lane's weight row and k slot: 8 codes (bytes 8 (kq & 1).. of piece
    // (pr, kq >> 1)) per 64-element chunk pr, and the row's scale piece
    const int nl = lane & 15, kq = lane >> 4;
    const int nrow = wave * 16 + nl;
    const uint8_t* wrow = a.w + (int64_t)tile * U * 9 * 1024 + nrow * 16;
    struct Wt { v2i q[4]; v4i s; };
    auto wload = [&](int u, Wt& t) {
        const uint8_t* p = wrow + (int64_t)u * 9 * 1024;
#pragma unroll
        for (int pr = 0; pr < 4; pr++) t.q[pr] = *(const v2i*)(p + (2 * pr + (kq >> 1)) * 1024 + 8 * (kq & 1));
        t.s = *(const v4i*)(p + 8 * 1024);
    };
    const int er = a.ew[(int64_t)tile * 64 + nrow];

    double S[NMT][4];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) S[mt][i] = 0.0;

    Wt wc, wn;
    v4i cv[NMT];
    float dv;
    wload(u0, wc);
    stage_load(u0, cv, dv);
    __syncthreads();                    // s_sm
    stage_store(0, cv, dv);
    __syncthreads();

    for (int u = u0; u < u1; u++) {
        const int buf = (u - u0) & 1;
        // the next unit in flight (the last one reloads itself: no branch)
        const int un = u + 1 < u1 ? u + 1 : u;
        wload(un, wn);
        stage_load(un, cv, dv);

        // this unit's scales and B operands
        const uint32_t h0 = (uint32_t)wc.s[0], hy = (uint32_t)wc.s[1], hz = (uint32_t)wc.s[2],
                       hw = (uint32_t)wc.s[3];
        const double dws = ldexp((double)cpv_h2f((uint16_t)(h0 & 0xffffu)), -er);
        const double dms = ldexp((double)cpv_h2f((uint16_t)(h0 >> 16)), -er);
        const uint32_t sc_lo = hy & 0x3f3f3f3fu, mn_lo = hz & 0x3f3f3f3fu;
        const uint32_t sc_hi = (hw & 0x0f0f0f0fu) | (((hy >> 6) & 0x03030303u) << 4);
        const uint32_t mn_hi = ((hw >> 4) & 0x0f0f0f0fu) | (((hz >> 6) & 0x03030303u) << 4);
        // per sub-block j: its B operands (codes, mn_j in every byte) built here, then
        // the four 16-row blocks; the dots are scaled by sc_j as they come
        int isum[NMT][4];
        v4i dmin[NMT];
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) {
            dmin[mt] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; i++) isum[mt][i] = 0;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t x0 = (uint32_t)wc.q[j >> 1][0], x1 = (uint32_t)wc.q[j >> 1][1];
            const int sh = 4 * (j & 1);   // sub-block 2 pr: low nibbles, 2 pr + 1: high
            const int64_t bq = pack2((x0 >> sh) & 0x0f0f0f0fu, (x1 >> sh) & 0x0f0f0f0fu);
            const uint32_t mw = j < 4 ? mn_lo : mn_hi;
            const uint32_t bb = __builtin_amdgcn_perm(mw, mw, (uint32_t)(j & 3) * 0x01010101u);
            const int64_t bm = pack2(bb, bb);
            const int scj = byte_at(j < 4 ? sc_lo : sc_hi, j & 3);
#pragma unroll
            for (int mt = 0; mt < NMT; mt++) {
                const int64_t av = *(const int64_t*)&s_codes[buf][mt * 16 + nl][8 * kq + 32 * j];
                const v4i d = mfma16(av, bq, v4i{0, 0, 0, 0});
                dmin[mt] = mfma16(av, bm, dmin[mt]);
#pragma unroll
                for (int i = 0; i < 4; i++) isum[mt][i] += __mul24(scj, d[i]);   // |dot| <= 32*15*127
            }
            // one sub-block at a time: the scaled dots are taken here (else the
            // compiler sinks them and keeps all 32 MFMA results live, which
            // costs the registers of a second wave per SIMD)
#pragma unroll
            for (int mt = 0; mt < NMT; mt++)
                asm volatile("" : "+v"(isum[mt][0]), "+v"(isum[mt][1]), "+v"(isum[mt][2]), "+v"(isum[mt][3]));
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) {
            const double* dd = &s_dad[buf][mt * 16 + 4 * kq];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const double da = dd[i];
                S[mt][i] += rint(dws * da * (double)isum[mt][i]) - rint(dms * da * (double)dmin[mt][i]);
            }
        }
        stage_store(buf ^ 1, cv, dv);
        __syncthreads();
        wc = wn;
    }

    // the sums: stored when this workgroup covers all of K, else added
    double* g = a.gsum + (int64_t)tile * 64 + nrow;
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = rbase + mt * 16 + 4 * kq + i;
            if (m < M) {
                double* p = g + (int64_t)(a.m0 + m) * a.n_pad;
                if (a.ksplit == 1) *p = S[mt][i];
                else unsafeAtomicAdd(p, S[mt][i]);
            }
        }
}

// The same for Q8_0 weights and activations (ggml's Q8_0 vec_dot_type).
// Per (activation row m, weight row n, 32-element block j) the dot is one
// 16x16x32 MFMA's entry, and the block's term is rounded on its own:
//     term = rint(dw_j * da_j * 2^-g * dot)          (binary64, exact product)
// eight terms per 256-element unit where Q4_K has two, so this kernel is
// bound by its binary64 VALU work.  A unit's 17 pieces: 16 of codes (block j
// in pieces 2j, 2j + 1), then the 8 block scales (f16).
// NMT: 16-row blocks of the 64 that hold rows (fewer when M <= 48)
template <int NMT>
__global__ __launch_bounds__(WT) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_wide_q80_kernel(WideArgs a)
{
    __shared__ __align__(16) uint8_t s_codes[2][16 * NMT][WROW];
    __shared__ double s_dad[2][16 * NMT + 1][8];   // da_j * 2^(win - Ea) per staged row and block (+ a dump row)
    __shared__ double s_sm[WBM];         // 2^(win - Ea(m)), 0 for an all-zero row

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int U = a.U, M = a.M, NDA = 8 * a.U;
    const int64_t Kp = (int64_t)U * 256;

    const int nb = gridDim.x, b0 = blockIdx.x;
    const int L = (nb & 7) == 0 ? (b0 & 7) * (nb >> 3) + (b0 >> 3) : b0;
    const int mb = L % a.mblocks, r0 = L / a.mblocks;
    const int ks = r0 % a.ksplit, tile = r0 / a.ksplit;
    const int u0 = ks * a.upk, u1 = min(U, u0 + a.upk);
    const int rbase = mb * WBM;

    for (int r = wave; r < WBM; r += WT / 64) {
        const int mr = a.m0 + min(rbase + r, M - 1);
        float mx = 0.0f;
        for (int c = lane; c < NDA; c += 64) mx = fmaxf(mx, fabsf(a.da[(int64_t)mr * NDA + c]));
        mx = cpv_wave_reduce(mx, cpv_op_max());
        if (lane == 0) {
            int e = CPV_E_EMPTY;
            if (mx > 0.0f) frexpf(mx, &e);
            s_sm[r] = e == CPV_E_EMPTY ? 0.0 : ldexp(1.0, a.win - e);
        }
    }

    const int8_t* qbase = a.qa + (int64_t)(a.m0 + rbase) * Kp;
    int soff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int p = tid + q * WT, r = p >> 4;
        soff[q] = (min(rbase + r, M - 1) - rbase) * (int)Kp + (p & 15) * 16;
    }
    // scales: thread tid stages blocks 2 (tid & 3), +1 of row tid >> 2
    const int srow = tid >> 2, sblk = 2 * (tid & 3);
    const float* sda = a.da + (int64_t)(a.m0 + min(rbase + srow, M - 1)) * NDA + sblk;
    auto stage_load = [&](int u, v4i* cv, float2& dv) {
#pragma unroll
        for (int q = 0; q < NMT; q++) cv[q] = *(const v4i*)(qbase + soff[q] + u * 256);
        dv = *(const float2*)(sda + 8 * u);
    };
    auto stage_store = [&](int buf, const v4i* cv, float2 dv) {
#pragma unroll
        for (int q = 0; q < NMT; q++) {
            const int p = tid + q * WT;
            *(v4i*)&s_codes[buf][p >> 4][(p & 15) * 16] = cv[q];
        }
        // (rows past the blocks write the dump row: a branch here made the
        // compiler hold every load across it, 256 VGPRs and spills)
        const int sr = srow < 16 * NMT ? srow : 16 * NMT;
        s_dad[buf][sr][sblk] = (double)dv.x * s_sm[srow];
        s_dad[buf][sr][sblk + 1] = (double)dv.y * s_sm[srow];
    };

    // this lane's weight row and k slot: 8 codes of block j (bytes 8 (kq & 1)
    // .. of piece 2j + (kq >> 1)), and the row's 8 block scales
    const int nl = lane & 15, kq = lane >> 4;
    const int nrow = wave * 16 + nl;
    const uint8_t* wrow = a.w + (int64_t)tile * U * 17 * 1024 + nrow * 16;
    struct Wt { v2i q[8]; v4i s; };
    auto wload = [&](int u, Wt& t) {
        const uint8_t* p = wrow + (int64_t)u * 17 * 1024;
#pragma unroll
        for (int j = 0; j < 8; j++) t.q[j] = *(const v2i*)(p + (2 * j + (kq >> 1)) * 1024 + 8 * (kq & 1));
        t.s = *(const v4i*)(p + 16 * 1024);
    };
    const int er = a.ew[(int64_t)tile * 64 + nrow];

    double S[NMT][4];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) S[mt][i] = 0.0;

    Wt wc, wn;
    v4i cv[NMT];
    float2 dv;
    wload(u0, wc);
    stage_load(u0, cv, dv);
    __syncthreads();                    // s_sm
    stage_store(0, cv, dv);
    __syncthreads();

    for (int u = u0; u < u1; u++) {
        const int buf = (u - u0) & 1;
        const int un = u + 1 < u1 ? u + 1 : u;
        wload(un, wn);
        stage_load(un, cv, dv);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t hw = (uint32_t)wc.s[j >> 1];
            const double dwj = ldexp((double)cpv_h2f((uint16_t)((j & 1) ? hw >> 16 : hw & 0xffffu)), -er);
            const int64_t bq = pack2((uint32_t)wc.q[j][0], (uint32_t)wc.q[j][1]);
#pragma unroll
            for (int mt = 0; mt < NMT; mt++) {
                const int64_t av = *(const int64_t*)&s_codes[buf][mt * 16 + nl][8 * kq + 32 * j];
                const v4i d = mfma16(av, bq, v4i{0, 0, 0, 0});
#pragma unroll
                for (int i = 0; i < 4; i++)
                    S[mt][i] += rint(dwj * s_dad[buf][mt * 16 + 4 * kq + i][j] * (double)d[i]);   // |dot| <= 32*127*127
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        stage_store(buf ^ 1, cv, dv);
        __syncthreads();
        wc = wn;
    }

    double* g = a.gsum + (int64_t)tile * 64 + nrow;
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = rbase + mt * 16 + 4 * kq + i;
            if (m < M) {
                double* p = g + (int64_t)(a.m0 + m) * a.n_pad;
                if (a.ksplit == 1) *p = S[mt][i];
                else unsafeAtomicAdd(p, S[mt][i]);
            }
        }
}

// The same for Q6_K weights (Q8_K activations).  Per (activation row m,
// weight row n, unit) the integer isum = sum_g sc_g * dot_g over the 16
// groups of 16 codes (q - 32), then one binary64 term rint(A * isum) as the
// contract has it.  Per 32-element chunk c (half h = c / 4, quarter s = c %
// 4) a lane's 8 codes are the low (s < 2) or high nibbles of ql bytes 64 h +
// 32 (s & 1) + 8 kq .., with qh bits 2 s, 2 s + 1 of bytes 32 h + 8 kq ..
// above them; the chunk's two groups go through two MFMAs whose B operands
// hold the codes in the group's k slots (kq < 2, kq >= 2) and zeros in the
// other's.  A unit's pieces: ql 0-7, qh 8-11, the 16 group scales 12; the
// unit's d (f16) lies in a region of its own after the tiles.
// NMT: 16-row blocks of the 64 that hold rows (fewer when M <= 48)
template <int NMT>
__global__ __launch_bounds__(WT) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_wide_q6k_kernel(WideArgs a)
{
    __shared__ __align__(16) uint8_t s_codes[2][16 * NMT][WROW];
    __shared__ double s_dad[2][16 * NMT];   // da * 2^(win - Ea) per staged row
    __shared__ double s_sm[WBM];        // 2^(win - Ea(m)), 0 for an all-zero row

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int U = a.U, M = a.M;
    const int64_t Kp = (int64_t)U * 256;

    const int nb = gridDim.x, b0 = blockIdx.x;
    const int L = (nb & 7) == 0 ? (b0 & 7) * (nb >> 3) + (b0 >> 3) : b0;
    const int mb = L % a.mblocks, r0 = L / a.mblocks;
    const int ks = r0 % a.ksplit, tile = r0 / a.ksplit;
    const int u0 = ks * a.upk, u1 = min(U, u0 + a.upk);
    const int rbase = mb * WBM;

    for (int r = wave; r < WBM; r += WT / 64) {
        const int mr = a.m0 + min(rbase + r, M - 1);
        float mx = 0.0f;
        for (int u = lane; u < U; u += 64) mx = fmaxf(mx, fabsf(a.da[(int64_t)mr * U + u]));
        mx = cpv_wave_reduce(mx, cpv_op_max());
        if (lane == 0) {
            int e = CPV_E_EMPTY;
            if (mx > 0.0f) frexpf(mx, &e);
            s_sm[r] = e == CPV_E_EMPTY ? 0.0 : ldexp(1.0, a.win - e);
        }
    }

    const int8_t* qbase = a.qa + (int64_t)(a.m0 + rbase) * Kp;
    int soff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int p = tid + q * WT, r = p >> 4;
        soff[q] = (min(rbase + r, M - 1) - rbase) * (int)Kp + (p & 15) * 16;
    }
    const float* sda = a.da + (int64_t)(a.m0 + min(rbase + (tid & 63), M - 1)) * U;
    auto stage_load = [&](int u, v4i* cv, float& dv) {
#pragma unroll
        for (int q = 0; q < NMT; q++) cv[q] = *(const v4i*)(qbase + soff[q] + u * 256);
        dv = sda[u];
    };
    auto stage_store = [&](int buf, const v4i* cv, float dv) {
#pragma unroll
        for (int q = 0; q < NMT; q++) {
            const int p = tid + q * WT;
            *(v4i*)&s_codes[buf][p >> 4][(p & 15) * 16] = cv[q];
        }
        if (tid < 16 * NMT) s_dad[buf][tid] = (double)dv * s_sm[tid];
    };

    const int nl = lane & 15, kq = lane >> 4;
    const int nrow = wave * 16 + nl;
    const uint8_t* wrow = a.w + (int64_t)tile * U * 13 * 1024 + nrow * 16;
    const uint16_t* drow = (const uint16_t*)(a.w + (int64_t)(a.n_pad / 64) * U * 13 * 1024) + (int64_t)tile * U * 64 + nrow;
    struct Wt { v2i ql[2][2]; v2i qh[2]; v4i s; uint32_t d; };
    auto wload = [&](int u, Wt& t) {
        const uint8_t* p = wrow + (int64_t)u * 13 * 1024 + 8 * (kq & 1);
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int s1 = 0; s1 < 2; s1++) t.ql[h][s1] = *(const v2i*)(p + (4 * h + 2 * s1 + (kq >> 1)) * 1024);
            t.qh[h] = *(const v2i*)(p + (8 + 2 * h + (kq >> 1)) * 1024);
        }
        t.s = *(const v4i*)(wrow + (int64_t)u * 13 * 1024 + 12 * 1024);
        t.d = drow[(int64_t)u * 64];
    };
    const int er = a.ew[(int64_t)tile * 64 + nrow];
    // the 4 codes of a dword as signed bytes q - 32 (q in 0..63: q ^ 32,
    // with bits 6 and 7 set where q < 32)
    auto centered = [](uint32_t q) {
        const uint32_t t = q ^ 0x20202020u;
        return t | (((t >> 5) & 0x01010101u) * 0xc0u);
    };

    double S[NMT][4];
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) S[mt][i] = 0.0;

    Wt wc, wn;
    v4i cv[NMT];
    float dv;
    wload(u0, wc);
    stage_load(u0, cv, dv);
    __syncthreads();                    // s_sm
    stage_store(0, cv, dv);
    __syncthreads();

    for (int u = u0; u < u1; u++) {
        const int buf = (u - u0) & 1;
        const int un = u + 1 < u1 ? u + 1 : u;
        wload(un, wn);
        stage_load(un, cv, dv);
        const double dws = ldexp((double)cpv_h2f((uint16_t)wc.d), -er);
        int isum[NMT][4];
#pragma unroll
        for (int mt = 0; mt < NMT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) isum[mt][i] = 0;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int h = c >> 2, sq = c & 3;
            uint32_t cw[2];
#pragma unroll
            for (int x = 0; x < 2; x++) {
                const uint32_t lo = ((uint32_t)wc.ql[h][sq & 1][x] >> (4 * (sq >> 1))) & 0x0f0f0f0fu;
                const uint32_t hi = (((uint32_t)wc.qh[h][x] >> (2 * sq)) & 0x03030303u) << 4;
                cw[x] = centered(lo | hi);
            }
            const int64_t bc = pack2(cw[0], cw[1]);
            const int64_t b0v = kq < 2 ? bc : 0, b1v = kq < 2 ? 0 : bc;   // group 2c, group 2c + 1
            const uint32_t sw = (uint32_t)wc.s[c >> 1];
            const int sc0 = (int)(int8_t)(sw >> (16 * (c & 1))), sc1 = (int)(int8_t)(sw >> (16 * (c & 1) + 8));
#pragma unroll
            for (int mt = 0; mt < NMT; mt++) {
                const int64_t av = *(const int64_t*)&s_codes[buf][mt * 16 + nl][8 * kq + 32 * c];
                const v4i d0 = mfma16(av, b0v, v4i{0, 0, 0, 0});
                const v4i d1 = mfma16(av, b1v, v4i{0, 0, 0, 0});
#pragma unroll
                for (int i = 0; i < 4; i++) isum[mt][i] += sc0 * d0[i] + sc1 * d1[i];   // |isum| < 2^28
            }
#pragma unroll
            for (int mt = 0; mt < NMT; mt++)
                asm volatile("" : "+v"(isum[mt][0]), "+v"(isum[mt][1]), "+v"(isum[mt][2]), "+v"(isum[mt][3]));
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int mt = 0; mt < NMT; mt++) {
            const double* dd = &s_dad[buf][mt * 16 + 4 * kq];
#pragma unroll
            for (int i = 0; i < 4; i++) S[mt][i] += rint(dws * dd[i] * (double)isum[mt][i]);
        }
        stage_store(buf ^ 1, cv, dv);
        __syncthreads();
        wc = wn;
    }

    double* g = a.gsum + (int64_t)tile * 64 + nrow;
#pragma unroll
    for (int mt = 0; mt < NMT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = rbase + mt * 16 + 4 * kq + i;
            if (m < M) {
                double* p = g + (int64_t)(a.m0 + m) * a.n_pad;
                if (a.ksplit == 1) *p = S[mt][i];
                else unsafeAtomicAdd(p, S[mt][i]);
            }
        }
}

}  // namespace

bool cpv_qgemm_wide_ok(const cpv_weight* w, int64_t m)
{
    // (Q6_K and Q8_0 from 9 rows: one 16-row block streams the weights once
    // where Q6_K's skinny kernel takes them in 8-row passes and Q8_0's runs
    // one wave per SIMD; Q4_K from 17, past its own 16-row kernel: at 24
    // rows 34 against 46 us, at 16 the 16-row kernel's 27 against 28 us)
    return (w->type == CPV_Q4_K && m > 16) || ((w->type == CPV_Q6_K || w->type == CPV_Q8_0) && m > 8);
}

cpv_status cpv_qgemm_wide(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, double* gsum, int win)
{
    const bool q80 = w->type == CPV_Q8_0, q6k = w->type == CPV_Q6_K;
    if ((w->type != CPV_Q4_K && !q80 && !q6k) || act->kq == q80 || act->U != (int)w->units || act->m < 1 ||
        act->m > INT32_MAX / 2)
        return cpv_fail(ctx, CPV_EINVAL, "qgemm_wide: weight or activation format not supported");
    if ((int64_t)WBM * act->U * 256 > INT32_MAX)   // the staging offsets within a row block are 32-bit
        return cpv_fail(ctx, CPV_EUNSUPPORTED, "qgemm_wide: k=%lld too long", (long long)w->k);
    WideArgs a;
    a.w = (const uint8_t*)w->data;
    a.ew = w->ew;
    a.qa = act->qa;
    a.da = act->da;
    a.gsum = gsum;
    a.n_pad = w->n_pad;
    a.U = act->U;
    a.M = (int)act->m;
    a.m0 = 0;
    a.win = win;
    a.tiles = (int)(w->n_pad / 64);
    a.mblocks = (a.M + WBM - 1) / WBM;
    // slice K when the grid would leave CUs idle (about 3 workgroups fit a CU)
    const int64_t blocks = (int64_t)a.tiles * a.mblocks, want = 3LL * ctx->cu_count;
    int ksplit = blocks >= want ? 1 : (int)((want + blocks - 1) / blocks);
    if (ksplit > a.U / 4) ksplit = a.U / 4 > 1 ? a.U / 4 : 1;
    a.upk = (a.U + ksplit - 1) / ksplit;
    a.ksplit = (a.U + a.upk - 1) / a.upk;
    const int64_t grid = blocks * a.ksplit;
    if (grid > INT32_MAX) return cpv_fail(ctx, CPV_EUNSUPPORTED, "qgemm_wide: grid of %lld", (long long)grid);
    const int ev = cpv_prof_mark(ctx);
    auto go = [=]() {
        if (q80 && a.M <= 16) qgemm_wide_q80_kernel<1><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (q80 && a.M <= 32) qgemm_wide_q80_kernel<2><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (q80) qgemm_wide_q80_kernel<4><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (q6k && a.M <= 16) qgemm_wide_q6k_kernel<1><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (q6k && a.M <= 32) qgemm_wide_q6k_kernel<2><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (q6k) qgemm_wide_q6k_kernel<4><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (a.M <= 16) qgemm_wide_kernel<1><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else if (a.M <= 32) qgemm_wide_kernel<2><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
        else qgemm_wide_kernel<4><<<(unsigned)grid, WT, 0, ctx->stream>>>(a);
    };
    go();
    CPV_HIP(ctx, hipGetLastError());
    if (ev >= 0) {  // algorithmic bytes: the weight, f32 activations in, f32 outputs
        const double wrow_b = q80 ? (double)(w->k / 32) * 34.0 : (double)(w->k / 256) * (q6k ? 210.0 : 144.0);
        const double bytes = (double)w->n * wrow_b + 4.0 * a.M * (double)w->k + 4.0 * a.M * (double)w->n;
        const int cls = q80 ? CPV_PROF_Q8_0_WIDE : q6k ? CPV_PROF_Q6_K_WIDE : CPV_PROF_Q4_K_WIDE;
        cpv_prof_add(ctx, ev, cls, bytes);
        cpv_prof_keep(ctx, cls, bytes, go);
    }
    return CPV_OK;
}
