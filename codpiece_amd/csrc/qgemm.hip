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
// Mapping.  A workgroup owns 16 weight rows and all of K.  Lane = r + 16 q of
// a wave handles row r and unit q of each pass of 4 units; the waves of the
// group take passes round-robin.  Activation codes for all of K are staged in
// LDS once per group; the 16 lanes of a q share every LDS read (broadcast).
// Weights come in through 128-bit loads that are contiguous per wave (see the
// repack in api.hip).  Partial sums reduce across q with shuffles and across
// waves through LDS, then one rounding to f32 per output.
#include <math.h>

#include "cpv_internal.h"

namespace {

constexpr int UNIT_STRIDE = 272;   // LDS bytes per 256 codes (+16 breaks bank aliasing)

__device__ __forceinline__ float h2f(uint32_t h) { return cpv_h2f((uint16_t)h); }

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

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
    float ax = fabsf(v);
    int ix = t;
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(ax, off);
        const int oi = __shfl_xor(ix, off);
        if (oa > ax || (oa == ax && oi < ix)) { ax = oa; ix = oi; }
    }
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
    int s16 = q;
    for (int off = 8; off > 0; off >>= 1) s16 += __shfl_xor(s16, off);
    int s32 = s16 + __shfl_xor(s16, 16);
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
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)roundf(v * id);
    const int64_t Kp = (int64_t)U * 256;
    qa[(int64_t)m * Kp + e] = (int8_t)q;
    if ((t & 31) == 0) da[((int64_t)m * U + u) * 8 + (t >> 5)] = cpv_h2f(cpv_f2h(d));
}

// ---------------------------------------------------------------- GEMM
struct GemmArgs {
    const uint8_t* w;      // repacked weight
    const int32_t* ew;     // [n_pad] row exponents
    const int8_t* qa;      // [M][Kp] codes
    const float* da;       // [M][U] (K-quants) or [M][U*8] (Q8_0)
    const int32_t* bs;     // [M][U*8] (Q4_K) or [M][U*16] (Q6_K)
    float* y;              // [M][N]
    int64_t N, n_pad;
    int P, U, M, m0, Mtot, win;
};

template <int TYPE>
struct Layout {
    static constexpr int PIECES = TYPE == CPV_Q4_K ? 8 : TYPE == CPV_Q6_K ? 13 : 16;
    static constexpr int DA_PER_UNIT = TYPE == CPV_Q8_0 ? 8 : 1;
    static constexpr int BS_PER_UNIT = TYPE == CPV_Q4_K ? 8 : TYPE == CPV_Q6_K ? 16 : 0;
};

template <int TYPE, int MT>
__host__ __device__ inline size_t gemm_lds_bytes(int U, int W)
{
    using L = Layout<TYPE>;
    return (size_t)MT * U * UNIT_STRIDE + (size_t)MT * U * L::DA_PER_UNIT * 8 +
           (size_t)MT * U * L::BS_PER_UNIT * 4 + (size_t)W * 16 * MT * 8;
}

template <int TYPE, int MT>
__global__ __launch_bounds__(512) void qgemm_kernel(GemmArgs a)
{
    using L = Layout<TYPE>;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ea[MT];
    const int U = a.U, P = a.P, M = a.M;
    const int tid = threadIdx.x, nthr = blockDim.x, W = nthr >> 6;
    uint8_t* s_qa = smem;
    double* s_da = (double*)(smem + (size_t)MT * U * UNIT_STRIDE);
    int32_t* s_bs = (int32_t*)(s_da + (size_t)MT * U * L::DA_PER_UNIT);
    double* s_red = (double*)(s_bs + (size_t)MT * U * L::BS_PER_UNIT);
    const int64_t Kp = (int64_t)U * 256;

    // stage codes (16 B at a time) and code sums
    for (int i = tid; i < M * U * 16; i += nthr) {
        const int m = i / (U * 16), rest = i % (U * 16), u = rest >> 4, c = rest & 15;
        const uint4 v = *(const uint4*)(a.qa + (int64_t)(a.m0 + m) * Kp + (int64_t)u * 256 + c * 16);
        *(uint4*)(s_qa + ((size_t)m * U + u) * UNIT_STRIDE + c * 16) = v;
    }
    if (L::BS_PER_UNIT)
        for (int i = tid; i < M * U * L::BS_PER_UNIT; i += nthr)
            s_bs[i] = a.bs[(int64_t)a.m0 * U * L::BS_PER_UNIT + i];
    // Ea(m): exponent of the row's largest activation scale
    if (tid < 64) {
        for (int m = 0; m < M; m++) {
            float mx = 0.0f;
            for (int i = tid; i < U * L::DA_PER_UNIT; i += 64)
                mx = fmaxf(mx, fabsf(a.da[(int64_t)(a.m0 + m) * U * L::DA_PER_UNIT + i]));
            for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            if (tid == 0) {
                int e = CPV_E_EMPTY;
                if (mx > 0.0f) frexpf(mx, &e);
                s_ea[m] = e;
            }
        }
    }
    __syncthreads();
    // activation scales pre-multiplied by 2^(win - Ea(m)) (exact)
    for (int i = tid; i < M * U * L::DA_PER_UNIT; i += nthr) {
        const int m = i / (U * L::DA_PER_UNIT);
        const int e = s_ea[m];
        const double v = (double)a.da[(int64_t)a.m0 * U * L::DA_PER_UNIT + i];
        s_da[i] = e == CPV_E_EMPTY ? 0.0 : ldexp(v, a.win - e);
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63, r = lane & 15, q = lane >> 4;
    const int64_t g = blockIdx.x;
    const int er = a.ew[g * 16 + r];
    const uint4* wq = (const uint4*)a.w;
    const int64_t groups = a.n_pad / 16;
    const int64_t region_a = groups * P * L::PIECES * 64;      // in uint4

    double acc[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = 0.0;

    for (int p = wave; p < P; p += W) {
        const int u = p * 4 + q;
        const uint4* src = wq + (g * P + p) * L::PIECES * 64 + lane;
        uint4 pc[L::PIECES];
#pragma unroll
        for (int i = 0; i < L::PIECES; i++) pc[i] = src[i * 64];

        if constexpr (TYPE == CPV_Q4_K) {
            const uint4 meta = wq[region_a + (g * P + p) * 64 + lane];
            const double dws = ldexp((double)h2f(meta.x & 0xffffu), -er);
            const double dms = ldexp((double)h2f(meta.x >> 16), -er);
            const uint32_t sc_lo = meta.y & 0x3f3f3f3fu, mn_lo = meta.z & 0x3f3f3f3fu;
            const uint32_t sc_hi = (meta.w & 0x0f0f0f0fu) | (((meta.y >> 6) & 0x03030303u) << 4);
            const uint32_t mn_hi = ((meta.w >> 4) & 0x0f0f0f0fu) | (((meta.z >> 6) & 0x03030303u) << 4);
            const uint32_t* nw = (const uint32_t*)pc;     // 32 dwords, chunk c = dwords 8c..8c+7
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m < M) {
                    const int* av = (const int*)(s_qa + ((size_t)m * U + u) * UNIT_STRIDE);
                    int isum = 0, imin = 0;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        int dlo = 0, dhi = 0;
#pragma unroll
                        for (int dd = 0; dd < 8; dd++) {
                            const uint32_t wv = nw[c * 8 + dd];
                            dlo = sdot4((int)(wv & 0x0f0f0f0fu), av[c * 16 + dd], dlo);
                            dhi = sdot4((int)((wv >> 4) & 0x0f0f0f0fu), av[c * 16 + 8 + dd], dhi);
                        }
                        const uint32_t scw = c < 2 ? sc_lo : sc_hi, mnw = c < 2 ? mn_lo : mn_hi;
                        const int j0 = (2 * c) & 3, j1 = (2 * c + 1) & 3;
                        isum += byte_of(scw, j0) * dlo + byte_of(scw, j1) * dhi;
                        const int32_t* bsu = s_bs + ((size_t)m * U + u) * 8;
                        imin += byte_of(mnw, j0) * bsu[2 * c] + byte_of(mnw, j1) * bsu[2 * c + 1];
                    }
                    const double das = s_da[(size_t)m * U + u];
                    acc[m] += rint(dws * das * (double)isum) - rint(dms * das * (double)imin);
                }
            }
        } else if constexpr (TYPE == CPV_Q6_K) {
            const uint16_t dbits = *((const uint16_t*)(wq + region_a) + (g * P + p) * 64 + lane);
            const double dws = ldexp((double)h2f(dbits), -er);
            const uint32_t* ql = (const uint32_t*)pc;         // 32 dwords
            const uint32_t* qh = ql + 32;                     // 16 dwords
            const uint32_t* scw = ql + 48;                    // 4 dwords, 16 int8 scales
            // unsigned 6-bit codes, element order, 64 dwords
            uint32_t code[64];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int dd = 0; dd < 8; dd++) {
                    const uint32_t l0 = ql[h * 16 + dd], l1 = ql[h * 16 + 8 + dd], hb = qh[h * 8 + dd];
                    code[h * 32 + 0 + dd] = (l0 & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4);
                    code[h * 32 + 8 + dd] = (l1 & 0x0f0f0f0fu) | (((hb >> 2) & 0x03030303u) << 4);
                    code[h * 32 + 16 + dd] = ((l0 >> 4) & 0x0f0f0f0fu) | (((hb >> 4) & 0x03030303u) << 4);
                    code[h * 32 + 24 + dd] = ((l1 >> 4) & 0x0f0f0f0fu) | (((hb >> 6) & 0x03030303u) << 4);
                }
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m < M) {
                    const int* av = (const int*)(s_qa + ((size_t)m * U + u) * UNIT_STRIDE);
                    const int32_t* bsu = s_bs + ((size_t)m * U + u) * 16;
                    int isum = 0;
#pragma unroll
                    for (int gi = 0; gi < 16; gi++) {
                        int dg = 0;
#pragma unroll
                        for (int dd = 0; dd < 4; dd++) dg = sdot4((int)code[gi * 4 + dd], av[gi * 4 + dd], dg);
                        const int sc = (int)(int8_t)byte_of(scw[gi >> 2], gi & 3);
                        isum += sc * (dg - 32 * bsu[gi]);
                    }
                    acc[m] += rint(dws * s_da[(size_t)m * U + u] * (double)isum);
                }
            }
        } else {
            const uint4 dq = wq[region_a + (g * P + p) * 64 + lane];
            const uint32_t dw4[4] = {dq.x, dq.y, dq.z, dq.w};
            const uint32_t* qs = (const uint32_t*)pc;         // 64 dwords, block b = 8b..8b+7
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m < M) {
                    const int* av = (const int*)(s_qa + ((size_t)m * U + u) * UNIT_STRIDE);
                    const double* das = s_da + ((size_t)m * U + u) * 8;
#pragma unroll
                    for (int b = 0; b < 8; b++) {
                        int isum = 0;
#pragma unroll
                        for (int dd = 0; dd < 8; dd++) isum = sdot4((int)qs[b * 8 + dd], av[b * 8 + dd], isum);
                        const uint32_t hb = (dw4[b >> 1] >> (16 * (b & 1))) & 0xffffu;
                        const double dws = ldexp((double)h2f(hb), -er);
                        acc[m] += rint(dws * das[b] * (double)isum);
                    }
                }
            }
        }
    }

    // exact reduction: over the 4 units of a row, then over waves
#pragma unroll
    for (int m = 0; m < MT; m++) {
        acc[m] += __shfl_xor(acc[m], 16);
        acc[m] += __shfl_xor(acc[m], 32);
    }
    if (q == 0)
#pragma unroll
        for (int m = 0; m < MT; m++) s_red[((size_t)wave * 16 + r) * MT + m] = acc[m];
    __syncthreads();
    for (int t = tid; t < 16 * M; t += nthr) {
        const int rr = t & 15, m = t >> 4;
        const int64_t row = g * 16 + rr;
        if (row >= a.N) continue;
        double s = 0.0;
        for (int w = 0; w < W; w++) s += s_red[((size_t)w * 16 + rr) * MT + m];
        const int ew = a.ew[row], ea = s_ea[m];
        float out = 0.0f;
        if (ew != CPV_E_EMPTY && ea != CPV_E_EMPTY) out = (float)ldexp(s, ew + ea - a.win);
        a.y[(int64_t)(a.m0 + m) * a.N + row] = out;
    }
}

// one launch of the GEMM; k and wbytes (the weight's row length and bytes)
// only feed the kernel timing
template <int TYPE, int MT>
cpv_status launch_mt(cpv_ctx* ctx, GemmArgs a, int W, int64_t k, double wbytes)
{
    const size_t lds = gemm_lds_bytes<TYPE, MT>(a.U, W);
    auto go = [=]() { qgemm_kernel<TYPE, MT><<<(unsigned)(a.n_pad / 16), W * 64, lds, ctx->stream>>>(a); };
    const int ev = cpv_prof_mark(ctx);
    go();
    CPV_HIP(ctx, hipGetLastError());
    if (ev >= 0) {  // algorithmic bytes: the weight, f32 activations in, f32 outputs
        const int cls = TYPE == CPV_Q4_K ? CPV_PROF_Q4_K : TYPE == CPV_Q6_K ? CPV_PROF_Q6_K : CPV_PROF_Q8_0;
        const double bytes = wbytes + 4.0 * a.M * (double)k + 4.0 * a.M * (double)a.N;
        cpv_prof_add(ctx, ev, cls, bytes);
        cpv_prof_keep(ctx, cls, bytes, go);
    }
    return CPV_OK;
}

template <int TYPE>
cpv_status launch_type(cpv_ctx* ctx, GemmArgs a, int W, int64_t k, double wbytes)
{
    // the register tile MT is the smallest instantiated size >= M
    if (a.M <= 1) return launch_mt<TYPE, 1>(ctx, a, W, k, wbytes);
    if (a.M <= 2) return launch_mt<TYPE, 2>(ctx, a, W, k, wbytes);
    if (a.M <= 4) return launch_mt<TYPE, 4>(ctx, a, W, k, wbytes);
    if (a.M <= 5) return launch_mt<TYPE, 5>(ctx, a, W, k, wbytes);
    if (a.M <= 8) return launch_mt<TYPE, 8>(ctx, a, W, k, wbytes);
    return launch_mt<TYPE, 16>(ctx, a, W, k, wbytes);
}

template <int TYPE>
size_t lds_for(int M, int U, int W)
{
    if (M <= 1) return gemm_lds_bytes<TYPE, 1>(U, W);
    if (M <= 2) return gemm_lds_bytes<TYPE, 2>(U, W);
    if (M <= 4) return gemm_lds_bytes<TYPE, 4>(U, W);
    if (M <= 5) return gemm_lds_bytes<TYPE, 5>(U, W);
    if (M <= 8) return gemm_lds_bytes<TYPE, 8>(U, W);
    return gemm_lds_bytes<TYPE, 16>(U, W);
}

static int isum_bits(int type) { return type == CPV_Q8_0 ? 20 : type == CPV_Q4_K ? 25 : 28; }

}  // namespace

int cpv_qgemm_window(int type, int64_t k)
{
    const int64_t terms = type == CPV_Q8_0 ? k / 32 : type == CPV_Q4_K ? 2 * (k / 256) : k / 256;
    int b = 0;
    while (((int64_t)1 << b) < terms + 1) b++;
    return 52 - isum_bits(type) - b;
}

size_t cpv_act_bytes(int type, int64_t k, int64_t m)
{
    const int64_t U = ((k + 255) / 256 + 3) / 4 * 4;
    const bool kq = type != CPV_Q8_0;
    const size_t qa_b = ((size_t)m * U * 256 + 255) & ~(size_t)255;
    const size_t da_b = ((size_t)m * U * (kq ? 1 : 8) * 4 + 255) & ~(size_t)255;
    const size_t bs_b = kq ? (size_t)m * U * (8 + 16) * 4 : 0;
    return qa_b + da_b + bs_b;
}

cpv_status cpv_quant_act(cpv_ctx* ctx, int type, const float* x, int64_t m, int64_t k, void* buf, cpv_act* out)
{
    const int U = (int)(((k + 255) / 256 + 3) / 4 * 4);
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

cpv_status cpv_qgemm_act(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, float* y)
{
    const bool kq = w->type != CPV_Q8_0;
    if (kq != act->kq || act->k != w->k || act->U != (int)(w->passes * 4))
        return cpv_fail(ctx, CPV_EINVAL, "qgemm: activation format does not match the weight");
    const int U = act->U;
    const int64_t m = act->m;
    const int P = (int)w->passes;
    const int per = (P + 7) / 8;
    const int W = (P + per - 1) / per;
    GemmArgs a;
    a.w = (const uint8_t*)w->data;
    a.ew = w->ew;
    a.qa = act->qa;
    a.da = act->da;
    a.bs = w->type == CPV_Q4_K ? act->bs32 : act->bs16;
    a.y = y;
    a.N = w->n;
    a.n_pad = w->n_pad;
    a.P = P;
    a.U = U;
    a.Mtot = (int)m;
    a.win = cpv_qgemm_window(w->type, w->k);
    // activation rows per launch: as many as fit the workgroup's LDS
    int chunk = m < 16 ? (int)m : 16;
    auto lds = [&](int c) {
        return w->type == CPV_Q4_K ? lds_for<CPV_Q4_K>(c, U, W)
             : w->type == CPV_Q6_K ? lds_for<CPV_Q6_K>(c, U, W) : lds_for<CPV_Q8_0>(c, U, W);
    };
    const size_t lds_cap = ctx->lds_max - 1024;    // less the static shared words
    while (chunk > 1 && lds(chunk) > lds_cap) chunk--;
    if (lds(chunk) > lds_cap)
        return cpv_fail(ctx, CPV_EUNSUPPORTED, "qgemm: k=%lld needs more LDS than a CU has", (long long)w->k);
    for (int64_t m0 = 0; m0 < m; m0 += chunk) {
        a.m0 = (int)m0;
        a.M = (int)((m - m0) < chunk ? (m - m0) : chunk);
        const double wb = (double)w->n * (double)(w->k / cpv_type_block(w->type)) * (double)cpv_type_size(w->type);
        cpv_status s2 = w->type == CPV_Q4_K ? launch_type<CPV_Q4_K>(ctx, a, W, w->k, wb)
                      : w->type == CPV_Q6_K ? launch_type<CPV_Q6_K>(ctx, a, W, w->k, wb)
                                            : launch_type<CPV_Q8_0>(ctx, a, W, w->k, wb);
        if (s2 != CPV_OK) return s2;
    }
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
    if (m < 1 || m > 64) return cpv_fail(ctx, CPV_EINVAL, "qgemm: m=%lld outside [1, 64]", (long long)m);
    if (w->ctx != ctx) return cpv_fail(ctx, CPV_EINVAL, "qgemm: weight belongs to another context");
    return cpv_qgemm_launch(ctx, w, x_dev, m, y_dev);
}
