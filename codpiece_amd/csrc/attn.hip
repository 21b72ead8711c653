// attn.hip — tree-masked GQA attention over the f16 KV cache, exact and
// order-free: the same bits whatever the grid, the split of the KV axis or
// the number of query rows in a call.
//
// Replaces the attention of build_attn_block (crates/codpiece-model/src/
// qwen35.rs:3182-3199): ggml_flash_attn_ext with prec F32 by default (the
// session's fa flag, qwen35.rs:534), or mul_mat(k, q) -> soft_max_ext(scale,
// mask) -> mul_mat(v, p).  Both ggml CPU paths round q to f16 (the f16
// cache's vec_dot_type) and sum in an order set by the SIMD width (and the
// FA kernel accumulates p.v in f16).  The contract here keeps the f16 q and
// makes every sum exact or fixed-order (the oracle's cpvo_attn states it):
//  1. scores: q16 and each cache row k16 become 15-bit fixed point relative
//     to their own largest element (qf = rint(q16 2^(14-Eq)), kf likewise);
//     s = (float)(sum_d qf kf * 2^(Eq+Ek-28)), the sum exact -- here on the
//     int8 MFMA with two signed 8-bit limbs per operand.
//  2. w = s * scale, mx = max over visible rows, e = expf(w - mx).
//  3. Z = sum rint(e 2^G) exactly (G = 62 - ceil_log2(n_vis + 1)),
//     inv = (float)(1 / (Z 2^-G)), p = f16(e * inv).
//  4. per 256-row chunk of the cache (absolute rows) P_c = fma chain over its
//     rows in increasing order; out = ((0 + P_0) + P_1) + ... in f32.
//
// Kernels: scores (grid: chunk x KV head x 32-row query block), softmax (one
// block per query row), pv (chunk x KV head x 8-row groups; lane = d), fold
// (per output element).  Scratch in the context workspace: w [T*H][n] f32,
// p [h_kv][n][LRp] f16 (LRp = query rows of a KV head, padded to 8),
// partials [chunks][T*H][D] f32.
//
// Layout.  K is [n_ctx][h_kv * d]; V is the transposed cache [h_kv * d][v_stride]
// (the reference's non-FA V layout, qwen35.rs:580-586): the KV axis is
// contiguous, the reduction axis of P V.
#include <math.h>

#include "cpv_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int CHUNK = 256;          // cache rows per chunk (the fold unit of the contract)
constexpr int QB = 32;              // query rows per scores workgroup
constexpr int E_EMPTY = -100000;    // exponent of an all-zero vector

__device__ __forceinline__ int ceil_log2_dev(int64_t v)
{
    int b = 0;
    while (((int64_t)1 << b) < v) b++;
    return b;
}

// visibility of cache row j for node t: context rows, then the node's
// ancestors and itself (tree, bit mask anc) or every node up to t (chain)
__device__ __forceinline__ bool visible(int64_t j, int64_t n_past, int t, bool tree, uint64_t anc)
{
    if (j < n_past) return true;
    const int64_t node = j - n_past;
    return tree ? ((anc >> node) & 1ull) != 0 : node <= t;
}

__device__ __forceinline__ uint64_t ancestors(const int32_t* parent, int t)
{
    uint64_t m = 0;
    for (int a = t; a >= 0; a = parent[a]) m |= 1ull << a;
    return m;
}

// 15-bit fixed point of an f16 value at exponent e, split into two signed
// 8-bit limbs: f = 256 hi + lo, lo in [-128, 127], |hi| <= 64
__device__ __forceinline__ void limbs(float v, int e, int8_t* hi, int8_t* lo)
{
    int f = 0;
    if (e != E_EMPTY) f = (int)rintf(ldexpf(v, 14 - e));
    const int h = (f + 128) >> 8;
    *hi = (int8_t)h;
    *lo = (int8_t)(f - 256 * h);
}

struct ScoreArgs {
    const float* q;           // [T][H][D]
    const uint16_t* kc;       // [n_ctx][Hkv*D]
    const int32_t* parent;    // [T] or null
    float* w;                 // [T*H][n]  scaled scores, -inf where invisible
    int64_t n_past, n;        // n = n_past + T rows in play
    int T, H, Hkv;
    float scale;
};

// scores of 32 query rows (of one KV head) against one 256-row chunk
template <int D>
__global__ __launch_bounds__(256) void attn_scores_kernel(ScoreArgs a)
{
    constexpr int TPR = D / 16;                // threads per row when converting (16 values each)
    constexpr int RPP = 256 / TPR;             // rows per pass
    __shared__ __align__(16) int8_t s_qh[QB][D], s_ql[QB][D];
    __shared__ __align__(16) int8_t s_kh[CHUNK][D], s_kl[CHUNK][D];
    __shared__ int s_eq[QB], s_ek[CHUNK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x, kh = blockIdx.y;
    const int G = a.H / a.Hkv, LR = G * a.T;
    const int64_t j0 = (int64_t)c * CHUNK;
    const int sub = tid % TPR;

    // ---- query rows lr = blockIdx.z * 32 + r: t = lr / G, head kh * G + lr % G
    for (int r = tid / TPR; r < QB; r += RPP) {
        const int lr = blockIdx.z * QB + r;
        float v[16];
        float mx = 0.0f;
        if (lr < LR) {
            const int t = lr / G, h = kh * G + lr % G;
            const float* src = a.q + ((int64_t)t * a.H + h) * D + sub * 16;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                v[i] = cpv_h2f(cpv_f2h(src[i]));
                mx = fmaxf(mx, fabsf(v[i]));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = 0.0f;
        }
        for (int off = 1; off < TPR; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        int e = E_EMPTY;
        if (mx > 0.0f) frexpf(mx, &e);
#pragma unroll
        for (int i = 0; i < 16; i++) limbs(v[i], e, &s_qh[r][sub * 16 + i], &s_ql[r][sub * 16 + i]);
        if (sub == 0) s_eq[r] = e;
    }
    // ---- the chunk's cache rows of this KV head
    for (int r = tid / TPR; r < CHUNK; r += RPP) {
        const int64_t j = j0 + r;
        float v[16];
        float mx = 0.0f;
        if (j < a.n) {
            const uint16_t* src = a.kc + j * (int64_t)a.Hkv * D + (int64_t)kh * D + sub * 16;
            const uint4 p0 = *(const uint4*)src, p1 = *(const uint4*)(src + 8);
            const uint32_t wds[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                v[i] = cpv_h2f((uint16_t)(wds[i >> 1] >> (16 * (i & 1))));
                mx = fmaxf(mx, fabsf(v[i]));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = 0.0f;
        }
        for (int off = 1; off < TPR; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        int e = E_EMPTY;
        if (mx > 0.0f) frexpf(mx, &e);
#pragma unroll
        for (int i = 0; i < 16; i++) limbs(v[i], e, &s_kh[r][sub * 16 + i], &s_kl[r][sub * 16 + i]);
        if (sub == 0) s_ek[r] = e;
    }
    __syncthreads();

    // ---- 2 x 16 output blocks of 16 x 16 (query rows x cache rows); 4 waves, 8 blocks each
    const bool tree = a.parent != nullptr;
    for (int blk = wave; blk < 2 * (CHUNK / 16); blk += 4) {
        const int qb = blk & 1, jb = blk >> 1;
        v4i hh = {0, 0, 0, 0}, mix = {0, 0, 0, 0}, ll = {0, 0, 0, 0};
        const int ar = qb * 16 + (lane & 15), bc = jb * 16 + (lane & 15), kg = (lane >> 4) * 16;
#pragma unroll
        for (int ks = 0; ks < D / 64; ks++) {
            const v4i qhv = *(const v4i*)&s_qh[ar][ks * 64 + kg], qlv = *(const v4i*)&s_ql[ar][ks * 64 + kg];
            const v4i khv = *(const v4i*)&s_kh[bc][ks * 64 + kg], klv = *(const v4i*)&s_kl[bc][ks * 64 + kg];
            hh = __builtin_amdgcn_mfma_i32_16x16x64_i8(qhv, khv, hh, 0, 0, 0);
            mix = __builtin_amdgcn_mfma_i32_16x16x64_i8(qhv, klv, mix, 0, 0, 0);
            mix = __builtin_amdgcn_mfma_i32_16x16x64_i8(qlv, khv, mix, 0, 0, 0);
            ll = __builtin_amdgcn_mfma_i32_16x16x64_i8(qlv, klv, ll, 0, 0, 0);
        }
        // lane holds rows 4 (lane/16) + i of the query block, cache row bc
        const int64_t j = j0 + bc;
        if (j >= a.n) continue;
        const int ek = s_ek[bc];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = qb * 16 + 4 * (lane >> 4) + i;
            const int lr = blockIdx.z * QB + r;
            if (lr >= LR) continue;
            const int t = lr / G, h = kh * G + lr % G;
            const uint64_t anc = tree ? ancestors(a.parent, t) : 0;
            float w = -INFINITY;
            if (visible(j, a.n_past, t, tree, anc)) {
                const int eq = s_eq[r];
                float s = 0.0f;
                if (eq != E_EMPTY && ek != E_EMPTY) {
                    const int64_t S = (int64_t)hh[i] * 65536 + (int64_t)mix[i] * 256 + (int64_t)ll[i];
                    s = (float)ldexp((double)S, eq + ek - 28);
                }
                w = s * a.scale;
            }
            a.w[((int64_t)t * a.H + h) * a.n + j] = w;
        }
    }
}

// one query row: max, exact normaliser, f16 probabilities (transposed per KV head)
__global__ __launch_bounds__(256) void attn_softmax_kernel(const float* __restrict__ w, int64_t n, int T, int H,
                                                           int Hkv, int LRp, uint16_t* __restrict__ p)
{
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = row / H, h = row % H, G = H / Hkv, kh = h / G, lr = t * G + h % G;
    const float* wr = w + (int64_t)row * n;
    __shared__ float s_m[4];
    __shared__ long long s_z[4];
    __shared__ int s_c[4];
    float mx = -INFINITY;
    int cnt = 0;
    for (int64_t j = tid; j < n; j += 256) {
        const float v = wr[j];
        if (v != -INFINITY) { mx = fmaxf(mx, v); cnt++; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        cnt += __shfl_xor(cnt, off);
    }
    if (lane == 0) { s_m[wave] = mx; s_c[wave] = cnt; }
    __syncthreads();
    mx = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    const int nvis = s_c[0] + s_c[1] + s_c[2] + s_c[3];
    const int Gz = 62 - ceil_log2_dev(nvis + 1);
    long long Z = 0;
    for (int64_t j = tid; j < n; j += 256) {
        const float v = wr[j];
        if (v != -INFINITY) Z += (long long)rint(ldexp((double)cpv_expf(v - mx), Gz));
    }
    for (int off = 32; off > 0; off >>= 1) Z += __shfl_xor(Z, off);
    if (lane == 0) s_z[wave] = Z;
    __syncthreads();
    Z = s_z[0] + s_z[1] + s_z[2] + s_z[3];
    const float inv = (float)(1.0 / ldexp((double)Z, -Gz));
    uint16_t* pr = p + (int64_t)kh * n * LRp + lr;
    for (int64_t j = tid; j < n; j += 256) {
        const float v = wr[j];
        pr[j * LRp] = v == -INFINITY ? (uint16_t)0 : cpv_f2h(cpv_expf(v - mx) * inv);
    }
}

// P_c for 8 query rows x D of one KV head and one chunk: lane = d, an fma chain over
// the chunk's rows in increasing order; the p of the 8 rows at a cache row is one
// uniform 16-byte load
template <int D>
__global__ __launch_bounds__(256) void attn_pv_kernel(const uint16_t* __restrict__ vt, int64_t v_stride,
                                                      const uint16_t* __restrict__ p, int64_t n, int LR, int LRp,
                                                      int T, int H, int Hkv, float* __restrict__ part)
{
    constexpr int WPR = D / 64;                // waves per 8-row group
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = blockIdx.x, kh = blockIdx.y;
    const int grp = blockIdx.z * (4 / WPR) + wave / WPR;   // 8-row group of this wave
    const int lr0 = grp * 8;
    if (lr0 >= LR) return;
    const int d = (wave % WPR) * 64 + lane;
    const int64_t j0 = (int64_t)c * CHUNK, j1 = j0 + CHUNK < n ? j0 + CHUNK : n;
    const uint16_t* vrow = vt + ((int64_t)kh * D + d) * v_stride;
    const uint16_t* pb = p + (int64_t)kh * n * LRp + lr0;
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; r++) acc[r] = 0.0f;
    int64_t j = j0;
    for (; j + 8 <= j1; j += 8) {
        const uint4 vv = *(const uint4*)(vrow + j);
        const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const float v = cpv_h2f((uint16_t)(vw[jj >> 1] >> (16 * (jj & 1))));
            const uint4 pp = *(const uint4*)(pb + (j + jj) * LRp);
            const uint32_t pw[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
            for (int r = 0; r < 8; r++) acc[r] = fmaf(cpv_h2f((uint16_t)(pw[r >> 1] >> (16 * (r & 1)))), v, acc[r]);
        }
    }
    for (; j < j1; j++) {
        const float v = cpv_h2f(vrow[j]);
        const uint4 pp = *(const uint4*)(pb + j * LRp);
        const uint32_t pw[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
        for (int r = 0; r < 8; r++) acc[r] = fmaf(cpv_h2f((uint16_t)(pw[r >> 1] >> (16 * (r & 1)))), v, acc[r]);
    }
    const int G = H / Hkv;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int lr = lr0 + r;
        if (lr >= LR) break;
        const int t = lr / G, h = kh * G + lr % G;
        part[((int64_t)c * T * H + (int64_t)t * H + h) * D + d] = acc[r];
    }
}

// out = ((0 + P_0) + P_1) + ... in chunk order
__global__ __launch_bounds__(256) void attn_fold_kernel(const float* __restrict__ part, int nchunk, int64_t total,
                                                        float* __restrict__ out)
{
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= total) return;
    float o = 0.0f;
    for (int c = 0; c < nchunk; c++) o = o + part[(int64_t)c * total + e];
    out[e] = o;
}

// one call over T query tokens (the scratch holds T*H rows)
template <int D>
cpv_status attn_block(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                      int64_t n_past, const int32_t* parent, int T, int H, int Hkv, float scale, float* out)
{
    const int64_t n = n_past + T;
    const int G = H / Hkv, LR = G * T, LRp = (LR + 7) / 8 * 8;
    const int nchunk = (int)((n + CHUNK - 1) / CHUNK);
    const size_t w_b = ((size_t)T * H * n * 4 + 255) & ~(size_t)255;
    const size_t p_b = ((size_t)Hkv * n * LRp * 2 + 255) & ~(size_t)255;
    const size_t part_b = (size_t)nchunk * T * H * D * 4;
    void* ws = nullptr;
    cpv_status st = cpv_workspace(ctx, w_b + p_b + part_b, &ws);
    if (st != CPV_OK) return st;
    float* w = (float*)ws;
    uint16_t* p = (uint16_t*)((uint8_t*)ws + w_b);
    float* part = (float*)((uint8_t*)ws + w_b + p_b);
    ScoreArgs sa;
    sa.q = q;
    sa.kc = kc;
    sa.parent = parent;
    sa.w = w;
    sa.n_past = n_past;
    sa.n = n;
    sa.T = T;
    sa.H = H;
    sa.Hkv = Hkv;
    sa.scale = scale;
    attn_scores_kernel<D><<<dim3((unsigned)nchunk, (unsigned)Hkv, (unsigned)((LR + QB - 1) / QB)), 256, 0,
                            ctx->stream>>>(sa);
    attn_softmax_kernel<<<(unsigned)(T * H), 256, 0, ctx->stream>>>(w, n, T, H, Hkv, LRp, p);
    const int rows_per_block = 8 * (4 / (D / 64));
    attn_pv_kernel<D><<<dim3((unsigned)nchunk, (unsigned)Hkv, (unsigned)((LR + rows_per_block - 1) / rows_per_block)),
                        256, 0, ctx->stream>>>(vt, v_stride, p, n, LR, LRp, T, H, Hkv, part);
    const int64_t total = (int64_t)T * H * D;
    attn_fold_kernel<<<(unsigned)((total + 255) / 256), 256, 0, ctx->stream>>>(part, nchunk, total, out);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

template <int D>
cpv_status attn_run(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                    int64_t n_past, const int32_t* parent, int t, int h, int h_kv, float scale, float* out)
{
    if (parent) return attn_block<D>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out);
    // a long chain runs in token blocks to bound the scratch: node t of a chain sees
    // the rows <= n_past + t, which is what a block starting at t0 sees with n_past + t0
    const int64_t n = n_past + t;
    int64_t tb = ((int64_t)192 << 20) / ((int64_t)h * n * 4 + 1);
    if (tb < 1) tb = 1;
    if (tb > t) tb = t;
    for (int t0 = 0; t0 < t; t0 += (int)tb) {
        const int tn = t - t0 < (int)tb ? t - t0 : (int)tb;
        cpv_status st = attn_block<D>(ctx, q + (int64_t)t0 * h * D, kc, vt, v_stride, n_past + t0, nullptr, tn, h,
                                      h_kv, scale, out + (int64_t)t0 * h * D);
        if (st != CPV_OK) return st;
    }
    return CPV_OK;
}

}  // namespace

cpv_status cpv_attn_launch(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                           int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                           float* out)
{
    auto go = [=]() {
        return d == 128 ? attn_run<128>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out)
                        : attn_run<64>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out);
    };
    const int ev = cpv_prof_mark(ctx);
    const cpv_status st = go();
    if (st == CPV_OK && ev >= 0) {  // algorithmic bytes: K and V rows once, q in, out
        const double bytes = 2.0 * 2.0 * (double)(n_past + t) * h_kv * d + 2.0 * 4.0 * t * h * d;
        cpv_prof_add(ctx, ev, CPV_PROF_ATTN, bytes);
        cpv_prof_keep(ctx, CPV_PROF_ATTN, bytes, [go]() { (void)go(); });
    }
    return st;
}

extern "C" cpv_status cpv_attn(cpv_ctx* ctx, const float* q_dev, const uint16_t* k_cache_dev,
                               const uint16_t* v_cache_t_dev, int64_t v_stride, int64_t n_past,
                               const int32_t* parent_dev, int t, int h, int h_kv, int d, float scale,
                               float* out_dev)
{
    if (!ctx || !q_dev || !k_cache_dev || !v_cache_t_dev || !out_dev)
        return cpv_fail(ctx, CPV_EINVAL, "attn: null argument");
    if (t < 1 || (parent_dev && t > 64) || t > 8192 || h < 1 || h_kv < 1 || h % h_kv || n_past < 0)
        return cpv_fail(ctx, CPV_EINVAL, "attn: bad shape t=%d h=%d h_kv=%d n_past=%lld", t, h, h_kv,
                        (long long)n_past);
    if (d != 64 && d != 128) return cpv_fail(ctx, CPV_EUNSUPPORTED, "attn: head dim %d (64 or 128)", d);
    if (v_stride < n_past + t || (v_stride % 8))
        return cpv_fail(ctx, CPV_EINVAL, "attn: v_stride %lld must be >= n_past + t and a multiple of 8",
                        (long long)v_stride);
    return cpv_attn_launch(ctx, q_dev, k_cache_dev, v_cache_t_dev, v_stride, n_past, parent_dev, t, h, h_kv, d,
                           scale, out_dev);
}
