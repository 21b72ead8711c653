// attn.hip — tree-masked GQA attention over the f16 KV cache (split-KV, MFMA).
//
// Replaces ggml_flash_attn_ext with prec F32 (crates/codpiece-model/src/
// qwen35.rs:3182-3187): out = softmax(scale * q k^T + mask) v, where a query
// node sees every context row and the rows of its ancestors and itself.
//
// Layout.  K is the FA cache layout [n_ctx][h_kv * d] (qwen35.rs:571-575).  V
// is the transposed cache [h_kv * d][v_stride] the reference uses without FA
// (qwen35.rs:580-586): the KV axis is contiguous, which is what the PV product
// needs as its reduction axis.
//
// Mapping.  Grid = (splits of the KV axis, h_kv).  A workgroup stages the
// G*T query rows of its KV head (G = h / h_kv) in LDS as f16 (ggml's CPU FA
// also converts q to f16), and its 4 waves walk 32-row KV tiles round-robin:
//   S  = Q K^T      v_mfma_f32_16x16x32_f16, K fragments straight from HBM
//   online softmax  f32, per query row, rows spread as the MFMA D layout
//   O += P V        v_mfma_f32_16x16x32_f16 twice, with P = P_hi + P_lo in f16
// Each wave keeps its own (m, l, O); the waves merge through LDS, each split
// writes (m, l, O) partials, and a second kernel combines the splits.
#include <math.h>

#include "cpv_internal.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int TILE = 32;           // KV rows per MFMA tile
constexpr int WAVES = 4;
constexpr int MAX_ROWS = 96;       // query rows per workgroup (a row block of one KV head)
constexpr int P_STRIDE = TILE + 8; // halves per P row in LDS (breaks bank aliasing)

__device__ __forceinline__ h8 load_h8(const uint16_t* p)
{
    const uint4 v = *(const uint4*)p;
    return __builtin_bit_cast(h8, v);
}

template <int D, int RT>
__global__ __launch_bounds__(256) void attn_split_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vt,
    int64_t v_stride, int64_t n_past, const int32_t* __restrict__ parent, int T, int H, int Hkv, float scale,
    int64_t chunk, float* __restrict__ part)
{
    constexpr int DC = D / 32;     // MFMA k-steps for q k^T
    constexpr int DT = D / 16;     // output column tiles
    const int G = H / Hkv;
    const int R = G * T;                         // query rows of this KV head
    const int row0 = blockIdx.z * MAX_ROWS;      // this workgroup's first row
    const int Rb = R - row0 < RT * 16 ? R - row0 : RT * 16;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
    const int64_t n_tot = n_past + T;
    const int64_t j_begin = (int64_t)split * chunk;
    const int64_t j_end = j_begin + chunk < n_tot ? j_begin + chunk : n_tot;
    const int ntiles = (int)((j_end - j_begin + TILE - 1) / TILE);

    __shared__ __align__(16) uint16_t s_q[RT * 16 * D];                      // f16 queries
    __shared__ __align__(16) uint16_t s_p[WAVES][2][RT * 16 * P_STRIDE];     // P hi / lo
    __shared__ uint64_t s_anc[64];
    __shared__ float s_ml[WAVES][2][RT * 16];

    // ancestor-or-self bitmask per node of a tree (a chain needs none)
    if (parent && tid < T) {
        uint64_t m = 0;
        int a = tid;
        for (int steps = 0; a >= 0 && a < T && steps <= T; steps++) {
            m |= 1ull << a;
            a = parent ? parent[a] : a - 1;
        }
        s_anc[tid] = m;
    }
    // query rows rho = t * G + gi of head kvh * G + gi, rounded to f16
    for (int i = tid; i < RT * 16 * D; i += blockDim.x) {
        const int rho = i / D, d = i % D;
        float v = 0.0f;
        if (rho < Rb) {
            const int t = (row0 + rho) / G, gi = (row0 + rho) % G;
            v = q[((int64_t)t * H + kvh * G + gi) * D + d];
        }
        s_q[i] = cpv_f2h(v);
    }
    __syncthreads();

    float m_run[RT][4], l_run[RT][4];
    f4 o[RT][DT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) { m_run[rt][i] = -INFINITY; l_run[rt][i] = 0.0f; }
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[rt][dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    const uint16_t* kh = kc + (int64_t)kvh * D;
    const int64_t k_row = (int64_t)Hkv * D;
    const int steps = (ntiles + WAVES - 1) / WAVES;
    for (int step = 0; step < steps; step++) {
        const int tile = step * WAVES + wave;
        const bool active = tile < ntiles;
        const int64_t j0 = j_begin + (int64_t)tile * TILE;
        if (active) {
            // K fragments for both 16-row column tiles: row j0 + 16 ct + l16, d = 32 dc + 8 g4
            h8 kf[2][DC];
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                const int64_t j = j0 + 16 * ct + l16;
#pragma unroll
                for (int dc = 0; dc < DC; dc++) {
                    if (j < j_end) kf[ct][dc] = load_h8(kh + j * k_row + 32 * dc + 8 * g4);
                    else kf[ct][dc] = h8{0, 0, 0, 0, 0, 0, 0, 0};
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                f4 s[2];
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int dc = 0; dc < DC; dc++) {
                        const h8 a = load_h8(s_q + (rt * 16 + l16) * D + 32 * dc + 8 * g4);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, kf[ct][dc], acc, 0, 0, 0);
                    }
                    s[ct] = acc;
                }
                // scale, mask, online softmax for rows rt*16 + 4 g4 + i
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int rho = rt * 16 + 4 * g4 + i;
                    const int node = rho < Rb ? (row0 + rho) / G : 0;
                    float sv[2];
#pragma unroll
                    for (int ct = 0; ct < 2; ct++) {
                        const int64_t j = j0 + 16 * ct + l16;
                        bool vis = j < j_end;
                        if (vis && j >= n_past)
                            vis = parent ? ((s_anc[node] >> (j - n_past)) & 1ull) != 0 : j - n_past <= node;
                        sv[ct] = vis ? s[ct][i] * scale : -INFINITY;
                    }
                    float mx = fmaxf(sv[0], sv[1]);
#pragma unroll
                    for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
                    const float m_new = fmaxf(m_run[rt][i], mx);
                    float p0 = 0.0f, p1 = 0.0f, alpha = 1.0f;
                    if (m_new != -INFINITY) {
                        alpha = expf(m_run[rt][i] - m_new);
                        p0 = expf(sv[0] - m_new);
                        p1 = expf(sv[1] - m_new);
                    }
                    float sum = p0 + p1;
#pragma unroll
                    for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off);
                    l_run[rt][i] = l_run[rt][i] * alpha + sum;
                    m_run[rt][i] = m_new;
#pragma unroll
                    for (int dt = 0; dt < DT; dt++) o[rt][dt][i] *= alpha;
                    // P for the PV product, split exactly into two f16 parts
                    const uint16_t h0 = cpv_f2h(p0), h1 = cpv_f2h(p1);
                    const uint16_t lo0 = cpv_f2h(p0 - cpv_h2f(h0)), lo1 = cpv_f2h(p1 - cpv_h2f(h1));
                    uint16_t* ph = s_p[wave][0] + (rt * 16 + 4 * g4 + i) * P_STRIDE;
                    uint16_t* pl = s_p[wave][1] + (rt * 16 + 4 * g4 + i) * P_STRIDE;
                    ph[l16] = h0;
                    ph[16 + l16] = h1;
                    pl[l16] = lo0;
                    pl[16 + l16] = lo1;
                }
            }
        }
        __syncthreads();
        if (active) {
            // V^T fragments: column d = 16 dt + l16, KV rows j0 + 8 g4 .. + 8
            h8 vf[DT];
            const int64_t jv = j0 + 8 * g4;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const uint16_t* src = vt + ((int64_t)kvh * D + 16 * dt + l16) * v_stride + jv;
                if (jv + 8 <= j_end) {
                    vf[dt] = load_h8(src);
                } else {
                    h8 v = {0, 0, 0, 0, 0, 0, 0, 0};
                    for (int e = 0; e < 8; e++)
                        if (jv + e < j_end) v[e] = __builtin_bit_cast(_Float16, src[e]);
                    vf[dt] = v;
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const h8 ahi = load_h8(s_p[wave][0] + (rt * 16 + l16) * P_STRIDE + 8 * g4);
                const h8 alo = load_h8(s_p[wave][1] + (rt * 16 + l16) * P_STRIDE + 8 * g4);
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, vf[dt], o[rt][dt], 0, 0, 0);
                    o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, vf[dt], o[rt][dt], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    // merge the waves' (m, l, O) through LDS, reusing the P buffers for O
    float* s_o = (float*)&s_p[0][0][0];          // RT*16 x D floats
    static_assert(sizeof(s_p) >= sizeof(float) * RT * 16 * D, "merge buffer");
    for (int w = 0; w < WAVES; w++) {
        if (wave == w) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int row = rt * 16 + 4 * g4 + i;
                    float scale_old = 0.0f, scale_new = 1.0f, m_tot = m_run[rt][i], l_tot = l_run[rt][i];
                    if (w > 0) {
                        const float mo = s_ml[0][0][row], lo = s_ml[0][1][row];
                        m_tot = fmaxf(mo, m_run[rt][i]);
                        scale_old = m_tot == -INFINITY ? 0.0f : expf(mo - m_tot);
                        scale_new = m_tot == -INFINITY ? 0.0f : expf(m_run[rt][i] - m_tot);
                        l_tot = lo * scale_old + l_run[rt][i] * scale_new;
                    }
#pragma unroll
                    for (int dt = 0; dt < DT; dt++) {
                        float* dst = s_o + row * D + 16 * dt + l16;
                        *dst = (w > 0 ? *dst * scale_old : 0.0f) + o[rt][dt][i] * scale_new;
                    }
                    if (l16 == 0) { s_ml[0][0][row] = m_tot; s_ml[0][1][row] = l_tot; }
                }
        }
        __syncthreads();
    }
    // partials: [split][kvh][rho] x (m, l, O[D])
    const int nsplit = gridDim.x;
    for (int i = tid; i < Rb * (D + 2); i += blockDim.x) {
        const int rho = i / (D + 2), c = i % (D + 2);
        const float v = c == 0 ? s_ml[0][0][rho] : c == 1 ? s_ml[0][1][rho] : s_o[rho * D + c - 2];
        part[(((int64_t)kvh * nsplit + split) * R + row0 + rho) * (D + 2) + c] = v;
    }
}

// combine the splits of one query row: out = sum_s e^{m_s-M} O_s / sum_s e^{m_s-M} l_s
__global__ void attn_combine_kernel(const float* __restrict__ part, int nsplit, int T, int H, int Hkv, int D,
                                    float* __restrict__ out)
{
    const int G = H / Hkv, R = G * T;
    const int rho = blockIdx.x % R, kvh = blockIdx.x / R;
    const float* base = part + ((int64_t)kvh * nsplit * R + rho) * (D + 2);
    const int64_t sstride = (int64_t)R * (D + 2);
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, base[s * sstride]);
    const int t = rho / G, gi = rho % G;
    float* o = out + ((int64_t)t * H + kvh * G + gi) * D;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float num = 0.0f, den = 0.0f;
        for (int s = 0; s < nsplit; s++) {
            const float* p = base + s * sstride;
            const float w = p[0] == -INFINITY ? 0.0f : expf(p[0] - M);
            num += w * p[2 + d];
            den += w * p[1];
        }
        o[d] = num / den;
    }
}

template <int D, int RT>
cpv_status launch(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                  int64_t n_past, const int32_t* parent, int T, int H, int Hkv, float scale, float* out)
{
    const int G = H / Hkv, R = G * T;
    const int64_t n_tot = n_past + T;
    // enough splits for ~4 workgroups per CU, chunks a whole number of wave-steps
    int64_t want = (int64_t)ctx->cu_count * 4 / Hkv;
    if (want < 1) want = 1;
    int64_t chunk = (n_tot + want - 1) / want;
    const int64_t step_rows = (int64_t)TILE * WAVES;
    chunk = (chunk + step_rows - 1) / step_rows * step_rows;
    const int nsplit = (int)((n_tot + chunk - 1) / chunk);
    void* ws = nullptr;
    cpv_status st = cpv_workspace(ctx, (size_t)Hkv * nsplit * R * (D + 2) * sizeof(float), &ws);
    if (st != CPV_OK) return st;
    dim3 grid((unsigned)nsplit, (unsigned)Hkv, (unsigned)((R + MAX_ROWS - 1) / MAX_ROWS));
    attn_split_kernel<D, RT><<<grid, 256, 0, ctx->stream>>>(q, kc, vt, v_stride, n_past, parent, T, H, Hkv,
                                                            scale, chunk, (float*)ws);
    CPV_HIP(ctx, hipGetLastError());
    attn_combine_kernel<<<(unsigned)(Hkv * R), D, 0, ctx->stream>>>((const float*)ws, nsplit, T, H, Hkv, D, out);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

template <int D>
cpv_status launch_rt(cpv_ctx* ctx, int rt, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t vs,
                     int64_t n_past, const int32_t* parent, int T, int H, int Hkv, float scale, float* out)
{
    switch (rt) {
    case 1: return launch<D, 1>(ctx, q, kc, vt, vs, n_past, parent, T, H, Hkv, scale, out);
    case 2: return launch<D, 2>(ctx, q, kc, vt, vs, n_past, parent, T, H, Hkv, scale, out);
    case 3: return launch<D, 3>(ctx, q, kc, vt, vs, n_past, parent, T, H, Hkv, scale, out);
    case 4: return launch<D, 4>(ctx, q, kc, vt, vs, n_past, parent, T, H, Hkv, scale, out);
    case 5: return launch<D, 5>(ctx, q, kc, vt, vs, n_past, parent, T, H, Hkv, scale, out);
    default: return launch<D, 6>(ctx, q, kc, vt, vs, n_past, parent, T, H, Hkv, scale, out);
    }
}

}  // namespace

cpv_status cpv_attn_launch(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                           int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                           float* out)
{
    const int R = (h / h_kv) * t;
    const int rt = ((R < MAX_ROWS ? R : MAX_ROWS) + 15) / 16;
    auto go = [=]() {
        return d == 128 ? launch_rt<128>(ctx, rt, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out)
                        : launch_rt<64>(ctx, rt, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out);
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
