// model.hip — the qwen35-layout verify round on the device.
//
// cpv_verify_step is Qwen35::step_fused_cached (crates/codpiece-model/src/
// qwen35.rs:1693-1948) for an all-attention qwen35 model: the trunk
// (build_inner, :2445-2786, with build_attn_block :3000-3198), the LM head and
// in-graph argmax (:2788-2821) and the fused MTP draft chain (:2840-2962).
// Every op follows the ggml CPU semantics the oracle restates:
//   rms_norm   exact sum of f32 squares, mean = (float)(sum/n),
//              scale = 1/sqrtf(mean + eps), y = (x*scale)*w
//   rope       NEOX pairs from a cos/sin table built on the host with ggml's
//              f32 theta recurrence (qwen35.rs:3053-3062 with text positions)
//   sigmoid    1/(1+expf(-x)); silu x/(1+expf(-x)); add / mul in f32
//   mul_mat    the exact-window GEMM of qgemm.hip
//   attention  attn.hip (the exact chunked contract the oracle restates:
//              fixed-point scores, exact normalisers, fixed-order sums)
// The K cache is [n_ctx][h_kv*d] and V is kept transposed [h_kv*d][n_ctx]
// (the reference's non-FA V layout), one pair per layer plus the MTP pair.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <map>
#include <string>
#include <type_traits>
#include <vector>

#include "cpv_internal.h"

namespace {

// ---------------------------------------------------------------- glue kernels
__device__ __forceinline__ int ceil_log2_dev(int64_t v)
{
    int b = 0;
    while (((int64_t)1 << b) < v) b++;
    return b;
}

// y = rms_norm(x) * w over rows of n; exact fixed-point sum of the f32 squares
// (order-free), then ggml's f32 tail.  One block of 1024 threads per row; the
// row is read once into registers (n <= RMS_PER * 1024), else re-read.
constexpr int RMS_PER = 24;

__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ x, int64_t xs,
                                                       const float* __restrict__ w, float* __restrict__ y,
                                                       int64_t ys, int n, float eps)
{
    const float* xr = x + (int64_t)blockIdx.x * xs;
    float* yr = y + (int64_t)blockIdx.x * ys;
    __shared__ float s_max[16];
    __shared__ long long s_sum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = (blockDim.x + 63) >> 6;
    const bool cached = n <= RMS_PER * (int)blockDim.x;
    float v[RMS_PER];
    float am = 0.0f;
    if (cached) {
#pragma unroll
        for (int j = 0; j < RMS_PER; j++) {
            const int i = tid + j * blockDim.x;
            const float xi = xr[i < n ? i : n - 1];          // every lane loads: no wait per element
            v[j] = i < n ? xi : 0.0f;
            am = fmaxf(am, fabsf(v[j]));
        }
    } else {
        for (int i = tid; i < n; i += blockDim.x) am = fmaxf(am, fabsf(xr[i]));
    }
    am = cpv_wave_reduce(am, cpv_op_max());
    if (lane == 0) s_max[wave] = am;
    __syncthreads();
    am = s_max[0];
    for (int i = 1; i < nw; i++) am = fmaxf(am, s_max[i]);
    double sum = 0.0;
    if (am > 0.0f) {
        int e;
        frexpf(am, &e);
        const int g = 2 * e - (62 - ceil_log2_dev(n + 1));
        long long S = 0;
        if (cached) {
#pragma unroll
            for (int j = 0; j < RMS_PER; j++) S += cpv_fixed_floor(v[j] * v[j], g);
        } else {
            for (int i = tid; i < n; i += blockDim.x) {
                const float sq = xr[i] * xr[i];
                S += cpv_fixed_floor(sq, g);
            }
        }
        S = cpv_wave_reduce(S, cpv_op_add());
        if (lane == 0) s_sum[wave] = S;
        __syncthreads();
        S = 0;
        for (int i = 0; i < nw; i++) S += s_sum[i];
        sum = ldexp((double)S, g);
    }
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (cached) {
#pragma unroll
        for (int j = 0; j < RMS_PER; j++) {
            const int i = tid + j * blockDim.x;
            if (i < n) {
                const float t = v[j] * scale;
                yr[i] = w ? t * w[i] : t;
            }
        }
    } else {
        for (int i = tid; i < n; i += blockDim.x) {
            const float t = xr[i] * scale;
            yr[i] = w ? t * w[i] : t;
        }
    }
}

// Per token t and head: q/k RMS norm over the head, NEOX rope at position
// rope_pos0 + t, then q to qout, and k and v (each rounded to f16) as limbs to
// row kv_row0 + t of the session's K and V caches.  Grid (T, H + Hkv), block hd.
struct PrepArgs {
    const float* qg;       // [T] rows of qs floats: [H][2*hd] query | output gate per head
    const float* kk;       // [T] rows of ks floats: [Hkv*hd]
    const float* vv;       // [T] rows of ks floats: [Hkv*hd]
    int64_t qs, ks;        // row strides (a fused q|k|v output shares one)
    const float* q_norm;   // [hd]
    const float* k_norm;   // [hd]
    const float* rope;     // [n_pos][n_rot/2][2]
    float* qout;           // [T][H][hd]
    int8_t* k_limbs;       // the K cache's limbs: rows of cpv_k_row_bytes(Hkv, hd), then the exponent plane
    int8_t* v_limbs;       // the V cache's limbs [Hkv*hd][v_stride / 16][CPV_ATTN_VLIMBS][16]
    int64_t v_stride;
    int64_t rope_pos0, kv_row0;
    const int32_t* pos_off;   // [T] position of token t = rope_pos0 + pos_off[t] (a tree's depths), or null: + t
    int H, Hkv, hd, n_rot, write;
    float eps;
    const int64_t* pos;       // when set (device memory, read at run time): rope_pos0 = pos[0] + rope_off,
    int pos_kv, rope_off;     // kv_row0 = pos[pos_kv]
};

__device__ __forceinline__ int64_t prep_rope0(const PrepArgs& a) { return a.pos ? a.pos[0] + a.rope_off : a.rope_pos0; }
__device__ __forceinline__ int64_t prep_kv0(const PrepArgs& a) { return a.pos ? a.pos[a.pos_kv] : a.kv_row0; }

// value vv of cache row `row`, column kh*hd + i, into the V cache: rounded to
// f16 (the cache's precision), then vq = rint(v 2^CPV_ATTN_VBITS) as signed
// 8-bit limbs, one per plane
__device__ __forceinline__ int8_t* v_limb_at(int8_t* v, int64_t col, int64_t v_stride, int64_t row)
{
    return v + (col * v_stride + (row & ~(int64_t)15)) * CPV_ATTN_VLIMBS + (row & 15);   // limb l at + 16 l
}

__device__ __forceinline__ void write_v_limbs(const PrepArgs& a, int kh, int i, int64_t row, float vv)
{
    int x = (int)rintf(ldexpf(cpv_h2f(cpv_f2h(vv)), CPV_ATTN_VBITS));
    int8_t* dst = v_limb_at(a.v_limbs, (int64_t)kh * a.hd + i, a.v_stride, row);
#pragma unroll
    for (int l = 0; l < CPV_ATTN_VLIMBS - 1; l++) {
        const int li = ((x + 128) & 255) - 128;
        dst[16 * l] = (int8_t)li;
        x = (x - li) >> 8;
    }
    dst[16 * (CPV_ATTN_VLIMBS - 1)] = (int8_t)x;
}

// key kk (element i of KV head kh, one thread each: the whole block) of cache
// row `row` into the K cache: rounded to f16, then the head's exponent and
// each element's two limbs (cpv_k_limbs)
__device__ __forceinline__ void write_k_limbs(const PrepArgs& a, int kh, int i, int64_t row, float kk, float* s_km)
{
    const float kf = cpv_h2f(cpv_f2h(kk));
    float km = cpv_wave_reduce(fabsf(kf), cpv_op_max());
    if ((i & 63) == 0) s_km[i >> 6] = km;
    __syncthreads();
    km = s_km[0];
    if (a.hd > 64) km = fmaxf(km, s_km[1]);
    const int e = cpv_exp_of_max(km);
    int8_t hi, lo;
    cpv_k_limbs(kf, e, &hi, &lo);
    const int64_t krow = cpv_k_row_bytes(a.Hkv, a.hd);
    int8_t* kr = a.k_limbs + row * krow;
    kr[(int64_t)kh * 2 * a.hd + i] = hi;
    kr[(int64_t)kh * 2 * a.hd + a.hd + i] = lo;
    if (i == 0) cpv_k_exps((int32_t*)a.k_limbs, a.Hkv, a.hd, a.v_stride)[(int64_t)kh * a.v_stride + row] = e;
}

__global__ __launch_bounds__(128) void qk_prep_kernel(PrepArgs a)
{
    const int64_t rope0 = prep_rope0(a), kv0 = prep_kv0(a);   // (read first: off the critical path)
    const int t = blockIdx.x, hh = blockIdx.y, i = threadIdx.x;
    const bool is_q = hh < a.H;
    const int kh = hh - a.H;
    const float* src = is_q ? a.qg + (int64_t)t * a.qs + (int64_t)hh * 2 * a.hd : a.kk + (int64_t)t * a.ks + (int64_t)kh * a.hd;
    const float* w = is_q ? a.q_norm : a.k_norm;
    __shared__ float s_v[128];
    __shared__ float s_am[2], s_km[2];
    __shared__ long long s_s[2];
    const float x = src[i];
    // rms over the head (n = hd <= 128: two waves at most)
    float am = fabsf(x);
    am = cpv_wave_reduce(am, cpv_op_max());
    if ((i & 63) == 0) s_am[i >> 6] = am;
    __syncthreads();
    am = s_am[0];
    if (a.hd > 64) am = fmaxf(am, s_am[1]);
    double sum = 0.0;
    if (am > 0.0f) {
        int e;
        frexpf(am, &e);
        const int g = 2 * e - (62 - ceil_log2_dev(a.hd + 1));
        long long S = cpv_fixed_floor(x * x, g);
        S = cpv_wave_reduce(S, cpv_op_add());
        if ((i & 63) == 0) s_s[i >> 6] = S;
        __syncthreads();
        S = s_s[0] + (a.hd > 64 ? s_s[1] : 0);
        sum = ldexp((double)S, g);
    }
    const float mean = (float)(sum / (double)a.hd);
    const float scale = 1.0f / sqrtf(mean + a.eps);
    const float v0 = x * scale;
    const float xn = w ? v0 * w[i] : v0;
    s_v[i] = xn;
    __syncthreads();
    float out = xn;
    const int half = a.n_rot / 2;
    if (i < a.n_rot) {
        const int p = i < half ? i : i - half;
        const float* cs = a.rope + (rope0 + (a.pos_off ? a.pos_off[t] : t)) * a.n_rot + 2 * p;
        const float c = cs[0], s = cs[1];
        const float x0 = s_v[p], x1 = s_v[p + half];
        if (i < half) {
            const float m0 = x0 * c, m1 = x1 * s;
            out = m0 - m1;
        } else {
            const float m0 = x0 * s, m1 = x1 * c;
            out = m0 + m1;
        }
    }
    if (is_q) {
        a.qout[((int64_t)t * a.H + hh) * a.hd + i] = out;
    } else if (a.write) {   // (block-uniform)
        const int64_t row = kv0 + t;
        const float vv = a.vv[(int64_t)t * a.ks + (int64_t)kh * a.hd + i];
        write_k_limbs(a, kh, i, row, out, s_km);
        write_v_limbs(a, kh, i, row, vv);
    }
}

// out[t][h*hd + i] = attn[t][h*hd + i] * sigmoid(gate), gate = qg[t*qs + h*2hd + hd + i]
__global__ void gate_mul_kernel(const float* __restrict__ attn, const float* __restrict__ qg, int64_t qs, int H,
                                int hd, int64_t total, float* __restrict__ out)
{
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = e / ((int64_t)H * hd);
        const int64_t r = e % ((int64_t)H * hd);
        const int64_t h = r / hd, i = r % hd;
        const float g = qg[t * qs + h * 2 * hd + hd + i];
        const float sig = 1.0f / (1.0f + cpv_expf(-g));
        out[e] = attn[e] * sig;
    }
}

__global__ void add_kernel(const float* a, const float* b, float* y, int64_t n)   // y may alias b
{
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x)
        y[e] = a[e] + b[e];
}

// act[t][i] = silu(g[t*gs + i]) * u[t*gs + i], silu(x) = x / (1 + expf(-x)); F per row
__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, int64_t gs, int64_t F,
                              float* __restrict__ y, int64_t n)
{
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = e / F, i = e % F;
        const float x = g[t * gs + i];
        const float s = x / (1.0f + cpv_expf(-x));
        y[e] = s * u[t * gs + i];
    }
}

// ---------------------------------------------------------------- fused row kernels
// One 1024-thread block per activation row.  Wave w holds the row's 256-element
// units u = w, w + 16, ...; lane l holds elements u*256 + 4l .. 4l + 3 of each,
// so every load and store is 16 (or 4) bytes wide and every per-unit step of
// the quantization is a wave reduction with no barrier.  A row kernel
// produces the row (from the residual and a GEMM result kept in the
// accumulator, or from the attention output and its gate, or from the
// gate|up GEMM through SwiGLU), optionally RMS-normalizes it, and optionally
// quantizes it for the next GEMM, with the same arithmetic as the separate
// kernels it replaces (add_kernel, rmsnorm_kernel, gate_mul_kernel,
// swiglu_kernel, quant_q8k_kernel / quant_q80_kernel).  Row lengths are
// multiples of 4.
constexpr int RB = 1024;     // most threads per row block
constexpr int RW = RB / 64;  // most waves
constexpr int RUU = 3;       // most units per wave: rows up to 3 * 16 * 256 = 12288 elements
constexpr int RQ = RUU * 4;  // most register slots per thread

enum { SRC_X = 0, SRC_ADD = 1, SRC_SET = 2, SRC_GATE = 3, SRC_SWIGLU = 4, SRC_GATE_FOLD = 5, SRC_CAT = 6 };
constexpr int FOLD_MAX = 512;   // attention chunks a SRC_GATE_FOLD row kernel folds (contexts to 64k)

struct RowArgs {
    int src;
    float* x;              // residual rows [T][xs] (SRC_X / _ADD / _SET read and write it)
    int64_t xs;
    cpv_gout g;            // kept GEMM result (SRC_ADD / _SET / _SWIGLU)
    const float* att;      // SRC_GATE: attention output [T][n] and gate [T][n]
    const float* gate;
    cpv_attn_part part;    // SRC_GATE_FOLD: the attention's chunk partials (rows = T * n / hd)
    int hd;                // SRC_GATE_FOLD: head dim
    int n;                 // row length
    const float* w;        // RMS norm weight, when norm
    int norm;
    float eps;
    float* y;              // optional f32 copy of the produced (normalized) row, stride ys
    int64_t ys;
    int quant;             // quantize the row into act (0: no)
    cpv_act act;
    // SRC_CAT: the row is [x row | x2 row], nseg elements each, each half
    // RMS-normalized on its own (weights w and w2), as two rmsnorm_kernel rows
    const float* x2;
    int64_t xs2;
    const float* w2;
    int nseg;
    // SRC_CAT with psum set: the block also stores conf_out[m], the softmax
    // peak of the previous draft link from its slice sums [T][CPV_AM_NB]
    const double* psum;
    float* conf_out;
};

// each block-wide reduction has its own LDS slots, so one barrier suffices
struct RowLds {
    float red_am[RW], red_am2[RW];
    long long red_s[RW], red_s2[RW];
};

// (the RW slots are read at once, those past the block's nw waves masked:
// a loop to nw would wait on each read in turn)
__device__ float row_max(float v, float* slot, int nw)
{
    const int tid = threadIdx.x;
    v = cpv_wave_reduce(v, cpv_op_max());
    if ((tid & 63) == 0) slot[tid >> 6] = v;
    __syncthreads();
    float sv[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) sv[i] = slot[i];
    float r = sv[0];
#pragma unroll
    for (int i = 1; i < RW; i++) r = i < nw ? fmaxf(r, sv[i]) : r;
    return r;
}

__device__ long long row_sum(long long v, long long* slot, int nw)
{
    const int tid = threadIdx.x;
    v = cpv_wave_reduce(v, cpv_op_add());
    if ((tid & 63) == 0) slot[tid >> 6] = v;
    __syncthreads();
    long long sv[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) sv[i] = slot[i];
    long long r = 0;
#pragma unroll
    for (int i = 0; i < RW; i++) r += i < nw ? sv[i] : 0;
    return r;
}

// NU units of 256 elements per wave, as many waves as the row's units need
// (each load slot past the row still costs the CU's load path a cycle per
// byte: with one block per row, that path bounds the kernel)
template <int SRC, int NU>
__global__ __launch_bounds__(RB) void row_kernel(RowArgs a)
{
    constexpr int RUU = NU, RQ = 4 * NU;
    __shared__ RowLds L;
    const int m = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
    const int n = a.n, U = (n + 255) / 256;
    constexpr bool kept = SRC == SRC_ADD || SRC == SRC_SET;
    float* xr = a.x + (int64_t)m * a.xs;
    // this lane's four elements of each of its units (clamped to element 0 when out of range)
    int e0[RUU];
    bool ok[RUU];
#pragma unroll
    for (int uu = 0; uu < RUU; uu++) {
        const int u = wave + nw * uu, e = u * 256 + 4 * lane;
        ok[uu] = u < U && e < n;
        e0[uu] = ok[uu] ? e : 0;
    }
    // ---- every input goes out first, unconditionally (a branch would make
    // the compiler wait for all of them at the join): x, the norm weight, a
    // kept result's sums and row exponents, and the scales that give Ea
    float v[RQ], wv[RQ];
    const float* wsrc = a.w ? a.w : xr;
    // SRC_CAT: a unit lies in one half (nseg is a multiple of 256)
    auto in_hi = [&](int uu) { return SRC == SRC_CAT && e0[uu] >= a.nseg; };
    // the previous link's slice sums, one per lane of the last wave
    const bool peak = SRC == SRC_CAT && a.psum != nullptr && wave == nw - 1;
    const double pv = peak ? a.psum[(int64_t)m * CPV_AM_NB + lane] : 0.0;
#pragma unroll
    for (int uu = 0; uu < RUU; uu++) {
        const float* xp = in_hi(uu) ? a.x2 + (int64_t)m * a.xs2 + (e0[uu] - a.nseg) : xr + e0[uu];
        const float* wp = in_hi(uu) ? a.w2 + (e0[uu] - a.nseg) : wsrc + e0[uu];
        const float4 xv = *(const float4*)xp;
        const float4 ww = *(const float4*)wp;
        const bool use_x = SRC == SRC_X || SRC == SRC_ADD || SRC == SRC_CAT;
        v[uu * 4 + 0] = use_x ? xv.x : 0.0f;
        v[uu * 4 + 1] = use_x ? xv.y : 0.0f;
        v[uu * 4 + 2] = use_x ? xv.z : 0.0f;
        v[uu * 4 + 3] = use_x ? xv.w : 0.0f;
        wv[uu * 4 + 0] = ww.x;
        wv[uu * 4 + 1] = ww.y;
        wv[uu * 4 + 2] = ww.z;
        wv[uu * 4 + 3] = ww.w;
    }
    if (kept) {
        // its sums and row exponents are loaded before anything is stored (the
        // stores further down could alias them), then Ea, then y = the
        // finalized sums, folded into x
        double* acc = a.g.acc + (int64_t)m * a.g.n_pad;
        double S[RQ];
        int ew[RQ];
#pragma unroll
        for (int uu = 0; uu < RUU; uu++) {
            const double2 s0 = *(const double2*)(acc + e0[uu]);
            const double2 s1 = *(const double2*)(acc + e0[uu] + 2);
            const int4 ev = *(const int4*)(a.g.ew + e0[uu]);
            S[uu * 4 + 0] = s0.x;
            S[uu * 4 + 1] = s0.y;
            S[uu * 4 + 2] = s1.x;
            S[uu * 4 + 3] = s1.y;
            ew[uu * 4 + 0] = ev.x;
            ew[uu * 4 + 1] = ev.y;
            ew[uu * 4 + 2] = ev.z;
            ew[uu * 4 + 3] = ev.w;
        }
        // Ea: every wave reduces the row's few scales itself (no block barrier)
        const float* dar = a.g.da + (int64_t)m * a.g.nda;
        float mx = fabsf(dar[lane < a.g.nda ? lane : 0]);
        if (lane >= a.g.nda) mx = 0.0f;
        for (int i = lane + 64; i < a.g.nda; i += 64) mx = fmaxf(mx, fabsf(dar[i]));
        const int ea = cpv_exp_of_max(cpv_wave_reduce(mx, cpv_op_max()));
#pragma unroll
        for (int j = 0; j < RQ; j++) {
            const float gv = cpv_gout_value(S[j], ew[j], ea, a.g.win);
            v[j] = SRC == SRC_ADD ? gv + v[j] : gv;
        }
    }
#pragma unroll
    for (int uu = 0; uu < RUU; uu++)
        if (!ok[uu])
#pragma unroll
            for (int k = 0; k < 4; k++) v[uu * 4 + k] = 0.0f;
    // the new x and the cleared accumulator entries are stored after the
    // norm's block reductions: a barrier waits for the stores issued before it
    auto store_kept = [&]() {
        if (!kept) return;
        double* acc = a.g.acc + (int64_t)m * a.g.n_pad;
#pragma unroll
        for (int uu = 0; uu < RUU; uu++)
            if (ok[uu]) {
                *(float4*)(xr + e0[uu]) = make_float4(v[uu * 4], v[uu * 4 + 1], v[uu * 4 + 2], v[uu * 4 + 3]);
                *(double2*)(acc + e0[uu]) = make_double2(0.0, 0.0);
                *(double2*)(acc + e0[uu] + 2) = make_double2(0.0, 0.0);
            }
    };
    if (!a.norm) store_kept();
    if (a.norm) {
        // exact fixed-point sum of the f32 squares, then ggml's f32 tail, over
        // the row (or over each half of a SRC_CAT row: hi selects the half)
        auto norm_scale = [&](bool hi, int len, float* red_am, long long* red_s) {
            float am = 0.0f;
#pragma unroll
            for (int uu = 0; uu < RUU; uu++)
                if (in_hi(uu) == hi)
#pragma unroll
                    for (int k = 0; k < 4; k++) am = fmaxf(am, fabsf(v[uu * 4 + k]));
            am = row_max(am, red_am, nw);
            double sum = 0.0;
            if (am > 0.0f) {
                int e;
                frexpf(am, &e);
                const int g2 = 2 * e - (62 - ceil_log2_dev(len + 1));
                long long S = 0;
#pragma unroll
                for (int uu = 0; uu < RUU; uu++)
                    if (in_hi(uu) == hi)
#pragma unroll
                        for (int k = 0; k < 4; k++) S += cpv_fixed_floor(v[uu * 4 + k] * v[uu * 4 + k], g2);
                sum = ldexp((double)row_sum(S, red_s, nw), g2);
            }
            const float mean = (float)(sum / (double)len);
            return 1.0f / sqrtf(mean + a.eps);
        };
        const float scale = norm_scale(false, SRC == SRC_CAT ? a.nseg : n, L.red_am, L.red_s);
        const float scale2 = SRC == SRC_CAT ? norm_scale(true, n - a.nseg, L.red_am2, L.red_s2) : scale;
        store_kept();
#pragma unroll
        for (int uu = 0; uu < RUU; uu++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int j = uu * 4 + k;
                const float tv = v[j] * (in_hi(uu) ? scale2 : scale);
                v[j] = ok[uu] ? (a.w ? tv * wv[j] : tv) : 0.0f;   // padding stays 0
            }
    }
    if (a.y) {
#pragma unroll
        for (int uu = 0; uu < RUU; uu++)
            if (ok[uu])
                *(float4*)(a.y + (int64_t)m * a.ys + e0[uu]) =
                    make_float4(v[uu * 4], v[uu * 4 + 1], v[uu * 4 + 2], v[uu * 4 + 3]);
    }
    if (peak) {
        // peak_fin_kernel's sum, in slice order
        double tot = 0.0;
        for (int b = 0; b < CPV_AM_NB; b++) tot += __shfl(pv, b);
        if (lane == 0) a.conf_out[m] = 1.0f * (float)(1.0 / tot);
    }
    if (!a.quant) return;
    const int64_t Kp = (int64_t)U * 256;
    int8_t* qa = const_cast<int8_t*>(a.act.qa);           // cpv_act is the GEMM's read-only view
    float* da = const_cast<float*>(a.act.da);
    int32_t* bs16 = const_cast<int32_t*>(a.act.bs16);
    int32_t* bs32 = const_cast<int32_t*>(a.act.bs32);
#pragma unroll
    for (int uu = 0; uu < RUU; uu++) {
        const int u = wave + nw * uu;
        if (u >= U) break;                                  // wave-uniform
        const float* x = v + uu * 4;
        uint32_t* qw = (uint32_t*)(qa + (int64_t)m * Kp + (int64_t)u * 256) + lane;
        int q[4];
        if (a.act.kq) {
            // Q8_K: the signed element of largest magnitude (first occurrence),
            // iscale = -127/max, q = min(127, rint(iscale * x)), d = 1/iscale, code sums
            float ax = fabsf(x[0]), sx = x[0];
            int ix = 4 * lane;
#pragma unroll
            for (int k = 1; k < 4; k++)
                if (fabsf(x[k]) > ax) { ax = fabsf(x[k]); ix = 4 * lane + k; sx = x[k]; }
            cpv_wave_amax(ax, ix, sx);
            float d = 0.0f;
            if (ax > 0.0f) {
                const float iscale = -127.0f / sx;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int vq = (int)rintf(iscale * x[k]);
                    q[k] = vq < 127 ? vq : 127;
                }
                d = 1.0f / iscale;
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) q[k] = 0;
            }
            *qw = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
                  ((uint32_t)(q[3] & 0xff) << 24);
            // code sums of 16 (4 lanes) and 32 (8 lanes) elements
            const int s16 = cpv_group_reduce<4>(q[0] + q[1] + q[2] + q[3], cpv_op_add());
            const int s32 = s16 + cpv_dpp<CPV_DPP_HMIRROR>(s16);
            if ((lane & 3) == 0) bs16[((int64_t)m * U + u) * 16 + (lane >> 2)] = s16;
            if ((lane & 7) == 0) bs32[((int64_t)m * U + u) * 8 + (lane >> 3)] = s32;
            if (lane == 0) da[(int64_t)m * U + u] = d;
        } else {
            // Q8_0 per 32-element block (8 lanes): d = amax/127, q = roundf(x * (1/d)), d kept as fp16
            float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
            amax = cpv_group_reduce<8>(amax, cpv_op_max());
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) q[k] = (int)roundf(x[k] * id);
            *qw = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
                  ((uint32_t)(q[3] & 0xff) << 24);
            if ((lane & 7) == 0) da[((int64_t)m * U + u) * 8 + (lane >> 3)] = cpv_h2f(cpv_f2h(d));
        }
    }
}

// The same for rows that need no row-wide reduction: the gated attention
// output (SRC_GATE) and SwiGLU of a kept gate|up result (SRC_SWIGLU), each
// quantized for the next GEMM.  One 256-thread block per (unit, row).
template <int SRC>
__global__ __launch_bounds__(256) void unit_kernel(RowArgs a)
{
    __shared__ float s_ax[4], s_sx[4];
    __shared__ int s_ix[4];
    const int u = blockIdx.x, m = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = a.n, U = (n + 255) / 256;
    const int e = u * 256 + t, ec = e < n ? e : n - 1;
    float val = 0.0f;
    if (SRC == SRC_GATE_FOLD) {
        // the attention output of this element's head (the fold of
        // attn_fold_kernel: chunks in order, factors expf(m_c - M), the
        // binary64 sum of the Z_c, one fma chain per element), times
        // sigmoid(gate).  A unit holds 256 / hd heads; hd threads per head.
        __shared__ float s_f[4][FOLD_MAX];
        __shared__ double s_z[4][FOLD_MAX];
        __shared__ float s_m[4][2], s_inv[4];
        const int hd = a.hd, rows = a.part.rows, H = n / hd;
        const int nchg = a.part.nchunk;                       // the grid's chunks: an upper bound
        const int lh = t / hd, tl = t - lh * hd;             // head within the unit, thread within the head
        const int h = ec / hd, rr = m * H + h;                // (clamped: a thread past n reads a valid head)
        const int wph = hd / 64;                              // waves per head
        // every grid chunk's max and sum are read (this thread's first ones
        // first) while the count of chunks in play comes from device memory;
        // those past it are never used.  The element's partials of the first
        // FB grid chunks go out next, into registers, so that the fma chain
        // waits on no load for them (loads complete in order: the first max
        // and sum do not wait for them)
        constexpr int FB = 48;
        const int c0 = tl < nchg ? tl : 0;
        const float gv = a.gate[(int64_t)m * n + ec];           // (the gate goes out first too)
        const float mc0 = a.part.mc[(int64_t)c0 * rows + rr];
        const int64_t zc0 = a.part.zc[(int64_t)c0 * rows + rr];
        const int nch = a.part.pos ? (int)((a.part.pos[a.part.pos_sel] + a.part.t + 127) / 128) : nchg;
        // (the compiler would otherwise issue the partials' loads first, and
        // the first max and the chunk count would wait for all of them)
        asm volatile("" ::: "memory");
        const float* pr = a.part.P + (int64_t)rr * hd + (ec - h * hd);
        const int64_t pcs = (int64_t)rows * hd;
        float pv[FB];
#pragma unroll
        for (int i = 0; i < FB; i++) pv[i] = pr[(int64_t)(i < nchg ? i : nchg - 1) * pcs];
        float M = -INFINITY;
        if (tl < nchg) {
            s_f[lh][tl] = mc0;
            s_z[lh][tl] = ldexp((double)zc0, -a.part.zbits);
        }
        for (int c = tl + hd; c < nchg; c += hd) {
            s_f[lh][c] = a.part.mc[(int64_t)c * rows + rr];
            s_z[lh][c] = ldexp((double)a.part.zc[(int64_t)c * rows + rr], -a.part.zbits);
        }
        for (int c = tl; c < nch; c += hd) M = fmaxf(M, s_f[lh][c]);
        M = cpv_wave_reduce(M, cpv_op_max());
        if (lane == 0) s_m[lh][wave - lh * wph] = M;
        __syncthreads();
        M = s_m[lh][0];
        for (int i = 1; i < wph; i++) M = fmaxf(M, s_m[lh][i]);
        for (int c = tl; c < nch; c += hd) {
            const float mc = s_f[lh][c];
            s_f[lh][c] = mc == -INFINITY ? 0.0f : cpv_expf(mc - M);
        }
        __syncthreads();
        if (tl == 0) {
            double Zt = 0.0;
            for (int c = 0; c < nch; c++) Zt = Zt + s_z[lh][c] * (double)s_f[lh][c];
            s_inv[lh] = (float)(1.0 / Zt);
        }
        // the element's fma chain over the chunks, in chunk order
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < FB; i++)
            if (i < nch) o = fmaf(pv[i], s_f[lh][i], o);
        if (nch > FB) o = cpv_fold_chain_from(pr, pcs, s_f[lh], nch, FB, o);
        __syncthreads();
        const float at = o * s_inv[lh];
        const float sig = 1.0f / (1.0f + cpv_expf(-gv));
        val = e < n ? at * sig : 0.0f;
    } else if (SRC == SRC_GATE) {
        const float gv = a.gate[(int64_t)m * n + ec], at = a.att[(int64_t)m * n + ec];
        const float sig = 1.0f / (1.0f + cpv_expf(-gv));
        val = e < n ? at * sig : 0.0f;
    } else {
        double* acc = a.g.acc + (int64_t)m * a.g.n_pad;
        const double S0 = acc[ec], S1 = acc[n + ec];
        const int e0 = a.g.ew[ec], e1 = a.g.ew[n + ec];
        // Ea: every wave reduces the row's few scales itself (no block barrier)
        float mx = 0.0f;
        for (int i = lane; i < a.g.nda; i += 64) mx = fmaxf(mx, fabsf(a.g.da[(int64_t)m * a.g.nda + i]));
        const int ea = cpv_exp_of_max(cpv_wave_reduce(mx, cpv_op_max()));
        if (e < n) {
            const float gv = cpv_gout_value(S0, e0, ea, a.g.win), uv = cpv_gout_value(S1, e1, ea, a.g.win);
            acc[e] = 0.0;
            acc[n + e] = 0.0;
            const float sl = gv / (1.0f + cpv_expf(-gv));
            val = sl * uv;
        }
    }
    if (!a.quant) return;
    int8_t* qa = const_cast<int8_t*>(a.act.qa);           // cpv_act is the GEMM's read-only view
    float* da = const_cast<float*>(a.act.da);
    const int64_t Kp = (int64_t)U * 256;
    if (a.act.kq) {
        // Q8_K: the signed element of largest magnitude (first occurrence),
        // iscale = -127/max, q = min(127, rint(iscale * x)), d = 1/iscale, code sums
        float ax = fabsf(val), sx = val;
        int ix = t;
        cpv_wave_amax(ax, ix, sx);
        if (lane == 0) { s_ax[wave] = ax; s_ix[wave] = ix; s_sx[wave] = sx; }
        __syncthreads();
        ax = s_ax[0];
        ix = s_ix[0];
        sx = s_sx[0];
        for (int w = 1; w < 4; w++)
            if (s_ax[w] > ax || (s_ax[w] == ax && s_ix[w] < ix)) { ax = s_ax[w]; ix = s_ix[w]; sx = s_sx[w]; }
        int q = 0;
        float d = 0.0f;
        if (ax > 0.0f) {
            const float iscale = -127.0f / sx;
            const int vq = (int)rintf(iscale * val);
            q = vq < 127 ? vq : 127;
            d = 1.0f / iscale;
        }
        qa[(int64_t)m * Kp + e] = (int8_t)q;
        const int s16 = cpv_group_reduce<16>(q, cpv_op_add());
        const int s32 = s16 + __shfl_xor(s16, 16);
        if ((t & 15) == 0) const_cast<int32_t*>(a.act.bs16)[((int64_t)m * U + u) * 16 + (t >> 4)] = s16;
        if ((t & 31) == 0) const_cast<int32_t*>(a.act.bs32)[((int64_t)m * U + u) * 8 + (t >> 5)] = s32;
        if (t == 0) da[(int64_t)m * U + u] = d;
    } else {
        // Q8_0 per 32-element block: d = amax/127, q = roundf(x * (1/d)), d kept as fp16
        float amax = fabsf(val);
        amax = cpv_group_reduce<16>(amax, cpv_op_max());
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        qa[(int64_t)m * Kp + e] = (int8_t)(int)roundf(val * id);
        if ((t & 31) == 0) da[((int64_t)m * U + u) * 8 + (t >> 5)] = cpv_h2f(cpv_f2h(d));
    }
}

// qk_prep_kernel on a kept q|gate|k|v GEMM result: each value is finalized
// (and its accumulator entry cleared) by the block that uses it; the query
// heads also write their output gate to gate_out [T][H][hd].
struct PrepKeptArgs {
    PrepArgs p;
    cpv_gout g;
    float* gate_out;
};

__global__ __launch_bounds__(128) void qk_prep_kept_kernel(PrepKeptArgs ka)
{
    const PrepArgs& a = ka.p;
    const int64_t rope0 = prep_rope0(a), kv0 = prep_kv0(a);   // (read first: off the critical path)
    const int t = blockIdx.x, hh = blockIdx.y, i = threadIdx.x;
    const bool is_q = hh < a.H;
    const int kh = hh - a.H;
    __shared__ float s_v[128];
    __shared__ float s_am[2], s_km[2];
    __shared__ long long s_s[2];
    // Ea of this token's activation row: every wave reduces its few scales
    // itself (no block barrier)
    float mx = 0.0f;
    for (int c = i & 63; c < ka.g.nda; c += 64) mx = fmaxf(mx, fabsf(ka.g.da[(int64_t)t * ka.g.nda + c]));
    const int ea = cpv_exp_of_max(cpv_wave_reduce(mx, cpv_op_max()));
    // this thread's two values: q and its gate, or k and v (their accumulator
    // entries are cleared at the end, after the block's barriers)
    const int64_t qoff = (int64_t)2 * a.H * a.hd;
    const int64_t n0 = is_q ? (int64_t)hh * 2 * a.hd + i : qoff + (int64_t)kh * a.hd + i;
    const int64_t n1 = is_q ? n0 + a.hd : n0 + (int64_t)a.Hkv * a.hd;
    double* acc = ka.g.acc + (int64_t)t * ka.g.n_pad;
    const float x = cpv_gout_value(acc[n0], ka.g.ew[n0], ea, ka.g.win);
    const float x1 = cpv_gout_value(acc[n1], ka.g.ew[n1], ea, ka.g.win);
    const float* w = is_q ? a.q_norm : a.k_norm;
    float am = fabsf(x);
    am = cpv_wave_reduce(am, cpv_op_max());
    if ((i & 63) == 0) s_am[i >> 6] = am;
    __syncthreads();
    am = s_am[0];
    if (a.hd > 64) am = fmaxf(am, s_am[1]);
    double sum = 0.0;
    if (am > 0.0f) {
        int e;
        frexpf(am, &e);
        const int g = 2 * e - (62 - ceil_log2_dev(a.hd + 1));
        long long S = cpv_fixed_floor(x * x, g);
        S = cpv_wave_reduce(S, cpv_op_add());
        if ((i & 63) == 0) s_s[i >> 6] = S;
        __syncthreads();
        S = s_s[0] + (a.hd > 64 ? s_s[1] : 0);
        sum = ldexp((double)S, g);
    }
    const float mean = (float)(sum / (double)a.hd);
    const float scale = 1.0f / sqrtf(mean + a.eps);
    const float v0 = x * scale;
    const float xn = w ? v0 * w[i] : v0;
    s_v[i] = xn;
    __syncthreads();
    float out = xn;
    const int half = a.n_rot / 2;
    if (i < a.n_rot) {
        const int p = i < half ? i : i - half;
        const float* cs = a.rope + (rope0 + (a.pos_off ? a.pos_off[t] : t)) * a.n_rot + 2 * p;
        const float c = cs[0], sn = cs[1];
        const float x0 = s_v[p], x1 = s_v[p + half];
        if (i < half) {
            const float m0 = x0 * c, m1 = x1 * sn;
            out = m0 - m1;
        } else {
            const float m0 = x0 * sn, m1 = x1 * c;
            out = m0 + m1;
        }
    }
    if (is_q) {
        a.qout[((int64_t)t * a.H + hh) * a.hd + i] = out;
        ka.gate_out[((int64_t)t * a.H + hh) * a.hd + i] = x1;
    } else if (a.write) {   // (block-uniform)
        const int64_t row = kv0 + t;
        write_k_limbs(a, kh, i, row, out, s_km);
        write_v_limbs(a, kh, i, row, x1);
    }
    acc[n0] = 0.0;
    acc[n1] = 0.0;
}

unsigned grid_for(int64_t n) { return (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096); }

}  // namespace

// ---------------------------------------------------------------- model
struct LayerW {
    cpv_weight *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
    cpv_weight *gate = nullptr, *up = nullptr, *down = nullptr;
    cpv_weight *qkv = nullptr, *gate_up = nullptr;   // stacked copies when the parts allow it
    float *attn_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct cpv_model {
    cpv_ctx* ctx = nullptr;
    cpv_hparams hp;
    std::vector<LayerW> layers;           // n_layer trunk layers, then the MTP layer
    cpv_weight *tok_embd = nullptr, *output = nullptr;
    float* output_norm = nullptr;
    // MTP extras (blk.{n_layer}.nextn.*)
    cpv_weight *eh_proj = nullptr, *mtp_embed = nullptr, *mtp_head = nullptr;
    float *enorm = nullptr, *hnorm = nullptr, *mtp_head_norm = nullptr;
    std::vector<void*> allocs;            // norm vectors
    std::vector<cpv_weight*> weights;
};

struct cpv_session {
    cpv_model* model = nullptr;
    int64_t n_ctx = 0, mtp_ctx = 0, v_stride = 0, mtp_v_stride = 0;
    int64_t n_past = 0, mtp_past = 0;
    int max_batch = 0;
    std::vector<int8_t*> kc;              // K caches as limbs, per layer; the last is the MTP cache
    std::vector<int8_t*> vt;              // V caches as limb planes (cpv_attn_launch), likewise
    float* rope = nullptr;                // [n_ctx + 2][n_rot/2][2]
    // activations, max_batch rows
    float *x, *xn, *qg, *kk, *vv, *q, *att, *gated, *o, *up, *gt, *act, *h, *logits, *e, *cat, *d, *dsa;
    float *mtp_logits, *hn;
    float *qkv, *gu;                      // outputs of the stacked q|k|v and gate|up GEMMs
    int32_t *tok, *preds, *chain;
    float* conf;
    void* actbuf;                         // quantized activations (two buffers, alternating:
    void* actbuf2;                        // a kept GEMM result refers to the scales of its input
    int act_i = 0;                        // while its consumer quantizes the next GEMM's input)
    size_t actbuf_bytes;
    float* tap = nullptr;                 // attention outputs of each call, when set
    int64_t tap_cap = 0, tap_off = 0;
    int32_t* tree_dev = nullptr;          // the last tree verify: parent [64], then depth [64]
    void** caches_dev = nullptr;          // the trunk's K caches [n_layer], then its V caches [n_layer]
    std::vector<int32_t> tree_parent;     // (host copy, to check a committed path)
    int64_t tree_base = -1;               // n_past before that verify; -1 when no tree is pending
    std::vector<int32_t> cand_host;       // the draft head's shortlist (host copy of cand_dev)
    int32_t* cand_dev = nullptr;          // [cand_cap]
    int64_t cand_cap = 0;
    cpv_weight* cand_head = nullptr;      // the draft head's rows cand_host
    int32_t* cand_idx = nullptr;          // [max_batch] a link's argmax within the shortlist
    int32_t* draft_io = nullptr;          // cpv_mtp_draft: the token in, then the draft and its gate out
    std::vector<void*> allocs;
    // round replay: the n_past and mtp_past of the call in flight in device
    // memory (the kernels that place rows read them there), and the rounds
    // captured as graphs, by shape (t, depth and the attention grids' chunk
    // counts), valid while the context's workspaces stay where they were
    int64_t* pos_dev = nullptr;           // [2]
    bool eager_only = false;              // set by a launch of the round that takes host positions
    bool replay = true;
    struct RoundGraph {
        int key[4];
        uint64_t ws_gen, used;
        hipGraphExec_t exec;
    };
    std::vector<RoundGraph> graphs;
    std::vector<std::array<int, 4>> warm;  // shapes run eagerly since the workspaces last moved
    uint64_t warm_gen = 0, clock = 0;
    int64_t n_captured = 0, n_replayed = 0;
    std::vector<std::array<int, 4>> unreplayable;
};

static cpv_status dev_alloc(cpv_ctx* ctx, std::vector<void*>& list, size_t bytes, void** out)
{
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) return cpv_hip_fail(ctx, e, "hipMalloc");
    list.push_back(p);
    *out = p;
    return CPV_OK;
}

extern "C" cpv_status cpv_model_create(cpv_ctx* ctx, const cpv_hparams* hp, cpv_model** out)
{
    if (!ctx || !hp || !out) return cpv_fail(ctx, CPV_EINVAL, "model: null argument");
    *out = nullptr;
    if (hp->n_layer < 1 || hp->n_embd < 1 || hp->n_head < 1 || hp->n_head_kv < 1 || hp->n_head % hp->n_head_kv ||
        (hp->head_dim != 64 && hp->head_dim != 128) || hp->n_rot < 0 || hp->n_rot > hp->head_dim ||
        (hp->n_rot & 1) || hp->n_ff < 1 || hp->n_vocab < 1)
        return cpv_fail(ctx, CPV_EINVAL, "model: unsupported hyper-parameters");
    cpv_model* m = new (std::nothrow) cpv_model();
    if (!m) return cpv_fail(ctx, CPV_ENOMEM, "model: host allocation");
    m->ctx = ctx;
    m->hp = *hp;
    m->layers.resize(hp->n_layer + (hp->has_mtp ? 1 : 0));
    *out = m;
    return CPV_OK;
}

extern "C" void cpv_model_free(cpv_model* m)
{
    if (!m) return;
    for (cpv_weight* w : m->weights) cpv_weight_free(w);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

static bool parse_blk(const std::string& name, int* il, std::string* rest)
{
    if (name.rfind("blk.", 0) != 0) return false;
    size_t dot = name.find('.', 4);
    if (dot == std::string::npos) return false;
    *il = atoi(name.substr(4, dot - 4).c_str());
    *rest = name.substr(dot + 1);
    return true;
}

extern "C" cpv_status cpv_model_set_tensor(cpv_model* m, const char* name_c, int type, const void* data,
                                           int on_device, int64_t ne0, int64_t ne1)
{
    if (!m || !name_c || !data || ne0 < 1 || ne1 < 1) return cpv_fail(m ? m->ctx : nullptr, CPV_EINVAL, "set_tensor: bad arguments");
    cpv_ctx* ctx = m->ctx;
    const std::string name(name_c);
    int il = -1;
    std::string rest;
    const bool blk = parse_blk(name, &il, &rest);
    const int nl = m->hp.n_layer;
    if (blk && (il < 0 || il >= (int)m->layers.size()))
        return cpv_fail(ctx, CPV_EINVAL, "set_tensor: %s: layer out of range", name_c);

    auto norm = [&](float** dst) -> cpv_status {
        if (type != CPV_F32 || ne1 != 1) return cpv_fail(ctx, CPV_EINVAL, "set_tensor: %s must be F32 [n]", name_c);
        void* p = nullptr;
        cpv_status st = dev_alloc(ctx, m->allocs, (size_t)ne0 * 4, &p);
        if (st != CPV_OK) return st;
        CPV_HIP(ctx, hipMemcpyAsync(p, data, (size_t)ne0 * 4, on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                    ctx->stream));
        CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
        *dst = (float*)p;
        return CPV_OK;
    };
    auto lin = [&](cpv_weight** dst) -> cpv_status {
        cpv_weight* w = nullptr;
        cpv_status st = on_device ? cpv_weight_from_device(ctx, type, data, ne1, ne0, &w)
                                  : cpv_weight_upload(ctx, type, data, ne1, ne0, &w);
        if (st != CPV_OK) return st;
        m->weights.push_back(w);
        *dst = w;
        return CPV_OK;
    };

    if (name == "token_embd.weight") return lin(&m->tok_embd);
    if (name == "output.weight") return lin(&m->output);
    if (name == "output_norm.weight") return norm(&m->output_norm);
    if (!blk) return cpv_fail(ctx, CPV_EINVAL, "set_tensor: unknown tensor %s", name_c);
    LayerW& L = m->layers[il];
    if (rest == "attn_norm.weight") return norm(&L.attn_norm);
    if (rest == "post_attention_norm.weight") return norm(&L.post_norm);
    if (rest == "attn_q_norm.weight") return norm(&L.q_norm);
    if (rest == "attn_k_norm.weight") return norm(&L.k_norm);
    if (rest == "attn_q.weight") return lin(&L.wq);
    if (rest == "attn_k.weight") return lin(&L.wk);
    if (rest == "attn_v.weight") return lin(&L.wv);
    if (rest == "attn_output.weight") return lin(&L.wo);
    if (rest == "ffn_gate.weight") return lin(&L.gate);
    if (rest == "ffn_up.weight") return lin(&L.up);
    if (rest == "ffn_down.weight") return lin(&L.down);
    if (il == nl) {
        if (rest == "nextn.eh_proj.weight") return lin(&m->eh_proj);
        if (rest == "nextn.enorm.weight") return norm(&m->enorm);
        if (rest == "nextn.hnorm.weight") return norm(&m->hnorm);
        if (rest == "nextn.embed_tokens.weight") return lin(&m->mtp_embed);
        if (rest == "nextn.shared_head_norm.weight") return norm(&m->mtp_head_norm);
        if (rest == "nextn.shared_head_head.weight") return lin(&m->mtp_head);
    }
    return cpv_fail(ctx, CPV_EINVAL, "set_tensor: unknown tensor %s", name_c);
}

extern "C" cpv_status cpv_model_ready(cpv_model* m)
{
    if (!m) return CPV_EINVAL;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    if (!m->tok_embd || !m->output_norm) return cpv_fail(ctx, CPV_EINVAL, "model: token_embd / output_norm missing");
    if (!m->output) m->output = m->tok_embd;           // tied head (qwen35.rs:2789)
    const int64_t E = hp.n_embd, hd = hp.head_dim, H = hp.n_head, Hkv = hp.n_head_kv, F = hp.n_ff;
    auto shape = [&](const cpv_weight* w, int64_t n, int64_t k, const char* what) -> cpv_status {
        if (!w) return cpv_fail(ctx, CPV_EINVAL, "model: %s missing", what);
        if (w->n != n || w->k != k)
            return cpv_fail(ctx, CPV_EINVAL, "model: %s is [%lld x %lld], want [%lld x %lld]", what, (long long)w->n,
                            (long long)w->k, (long long)n, (long long)k);
        return CPV_OK;
    };
    cpv_status st;
    if ((st = shape(m->tok_embd, hp.n_vocab, E, "token_embd")) || (st = shape(m->output, hp.n_vocab, E, "output")))
        return st;
    for (size_t il = 0; il < m->layers.size(); il++) {
        const LayerW& L = m->layers[il];
        if (!L.attn_norm || !L.post_norm || !L.q_norm || !L.k_norm)
            return cpv_fail(ctx, CPV_EINVAL, "model: layer %zu norms missing", il);
        if ((!L.qkv && ((st = shape(L.wq, 2 * H * hd, E, "attn_q")) || (st = shape(L.wk, Hkv * hd, E, "attn_k")) ||
                        (st = shape(L.wv, Hkv * hd, E, "attn_v")))) ||
            (st = shape(L.wo, E, H * hd, "attn_output")) ||
            (!L.gate_up && ((st = shape(L.gate, F, E, "ffn_gate")) || (st = shape(L.up, F, E, "ffn_up")))) ||
            (st = shape(L.down, E, F, "ffn_down")))
            return st;
    }
    if (hp.has_mtp) {
        if (!m->enorm || !m->hnorm) return cpv_fail(ctx, CPV_EINVAL, "model: nextn norms missing");
        if ((st = shape(m->eh_proj, E, 2 * E, "nextn.eh_proj"))) return st;
        if (!m->mtp_embed) m->mtp_embed = m->tok_embd;
        if (!m->mtp_head) m->mtp_head = m->output;
        if (!m->mtp_head_norm) m->mtp_head_norm = m->output_norm;
    }
    // Stack q|k|v and gate|up into one weight each where the parts allow it
    // (same type, whole 64-row tiles): one activation pass and one GEMM launch
    // instead of three / two.  The parts are freed.
    auto release = [&](cpv_weight* w) {
        for (size_t i = 0; i < m->weights.size(); i++)
            if (m->weights[i] == w) {
                cpv_weight_free(w);
                m->weights.erase(m->weights.begin() + (long)i);
                return;
            }
    };
    for (LayerW& L : m->layers) {
        if (!L.qkv && L.wq->type == L.wk->type && L.wk->type == L.wv->type && L.wq->n % 64 == 0 && L.wk->n % 64 == 0) {
            cpv_weight* parts[3] = {L.wq, L.wk, L.wv};
            if ((st = cpv_weight_concat(ctx, parts, 3, &L.qkv))) return st;
            m->weights.push_back(L.qkv);
            release(L.wq);
            release(L.wk);
            release(L.wv);
            L.wq = L.wk = L.wv = nullptr;
        }
        if (!L.gate_up && L.gate->type == L.up->type && L.gate->n % 64 == 0) {
            cpv_weight* parts[2] = {L.gate, L.up};
            if ((st = cpv_weight_concat(ctx, parts, 2, &L.gate_up))) return st;
            m->weights.push_back(L.gate_up);
            release(L.gate);
            release(L.up);
            L.gate = L.up = nullptr;
        }
    }
    return CPV_OK;
}

// ---------------------------------------------------------------- session
extern "C" void cpv_session_free(cpv_session* s)
{
    if (!s) return;
    (void)hipStreamSynchronize(s->model->ctx->stream);
    for (auto& g : s->graphs) (void)hipGraphExecDestroy(g.exec);
    for (void* p : s->allocs) (void)hipFree(p);
    if (s->cand_dev) (void)hipFree(s->cand_dev);
    if (s->cand_head) cpv_weight_free(s->cand_head);
    delete s;
}

extern "C" cpv_status cpv_session_create(cpv_model* m, int64_t n_ctx, int32_t max_batch, cpv_session** out)
{
    if (!m || !out || n_ctx < 1 || max_batch < 1 || max_batch > 4096)
        return cpv_fail(m ? m->ctx : nullptr, CPV_EINVAL, "session: bad arguments");
    cpv_ctx* ctx = m->ctx;
    *out = nullptr;
    const cpv_hparams& hp = m->hp;
    cpv_session* s = new (std::nothrow) cpv_session();
    if (!s) return cpv_fail(ctx, CPV_ENOMEM, "session: host allocation");
    s->model = m;
    s->n_ctx = n_ctx;
    s->mtp_ctx = n_ctx < 16384 ? n_ctx : 16384;       // mtp_ctx_cap (qwen35.rs:366-373)
    s->v_stride = (n_ctx + 15) / 16 * 16;          // (16-byte limb segments)
    s->mtp_v_stride = (s->mtp_ctx + 15) / 16 * 16;
    s->max_batch = max_batch;
    const int64_t E = hp.n_embd, hd = hp.head_dim, H = hp.n_head, Hkv = hp.n_head_kv, F = hp.n_ff, V = hp.n_vocab;
    const int64_t T = max_batch;
    cpv_status st = CPV_OK;
    auto A = [&](size_t bytes, void** p) {
        if (st == CPV_OK) st = dev_alloc(ctx, s->allocs, bytes, p);
    };
    const size_t layers = m->layers.size();
    s->kc.resize(layers);
    s->vt.resize(layers);
    for (size_t il = 0; il < layers; il++) {
        const bool mtp = (int)il == hp.n_layer;
        const int64_t rows = mtp ? s->mtp_ctx : n_ctx, vs = mtp ? s->mtp_v_stride : s->v_stride;
        (void)rows;
        A((size_t)cpv_k_cache_bytes((int)Hkv, (int)hd, vs), (void**)&s->kc[il]);
        A((size_t)CPV_ATTN_VLIMBS * Hkv * hd * vs, (void**)&s->vt[il]);
        if (st == CPV_OK)
            CPV_HIP(ctx, hipMemsetAsync(s->vt[il], 0, (size_t)CPV_ATTN_VLIMBS * Hkv * hd * vs, ctx->stream));
    }
    A((size_t)T * E * 4, (void**)&s->x);
    A((size_t)T * 2 * E * 4, (void**)&s->xn);
    A((size_t)T * 2 * H * hd * 4, (void**)&s->qg);
    A((size_t)T * Hkv * hd * 4, (void**)&s->kk);
    A((size_t)T * Hkv * hd * 4, (void**)&s->vv);
    A((size_t)T * H * hd * 4, (void**)&s->q);
    A((size_t)T * H * hd * 4, (void**)&s->att);
    A((size_t)T * H * hd * 4, (void**)&s->gated);
    A((size_t)T * E * 4, (void**)&s->o);
    A((size_t)T * F * 4, (void**)&s->up);
    A((size_t)T * F * 4, (void**)&s->gt);
    A((size_t)T * F * 4, (void**)&s->act);
    A((size_t)T * (2 * H + 2 * Hkv) * hd * 4, (void**)&s->qkv);
    A((size_t)T * 2 * F * 4, (void**)&s->gu);
    A((size_t)T * E * 4, (void**)&s->h);
    A((size_t)T * V * 4, (void**)&s->logits);
    A((size_t)T * V * 4, (void**)&s->mtp_logits);
    A((size_t)T * E * 4, (void**)&s->hn);
    A((size_t)T * E * 4, (void**)&s->e);
    A((size_t)T * 2 * E * 4, (void**)&s->cat);
    A((size_t)T * E * 4, (void**)&s->d);
    A((size_t)T * E * 4, (void**)&s->dsa);
    A((size_t)T * 4, (void**)&s->tok);
    A((size_t)T * 4, (void**)&s->preds);
    A((size_t)16 * T * 4, (void**)&s->chain);
    A((size_t)16 * T * 4, (void**)&s->conf);
    A((size_t)2 * CPV_TREE_MAX * 4, (void**)&s->tree_dev);
    A(2 * sizeof(int64_t), (void**)&s->pos_dev);
    A((size_t)T * 4, (void**)&s->cand_idx);
    A(4 * sizeof(int32_t), (void**)&s->draft_io);
    A((size_t)2 * hp.n_layer * sizeof(void*), (void**)&s->caches_dev);
    if (st == CPV_OK) {
        std::vector<void*> cp(2 * hp.n_layer);
        for (int il = 0; il < hp.n_layer; il++) {
            cp[il] = s->kc[il];
            cp[hp.n_layer + il] = s->vt[il];
        }
        // (synchronous: the host vector goes away on return)
        hipError_t e = hipMemcpy(s->caches_dev, cp.data(), cp.size() * sizeof(void*), hipMemcpyHostToDevice);
        if (e != hipSuccess) st = cpv_hip_fail(ctx, e, "hipMemcpy");
    }
    const int64_t kmax = (2 * E > F ? 2 * E : F) > H * hd ? (2 * E > F ? 2 * E : F) : H * hd;
    s->actbuf_bytes = cpv_act_bytes(CPV_Q4_K, kmax, T) > cpv_act_bytes(CPV_Q8_0, kmax, T)
                    ? cpv_act_bytes(CPV_Q4_K, kmax, T) : cpv_act_bytes(CPV_Q8_0, kmax, T);
    A(s->actbuf_bytes, &s->actbuf);
    A(s->actbuf_bytes, &s->actbuf2);
    // rope table: positions up to n_ctx + 1 (the MTP head runs one position ahead)
    const int64_t npos = n_ctx + 2, nrot = hp.n_rot;
    if (st == CPV_OK && nrot > 0) {
        std::vector<float> tab((size_t)npos * nrot);
        const float theta_scale = powf(hp.freq_base, -2.0f / (float)nrot);
        const int32_t* sec = hp.rope_sections;
        const int sect = sec[0] + sec[1] + sec[2] + sec[3];
        for (int64_t p = 0; p < npos; p++) {
            float th_t = (float)p, th_h = (float)p, th_w = (float)p, th_e = 0.0f;
            for (int64_t i = 0; i < nrot / 2; i++) {
                float theta = th_t;
                if (sect > 0) {
                    const int sc = (int)(i % sect);
                    if (sc % 3 == 1 && sc < 3 * sec[1]) theta = th_h;
                    else if (sc % 3 == 2 && sc < 3 * sec[2]) theta = th_w;
                    else if (sc % 3 == 0 && sc < 3 * sec[0]) theta = th_t;
                    else theta = th_e;
                }
                tab[(size_t)p * nrot + 2 * i] = cosf(theta);
                tab[(size_t)p * nrot + 2 * i + 1] = sinf(theta);
                th_t *= theta_scale;
                th_h *= theta_scale;
                th_w *= theta_scale;
                th_e *= theta_scale;
            }
        }
        A(tab.size() * 4, (void**)&s->rope);
        if (st == CPV_OK) {
            CPV_HIP(ctx, hipMemcpyAsync(s->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, ctx->stream));
            CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
        }
    }
    if (st != CPV_OK) {
        cpv_session_free(s);
        return st;
    }
    *out = s;
    return CPV_OK;
}

extern "C" cpv_status cpv_session_set_pos(cpv_session* s, int64_t n_past, int64_t mtp_past)
{
    if (!s || n_past < 0 || n_past > s->n_ctx || mtp_past < 0 || mtp_past > s->mtp_ctx)
        return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "session: position out of range");
    s->n_past = n_past;
    s->mtp_past = mtp_past;
    s->tree_base = -1;
    return CPV_OK;
}

extern "C" cpv_status cpv_session_set_attn_tap(cpv_session* s, float* tap_dev, int64_t capacity_floats)
{
    if (!s || capacity_floats < 0 || (!tap_dev && capacity_floats))
        return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "set_attn_tap: bad arguments");
    s->tap = tap_dev;
    s->tap_cap = tap_dev ? capacity_floats : 0;
    s->tap_off = 0;
    return CPV_OK;
}

extern "C" cpv_status cpv_session_set_replay(cpv_session* s, int on)
{
    if (!s) return CPV_EINVAL;
    s->replay = on != 0;
    return CPV_OK;
}

extern "C" cpv_status cpv_session_replay_stats(const cpv_session* s, int64_t* captured, int64_t* replayed)
{
    if (!s || !captured || !replayed) return CPV_EINVAL;
    *captured = s->n_captured;
    *replayed = s->n_replayed;
    return CPV_OK;
}

extern "C" cpv_status cpv_session_get_pos(const cpv_session* s, int64_t* n_past, int64_t* mtp_past)
{
    if (!s) return CPV_EINVAL;
    if (n_past) *n_past = s->n_past;
    if (mtp_past) *mtp_past = s->mtp_past;
    return CPV_OK;
}

// ---------------------------------------------------------------- forward
namespace {

void* next_act(cpv_session* s)
{
    s->act_i ^= 1;
    return s->act_i ? s->actbuf2 : s->actbuf;
}

cpv_status rmsnorm(cpv_ctx* ctx, const float* x, int64_t xs, const float* w, float* y, int64_t ys, int64_t rows,
                   int n, float eps)
{
    rmsnorm_kernel<<<(unsigned)rows, 1024, 0, ctx->stream>>>(x, xs, w, y, ys, n, eps);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

cpv_status row_launch(cpv_ctx* ctx, const RowArgs& a, int T)
{
    const dim3 ugrid((unsigned)((a.n + 255) / 256), (unsigned)T);
    const bool rowk = a.src <= SRC_SET || a.src == SRC_CAT;
    if (rowk) {
        // row_kernel: 16-byte accesses of every row it reads or writes
        auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
        const bool kept = a.src == SRC_ADD || a.src == SRC_SET;
        if (a.n % 4 || a.xs % 4 || !a.x || !al(a.x) || (a.w && !al(a.w)) || (a.y && (a.ys % 4 || !al(a.y))) ||
            (kept && (!al(a.g.acc) || a.g.n_pad % 4 || !al(a.g.ew))))
            return cpv_fail(ctx, CPV_EUNSUPPORTED, "row kernel: rows of %d need 16-byte aligned rows of a multiple of 4",
                            a.n);
        if (a.src == SRC_CAT && (a.nseg % 256 || a.n != 2 * a.nseg || !a.w || !a.w2 || !al(a.w2) || !a.x2 ||
                                 !al(a.x2) || a.xs2 % 4))
            return cpv_fail(ctx, CPV_EUNSUPPORTED, "row kernel: halves of %d need whole units and both weights", a.nseg);
        if (a.src == SRC_CAT && a.psum && !a.conf_out) return cpv_fail(ctx, CPV_EINVAL, "row kernel: a peak needs its output");
    }
    // row_kernel: the fewest units per wave that 16 waves cover, and the waves that many units need
    const int U = (a.n + 255) / 256, nu = (U + RW - 1) / RW, nt = 64 * ((U + nu - 1) / nu);
    if (rowk && nu > RUU)
        return cpv_fail(ctx, CPV_EUNSUPPORTED, "row kernel: rows of %d exceed %d elements", a.n, RQ * RB);
    auto rows = [&](auto src) {
        constexpr int S = decltype(src)::value;
        if (nu == 1) row_kernel<S, 1><<<(unsigned)T, (unsigned)nt, 0, ctx->stream>>>(a);
        else if (nu == 2) row_kernel<S, 2><<<(unsigned)T, (unsigned)nt, 0, ctx->stream>>>(a);
        else row_kernel<S, 3><<<(unsigned)T, (unsigned)nt, 0, ctx->stream>>>(a);
    };
    switch (a.src) {
    case SRC_X: rows(std::integral_constant<int, SRC_X>()); break;
    case SRC_ADD: rows(std::integral_constant<int, SRC_ADD>()); break;
    case SRC_SET: rows(std::integral_constant<int, SRC_SET>()); break;
    case SRC_CAT: rows(std::integral_constant<int, SRC_CAT>()); break;
    case SRC_GATE: unit_kernel<SRC_GATE><<<ugrid, 256, 0, ctx->stream>>>(a); break;
    case SRC_GATE_FOLD:
        if (a.hd % 64 || 256 % a.hd || a.n % a.hd || a.part.nchunk > FOLD_MAX)
            return cpv_fail(ctx, CPV_EUNSUPPORTED, "gate fold: head dim %d, %d chunks", a.hd, a.part.nchunk);
        unit_kernel<SRC_GATE_FOLD><<<ugrid, 256, 0, ctx->stream>>>(a);
        break;
    default: unit_kernel<SRC_SWIGLU><<<ugrid, 256, 0, ctx->stream>>>(a); break;
    }
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

// fold a kept GEMM result into x (SRC_ADD: x += y, SRC_SET: x = y), nothing else
cpv_status apply_kept(cpv_session* s, float* x, int T, const cpv_gout& g, int src)
{
    RowArgs r{};
    r.src = src;
    r.x = x;
    r.xs = s->model->hp.n_embd;
    r.g = g;
    r.n = (int)s->model->hp.n_embd;
    return row_launch(s->model->ctx, r, T);
}

// one attention block + FFN block of layer L on x (in place), T rows, one
// kernel per op: the path for unstacked weights
// a draft tree on the device: parent[i] (-1: a child of the context) and the
// depth of node i, whose position is the round's base position + depth
struct Tree {
    const int32_t* parent;
    const int32_t* depth;
};

// the session's positions into its device copy, for the call's kernels
__global__ void set_pos_kernel(int64_t* __restrict__ pos, int64_t n_past, int64_t mtp_past)
{
    if (threadIdx.x == 0) {
        pos[0] = n_past;
        pos[1] = mtp_past;
    }
}

cpv_status set_pos_dev(cpv_session* s)
{
    cpv_ctx* ctx = s->model->ctx;
    set_pos_kernel<<<1, 64, 0, ctx->stream>>>(s->pos_dev, s->n_past, s->mtp_past);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

// the device position a block reads: KV rows from pos[kv] (0: n_past, 1:
// mtp_past), rope positions pos[0] + rope_off (the host values rope_pos0,
// kv_row0 and attn_past of the same call size the grids)
struct PosSel {
    int kv, rope_off;
};

cpv_status block_unfused(cpv_session* s, const LayerW& L, float* x, int T, int64_t rope_pos0, int64_t kv_row0,
                 int64_t attn_past, int8_t* kc, int8_t* vt, int64_t v_stride, bool write,
                 const Tree* tree, PosSel ps)
{
    const int32_t* parent = tree ? tree->parent : nullptr;
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    const int64_t E = hp.n_embd, hd = hp.head_dim, H = hp.n_head, Hkv = hp.n_head_kv, F = hp.n_ff;
    cpv_status st;
    cpv_act act;
    // attention (build_attn_block)
    if ((st = rmsnorm(ctx, x, E, L.attn_norm, s->xn, E, T, (int)E, hp.rms_eps))) return st;
    PrepArgs pa;
    if (L.qkv) {
        // one GEMM for q|gate, k and v: row stride 2*H*hd + 2*Hkv*hd
        if ((st = cpv_quant_act(ctx, L.qkv->type, s->xn, T, E, next_act(s), &act))) return st;
        if ((st = cpv_qgemm_act(ctx, L.qkv, &act, s->qkv))) return st;
        pa.qg = s->qkv;
        pa.kk = s->qkv + 2 * H * hd;
        pa.vv = pa.kk + Hkv * hd;
        pa.qs = pa.ks = L.qkv->n;
    } else {
        if ((st = cpv_quant_act(ctx, L.wq->type, s->xn, T, E, next_act(s), &act))) return st;
        if ((st = cpv_qgemm_act(ctx, L.wq, &act, s->qg))) return st;
        if (L.wk->type != L.wq->type && (st = cpv_quant_act(ctx, L.wk->type, s->xn, T, E, next_act(s), &act))) return st;
        if ((st = cpv_qgemm_act(ctx, L.wk, &act, s->kk))) return st;
        if (L.wv->type != L.wk->type && (st = cpv_quant_act(ctx, L.wv->type, s->xn, T, E, next_act(s), &act))) return st;
        if ((st = cpv_qgemm_act(ctx, L.wv, &act, s->vv))) return st;
        pa.qg = s->qg;
        pa.kk = s->kk;
        pa.vv = s->vv;
        pa.qs = 2 * H * hd;
        pa.ks = Hkv * hd;
    }
    pa.q_norm = L.q_norm;
    pa.k_norm = L.k_norm;
    pa.rope = s->rope;
    pa.qout = s->q;
    pa.k_limbs = kc;
    pa.v_limbs = vt;
    pa.v_stride = v_stride;
    pa.rope_pos0 = rope_pos0;
    pa.kv_row0 = kv_row0;
    pa.pos_off = tree ? tree->depth : nullptr;
    pa.H = (int)H;
    pa.Hkv = (int)Hkv;
    pa.hd = (int)hd;
    pa.n_rot = hp.n_rot;
    pa.write = write ? 1 : 0;
    pa.eps = hp.rms_eps;
    pa.pos = s->pos_dev;
    pa.pos_kv = ps.kv;
    pa.rope_off = ps.rope_off;
    s->eager_only = true;   // (the attention below takes host positions)
    qk_prep_kernel<<<dim3((unsigned)T, (unsigned)(H + Hkv)), (unsigned)hd, 0, ctx->stream>>>(pa);
    CPV_HIP(ctx, hipGetLastError());
    const float kq_scale = 1.0f / sqrtf((float)hd);
    if ((st = cpv_attn_launch(ctx, s->q, nullptr, nullptr, v_stride, attn_past, parent, T, (int)H, (int)Hkv, (int)hd,
                              kq_scale, s->att, vt, kc)))
        return st;
    if (s->tap) {
        const int64_t n = (int64_t)T * H * hd;
        if (s->tap_off + n <= s->tap_cap)
            CPV_HIP(ctx, hipMemcpyAsync(s->tap + s->tap_off, s->att, (size_t)n * 4, hipMemcpyDeviceToDevice, ctx->stream));
        s->tap_off += n;
    }
    gate_mul_kernel<<<grid_for(T * H * hd), 256, 0, ctx->stream>>>(s->att, pa.qg, pa.qs, (int)H, (int)hd, T * H * hd,
                                                                  s->gated);
    if ((st = cpv_quant_act(ctx, L.wo->type, s->gated, T, H * hd, next_act(s), &act))) return st;
    if ((st = cpv_qgemm_act(ctx, L.wo, &act, s->o))) return st;
    add_kernel<<<grid_for(T * E), 256, 0, ctx->stream>>>(s->o, x, x, T * E);
    // FFN
    if ((st = rmsnorm(ctx, x, E, L.post_norm, s->xn, E, T, (int)E, hp.rms_eps))) return st;
    if (L.gate_up) {
        // one GEMM for gate|up: row stride 2F
        if ((st = cpv_quant_act(ctx, L.gate_up->type, s->xn, T, E, next_act(s), &act))) return st;
        if ((st = cpv_qgemm_act(ctx, L.gate_up, &act, s->gu))) return st;
        swiglu_kernel<<<grid_for(T * F), 256, 0, ctx->stream>>>(s->gu, s->gu + F, 2 * F, F, s->act, T * F);
    } else {
        if ((st = cpv_quant_act(ctx, L.up->type, s->xn, T, E, next_act(s), &act))) return st;
        if ((st = cpv_qgemm_act(ctx, L.up, &act, s->up))) return st;
        if (L.gate->type != L.up->type && (st = cpv_quant_act(ctx, L.gate->type, s->xn, T, E, next_act(s), &act)))
            return st;
        if ((st = cpv_qgemm_act(ctx, L.gate, &act, s->gt))) return st;
        swiglu_kernel<<<grid_for(T * F), 256, 0, ctx->stream>>>(s->gt, s->up, F, F, s->act, T * F);
    }
    if ((st = cpv_quant_act(ctx, L.down->type, s->act, T, F, next_act(s), &act))) return st;
    if ((st = cpv_qgemm_act(ctx, L.down, &act, s->d))) return st;
    add_kernel<<<grid_for(T * E), 256, 0, ctx->stream>>>(s->d, x, x, T * E);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

bool fusable(const cpv_model* m, const LayerW& L)
{
    const cpv_hparams& hp = m->hp;
    // the residual rows go through row_kernel (RQ elements per thread); the
    // gated attention output and SwiGLU rows through unit_kernel (any length)
    return L.qkv && L.gate_up && hp.n_embd <= (int64_t)RQ * RB;
}

// One attention block + FFN block of layer L on x (in place), T rows.  pend,
// when given, is a kept GEMM result folded into x first (pend_src: SRC_ADD or
// SRC_SET).  On return *out holds the block's FFN down projection as a kept
// result still to be added to x (the next block, the final norm or apply_kept
// folds it in), or out->acc is null when the block already added it.
// Launches per block: norm+quant, q|k|v GEMM, prep, attention (2), gate+quant,
// wo GEMM, residual+norm+quant, gate|up GEMM, SwiGLU+quant, down GEMM.
cpv_status block(cpv_session* s, const LayerW& L, float* x, int T, int64_t rope_pos0, int64_t kv_row0,
                 int64_t attn_past, int8_t* kc, int8_t* vt, int64_t v_stride, bool write, const cpv_gout* pend,
                 int pend_src, cpv_gout* out, PosSel ps, const Tree* tree = nullptr)
{
    const int32_t* parent = tree ? tree->parent : nullptr;
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    const int64_t E = hp.n_embd, hd = hp.head_dim, H = hp.n_head, Hkv = hp.n_head_kv, F = hp.n_ff;
    cpv_status st;
    out->acc = nullptr;
    if (!fusable(m, L)) {
        if (pend && (st = apply_kept(s, x, T, *pend, pend_src))) return st;
        return block_unfused(s, L, x, T, rope_pos0, kv_row0, attn_past, kc, vt, v_stride, write, tree, ps);
    }
    // attention norm (after the pending residual term) and the q|k|v input
    RowArgs r{};
    r.src = pend ? pend_src : SRC_X;
    r.x = x;
    r.xs = E;
    if (pend) r.g = *pend;
    r.n = (int)E;
    r.w = L.attn_norm;
    r.norm = 1;
    r.eps = hp.rms_eps;
    r.quant = 1;
    cpv_act_layout(L.qkv->type, T, E, next_act(s), &r.act);
    if ((st = row_launch(ctx, r, T))) return st;
    cpv_gout g;
    if ((st = cpv_qgemm_keep(ctx, L.qkv, &r.act, &g))) return st;
    // q/k norm, rope, KV write, output gate
    PrepKeptArgs pk;
    PrepArgs& pa = pk.p;
    pa.qg = pa.kk = pa.vv = nullptr;
    pa.qs = pa.ks = 0;
    pa.q_norm = L.q_norm;
    pa.k_norm = L.k_norm;
    pa.rope = s->rope;
    pa.qout = s->q;
    pa.k_limbs = kc;
    pa.v_limbs = vt;
    pa.v_stride = v_stride;
    pa.rope_pos0 = rope_pos0;
    pa.kv_row0 = kv_row0;
    pa.pos_off = tree ? tree->depth : nullptr;
    pa.H = (int)H;
    pa.Hkv = (int)Hkv;
    pa.hd = (int)hd;
    pa.n_rot = hp.n_rot;
    pa.write = write ? 1 : 0;
    pa.eps = hp.rms_eps;
    pa.pos = s->pos_dev;
    pa.pos_kv = ps.kv;
    pa.rope_off = ps.rope_off;
    pk.g = g;
    pk.gate_out = s->qg;
    qk_prep_kept_kernel<<<dim3((unsigned)T, (unsigned)(H + Hkv)), (unsigned)hd, 0, ctx->stream>>>(pk);
    CPV_HIP(ctx, hipGetLastError());
    const float kq_scale = 1.0f / sqrtf((float)hd);
    // attention output times sigmoid(gate), the wo input: the gate kernel folds
    // the attention's chunk partials itself, unless the tap wants the output or
    // the partials do not come in one block
    RowArgs r2{};
    r2.gate = s->qg;
    r2.n = (int)(H * hd);
    r2.quant = 1;
    cpv_attn_part part{};
    // the attention's 128-row chunks, and the grid's: a multiple of 8, so that
    // one grid serves every position of a 1024-row range (a replayed round)
    const int64_t nch = (attn_past + T + 127) / 128, nch_grid = (nch + 7) / 8 * 8;
    const bool fold = !s->tap && hd % 64 == 0 && 256 % hd == 0 && nch_grid <= FOLD_MAX &&
                      cpv_attn_partials(ctx, s->q, nullptr, nullptr, v_stride, attn_past, parent, T, (int)H, (int)Hkv, (int)hd,
                                        kq_scale, &part, s->pos_dev, ps.kv, (int)nch_grid,
                                        ps.kv == 0 ? s->n_ctx : s->mtp_ctx, vt, kc) == CPV_OK;
    if (fold) {
        r2.src = SRC_GATE_FOLD;
        r2.part = part;
        r2.hd = (int)hd;
    } else {
        s->eager_only = true;   // (host positions)
        if ((st = cpv_attn_launch(ctx, s->q, nullptr, nullptr, v_stride, attn_past, parent, T, (int)H, (int)Hkv, (int)hd,
                                  kq_scale, s->att, vt, kc)))
            return st;
        if (s->tap) {
            const int64_t n = (int64_t)T * H * hd;
            if (s->tap_off + n <= s->tap_cap)
                CPV_HIP(ctx,
                        hipMemcpyAsync(s->tap + s->tap_off, s->att, (size_t)n * 4, hipMemcpyDeviceToDevice, ctx->stream));
            s->tap_off += n;
        }
        r2.src = SRC_GATE;
        r2.att = s->att;
    }
    cpv_act_layout(L.wo->type, T, H * hd, next_act(s), &r2.act);
    if ((st = row_launch(ctx, r2, T))) return st;
    if ((st = cpv_qgemm_keep(ctx, L.wo, &r2.act, &g))) return st;
    // residual add, FFN norm, the gate|up input
    RowArgs r3{};
    r3.src = SRC_ADD;
    r3.x = x;
    r3.xs = E;
    r3.g = g;
    r3.n = (int)E;
    r3.w = L.post_norm;
    r3.norm = 1;
    r3.eps = hp.rms_eps;
    r3.quant = 1;
    cpv_act_layout(L.gate_up->type, T, E, next_act(s), &r3.act);
    if ((st = row_launch(ctx, r3, T))) return st;
    if ((st = cpv_qgemm_keep(ctx, L.gate_up, &r3.act, &g))) return st;
    // SwiGLU, the down input
    RowArgs r4{};
    r4.src = SRC_SWIGLU;
    r4.g = g;
    r4.n = (int)F;
    r4.quant = 1;
    cpv_act_layout(L.down->type, T, F, next_act(s), &r4.act);
    if ((st = row_launch(ctx, r4, T))) return st;
    return cpv_qgemm_keep(ctx, L.down, &r4.act, out);
}

cpv_status project(cpv_session* s, const cpv_weight* w, const float* x, int T, float* y)
{
    cpv_act act;
    cpv_status st = cpv_quant_act(s->model->ctx, w->type, x, T, w->k, next_act(s), &act);
    if (st != CPV_OK) return st;
    return cpv_qgemm_act(s->model->ctx, w, &act, y);
}

// x (+ a kept result) -> RMS norm with w -> y (f32) and the input of head w_head,
// whose logits go to logits
// rms(x) with weight w into y, then the head's logits; with keep, the head's
// result stays in the accumulator (*keep, for cpv_argmax_peak_rows to
// finalize), else keep->acc is null and the logits are stored
cpv_status norm_head(cpv_session* s, float* x, int T, const cpv_gout* pend, const float* w, float* y,
                     const cpv_weight* w_head, float* logits, cpv_gout* keep = nullptr)
{
    if (keep) keep->acc = nullptr;
    cpv_model* m = s->model;
    const cpv_hparams& hp = m->hp;
    if (hp.n_embd > (int64_t)RQ * RB) {     // rows too long for row_kernel (never with a kept result)
        cpv_status st = rmsnorm(m->ctx, x, hp.n_embd, w, y, hp.n_embd, T, (int)hp.n_embd, hp.rms_eps);
        return st != CPV_OK ? st : project(s, w_head, y, T, logits);
    }
    RowArgs r{};
    r.src = pend ? SRC_ADD : SRC_X;
    r.x = x;
    r.xs = hp.n_embd;
    if (pend) r.g = *pend;
    r.n = hp.n_embd;
    r.w = w;
    r.norm = 1;
    r.eps = hp.rms_eps;
    r.y = y;
    r.ys = hp.n_embd;
    r.quant = 1;
    cpv_act_layout(w_head->type, T, hp.n_embd, next_act(s), &r.act);
    cpv_status st = row_launch(m->ctx, r, T);
    if (st != CPV_OK) return st;
    if (keep) return cpv_qgemm_keep(m->ctx, w_head, &r.act, keep);
    return cpv_qgemm_act(m->ctx, w_head, &r.act, logits);
}

}  // namespace

extern "C" cpv_status cpv_prefill(cpv_session* s, const int32_t* tokens_dev, int t)
{
    if (!s || !tokens_dev || t < 1 || t > s->max_batch)
        return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "prefill: bad arguments");
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    if (s->n_past + t > s->n_ctx) return cpv_fail(ctx, CPV_EINVAL, "prefill: context overflow");
    cpv_status st;
    s->tap_off = 0;
    s->tree_base = -1;
    if ((st = set_pos_dev(s)) != CPV_OK) return st;
    CPV_HIP(ctx, hipMemcpyAsync(s->tok, tokens_dev, (size_t)t * 4, hipMemcpyDeviceToDevice, ctx->stream));
    if ((st = cpv_get_rows(ctx, m->tok_embd, s->tok, t, s->x))) return st;
    cpv_gout pend{}, nxt{};
    for (int il = 0; il < m->hp.n_layer; il++) {
        if ((st = block(s, m->layers[il], s->x, t, s->n_past, s->n_past, s->n_past, s->kc[il], s->vt[il], s->v_stride,
                        true, pend.acc ? &pend : nullptr, SRC_ADD, &nxt, PosSel{0, 0})))
            return st;
        pend = nxt;
    }
    if (pend.acc && (st = apply_kept(s, s->x, t, pend, SRC_ADD))) return st;
    s->n_past += t;
    return CPV_OK;
}

namespace {

// a shortlist link's drafts: ids[i] = cands[idx[i]]
__global__ void map_cands_kernel(const int32_t* __restrict__ idx, const int32_t* __restrict__ cands, int t,
                                 int32_t* __restrict__ ids)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < t) ids[i] = cands[idx[i]];
}

// the draft head over `cands` (host, ids < V): uploaded and gathered when they
// differ from the last shortlist; the device buffers a previous round may still
// read are replaced only after the stream drains
cpv_status set_cands(cpv_session* s, const int32_t* cands, int n)
{
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    if ((size_t)n == s->cand_host.size() && std::equal(cands, cands + n, s->cand_host.begin())) return CPV_OK;
    for (int j = 0; j < n; j++)
        if (cands[j] < 0 || cands[j] >= m->hp.n_vocab)
            return cpv_fail(ctx, CPV_EINVAL, "verify_step: candidate %d = %d outside the vocabulary", j, cands[j]);
    CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
    s->cand_host.clear();
    if (s->cand_head) {
        cpv_weight_free(s->cand_head);
        s->cand_head = nullptr;
    }
    if (n > s->cand_cap) {
        if (s->cand_dev) (void)hipFree(s->cand_dev);
        s->cand_dev = nullptr;
        s->cand_cap = 0;
        CPV_HIP(ctx, hipMalloc((void**)&s->cand_dev, (size_t)n * 4));
        s->cand_cap = n;
    }
    CPV_HIP(ctx, hipMemcpy(s->cand_dev, cands, (size_t)n * 4, hipMemcpyHostToDevice));
    cpv_status st = cpv_weight_gather(ctx, m->mtp_head, s->cand_dev, n, &s->cand_head);
    if (st != CPV_OK) return st;
    s->cand_host.assign(cands, cands + n);
    return CPV_OK;
}

}  // namespace

namespace {

// a standalone draft link's inputs: its rope position and MTP row into the
// session's device positions, its token into draft_io[0]
__global__ void draft_setup_kernel(int64_t* __restrict__ pos, int64_t rope_pos, int64_t mtp_row,
                                   int32_t* __restrict__ io, int32_t token)
{
    if (threadIdx.x == 0) {
        pos[0] = rope_pos;
        pos[1] = mtp_row;
        io[0] = token;
    }
}

}  // namespace

extern "C" cpv_status cpv_mtp_draft(cpv_session* s, const float* hidden_dev, int32_t token, int64_t pos, float p_min,
                                    cpv_draft_out* out)
{
    if (!s || !hidden_dev || !out) return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "mtp_draft: null argument");
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    const int64_t E = hp.n_embd, V = hp.n_vocab;
    if (!hp.has_mtp) return cpv_fail(ctx, CPV_EINVAL, "mtp_draft: the model has no MTP head");
    if (token < 0 || token >= V) return cpv_fail(ctx, CPV_EINVAL, "mtp_draft: token %d outside the vocabulary", token);
    // the rope table covers positions 0 .. n_ctx + 1
    if (pos < 0 || pos > s->n_ctx + 1) return cpv_fail(ctx, CPV_EINVAL, "mtp_draft: position %lld out of range", (long long)pos);
    // the reference writes row mtp_past with no check (qwen35.rs:2177-2181);
    // here a full MTP cache is an error
    if (s->mtp_past + 1 > s->mtp_ctx)
        return cpv_fail(ctx, CPV_EINVAL, "mtp_draft: the MTP cache is full (%lld rows)", (long long)s->mtp_ctx);
    cpv_status st;
    s->tap_off = 0;
    draft_setup_kernel<<<1, 64, 0, ctx->stream>>>(s->pos_dev, pos, s->mtp_past, s->draft_io, token);
    CPV_HIP(ctx, hipGetLastError());
    if ((st = cpv_get_rows(ctx, m->mtp_embed, s->draft_io, 1, s->e))) return st;
    cpv_act act;
    if (2 * E <= (int64_t)RQ * RB && E % 256 == 0) {
        RowArgs rc{};
        rc.src = SRC_CAT;
        rc.x = s->e;
        rc.xs = E;
        rc.x2 = hidden_dev;
        rc.xs2 = E;
        rc.nseg = (int)E;
        rc.n = (int)(2 * E);
        rc.w = m->enorm;
        rc.w2 = m->hnorm;
        rc.norm = 1;
        rc.eps = hp.rms_eps;
        rc.quant = 1;
        cpv_act_layout(m->eh_proj->type, 1, 2 * E, next_act(s), &rc.act);
        if ((st = row_launch(ctx, rc, 1))) return st;
        act = rc.act;
    } else {
        if ((st = rmsnorm(ctx, s->e, E, m->enorm, s->cat, 2 * E, 1, (int)E, hp.rms_eps))) return st;
        if ((st = rmsnorm(ctx, hidden_dev, E, m->hnorm, s->cat + E, 2 * E, 1, (int)E, hp.rms_eps))) return st;
        if ((st = cpv_quant_act(ctx, m->eh_proj->type, s->cat, 1, 2 * E, next_act(s), &act))) return st;
    }
    cpv_gout eh, nxt;
    if ((st = cpv_qgemm_keep(ctx, m->eh_proj, &act, &eh))) return st;
    // the MTP layer: K/V written at row mtp_past, rows 0..mtp_past attended
    // (mtp_graph.rs:179-195 via build_attn_block), rope position pos
    if ((st = block(s, m->layers[hp.n_layer], s->dsa, 1, pos, s->mtp_past, s->mtp_past, s->kc[hp.n_layer],
                    s->vt[hp.n_layer], s->mtp_v_stride, true, &eh, SRC_SET, &nxt, PosSel{1, 0})))
        return st;
    // h_out = rms(cur, shared_head_norm or output_norm), then the head (mtp_graph.rs:218-245)
    cpv_gout mk;
    if ((st = norm_head(s, s->dsa, 1, nxt.acc ? &nxt : nullptr, m->mtp_head_norm, s->hn, m->mtp_head, s->mtp_logits,
                        &mk)))
        return st;
    if ((st = cpv_argmax_gate_rows(ctx, s->mtp_logits, 1, V, s->draft_io + 1, p_min, s->draft_io + 2,
                                   mk.acc ? &mk : nullptr)))
        return st;
    s->mtp_past += 1;
    out->logits_dev = s->mtp_logits;
    out->hidden_dev = s->hn;
    out->draft_dev = s->draft_io + 1;
    out->keep_dev = s->draft_io + 2;
    return CPV_OK;
}

extern "C" cpv_status cpv_verify_step(cpv_session* s, const int32_t* tokens_dev, int t, int depth,
                                      const float* noise_dev, cpv_round_out* out)
{
    return cpv_verify_step_cands(s, tokens_dev, t, depth, noise_dev, nullptr, 0, out);
}

namespace {

// the round's launches after its tokens are in s->tok and its positions in
// s->pos_dev: the trunk, the LM head and its argmax, the MTP chain
cpv_status round_body(cpv_session* s, int t, int depth, const float* noise_dev, bool shortlist, int n_cand)
{
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    const int64_t E = hp.n_embd, V = hp.n_vocab;
    cpv_status st;
    if ((st = cpv_get_rows(ctx, m->tok_embd, s->tok, t, s->x))) return st;
    cpv_gout pend{}, nxt{};
    for (int il = 0; il < hp.n_layer; il++) {
        if ((st = block(s, m->layers[il], s->x, t, s->n_past, s->n_past, s->n_past, s->kc[il], s->vt[il], s->v_stride,
                        true, pend.acc ? &pend : nullptr, SRC_ADD, &nxt, PosSel{0, 0})))
            return st;
        pend = nxt;
    }
    // LM head and in-graph argmax (qwen35.rs:2788-2821)
    cpv_gout hk;
    if ((st = norm_head(s, s->x, t, pend.acc ? &pend : nullptr, m->output_norm, s->h, m->output, s->logits, &hk)))
        return st;
    // with a draft chain, the argmax's last pass also writes the winners'
    // embedding rows for link 0 (each link's peak pass those for the next
    // one), and with the chain in row kernels each link's peak but the last
    // is finished by the next link's row kernel
    const bool cat = depth > 0 && 2 * E <= (int64_t)RQ * RB && E % 256 == 0;
    cpv_am_fin pfin{};
    if ((st = cpv_argmax_peak_rows(ctx, s->logits, noise_dev, t, V, s->preds, nullptr, hk.acc ? &hk : nullptr,
                                   nullptr, depth > 0 ? m->mtp_embed : nullptr, s->e)))
        return st;
    // fused MTP draft chain (qwen35.rs:2840-2962)
    if (depth > 0) {
        const LayerW& ML = m->layers[hp.n_layer];
        const float* h_src = s->h;
        for (int step = 0; step < depth; step++) {
            cpv_act act;
            if (cat) {
                // concat(enorm(e), hnorm(h)) normalized and quantized in one row
                // kernel, which also finishes the previous link's peak
                RowArgs rc{};
                rc.src = SRC_CAT;
                rc.x = s->e;
                rc.xs = E;
                if (step > 0) {
                    rc.psum = pfin.psum;
                    rc.conf_out = s->conf + (size_t)(step - 1) * t;
                }
                rc.x2 = h_src;
                rc.xs2 = E;
                rc.nseg = (int)E;
                rc.n = (int)(2 * E);
                rc.w = m->enorm;
                rc.w2 = m->hnorm;
                rc.norm = 1;
                rc.eps = hp.rms_eps;
                rc.quant = 1;
                cpv_act_layout(m->eh_proj->type, t, 2 * E, next_act(s), &rc.act);
                if ((st = row_launch(ctx, rc, t))) return st;
                act = rc.act;
            } else {
                if ((st = rmsnorm(ctx, s->e, E, m->enorm, s->cat, 2 * E, t, (int)E, hp.rms_eps))) return st;
                if ((st = rmsnorm(ctx, h_src, E, m->hnorm, s->cat + E, 2 * E, t, (int)E, hp.rms_eps))) return st;
                if ((st = cpv_quant_act(ctx, m->eh_proj->type, s->cat, t, 2 * E, next_act(s), &act))) return st;
            }
            cpv_gout eh;
            if ((st = cpv_qgemm_keep(ctx, m->eh_proj, &act, &eh))) return st;
            // positions rope_base + i + 1, rows mtp_past + i; only link 0 writes (:1858-1866, :2898-2906)
            if ((st = block(s, ML, s->dsa, t, s->n_past + 1, s->mtp_past, s->mtp_past, s->kc[hp.n_layer],
                            s->vt[hp.n_layer], s->mtp_v_stride, step == 0, &eh, SRC_SET, &nxt, PosSel{1, 1})))
                return st;
            // h_next = rms(d, shared_head_norm or output_norm), then the draft head,
            // over the shortlist when one is given (qwen35.rs:2925-2931)
            cpv_gout mk;
            if ((st = norm_head(s, s->dsa, t, nxt.acc ? &nxt : nullptr, m->mtp_head_norm, s->hn,
                                shortlist ? s->cand_head : m->mtp_head, s->mtp_logits, &mk)))
                return st;
            int32_t* ids = s->chain + (size_t)step * t;
            const bool more = step + 1 < depth;
            if ((st = cpv_argmax_peak_rows(ctx, s->mtp_logits, nullptr, t, shortlist ? n_cand : V,
                                           shortlist ? s->cand_idx : ids, s->conf + (size_t)step * t,
                                           mk.acc ? &mk : nullptr, cat && more ? &pfin : nullptr,
                                           more ? m->mtp_embed : nullptr, s->e)))
                return st;
            if (shortlist) {
                // drafts are candidates; the next link embeds the argmax itself (the
                // index into the shortlist, embedded by the peak pass above), as the
                // graph does (tok_src = ids, qwen35.rs:2958; the ids map back on the host, :1904-1910)
                map_cands_kernel<<<(unsigned)((t + 255) / 256), 256, 0, ctx->stream>>>(s->cand_idx, s->cand_dev, t, ids);
                CPV_HIP(ctx, hipGetLastError());
            }
            // the next link feeds on this link's prediction (its embedding in e) and
            // hidden (read by its hnorm before its own head overwrites hn)
            h_src = s->hn;
        }
    }
    return CPV_OK;
}

// the attention grid's chunk count for `rows` cache rows (as block() sizes it)
int chunk_bucket(int64_t rows) { return (int)(((rows + 127) / 128 + 7) / 8 * 8); }

// A greedy round of shape key replayed from its graph (*done set).  A shape's
// first round runs eagerly (so that every workspace it uses has its size);
// its second is captured, instantiated and launched.  A capture that fails,
// or a round with a launch that takes host positions, leaves the shape to
// eager rounds.  Graphs hold workspace addresses: a move of any workspace
// (ws_gen) retires them.
cpv_status replay_round(cpv_session* s, const std::array<int, 4>& key, bool* done)
{
    cpv_ctx* ctx = s->model->ctx;
    *done = false;
    if (s->warm_gen != ctx->ws_gen) {
        s->warm.clear();
        s->warm_gen = ctx->ws_gen;
    }
    auto same = [&](const int* k) { return std::equal(key.begin(), key.end(), k); };
    for (auto& g : s->graphs)
        if (same(g.key) && g.ws_gen == ctx->ws_gen) {
            CPV_HIP(ctx, hipGraphLaunch(g.exec, ctx->stream));
            g.used = ++s->clock;
            s->n_replayed++;
            *done = true;
            return CPV_OK;
        }
    if (std::find(s->unreplayable.begin(), s->unreplayable.end(), key) != s->unreplayable.end()) return CPV_OK;
    if (std::find(s->warm.begin(), s->warm.end(), key) == s->warm.end()) {
        s->warm.push_back(key);
        return CPV_OK;
    }
    // captured on a stream of its own (nothing runs while capturing), replayed on the caller's
    const uint64_t gen0 = ctx->ws_gen;
    const hipStream_t home = ctx->stream;
    if ((!ctx->cap_stream && hipStreamCreateWithFlags(&ctx->cap_stream, hipStreamNonBlocking) != hipSuccess) ||
        hipStreamBeginCapture(ctx->cap_stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        (void)hipGetLastError();
        s->unreplayable.push_back(key);
        return CPV_OK;
    }
    ctx->stream = ctx->cap_stream;
    s->eager_only = false;
    ctx->grow_refused = false;
    const cpv_status st = round_body(s, key[0], key[1], nullptr, false, 0);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->cap_stream, &graph);
    ctx->stream = home;
    hipGraphExec_t exec = nullptr;
    const bool ok = st == CPV_OK && e == hipSuccess && graph && !s->eager_only && ctx->ws_gen == gen0 &&
                    hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    if (!ok) {   // (nothing was launched: the round runs eagerly)
        if (ctx->grow_refused) {
            // a buffer had to grow: the eager round grows it, and the shape
            // is warmed again before its next capture
            ctx->grow_refused = false;
            s->warm.erase(std::remove(s->warm.begin(), s->warm.end(), key), s->warm.end());
        } else {
            s->unreplayable.push_back(key);
        }
        return CPV_OK;
    }
    constexpr size_t MAX_GRAPHS = 8;
    if (s->graphs.size() >= MAX_GRAPHS) {
        size_t lru = 0;
        for (size_t i = 1; i < s->graphs.size(); i++)
            if (s->graphs[i].used < s->graphs[lru].used) lru = i;
        CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));   // (it may still be running)
        (void)hipGraphExecDestroy(s->graphs[lru].exec);
        s->graphs.erase(s->graphs.begin() + (long)lru);
    }
    cpv_session::RoundGraph g;
    std::copy(key.begin(), key.end(), g.key);
    g.ws_gen = gen0;
    g.used = ++s->clock;
    g.exec = exec;
    s->graphs.push_back(g);
    CPV_HIP(ctx, hipGraphLaunch(exec, ctx->stream));
    s->n_captured++;
    s->n_replayed++;
    *done = true;
    return CPV_OK;
}

}  // namespace

extern "C" cpv_status cpv_verify_step_cands(cpv_session* s, const int32_t* tokens_dev, int t, int depth,
                                            const float* noise_dev, const int32_t* cands_host, int n_cand,
                                            cpv_round_out* out)
{
    if (!s || !tokens_dev || !out || t < 1 || t > s->max_batch || depth < 0 || depth > 16 || n_cand < 0 ||
        (n_cand > 0 && !cands_host))
        return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "verify_step: bad arguments");
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    const int64_t E = hp.n_embd, V = hp.n_vocab;
    if (n_cand > V) return cpv_fail(ctx, CPV_EINVAL, "verify_step: %d candidates for a vocabulary of %lld", n_cand,
                                    (long long)V);
    if (s->n_past + t > s->n_ctx) return cpv_fail(ctx, CPV_EINVAL, "verify_step: context overflow");  // qwen35.rs:1718-1720
    if (depth > 0 && !hp.has_mtp) return cpv_fail(ctx, CPV_EINVAL, "verify_step: model has no MTP head");
    const bool shortlist = depth > 0 && n_cand > 0;
    cpv_status st0;
    if (shortlist && (st0 = set_cands(s, cands_host, n_cand)) != CPV_OK) return st0;
    // the draft head's window is bounded; when it fills, it restarts (qwen35.rs:1730-1735)
    if (s->mtp_past + t > s->mtp_ctx) s->mtp_past = 0;
    cpv_status st;
    s->tap_off = 0;
    s->tree_base = -1;
    if ((st = set_pos_dev(s)) != CPV_OK) return st;
    CPV_HIP(ctx, hipMemcpyAsync(s->tok, tokens_dev, (size_t)t * 4, hipMemcpyDeviceToDevice, ctx->stream));
    // greedy rounds without a shortlist, a tap or the profiler replay a graph of their shape
    bool done = false;
    if (s->replay && !shortlist && !noise_dev && !s->tap && !ctx->prof) {
        const std::array<int, 4> key{t, depth, chunk_bucket(s->n_past + t), depth > 0 ? chunk_bucket(s->mtp_past + t) : 0};
        if ((st = replay_round(s, key, &done)) != CPV_OK) return st;
    }
    if (!done && (st = round_body(s, t, depth, noise_dev, shortlist, n_cand)) != CPV_OK) return st;
    s->n_past += t;
    out->n_past = s->n_past;
    out->preds_dev = s->preds;
    out->chain_dev = s->chain;
    out->conf_dev = s->conf;
    out->logits_dev = s->logits;
    out->hidden_dev = s->h;
    return CPV_OK;
}

// ---------------------------------------------------------------- draft trees
// A tree verify is step_verify over a draft tree rather than a chain: no
// counterpart in the reference, whose rounds verify a linear draft and rewind
// it (engine.rs:2533-2540).  Node i is written at KV row n_past + i, placed at
// position n_past + depth(i) and sees the context and its ancestors; a commit
// then keeps one root-to-node path as contiguous context rows.

namespace {

struct TreeSetup {
    int8_t parent[CPV_TREE_MAX], depth[CPV_TREE_MAX];
    int t;
};

// the host-checked tree, passed by value, into the session's device copy
__global__ void tree_setup_kernel(TreeSetup ts, int32_t* __restrict__ tree)
{
    const int i = threadIdx.x;
    if (i < ts.t) {
        tree[i] = ts.parent[i];
        tree[CPV_TREE_MAX + i] = ts.depth[i];
    }
}

struct CompactArgs {
    void* const* caches;       // K caches [n_layer], then V caches [n_layer] (limbs)
    int64_t base, v_stride;
    int n_layer, kpieces, width, n;   // kpieces: 16-byte pieces of a K row; width: h_kv * head_dim
    int h_kv;
    int8_t path[CPV_TREE_MAX];
};

// rows base + path[j] -> base + j of every trunk K cache (16-byte pieces of a
// row, then one KV head's exponents per thread) and columns likewise of every
// V cache (one limb of one column per thread).  Since
// path[j] >= j, writing row j never touches a source of a later j: each thread
// moves its slice in order, eight rows at a time (all eight read before any is
// written).
__global__ __launch_bounds__(256) void compact_kernel(CompactArgs a)
{
    const int layer = blockIdx.y;
    const int g = blockIdx.x * 256 + threadIdx.x, npiece = a.kpieces;
    if (g < npiece) {
        uint4* kc = (uint4*)a.caches[layer];
        for (int j0 = 0; j0 < a.n; j0 += 8) {
            uint4 v[8];
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (j0 + q < a.n) v[q] = kc[(a.base + a.path[j0 + q]) * npiece + g];
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (j0 + q < a.n) kc[(a.base + j0 + q) * npiece + g] = v[q];
        }
    } else if (g >= npiece + CPV_ATTN_VLIMBS * a.width) {
        const int kh = g - npiece - CPV_ATTN_VLIMBS * a.width;
        if (kh < a.h_kv) {
            int32_t* ke = (int32_t*)((int8_t*)a.caches[layer] + a.v_stride * (int64_t)npiece * 16) + kh * a.v_stride;
            for (int j0 = 0; j0 < a.n; j0 += 8) {
                int32_t v[8];
#pragma unroll
                for (int q = 0; q < 8; q++)
                    if (j0 + q < a.n) v[q] = ke[a.base + a.path[j0 + q]];
#pragma unroll
                for (int q = 0; q < 8; q++)
                    if (j0 + q < a.n) ke[a.base + j0 + q] = v[q];
            }
        }
    } else {
        const int vr = g - npiece, limb = vr / a.width, col = vr - limb * a.width;
        int8_t* vc = (int8_t*)a.caches[a.n_layer + layer] + 16 * limb;
        for (int j0 = 0; j0 < a.n; j0 += 8) {
            int8_t v[8];
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (j0 + q < a.n) v[q] = *v_limb_at(vc, col, a.v_stride, a.base + a.path[j0 + q]);
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (j0 + q < a.n) *v_limb_at(vc, col, a.v_stride, a.base + j0 + q) = v[q];
        }
    }
}

}  // namespace

extern "C" cpv_status cpv_verify_tree(cpv_session* s, const int32_t* tokens_dev, const int32_t* parent_host, int t,
                                      const float* noise_dev, cpv_round_out* out)
{
    if (!s || !tokens_dev || !parent_host || !out || t < 1 || t > CPV_TREE_MAX || t > s->max_batch)
        return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "verify_tree: bad arguments");
    cpv_model* m = s->model;
    cpv_ctx* ctx = m->ctx;
    const cpv_hparams& hp = m->hp;
    const int64_t V = hp.n_vocab;
    if (s->n_past + t > s->n_ctx) return cpv_fail(ctx, CPV_EINVAL, "verify_tree: context overflow");
    TreeSetup ts{};
    ts.t = t;
    for (int i = 0; i < t; i++) {
        const int p = parent_host[i];
        if (p < -1 || p >= i)
            return cpv_fail(ctx, CPV_EINVAL, "verify_tree: parent[%d] = %d (parents precede their children)", i, p);
        ts.parent[i] = (int8_t)p;
        ts.depth[i] = (int8_t)(p < 0 ? 0 : ts.depth[p] + 1);
    }
    s->tap_off = 0;
    s->tree_base = -1;
    cpv_status st;
    tree_setup_kernel<<<1, CPV_TREE_MAX, 0, ctx->stream>>>(ts, s->tree_dev);
    CPV_HIP(ctx, hipGetLastError());
    const Tree tree{s->tree_dev, s->tree_dev + CPV_TREE_MAX};
    if ((st = set_pos_dev(s)) != CPV_OK) return st;
    CPV_HIP(ctx, hipMemcpyAsync(s->tok, tokens_dev, (size_t)t * 4, hipMemcpyDeviceToDevice, ctx->stream));
    if ((st = cpv_get_rows(ctx, m->tok_embd, s->tok, t, s->x))) return st;
    cpv_gout pend{}, nxt{};
    for (int il = 0; il < hp.n_layer; il++) {
        if ((st = block(s, m->layers[il], s->x, t, s->n_past, s->n_past, s->n_past, s->kc[il], s->vt[il], s->v_stride,
                        true, pend.acc ? &pend : nullptr, SRC_ADD, &nxt, PosSel{0, 0}, &tree)))
            return st;
        pend = nxt;
    }
    cpv_gout hk;
    if ((st = norm_head(s, s->x, t, pend.acc ? &pend : nullptr, m->output_norm, s->h, m->output, s->logits, &hk)))
        return st;
    if ((st = cpv_argmax_peak_rows(ctx, s->logits, noise_dev, t, V, s->preds, nullptr, hk.acc ? &hk : nullptr)))
        return st;
    s->tree_parent.assign(parent_host, parent_host + t);
    s->tree_base = s->n_past;
    s->n_past += t;
    out->n_past = s->n_past;
    out->preds_dev = s->preds;
    out->chain_dev = s->chain;
    out->conf_dev = s->conf;
    out->logits_dev = s->logits;
    out->hidden_dev = s->h;
    return CPV_OK;
}

extern "C" cpv_status cpv_session_commit_branch(cpv_session* s, const int32_t* path_host, int n)
{
    if (!s || (n > 0 && !path_host) || n < 0)
        return cpv_fail(s ? s->model->ctx : nullptr, CPV_EINVAL, "commit_branch: bad arguments");
    cpv_ctx* ctx = s->model->ctx;
    const cpv_hparams& hp = s->model->hp;
    if (s->tree_base < 0) return cpv_fail(ctx, CPV_EINVAL, "commit_branch: no tree verify to commit");
    const int t = (int)s->tree_parent.size();
    if (n > t) return cpv_fail(ctx, CPV_EINVAL, "commit_branch: path of %d nodes in a tree of %d", n, t);
    CompactArgs a{};
    bool moved = false;
    for (int j = 0; j < n; j++) {
        const int v = path_host[j];
        if (v < 0 || v >= t || s->tree_parent[v] != (j == 0 ? -1 : path_host[j - 1]))
            return cpv_fail(ctx, CPV_EINVAL, "commit_branch: path[%d] = %d does not continue a root-to-node path", j, v);
        a.path[j] = (int8_t)v;
        moved |= v != j;
    }
    if (moved) {
        a.caches = s->caches_dev;
        a.base = s->tree_base;
        a.v_stride = s->v_stride;
        a.n_layer = hp.n_layer;
        a.kpieces = (int)(cpv_k_row_bytes((int)hp.n_head_kv, (int)hp.head_dim) / 16);
        a.width = (int)(hp.n_head_kv * hp.head_dim);
        a.h_kv = (int)hp.n_head_kv;
        a.n = n;
        const int threads = a.kpieces + CPV_ATTN_VLIMBS * a.width + a.h_kv;
        compact_kernel<<<dim3((unsigned)((threads + 255) / 256), (unsigned)hp.n_layer), 256, 0, ctx->stream>>>(a);
        CPV_HIP(ctx, hipGetLastError());
    }
    s->n_past = s->tree_base + n;
    s->tree_base = -1;
    return CPV_OK;
}
