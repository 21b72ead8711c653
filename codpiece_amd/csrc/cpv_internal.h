// cpv_internal.h — shared definitions of libcpv (HIP, gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <functional>
#include <string>
#include <vector>

#include "../../include/cpv.h"

struct cpv_ctx {
    int device = 0;
    int cu_count = 0;
    size_t lds_max = 0;       // shared memory per workgroup (bytes)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    hipStream_t cap_stream = nullptr;   // graph captures (the caller's stream may be the null stream)
    std::string err;
    // scratch owned by the context, grown on demand (never inside a capture)
    void* ws = nullptr;
    size_t ws_bytes = 0;
    uint64_t ws_gen = 0;      // bumped whenever ws (or the GEMM accumulator) is reallocated
    // the split-K GEMM accumulator [rows][n_pad] f64: zero between uses (each
    // finalize, and each fused consumer of a kept result, leaves it zero)
    double* gsum = nullptr;
    size_t gsum_bytes = 0;
    // partial results of the row reductions (argmax / softmax peak), grown on demand
    void* red = nullptr;
    size_t red_bytes = 0;
    // this device's address of the file-scope scratch of cpv_qgemm_noalloc
    void* scratch = nullptr;
    // set when a buffer was not grown because the stream was being captured
    bool grow_refused = false;
    // kernel timing (cpv_profile_start / _stop): event pairs around launches,
    // and each launch kept for cpv_profile_replay
    struct prof_rec { int cls, ev0, ev1; double bytes; };
    struct prof_launch { int cls; double bytes; uint64_t ws_gen; std::function<void()> go; };
    bool prof = false;
    std::vector<hipEvent_t> prof_ev;      // reused from one profile to the next
    std::vector<prof_rec> prof_recs;
    std::vector<prof_launch> prof_launches;
    size_t prof_used = 0;
};

// kernel timing: cpv_prof_mark records an event on the context's stream and
// returns its index (-1 when not profiling); cpv_prof_add closes a launch of
// class `cls` that moved `bytes` algorithmic bytes, opened by mark `ev0`
int  cpv_prof_mark(cpv_ctx* ctx);
void cpv_prof_add(cpv_ctx* ctx, int ev0, int cls, double bytes);
// keep a launch (its kernel and arguments) for cpv_profile_replay
void cpv_prof_keep(cpv_ctx* ctx, int cls, double bytes, std::function<void()> go);

struct cpv_weight {
    cpv_ctx* ctx = nullptr;
    int type = 0;
    int64_t n = 0, k = 0;     // logical rows and row length
    int64_t n_pad = 0;        // rows padded to the 64-row tiles of the GEMM
    int64_t units = 0;        // 256-element units per row (a super-block, or 8 Q8_0 blocks)
    void* data = nullptr;     // repacked tiles, layout per type (api.hip)
    size_t data_bytes = 0;
    int32_t* ew = nullptr;    // [n_pad] frexp exponent of the row's largest scale
};

// rows[0..n) (device, each < src->n) of a repacked weight as a new weight
cpv_status cpv_weight_gather(cpv_ctx* ctx, const cpv_weight* src, const int32_t* rows_dev, int64_t n,
                             cpv_weight** out);

// error helpers: record a message on the context and return the status
cpv_status cpv_fail(cpv_ctx* ctx, cpv_status st, const char* fmt, ...);
cpv_status cpv_hip_fail(cpv_ctx* ctx, hipError_t e, const char* what);

#define CPV_HIP(ctx, expr)                                             \
    do {                                                               \
        hipError_t e_ = (expr);                                        \
        if (e_ != hipSuccess) return cpv_hip_fail((ctx), e_, #expr);   \
    } while (0)

// look up this device's address of cpv_qgemm_noalloc's scratch (once per
// device; ctx->device must be current)
cpv_status cpv_noalloc_setup(cpv_ctx* ctx);

// grow the context workspace to at least `bytes` (synchronises the stream
// before freeing an old buffer the queued work may still use)
cpv_status cpv_workspace(cpv_ctx* ctx, size_t bytes, void** out);

// Whether ctx->stream is being captured into a graph.  A buffer that would
// have to grow then is not grown (a capture may record no synchronisation,
// allocation or memset): the call fails with CPV_EUNSUPPORTED and sets
// ctx->grow_refused, and a round being captured runs eagerly instead.
bool cpv_capturing(cpv_ctx* ctx);
cpv_status cpv_refuse_growth(cpv_ctx* ctx, const char* what, size_t bytes);

// bytes per block / elements per block of a GGUF type
int64_t cpv_type_block(int type);
int64_t cpv_type_size(int type);

// sentinel exponent of an all-zero scale set
constexpr int CPV_E_EMPTY = -100000;

// exact-window constants shared by the launcher and the kernels
int cpv_qgemm_window(int type, int64_t k);

// IEEE binary16 <-> binary32 (exact / round-to-nearest-even).  The narrowing
// is done on the bits: a plain (_Float16) conversion lets the compiler fuse a
// preceding f32 multiply or add into one v_fma_mix (a single rounding to f16
// instead of f32 then f16), which differs at f32 ties.
__host__ __device__ __forceinline__ float cpv_h2f(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}
// f32 -> f16, round to nearest even (subnormals kept, overflow to inf), NaN
// as the quiet NaN 0x7e00 with the input's sign: v_cvt_f16_f32 under the
// default mode, which equals the bit-level rounding rule for every f32 input
// but NaN payloads (compared over all 2^32 inputs on gfx950).  The empty asm
// keeps the compiler from folding a product into the conversion
// (v_mad_mixlo_f16 rounds a * b once, where the contract rounds it to f32
// first).
__device__ __forceinline__ uint16_t cpv_f2h(float f)
{
    asm volatile("" : "+v"(f));
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    return (x & 0x7fffffffu) > 0x7f800000u ? (uint16_t)(((x >> 16) & 0x8000u) | 0x7e00u) : h;
}

// 2^(i/32) in binary64, stored minus i << 47
#define CPV_EXP2F_TAB { \
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull }

// expf evaluated as glibc (>= 2.27) evaluates it, which is the libm expf the
// reference's Rust f32::exp calls: k = round(x * 32/ln2), e^x = 2^(k/32) * p(r)
// with a 32-entry table of 2^(i/32) (stored minus i<<47) and the published
// cubic, in binary64 with fused multiply-adds, rounded once to f32.  Used
// wherever the reference applies exp on the verify path (sigmoid, SiLU, the
// sampler), so results match the CPU bit for bit.  cpv_expf_t takes the table
// from the caller (a copy in LDS keeps global loads out of a kernel's phase).
__host__ __device__ __forceinline__ float cpv_expf_core(float x, const uint64_t* tab)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __builtin_bit_cast(double, tab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}
__host__ __device__ __forceinline__ float cpv_expf_t(float x, const uint64_t* tab)
{
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_huge_valf();
    if (x < -0x1.9fe368p6f) return 0.0f;
    return cpv_expf_core(x, tab);
}
// the same values with no branches: the main path on x clamped to its range
// (NaN to the low end), kept there by an empty asm statement the compiler
// cannot sink into a branch, then the special cases selected
__device__ __forceinline__ float cpv_expf_sel(float x, const uint64_t* tab)
{
    constexpr float lo = -0x1.9fe368p6f, hi = 0x1.62e42ep6f;
    float y = cpv_expf_core(fminf(fmaxf(x, lo), hi), tab);
    __asm__ volatile("" : "+v"(y));
    return x != x ? x + x : x > hi ? __builtin_huge_valf() : x < lo ? 0.0f : y;
}
__host__ __device__ __forceinline__ float cpv_expf(float x)
{
    constexpr uint64_t tab[32] = CPV_EXP2F_TAB;
    return cpv_expf_t(x, tab);
}

// ---- reductions across lanes through DPP row permutations (no LDS round
// trip, unlike a shuffle).  Every lane of the wave must be active.  The
// operations used with them (max, integer sums, a strict total order) give
// the same result in any order.
//   XOR1 = quad_perm [1,0,3,2], XOR2 = quad_perm [2,3,0,1]: lane ^ 1, lane ^ 2;
//   HMIRROR = row_half_mirror (i <-> 7 - i in 8 lanes), MIRROR = row_mirror
//   (i <-> 15 - i in 16): once the quads (eights) agree on a value, each pairs
//   them with the other quad (eight) of the group.
enum { CPV_DPP_XOR1 = 0xb1, CPV_DPP_XOR2 = 0x4e, CPV_DPP_MIRROR = 0x140, CPV_DPP_HMIRROR = 0x141 };

template <int C>
__device__ __forceinline__ int cpv_dpp(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, C, 0xf, 0xf, false);
}
template <int C>
__device__ __forceinline__ float cpv_dpp(float v)
{
    return __builtin_bit_cast(float, cpv_dpp<C>(__builtin_bit_cast(int, v)));
}
template <int C>
__device__ __forceinline__ long long cpv_dpp(long long v)
{
    const int lo = cpv_dpp<C>((int)(uint32_t)v), hi = cpv_dpp<C>((int)(v >> 32));
    return (long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
template <int C>
__device__ __forceinline__ unsigned long long cpv_dpp(unsigned long long v)
{
    return (unsigned long long)cpv_dpp<C>((long long)v);
}
__device__ __forceinline__ int cpv_readlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float cpv_readlane(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ long long cpv_readlane(long long v, int l)
{
    const int lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l), hi = __builtin_amdgcn_readlane((int)(v >> 32), l);
    return (long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ unsigned long long cpv_readlane(unsigned long long v, int l)
{
    return (unsigned long long)cpv_readlane((long long)v, l);
}

// op over each group of N consecutive lanes (N = 2, 4, 8, 16), in every lane of the group
template <int N, class T, class Op>
__device__ __forceinline__ T cpv_group_reduce(T v, Op op)
{
    static_assert(N == 2 || N == 4 || N == 8 || N == 16, "group of 2, 4, 8 or 16 lanes");
    v = op(v, cpv_dpp<CPV_DPP_XOR1>(v));
    if constexpr (N >= 4) v = op(v, cpv_dpp<CPV_DPP_XOR2>(v));
    if constexpr (N >= 8) v = op(v, cpv_dpp<CPV_DPP_HMIRROR>(v));
    if constexpr (N >= 16) v = op(v, cpv_dpp<CPV_DPP_MIRROR>(v));
    return v;
}
// op over the whole wave (a wave-uniform value)
template <class T, class Op>
__device__ __forceinline__ T cpv_wave_reduce(T v, Op op)
{
    v = cpv_group_reduce<16>(v, op);
    return op(op(cpv_readlane(v, 0), cpv_readlane(v, 16)), op(cpv_readlane(v, 32), cpv_readlane(v, 48)));
}
struct cpv_op_max { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct cpv_op_umax {
    __device__ unsigned long long operator()(unsigned long long a, unsigned long long b) const { return a > b ? a : b; }
};
struct cpv_op_add { template <class T> __device__ T operator()(T a, T b) const { return a + b; } };

// the signed element of largest magnitude over the wave, the lowest index
// among equal magnitudes (a strict order, so any reduction order agrees);
// every lane ends with it
__device__ __forceinline__ void cpv_amax_take(float& ax, int& ix, float& sx, float oa, int oi, float os)
{
    if (oa > ax || (oa == ax && oi < ix)) {
        ax = oa;
        ix = oi;
        sx = os;
    }
}
template <int C>
__device__ __forceinline__ void cpv_amax_dpp(float& ax, int& ix, float& sx)
{
    cpv_amax_take(ax, ix, sx, cpv_dpp<C>(ax), cpv_dpp<C>(ix), cpv_dpp<C>(sx));
}
__device__ __forceinline__ void cpv_wave_amax(float& ax, int& ix, float& sx)
{
    cpv_amax_dpp<CPV_DPP_XOR1>(ax, ix, sx);
    cpv_amax_dpp<CPV_DPP_XOR2>(ax, ix, sx);
    cpv_amax_dpp<CPV_DPP_HMIRROR>(ax, ix, sx);
    cpv_amax_dpp<CPV_DPP_MIRROR>(ax, ix, sx);
    float a0 = cpv_readlane(ax, 0), s0 = cpv_readlane(sx, 0);
    int i0 = cpv_readlane(ix, 0);
#pragma unroll
    for (int l = 16; l < 64; l += 16) cpv_amax_take(a0, i0, s0, cpv_readlane(ax, l), cpv_readlane(ix, l), cpv_readlane(sx, l));
    ax = a0;
    ix = i0;
    sx = s0;
}

// quantized activations shared by every GEMM that reads the same input
struct cpv_act {
    const int8_t* qa;        // [m][U*256] codes
    const float* da;         // [m][U] (Q8_K) or [m][U*8] (Q8_0) scales
    const int32_t* bs32;     // [m][U*8] 32-code sums (Q8_K)
    const int32_t* bs16;     // [m][U*16] 16-code sums (Q8_K)
    int64_t m, k;
    int U;
    bool kq;                 // Q8_K (for Q4_K / Q6_K weights) or Q8_0
};
size_t cpv_act_bytes(int type, int64_t k, int64_t m);
// the cpv_act views of buf for m rows of length k (no work launched)
void cpv_act_layout(int type, int64_t m, int64_t k, void* buf, cpv_act* out);
cpv_status cpv_quant_act(cpv_ctx* ctx, int type, const float* x, int64_t m, int64_t k, void* buf, cpv_act* out);
cpv_status cpv_qgemm_act(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, float* y);

// The GEMMs for many activation rows (qgemm_wide.hip): the same accumulator
// sums as cpv_qgemm_act's skinny kernels, on the 16x16x32 int8 MFMA, for all
// act->m rows in one launch; cpv_qgemm_act takes them above 16 rows for
// Q4_K and above 8 for Q6_K and Q8_0 (cpv_qgemm_wide_ok).
bool cpv_qgemm_wide_ok(const cpv_weight* w, int64_t m);
cpv_status cpv_qgemm_wide(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, double* gsum, int win);

// A GEMM result kept in the accumulator for a fused consumer: row m, output n
// is cpv_gout_value(acc[m * n_pad + n], ew[n], Ea(m), win) with Ea(m) the
// frexp exponent of max |da[m][0..nda)|; the consumer reads each entry once
// and writes it back to zero.
struct cpv_gout {
    double* acc;
    int64_t n_pad, n;
    const int32_t* ew;
    const float* da;
    int nda, win;
};
cpv_status cpv_qgemm_keep(cpv_ctx* ctx, const cpv_weight* w, const cpv_act* act, cpv_gout* out);

// floor(sq * 2^-g) for a non-negative finite f32 sq, as an integer: sq is its
// 24-bit mantissa times a power of two, so the floor is a shift (the same value
// as floor(ldexp((double)sq, -g)), without binary64 arithmetic).  Callers keep
// the result below 2^63.
__host__ __device__ __forceinline__ long long cpv_fixed_floor(float sq, int g)
{
    const uint32_t b = __builtin_bit_cast(uint32_t, sq);
    const uint32_t be = b >> 23;
    const long long mant = (long long)((b & 0x7fffffu) | (be ? 0x800000u : 0u));
    const int sh = (int)(be ? be : 1u) - 150 - g;           // sq = mant * 2^(sh + g)
    // one of the two shifts is zero; no branch (a right shift by 24 or more clears mant)
    const int ls = sh > 0 ? (sh < 63 ? sh : 63) : 0;
    const int rs = sh < 0 ? (-sh < 63 ? -sh : 63) : 0;
    return (mant << ls) >> rs;
}

__host__ __device__ __forceinline__ int cpv_exp_of_max(float mx)
{
    int e = CPV_E_EMPTY;
    if (mx > 0.0f) frexpf(mx, &e);
    return e;
}
__host__ __device__ __forceinline__ float cpv_gout_value(double S, int ew, int ea, int win)
{
    return (ew == CPV_E_EMPTY || ea == CPV_E_EMPTY) ? 0.0f : (float)ldexp(S, ew + ea - win);
}

// rows of several weights stacked into a new weight (same type and k, every
// part but the last in whole 64-row tiles)
cpv_status cpv_weight_concat(cpv_ctx* ctx, cpv_weight* const* parts, int np, cpv_weight** out);

// Row argmax (first maximum, as cpv_argmax_rows) and, when peak_out is not
// null, the softmax peak expf(0) * (float)(1 / sum_i expf(x_i - max)) of each
// row (the sum in binary64), in two passes over 64 slices per row.  With
// kept, the rows are first finalized from that kept GEMM result (n = kept->n)
// into x, in the first pass.
// With emb, the pass that stores idx_out also stores emb_out[r] = row
// idx_out[r] of that embedding table, as cpv_get_rows would.  With fin and
// peak_out, the peak's last pass is left to the kernel that consumes it: fin
// receives the peak's slice sums [rows][CPV_AM_NB] (cpv_peak_of's order),
// valid until the next argmax call on the context.
struct cpv_am_fin {
    const double* psum;
};
cpv_status cpv_argmax_peak_rows(cpv_ctx* ctx, const float* x, const float* noise, int64_t rows, int64_t n,
                                int32_t* idx_out, float* peak_out, const cpv_gout* kept = nullptr,
                                cpv_am_fin* fin = nullptr, const cpv_weight* emb = nullptr, float* emb_out = nullptr);
constexpr int CPV_AM_NB = 64;   // slices per row of the argmax and peak passes
// a row's argmax from its slice keys: key = (order-preserving value bits) << 32
// | (2^32 - 1 - index), 0 for a slice with no value above -inf; no winner gives 0
__device__ __forceinline__ int32_t cpv_am_index(unsigned long long best)
{
    return best ? (int32_t)(0xffffffffu - (uint32_t)best) : 0;
}
// the softmax peak from a row's slice sums, added in slice order
__device__ __forceinline__ float cpv_peak_of(const double* psum_row)
{
    double tot = 0.0;
    for (int b = 0; b < CPV_AM_NB; b++) tot += psum_row[b];
    return 1.0f * (float)(1.0 / tot);
}

// elements e .. e+3 (e a multiple of 4) of weight row `row` (0 <= row < n),
// dequantized from the repacked layout (64-row tiles of U units, PIECES KiB
// per tile and unit, a row's 16 bytes per KiB; Q6_K's f16 scales after the
// tiles) with ggml's f32 formulas:
//   Q8_0: q * d;  Q4_K: (d*sc)*q - (dmin*m);  Q6_K: d*sc*q, left to right.
// The four codes of each kind sit in one dword of a 16-byte piece.
template <int TYPE>
__device__ __forceinline__ void cpv_dequant4(const uint8_t* data, int64_t n, int64_t U, int64_t row, int64_t e,
                                             float* out)
{
    constexpr int PIECES = TYPE == CPV_Q4_K ? 9 : TYPE == CPV_Q6_K ? 13 : 17;
    const int64_t t = row / 64, u = e / 256;
    const int lane = (int)(row % 64), el = (int)(e % 256);
    const uint8_t* slab = data + (t * U + u) * PIECES * 1024 + lane * 16;
    // the dword holding block bytes idx .. idx+3 of the piece run
    auto dword_at = [&](int idx) { return *(const uint32_t*)(slab + (idx / 16) * 1024 + idx % 16); };
    if constexpr (TYPE == CPV_Q4_K) {
        const uint4 meta = *(const uint4*)(slab + 8 * 1024);   // d, dmin, then 12 bytes of scales and mins
        const uint32_t sw[3] = {meta.y, meta.z, meta.w};
        auto s = [&](int i) { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
        const int j = el / 32, l = el % 32;
        const uint32_t codes = dword_at((j / 2) * 32 + l);
        int sc, m;
        if (j < 4) {
            sc = s(j) & 63;
            m = s(j + 4) & 63;
        } else {
            sc = (s(j + 4) & 0xF) | ((s(j - 4) >> 6) << 4);
            m = (s(j + 4) >> 4) | ((s(j) >> 6) << 4);
        }
        const float d = cpv_h2f((uint16_t)(meta.x & 0xffffu));
        const float dm = cpv_h2f((uint16_t)(meta.x >> 16));
        const float d1 = d * (float)sc, m1 = dm * (float)m;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t byte = (codes >> (8 * k)) & 0xffu;
            const int code = (j & 1) ? (int)(byte >> 4) : (int)(byte & 15);
            out[k] = d1 * (float)code - m1;
        }
    } else if constexpr (TYPE == CPV_Q6_K) {
        const int h = el / 128, l = el % 128, l32 = l % 32, quad = l / 32;
        const uint32_t ql = dword_at(h * 64 + l32 + (quad & 1) * 32);
        const uint32_t qh = dword_at(128 + h * 32 + l32);
        const int8_t sc = (int8_t)slab[((192 + el / 16) / 16) * 1024 + (192 + el / 16) % 16];
        const float d = cpv_h2f(*(const uint16_t*)(data + ((n + 63) / 64) * U * 13 * 1024 + ((t * U + u) * 64 + lane) * 2));
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t qlb = (ql >> (8 * k)) & 0xffu, qhb = (qh >> (8 * k)) & 0xffu;
            const int lo = (quad < 2) ? (int)(qlb & 15) : (int)(qlb >> 4);
            const int code = (lo | (int)(((qhb >> (2 * quad)) & 3) << 4)) - 32;
            out[k] = d * (float)sc * (float)code;
        }
    } else {
        const uint32_t codes = dword_at(el);
        const float d = cpv_h2f(*(const uint16_t*)(slab + 16 * 1024 + (el / 32) * 2));
#pragma unroll
        for (int k = 0; k < 4; k++) out[k] = (float)(int8_t)((codes >> (8 * k)) & 0xffu) * d;
    }
}
// the same for a weight type known at run time (CPV_Q8_0, CPV_Q4_K or CPV_Q6_K)
__device__ __forceinline__ void cpv_dequant4_t(int type, const uint8_t* data, int64_t n, int64_t U, int64_t row,
                                               int64_t e, float* out)
{
    if (type == CPV_Q4_K) cpv_dequant4<CPV_Q4_K>(data, n, U, row, e, out);
    else if (type == CPV_Q6_K) cpv_dequant4<CPV_Q6_K>(data, n, U, row, e, out);
    else cpv_dequant4<CPV_Q8_0>(data, n, U, row, e, out);
}

// Row argmax (first maximum) and the re-draft gate of each row: keep_out[r] =
// 0 when p_min > 0 and 1 / lse < p_min, else 1, with lse the index-order f32
// sum of expf(x_i - max) (engine.rs:2598-2606), decided exactly: a binary64
// bound pass settles rows whose 1 / lse is clear of p_min by more than the f32
// sum's rounding can move it, and the others run the sequential fold.  keep_out
// may be null when p_min <= 0.  With kept, as cpv_argmax_peak_rows.
cpv_status cpv_argmax_gate_rows(cpv_ctx* ctx, const float* x, int64_t rows, int64_t n, int32_t* idx_out, float p_min,
                                int32_t* keep_out, const cpv_gout* kept = nullptr);
// the gate's decision from the bound pass's pairs sw [rows][nb][2] (sw null:
// every row keeps), the argmax idx giving each row's max (sample.hip)
cpv_status cpv_gate_fin_launch(cpv_ctx* ctx, const float* x, int64_t rows, int64_t n, const int32_t* idx,
                               const double* sw, int nb, float p_min, int32_t* keep_out);

// internal launchers
cpv_status cpv_repack_launch(cpv_ctx* ctx, cpv_weight* w, const void* aos_dev);
// the V cache of a session as limbs: vq = rint(f16(v) 2^CPV_ATTN_VBITS)
// (|vq| < 2^30) as CPV_ATTN_VLIMBS signed 8-bit limbs, laid out
// [Hkv*D][v_stride / 16][limb][16 rows] (v_stride a multiple of 16): the
// limbs of 16 consecutive rows of one column are 64 contiguous bytes, which
// attention's P V reads straight into the int8 MFMA
constexpr int CPV_ATTN_VBITS = 14;
constexpr int CPV_ATTN_VLIMBS = 4;

// the K cache of a session as limbs: per row and KV head, each f16 value kf
// as the 15-bit fixed point rint(kf 2^(14 - e)), e the frexp exponent of the
// head's largest |kf| (CPV_E_EMPTY for an all-zero head), split into two
// signed 8-bit limbs f = 256 hi + lo (lo in [-128, 127]): d hi bytes, then d
// lo bytes per head, rows of cpv_k_row_bytes; then, after v_stride rows (the
// V cache's stride, at least the row count), the exponents as an int32 plane
// [h_kv][v_stride], so that a chunk's exponents of one head are contiguous.
// Attention's scores take the limbs straight into the int8 MFMA.
__host__ __device__ __forceinline__ int64_t cpv_k_row_bytes(int h_kv, int d)
{
    return (int64_t)h_kv * 2 * d;
}
__host__ __device__ __forceinline__ int64_t cpv_k_cache_bytes(int h_kv, int d, int64_t v_stride)
{
    return v_stride * cpv_k_row_bytes(h_kv, d) + (int64_t)h_kv * v_stride * 4;
}
template <class T>
__host__ __device__ __forceinline__ T* cpv_k_exps(T* kc, int h_kv, int d, int64_t v_stride)
{
    return (T*)((int8_t*)kc + v_stride * cpv_k_row_bytes(h_kv, d));
}
__device__ __forceinline__ int cpv_k_fixed(float kf, int e)
{
    return e != CPV_E_EMPTY ? (int)rintf(ldexpf(kf, 14 - e)) : 0;
}
__device__ __forceinline__ void cpv_k_limbs(float kf, int e, int8_t* hi, int8_t* lo)
{
    const int f = cpv_k_fixed(kf, e);
    const int h = (f + 128) >> 8;
    *hi = (int8_t)h;
    *lo = (int8_t)(f - 256 * h);
}

// attention over the API's caches (kc f16 [n_ctx][h_kv*d], vt f16 transposed)
// or a session's (vl and kl set: the limb caches above; kc and vt unused)
cpv_status cpv_attn_launch(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                           int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                           float* out, const int8_t* vl = nullptr, const int8_t* kl = nullptr);
cpv_status cpv_qgemm_launch(cpv_ctx* ctx, const cpv_weight* w, const float* x, int64_t m, float* y);

// the attention's chunk partials for a consumer that folds them itself (chains
// only, when t tokens run as one block; else CPV_EUNSUPPORTED, nothing launched):
// P [nchunk][rows][d] f32, mc [nchunk][rows] f32, zc [nchunk][rows] int64 in
// the context workspace, rows = t * h, row = token * h + head
struct cpv_attn_part {
    const float* P;
    const float* mc;
    const long long* zc;
    int nchunk, rows;
    int zbits;            // zc holds Z_c 2^zbits
    const int64_t* pos;   // when set, the chunks in play are ceil((pos[pos_sel] + t) / 128)
    int pos_sel, t;       // (device memory; nchunk is then the grid's, an upper bound)
};
// o = fmaf(p[c * cs], f[c], o) for c = 0 .. n-1 in order from +0 (the
// attention's fold over its chunk partials, n >= 1): each batch of loads goes
// out, at clamped in-bounds indexes and without a branch, one batch ahead of
// the chain that consumes it
// (from chunk c0 on, after the fold o of the chunks before it)
template <int B = 16>
__device__ __forceinline__ float cpv_fold_chain_from(const float* p, int64_t cs, const float* f, int n, int c0,
                                                     float o)
{
    float cur[B];
#pragma unroll
    for (int i = 0; i < B; i++) cur[i] = p[(int64_t)(c0 + i < n ? c0 + i : n - 1) * cs];
    int c = c0;
    for (; c + B <= n; c += B) {
        float nxt[B];
#pragma unroll
        for (int i = 0; i < B; i++) {
            const int k = c + B + i;
            nxt[i] = p[(int64_t)(k < n ? k : n - 1) * cs];
        }
#pragma unroll
        for (int i = 0; i < B; i++) o = fmaf(cur[i], f[c + i], o);
#pragma unroll
        for (int i = 0; i < B; i++) cur[i] = nxt[i];
    }
#pragma unroll
    for (int i = 0; i < B; i++)
        if (c + i < n) o = fmaf(cur[i], f[c + i], o);
    return o;
}
template <int B = 16>
__device__ __forceinline__ float cpv_fold_chain(const float* p, int64_t cs, const float* f, int n)
{
    return cpv_fold_chain_from<B>(p, cs, f, n, 0, 0.0f);
}
cpv_status cpv_attn_partials(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                             int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                             cpv_attn_part* part, const int64_t* pos = nullptr, int pos_sel = 0,
                             int nchunk_grid = 0, int64_t kv_rows = 0, const int8_t* vl = nullptr,
                             const int8_t* kl = nullptr);
