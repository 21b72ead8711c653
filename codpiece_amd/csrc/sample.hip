// sample.hip — target distributions and speculative acceptance on the device.
//
// The reference builds each target distribution on the host
// (Sampler::build, crates/codpiece-sample/src/lib.rs:229-376) with f32
// arithmetic whose sums are sequential folds in candidate order, and decides
// a round with Dist::{prob_of, draw, draw_excluding} (:387-436) in the engine
// loop (crates/codpiece-server/src/engine.rs:2326-2461).  Here one 1024-thread
// workgroup builds the distribution of one verified row and a second kernel,
// one workgroup per sequence, walks the drafts.  Results equal the CPU
// sampler bit for bit:
//
//  * Sequential f32 sums without a sequential loop.  While a running sum s
//    stays inside one binade [2^E, 2^(E+1)) every float there is a multiple
//    of u = ulp(s), so fl(s + x) = s + u*round(x/u), where round is to
//    nearest and a tie goes to the even multiple: the step depends on s only
//    through the parity of s/u.  Each element is therefore a map on integers
//    S -> S + d[S & 1], the maps compose associatively, and a block scan of
//    them gives every prefix of the fold exactly.  The first element whose
//    prefix would leave the binade is added in hardware f32 and the scan
//    resumes from there in the new binade; sums of non-negative terms only
//    climb, so there are at most ~40 such restarts.
//  * Candidate order (logit descending, id ascending; cmp_desc, lib.rs:
//    453-459) as a stream of sorted bands: a radix histogram over the 64-bit
//    key (order-flipped logit bits, id) picks the next <= 16384 keys, which
//    are gathered, packed into 50 bits (key << 18 | id) and radix-sorted in
//    LDS by rocPRIM's block sort.  Only as much of the order as the filter
//    needs is produced.
//  * exp is the glibc expf restatement (cpv_expf); divisions are IEEE; the
//    library is built without contraction, so every a*b+c rounds twice as
//    in the Rust source.
#include "cpv_internal.h"

#include <float.h>
#include <math.h>

#include <rocprim/block/block_radix_sort.hpp>

namespace {

constexpr int SB = 1024;               // threads per sampler workgroup
constexpr int SWV = SB / 64;           // waves per workgroup
constexpr int FIPT = 8;                // fold: elements per thread per window
constexpr int BU = 8;                  // strided loops: loads issued ahead of their uses
constexpr uint32_t FTOP = 1u << 24;    // fold: ulps from 0 to the top of a binade
constexpr uint32_t FSAT = 1u << 26;    // fold: saturation of a composed step
constexpr int FOLD_SEQ = 1024;         // folds: leading elements added by one thread
constexpr int BAND = 16384;            // sorted band held in LDS as u64 keys
constexpr int HIST_MAX = 4096;         // penalty window input limit (4 per thread)
constexpr int VMAX = 262144;           // ids fit the low 18 bits of a key
// a band in candidate order: a block radix sort of 16 keys per thread, each
// key (desc_key, id) packed into 50 bits, 5 bits per pass with match ranking
// (377 µs per B = 1 acceptance call against 391 with rocPRIM's default 8);
// its storage overlays the key buffer.  Bands of up to SMALL_BAND keys sort
// with 4 keys per thread.
using band_sort_t = rocprim::block_radix_sort<unsigned long long, SB, BAND / SB, rocprim::empty_type, 1, 1, 5,
                                              rocprim::block_radix_rank_algorithm::match>;
constexpr int SMALL_BAND = 4096;
using small_sort_t = rocprim::block_radix_sort<unsigned long long, SB, SMALL_BAND / SB>;
constexpr int KEY_BITS = 50;
// a first band split at histogram-bin boundaries into parts that workgroups
// of their own sort: bin b (keys from offset o_b of the band on) joins part
// o_b / PSPAN, so a part spans at most PSPAN keys plus its last bin, and
// holds at most SMALL_BAND keys while no bin exceeds PSPAN
constexpr int PSPAN = 2048;
constexpr int MAXP = BAND / PSPAN;
constexpr size_t SAMPLE_LDS_KEYS =
    (((size_t)BAND * 8 > sizeof(band_sort_t::storage_type) ? (size_t)BAND * 8 : sizeof(band_sort_t::storage_type)) +
     255) & ~(size_t)255;
static_assert(sizeof(small_sort_t::storage_type) <= SAMPLE_LDS_KEYS, "the small sort fits the key buffer");
// band_part_kernel's key buffer: one part (two workgroups share a CU)
constexpr size_t PART_LDS_KEYS =
    (((size_t)SMALL_BAND * 8 > sizeof(small_sort_t::storage_type) ? (size_t)SMALL_BAND * 8
                                                                   : sizeof(small_sort_t::storage_type)) +
     255) & ~(size_t)255;

// ------------------------------------------------------------ block scratch
struct FMap { uint32_t d0, d1; };      // S -> S + (S even ? d0 : d1)

struct Small {
    FMap wtot[SWV];
    unsigned long long slot[2][2];     // per pass: first binade exit, first predicate hit
    uint32_t scan[SWV];
    float wf[SWV];
    int wi[SWV];
    int iv[8];
    unsigned long long last;           // the last key of a band
    int poff[8], pend[8], pfill[8];    // a partitioned band: each part's offset, end and fill
    float pf1[8], pf2[8];              // each part's estimated sums of exp(l - max) and exp((l - max) / T)
    unsigned long long wmax[SWV], wmin[SWV];
};

// for (i = tid; i < n; i += SB) use(i, load(i)), with BU loads in flight:
// every load of a batch is issued (at a clamped index) before the first use
template <class L, class U>
__device__ __forceinline__ void strided(int n, L load, U use)
{
    for (int i0 = threadIdx.x; i0 < n; i0 += SB * BU) {
        decltype(load(0)) v[BU];
#pragma unroll
        for (int q = 0; q < BU; q++) {
            const int i = i0 + q * SB;
            v[q] = load(i < n ? i : n - 1);
        }
#pragma unroll
        for (int q = 0; q < BU; q++) {
            const int i = i0 + q * SB;
            if (i < n) use(i, v[q]);
        }
    }
}

// use(i, x[i]) for every i < n in some order, for a row x of floats: 16-byte
// loads, BU of them in flight per thread (4x the bytes of strided, for the
// latency-bound passes over a whole vocabulary row); rows that are not
// 16-byte aligned, or whose length is not a multiple of 4, take strided
template <class U>
__device__ __forceinline__ void row_pass(const float* x, int n, U use)
{
    if ((n & 3) || ((uintptr_t)x & 15)) {
        strided(n, [&](int i) { return x[i]; }, use);
        return;
    }
    const int n4 = n >> 2;
    const float4* x4 = (const float4*)x;
    for (int j0 = threadIdx.x; j0 < n4; j0 += SB * BU) {
        float4 v[BU];
#pragma unroll
        for (int q = 0; q < BU; q++) {
            const int j = j0 + q * SB;
            v[q] = x4[j < n4 ? j : n4 - 1];
        }
#pragma unroll
        for (int q = 0; q < BU; q++) {
            const int j = j0 + q * SB;
            if (j < n4) {
                use(4 * j, v[q].x);
                use(4 * j + 1, v[q].y);
                use(4 * j + 2, v[q].z);
                use(4 * j + 3, v[q].w);
            }
        }
    }
}

// the step of m for an S of parity par (arithmetic select: a ?: on the two
// fields lets the compiler address a register array by parity)
__device__ __forceinline__ uint32_t fsel(FMap m, uint32_t par)
{
    return m.d0 ^ ((m.d0 ^ m.d1) & (0u - (par & 1u)));
}

// f then g
__device__ __forceinline__ FMap fcomp(FMap f, FMap g)
{
    const uint32_t a = f.d0 + fsel(g, f.d0);
    const uint32_t b = f.d1 + fsel(g, f.d1 + 1u);
    return {a < FSAT ? a : FSAT, b < FSAT ? b : FSAT};
}

// Scans through DPP (no LDS round trip): row_shr:1,2,4,8 within each row of 16
// lanes, then row_bcast:15 (rows 1 and 3 take the last lane of the row before)
// and row_bcast:31 (rows 2 and 3 take lane 31).  A lane without a source keeps
// `old` = the identity, and every step combines the earlier lanes' value
// first, so a non-commutative composition scans in lane order.
template <int C, int RM>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, C, RM, 0xf, false);
}
template <int C, int RM>
__device__ __forceinline__ FMap dpp_map(FMap f)
{
    return {dpp_u32<C, RM>(f.d0), dpp_u32<C, RM>(f.d1)};
}
// inclusive scan of the wave's maps (lane i: lanes 0..i composed in order)
__device__ __forceinline__ FMap wave_scan_maps(FMap v)
{
    v = fcomp(dpp_map<0x111, 0xf>(v), v);
    v = fcomp(dpp_map<0x112, 0xf>(v), v);
    v = fcomp(dpp_map<0x114, 0xf>(v), v);
    v = fcomp(dpp_map<0x118, 0xf>(v), v);
    v = fcomp(dpp_map<0x142, 0xa>(v), v);
    v = fcomp(dpp_map<0x143, 0xc>(v), v);
    return v;
}
// inclusive scan of the first 16 lanes (the lanes past them are not used)
__device__ __forceinline__ FMap row_scan_maps(FMap v)
{
    v = fcomp(dpp_map<0x111, 0xf>(v), v);
    v = fcomp(dpp_map<0x112, 0xf>(v), v);
    v = fcomp(dpp_map<0x114, 0xf>(v), v);
    v = fcomp(dpp_map<0x118, 0xf>(v), v);
    return v;
}
__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v)
{
    v += dpp_u32<0x111, 0xf>(v);
    v += dpp_u32<0x112, 0xf>(v);
    v += dpp_u32<0x114, 0xf>(v);
    v += dpp_u32<0x118, 0xf>(v);
    v += dpp_u32<0x142, 0xa>(v);
    v += dpp_u32<0x143, 0xc>(v);
    return v;
}

// the step x/u rounded to nearest, for x >= 0 finite and u = 2^(eb - 150)
// (eb = the biased exponent of the binade, 1 for the subnormal range)
__device__ __forceinline__ FMap fmap_of(float x, int eb)
{
    const uint32_t xb = __float_as_uint(x);
    int xe = (int)(xb >> 23);
    uint32_t m = xb & 0x7fffffu;
    if (xe == 0) xe = 1;
    else m |= 0x800000u;
    const int sh = eb - xe;                      // x/u = m * 2^-sh
    if (sh <= 0) {
        if (m == 0) return {0, 0};
        const uint32_t X = (-sh >= 3) ? FSAT : (m << (-sh));
        return {X, X};
    }
    if (sh >= 26) return {0, 0};                 // below a quarter ulp
    const uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem != half) {
        const uint32_t d = q + (rem > half ? 1u : 0u);
        return {d, d};
    }
    return {q + (q & 1u), q + ((q & 1u) ^ 1u)};  // tie: to the even multiple
}

__device__ __forceinline__ int f_eb(float s)
{
    const int e = (int)(__float_as_uint(s) >> 23);
    return e ? e : 1;
}
__device__ __forceinline__ uint32_t f_S(float s)
{
    const uint32_t b = __float_as_uint(s);
    return (b >> 23) ? ((b & 0x7fffffu) | 0x800000u) : b;
}
__device__ __forceinline__ float f_make(int eb, uint32_t S)
{
    return __uint_as_float(((uint32_t)(eb - 1) << 23) + S);
}

enum { F_NONE = 0, F_GE = 1, F_GT = 2 };

struct FoldRes {
    float sum;    // the fold of all n elements (idx < 0), or the prefix at idx
    int idx;      // first index whose prefix meets the predicate, or -1
};

__device__ __forceinline__ bool fpred(int mode, float v, float thr)
{
    return mode == F_GE ? v >= thr : v > thr;
}

// one thread: t = t + x(i) for i < n in order; with a predicate, up to its
// first hit (*hit = that index, t = the prefix there).  The prefixes only
// grow, so the predicate is tested once per 16 elements, on the last prefix,
// and inside those 16 only when it holds there.  Elements past n enter as 0,
// which leaves a sum unchanged.
template <class X>
__device__ __forceinline__ float head_fold(X x_at, int n, float t, float thr, int pmode, int* hit)
{
    if (pmode == F_NONE) {
#pragma unroll 16
        for (int i = 0; i < n; i++) t = t + x_at(i);
        return t;
    }
    for (int i0 = 0; i0 < n; i0 += 16) {
        float v[16], tq[16];
#pragma unroll
        for (int q = 0; q < 16; q++) v[q] = x_at(i0 + q < n ? i0 + q : n - 1);
        float u = t;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            u = u + (i0 + q < n ? v[q] : 0.0f);
            tq[q] = u;
        }
        if (fpred(pmode, u, thr)) {
#pragma unroll
            for (int q = 15; q >= 0; q--)
                if (fpred(pmode, tq[q], thr)) { *hit = i0 + q; t = tq[q]; }
            return t;
        }
        t = u;
    }
    *hit = -1;
    return t;
}

// Sequential f32 fold s = s + x(i), i = 0..n-1, of non-negative finite x,
// bit-identical to the loop, with an optional monotone predicate on the
// running value (F_GE: s_i >= thr, F_GT: s_i > thr) whose first hit ends the
// fold.  Called by every thread of the block with the same arguments.  With
// seq > 0 one thread adds the first seq elements itself, in order, with the
// predicate on its prefixes (head_fold): a sum leaves a binade every time it doubles and
// each exit costs a block pass, so a fold from 0 over values of one size, or
// over values sorted largest first from 1, meets most of its exits in its
// first few hundred elements.  That thread reads head[i] (LDS, staged by the
// caller) when head is given, else x_at(i) (then a plain load, so that the
// loop can issue its loads ahead).  With ck, thread 0 stores the running sum
// after the first seq elements in ck[0] and after each window w of SB * FIPT
// elements in ck[1 + w] (fold_search starts from them).
template <class X>
__device__ FoldRes block_fold(X x_at, int n, float s, float thr, int pmode, Small* sm, int seq = 0,
                              const float* head = nullptr, float* ck = nullptr)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __syncthreads();
    if (tid < 4) (&sm->slot[0][0])[tid] = ~0ull;
    int start0 = 0;
    if (seq > 0) {
        start0 = seq < n ? seq : n;
        if (tid == 0) {
            int hit = -1;
            const float t = head ? head_fold([&](int i) { return head[i]; }, start0, s, thr, pmode, &hit)
                                 : head_fold(x_at, start0, s, thr, pmode, &hit);
            sm->wf[0] = t;
            sm->iv[5] = hit;
        }
        __syncthreads();
        s = sm->wf[0];
        const int hit = sm->iv[5];
        if (hit >= 0) return {s, hit};
    }
    if (ck && tid == 0) ck[0] = s;
    __syncthreads();
    int it = 0, win = 0;
    for (int start = start0; start < n; start += SB * FIPT, win++) {
        const int base = start + tid * FIPT;
        float xv[FIPT];
#pragma unroll
        for (int q = 0; q < FIPT; q++) {
            const int i = base + q;
            xv[q] = x_at(i < n ? i : n - 1);
        }
#pragma unroll
        for (int q = 0; q < FIPT; q++)
            if (base + q >= n) xv[q] = 0.0f;
        // passes over the window held in registers; a pass that leaves the
        // binade is redone from the exit on, in the new binade, with the
        // elements up to the exit masked out
        int done = start - 1;
        for (;;) {
            const int eb = f_eb(s);
            const uint32_t S0 = f_S(s);
            FMap m[FIPT];
            FMap acc = {0u, 0u};
#pragma unroll
            for (int q = 0; q < FIPT; q++) {
                m[q] = base + q > done ? fmap_of(xv[q], eb) : FMap{0u, 0u};
                acc = fcomp(acc, m[q]);
            }
            const FMap inc = wave_scan_maps(acc);
            const FMap ex = dpp_map<0x138, 0xf>(inc);      // wave_shr:1 (lane 0: the identity)
            if (lane == 63) sm->wtot[wave] = inc;
            unsigned long long* slot = sm->slot[it & 1];
            __syncthreads();
            if (tid < 2) sm->slot[(it + 1) & 1][tid] = ~0ull;
            // the waves' totals, scanned by every wave on its first SWV lanes
            static_assert(SWV == 16, "one DPP row holds the wave totals");
            const FMap wi = row_scan_maps(lane < SWV ? sm->wtot[lane] : FMap{0u, 0u});
            FMap wp = {0u, 0u}, tot;
            const int src = __builtin_amdgcn_readfirstlane(wave > 0 ? wave - 1 : 0);
            wp.d0 = (uint32_t)__builtin_amdgcn_readlane((int)wi.d0, src);
            wp.d1 = (uint32_t)__builtin_amdgcn_readlane((int)wi.d1, src);
            if (wave == 0) wp = {0u, 0u};
            tot.d0 = (uint32_t)__builtin_amdgcn_readlane((int)wi.d0, SWV - 1);
            tot.d1 = (uint32_t)__builtin_amdgcn_readlane((int)wi.d1, SWV - 1);
            const FMap pre = fcomp(wp, ex);
            uint32_t S = S0 + fsel(pre, S0);
            bool live = true;
#pragma unroll
            for (int q = 0; q < FIPT; q++) {
                const int i = base + q;
                if (live && i > done && i < n && S < FTOP) {
                    const uint32_t Sp = S;
                    S = Sp + fsel(m[q], Sp);
                    if (S >= FTOP) {
                        // leaves the binade: this add is done in f32 by the hardware
                        const float sn = f_make(eb, Sp) + xv[q];
                        atomicMin(&slot[0], ((unsigned long long)i << 32) | __float_as_uint(sn));
                        live = false;
                    } else if (pmode != F_NONE) {
                        const float sv = f_make(eb, S);
                        if (fpred(pmode, sv, thr)) {
                            atomicMin(&slot[1], ((unsigned long long)i << 32) | __float_as_uint(sv));
                            live = false;
                        }
                    }
                }
            }
            __syncthreads();
            const unsigned long long cr = slot[0], pr = slot[1];
            it++;
            // a predicate hit can only precede the first exit: later prefixes
            // are saturated and never tested
            if (pr != ~0ull) return {__uint_as_float((uint32_t)pr), (int)(pr >> 32)};
            if (cr == ~0ull) {
                s = f_make(eb, S0 + fsel(tot, S0));
                if (ck && tid == 0) ck[1 + win] = s;
                break;
            }
            const int ci = (int)(cr >> 32);
            const float sn = __uint_as_float((uint32_t)cr);
            if (pmode != F_NONE && fpred(pmode, sn, thr)) return {sn, ci};
            s = sn;
            done = ci;
        }
    }
    return {s, -1};
}

// ------------------------------------------------------------ block helpers
// exclusive scan of one u32 per thread; *total gets the block sum
__device__ uint32_t block_excl_scan(uint32_t v, Small* sm, uint32_t* total)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t inc = wave_scan_add(v);
    __syncthreads();
    if (lane == 63) sm->scan[wave] = inc;
    __syncthreads();
    uint32_t wp = 0, tot = 0;
    for (int w = 0; w < SWV; w++) {
        const uint32_t c = sm->scan[w];
        if (w < wave) wp += c;
        tot += c;
    }
    *total = tot;
    return wp + inc - v;
}

// fmaxf over x(i), i < n (f32::max semantics: a NaN operand is ignored)
template <class X>
__device__ float block_max(X x_at, int n, Small* sm)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float m = -INFINITY;
    strided(n, x_at, [&](int, float v) { m = fmaxf(m, v); });
    m = cpv_wave_reduce(m, cpv_op_max());
    __syncthreads();
    if (lane == 0) sm->wf[wave] = m;
    __syncthreads();
    float r = -INFINITY;
    for (int w = 0; w < SWV; w++) r = fmaxf(r, sm->wf[w]);
    return r;
}

// index of the first strict maximum of x(i), i < n (values that are not
// above -inf, NaN included, never win); `dflt` when nothing wins
template <class X>
__device__ int block_argmax(X x_at, int n, int dflt, Small* sm)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    strided(n, x_at, [&](int i, float v) {
        if (v > best) { best = v; idx = i; }
    });
    {
        float unused = 0.0f;
        cpv_wave_amax(best, idx, unused);   // (best, lowest index) is a strict order
    }
    __syncthreads();
    if (lane == 0) { sm->wf[wave] = best; sm->wi[wave] = idx; }
    __syncthreads();
    best = -INFINITY;
    idx = 0x7fffffff;
    for (int w = 0; w < SWV; w++)
        if (sm->wf[w] > best || (sm->wf[w] == best && sm->wi[w] < idx)) { best = sm->wf[w]; idx = sm->wi[w]; }
    return idx == 0x7fffffff ? dflt : idx;
}

// number of i < n with pred(i)
template <class Pred>
__device__ int block_count(Pred pred, int n, Small* sm)
{
    int c = 0;
    for (int i = threadIdx.x; i < n; i += SB) c += pred(i) ? 1 : 0;
    uint32_t tot;
    (void)block_excl_scan((uint32_t)c, sm, &tot);
    return (int)tot;
}

// smallest i < n with pred(i), or -1 (pred evaluated BU indices at a time,
// at clamped indices, so that its loads are issued together)
template <class Pred>
__device__ int block_first(Pred pred, int n, Small* sm)
{
    __syncthreads();
    if (threadIdx.x == 0) sm->iv[7] = 0x7fffffff;
    __syncthreads();
    int mine = 0x7fffffff;
    for (int i0 = threadIdx.x; i0 < n && mine == 0x7fffffff; i0 += SB * BU) {
        bool h[BU];
#pragma unroll
        for (int q = 0; q < BU; q++) {
            const int i = i0 + q * SB;
            h[q] = pred(i < n ? i : n - 1) && i < n;
        }
#pragma unroll
        for (int q = BU - 1; q >= 0; q--)
            if (h[q]) mine = i0 + q * SB;
    }
    if (mine != 0x7fffffff) atomicMin(&sm->iv[7], mine);
    __syncthreads();
    const int r = sm->iv[7];
    return r == 0x7fffffff ? -1 : r;
}

// largest i < n with pred(i), or -1
template <class Pred>
__device__ int block_last(Pred pred, int n, Small* sm)
{
    __syncthreads();
    if (threadIdx.x == 0) sm->iv[6] = -1;
    __syncthreads();
    int mine = -1;
    for (int i0 = threadIdx.x; i0 < n; i0 += SB * BU) {
        bool h[BU];
#pragma unroll
        for (int q = 0; q < BU; q++) {
            const int i = i0 + q * SB;
            h[q] = pred(i < n ? i : n - 1) && i < n;
        }
#pragma unroll
        for (int q = 0; q < BU; q++)
            if (h[q]) mine = i0 + q * SB;
    }
    if (mine >= 0) atomicMax(&sm->iv[6], mine);
    __syncthreads();
    return sm->iv[6];
}

// Folds from 0 over values in candidate order (largest first) meet most of
// their binade exits in the first elements: those go to the fold's
// one-thread head, staged in LDS by the whole block first (the values may
// gather, and one thread's loads from memory would wait one by one).  A
// draw's two folds over the same values share the staging, and the search
// starts at the last checkpoint of the total's fold below the target.
struct FoldLds {
    float head[FOLD_SEQ];
    float ck[40];   // ck[0] after the head, ck[1 + w] after window w
};
static_assert((VMAX + SB * FIPT - 1) / (SB * FIPT) + 1 <= 40, "a checkpoint per fold window");

template <class X>
__device__ void stage_head(X x_at, int n, FoldLds* fl)
{
    const int ns = n < FOLD_SEQ ? n : FOLD_SEQ;
    __syncthreads();
    for (int i = threadIdx.x; i < ns; i += SB) fl->head[i] = x_at(i);
    __syncthreads();
}

// the fold of x over n elements from 0, staged head first, with checkpoints
template <class X>
__device__ float staged_total(X x_at, int n, FoldLds* fl, Small* sm)
{
    stage_head(x_at, n, fl);
    return block_fold(x_at, n, 0.0f, 0.0f, F_NONE, sm, FOLD_SEQ, fl->head, fl->ck).sum;
}

// the first prefix of the same fold meeting the predicate, from the last
// checkpoint that does not (the prefixes are monotone: the values are >= 0
// and f32 addition rounds monotonically)
template <class X>
__device__ FoldRes fold_search(X x_at, int n, float thr, int pmode, FoldLds* fl, Small* sm)
{
    __syncthreads();
    const int ns = n < FOLD_SEQ ? n : FOLD_SEQ;
    const int nw = (n - ns + SB * FIPT - 1) / (SB * FIPT);
    int j = -1;
    for (int c = 0; c <= nw && !fpred(pmode, fl->ck[c], thr); c++) j = c;
    if (j < 0) return block_fold(x_at, n, 0.0f, thr, pmode, sm, FOLD_SEQ, fl->head);
    const int p0 = ns + j * SB * FIPT;
    const float c0 = fl->ck[j];
    if (p0 >= n) return {c0, -1};
    FoldRes r = block_fold([&](int i) { return x_at(p0 + i); }, n - p0, c0, thr, pmode, sm);
    if (r.idx >= 0) r.idx += p0;
    return r;
}

// ------------------------------------------------------------ candidate order
// u32 that ascends as the logit descends (-0 ranks with +0)
__device__ __forceinline__ uint32_t desc_key(float l)
{
    uint32_t b = __float_as_uint(l);
    if (b == 0x80000000u) b = 0;
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ~ord;
}
__device__ __forceinline__ unsigned long long cand_key(float l, int i)
{
    return ((unsigned long long)desc_key(l) << 32) | (uint32_t)i;
}

// the band's cnt keys (keys[0..cnt), any order) sorted in LDS, IPT per
// thread, and written out as ids and logits at sid/sl[pos...]; sm->last gets
// the last key
template <class Sort, int IPT>
__device__ __forceinline__ void sort_emit(const float* lg, int cnt, int pos, int32_t* sid, float* sl,
                                          unsigned long long* keys, Small* sm, int (&oid)[IPT], float (&olv)[IPT])
{
    const int tid = threadIdx.x;
    unsigned long long k[IPT];
#pragma unroll
    for (int q = 0; q < IPT; q++) {
        const int t = tid * IPT + q;
        const unsigned long long key = t < cnt ? keys[t] : ~0ull;
        k[q] = key == ~0ull ? (1ull << KEY_BITS) - 1 : ((key >> 32) << 18) | (key & 0x3ffffull);
    }
    __syncthreads();                           // the key buffer becomes the sort's storage
    Sort().sort_to_striped(k, *reinterpret_cast<typename Sort::storage_type*>(keys), 0, KEY_BITS);
    // thread t now holds positions t, t + SB, ... of the band (striped: the
    // stores coalesce); every logit load goes out before the first store
    // (padding keys read id 0).  The positions are formed anew here: values
    // kept across the sort were spilled and reloaded one store at a time.
    int tb = tid;
    asm volatile("" : "+v"(tb));
    float lv[IPT];
#pragma unroll
    for (int q = 0; q < IPT; q++) {
        const int t = tb + q * SB;
        lv[q] = lg[t < cnt ? (int)(k[q] & 0x3ffffull) : 0];
    }
#pragma unroll
    for (int q = 0; q < IPT; q++) {
        const int t = tb + q * SB;
        if (t < cnt) {
            sid[pos + t] = (int)(k[q] & 0x3ffffull);
            sl[pos + t] = lv[q];
            if (t == cnt - 1) sm->last = ((k[q] >> 18) << 32) | (k[q] & 0x3ffffull);
        }
        oid[q] = (int)(k[q] & 0x3ffffull);
        olv[q] = lv[q];
    }
    __syncthreads();
}
template <class Sort, int IPT>
__device__ __forceinline__ void sort_emit(const float* lg, int cnt, int pos, int32_t* sid, float* sl,
                                          unsigned long long* keys, Small* sm)
{
    int oid[IPT];
    float olv[IPT];
    sort_emit<Sort, IPT>(lg, cnt, pos, sid, sl, keys, sm, oid, olv);
}

// the split top-p build's state per row: the row maximum in EXP_SPLIT
// parts, then what its first launch leaves for the second
constexpr int EXP_SPLIT = 32;
struct DistState {
    float sum1;                 // the index-order sum of exp(l - max)
    int cnt;                    // size of the first band
    unsigned long long last;    // its last key
    float pmax[EXP_SPLIT];      // fmaxf over each part of the row
    double psum[EXP_SPLIT];     // each part's exponentials summed in binary64 (a forecast only)
    FMap pmap[EXP_SPLIT];       // each part's fold steps composed in binade peb
    int peb[EXP_SPLIT];         // the binade the forecast puts the fold in at the part's start
    int np;                     // the first band in parts (band_part_kernel sorts them), or 0
    int boff[MAXP], bcnt[MAXP]; // each part's offset in the band and size
    unsigned long long first;   // the band's first key
    float bf1[MAXP], bf2[MAXP]; // each part's estimated sums of exp(l - max) and exp((l - max) / T)
    FMap m1[MAXP], m2[MAXP];    // each part's top-p fold (pr / sum1) and final-sum (exp(l / T - mx2)) steps
    int eb1[MAXP], eb2[MAXP];   // composed in these binades
};

// The next band of the candidate order after key *last (all keys when
// have_last is false): at most BAND keys, ending early at a histogram bin
// boundary once `want` are in.  band_select leaves the last level's
// histogram in the key buffer and describes the band: the keys after *last
// and up to hi, which share `prefix` on the bits `fixed` and lie in bins
// first..j of the level at shift sh; tot = 0: no key is left.
struct BandSel {
    unsigned long long prefix, fixed, hi;
    int sh, nb, first, j;
    uint32_t tot;
};

__device__ BandSel band_select(const float* lg, int V, bool have_last, unsigned long long last, int want,
                               unsigned long long* keys, Small* sm)
{
    const int tid = threadIdx.x;
    uint32_t* hist = (uint32_t*)keys;
    BandSel b{};
    b.hi = ~0ull;
    // bit fields of the key: desc_key in 63..32 (12 + 12 + 8), id in 17..0 (9 + 9)
    const int SH[5] = {52, 40, 32, 9, 0};
    const int WD[5] = {12, 12, 8, 9, 9};
    for (int lev = 0; lev < 5; lev++) {
        const int sh = SH[lev], nb = 1 << WD[lev];
        __syncthreads();
        for (int q = tid; q < nb; q += SB) hist[q] = 0;
        __syncthreads();
        const unsigned long long prefix = b.prefix, fixed = b.fixed;
        row_pass(lg, V, [&](int i, float l) {
            const unsigned long long key = cand_key(l, i);
            if ((have_last && key <= last) || (key & fixed) != prefix) return;
            atomicAdd(&hist[(key >> sh) & (unsigned long long)(nb - 1)], 1u);
        });
        __syncthreads();
        uint32_t c[4], s = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int bq = tid * 4 + q;
            c[q] = bq < nb ? hist[bq] : 0u;
            s += c[q];
        }
        uint32_t tot;
        const uint32_t ex = block_excl_scan(s, sm, &tot);
        if (tid == 0) { sm->iv[0] = -1; sm->iv[1] = 0x7fffffff; sm->iv[2] = 0x7fffffff; }
        __syncthreads();
        uint32_t run = ex;
        int my_cap = -1, my_want = 0x7fffffff, my_first = 0x7fffffff;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int bq = tid * 4 + q;
            if (bq < nb) {
                run += c[q];
                if (run <= (uint32_t)BAND) my_cap = bq;
                if (run >= (uint32_t)want && my_want == 0x7fffffff) my_want = bq;
                if (c[q] && my_first == 0x7fffffff) my_first = bq;
            }
        }
        if (my_cap >= 0) atomicMax(&sm->iv[0], my_cap);
        if (my_want != 0x7fffffff) atomicMin(&sm->iv[1], my_want);
        if (my_first != 0x7fffffff) atomicMin(&sm->iv[2], my_first);
        __syncthreads();
        const int jcap = sm->iv[0], jwant = sm->iv[1], first = sm->iv[2];
        b.tot = tot;
        if (tot == 0) return b;
        if (jcap >= first) {
            b.j = jwant < jcap ? jwant : jcap;
            b.hi = prefix | ((unsigned long long)b.j << sh) | ((1ull << sh) - 1ull);
            b.sh = sh;
            b.nb = nb;
            b.first = first;
            return b;
        }
        // the first non-empty bin alone holds more than a band: refine it
        b.prefix |= (unsigned long long)first << sh;
        b.fixed |= (unsigned long long)(nb - 1) << sh;
    }
    return b;   // (not reached: the last level's bins hold one key each)
}

// the band's keys gathered into the key buffer, sorted and written out at
// sid/sl[pos...]; *last_io advances to the band's last key
__device__ int band_sort_emit(const float* lg, int V, bool have_last, BandSel b,
                              unsigned long long* last_io, int pos, int32_t* sid, float* sl,
                              unsigned long long* keys, Small* sm)
{
    const int tid = threadIdx.x;
    const unsigned long long last = *last_io, hi = b.hi;
    __syncthreads();
    if (tid == 0) sm->iv[3] = 0;
    __syncthreads();
    row_pass(lg, V, [&](int i, float l) {
        const unsigned long long key = cand_key(l, i);
        if ((have_last && key <= last) || key > hi) return;
        keys[atomicAdd(&sm->iv[3], 1)] = key;   // (the band is sorted below: any order)
    });
    __syncthreads();
    const int cnt = sm->iv[3];
    if (cnt <= SMALL_BAND) sort_emit<small_sort_t, SMALL_BAND / SB>(lg, cnt, pos, sid, sl, keys, sm);
    else sort_emit<band_sort_t, BAND / SB>(lg, cnt, pos, sid, sl, keys, sm);
    *last_io = sm->last;
    __syncthreads();
    return cnt;
}

// Writes ids and logits to sid/sl[pos...], advances *last and returns the
// band size.
__device__ __noinline__ int emit_band(const float* lg, int V, bool have_last, unsigned long long* last_io, int want,
                                      int pos, int32_t* sid, float* sl, unsigned long long* keys, Small* sm)
{
    const BandSel b = band_select(lg, V, have_last, *last_io, want, keys, sm);
    if (b.tot == 0) return 0;
    return band_sort_emit(lg, V, have_last, b, last_io, pos, sid, sl, keys, sm);
}

// The first band for workgroups of its own to sort (the split top-p build):
// its keys gathered into bkeys, part by part (parts of whole bins of a
// histogram over the band's key range, each sorted by band_part_kernel).  Returns the band size and sets *last to its
// last key and *np to the number of parts; or -1 (np = 0) when a part would
// exceed SMALL_BAND keys, for the caller to emit the band itself.
__device__ __noinline__ int emit_band_parts(const float* lg, int V, float mx, float T, unsigned long long* last,
                                            unsigned long long* bkeys, DistState* st, int* np,
                                            unsigned long long* keys, Small* sm)
{
    const int tid = threadIdx.x;
    *np = 0;
    const BandSel b = band_select(lg, V, false, 0ull, BAND, keys, sm);
    if (b.tot == 0) return 0;
    // the band's keys lie in [klo, hi]: a histogram of its own over that
    // range, 4096 bins of 2^bs keys (the selection's bins are too coarse to
    // part: near a band's edge one holds thousands of keys)
    const unsigned long long klo = b.prefix | ((unsigned long long)b.first << b.sh), hi = b.hi;
    const unsigned long long span = hi - klo;
    const int bs = span >> 12 ? 64 - __clzll((long long)span) - 12 : 0;   // span >> bs < 4096
    uint32_t* hist = (uint32_t*)keys;
    uint8_t* part_of = (uint8_t*)keys + 4 * 4096;   // (after the histogram)
    __syncthreads();
    for (int q = tid; q < 4096; q += SB) hist[q] = 0;
    __syncthreads();
    row_pass(lg, V, [&](int i, float l) {
        const unsigned long long key = cand_key(l, i);
        if (key > hi || key < klo) return;
        atomicAdd(&hist[(int)((key - klo) >> bs)], 1u);
    });
    __syncthreads();
    // part of each bin (its offset in the band / PSPAN), each part's range
    uint32_t c[4], s = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        c[q] = hist[tid * 4 + q];
        s += c[q];
    }
    uint32_t tot;
    uint32_t off = block_excl_scan(s, sm, &tot);
    if (tid < MAXP) {
        sm->poff[tid] = 0x7fffffff;
        sm->pend[tid] = 0;
        sm->pfill[tid] = 0;
        sm->pf1[tid] = 0.0f;
        sm->pf2[tid] = 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int bq = tid * 4 + q;
        if (c[q]) {
            const int k = (int)(off / PSPAN);
            part_of[bq] = (uint8_t)k;
            atomicMin(&sm->poff[k], (int)off);
            atomicMax(&sm->pend[k], (int)(off + c[q]));
            // the part's sums estimated from the bin's largest logit (they set
            // the binades the parts' fold steps are composed in: speed only)
            const uint32_t ord = ~(uint32_t)((klo + ((unsigned long long)bq << bs)) >> 32);
            const float lb = __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
            atomicAdd(&sm->pf1[k], (float)c[q] * __expf(lb - mx));
            atomicAdd(&sm->pf2[k], (float)c[q] * __expf((lb - mx) / T));
        }
        off += c[q];
    }
    __syncthreads();
    bool fits = true;
    for (int k = 0; k < MAXP; k++)
        if (sm->pend[k] - (sm->poff[k] < sm->pend[k] ? sm->poff[k] : sm->pend[k]) > SMALL_BAND) fits = false;
    if (!fits) return -1;
    unsigned long long kmx = 0ull, kmn = ~0ull;   // (the band is not empty)
    row_pass(lg, V, [&](int i, float l) {
        const unsigned long long key = cand_key(l, i);
        if (key > hi || key < klo) return;
        const int k = part_of[(int)((key - klo) >> bs)];
        bkeys[sm->poff[k] + atomicAdd(&sm->pfill[k], 1)] = key;
        kmx = key > kmx ? key : kmx;
        kmn = key < kmn ? key : kmn;
    });
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long y = __shfl_xor(kmx, o), z = __shfl_xor(kmn, o);
        kmx = y > kmx ? y : kmx;
        kmn = z < kmn ? z : kmn;
    }
    if ((tid & 63) == 0) {
        sm->wmax[tid >> 6] = kmx;
        sm->wmin[tid >> 6] = kmn;
    }
    __syncthreads();
    if (tid == 0) {
        unsigned long long m = sm->wmax[0], n = sm->wmin[0];
        for (int w = 1; w < SWV; w++) {
            m = sm->wmax[w] > m ? sm->wmax[w] : m;
            n = sm->wmin[w] < n ? sm->wmin[w] : n;
        }
        sm->last = m;
        st->first = n;
    }
    __syncthreads();
    if (tid < MAXP) {
        const bool used = sm->pend[tid] > 0;
        st->boff[tid] = used ? sm->poff[tid] : 0;
        st->bcnt[tid] = used ? sm->pend[tid] - sm->poff[tid] : 0;
        st->bf1[tid] = sm->pf1[tid];
        st->bf2[tid] = sm->pf2[tid];
    }
    *last = sm->last;
    *np = MAXP;
    __syncthreads();
    return (int)tot;
}

// ------------------------------------------------------------ distributions

struct DistArgs {
    const float* p_logits;      // spec: [B][k+1][V]; direct: [rows][V]
    const float* q_logits;      // spec only: [B][k][V] or NULL
    const int32_t* draft;       // spec only: [B][k]
    const int32_t* hist;        // [B or rows][hist_len] or NULL
    int B, k, V, hist_len, nrow_p, direct;
    cpv_sampler_params prm;
    float ln_min_p;             // logf(min_p), evaluated by the host's libm
    int pen_on;
    float* pen;                 // [rows][V] penalised copies (pen_on)
    int32_t* sid;               // [rows][V] candidate ids in candidate order
    float* sl;                  // [rows][V] their (penalised, untempered) logits
    float* pr;                  // [rows][V] their probabilities
    int32_t* hdr;               // [rows] candidate count
    int phase;                  // 0: the whole build; top-p split: 1 (two workgroups per row), then 2
    int pre_exp;                // top-p: pr already holds expf(l - max) (exp_kernel)
    DistState* st;              // [rows] (phases 1 and 2)
    unsigned long long* bkeys;  // [rows][BAND] the first band's keys, part by part (phase 1)
    float* e2;                  // [rows][BAND] exp(l / T - mx2) of the first band's candidates (band parts)
    int parts;                  // phase 1 leaves the first band in parts (band_part_kernel follows)
};

// Penalties (lib.rs:233-266): a dense copy of the row in which every token
// of the window carries its penalised logit.  The window is the last
// penalty_last_n of the history (valid entries, oldest first) followed by
// the row's preceding drafts (Sampler::accept after each kept draft,
// engine.rs:2368-2369).
__device__ const float* apply_penalties(const float* logits, float* pen, int V, const int32_t* hist, int hist_len,
                                        const int32_t* drafts, int nd, const cpv_sampler_params& P, int* win,
                                        Small* sm)
{
    const int tid = threadIdx.x;
    int valid[4], c = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int a = tid * 4 + q;
        valid[q] = (hist && a < hist_len && hist[a] >= 0) ? 1 : 0;
        c += valid[q];
    }
    uint32_t L;
    uint32_t p = block_excl_scan((uint32_t)c, sm, &L);
    const int total = (int)L + nd, cap = P.penalty_last_n;
    const int start = total > cap ? total - cap : 0;
    const int wn = total - start;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (valid[q]) {
            if ((int)p >= start) win[p - start] = hist[tid * 4 + q];
            p++;
        }
    }
    for (int d = tid; d < nd; d += SB) {
        const int at = (int)L + d;
        if (at >= start) win[at - start] = drafts[d];
    }
    strided(V, [&](int i) { return logits[i]; }, [&](int i, float l) { pen[i] = l; });
    __syncthreads();
    for (int a = tid; a < wn; a += SB) {
        const int tok = win[a];
        if (tok < 0 || tok >= V) continue;
        bool first = true;
        int count = 0;
        for (int b = 0; b < wn; b++) {
            if (win[b] == tok) {
                if (b < a) first = false;
                count++;
            }
        }
        if (!first) continue;
        float l = logits[tok];
        if (l <= 0.0f) l *= P.penalty_repeat;
        else l /= P.penalty_repeat;
        const float sub = (float)count * P.penalty_freq;
        l -= sub + P.penalty_present;
        pen[tok] = l;
    }
    __syncthreads();
    return pen;
}

// the logits row `row` of the build (penalties off)
__device__ __forceinline__ const float* row_logits(const DistArgs& a, int row)
{
    if (a.direct || row < a.nrow_p) return a.p_logits + (size_t)row * a.V;
    return a.q_logits + (size_t)(row - a.nrow_p) * a.V;
}

// The split top-p build's first two launches, EXP_SPLIT workgroups per row:
// the row maximum in parts (fmaxf is order-free), then pr[i] = expf(l - max)
// by index, as the one-workgroup build computes them.
// the part's element range, in whole float4s (parts start at multiples of 4)
__device__ __forceinline__ void exp_part(int V, int part, int* i0, int* i1)
{
    const int per = (((V + EXP_SPLIT - 1) / EXP_SPLIT) + 3) & ~3;
    *i0 = min(V, part * per);
    *i1 = min(V, *i0 + per);
}

// 16-byte accesses when the row allows them
__device__ __forceinline__ bool vec4_ok(const void* p, int V) { return !(V & 3) && !((uintptr_t)p & 15); }

__global__ __launch_bounds__(256) void rowmax_part_kernel(DistArgs a)
{
    const int part = blockIdx.x, row = blockIdx.y, V = a.V, tid = threadIdx.x;
    const float* lg = row_logits(a, row);
    int i0, i1;
    exp_part(V, part, &i0, &i1);
    float m = -INFINITY;
    if (vec4_ok(lg, V)) {
        const float4* l4 = (const float4*)lg;
        for (int j = (i0 >> 2) + tid; j < (i1 >> 2); j += 256) {
            const float4 v = l4[j];
            m = fmaxf(m, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
        }
    } else {
        for (int i = i0 + tid; i < i1; i += 256) m = fmaxf(m, lg[i]);
    }
    m = cpv_wave_reduce(m, cpv_op_max());
    __shared__ float s_m[4];
    if ((tid & 63) == 0) s_m[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) a.st[row].pmax[part] = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
}

__global__ __launch_bounds__(256) void exp_kernel(DistArgs a)
{
    const int part = blockIdx.x, row = blockIdx.y, V = a.V, tid = threadIdx.x;
    const float* lg = row_logits(a, row);
    float mx = -INFINITY;
    for (int q = 0; q < EXP_SPLIT; q++) mx = fmaxf(mx, a.st[row].pmax[q]);
    float* pr = a.pr + (size_t)row * V;
    int i0, i1;
    exp_part(V, part, &i0, &i1);
    double ps = 0.0;             // (the part's sum, for the fold's forecast)
    if (vec4_ok(lg, V) && vec4_ok(pr, V)) {
        const float4* l4 = (const float4*)lg;
        float4* p4 = (float4*)pr;
        for (int j = (i0 >> 2) + tid; j < (i1 >> 2); j += 256) {
            const float4 v = l4[j];
            const float4 e = make_float4(cpv_expf(v.x - mx), cpv_expf(v.y - mx), cpv_expf(v.z - mx), cpv_expf(v.w - mx));
            p4[j] = e;
            ps += ((double)e.x + (double)e.y) + ((double)e.z + (double)e.w);
        }
    } else {
        for (int i = i0 + tid; i < i1; i += 256) {
            pr[i] = cpv_expf(lg[i] - mx);
            ps += (double)pr[i];
        }
    }
    for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
    __shared__ double s_ps[4];
    if ((tid & 63) == 0) s_ps[tid >> 6] = ps;
    __syncthreads();
    if (tid == 0) a.st[row].psum[part] = (s_ps[0] + s_ps[1]) + (s_ps[2] + s_ps[3]);
}

// The index-order fold's steps over each part, composed ahead (EXP_SPLIT
// workgroups per row, after exp_kernel): the binary64 sums of the parts
// before it forecast the binade the fold is in when it reaches the part;
// the part's per-element maps S -> S + d[S & 1] in that binade (fmap_of),
// composed in index order, are its whole step there.  The fold takes the
// step only when it does reach the part in that binade and the step keeps
// it below the binade's top (so no element left it); else it folds the
// part element by element (dist_kernel).  The forecast sets only the speed.
__global__ __launch_bounds__(256) void fmap_kernel(DistArgs a)
{
    const int part = blockIdx.x, row = blockIdx.y, V = a.V, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    DistState& st = a.st[row];
    double before = 0.0;
    for (int q = 0; q < part; q++) before += st.psum[q];
    const int eb = f_eb((float)before);
    const float* pr = a.pr + (size_t)row * V;
    int i0, i1;
    exp_part(V, part, &i0, &i1);
    // thread t composes the contiguous run [i0 + t c, i0 + (t + 1) c)
    const int c = (i1 - i0 + 255) / 256, b0 = i0 + tid * c, b1 = b0 + c < i1 ? b0 + c : i1;
    FMap m = {0u, 0u};
    for (int i = b0; i < b1; i++) m = fcomp(m, fmap_of(pr[i], eb));
    m = wave_scan_maps(m);                     // lane 63: the wave's runs in order
    __shared__ FMap s_w[4];
    if (lane == 63) s_w[wave] = m;
    __syncthreads();
    if (tid == 0) {
        const FMap t = fcomp(fcomp(s_w[0], s_w[1]), fcomp(s_w[2], s_w[3]));
        st.pmap[part] = t;
        st.peb[part] = eb;
    }
}

// Sampler::build for one row (lib.rs:229-376), leaving the distribution as
// n candidates (sid, sl, pr) in candidate order.
__global__ __launch_bounds__(SB) void dist_kernel(DistArgs a)
{
    extern __shared__ __align__(16) unsigned char sdyn[];
    unsigned long long* keys = (unsigned long long*)sdyn;
    Small* sm = (Small*)(sdyn + SAMPLE_LDS_KEYS);
    FoldLds* fl = (FoldLds*)(sdyn + SAMPLE_LDS_KEYS + sizeof(Small));
    // the split top-p build: after rowmax_part_kernel and exp_kernel, in
    // phase 1 workgroup 2 r sums row r's exponentials in index order while
    // workgroup 2 r + 1 emits its first band (the two need nothing from each
    // other); phase 2 goes on from both
    const int tid = threadIdx.x, row = a.phase == 1 ? (int)(blockIdx.x >> 1) : (int)blockIdx.x, V = a.V;
    const int role = a.phase == 1 ? (int)(blockIdx.x & 1) : 0;
    const cpv_sampler_params& P = a.prm;
    const float* logits;
    const int32_t* hist = nullptr;
    const int32_t* drafts = nullptr;
    int nd = 0;
    if (a.direct) {
        logits = a.p_logits + (size_t)row * V;
        if (a.hist) hist = a.hist + (size_t)row * a.hist_len;
    } else {
        int b, j;
        if (row < a.nrow_p) {
            b = row / (a.k + 1);
            j = row % (a.k + 1);
            logits = a.p_logits + (size_t)row * V;
        } else {
            const int r = row - a.nrow_p;
            b = r / a.k;
            j = r % a.k;
            logits = a.q_logits + (size_t)r * V;
        }
        if (a.hist) hist = a.hist + (size_t)b * a.hist_len;
        drafts = a.draft + (size_t)b * a.k;
        nd = j;
    }
    const size_t off = (size_t)row * V;
    int32_t* sid = a.sid + off;
    float* sl = a.sl + off;
    float* pr = a.pr + off;
    const float* lg = logits;
    if (a.pen_on) lg = apply_penalties(logits, a.pen + off, V, hist, a.hist_len, drafts, nd, P, (int*)keys, sm);

    if (P.temp <= 0.0f) {                                  // :324-337 point mass at the first maximum
        const int best = block_argmax([&](int i) { return lg[i]; }, V, 0, sm);
        if (tid == 0) {
            sid[0] = best;
            sl[0] = lg[best];
            pr[0] = 1.0f;
            a.hdr[row] = 1;
        }
        return;
    }

    const bool top_k = P.top_k > 0 && P.top_k < V;         // :272-280
    const bool min_p = !top_k && P.min_p > 0.0f;           // :281-295
    const bool top_p = !top_k && !min_p && P.top_p < 1.0f; // :296-316
    // (the split build needs no maximum here: exp_kernel has used it, and
    // top-p's final softmax is relative to the first candidate)
    const float mx = a.phase != 0 || a.pre_exp ? 0.0f : block_max([&](int i) { return lg[i]; }, V, sm);
    int n;
    if (top_k || min_p || top_p) {
        int M = 0, emitted = 0;
        unsigned long long last = 0;
        if (top_k) {
            M = P.top_k > P.min_keep ? P.top_k : P.min_keep;
            if (M > V) M = V;
        } else if (min_p) {
            const float floor_l = mx + a.ln_min_p;
            M = block_count([&](int i) { return lg[i] >= floor_l; }, V, sm);
        } else {
            // softmax over the vocabulary in index order, then the probe:
            // the smallest of 1024, 8192, ... (capped at V) whose sorted
            // prefix covers top_p, and the cut inside it (:343-358), both
            // read off one fold of the probabilities in candidate order
            // e_i = expf(l_i - max) once, by index, in the probabilities' row (the
            // final probabilities overwrite it at the end)
            float sum1 = 0.0f;
            int cnt;
            if (a.phase == 2) {
                sum1 = a.st[row].sum1;
                cnt = a.st[row].cnt;
                last = a.st[row].last;
            } else {
                if (role == 0) {
                    if (!a.pre_exp) {   // (else they come from exp_kernel)
                        strided(V, [&](int i) { return lg[i]; }, [&](int i, float l) { pr[i] = cpv_expf(l - mx); });
                        __syncthreads();
                    }
                    if (a.pre_exp) {
                        // part by part: the composed step where it applies, else element by element
                        const DistState& st = a.st[row];
                        for (int part = 0; part < EXP_SPLIT; part++) {
                            int i0, i1;
                            exp_part(V, part, &i0, &i1);
                            if (i1 <= i0) continue;
                            const int eb = f_eb(sum1);
                            if (part > 0 && eb == st.peb[part]) {
                                const uint32_t S0 = f_S(sum1), S = S0 + fsel(st.pmap[part], S0);
                                if (S < FTOP) {
                                    sum1 = f_make(eb, S);
                                    continue;
                                }
                            }
                            auto pv = [&](int i) { return pr[i0 + i]; };
                            if (part == 0) stage_head(pv, i1 - i0, fl);
                            sum1 = block_fold(pv, i1 - i0, sum1, 0.0f, F_NONE, sm, part == 0 ? FOLD_SEQ : 0,
                                              fl->head).sum;
                        }
                    } else {
                        auto pv = [&](int i) { return pr[i]; };
                        stage_head(pv, V, fl);
                        sum1 = block_fold(pv, V, 0.0f, 0.0f, F_NONE, sm, FOLD_SEQ, fl->head).sum;
                    }
                    if (a.phase == 1) {
                        if (tid == 0) a.st[row].sum1 = sum1;
                        return;
                    }
                }
                if (a.phase == 1) {
                    // the band's keys in parts for band_part_kernel to sort,
                    // or the band sorted here
                    DistState& st = a.st[row];
                    int np = 0;
                    cnt = -1;
                    if (a.parts) {
                        float mxr = -INFINITY;
                        for (int q = 0; q < EXP_SPLIT; q++) mxr = fmaxf(mxr, st.pmax[q]);
                        cnt = emit_band_parts(lg, V, mxr, P.temp, &last, a.bkeys + (size_t)row * BAND, &st, &np, keys,
                                              sm);
                    }
                    if (cnt < 0) cnt = emit_band(lg, V, false, &last, BAND, 0, sid, sl, keys, sm);
                    if (tid == 0) {
                        st.cnt = cnt;
                        st.last = last;
                        st.np = np;
                    }
                    return;
                }
                cnt = emit_band(lg, V, false, &last, BAND, 0, sid, sl, keys, sm);
            }
            float s = 0.0f;
            int ifirst = -1;
            if (a.phase == 2 && a.st[row].np > 0 && cnt > 0) {
                // the first band in parts: each part's composed step where it
                // applies and leaves the sum below top_p (the fold's values
                // only grow, so no element of the part meets the predicate),
                // else the part element by element
                const DistState& st = a.st[row];
                for (int p = 0; p < st.np; p++) {
                    const int pc = st.bcnt[p], po = st.boff[p];
                    if (pc <= 0) continue;
                    const int eb = f_eb(s);
                    if (eb == st.eb1[p]) {
                        const uint32_t S0 = f_S(s), S = S0 + fsel(st.m1[p], S0);
                        if (S < FTOP && !(f_make(eb, S) >= P.top_p)) {
                            s = f_make(eb, S);
                            continue;
                        }
                    }
                    const int32_t* band = sid + po;
                    auto bv = [&](int i) { return pr[band[i]] / sum1; };
                    const int seq = s == 0.0f ? FOLD_SEQ : 0;
                    if (seq) stage_head(bv, pc, fl);
                    const FoldRes r = block_fold(bv, pc, s, P.top_p, F_GE, sm, seq, fl->head);
                    if (r.idx >= 0) {
                        ifirst = po + r.idx;
                        break;
                    }
                    s = r.sum;
                }
                emitted = cnt;
                if (ifirst < 0 && emitted < V) cnt = emit_band(lg, V, true, &last, BAND, emitted, sid, sl, keys, sm);
                else cnt = 0;
            }
            while (cnt > 0) {
                const int32_t* band = sid + emitted;
                auto bv = [&](int i) { return pr[band[i]] / sum1; };
                const int seq = s == 0.0f ? FOLD_SEQ : 0;
                if (seq) stage_head(bv, cnt, fl);
                const FoldRes r = block_fold(bv, cnt, s, P.top_p, F_GE, sm, seq, fl->head);
                if (r.idx >= 0) ifirst = emitted + r.idx;
                emitted += cnt;
                if (r.idx >= 0) break;
                s = r.sum;
                if (emitted >= V) break;
                cnt = emit_band(lg, V, true, &last, BAND, emitted, sid, sl, keys, sm);
            }
            int probe = V < 1024 ? V : 1024;
            if (ifirst < 0) probe = V;
            else
                while (probe < ifirst + 1) probe = probe * 8 < V ? probe * 8 : V;
            M = probe;
            if (probe > 1 && ifirst >= 0) {
                const int keep = ifirst + 1 > P.min_keep ? ifirst + 1 : P.min_keep;
                if (keep <= probe) M = keep;
            }
        }
        while (emitted < M) {
            const int cnt = emit_band(lg, V, emitted > 0, &last, M - emitted, emitted, sid, sl, keys, sm);
            if (cnt <= 0) break;
            emitted += cnt;
        }
        n = M;
        if (!top_p && P.top_p < 1.0f && n > 1) {           // :343-358 after a re-softmax over the survivors
            const float l0 = sl[0];
            strided(n, [&](int i) { return sl[i]; }, [&](int i, float l) { pr[i] = cpv_expf(l - l0); });
            __syncthreads();
            auto pv = [&](int i) { return pr[i]; };
            stage_head(pv, n, fl);
            const float sA = block_fold(pv, n, 0.0f, 0.0f, F_NONE, sm, FOLD_SEQ, fl->head).sum;
            auto qv = [&](int i) { return pr[i] / sA; };
            stage_head(qv, n, fl);
            const FoldRes r = block_fold(qv, n, 0.0f, P.top_p, F_GE, sm, FOLD_SEQ, fl->head);
            if (r.idx >= 0) {
                const int keep = r.idx + 1 > P.min_keep ? r.idx + 1 : P.min_keep;
                if (keep <= n) n = keep;
            }
        }
        if (top_k && P.min_p > 0.0f && n > 1) {            // :360-369
            const float floor_l = sl[0] + a.ln_min_p;
            const int nn = n;
            int keep = block_count([&](int i) { return sl[i] >= floor_l; }, nn, sm);
            if (keep < 1) keep = 1;
            if (keep < P.min_keep) keep = P.min_keep;
            if (keep < n) n = keep;
        }
    } else {                                               // :317-322 the vocabulary in index order
        for (int i = tid; i < V; i += SB) {
            sid[i] = i;
            sl[i] = lg[i];
        }
        __syncthreads();
        n = V;
    }
    // :371-374 temperature, then softmax over the survivors (:461-471)
    const float T = P.temp;
    const float mx2 = (top_k || min_p || top_p ? sl[0] : mx) / T;
    __syncthreads();
    if (top_p && a.phase == 2 && a.st[row].np > 0 && n <= a.st[row].cnt) {
        // the survivors lie in the first band: its parts' e2 and composed
        // steps (band_part_kernel), the steps where they apply, whole parts
        // below n; the rest element by element
        const DistState& st = a.st[row];
        const float* e2 = a.e2 + (size_t)row * BAND;
        float s2 = 0.0f;
        for (int p = 0; p < st.np; p++) {
            const int pc = st.bcnt[p], po = st.boff[p];
            if (pc <= 0 || po >= n) continue;
            const int len = n - po < pc ? n - po : pc;
            const int eb = f_eb(s2);
            if (len == pc && eb == st.eb2[p]) {
                const uint32_t S0 = f_S(s2), S = S0 + fsel(st.m2[p], S0);
                if (S < FTOP) {
                    s2 = f_make(eb, S);
                    continue;
                }
            }
            auto ev = [&](int i) { return e2[po + i]; };
            if (po == 0) stage_head(ev, len, fl);
            s2 = block_fold(ev, len, s2, 0.0f, F_NONE, sm, po == 0 ? FOLD_SEQ : 0, fl->head).sum;
        }
        __syncthreads();
        strided(n, [&](int i) { return e2[i]; }, [&](int i, float e) { pr[i] = e / s2; });
        if (tid == 0) a.hdr[row] = n;
        return;
    }
    strided(n, [&](int i) { return sl[i]; }, [&](int i, float l) { pr[i] = cpv_expf(l / T - mx2); });
    __syncthreads();
    auto pv2 = [&](int i) { return pr[i]; };
    stage_head(pv2, n, fl);
    const float s2 = block_fold(pv2, n, 0.0f, 0.0f, F_NONE, sm, FOLD_SEQ, fl->head).sum;
    __syncthreads();
    strided(n, [&](int i) { return pr[i]; }, [&](int i, float e) { pr[i] = e / s2; });
    if (tid == 0) a.hdr[row] = n;
}

// The split top-p build's first band, part by part (after phase 1, before
// phase 2): workgroup (p, row) sorts part p's keys, whole histogram bins of
// the band in order, and writes their ids and logits at the part's offset.
// It then composes the part's steps of the two folds phase 2 runs over the
// band in candidate order: the top-p fold of pr[id] / sum1 and the final
// softmax sum of e2 = exp(l / T - mx2) (mx2 = the first candidate's l / T;
// the e2 are kept for phase 2), each in the binade its estimated sums put the
// fold in at the part's start.  Phase 2 takes a part's step only where it
// applies (the fmap_kernel rule), else folds the part element by element.
__global__ __launch_bounds__(SB) void band_part_kernel(DistArgs a)
{
    extern __shared__ __align__(16) unsigned char sdyn[];
    unsigned long long* keys = (unsigned long long*)sdyn;
    Small* sm;
    const int p = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    DistState& st = a.st[row];
    if (p >= st.np) return;
    sm = (Small*)(sdyn + PART_LDS_KEYS);
    const int cnt = st.bcnt[p], off = st.boff[p];
    if (cnt <= 0) return;
    const unsigned long long* src = a.bkeys + (size_t)row * BAND + off;
    for (int t = tid; t < cnt; t += SB) keys[t] = src[t];
    __syncthreads();
    const size_t ro = (size_t)row * a.V;
    const float* lg = row_logits(a, row);
    constexpr int IPT = SMALL_BAND / SB;
    int id[IPT];
    float lv[IPT];
    sort_emit<small_sort_t, IPT>(lg, cnt, off, a.sid + ro, a.sl + ro, keys, sm, id, lv);
    // this thread's positions tid + q SB: their terms (0 past the part)
    const float sum1 = st.sum1, T = a.prm.temp;
    const float mx2 = lg[(int)(st.first & 0x3ffffull)] / T;
    const float* pr = a.pr + ro;
    float* e2 = a.e2 + (size_t)row * BAND;
    float t1[IPT], t2[IPT];
#pragma unroll
    for (int q = 0; q < IPT; q++) {
        const int t = tid + q * SB;
        t1[q] = t < cnt ? pr[id[q]] / sum1 : 0.0f;
        t2[q] = t < cnt ? cpv_expf(lv[q] / T - mx2) : 0.0f;
        if (t < cnt) e2[off + t] = t2[q];
    }
    double f1 = 0.0, f2 = 0.0;
    for (int q = 0; q < p; q++) {
        f1 += (double)st.bf1[q];
        f2 += (double)st.bf2[q];
    }
    const int eb1 = f_eb((float)(f1 / (double)sum1)), eb2 = f_eb((float)f2);
    // the maps composed in position order: each stride of SB positions over
    // the waves in order, then the strides in order
    FMap c1 = {0u, 0u}, c2 = {0u, 0u};
#pragma unroll
    for (int q = 0; q < IPT; q++) {
        const FMap w1 = wave_scan_maps(fmap_of(t1[q], eb1)), w2 = wave_scan_maps(fmap_of(t2[q], eb2));
        __syncthreads();
        if (lane == 63) {
            sm->wtot[wave] = w1;
            sm->wi[wave] = (int)w2.d0;
            sm->scan[wave] = w2.d1;
        }
        __syncthreads();
        if (tid == 0)
            for (int w = 0; w < SWV; w++) {
                c1 = fcomp(c1, sm->wtot[w]);
                c2 = fcomp(c2, FMap{(uint32_t)sm->wi[w], sm->scan[w]});
            }
    }
    if (tid == 0) {
        st.m1[p] = c1;
        st.m2[p] = c2;
        st.eb1[p] = eb1;
        st.eb2[p] = eb2;
    }
}

// ------------------------------------------------------------ acceptance
// Philox4x64-10 (Salmon, Moraes, Dror, Shaw, SC'11): counter (c0, c1, c2, c3),
// key (seed, 0); the uniform is the top 24 bits of the first output word.
__device__ float philox_u01(uint64_t seed, uint64_t c0, uint64_t c1, uint64_t c2, uint64_t c3)
{
    uint64_t x0 = c0, x1 = c1, x2 = c2, x3 = c3, k0 = seed, k1 = 0;
    for (int r = 0; r < 10; r++) {
        const uint64_t lo0 = 0xD2E7470EE14C6C93ull * x0, hi0 = __umul64hi(0xD2E7470EE14C6C93ull, x0);
        const uint64_t lo1 = 0xCA5A826395121157ull * x2, hi1 = __umul64hi(0xCA5A826395121157ull, x2);
        const uint64_t n0 = hi1 ^ x1 ^ k0, n2 = hi0 ^ x3 ^ k1;
        x0 = n0;
        x1 = lo1;
        x2 = n2;
        x3 = lo0;
        k0 += 0x9E3779B97F4A7C15ull;
        k1 += 0xBB67AE8584CAA73Bull;
    }
    return (float)(x0 >> 40) / 16777216.0f;
}

struct DecideArgs {
    const int32_t* draft;       // [B][k]
    const float* u;             // [B][k+1][2] or NULL (Philox)
    uint64_t seed, round;
    const float* noise;         // [B][k+1][V] (GUMBEL)
    int B, k, V, mode, has_q, nrow_p;
    float T, inv_t;
    const int32_t* sid;
    const float* sl;
    const float* pr;
    const int32_t* hdr;
    float* qdense;              // [B][V] (has_q)
    int32_t* out_tok;           // [B][k+1]
    int32_t* out_n;             // [B]
};

struct Row {
    const int32_t* sid;
    const float* sl;
    const float* pr;
    int n;
};

__device__ __forceinline__ Row dist_row(const DecideArgs& a, int row)
{
    const size_t off = (size_t)row * a.V;
    return {a.sid + off, a.sl + off, a.pr + off, a.hdr[row]};
}

// Dist::draw (lib.rs:395-404): the first candidate whose cumulative
// probability exceeds r, else the last
__device__ int dist_draw(const Row& d, float r, Small* sm, FoldLds* fl)
{
    auto pv = [&](int i) { return d.pr[i]; };
    stage_head(pv, d.n, fl);
    const FoldRes f = block_fold(pv, d.n, 0.0f, r, F_GT, sm, FOLD_SEQ, fl->head);
    return f.idx >= 0 ? d.sid[f.idx] : d.sid[d.n - 1];
}

// Dist::draw_excluding (lib.rs:408-436).  Adding 0 leaves an f32 sum
// unchanged, so skipping x is folding it as 0.
__device__ int dist_draw_excluding(const Row& d, int x, float r, Small* sm, FoldLds* fl)
{
    auto val = [&](int i) { return d.sid[i] == x ? 0.0f : d.pr[i]; };
    const float total = staged_total(val, d.n, fl, sm);
    if (total <= 0.0f) return dist_draw(d, r, sm, fl);
    const float target = r * total;
    const FoldRes f = fold_search(val, d.n, target, F_GT, fl, sm);
    if (f.idx >= 0) return d.sid[f.idx];
    if (d.sid[d.n - 1] != x || d.n < 2) return d.sid[d.n - 1];
    return d.sid[d.n - 2];
}

// the general rule's residual max(0, p - q) over p's candidates in p's order
__device__ int dist_draw_residual(const Row& p, const Row& q, float* qd, int V, float r, Small* sm, FoldLds* fl)
{
    if ((V & 3) == 0 && ((uintptr_t)qd & 15) == 0) {
        for (int i = threadIdx.x; i < V / 4; i += SB) ((float4*)qd)[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
        for (int i = threadIdx.x; i < V; i += SB) qd[i] = 0.0f;
    }
    __syncthreads();
    strided(q.n, [&](int i) { return make_int2(q.sid[i], __float_as_int(q.pr[i])); },
            [&](int, int2 e) { qd[e.x] = __int_as_float(e.y); });
    __syncthreads();
    auto val = [&](int i) {
        const float d = p.pr[i] - qd[p.sid[i]];
        return d > 0.0f ? d : 0.0f;
    };
    const float total = staged_total(val, p.n, fl, sm);
    if (total <= 0.0f) return dist_draw(p, r, sm, fl);
    const float target = r * total;
    const FoldRes f = fold_search(val, p.n, target, F_GT, fl, sm);
    if (f.idx >= 0) return p.sid[f.idx];
    const int l = block_last([&](int i) { return p.pr[i] - qd[p.sid[i]] > 0.0f; }, p.n, sm);
    return l >= 0 ? p.sid[l] : p.sid[p.n - 1];
}

// Sampler::sample_coupled (lib.rs:197-216): the first candidate maximising
// tempered logit + T-scaled noise / T
__device__ int coupled_argmax(const DecideArgs& a, const Row& d, const float* noise_row, Small* sm)
{
    const float T = a.T, inv_t = a.inv_t;
    const bool tempered = T > 0.0f;
    const int i = block_argmax(
        [&](int c) {
            const float tl = tempered ? d.sl[c] / T : d.sl[c];
            return tl + noise_row[d.sid[c]] * inv_t;
        },
        d.n, 0, sm);
    return d.sid[i];
}

__device__ __forceinline__ float uniform(const DecideArgs& a, int b, int j, int r)
{
    if (a.u) return a.u[((size_t)b * (a.k + 1) + j) * 2 + r];
    return philox_u01(a.seed, (uint64_t)b, (uint64_t)j, (uint64_t)r, a.round);
}

// engine.rs:2326-2461 for one sequence: walk the drafts, stop at the first
// rejection, then the replacement or the bonus token
__global__ __launch_bounds__(SB) void decide_kernel(DecideArgs a)
{
    __shared__ Small sm_s;
    __shared__ FoldLds fl_s;
    Small* sm = &sm_s;
    FoldLds* fl = &fl_s;
    const int b = blockIdx.x, tid = threadIdx.x, K1 = a.k + 1, V = a.V;
    int n_keep = 0, rep = 0;
    bool have_rep = false;
    for (int j = 0; j < a.k; j++) {
        const Row d = dist_row(a, b * K1 + j);
        const int x = a.draft[(size_t)b * a.k + j];
        bool keep;
        if (a.mode == CPV_ACCEPT_GUMBEL) {
            const int commit = coupled_argmax(a, d, a.noise + ((size_t)b * K1 + j) * V, sm);
            keep = x == commit;
            if (!keep) { rep = commit; have_rep = true; }
        } else {
            const float u0 = uniform(a, b, j, 0), u1 = uniform(a, b, j, 1);
            const int pos = block_first([&](int i) { return d.sid[i] == x; }, d.n, sm);
            const float px = pos >= 0 ? d.pr[pos] : 0.0f;
            if (!a.has_q) {
                keep = u0 < px;
                if (!keep) { rep = dist_draw_excluding(d, x, u1, sm, fl); have_rep = true; }
            } else {
                const Row q = dist_row(a, a.nrow_p + b * a.k + j);
                const int qpos = block_first([&](int i) { return q.sid[i] == x; }, q.n, sm);
                const float qx = qpos >= 0 ? q.pr[qpos] : 0.0f;
                keep = u0 * qx < px;
                if (!keep) {
                    rep = dist_draw_residual(d, q, a.qdense + (size_t)b * V, V, u1, sm, fl);
                    have_rep = true;
                }
            }
        }
        if (!keep) break;
        if (tid == 0) a.out_tok[(size_t)b * K1 + n_keep] = x;
        n_keep++;
    }
    int next;
    if (have_rep) {
        next = rep;
    } else {
        const Row d = dist_row(a, b * K1 + n_keep);
        if (a.mode == CPV_ACCEPT_GUMBEL) next = coupled_argmax(a, d, a.noise + ((size_t)b * K1 + n_keep) * V, sm);
        else next = dist_draw(d, uniform(a, b, n_keep, 0), sm, fl);
    }
    if (tid == 0) {
        a.out_tok[(size_t)b * K1 + n_keep] = next;
        a.out_n[b] = n_keep;
    }
}

// greedy, and gumbel when the coupling is exact: the drafts are kept while
// they equal the row argmax (of logits + noise), and the row after the last
// kept draft gives the next token
__global__ void decide_argmax_kernel(const int32_t* __restrict__ am, const int32_t* __restrict__ draft, int B, int k,
                                     int32_t* __restrict__ out_tok, int32_t* __restrict__ out_n)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int K1 = k + 1;
    int n_keep = 0;
    while (n_keep < k && am[(size_t)b * K1 + n_keep] == draft[(size_t)b * k + n_keep]) {
        out_tok[(size_t)b * K1 + n_keep] = draft[(size_t)b * k + n_keep];
        n_keep++;
    }
    out_tok[(size_t)b * K1 + n_keep] = am[(size_t)b * K1 + n_keep];
    out_n[b] = n_keep;
}

bool penalties_on(const cpv_sampler_params* p)
{
    return !(p->penalty_repeat == 1.0f && p->penalty_freq == 0.0f && p->penalty_present == 0.0f);
}

bool coupling_is_exact(const cpv_sampler_params* p)       // lib.rs:70-78
{
    return p->temp > 0.0f && p->top_k == 0 && p->top_p >= 1.0f && p->min_p <= 0.0f && !penalties_on(p);
}

cpv_status check_params(cpv_ctx* ctx, const cpv_sampler_params* p, int hist_len)
{
    if (!p) return cpv_fail(ctx, CPV_EINVAL, "sampler: params is NULL");
    if (p->top_k < 0 || p->min_keep < 0 || p->penalty_last_n < 0)
        return cpv_fail(ctx, CPV_EINVAL, "sampler: top_k, min_keep and penalty_last_n are counts (>= 0)");
    if (p->min_p > 1.0f)
        return cpv_fail(ctx, CPV_EINVAL, "sampler: min_p above 1 leaves no candidate");
    if (hist_len < 0 || hist_len > HIST_MAX)
        return cpv_fail(ctx, CPV_EINVAL, "sampler: hist_len must be in [0, %d]", HIST_MAX);
    return CPV_OK;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct DistBufs {
    int32_t* hdr;
    DistState* st;
    unsigned long long* bkeys;
    float* e2;
    int32_t* sid;
    float* sl;
    float* pr;
    float* pen;
    void* tail;                 // first byte after the distribution buffers
};

size_t dist_bytes(int rows, int V, bool pen)
{
    const size_t rv = align256((size_t)rows * V * 4);
    return align256((size_t)rows * 4) + align256((size_t)rows * sizeof(DistState)) +
           align256((size_t)rows * BAND * 8) + align256((size_t)rows * BAND * 4) + 3 * rv + (pen ? rv : 0);
}

DistBufs dist_carve(void* ws, int rows, int V, bool pen)
{
    uint8_t* p = (uint8_t*)ws;
    const size_t rv = align256((size_t)rows * V * 4);
    DistBufs d;
    d.hdr = (int32_t*)p;
    p += align256((size_t)rows * 4);
    d.st = (DistState*)p;
    p += align256((size_t)rows * sizeof(DistState));
    d.bkeys = (unsigned long long*)p;
    p += align256((size_t)rows * BAND * 8);
    d.e2 = (float*)p;
    p += align256((size_t)rows * BAND * 4);
    d.sid = (int32_t*)p;
    p += rv;
    d.sl = (float*)p;
    p += rv;
    d.pr = (float*)p;
    p += rv;
    d.pen = pen ? (float*)p : nullptr;
    if (pen) p += rv;
    d.tail = p;
    return d;
}

cpv_status dist_launch(cpv_ctx* ctx, DistArgs& a, int rows)
{
    const size_t lds = SAMPLE_LDS_KEYS + sizeof(Small) + sizeof(FoldLds);
    if (lds > ctx->lds_max) return cpv_fail(ctx, CPV_EUNSUPPORTED, "sampler: needs %zu bytes of LDS", lds);
    const int e0 = cpv_prof_mark(ctx);
    // top-p without penalties: the maximum and the exponentials over
    // EXP_SPLIT workgroups per row; then, when two workgroups per row fit the
    // CUs, the index-order sum and the first band side by side (two
    // workgroups per row), then the rest
    const cpv_sampler_params& P = a.prm;
    const bool top_k = P.top_k > 0 && P.top_k < a.V;
    a.pre_exp = P.temp > 0.0f && !top_k && !(P.min_p > 0.0f) && P.top_p < 1.0f && !a.pen_on;
    if (a.pre_exp) {
        rowmax_part_kernel<<<dim3(EXP_SPLIT, (unsigned)rows), 256, 0, ctx->stream>>>(a);
        exp_kernel<<<dim3(EXP_SPLIT, (unsigned)rows), 256, 0, ctx->stream>>>(a);
        fmap_kernel<<<dim3(EXP_SPLIT, (unsigned)rows), 256, 0, ctx->stream>>>(a);
    }
    if (a.pre_exp && 2 * rows <= ctx->cu_count) {
        // the first band in parts while the part workgroups fit the CUs two to a CU
        a.parts = rows * MAXP <= 2 * ctx->cu_count;
        a.phase = 1;
        dist_kernel<<<(unsigned)(2 * rows), SB, lds, ctx->stream>>>(a);
        if (a.parts)
            band_part_kernel<<<dim3(MAXP, (unsigned)rows), SB, PART_LDS_KEYS + sizeof(Small), ctx->stream>>>(a);
        a.phase = 2;
        dist_kernel<<<(unsigned)rows, SB, lds, ctx->stream>>>(a);
    } else {
        a.phase = 0;
        dist_kernel<<<(unsigned)rows, SB, lds, ctx->stream>>>(a);
    }
    CPV_HIP(ctx, hipGetLastError());
    cpv_prof_add(ctx, e0, CPV_PROF_SAMPLE, (double)rows * a.V * 4.0);
    return CPV_OK;
}

// The re-draft gate's decision for row blockIdx.x: 1 / lse < p_min, lse the
// index-order f32 sum of e_i = expf(x_i - max) (engine.rs:2598-2606; the CLI
// spec path's softmax_prob at the argmax, crates/codpiece-cli/src/main.rs:
// 946-954, is the same value).  The bound pass gives S = sum e_i and W =
// sum e_i (n - i) in binary64.  The f32 loop's k-th add rounds its prefix by
// at most 2^-24 relative and carries the earlier errors with factors (1 +
// 2^-24) at most n times, so |lse - S| <= 2^-24 (1 + 2^-24)^n W, and for n <=
// 2^18 (a factor below 1.016), B = 0x1.1p-24 W + 2^-40 S covers it (the
// 2^-40 S for the binary64 sums themselves, each term of which passes
// through fewer than 2^7 adds).  1 / lse then lies in [1 / (S + B), 1 / (S - B)]: below
// p (1 - 2^-23) it rounds to an f32 below p_min, and from p_min up it rounds
// to p_min or above.  Rows in between run the sequential fold (block_fold
// over the same e_i, bit-identical to the loop).  A sum that is not finite and
// at least 1 (a NaN, or no finite logit) makes 1 / lse a NaN or 0 in the
// reference; it keeps the draft on NaN, as a NaN compares false.
__global__ __launch_bounds__(SB) void gate_fin_kernel(const float* __restrict__ x, int n,
                                                      const int32_t* __restrict__ idx, const double* __restrict__ sw,
                                                      int nb, float p_min, int32_t* __restrict__ keep)
{
    __shared__ Small sm;
    __shared__ int s_dec;
    const int64_t row = blockIdx.x;
    const float* xr = x + row * (int64_t)n;
    if (threadIdx.x == 0) {
        int dec = 1;
        if (sw && p_min > 0.0f) {
            double S = 0.0, W = 0.0;
            for (int b = 0; b < nb; b++) {
                S += sw[(row * nb + b) * 2];
                W += sw[(row * nb + b) * 2 + 1];
            }
            if (S >= 1.0 && S < 1e30) {
                const double B = 0x1.1p-24 * W + 0x1p-40 * S;
                const double rmax = 1.0 / (S - B), rmin = 1.0 / (S + B);
                const double p = (double)p_min;
                if (rmax * (1.0 + 0x1p-40) < p * (1.0 - 0x1p-23)) dec = 0;
                else if (rmin * (1.0 - 0x1p-40) >= p) dec = 1;
                else dec = 2;
            }
        }
        s_dec = dec;
    }
    __syncthreads();
    int dec = s_dec;
    if (dec == 2) {
        const float m = xr[idx[row]];
        const FoldRes r = block_fold([&](int i) { return cpv_expf(xr[i] - m); }, n, 0.0f, 0.0f, F_NONE, &sm, FOLD_SEQ);
        const float g = 1.0f / r.sum;
        dec = g < p_min ? 0 : 1;
    }
    if (threadIdx.x == 0) keep[row] = dec;
}

}  // namespace

cpv_status cpv_gate_fin_launch(cpv_ctx* ctx, const float* x, int64_t rows, int64_t n, const int32_t* idx,
                               const double* sw, int nb, float p_min, int32_t* keep_out)
{
    if (n > VMAX) return cpv_fail(ctx, CPV_EUNSUPPORTED, "redraft gate: rows longer than %d", VMAX);
    gate_fin_kernel<<<(unsigned)rows, SB, 0, ctx->stream>>>(x, (int)n, idx, sw, nb, p_min, keep_out);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

extern "C" cpv_status cpv_distribution(cpv_ctx* ctx, const float* logits_dev, int rows, int v,
                                       const cpv_sampler_params* params, const int32_t* hist_dev, int hist_len,
                                       int32_t* ids_dev, float* probs_dev, int32_t* n_dev)
{
    if (!ctx) return CPV_EINVAL;
    if (!logits_dev || !ids_dev || !probs_dev || !n_dev || rows < 0 || v < 1 || v > VMAX)
        return cpv_fail(ctx, CPV_EINVAL, "distribution: bad arguments (1 <= v <= %d)", VMAX);
    cpv_status st = check_params(ctx, params, hist_dev ? hist_len : 0);
    if (st) return st;
    if (rows == 0) return CPV_OK;
    const bool pen = penalties_on(params) && params->penalty_last_n > 0 && hist_dev && hist_len > 0;
    void* ws = nullptr;
    if ((st = cpv_workspace(ctx, dist_bytes(rows, v, pen), &ws))) return st;
    DistBufs d = dist_carve(ws, rows, v, pen);
    DistArgs a{};
    a.p_logits = logits_dev;
    a.hist = hist_dev;
    a.V = v;
    a.hist_len = hist_dev ? hist_len : 0;
    a.direct = 1;
    a.prm = *params;
    a.ln_min_p = params->min_p > 0.0f ? logf(params->min_p) : 0.0f;
    a.pen_on = pen;
    a.pen = d.pen;
    a.sid = ids_dev;
    a.sl = d.sl;
    a.pr = probs_dev;
    a.hdr = n_dev;
    a.st = d.st;
    a.bkeys = d.bkeys;
    a.e2 = d.e2;
    return dist_launch(ctx, a, rows);
}

extern "C" cpv_status cpv_spec_accept(cpv_ctx* ctx, const float* p_logits_dev, const float* q_logits_dev,
                                      const int32_t* draft_dev, int b, int k, int v,
                                      const cpv_sampler_params* params, int mode, const float* u_dev,
                                      uint64_t philox_seed, uint64_t philox_round, const float* noise_dev,
                                      const int32_t* hist_dev, int hist_len, int32_t* out_tok_dev,
                                      int32_t* out_n_dev)
{
    if (!ctx) return CPV_EINVAL;
    if (!p_logits_dev || (k > 0 && !draft_dev) || !out_tok_dev || !out_n_dev || b < 1 || k < 0 || k > 15 || v < 1 ||
        v > VMAX)
        return cpv_fail(ctx, CPV_EINVAL, "spec_accept: bad arguments (b >= 1, 0 <= k <= 15, 1 <= v <= %d)", VMAX);
    if (mode != CPV_ACCEPT_GREEDY && mode != CPV_ACCEPT_REJECT && mode != CPV_ACCEPT_GUMBEL)
        return cpv_fail(ctx, CPV_EINVAL, "spec_accept: unknown mode %d", mode);
    if (mode == CPV_ACCEPT_GUMBEL && !noise_dev) return cpv_fail(ctx, CPV_EINVAL, "spec_accept: gumbel needs noise");
    cpv_status st;
    const int K1 = k + 1, nrow_p = b * K1;
    if (mode == CPV_ACCEPT_GREEDY || (mode == CPV_ACCEPT_GUMBEL && params && coupling_is_exact(params))) {
        void* ws = nullptr;
        if ((st = cpv_workspace(ctx, align256((size_t)nrow_p * 4), &ws))) return st;
        int32_t* am = (int32_t*)ws;
        if ((st = cpv_argmax_rows(ctx, p_logits_dev, mode == CPV_ACCEPT_GUMBEL ? noise_dev : nullptr, nrow_p, v, am)))
            return st;
        decide_argmax_kernel<<<(unsigned)((b + 63) / 64), 64, 0, ctx->stream>>>(am, draft_dev, b, k, out_tok_dev,
                                                                                out_n_dev);
        CPV_HIP(ctx, hipGetLastError());
        return CPV_OK;
    }
    if ((st = check_params(ctx, params, hist_dev ? hist_len : 0))) return st;
    const bool has_q = mode == CPV_ACCEPT_REJECT && q_logits_dev && k > 0;
    const int rows = nrow_p + (has_q ? b * k : 0);
    const bool pen = penalties_on(params) && params->penalty_last_n > 0;
    const size_t db = dist_bytes(rows, v, pen);
    const size_t qb = has_q ? align256((size_t)b * v * 4) : 0;
    void* ws = nullptr;
    if ((st = cpv_workspace(ctx, db + qb, &ws))) return st;
    DistBufs d = dist_carve(ws, rows, v, pen);
    DistArgs a{};
    a.p_logits = p_logits_dev;
    a.q_logits = has_q ? q_logits_dev : nullptr;
    a.draft = draft_dev;
    a.hist = hist_dev;
    a.B = b;
    a.k = k;
    a.V = v;
    a.hist_len = hist_dev ? hist_len : 0;
    a.nrow_p = nrow_p;
    a.direct = 0;
    a.prm = *params;
    a.ln_min_p = params->min_p > 0.0f ? logf(params->min_p) : 0.0f;
    a.pen_on = pen;
    a.pen = d.pen;
    a.sid = d.sid;
    a.sl = d.sl;
    a.pr = d.pr;
    a.hdr = d.hdr;
    a.st = d.st;
    a.bkeys = d.bkeys;
    a.e2 = d.e2;
    if ((st = dist_launch(ctx, a, rows))) return st;
    DecideArgs c{};
    c.draft = draft_dev;
    c.u = u_dev;
    c.seed = philox_seed;
    c.round = philox_round;
    c.noise = noise_dev;
    c.B = b;
    c.k = k;
    c.V = v;
    c.mode = mode;
    c.has_q = has_q;
    c.nrow_p = nrow_p;
    c.T = params->temp;
    c.inv_t = 1.0f / fmaxf(params->temp, FLT_MIN);
    c.sid = d.sid;
    c.sl = d.sl;
    c.pr = d.pr;
    c.hdr = d.hdr;
    c.qdense = has_q ? (float*)d.tail : nullptr;
    c.out_tok = out_tok_dev;
    c.out_n = out_n_dev;
    decide_kernel<<<(unsigned)b, SB, 0, ctx->stream>>>(c);
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}
