// attn.hip — tree-masked GQA attention over the f16 KV cache, exact and
// order-free: the same bits whatever the grid or the number of query rows in
// a call (the oracle's cpvo_attn states the contract).
//
// Replaces the attention of build_attn_block (crates/codpiece-model/src/
// qwen35.rs:3182-3199), by default ggml_flash_attn_ext with prec F32 (the
// session's fa flag, qwen35.rs:534): q rounded to f16, weights expf(s - max),
// the normalisation deferred to the end.  Here every sum is exact or in a
// fixed order:
//  1. scores: q16 and each cache row k16 become 15-bit fixed point relative
//     to their own largest element (qf = rint(q16 2^(14-Eq)), kf likewise);
//     s = (float)(sum_d qf kf * 2^(Eq+Ek-28)), the sum exact -- here on the
//     int8 MFMA with two signed 8-bit limbs per operand; w = s * scale.
//  2. per chunk c of 128 cache rows (absolute rows), over its visible rows:
//     m_c = max w, e = expf(w - m_c), the weight p = rint(e 2^22) and each
//     value vq = rint(f16(v) 2^14), both integers; S_c = sum p vq and
//     Z_c = sum p, exact -- here on the int8 MFMA (3 signed 8-bit limbs of p,
//     4 of vq); P_c = (float)S_c * 2^-36.
//  3. M = max m_c, f_c = expf(m_c - M); in chunk order Zt += (Z_c 2^-22) f_c
//     (binary64) and O = fma(P_c, f_c, O) (f32); out = O * (float)(1 / Zt).
//
// Kernels: chunk (grid: chunk x KV head x query block of 32, 48 or 80 rows;
// scores on the MFMA, then the chunk's softmax and its P_c in the same
// workgroup) and fold (one block per query row), and over the API's caches a
// first launch that makes the query rows' limbs once.  Scratch in the context
// workspace: P (per chunk and query row, D f32: [chunks][T*H][D] for a
// consumer's fold, [T*H][chunks][D] for the fold here), m [chunks][T*H] f32,
// Z [chunks][T*H] int64, the query limbs.
//
// Layout.  A session's caches hold limbs, written once per row and read by
// the MFMAs with no conversion: K as each row's hi and lo limbs per KV head
// (cpv_k_row_bytes), then the heads' exponents as a plane [h_kv][v_stride]
// (a chunk's 128 exponents of one head in 512 contiguous bytes), V as vq's
// limbs, [h_kv * d][v_stride / 16][4][16].  The API's caches (cpv_attn) are f16:
// K [n_ctx][h_kv * d] and the transposed V [h_kv * d][v_stride] (the
// reference's non-FA V layout, qwen35.rs:580-586), converted in the kernel.
// Either way the KV axis is the reduction axis of P V.
#include <math.h>

#include "cpv_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int CHUNK = 128;          // cache rows per chunk (the unit of the contract)
constexpr int PBITS = 22;           // a weight e in (0, 1] as p = rint(e 2^22): PL limbs
constexpr int PL = 3;
constexpr int VBITS = CPV_ATTN_VBITS;   // an f16 value v as vq = rint(v 2^14): |vq| < 2^30, VLIMBS limbs
constexpr int VLIMBS = CPV_ATTN_VLIMBS;
constexpr int QB_CHAIN = 32;        // query rows per chunk workgroup: chains, prefill, fewer than 512 units;
constexpr int QB_WIDE = 48;         //   from 512 (chunk, KV head) units on, when a KV head has more than 32,
constexpr int QB_TREE = 80;         //   or, over the API's caches, 49 to 80 (a 16-node tree's 5 x 16)
constexpr int E_EMPTY = CPV_E_EMPTY;   // exponent of an all-zero vector

__device__ __forceinline__ int ceil_log2_dev(int64_t v)
{
    int b = 0;
    while (((int64_t)1 << b) < v) b++;
    return b;
}

// node t and its ancestors; a link that does not point to an earlier node
// ends the walk (so a malformed array cannot loop)
__device__ __forceinline__ uint64_t ancestors(const int32_t* parent, int t)
{
    uint64_t m = 0;
    for (int a = t; a >= 0 && a < 64;) {
        m |= 1ull << a;
        const int p = parent[a];
        if (p >= a) break;
        a = p;
    }
    return m;
}

struct ChunkArgs {
    const float* q;           // [T][H][D] (LC kernels)
    const int8_t* qlim;       // the same rows (t * H + h) as limbs (the others): [T*H][2][D], the D hi
    const int32_t* qexp;      //   limbs then the D lo; [T*H] the rows' exponents
    const uint16_t* kc;       // [n_ctx][Hkv*D]
    const uint16_t* vt;       // [Hkv*D][v_stride]
    const int32_t* parent;    // [T] or null
    float* P;                 // partial of chunk c, query row r: P + c p_cs + r p_rs, D floats
    int64_t p_cs, p_rs;       //   ([chunks][T*H][D] for a consumer's fold, [T*H][chunks][D] for attn_fold_kernel)
    float* mc;                // [chunks][T*H]
    long long* zc;            // [chunks][T*H]
    int64_t n_past, n, v_stride;   // n = n_past + T rows in play
    int T, H, Hkv;
    float scale;
    const int64_t* pos;       // when set, n_past is pos[pos_sel] (device memory, read at run
    int pos_sel;              // time) and the grid may hold chunks past the end, which exit
    int64_t kv_rows;          // rows the K cache holds (loads stay below it; v_stride for V)
    const int8_t* vl;         // the session's V cache as limbs (LC kernels): [Hkv*D][v_stride / 16][VLIMBS][16]
    const int8_t* kl;         // the session's K cache as limbs (LC kernels): rows of k_row bytes, then
    int64_t k_row;            // the exponent plane [Hkv][v_stride] (cpv_k_exps)
    int fwd;                  // chunks in dispatch order first to last (no pos)
};

// an integer as L signed 8-bit limbs, x = sum l_i 256^i with l_i in
// [-128, 127] below the top limb (which takes the rest), as the bytes of one
// dword: byte i of x + K (K = 128 in each lower byte) is l_i + 128 below the
// top, the top limb itself last, so XOR with K leaves each l_i
template <int L>
__device__ __forceinline__ uint32_t packed_limbs(int x)
{
    constexpr uint32_t K = 0x80808080u >> (8 * (5 - L));
    return ((uint32_t)x + K) ^ K;
}

// out[p] = byte p of w[0], w[1], w[2], w[3] (w[0]'s lowest), p < L: four
// values' limb p side by side, as the MFMA operands take them
// (v_perm_b32 picks bytes 0-3 from its second source, 4-7 from its first)
template <int L>
__device__ __forceinline__ void limb_transpose(const uint32_t* w, uint32_t* out)
{
    const uint32_t a01 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);   // w0.0 w1.0 w0.1 w1.1
    const uint32_t a23 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
    out[0] = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
    if constexpr (L > 2) {
        const uint32_t b01 = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);   // w0.2 w1.2 w0.3 w1.3
        const uint32_t b23 = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
        out[2] = __builtin_amdgcn_perm(b23, b01, 0x05040100u);
        if constexpr (L > 3) out[3] = __builtin_amdgcn_perm(b23, b01, 0x07060302u);
    }
}

// the limbs of 16 f16-exact values at the exponent of the largest |value| of
// their row (a row spans TPR consecutive lanes): lo[j] and hi[j] hold values
// 4j .. 4j + 3
template <int TPR>
__device__ __forceinline__ int row_limbs(const float* v, uint32_t* hi, uint32_t* lo)
{
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = cpv_group_reduce<TPR>(mx, cpv_op_max());   // a row's lanes are all active or all idle
    int e = E_EMPTY;
    if (mx > 0.0f) frexpf(mx, &e);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t w[4], t[2];
#pragma unroll
        for (int k = 0; k < 4; k++) w[k] = packed_limbs<2>(cpv_k_fixed(v[4 * j + k], e));
        limb_transpose<2>(w, t);
        lo[j] = t[0];
        hi[j] = t[1];
    }
    return e;
}

// The query rows as the chunk kernels take them (once per call, not once per
// chunk): each element rounded to f16, the row's exponent, the two limbs.
// TPR lanes per row, 16 values each.
template <int D>
__global__ __launch_bounds__(256) void q_limbs_kernel(const float* __restrict__ q, int rows, int8_t* __restrict__ qlim,
                                                      int32_t* __restrict__ qexp)
{
    constexpr int TPR = D / 16;
    const int g = blockIdx.x * 256 + threadIdx.x, row = g / TPR, sub = g % TPR;
    const int rc = row < rows ? row : rows - 1;   // (the row's lanes reduce together: all active)
    const float4* src = (const float4*)(q + (int64_t)rc * D + sub * 16);
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 x = src[i];
        v[4 * i + 0] = cpv_h2f(cpv_f2h(x.x));
        v[4 * i + 1] = cpv_h2f(cpv_f2h(x.y));
        v[4 * i + 2] = cpv_h2f(cpv_f2h(x.z));
        v[4 * i + 3] = cpv_h2f(cpv_f2h(x.w));
    }
    uint32_t hi[4], lo[4];
    const int e = row_limbs<TPR>(v, hi, lo);
    if (row < rows) {
        int8_t* dst = qlim + (int64_t)row * 2 * D + sub * 16;
        *(uint4*)dst = uint4{hi[0], hi[1], hi[2], hi[3]};
        *(uint4*)(dst + D) = uint4{lo[0], lo[1], lo[2], lo[3]};
        if (sub == 0) qexp[row] = e;
    }
}

// one 128-row chunk of the cache against QB query rows of one KV head
constexpr int CT = 512;             // threads of a chunk workgroup (8 waves)

// LC: K and V come from a session's limb caches (a.kl, a.vl); else from the
// API's f16 caches (a.kc, a.vt), converted here.  QB: query rows per
// workgroup, a multiple of 16 (MFMA row blocks)
template <int D, bool LC, int QB>
__global__ __launch_bounds__(CT) void attn_chunk_kernel(ChunkArgs a)
{
    static_assert(QB % 16 == 0, "16-row query blocks");
    constexpr int QBB = QB / 16;               // query row blocks
    constexpr int TPR = D / 16;                // threads per row when converting (16 values each)
    constexpr int RPP = CT / TPR;              // rows per pass
    constexpr int QP = (QB + RPP - 1) / RPP;   // query conversion passes
    // rows padded by 16 bytes (limbs) and 4 floats (scores): the MFMA operand
    // reads and the score writes then fall on distinct LDS banks.  One buffer
    // holds the phases in turn: the K limbs at 0 and the query limbs after
    // them until the score MFMAs are done; the weights' limbs at 0 once the
    // scores are done.  The scores lie after the query limbs, or, for more
    // than 32 query rows (OVL), at PBUF over both (a barrier after the score
    // MFMAs): 52 KB a workgroup at 48 rows and d = 128, so that two share a
    // CU (at 78 KB one ran per CU).  Past 48 rows the scores wait in
    // registers and go through the LDS and the softmax WR rows at a time.
    constexpr bool OVL = QB > QB_CHAIN;
    constexpr int WR = QB > QB_WIDE ? QB_WIDE : QB, NH = (QB + WR - 1) / WR;
    static_assert(WR % 16 == 0, "score halves of whole row blocks");
    constexpr int KBUF = 2 * CHUNK * (D + 16), PBUF = PL * QB * (CHUNK + 16);
    constexpr int QS = 2 * QB * (D + 16), WS = WR * (CHUNK + 4) * (int)sizeof(float);
    constexpr int KQ = (KBUF > PBUF ? KBUF : PBUF) + QS;
    constexpr int WOFF = OVL ? PBUF : KQ;
    constexpr int UBUF = KQ > WOFF + WS ? KQ : WOFF + WS;
    static_assert(PBUF % 16 == 0 && KBUF % 16 == 0, "16-byte aligned phases");
    __shared__ __align__(16) int8_t s_buf[UBUF];
    int8_t(*s_kh)[D + 16] = (int8_t(*)[D + 16]) & s_buf[0];
    int8_t(*s_kl)[D + 16] = (int8_t(*)[D + 16]) & s_buf[CHUNK * (D + 16)];
    int8_t(*s_qh)[D + 16] = (int8_t(*)[D + 16]) & s_buf[KQ - QS];
    int8_t(*s_ql)[D + 16] = (int8_t(*)[D + 16]) & s_buf[KQ - QS + QB * (D + 16)];
    float(*s_w)[CHUNK + 4] = (float(*)[CHUNK + 4]) & s_buf[WOFF];                // scores
    int8_t(*s_p)[QB][CHUNK + 16] = (int8_t(*)[QB][CHUNK + 16]) & s_buf[0];      // [PL][query row][cache row]
    __shared__ int s_eq[QB], s_ek[CHUNK];
    __shared__ unsigned long long s_anc[QB];
    __shared__ int s_vis[QB], s_orow[QB];      // (per query row; set with its limbs)
    __shared__ uint64_t s_etab[32];                     // the expf table
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 32) {
        constexpr uint64_t etab[32] = CPV_EXP2F_TAB;
        s_etab[tid] = etab[tid];
    }
    // KV head fastest, chunks last to first: the first blocks dispatched are
    // those past the end (which exit at once) and the short last chunk (which
    // costs little below), so the blocks that a full grid places on a CU
    // beside another are full chunks beside those.  A grid of more blocks
    // than two a CU (fwd) runs first to last: the short chunk then comes in
    // the last round, not a full one.
    const int cq = (int)(blockIdx.x / a.Hkv), kh = blockIdx.x % a.Hkv;
    const int c = a.fwd ? cq : (int)(gridDim.x / a.Hkv) - 1 - cq;
    const int64_t j0 = (int64_t)c * CHUNK;
    const int G = a.H / a.Hkv, LR = G * a.T;
    const int sub = tid % TPR;
    const bool tree = a.parent != nullptr;

    // The grid's last 8 chunks may lie past the end or hold the short last
    // one (a replayed round's grid serves a 1024-row range).  There n_past is
    // read first: a chunk past the end exits before any load, and a bounded
    // chunk's loads stay below row n (the rows past it read row n - 1 again).
    const bool tail = a.pos != nullptr && c >= (int)(gridDim.x / a.Hkv) - 8;
    const bool bounded = a.pos == nullptr || tail;
    int64_t n_past = a.n_past;
    if (tail) {
        n_past = a.pos[a.pos_sel];
        if (j0 >= n_past + a.T) return;        // (the whole workgroup, before any barrier)
    }
    const int64_t lim = bounded ? n_past + a.T : a.kv_rows;   // (a.kv_rows = n without positions)

    // ---- q and K go out first, at clamped (in-bounds) rows, with no branch
    // around a load (a branch makes the compiler wait for every load at the join)
    constexpr int KP = CHUNK / RPP > 0 ? CHUNK / RPP : 1;   // K passes
    const int rq = tid / TPR;                  // query row converted by this thread in pass 0
    // (LC: the f32 rows, made into limbs below; else their limbs as made by
    // q_limbs_kernel, once per call)
    float4 qv[LC ? QP : 1][4];
    uint4 qlv[LC ? 1 : QP][2];
    int qev[LC ? 1 : QP];
#pragma unroll
    for (int qp = 0; qp < QP; qp++) {          // (rows past QB or LR read row 0)
        const int lrq = blockIdx.z * QB + rq + qp * RPP;
        const int lrc = rq + qp * RPP < QB && lrq < LR ? lrq : 0;
        const int64_t qrow = (int64_t)(lrc / G) * a.H + kh * G + lrc % G;
        if constexpr (LC) {
            const float* src = a.q + qrow * D + sub * 16;
#pragma unroll
            for (int i = 0; i < 4; i++) qv[qp][i] = ((const float4*)src)[i];
        } else {
            const int8_t* src = a.qlim + qrow * 2 * D + sub * 16;
            qlv[qp][0] = *(const uint4*)src;
            qlv[qp][1] = *(const uint4*)(src + D);
            qev[qp] = a.qexp[qrow];
        }
    }
    // (elsewhere rows clamped to the cache's: the chunk's end is known once n_past is)
    // LC: kv[p] = 16 hi limbs, 16 lo limbs of the row's head, ekv[p] its exponent
    uint4 kv[KP][2];
    int ekv[KP];
#pragma unroll
    for (int p = 0; p < KP; p++) {
        const int64_t row = j0 + rq + p * RPP, rc = row < lim ? row : lim - 1;
        if constexpr (LC) {
            const int8_t* src = a.kl + rc * a.k_row + (int64_t)kh * 2 * D + sub * 16;
            kv[p][0] = *(const uint4*)src;
            kv[p][1] = *(const uint4*)(src + D);
            ekv[p] = *(const int32_t*)(a.kl + a.v_stride * a.k_row + 4 * ((int64_t)kh * a.v_stride + rc));
        } else {
            const uint16_t* src = a.kc + rc * (int64_t)a.Hkv * D + (int64_t)kh * D + sub * 16;
            kv[p][0] = *(const uint4*)src;
            kv[p][1] = *(const uint4*)(src + 8);
        }
    }
    if (a.pos && !tail) n_past = a.pos[a.pos_sel];
    const int64_t n_all = n_past + a.T;
    if (j0 >= n_all) return;                   // a chunk past the end (the whole workgroup, before any barrier)
    const int nj = (int)(n_all - j0 < CHUNK ? n_all - j0 : CHUNK);
    // ---- query rows lr = blockIdx.z * QB + r: token t = lr / G, head kh * G + lr % G
#pragma unroll
    for (int qp = 0; qp < QP; qp++) {
        const int r = rq + qp * RPP;
        if (r >= QB) break;                    // (threads past the block's rows in the last pass)
        const int lrq = blockIdx.z * QB + r;
        const bool qok = lrq < LR;
        const int lrc = qok ? lrq : 0;
        // (a row past LR: all-zero limbs, as an all-zero row has)
        int e;
        if constexpr (LC) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[4 * i + 0] = qok ? cpv_h2f(cpv_f2h(qv[qp][i].x)) : 0.0f;
                v[4 * i + 1] = qok ? cpv_h2f(cpv_f2h(qv[qp][i].y)) : 0.0f;
                v[4 * i + 2] = qok ? cpv_h2f(cpv_f2h(qv[qp][i].z)) : 0.0f;
                v[4 * i + 3] = qok ? cpv_h2f(cpv_f2h(qv[qp][i].w)) : 0.0f;
            }
            uint32_t hi[4], lo[4];
            e = row_limbs<TPR>(v, hi, lo);
            *(uint4*)&s_qh[r][sub * 16] = uint4{hi[0], hi[1], hi[2], hi[3]};
            *(uint4*)&s_ql[r][sub * 16] = uint4{lo[0], lo[1], lo[2], lo[3]};
        } else {
            *(uint4*)&s_qh[r][sub * 16] = qok ? qlv[qp][0] : uint4{0, 0, 0, 0};
            *(uint4*)&s_ql[r][sub * 16] = qok ? qlv[qp][1] : uint4{0, 0, 0, 0};
            e = qok ? qev[qp] : E_EMPTY;
        }
        if (sub == 0) {
            // the row's visible cache rows in this chunk: the first s_vis of
            // them (the context, and for a chain its nodes up to t), then for
            // a tree the ancestors' bits of s_anc; nothing for a row past LR
            const int t = lrc / G;
            const int64_t vis = (tree ? n_past : n_past + t + 1) - j0;
            s_eq[r] = e;
            s_vis[r] = !qok ? 0 : vis < 0 ? 0 : vis < nj ? (int)vis : nj;
            s_anc[r] = (tree && qok) ? ancestors(a.parent, t) : 0ull;
            s_orow[r] = t * a.H + kh * G + lrc % G;
        }
    }
    // ---- the chunk's cache rows of this KV head
#pragma unroll
    for (int p = 0; p < KP; p++) {
        const int r = rq + p * RPP;
        if (r >= CHUNK) break;                 // (threads past the chunk when d = 64)
        if constexpr (LC) {
            // the cache's limbs as they are; rows past the chunk's end as an all-zero row
            const bool in = r < nj;
            *(uint4*)&s_kh[r][sub * 16] = in ? kv[p][0] : uint4{0, 0, 0, 0};
            *(uint4*)&s_kl[r][sub * 16] = in ? kv[p][1] : uint4{0, 0, 0, 0};
            if (sub == 0) s_ek[r] = in ? ekv[p] : E_EMPTY;
            continue;
        }
        const uint32_t wds[8] = {kv[p][0].x, kv[p][0].y, kv[p][0].z, kv[p][0].w,
                                 kv[p][1].x, kv[p][1].y, kv[p][1].z, kv[p][1].w};
        uint32_t hi[4] = {0, 0, 0, 0}, lo[4] = {0, 0, 0, 0};   // (what row_limbs gives an all-zero row)
        int e = E_EMPTY;
        if (r < nj) {                          // the same for the TPR lanes of a row
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = cpv_h2f((uint16_t)(wds[i >> 1] >> (16 * (i & 1))));
            e = row_limbs<TPR>(v, hi, lo);
        }
        *(uint4*)&s_kh[r][sub * 16] = uint4{hi[0], hi[1], hi[2], hi[3]};
        *(uint4*)&s_kl[r][sub * 16] = uint4{lo[0], lo[1], lo[2], lo[3]};
        if (sub == 0) s_ek[r] = e;
    }
    // ---- this wave's V operands, in flight through the scores and the
    // softmax: d-block cb (16 columns), the chunk's rows in two 64-row steps;
    // lane (c16, g4) holds column 16 cb + c16 and rows 64 ks + 16 g4 .. +15,
    // the B operands of the P V MFMAs, as the VLIMBS signed 8-bit limbs of
    // vq = rint(v 2^VBITS).  Segments past the cache's end (wholly: v_stride
    // is a multiple of 16, or of 8 for halves) read its last one, and in a
    // bounded chunk those past n read the one holding row n - 1; those rows
    // carry weight 0.
    constexpr int NCB = D / 16;                 // d-blocks
    static_assert((CT / 64) % NCB == 0, "waves per d-block");
    const int cb = wave % NCB, c16 = lane & 15, g4 = lane >> 4;
    const int dcol = cb * 16 + c16;
    v4i vb[2][VLIMBS];
    const int64_t vlast16 = bounded ? (lim - 1) & ~(int64_t)15 : a.v_stride - 16;
    const int64_t vlast8 = bounded ? (lim - 1) & ~(int64_t)7 : a.v_stride - 8;
    uint4 vraw[2][2];
    if constexpr (LC) {
        // (a segment's limbs lie together: one 64-byte read)
        const int8_t* vbase = a.vl + ((int64_t)kh * D + dcol) * a.v_stride * VLIMBS;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int64_t sj = j0 + ks * 64 + g4 * 16, sjc = sj <= vlast16 ? sj : vlast16;
#pragma unroll
            for (int l = 0; l < VLIMBS; l++) vb[ks][l] = *(const v4i*)(vbase + sjc * VLIMBS + 16 * l);
        }
    } else {
        const uint16_t* vrow = a.vt + ((int64_t)kh * D + dcol) * a.v_stride;
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int64_t sj = j0 + ks * 64 + g4 * 16 + 8 * h, sjc = sj <= vlast8 ? sj : vlast8;
                vraw[ks][h] = *(const uint4*)(vrow + sjc);
            }
    }
    __syncthreads();

    // ---- scores: QBB x 8 blocks of 16 x 16 (query rows x cache rows); wave
    // w takes blocks w + 8 b, b < QBB, side by side, so that their MFMA
    // chains interleave.  A block past the chunk's end meets all-zero K rows
    // (S = 0) and is written as -inf, as every invisible score is; a chunk of
    // at most 64 rows (the short last one) has only its first half read
    // below, and the softmax and P V skip the second
    const bool half = nj <= CHUNK / 2;
    float scv[NH > 1 ? QBB : 1][4];            // this lane's scores (masked), past 48 rows
    {
        const int kg = (lane >> 4) * 16;
        v4i hh[QBB], mix[QBB], ll[QBB];
#pragma unroll
        for (int b = 0; b < QBB; b++) hh[b] = mix[b] = ll[b] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < D / 64; ks++)
#pragma unroll
            for (int b = 0; b < QBB; b++) {
                const int blk = wave + (CT / 64) * b, qb = blk % QBB, jb = blk / QBB;
                const int ar = qb * 16 + (lane & 15), bc = jb * 16 + (lane & 15);
                const v4i qhv = *(const v4i*)&s_qh[ar][ks * 64 + kg], qlv = *(const v4i*)&s_ql[ar][ks * 64 + kg];
                const v4i khv = *(const v4i*)&s_kh[bc][ks * 64 + kg], klv = *(const v4i*)&s_kl[bc][ks * 64 + kg];
                hh[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qhv, khv, hh[b], 0, 0, 0);
                mix[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qhv, klv, mix[b], 0, 0, 0);
                mix[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qlv, khv, mix[b], 0, 0, 0);
                ll[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qlv, klv, ll[b], 0, 0, 0);
            }
        if constexpr (OVL) __syncthreads();   // (the scores overwrite the q and K limbs)
#pragma unroll
        for (int b = 0; b < QBB; b++) {
            const int blk = wave + (CT / 64) * b, qb = blk % QBB, jb = blk / QBB;
            const int bc = jb * 16 + (lane & 15);
            // lane holds query rows 4 (lane/16) + i of the block, cache row bc.
            // S = hh 2^16 + mix 2^8 + ll is exact in binary64 (|S| < 2^37), the
            // score one rounding of S 2^(eq+ek-28): 0 when either row is all
            // zero, as its limbs are
            const int ek = s_ek[bc];
            const int64_t node = j0 + bc - n_past;   // (a tree node when in [0, 64))
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = qb * 16 + 4 * (lane >> 4) + i;
                bool vis = bc < s_vis[r];
                if (tree) vis = vis || ((uint64_t)node < 64 && ((s_anc[r] >> node) & 1ull));
                const double S = __builtin_fma((double)hh[b][i], 65536.0, (double)(mix[b][i] * 256 + ll[b][i]));
                const float sc = (float)ldexp(S, s_eq[r] + ek - 28);
                const float wv = vis ? sc * a.scale : -INFINITY;
                if constexpr (NH == 1) s_w[r][bc] = wv;
                else scv[b][i] = wv;
            }
        }
    }

    // ---- the chunk's softmax: SPR threads per query row, 8 cache rows each
    // (4 part + 64 i + k: 16-byte reads of the scores, one dword per limb
    // written), CT / SPR rows per pass; the weights in fixed point,
    // p = rint(e 2^PBITS), as PL signed 8-bit limbs, and Z_c = sum p.  The
    // scores of rows h WR .. (h + 1) WR - 1 go to the LDS first (the blocks
    // of a wave's b are whole in one of them: wave-uniform).
    constexpr int SPR = CHUNK / 8, SRP = CT / SPR;
    static_assert(WR % (SRP / 2) == 0 && QB % (SRP / 2) == 0, "softmax passes of whole waves");
#pragma unroll
    for (int h = 0; h < NH; h++) {
    if constexpr (NH > 1) {
        if (h > 0) __syncthreads();            // (the previous rows' scores are read)
#pragma unroll
        for (int b = 0; b < QBB; b++) {
            const int blk = wave + (CT / 64) * b, qb = blk % QBB, jb = blk / QBB;
            if (qb * 16 / WR != h) continue;
            const int bc = jb * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; i++) s_w[qb * 16 + 4 * (lane >> 4) + i - h * WR][bc] = scv[b][i];
        }
    }
    __syncthreads();
    const int rend = (h + 1) * WR < QB ? (h + 1) * WR : QB;
#pragma unroll
    for (int r0 = h * WR; r0 < rend; r0 += SRP) {
        const int r = r0 + tid / SPR, part = tid % SPR;
        if (r >= rend) break;                  // (a half pass: whole waves past the rows)
        const int lr = blockIdx.z * QB + r;
        float w[8];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float4 w4 = i == 0 || !half ? *(const float4*)&s_w[r - h * WR][4 * part + 64 * i]
                                              : float4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            w[4 * i] = w4.x;
            w[4 * i + 1] = w4.y;
            w[4 * i + 2] = w4.z;
            w[4 * i + 3] = w4.w;
        }
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; i++) m = fmaxf(m, w[i]);
        m = cpv_group_reduce<SPR>(m, cpv_op_max());
        int z = 0;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if (i == 1 && half) break;
            uint32_t wq[4], pk[PL];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float wv = w[4 * i + k];
                const int qe = (int)rintf(ldexpf(cpv_expf_sel(wv - m, s_etab), PBITS));   // (every lane)
                const int q = wv != -INFINITY ? qe : 0;
                z += q;
                wq[k] = packed_limbs<PL>(q);
            }
            limb_transpose<PL>(wq, pk);
#pragma unroll
            for (int p = 0; p < PL; p++) *(uint32_t*)&s_p[p][r][4 * part + 64 * i] = pk[p];
        }
        z = cpv_group_reduce<SPR>(z, cpv_op_add());
        if (part == 0 && lr < LR) {
            const int64_t row = (int64_t)c * a.T * a.H + s_orow[r];
            a.mc[row] = m;
            a.zc[row] = z;
        }
    }
    }
    // (the f16 cache's values into limbs meanwhile)
    if constexpr (!LC) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            uint32_t pk[VLIMBS][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {      // values 4j .. 4j + 3 of the segment: half j / 2 of the raw read
                const uint4 raw = vraw[ks][j >> 1];
                const uint32_t wd[2] = {(j & 1) ? raw.z : raw.x, (j & 1) ? raw.w : raw.y};
                uint32_t w[4], t[VLIMBS];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    w[k] = packed_limbs<VLIMBS>(
                        (int)rintf(ldexpf(cpv_h2f((uint16_t)(wd[k >> 1] >> (16 * (k & 1)))), VBITS)));
                limb_transpose<VLIMBS>(w, t);
#pragma unroll
                for (int p = 0; p < VLIMBS; p++) pk[p][j] = t[p];
            }
#pragma unroll
            for (int p = 0; p < VLIMBS; p++) vb[ks][p] = v4i{(int)pk[p][0], (int)pk[p][1], (int)pk[p][2], (int)pk[p][3]};
        }
    }
    __syncthreads();

    // ---- P_c on the int8 MFMA: for row block rb (16 query rows) and this
    // wave's d-block, the limb products p_a v_b go to accumulator a + b
    // (weight 2^(8 (a + b))); S = sum of them exactly in int64 (|S| < 2^59);
    // P_c = (float)S * 2^-(PBITS + VBITS).  A lane holds D rows 4 g4 .. +3 of
    // column c16.  Where the wave's values of a 64-row step all have a zero
    // top limb (|v| < 2^(8 (VLIMBS - 1) - 1 - VBITS), 512 for f16 values at
    // 2^14), that limb's products are zero and their MFMAs are skipped.
    bool vtop[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const v4i t = vb[ks][VLIMBS - 1];
        vtop[ks] = __builtin_amdgcn_ballot_w64((t[0] | t[1] | t[2] | t[3]) != 0) != 0;   // (wave-uniform)
    }
    for (int rb = wave / NCB; rb < QB / 16; rb += CT / 64 / NCB) {
        if (blockIdx.z * QB + rb * 16 >= LR) break;   // (wave-uniform) past the query rows
        v4i acc[PL + VLIMBS - 1];
#pragma unroll
        for (int q = 0; q < PL + VLIMBS - 1; q++) acc[q] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            if (ks == 1 && half) break;
            v4i pa[PL];
#pragma unroll
            for (int p = 0; p < PL; p++) pa[p] = *(const v4i*)&s_p[p][rb * 16 + c16][ks * 64 + g4 * 16];
#pragma unroll
            for (int p = 0; p < PL; p++)
#pragma unroll
                for (int l = 0; l < VLIMBS - 1; l++)
                    acc[p + l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa[p], vb[ks][l], acc[p + l], 0, 0, 0);
            if (vtop[ks]) {
#pragma unroll
                for (int p = 0; p < PL; p++)
                    acc[p + VLIMBS - 1] =
                        __builtin_amdgcn_mfma_i32_16x16x64_i8(pa[p], vb[ks][VLIMBS - 1], acc[p + VLIMBS - 1], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int lr = blockIdx.z * QB + rb * 16 + 4 * g4 + i;
            if (lr >= LR) break;
            float pc;
            if (!vtop[0] && !vtop[1]) {
                // (wave-uniform) no top value limb: |vq| < 2^23, so |S| < 2^22 2^23
                // 128 < 2^52 and every step of the limb sum below is exact in
                // binary64; one rounding to f32, as from the int64 sum
                double Sd = (double)acc[PL + VLIMBS - 3][i];
#pragma unroll
                for (int q = PL + VLIMBS - 4; q >= 0; q--) Sd = __builtin_fma(Sd, 256.0, (double)acc[q][i]);
                pc = (float)Sd;
            } else {
                int64_t S = 0;
#pragma unroll
                for (int q = 0; q < PL + VLIMBS - 1; q++) S += (int64_t)acc[q][i] * ((int64_t)1 << (8 * q));
                pc = (float)S;
            }
            a.P[(int64_t)c * a.p_cs + (int64_t)s_orow[rb * 16 + 4 * g4 + i] * a.p_rs + dcol] =
                ldexpf(pc, -(PBITS + VBITS));
        }
    }
}

// one query row: the chunks folded in order, then the normalisation.  The
// chunk maxima, sums and factors are staged in LDS; empty chunks (no visible
// row) carry factor 0 and zero partials, which leave both folds unchanged.
// Threads 0 .. D-1 fold one column each; a third wave's first lane sums Z
// meanwhile (a serial binary64 chain, off the folds' path).
template <int D>
__global__ __launch_bounds__(D + 64) void attn_fold_kernel(const float* __restrict__ P, const float* __restrict__ mc,
                                                           const long long* __restrict__ zc, int nchunk, int rows,
                                                           float* __restrict__ out)
{
    constexpr int NT = D + 64, NW = NT / 64;
    extern __shared__ double s_dyn[];          // [nchunk] Z_c 2^-PBITS, then [nchunk] factors f_c
    double* s_z = s_dyn;
    float* s_f = (float*)(s_dyn + nchunk);
    __shared__ float s_red[NW];
    __shared__ float s_inv;
    const int row = blockIdx.x, d = threadIdx.x, lane = d & 63, wave = d >> 6;
    float M = -INFINITY;
    for (int c = d; c < nchunk; c += NT) {
        const float m = mc[(int64_t)c * rows + row];
        s_f[c] = m;
        s_z[c] = ldexp((double)zc[(int64_t)c * rows + row], -PBITS);
        M = fmaxf(M, m);
    }
    M = cpv_wave_reduce(M, cpv_op_max());
    if (lane == 0) s_red[wave] = M;
    __syncthreads();
    M = s_red[0];
    for (int i = 1; i < NW; i++) M = fmaxf(M, s_red[i]);
    for (int c = d; c < nchunk; c += NT) {
        const float m = s_f[c];
        s_f[c] = m == -INFINITY ? 0.0f : cpv_expf(m - M);
    }
    __syncthreads();
    float o = 0.0f;
    if (d < D) {                               // (wave-uniform)
        // (a row's partials lie together: [rows][nchunk][D])
        o = cpv_fold_chain<32>(P + (int64_t)row * nchunk * D + d, D, s_f, nchunk);
    } else if (d == D) {
        double Zt = 0.0;
        for (int c = 0; c < nchunk; c++) Zt = Zt + s_z[c] * (double)s_f[c];
        s_inv = (float)(1.0 / Zt);
    }
    __syncthreads();
    if (d < D) out[(int64_t)row * D + d] = o * s_inv;
}

// one call over T query tokens (the scratch holds T*H rows per chunk); with
// out null only the chunk partials are produced (into *part), for a consumer
// that folds them itself
// With pos set (partials only), the grid and the scratch are sized for
// nchunk_grid chunks, at least the call's, and n_past is read on the device.
// Over the API's caches the queries are made into limbs first
// (q_limbs_kernel, once per call); a session's LC kernels convert their own
// (about as fast at a verify's few rows, with no launch of its own).
template <int D>
cpv_status attn_block(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                      int64_t n_past, const int32_t* parent, int T, int H, int Hkv, float scale, float* out,
                      cpv_attn_part* part = nullptr, const int64_t* pos = nullptr, int pos_sel = 0,
                      int nchunk_grid = 0, int64_t kv_rows = 0, const int8_t* vl = nullptr,
                      const int8_t* kl = nullptr)
{
    if ((vl != nullptr) != (kl != nullptr))
        return cpv_fail(ctx, CPV_EINVAL, "attention: a session's K and V limb caches go together");
    const int64_t n = n_past + T;
    const int G = H / Hkv, LR = G * T, rows = T * H;
    int nchunk = (int)((n + CHUNK - 1) / CHUNK);
    if (pos && (out || kv_rows < n))
        return cpv_fail(ctx, CPV_EINVAL, "attention: device positions are for partials over a cache of >= n rows");
    if (pos && nchunk_grid > nchunk) nchunk = nchunk_grid;
    const size_t P_b = ((size_t)nchunk * rows * D * 4 + 255) & ~(size_t)255;
    const size_t m_b = ((size_t)nchunk * rows * 4 + 255) & ~(size_t)255;
    const size_t z_b = ((size_t)nchunk * rows * 8 + 255) & ~(size_t)255;
    const size_t ql_b = vl ? 0 : (((size_t)rows * 2 * D + 255) & ~(size_t)255) + (size_t)rows * 4;
    void* ws = nullptr;
    cpv_status st = cpv_workspace(ctx, P_b + m_b + z_b + ql_b, &ws);
    if (st != CPV_OK) return st;
    ChunkArgs ca;
    ca.q = q;
    ca.qlim = nullptr;
    ca.qexp = nullptr;
    if (!vl) {
        int8_t* ql = (int8_t*)ws + P_b + m_b + z_b;
        int32_t* qe = (int32_t*)(ql + (((size_t)rows * 2 * D + 255) & ~(size_t)255));
        q_limbs_kernel<D><<<(unsigned)(((int64_t)rows * (D / 16) + 255) / 256), 256, 0, ctx->stream>>>(q, rows, ql, qe);
        ca.qlim = ql;
        ca.qexp = qe;
    }
    ca.kc = kc;
    ca.vt = vt;
    ca.parent = parent;
    ca.P = (float*)ws;
    ca.p_cs = out ? D : (int64_t)rows * D;
    ca.p_rs = out ? (int64_t)nchunk * D : D;
    ca.mc = (float*)((uint8_t*)ws + P_b);
    ca.zc = (long long*)((uint8_t*)ws + P_b + m_b);
    ca.n_past = n_past;
    ca.n = n;
    ca.v_stride = v_stride;
    ca.T = T;
    ca.H = H;
    ca.Hkv = Hkv;
    ca.scale = scale;
    ca.pos = pos;
    ca.pos_sel = pos_sel;
    ca.kv_rows = pos ? kv_rows : n;
    ca.vl = vl;
    ca.kl = kl;
    ca.k_row = cpv_k_row_bytes(Hkv, D);
    if (vl && (v_stride % 16 || ((uintptr_t)vl & 15) || ((uintptr_t)kl & 15)))
        return cpv_fail(ctx, CPV_EINVAL, "attention: limb caches need 16-byte aligned rows");
    // a KV head's rows past 32 in blocks of 48 once there are 512 (chunk, KV
    // head) units or more (a 16-node tree's 80 rows in two workgroups per
    // chunk, not three): each stages and converts the chunk's K and V once for
    // more rows, and two still fit a CU.  With fewer units the 32-row blocks'
    // extra workgroups take no more passes over the CUs, and their shorter
    // chains win (the 16-node tree at 4101 rows: 9.59 against 9.71 ms; at
    // 32768 over the API's caches: 200 against 182 us)
    // Over the API's f16 caches, 49 to 80 rows (a 16-node tree's) go in one
    // 80-row block: the chunk's K and V are loaded and converted to limbs
    // once for all of them, not once per 48-row block.
    const bool wide = LR > QB_CHAIN && (int64_t)nchunk * Hkv >= 512;
    const bool tree_blk = wide && !vl && LR > QB_WIDE && LR <= QB_TREE;
    const int QB = tree_blk ? QB_TREE : wide ? QB_WIDE : QB_CHAIN;
    const dim3 cgrid((unsigned)(nchunk * Hkv), 1u, (unsigned)((LR + QB - 1) / QB));
    ca.fwd = !pos && (int64_t)cgrid.x * cgrid.z > 2 * (int64_t)ctx->cu_count;
    if (tree_blk) {
        attn_chunk_kernel<D, false, QB_TREE><<<cgrid, CT, 0, ctx->stream>>>(ca);
    } else if (wide) {
        if (vl) attn_chunk_kernel<D, true, QB_WIDE><<<cgrid, CT, 0, ctx->stream>>>(ca);
        else attn_chunk_kernel<D, false, QB_WIDE><<<cgrid, CT, 0, ctx->stream>>>(ca);
    } else {
        if (vl) attn_chunk_kernel<D, true, QB_CHAIN><<<cgrid, CT, 0, ctx->stream>>>(ca);
        else attn_chunk_kernel<D, false, QB_CHAIN><<<cgrid, CT, 0, ctx->stream>>>(ca);
    }
    if (out)
        attn_fold_kernel<D><<<(unsigned)rows, D + 64, (size_t)nchunk * 12, ctx->stream>>>(ca.P, ca.mc, ca.zc, nchunk,
                                                                                  rows, out);
    CPV_HIP(ctx, hipGetLastError());
    if (part) {
        part->P = ca.P;
        part->mc = ca.mc;
        part->zc = ca.zc;
        part->nchunk = nchunk;
        part->rows = rows;
        part->zbits = PBITS;
        part->pos = pos;
        part->pos_sel = pos_sel;
        part->t = T;
    }
    return CPV_OK;
}

// the chain's scratch per token, and whether T tokens run as one block
template <int D>
bool attn_one_block(int64_t n_past, int t, int h)
{
    const int64_t n = n_past + t;
    const int64_t per_token = (int64_t)h * ((n + CHUNK - 1) / CHUNK) * (D * 4 + 12);
    return ((int64_t)192 << 20) / (per_token + 1) >= t;
}

template <int D>
cpv_status attn_run(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                    int64_t n_past, const int32_t* parent, int t, int h, int h_kv, float scale, float* out,
                    const int8_t* vl, const int8_t* kl)
{
    if (parent)
        return attn_block<D>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out, nullptr, nullptr, 0, 0,
                             0, vl, kl);
    // a long chain runs in token blocks to bound the scratch: node t of a chain sees
    // the rows <= n_past + t, which is what a block starting at t0 sees with n_past + t0
    const int64_t n = n_past + t;
    const int64_t per_token = (int64_t)h * ((n + CHUNK - 1) / CHUNK) * (D * 4 + 12);   // (attn_one_block)
    int64_t tb = ((int64_t)192 << 20) / (per_token + 1);
    if (tb < 1) tb = 1;
    if (tb > t) tb = t;
    for (int t0 = 0; t0 < t; t0 += (int)tb) {
        const int tn = t - t0 < (int)tb ? t - t0 : (int)tb;
        cpv_status st = attn_block<D>(ctx, q + (int64_t)t0 * h * D, kc, vt, v_stride, n_past + t0, nullptr, tn, h,
                                      h_kv, scale, out + (int64_t)t0 * h * D, nullptr, nullptr, 0, 0, 0, vl, kl);
        if (st != CPV_OK) return st;
    }
    return CPV_OK;
}

}  // namespace

cpv_status cpv_attn_launch(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                           int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                           float* out, const int8_t* vl, const int8_t* kl)
{
    auto go = [=]() {
        return d == 128 ? attn_run<128>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out, vl, kl)
                        : attn_run<64>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, out, vl, kl);
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

cpv_status cpv_attn_partials(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                             int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                             cpv_attn_part* part, const int64_t* pos, int pos_sel, int nchunk_grid, int64_t kv_rows,
                             const int8_t* vl, const int8_t* kl)
{
    const int64_t grid_past = pos && (int64_t)nchunk_grid * CHUNK - t > n_past ? (int64_t)nchunk_grid * CHUNK - t : n_past;
    if ((d != 64 && d != 128) || (parent && t > 64) ||
        !(d == 128 ? attn_one_block<128>(grid_past, t, h) : attn_one_block<64>(grid_past, t, h)))
        return CPV_EUNSUPPORTED;   // (no message: the caller takes the unfused path)
    // (a profile replay runs after the caller's frame is gone: its partials'
    // description goes to a scratch copy, not to *part)
    auto go = [=](bool replay) {
        cpv_attn_part scratch{};
        cpv_attn_part* pt = replay ? &scratch : part;
        return d == 128 ? attn_block<128>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, nullptr, pt,
                                          pos, pos_sel, nchunk_grid, kv_rows, vl, kl)
                        : attn_block<64>(ctx, q, kc, vt, v_stride, n_past, parent, t, h, h_kv, scale, nullptr, pt,
                                         pos, pos_sel, nchunk_grid, kv_rows, vl, kl);
    };
    const int ev = cpv_prof_mark(ctx);
    const cpv_status st = go(false);
    if (st == CPV_OK && ev >= 0) {  // algorithmic bytes: K and V rows once, q in (the fold is the consumer's)
        const double bytes = 2.0 * 2.0 * (double)(n_past + t) * h_kv * d + 4.0 * t * h * d;
        cpv_prof_add(ctx, ev, CPV_PROF_ATTN, bytes);
        cpv_prof_keep(ctx, CPV_PROF_ATTN, bytes, [go]() { (void)go(true); });
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
