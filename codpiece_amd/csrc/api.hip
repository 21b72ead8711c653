// api.hip — context, errors, weight upload/repack, get_rows, argmax.
//
// Weight repack.  ggml stores a quantized row as consecutive blocks (Q4_K 144 B,
// Q6_K 210 B, Q8_0 34 B).  The GEMM kernel gives each lane of a wave one row of
// a 64-row tile and walks the row one 256-element unit at a time, so the
// repack orders the bytes the way one wave instruction reads them: per (tile,
// unit), piece-major, then lane, 16 bytes per lane (see repack_kernel).  Every
// 128-bit load of the kernel is then a contiguous 1 KiB read, and the total
// size equals ggml's (plus zero padding of the last tile).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "cpv_internal.h"

// ---------------------------------------------------------------- errors
cpv_status cpv_fail(cpv_ctx* ctx, cpv_status st, const char* fmt, ...)
{
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return st;
}

cpv_status cpv_hip_fail(cpv_ctx* ctx, hipError_t e, const char* what)
{
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        return cpv_fail(ctx, CPV_ENOMEM, "%s: out of device memory", what);
    }
    return cpv_fail(ctx, CPV_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

int64_t cpv_type_block(int type)
{
    switch (type) {
    case CPV_Q8_0: return 32;
    case CPV_Q4_K: case CPV_Q6_K: return 256;
    case CPV_F32: case CPV_F16: return 1;
    default: return -1;
    }
}

int64_t cpv_type_size(int type)
{
    switch (type) {
    case CPV_Q8_0: return 34;
    case CPV_Q4_K: return 144;
    case CPV_Q6_K: return 210;
    case CPV_F32: return 4;
    case CPV_F16: return 2;
    default: return -1;
    }
}

// ---------------------------------------------------------------- context
extern "C" cpv_status cpv_init(int device, cpv_ctx** out)
{
    if (!out) return CPV_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return CPV_EDEVICE;
    if (hipSetDevice(device) != hipSuccess) return CPV_EDEVICE;
    cpv_ctx* c = new (std::nothrow) cpv_ctx();
    if (!c) return CPV_ENOMEM;
    c->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) { delete c; return CPV_EDEVICE; }
    c->cu_count = prop.multiProcessorCount;
    c->lds_max = prop.sharedMemPerBlock;
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return CPV_EDEVICE;
    }
    c->stream = c->own_stream;
    if (cpv_noalloc_setup(c) != CPV_OK) {
        // only cpv_qgemm_noalloc uses the scratch, and it reports CPV_EDEVICE
        // itself while ctx->scratch is null; the rest of the library works
        c->scratch = nullptr;
        (void)hipGetLastError();
    }
    *out = c;
    return CPV_OK;
}

extern "C" void cpv_free(cpv_ctx* ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->gsum) (void)hipFree(ctx->gsum);
    if (ctx->red) (void)hipFree(ctx->red);
    for (hipEvent_t e : ctx->prof_ev) (void)hipEventDestroy(e);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    if (ctx->cap_stream) (void)hipStreamDestroy(ctx->cap_stream);
    delete ctx;
}

extern "C" const char* cpv_last_error(const cpv_ctx* ctx)
{
    return ctx ? ctx->err.c_str() : "null context";
}

extern "C" cpv_status cpv_set_stream(cpv_ctx* ctx, void* s)
{
    if (!ctx) return CPV_EINVAL;
    ctx->stream = (hipStream_t)s;
    return CPV_OK;
}

extern "C" void* cpv_get_stream(const cpv_ctx* ctx)
{
    return ctx ? (void*)ctx->stream : nullptr;
}

extern "C" cpv_status cpv_sync(cpv_ctx* ctx)
{
    if (!ctx) return CPV_EINVAL;
    CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return CPV_OK;
}

// ---------------------------------------------------------------- timing
int cpv_prof_mark(cpv_ctx* ctx)
{
    if (!ctx->prof) return -1;
    if (ctx->prof_used == ctx->prof_ev.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) {
            ctx->prof = false;               // out of events: stop timing, keep computing
            return -1;
        }
        ctx->prof_ev.push_back(e);
    }
    if (hipEventRecord(ctx->prof_ev[ctx->prof_used], ctx->stream) != hipSuccess) return -1;
    return (int)ctx->prof_used++;
}

void cpv_prof_add(cpv_ctx* ctx, int ev0, int cls, double bytes)
{
    const int ev1 = cpv_prof_mark(ctx);
    if (ev0 >= 0 && ev1 >= 0) ctx->prof_recs.push_back({cls, ev0, ev1, bytes});
}

void cpv_prof_keep(cpv_ctx* ctx, int cls, double bytes, std::function<void()> go)
{
    ctx->prof_launches.push_back({cls, bytes, ctx->ws_gen, std::move(go)});
}

extern "C" cpv_status cpv_profile_start(cpv_ctx* ctx)
{
    if (!ctx) return CPV_EINVAL;
    ctx->prof = true;
    ctx->prof_used = 0;
    ctx->prof_recs.clear();
    ctx->prof_launches.clear();
    return CPV_OK;
}

extern "C" cpv_status cpv_profile_replay(cpv_ctx* ctx, int cls, int reps, double* ms_per_launch,
                                         double* bytes_per_launch)
{
    if (!ctx || cls < 0 || cls >= CPV_PROF_CLASSES || reps < 1 || !ms_per_launch)
        return cpv_fail(ctx, CPV_EINVAL, "profile_replay: bad arguments");
    if (ctx->prof) return cpv_fail(ctx, CPV_EINVAL, "profile_replay: stop the profile first");
    std::vector<const cpv_ctx::prof_launch*> sel;
    double bytes = 0.0;
    for (const auto& l : ctx->prof_launches)
        if (l.cls == cls) {
            if (l.ws_gen != ctx->ws_gen)
                return cpv_fail(ctx, CPV_EINVAL, "profile_replay: the workspace moved since the profile");
            sel.push_back(&l);
            bytes += l.bytes;
        }
    if (sel.empty()) return cpv_fail(ctx, CPV_EINVAL, "profile_replay: no launches of class %d recorded", cls);
    hipEvent_t e0, e1;
    CPV_HIP(ctx, hipEventCreate(&e0));
    CPV_HIP(ctx, hipEventCreate(&e1));
    CPV_HIP(ctx, hipEventRecord(e0, ctx->stream));
    for (int r = 0; r < reps; r++)
        for (const auto* l : sel) l->go();
    CPV_HIP(ctx, hipEventRecord(e1, ctx->stream));
    CPV_HIP(ctx, hipEventSynchronize(e1));
    float ms = 0.0f;
    CPV_HIP(ctx, hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    CPV_HIP(ctx, hipGetLastError());
    // a replayed GEMM without its consumer leaves sums in the split-K
    // accumulator, which every GEMM expects to find zero
    if (ctx->gsum) {
        CPV_HIP(ctx, hipMemsetAsync(ctx->gsum, 0, ctx->gsum_bytes, ctx->stream));
        CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
    }
    *ms_per_launch = (double)ms / ((double)reps * (double)sel.size());
    if (bytes_per_launch) *bytes_per_launch = bytes / (double)sel.size();
    return CPV_OK;
}

extern "C" cpv_status cpv_profile_stop(cpv_ctx* ctx, cpv_prof_stat* out)
{
    if (!ctx || !out) return cpv_fail(ctx, CPV_EINVAL, "profile_stop: null argument");
    const bool was = ctx->prof;
    ctx->prof = false;
    for (int c = 0; c < CPV_PROF_CLASSES; c++) out[c] = cpv_prof_stat{0, 0.0, 0.0};
    if (!was) return cpv_fail(ctx, CPV_EINVAL, "profile_stop: no profile running");
    CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (const auto& r : ctx->prof_recs) {
        float ms = 0.0f;
        CPV_HIP(ctx, hipEventElapsedTime(&ms, ctx->prof_ev[r.ev0], ctx->prof_ev[r.ev1]));
        out[r.cls].launches++;
        out[r.cls].ms += ms;
        out[r.cls].bytes += r.bytes;
    }
    ctx->prof_recs.clear();
    ctx->prof_used = 0;
    return CPV_OK;
}

bool cpv_capturing(cpv_ctx* ctx)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

cpv_status cpv_refuse_growth(cpv_ctx* ctx, const char* what, size_t bytes)
{
    ctx->grow_refused = true;
    return cpv_fail(ctx, CPV_EUNSUPPORTED, "%s: growing to %zu bytes while the stream is being captured "
                                           "(run the call once outside the capture first)", what, bytes);
}

cpv_status cpv_workspace(cpv_ctx* ctx, size_t bytes, void** out)
{
    if (bytes <= ctx->ws_bytes) {
        *out = ctx->ws;
        return CPV_OK;
    }
    if (cpv_capturing(ctx)) return cpv_refuse_growth(ctx, "workspace", bytes);
    if (ctx->ws) {
        CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
        CPV_HIP(ctx, hipFree(ctx->ws));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    size_t sz = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    CPV_HIP(ctx, hipMalloc(&ctx->ws, sz));
    ctx->ws_bytes = sz;
    ctx->ws_gen++;
    *out = ctx->ws;
    return CPV_OK;
}

// ---------------------------------------------------------------- repack
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return cpv_h2f(h); }

// Tile layout of a repacked weight.  Rows are padded to tiles of 64; for
// tile t and 256-element unit u the slab (t*U + u) holds PIECES x 64 lanes x
// 16 bytes, lane = row within the tile, so the wave that owns the tile reads
// each piece as one contiguous KiB:
//   Q4_K  pieces 0-7 = qs (block bytes 16..143), piece 8 = d, dmin, scales[12]
//   Q6_K  pieces 0-12 = ql, qh, scales (block bytes 0..207); the f16 d of
//         every (row, unit) follows all slabs as [t*U + u][lane] u16
//   Q8_0  pieces 0-15 = the codes of the unit's 8 blocks, piece 16 = their 8 d
// Missing rows and units are zero (their Ew is empty, so they contribute 0).
template <int TYPE>
__global__ void repack_kernel(const uint8_t* __restrict__ aos, uint8_t* __restrict__ out, int64_t n,
                              int64_t k, int64_t U, int64_t total)
{
    constexpr int PIECES = TYPE == CPV_Q4_K ? 9 : TYPE == CPV_Q6_K ? 13 : 17;
    constexpr int BSZ = TYPE == CPV_Q4_K ? 144 : TYPE == CPV_Q6_K ? 210 : 34;
    constexpr int BLK = TYPE == CPV_Q8_0 ? 32 : 256;
    const int64_t nblk = k / BLK;
    const int64_t rb = nblk * BSZ;
    const int64_t tiles = (n + 63) / 64;
    const int64_t region_a = tiles * U * PIECES * 1024;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t src = -1;
        if (i < region_a) {
            const int b = (int)(i & 15);
            const int lane = (int)((i >> 4) & 63);
            const int piece = (int)((i >> 10) % PIECES);
            const int64_t slab = (i >> 10) / PIECES;
            const int64_t t = slab / U, u = slab % U;
            const int64_t row = t * 64 + lane;
            if (row < n) {
                if (TYPE == CPV_Q4_K) {
                    if (u < nblk) src = row * rb + u * 144 + (piece < 8 ? 16 + 16 * piece : 0) + b;
                } else if (TYPE == CPV_Q6_K) {
                    if (u < nblk) src = row * rb + u * 210 + 16 * piece + b;
                } else if (piece < 16) {
                    const int64_t blk = u * 8 + piece / 2;
                    if (blk < nblk) src = row * rb + blk * 34 + 2 + 16 * (piece & 1) + b;
                } else {
                    const int64_t blk = u * 8 + b / 2;
                    if (blk < nblk) src = row * rb + blk * 34 + (b & 1);
                }
            }
        } else {
            // Q6_K d region
            const int64_t j = i - region_a;
            const int b = (int)(j & 1);
            const int lane = (int)((j >> 1) & 63);
            const int64_t slab = j >> 7;
            const int64_t t = slab / U, u = slab % U;
            const int64_t row = t * 64 + lane;
            if (row < n && u < nblk) src = row * rb + u * 210 + 208 + b;
        }
        out[i] = src >= 0 ? aos[src] : 0;
    }
}

// Ew(row): frexp exponent of the row's largest scale magnitude (d and dmin for
// Q4_K, d for Q6_K / Q8_0; Q6_K's int8 group scales ride in the integer sum).
template <int TYPE>
__global__ void row_exponent_kernel(const uint8_t* __restrict__ aos, int32_t* __restrict__ ew,
                                    int64_t n, int64_t n_pad, int64_t k)
{
    constexpr int BSZ = TYPE == CPV_Q4_K ? 144 : TYPE == CPV_Q6_K ? 210 : 34;
    constexpr int BLK = TYPE == CPV_Q8_0 ? 32 : 256;
    const int64_t nblk = k / BLK;
    const int64_t row = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (row >= n_pad) return;
    if (row >= n) { ew[row] = CPV_E_EMPTY; return; }
    const uint8_t* r = aos + row * nblk * BSZ;
    float mx = 0.0f;
    for (int64_t b = 0; b < nblk; b++) {
        const uint8_t* bl = r + b * BSZ;
        if (TYPE == CPV_Q4_K) {
            const uint16_t d = (uint16_t)(bl[0] | (bl[1] << 8)), dm = (uint16_t)(bl[2] | (bl[3] << 8));
            mx = fmaxf(mx, fabsf(f16_to_f32(d)));
            mx = fmaxf(mx, fabsf(f16_to_f32(dm)));
        } else if (TYPE == CPV_Q6_K) {
            const uint16_t d = (uint16_t)(bl[208] | (bl[209] << 8));
            mx = fmaxf(mx, fabsf(f16_to_f32(d)));
        } else {
            const uint16_t d = (uint16_t)(bl[0] | (bl[1] << 8));
            mx = fmaxf(mx, fabsf(f16_to_f32(d)));
        }
    }
    int e = CPV_E_EMPTY;
    if (mx > 0.0f) frexpf(mx, &e);
    ew[row] = e;
}

static void weight_geometry(cpv_weight* w)
{
    w->units = (w->k + 255) / 256;
    w->n_pad = (w->n + 63) / 64 * 64;
    const int64_t slots = w->n_pad * w->units;          // (row, unit) pairs
    switch (w->type) {
    case CPV_Q4_K: w->data_bytes = (size_t)slots * 144; break;
    case CPV_Q6_K: w->data_bytes = (size_t)slots * (208 + 2); break;
    default: w->data_bytes = (size_t)slots * (256 + 16); break;
    }
}

cpv_status cpv_repack_launch(cpv_ctx* ctx, cpv_weight* w, const void* aos_dev)
{
    const int64_t total = (int64_t)w->data_bytes;
    const int threads = 256;
    const int64_t want = (total + threads - 1) / threads;
    const int blocks = (int)(want < 65536 ? want : 65536);
    const uint8_t* a = (const uint8_t*)aos_dev;
    uint8_t* o = (uint8_t*)w->data;
    const int eblocks = (int)((w->n_pad + 255) / 256);
    switch (w->type) {
    case CPV_Q4_K:
        repack_kernel<CPV_Q4_K><<<blocks, threads, 0, ctx->stream>>>(a, o, w->n, w->k, w->units, total);
        row_exponent_kernel<CPV_Q4_K><<<eblocks, 256, 0, ctx->stream>>>(a, w->ew, w->n, w->n_pad, w->k);
        break;
    case CPV_Q6_K:
        repack_kernel<CPV_Q6_K><<<blocks, threads, 0, ctx->stream>>>(a, o, w->n, w->k, w->units, total);
        row_exponent_kernel<CPV_Q6_K><<<eblocks, 256, 0, ctx->stream>>>(a, w->ew, w->n, w->n_pad, w->k);
        break;
    default:
        repack_kernel<CPV_Q8_0><<<blocks, threads, 0, ctx->stream>>>(a, o, w->n, w->k, w->units, total);
        row_exponent_kernel<CPV_Q8_0><<<eblocks, 256, 0, ctx->stream>>>(a, w->ew, w->n, w->n_pad, w->k);
        break;
    }
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

static cpv_status weight_create(cpv_ctx* ctx, int type, const void* bytes, bool on_device, int64_t n,
                                int64_t k, cpv_weight** out)
{
    if (!ctx || !bytes || !out || n <= 0 || k <= 0) return cpv_fail(ctx, CPV_EINVAL, "weight: bad arguments");
    *out = nullptr;
    if (type != CPV_Q8_0 && type != CPV_Q4_K && type != CPV_Q6_K)
        return cpv_fail(ctx, CPV_EUNSUPPORTED, "weight: type %d not supported (Q8_0, Q4_K, Q6_K)", type);
    const int64_t blk = cpv_type_block(type);
    if (k % blk) return cpv_fail(ctx, CPV_EINVAL, "weight: k=%lld not a multiple of %lld", (long long)k, (long long)blk);
    CPV_HIP(ctx, hipSetDevice(ctx->device));
    cpv_weight* w = new (std::nothrow) cpv_weight();
    if (!w) return cpv_fail(ctx, CPV_ENOMEM, "weight: host allocation");
    w->ctx = ctx;
    w->type = type;
    w->n = n;
    w->k = k;
    weight_geometry(w);
    const size_t aos_bytes = (size_t)n * (size_t)(k / blk) * (size_t)cpv_type_size(type);
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&w->data, w->data_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&w->ew, sizeof(int32_t) * (size_t)w->n_pad);
    if (e == hipSuccess && !on_device) e = hipMalloc(&tmp, aos_bytes);
    if (e == hipSuccess && !on_device) e = hipMemcpyAsync(tmp, bytes, aos_bytes, hipMemcpyHostToDevice, ctx->stream);
    cpv_status st = CPV_OK;
    if (e != hipSuccess) st = cpv_hip_fail(ctx, e, "weight upload");
    if (st == CPV_OK) st = cpv_repack_launch(ctx, w, on_device ? bytes : tmp);
    if (tmp) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(tmp);
    }
    if (st != CPV_OK) {
        if (w->data) (void)hipFree(w->data);
        if (w->ew) (void)hipFree(w->ew);
        delete w;
        return st;
    }
    *out = w;
    return CPV_OK;
}

extern "C" cpv_status cpv_weight_upload(cpv_ctx* ctx, int type, const void* host_bytes, int64_t n_rows,
                                        int64_t k, cpv_weight** out)
{
    return weight_create(ctx, type, host_bytes, false, n_rows, k, out);
}

extern "C" cpv_status cpv_weight_from_device(cpv_ctx* ctx, int type, const void* dev_bytes, int64_t n_rows,
                                             int64_t k, cpv_weight** out)
{
    return weight_create(ctx, type, dev_bytes, true, n_rows, k, out);
}

// Rows `rows[0..n)` of a repacked weight as a new one of n rows (get_rows on
// a quantized weight, as a draft head's shortlist takes it, qwen35.rs:2929):
// the 16-byte pieces of every (tile, unit) slab move lane by lane, then the
// Q6_K d region and the row exponents; rows past n are empty.
template <int TYPE>
__global__ void gather_kernel(const uint8_t* __restrict__ src, const int32_t* __restrict__ ew_s, int64_t n_pad_s,
                              const int32_t* __restrict__ rows, int64_t n, int64_t U, uint8_t* __restrict__ dst,
                              int32_t* __restrict__ ew_d, int64_t n_pad_d)
{
    constexpr int PIECES = TYPE == CPV_Q4_K ? 9 : TYPE == CPV_Q6_K ? 13 : 17;
    const int64_t tiles_d = n_pad_d / 64;
    const int64_t npieces = tiles_d * U * PIECES * 64;
    const int64_t nd6 = TYPE == CPV_Q6_K ? tiles_d * U * 64 : 0;
    const int64_t total = npieces + nd6 + n_pad_d;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        if (i < npieces) {
            const int lane = (int)(i & 63);
            const int64_t sp = i >> 6, piece = sp % PIECES, slab = sp / PIECES;
            const int64_t row = (slab / U) * 64 + lane, u = slab % U;
            uint4 v = {0u, 0u, 0u, 0u};
            if (row < n) {
                const int64_t r = rows[row];
                v = *(const uint4*)(src + (((r / 64) * U + u) * PIECES + piece) * 1024 + (r % 64) * 16);
            }
            *(uint4*)(dst + (slab * PIECES + piece) * 1024 + lane * 16) = v;
        } else if (i < npieces + nd6) {
            const int64_t j = i - npieces;
            const int lane = (int)(j & 63);
            const int64_t slab = j >> 6, row = (slab / U) * 64 + lane, u = slab % U;
            const uint16_t* d6s = (const uint16_t*)(src + (n_pad_s / 64) * U * PIECES * 1024);
            uint16_t* d6d = (uint16_t*)(dst + tiles_d * U * PIECES * 1024);
            uint16_t v = 0;
            if (row < n) {
                const int64_t r = rows[row];
                v = d6s[((r / 64) * U + u) * 64 + r % 64];
            }
            d6d[slab * 64 + lane] = v;
        } else {
            const int64_t row = i - npieces - nd6;
            ew_d[row] = row < n ? ew_s[rows[row]] : CPV_E_EMPTY;
        }
    }
}

cpv_status cpv_weight_gather(cpv_ctx* ctx, const cpv_weight* src, const int32_t* rows_dev, int64_t n,
                             cpv_weight** out)
{
    *out = nullptr;
    cpv_weight* w = new (std::nothrow) cpv_weight();
    if (!w) return cpv_fail(ctx, CPV_ENOMEM, "gather: host allocation");
    w->ctx = ctx;
    w->type = src->type;
    w->n = n;
    w->k = src->k;
    weight_geometry(w);
    hipError_t e = hipMalloc(&w->data, w->data_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&w->ew, sizeof(int32_t) * (size_t)w->n_pad);
    if (e != hipSuccess) {
        if (w->data) (void)hipFree(w->data);
        delete w;
        return cpv_hip_fail(ctx, e, "gather: hipMalloc");
    }
    const int64_t pieces = (int64_t)(w->data_bytes / 16) + w->n_pad;
    const unsigned blocks = (unsigned)((pieces + 255) / 256 < 4096 ? (pieces + 255) / 256 : 4096);
    const uint8_t* s = (const uint8_t*)src->data;
    uint8_t* d = (uint8_t*)w->data;
    switch (w->type) {
    case CPV_Q4_K:
        gather_kernel<CPV_Q4_K><<<blocks, 256, 0, ctx->stream>>>(s, src->ew, src->n_pad, rows_dev, n, w->units, d, w->ew,
                                                                 w->n_pad);
        break;
    case CPV_Q6_K:
        gather_kernel<CPV_Q6_K><<<blocks, 256, 0, ctx->stream>>>(s, src->ew, src->n_pad, rows_dev, n, w->units, d, w->ew,
                                                                 w->n_pad);
        break;
    default:
        gather_kernel<CPV_Q8_0><<<blocks, 256, 0, ctx->stream>>>(s, src->ew, src->n_pad, rows_dev, n, w->units, d, w->ew,
                                                                 w->n_pad);
        break;
    }
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(w->data);
        (void)hipFree(w->ew);
        delete w;
        return cpv_hip_fail(ctx, e, "gather");
    }
    *out = w;
    return CPV_OK;
}

// Rows of several weights stacked into one (same type and k; every part but
// the last a whole number of 64-row tiles, so the tiles just follow each
// other): the tile slabs of the parts in order, then, for Q6_K, their d
// regions in order, and their row exponents.  The parts stay as they are.
cpv_status cpv_weight_concat(cpv_ctx* ctx, cpv_weight* const* parts, int np, cpv_weight** out)
{
    *out = nullptr;
    if (np < 1) return cpv_fail(ctx, CPV_EINVAL, "weight_concat: no parts");
    const int type = parts[0]->type;
    const int64_t k = parts[0]->k;
    int64_t n = 0;
    for (int i = 0; i < np; i++) {
        if (parts[i]->type != type || parts[i]->k != k)
            return cpv_fail(ctx, CPV_EINVAL, "weight_concat: parts differ in type or k");
        if (i + 1 < np && parts[i]->n % 64)
            return cpv_fail(ctx, CPV_EINVAL, "weight_concat: part %d has %lld rows, not whole tiles", i,
                            (long long)parts[i]->n);
        n += parts[i]->n;
    }
    cpv_weight* w = new (std::nothrow) cpv_weight();
    if (!w) return cpv_fail(ctx, CPV_ENOMEM, "weight_concat: host allocation");
    w->ctx = ctx;
    w->type = type;
    w->n = n;
    w->k = k;
    weight_geometry(w);
    hipError_t e = hipMalloc(&w->data, w->data_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&w->ew, sizeof(int32_t) * (size_t)w->n_pad);
    const size_t slab = (size_t)w->units * (type == CPV_Q4_K ? 9 : type == CPV_Q6_K ? 13 : 17) * 1024;
    size_t off_a = 0, off_d = (size_t)(w->n_pad / 64) * slab, off_e = 0;
    for (int i = 0; i < np && e == hipSuccess; i++) {
        const cpv_weight* q = parts[i];
        const size_t ra = (size_t)(q->n_pad / 64) * slab;
        e = hipMemcpyAsync((uint8_t*)w->data + off_a, q->data, ra, hipMemcpyDeviceToDevice, ctx->stream);
        off_a += ra;
        if (e == hipSuccess && type == CPV_Q6_K) {
            const size_t rd = (size_t)(q->n_pad / 64) * w->units * 64 * 2;
            e = hipMemcpyAsync((uint8_t*)w->data + off_d, (const uint8_t*)q->data + ra, rd, hipMemcpyDeviceToDevice,
                               ctx->stream);
            off_d += rd;
        }
        if (e == hipSuccess)
            e = hipMemcpyAsync(w->ew + off_e, q->ew, sizeof(int32_t) * (size_t)q->n_pad, hipMemcpyDeviceToDevice,
                               ctx->stream);
        off_e += (size_t)q->n_pad;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        if (w->data) (void)hipFree(w->data);
        if (w->ew) (void)hipFree(w->ew);
        delete w;
        return cpv_hip_fail(ctx, e, "weight_concat");
    }
    *out = w;
    return CPV_OK;
}

extern "C" void cpv_weight_free(cpv_weight* w)
{
    if (!w) return;
    if (w->ctx) {
        (void)hipSetDevice(w->ctx->device);
        (void)hipStreamSynchronize(w->ctx->stream);
    }
    if (w->data) (void)hipFree(w->data);
    if (w->ew) (void)hipFree(w->ew);
    delete w;
}

extern "C" cpv_status cpv_weight_info(const cpv_weight* w, int* type, int64_t* n_rows, int64_t* k,
                                      int64_t* bytes)
{
    if (!w) return CPV_EINVAL;
    if (type) *type = w->type;
    if (n_rows) *n_rows = w->n;
    if (k) *k = w->k;
    if (bytes) *bytes = (int64_t)w->data_bytes;
    return CPV_OK;
}

// ---------------------------------------------------------------- get_rows
// Dequantize from the repacked layout with ggml's f32 formulas
// (cpv_dequant4), four elements per thread
template <int TYPE>
__global__ void get_rows_kernel(const uint8_t* __restrict__ data, const int32_t* __restrict__ rows,
                                int64_t nrows, int64_t n, int64_t k, int64_t U, float* __restrict__ out)
{
    const int64_t r_out = blockIdx.y;
    if (r_out >= nrows) return;
    const int64_t row = rows[r_out];
    for (int64_t e = 4 * (blockIdx.x * (int64_t)blockDim.x + threadIdx.x); e < k; e += 4 * (int64_t)gridDim.x * blockDim.x) {
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (row >= 0 && row < n) cpv_dequant4<TYPE>(data, n, U, row, e, v);
#pragma unroll
        for (int i = 0; i < 4; i++) out[r_out * k + e + i] = v[i];
    }
}

extern "C" cpv_status cpv_get_rows(cpv_ctx* ctx, const cpv_weight* w, const int32_t* rows_dev, int64_t n,
                                   float* out_dev)
{
    if (!ctx || !w || !rows_dev || !out_dev || n < 0) return cpv_fail(ctx, CPV_EINVAL, "get_rows: bad arguments");
    if (n == 0) return CPV_OK;
    if (n > 65535) return cpv_fail(ctx, CPV_EINVAL, "get_rows: at most 65535 rows per call");
    // (four elements per thread: rows are whole 32-element blocks)
    dim3 grid((unsigned)((w->k + 1023) / 1024), (unsigned)n);
    const uint8_t* d = (const uint8_t*)w->data;
    switch (w->type) {
    case CPV_Q4_K: get_rows_kernel<CPV_Q4_K><<<grid, 256, 0, ctx->stream>>>(d, rows_dev, n, w->n, w->k, w->units, out_dev); break;
    case CPV_Q6_K: get_rows_kernel<CPV_Q6_K><<<grid, 256, 0, ctx->stream>>>(d, rows_dev, n, w->n, w->k, w->units, out_dev); break;
    default: get_rows_kernel<CPV_Q8_0><<<grid, 256, 0, ctx->stream>>>(d, rows_dev, n, w->n, w->k, w->units, out_dev); break;
    }
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

// ---------------------------------------------------------------- argmax
// ggml_argmax: the first index of the maximum; values that are not > -inf
// (and NaN) never win, and a row with no winner gives 0.  Pass 1 reduces each
// of 64 slices of a row to a key, (order-preserving bits of the value) << 32 |
// (2^32 - 1 - index), so the integer maximum of the keys is the largest value
// at its first index (-0 is keyed as +0, which compares equal); 0 = no winner.
// Pass 2 reduces a row's keys.
constexpr int AM_NB = CPV_AM_NB;

__device__ __forceinline__ unsigned long long am_key(float v, int64_t i)
{
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0;
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
}

__device__ __forceinline__ float am_value(unsigned long long key)
{
    const uint32_t ord = (uint32_t)(key >> 32);
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}

__device__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* s)
{
    v = cpv_wave_reduce(v, cpv_op_umax());
    const int tid = threadIdx.x, nw = blockDim.x >> 6;
    if ((tid & 63) == 0) s[tid >> 6] = v;
    __syncthreads();
    unsigned long long r = 0;
    for (int w = 0; w < nw; w++) r = s[w] > r ? s[w] : r;
    return r;
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const float* __restrict__ x, const float* __restrict__ nz,
                                                          int64_t n, int64_t chunk, unsigned long long* __restrict__ part)
{
    __shared__ unsigned long long s_k[4];
    const int64_t row = blockIdx.y, i0 = (int64_t)blockIdx.x * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    const float* xr = x + row * n;
    const float* nr = nz ? nz + row * n : nullptr;
    unsigned long long best = 0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) {
        const float v = nr ? xr[i] + nr[i] : xr[i];
        if (v > -INFINITY) {
            const unsigned long long k = am_key(v, i);
            best = k > best ? k : best;
        }
    }
    best = block_max_u64(best, s_k);
    if (threadIdx.x == 0) part[row * AM_NB + blockIdx.x] = best;
}

// argmax_part_kernel over a GEMM result kept in the accumulator: each entry
// is finalized as qgemm_finalize_kernel does (and the accumulator cleared),
// stored to y, then keyed; Ea of the row comes from a wave reduction per wave
__global__ __launch_bounds__(256) void argmax_kept_part_kernel(cpv_gout g, const float* __restrict__ nz, int64_t chunk,
                                                               float* __restrict__ y,
                                                               unsigned long long* __restrict__ part)
{
    __shared__ unsigned long long s_k[4];
    const int64_t n = g.n, row = blockIdx.y, i0 = (int64_t)blockIdx.x * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    const int lane = threadIdx.x & 63;
    const float* dar = g.da + row * g.nda;
    float mx = 0.0f;
    for (int i = lane; i < g.nda; i += 64) mx = fmaxf(mx, fabsf(dar[i]));
    const int ea = cpv_exp_of_max(cpv_wave_reduce(mx, cpv_op_max()));
    double* acc = g.acc + row * g.n_pad;
    float* yr = y + row * n;
    const float* nr = nz ? nz + row * n : nullptr;
    unsigned long long best = 0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) {
        const double S = acc[i];
        acc[i] = 0.0;
        const float x = cpv_gout_value(S, g.ew[i], ea, g.win);
        yr[i] = x;
        const float v = nr ? x + nr[i] : x;
        if (v > -INFINITY) {
            const unsigned long long k = am_key(v, i);
            best = k > best ? k : best;
        }
    }
    best = block_max_u64(best, s_k);
    if (threadIdx.x == 0) part[row * AM_NB + blockIdx.x] = best;
}

__global__ __launch_bounds__(64) void argmax_fin_kernel(const unsigned long long* __restrict__ part,
                                                        int32_t* __restrict__ out)
{
    const int64_t row = blockIdx.x;
    const unsigned long long v = cpv_wave_reduce(part[row * AM_NB + threadIdx.x], cpv_op_umax());
    if (threadIdx.x == 0) out[row] = cpv_am_index(v);
}

// The embedding table of a draft chain's next link (data null: none): the
// blocks of a row write the table's row tok, the row's argmax, to out[row],
// four elements per thread, as get_rows_kernel does
struct EmbArgs {
    const uint8_t* data;
    int type;
    int64_t n, k, U;
    float* out;
};

__device__ __forceinline__ void embed_share(const EmbArgs& e, int64_t row, int64_t tok)
{
    if (!e.data) return;
    for (int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x); i < e.k; i += 4 * (int64_t)gridDim.x * blockDim.x) {
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (tok >= 0 && tok < e.n) cpv_dequant4_t(e.type, e.data, e.n, e.U, tok, i, v);
#pragma unroll
        for (int k = 0; k < 4; k++) e.out[row * e.k + i + k] = v[k];
    }
}

// argmax_fin_kernel's index, with the winners' embedding rows: every block
// reduces its row's keys
__global__ __launch_bounds__(256) void argmax_embed_kernel(const unsigned long long* __restrict__ part,
                                                           int32_t* __restrict__ idx_out, EmbArgs emb)
{
    const int64_t row = blockIdx.y;
    const int32_t tok = cpv_am_index(cpv_wave_reduce(part[row * AM_NB + (threadIdx.x & 63)], cpv_op_umax()));
    if (blockIdx.x == 0 && threadIdx.x == 0) idx_out[row] = tok;
    embed_share(emb, row, tok);
}

// softmax peak: each slice's sum of expf(x - max) in binary64 (max from the
// argmax keys), then the row's slices added in order.  Every block reduces
// the row's argmax keys itself; block 0 stores the row's argmax index, as
// argmax_fin_kernel would, and the first blocks the winners' embedding rows
__global__ __launch_bounds__(256) void peak_part_kernel(const float* __restrict__ x, int64_t n, int64_t chunk,
                                                        const unsigned long long* __restrict__ part,
                                                        double* __restrict__ psum, int32_t* __restrict__ idx_out,
                                                        EmbArgs emb)
{
    __shared__ double s_d[4];
    const int64_t row = blockIdx.y, i0 = (int64_t)blockIdx.x * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    const unsigned long long k = cpv_wave_reduce(part[row * AM_NB + (threadIdx.x & 63)], cpv_op_umax());
    if (blockIdx.x == 0 && threadIdx.x == 0) idx_out[row] = cpv_am_index(k);
    const float mx = k ? am_value(k) : -INFINITY;
    const float* xr = x + row * n;
    double sum = 0.0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) sum += (double)cpv_expf(xr[i] - mx);
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((threadIdx.x & 63) == 0) s_d[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) psum[row * AM_NB + blockIdx.x] = (s_d[0] + s_d[1]) + (s_d[2] + s_d[3]);
    embed_share(emb, row, cpv_am_index(k));
}

__global__ void peak_fin_kernel(const double* __restrict__ psum, int64_t rows, float* __restrict__ out)
{
    const int64_t row = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (row >= rows) return;
    out[row] = cpv_peak_of(psum + row * AM_NB);
}

// the re-draft gate's bound pass: each slice's S = sum of e_i = expf(x_i -
// max) and W = sum of e_i (n - i), both in binary64 (max from the argmax
// keys).  W bounds the rounding of the index-order f32 sum: every prefix of
// that sum rounds with a relative error of at most 2^-24, and e_i is in the
// n - i prefixes from i on.  Block 0 stores the row's argmax index.
__global__ __launch_bounds__(256) void gate_part_kernel(const float* __restrict__ x, int64_t n, int64_t chunk,
                                                        const unsigned long long* __restrict__ part,
                                                        double* __restrict__ sw, int32_t* __restrict__ idx_out)
{
    __shared__ double s_d[4][2];
    const int64_t row = blockIdx.y, i0 = (int64_t)blockIdx.x * chunk;
    const int64_t i1 = i0 + chunk < n ? i0 + chunk : n;
    const unsigned long long k = cpv_wave_reduce(part[row * AM_NB + (threadIdx.x & 63)], cpv_op_umax());
    if (blockIdx.x == 0 && threadIdx.x == 0) idx_out[row] = cpv_am_index(k);
    const float mx = k ? am_value(k) : -INFINITY;
    const float* xr = x + row * n;
    double S = 0.0, W = 0.0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) {
        const double e = (double)cpv_expf(xr[i] - mx);
        S += e;
        W += e * (double)(n - i);
    }
    for (int off = 32; off > 0; off >>= 1) {
        S += __shfl_xor(S, off);
        W += __shfl_xor(W, off);
    }
    if ((threadIdx.x & 63) == 0) {
        s_d[threadIdx.x >> 6][0] = S;
        s_d[threadIdx.x >> 6][1] = W;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        const int c = threadIdx.x;
        sw[(row * AM_NB + blockIdx.x) * 2 + c] = (s_d[0][c] + s_d[1][c]) + (s_d[2][c] + s_d[3][c]);
    }
}

// the reduction buffer for `rows` rows: argmax keys [rows][AM_NB], then
// binary64 pairs [rows][AM_NB][2] (the peak's sums use the first half)
static cpv_status reduce_buffer(cpv_ctx* ctx, int64_t rows, unsigned long long** keys, double** sums)
{
    const size_t need = (size_t)rows * AM_NB * 24;
    if (need > ctx->red_bytes) {
        if (cpv_capturing(ctx)) return cpv_refuse_growth(ctx, "reduction buffer", need);
        CPV_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->red) (void)hipFree(ctx->red);
        ctx->red = nullptr;
        ctx->red_bytes = 0;
        const size_t bs = need > ((size_t)1 << 20) ? need : ((size_t)1 << 20);
        CPV_HIP(ctx, hipMalloc(&ctx->red, bs));
        ctx->red_bytes = bs;
        ctx->ws_gen++;
    }
    *keys = (unsigned long long*)ctx->red;
    *sums = (double*)(*keys + rows * AM_NB);
    return CPV_OK;
}

cpv_status cpv_argmax_gate_rows(cpv_ctx* ctx, const float* x, int64_t rows, int64_t n, int32_t* idx_out, float p_min,
                                int32_t* keep_out, const cpv_gout* kept)
{
    unsigned long long* part;
    double* sw;
    cpv_status st = reduce_buffer(ctx, rows, &part, &sw);
    if (st != CPV_OK) return st;
    const int64_t chunk = (n + AM_NB - 1) / AM_NB;
    const dim3 grid(AM_NB, (unsigned)rows);
    if (kept) argmax_kept_part_kernel<<<grid, 256, 0, ctx->stream>>>(*kept, nullptr, chunk, const_cast<float*>(x), part);
    else argmax_part_kernel<<<grid, 256, 0, ctx->stream>>>(x, nullptr, n, chunk, part);
    CPV_HIP(ctx, hipGetLastError());
    if (!(p_min > 0.0f)) {
        argmax_fin_kernel<<<(unsigned)rows, 64, 0, ctx->stream>>>(part, idx_out);
        CPV_HIP(ctx, hipGetLastError());
        return keep_out ? cpv_gate_fin_launch(ctx, x, rows, n, idx_out, nullptr, 0, p_min, keep_out) : CPV_OK;
    }
    gate_part_kernel<<<grid, 256, 0, ctx->stream>>>(x, n, chunk, part, sw, idx_out);
    CPV_HIP(ctx, hipGetLastError());
    return cpv_gate_fin_launch(ctx, x, rows, n, idx_out, sw, AM_NB, p_min, keep_out);
}

cpv_status cpv_argmax_peak_rows(cpv_ctx* ctx, const float* x, const float* noise, int64_t rows, int64_t n,
                                int32_t* idx_out, float* peak_out, const cpv_gout* kept, cpv_am_fin* fin,
                                const cpv_weight* emb, float* emb_out)
{
    unsigned long long* part;
    double* psum;
    cpv_status st = reduce_buffer(ctx, rows, &part, &psum);
    if (st != CPV_OK) return st;
    const int64_t chunk = (n + AM_NB - 1) / AM_NB;
    const dim3 grid(AM_NB, (unsigned)rows);
    if (kept) argmax_kept_part_kernel<<<grid, 256, 0, ctx->stream>>>(*kept, noise, chunk, const_cast<float*>(x), part);
    else argmax_part_kernel<<<grid, 256, 0, ctx->stream>>>(x, noise, n, chunk, part);
    EmbArgs ea{};
    if (emb) ea = EmbArgs{(const uint8_t*)emb->data, emb->type, emb->n, emb->k, emb->units, emb_out};
    if (peak_out) {
        peak_part_kernel<<<grid, 256, 0, ctx->stream>>>(x, n, chunk, part, psum, idx_out, ea);
        if (!fin) peak_fin_kernel<<<(unsigned)((rows + 63) / 64), 64, 0, ctx->stream>>>(psum, rows, peak_out);
    } else if (emb) {
        argmax_embed_kernel<<<dim3((unsigned)((emb->k + 1023) / 1024), (unsigned)rows), 256, 0, ctx->stream>>>(part, idx_out,
                                                                                                          ea);
    } else {
        argmax_fin_kernel<<<(unsigned)rows, 64, 0, ctx->stream>>>(part, idx_out);
    }
    if (fin) fin->psum = peak_out ? psum : nullptr;
    CPV_HIP(ctx, hipGetLastError());
    return CPV_OK;
}

extern "C" cpv_status cpv_redraft_gate(cpv_ctx* ctx, const float* logits_dev, int64_t rows, int64_t v,
                                       float p_min, int32_t* argmax_dev, int32_t* keep_dev)
{
    if (!ctx || !logits_dev || !argmax_dev || !keep_dev || rows < 0 || rows > 65535 || v <= 0 || v > 262144)
        return cpv_fail(ctx, CPV_EINVAL, "redraft_gate: bad arguments");
    if (rows == 0) return CPV_OK;
    return cpv_argmax_gate_rows(ctx, logits_dev, rows, v, argmax_dev, p_min, keep_dev, nullptr);
}

extern "C" cpv_status cpv_argmax_rows(cpv_ctx* ctx, const float* x_dev, const float* noise_dev, int64_t rows,
                                      int64_t n, int32_t* out_dev)
{
    if (!ctx || !x_dev || !out_dev || rows < 0 || n <= 0 || n > 0x7fffffff || rows > 65535)
        return cpv_fail(ctx, CPV_EINVAL, "argmax: bad arguments");
    if (rows == 0) return CPV_OK;
    return cpv_argmax_peak_rows(ctx, x_dev, noise_dev, rows, n, out_dev, nullptr);
}
