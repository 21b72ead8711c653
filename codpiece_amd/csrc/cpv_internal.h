// cpv_internal.h — shared definitions of libcpv (HIP, gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/cpv.h"

struct cpv_ctx {
    int device = 0;
    int cu_count = 0;
    size_t lds_max = 0;       // shared memory per workgroup (bytes)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    // scratch owned by the context, grown on demand (never inside a capture)
    void* ws = nullptr;
    size_t ws_bytes = 0;
};

struct cpv_weight {
    cpv_ctx* ctx = nullptr;
    int type = 0;
    int64_t n = 0, k = 0;     // logical rows and row length
    int64_t n_pad = 0;        // rows padded to the 16-row groups of the GEMM
    int64_t units = 0;        // super-blocks (K-quants) or 32-blocks (Q8_0) per row
    int64_t passes = 0;       // 256-element passes per row (padded)
    void* data = nullptr;     // repacked blocks, layout per type (qgemm.hip)
    size_t data_bytes = 0;
    void* aos = nullptr;      // ggml row layout, kept for get_rows
    size_t aos_bytes = 0;
    int32_t* ew = nullptr;    // [n_pad] frexp exponent of the row's largest scale
};

// error helpers: record a message on the context and return the status
cpv_status cpv_fail(cpv_ctx* ctx, cpv_status st, const char* fmt, ...);
cpv_status cpv_hip_fail(cpv_ctx* ctx, hipError_t e, const char* what);

#define CPV_HIP(ctx, expr)                                             \
    do {                                                               \
        hipError_t e_ = (expr);                                        \
        if (e_ != hipSuccess) return cpv_hip_fail((ctx), e_, #expr);   \
    } while (0)

// grow the context workspace to at least `bytes` (synchronises the stream
// before freeing an old buffer the queued work may still use)
cpv_status cpv_workspace(cpv_ctx* ctx, size_t bytes, void** out);

// bytes per block / elements per block of a GGUF type
int64_t cpv_type_block(int type);
int64_t cpv_type_size(int type);

// sentinel exponent of an all-zero scale set
constexpr int CPV_E_EMPTY = -100000;

// exact-window constants shared by the launcher and the kernels
int cpv_qgemm_window(int type, int64_t k);

// IEEE binary16 <-> binary32 (exact / round-to-nearest-even)
__host__ __device__ __forceinline__ float cpv_h2f(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}
__host__ __device__ __forceinline__ uint16_t cpv_f2h(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// internal launchers
cpv_status cpv_repack_launch(cpv_ctx* ctx, cpv_weight* w, const void* aos_dev);
cpv_status cpv_attn_launch(cpv_ctx* ctx, const float* q, const uint16_t* kc, const uint16_t* vt, int64_t v_stride,
                           int64_t n_past, const int32_t* parent, int t, int h, int h_kv, int d, float scale,
                           float* out);
cpv_status cpv_qgemm_launch(cpv_ctx* ctx, const cpv_weight* w, const float* x, int64_t m, float* y);
