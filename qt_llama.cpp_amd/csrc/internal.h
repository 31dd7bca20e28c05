// internal.h -- host-side internals shared by the backend's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/mrml_hip.h"

struct mrml_hip_ctx {
    int32_t device = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    void *ws = nullptr;     // scratch: activation packs and partial results
    size_t ws_bytes = 0;
    std::string err;
};

namespace mrml {

// Record a failure on the context and return `code`.
int fail(mrml_hip_ctx *ctx, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
// Record a HIP error (with the call that produced it) and return MRML_HIP_E_HIP.
int hip_fail(mrml_hip_ctx *ctx, hipError_t e, const char *what);
// Make hipSetDevice(ctx->device) current; returns 0 or an error code.
int enter(mrml_hip_ctx *ctx);
// Check the launch that just happened.
int check_launch(mrml_hip_ctx *ctx, const char *kernel);
// Ensure at least `bytes` of scratch; returns its device pointer or null on failure.
void *workspace(mrml_hip_ctx *ctx, size_t bytes);

__host__ __device__ inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Launchers implemented in the kernel translation units.  All return 0 or a
// negative status and assume arguments were validated by the ABI layer.
int launch_quantize_q8_0(mrml_hip_ctx *ctx, const float *x, void *gguf, void *pack, int32_t n);
int launch_repack_q4_0(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols);
int launch_repack_q8_0(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols);
int launch_repack_q4_k(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols);
int launch_zero(mrml_hip_ctx *ctx, void *dst, size_t bytes);
int launch_copy(mrml_hip_ctx *ctx, void *dst, const void *src, size_t bytes);

// Q4_0 x Q8_0 matvec family; `xpack` is an activation pack for `cols`.
int launch_gemv_q4_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                     int32_t rows, int32_t cols);
int launch_gemv_q4_0_gguf(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                          int32_t rows, int32_t cols);
// f32-input forms: quantise x inside the kernel where a fixed instance exists.
int launch_gemv_q4_0_x(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols);
int launch_gemv_q4_0_geglu_x(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                             void *act_pack, int32_t rows, int32_t cols);
int launch_gemv_q4_0_qkv_x(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *x,
                           float *y, int32_t q_rows, int32_t kv_rows, int32_t cols);
int launch_gemv_q4_0_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack,
                           float *act, int32_t rows, int32_t cols);
int launch_gemv_q4_0_qkv(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv,
                         const void *xpack, float *y, int32_t q_rows, int32_t kv_rows,
                         int32_t cols);
int launch_gemv_q8_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                     int32_t rows, int32_t cols, int32_t softcap);
int launch_gemv_q4_k(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y,
                     int32_t rows, int32_t cols);
int launch_argmax_f32(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out);

}  // namespace mrml
