// runtime.hip -- the C ABI (include/mrml_hip.h): context, memory, argument
// validation and dispatch to the kernel launchers.
//
// Replaces the CUDA driver-API host layer of the reference
// (crates/mrml-tensor/src/cuda.rs): there, a dlopen'd libcuda, a PTX module
// and a per-device stream; here, libamdhip64 linked directly, gfx950 code
// objects linked into this library, and one stream per context.

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "device.h"
#include "exact_sum.h"
#include "internal.h"

namespace mrml {

int fail(mrml_hip_ctx *ctx, int code, const char *fmt, ...)
{
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return code;
}

int hip_fail(mrml_hip_ctx *ctx, hipError_t e, const char *what)
{
    return fail(ctx, MRML_HIP_E_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

int enter(mrml_hip_ctx *ctx)
{
    hipError_t e = hipSetDevice(ctx->device);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipSetDevice");
}

int check_launch(mrml_hip_ctx *ctx, const char *kernel)
{
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(ctx, e, kernel);
}

void *workspace(mrml_hip_ctx *ctx, size_t bytes)
{
    if (bytes <= ctx->ws_bytes) return ctx->ws;
    size_t want = align_up(bytes, (size_t)1 << 20);
    if (ctx->ws) {
        // The old scratch may still be read by queued work.
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) { hip_fail(ctx, e, "hipStreamSynchronize (workspace)"); return nullptr; }
        (void)hipFree(ctx->ws);
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        fail(ctx, MRML_HIP_E_ALLOC, "workspace hipMalloc(%zu): %s", want, hipGetErrorString(e));
        return nullptr;
    }
    ctx->ws = p;
    ctx->ws_bytes = want;
    return p;
}

bool host_expf_fused()
{
    static const bool fused = __builtin_cpu_supports("fma") && __builtin_cpu_supports("avx2");
    return fused;
}

int fill_rope_freqs(mrml_hip_ctx *ctx, float *d_freqs, int head_dim, float base)
{
    float (*volatile f_pow)(float, float) = powf;  // the C library's powf, not a folded constant
    std::vector<float> f(head_dim / 2);
    for (int i = 0; i < head_dim / 2; ++i) f[i] = f_pow(base, (float)(2 * i) / (float)head_dim);
    hipError_t e = hipMemcpyAsync(d_freqs, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MRML_HIP_OK : hip_fail(ctx, e, "rope frequencies upload");
}

int fill_rope_table(mrml_hip_ctx *ctx, float *d_table, int n_pos, int head_dim, float base, float freq_scale)
{
    // Called through pointers so the compiler keeps three separate libm calls
    // (the reference calls powf, cosf and sinf; a merged sincosf is a
    // different routine).
    float (*volatile f_pow)(float, float) = powf;
    float (*volatile f_cos)(float) = cosf;
    float (*volatile f_sin)(float) = sinf;
    const int half = head_dim / 2;
    std::vector<float> inv(half), tab((size_t)n_pos * half * 2);
    for (int i = 0; i < half; ++i) inv[i] = f_pow(base, (float)(2 * i) / (float)head_dim);
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float theta = (float)p * freq_scale / inv[i];  // ops.rs:185-208 order
            tab[((size_t)p * half + i) * 2] = f_cos(theta);
            tab[((size_t)p * half + i) * 2 + 1] = f_sin(theta);
        }
    hipError_t e = hipMemcpyAsync(d_table, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MRML_HIP_OK : hip_fail(ctx, e, "rope table upload");
}

}  // namespace mrml

using namespace mrml;

extern "C" {

const char *mrml_hip_status_string(int status)
{
    switch (status) {
    case MRML_HIP_OK: return "ok";
    case MRML_HIP_E_INVALID: return "invalid argument";
    case MRML_HIP_E_ALLOC: return "allocation failed";
    case MRML_HIP_E_HIP: return "HIP runtime error";
    case MRML_HIP_E_UNSUPPORTED: return "unsupported";
    case MRML_HIP_E_NODEVICE: return "no gfx950 device";
    case MRML_HIP_E_FORMAT: return "malformed GGUF file";
    case MRML_HIP_E_IO: return "file I/O error";
    case MRML_HIP_E_NOTFOUND: return "not found";
    default: return "unknown status";
    }
}

int mrml_hip_device_count(int32_t *count)
{
    if (!count) return MRML_HIP_E_INVALID;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return MRML_HIP_OK;
}

int mrml_hip_create(int32_t device, mrml_hip_ctx **out)
{
    if (!out) return MRML_HIP_E_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return MRML_HIP_E_NODEVICE;
    mrml_hip_ctx *ctx = new (std::nothrow) mrml_hip_ctx();
    if (!ctx) return MRML_HIP_E_ALLOC;
    ctx->device = device;
    if (hipSetDevice(device) != hipSuccess || hipGetDeviceProperties(&ctx->props, device) != hipSuccess) {
        delete ctx;
        return MRML_HIP_E_NODEVICE;
    }
    // The kernels are compiled for gfx950 only.
    if (std::strncmp(ctx->props.gcnArchName, "gfx950", 6) != 0) {
        delete ctx;
        return MRML_HIP_E_NODEVICE;
    }
    // Default priority, non-blocking with respect to the null stream.
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return MRML_HIP_E_HIP;
    }
    // The device address of the allocation-free GEMM's scratch (once per device).
    if (gemm_noalloc_scratch(ctx, &ctx->noalloc_scratch) != MRML_HIP_OK) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return MRML_HIP_E_HIP;
    }
    *out = ctx;
    return MRML_HIP_OK;
}

int mrml_hip_destroy(mrml_hip_ctx *ctx)
{
    if (!ctx) return MRML_HIP_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return MRML_HIP_OK;
}

const char *mrml_hip_last_error(const mrml_hip_ctx *ctx)
{
    return ctx ? ctx->err.c_str() : "null context";
}

int mrml_hip_sync(mrml_hip_ctx *ctx)
{
    CTX_GUARD(ctx);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    // Kernels whose bounded waits gave up went on with wrong data.
    uint32_t t_gemv = 0, t_decode = 0;
    if ((e = wait_guard_gemv(-1, &t_gemv)) != hipSuccess) return hip_fail(ctx, e, "wait guard (matvec)");
    if ((e = wait_guard_decode(-1, &t_decode)) != hipSuccess) return hip_fail(ctx, e, "wait guard (decode)");
    if (t_gemv + t_decode)
        return fail(ctx, MRML_HIP_E_HIP,
                    "%u bounded LDS-counter waits gave up (%u matvec, %u decode): the results since the last sync "
                    "are wrong", t_gemv + t_decode, t_gemv, t_decode);
    return MRML_HIP_OK;
}

int mrml_hip_set_wait_limit(mrml_hip_ctx *ctx, int32_t polls)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, polls <= (1 << 24), "set_wait_limit: polls=%d above 2^24", polls);
    if (polls < 0) polls = mrml_xsum::kSyncSpin;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = wait_guard_gemv(polls, nullptr);
    if (e == hipSuccess) e = wait_guard_decode(polls, nullptr);
    return e == hipSuccess ? MRML_HIP_OK : hip_fail(ctx, e, "set_wait_limit");
}

int mrml_hip_device_info_get(mrml_hip_ctx *ctx, mrml_hip_device_info *info)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, info, "info is null");
    std::memset(info, 0, sizeof *info);
    std::snprintf(info->name, sizeof info->name, "%s", ctx->props.gcnArchName);
    info->compute_units = ctx->props.multiProcessorCount;
    info->clock_khz = ctx->props.clockRate;
    int rv = 0;
    (void)hipRuntimeGetVersion(&rv);
    info->runtime_version = rv;
    info->abi_version = MRML_HIP_ABI_VERSION;
    info->total_memory = ctx->props.totalGlobalMem;
    info->l2_bytes = (uint64_t)ctx->props.l2CacheSize;
    return MRML_HIP_OK;
}

int mrml_hip_memory_info(mrml_hip_ctx *ctx, uint64_t *free_bytes, uint64_t *total_bytes)
{
    CTX_GUARD(ctx);
    size_t f = 0, t = 0;
    hipError_t e = hipMemGetInfo(&f, &t);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMemGetInfo");
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return MRML_HIP_OK;
}

void *mrml_hip_stream(mrml_hip_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int mrml_hip_reserve_workspace(mrml_hip_ctx *ctx, size_t bytes)
{
    CTX_GUARD(ctx);
    return workspace(ctx, bytes) ? MRML_HIP_OK : MRML_HIP_E_ALLOC;
}

int mrml_hip_workspace_bytes(mrml_hip_ctx *ctx, size_t *bytes)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, bytes, "workspace_bytes: null output");
    *bytes = ctx->ws_bytes;
    return MRML_HIP_OK;
}

int mrml_hip_graph_begin(mrml_hip_ctx *ctx)
{
    CTX_GUARD(ctx);
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipStreamBeginCapture");
}

int mrml_hip_graph_end(mrml_hip_ctx *ctx, void **graph_exec_out)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, graph_exec_out, "graph_exec_out is null");
    *graph_exec_out = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphInstantiate");
    *graph_exec_out = (void *)exec;
    return MRML_HIP_OK;
}

int mrml_hip_graph_launch(mrml_hip_ctx *ctx, void *graph_exec)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, graph_exec, "graph_exec is null");
    hipError_t e = hipGraphLaunch((hipGraphExec_t)graph_exec, ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipGraphLaunch");
}

int mrml_hip_graph_destroy(mrml_hip_ctx *ctx, void *graph_exec)
{
    CTX_GUARD(ctx);
    if (!graph_exec) return MRML_HIP_OK;
    hipError_t e = hipGraphExecDestroy((hipGraphExec_t)graph_exec);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipGraphExecDestroy");
}

int mrml_hip_malloc(mrml_hip_ctx *ctx, size_t bytes, void **d_out)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, d_out, "d_out is null");
    *d_out = nullptr;
    hipError_t e = hipMalloc(d_out, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(ctx, MRML_HIP_E_ALLOC, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return MRML_HIP_OK;
}

int mrml_hip_free(mrml_hip_ctx *ctx, void *d_ptr)
{
    CTX_GUARD(ctx);
    if (!d_ptr) return MRML_HIP_OK;
    hipError_t e = hipFree(d_ptr);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipFree");
}

int mrml_hip_memcpy_h2d(mrml_hip_ctx *ctx, void *d_dst, const void *h_src, size_t bytes)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, d_dst && h_src, "null pointer");
    hipError_t e = hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipMemcpy H2D");
}

int mrml_hip_memcpy_d2h(mrml_hip_ctx *ctx, void *h_dst, const void *d_src, size_t bytes)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, h_dst && d_src, "null pointer");
    hipError_t e = hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipMemcpy D2H");
}

int mrml_hip_memcpy_h2d_async(mrml_hip_ctx *ctx, void *d_dst, const void *h_src, size_t bytes)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, d_dst && h_src, "null pointer");
    hipError_t e = hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipMemcpyAsync H2D");
}

int mrml_hip_memcpy_d2d_async(mrml_hip_ctx *ctx, void *d_dst, const void *d_src, size_t bytes)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, d_dst && d_src, "null pointer");
    hipError_t e = hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(ctx, e, "hipMemcpyAsync D2D");
}

int mrml_hip_zero_async(mrml_hip_ctx *ctx, void *d_dst, size_t bytes)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, d_dst, "null pointer");
    return launch_zero(ctx, d_dst, bytes);
}

int mrml_hip_copy_kernel(mrml_hip_ctx *ctx, void *d_dst, const void *d_src, size_t bytes)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, d_dst && d_src, "null pointer");
    REQUIRE(ctx, bytes % 16 == 0 && ((uintptr_t)d_dst % 16) == 0 && ((uintptr_t)d_src % 16) == 0,
            "copy_kernel: bytes and pointers must be 16-byte aligned");
    return launch_copy(ctx, d_dst, d_src, bytes);
}

int mrml_hip_read_kernel(mrml_hip_ctx *ctx, const void *d_src, size_t bytes, void *d_sink)
{
    CTX_GUARD(ctx);
    if (!bytes) return MRML_HIP_OK;
    REQUIRE(ctx, d_src && d_sink, "null pointer");
    REQUIRE(ctx, bytes % 16 == 0 && ((uintptr_t)d_src % 16) == 0 && ((uintptr_t)d_sink % 4) == 0,
            "read_kernel: bytes and source must be 16-byte aligned");
    REQUIRE(ctx, bytes / 16 / (256 * 8) < (1u << 31), "read_kernel: %zu bytes is too many", bytes);
    return launch_read(ctx, d_src, bytes, d_sink);
}

// ---- layout conversion ----------------------------------------------------

int mrml_hip_repack_q4_0(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, src && dst, "null pointer");
    REQUIRE(ctx, rows > 0 && cols > 0 && cols % 32 == 0, "repack_q4_0: rows=%d cols=%d (cols %% 32 != 0?)", rows, cols);
    REQUIRE(ctx, src != dst, "repack_q4_0: in-place conversion is not supported");
    return launch_repack_q4_0(ctx, src, dst, rows, cols);
}

int mrml_hip_repack_q8_0(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, src && dst, "null pointer");
    REQUIRE(ctx, rows > 0 && cols > 0 && cols % 32 == 0, "repack_q8_0: rows=%d cols=%d", rows, cols);
    REQUIRE(ctx, src != dst, "repack_q8_0: in-place conversion is not supported");
    return launch_repack_q8_0(ctx, src, dst, rows, cols);
}

int mrml_hip_repack_q4_k(mrml_hip_ctx *ctx, const void *src, void *dst, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, src && dst, "null pointer");
    REQUIRE(ctx, rows > 0 && cols > 0 && cols % 256 == 0, "repack_q4_k: rows=%d cols=%d (cols %% 256 != 0?)", rows, cols);
    REQUIRE(ctx, src != dst, "repack_q4_k: in-place conversion is not supported");
    return launch_repack_q4_k(ctx, src, dst, rows, cols);
}

// ---- quantiser ------------------------------------------------------------

size_t mrml_hip_q8_0_pack_bytes(int32_t n) { return n > 0 ? act_pack_bytes(n / 32) : 0; }

int mrml_hip_quantize_q8_0(mrml_hip_ctx *ctx, const float *x, void *gguf, void *pack, int32_t n)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, x, "x is null");
    REQUIRE(ctx, gguf || pack, "quantize_q8_0: no output requested");
    REQUIRE(ctx, n > 0 && n % 32 == 0, "quantize_q8_0: n=%d is not a positive multiple of 32", n);
    REQUIRE(ctx, ((uintptr_t)x & 15) == 0 && ((uintptr_t)pack & 15) == 0 && ((uintptr_t)gguf & 1) == 0,
            "quantize_q8_0: x and pack must be 16-byte aligned, gguf 2-byte aligned");
    return launch_quantize_q8_0(ctx, x, gguf, pack, n);
}

// Quantise x into the scratch pack; returns the pack or null (error recorded).
static void *quantize_to_scratch(mrml_hip_ctx *ctx, const float *x, int32_t cols, size_t extra_bytes = 0)
{
    void *ws = workspace(ctx, act_pack_bytes(cols / 32) + extra_bytes);
    if (!ws) return nullptr;
    if (launch_quantize_q8_0(ctx, x, nullptr, ws, cols)) return nullptr;
    return ws;
}

#define CHECK_MATVEC(ctx, w, x, y, rows, cols, mult)                                          \
    do {                                                                                      \
        REQUIRE(ctx, (w) && (x) && (y), "null pointer");                                      \
        REQUIRE(ctx, ((uintptr_t)(x) & 15) == 0, "x / pack must be 16-byte aligned");          \
        REQUIRE(ctx, (rows) > 0 && (cols) > 0 && (cols) % (mult) == 0,                        \
                "rows=%d cols=%d: need rows > 0 and cols a positive multiple of %d",          \
                (int)(rows), (int)(cols), (int)(mult));                                       \
    } while (0)

int mrml_hip_gemv_q4_0(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, x, y, rows, cols, 32);
    return launch_gemv_q4_0_x(ctx, w, x, y, rows, cols);
}

int mrml_hip_gemv_q4_0_q8(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, xpack, y, rows, cols, 32);
    return launch_gemv_q4_0(ctx, w, xpack, y, rows, cols);
}

int mrml_hip_gemv_q4_0_q8_relaxed(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows,
                                  int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, xpack, y, rows, cols, 32);
    return launch_gemv_q4_0(ctx, w, xpack, y, rows, cols, true);
}

int mrml_hip_gemv_q4_0_gguf(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, x, y, rows, cols, 32);
    void *xp = quantize_to_scratch(ctx, x, cols);
    if (!xp) return MRML_HIP_E_ALLOC;
    return launch_gemv_q4_0_gguf(ctx, w, xp, y, rows, cols);
}

int mrml_hip_gemv_q4_0_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                             int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wg, x, act, rows, cols, 32);
    REQUIRE(ctx, wu, "w_up is null");
    return launch_gemv_q4_0_geglu_x(ctx, wg, wu, x, act, nullptr, rows, cols);
}

int mrml_hip_gemv_q4_0_geglu_pack(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                                  void *act_pack, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wg, x, act_pack, rows, cols, 32);
    REQUIRE(ctx, wu, "w_up is null");
    REQUIRE(ctx, rows % 32 == 0, "rows=%d is not a multiple of 32", rows);
    return launch_gemv_q4_0_geglu_x(ctx, wg, wu, x, act, act_pack, rows, cols);
}

int mrml_hip_ffn_geglu_q4_0(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *wd, const float *x,
                            float *act, float *y, int32_t dim, int32_t ffn)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wg, x, y, ffn, dim, 32);
    REQUIRE(ctx, wu && wd, "null pointer");
    REQUIRE(ctx, ffn % 32 == 0, "ffn=%d is not a multiple of 32", ffn);
    if (ffn_split_ok(dim, ffn)) {
        // the balanced GeGLU (one workgroup per CU) forming the pack blocks it
        // owns whole, then the down projection quantising the rest from the
        // f32 outputs: the same Q8_0 bits as one quantiser over all of them
        const size_t pk = align_up(act_pack_bytes(ffn / 32), 256);
        uint8_t *ws = (uint8_t *)workspace(ctx, pk + (act ? 0 : (size_t)ffn * sizeof(float)));
        if (!ws) return MRML_HIP_E_ALLOC;
        float *a = act ? act : reinterpret_cast<float *>(ws + pk);
        REQUIRE(ctx, ((uintptr_t)a & 15) == 0, "ffn_geglu_q4_0: act must be 16-byte aligned");
        return launch_ffn_split(ctx, wg, wu, wd, x, a, ws, y, dim, ffn);
    }
    void *pk = workspace(ctx, act_pack_bytes(ffn / 32));
    if (!pk) return MRML_HIP_E_ALLOC;
    if (int rc = launch_gemv_q4_0_geglu_x(ctx, wg, wu, x, act, pk, ffn, dim)) return rc;
    return launch_gemv_q4_0(ctx, wd, pk, y, dim, ffn);
}

int mrml_hip_ffn_split_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                             void *act_pack, const void *wd_next, int32_t dim, int32_t ffn)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wg, x, act, ffn, dim, 32);
    REQUIRE(ctx, wu && act_pack, "null pointer");
    REQUIRE(ctx, ffn_split_ok(dim, ffn), "ffn_split_geglu: dim=%d ffn=%d is not a shape of the split form", dim, ffn);
    REQUIRE(ctx, ((uintptr_t)act_pack & 15) == 0, "ffn_split_geglu: act_pack must be 16-byte aligned");
    return launch_geglu_split(ctx, wg, wu, x, act, act_pack, ffn, dim, wd_next);
}

int mrml_hip_ffn_split_down(mrml_hip_ctx *ctx, const void *wd, const void *act_pack, const float *act, float *y,
                            int32_t dim, int32_t ffn)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wd, act, y, dim, ffn, 32);
    REQUIRE(ctx, act_pack, "null pointer");
    REQUIRE(ctx, ffn_split_ok(dim, ffn), "ffn_split_down: dim=%d ffn=%d is not a shape of the split form", dim, ffn);
    REQUIRE(ctx, ((uintptr_t)act_pack & 15) == 0, "ffn_split_down: act_pack must be 16-byte aligned");
    return launch_down_mix(ctx, wd, act_pack, act, y, dim, ffn);
}

int mrml_hip_gemv_q4_0_geglu_q8(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack,
                                float *act, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wg, xpack, act, rows, cols, 32);
    REQUIRE(ctx, wu, "w_up is null");
    return launch_gemv_q4_0_geglu(ctx, wg, wu, xpack, act, rows, cols);
}

int mrml_hip_gemv_q4_0_qkv_q8(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv,
                              const void *xpack, float *y, int32_t q_rows, int32_t kv_rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wq, xpack, y, q_rows, cols, 32);
    REQUIRE(ctx, wk && wv, "null pointer");
    REQUIRE(ctx, kv_rows > 0, "kv_rows=%d", kv_rows);
    return launch_gemv_q4_0_qkv(ctx, wq, wk, wv, xpack, y, q_rows, kv_rows, cols);
}

int mrml_hip_gemv_q4_0_qkv(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *x,
                           float *y, int32_t q_rows, int32_t kv_rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, wq, x, y, q_rows, cols, 32);
    REQUIRE(ctx, wk && wv, "null pointer");
    REQUIRE(ctx, kv_rows > 0, "kv_rows=%d", kv_rows);
    return launch_gemv_q4_0_qkv_x(ctx, wq, wk, wv, x, y, q_rows, kv_rows, cols);
}

int mrml_hip_gemv_q8_0(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols,
                       int32_t softcap)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, x, y, rows, cols, 32);
    void *xp = quantize_to_scratch(ctx, x, cols);
    if (!xp) return MRML_HIP_E_ALLOC;
    return launch_gemv_q8_0(ctx, w, xp, y, rows, cols, softcap);
}

int mrml_hip_gemv_q8_0_q8(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols,
                          int32_t softcap)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, xpack, y, rows, cols, 32);
    return launch_gemv_q8_0(ctx, w, xpack, y, rows, cols, softcap);
}

int mrml_hip_gemv_q4_k_q8(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, xpack, y, rows, cols, 256);
    return launch_gemv_q4_k(ctx, w, xpack, y, rows, cols);
}

int mrml_hip_gemv_q4_k(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols)
{
    CTX_GUARD(ctx);
    CHECK_MATVEC(ctx, w, x, y, rows, cols, 256);
    void *xp = quantize_to_scratch(ctx, x, cols);
    if (!xp) return MRML_HIP_E_ALLOC;
    return launch_gemv_q4_k(ctx, w, xp, y, rows, cols);
}

#define CHECK_GEMM(ctx, w, x, y, rows, cols, batch)                                                  \
    do {                                                                                             \
        REQUIRE(ctx, (w) && (x) && (y), "null pointer");                                             \
        REQUIRE(ctx, ((uintptr_t)(x) & 15) == 0 && ((uintptr_t)(y) & 15) == 0,                       \
                "x / pack and y must be 16-byte aligned");                                           \
        REQUIRE(ctx, gemm_shape_ok(rows, cols, batch),                                               \
                "gemm rows=%d cols=%d batch=%d: need rows > 0, cols %% 32 == 0, batch > 0 "           \
                "and W / activations below 2 GiB",                                                   \
                (int)(rows), (int)(cols), (int)(batch));                                             \
        REQUIRE(ctx, (int64_t)(batch) * (cols) <= INT32_MAX && (int64_t)(batch) * (rows) <= INT32_MAX, \
                "gemm batch=%d too large for rows=%d cols=%d", (int)(batch), (int)(rows), (int)(cols)); \
    } while (0)

int mrml_hip_gemm_q4_0(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols,
                       int32_t batch)
{
    CTX_GUARD(ctx);
    CHECK_GEMM(ctx, w, x, y, rows, cols, batch);
    void *gp = workspace(ctx, gemm_pack_bytes(cols, batch));
    if (!gp) return MRML_HIP_E_ALLOC;
    int rc = launch_gemm_pack_quantize(ctx, x, gp, cols, batch);
    return rc ? rc : launch_gemm_q4_0(ctx, w, gp, y, rows, cols, batch);
}

int mrml_hip_gemm_q4_0_relaxed(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows,
                               int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    CHECK_GEMM(ctx, w, x, y, rows, cols, batch);
    void *gp = workspace(ctx, gemm_pack_bytes(cols, batch));
    if (!gp) return MRML_HIP_E_ALLOC;
    int rc = launch_gemm_pack_quantize(ctx, x, gp, cols, batch);
    return rc ? rc : launch_gemm_q4_0(ctx, w, gp, y, rows, cols, batch, 0, true);
}

int mrml_hip_gemm_q4_0_noalloc(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows,
                               int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    CHECK_GEMM(ctx, w, x, y, rows, cols, batch);
    const size_t need = gemm_pack_bytes(cols, batch);
    REQUIRE(ctx, need <= gemm_noalloc_scratch_bytes(),
            "gemm_q4_0_noalloc: cols=%d batch=%d needs a %zu-byte GEMM pack, above the %zu-byte device scratch "
            "(at most %zu token groups of 32 x cols/32 blocks x 1152 bytes)",
            cols, batch, need, gemm_noalloc_scratch_bytes(), gemm_noalloc_scratch_bytes() / ((size_t)(cols / 32) * 1152));
    void *gp = ctx->noalloc_scratch;
    if (!gp) return fail(ctx, MRML_HIP_E_HIP, "gemm_q4_0_noalloc: the device scratch address is unknown");
    int rc = launch_gemm_pack_quantize(ctx, x, gp, cols, batch);
    return rc ? rc : launch_gemm_q4_0(ctx, w, gp, y, rows, cols, batch);
}

size_t mrml_hip_gemm_q4_0_noalloc_max_pack_bytes(void) { return gemm_noalloc_scratch_bytes(); }

int mrml_hip_gemm_q4_0_q8(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows,
                          int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    CHECK_GEMM(ctx, w, xpack, y, rows, cols, batch);
    void *gp = workspace(ctx, gemm_pack_bytes(cols, batch));
    if (!gp) return MRML_HIP_E_ALLOC;
    int rc = launch_gemm_pack_from_act(ctx, xpack, gp, cols, batch);
    return rc ? rc : launch_gemm_q4_0(ctx, w, gp, y, rows, cols, batch);
}

int mrml_hip_gemm_q4_0_qkv(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *x,
                           float *y, int32_t q_rows, int32_t kv_rows, int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, wk && wv, "gemm_q4_0_qkv: null pointer");
    CHECK_GEMM(ctx, wq, x, y, q_rows, cols, batch);
    REQUIRE(ctx, gemm_shape_ok(kv_rows, cols, batch), "gemm_q4_0_qkv: kv_rows=%d must be positive", kv_rows);
    const int32_t total = q_rows + 2 * kv_rows;
    REQUIRE(ctx, (int64_t)batch * total <= INT32_MAX, "gemm_q4_0_qkv: batch=%d too large", batch);
    void *gp = workspace(ctx, gemm_pack_bytes(cols, batch));
    if (!gp) return MRML_HIP_E_ALLOC;
    // one GEMM pack for the three products, run as one launch over the
    // stacked rows; each writes its column range of the stacked
    // [batch][q | k | v] rows (row stride q_rows + 2*kv_rows)
    if (int rc = launch_gemm_pack_quantize(ctx, x, gp, cols, batch)) return rc;
    const void *w3[3] = {wq, wk, wv};
    const int32_t r3[3] = {q_rows, kv_rows, kv_rows};
    return launch_gemm_q4_0_stacked(ctx, w3, r3, 3, gp, y, cols, batch, total);
}

int mrml_hip_gemm_q4_0_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                             int32_t rows, int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, wu, "gemm_q4_0_geglu: null pointer");
    CHECK_GEMM(ctx, wg, x, act, rows, cols, batch);
    // workspace: the GEMM pack, then the gate and up products [batch][rows]
    const size_t pk = align_up(gemm_pack_bytes(cols, batch), 256), n = (size_t)batch * rows;
    uint8_t *ws = (uint8_t *)workspace(ctx, pk + 2 * n * sizeof(float));
    if (!ws) return MRML_HIP_E_ALLOC;
    float *g = reinterpret_cast<float *>(ws + pk), *u = g + n;
    if (int rc = launch_gemm_pack_quantize(ctx, x, ws, cols, batch)) return rc;
    if (int rc = launch_gemm_q4_0(ctx, wg, ws, g, rows, cols, batch)) return rc;
    if (int rc = launch_gemm_q4_0(ctx, wu, ws, u, rows, cols, batch)) return rc;
    return launch_geglu_rows(ctx, g, u, act, (int)n);
}

size_t mrml_hip_gemm_pack_bytes(int32_t cols, int32_t batch)
{
    return (cols > 0 && cols % 32 == 0 && batch > 0) ? gemm_pack_bytes(cols, batch) : 0;
}

int mrml_hip_quantize_q8_0_gemm(mrml_hip_ctx *ctx, const float *x, void *gpack, int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    CHECK_GEMM(ctx, gpack, x, gpack, 32, cols, batch);
    return launch_gemm_pack_quantize(ctx, x, gpack, cols, batch);
}

int mrml_hip_gemm_q4_0_gpack(mrml_hip_ctx *ctx, const void *w, const void *gpack, float *y, int32_t rows,
                             int32_t cols, int32_t batch)
{
    CTX_GUARD(ctx);
    CHECK_GEMM(ctx, w, gpack, y, rows, cols, batch);
    return launch_gemm_q4_0(ctx, w, gpack, y, rows, cols, batch);
}

int mrml_hip_argmax_f32(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, x && out, "null pointer");
    REQUIRE(ctx, n > 0, "argmax: n=%d", n);
    return launch_argmax_f32(ctx, x, n, out);
}

int mrml_hip_vocab_topk(mrml_hip_ctx *ctx, const float *logits, const uint8_t *valid, const int32_t *recent,
                        float *scores, int32_t *ids, int32_t vocab, int32_t n_recent, int32_t generated_count,
                        int32_t k, int32_t partitions)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, logits && scores && ids && (recent || n_recent == 0), "vocab_topk: null pointer");
    REQUIRE(ctx, n_recent >= 0 && n_recent <= 32, "vocab_topk: n_recent=%d outside 0..32", n_recent);
    REQUIRE(ctx, vocab_topk_ok(vocab, k, partitions),
            "vocab_topk: vocab=%d, k=%d, partitions=%d unsupported (k 1..64, 1 <= partitions <= vocab, "
            "partitions of at most 2097152 ids)",
            vocab, k, partitions);
    void *ws = workspace(ctx, vocab_topk_scratch_bytes(vocab, k, partitions));
    if (!ws) return MRML_HIP_E_ALLOC;
    return launch_vocab_topk(ctx, logits, valid, recent, scores, ids, vocab, n_recent, generated_count, k,
                             partitions, ws);
}

int mrml_hip_vocab_select(mrml_hip_ctx *ctx, const float *logits, int32_t vocab, const uint8_t *valid,
                          const int32_t *recent, int32_t n_recent, int32_t generated_count, int32_t scoring,
                          float temperature, uint64_t pos, int32_t k, int32_t *token, float *scores, int32_t *ids)
{
    CTX_GUARD(ctx);
    REQUIRE(ctx, logits && (recent || n_recent == 0), "vocab_select: null pointer");
    REQUIRE(ctx, n_recent >= 0 && n_recent <= 32, "vocab_select: n_recent=%d outside 0..32", n_recent);
    REQUIRE(ctx, scoring == MRML_HIP_SCORE_CPU || scoring == MRML_HIP_SCORE_DEVICE,
            "vocab_select: scoring=%d is neither CPU (0) nor DEVICE (1)", scoring);
    REQUIRE(ctx, temperature == temperature, "vocab_select: temperature is NaN");
    REQUIRE(ctx, vocab_select_ok(vocab, k), "vocab_select: vocab=%d with k=%d unsupported (k 1..64, vocab <= 2097152)",
            vocab, k);
    void *ws = workspace(ctx, vocab_select_scratch_bytes(vocab, k));
    if (!ws) return MRML_HIP_E_ALLOC;
    return launch_vocab_select(ctx, logits, vocab, valid, recent, n_recent, generated_count, scoring, temperature,
                               pos, k, token, scores, ids, ws, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
}

}  // extern "C"
