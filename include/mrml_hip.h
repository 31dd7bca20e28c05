/*
 * mrml_hip.h -- C ABI of the MI355X (gfx950) backend for the MRML decode hot
 * path: GGUF block-quantised matrix-vector products (Q4_0, Q8_0, Q4_K) and the
 * small-batch Q4_0 product, plus the ops around them in a token step.
 *
 * It replaces the CUDA operator surface of mitchellrenouf/QT_llama.cpp,
 * `CudaDevice` / `CudaBuffer` in crates/mrml-tensor/src/cuda.rs; each entry
 * point names the reference method it stands in for.  The arithmetic is the
 * reference's CPU path (crates/mrml-tensor/src/quant.rs, ops.rs): activations
 * are quantised to Q8_0 with the reference routine and every block dot is an
 * exact integer sum, folded into f32 in block order without FMA, so matvec
 * outputs are bit-identical to the CPU kernels.
 *
 * Conventions
 *  - Every function returns 0 (MRML_HIP_OK) or a negative MRML_HIP_E_* code;
 *    nothing aborts or throws across the ABI.  mrml_hip_last_error(ctx) holds
 *    the message of the last failure on that context.
 *  - Pointers named d_* are device pointers (from mrml_hip_malloc or any
 *    hipMalloc'd memory on the context's device); h_* are host pointers.
 *  - All ops are asynchronous on the context's single stream and ordered on
 *    it.  A context is used from one thread at a time (the reference
 *    serialises every CudaDevice call behind one lock, engine.rs:6-8).
 *  - Dimensions are int32 like the reference's launch arguments; `cols` must be
 *    a multiple of 32 (256 for Q4_K), as the reference's kernel schemas require
 *    (crates/mrml-kernel/src/virtual_gpu.rs:2897-3125).
 *  - Activation vectors (f32 x) and Q8_0 activation packs are read in 16-byte
 *    units and must be 16-byte aligned (hipMalloc returns 256-byte aligned
 *    memory; whole-block offsets keep the alignment); misaligned pointers are
 *    rejected with MRML_HIP_E_INVALID.
 *  - Weight layouts: the *_gguf entry points read the raw GGUF bytes the
 *    reference uploads unchanged (model.rs:651-705).  The other weight
 *    arguments take the backend layout written by mrml_hip_repack_* (the same
 *    number of bytes as the GGUF tensor, split into a 16-byte-aligned quant
 *    plane and a scale plane), which is what the fast kernels stream.
 */
#ifndef MRML_HIP_H
#define MRML_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MRML_HIP_ABI_VERSION 1

enum {
    MRML_HIP_OK = 0,
    MRML_HIP_E_INVALID = -1,     /* bad argument: shape, null pointer, alignment */
    MRML_HIP_E_ALLOC = -2,       /* device or host allocation failed */
    MRML_HIP_E_HIP = -3,         /* a HIP runtime call failed (message has the HIP error) */
    MRML_HIP_E_UNSUPPORTED = -4, /* shape or format this build does not implement */
    MRML_HIP_E_NODEVICE = -5     /* no gfx950 device at that index */
};

/* GGUF tensor type ids (crates/mrml-tensor/src/types.rs:7-30, gguf.rs:121-133) */
enum { MRML_HIP_Q4_0 = 2, MRML_HIP_Q8_0 = 8, MRML_HIP_Q4_K = 12 };

typedef struct mrml_hip_ctx mrml_hip_ctx;

/* CudaDeviceInfo (cuda.rs:1860-1878) with AMD fields. */
typedef struct mrml_hip_device_info {
    char     name[64];       /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t  compute_units;  /* CudaDeviceInfo::multiprocessors */
    int32_t  clock_khz;
    int32_t  runtime_version;
    int32_t  abi_version;
    uint64_t total_memory;
    uint64_t l2_bytes;
} mrml_hip_device_info;

/* ---- lifecycle: CudaDevice::{count, is_available, new, sync, device_info,
 *      get_memory_info} (cuda.rs:1957-2100) --------------------------------- */
int         mrml_hip_device_count(int32_t *count);
int         mrml_hip_create(int32_t device, mrml_hip_ctx **out);
int         mrml_hip_destroy(mrml_hip_ctx *ctx);
const char *mrml_hip_last_error(const mrml_hip_ctx *ctx);
const char *mrml_hip_status_string(int status);
int         mrml_hip_sync(mrml_hip_ctx *ctx);
int         mrml_hip_device_info_get(mrml_hip_ctx *ctx, mrml_hip_device_info *info);
int         mrml_hip_memory_info(mrml_hip_ctx *ctx, uint64_t *free_bytes, uint64_t *total_bytes);
/* The context's hipStream_t, for callers that record events on it. */
void       *mrml_hip_stream(mrml_hip_ctx *ctx);
/* Grow the internal scratch (activation packs, partial results) to at least
 * `bytes` now, so later ops never allocate (e.g. under stream capture). */
int         mrml_hip_reserve_workspace(mrml_hip_ctx *ctx, size_t bytes);

/* ---- graphs: CudaDevice::{capture, launch_graph} and CudaGraphExec
 *      (cuda.rs:1841-1858, 1957-2003).  Ops issued on the context between
 *      begin and end are recorded, not run; launch replays them on the
 *      stream.  Ops that would grow the workspace fail during capture, so call
 *      mrml_hip_reserve_workspace (or run the ops once) first. --------------- */
int mrml_hip_graph_begin(mrml_hip_ctx *ctx);
int mrml_hip_graph_end(mrml_hip_ctx *ctx, void **graph_exec_out);
int mrml_hip_graph_launch(mrml_hip_ctx *ctx, void *graph_exec);
int mrml_hip_graph_destroy(mrml_hip_ctx *ctx, void *graph_exec);

/* ---- memory: CudaBuffer::{alloc_on, from_host_on, copy_from_host,
 *      copy_to_host} (cuda.rs:1350-1490), CudaDevice::copy_from_host_async
 *      (cuda.rs:2334-2376) ------------------------------------------------------ */
int mrml_hip_malloc(mrml_hip_ctx *ctx, size_t bytes, void **d_out);
int mrml_hip_free(mrml_hip_ctx *ctx, void *d_ptr);
/* Synchronous on the context stream (the reference's copy_to_host is a
 * blocking cuMemcpyDtoH, cuda.rs:1443-1464). */
int mrml_hip_memcpy_h2d(mrml_hip_ctx *ctx, void *d_dst, const void *h_src, size_t bytes);
int mrml_hip_memcpy_d2h(mrml_hip_ctx *ctx, void *h_dst, const void *d_src, size_t bytes);
int mrml_hip_memcpy_h2d_async(mrml_hip_ctx *ctx, void *d_dst, const void *h_src, size_t bytes);
int mrml_hip_memcpy_d2d_async(mrml_hip_ctx *ctx, void *d_dst, const void *d_src, size_t bytes);
/* Zero-fill with a kernel (safe to record in a captured graph). */
int mrml_hip_zero_async(mrml_hip_ctx *ctx, void *d_dst, size_t bytes);
/* Device-to-device copy by a plain streaming kernel (16-byte aligned).  No
 * reference counterpart: the bandwidth ceiling and the known-size kernel that
 * calibrates HBM byte counters in the measurements. */
int mrml_hip_copy_kernel(mrml_hip_ctx *ctx, void *d_dst, const void *d_src, size_t bytes);

/* ---- weight layout conversion (upload path; model.rs:651-705 uploads GGUF
 *      bytes unchanged, this backend converts them once after upload) ------- */
/* GGUF Q4_0 (18 B / 32 weights) -> backend Q4_0: quant plane
 * [rows][cols/32][16 B] followed by scale plane [rows][cols/32] f16.
 * d_src and d_dst must not overlap. */
int mrml_hip_repack_q4_0(mrml_hip_ctx *ctx, const void *d_src_gguf, void *d_dst,
                         int32_t rows, int32_t cols);
/* GGUF Q8_0 (34 B / 32) -> quant plane [rows][cols/32][32 B] + scale plane f16. */
int mrml_hip_repack_q8_0(mrml_hip_ctx *ctx, const void *d_src_gguf, void *d_dst,
                         int32_t rows, int32_t cols);
/* GGUF Q4_K (144 B / 256) -> quant plane [rows][cols/256][128 B] + header plane
 * [rows][cols/256][16 B] = {f16 d, f16 dmin, u8 scales[12]}. */
int mrml_hip_repack_q4_k(mrml_hip_ctx *ctx, const void *d_src_gguf, void *d_dst,
                         int32_t rows, int32_t cols);

/* ---- activation quantisation: quant::quantize_f32_to_q8_0 (quant.rs:193-228)
 * d_x: n f32.  d_q8_gguf (nullable): n/32*34 GGUF Q8_0 bytes.  d_pack
 * (nullable): the backend activation pack of n/32*40 bytes = int8 quants
 * [n/32][32], then f32 block scales [n/32] (the f16 scale widened), then
 * int32 block sums [n/32]. */
int mrml_hip_quantize_q8_0(mrml_hip_ctx *ctx, const float *d_x, void *d_q8_gguf,
                           void *d_pack, int32_t n);
size_t mrml_hip_q8_0_pack_bytes(int32_t n);

/* ---- matrix-vector products ------------------------------------------------ */
/* CudaDevice::gemv_q4_0 (cuda.rs:2286-2306) with the CPU semantics of
 * ops::mat_vec_mul_q4_0 (ops.rs:162-180): y[r] = dot(W[r], Q8_0(x)).
 * d_w: backend Q4_0 layout; d_x: cols f32; d_y: rows f32. */
int mrml_hip_gemv_q4_0(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                       int32_t rows, int32_t cols);
/* ops::mat_vec_mul_q4_0_q8_0 (ops.rs:221-260): x already quantised, as an
 * activation pack from mrml_hip_quantize_q8_0. */
int mrml_hip_gemv_q4_0_q8(mrml_hip_ctx *ctx, const void *d_w, const void *d_xpack, float *d_y,
                          int32_t rows, int32_t cols);
/* As mrml_hip_gemv_q4_0 on raw GGUF Q4_0 bytes (no repack needed). */
int mrml_hip_gemv_q4_0_gguf(mrml_hip_ctx *ctx, const void *d_w_gguf, const float *d_x,
                            float *d_y, int32_t rows, int32_t cols);
/* CudaDevice::gemv_q4_0_geglu (cuda.rs:2521-2544) with CPU semantics
 * (model.rs:2093-2105): act[r] = gelu_tanh(g[r]) * u[r], g and u the two
 * products over one Q8_0(x).  rows = ffn width, cols = model width. */
int mrml_hip_gemv_q4_0_geglu(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up,
                             const float *d_x, float *d_act, int32_t rows, int32_t cols);
/* One Gemma-style FFN, y = W_down * Q8_0(GeGLU(W_gate x, W_up x)) (model.rs:
 * 2093-2108 with a dense GeGLU FFN): two launches, the first quantising x
 * itself and writing the Q8_0 pack of the activation for the second.  d_act
 * (nullable) also receives the f32 activation.  dim = model width (cols of
 * gate/up, rows of down), ffn = hidden width. */
int mrml_hip_ffn_geglu_q4_0(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up,
                            const void *d_w_down, const float *d_x, float *d_act, float *d_y,
                            int32_t dim, int32_t ffn);
/* The first launch of mrml_hip_ffn_geglu_q4_0 on its own: act = GeGLU of the
 * two products over Q8_0(x), written as f32 (d_act, nullable) and as the
 * activation pack of its rows values (d_act_pack, rows/32*40 bytes). */
int mrml_hip_gemv_q4_0_geglu_pack(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up,
                                  const float *d_x, float *d_act, void *d_act_pack,
                                  int32_t rows, int32_t cols);
/* As mrml_hip_gemv_q4_0_geglu with x already quantised (activation pack):
 * the shared Q8_0 input of model.rs:2096-2103. */
int mrml_hip_gemv_q4_0_geglu_q8(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up,
                                const void *d_xpack, float *d_act, int32_t rows, int32_t cols);
/* CudaDevice::gemv_q4_0_qkv (cuda.rs:2378-2404): d_y = [Wq x | Wk x | Wv x]. */
int mrml_hip_gemv_q4_0_qkv(mrml_hip_ctx *ctx, const void *d_wq, const void *d_wk,
                           const void *d_wv, const float *d_x, float *d_y,
                           int32_t q_rows, int32_t kv_rows, int32_t cols);
/* As mrml_hip_gemv_q4_0_qkv with x already quantised (model.rs:1389-1401). */
int mrml_hip_gemv_q4_0_qkv_q8(mrml_hip_ctx *ctx, const void *d_wq, const void *d_wk,
                              const void *d_wv, const void *d_xpack, float *d_y,
                              int32_t q_rows, int32_t kv_rows, int32_t cols);
/* CudaDevice::gemv_q8_0 (cuda.rs:2546-2577) with the CPU semantics of the
 * vocabulary loop (model.rs:2842-2853): y[r] = dot_q8_0_q8_0(W[r], Q8_0(x)),
 * then 30*tanh(y/30) when softcap != 0.  d_w: backend Q8_0 layout. */
int mrml_hip_gemv_q8_0(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                       int32_t rows, int32_t cols, int32_t softcap);
/* Q4_K (build-defined semantics, GGUF layout; the reference has no Q4_K dot):
 * y[r] = sum over sub-blocks j of
 *        (float)isum_j*((d*sc_j)*d_a) - (float)bsum_j*((dmin*m_j)*d_a),
 * folded in order.  d_w: backend Q4_K layout. */
int mrml_hip_gemv_q4_k(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                       int32_t rows, int32_t cols);

/* Greedy pick over n f32 scores (model.rs:2869-2888; GPU tie rule
 * kernels.rs:1144-1145): index of the maximum, lowest index on ties, NaN
 * never wins.  d_out: one int32 on the device. */
int mrml_hip_argmax_f32(mrml_hip_ctx *ctx, const float *d_x, int32_t n, int32_t *d_out);

#ifdef __cplusplus
}
#endif
#endif
