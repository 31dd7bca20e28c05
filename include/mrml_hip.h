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

#define MRML_HIP_ABI_VERSION 2

enum {
    MRML_HIP_OK = 0,
    MRML_HIP_E_INVALID = -1,     /* bad argument: shape, null pointer, alignment */
    MRML_HIP_E_ALLOC = -2,       /* device or host allocation failed */
    MRML_HIP_E_HIP = -3,         /* a HIP runtime call failed (message has the HIP error) */
    MRML_HIP_E_UNSUPPORTED = -4, /* shape or format this build does not implement */
    MRML_HIP_E_NODEVICE = -5,    /* no gfx950 device at that index */
    MRML_HIP_E_FORMAT = -6,      /* malformed or unsupported GGUF file */
    MRML_HIP_E_IO = -7,          /* a file could not be opened or read */
    MRML_HIP_E_NOTFOUND = -8     /* no GGUF tensor or metadata key of that name */
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
/* Waits for the context's stream.  Also fails with MRML_HIP_E_HIP when a
 * kernel's bounded wait for other waves of its workgroup gave up since the
 * last sync on the device (its results are then wrong). */
int         mrml_hip_sync(mrml_hip_ctx *ctx);
/* Poll limit of those bounded waits on the context's device (every context
 * on it): polls < 0 restores the default (2^20), 0 makes every wait give up
 * at once.  No reference counterpart: it lets a test drive the error path of
 * mrml_hip_sync with every kernel still exiting normally. */
int         mrml_hip_set_wait_limit(mrml_hip_ctx *ctx, int32_t polls);
int         mrml_hip_device_info_get(mrml_hip_ctx *ctx, mrml_hip_device_info *info);
int         mrml_hip_memory_info(mrml_hip_ctx *ctx, uint64_t *free_bytes, uint64_t *total_bytes);
/* The context's hipStream_t, for callers that record events on it. */
void       *mrml_hip_stream(mrml_hip_ctx *ctx);
/* Grow the internal scratch (activation packs, partial results) to at least
 * `bytes` now, so later ops never allocate (e.g. under stream capture). */
int         mrml_hip_reserve_workspace(mrml_hip_ctx *ctx, size_t bytes);
/* Current size of that scratch in bytes.  No reference counterpart: it lets a
 * caller check that a sequence of ops (a captured prefill, say) grew nothing. */
int         mrml_hip_workspace_bytes(mrml_hip_ctx *ctx, size_t *bytes);

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
/* Streaming read of `bytes` (16-byte aligned) with the weight streams'
 * non-temporal loads, writing nothing but (rarely) a word of the 1 KiB
 * d_sink.  No reference counterpart: the read-only floor that a matvec
 * streaming the same bytes in one launch cannot beat. */
int mrml_hip_read_kernel(mrml_hip_ctx *ctx, const void *d_src, size_t bytes, void *d_sink);

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
/* GGUF Q4_K (144 B / 256) -> quant plane [rows][cols/32][16 B], one run per
 * 32-weight sub-block in Q4_0 nibble order (byte i: weight i low, weight
 * i+16 high), + header plane [rows][cols/256][16 B] = {f16 d, f16 dmin,
 * u8 scales[12]}. */
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
/* mrml_hip_gemv_q4_0_q8 on the tolerance path: the same integer block dots
 * and block terms, each row's f32 sum added in tree order (lane sums, then
 * a wave butterfly) instead of block order, nine rows a workgroup -- the
 * token step's output and down projections under MRML_HIP_NUMERICS_FAST.
 * Outputs within 1e-5 of the exact product relative to the largest output.
 * Block counts that are neither a multiple of 64 nor above 256, or above
 * 320, run the exact kernels.  No counterpart in the reference. */
int mrml_hip_gemv_q4_0_q8_relaxed(mrml_hip_ctx *ctx, const void *d_w, const void *d_xpack, float *d_y,
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
 * (nullable, 16-byte aligned) also receives the f32 activation.  dim = model
 * width (cols of gate/up, rows of down), ffn = hidden width.  At the
 * Gemma-2-2B shape (dim 2304, ffn 9216) the launches are the split form of
 * mrml_hip_ffn_split_geglu / _down; the result is the same bits either way. */
int mrml_hip_ffn_geglu_q4_0(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up,
                            const void *d_w_down, const float *d_x, float *d_act, float *d_y,
                            int32_t dim, int32_t ffn);
/* The split form's two launches on their own (no reference counterpart: the
 * FFN entry point above, for callers that interleave other work).  The
 * GeGLU runs one 36-row workgroup per CU: 32 rows of one activation block and
 * 4 of the tail, and writes the f32 activation (d_act, required) and the
 * Q8_0 pack entries of the blocks it holds whole (d_act_pack, ffn/32*40
 * bytes); the down projection takes both, quantising the tail blocks from
 * d_act itself.  Only the shapes of the split form (dim/32 in {64, 72}, ffn
 * = 9216 = 256 x 36) are served; others return MRML_HIP_E_INVALID.
 * d_w_down_next (nullable): the down projection the caller launches next (a
 * dim x ffn Q4_0 matrix in the backend layout: dim*ffn/32*18 bytes, read
 * only); when it runs nine rows a workgroup (dim a multiple of 2304) the GeGLU
 * reads its rows ahead into the caches while its own weights finish streaming
 * (the results do not depend on it; mrml_hip_ffn_geglu_q4_0 passes its
 * d_w_down). */
int mrml_hip_ffn_split_geglu(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up, const float *d_x,
                             float *d_act, void *d_act_pack, const void *d_w_down_next, int32_t dim, int32_t ffn);
int mrml_hip_ffn_split_down(mrml_hip_ctx *ctx, const void *d_w_down, const void *d_act_pack, const float *d_act,
                            float *d_y, int32_t dim, int32_t ffn);
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
/* As mrml_hip_gemv_q8_0 with x already quantised (an activation pack from
 * mrml_hip_quantize_q8_0): the vocabulary loop quantises its input once
 * (model.rs:2842-2853). */
int mrml_hip_gemv_q8_0_q8(mrml_hip_ctx *ctx, const void *d_w, const void *d_xpack, float *d_y,
                          int32_t rows, int32_t cols, int32_t softcap);
/* Q4_K (build-defined semantics, GGUF layout; the reference has no Q4_K dot):
 * y[r] = sum over sub-blocks j of
 *        (float)isum_j*((d*sc_j)*d_a) - (float)bsum_j*((dmin*m_j)*d_a),
 * folded in order.  d_w: backend Q4_K layout. */
int mrml_hip_gemv_q4_k(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                       int32_t rows, int32_t cols);
/* As mrml_hip_gemv_q4_k with x already quantised (activation pack). */
int mrml_hip_gemv_q4_k_q8(mrml_hip_ctx *ctx, const void *d_w, const void *d_xpack, float *d_y,
                          int32_t rows, int32_t cols);

/* ---- batched (prefill) products ------------------------------------------- */
/* CudaDevice::gemm_q4_0 (cuda.rs:2308-2332; layout of kernels.rs:343-400):
 * d_x is [batch][cols] f32, d_y is [batch][rows] f32, and
 * d_y[m][r] = dot(W[r], Q8_0(x[m])) with the CPU semantics of
 * ops::mat_vec_mul_q4_0 (ops.rs:162-180) for every token m, each output
 * bit-identical to mrml_hip_gemv_q4_0 on that token.  The integer block dots
 * run on int8 MFMA.  Any rows (the reference grid is ceil(rows / 8),
 * cuda.rs:627-673), cols % 32 == 0; W and the activations each below 2 GiB.  Uses the context workspace (batch/32 * cols/32 * 1152
 * bytes rounded up) for the activations in MFMA order. */
int mrml_hip_gemm_q4_0(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                       int32_t rows, int32_t cols, int32_t batch);
/* mrml_hip_gemm_q4_0 with the tolerance path's fold: the integer block sums
 * stay exact, each block term joins its output's sum with one FMA (one
 * rounding instead of two), so outputs are within 1e-5 of the exact
 * product relative to the largest output (the GEMM's time is its f32 fold;
 * this removes a quarter of the fold's instructions).  The prefill of a
 * MRML_HIP_NUMERICS_FAST model uses it. */
int mrml_hip_gemm_q4_0_relaxed(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                               int32_t rows, int32_t cols, int32_t batch);
/* As mrml_hip_gemm_q4_0 with the batch already quantised: d_xpack is the
 * activation pack of batch*cols values (mrml_hip_quantize_q8_0 over the
 * whole [batch][cols] array), token m's block b at index m*(cols/32)+b. */
int mrml_hip_gemm_q4_0_q8(mrml_hip_ctx *ctx, const void *d_w, const void *d_xpack, float *d_y,
                          int32_t rows, int32_t cols, int32_t batch);
/* The batch quantised once for several products over the same activations
 * (gate and up, or Q/K/V, share their input: model.rs:2452-2560): Q8_0 of
 * every token (quant.rs:193-228) written as a GEMM pack, the MFMA operand
 * order of these kernels, mrml_hip_gemm_pack_bytes(cols, batch) bytes. */
size_t mrml_hip_gemm_pack_bytes(int32_t cols, int32_t batch);
int mrml_hip_quantize_q8_0_gemm(mrml_hip_ctx *ctx, const float *d_x, void *d_gpack, int32_t cols,
                                int32_t batch);
/* As mrml_hip_gemm_q4_0 over a GEMM pack; no workspace. */
int mrml_hip_gemm_q4_0_gpack(mrml_hip_ctx *ctx, const void *d_w, const void *d_gpack, float *d_y,
                             int32_t rows, int32_t cols, int32_t batch);

/* CudaDevice::gemm_q4_0_qkv (cuda.rs:2406-2436; layout of kernels.rs:402-469):
 * d_x [batch][cols] f32, d_y [batch][q_rows + 2*kv_rows] f32 = the stacked
 * q | k | v of every token, each output bit-identical to mrml_hip_gemv_q4_0
 * on that token (the CPU path of model.rs:1388-1402).  One Q8_0 GEMM pack of
 * the batch (workspace) feeds the three products.  q_rows, kv_rows, cols
 * multiples of 32. */
int mrml_hip_gemm_q4_0_qkv(mrml_hip_ctx *ctx, const void *d_wq, const void *d_wk, const void *d_wv,
                           const float *d_x, float *d_y, int32_t q_rows, int32_t kv_rows, int32_t cols,
                           int32_t batch);
/* CudaDevice::gemm_q4_0_geglu (cuda.rs:2699-2725; layout of kernels.rs:597-
 * 673): d_act [batch][rows] = gelu_tanh(g) * u with g, u the two products
 * over Q8_0(x) of every token -- per token bit-identical to
 * mrml_hip_gemv_q4_0_geglu (CPU semantics model.rs:2093-2105, the host
 * libm's tanhf).  Workspace: the GEMM pack and 2*batch*rows floats. */
int mrml_hip_gemm_q4_0_geglu(mrml_hip_ctx *ctx, const void *d_w_gate, const void *d_w_up, const float *d_x,
                             float *d_act, int32_t rows, int32_t cols, int32_t batch);

/* As mrml_hip_gemm_q4_0 (same arguments, same bit-identical outputs), but
 * it allocates nothing: no hipMalloc, no workspace growth.  No counterpart in
 * the reference; it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).
 * The GEMM pack of the activations goes to a fixed device scratch of
 * mrml_hip_gemm_q4_0_noalloc_max_pack_bytes() bytes (8 MiB: batch up to 3232
 * tokens at cols 2304, 800 at cols 9216), one per GPU for the life of the
 * process; shapes whose pack, mrml_hip_gemm_pack_bytes(cols, batch), is
 * larger fail with MRML_HIP_E_INVALID.  Every call on a GPU shares that
 * scratch, so calls that overlap on one GPU (several contexts or streams at
 * once) race; calls ordered on one context are safe. */
int mrml_hip_gemm_q4_0_noalloc(mrml_hip_ctx *ctx, const void *d_w, const float *d_x, float *d_y,
                               int32_t rows, int32_t cols, int32_t batch);
size_t mrml_hip_gemm_q4_0_noalloc_max_pack_bytes(void);

/* Greedy pick over n f32 scores (model.rs:2869-2888; GPU tie rule
 * kernels.rs:1144-1145): index of the maximum, lowest index on ties, NaN
 * never wins.  d_out: one int32 on the device. */
int mrml_hip_argmax_f32(mrml_hip_ctx *ctx, const float *d_x, int32_t n, int32_t *d_out);

/* Vocabulary scoring of step_generation.  Candidates: ids with
 * d_valid[id] != 0 (d_valid nullable: all), minus 1, 2, 105 and 106 while
 * generated_count < 4 (model.rs:2845-2850).  Scores:
 *   MRML_HIP_SCORE_CPU (the CPU path, model.rs:2851-2856): d_logits are raw
 *     dot products; score = 30*tanh(logit/30) (the host libm's tanhf, bit
 *     for bit), minus 3.5 once when id is among the recent ids;
 *   MRML_HIP_SCORE_DEVICE (the device path, kernels.rs:1110-1123): d_logits
 *     come softcapped from the Q8 GEMV; score = logit minus 1.8 per
 *     occurrence of id among the recent ids.
 * NaN scores are no candidates.  Ranking: score descending, equal scores by
 * ascending id (kernels.rs:1144-1145; the host sorts of the reference leave
 * that order open).  d_recent: n_recent (0..32) ids on the device. */
enum { MRML_HIP_SCORE_CPU = 0, MRML_HIP_SCORE_DEVICE = 1 };

/* CudaDevice::vocab_topk (cuda.rs:3052-3111; kernels.rs:1085-1228): device
 * scoring; partition p covers ids [vocab*p/partitions,
 * vocab*(p+1)/partitions) and gets its k best (score, id) at
 * d_scores/d_ids[p*k ..], (-inf, -1) past its candidates.  k 1..64; any
 * partition size (the reference's generic kernel) up to 2,097,152 ids. */
int mrml_hip_vocab_topk(mrml_hip_ctx *ctx, const float *d_logits, const uint8_t *d_valid, const int32_t *d_recent,
                        float *d_scores, int32_t *d_ids, int32_t vocab, int32_t n_recent, int32_t generated_count,
                        int32_t k, int32_t partitions);

/* The whole next-token pick of step_generation (model.rs:2842-2907) on the
 * device: the k best candidates over the vocabulary, then temperature <= 0:
 * the best; else p_i = expf((s_i - s_0) / max(temperature, 0.1)) summed in
 * rank order and the first i with rng <= (acc += p_i / sum), rng =
 * (f32)((pos * 6364136223846793005 + 1) >> 33) / (f32)UINT32_MAX with pos the
 * reference's state.pos (the position after the token whose logits these
 * are); no candidate: token 506.  d_token (one int32), d_scores / d_ids (k
 * entries, -inf / -1 past the candidates) are nullable.  k 1..64 (the
 * reference draws from 40), vocab up to 2,097,152.  Bit-identical to the
 * reference CPU path's choice given its scores. */
int mrml_hip_vocab_select(mrml_hip_ctx *ctx, const float *d_logits, int32_t vocab, const uint8_t *d_valid,
                          const int32_t *d_recent, int32_t n_recent, int32_t generated_count, int32_t scoring,
                          float temperature, uint64_t pos, int32_t k, int32_t *d_token, float *d_scores,
                          int32_t *d_ids);

/* ---- the rest of the token step ---------------------------------------------
 * Every op keeps the CPU path's operation order: sums the reference evaluates
 * sequentially in f32 (RMSNorm's sum of squares, the attention dots, softmax
 * denominator and weighted sum of values) give the same bits here, and expf /
 * tanhf / the RoPE table reproduce the host C library's results, so these
 * outputs are bit-identical to the CPU path too.  Where an op takes both
 * `pos` and `d_pos`, a non-null d_pos (one int32 on the device) is read when
 * the op executes, so a captured graph serves every position. */

/* CudaDevice::rms_norm (cuda.rs:2102-2180; CPU ops.rs:24-79):
 * out = (x * (1/sqrt(sum(x^2)/dim + eps))) * w.  d_w nullable (no weight).
 * d_out (f32) and d_pack (the Q8_0 activation pack of the result, for the
 * next matvec) are each nullable, not both.  dim % 32 == 0, dim <= 12288. */
int mrml_hip_rms_norm(mrml_hip_ctx *ctx, const float *d_x, const float *d_w, float *d_out, void *d_pack,
                      int32_t dim, float eps);
/* CudaDevice::rms_norm_batch (cuda.rs:2102-2180): rms_norm of each of
 * `batch` consecutive vectors of dim values, d_x and d_out [batch][dim], d_w
 * nullable; each row bit-identical to mrml_hip_rms_norm. */
int mrml_hip_rms_norm_batch(mrml_hip_ctx *ctx, const float *d_x, const float *d_w, float *d_out, int32_t dim,
                            int32_t batch, float eps);
/* Gemma-2 sandwich-norm residual, then the next block's pre-norm (the
 * per-layer order of model.rs:1185-2260):
 *   h += rms_norm(t, w_post);  xn = rms_norm(h, w_next) -> d_xn, d_pack (nullable). */
int mrml_hip_residual_rms_norm(mrml_hip_ctx *ctx, const float *d_t, const float *d_w_post, float *d_h,
                               const float *d_w_next, float *d_xn, void *d_pack, int32_t dim, float eps);
/* CudaDevice::embedding_q8_0 (cuda.rs:2625-2656; CPU model.rs:1164-1182):
 * out[i] = (q_i * d) * scale for row `token` of a backend-layout Q4_0 or Q8_0
 * table (type MRML_HIP_Q4_0 / MRML_HIP_Q8_0).  d_token overrides token. */
int mrml_hip_embedding(mrml_hip_ctx *ctx, const void *d_table, int32_t type, int32_t token,
                       const int32_t *d_token, float *d_out, int32_t dim, int32_t vocab, float scale);
/* RoPE angle table for positions 0..n_pos-1: d_table[(pos*head_dim/2 + i)*2]
 * = cosf(theta), +1 = sinf(theta), theta = pos*freq_scale /
 * powf(freq_base, 2i/head_dim) (ops.rs:185-208), computed on the host with
 * the C library the reference calls, so table-driven RoPE is bit-exact.
 * Synchronous (uploads n_pos*head_dim floats); call before graph capture. */
int mrml_hip_rope_table(mrml_hip_ctx *ctx, float *d_table, int32_t n_pos, int32_t head_dim, float freq_base,
                        float freq_scale);
/* CudaDevice::qkv_postprocess (cuda.rs:2438-2476) without the Gemma-4 head
 * norms: NeoX RoPE (ops.rs:185-208; theta = pos*freq_scale /
 * freq_base^(2i/head_dim)) on the q and k heads of d_qkv = [q | k | v] in
 * place, then k and v stored as f16 (round to nearest even) at cache row
 * pos % capacity of [capacity][n_kv_heads][head_dim] caches.  cos/sin come
 * from d_table (nullable; from mrml_hip_rope_table) for pos < n_table, else
 * are evaluated on the device: powf in double precision rounded once, then
 * cosf and sinf in the host C library's algorithm (glibc's, bit for bit), so
 * the rotation has the CPU path's bits unless the host's powf rounds a pair's
 * frequency the other way (none at base 10000). */
int mrml_hip_rope_kv_append_f16(mrml_hip_ctx *ctx, float *d_qkv, uint16_t *d_k_cache, uint16_t *d_v_cache,
                                int32_t pos, const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads,
                                int32_t head_dim, float freq_base, float freq_scale, int32_t capacity,
                                const float *d_table, int32_t n_table);
/* CudaDevice::qkv_postprocess_batch (cuda.rs:2478-2519, the kernel at
 * kernels.rs:1231-1330; called by prefill_cuda, model.rs:2485-2501) without
 * the Gemma-4 head norms: `batch` stacked [q | k | v] rows of d_qkv, row i
 * rotated at position start_pos + i as mrml_hip_rope_kv_append_f16 rotates
 * one row, its k and v stored at cache row (cache_start + i) % capacity in
 * the caches' formats (KvCacheFormat::cuda_code, kv_cache.rs:16-31): 0 f16
 * (round to nearest even), 1 Q8_0 or 2 Q4_0 blocks of 32 along each head
 * (quantize_f32_to_q8_0 / _q4_0, quant.rs:193-228, 372-389, as
 * KvCacheRow::from_f32 stores them; head_dim % 32 == 0), rows of
 * n_kv_heads*head_dim/32 blocks of 34 or 18 bytes.  batch <= capacity (rows
 * of one call never share a cache row).  freq_scale 1 is the reference's
 * (the batched kernel has none). */
int mrml_hip_rope_kv_append_f16_batch(mrml_hip_ctx *ctx, float *d_qkv, uint16_t *d_k_cache, uint16_t *d_v_cache,
                                      int32_t start_pos, int32_t cache_start, int32_t batch, int32_t n_heads,
                                      int32_t n_kv_heads, int32_t head_dim, float freq_base, float freq_scale,
                                      int32_t capacity, int32_t k_format, int32_t v_format, const float *d_table,
                                      int32_t n_table);
/* CudaDevice::rope_256k (cuda.rs:2248-2285): rope_1d_batched (ops.rs:185-208)
 * of n_heads contiguous heads of head_dim floats in d_vec, in place, at
 * position pos; cos/sin from d_table (nullable) for pos < n_table, else
 * evaluated on the device as mrml_hip_rope_kv_append_f16 does (any position:
 * the large-argument reduction matches the host's too).  head_dim
 * even, at most 1024. */
int mrml_hip_rope(mrml_hip_ctx *ctx, float *d_vec, int32_t pos, int32_t head_dim, int32_t n_heads, float freq_base,
                  float freq_scale, const float *d_table, int32_t n_table);
/* CudaDevice::geglu (cuda.rs:2215-2246): d_out[i] = gelu_tanh(d_gate[i]) *
 * d_up[i] for i < n (ops.rs:99-114), bit-identical to the CPU path. */
int mrml_hip_geglu(mrml_hip_ctx *ctx, const float *d_gate, const float *d_up, float *d_out, int32_t n);
/* CudaDevice::swiglu (cuda.rs:2182-2213): d_out[i] = silu(d_gate[i]) *
 * d_up[i], silu(x) = x / (1 + expf(-x)) (ops.rs:116-130), expf the host C
 * library's, bit-identical to the CPU path. */
int mrml_hip_swiglu(mrml_hip_ctx *ctx, const float *d_gate, const float *d_up, float *d_out, int32_t n);
/* CudaDevice::add (cuda.rs:2579-2593): d_out[i] = d_a[i] + d_b[i] for i < n
 * (one IEEE f32 add each; d_out may alias an input). */
int mrml_hip_add(mrml_hip_ctx *ctx, const float *d_a, const float *d_b, float *d_out, int32_t n);
/* CudaDevice::attention_causal (cuda.rs:2658-2697; CPU model.rs:1457-1590)
 * for one token: out[h] = softmax(scale * q[h] . K[t]) . V[t] over the last
 * min(n_past+1, capacity) cache rows, kv head h / (n_heads / n_kv_heads),
 * in the CPU path's operation order (sequential dots, softmax sum and
 * weighted sum; the host C library's expf).  head_dim a multiple of 32 up
 * to 512, groups of at most 16, capacity at most 2^20: past 6144 the
 * window's exps are summed in LDS-staged chunks, each chunk's exact
 * sequential sum continuing the running sum (the same bits; the reference
 * streams such windows through its online-softmax kernel,
 * kernels.rs:1463-1561).  d_out (f32) and d_pack (Q8_0 pack of the
 * n_heads*head_dim output) nullable, not both. */
int mrml_hip_attn_decode_f16(mrml_hip_ctx *ctx, const float *d_q, const uint16_t *d_k_cache,
                             const uint16_t *d_v_cache, float *d_out, void *d_pack, int32_t n_past,
                             const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                             float scale, int32_t capacity);

/* The same attention split over tiles of 32 positions of the window (flash
 * decoding: per tile and head the max, the exp sum and the weighted values
 * in f32 tree order, then a merge in tile order): the FAST numerics of the
 * token step (MRML_HIP_NUMERICS_FAST).  Within 1e-5 of the CPU path relative
 * to the output's largest magnitude, not bit-identical.  Same arguments and
 * limits as mrml_hip_attn_decode_f16 (attention_causal, cuda.rs:2658-2697);
 * shapes other than head_dim 256 with groups up to 8 run the exact form. */
int mrml_hip_attn_decode_f16_split(mrml_hip_ctx *ctx, const float *d_q, const uint16_t *d_k_cache,
                                   const uint16_t *d_v_cache, float *d_out, void *d_pack, int32_t n_past,
                                   const int32_t *d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                   float scale, int32_t capacity);

/* CudaDevice::attention_causal with the reference's own argument list
 * (cuda.rs:2658-2697; the window rule of kernels.rs:1398-1404): q holds
 * n_heads*head_dim floats, the caches capacity rows (row = position %
 * capacity), n_past the query's position; sliding_window > 0 limits the
 * window to the last sliding_window positions (<= 0: no limit beyond the
 * capacity).  The arithmetic of mrml_hip_attn_decode_f16, bit-identical to
 * the CPU path over the same rows.  k_format / v_format: the cache formats
 * of KvCacheFormat::cuda_code (kv_cache.rs:16-22): 0 f16 rows, 1 Q8_0 and
 * 2 Q4_0 blocks (rows as mrml_hip_rope_kv_append_f16_batch stores them);
 * scores are then KvCacheRow::dot_head -- the block-ordered Q8_0 x Q8_0 or
 * Q4_0 x Q8_0 fold against quantize_f32_to_q8_0(q_h) -- times scale, and the
 * values add (f16(d) * p) * q per value (add_head_scaled,
 * kv_cache.rs:73-125).  Other codes return MRML_HIP_E_UNSUPPORTED.  Limits
 * as mrml_hip_attn_decode_f16. */
int mrml_hip_attention_causal(mrml_hip_ctx *ctx, const float *d_q, const uint16_t *d_k_cache,
                              const uint16_t *d_v_cache, float *d_out, int32_t n_past, int32_t n_heads,
                              int32_t n_kv_heads, int32_t head_dim, float scale, int32_t sliding_window,
                              int32_t capacity, int32_t k_format, int32_t v_format);
/* The same on the tolerance path (mrml_hip_attn_decode_f16_split's split-K
 * arithmetic, within 1e-5 of the CPU path). */
int mrml_hip_attention_causal_split(mrml_hip_ctx *ctx, const float *d_q, const uint16_t *d_k_cache,
                                    const uint16_t *d_v_cache, float *d_out, int32_t n_past, int32_t n_heads,
                                    int32_t n_kv_heads, int32_t head_dim, float scale, int32_t sliding_window,
                                    int32_t capacity, int32_t k_format, int32_t v_format);

/* CudaDevice::attention_prefill (cuda.rs:2727-2770; called by prefill_cuda,
 * model.rs:2503-2522): `batch` queries at positions cache_start + i over
 * caches that already hold every row's K/V; query row i starts i * q_stride
 * floats into d_q (the reference's q.len() / batch, >= n_heads*head_dim),
 * output row i (n_heads*head_dim floats) at d_out + i*n_heads*head_dim.  Row
 * i is bit-identical to mrml_hip_attention_causal at n_past = cache_start + i
 * with the same sliding window, capacity and formats. */
int mrml_hip_attention_prefill(mrml_hip_ctx *ctx, const float *d_q, int32_t q_stride, const uint16_t *d_k_cache,
                               const uint16_t *d_v_cache, float *d_out, int32_t cache_start, int32_t batch,
                               int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                               int32_t sliding_window, int32_t capacity, int32_t k_format, int32_t v_format);

/* ---- Gemma-2-shape token step (model.rs forward_token, model.rs:1185-2260,
 * and greedy selection, model.rs:2833-2907) ----------------------------------- */
/* Numerics of the token step.  EXACT (0, the default): every op in the CPU
 * path's operation order, logits bit-identical to the reference CPU step.
 * FAST: the residual RMSNorm sums are deterministic tree sums, decode
 * attention is split over tiles of the window (flash decoding) with
 * tree-order softmax and value sums, and the output and down projections
 * add each row in tree order (mrml_hip_gemv_q4_0_q8_relaxed); the other
 * matvecs stay bit-exact given their inputs.  Each changed op is within
 * 1e-5 of the CPU path relative to its
 * output's largest magnitude, and greedy tokens are checked against the
 * reference CPU step (north_star: <= 1e-5 max-rel, identical greedy tokens). */
enum { MRML_HIP_NUMERICS_EXACT = 0, MRML_HIP_NUMERICS_FAST = 1 };

typedef struct mrml_hip_gemma2_config {
    int32_t n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, ctx_len;
    float   rope_base, eps, attn_scale;
    int32_t tie_type; /* MRML_HIP_Q4_0 or MRML_HIP_Q8_0: tied embedding / LM-head table */
    int32_t numerics; /* MRML_HIP_NUMERICS_EXACT (0) or MRML_HIP_NUMERICS_FAST */
    /* Per-layer attention windows (model.rs:590, 1465-1467): with
     * sliding_window > 0 and swa_period > 0, layer l attends the last
     * sliding_window positions unless l % swa_period == swa_period - 1 (a
     * global layer, the whole cache).  Gemma-2: 4096 and 2 (local layers
     * 0, 2, ...); the reference's 5 local : 1 global pattern: period 6.
     * 0 and 0: every layer global. */
    int32_t sliding_window, swa_period;
} mrml_hip_gemma2_config;

/* Device pointers of one layer: matrices in the backend Q4_0 layout, norm
 * weights f32[dim]. */
typedef struct mrml_hip_gemma2_layer {
    const void  *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    const float *attn_norm, *post_attn_norm, *ffn_norm, *post_ffw_norm;
} mrml_hip_gemma2_layer;

typedef struct mrml_hip_gemma2 mrml_hip_gemma2;

/* Bind weights (not copied; they must outlive the model) and allocate the
 * step's activation buffers. */
int mrml_hip_gemma2_create(mrml_hip_ctx *ctx, const mrml_hip_gemma2_config *cfg, const void *d_tok_embd,
                           const float *d_output_norm, const mrml_hip_gemma2_layer *layers,
                           mrml_hip_gemma2 **out);
int mrml_hip_gemma2_destroy(mrml_hip_ctx *ctx, mrml_hip_gemma2 *model);
/* Enqueue one token step.  d_state = {token, pos} (two int32 on the device)
 * is read when the step executes; its last kernel records the pick (the
 * greedy argmax with lowest index on ties, or the sampler's choice, see
 * mrml_hip_gemma2_set_sampler) in d_argmax (nullable) and in d_hist[pos]
 * (nullable, pos < hist_cap), then advances the state: pos += 1 and token =
 * d_prompt[pos] while pos < prompt_len (prefill), else the pick.  Caches
 * are [n_layers][ctx_len][n_kv_heads][head_dim] f16.  d_logits (nullable)
 * receives the vocab logits.  A graph captured around one call replays for
 * every token. */
int mrml_hip_gemma2_step(mrml_hip_ctx *ctx, mrml_hip_gemma2 *model, int32_t *d_state, uint16_t *d_k_cache,
                         uint16_t *d_v_cache, float *d_logits, int32_t *d_argmax, int32_t *d_hist,
                         int32_t hist_cap, const int32_t *d_prompt, int32_t prompt_len);
/* Prefill (prefill_cuda, model.rs:2395-2638): the token steps of positions
 * pos0 .. pos0+n_tokens-1 for the tokens d_tokens[0..n_tokens) (device
 * int32), in chunks of up to 512 tokens whose seven projections per layer run
 * as batched Q4_0 products on MFMA (mrml_hip_gemm_q4_0).  Every op keeps the
 * token step's arithmetic, so the caches end bit-identical to n_tokens calls
 * of mrml_hip_gemma2_step; the last token's logits go to d_logits (nullable:
 * the model's own buffer) and its greedy argmax to d_argmax (nullable).
 * Positions may pass ctx_len: a chunk that wraps the ring appends and
 * attends token by token (its products stay batched), as the token steps
 * do.  RoPE angles come from the model's host-computed table for positions
 * below ctx_len and past it from host-computed powf values and the host C
 * library's cosf/sinf algorithm on the device, bit-exact at every position.
 * The first call
 * allocates the chunk buffers (freed by mrml_hip_gemma2_destroy) unless
 * mrml_hip_gemma2_reserve_prefill has; every later call allocates nothing
 * and records no memset, so it can be captured into a graph, which then
 * replays the same positions over the same token buffer. */
int mrml_hip_gemma2_prefill(mrml_hip_ctx *ctx, mrml_hip_gemma2 *model, const int32_t *d_tokens, int32_t n_tokens,
                            int32_t pos0, uint16_t *d_k_cache, uint16_t *d_v_cache, float *d_logits,
                            int32_t *d_argmax);
/* Allocate the prefill's chunk buffers now (synchronous; idempotent), so
 * that the next mrml_hip_gemma2_prefill can be captured.  No counterpart in
 * the reference, whose prefill_cuda takes pooled buffers per call. */
int mrml_hip_gemma2_reserve_prefill(mrml_hip_ctx *ctx, mrml_hip_gemma2 *model);
/* The pick of mrml_hip_gemma2_step and _prefill (step_generation,
 * model.rs:2713-2907): with a sampler, the CPU path's scoring
 * (MRML_HIP_SCORE_CPU of mrml_hip_vocab_select: masks, 30*tanh softcap,
 * -3.5 for the tokens of the last 32 positions) and its draw at the
 * sampler's temperature over the top_k best (greedy when temperature <= 0),
 * the generated count being pos - (prompt_len - 1) in a step and 0 after a
 * prefill; without one (NULL, the default), the plain argmax.  The model
 * keeps the tokens of the last 32 positions it processed (steps and
 * prefills both record them).  Applies to calls enqueued, or graphs
 * captured, after this call. */
typedef struct mrml_hip_sampler {
    const uint8_t *d_valid; /* nullable: every id valid; else vocab bytes on the device */
    float          temperature;
    int32_t        top_k;   /* 1..64 (the reference: 40) */
} mrml_hip_sampler;
int mrml_hip_gemma2_set_sampler(mrml_hip_ctx *ctx, mrml_hip_gemma2 *model, const mrml_hip_sampler *sampler);
/* The model's own residual stream h (f32[dim]) and logits (f32[vocab]). */
int mrml_hip_gemma2_activations(mrml_hip_ctx *ctx, mrml_hip_gemma2 *model, float **d_h, float **d_logits);

/* ---- GGUF container reader (host only; GgufFile, crates/mrml-tensor/src/
 * gguf.rs:78-184) -----------------------------------------------------------
 * Version 2 and 3 files.  Tensors and metadata keys are indexed in key-byte
 * order, a repeated name keeping its last entry (the reference's OrderedMap,
 * crates/mrml-runtime/src/map.rs:38-49).  Tensor bytes are read on demand,
 * like GgufFile::read_tensor_bytes.  Errors are MRML_HIP_E_FORMAT (the
 * reference's "Invalid GGUF magic number", "Unsupported GGUF version",
 * "Unsupported GGUF dtype ID", "Unknown GGUF value type ID", non-UTF-8
 * strings, truncation), MRML_HIP_E_IO and MRML_HIP_E_NOTFOUND; the message of
 * the calling thread's last failure is mrml_gguf_last_error(). */
typedef struct mrml_gguf mrml_gguf;

typedef struct {
    const char *name;    /* valid until mrml_gguf_close */
    int32_t type;        /* GGUF type id: 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K, 16 IQ4_XS, 30 BF16 */
    int32_t n_dims;      /* min(stored n_dims, 4) */
    uint64_t dims[4];    /* ggml order (dims[0] = elements per row); unused dims are 1 */
    uint64_t offset;     /* from the data section start */
    uint64_t size_bytes; /* numel / block size * block bytes (gguf.rs:146-147) */
} mrml_gguf_tensor_info;

/* GgufFile::open (gguf.rs:80-171): parses the header, metadata and tensor
 * directory. */
int mrml_gguf_open(const char *path, mrml_gguf **out);
int mrml_gguf_close(mrml_gguf *g);
const char *mrml_gguf_last_error(void);
/* version, data section offset (gguf.rs:153-163), tensor and key counts; each
 * output nullable. */
int mrml_gguf_header(const mrml_gguf *g, uint32_t *version, uint64_t *data_offset, int64_t *n_tensors,
                     int64_t *n_meta);
int mrml_gguf_tensor(const mrml_gguf *g, int64_t index, mrml_gguf_tensor_info *info);
/* GgufFile::tensors.get(name) */
int mrml_gguf_find_tensor(const mrml_gguf *g, const char *name, int64_t *index);
/* GgufFile::read_tensor_bytes (gguf.rs:173-183) into a host buffer of at
 * least size_bytes. */
int mrml_gguf_read_tensor(const mrml_gguf *g, int64_t index, void *h_dst, uint64_t dst_bytes);
/* Metadata key `index` in key order and its value type id (0..12). */
int mrml_gguf_meta_key(const mrml_gguf *g, int64_t index, const char **key, int32_t *type);
/* GgufValue::as_u32 / as_f32 / as_str (gguf.rs:25-53) of metadata `key`:
 * MRML_HIP_E_INVALID when the value has no such reading. */
int mrml_gguf_meta_u32(const mrml_gguf *g, const char *key, uint32_t *out);
int mrml_gguf_meta_f32(const mrml_gguf *g, const char *key, float *out);
int mrml_gguf_meta_str(const mrml_gguf *g, const char *key, const char **out, uint64_t *len);
/* GgufValue::as_array (gguf.rs:55-60): item type and length. */
int mrml_gguf_meta_array(const mrml_gguf *g, const char *key, int32_t *item_type, uint64_t *len);

#ifdef __cplusplus
}
#endif
#endif
