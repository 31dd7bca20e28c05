// gemv_q4_0.hip -- batch-1 Q4_0 x Q8_0 matrix-vector products for gfx950.
//
// Semantics (crates/mrml-tensor/src/quant.rs:335-369, ops.rs:221-260):
//   isum_b = sum_i ((qs&15)-8)*a[i] + ((qs>>4)-8)*a[i+16]       exact int32
//   y[r]   = (...((0 + isum_0*(dw_0*da_0)) + isum_1*(dw_1*da_1)) ...)
// in block order, each product and each sum rounded separately (this file is
// compiled with -ffp-contract=off), so y is bit-identical to the CPU path.
//
// Three kernel shapes, chosen by measurement on MI355X:
//
//  * 16 lanes per row ("fold16"), for rows of <= ~128 blocks (cols 2048,
//    2304): one 64-lane wave owns 4 rows; lane j takes blocks 16*it + j, one
//    16-byte load each, so the 16 lanes of a row read 256 contiguous bytes.
//    The ordered fold is a chain of 16 row_ror:1 DPP adds per iteration;
//    after step k lane k holds the running sum through block 16*it + k and
//    lane 15 ends with the row.  A staging wave copies the activation pack
//    (or quantises f32 x itself) into LDS while the compute waves' weight
//    loads are in flight.
//
//  * Relay ("relay"), for long rows (cols 9216): a workgroup of S waves owns 4
//    rows and splits the row's iterations between them, so each wave issues
//    and computes only 1/S of the row (per-wave work, not bandwidth, bounds
//    the plain layout on long rows).  Each lane loads its own activation
//    blocks straight from the pack.  The block terms go to LDS and the
//    running sums are relayed wave to wave in iteration order (S-1
//    barriers); the fold itself is plain adds in the 4 fold lanes.
//
//  * Runtime block count ("any"): the fold16 structure with nb a kernel
//    argument, for every other shape.
//
// The GeGLU kernel can also quantise x itself and emit the Q8_0 pack of its
// output for the next (down) projection, so an FFN is two launches.

#include "device.h"
#include "internal.h"
#include "norm_block.h"

namespace mrml {

namespace {

constexpr uint32_t kNib = 0x0F0F0F0Fu;

// Exact integer block dot of one Q4_0 block (16 packed bytes) with the
// matching Q8_0 activation quants (a0 = a[0..15], a1 = a[16..31]) and their sum.
__device__ __forceinline__ int32_t q4_0_isum(uint4 w, int4 a0, int4 a1, int32_t asum)
{
    int32_t s = sdot4(w.x & kNib, (uint32_t)a0.x, 0);
    s = sdot4(w.y & kNib, (uint32_t)a0.y, s);
    s = sdot4(w.z & kNib, (uint32_t)a0.z, s);
    s = sdot4(w.w & kNib, (uint32_t)a0.w, s);
    s = sdot4((w.x >> 4) & kNib, (uint32_t)a1.x, s);
    s = sdot4((w.y >> 4) & kNib, (uint32_t)a1.y, s);
    s = sdot4((w.z >> 4) & kNib, (uint32_t)a1.z, s);
    s = sdot4((w.w >> 4) & kNib, (uint32_t)a1.w, s);
    return s - 8 * asum;  // nibble offset: sum (q-8)*a = sum q*a - 8*sum a
}

// Quantise f32 x (NB blocks) into a split-nibble activation pack in LDS with
// NQ waves (this is wave qw): eight blocks per wave step, 8 lanes of 4 values
// each per block; all of a wave's loads are issued before the first block is
// quantised.
template <int NB, int NQ>
__device__ __forceinline__ void quantize_into_lds(const float *__restrict__ x, uint8_t *pack, int qw)
{
    constexpr int K = (NB + 8 * NQ - 1) / (8 * NQ);
    const int lane = threadIdx.x & 63, g = lane >> 3, l = lane & 7;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    float4 v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        int b = 8 * (qw + NQ * k) + g;
        b = b < NB ? b : NB - 1;
        v[k] = x4[b * 8 + l];
    }
    __builtin_amdgcn_s_barrier();  // x's loads are issued (stage_split_pack's ISSUE_BARRIER)
    uint32_t *pq = reinterpret_cast<uint32_t *>(pack);
    float *pd = reinterpret_cast<float *>(pack + NB * 32);
    int32_t *ps = reinterpret_cast<int32_t *>(pack + NB * 36);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int b = 8 * (qw + NQ * k) + g;
        uint32_t dbits;
        int s;
        const uint32_t q = q8_split8(q8_0_block8x4(v[k], dbits, s), l, s);
        if (b < NB) {
            pq[b * 8 + l] = q;
            if (l == 0) {
                pd[b] = f16_bits_to_f32(dbits);
                ps[b] = s;
            }
        }
    }
}

// ---- 16 lanes per row: registers, loads and the DPP fold --------------------

// Per-lane registers of one row: ITERS 16-byte quant blocks and, per block,
// the 32-bit word of the scale plane that holds its f16 scale (a 4-byte load
// keeps each scale in its own register, so no load is consumed early).
template <int ITERS>
struct RowRegs {
    uint4 w[ITERS];
    uint32_t d[ITERS];
};

// Issue every load of one row (lane j, blocks 16*it + j); blocks past the row
// end load a clamped in-bounds block and are masked out of the fold.  ODD:
// the matrix has an odd number of blocks, so the 4-byte word holding the
// last scale would reach 2 bytes past the scale plane; every scale is then
// read with a 2-byte load instead (the word's low half).
template <int ITERS, bool ODD = false>
__device__ __forceinline__ void load_row(RowRegs<ITERS> &r, const uint8_t *__restrict__ w, size_t nblk,
                                         size_t base, int nb, int j)
{
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(w + nblk * 16);
    const uint16_t *dh = reinterpret_cast<const uint16_t *>(w + nblk * 16);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int b = it * 16 + j;
        b = b < nb ? b : nb - 1;
        r.w[it] = load_stream16(qs + base + b);
        r.d[it] = ODD ? (uint32_t)dh[base + b] : dw[(base + b) >> 1];
    }
}

// Block term of iteration `it` (masked to +0 past the row end) against a
// split-nibble pack in LDS.  Computed unconditionally, so the compiler has
// no conditional block to sink the weight load into (which would delay its
// issue).
template <int ITERS, bool ODD = false>
__device__ __forceinline__ float row_term(const RowRegs<ITERS> &r, int it, const uint8_t *pack, size_t base, int nb,
                                          int j)
{
    const int b = it * 16 + j;
    const int bc = b < nb ? b : nb - 1;
    const uint4 *aq = reinterpret_cast<const uint4 *>(pack);
    const float *ad = reinterpret_cast<const float *>(pack + nb * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(pack + nb * 36);
    const uint4 w = r.w[it], lo = aq[2 * bc], hi = aq[2 * bc + 1];
    const int32_t isum = q4_0_isum_split(w.x, w.y, w.z, w.w, lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w, ac[bc]);
    const uint32_t word = r.d[it];
    const uint32_t dbits = (!ODD && ((base + bc) & 1)) ? word >> 16 : word & 0xffffu;
    const float t = (float)isum * (f16_bits_to_f32(dbits) * ad[bc]);
    return b < nb ? t : 0.0f;
}

// Ordered fold; the row result is valid in lane 15 of the DPP row.  Masked
// tail terms are +0, which leaves a running sum unchanged (the sum starts at
// +0 and round-to-nearest never turns it into -0).
template <int ITERS, bool ODD = false>
__device__ __forceinline__ float fold_row(const RowRegs<ITERS> &r, const uint8_t *pack, size_t base, int nb, int j)
{
    float s = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const float t = row_term<ITERS, ODD>(r, it, pack, base, nb, j);
#pragma unroll
        for (int k = 0; k < 16; ++k) s = fold16(s, t);
    }
    return s;
}

// Two rows (gate and up) with interleaved chains.
template <int ITERS>
__device__ __forceinline__ void fold_row2(const RowRegs<ITERS> &ra, const RowRegs<ITERS> &rb, const uint8_t *pack,
                                          size_t base, int nb, int j, float &sa, float &sb)
{
    sa = 0.0f;
    sb = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const float ta = row_term<ITERS>(ra, it, pack, base, nb, j);
        const float tb = row_term<ITERS>(rb, it, pack, base, nb, j);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            sa = fold16(sa, ta);
            sb = fold16(sb, tb);
        }
    }
}

// ---- transposed fold ----------------------------------------------------------
// The same ordered fold (s = +0, then s = s + t[b] in block order) with one
// lane per row instead of 16: the compute lanes store their block terms to
// LDS, T[chain][b] at a stride of t_stride floats, and after a barrier one
// lane per chain adds a row's terms in order -- one add instruction per
// block for up to 64 rows, where the DPP fold spends 16 per 16 blocks per 4
// rows.  A chain has a slot for every lane's block of every iteration
// (ITERS*16 >= NB; the slots past NB hold the masked +0 terms and are never
// read), so the stores are unconditional: a store under `b < NB` lets the
// compiler sink the whole term, weight load included, into the branch and
// issue the last iteration's loads only after the first terms.  The stride
// is an odd number of 16-byte segments, so the float4 reads of 64 chains
// spread over the banks.
template <int NB>
constexpr int t_stride()
{
    static_assert(NB % 4 == 0, "float4 reads of the terms");
    constexpr int n = (NB + 15) / 16 * 16;
    return (n / 4) % 2 ? n : n + 4;
}

// Two rows (gate and up): the term chains of both, computed interleaved.
template <int NB, int ITERS>
__device__ __forceinline__ void store_terms2(const RowRegs<ITERS> &ra, const RowRegs<ITERS> &rb, const uint8_t *pack,
                                             size_t base, int j, float *T, int chain_a, int chain_b)
{
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const float ta = row_term<ITERS>(ra, it, pack, base, NB, j);
        const float tb = row_term<ITERS>(rb, it, pack, base, NB, j);
        T[chain_a * t_stride<NB>() + it * 16 + j] = ta;
        T[chain_b * t_stride<NB>() + it * 16 + j] = tb;
    }
}

// store_terms2 with every pack read of the lane (its blocks j, 16 + j, ...:
// two 16-byte quant words, the scale and the constant of each) issued at
// once, before the first term: the LDS latency is paid once instead of once
// per iteration (the weights' loads set the pace after that).
template <int NB, int ITERS>
__device__ __forceinline__ void store_terms2_pre(const RowRegs<ITERS> &ra, const RowRegs<ITERS> &rb,
                                                 const uint8_t *pack, size_t base, int j, float *T, int chain_a,
                                                 int chain_b)
{
    const uint4 *aq = reinterpret_cast<const uint4 *>(pack);
    const float *ad = reinterpret_cast<const float *>(pack + NB * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(pack + NB * 36);
    uint4 lo[ITERS], hi[ITERS];
    float d[ITERS];
    int32_t c[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int b = it * 16 + j, bc = b < NB ? b : NB - 1;
        lo[it] = aq[2 * bc];
        hi[it] = aq[2 * bc + 1];
        d[it] = ad[bc];
        c[it] = ac[bc];
    }
    asm volatile("" ::: "memory");  // every pack read above is issued before the terms' stores
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int b = it * 16 + j, bc = b < NB ? b : NB - 1;
        float t[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const RowRegs<ITERS> &r = m ? rb : ra;
            const uint4 w = r.w[it];
            const int32_t isum = q4_0_isum_split(w.x, w.y, w.z, w.w, lo[it].x, lo[it].y, lo[it].z, lo[it].w,
                                                 hi[it].x, hi[it].y, hi[it].z, hi[it].w, c[it]);
            const uint32_t dbits = ((base + bc) & 1) ? r.d[it] >> 16 : r.d[it] & 0xffffu;
            const float tv = (float)isum * (f16_bits_to_f32(dbits) * d[it]);
            t[m] = b < NB ? tv : 0.0f;
        }
        T[chain_a * t_stride<NB>() + it * 16 + j] = t[0];
        T[chain_b * t_stride<NB>() + it * 16 + j] = t[1];
    }
}

// The ordered sum of chain `chain` (all NB/4 reads issued before the adds).
template <int NB>
__device__ __forceinline__ float fold_chain(const float *T, int chain)
{
    const float4 *p = reinterpret_cast<const float4 *>(T + chain * t_stride<NB>());
    float4 v[NB / 4];
#pragma unroll
    for (int k = 0; k < NB / 4; ++k) v[k] = p[k];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NB / 4; ++k) {
        s = s + v[k].x;
        s = s + v[k].y;
        s = s + v[k].z;
        s = s + v[k].w;
    }
    return s;
}

// Value of lane (lane ^ M) (M = 16 or 32: across DPP rows, so through the
// LDS crossbar; no LDS memory is touched).
template <int M>
__device__ __forceinline__ float lane_xor(float v)
{
    const int lane = threadIdx.x & 63;
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ M) << 2, __builtin_bit_cast(int, v)));
}

// Row of matrix set {wq | wk | wv} for a stacked output row.
struct QkvSel {
    const uint8_t *w;
    int local, mrows;
};
__device__ __forceinline__ QkvSel qkv_select(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, int row,
                                             int q_rows, int kv_rows)
{
    if (row < q_rows) return {wq, row, q_rows};
    if (row < q_rows + kv_rows) return {wk, row - q_rows, kv_rows};
    return {wv, row - q_rows - kv_rows, kv_rows};
}

// ---- fold16 kernels, block count NB fixed at compile time --------------------
// NQ leading waves prepare the activation pack in LDS: QX = false copies a
// pack, QX = true quantises f32 x; the WAVES compute waves own 4 rows each.

constexpr int kNQ = 4;  // staging waves when quantising x in the kernel

template <int NB, bool QX>
__device__ __forceinline__ void prepare_pack(const void *xin, uint8_t *lds, int wave)
{
    static_assert(NB <= kStageMax, "one staging batch");
    if constexpr (QX) quantize_into_lds<NB, kNQ>(reinterpret_cast<const float *>(xin), lds, wave);
    else stage_split_pack<true>(reinterpret_cast<const uint8_t *>(xin), lds, NB);
}

template <bool QX>
constexpr int stage_waves() { return QX ? kNQ : 1; }

template <int NB, int WAVES, bool QX>
__global__ __launch_bounds__(64 * (WAVES + (QX ? kNQ : 1))) void gemv_q4_0_kernel(
    const uint8_t *__restrict__ w, const void *xin, float *__restrict__ y, int rows)
{
    constexpr int NS = stage_waves<QX>(), ITERS = (NB + 15) / 16;
    extern __shared__ __align__(16) uint8_t lds[];
    const int wave = threadIdx.x >> 6;
    if (wave < NS) {
        prepare_pack<NB, QX>(xin, lds, wave);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int row_raw = (blockIdx.x * WAVES + wave - NS) * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const size_t base = (size_t)row * NB;
    RowRegs<ITERS> r;
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
    load_row<ITERS>(r, w, (size_t)rows * NB, base, NB, j);
    __syncthreads();
    const float s = fold_row<ITERS>(r, lds, base, NB, j);
    if (j == 15 && row_raw < rows) y[row_raw] = s;
}

template <int NB, int WAVES, bool QX>
__global__ __launch_bounds__(64 * (WAVES + (QX ? kNQ : 1))) void gemv_q4_0_qkv_kernel(
    const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wk, const uint8_t *__restrict__ wv, const void *xin,
    float *__restrict__ y, int q_rows, int kv_rows)
{
    constexpr int NS = stage_waves<QX>(), ITERS = (NB + 15) / 16;
    extern __shared__ __align__(16) uint8_t lds[];
    const int wave = threadIdx.x >> 6;
    if (wave < NS) {
        prepare_pack<NB, QX>(xin, lds, wave);
        __syncthreads();
        return;
    }
    const int total = q_rows + 2 * kv_rows;
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int row_raw = (blockIdx.x * WAVES + wave - NS) * 4 + (lane >> 4);
    const QkvSel m = qkv_select(wq, wk, wv, row_raw < total ? row_raw : total - 1, q_rows, kv_rows);
    const size_t base = (size_t)m.local * NB;
    RowRegs<ITERS> r;
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
    load_row<ITERS>(r, m.w, (size_t)m.mrows * NB, base, NB, j);
    __syncthreads();
    const float s = fold_row<ITERS>(r, lds, base, NB, j);
    if (j == 15 && row_raw < total) y[row_raw] = s;
}

// Gate+up with the GeGLU epilogue (model.rs:2093-2105, ops.rs:99-114).  The
// R = 4*WAVES rows of a workgroup are folded by its first compute wave, one
// lane per chain (gate rows in lanes [0,R), up rows in [R,2R)).  With EMIT,
// a workgroup owns 32 rows (WAVES = 8) and that wave also writes the Q8_0
// pack of its 32 outputs (one activation block) for the next projection;
// act may then be null.
template <int NB, int WAVES, bool QX, bool EMIT>
__global__ __launch_bounds__(64 * (WAVES + (QX ? kNQ : 1))) void gemv_q4_0_geglu_kernel(
    const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu, const void *xin, float *__restrict__ act,
    uint8_t *__restrict__ act_pack, int rows)
{
    static_assert(!EMIT || WAVES == 8, "the output pack block needs 32 rows per workgroup");
    static_assert(WAVES == 4 || WAVES == 8, "gate/up lanes pair across 16 or 32 lanes");
    constexpr int NS = stage_waves<QX>(), ITERS = (NB + 15) / 16, R = 4 * WAVES;
    extern __shared__ __align__(16) uint8_t lds[];
    float *T = reinterpret_cast<float *>(lds + (NB * 40 + 15) / 16 * 16);
    const int wave = threadIdx.x >> 6;
    if (wave < NS) {
        prepare_pack<NB, QX>(xin, lds, wave);
        __syncthreads();  // the pack is whole
        __syncthreads();  // every term is stored
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int rl = (wave - NS) * 4 + (lane >> 4);
    const int row_raw = blockIdx.x * R + rl;
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    RowRegs<ITERS> rg, ru;
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
    load_row<ITERS>(rg, wg, nblk, base, NB, j);
    load_row<ITERS>(ru, wu, nblk, base, NB, j);
    __syncthreads();
    store_terms2<NB, ITERS>(rg, ru, lds, base, j, T, rl, R + rl);
    __syncthreads();
    if (wave != NS) return;
    const float s = fold_chain<NB>(T, lane < 2 * R ? lane : 0);
    const float p = lane_xor<R>(s);
    const bool up = (lane & R) != 0;
    const float a = gelu_tanh(up ? p : s) * (up ? s : p);  // row (lane mod R)'s output, in both lanes of the pair
    const int out = blockIdx.x * R + (lane & (R - 1));
    if (act && lane < R && out < rows) act[out] = a;
    if constexpr (EMIT) {
        uint32_t dbits;
        int qs;
        const int q = q8_0_block32(a, dbits, qs);
        const int blk = blockIdx.x, nbo = rows / 32;
        if (lane < 32) {
            act_pack[(size_t)blk * 32 + lane] = (uint8_t)(int8_t)q;
            if (lane == 0) {
                reinterpret_cast<float *>(act_pack + (size_t)nbo * 32)[blk] = f16_bits_to_f32(dbits);
                reinterpret_cast<int32_t *>(act_pack + (size_t)nbo * 36)[blk] = qs;
            }
        }
    }
}

// LDS of the GeGLU kernel: the pack, then 2R term chains.
template <int NB>
constexpr size_t geglu_lds(int waves)
{
    return (NB * 40 + 15) / 16 * 16 + (size_t)2 * 4 * waves * t_stride<NB>() * sizeof(float);
}

// Two chains of one lane (gate and up of a row), added in block order,
// interleaved.
template <int NB>
__device__ __forceinline__ void fold_chain2(const float *T, int ca, int cb, float &sa, float &sb)
{
    const float4 *pa = reinterpret_cast<const float4 *>(T + ca * t_stride<NB>());
    const float4 *pb = reinterpret_cast<const float4 *>(T + cb * t_stride<NB>());
    float4 va[NB / 4], vb[NB / 4];
#pragma unroll
    for (int k = 0; k < NB / 4; ++k) {
        va[k] = pa[k];
        vb[k] = pb[k];
    }
    sa = 0.0f;
    sb = 0.0f;
#pragma unroll
    for (int k = 0; k < NB / 4; ++k) {
        sa = sa + va[k].x;
        sb = sb + vb[k].x;
        sa = sa + va[k].y;
        sb = sb + vb[k].y;
        sa = sa + va[k].z;
        sb = sb + vb[k].z;
        sa = sa + va[k].w;
        sb = sb + vb[k].w;
    }
}

// Gate+up GeGLU with f32 output, rows spread evenly over the CUs: W compute
// waves own R = 4W rows (W = 9: 36 rows, 256 workgroups for 9216 rows, one
// per CU; 32-row workgroups would put two on 32 CUs, which then finish about
// 2 us after the rest).  x is quantised in the kernel (kNQ staging waves);
// lane r < R of the first compute wave adds both chains of row r.  Used
// where act is wanted in f32 only: an FFN emits the Q8_0 pack from 32-row
// workgroups instead, since forming the pack inside each down-projection
// workgroup (576 of them) costs far more than the imbalance.
template <int NB, int W>
__global__ __launch_bounds__(64 * (W + kNQ)) void gemv_q4_0_geglu_f32_kernel(
    const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu, const float *__restrict__ x,
    float *__restrict__ act, int rows)
{
    constexpr int NS = kNQ, ITERS = (NB + 15) / 16, R = 4 * W;
    static_assert(R <= 64, "one fold lane per row");
    extern __shared__ __align__(16) uint8_t lds[];
    float *T = reinterpret_cast<float *>(lds + (NB * 40 + 15) / 16 * 16);
    const int wave = threadIdx.x >> 6;
    if (wave < NS) {
        quantize_into_lds<NB, kNQ>(x, lds, wave);
        __syncthreads();  // the pack is whole
        __syncthreads();  // every term is stored
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int rl = (wave - NS) * 4 + (lane >> 4);
    const int row_raw = blockIdx.x * R + rl;
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    RowRegs<ITERS> rg, ru;
    __builtin_amdgcn_s_barrier();  // x's loads are issued
    load_row<ITERS>(rg, wg, nblk, base, NB, j);
    load_row<ITERS>(ru, wu, nblk, base, NB, j);
    __syncthreads();
    store_terms2<NB, ITERS>(rg, ru, lds, base, j, T, rl, R + rl);
    __syncthreads();
    if (wave != NS) return;
    float g, u;
    fold_chain2<NB>(T, lane < R ? lane : 0, lane < R ? R + lane : R, g, u);
    const int out = blockIdx.x * R + lane;
    if (lane < R && out < rows) act[out] = gelu_tanh(g) * u;
}

template <int NB, int W>
constexpr size_t geglu_f32_lds() { return (NB * 40 + 15) / 16 * 16 + (size_t)2 * 4 * W * t_stride<NB>() * sizeof(float); }

// The balanced GeGLU that still emits most of the Q8_0 activation pack: R =
// 4W = 32 + E rows per workgroup, G workgroups, rows = G*R with G*E a
// multiple of 32.  Workgroup w owns the whole 32-row block w (rows 32w..) and
// E rows of the tail, 32G + E*w .. + E-1, so each workgroup has the same
// bytes (one per CU at the Gemma-2-2B FFN: 256 x 36 rows) and the block's
// pack entry (quant.rs:193-228 over its 32 outputs) is formed inside it.  The
// G*E/32 tail blocks straddle workgroups; their pack entries are left
// unwritten, and the consumer quantises them from the f32 outputs (act,
// always written).  x is quantised by kNQ staging waves and the fold runs
// after all terms are stored (a fold pipelined with the stream through
// per-iteration counters, and x quantised by the compute waves themselves,
// each measured slower: 8.5 and 8.7 against 7.9 us).
// The compute waves of the split GeGLU (waves NS.. of the workgroup): issue
// the rows' weight loads after the staging waves' barrier, run hook (the
// compute waves' share of staging the pack, with the barriers it takes),
// fold against the pack in lds, and emit act and the pack block blockIdx.x.
// The staging waves take the same barriers (one s_barrier after their loads
// are issued, hook's, then three __syncthreads) and leave.
struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

// The next product's rows, read ahead into the caches by the split GeGLU's
// staging waves while its own weights finish streaming: the down projection
// that follows runs nine rows a workgroup, workgroup w rows 9w .. 9w+8, on the
// XCD of the GeGLU's workgroup w (workgroups go to XCDs by index), so
// workgroup w reads those rows' quants and scales (46.6 KB at the Gemma-2
// shape) and the down projection then finds them in its L2 instead of
// waiting out an HBM round trip for its whole stream: the HBM is otherwise
// idle during the GeGLU's tail (the fold, GELU and block quantisation) and
// the launch gap.  Loads are issued after the pack barrier, behind the
// compute waves' weight loads, and held in registers until the waves leave
// (nothing is stored; the registers keep the loads from being dropped).
// rows_next / gridDim.x rows a workgroup; a region above 12 loads a
// staging thread is read only in part.  Nothing is read when w_next is null.
// (The decode step's residual-norm GeGLU does not read ahead: there the pack
// is whole only after the norm's exact sums, so the loads went out late and
// held the kernel's end: 847 -> 821 tok/s.)
struct PrefetchRegs {
    static constexpr int kQ = 12, kS = 2;  // 16-byte loads per staging thread (4 staging waves)
    uint4 q[kQ], s[kS];
};

__device__ __forceinline__ void prefetch_rows(PrefetchRegs &r, const uint8_t *w_next, int rows_next, int nb_next)
{
    if (!w_next) return;
    const int per = rows_next / (int)gridDim.x, t = threadIdx.x;  // staging threads 0 .. 64*kNQ-1
    const size_t qn = (size_t)per * nb_next * 16, q0 = (size_t)blockIdx.x * qn;
    const size_t sn = (size_t)per * nb_next * 2, s0 = (size_t)rows_next * nb_next * 16 + (size_t)blockIdx.x * sn;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w_next + q0), *ss = reinterpret_cast<const uint4 *>(w_next + s0);
#pragma unroll
    for (int k = 0; k < PrefetchRegs::kQ; ++k) {
        const size_t i = (size_t)t + 64 * kNQ * k;
        r.q[k] = qs[i * 16 < qn ? i : 0];
    }
#pragma unroll
    for (int k = 0; k < PrefetchRegs::kS; ++k) {
        const size_t i = (size_t)t + 64 * kNQ * k;
        r.s[k] = ss[i * 16 + 16 <= sn ? i : 0];
    }
}

// Keeps the read-ahead loads live until the wave leaves.
__device__ __forceinline__ void prefetch_hold(const PrefetchRegs &r, const uint8_t *w_next)
{
    if (!w_next) return;
#pragma unroll
    for (int k = 0; k < PrefetchRegs::kQ; ++k) asm volatile("" ::"v"(r.q[k].x));
#pragma unroll
    for (int k = 0; k < PrefetchRegs::kS; ++k) asm volatile("" ::"v"(r.s[k].x));
}

template <int NB, int W, int NS, class Hook = NoHook>
__device__ __forceinline__ void geglu_split_compute(const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu,
                                                    float *__restrict__ act, uint8_t *__restrict__ act_pack, int rows,
                                                    uint8_t *lds, float *T, int wave, Hook hook = Hook())
{
    constexpr int ITERS = (NB + 15) / 16, R = 4 * W, E = R - 32;
    static_assert(R <= 64 && E > 0, "one fold lane per row, a tail share per workgroup");
    const int G = gridDim.x;
    auto row_of = [&](int rl) { return rl < 32 ? 32 * (int)blockIdx.x + rl : 32 * G + E * (int)blockIdx.x + rl - 32; };
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int rl = (wave - NS) * 4 + (lane >> 4);
    const int row = row_of(rl);
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    RowRegs<ITERS> rg, ru;
    __builtin_amdgcn_s_barrier();  // the staging waves' loads are issued
    load_row<ITERS>(rg, wg, nblk, base, NB, j);
    load_row<ITERS>(ru, wu, nblk, base, NB, j);
    hook();  // work of the waves that also take part in staging the pack
    __syncthreads();
    store_terms2_pre<NB, ITERS>(rg, ru, lds, base, j, T, rl, R + rl);
    __syncthreads();
    // the gate chains and GELU in one wave, the up chains in the next (two
    // dependent chains of 72 adds in one wave ran one after the other)
    float *ushare = reinterpret_cast<float *>(lds);  // the pack is no longer read
    if (wave != NS) {
        if (wave == NS + 1) ushare[lane] = fold_chain<NB>(T, lane < R ? R + lane : R);
        __syncthreads();  // the up sums are shared (every wave takes part)
        return;
    }
    const float gg = gelu_tanh(fold_chain<NB>(T, lane < R ? lane : 0));
    __syncthreads();
    const float a = gg * ushare[lane];
    if (lane < R) act[row_of(lane)] = a;
    uint32_t dbits;
    int qs;
    const int q = q8_0_block32(a, dbits, qs);  // lanes 0..31: block blockIdx.x
    const int blk = blockIdx.x, nbo = rows / 32;
    if (lane < 32) {
        act_pack[(size_t)blk * 32 + lane] = (uint8_t)(int8_t)q;
        if (lane == 0) {
            reinterpret_cast<float *>(act_pack + (size_t)nbo * 32)[blk] = f16_bits_to_f32(dbits);
            reinterpret_cast<int32_t *>(act_pack + (size_t)nbo * 36)[blk] = qs;
        }
    }
}

template <int NB, int W>
__global__ __launch_bounds__(64 * (W + kNQ)) void gemv_q4_0_geglu_split_kernel(
    const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu, const float *__restrict__ x,
    float *__restrict__ act, uint8_t *__restrict__ act_pack, int rows, const uint8_t *w_next, int rows_next,
    int nb_next)
{
    extern __shared__ __align__(16) uint8_t lds[];
    float *T = reinterpret_cast<float *>(lds + (NB * 40 + 15) / 16 * 16);
    const int wave = threadIdx.x >> 6;
    if (wave < kNQ) {
        quantize_into_lds<NB, kNQ>(x, lds, wave);  // takes the first barrier
        __syncthreads();  // the pack is whole
        PrefetchRegs pf;
        prefetch_rows(pf, w_next, rows_next, nb_next);
        __syncthreads();  // every term is stored
        __syncthreads();  // the up sums are shared
        prefetch_hold(pf, w_next);
        return;
    }
    geglu_split_compute<NB, W, kNQ>(wg, wu, act, act_pack, rows, lds, T, wave);
}

// ---- the Gemma-2 sandwich residual ahead of the rows ---------------------------
// Each workgroup first forms h_out = h_in + rms_norm(t, w_post) and
// the Q8_0 pack of rms_norm(h_out, w_norm) in its own LDS (norm_block.h;
// the same bits in every workgroup, workgroup 0 stores h_out), then its
// compute waves fold 4 rows each against that pack.  The compute waves issue their
// weight loads once the norm's operands have arrived, so the norm's exact
// sums run while the weights stream in (its barriers wait on LDS only).  h_out must not alias h_in: other workgroups still read h_in.
// dim = NB*32 <= 4*576 (one float4 chunk per thread).
constexpr int kResWaves = 9;
// Row waves of the fused q|k|v: 16 rows a workgroup, so the 4096 rows of the
// Gemma-2 shape fill 256 workgroups (one per CU) instead of 128 of 32 rows;
// every workgroup forms the norm, the waves past CW only for that.  Measured
// in the token step: 771 -> 780 tok/s (EXACT), 1032 -> 1049 (FAST).
constexpr int kQkvResRowWaves = 4;

template <int NB>
__device__ __forceinline__ uint8_t *resnorm_pack_lds(uint8_t *lds) { return lds; }
template <int NB>
__device__ __forceinline__ mrml_xsum::Shared4 *resnorm_shared(uint8_t *lds)
{
    return reinterpret_cast<mrml_xsum::Shared4 *>(lds + (NB * 40 + 15) / 16 * 16 + 64 * sizeof(float));
}

// Gate+up with the GeGLU epilogue and the output's Q8_0 pack, the
// post-attention residual fused ahead: 16 waves own 64 rows (two output
// blocks), 144 workgroups for 9216 rows, so every workgroup is resident at
// once.
constexpr int kGegluResWaves = 16;

// ---- the residual norm in a group of waves, the weight stream beside it --------
// In the fused residual + GeGLU the two norms run in the first kNormWaves
// waves only (exact_sum.h's group form, synchronised by an LDS counter)
// while the other waves issue their weight loads at once: a wave issuing
// loads into a full memory pipeline stalls, and with workgroup barriers
// inside the norm every stall held the norm back.  The norm waves
// issue their own rows' loads once the pack is written; everyone meets at one
// workgroup barrier before the terms.  Norm lane l of wave w holds the KN
// consecutive values k = KN*(64w + l) + i.
constexpr int kNormWaves = 4;

template <int NB, int NW = kNormWaves>
constexpr int norm_kn() { return (NB * 32 + 64 * NW - 1) / (64 * NW); }

// LDS: pack | GroupShared | sync counter | xn (dim floats) + events (dim + pad),
// the term chains reusing that last area once the pack is whole.
template <int NB>
constexpr size_t rn2_group_off() { return (NB * 40 + 15) / 16 * 16; }
template <int NB>
constexpr size_t rn2_area_off() { return rn2_group_off<NB>() + (sizeof(mrml_xsum::GroupShared) + 16 + 15) / 16 * 16; }
template <int NB>
constexpr size_t rn2_area_bytes(int chains)
{
    const size_t norm = (size_t)(NB * 32 + mrml_xsum::group_events(NB * 32)) * sizeof(float);
    const size_t terms = (size_t)chains * t_stride<NB>() * sizeof(float);
    return norm > terms ? norm : terms;
}

// The group's operands: lane values k = KN*(64w + l) + i of t, h_in, w_post,
// w_norm.  Loaded unconditionally (a missing weight reads t and is replaced
// by 1 in the norm) so that all of them are issued at once, before the
// workgroup barrier that lets the other waves issue their weight loads.
template <int NB, int NW = kNormWaves>
struct GroupNormOps {
    float t[norm_kn<NB, NW>()], h[norm_kn<NB, NW>()], p[norm_kn<NB, NW>()], n[norm_kn<NB, NW>()];
};

template <int NB, int NW = kNormWaves>
__device__ __forceinline__ void group_norm_load(GroupNormOps<NB, NW> &o, const float *__restrict__ t,
                                                const float *__restrict__ w_post, const float *h_in,
                                                const float *__restrict__ w_norm, int wave)
{
    constexpr int DIM = NB * 32, KN = norm_kn<NB, NW>();
    const int k0 = KN * (64 * wave + (threadIdx.x & 63));
    const float *pp = w_post ? w_post : t, *pn = w_norm ? w_norm : t;
#pragma unroll
    for (int i = 0; i < KN; ++i) {
        const int k = k0 + i < DIM ? k0 + i : DIM - 1;
        o.t[i] = t[k];
        o.h[i] = h_in[k];
        o.p[i] = pp[k];
        o.n[i] = pn[k];
    }
}

// The residual norm of the group: h_out = h_in + rms_norm(t, w_post) (stored
// when h_out is set), rms_norm(h_out, w_norm) to area[0, dim) and (EMIT) its
// split pack at pack.  Called by the NW group waves only (group wave index
// `wave`).  Without EMIT the caller publishes area with a workgroup barrier
// and emits the pack itself.
// FAST (the decode step's tolerance path): both sums are deterministic tree
// sums (exact_sum.h's group_tree_sum) instead of the sequential-order ones.
template <int NB, bool FAST = false, int NW = kNormWaves, bool EMIT = true>
__device__ __forceinline__ void group_residual_norm(GroupNormOps<NB, NW> &o, bool has_post, bool has_norm,
                                                    float *h_out, float eps, uint8_t *pack, uint8_t *lds_group,
                                                    float *area, int wave, int polls)
{
    static_assert(NW <= 8, "group tree sums hold 8 wave totals per slot");
    constexpr int DIM = NB * 32, KN = norm_kn<NB, NW>(), N4 = DIM / 4;
    const int lane = threadIdx.x & 63, k0 = KN * (64 * wave + lane);
    auto *gs = reinterpret_cast<mrml_xsum::GroupShared *>(lds_group);
    mrml_xsum::GroupSync sync{reinterpret_cast<uint32_t *>(lds_group + sizeof(mrml_xsum::GroupShared)), 0u,
                              (uint32_t)NW, polls};
    float sq[KN];
#pragma unroll
    for (int i = 0; i < KN; ++i) sq[i] = o.t[i] * o.t[i];
    float *xn = area, *evl = area + DIM;
    auto sum_sq = [&](int slot) {
        if constexpr (FAST) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < KN; ++i) a += k0 + i < DIM ? sq[i] : 0.0f;
            return mrml_xsum::group_tree_sum(a, wave, sync, *gs, slot);
        } else {
            return mrml_xsum::group_seq_sum_nonneg<KN>(sq, DIM, wave, sync, *gs, evl);
        }
    };
    const float s1 = rms_scale(sum_sq(0), DIM, eps);
#pragma unroll
    for (int i = 0; i < KN; ++i) {
        float tn = o.t[i] * s1;
        if (has_post) tn = tn * o.p[i];
        o.h[i] = o.h[i] + tn;
        if (h_out && k0 + i < DIM) h_out[k0 + i] = o.h[i];
        sq[i] = o.h[i] * o.h[i];
    }
    const float s2 = rms_scale(sum_sq(1), DIM, eps);
#pragma unroll
    for (int i = 0; i < KN; ++i) {
        float v = o.h[i] * s2;
        if (has_norm) v = v * o.n[i];
        if (k0 + i < DIM) xn[k0 + i] = v;
    }
    if constexpr (EMIT) {
        sync();
        // Q8_0 blocks: 8 consecutive lanes per block, chunk c = 64w + l + 64*NW*m
        const float4 *x4 = reinterpret_cast<const float4 *>(xn);
#pragma unroll
        for (int m = 0; m < (N4 + 64 * NW - 1) / (64 * NW); ++m) {
            const int c = 64 * wave + lane + 64 * NW * m;
            emit_q8<true>(x4[c < N4 ? c : N4 - 1], c, N4, pack, NB);
        }
    }
}

template <int NB, bool FAST>
__global__ __launch_bounds__(64 * kGegluResWaves) void gemv_q4_0_geglu_resnorm_kernel(
    const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu, const float *__restrict__ t,
    const float *__restrict__ w_post, const float *h_in, float *h_out, const float *__restrict__ w_norm, float eps,
    uint8_t *__restrict__ act_pack, int rows)
{
    constexpr int ITERS = (NB + 15) / 16;
    static_assert(2 * 64 <= 128, "chains");
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *lds_group = lds + rn2_group_off<NB>();
    float *area = reinterpret_cast<float *>(lds + rn2_area_off<NB>());
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15;
    // the norm's operands are issued first, so they do not queue behind the
    // weights; the barrier also publishes the zeroed sync counter
    const int polls = mrml_xsum::wait_polls();
    GroupNormOps<NB> ops;
    if (wave < kNormWaves) group_norm_load<NB>(ops, t, w_post, h_in, w_norm, wave);
    if (threadIdx.x == 0) *reinterpret_cast<uint32_t *>(lds_group + sizeof(mrml_xsum::GroupShared)) = 0u;
    __syncthreads();
    const int rl = wave * 4 + (lane >> 4);
    const int row = blockIdx.x * 64 + rl;  // rows % 64 == 0
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    RowRegs<ITERS> rg, ru;
    if (wave >= kNormWaves) {
        load_row<ITERS>(rg, wg, nblk, base, NB, j);
        load_row<ITERS>(ru, wu, nblk, base, NB, j);
    } else {
        group_residual_norm<NB, FAST>(ops, w_post != nullptr, w_norm != nullptr, blockIdx.x == 0 ? h_out : nullptr,
                                      eps, lds, lds_group, area, wave, polls);
        load_row<ITERS>(rg, wg, nblk, base, NB, j);
        load_row<ITERS>(ru, wu, nblk, base, NB, j);
    }
    __syncthreads();  // the pack is whole; the norm's area is free
    float *T = area;
    store_terms2<NB, ITERS>(rg, ru, lds, base, j, T, rl, 64 + rl);
    __syncthreads();  // every term is stored
    if (wave < 2) {
        const float s = fold_chain<NB>(T, (lane >> 5) * 64 + 32 * wave + (lane & 31));
        const float p = lane_xor<32>(s);
        const bool up = lane >= 32;
        const float a = gelu_tanh(up ? p : s) * (up ? s : p);
        uint32_t dbits;
        int qs;
        const int q = q8_0_block32(a, dbits, qs);
        const int blk = 2 * blockIdx.x + wave, nbo = rows / 32;
        if (lane < 32 && blk < nbo) {
            act_pack[(size_t)blk * 32 + lane] = (uint8_t)(int8_t)q;
            if (lane == 0) {
                reinterpret_cast<float *>(act_pack + (size_t)nbo * 32)[blk] = f16_bits_to_f32(dbits);
                reinterpret_cast<int32_t *>(act_pack + (size_t)nbo * 36)[blk] = qs;
            }
        }
    }
}

template <int NB>
constexpr size_t geglu_resnorm_lds() { return rn2_area_off<NB>() + rn2_area_bytes<NB>(128); }

// The split GeGLU with the post-attention residual ahead (the decode step's
// FFN): h_out = h_in + rms_norm(t, w_post) and the split pack of
// rms_norm(h_out, w_norm) (group_residual_norm: the same bits in every
// workgroup, workgroup 0 stores h_out) form while the weights stream; the
// rows, the fold and the emitted pack blocks are gemv_q4_0_geglu_split_kernel's.
// The norm's two sums run in the kResSplitNW = kNQ staging waves (a group of
// 8 with four compute waves measured slower: a compute wave first issues its
// weight loads into the full memory pipeline, and the group's syncs wait for
// it); every wave of the first NB*8/64 then quantises one 4-value chunk of
// the normalised vector (three chunks per lane in the group alone took
// 1.8 us, one chunk in nine waves 0.5 us).
// LDS: the rn2 layout, its last area holding the normalised vector and the
// events, then the terms.
constexpr int kResSplitNW = kNQ;
static_assert(kNQ == kNormWaves, "the staging waves lead the group");
template <int NB, int W, bool FAST>
__global__ __launch_bounds__(64 * (W + kNQ)) void gemv_q4_0_geglu_resnorm_split_kernel(
    const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu, const float *__restrict__ t,
    const float *__restrict__ w_post, const float *h_in, float *h_out, const float *__restrict__ w_norm, float eps,
    float *__restrict__ act, uint8_t *__restrict__ act_pack, int rows)
{
    constexpr int NW = kResSplitNW, N4 = NB * 8;
    static_assert(NW <= kNQ + W && N4 % 64 == 0 && N4 <= 64 * (W + kNQ), "group waves; whole waves of chunks");
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *lds_group = lds + rn2_group_off<NB>();
    float *area = reinterpret_cast<float *>(lds + rn2_area_off<NB>());
    const int wave = threadIdx.x >> 6;
    const bool in_group = wave < NW;
    const int polls = mrml_xsum::wait_polls();
    GroupNormOps<NB, NW> ops;
    if (in_group) group_norm_load<NB, NW>(ops, t, w_post, h_in, w_norm, wave);
    if (threadIdx.x == 0) *reinterpret_cast<uint32_t *>(lds_group + sizeof(mrml_xsum::GroupShared)) = 0u;
    // the norm's operand loads are issued and the sync counter is zero
    // before any weight load (the compute part's first barrier is this one)
    auto norm_and_emit = [&]() {
        if (in_group)
            group_residual_norm<NB, FAST, NW, false>(ops, w_post != nullptr, w_norm != nullptr,
                                                     blockIdx.x == 0 ? h_out : nullptr, eps, lds, lds_group, area,
                                                     wave, polls);
        __syncthreads();  // the normalised vector is in area
        if (wave < N4 / 64) emit_q8<true>(reinterpret_cast<const float4 *>(area)[threadIdx.x], threadIdx.x, N4, lds, NB);
    };
    if (wave < kNQ) {
        mrml_xsum::lds_barrier();
        norm_and_emit();
        __syncthreads();  // the pack is whole
        __syncthreads();  // every term is stored
        __syncthreads();  // the up sums are shared
        return;
    }
    geglu_split_compute<NB, W, kNQ>(wg, wu, act, act_pack, rows, lds, area, wave, norm_and_emit);
}

template <int NB, int W>
constexpr size_t geglu_resnorm_split_lds() { return rn2_area_off<NB>() + rn2_area_bytes<NB>(8 * W); }


// The stacked q|k|v matvec, the post-FFN residual of the previous block and
// this block's pre-attention norm fused ahead: all kResWaves waves form the
// norm (one float4 of it per thread), waves 1..CW then own 4 rows each.
template <int NB, bool FAST, int CW>
__global__ __launch_bounds__(64 * kResWaves) void gemv_q4_0_qkv_resnorm_kernel(
    const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wk, const uint8_t *__restrict__ wv,
    const float *__restrict__ t, const float *__restrict__ w_post, const float *h_in, float *h_out,
    const float *__restrict__ w_norm, float eps, float *__restrict__ y, int q_rows, int kv_rows)
{
    static_assert(NB * 8 <= 64 * kResWaves, "one float4 chunk per thread");
    static_assert(CW >= 1 && CW < kResWaves, "row waves after the first");
    constexpr int ITERS = (NB + 15) / 16;
    extern __shared__ __align__(16) uint8_t lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15;
    const ResidualOps ops = residual_load(t, w_post, h_in, w_norm, NB * 8);
    wait_vm_loads();  // the norm then waits on no weight load
    const int total = q_rows + 2 * kv_rows;
    const bool rows_wave = wave > 0 && wave <= CW;
    const int row_raw = (blockIdx.x * CW + wave - 1) * 4 + (lane >> 4);
    const QkvSel m = qkv_select(wq, wk, wv, row_raw < 0 ? 0 : (row_raw < total ? row_raw : total - 1), q_rows, kv_rows);
    const size_t base = (size_t)m.local * NB;
    RowRegs<ITERS> r;
    if (rows_wave) load_row<ITERS>(r, m.w, (size_t)m.mrows * NB, base, NB, j);
    residual_norm1<true, FAST>(ops, w_post != nullptr, w_norm != nullptr, eps, blockIdx.x == 0 ? h_out : nullptr,
                               nullptr, resnorm_pack_lds<NB>(lds), NB * 32, *resnorm_shared<NB>(lds));
    mrml_xsum::lds_barrier();  // the pack is whole
    if (rows_wave) {
        const float s = fold_row<ITERS>(r, lds, base, NB, j);
        if (j == 15 && row_raw >= 0 && row_raw < total) y[row_raw] = s;
    }
}

// ---- relay kernel for long rows ------------------------------------------------
// S waves, 4 rows (16 lanes per row).  Wave s owns iterations
// [s*IPW, s*IPW + IPW); each lane loads its weight block, scale word and
// activation block (quants, scale, sum) straight from global memory, all
// issued before any is used.  Terms go to T[s][m][k][lane]; then, in wave
// order, wave s continues the running sums of wave s-1 over its own terms
// (lane r < 4 folds row r) and hands them on through LDS.

template <int NB, int S, int NMAT>
__global__ __launch_bounds__(64 * S) void gemv_q4_0_relay_kernel(const uint8_t *__restrict__ w0,
                                                                 const uint8_t *__restrict__ w1,
                                                                 const uint8_t *__restrict__ xpack,
                                                                 float *__restrict__ y, int rows)
{
    constexpr int ITERS = (NB + 15) / 16, IPW = (ITERS + S - 1) / S;
    __shared__ __align__(16) float T[S][NMAT][IPW][64];
    __shared__ float slot[NMAT][4];
    const int lane = threadIdx.x & 63, j = lane & 15, ws = threadIdx.x >> 6;
    const int row_raw = blockIdx.x * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    const int4 *aq = reinterpret_cast<const int4 *>(xpack);
    const float *ad = reinterpret_cast<const float *>(xpack + NB * 32);
    const int32_t *as = reinterpret_cast<const int32_t *>(xpack + NB * 36);

    int4 a0[IPW], a1[IPW];
    float da[IPW];
    int32_t sa[IPW];
    uint4 wr[NMAT][IPW];
    uint32_t dr[NMAT][IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        int it = ws * IPW + k;
        it = it < ITERS ? it : ITERS - 1;
        int b = it * 16 + j;
        b = b < NB ? b : NB - 1;
        a0[k] = aq[2 * b];
        a1[k] = aq[2 * b + 1];
        da[k] = ad[b];
        sa[k] = as[b];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint8_t *w = m ? w1 : w0;
            wr[m][k] = load_stream16(reinterpret_cast<const uint4 *>(w) + base + b);
            dr[m][k] = reinterpret_cast<const uint32_t *>(w + nblk * 16)[(base + b) >> 1];
        }
    }
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        const int it = ws * IPW + k;
        const int b = it * 16 + j;
        const int bc = b < NB ? b : NB - 1;
        const bool live = it < ITERS && b < NB;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const int32_t isum = q4_0_isum(wr[m][k], a0[k], a1[k], sa[k]);
            const uint32_t dbits = ((base + bc) & 1) ? dr[m][k] >> 16 : dr[m][k] & 0xffffu;
            const float t = (float)isum * (f16_bits_to_f32(dbits) * da[k]);
            T[ws][m][k][lane] = live ? t : 0.0f;
        }
    }
    float acc[NMAT];
    const int fr = lane & 3;
#pragma unroll
    for (int r = 0; r < S; ++r) {
        if (ws == r) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                float s = r == 0 ? 0.0f : slot[m][fr];
#pragma unroll
                for (int k = 0; k < IPW; ++k) {
                    const float4 *v = reinterpret_cast<const float4 *>(&T[ws][m][k][fr * 16]);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 x = v[q];
                        s = s + x.x;
                        s = s + x.y;
                        s = s + x.z;
                        s = s + x.w;
                    }
                }
                acc[m] = s;
            }
            if (r < S - 1 && lane < 4) {
#pragma unroll
                for (int m = 0; m < NMAT; ++m) slot[m][lane] = acc[m];
            }
        }
        if (r < S - 1) __syncthreads();
    }
    if (ws == S - 1 && lane < 4) {
        const int out = blockIdx.x * 4 + lane;
        if (out < rows) y[out] = NMAT == 1 ? acc[0] : gelu_tanh(acc[0]) * acc[NMAT - 1];
    }
}

// ---- long rows: the row split over waves, the ordered fold pipelined ----------
// 4 rows per workgroup.  Wave 0 stages the activation pack into LDS in split
// form, then folds; compute wave s owns iterations it = s, s+S, s+2S, ... of
// all 4 rows (16 lanes per row, lane j: block 16*it + j) and loads only
// weights.  Its loads go out iteration-major across the waves, so the data,
// and the terms, arrive roughly in block order.  Each wave stores the terms
// of its round-k iteration to T[it][row][j] and then counts it in cnt[k];
// wave 0's lanes r < 4 add row r's terms of a round, in block order, once all
// of the round's waves have counted, so only the last round's adds remain
// once the stream ends.  The waits are bounded (exact_sum.h's bounded_wait).
template <int NB, int S>
constexpr int long_ipw() { return (NB / 16 + S - 1) / S; }

template <int NB, int S>
constexpr size_t long_t_off() { return ((size_t)NB * 40 + 64 * sizeof(uint32_t) + 15) / 16 * 16; }

template <int NB, int S>
constexpr size_t long_lds() { return long_t_off<NB, S>() + (size_t)S * long_ipw<NB, S>() * 64 * sizeof(float); }

// A fold lane's ordered sum of its row's terms, round by round: round k is
// iterations S*k .. S*k+S-1 (4 float4 of terms each, at tv[it*16 ..]), ready
// once q * (its live waves) have counted it in flag[k].  Round k's reads are
// issued before round k-1's adds, so a lane that has fallen behind the stream
// pays no LDS round trip per round.
template <int NB, int S>
__device__ __forceinline__ float long_fold(const float4 *tv, const uint32_t *flag, uint32_t q, int polls)
{
    constexpr int ITERS = NB / 16, IPW = long_ipw<NB, S>();
    float4 v[2][4 * S];
    float acc = 0.0f;
    auto want = [&](int k) { return q * (uint32_t)(ITERS - S * k < S ? ITERS - S * k : S); };  // live waves
    auto rd = [&](int k) {
#pragma unroll
        for (int i = 0; i < 4 * S; ++i) v[k & 1][i] = tv[(S * k + (i >> 2)) * 16 + (i & 3)];
    };
    auto add = [&](int k) {
#pragma unroll
        for (int i = 0; i < 4 * S; ++i) {
            if (S * k + (i >> 2) < ITERS) {  // uniform
                acc = acc + v[k & 1][i].x;
                acc = acc + v[k & 1][i].y;
                acc = acc + v[k & 1][i].z;
                acc = acc + v[k & 1][i].w;
            }
        }
    };
    mrml_xsum::bounded_wait(&flag[0], want(0), polls);
    asm volatile("" ::: "memory");
    rd(0);
#pragma unroll
    for (int k = 1; k < IPW; ++k) {
        mrml_xsum::bounded_wait(&flag[k], want(k), polls);
        asm volatile("" ::: "memory");
        rd(k);
        __builtin_amdgcn_sched_barrier(0);  // round k's reads issued before round k-1's adds
        add(k - 1);
        asm volatile("" : "+v"(acc) : : "memory");  // and those adds done before the next wait
    }
    add(IPW - 1);
    return acc;
}

template <int NB, int S>
__global__ __launch_bounds__(64 * (S + 1)) void gemv_q4_0_long_kernel(const uint8_t *__restrict__ w,
                                                                    const uint8_t *xpack, float *__restrict__ y,
                                                                    int rows)
{
    constexpr int ITERS = NB / 16, IPW = long_ipw<NB, S>();
    static_assert(NB % 16 == 0 && NB <= kStageMax, "whole iterations; one staging batch");
    static_assert(IPW <= 64, "one count per round");
    extern __shared__ __align__(16) uint8_t lds[];
    uint32_t *flag = reinterpret_cast<uint32_t *>(lds + NB * 40);  // cnt[k] of the text
    float *T = reinterpret_cast<float *>(lds + long_t_off<NB, S>());
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave == 0) {
        const int polls = mrml_xsum::wait_polls();  // before the pack's loads
        flag[lane] = 0u;  // zero before the issue barrier inside the staging
        stage_split_pack<true>(xpack, lds, NB);
        __syncthreads();  // the pack is whole
        if (lane >= 4) return;
        const float acc = long_fold<NB, S>(reinterpret_cast<const float4 *>(T) + lane * 4, flag, 1u, polls);
        const int out = blockIdx.x * 4 + lane;
        if (out < rows) y[out] = acc;
        return;
    }
    __builtin_amdgcn_s_barrier();  // the pack's loads and the zeroed flags are in
    const int sw = wave - 1, j = lane & 15, rsub = lane >> 4;
    const int row_raw = blockIdx.x * 4 + rsub;
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(w + nblk * 16);
    uint4 wq[IPW];
    uint32_t wd[IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        int it = sw + S * k;
        it = it < ITERS ? it : ITERS - 1;
        const int b = it * 16 + j;
        wq[k] = load_stream16(qs + base + b);
        wd[k] = dw[(base + b) >> 1];
    }
    __syncthreads();
    const uint4 *aq = reinterpret_cast<const uint4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + NB * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(lds + NB * 36);
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        const int it = sw + S * k;
        const int b = (it < ITERS ? it : ITERS - 1) * 16 + j;
        const uint4 q = wq[k], lo = aq[2 * b], hi = aq[2 * b + 1];
        const int32_t isum = q4_0_isum_split(q.x, q.y, q.z, q.w, lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w, ac[b]);
        const uint32_t dbits = ((base + b) & 1) ? wd[k] >> 16 : wd[k] & 0xffffu;
        // every store unconditional (padding iterations of the last waves
        // included), so no weight load is sunk into a branch
        T[((sw + S * k) * 4 + rsub) * 16 + j] = (float)isum * (f16_bits_to_f32(dbits) * ad[b]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the terms are in LDS before the count
        if (lane == 0 && it < ITERS)
            __hip_atomic_fetch_add(&flag[k], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// The long-row kernel over a pack whose blocks [nmain, NB) are missing (the
// split GeGLU's tail blocks): wave 0 stages blocks [0, nmain) from the pack
// and then folds, as in gemv_q4_0_long_kernel; the tail blocks are quantised
// from the f32 activations x (quant.rs:193-228) by wave 1 and the S compute
// waves, one step of 8 blocks each (a quantiser step is a long dependent
// chain, so one wave doing all of them sat on the critical path: +1.25 us).
// Every wave issues its x loads before the workgroup's issue barrier and the
// compute waves their weight loads right after it, so the quantisation runs
// while the weights stream in.  Requires NB - nmain <= 8 * (S + 1).
template <int NB, int S>
__device__ __forceinline__ void mix_tail_load(const float *__restrict__ x, float4 &v, int nmain, int step)
{
    const int lane = threadIdx.x & 63, g = lane >> 3, l = lane & 7;
    int b = nmain + 8 * step + g;
    b = b < NB ? b : NB - 1;
    v = reinterpret_cast<const float4 *>(x)[b * 8 + l];
}

template <int NB, int S>
__device__ __forceinline__ void mix_tail_quantize(const float4 &v, uint8_t *lds, int nmain, int step)
{
    const int lane = threadIdx.x & 63, g = lane >> 3, l = lane & 7;
    const int b = nmain + 8 * step + g;
    uint32_t dbits;
    int sum;
    const uint32_t q = q8_split8(q8_0_block8x4(v, dbits, sum), l, sum);  // every lane takes part
    if (b < NB) {
        reinterpret_cast<uint32_t *>(lds)[b * 8 + l] = q;
        if (l == 0) {
            reinterpret_cast<float *>(lds + NB * 32)[b] = f16_bits_to_f32(dbits);
            reinterpret_cast<int32_t *>(lds + NB * 36)[b] = sum;
        }
    }
}

// Q row quads a workgroup (4Q row slots, the first rpw of them real rows
// blockIdx.x*rpw ..; the other slots repeat the last real row, their loads
// L2 hits, their sums never stored): Q = 1, rpw = 4 is the plain layout;
// Q = 3, rpw = 9 puts the 2304 rows of the Gemma-2 down projection on
// exactly 256 workgroups, one per CU (576 workgroups of 4 rows left 64 CUs
// a third workgroup: rows 2048 take 5.04 us, 2304 take 5.84).  Quad q's S
// compute waves write its terms to their own slice of T; the round counters
// count every quad's waves; fold lane s folds slot s.
template <int NB, int S, int Q>
constexpr size_t long_mix_lds() { return long_t_off<NB, S>() + (size_t)Q * S * long_ipw<NB, S>() * 64 * sizeof(float); }

template <int NB, int S, int Q>
__global__ __launch_bounds__(64 * (Q * S + 2)) void gemv_q4_0_long_mix_kernel(const uint8_t *__restrict__ w,
                                                                            const uint8_t *xpack,
                                                                            const float *__restrict__ x,
                                                                            float *__restrict__ y, int rows,
                                                                            int nmain, int rpw)
{
    constexpr int ITERS = NB / 16, IPW = long_ipw<NB, S>(), QT = S * IPW * 64;  // floats of T per quad
    static_assert(NB % 16 == 0 && NB <= kStageMax, "whole iterations; one staging batch");
    static_assert(IPW <= 64 && 4 * Q <= 64, "one count per round; one fold lane per slot");
    extern __shared__ __align__(16) uint8_t lds[];
    uint32_t *flag = reinterpret_cast<uint32_t *>(lds + NB * 40);
    float *T = reinterpret_cast<float *>(lds + long_t_off<NB, S>());
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (int)blockIdx.x * rpw;
    auto row_of = [&](int slot) {  // slots past rpw repeat the last real row; rows past the matrix its last
        const int r = row0 + (slot < rpw ? slot : rpw - 1);
        return r < rows ? r : rows - 1;
    };
    if (wave == 1) {
        float4 v;
        mix_tail_load<NB, S>(x, v, nmain, 0);
        __builtin_amdgcn_s_barrier();  // the loads are issued
        mix_tail_quantize<NB, S>(v, lds, nmain, 0);
        __syncthreads();  // the pack is whole
        return;
    }
    if (wave == 0) {
        const int polls = mrml_xsum::wait_polls();
        flag[lane] = 0u;  // zero before the issue barrier inside the staging
        stage_split_pack<true>(xpack, lds, NB, nmain);
        __syncthreads();  // the pack is whole
        if (lane >= 4 * Q) return;
        const float4 *tv = reinterpret_cast<const float4 *>(T + (lane >> 2) * QT) + (lane & 3) * 4;
        const float acc = long_fold<NB, S>(tv, flag, (uint32_t)Q, polls);  // every quad's waves count
        const int out = row0 + lane;
        if (lane < rpw && out < rows) y[out] = acc;
        return;
    }
    const int cw = wave - 2, qd = cw / S, sw = cw - qd * S, j = lane & 15, rsub = lane >> 4;
    float4 xv;
    if (qd == 0) mix_tail_load<NB, S>(x, xv, nmain, sw + 1);  // before the weights: an L2 hit behind HBM misses waits
    __builtin_amdgcn_s_barrier();  // the pack's loads and the zeroed flags are in
    const int row = row_of(4 * qd + rsub);
    const size_t nblk = (size_t)rows * NB, base = (size_t)row * NB;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(w + nblk * 16);
    uint4 wq[IPW];
    uint32_t wd[IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        int it = sw + S * k;
        it = it < ITERS ? it : ITERS - 1;
        const int b = it * 16 + j;
        wq[k] = load_stream16(qs + base + b);
        wd[k] = dw[(base + b) >> 1];
    }
    if (qd == 0) mix_tail_quantize<NB, S>(xv, lds, nmain, sw + 1);
    __syncthreads();
    const uint4 *aq = reinterpret_cast<const uint4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + NB * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(lds + NB * 36);
    float *Tq = T + qd * QT;
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        const int it = sw + S * k;
        const int b = (it < ITERS ? it : ITERS - 1) * 16 + j;
        const uint4 q = wq[k], lo = aq[2 * b], hi = aq[2 * b + 1];
        const int32_t isum = q4_0_isum_split(q.x, q.y, q.z, q.w, lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w, ac[b]);
        const uint32_t dbits = ((base + b) & 1) ? wd[k] >> 16 : wd[k] & 0xffffu;
        Tq[((sw + S * k) * 4 + rsub) * 16 + j] = (float)isum * (f16_bits_to_f32(dbits) * ad[b]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the terms are in LDS before the count
        if (lane == 0 && it < ITERS)
            __hip_atomic_fetch_add(&flag[k], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// ---- relaxed rows: the tolerance path's matvec -----------------------------------
// kRelaxR rows per workgroup, one wave per row (lane l: blocks l, l+64, ...),
// wave 0 staging the pack.  Every integer block dot and every block term is
// the exact kernels' own; each lane adds its terms and the wave adds the
// lanes' sums in a butterfly, so only the order of the f32 additions differs
// from the block-ordered fold (outputs within a few ulps of it; the tests
// bound them at 1e-5 relative to the largest output).  Nine rows a
// workgroup put the 2304 rows of Gemma-2's output and down projections on
// exactly 256 workgroups, one per CU, where the exact long-row kernel needs
// 576 small ones to hide its ordered fold.  ODD: the scale plane holds an
// odd number of f16 scales and is read with 2-byte loads.
constexpr int kRelaxR = 9;

template <int K, bool ODD>
__global__ __launch_bounds__(64 * (kRelaxR + 1)) void gemv_q4_0_relaxed_kernel(const uint8_t *__restrict__ w,
                                                                               const uint8_t *xpack,
                                                                               float *__restrict__ y, int rows, int nb)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave == 0) {
        stage_split_pack<true>(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int row_raw = blockIdx.x * kRelaxR + wave - 1;
    const int row = row_raw < rows ? row_raw : rows - 1;  // tail rows recompute the last row
    const size_t nblk = (size_t)rows * nb, base = (size_t)row * nb;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(w + nblk * 16);
    const uint16_t *dh = reinterpret_cast<const uint16_t *>(w + nblk * 16);
    uint4 wq[K];
    uint32_t wd[K];
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
#pragma unroll
    for (int k = 0; k < K; ++k) {
        int b = 64 * k + lane;
        b = b < nb ? b : nb - 1;
        wq[k] = load_stream16(qs + base + b);
        wd[k] = ODD ? (uint32_t)dh[base + b] : dw[(base + b) >> 1];
    }
    __syncthreads();
    const uint4 *aq = reinterpret_cast<const uint4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(lds + nb * 36);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int bt = 64 * k + lane, b = bt < nb ? bt : nb - 1;
        const uint4 q = wq[k], lo = aq[2 * b], hi = aq[2 * b + 1];
        const int32_t isum = q4_0_isum_split(q.x, q.y, q.z, q.w, lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w, ac[b]);
        const uint32_t dbits = (!ODD && ((base + b) & 1)) ? wd[k] >> 16 : wd[k] & 0xffffu;
        const float tv = (float)isum * (f16_bits_to_f32(dbits) * ad[b]);
        s += bt < nb ? tv : 0.0f;
    }
    s = mrml_xsum::wave_sum_f32(s);
    if (lane == 0 && row_raw < rows) y[row_raw] = s;
}

// ---- runtime block count (fold16) -----------------------------------------------

template <int ITERS, int WAVES, bool ODD = false>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_0_any_kernel(const uint8_t *__restrict__ w,
                                                                     const uint8_t *xpack,
                                                                     float *__restrict__ y, int rows, int nb)
{
    extern __shared__ __align__(16) uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_split_pack<true>(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int row_raw = (blockIdx.x * WAVES + (threadIdx.x >> 6) - 1) * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;
    const size_t base = (size_t)row * nb;
    RowRegs<ITERS> r;
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
    load_row<ITERS, ODD>(r, w, (size_t)rows * nb, base, nb, j);
    __syncthreads();
    const float s = fold_row<ITERS, ODD>(r, lds, base, nb, j);
    if (j == 15 && row_raw < rows) y[row_raw] = s;
}

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_0_geglu_any_kernel(const uint8_t *__restrict__ wg,
                                                                           const uint8_t *__restrict__ wu,
                                                                           const uint8_t *xpack,
                                                                           float *__restrict__ act, int rows,
                                                                           int nb)
{
    extern __shared__ __align__(16) uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_split_pack<true>(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int row_raw = (blockIdx.x * WAVES + (threadIdx.x >> 6) - 1) * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;
    const size_t nblk = (size_t)rows * nb, base = (size_t)row * nb;
    RowRegs<ITERS> rg, ru;
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
    load_row<ITERS>(rg, wg, nblk, base, nb, j);
    load_row<ITERS>(ru, wu, nblk, base, nb, j);
    __syncthreads();
    float g, u;
    fold_row2<ITERS>(rg, ru, lds, base, nb, j, g, u);
    if (j == 15 && row_raw < rows) act[row_raw] = gelu_tanh(g) * u;
}

template <int ITERS, int WAVES>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q4_0_qkv_any_kernel(const uint8_t *__restrict__ wq,
                                                                         const uint8_t *__restrict__ wk,
                                                                         const uint8_t *__restrict__ wv,
                                                                         const uint8_t *xpack,
                                                                         float *__restrict__ y, int q_rows,
                                                                         int kv_rows, int nb)
{
    extern __shared__ __align__(16) uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_split_pack<true>(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int total = q_rows + 2 * kv_rows;
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int row_raw = (blockIdx.x * WAVES + (threadIdx.x >> 6) - 1) * 4 + (lane >> 4);
    const QkvSel m = qkv_select(wq, wk, wv, row_raw < total ? row_raw : total - 1, q_rows, kv_rows);
    const size_t base = (size_t)m.local * nb;
    RowRegs<ITERS> r;
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
    load_row<ITERS>(r, m.w, (size_t)m.mrows * nb, base, nb, j);
    __syncthreads();
    const float s = fold_row<ITERS>(r, lds, base, nb, j);
    if (j == 15 && row_raw < total) y[row_raw] = s;
}

// ---- raw GGUF layout --------------------------------------------------------
// The four rows of a wave are one contiguous span of 4*nb*18 bytes.  The
// wave copies the span into LDS with 16-byte loads when it is 16-byte
// aligned, else with 2-byte loads, and reads each 18-byte block back from
// LDS.  One wave per workgroup.
template <int ITERS>
__global__ __launch_bounds__(64) void gemv_q4_0_gguf_kernel(const uint8_t *__restrict__ w,
                                                            const uint8_t *xpack,
                                                            float *__restrict__ y, int rows, int nb)
{
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *act = lds;                                    // nb*40 bytes
    uint8_t *tile = lds + align_up((size_t)nb * 40, 16);   // 4 rows of raw blocks
    const int lane = threadIdx.x, j = lane & 15, rsub = lane >> 4;
    const int row0 = blockIdx.x * 4;
    const int nrows = rows - row0 < 4 ? rows - row0 : 4;
    const size_t row_bytes = (size_t)nb * 18;
    const uint8_t *span = w + (size_t)row0 * row_bytes;
    const size_t span_bytes = (size_t)nrows * row_bytes;
    if (((uintptr_t)span & 15u) == 0 && (span_bytes & 15u) == 0) {
        const uint4 *s = reinterpret_cast<const uint4 *>(span);
        uint4 *d = reinterpret_cast<uint4 *>(tile);
        for (size_t i = lane; i < span_bytes / 16; i += 64) d[i] = s[i];
    } else {
        const uint16_t *s = reinterpret_cast<const uint16_t *>(span);
        uint16_t *d = reinterpret_cast<uint16_t *>(tile);
        for (size_t i = lane; i < span_bytes / 2; i += 64) d[i] = s[i];
    }
    stage_split_pack(xpack, act, nb);
    __syncthreads();
    const int row = rsub < nrows ? rsub : nrows - 1;
    const uint16_t *rowp = reinterpret_cast<const uint16_t *>(tile + (size_t)row * row_bytes);
    const uint4 *aq = reinterpret_cast<const uint4 *>(act);
    const float *ad = reinterpret_cast<const float *>(act + nb * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(act + nb * 36);
    float s = 0.0f;
    for (int it = 0; it < ITERS; ++it) {
        const int b = it * 16 + j;
        const int bc = b < nb ? b : nb - 1;
        const uint16_t *blk = rowp + bc * 9;  // 18 bytes = 9 halfwords
        const uint4 lo = aq[2 * bc], hi = aq[2 * bc + 1];
        const int32_t isum = q4_0_isum_split(blk[1] | ((uint32_t)blk[2] << 16), blk[3] | ((uint32_t)blk[4] << 16),
                                             blk[5] | ((uint32_t)blk[6] << 16), blk[7] | ((uint32_t)blk[8] << 16),
                                             lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w, ac[bc]);
        const float tv = (float)isum * (f16_bits_to_f32(blk[0]) * ad[bc]);
        const float t = b < nb ? tv : 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) s = fold16(s, t);
    }
    if (j == 15 && rsub < nrows) y[row0 + rsub] = s;
}

// ---- dispatch ---------------------------------------------------------------

// Waves per workgroup of the runtime-nb kernels.
inline int waves_for(int rows) { return rows >= 8192 ? 4 : (rows >= 2048 ? 2 : 1); }

// The smallest compiled iteration count >= iters (iterations past a row's
// last block are masked, so a larger instance gives the same result).
static int iters_round(int iters)
{
    static const int kInst[] = {1, 2, 3, 4, 5, 6, 8, 9, 12, 16, 18, 20};
    for (int v : kInst)
        if (v >= iters) return v;
    return 0;
}

#define MRML_DISPATCH_ITERS(ITERS_VAL, BODY)                 \
    switch (iters_round(ITERS_VAL)) {                        \
    case 1: { constexpr int IT = 1; BODY; } break;           \
    case 2: { constexpr int IT = 2; BODY; } break;           \
    case 3: { constexpr int IT = 3; BODY; } break;           \
    case 4: { constexpr int IT = 4; BODY; } break;           \
    case 5: { constexpr int IT = 5; BODY; } break;           \
    case 6: { constexpr int IT = 6; BODY; } break;           \
    case 8: { constexpr int IT = 8; BODY; } break;           \
    case 9: { constexpr int IT = 9; BODY; } break;           \
    case 12: { constexpr int IT = 12; BODY; } break;         \
    case 16: { constexpr int IT = 16; BODY; } break;         \
    case 18: { constexpr int IT = 18; BODY; } break;         \
    case 20: { constexpr int IT = 20; BODY; } break;         \
    default: return fail(ctx, MRML_HIP_E_UNSUPPORTED,        \
                         "q4_0 matvec: cols=%d (%d blocks) has no kernel instance", nb * 32, nb); \
    }

#define MRML_DISPATCH_WAVES(WAVES_VAL, BODY)                 \
    switch (WAVES_VAL) {                                     \
    case 1: { constexpr int WV = 1; BODY; } break;           \
    case 2: { constexpr int WV = 2; BODY; } break;           \
    default: { constexpr int WV = 4; BODY; } break;          \
    }

// Fixed-shape instances (the block counts of the Gemma-2-2B projections).
constexpr int kFoldWaves = 4;   // fold16 compute waves per workgroup
constexpr int kRelayS = 6;      // relay waves per 4 rows for 288-block rows (gate/up pairs)
constexpr int kLongS = 3;       // compute waves per 4 rows of the long-row kernel
constexpr int kCUs = 256;       // MI355X compute units: workgroup counts that divide among them evenly

inline bool fold16_shape(int nb) { return nb == 64 || nb == 72; }
inline bool relay_shape(int nb) { return nb == 288; }

}  // namespace

// The FFN's two launches in the balanced split form (gemv_q4_0_geglu_split_kernel
// + gemv_q4_0_long_mix_kernel): the Gemma-2-2B FFN shape, 9216 = 256 x 36 rows.
constexpr int kSplitW = 9;  // 36 rows a workgroup: 32 of one block, 4 of the tail
bool ffn_split_ok(int dim, int ffn)
{
    const int R = 4 * kSplitW, E = R - 32;
    if (!(relay_shape(ffn / 32) && fold16_shape(dim / 32) && ffn % R == 0)) return false;
    const int G = ffn / R;
    return (G * E) % 32 == 0 && G * E / 32 <= 8 * (kLongS + 1) && (((int64_t)dim * (ffn / 32)) & 1) == 0 &&
           (((int64_t)ffn * (dim / 32)) & 1) == 0;
}

namespace {

#define MRML_FOLD16_NB(NB_VAL, BODY)                                                  \
    switch (NB_VAL) {                                                                 \
    case 64: { constexpr int NB = 64; BODY; } break;                                  \
    case 72: { constexpr int NB = 72; BODY; } break;                                  \
    default: break;                                                                   \
    }

size_t pack_lds(int nb) { return align_up((size_t)nb * 40, 16); }

}  // namespace

// The scale plane is read as 4-byte words, so the block count of each matrix
// (rows * cols/32) must be even: cols % 64 == 0 or an even row count.
// A matrix with an odd number of blocks (rows * cols/32) keeps its last
// scale in the first half of a 4-byte word that would reach past the scale
// plane.  The fixed-shape kernels read scales as words, so such a matrix
// goes through the runtime-block-count kernel with 2-byte scale loads
// (ODD), and the fused entry points split into plain matvecs.
static bool odd_blocks(int32_t rows, int nb) { return (((int64_t)rows * nb) & 1) != 0; }

static int check_even(mrml_hip_ctx *ctx, int32_t rows, int nb)
{
    if (odd_blocks(rows, nb))
        return fail(ctx, MRML_HIP_E_UNSUPPORTED,
                    "q4_0 fused matvec: rows*cols/32 = %lld is odd (the unfused entry points serve it)",
                    (long long)rows * nb);
    return 0;
}

// act[i] = gelu_tanh(g[i]) * u[i]: the GeGLU epilogue of the matvec kernels
// (model.rs:2093-2105, ops.rs:99-114), elementwise.
__global__ void geglu_rows_kernel(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ act,
                                  int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) act[i] = gelu_tanh(g[i]) * u[i];
}

int launch_geglu_rows(mrml_hip_ctx *ctx, const float *g, const float *u, float *act, int n)
{
    hipLaunchKernelGGL(geglu_rows_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, g, u, act, n);
    return check_launch(ctx, "geglu_rows_kernel");
}

static int launch_gemv_q4_0_odd(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int nb)
{
    const int iters = (nb + 15) / 16;
    if (nb > kStageMax)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q4_0 matvec: cols=%d with an odd block count above %d", nb * 32,
                    kStageMax * 32);
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_any_kernel<IT, WV, true>), grid, dim3(64 * (WV + 1)), pack_lds(nb),
                           ctx->stream, (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb);
    }));
    return check_launch(ctx, "gemv_q4_0_any_kernel");
}

// GeGLU of an odd-block shape: the two products into gu (2*rows floats),
// then the elementwise epilogue into act.
static int geglu_odd(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack, float *act, float *gu,
                     int32_t rows, int nb)
{
    if (int rc = launch_gemv_q4_0_odd(ctx, wg, xpack, gu, rows, nb)) return rc;
    if (int rc = launch_gemv_q4_0_odd(ctx, wu, xpack, gu + rows, rows, nb)) return rc;
    return launch_geglu_rows(ctx, gu, gu + rows, act, rows);
}

// The relaxed rows kernel where its 64-block groups are nearly full (block
// counts that are multiples of 64, or above 256); other shapes keep the
// exact kernels, which meet the tolerance trivially.
static bool relaxed_rows_shape(int nb) { return nb <= kStageMax && (nb % 64 == 0 || nb > 256); }

static int launch_gemv_q4_0_relaxed(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows,
                                    int nb)
{
    const dim3 grid((rows + kRelaxR - 1) / kRelaxR), block(64 * (kRelaxR + 1));
    const int groups = (nb + 63) / 64;
    const bool odd = odd_blocks(rows, nb);
#define MRML_RELAXED_K(KK)                                                                                       \
    case KK:                                                                                                     \
        if (odd)                                                                                                 \
            hipLaunchKernelGGL((gemv_q4_0_relaxed_kernel<KK, true>), grid, block, pack_lds(nb), ctx->stream,     \
                               (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb);                         \
        else                                                                                                     \
            hipLaunchKernelGGL((gemv_q4_0_relaxed_kernel<KK, false>), grid, block, pack_lds(nb), ctx->stream,    \
                               (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb);                         \
        break;
    switch (groups) {
        MRML_RELAXED_K(1)
        MRML_RELAXED_K(2)
        MRML_RELAXED_K(3)
        MRML_RELAXED_K(4)
        MRML_RELAXED_K(5)
        default:
            return fail(ctx, MRML_HIP_E_UNSUPPORTED, "relaxed q4_0 matvec: %d blocks per row", nb);
    }
#undef MRML_RELAXED_K
    return check_launch(ctx, "gemv_q4_0_relaxed_kernel");
}

int launch_gemv_q4_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols,
                     bool relaxed)
{
    const int nb = cols / 32;
    if (relaxed && relaxed_rows_shape(nb)) return launch_gemv_q4_0_relaxed(ctx, w, xpack, y, rows, nb);
    if (odd_blocks(rows, nb)) return launch_gemv_q4_0_odd(ctx, w, xpack, y, rows, nb);
    if (fold16_shape(nb)) {
        const dim3 grid(((rows + 3) / 4 + kFoldWaves - 1) / kFoldWaves);
        MRML_FOLD16_NB(nb, {
            hipLaunchKernelGGL((gemv_q4_0_kernel<NB, kFoldWaves, false>), grid, dim3(64 * (kFoldWaves + 1)),
                               pack_lds(NB), ctx->stream, (const uint8_t *)w, xpack, y, rows);
        });
        return check_launch(ctx, "gemv_q4_0_kernel");
    }
    if (relay_shape(nb)) {
        hipLaunchKernelGGL((gemv_q4_0_long_kernel<288, kLongS>), dim3((rows + 3) / 4), dim3(64 * (kLongS + 1)),
                           (long_lds<288, kLongS>()), ctx->stream, (const uint8_t *)w, (const uint8_t *)xpack, y, rows);
        return check_launch(ctx, "gemv_q4_0_long_kernel");
    }
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_any_kernel<IT, WV>), grid, dim3(64 * (WV + 1)), pack_lds(nb), ctx->stream,
                           (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb);
    }));
    return check_launch(ctx, "gemv_q4_0_any_kernel");
}

// f32 input: quantised inside the kernel where a fixed instance exists, else
// through the scratch pack.
// The split form's two launches.  GeGLU: x (cols f32) -> act (rows f32) and
// the pack of its whole blocks (act_pack_bytes(rows / 32) bytes; the tail
// blocks [split_main_blocks(rows), rows / 32) left out).  Down: the pack's
// whole blocks plus the tail blocks quantised from act -> y (rows f32).
int split_main_blocks(int ffn) { return ffn / (4 * kSplitW); }

// The down projection's weights to read ahead in the split GeGLU (the
// GeGLU's workgroup w holds rows 9w .. 9w+8 of it, the down projection's own
// workgroup w), or null when the down projection runs another layout.
static const uint8_t *split_prefetch(const void *wd, int32_t dim, int32_t ffn)
{
    return (wd && dim % (9 * kCUs) == 0 && dim / 9 == split_main_blocks(ffn)) ? (const uint8_t *)wd : nullptr;
}

int launch_geglu_split(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act, void *pack,
                       int32_t rows, int32_t cols, const void *wd)
{
    const uint8_t *pf = split_prefetch(wd, cols, rows);
    MRML_FOLD16_NB(cols / 32, {
        hipLaunchKernelGGL((gemv_q4_0_geglu_split_kernel<NB, kSplitW>), dim3(split_main_blocks(rows)),
                           dim3(64 * (kSplitW + kNQ)), (geglu_f32_lds<NB, kSplitW>()), ctx->stream,
                           (const uint8_t *)wg, (const uint8_t *)wu, x, act, (uint8_t *)pack, rows, pf, cols,
                           rows / 32);
    });
    return check_launch(ctx, "gemv_q4_0_geglu_split_kernel");
}

int launch_geglu_resnorm_split(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *t,
                               const float *w_post, const float *h_in, float *h_out, const float *w_norm, float eps,
                               float *act, void *pack, int32_t rows, int32_t cols, bool fast)
{
    if (!ffn_split_ok(cols, rows) || h_in == h_out)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "geglu_resnorm_split: no instance for %dx%d (or h_in == h_out)", rows,
                    cols);
    MRML_FOLD16_NB(cols / 32, {
        if (fast)
            hipLaunchKernelGGL((gemv_q4_0_geglu_resnorm_split_kernel<NB, kSplitW, true>), dim3(split_main_blocks(rows)),
                               dim3(64 * (kSplitW + kNQ)), (geglu_resnorm_split_lds<NB, kSplitW>()), ctx->stream,
                               (const uint8_t *)wg, (const uint8_t *)wu, t, w_post, h_in, h_out, w_norm, eps, act,
                               (uint8_t *)pack, rows);
        else
            hipLaunchKernelGGL((gemv_q4_0_geglu_resnorm_split_kernel<NB, kSplitW, false>),
                               dim3(split_main_blocks(rows)), dim3(64 * (kSplitW + kNQ)),
                               (geglu_resnorm_split_lds<NB, kSplitW>()), ctx->stream, (const uint8_t *)wg,
                               (const uint8_t *)wu, t, w_post, h_in, h_out, w_norm, eps, act, (uint8_t *)pack, rows);
    });
    return check_launch(ctx, "gemv_q4_0_geglu_resnorm_split_kernel");
}

int launch_down_mix(mrml_hip_ctx *ctx, const void *wd, const void *pack, const float *act, float *y, int32_t rows,
                    int32_t cols)
{
    if (rows % (9 * kCUs) == 0) {
        // nine rows a workgroup (three quads): a whole number of workgroups per CU
        hipLaunchKernelGGL((gemv_q4_0_long_mix_kernel<288, kLongS, 3>), dim3(rows / 9), dim3(64 * (3 * kLongS + 2)),
                           (long_mix_lds<288, kLongS, 3>()), ctx->stream, (const uint8_t *)wd, (const uint8_t *)pack,
                           act, y, rows, split_main_blocks(cols), 9);
    } else {
        hipLaunchKernelGGL((gemv_q4_0_long_mix_kernel<288, kLongS, 1>), dim3((rows + 3) / 4), dim3(64 * (kLongS + 2)),
                           (long_mix_lds<288, kLongS, 1>()), ctx->stream, (const uint8_t *)wd, (const uint8_t *)pack,
                           act, y, rows, split_main_blocks(cols), 4);
    }
    return check_launch(ctx, "gemv_q4_0_long_mix_kernel");
}

int launch_ffn_split(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *wd, const float *x, float *act,
                     void *pack, float *y, int32_t dim, int32_t ffn)
{
    if (int rc = launch_geglu_split(ctx, wg, wu, x, act, pack, ffn, dim, wd)) return rc;
    return launch_down_mix(ctx, wd, pack, act, y, dim, ffn);
}

int launch_gemv_q4_0_x(mrml_hip_ctx *ctx, const void *w, const float *x, float *y, int32_t rows, int32_t cols)
{
    const int nb = cols / 32;
    if (fold16_shape(nb) && !odd_blocks(rows, nb)) {
        const dim3 grid(((rows + 3) / 4 + kFoldWaves - 1) / kFoldWaves);
        MRML_FOLD16_NB(nb, {
            hipLaunchKernelGGL((gemv_q4_0_kernel<NB, kFoldWaves, true>), grid, dim3(64 * (kFoldWaves + kNQ)),
                               pack_lds(NB), ctx->stream, (const uint8_t *)w, (const void *)x, y, rows);
        });
        return check_launch(ctx, "gemv_q4_0_kernel");
    }
    void *pk = workspace(ctx, act_pack_bytes(nb));
    if (!pk) return MRML_HIP_E_ALLOC;
    if (int rc = launch_quantize_q8_0(ctx, x, nullptr, pk, cols)) return rc;
    return launch_gemv_q4_0(ctx, w, pk, y, rows, cols);
}

int launch_gemv_q4_0_geglu(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack, float *act,
                           int32_t rows, int32_t cols)
{
    const int nb = cols / 32;
    if (odd_blocks(rows, nb)) {  // xpack is never the workspace here (launch_gemv_q4_0_geglu_x handles its own)
        float *gu = (float *)workspace(ctx, (size_t)2 * rows * sizeof(float));
        if (!gu) return MRML_HIP_E_ALLOC;
        return geglu_odd(ctx, wg, wu, xpack, act, gu, rows, nb);
    }
    if (fold16_shape(nb)) {
        const dim3 grid(((rows + 3) / 4 + kFoldWaves - 1) / kFoldWaves);
        MRML_FOLD16_NB(nb, {
            hipLaunchKernelGGL((gemv_q4_0_geglu_kernel<NB, kFoldWaves, false, false>), grid,
                               dim3(64 * (kFoldWaves + 1)), geglu_lds<NB>(kFoldWaves), ctx->stream, (const uint8_t *)wg,
                               (const uint8_t *)wu, xpack, act, (uint8_t *)nullptr, rows);
        });
        return check_launch(ctx, "gemv_q4_0_geglu_kernel");
    }
    if (relay_shape(nb)) {
        hipLaunchKernelGGL((gemv_q4_0_relay_kernel<288, kRelayS, 2>), dim3((rows + 3) / 4), dim3(64 * kRelayS), 0,
                           ctx->stream, (const uint8_t *)wg, (const uint8_t *)wu, (const uint8_t *)xpack, act, rows);
        return check_launch(ctx, "gemv_q4_0_relay_kernel");
    }
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_geglu_any_kernel<IT, WV>), grid, dim3(64 * (WV + 1)), pack_lds(nb),
                           ctx->stream, (const uint8_t *)wg, (const uint8_t *)wu, (const uint8_t *)xpack, act, rows,
                           nb);
    }));
    return check_launch(ctx, "gemv_q4_0_geglu_any_kernel");
}

// f32 input, optional f32 output, optional Q8_0 pack of the output (for the
// next projection).  One launch when the shape has a fixed instance and
// rows % 32 == 0; otherwise quantise / run / quantise separately.
int launch_gemv_q4_0_geglu_emit(mrml_hip_ctx *ctx, const void *wg, const void *wu, const void *xpack, float *act,
                                void *act_pack, int32_t rows, int32_t cols)
{
    const int nb = cols / 32;
    if (odd_blocks(rows, nb)) {
        float *gu = (float *)workspace(ctx, (size_t)3 * rows * sizeof(float));
        if (!gu) return MRML_HIP_E_ALLOC;
        float *out = act ? act : gu + 2 * (size_t)rows;
        if (int rc = geglu_odd(ctx, wg, wu, xpack, out, gu, rows, nb)) return rc;
        return launch_quantize_q8_0(ctx, out, nullptr, act_pack, rows);
    }
    if (fold16_shape(nb) && rows % 32 == 0) {
        MRML_FOLD16_NB(nb, {
            hipLaunchKernelGGL((gemv_q4_0_geglu_kernel<NB, 8, false, true>), dim3(rows / 32), dim3(64 * 9),
                               geglu_lds<NB>(8), ctx->stream, (const uint8_t *)wg,
                               (const uint8_t *)wu, xpack, act, (uint8_t *)act_pack, rows);
        });
        return check_launch(ctx, "gemv_q4_0_geglu_kernel");
    }
    float *out = act;
    if (!out) {
        out = (float *)workspace(ctx, (size_t)rows * sizeof(float));
        if (!out) return MRML_HIP_E_ALLOC;
    }
    if (int rc = launch_gemv_q4_0_geglu(ctx, wg, wu, xpack, out, rows, cols)) return rc;
    return launch_quantize_q8_0(ctx, out, nullptr, act_pack, rows);
}

// f32 in, f32 out on the balanced kernel (36 rows per workgroup).
constexpr int kGegluF32W = 9;

static int launch_geglu_f32(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                            int32_t rows, int nb)
{
    constexpr int R = 4 * kGegluF32W;
    MRML_FOLD16_NB(nb, {
        hipLaunchKernelGGL((gemv_q4_0_geglu_f32_kernel<NB, kGegluF32W>), dim3((rows + R - 1) / R),
                           dim3(64 * (kGegluF32W + kNQ)), (geglu_f32_lds<NB, kGegluF32W>()), ctx->stream,
                           (const uint8_t *)wg, (const uint8_t *)wu, x, act, rows);
    });
    return check_launch(ctx, "gemv_q4_0_geglu_f32_kernel");
}

int launch_gemv_q4_0_geglu_x(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *x, float *act,
                             void *act_pack, int32_t rows, int32_t cols)
{
    const int nb = cols / 32;
    if (odd_blocks(rows, nb)) {
        // one workspace: x's pack, then g, u and (without act) the output
        const size_t in_bytes = align_up(act_pack_bytes(nb), 16);
        uint8_t *ws = (uint8_t *)workspace(ctx, in_bytes + (size_t)3 * rows * sizeof(float));
        if (!ws) return MRML_HIP_E_ALLOC;
        float *gu = reinterpret_cast<float *>(ws + in_bytes), *out = act ? act : gu + 2 * (size_t)rows;
        if (int rc = launch_quantize_q8_0(ctx, x, nullptr, ws, cols)) return rc;
        if (int rc = geglu_odd(ctx, wg, wu, ws, out, gu, rows, nb)) return rc;
        if (act_pack) return launch_quantize_q8_0(ctx, out, nullptr, act_pack, rows);
        return MRML_HIP_OK;
    }
    if (fold16_shape(nb) && !act_pack) return launch_geglu_f32(ctx, wg, wu, x, act, rows, nb);
    if (fold16_shape(nb) && (!act_pack || rows % 32 == 0)) {
        if (act_pack) {
            MRML_FOLD16_NB(nb, {
                hipLaunchKernelGGL((gemv_q4_0_geglu_kernel<NB, 8, true, true>), dim3(rows / 32), dim3(64 * (8 + kNQ)),
                                   geglu_lds<NB>(8), ctx->stream, (const uint8_t *)wg, (const uint8_t *)wu, (const void *)x, act,
                                   (uint8_t *)act_pack, rows);
            });
        } else {
            const dim3 grid(((rows + 3) / 4 + kFoldWaves - 1) / kFoldWaves);
            MRML_FOLD16_NB(nb, {
                hipLaunchKernelGGL((gemv_q4_0_geglu_kernel<NB, kFoldWaves, true, false>), grid,
                                   dim3(64 * (kFoldWaves + kNQ)), geglu_lds<NB>(kFoldWaves), ctx->stream, (const uint8_t *)wg,
                                   (const uint8_t *)wu, (const void *)x, act, (uint8_t *)nullptr, rows);
            });
        }
        return check_launch(ctx, "gemv_q4_0_geglu_kernel");
    }
    const size_t in_bytes = act_pack_bytes(nb);
    uint8_t *ws = (uint8_t *)workspace(ctx, in_bytes + (size_t)rows * sizeof(float));
    if (!ws) return MRML_HIP_E_ALLOC;
    float *out = act ? act : reinterpret_cast<float *>(ws + in_bytes);
    if (int rc = launch_quantize_q8_0(ctx, x, nullptr, ws, cols)) return rc;
    if (int rc = launch_gemv_q4_0_geglu(ctx, wg, wu, ws, out, rows, cols)) return rc;
    if (act_pack) return launch_quantize_q8_0(ctx, out, nullptr, act_pack, rows);
    return MRML_HIP_OK;
}

int launch_gemv_q4_0_qkv(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const void *xpack,
                         float *y, int32_t q_rows, int32_t kv_rows, int32_t cols)
{
    const int nb = cols / 32;
    if (odd_blocks(q_rows, nb) || odd_blocks(kv_rows, nb)) {  // three plain products into the stacked rows
        if (int rc = launch_gemv_q4_0(ctx, wq, xpack, y, q_rows, cols)) return rc;
        if (int rc = launch_gemv_q4_0(ctx, wk, xpack, y + q_rows, kv_rows, cols)) return rc;
        return launch_gemv_q4_0(ctx, wv, xpack, y + q_rows + kv_rows, kv_rows, cols);
    }
    const int total = q_rows + 2 * kv_rows;
    if (fold16_shape(nb)) {
        const dim3 grid(((total + 3) / 4 + kFoldWaves - 1) / kFoldWaves);
        MRML_FOLD16_NB(nb, {
            hipLaunchKernelGGL((gemv_q4_0_qkv_kernel<NB, kFoldWaves, false>), grid, dim3(64 * (kFoldWaves + 1)),
                               pack_lds(NB), ctx->stream, (const uint8_t *)wq, (const uint8_t *)wk,
                               (const uint8_t *)wv, xpack, y, q_rows, kv_rows);
        });
        return check_launch(ctx, "gemv_q4_0_qkv_kernel");
    }
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(total);
    const dim3 grid(((total + 3) / 4 + waves - 1) / waves);
    MRML_DISPATCH_ITERS(iters, MRML_DISPATCH_WAVES(waves, {
        hipLaunchKernelGGL((gemv_q4_0_qkv_any_kernel<IT, WV>), grid, dim3(64 * (WV + 1)), pack_lds(nb), ctx->stream,
                           (const uint8_t *)wq, (const uint8_t *)wk, (const uint8_t *)wv, (const uint8_t *)xpack,
                           y, q_rows, kv_rows, nb);
    }));
    return check_launch(ctx, "gemv_q4_0_qkv_any_kernel");
}

int launch_gemv_q4_0_qkv_x(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *x,
                           float *y, int32_t q_rows, int32_t kv_rows, int32_t cols)
{
    const int nb = cols / 32;
    const int total = q_rows + 2 * kv_rows;
    if (fold16_shape(nb) && !odd_blocks(q_rows, nb) && !odd_blocks(kv_rows, nb)) {
        const dim3 grid(((total + 3) / 4 + kFoldWaves - 1) / kFoldWaves);
        MRML_FOLD16_NB(nb, {
            hipLaunchKernelGGL((gemv_q4_0_qkv_kernel<NB, kFoldWaves, true>), grid, dim3(64 * (kFoldWaves + kNQ)),
                               pack_lds(NB), ctx->stream, (const uint8_t *)wq, (const uint8_t *)wk,
                               (const uint8_t *)wv, (const void *)x, y, q_rows, kv_rows);
        });
        return check_launch(ctx, "gemv_q4_0_qkv_kernel");
    }
    void *pk = workspace(ctx, act_pack_bytes(nb));
    if (!pk) return MRML_HIP_E_ALLOC;
    if (int rc = launch_quantize_q8_0(ctx, x, nullptr, pk, cols)) return rc;
    return launch_gemv_q4_0_qkv(ctx, wq, wk, wv, pk, y, q_rows, kv_rows, cols);
}

// The Gemma-2 residual fused ahead of the gate/up GeGLU (act pack out) or of
// the q|k|v matvec.  resnorm_shape() says whether a fused instance exists;
// otherwise the caller runs the residual norm and the matvec separately.
bool resnorm_shape(int cols) { return fold16_shape(cols / 32) && cols % 32 == 0; }

static size_t resnorm_lds(int nb) { return pack_lds(nb) + 64 * sizeof(float) + sizeof(mrml_xsum::Shared4); }


int launch_geglu_resnorm(mrml_hip_ctx *ctx, const void *wg, const void *wu, const float *t, const float *w_post,
                         const float *h_in, float *h_out, const float *w_norm, float eps, void *act_pack, int32_t rows,
                         int32_t cols, bool fast)
{
    const int nb = cols / 32;
    if (!resnorm_shape(cols) || rows % 64 != 0 || h_in == h_out)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "geglu_resnorm: no fused instance for %dx%d (or h_in == h_out)", rows,
                    cols);
    if (int rc = check_even(ctx, rows, nb)) return rc;
    MRML_FOLD16_NB(nb, {
        if (fast)
            hipLaunchKernelGGL((gemv_q4_0_geglu_resnorm_kernel<NB, true>), dim3(rows / 64), dim3(64 * kGegluResWaves),
                               geglu_resnorm_lds<NB>(), ctx->stream, (const uint8_t *)wg, (const uint8_t *)wu, t,
                               w_post, h_in, h_out, w_norm, eps, (uint8_t *)act_pack, rows);
        else
            hipLaunchKernelGGL((gemv_q4_0_geglu_resnorm_kernel<NB, false>), dim3(rows / 64),
                               dim3(64 * kGegluResWaves), geglu_resnorm_lds<NB>(), ctx->stream, (const uint8_t *)wg,
                               (const uint8_t *)wu, t, w_post, h_in, h_out, w_norm, eps, (uint8_t *)act_pack, rows);
    });
    return check_launch(ctx, "gemv_q4_0_geglu_resnorm_kernel");
}

int launch_qkv_resnorm(mrml_hip_ctx *ctx, const void *wq, const void *wk, const void *wv, const float *t,
                       const float *w_post, const float *h_in, float *h_out, const float *w_norm, float eps, float *y,
                       int32_t q_rows, int32_t kv_rows, int32_t cols, bool fast)
{
    const int nb = cols / 32;
    if (!resnorm_shape(cols) || h_in == h_out)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "qkv_resnorm: no fused instance for cols=%d (or h_in == h_out)", cols);
    if (int rc = check_even(ctx, q_rows, nb)) return rc;
    if (int rc = check_even(ctx, kv_rows, nb)) return rc;
    const int total = q_rows + 2 * kv_rows;
    constexpr int CW = kQkvResRowWaves, RPW = 4 * CW;
    MRML_FOLD16_NB(nb, {
        if (fast)
            hipLaunchKernelGGL((gemv_q4_0_qkv_resnorm_kernel<NB, true, CW>), dim3((total + RPW - 1) / RPW),
                               dim3(64 * kResWaves), resnorm_lds(NB), ctx->stream, (const uint8_t *)wq,
                               (const uint8_t *)wk, (const uint8_t *)wv, t, w_post, h_in, h_out, w_norm, eps, y,
                               q_rows, kv_rows);
        else
            hipLaunchKernelGGL((gemv_q4_0_qkv_resnorm_kernel<NB, false, CW>), dim3((total + RPW - 1) / RPW),
                               dim3(64 * kResWaves), resnorm_lds(NB), ctx->stream, (const uint8_t *)wq,
                               (const uint8_t *)wk, (const uint8_t *)wv, t, w_post, h_in, h_out, w_norm, eps, y,
                               q_rows, kv_rows);
    });
    return check_launch(ctx, "gemv_q4_0_qkv_resnorm_kernel");
}

int launch_gemv_q4_0_gguf(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows,
                          int32_t cols)
{
    const int nb = cols / 32;
    const int iters = (nb + 15) / 16;
    const size_t lds = align_up((size_t)nb * 40, 16) + (size_t)4 * nb * 18;
    if (lds > 160 * 1024)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "gemv_q4_0_gguf: cols=%d needs %zu bytes of LDS", cols, lds);
    const dim3 grid((rows + 3) / 4);
    MRML_DISPATCH_ITERS(iters, {
        hipLaunchKernelGGL((gemv_q4_0_gguf_kernel<IT>), grid, dim3(64), lds, ctx->stream, (const uint8_t *)w,
                           (const uint8_t *)xpack, y, rows, nb);
    });
    return check_launch(ctx, "gemv_q4_0_gguf_kernel");
}

hipError_t wait_guard_gemv(int polls, uint32_t *timeouts) { return mrml_xsum::wait_guard_io(polls, timeouts); }

}  // namespace mrml
