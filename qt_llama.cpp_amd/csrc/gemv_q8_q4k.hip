// gemv_q8_q4k.hip -- batch-1 Q8_0 and Q4_K matrix-vector products and the
// greedy argmax, gfx950.  Same wave mapping and ordered DPP fold as the Q4_0
// kernels (one 16-lane DPP row per matrix row, 4 rows per wave); this file
// is compiled with -ffp-contract=off.

#include "device.h"
#include "internal.h"
#include "libm_f32.h"

namespace mrml {

namespace {


// Wave 0 of each workgroup copies the activation pack into LDS; the compute
// waves issue only their weight loads (see gemv_q4_0.hip).
__device__ __forceinline__ void stage_pack_wave(const uint8_t *src, uint8_t *lds, int nb)
{
    const int n16 = (nb * 40 + 15) >> 4;
    const uint4 *s = reinterpret_cast<const uint4 *>(src);
    uint4 *d = reinterpret_cast<uint4 *>(lds);
    for (int i = threadIdx.x; i < n16; i += 64) d[i] = s[i];
}

// ---- Q8_0 (quant.rs:563-577 semantics; model.rs:2842-2853 softcap) ---------
// Backend layout: quant plane [rows*nb][32 B], scale plane [rows*nb] f16.

// ODD: the matrix has an odd number of blocks, so the 4-byte word of the last
// scale would reach past the scale plane; scales are then read with 2-byte
// loads.
template <int ITERS, int WAVES, bool ODD>
__global__ __launch_bounds__(64 * (WAVES + 1)) void gemv_q8_0_kernel(const uint8_t *__restrict__ w,
                                                                     const uint8_t *xpack,
                                                                     float *__restrict__ y, int rows, int nb,
                                                                     int softcap)
{
    extern __shared__ uint8_t lds[];
    if (threadIdx.x < 64) {
        stage_pack_wave(xpack, lds, nb);
        __syncthreads();
        return;
    }
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int quad = blockIdx.x * WAVES + (threadIdx.x >> 6) - 1;
    const int row_raw = quad * 4 + (lane >> 4);
    const int row = row_raw < rows ? row_raw : rows - 1;
    const size_t nblk = (size_t)rows * nb;
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint16_t *dp = reinterpret_cast<const uint16_t *>(w + nblk * 32);
    const size_t base = (size_t)row * nb;

    // Scales are read as the 4-byte word holding them (see gemv_q4_0.hip);
    // tail lanes load a clamped in-bounds block and are masked in the fold.
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(dp);
    uint4 w0[ITERS], w1[ITERS];
    uint32_t d[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int b = it * 16 + j;
        b = b < nb ? b : nb - 1;
        w0[it] = load_stream16(qs + 2 * (base + b));
        w1[it] = load_stream16(qs + 2 * (base + b) + 1);
        d[it] = ODD ? (uint32_t)dp[base + b] : dw[(base + b) >> 1];
    }
    __syncthreads();
    const int4 *aq = reinterpret_cast<const int4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    float s = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int bt = it * 16 + j;
        const int b = bt < nb ? bt : nb - 1;
        {
            const int4 a0 = aq[2 * b], a1 = aq[2 * b + 1];
            int32_t isum = sdot4(w0[it].x, (uint32_t)a0.x, 0);
            isum = sdot4(w0[it].y, (uint32_t)a0.y, isum);
            isum = sdot4(w0[it].z, (uint32_t)a0.z, isum);
            isum = sdot4(w0[it].w, (uint32_t)a0.w, isum);
            isum = sdot4(w1[it].x, (uint32_t)a1.x, isum);
            isum = sdot4(w1[it].y, (uint32_t)a1.y, isum);
            isum = sdot4(w1[it].z, (uint32_t)a1.z, isum);
            isum = sdot4(w1[it].w, (uint32_t)a1.w, isum);
            const size_t blk = base + b;
            const float tv = (float)isum * (f16_bits_to_f32((!ODD && (blk & 1)) ? d[it] >> 16 : d[it] & 0xffffu) * ad[b]);
            const float t = bt < nb ? tv : 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) s = fold16(s, t);
        }
    }
    if (j == 15 && row_raw < rows) y[row_raw] = softcap ? 30.0f * mrml_libm::tanhf(s / 30.0f) : s;
}

// ---- Q4_K (build-defined semantics over the GGUF super-block) ---------------
// Backend layout (repack_q4_k_kernel): quant plane [rows*nsb*8][16 B], one
// 16-byte run per 32-weight sub-block in Q4_0 nibble order, then the header
// plane [rows*nsb][16 B] = {f16 d, f16 dmin, 96-bit field of the 6-bit
// scales (bits 6j..) and mins (bits 48+6j..)}.  The rows then stream like
// Q4_0 rows of 8*nsb blocks: lane j of a 16-lane row owns sub-blocks
// 16*it + j (sub-block j & 7 of its super-block in every iteration).  Term
// of a sub-block:
//   t = (float)isum * ((d * sc) * da) - bsum * ((dmin * m) * da),
//   isum = sum q*a (q = 0..15), bsum = sum a (the activation block's sum,
//   staged as an exact float),
// the integer dot on the split-nibble pack (stage_split_pack's KQ form: 8
// dot8 and 4 xor per sub-block).  The 8 lanes of a super-block share its
// header: each lane loads one 4-byte word of it (lane j: word j & 3, so
// every quad of lanes holds the whole header) and gets the other three by
// DPP quad broadcasts.
//
// The fold is transposed: the compute waves store each row's terms to LDS,
// T[row][b] (every slot of every iteration, the ones past the row end +0),
// and after a barrier lane r of the staging wave adds row r's terms in
// sub-block order (super-blocks, then sub-blocks: the oracle's order).  One
// add per sub-block for up to 64 rows, where a 16-lane DPP fold spends 16
// dependent adds per 16 sub-blocks per 4 rows: the DPP fold made this kernel
// VALU-bound at the 256000-row head.  The trailing +0 slots leave the sum
// unchanged (it is never -0: it starts at +0, and a sum of floats that is
// exactly zero rounds to +0).

template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K | (K << 2) | (K << 4) | (K << 6), 0xf, 0xf, false);
}

// T row stride in floats: every slot of ITERS iterations, an odd number of
// 16-byte segments (the fold lanes' float4 reads spread over the banks).
template <int ITERS>
constexpr int q4k_t_stride() { return (ITERS * 4) % 2 ? ITERS * 16 : ITERS * 16 + 4; }

inline size_t q4k_t_off(int nb) { return ((size_t)nb * 44 + 15) & ~(size_t)15; }

// Dynamic LDS of a launch: the pack with block sums, then T.
template <int ITERS>
size_t q4k_lds(int nb, int waves) { return q4k_t_off(nb) + (size_t)4 * waves * q4k_t_stride<ITERS>() * sizeof(float); }

template <int ITERS, int W>
__global__ __launch_bounds__(64 * (W + 1)) void gemv_q4_k_kernel(const uint8_t *__restrict__ w,
                                                                 const uint8_t *xpack,
                                                                 float *__restrict__ y, int rows, int nsb)
{
    constexpr int TS = q4k_t_stride<ITERS>();
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = nsb * 8;  // sub-blocks per row = activation blocks
    float *T = reinterpret_cast<float *>(lds + (((size_t)nb * 44 + 15) & ~(size_t)15));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (int)blockIdx.x * 4 * W;
    if (wave == 0) {
        stage_split_pack<true, true>(xpack, lds, nb);
        __syncthreads();  // the pack is whole
        __syncthreads();  // the terms are in
        if (lane < 4 * W) {
            const float4 *p = reinterpret_cast<const float4 *>(T + lane * TS);
            float s = 0.0f;
#pragma unroll
            for (int k0 = 0; k0 < ITERS * 4; k0 += 4) {
                float4 v[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k0 + k < ITERS * 4) v[k] = p[k0 + k];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (k0 + k < ITERS * 4) {
                        s = s + v[k].x;
                        s = s + v[k].y;
                        s = s + v[k].z;
                        s = s + v[k].w;
                    }
                }
            }
            if (row0 + lane < rows) y[row0 + lane] = s;
        }
        return;
    }
    const int j = lane & 15, rl = (wave - 1) * 4 + (lane >> 4);
    const int row = row0 + rl < rows ? row0 + rl : rows - 1;  // tail rows recompute the last row
    const uint4 *qs = reinterpret_cast<const uint4 *>(w);
    const uint32_t *hp = reinterpret_cast<const uint32_t *>(w + (size_t)rows * nb * 16);
    const size_t base = (size_t)row * nb, hbase = (size_t)row * nsb;
    const int sh_sc = 6 * (j & 7), sh_m = 16 + 6 * (j & 7);

    // every load of the row first; past the row end a clamped in-bounds
    // sub-block, masked out of the fold
    uint4 q[ITERS];
    uint32_t hw[ITERS];
    __builtin_amdgcn_s_barrier();  // the pack's loads are issued
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        int b = it * 16 + j;
        b = b < nb ? b : nb - 1;
        q[it] = load_stream16(qs + base + b);
        hw[it] = hp[(hbase + (b >> 3)) * 4 + (j & 3)];
    }
    __syncthreads();
    const uint4 *aq = reinterpret_cast<const uint4 *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    const int32_t *ac = reinterpret_cast<const int32_t *>(lds + nb * 36);
    const float *as = reinterpret_cast<const float *>(lds + nb * 40);
    float *Tr = T + rl * TS;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int bt = it * 16 + j;
        const int b = bt < nb ? bt : nb - 1;
        const uint4 wq = q[it], lo = aq[2 * b], hi = aq[2 * b + 1];
        const int32_t isum = q4_0_isum_split(wq.x, wq.y, wq.z, wq.w, lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w,
                                             ac[b]);
        const uint32_t h0 = quad_bcast<0>(hw[it]), h1 = quad_bcast<1>(hw[it]), h2 = quad_bcast<2>(hw[it]),
                       h3 = quad_bcast<3>(hw[it]);
        const uint64_t f_sc = (uint64_t)h1 | ((uint64_t)h2 << 32), f_m = (uint64_t)h2 | ((uint64_t)h3 << 32);
        const uint32_t sc = (uint32_t)(f_sc >> sh_sc) & 63u, m = (uint32_t)(f_m >> sh_m) & 63u;
        const float d = f16_bits_to_f32(h0 & 0xffffu);
        const float dmin = f16_bits_to_f32(h0 >> 16);
        const float da = ad[b];
        const float ds = (d * (float)sc) * da;
        const float dm = (dmin * (float)m) * da;
        const float tv = (float)isum * ds - as[b] * dm;
        Tr[it * 16 + j] = bt < nb ? tv : 0.0f;
    }
    __syncthreads();
}

// ---- argmax (lowest index on ties, NaN never wins) ---------------------------

__device__ __forceinline__ bool better(float av, int ai, float bv, int bi)
{
    const bool an = av != av, bn = bv != bv;
    if (an || bn) return (an && bn) ? ai < bi : bn;
    return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ void block_best(float &v, int &i)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        if (better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wave] = v; si[wave] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < nw; ++k)
            if (better(sv[k], si[k], v, i)) { v = sv[k]; i = si[k]; }
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ x, int n,
                                                             float *__restrict__ pv, int *__restrict__ pi)
{
    float v = __builtin_nanf("");
    int i = 0x7fffffff;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < n; k += gridDim.x * blockDim.x) {
        const float xv = x[k];
        if (better(xv, k, v, i)) { v = xv; i = k; }
    }
    block_best(v, i);
    if (threadIdx.x == 0) { pv[blockIdx.x] = v; pi[blockIdx.x] = i; }
}

// With `state` = {token, pos} (device), also advances a decode loop kept on
// the device: hist[pos] = the argmax (when pos < hist_cap); pos += 1; token =
// prompt[pos] while pos < prompt_len (prefill), else the argmax.
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *__restrict__ pv, const int *__restrict__ pi,
                                                           int parts, int32_t *__restrict__ out,
                                                           int32_t *__restrict__ state, int32_t *__restrict__ hist,
                                                           int hist_cap, const int32_t *__restrict__ prompt,
                                                           int prompt_len, int2 *__restrict__ ring)
{
    float v = __builtin_nanf("");
    int i = 0x7fffffff;
    for (int k = threadIdx.x; k < parts; k += blockDim.x)
        if (better(pv[k], pi[k], v, i)) { v = pv[k]; i = pi[k]; }
    block_best(v, i);
    if (threadIdx.x == 0) {
        if (out) *out = i;
        if (state) {
            const int cur = state[1];
            if (ring && cur >= 0) ring[cur % 32] = make_int2(cur, state[0]);  // the token processed at cur
            if (hist && cur >= 0 && cur < hist_cap) hist[cur] = i;
            const int pos = cur + 1;
            state[0] = (prompt && pos < prompt_len) ? prompt[pos] : i;
            state[1] = pos;
        }
    }
}

// ---- vocabulary scoring and the next-token pick (model.rs:2842-2907) -----------
// Candidates are ranked by a 64-bit key: the score's bits made order-
// preserving as an unsigned number in the high word, ~id in the low word, so
// a larger key is a larger score or, on equal scores, a lower id.  Key 0
// marks "no candidate" (masked, NaN, or past the end).
__device__ __forceinline__ uint64_t cand_key(float s, int id)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, s);
    const uint32_t o = (u >> 31) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)id;
}
__device__ __forceinline__ float key_score(uint64_t k)
{
    const uint32_t o = (uint32_t)(k >> 32);
    return __builtin_bit_cast(float, (o >> 31) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)~(uint32_t)k; }

__device__ __forceinline__ uint64_t wave_max(uint64_t v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, 64);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// The workgroup's largest v, in every thread (red: one entry per wave).
template <typename T>
__device__ __forceinline__ T block_max(T v, T *red)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (int)(blockDim.x >> 6);
    v = wave_max(v);
    __syncthreads();  // red is free
    if (lane == 0) red[wave] = v;
    __syncthreads();
    T m = red[0];
    for (int w = 1; w < nw; ++w) m = red[w] > m ? red[w] : m;
    return m;
}

// The k-th largest of vals[0..n) (LDS), counted with multiplicity: the
// largest v with at least k values >= v; `none` when n < k.  Every thread.
template <typename T>
__device__ __forceinline__ T kth_largest(const T *vals, int n, int k, T none, T *red)
{
    T best = none;
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
        const T v = vals[t];
        int c = 0;
        for (int u = 0; u < n; ++u) c += vals[u] >= v ? 1 : 0;
        if (c >= k && v > best) best = v;
    }
    return block_max(best, red);
}

// top[0..k) = the k largest of the n_surv distinct non-zero keys in surv
// (LDS), descending, then zeros: each key's rank is the number of larger
// ones.  Ends with a barrier.
__device__ __forceinline__ void rank_survivors(const uint64_t *surv, int n_surv, int k, uint64_t *top)
{
    for (int s = threadIdx.x; s < n_surv; s += blockDim.x) {
        const uint64_t x = surv[s];
        int r = 0;
        for (int u = 0; u < n_surv && r < k; ++u) r += surv[u] > x ? 1 : 0;  // k or more: placed nowhere
        if (r < k) top[r] = x;
    }
    for (int i = n_surv + (int)threadIdx.x; i < k; i += blockDim.x) top[i] = 0;
    __syncthreads();
}

template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&keys)[N])
{
#pragma unroll
    for (int i = 1; i < N; ++i)
#pragma unroll
        for (int j = i; j > 0; --j)
            if (keys[j] > keys[j - 1]) {
                const uint64_t t = keys[j];
                keys[j] = keys[j - 1];
                keys[j - 1] = t;
            }
}

constexpr int kVocabPerThread = 8;     // candidates per thread of a partition
constexpr int kVocabThreads = 256;
constexpr int kVocabPart = kVocabPerThread * kVocabThreads;  // ids per partition
constexpr int kSelectThreads = 1024;   // also the most lists one merge takes
constexpr int kTopKMax = 64;
constexpr int kRecentMax = 32;
// 30*tanh(x/30) from the hardware exp and reciprocal is within this of the
// host libm's value (both are within a few 1e-6 of the true one); only
// candidates whose interval can reach the partition's k-th best get the
// exact evaluation.
constexpr float kSoftcapSlack = 1e-3f;

__device__ __forceinline__ float softcap_approx(float x)
{
    const float e = __expf(x * (2.0f / 30.0f));
    return 30.0f * (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f));
}

// top[0..k) = the k largest of the n_surv distinct keys in surv (LDS), which
// hold n_seg descending segments (segment j: seg_len[j] keys from
// seg_off[j]; surv_seg[s] = the segment of key s): a key's rank is its
// place in its own segment plus, for every other segment, the number of
// larger keys there (binary search).  Ends with a barrier.
__device__ __forceinline__ void rank_segments(const uint64_t *surv, const uint8_t *surv_seg, int n_surv,
                                              const int *seg_off, const int *seg_len, int n_seg, int k, uint64_t *top)
{
    for (int s = threadIdx.x; s < n_surv; s += blockDim.x) {
        const uint64_t x = surv[s];
        const int own = surv_seg[s];
        int r = s - seg_off[own];
        for (int j = 0; j < n_seg && r < k; ++j) {  // a rank of k or more places nowhere
            if (j == own) continue;
            const uint64_t *sj = surv + seg_off[j];
            const int len = seg_len[j];
            if (sj[len - 1] > x) {  // the whole segment is larger
                r += len;
                continue;
            }
            if (sj[0] < x) continue;  // the whole segment is smaller
            int lo = 0, hi = len;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (sj[mid] > x) lo = mid + 1;
                else hi = mid;
            }
            r += lo;
        }
        if (r < k) top[r] = x;
    }
    for (int i = n_surv + (int)threadIdx.x; i < k; i += blockDim.x) top[i] = 0;
    __syncthreads();
}

// LDS of merge_lists.
struct MergeShared {
    uint64_t heads[kSelectThreads];
    uint64_t surv[kTopKMax * kTopKMax];
    uint8_t surv_seg[kTopKMax * kTopKMax];
    int seg_off[kTopKMax], seg_len[kTopKMax], seg_list[kTopKMax];
    uint64_t red[kSelectThreads / 64];
    int n_surv, n_seg;
};

// The k largest keys (k <= 64) of n_lists descending lists of k keys at
// lists[i*k ..] (global), to top[0..k) in LDS.  k == 1: the maximum.  Else
// L = the k-th largest list head: exactly the k lists whose head is >= L
// (fewer when L is 0) hold the answer, so their keys >= L (at most k*k, a
// prefix of each) are ranked -- by counting when few, else per segment.
// n_lists <= blockDim.  Ends with a barrier.
__device__ __forceinline__ void merge_lists(const uint64_t *__restrict__ lists, int n_lists, int k, uint64_t *top,
                                            MergeShared &m)
{
    if (k == 1) {
        uint64_t b = 0;
        for (int t = threadIdx.x; t < n_lists; t += blockDim.x) b = lists[t] > b ? lists[t] : b;
        b = block_max(b, m.red);
        if (threadIdx.x == 0) top[0] = b;
        __syncthreads();
        return;
    }
    const int t = threadIdx.x;
    if (t == 0) {
        m.n_surv = 0;
        m.n_seg = 0;
    }
    m.heads[t] = t < n_lists ? lists[(size_t)t * k] : 0;
    __syncthreads();
    uint64_t L = kth_largest(m.heads, n_lists, k, (uint64_t)0, m.red);
    L = L ? L : 1;
    // the lists with a head >= L (at most k: the heads are distinct keys or 0)
    if (t < n_lists && m.heads[t] >= L) {
        const int sg = atomicAdd(&m.n_seg, 1);
        m.seg_list[sg] = t;
        m.seg_len[sg] = 0;
    }
    __syncthreads();
    // every key of those lists loaded at once, (segment, place) pairs over
    // the block; a list's keys >= L are a prefix of it (descending), so its
    // length is the largest place that passes, plus one
    const int ns = m.n_seg, npairs = ns * k;
    constexpr int kPairs = kTopKMax * kTopKMax / kSelectThreads;
    static_assert(kPairs * kSelectThreads == kTopKMax * kTopKMax, "whole pairs per thread");
    uint64_t pk[kPairs];
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const int q = t + i * kSelectThreads;
        pk[i] = q < npairs ? lists[(size_t)m.seg_list[q / k] * k + q % k] : 0;
    }
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const int q = t + i * kSelectThreads;
        if (q < npairs && pk[i] >= L) atomicMax(&m.seg_len[q / k], q % k + 1);
    }
    __syncthreads();
    if (t == 0) {
        int off = 0;
        for (int sg = 0; sg < ns; ++sg) {
            m.seg_off[sg] = off;
            off += m.seg_len[sg];
        }
        m.n_surv = off;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const int q = t + i * kSelectThreads, sg = q / k, j = q % k;
        if (q < npairs && j < m.seg_len[sg]) {
            m.surv[m.seg_off[sg] + j] = pk[i];
            m.surv_seg[m.seg_off[sg] + j] = (uint8_t)sg;
        }
    }
    __syncthreads();
    if (m.n_surv <= 4 * kTopKMax) rank_survivors(m.surv, m.n_surv, k, top);
    else rank_segments(m.surv, m.surv_seg, m.n_surv, m.seg_off, m.seg_len, m.n_seg, k, top);
}

// Where the scores of one vocabulary pick come from.  recent: the n_recent
// (<= 32) ids of a caller's list, or, with ring, the tokens of positions
// cur-31 .. cur from the ring of {position, token} entries (slot q % 32),
// cur being state[1] (the token state[0] is taken from the state itself)
// or host_cur.  With state, the generated count is cur - (prompt_len - 1).
struct VocabScoring {
    const float *logits;
    const uint8_t *valid;
    const int32_t *recent;
    const int2 *ring;
    const int32_t *state;
    long long host_cur;
    int vocab, n_recent, generated_count, prompt_len, scoring;
};

// Entry l (0..31) of the recent-token list, or -1.
__device__ __forceinline__ int recent_entry(const VocabScoring &v, int l)
{
    if (!v.ring) return l < v.n_recent ? v.recent[l] : -1;
    const long long cur = v.state ? (long long)v.state[1] : v.host_cur;
    if (v.state && l == 0) return v.state[0];
    const long long q = cur - l;
    if (q < 0) return -1;
    const int2 e = v.ring[q % kRecentMax];
    return e.x == (int)q ? e.y : -1;
}

// Block b scores chunk b % chunks (up to 2048 ids) of partition b / chunks,
// whose ids are [vocab*p/parts, vocab*(p+1)/parts) as in the reference's
// launch (kernels.rs:1100-1103), and writes its k best keys to keys_out[b*k..];
// with out_scores (chunks == 1), also the partition's (score, id) list, past
// the candidates (-inf, -1) (kernels.rs:1160-1167).
__global__ __launch_bounds__(kVocabThreads) void vocab_topk_partial_kernel(VocabScoring v, int parts, int chunks,
                                                                           int k, uint64_t *__restrict__ keys_out,
                                                                           float *__restrict__ out_scores,
                                                                           int32_t *__restrict__ out_ids)
{
    constexpr int N = kVocabPerThread;
    __shared__ int32_t rec[kRecentMax];
    __shared__ int n_rec, n_surv, n_cand;
    __shared__ float fred[kVocabThreads / 64], fvals[kVocabThreads];
    __shared__ float c_val[kVocabPart];
    __shared__ uint16_t c_meta[kVocabPart];
    __shared__ uint64_t c_key[kVocabPart];
    __shared__ uint64_t kred[kVocabThreads / 64], heads[kVocabThreads];
    __shared__ uint64_t surv[N * kTopKMax];
    __shared__ uint64_t top[kTopKMax];
    int gen = v.generated_count;
    if (v.state) {
        const long long cur = v.state[1];
        const long long first = v.prompt_len > 0 ? v.prompt_len - 1 : 0;
        gen = cur > first ? (int)(cur - first) : 0;
    }
    const int p = (int)blockIdx.x / chunks, c = (int)blockIdx.x % chunks;
    const int pa = (int)((long long)v.vocab * p / parts), pe = (int)((long long)v.vocab * (p + 1) / parts);
    const int start = pa + c * kVocabPart, end = min(start + kVocabPart, pe);
    // the logits and masks are loaded first: nothing below waits twice
    float x[N];
    bool cand[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int id = start + i * kVocabThreads + (int)threadIdx.x;
        cand[i] = id < end && !(gen < 4 && (id == 1 || id == 2 || id == 105 || id == 106));
        x[i] = v.logits[cand[i] ? id : pa];  // pa < pe <= vocab: in bounds for an empty chunk too
        if (v.valid) cand[i] = cand[i] && v.valid[cand[i] ? id : pa];
    }
    // the recent ids inside [start, end), compacted by wave 0
    if (threadIdx.x < 64) {
        const int id = threadIdx.x < kRecentMax ? recent_entry(v, threadIdx.x) : -1;
        const bool in = id >= start && id < end;
        const uint64_t m = __ballot(in);
        if (in) rec[__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] = id;
        if (threadIdx.x == 0) {
            n_rec = __popcll(m);
            n_surv = 0;
            n_cand = 0;
        }
    }
    __syncthreads();
    const int nr = n_rec;
    // scores: exact for the device path; for the CPU path an interval
    // [lo, hi] around 30*tanh(x/30) minus the penalty
    float lo[N], hi[N];
    bool pen[N];
    float mlo = -INFINITY;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int id = start + i * kVocabThreads + (int)threadIdx.x;
        pen[i] = false;
        if (v.scoring == 0) {
            for (int r = 0; r < nr; ++r)
                if (rec[r] == id) pen[i] = true;
            const float a = softcap_approx(x[i]);
            lo[i] = (a - kSoftcapSlack) - (pen[i] ? 3.5f : 0.0f);
            hi[i] = (a + kSoftcapSlack) - (pen[i] ? 3.5f : 0.0f);
        } else {
            float sc = x[i];
            for (int r = 0; r < nr; ++r)
                if (rec[r] == id) sc -= 1.8f;  // per occurrence, in list order
            lo[i] = hi[i] = sc;
        }
        if (!cand[i] || x[i] != x[i]) {
            cand[i] = false;
            lo[i] = -INFINITY;
        }
        mlo = lo[i] > mlo ? lo[i] : mlo;
    }
    // T: a lower bound of the partition's k-th best score (the k-th largest
    // per-thread best lower end); only candidates with hi >= T can place.
    // They are compacted (element, value, penalty) for one exact pass.
    float T;
    if (k == 1) {
        T = block_max(mlo, fred);
    } else {
        fvals[threadIdx.x] = mlo;
        __syncthreads();
        T = kth_largest(fvals, kVocabThreads, k, -INFINITY, fred);
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (cand[i] && hi[i] >= T) {
            const int slot = atomicAdd(&n_cand, 1);
            c_val[slot] = v.scoring == 0 ? x[i] : lo[i];
            c_meta[slot] = (uint16_t)((i * kVocabThreads + (int)threadIdx.x) | (pen[i] ? 0x8000 : 0));
        }
    __syncthreads();
    const int nc = n_cand;
#pragma unroll 1
    for (int s = threadIdx.x; s < nc; s += kVocabThreads) {
        const int e = c_meta[s] & 0x7fff, id = start + e;
        float sc = c_val[s];
        if (v.scoring == 0) {  // the CPU path's exact score
            sc = 30.0f * mrml_libm::tanhf(sc / 30.0f);
            if (c_meta[s] & 0x8000) sc -= 3.5f;
        }
        c_key[s] = sc == sc ? cand_key(sc, id) : 0;
    }
    __syncthreads();
    uint64_t keys[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int s = i * kVocabThreads + (int)threadIdx.x;
        keys[i] = s < nc ? c_key[s] : 0;
    }
    if (k == 1) {
        uint64_t b = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) b = keys[i] > b ? keys[i] : b;
        b = block_max(b, kred);
        if (threadIdx.x == 0) top[0] = b;
        __syncthreads();
    } else {
        // exact top k: L = the k-th largest per-thread best key; the k
        // threads at or above it hold every answer (at most 8k keys >= L)
        sort_desc(keys);
        heads[threadIdx.x] = keys[0];
        __syncthreads();
        uint64_t L = kth_largest(heads, kVocabThreads, k, (uint64_t)0, kred);
        L = L ? L : 1;
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (keys[i] >= L) surv[atomicAdd(&n_surv, 1)] = keys[i];
        __syncthreads();
        rank_survivors(surv, n_surv, k, top);
    }
    for (int r = threadIdx.x; r < k; r += blockDim.x) {
        const uint64_t key = top[r];
        keys_out[(size_t)blockIdx.x * k + r] = key;
        if (out_scores) {
            out_scores[(size_t)p * k + r] = key ? key_score(key) : -INFINITY;
            out_ids[(size_t)p * k + r] = key ? key_id(key) : -1;
        }
    }
}

// Partition blockIdx.x's k best from its chunks' lists (partitions of more
// than 2048 ids: the reference's serial kernel, kernels.rs:1170-1228).
__global__ __launch_bounds__(kSelectThreads) void vocab_topk_merge_kernel(const uint64_t *__restrict__ keys_in,
                                                                         int chunks, int k,
                                                                         float *__restrict__ out_scores,
                                                                         int32_t *__restrict__ out_ids)
{
    __shared__ MergeShared ms;
    __shared__ uint64_t top[kTopKMax];
    merge_lists(keys_in + (size_t)blockIdx.x * chunks * k, chunks, k, top, ms);
    for (int r = threadIdx.x; r < k; r += blockDim.x) {
        const uint64_t key = top[r];
        out_scores[(size_t)blockIdx.x * k + r] = key ? key_score(key) : -INFINITY;
        out_ids[(size_t)blockIdx.x * k + r] = key ? key_id(key) : -1;
    }
}

// Merges the partitions' keys into the k best (descending) and picks the
// token: temperature <= 0 -> the first; else the softmax draw of the CPU path
// with its LCG (the exponentials in parallel, the sums in the reference's
// order).  Writes out_token (nullable), out_scores / out_ids (nullable, k
// entries, -inf / -1 past the candidates) and, with state, advances the
// decode loop as argmax_final_kernel does and records {pos, token} in ring.
__global__ __launch_bounds__(kSelectThreads) void vocab_select_kernel(
    const uint64_t *__restrict__ part, int n_part, int k, float temperature, unsigned long long pos_arg,
    int expf_fused, int32_t *__restrict__ out_token, float *__restrict__ out_scores, int32_t *__restrict__ out_ids,
    int32_t *__restrict__ state, int2 *__restrict__ ring, int32_t *__restrict__ hist, int hist_cap,
    const int32_t *__restrict__ prompt, int prompt_len)
{
    __shared__ MergeShared ms;
    __shared__ uint64_t top[kTopKMax];
    __shared__ float probs[kTopKMax], quot[kTopKMax];
    merge_lists(part, n_part, k, top, ms);
    const int t = threadIdx.x;
    int n = 0;
    for (int i = 0; i < k; ++i) n += top[i] != 0 ? 1 : 0;  // the candidates lead, zeros follow
    // the CPU path's state.pos: the position after the token just processed
    const unsigned long long pos = state ? (unsigned long long)state[1] + 1ull : pos_arg;
    const bool draw = n > 0 && temperature > 0.0f;
    if (draw) {
        const float s0 = key_score(top[0]);
        const float temp = temperature > 0.1f ? temperature : 0.1f;
        if (t < n) probs[t] = mrml_libm::expf((key_score(top[t]) - s0) / temp, expf_fused != 0);
        __syncthreads();
        if (t < n) {
            float sum_exp = 0.0f;
            for (int i = 0; i < n; ++i) sum_exp += probs[i];
            quot[t] = probs[t] / sum_exp;
        }
        __syncthreads();
    }
    if (t != 0) return;
    if (out_scores || out_ids)
        for (int i = 0; i < k; ++i) {
            if (out_scores) out_scores[i] = i < n ? key_score(top[i]) : -INFINITY;
            if (out_ids) out_ids[i] = i < n ? key_id(top[i]) : -1;
        }
    int token = n ? key_id(top[0]) : 506;
    if (draw) {
        float sum_exp = 0.0f;
        for (int i = 0; i < n; ++i) sum_exp += probs[i];
        if (sum_exp > 0.0f) {
            const float rng = (float)((pos * 6364136223846793005ull + 1ull) >> 33) / (float)0xffffffffu;
            float acc = 0.0f;
            for (int i = 0; i < n; ++i) {
                acc += quot[i];
                if (rng <= acc) {
                    token = key_id(top[i]);
                    break;
                }
            }
        }
    }
    if (out_token) *out_token = token;
    if (state) {
        const int cur = state[1];
        if (ring && cur >= 0) ring[cur % kRecentMax] = make_int2(cur, state[0]);  // the token processed at cur
        if (hist && cur >= 0 && cur < hist_cap) hist[cur] = token;
        const int next = cur + 1;
        state[0] = (prompt && next < prompt_len) ? prompt[next] : token;
        state[1] = next;
    }
}

// The ring entries of positions pos0 .. pos0+n-1 (the last 32 of them) for
// tokens[0..n): the recent-token history of a batched prefill.
__global__ void recent_ring_write_kernel(int2 *__restrict__ ring, const int32_t *__restrict__ tokens, int n, int pos0)
{
    const int i = n - 1 - (int)threadIdx.x;
    if (threadIdx.x < kRecentMax && i >= 0) ring[(pos0 + i) % kRecentMax] = make_int2(pos0 + i, tokens[i]);
}

inline int waves_for(int rows) { return rows >= 8192 ? 4 : (rows >= 2048 ? 2 : 1); }

// The smallest compiled iteration count >= iters (iterations past a row's
// last block are masked, so a larger instance gives the same result), or 0.
inline int iters_instance(int iters)
{
    static const int kInst[] = {1, 2, 3, 4, 5, 6, 8, 9, 12, 16, 18, 20};
    for (int v : kInst)
        if (v >= iters) return v;
    return 0;
}

#define MRML_DISPATCH_WAVES(WAVES_VAL, BODY)                 \
    switch (WAVES_VAL) {                                     \
    case 1: { constexpr int WV = 1; BODY; } break;           \
    case 2: { constexpr int WV = 2; BODY; } break;           \
    default: { constexpr int WV = 4; BODY; } break;          \
    }

}  // namespace

int launch_gemv_q8_0(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols,
                     int32_t softcap)
{
    const int nb = cols / 32;
    const bool odd = (((int64_t)rows * nb) & 1) != 0;
    const int iters = (nb + 15) / 16;
    const int waves = waves_for(rows);
    const dim3 grid(((rows + 3) / 4 + waves - 1) / waves);
    const size_t lds = act_pack_bytes(nb);
#define Q8_CASE(N)                                                                                           \
    case N:                                                                                                  \
        MRML_DISPATCH_WAVES(waves, {                                                                         \
            if (odd)                                                                                         \
                hipLaunchKernelGGL((gemv_q8_0_kernel<N, WV, true>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,   \
                                   (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb, softcap);       \
            else                                                                                             \
                hipLaunchKernelGGL((gemv_q8_0_kernel<N, WV, false>), grid, dim3(64 * (WV + 1)), lds, ctx->stream,  \
                                   (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nb, softcap);       \
        });                                                                                                  \
        break;
    switch (iters_instance(iters)) {
        Q8_CASE(1) Q8_CASE(2) Q8_CASE(3) Q8_CASE(4) Q8_CASE(5) Q8_CASE(6) Q8_CASE(8) Q8_CASE(9)
        Q8_CASE(12) Q8_CASE(16) Q8_CASE(18) Q8_CASE(20)
    default:
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q8_0 matvec: cols=%d has no kernel instance", cols);
    }
#undef Q8_CASE
    return check_launch(ctx, "gemv_q8_0_kernel");
}

int launch_gemv_q4_k(mrml_hip_ctx *ctx, const void *w, const void *xpack, float *y, int32_t rows, int32_t cols)
{
    const int nsb = cols / 256, nb = nsb * 8;
    const int iters = (nb + 15) / 16;
    if (nb > kStageMax)
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q4_k matvec: cols=%d above %d", cols, kStageMax * 32);
    // compute waves per workgroup (4 rows each); 8 waves of 32 rows with one
    // fold lane per row measured slower at the 256000-row head (57.4 against
    // 51.8 us for 4 waves)
    const int waves = waves_for(rows);
    const dim3 grid((rows + 4 * waves - 1) / (4 * waves));
#define QK_CASE(N)                                                                                           \
    case N:                                                                                                  \
        switch (waves) {                                                                                     \
        case 1: hipLaunchKernelGGL((gemv_q4_k_kernel<N, 1>), grid, dim3(64 * 2), q4k_lds<N>(nb, 1),            \
                                   ctx->stream, (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nsb); break; \
        case 2: hipLaunchKernelGGL((gemv_q4_k_kernel<N, 2>), grid, dim3(64 * 3), q4k_lds<N>(nb, 2),            \
                                   ctx->stream, (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nsb); break; \
        default: hipLaunchKernelGGL((gemv_q4_k_kernel<N, 4>), grid, dim3(64 * 5), q4k_lds<N>(nb, 4),           \
                                    ctx->stream, (const uint8_t *)w, (const uint8_t *)xpack, y, rows, nsb); break; \
        }                                                                                                    \
        break;
    switch (iters_instance(iters)) {
        QK_CASE(1) QK_CASE(2) QK_CASE(3) QK_CASE(4) QK_CASE(5) QK_CASE(6) QK_CASE(8) QK_CASE(9) QK_CASE(12)
        QK_CASE(16) QK_CASE(18) QK_CASE(20)
    default:
        return fail(ctx, MRML_HIP_E_UNSUPPORTED, "q4_k matvec: cols=%d has no kernel instance", cols);
    }
#undef QK_CASE
    return check_launch(ctx, "gemv_q4_k_kernel");
}

int vocab_parts(int32_t vocab) { return (vocab + kVocabPart - 1) / kVocabPart; }

size_t vocab_select_scratch_bytes(int32_t vocab, int32_t k) { return (size_t)vocab_parts(vocab) * k * 8; }

bool vocab_select_ok(int32_t vocab, int32_t k)
{
    return vocab > 0 && k >= 1 && k <= kTopKMax && vocab_parts(vocab) <= kSelectThreads;
}

int vocab_topk_chunks(int32_t vocab, int32_t parts)
{
    const long long most = ((long long)vocab + parts - 1) / parts;  // the largest partition's ids
    return (int)((most + kVocabPart - 1) / kVocabPart);
}

bool vocab_topk_ok(int32_t vocab, int32_t k, int32_t parts)
{
    return vocab > 0 && parts >= 1 && parts <= vocab && k >= 1 && k <= kTopKMax &&
           vocab_topk_chunks(vocab, parts) <= kSelectThreads;
}

size_t vocab_topk_scratch_bytes(int32_t vocab, int32_t k, int32_t parts)
{
    return (size_t)parts * vocab_topk_chunks(vocab, parts) * k * 8;
}

namespace {
VocabScoring scoring_of(const float *logits, int32_t vocab, const uint8_t *valid, const int32_t *recent,
                        int32_t n_recent, int32_t generated_count, int32_t scoring, const int32_t *state,
                        const void *ring, long long host_cur, int prompt_len)
{
    VocabScoring v;
    v.logits = logits;
    v.valid = valid;
    v.recent = recent;
    v.ring = (const int2 *)ring;
    v.state = state;
    v.host_cur = host_cur;
    v.vocab = vocab;
    v.n_recent = n_recent;
    v.generated_count = generated_count;
    v.prompt_len = prompt_len;
    v.scoring = scoring;
    return v;
}
}  // namespace

size_t recent_ring_bytes() { return kRecentMax * sizeof(int2); }

int launch_recent_ring_write(mrml_hip_ctx *ctx, void *ring, const int32_t *tokens, int n, int pos0)
{
    hipLaunchKernelGGL(recent_ring_write_kernel, dim3(1), dim3(kRecentMax), 0, ctx->stream, (int2 *)ring, tokens, n,
                       pos0);
    return check_launch(ctx, "recent_ring_write_kernel");
}

int launch_vocab_topk(mrml_hip_ctx *ctx, const float *logits, const uint8_t *valid, const int32_t *recent,
                      float *out_scores, int32_t *out_ids, int32_t vocab, int32_t n_recent, int32_t generated_count,
                      int32_t k, int32_t parts, void *scratch)
{
    const int chunks = vocab_topk_chunks(vocab, parts);
    const VocabScoring v = scoring_of(logits, vocab, valid, recent, n_recent, generated_count, 1, nullptr, nullptr, 0, 0);
    uint64_t *keys = reinterpret_cast<uint64_t *>(scratch);
    hipLaunchKernelGGL(vocab_topk_partial_kernel, dim3(parts * chunks), dim3(kVocabThreads), 0, ctx->stream, v, parts,
                       chunks, k, keys, chunks == 1 ? out_scores : nullptr, chunks == 1 ? out_ids : nullptr);
    if (int rc = check_launch(ctx, "vocab_topk_partial_kernel")) return rc;
    if (chunks == 1) return MRML_HIP_OK;
    hipLaunchKernelGGL(vocab_topk_merge_kernel, dim3(parts), dim3(kSelectThreads), 0, ctx->stream,
                       (const uint64_t *)keys, chunks, k, out_scores, out_ids);
    return check_launch(ctx, "vocab_topk_merge_kernel");
}

int launch_vocab_select(mrml_hip_ctx *ctx, const float *logits, int32_t vocab, const uint8_t *valid,
                        const int32_t *recent, int32_t n_recent, int32_t generated_count, int32_t scoring,
                        float temperature, uint64_t pos, int32_t k, int32_t *out_token, float *out_scores,
                        int32_t *out_ids, void *scratch, int32_t *state, void *ring, long long host_cur, int32_t *hist,
                        int hist_cap, const int32_t *prompt, int prompt_len)
{
    const int parts = vocab_parts(vocab);
    const VocabScoring v = scoring_of(logits, vocab, valid, recent, n_recent, generated_count, scoring, state, ring,
                                      host_cur, prompt_len);
    uint64_t *keys = reinterpret_cast<uint64_t *>(scratch);
    hipLaunchKernelGGL(vocab_topk_partial_kernel, dim3(parts), dim3(kVocabThreads), 0, ctx->stream, v, parts, 1, k,
                       keys, nullptr, nullptr);
    if (int rc = check_launch(ctx, "vocab_topk_partial_kernel")) return rc;
    hipLaunchKernelGGL(vocab_select_kernel, dim3(1), dim3(kSelectThreads), 0, ctx->stream, (const uint64_t *)keys,
                       parts, k, temperature, (unsigned long long)pos, (int)host_expf_fused(), out_token, out_scores,
                       out_ids, state, (int2 *)ring, hist, hist_cap, prompt, prompt_len);
    return check_launch(ctx, "vocab_select_kernel");
}

int argmax_parts(int32_t n)
{
    const int parts = (n + 2047) / 2048;
    return parts > 1024 ? 1024 : parts;
}

int launch_argmax_step(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out, void *scratch, int32_t *state,
                       int32_t *hist, int hist_cap, const int32_t *prompt, int prompt_len, void *ring)
{
    const int parts = argmax_parts(n);
    float *pv = reinterpret_cast<float *>(scratch);
    int *pi = reinterpret_cast<int *>(reinterpret_cast<uint8_t *>(scratch) + (size_t)parts * 4);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(256), 0, ctx->stream, x, n, pv, pi);
    int rc = check_launch(ctx, "argmax_partial_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, ctx->stream, pv, pi, parts, out, state, hist,
                       hist_cap, prompt, prompt_len, (int2 *)ring);
    return check_launch(ctx, "argmax_final_kernel");
}

int launch_argmax_f32(mrml_hip_ctx *ctx, const float *x, int32_t n, int32_t *out)
{
    void *ws = workspace(ctx, (size_t)argmax_parts(n) * 8);
    if (!ws) return MRML_HIP_E_ALLOC;
    return launch_argmax_step(ctx, x, n, out, ws, nullptr, nullptr, 0, nullptr, 0, nullptr);
}

}  // namespace mrml
