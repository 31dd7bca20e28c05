// exact_sum.h -- the sequential f32 sum of non-negative terms, evaluated in
// parallel with the same result bit for bit.
//
// The reference sums squares (RMSNorm, ops.rs:24-79) and softmax terms
// (ops.rs:133-158) in a loop: s = 0; s = RN(s + a_k), k = 0..n-1.  A single
// GPU lane doing that costs one dependent add (plus operand traffic) per
// term.  For a_k >= 0 the loop can be compressed exactly:
//
//  * While s stays in one binade [2^e, 2^(e+1)) the representable values
//    are the multiples of u = 2^(e-23), so RN(s + a_k) = s + u * RNI(a_k/u)
//    (round to nearest integer), where only an exact tie (a_k/u = n + 1/2)
//    depends on s (its parity).  Steps that provably start and end in the
//    same binade and are not ties therefore each add a fixed integer number
//    of ulps, and a run of them adds u * (sum of those integers) -- an
//    exactly representable amount, so one f32 add reproduces the whole run.
//  * "Provably" uses approximate prefix sums P_k (any summation order): the
//    sequential s_k satisfies |s_k - P_k| <= (k+1) 2^-24 s_k (each rounding
//    errs by at most 2^-24 relative and s is non-decreasing), and a tree of
//    depth D adds at most D 2^-24 relative error to P_k; a step is classed
//    safe when P_{k-1} and P_k clear the binade boundaries by twice that.
//  * Every other step (the first, crossings of a binade boundary, ties,
//    s near 0) stays an event of its own, s = RN(s + a_k).
//
// So the sum becomes a short sequential f32 sum over events (each run's exact
// addend, each unsafe term) whose result equals the original loop's.  The
// classification is per term and order-free; only the ~tens of events are
// added in sequence.  Functions are host+device so the host tests can run
// the same classification against the plain loop.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MRML_XS_HD __host__ __device__ __forceinline__
#else
#define MRML_XS_HD static inline
#endif

namespace mrml_xsum {

MRML_XS_HD float pow2f(int e)  // 2^e for -126 <= e <= 127
{
    return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
}

// Depth allowance of the approximate prefix sums (terms per thread plus the
// scan levels of a workgroup of up to 1024 threads): P_k is within
// kDepth * 2^-24 of the exact prefix sum, relatively.
constexpr int kDepth = 64;

struct Step {
    int safe;   // 1: the step adds exactly inc * u
    int inc;    // integer number of ulps added
    float u;    // ulp of the binade the step stays in
};

// Twice the relative error bound of the approximate prefix sums up to term
// k: the classification's margin.  A term may be classed with the margin of
// a later k (a larger margin only classes more steps unsafe); 1 - rho and
// 1 + rho are exact floats for k < 2^22.
MRML_XS_HD float margin(int k) { return (float)(2 * (k + 1 + kDepth)) * 0x1p-24f; }

// Classify step k (a = a_k >= 0 finite, pm ~ P_{k-1}, pk ~ P_k; first: k == 0)
// with omr = 1 - rho, opr = 1 + rho for a margin rho >= margin(k).  The
// powers of two come from the exponent field of P_{k-1}: 2^e, 2^(e+1), the
// ulp 2^(e-23) and its inverse 2^(23-e).  Written without early returns: on
// the GPU the lanes of a wave evaluate it in step.
MRML_XS_HD Step classify(float a, float pm, float pk, bool first, float omr, float opr)
{
    const bool in_range = !first && pm >= 0x1p-100f && pk < 0x1p+120f;
    const uint32_t lob = __builtin_bit_cast(uint32_t, in_range ? pm : 1.0f) & 0x7f800000u;  // keeps e in range
    const float lo = __builtin_bit_cast(float, lob);                  // 2^e
    const float hi = __builtin_bit_cast(float, lob + 0x00800000u);    // 2^(e+1)
    const float u = __builtin_bit_cast(float, lob - 0x0b800000u);     // 2^(e-23): exponent field minus 23
    const float iu = __builtin_bit_cast(float, 0x8a800000u - lob);    // 2^(23-e): field 277 - (e+127)
    const bool starts_in = pm * omr >= lo;       // s_{k-1} surely >= 2^e
    const bool ends_in = pk * opr + u < hi;      // s_{k-1} + a_k surely < 2^(e+1) - u
    const float q = a * iu;                      // exact when safe: a < 2^(e+1)
    const float r = __builtin_floorf(q);
    const float f = q - r;                       // exact
    Step st;
    st.safe = (in_range && starts_in && ends_in && f != 0.5f) ? 1 : 0;  // a tie depends on s's parity
    st.inc = st.safe ? (int)r + (f > 0.5f ? 1 : 0) : 0;
    st.u = u;
    return st;
}

MRML_XS_HD Step classify(float a, float pm, float pk, int k)
{
    const float rho = margin(k);
    return classify(a, pm, pk, k == 0, 1.0f - rho, 1.0f + rho);
}

#if defined(__HIPCC__)

// ---- workgroup implementation ---------------------------------------------------

constexpr int kMaxPerThread = 16;  // terms per thread (n <= 16 * blockDim)
constexpr int kEventCap = 512;     // events held in LDS; more falls back to the plain loop

// LDS of one call: n bytes of flags plus this struct (16-byte aligned).
struct Shared {
    float add[kEventCap];  // event addends, in order
    float u[kEventCap];    // ulp of a run (0 for a single term)
    int Rs[kEventCap];     // a run's ulp prefix before its first term
    int Re[kEventCap];     // a run's ulp prefix after its last term
    float wtot[16];        // per-wave totals of the approximate prefix scan
    int wcnt[16];          // per-wave event counts
    int winc[16];          // per-wave sums of the safe terms' ulp counts
    float result;
};

// Inclusive scans over the 64 lanes of a wave with DPP: row_shr 1, 2, 4, 8
// within each 16-lane row (lanes shifted in from outside the row read 0),
// then row_bcast 15 and 31 carry row totals into the following rows.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i32(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, true);
}

__device__ __forceinline__ int wave_incl_scan_i32(int v)
{
    v += dpp_i32<0x111, 0xf>(v);  // row_shr:1
    v += dpp_i32<0x112, 0xf>(v);  // row_shr:2
    v += dpp_i32<0x114, 0xf>(v);  // row_shr:4
    v += dpp_i32<0x118, 0xf>(v);  // row_shr:8
    v += dpp_i32<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_i32<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float v)
{
    return __builtin_bit_cast(float, dpp_i32<CTRL, ROW_MASK>(__builtin_bit_cast(int, v)));
}

__device__ __forceinline__ float wave_incl_scan_f32(float v)
{
    v += dpp_f32<0x111, 0xf>(v);
    v += dpp_f32<0x112, 0xf>(v);
    v += dpp_f32<0x114, 0xf>(v);
    v += dpp_f32<0x118, 0xf>(v);
    v += dpp_f32<0x142, 0xa>(v);
    v += dpp_f32<0x143, 0xc>(v);
    return v;
}

// s = 0; s = RN(s + a[k]) for k = 0..n-1 over a[] in LDS (a[k] >= 0, finite),
// computed by the whole workgroup (blockDim a multiple of 64, at most 1024,
// n <= kMaxPerThread * blockDim).  flags: n bytes of LDS.  Returns the
// result in every thread; ends with a barrier, so a and x may be reused.
__device__ float block_seq_sum_nonneg(const float *a, int n, uint8_t *flags, Shared &x)
{
    const int nt = blockDim.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int C = (n + nt - 1) / nt;
    const int k0 = tid * C;
    // approximate prefix sums: thread-local sequential, then the block scan
    float av[kMaxPerThread], lp[kMaxPerThread];
    float run = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerThread; ++i) {
        av[i] = 0.0f;
        if (i < C) {
            const int k = k0 + i;
            av[i] = k < n ? a[k] : 0.0f;
            run += av[i];
            lp[i] = run;
        }
    }
    const float wincl = wave_incl_scan_f32(run);
    if (lane == 63) x.wtot[wave] = wincl;
    __syncthreads();
    // exclusive prefix from the previous lane's inclusive one (wincl - run
    // would lose the relative accuracy the classification relies on)
    float base = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, wincl), 0x138,
                                                                        0xf, 0xf, true));  // wave_shr:1
    for (int w = 0; w < wave; ++w) base += x.wtot[w];
    // classify each term, flag the unsafe ones
    int inc[kMaxPerThread];  // ulps added by a safe term, -1 for an unsafe one
    float uu[kMaxPerThread];
    int my_inc = 0;
#pragma unroll
    for (int i = 0; i < kMaxPerThread; ++i) {
        inc[i] = -1;
        uu[i] = 0.0f;
        if (i < C) {
            const int k = k0 + i;
            if (k < n) {
                const float pm = i ? base + lp[i - 1] : base;
                const Step st = classify(av[i], pm, base + lp[i], k);
                inc[i] = st.safe ? st.inc : -1;
                uu[i] = st.u;
                flags[k] = st.safe ? 0 : 1;
                my_inc += st.safe ? st.inc : 0;
            }
        }
    }
    __syncthreads();
    // events: every unsafe term, and every safe term that follows an unsafe
    // one; with the running count of safe ulps, a run's total is its end
    // prefix minus its start prefix
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < kMaxPerThread; ++i) {
        const int k = k0 + i;
        if (i < C && k < n && (flags[k] || k == 0 || flags[k - 1])) ++cnt;
    }
    const int cincl = wave_incl_scan_i32(cnt);
    const int iincl = wave_incl_scan_i32(my_inc);
    if (lane == 63) {
        x.wcnt[wave] = cincl;
        x.winc[wave] = iincl;
    }
    __syncthreads();
    int ebase = cincl - cnt, ibase = iincl - my_inc, nev = 0;
    for (int w = 0; w < nw; ++w) {
        if (w < wave) {
            ebase += x.wcnt[w];
            ibase += x.winc[w];
        }
        nev += x.wcnt[w];
    }
    if (nev > kEventCap) {
        // too many events for LDS (e.g. many exact ties): the plain loop
        if (tid < 64) {
            float s = 0.0f;
            for (int k = 0; k < n; ++k) s += a[k];
            if (tid == 0) x.result = s;
        }
        __syncthreads();
        const float r = x.result;
        __syncthreads();
        return r;
    }
    int E = ebase - 1, pre = ibase;
#pragma unroll
    for (int i = 0; i < kMaxPerThread; ++i) {
        const int k = k0 + i;
        if (i < C && k < n) {
            const bool start = flags[k] || k == 0 || flags[k - 1];
            const bool last = k == n - 1 || flags[k + 1];  // the next term starts an event
            if (start) ++E;
            if (inc[i] < 0) {
                x.add[E] = av[i];
                x.u[E] = 0.0f;
            } else {
                if (start) {
                    x.u[E] = uu[i];
                    x.Rs[E] = pre;  // each run has one first and one last term
                }
                pre += inc[i];
                if (last) x.Re[E] = pre;
            }
        }
    }
    __syncthreads();
    for (int j = tid; j < nev; j += nt)
        if (x.u[j] > 0.0f) x.add[j] = (float)(x.Re[j] - x.Rs[j]) * x.u[j];  // exact: < 2^24 ulps, u a power of 2
    __syncthreads();
    if (tid < 64) {
        float s = 0.0f;
        int j = 0;
        for (; j + 8 <= nev; j += 8) {
            float4 b0 = *reinterpret_cast<const float4 *>(&x.add[j]);
            float4 b1 = *reinterpret_cast<const float4 *>(&x.add[j + 4]);
            s += b0.x;
            s += b0.y;
            s += b0.z;
            s += b0.w;
            s += b1.x;
            s += b1.y;
            s += b1.z;
            s += b1.w;
        }
        for (; j < nev; ++j) s += x.add[j];
        if (tid == 0) x.result = s;
    }
    __syncthreads();
    const float r = x.result;
    __syncthreads();
    return r;
}

// The same sum when thread t holds terms 4t..4t+3 in registers (n <= 4 *
// blockDim; terms at or past n are ignored) -- the layout of the norm
// kernels.  Each wave forms the events of its own 256 terms: its first term
// always starts an event and its last always ends one (splitting a run of
// exact steps keeps every partial sum exact), so no flag or ulp count
// crosses a wave.  Each event is written by one term: an unsafe term writes
// its value, a run's last term writes (Re - Rs) * u, where Rs (the wave's
// ulp prefix before the run's first term) reaches it by a max-scan (the
// prefix never decreases).  The prefix stays below 2^31: the safe steps in
// one binade add fewer than 2^23 ulps, and s visits each binade once.
// The events land in block order after the waves' counts are exchanged
// (each lane's event stores unconditional: a lane with no event writes the
// trash word); every wave then adds them itself, the same adds in the same
// order, with operands from broadcast LDS reads (a register chain: v_readlane
// operands would cost several times more per add), so no barrier broadcasts
// the result.  Three barriers, all LDS-only (pending global stores are not
// waited for).  A following call may reuse x at once (its writes to the list
// come after its second barrier); other LDS the caller reuses needs the
// caller's own barrier.
constexpr int kPadEvents = 32;  // zeros after the last event (the walk reads groups of 32)

struct Shared4 {
    float ev[16 * 256 + kPadEvents];  // event addends in order (at most one per term)
    float wtot[16];                   // per-wave totals of the approximate prefix scan
    int wcnt[16];                     // per-wave event counts
    float trash;                      // target of the event stores of lanes that have no event
};

__device__ __forceinline__ void lds_barrier()  // s_barrier after this wave's LDS accesses
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ int wave_shr1_i32(int v)  // lane l gets lane l-1 (lane 0: 0)
{
    return __builtin_amdgcn_update_dpp(0, v, 0x138, 0xf, 0xf, true);
}
__device__ __forceinline__ int wave_shl1_i32(int v)  // lane l gets lane l+1 (lane 63: 0)
{
    return __builtin_amdgcn_update_dpp(0, v, 0x130, 0xf, 0xf, true);
}

// inclusive max-scan over the wave (the same DPP steps as the sums above)
__device__ __forceinline__ uint32_t wave_incl_max_u32(uint32_t v)
{
    auto mx = [](uint32_t a, int b) { return a > (uint32_t)b ? a : (uint32_t)b; };
    v = mx(v, dpp_i32<0x111, 0xf>((int)v));
    v = mx(v, dpp_i32<0x112, 0xf>((int)v));
    v = mx(v, dpp_i32<0x114, 0xf>((int)v));
    v = mx(v, dpp_i32<0x118, 0xf>((int)v));
    v = mx(v, dpp_i32<0x142, 0xa>((int)v));
    v = mx(v, dpp_i32<0x143, 0xc>((int)v));
    return v;
}

// inclusive scans within each 16-lane row (row 0 carries the per-wave values)
__device__ __forceinline__ int row_incl_scan_i32(int v)
{
    v += dpp_i32<0x111, 0xf>(v);
    v += dpp_i32<0x112, 0xf>(v);
    v += dpp_i32<0x114, 0xf>(v);
    v += dpp_i32<0x118, 0xf>(v);
    return v;
}
__device__ __forceinline__ float row_incl_scan_f32(float v)
{
    v += dpp_f32<0x111, 0xf>(v);
    v += dpp_f32<0x112, 0xf>(v);
    v += dpp_f32<0x114, 0xf>(v);
    v += dpp_f32<0x118, 0xf>(v);
    return v;
}

__device__ __forceinline__ float readlane_f32(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float block_seq_sum_nonneg4(float4 v, int n, Shared4 &x)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int k0 = 4 * tid;
    const int wv = __builtin_amdgcn_readfirstlane(wave);  // uniform: the readlane index
    // (a wave past n has no terms and no events; it runs the same steps)
    float a[4] = {v.x, v.y, v.z, v.w};
    float lp[4], run = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = k0 + i < n ? a[i] : 0.0f;
        run += a[i];
        lp[i] = run;
    }
    // approximate prefix: thread-local, wave scan, earlier waves' totals
    const float wincl = wave_incl_scan_f32(run);
    if (lane == 63) x.wtot[wave] = wincl;
    lds_barrier();
    const float wt = lane < wave ? x.wtot[lane] : 0.0f;  // lane < wave <= 15: row 0
    const float base =
        __builtin_bit_cast(float, wave_shr1_i32(__builtin_bit_cast(int, wincl))) + readlane_f32(row_incl_scan_f32(wt), 15);
    // classify; unsafe: bit i set for an unsafe term, stop: unsafe or past n
    uint32_t inc[4], my_inc = 0;
    float uu[4];
    int unsafe = 0, stop = 0;
    const float rho = margin(k0 + 3), omr = 1.0f - rho, opr = 1.0f + rho;  // the thread's last term's margin
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = k0 + i;
        const Step st = classify(a[i], i ? base + lp[i - 1] : base, base + lp[i], k == 0, omr, opr);
        const bool in = k < n;
        inc[i] = (in && st.safe) ? (uint32_t)st.inc : 0u;
        uu[i] = st.u;
        unsafe |= (in && !st.safe) ? (1 << i) : 0;
        stop |= (!in || !st.safe) ? (1 << i) : 0;
        my_inc += inc[i];
    }
    // event starts: an unsafe term, a term after an unsafe one, the wave's
    // first term; run ends: a safe term before a stop, the wave's last term
    const int pv = wave_shr1_i32(unsafe), nx = wave_shl1_i32(stop);  // every lane takes part
    const int prev = lane == 0 ? 8 : pv, next = lane == 63 ? 1 : nx;
    int starts = 0, ends = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool in = k0 + i < n, uns = (unsafe >> i) & 1;
        const bool before = i ? (unsafe >> (i - 1)) & 1 : (prev >> 3) & 1;
        const bool after = i < 3 ? (stop >> (i + 1)) & 1 : next & 1;
        starts |= (in && (uns || before)) ? (1 << i) : 0;
        ends |= (in && !uns && after) ? (1 << i) : 0;
    }
    const int cnt = __builtin_popcount(starts);
    const int cincl = wave_incl_scan_i32(cnt);
    const uint32_t iincl = (uint32_t)wave_incl_scan_i32((int)my_inc);
    // Rs of this thread's latest run start, max-scanned over the wave
    uint32_t r = iincl - my_inc, mine = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (((starts & ~unsafe) >> i) & 1) mine = r;
        r += inc[i];
    }
    uint32_t rs = (uint32_t)wave_shr1_i32((int)wave_incl_max_u32(mine));
    if (lane == 63) x.wcnt[wave] = cincl;
    lds_barrier();
    // this wave's offset in the block's list, and the list's length
    const int cw = lane < nw ? x.wcnt[lane] : 0;  // row 0
    const int ci = row_incl_scan_i32(cw);
    const int nev = __builtin_amdgcn_readlane(ci, 15);
    const int goff = wv ? __builtin_amdgcn_readlane(ci, wv - 1) : 0;
    float *const trash = &x.trash;
    {
        float *pz = (wave == 0 && lane < kPadEvents) ? x.ev + nev + lane : trash;
        *pz = 0.0f;
    }
    float *ev = x.ev + goff;
    int e = cincl - cnt;  // events started before this thread's terms
    r = iincl - my_inc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool st = (starts >> i) & 1, uns = (unsafe >> i) & 1, en = (ends >> i) & 1;
        e += st ? 1 : 0;
        rs = (st && !uns) ? r : rs;
        const uint32_t re = r + inc[i];
        // an unsafe term adds itself; a run's last term its run's exact total
        // (< 2^23 ulps, u a power of 2)
        const float val = uns ? a[i] : (float)(int)(re - rs) * uu[i];
        float *dst = (uns || en) ? ev + (e - 1) : trash;
        *dst = val;
        r = re;
    }
    lds_barrier();
    // the ordered sum, 32 events per batch: every 16-byte read of a batch
    // issued before its first add (an LDS read takes a few hundred cycles
    // under load; the scheduling barrier keeps the reads ahead), the zero pad
    // completing the last batch (+0 leaves s unchanged: s >= +0)
    const float4 *e4 = reinterpret_cast<const float4 *>(x.ev);
    const int n4 = (nev + 3) >> 2;
    float s = 0.0f;
    int q0 = 0;
    do {
        float4 b[kPadEvents / 4];
#pragma unroll
        for (int q = 0; q < kPadEvents / 4; ++q) b[q] = e4[q0 + q];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < kPadEvents / 4; ++q) {
            s += b[q].x;
            s += b[q].y;
            s += b[q].z;
            s += b[q].w;
        }
        q0 += kPadEvents / 4;
    } while (q0 < n4);
    return s;
}

// ---- tree sums (the tolerance path) ---------------------------------------------
// Sums in a fixed tree order -- deterministic from run to run, but not the
// reference's sequential order: they serve the decode step's tolerance path,
// where each RMSNorm sum is a few tree levels instead of an exact
// sequential-order evaluation.

// Sum over the 64 lanes of the wave, the same value in every lane (an xor
// butterfly: at each level both partners add the same two values).
__device__ __forceinline__ float wave_sum_f32(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum over the workgroup (every thread passes its value; the result in
// every thread).  red: blockDim/64 floats of LDS.  Two LDS-only barriers,
// so outstanding global loads are not waited for; red may be reused after
// the call.
__device__ __forceinline__ float block_tree_sum(float v, float *red)
{
    v = wave_sum_f32(v);
    const int nw = (int)(blockDim.x >> 6);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float s = 0.0f;
    for (int w = 0; w < nw; ++w) s += red[w];
    lds_barrier();
    return s;
}

// ---- a group of waves with its own barrier ------------------------------------
// The register form for the nw (<= 16) waves of a group inside a workgroup,
// K terms per lane: lane l of group wave gw holds terms k = K*(64*gw + l) + i.
// Classification, runs and the ordered walk are those above; the group's
// barrier is an LDS counter (GroupSync), so the workgroup's other waves never
// wait on the sum -- they can be stalled issuing loads meanwhile.

// ---- bounded waits on LDS counters ---------------------------------------------
// A wave waiting for other waves of its workgroup polls an LDS counter at most
// g_wait_polls times (default kSyncSpin), so a wait that never completes
// cannot keep the device busy.  A wait that gives up lets the wave go on (its
// LDS reads stay in bounds, the values are wrong) and adds one to
// g_wait_timeouts; the host reads and clears that count when it synchronizes
// and reports the failure (mrml_hip_sync returns MRML_HIP_E_HIP), so wrong
// data never comes back with a success status.  Each translation unit that
// includes this header has its own pair of words (no relocatable device
// code); wait_guard_io() below is that unit's host access to them.
constexpr int kSyncSpin = 1 << 20;

static __device__ int g_wait_polls = kSyncSpin;
static __device__ uint32_t g_wait_timeouts = 0u;

// The poll limit, read once at a kernel's start (before its weight loads are
// queued, so the read does not wait behind them) and passed to the waits.
__device__ __forceinline__ int wait_polls()
{
    const int polls = __builtin_amdgcn_readfirstlane(g_wait_polls);
    asm volatile("" ::"s"(polls));  // the value is in hand here, not fetched at the first wait
    return polls;
}

// Waits until the wave-uniform value of *ctr reaches target, polling at most
// `polls` times; false (and one timeout recorded per wave) if it gives up.
__device__ __forceinline__ bool bounded_wait(const uint32_t *ctr, uint32_t target, int polls)
{
#pragma unroll 1
    for (int i = 0; i < polls; ++i) {
        const uint32_t v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (__builtin_amdgcn_readfirstlane(v) >= target) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&g_wait_timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

// Host side, for the current device: polls >= 0 sets this unit's poll limit
// (0: every wait gives up at once), polls < 0 leaves it; timeouts (nullable)
// receives the count of waits given up since the last call, which is then
// cleared.
static inline hipError_t wait_guard_io(int polls, uint32_t *timeouts)
{
    hipError_t e = hipSuccess;
    if (polls >= 0) e = hipMemcpyToSymbol(HIP_SYMBOL(g_wait_polls), &polls, sizeof polls);
    if (e == hipSuccess && timeouts) {
        e = hipMemcpyFromSymbol(timeouts, HIP_SYMBOL(g_wait_timeouts), sizeof *timeouts);
        if (e == hipSuccess && *timeouts) {
            const uint32_t zero = 0u;
            e = hipMemcpyToSymbol(HIP_SYMBOL(g_wait_timeouts), &zero, sizeof zero);
        }
    }
    return e;
}

// A barrier among the nw waves of a group: each wave adds 1 to an LDS counter
// once its own LDS accesses are done and waits (bounded_wait) until the
// counter reaches nw times its number of syncs so far.  The counter is zeroed
// (and the zero made visible by a workgroup barrier) before the group's first
// sync.
struct GroupSync {
    uint32_t *ctr;
    uint32_t target;
    uint32_t nw;
    int polls;  // wait_polls(), read at the kernel's start
    __device__ __forceinline__ void operator()()
    {
        target += nw;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        bounded_wait(ctr, target, polls);
        asm volatile("" ::: "memory");
    }
};

// LDS of a group sum: the event list (at most one event per term) and the
// zero pad the walk reads past it, at evl, sized by the caller:
// group_events(n) floats.
constexpr int kGroupWalk = 32;  // events per walk batch (eight 16-byte reads)
constexpr int group_events(int n) { return n + kGroupWalk; }

struct GroupShared {
    float wtot[16];
    int wcnt[16];
    float result;
    float trash;  // target of the event stores of lanes that have no event
};

// Tree sum over the nw (<= 8) waves of a group: the wave totals go to
// x.wtot[8*slot + gw] (slot 0 or 1, so two sums in a row need no extra
// sync), one group sync, then every lane adds them in wave order.
__device__ __forceinline__ float group_tree_sum(float v, int gw, GroupSync &sync, GroupShared &x, int slot)
{
    v = wave_sum_f32(v);
    if ((threadIdx.x & 63) == 0) x.wtot[8 * slot + gw] = v;
    sync();
    float s = 0.0f;
    for (int w = 0; w < (int)sync.nw; ++w) s += x.wtot[8 * slot + w];
    return s;
}

// Sum of the terms held by the group (n terms in all), bit for bit the
// sequential loop.  Every lane of the nw waves calls it; gw is the wave's
// index in the group (uniform).  The workgroup form's steps with three group
// syncs: the wave totals, the event counts, the event list.  Each lane's
// event stores are unconditional (a lane with no event writes the trash
// word), and every wave walks the list itself, the same adds in the same
// order, so no fourth sync broadcasts the result.  The caller may start the
// next sum at once: its first LDS writes (the wave totals, then the counts
// and events after its syncs) land only after every wave has passed this
// sum's last sync.
template <int K>
__device__ __forceinline__ float group_seq_sum_nonneg(const float (&av)[K], int n, int gw, GroupSync &sync,
                                                      GroupShared &x, float *evl)
{
    static_assert(K >= 1 && K <= 32 && K + 12 <= kDepth, "masks in 32 bits; prefix depth within the margin");
    const int lane = threadIdx.x & 63, nw = (int)sync.nw;
    const int k0 = K * (64 * gw + lane);
    float a[K], lp[K], run = 0.0f;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        a[i] = k0 + i < n ? av[i] : 0.0f;
        run += a[i];
        lp[i] = run;
    }
    const float wincl = wave_incl_scan_f32(run);
    if (lane == 63) x.wtot[gw] = wincl;
    sync();
    const float wt = lane < gw ? x.wtot[lane] : 0.0f;  // lane < gw <= 15: row 0
    const float base =
        __builtin_bit_cast(float, wave_shr1_i32(__builtin_bit_cast(int, wincl))) + readlane_f32(row_incl_scan_f32(wt), 15);
    uint32_t inc[K], my_inc = 0;
    float uu[K];
    uint32_t unsafe = 0, stop = 0;
    const float rho = margin(k0 + K - 1), omr = 1.0f - rho, opr = 1.0f + rho;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const int k = k0 + i;
        const Step st = classify(a[i], i ? base + lp[i - 1] : base, base + lp[i], k == 0, omr, opr);
        const bool in = k < n;
        inc[i] = (in && st.safe) ? (uint32_t)st.inc : 0u;
        uu[i] = st.u;
        unsafe |= (in && !st.safe) ? (1u << i) : 0u;
        stop |= (!in || !st.safe) ? (1u << i) : 0u;
        my_inc += inc[i];
    }
    const uint32_t pv = (uint32_t)wave_shr1_i32((int)unsafe), nx = (uint32_t)wave_shl1_i32((int)stop);
    const uint32_t prev = lane == 0 ? (1u << (K - 1)) : pv, next = lane == 63 ? 1u : nx;
    uint32_t starts = 0, ends = 0;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const bool in = k0 + i < n, uns = (unsafe >> i) & 1u;
        const bool before = i ? (unsafe >> (i - 1)) & 1u : (prev >> (K - 1)) & 1u;
        const bool after = i < K - 1 ? (stop >> (i + 1)) & 1u : next & 1u;
        starts |= (in && (uns || before)) ? (1u << i) : 0u;
        ends |= (in && !uns && after) ? (1u << i) : 0u;
    }
    const int cnt = __builtin_popcount(starts);
    const int cincl = wave_incl_scan_i32(cnt);
    const uint32_t iincl = (uint32_t)wave_incl_scan_i32((int)my_inc);
    uint32_t r = iincl - my_inc, mine = 0;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        if (((starts & ~unsafe) >> i) & 1u) mine = r;
        r += inc[i];
    }
    uint32_t rs = (uint32_t)wave_shr1_i32((int)wave_incl_max_u32(mine));
    if (lane == 63) x.wcnt[gw] = cincl;
    sync();
    // The counts, offsets and stores are clamped to the n-term event list.
    // The clamps change nothing while every wait completes (each term makes
    // at most one event); after a wait that gave up (stale counts) they keep
    // every LDS access inside the list and the walk below finite.
    const int cw = lane < nw ? (int)min((uint32_t)x.wcnt[lane], (uint32_t)(64 * K)) : 0;  // row 0
    const int ci = row_incl_scan_i32(cw);
    const int nev = min(__builtin_amdgcn_readlane(ci, 15), n);
    const int goff = gw ? min(__builtin_amdgcn_readlane(ci, gw - 1), n) : 0;
    float *const trash = &x.trash;
    {
        float *pz = (gw == 0 && lane < kGroupWalk) ? evl + nev + lane : trash;
        *pz = 0.0f;
    }
    float *ev = evl + goff;
    const int ecap = n - goff;  // events this wave may store
    int e = cincl - cnt;
    r = iincl - my_inc;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const bool st = (starts >> i) & 1u, uns = (unsafe >> i) & 1u, en = (ends >> i) & 1u;
        e += st ? 1 : 0;
        rs = (st && !uns) ? r : rs;
        const uint32_t re = r + inc[i];
        // an unsafe term adds itself; a run's last term its run's exact total
        // (< 2^23 ulps, u a power of 2)
        const float val = uns ? a[i] : (float)(int)(re - rs) * uu[i];
        float *dst = ((uns || en) && e <= ecap) ? ev + (e - 1) : trash;
        *dst = val;
        r = re;
    }
    sync();
    // the ordered walk, kGroupWalk events per batch: every 16-byte read of a
    // batch issued before its first add (the zero pad completes the last
    // batch; +0 leaves s unchanged: s >= +0)
    const float4 *e4 = reinterpret_cast<const float4 *>(evl);
    const int n4 = (nev + 3) >> 2;
    float s = 0.0f;
    int q0 = 0;
    do {
        float4 b[kGroupWalk / 4];
#pragma unroll
        for (int q = 0; q < kGroupWalk / 4; ++q) b[q] = e4[q0 + q];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < kGroupWalk / 4; ++q) {
            s += b[q].x;
            s += b[q].y;
            s += b[q].z;
            s += b[q].w;
        }
        q0 += kGroupWalk / 4;
    } while (q0 < n4);
    return s;
}

#endif  // __HIPCC__

}  // namespace mrml_xsum
