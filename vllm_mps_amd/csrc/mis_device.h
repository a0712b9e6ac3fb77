// mis_device.h -- device-side primitives of the sampler kernels: dtype loads,
// temperature scaling, wave64 / workgroup reductions and scans, histogram
// search, raw-key interval search and a latency-hiding row scan.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mis_common.h"
#include "mis_layout.h"

namespace mis {

// ------------------------------------------------------------------ dtype io

template <int DT> struct Traits;
template <> struct Traits<F32> { static constexpr int VEC = 4, ESZ = 4; };
template <> struct Traits<F16> { static constexpr int VEC = 8, ESZ = 2; };
template <> struct Traits<BF16> { static constexpr int VEC = 8, ESZ = 2; };

template <int DT> __device__ __forceinline__ float cvt16(uint32_t h)
{
    if (DT == F16) { _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h); return (float)v; }
    return bits_f32(h << 16);
}

// logits live in global memory: load through the global address space so
// the compiler emits global_load rather than flat_load
#define MIS_GLOBAL __attribute__((address_space(1)))

template <int DT> __device__ __forceinline__ float load1(const char *rowp, int64_t j)
{
    if (DT == F32) return ((const MIS_GLOBAL float *)rowp)[j];
    return cvt16<DT>(((const MIS_GLOBAL uint16_t *)rowp)[j]);
}

// VEC elements from a 16-byte aligned address
template <int DT> __device__ __forceinline__ void loadvec(const char *rowp, int64_t j0, float *out)
{
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = *(const MIS_GLOBAL u32x4 *)(rowp + j0 * Traits<DT>::ESZ);
    if (DT == F32) {
        out[0] = bits_f32(v.x); out[1] = bits_f32(v.y); out[2] = bits_f32(v.z); out[3] = bits_f32(v.w);
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) { out[2 * i] = cvt16<DT>(w[i] & 0xffffu); out[2 * i + 1] = cvt16<DT>(w[i] >> 16); }
    }
}

// y = dtype(f32(x) / T): IEEE binary32 division (hipcc's correctly rounded
// divide), then round-to-nearest-even into the 16-bit dtype.
template <int DT> __device__ __forceinline__ float scale_y(float x, float T)
{
    const float q = x / T;
    return DT == F32 ? q : rn_dtype(q, DT);
}

// The same quotient through the row's reciprocal r = RN(1/T): div_rcp()
// (mis_common.h), the generic division where it does not apply.
template <int DT> __device__ __forceinline__ float scale_r(float x, float T, float r)
{
    const float q = div_rcp(x, T, r);
    return DT == F32 ? q : rn_dtype(q, DT);
}

// scale_r over N register values in place, with the generic division taken
// in one wave-uniform branch for the (rare) elements that need it instead of
// a branch per element.  N <= 64.
template <int DT, int N> __device__ __forceinline__ void scale_all(float (&x)[N], float T, float r)
{
    static_assert(N <= 64, "one mask bit per element");
    if (T == 1.0f) {
        // x / 1 == x exactly, and x (a value of the row's dtype) rounds to
        // itself: only NaN elements, which the division quiets, take the
        // general formula
        uint64_t nan = 0ull;
#pragma unroll
        for (int i = 0; i < N; ++i) nan |= x[i] != x[i] ? (1ull << i) : 0ull;
        if (__ballot(nan != 0ull) != 0ull) {
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (nan & (1ull << i)) x[i] = DT == F32 ? x[i] / T : rn_dtype(x[i] / T, DT);
        }
        return;
    }
    uint64_t slow = 0ull;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float xi = x[i];
        const float q0 = xi * r;
        const bool sl = !div_rcp_safe(xi, q0);
        const float q = div_rcp_core(xi, T, r, q0);
        x[i] = sl ? xi : q;
        slow |= sl ? (1ull << i) : 0ull;
    }
    if (__ballot(slow != 0ull) != 0ull) {
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (slow & (1ull << i)) x[i] = x[i] / T;
    }
    if (DT != F32) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = rn_dtype(x[i], DT);
    }
}

// exp(y - ym) for y <= ym in binary32 with a bounded relative error: the
// difference and its base-2 scaling are formed in binary64 (exact difference,
// one rounding of 2^-53), split into n + f with |f| <= 1/2, and 2^f comes from
// the hardware exp2 (1 ulp) on the f32-rounded f (2^-26 absolute).  Relative
// error <= 1.3e-7 while the result is normal; WEXP_REL_ERR bounds it with
// margin.  Results below 2^-126 lose relative precision (absolute error
// <= 2^-149), which the callers' bounds cover through an absolute term.
constexpr double WEXP_REL_ERR = 4.8e-7;   // 2^-21
constexpr double WEXP_ABS_ERR = 1.5e-45;  // one subnormal ulp per element
__device__ __forceinline__ float wexp(float y, float ym)
{
    const double t = ((double)y - (double)ym) * 1.4426950408889634;
    if (!(t > -1000.0)) return 0.0f;  // y = -inf (or below every subnormal)
    const double n = rint(t);
    const float f = (float)(t - n);
    const float p = __builtin_amdgcn_exp2f(f);
    const int ni = n < -300.0 ? -300 : (int)n;
    return ldexpf(p, ni);
}

// ------------------------------------------------------------------ wave / block

// Workgroup-uniform values read back from LDS: moving them to scalar
// registers frees vector registers and lets loads through them go scalar.
__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ int32_t uni(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uni(float v) { return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ double uni(double v)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

template <class T> __device__ __forceinline__ T wave_sum(T v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <class T> __device__ __forceinline__ T wave_max(T v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { T w = __shfl_xor(v, o, 64); v = w > v ? w : v; }
    return v;
}
template <class T> __device__ __forceinline__ T wave_min(T v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { T w = __shfl_xor(v, o, 64); v = w < v ? w : v; }
    return v;
}
// (key desc, idx asc) arg-max
__device__ __forceinline__ void wave_argmax(uint32_t &k, int32_t &i)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t k2 = __shfl_xor(k, o, 64);
        const int32_t i2 = __shfl_xor(i, o, 64);
        if (k2 > k || (k2 == k && i2 < i)) { k = k2; i = i2; }
    }
}
template <class T> __device__ __forceinline__ T wave_incl_scan(T v)
{
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T w = __shfl_up(v, o, 64);
        if (l >= o) v += w;
    }
    return v;
}

// Slot of this lane in an append to a list whose fill is *counter (LDS): one
// atomic per wave instead of one per element.  Valid where pred holds; lanes
// not executing the call take no part.
__device__ __forceinline__ uint32_t wave_append(bool pred, uint32_t *counter)
{
    const uint64_t mk = __ballot(pred);
    if (mk == 0ull) return 0u;
    const int lead = __builtin_ctzll(__ballot(1));
    uint32_t base = 0u;
    if (lane_id() == lead) base = atomicAdd(counter, (uint32_t)__popcll(mk));
    base = (uint32_t)__shfl((int)base, lead, 64);
    return base + (uint32_t)__popcll(mk & ((1ull << lane_id()) - 1ull));
}

// LDS scratch for the block reductions of up to 16 waves (1024 threads);
// the helpers take the block's wave count NW as a template argument
constexpr int NWAVE_MAX = 16;
struct Red { double d[NWAVE_MAX + 1]; int64_t l[NWAVE_MAX + 1]; uint32_t u[NWAVE_MAX + 1]; float f[NWAVE_MAX + 1]; };

template <class T> __device__ __forceinline__ T *red_of(Red &r);
template <> __device__ __forceinline__ double *red_of<double>(Red &r) { return r.d; }
template <> __device__ __forceinline__ int64_t *red_of<int64_t>(Red &r) { return r.l; }
template <> __device__ __forceinline__ uint32_t *red_of<uint32_t>(Red &r) { return r.u; }
template <> __device__ __forceinline__ float *red_of<float>(Red &r) { return r.f; }

template <class T, int NW = NWAVE> __device__ __forceinline__ T block_excl_scan(T v, Red &rr, T *total)
{
    T *red = red_of<T>(rr);
    const T inc = wave_incl_scan(v);
    if (lane_id() == 63) red[wave_id()] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        T run = T(0);
        for (int w = 0; w < NW; ++w) { const T t = red[w]; red[w] = run; run += t; }
        red[NW] = run;
    }
    __syncthreads();
    const T res = inc - v + red[wave_id()];
    *total = red[NW];
    __syncthreads();
    return res;
}
template <class T, int NW = NWAVE> __device__ __forceinline__ T block_sum(T v, Red &rr)
{
    T *red = red_of<T>(rr);
    v = wave_sum(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    T t = T(0);
    for (int w = 0; w < NW; ++w) t += red[w];
    __syncthreads();
    return t;
}
template <class T, int NW = NWAVE> __device__ __forceinline__ T block_max(T v, Red &rr)
{
    T *red = red_of<T>(rr);
    v = wave_max(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    T t = red[0];
    for (int w = 1; w < NW; ++w) t = red[w] > t ? red[w] : t;
    __syncthreads();
    return t;
}
template <class T, int NW = NWAVE> __device__ __forceinline__ T block_min(T v, Red &rr)
{
    T *red = red_of<T>(rr);
    v = wave_min(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    T t = red[0];
    for (int w = 1; w < NW; ++w) t = red[w] < t ? red[w] : t;
    __syncthreads();
    return t;
}

// Descending search over a histogram in LDS, run by one whole wave.  Finds
// the first bin b from the top (index nbins-1 downwards) where
// sum_{b' >= b} h[b'] >= target; *above = sum of the bins strictly above b.
// If the target is never reached (rounding) it returns the lowest non-empty
// bin.  nbins must be a multiple of 64.
template <class T>
__device__ __forceinline__ int wave_find_desc(const T *h, int nbins, T target, T *above)
{
    const int l = lane_id();
    const int per = nbins / 64;
    T s = T(0);
    for (int i = 0; i < per; ++i) s += h[nbins - 1 - (l * per + i)];
    const T inc = wave_incl_scan(s);
    const uint64_t mask = __ballot(inc >= target);
    int bsel = 0;
    T abv = T(0);
    int first;
    if (mask == 0ull) {
        const uint64_t ne = __ballot(s > T(0));
        if (ne == 0ull) { *above = T(0); return 0; }
        first = 63 - __builtin_clzll(ne);
        if (l == first) {
            T run = inc - s;
            for (int i = 0; i < per; ++i) {
                const int b = nbins - 1 - (l * per + i);
                if (h[b] > T(0)) { bsel = b; abv = run; }
                run += h[b];
            }
        }
    } else {
        first = __builtin_ctzll(mask);
        if (l == first) {
            T run = inc - s;
            bsel = nbins - 1 - (l * per + per - 1);
            abv = run;
            for (int i = 0; i < per; ++i) {
                const int b = nbins - 1 - (l * per + i);
                if (run + h[b] >= target) { bsel = b; abv = run; break; }
                run += h[b];
            }
        }
    }
    bsel = __shfl(bsel, first, 64);
    abv = __shfl(abv, first, 64);
    *above = abv;
    return bsel;
}

// Descending search over a count histogram in LDS by the whole block (NTH
// threads, nbins a multiple of NTH, at most 4 bins per thread): the bin b
// where the count from the top reaches `target` (which must be at most the
// total); *above = the count strictly above b.  slot: two LDS words.
template <int NTH>
__device__ __forceinline__ int block_find_desc(const uint32_t *h, int nbins, uint32_t target, uint32_t *above, Red &rr,
                                               uint32_t *slot)
{
    const int per = nbins / NTH, t = threadIdx.x;
    uint32_t v[4] = {0u, 0u, 0u, 0u}, s = 0u;
    for (int q = 0; q < per && q < 4; ++q) { v[q] = h[nbins - 1 - (t * per + q)]; s += v[q]; }
    uint32_t tot;
    const uint32_t ex = block_excl_scan<uint32_t, NTH / 64>(s, rr, &tot);
    if (t == 0) { slot[0] = 0u; slot[1] = tot; }
    __syncthreads();
    if (ex < target && ex + s >= target) {
        uint32_t run = ex;
        for (int q = 0; q < per && q < 4; ++q) {
            if (run + v[q] >= target) { slot[0] = (uint32_t)(nbins - 1 - (t * per + q)); slot[1] = run; break; }
            run += v[q];
        }
    }
    __syncthreads();
    const int b = (int)slot[0];
    *above = slot[1];
    __syncthreads();
    return b;
}

// Ascending search over n <= 64*per values in LDS, run by one whole wave:
// the first index i whose inclusive prefix sum exceeds `target` (indices with
// zero value never qualify); *before = sum of the values before i.  When
// rounding leaves the target out of reach, the last index with a nonzero
// value.  Returns -1 when every value is zero.
__device__ __forceinline__ int wave_find_asc(const double *v, int n, double target, double *before)
{
    const int l = lane_id();
    const int per = (n + 63) / 64;
    const int b0 = l * per, b1 = b0 + per < n ? b0 + per : n;
    double s = 0.0;
    for (int i = b0; i < b1; ++i) s += v[i];
    const double inc = wave_incl_scan(s);
    const uint64_t mask = __ballot(inc > target);
    int sel = -1;
    double bef = 0.0;
    int owner;
    if (mask != 0ull) {
        owner = __builtin_ctzll(mask);
        if (l == owner) {
            double run = inc - s;
            int last = -1;
            double lastbef = 0.0;
            for (int i = b0; i < b1; ++i) {
                if (v[i] > 0.0) {
                    if (run + v[i] > target) { sel = i; bef = run; break; }
                    last = i; lastbef = run;
                }
                run += v[i];
            }
            if (sel < 0) { sel = last; bef = lastbef; }
        }
    } else {
        const uint64_t ne = __ballot(s > 0.0);
        if (ne == 0ull) { *before = 0.0; return -1; }
        owner = 63 - __builtin_clzll(ne);
        if (l == owner) {
            double run = inc - s;
            for (int i = b0; i < b1; ++i) {
                if (v[i] > 0.0) { sel = i; bef = run; }
                run += v[i];
            }
        }
    }
    sel = __shfl(sel, owner, 64);
    bef = __shfl(bef, owner, 64);
    *before = bef;
    return sel;
}

// Sort, descending, of k[0..n) with payload e (n <= CAP; CAP and the block
// size NTH powers of two), by all threads of the block; afterwards entries
// n .. CAP-1 hold key 0 and payload 0, and every real key must be > 0.
// Up to RANK_N entries: each of the first n threads counts the keys above
// its own (equal keys ordered by position) and writes its pair to that rank.
// Beyond: a bitonic sort, element i in thread i / PT (PT = CAP / NTH, at most
// 4) at register slot i % PT: compare-exchanges between slots of one thread
// work on registers, between lanes of one wave on shuffles, and only partners
// in other waves go through LDS (k and e, CAP entries each).
constexpr int RANK_N = 256;
template <int NTH, int CAP>
__device__ __forceinline__ void block_sort_desc(uint64_t *k, double *e, int n)
{
    constexpr int PT = CAP / NTH;
    static_assert(PT == 1 || PT == 2 || PT == 4, "1, 2 or 4 elements per thread");
    static_assert(RANK_N <= NTH, "one element per thread in the rank sort");
    const int tid = threadIdx.x;
    if (n <= RANK_N) {
        __syncthreads();
        uint64_t kt = 0ull;
        double et = 0.0;
        int rank = 0;
        if (tid < n) {
            kt = k[tid];
            et = e[tid];
            for (int j = 0; j < n; ++j) {
                const uint64_t kj = k[j];
                rank += (kj > kt || (kj == kt && j < tid)) ? 1 : 0;
            }
        }
        __syncthreads();
        if (tid < n) { k[rank] = kt; e[rank] = et; }
        for (int i = n + tid; i < CAP; i += NTH) { k[i] = 0ull; e[i] = 0.0; }
        __syncthreads();
        return;
    }
    int npow = 1;
    while (npow < n) npow <<= 1;
    uint64_t kv[PT];
    double ev[PT];
#pragma unroll
    for (int r = 0; r < PT; ++r) {
        const int i = tid * PT + r;
        kv[r] = i < n ? k[i] : 0ull;
        ev[r] = i < n ? e[i] : 0.0;
    }
    // the pair (r, r + jj) of one thread, stage (kk, jj)
    auto cx = [&](int r, int p, int kk) {
        const int i = tid * PT + r;
        const bool desc = (i & kk) == 0;
        if (desc ? (kv[r] < kv[p]) : (kv[r] > kv[p])) {
            const uint64_t tk = kv[r]; kv[r] = kv[p]; kv[p] = tk;
            const double te = ev[r]; ev[r] = ev[p]; ev[p] = te;
        }
    };
    for (int kk = 2; kk <= npow; kk <<= 1) {
        for (int j = kk >> 1; j > 0; j >>= 1) {
            if (j < PT) {
                if constexpr (PT == 2) {
                    cx(0, 1, kk);
                } else if constexpr (PT == 4) {
                    if (j == 1) { cx(0, 1, kk); cx(2, 3, kk); }
                    else { cx(0, 2, kk); cx(1, 3, kk); }
                }
            } else if (j < PT * 64) {
                const int lm = j / PT;
#pragma unroll
                for (int r = 0; r < PT; ++r) {
                    const int i = tid * PT + r;
                    const uint64_t k2 = __shfl_xor(kv[r], lm, 64);
                    const double e2 = __shfl_xor(ev[r], lm, 64);
                    const bool take_max = ((i & j) == 0) == ((i & kk) == 0);
                    if (take_max ? (k2 > kv[r]) : (k2 < kv[r])) { kv[r] = k2; ev[r] = e2; }
                }
            } else {
                __syncthreads();
#pragma unroll
                for (int r = 0; r < PT; ++r) { k[tid * PT + r] = kv[r]; e[tid * PT + r] = ev[r]; }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < PT; ++r) {
                    const int i = tid * PT + r;
                    const uint64_t k2 = k[i ^ j];
                    const double e2 = e[i ^ j];
                    const bool take_max = ((i & j) == 0) == ((i & kk) == 0);
                    if (take_max ? (k2 > kv[r]) : (k2 < kv[r])) { kv[r] = k2; ev[r] = e2; }
                }
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < PT; ++r) { k[tid * PT + r] = kv[r]; e[tid * PT + r] = ev[r]; }
    __syncthreads();
}

// ------------------------------------------------------------------ raw-key intervals
//
// The scaled value y = scale(x) is a non-decreasing function of the raw
// logit x, so the set of raw values whose scaled key lies in [klo, khi] is an
// interval of raw keys.  Filtering raw keys first avoids a division for every
// element a scan does not need.

template <int DT> __device__ __forceinline__ uint32_t rk_of_xkey(uint32_t xk, float T)
{
    return row_key(scale_y<DT>(f32_of_key(xk), T), DT);
}

// Smallest raw key (over all non-NaN floats) whose scaled key is >= target;
// 0xff800001 when none.  Executed by one whole wave (64-ary search).
template <int DT> __device__ __forceinline__ uint32_t x_lower(uint32_t target, float T)
{
    const uint32_t XLO = 0x007fffffu, XHI = 0xff800000u;  // -inf .. +inf
    const int l0 = lane_id();
    {
        // one window of 64 raw keys around a guess first: the boundary lies
        // within a few ulps of b * T, b the least scaled value that reaches
        // target (fp32: its value; 16-bit: the midpoint to the next lower
        // value, where round-to-nearest starts to give target).  The
        // predicate is monotone, so false at the window's first key and true
        // at a later one fixes the boundary; otherwise the full search runs.
        float b;
        if (DT == F32) {
            b = f32_of_key(target);
        } else {
            // 16-bit row keys are multiples of 2^16: the least one >= target
            // (0 when none: a NaN guess, which skips the window)
            const uint32_t t16 = (target & 0xffffu) ? (target | 0xffffu) + 1u : target;
            const float v = value_of_row_key(t16, DT);
            const float w = t16 >= 0x10000u ? value_of_row_key(t16 - 0x10000u, DT) : -INFINITY;
            b = 0.5f * v + 0.5f * w;
        }
        const float gx = b * T;
        if (fabsf(gx) < INFINITY) {  // finite (NaN fails too)
            const uint32_t gk = key_of_f32(gx);
            uint32_t base = gk > XLO + 32u ? gk - 32u : XLO;
            if (base > XHI - 63u) base = XHI - 63u;
            const uint64_t mask = __ballot(rk_of_xkey<DT>(base + (uint32_t)l0, T) >= target);
            if (mask != 0ull && (mask & 1ull) == 0ull) return base + (uint32_t)__builtin_ctzll(mask);
        }
    }
    if (rk_of_xkey<DT>(XLO, T) >= target) return XLO;
    if (rk_of_xkey<DT>(XHI, T) < target) return XHI + 1u;
    uint64_t lo = XLO, hi = XHI;  // pred(lo) false, pred(hi) true
    const int l = lane_id();
    while (hi - lo > 1) {
        uint64_t step = (hi - lo) / 64;
        if (step == 0) step = 1;
        const uint64_t p = lo + (uint64_t)(l + 1) * step;
        const bool pred = p >= hi ? true : (rk_of_xkey<DT>((uint32_t)p, T) >= target);
        const uint64_t mask = __ballot(pred);
        if (mask == 0ull) { lo = lo + 64 * step; continue; }
        const int f = __builtin_ctzll(mask);
        const uint64_t nhi = lo + (uint64_t)(f + 1) * step;
        if (nhi < hi) hi = nhi;
        lo = lo + (uint64_t)f * step;
    }
    return (uint32_t)hi;
}

// Largest raw key whose scaled key is <= target (0x007ffffe when none).
template <int DT> __device__ __forceinline__ uint32_t x_upper(uint32_t target, float T)
{
    if (target == 0xffffffffu) return 0xff800000u;
    return x_lower<DT>(target + 1u, T) - 1u;
}

// ------------------------------------------------------------------ row scans

// Calls f(j, x) for every j in [jb, je) of a row.  Each thread issues UNROLL
// 16-byte loads before consuming any, so a single workgroup keeps
// NT * UNROLL * 16 bytes in flight.  jb must be a multiple of the vector
// width when vec_ok.  All threads of the block must call it.
template <int DT, int UNROLL, class F>
__device__ __forceinline__ void scan_range(const char *rowp, int64_t jb, int64_t je, int vec_ok, F &&f)
{
    constexpr int VEC = Traits<DT>::VEC;
    const int64_t tile = (int64_t)NT * VEC * UNROLL;
    for (int64_t t0 = jb; t0 < je; t0 += tile) {
        float xs[UNROLL][VEC];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t j0 = t0 + ((int64_t)u * NT + threadIdx.x) * VEC;
            if (vec_ok && j0 + VEC <= je) {
                loadvec<DT>(rowp, j0, xs[u]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) xs[u][e] = (j0 + e < je) ? load1<DT>(rowp, j0 + e) : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t j0 = t0 + ((int64_t)u * NT + threadIdx.x) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                if (j0 + e < je) f(j0 + e, xs[u][e]);
        }
    }
}

}  // namespace mis
