// mis_sampler.hip -- MI355X (gfx950) decode-step token sampler behind the C ABI
// declared in include/mis_sampler.h.
//
// One call = up to three stream-ordered launches:
//   K1 k_chunk  grid (G, B), 256 threads.  Each workgroup holds one chunk of
//               one logits row in registers (a single coalesced 16-byte-vector
//               read of HBM) and reduces it to a chunk summary: argmax of the
//               raw logits, the chunk max of the scaled logits, and -- by row
//               mode -- the chunk-local top-k' candidates, or the float64
//               softmax mass with a 256-bin histogram (top byte of the order
//               key) of counts and masses.
//   K2 k_final  grid (B), 1024 threads.  Merges the G summaries of a row,
//               resolves the top-k threshold and the top-p cut, and draws the
//               token by inverse CDF in vocabulary order.  Re-reads of the row
//               (L2 / MALL) happen only to refine a histogram bin or to scan
//               one chunk for the draw.
//   K3 k_emit   grid (G, B), 256 threads, only when the caller asks for the
//               debug probabilities / keep bitmask.
//
// Semantics follow model/sampler.py:18-60 per row (see the oracle for the
// exact contract):  greedy argmax (ties -> lowest index) when T == 0;
// y = dtype(f32(x) / T); top-k keeps y >= k'-th largest (all ties); top-p on
// the stable descending order with float64 masses (fp32 rows) or torch's
// 16-bit rounding chain (fp16/bf16 rows); the draw is
// min{i : sum_{j<=i} w_j > u * sum w} over the kept weights w = exp(y - m).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mis_common.h"
#include "mis_sampler.h"

namespace mis {

constexpr int K1_THREADS = 256;
constexpr int K2_THREADS = 512;
constexpr int K3_THREADS = 256;
constexpr int K2_WAVES = K2_THREADS / 64;
constexpr int K_SMALL = 1024;      // largest k' served by the candidate path
constexpr int CAND_CAP = 2048;     // candidates one chunk may emit
constexpr int SURV_CAP = 4096;     // top-k survivors the finalize holds in LDS
constexpr int G_MAX = 1024;        // chunks per row
constexpr int REGION_BINS = 16;    // L1 bins per 16-bit chain pass (16 x 256 keys)
constexpr int RUN_CAP = REGION_BINS * 256;
constexpr int TIE_CAP = 4096;
constexpr uint32_t NCAND_OVERFLOW = 0xffffffffu;
constexpr int32_t IDX_ALL = 0x7fffffff;

enum : int { M_BAD = 0, M_GREEDY = 1, M_SMALLK = 2, M_LARGEK = 3, M_TOPP = 4, M_TEMP = 5 };
enum : uint32_t { FLAG_NAN = 1u, FLAG_PINF = 2u };

// ------------------------------------------------------------------ layout

struct ChunkSum {           // 32 bytes per (row, chunk)
    uint32_t xkey;          // argmax key of the raw logits (NaN = 0xffffffff)
    int32_t xarg;           // first index holding it
    float ymax;             // max scaled logit of the chunk
    uint32_t flags;
    uint32_t ncand;         // candidates written (small-k rows) or NCAND_OVERFLOW
    uint32_t pad;
    double S;               // sum exp(y - ymax) over the chunk (float64)
};

struct RowOut {             // 48 bytes per row, read by k_emit
    int64_t id;
    int32_t status;
    int32_t mode;
    float m;                // row max of the scaled logits
    uint32_t cut_key;       // kept iff key > cut_key or (key == cut_key and j <= cut_i)
    int32_t cut_i;
    int32_t pad;
    double S;               // sum of kept weights exp(y - m)
    double pad2;
};

struct Cand { uint32_t key; int32_t idx; };

struct Layout {
    int64_t B, V;
    int ept, G;
    size_t rowout, chunks, l1cnt, l1mass, cand, total;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static Layout make_layout(int64_t B, int64_t V)
{
    Layout L;
    L.B = B; L.V = V;
    static const int opts[4] = {64, 32, 16, 8};
    L.ept = 8;
    for (int i = 0; i < 4; ++i) {
        int64_t G = (V + (int64_t)K1_THREADS * opts[i] - 1) / ((int64_t)K1_THREADS * opts[i]);
        if (B * G >= 1024 && G <= G_MAX) { L.ept = opts[i]; break; }
    }
    L.G = (int)((V + (int64_t)K1_THREADS * L.ept - 1) / ((int64_t)K1_THREADS * L.ept));
    if (L.G > G_MAX) {  // very large vocabularies: widest chunks
        L.ept = 64;
        L.G = (int)((V + (int64_t)K1_THREADS * 64 - 1) / ((int64_t)K1_THREADS * 64));
    }
    size_t off = 0;
    L.rowout = off; off = align256(off + sizeof(RowOut) * (size_t)B);
    L.chunks = off; off = align256(off + sizeof(ChunkSum) * (size_t)B * L.G);
    L.l1cnt = off;  off = align256(off + sizeof(uint32_t) * 256 * (size_t)B * L.G);
    L.l1mass = off; off = align256(off + sizeof(double) * 256 * (size_t)B * L.G);
    L.cand = off;   off = align256(off + sizeof(Cand) * (size_t)CAND_CAP * B * L.G);
    L.total = off;
    return L;
}

// ------------------------------------------------------------------ row plan

struct RowPlan { int mode; int kk; int topp; float T; float top_p; float u; };

__device__ __forceinline__ RowPlan plan_row(const mis_row_params &P, int64_t V)
{
    RowPlan r;
    r.T = P.temperature; r.top_p = P.top_p; r.u = P.uniform; r.kk = 0; r.topp = 0;
    bool bad = !(P.temperature >= 0.0f) || P.top_k < 0 || !(P.top_p > 0.0f) || !(P.uniform == P.uniform);
    if (bad) { r.mode = M_BAD; return r; }
    if (P.temperature == 0.0f) { r.mode = M_GREEDY; return r; }
    int64_t kk = P.top_k > 0 ? ((int64_t)P.top_k < V ? (int64_t)P.top_k : V) : 0;
    if (kk >= V) kk = 0;  // k' = V keeps every element
    r.kk = (int)kk;
    r.topp = P.top_p < 1.0f;
    if (kk > 0 && kk <= K_SMALL) r.mode = M_SMALLK;
    else if (kk > 0) r.mode = M_LARGEK;
    else if (r.topp) r.mode = M_TOPP;
    else r.mode = M_TEMP;
    return r;
}

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

template <int DT> __device__ __forceinline__ float load1(const char *rowp, int64_t j)
{
    if (DT == F32) return reinterpret_cast<const float *>(rowp)[j];
    return cvt16<DT>(reinterpret_cast<const uint16_t *>(rowp)[j]);
}

template <int DT> __device__ __forceinline__ void loadvec(const char *rowp, int64_t j0, float *out)
{
    uint4 v = *reinterpret_cast<const uint4 *>(rowp + j0 * Traits<DT>::ESZ);
    if (DT == F32) {
        out[0] = bits_f32(v.x); out[1] = bits_f32(v.y); out[2] = bits_f32(v.z); out[3] = bits_f32(v.w);
    } else {
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) { out[2 * i] = cvt16<DT>(w[i] & 0xffffu); out[2 * i + 1] = cvt16<DT>(w[i] >> 16); }
    }
}

// y = dtype(f32(x) / T): IEEE division (hipcc's default correctly rounded
// f32 divide), then RNE to the 16-bit dtype.
template <int DT> __device__ __forceinline__ float scale_y(float x, float T)
{
    float q = x / T;
    return DT == F32 ? q : rn_dtype(q, DT);
}

// ------------------------------------------------------------------ wave / block helpers

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

// (key desc, idx asc) arg-max reduction
__device__ __forceinline__ void wave_argmax(uint32_t &k, int32_t &i)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t k2 = __shfl_xor(k, o, 64);
        int32_t i2 = __shfl_xor(i, o, 64);
        if (k2 > k || (k2 == k && i2 < i)) { k = k2; i = i2; }
    }
}

template <class T> __device__ __forceinline__ T wave_incl_scan(T v)
{
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        T w = __shfl_up(v, o, 64);
        if (l >= o) v += w;
    }
    return v;
}

// Block-wide exclusive scan; `red` is LDS scratch of >= NW entries.  Returns
// the exclusive prefix of this thread and writes the block total to *total.
template <int NT, class T> __device__ T block_excl_scan(T v, T *red, T *total)
{
    constexpr int NW = NT / 64;
    T inc = wave_incl_scan(v);
    if (lane_id() == 63) red[wave_id()] = inc;
    __syncthreads();
    if (wave_id() == 0) {
        T t = lane_id() < NW ? red[lane_id()] : T(0);
        T ti = wave_incl_scan(t);
        if (lane_id() < NW) red[lane_id()] = ti - t;
        if (lane_id() == NW - 1) red[NW] = ti;
    }
    __syncthreads();
    T res = inc - v + red[wave_id()];
    *total = red[NW];
    __syncthreads();
    return res;
}

template <int NT, class T> __device__ T block_sum(T v, T *red)
{
    constexpr int NW = NT / 64;
    v = wave_sum(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    T t = T(0);
    for (int w = 0; w < NW; ++w) t += red[w];
    __syncthreads();
    return t;
}

template <int NT, class T> __device__ T block_max(T v, T *red)
{
    constexpr int NW = NT / 64;
    v = wave_max(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    T t = red[0];
    for (int w = 1; w < NW; ++w) t = red[w] > t ? red[w] : t;
    __syncthreads();
    return t;
}

template <int NT, class T> __device__ T block_min(T v, T *red)
{
    constexpr int NW = NT / 64;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { T w = __shfl_xor(v, o, 64); v = w < v ? w : v; }
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    T t = red[0];
    for (int w = 1; w < NW; ++w) t = red[w] < t ? red[w] : t;
    __syncthreads();
    return t;
}

// Descending search over a histogram held in LDS (run by one whole wave).
// Finds the first bin b (from the top) where acc + sum_{b' >= b} h[b'] >= target
// and returns b with *above = sum of bins strictly above b.  If the target is
// never reached (rounding), returns the lowest non-empty bin.
template <class T>
__device__ int wave_find_desc(const T *h, int nbins, T target, T *above)
{
    const int l = lane_id();
    const int per = nbins / 64;
    // lane l owns bins [nbins-1 - l*per, nbins - (l+1)*per] in descending order
    T s = T(0);
    for (int i = 0; i < per; ++i) s += h[nbins - 1 - (l * per + i)];
    T inc = wave_incl_scan(s);
    uint64_t mask = __ballot(inc >= target);
    int first;
    if (mask == 0ull) {
        // not reached: lowest non-empty bin
        uint64_t ne = __ballot(s > T(0));
        if (ne == 0ull) { *above = T(0); return 0; }
        first = 63 - __builtin_clzll(ne);
        T before = __shfl(inc - s, first, 64);
        int bsel = 0;
        T abv = before;
        if (l == first) {
            T run = before;
            for (int i = 0; i < per; ++i) {
                int b = nbins - 1 - (l * per + i);
                if (h[b] > T(0)) { bsel = b; abv = run; }
                run += h[b];
            }
        }
        bsel = __shfl(bsel, first, 64);
        abv = __shfl(abv, first, 64);
        *above = abv;
        return bsel;
    }
    first = __builtin_ctzll(mask);
    int bsel = 0;
    T abv = T(0);
    if (l == first) {
        T run = inc - s;
        bsel = nbins - 1 - (l * per + per - 1);
        abv = run;
        for (int i = 0; i < per; ++i) {
            int b = nbins - 1 - (l * per + i);
            if (run + h[b] >= target) { bsel = b; abv = run; break; }
            run += h[b];
        }
    }
    bsel = __shfl(bsel, first, 64);
    abv = __shfl(abv, first, 64);
    *above = abv;
    return bsel;
}

// ------------------------------------------------------------------ K1: chunk pass

template <int DT, int EPT>
__global__ __launch_bounds__(K1_THREADS) void k_chunk(const char *__restrict__ logits, int64_t V,
                                                      int64_t stride_bytes, int vec_ok,
                                                      const mis_row_params *__restrict__ params,
                                                      Layout L, char *__restrict__ ws)
{
    constexpr int VEC = Traits<DT>::VEC, NV = EPT / VEC, CH = K1_THREADS * EPT;
    const int tid = threadIdx.x, chunk = blockIdx.x, row = blockIdx.y;
    const int64_t base = (int64_t)chunk * CH;
    const char *rowp = logits + (int64_t)row * stride_bytes;
    const RowPlan pl = plan_row(params[row], V);
    ChunkSum *cs = reinterpret_cast<ChunkSum *>(ws + L.chunks) + (size_t)row * L.G + chunk;

    __shared__ uint32_t s_u[256];
    __shared__ double s_d[256];
    __shared__ uint32_t s_red_u[8];
    __shared__ int32_t s_red_i[8];
    __shared__ double s_red_d[8];
    __shared__ uint32_t s_bcast[4];

    float x[EPT];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int64_t j0 = base + ((int64_t)v * K1_THREADS + tid) * VEC;
        if (vec_ok && j0 + VEC <= V) {
            loadvec<DT>(rowp, j0, &x[v * VEC]);
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) x[v * VEC + e] = (j0 + e < V) ? load1<DT>(rowp, j0 + e) : 0.0f;
        }
    }
    auto idx_of = [&](int i) -> int64_t { return base + ((int64_t)(i / VEC) * K1_THREADS + tid) * VEC + (i % VEC); };

    // ---- argmax of the raw logits (every mode)
    uint32_t bk = 0u;
    int32_t bi = IDX_ALL;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int64_t j = idx_of(i);
        if (j < V) {
            uint32_t k = argmax_key(x[i]);
            if (k > bk) { bk = k; bi = (int32_t)j; }  // ascending j per thread: first wins
        }
    }
    wave_argmax(bk, bi);
    if (lane_id() == 0) { s_red_u[wave_id()] = bk; s_red_i[wave_id()] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < K1_THREADS / 64; ++w) {
            if (s_red_u[w] > bk || (s_red_u[w] == bk && s_red_i[w] < bi)) { bk = s_red_u[w]; bi = s_red_i[w]; }
        }
        s_bcast[0] = bk;
        s_bcast[1] = (uint32_t)bi;
    }
    __syncthreads();
    bk = s_bcast[0];
    bi = (int32_t)s_bcast[1];

    if (pl.mode == M_BAD || pl.mode == M_GREEDY) {
        if (tid == 0) { cs->xkey = bk; cs->xarg = bi; cs->ymax = 0.0f; cs->flags = 0; cs->ncand = 0; cs->S = 0.0; }
        return;
    }

    uint32_t flags = 0;
    float ymax;
    if (bk == 0xffffffffu) { flags |= FLAG_NAN; ymax = 0.0f; }
    else ymax = scale_y<DT>(f32_of_key(bk), pl.T);  // scaling is monotone
    if (ymax == INFINITY) flags |= FLAG_PINF;
    if (flags) {
        if (tid == 0) { cs->xkey = bk; cs->xarg = bi; cs->ymax = ymax; cs->flags = flags; cs->ncand = 0; cs->S = 0.0; }
        return;
    }

    if (pl.mode == M_SMALLK) {
        const uint32_t kneg = row_key(-INFINITY, DT);
        uint32_t key[EPT];
        uint32_t nfin = 0;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int64_t j = idx_of(i);
            key[i] = (j < V) ? row_key(scale_y<DT>(x[i], pl.T), DT) : 0u;
            nfin += key[i] > kneg ? 1u : 0u;
        }
        nfin = block_sum<K1_THREADS>(nfin, s_red_u);
        // threshold: candidates are the finite elements with key >= thr
        uint32_t thr = kneg + 1u;
        if (nfin > (uint32_t)pl.kk) {
            uint32_t prefix = 0u, rem = (uint32_t)pl.kk;
            const int nlev = DT == F32 ? 4 : 2;
            for (int lev = 0; lev < nlev; ++lev) {
                const int shift = 24 - 8 * lev;
                s_u[tid] = 0u;
                __syncthreads();
#pragma unroll
                for (int i = 0; i < EPT; ++i) {
                    const uint32_t k = key[i];
                    bool in = k > kneg && (lev == 0 || (k >> (shift + 8)) == (prefix >> (shift + 8)));
                    if (in) atomicAdd(&s_u[(k >> shift) & 255u], 1u);
                }
                __syncthreads();
                if (wave_id() == 0) {
                    uint32_t above;
                    int d = wave_find_desc<uint32_t>(s_u, 256, rem, &above);
                    if (lane_id() == 0) { s_bcast[0] = (uint32_t)d; s_bcast[1] = above; s_bcast[2] = s_u[d]; }
                }
                __syncthreads();
                const uint32_t d = s_bcast[0], above = s_bcast[1], incnt = s_bcast[2];
                rem -= above;
                prefix |= d << shift;
                __syncthreads();
                if (incnt == rem) break;  // the whole bin is inside the top k'
            }
            thr = prefix;
        }
        uint32_t mine = 0;
#pragma unroll
        for (int i = 0; i < EPT; ++i) mine += (key[i] > kneg && key[i] >= thr) ? 1u : 0u;
        uint32_t total;
        uint32_t off = block_excl_scan<K1_THREADS>(mine, s_red_u, &total);
        if (total <= (uint32_t)CAND_CAP) {
            Cand *cand = reinterpret_cast<Cand *>(ws + L.cand) + ((size_t)row * L.G + chunk) * CAND_CAP;
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                if (key[i] > kneg && key[i] >= thr) {
                    Cand c; c.key = key[i]; c.idx = (int32_t)idx_of(i);
                    cand[off++] = c;
                }
            }
        }
        if (tid == 0) {
            cs->xkey = bk; cs->xarg = bi; cs->ymax = ymax; cs->flags = 0;
            cs->ncand = total <= (uint32_t)CAND_CAP ? total : NCAND_OVERFLOW; cs->S = 0.0;
        }
        return;
    }

    // M_TOPP / M_LARGEK / M_TEMP: float64 softmax mass relative to the chunk max
    const bool hist = pl.mode != M_TEMP;
    if (hist) { s_u[tid] = 0u; s_d[tid] = 0.0; }
    __syncthreads();
    double S = 0.0;
    const double ym = (double)ymax;
    const bool allneg = (ymax == -INFINITY);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int64_t j = idx_of(i);
        if (j < V) {
            const float y = scale_y<DT>(x[i], pl.T);
            const double e = allneg ? 0.0 : exp((double)y - ym);
            S += e;
            if (hist) {
                const uint32_t b = row_key(y, DT) >> 24;
                atomicAdd(&s_u[b], 1u);
                atomicAdd(&s_d[b], e);
            }
        }
    }
    S = block_sum<K1_THREADS>(S, s_red_d);
    if (hist) {
        uint32_t *gc = reinterpret_cast<uint32_t *>(ws + L.l1cnt) + ((size_t)row * L.G + chunk) * 256;
        double *gm = reinterpret_cast<double *>(ws + L.l1mass) + ((size_t)row * L.G + chunk) * 256;
        gc[tid] = s_u[tid];
        gm[tid] = s_d[tid];
    }
    if (tid == 0) { cs->xkey = bk; cs->xarg = bi; cs->ymax = ymax; cs->flags = 0; cs->ncand = 0; cs->S = S; }
}

// ------------------------------------------------------------------ K2: finalize

struct K2Shared {
    union {
        struct { uint32_t cnt[4096]; double mass[4096]; } h;                       // 48 KB
        struct { uint64_t sk[SURV_CAP]; double e[SURV_CAP]; uint64_t sk2[SURV_CAP]; } s;  // 96 KB
        struct { uint32_t cnt[RUN_CAP]; uint32_t rkey[RUN_CAP]; uint32_t rcnt[RUN_CAP]; float rp[RUN_CAP]; } r;  // 64 KB
        struct { int32_t idx[TIE_CAP]; } t;
    } u;
    double l1m[256];
    uint32_t l1c[256];
    double cw[G_MAX];          // per-chunk kept weight
    double chs[G_MAX];         // per-chunk rescale exp(ymax_c - m)
    double red_d[K2_WAVES + 1];
    float red_f[K2_WAVES + 1];
    int64_t red_l[K2_WAVES + 1];
    uint32_t red_u[K2_WAVES + 1];
    int32_t red_i[K2_WAVES + 1];
    uint64_t red_q[K2_WAVES + 1];
    uint32_t bu[8];
    int32_t bi[8];
    double bd[8];
    float bf[8];
};

struct K2Ctx {
    const char *rowp;
    int64_t V;
    int vec_ok;
    float T;
    float m;          // row max of y
    int G;
    int ept;
    int64_t CH;
};

// rk(x) = row key of the scaled value of raw x
template <int DT> __device__ __forceinline__ uint32_t rk_of_xkey(uint32_t xk, float T)
{
    return row_key(scale_y<DT>(f32_of_key(xk), T), DT);
}

// Smallest raw key xk (over all non-NaN floats) with rk(xk) >= target
// (0xff800001 if none).  One wave, 64-ary search.
template <int DT> __device__ uint32_t x_lower(uint32_t target, float T)
{
    const uint32_t XLO = 0x007fffffu, XHI = 0xff800000u;  // -inf .. +inf
    if (rk_of_xkey<DT>(XLO, T) >= target) return XLO;
    if (rk_of_xkey<DT>(XHI, T) < target) return XHI + 1u;
    uint64_t lo = XLO, hi = XHI;  // pred(lo) false, pred(hi) true
    const int l = lane_id();
    while (hi - lo > 1) {
        uint64_t step = (hi - lo) / 64;
        if (step == 0) step = 1;
        uint64_t p = lo + (uint64_t)(l + 1) * step;
        bool pred = p >= hi ? true : (rk_of_xkey<DT>((uint32_t)p, T) >= target);
        uint64_t mask = __ballot(pred);
        if (mask == 0ull) { lo = lo + 64 * step; continue; }
        int f = __builtin_ctzll(mask);
        uint64_t nhi = lo + (uint64_t)(f + 1) * step;
        if (nhi < hi) hi = nhi;
        lo = lo + (uint64_t)f * step;
    }
    return (uint32_t)hi;
}

// Largest raw key xk with rk(xk) <= target (XLO-1 if none).
template <int DT> __device__ uint32_t x_upper(uint32_t target, float T)
{
    if (target == 0xffffffffu) return 0xff800000u;
    uint32_t lb = x_lower<DT>(target + 1u, T);
    return lb - 1u;
}

// One pass over the row; calls f(j, y, key) for elements whose raw key lies in
// [xklo, xkhi].  All threads of the block must call it.
template <int DT, class F>
__device__ void rescan(const K2Ctx &c, uint32_t xklo, uint32_t xkhi, F &&f)
{
    constexpr int VEC = Traits<DT>::VEC;
    if (xklo > xkhi) return;
    for (int64_t t0 = 0; t0 < c.V; t0 += (int64_t)K2_THREADS * VEC) {
        const int64_t j0 = t0 + (int64_t)threadIdx.x * VEC;
        float xs[VEC];
        if (c.vec_ok && j0 + VEC <= c.V) loadvec<DT>(c.rowp, j0, xs);
        else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) xs[e] = (j0 + e < c.V) ? load1<DT>(c.rowp, j0 + e) : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            if (j0 + e < c.V) {
                const uint32_t xk = key_of_f32(xs[e]);
                if (xk >= xklo && xk <= xkhi) {
                    const float y = scale_y<DT>(xs[e], c.T);
                    f(j0 + e, y, row_key(y, DT));
                }
            }
        }
    }
}

// Raw-key interval covering the scaled-key interval [klo, khi].
template <int DT> __device__ void x_interval(K2Shared &sh, uint32_t klo, uint32_t khi, float T, uint32_t *xlo, uint32_t *xhi)
{
    __syncthreads();
    if (wave_id() == 0) {
        uint32_t a = x_lower<DT>(klo, T);
        uint32_t b = x_upper<DT>(khi, T);
        if (lane_id() == 0) { sh.bu[6] = a; sh.bu[7] = b; }
    }
    __syncthreads();
    *xlo = sh.bu[6];
    *xhi = sh.bu[7];
    __syncthreads();
}

__device__ __forceinline__ bool kept_by_cut(uint32_t key, int64_t j, uint32_t cut_key, int32_t cut_i)
{
    return key > cut_key || (key == cut_key && j <= (int64_t)cut_i);
}

// Radix descent over the row keys >= floor_key.  Level 1 comes from the
// 256-bin histogram in sh.l1c / sh.l1m; later levels re-read the row.
// by_mass: find the key where the running mass (descending) reaches target;
// otherwise the key where the running count reaches target.  Returns the
// fully resolved key; *acc = mass (or count) strictly above it; *kcnt =
// number of elements holding exactly that key.
template <int DT>
__device__ __noinline__ uint32_t descend(K2Shared &sh, const K2Ctx &c, bool by_mass, double target, uint32_t floor_key,
                            double *acc_out, uint32_t *kcnt)
{
    double acc = 0.0;
    uint32_t prefix = 0u;
    // level 1
    __syncthreads();
    if (wave_id() == 0) {
        int b;
        if (by_mass) { double ab; b = wave_find_desc<double>(sh.l1m, 256, target, &ab); if (lane_id() == 0) sh.bd[0] = ab; }
        else { uint32_t ab; b = wave_find_desc<uint32_t>(sh.l1c, 256, (uint32_t)target, &ab); if (lane_id() == 0) sh.bd[0] = (double)ab; }
        if (lane_id() == 0) { sh.bu[0] = (uint32_t)b; sh.bu[1] = sh.l1c[b]; }
    }
    __syncthreads();
    prefix = sh.bu[0] << 24;
    acc = sh.bd[0];
    uint32_t bincnt = sh.bu[1];
    const int nlev = DT == F32 ? 2 : 1;
    for (int lev = 0; lev < nlev; ++lev) {
        const int bits = DT == F32 ? 12 : 8;
        const int shift = DT == F32 ? (lev == 0 ? 12 : 0) : 16;
        const int nb = 1 << bits;
        const uint32_t freemask = (lev == 0) ? 0x00ffffffu : 0x00000fffu;
        for (int i = threadIdx.x; i < nb; i += K2_THREADS) { sh.u.h.cnt[i] = 0u; sh.u.h.mass[i] = 0.0; }
        uint32_t klo = prefix, khi = prefix | freemask;
        if (klo < floor_key) klo = floor_key;
        uint32_t xlo, xhi;
        x_interval<DT>(sh, klo, khi, c.T, &xlo, &xhi);
        const double m = (double)c.m;
        rescan<DT>(c, xlo, xhi, [&](int64_t, float y, uint32_t key) {
            if (key < klo || key > khi) return;
            const uint32_t b = (key >> shift) & (uint32_t)(nb - 1);
            atomicAdd(&sh.u.h.cnt[b], 1u);
            if (by_mass) atomicAdd(&sh.u.h.mass[b], exp((double)y - m));
        });
        __syncthreads();
        if (wave_id() == 0) {
            int b;
            if (by_mass) { double ab; b = wave_find_desc<double>(sh.u.h.mass, nb, target - acc, &ab); if (lane_id() == 0) sh.bd[0] = ab; }
            else { uint32_t ab; b = wave_find_desc<uint32_t>(sh.u.h.cnt, nb, (uint32_t)(target - acc), &ab); if (lane_id() == 0) sh.bd[0] = (double)ab; }
            if (lane_id() == 0) { sh.bu[0] = (uint32_t)b; sh.bu[1] = sh.u.h.cnt[b]; }
        }
        __syncthreads();
        prefix |= sh.bu[0] << shift;
        acc += sh.bd[0];
        bincnt = sh.bu[1];
        __syncthreads();
    }
    *acc_out = acc;
    *kcnt = bincnt;
    return prefix;
}

// Index of the t-th (1-based) element, in index order, whose scaled key is
// exactly `key`.
template <int DT>
__device__ __noinline__ int32_t tie_index(K2Shared &sh, const K2Ctx &c, uint32_t key, uint32_t t)
{
    uint32_t xlo, xhi;
    x_interval<DT>(sh, key, key, c.T, &xlo, &xhi);
    if (threadIdx.x == 0) sh.bu[2] = 0u;
    __syncthreads();
    rescan<DT>(c, xlo, xhi, [&](int64_t j, float, uint32_t k) {
        if (k != key) return;
        uint32_t p = atomicAdd(&sh.bu[2], 1u);
        if (p < (uint32_t)TIE_CAP) sh.u.t.idx[p] = (int32_t)j;
    });
    __syncthreads();
    const uint32_t n = sh.bu[2];
    if (n <= (uint32_t)TIE_CAP) {
        // rank of each collected index; the one with rank t-1 is the answer
        for (uint32_t i = threadIdx.x; i < n; i += K2_THREADS) {
            const int32_t v = sh.u.t.idx[i];
            uint32_t r = 0;
            for (uint32_t q = 0; q < n; ++q) r += sh.u.t.idx[q] < v ? 1u : 0u;
            if (r == t - 1u) sh.bi[0] = v;
        }
        __syncthreads();
        int32_t res = sh.bi[0];
        __syncthreads();
        return res;
    }
    // many ties: bisect on the index with counting passes
    int64_t lo = 0, hi = c.V - 1;  // find smallest idx with count(ties <= idx) >= t
    while (lo < hi) {
        const int64_t mid = lo + (hi - lo) / 2;
        if (threadIdx.x == 0) sh.bu[3] = 0u;
        __syncthreads();
        uint32_t mine = 0;
        rescan<DT>(c, xlo, xhi, [&](int64_t j, float, uint32_t k) { if (k == key && j <= mid) mine++; });
        mine = block_sum<K2_THREADS>(mine, sh.red_u);
        if (mine >= t) hi = mid; else lo = mid + 1;
    }
    return (int32_t)lo;
}

// Sequential walk of the 16-bit top-p chain over runs (one thread).  On
// return *found says whether some rank triggered removal; then the cut keeps
// `*t_keep` elements of run *run_at (0 means the cut is the previous run).
__device__ bool chain_walk(const uint32_t *rkey, const uint32_t *rcnt, const float *rp, int nruns, float &F,
                           float thr16, int dt, int *run_at, uint32_t *t_keep)
{
    for (int r = 0; r < nruns; ++r) {
        const float p = rp[r];
        const uint32_t n = rcnt[r];
        const float Fend = chain_add_n(F, p, n);
        if (chain_E(Fend, p, dt) >= thr16) {
            uint32_t lo = 0, hi = n - 1;  // first t in [0, n) whose E triggers
            while (lo < hi) {
                const uint32_t mid = lo + (hi - lo) / 2;
                if (chain_E(chain_add_n(F, p, (uint64_t)mid + 1), p, dt) >= thr16) hi = mid; else lo = mid + 1;
            }
            *run_at = r;
            *t_keep = lo;
            return true;
        }
        F = Fend;
    }
    return false;
}

// Per-chunk kept weight for the draw, then the inverse-CDF pick inside the
// chosen chunk.  sh.cw[c] must hold the kept weight of chunk c.
template <int DT>
__device__ __noinline__ int64_t draw_from_chunks(K2Shared &sh, const K2Ctx &c, float u, uint32_t cut_key, int32_t cut_i, double *S_out)
{
    __syncthreads();
    if (threadIdx.x == 0) {
        double S = 0.0;
        for (int g = 0; g < c.G; ++g) S += sh.cw[g];
        double target = (double)u * S;
        double cum = 0.0;
        int gsel = -1;
        for (int g = 0; g < c.G; ++g) {
            if (sh.cw[g] > 0.0) {
                if (cum + sh.cw[g] > target) { gsel = g; break; }
                cum += sh.cw[g];
            }
        }
        if (gsel < 0) {  // rounding: last chunk with weight
            for (int g = c.G - 1; g >= 0; --g) if (sh.cw[g] > 0.0) { gsel = g; break; }
            cum = 0.0;
            for (int g = 0; g < gsel; ++g) cum += sh.cw[g];
            target = cum + sh.cw[gsel];  // pick the last kept element of that chunk
        }
        sh.bd[0] = S;
        sh.bd[1] = target - cum;
        sh.bi[0] = gsel;
    }
    __syncthreads();
    const double S = sh.bd[0], resid = sh.bd[1];
    const int g = sh.bi[0];
    *S_out = S;
    if (g < 0) return -1;
    // scan chunk g in index order: thread t owns a contiguous slice
    const int64_t cbeg = (int64_t)g * c.CH;
    const int64_t cend = cbeg + c.CH < c.V ? cbeg + c.CH : c.V;
    const int64_t per = (c.CH + K2_THREADS - 1) / K2_THREADS;
    const int64_t jb = cbeg + (int64_t)threadIdx.x * per;
    const int64_t je = jb + per < cend ? jb + per : cend;
    const double m = (double)c.m;
    double local = 0.0;
    int64_t lastk = -1;
    for (int64_t j = jb; j < je; ++j) {
        const float y = scale_y<DT>(load1<DT>(c.rowp, j), c.T);
        const uint32_t key = row_key(y, DT);
        if (y != -INFINITY && kept_by_cut(key, j, cut_key, cut_i)) { local += exp((double)y - m); lastk = j; }
    }
    double tot;
    const double before = block_excl_scan<K2_THREADS>(local, sh.red_d, &tot);
    if (threadIdx.x == 0) { sh.red_q[0] = 0xffffffffffffffffull; }
    __syncthreads();
    if (local > 0.0 && before <= resid && resid < before + local) {
        double run = before;
        int64_t pick = lastk;
        for (int64_t j = jb; j < je; ++j) {
            const float y = scale_y<DT>(load1<DT>(c.rowp, j), c.T);
            const uint32_t key = row_key(y, DT);
            if (y != -INFINITY && kept_by_cut(key, j, cut_key, cut_i)) {
                run += exp((double)y - m);
                if (run > resid) { pick = j; break; }
            }
        }
        atomicMin((unsigned long long *)&sh.red_q[0], (unsigned long long)pick);
    }
    __syncthreads();
    uint64_t pk = sh.red_q[0];
    if (pk == 0xffffffffffffffffull) {
        // residual beyond the recomputed total: last kept element of the chunk
        int64_t lk = block_max<K2_THREADS>((int64_t)lastk, sh.red_l);
        return lk;
    }
    __syncthreads();
    return (int64_t)pk;
}

// Bitonic sort (descending) of n_pow2 uint64 keys in LDS by the whole block.
__device__ void bitonic_desc(uint64_t *a, int n)
{
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += K2_THREADS) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const bool desc = (i & k) == 0;
                    const uint64_t x = a[i], y = a[ixj];
                    if (desc ? (x < y) : (x > y)) { a[i] = y; a[ixj] = x; }
                }
            }
            __syncthreads();
        }
    }
}

template <int DT>
__device__ void write_row(RowOut *ro, int64_t *out_ids, int32_t *out_status, int row, int64_t id, int status, int mode,
                          float m, uint32_t cut_key, int32_t cut_i, double S)
{
    if (threadIdx.x == 0) {
        ro->id = status == MIS_ROW_OK ? id : -1;
        ro->status = status;
        ro->mode = mode;
        ro->m = m;
        ro->cut_key = cut_key;
        ro->cut_i = cut_i;
        ro->S = S;
        out_ids[row] = status == MIS_ROW_OK ? id : -1;
        if (out_status) out_status[row] = status;
    }
}

// generic full-row path: top-k by count descent (k' may be any size) and/or
// top-p, with every histogram level re-read from the row.
template <int DT>
__device__ __noinline__ void final_generic(K2Shared &sh, K2Ctx &c, const RowPlan &pl, bool have_l1, RowOut *ro,
                              int64_t *out_ids, int32_t *out_status, int row, const uint32_t *gl1c, const double *gl1m);

template <int DT>
__device__ __noinline__ void topp_cut(K2Shared &sh, const K2Ctx &c, const RowPlan &pl, uint32_t floor_key, double S,
                         uint32_t *cut_key, int32_t *cut_i, int *status);

template <int DT>
__global__ __launch_bounds__(K2_THREADS) void k_final(const char *__restrict__ logits, int64_t V, int64_t stride_bytes,
                                                      int vec_ok, const mis_row_params *__restrict__ params, Layout L,
                                                      char *__restrict__ ws, int64_t *__restrict__ out_ids,
                                                      int32_t *__restrict__ out_status)
{
    __shared__ K2Shared sh;
    const int row = blockIdx.x;
    const RowPlan pl = plan_row(params[row], V);
    RowOut *ro = reinterpret_cast<RowOut *>(ws + L.rowout) + row;
    const ChunkSum *cs = reinterpret_cast<const ChunkSum *>(ws + L.chunks) + (size_t)row * L.G;
    const uint32_t kneg = row_key(-INFINITY, DT);

    if (pl.mode == M_BAD) {
        write_row<DT>(ro, out_ids, out_status, row, -1, MIS_ROW_BAD_PARAM, pl.mode, 0.f, 0u, 0, 0.0);
        return;
    }
    // ---- merge chunk summaries
    uint32_t bk = 0u; int32_t bi = IDX_ALL; uint32_t fl = 0u; float ym = -INFINITY;
    for (int g = threadIdx.x; g < L.G; g += K2_THREADS) {
        const ChunkSum s = cs[g];
        if (s.xkey > bk || (s.xkey == bk && s.xarg < bi)) { bk = s.xkey; bi = s.xarg; }
        fl |= s.flags;
        ym = s.ymax > ym ? s.ymax : ym;
    }
    wave_argmax(bk, bi);
    if (lane_id() == 0) { sh.red_u[wave_id()] = bk; sh.red_i[wave_id()] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < K2_WAVES; ++w)
            if (sh.red_u[w] > bk || (sh.red_u[w] == bk && sh.red_i[w] < bi)) { bk = sh.red_u[w]; bi = sh.red_i[w]; }
        sh.bu[0] = bk; sh.bi[0] = bi;
    }
    __syncthreads();
    bk = sh.bu[0]; bi = sh.bi[0];
    __syncthreads();
    if (pl.mode == M_GREEDY) {
        write_row<DT>(ro, out_ids, out_status, row, bi, MIS_ROW_OK, pl.mode, 0.f, 0u, bi, 1.0);
        return;
    }
    fl = block_sum<K2_THREADS>(fl ? 1u : 0u, sh.red_u);  // chunks carrying NaN / +inf
    const float m = block_max<K2_THREADS>(ym, sh.red_f);
    if (fl != 0u || m == -INFINITY || !(m == m)) {
        write_row<DT>(ro, out_ids, out_status, row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
        return;
    }

    K2Ctx c;
    c.rowp = logits + (int64_t)row * stride_bytes;
    c.V = V; c.vec_ok = vec_ok; c.T = pl.T; c.m = m; c.G = L.G; c.ept = L.ept;
    c.CH = (int64_t)K1_THREADS * L.ept;
    const double md = (double)m;
    for (int g = threadIdx.x; g < L.G; g += K2_THREADS) sh.chs[g] = exp((double)cs[g].ymax - md);
    __syncthreads();

    if (pl.mode == M_TEMP) {
        for (int g = threadIdx.x; g < L.G; g += K2_THREADS) sh.cw[g] = cs[g].ymax == -INFINITY ? 0.0 : cs[g].S * sh.chs[g];
        double S;
        int64_t id = draw_from_chunks<DT>(sh, c, pl.u, kneg, -1, &S);
        write_row<DT>(ro, out_ids, out_status, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, kneg, -1, S);
        return;
    }

    const uint32_t *gl1c = reinterpret_cast<const uint32_t *>(ws + L.l1cnt) + (size_t)row * L.G * 256;
    const double *gl1m = reinterpret_cast<const double *>(ws + L.l1mass) + (size_t)row * L.G * 256;

    if (pl.mode == M_SMALLK) {
        // ---- candidate path
        uint32_t ncand_tot = 0, ovf = 0;
        for (int g = threadIdx.x; g < L.G; g += K2_THREADS) {
            const uint32_t n = cs[g].ncand;
            if (n == NCAND_OVERFLOW) ovf = 1; else ncand_tot += n;
        }
        ovf = block_sum<K2_THREADS>(ovf, sh.red_u);
        ncand_tot = block_sum<K2_THREADS>(ncand_tot, sh.red_u);
        if (ovf == 0) {
            const Cand *cand = reinterpret_cast<const Cand *>(ws + L.cand) + (size_t)row * L.G * CAND_CAP;
            // k'-th largest key among the candidates
            // fewer than k' candidates means fewer than k' finite elements in
            // the row: every finite element survives
            uint32_t thr = kneg + 1u;
            if (ncand_tot >= (uint32_t)pl.kk) {
                uint32_t prefix = 0u, rem = (uint32_t)pl.kk;
                const int nlev = DT == F32 ? 4 : 2;
                for (int lev = 0; lev < nlev; ++lev) {
                    const int shift = 24 - 8 * lev;
                    for (int i = threadIdx.x; i < 256; i += K2_THREADS) sh.u.h.cnt[i] = 0u;
                    __syncthreads();
                    for (int g = 0; g < L.G; ++g) {
                        const uint32_t n = cs[g].ncand;
                        for (uint32_t i = threadIdx.x; i < n; i += K2_THREADS) {
                            const uint32_t k = cand[(size_t)g * CAND_CAP + i].key;
                            if (lev == 0 || (k >> (shift + 8)) == (prefix >> (shift + 8))) atomicAdd(&sh.u.h.cnt[(k >> shift) & 255u], 1u);
                        }
                    }
                    __syncthreads();
                    if (wave_id() == 0) {
                        uint32_t above;
                        int d = wave_find_desc<uint32_t>(sh.u.h.cnt, 256, rem, &above);
                        if (lane_id() == 0) { sh.bu[0] = (uint32_t)d; sh.bu[1] = above; sh.bu[2] = sh.u.h.cnt[d]; }
                    }
                    __syncthreads();
                    rem -= sh.bu[1];
                    prefix |= sh.bu[0] << shift;
                    __syncthreads();
                    // no early exit here: the threshold is applied to the whole
                    // row, so it must be the exact k'-th key
                }
                thr = prefix;
            }
            // survivors into LDS
            if (threadIdx.x == 0) sh.bu[3] = 0u;
            __syncthreads();
            for (int g = 0; g < L.G; ++g) {
                const uint32_t n = cs[g].ncand;
                for (uint32_t i = threadIdx.x; i < n; i += K2_THREADS) {
                    const Cand cd = cand[(size_t)g * CAND_CAP + i];
                    if (cd.key >= thr) {
                        const uint32_t p = atomicAdd(&sh.bu[3], 1u);
                        if (p < (uint32_t)SURV_CAP)
                            sh.u.s.sk[p] = ((uint64_t)cd.key << 32) | (uint64_t)(0xffffffffu - (uint32_t)cd.idx);
                    }
                }
            }
            __syncthreads();
            const uint32_t ns = sh.bu[3];
            __syncthreads();
            if (ns <= (uint32_t)SURV_CAP && ns > 0) {
                int npow = 1;
                while (npow < (int)ns) npow <<= 1;
                for (int i = threadIdx.x; i < npow; i += K2_THREADS) if (i >= (int)ns) sh.u.s.sk[i] = 0ull;
                __syncthreads();
                bitonic_desc(sh.u.s.sk, npow);  // key desc, idx asc
                for (int i = threadIdx.x; i < (int)ns; i += K2_THREADS)
                    sh.u.s.e[i] = exp((double)value_of_row_key((uint32_t)(sh.u.s.sk[i] >> 32), DT) - md);
                __syncthreads();
                uint32_t nkeep = ns;
                int status = MIS_ROW_OK;
                if (pl.topp) {
                    if (DT == F32) {
                        // exclusive prefix of the masses in sorted order
                        double Stot = 0.0;
                        for (int i0 = 0; i0 < (int)ns; i0 += K2_THREADS) {
                            const int i = i0 + threadIdx.x;
                            double v = i < (int)ns ? sh.u.s.e[i] : 0.0, tot;
                            double ex = block_excl_scan<K2_THREADS>(v, sh.red_d, &tot);
                            if (i < (int)ns) sh.u.s.sk2[i] = f64_bits(Stot + ex);
                            Stot += tot;
                        }
                        __syncthreads();
                        const double A = (double)pl.top_p * Stot;
                        uint32_t first = ns;
                        for (int i = threadIdx.x; i < (int)ns; i += K2_THREADS)
                            if (bits_f64(sh.u.s.sk2[i]) >= A) first = first < (uint32_t)i ? first : (uint32_t)i;
                        first = block_min<K2_THREADS>(first, sh.red_u);
                        nkeep = first;
                    } else {
                        // 16-bit chain over runs of equal keys (sorted survivors)
                        if (threadIdx.x == 0) {
                            const float thr16 = rn_dtype(pl.top_p, DT);
                            double Stot = 0.0;
                            for (int i = (int)ns - 1; i >= 0; --i) Stot += sh.u.s.e[i];
                            float F = 0.0f;
                            uint32_t r0 = ns;
                            int i = 0;
                            while (i < (int)ns) {
                                const uint32_t key = (uint32_t)(sh.u.s.sk[i] >> 32);
                                int jn = i + 1;
                                while (jn < (int)ns && (uint32_t)(sh.u.s.sk[jn] >> 32) == key) ++jn;
                                const float p = rn_dtype((float)(sh.u.s.e[i] / Stot), DT);
                                const uint32_t n = (uint32_t)(jn - i);
                                const float Fend = chain_add_n(F, p, n);
                                if (chain_E(Fend, p, DT) >= thr16) {
                                    uint32_t lo = 0, hi = n - 1;
                                    while (lo < hi) {
                                        const uint32_t mid = lo + (hi - lo) / 2;
                                        if (chain_E(chain_add_n(F, p, (uint64_t)mid + 1), p, DT) >= thr16) hi = mid; else lo = mid + 1;
                                    }
                                    r0 = (uint32_t)i + lo;
                                    break;
                                }
                                F = Fend;
                                i = jn;
                            }
                            sh.bu[4] = r0;
                        }
                        __syncthreads();
                        nkeep = sh.bu[4];
                        __syncthreads();
                    }
                    if (nkeep == 0) status = MIS_ROW_INVALID;
                }
                if (status == MIS_ROW_OK) {
                    uint32_t cut_key;
                    int32_t cut_i;
                    if (pl.topp) {
                        const uint64_t q = sh.u.s.sk[nkeep - 1];
                        cut_key = (uint32_t)(q >> 32);
                        cut_i = (int32_t)(0xffffffffu - (uint32_t)q);
                    } else {
                        cut_key = thr; cut_i = IDX_ALL;
                    }
                    // kept set in index order: sk2 = idx << 32 | slot (ascending)
                    int npw = 1;
                    while (npw < (int)nkeep) npw <<= 1;
                    for (int i = threadIdx.x; i < npw; i += K2_THREADS) {
                        uint64_t v;
                        if (i < (int)nkeep) v = ((uint64_t)(0xffffffffu - (uint32_t)sh.u.s.sk[i]) << 32) | (uint64_t)i;
                        else v = 0xffffffffffffffffull;
                        sh.u.s.sk2[i] = ~v;  // sort descending on complement = ascending on v
                    }
                    __syncthreads();
                    bitonic_desc(sh.u.s.sk2, npw);
                    double SK = 0.0;
                    for (int i0 = 0; i0 < (int)nkeep; i0 += K2_THREADS) {
                        const int i = i0 + threadIdx.x;
                        double v = 0.0;
                        if (i < (int)nkeep) v = sh.u.s.e[(uint32_t)(~sh.u.s.sk2[i])];
                        double tot;
                        (void)block_excl_scan<K2_THREADS>(v, sh.red_d, &tot);
                        SK += tot;
                    }
                    const double target = (double)pl.u * SK;
                    double run = 0.0;
                    int64_t pick = -1;
                    if (threadIdx.x == 0) {
                        for (int i = 0; i < (int)nkeep; ++i) {
                            const uint64_t v = ~sh.u.s.sk2[i];
                            const uint32_t slot = (uint32_t)v;
                            run += sh.u.s.e[slot];
                            pick = (int64_t)(v >> 32);
                            if (run > target) break;
                        }
                        sh.bd[2] = (double)pick;
                    }
                    __syncthreads();
                    pick = (int64_t)sh.bd[2];
                    write_row<DT>(ro, out_ids, out_status, row, pick, MIS_ROW_OK, pl.mode, m, cut_key, cut_i, SK);
                } else {
                    write_row<DT>(ro, out_ids, out_status, row, -1, status, pl.mode, m, 0u, 0, 0.0);
                }
                return;
            }
        }
        // overflow: fall through to the generic path
        final_generic<DT>(sh, c, pl, false, ro, out_ids, out_status, row, gl1c, gl1m);
        return;
    }

    if (pl.mode == M_LARGEK) {
        final_generic<DT>(sh, c, pl, true, ro, out_ids, out_status, row, gl1c, gl1m);
        return;
    }

    // ---- M_TOPP with chunk histograms
    for (int b = threadIdx.x; b < 256; b += K2_THREADS) {
        double mm = 0.0; uint32_t cc = 0;
        for (int g = 0; g < L.G; ++g) { mm += gl1m[(size_t)g * 256 + b] * sh.chs[g]; cc += gl1c[(size_t)g * 256 + b]; }
        sh.l1m[b] = mm; sh.l1c[b] = cc;
    }
    double S = 0.0;
    for (int g = threadIdx.x; g < L.G; g += K2_THREADS) S += cs[g].ymax == -INFINITY ? 0.0 : cs[g].S * sh.chs[g];
    S = block_sum<K2_THREADS>(S, sh.red_d);
    uint32_t cut_key; int32_t cut_i; int status;
    topp_cut<DT>(sh, c, pl, 0u, S, &cut_key, &cut_i, &status);
    if (status != MIS_ROW_OK) {
        write_row<DT>(ro, out_ids, out_status, row, -1, status, pl.mode, m, 0u, 0, 0.0);
        return;
    }
    // per-chunk kept weight: whole L1 bins above the cut's bin from the chunk
    // histograms, the cut's bin from one filtered re-read
    const uint32_t cb = cut_key >> 24;
    for (int g = threadIdx.x; g < L.G; g += K2_THREADS) {
        double w = 0.0;
        for (int b = cb + 1; b < 256; ++b) w += gl1m[(size_t)g * 256 + b];
        sh.cw[g] = w * sh.chs[g];
    }
    __syncthreads();
    {
        uint32_t xlo, xhi;
        x_interval<DT>(sh, cut_key, (cb << 24) | 0x00ffffffu, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t j, float y, uint32_t key) {
            if ((key >> 24) != cb) return;
            if (kept_by_cut(key, j, cut_key, cut_i)) atomicAdd(&sh.cw[j / c.CH], exp((double)y - md));
        });
    }
    double SK;
    int64_t id = draw_from_chunks<DT>(sh, c, pl.u, cut_key, cut_i, &SK);
    write_row<DT>(ro, out_ids, out_status, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, cut_key, cut_i, SK);
}

// Top-p cut over elements with key >= floor_key.  sh.l1m / sh.l1c must hold
// the 256-bin histogram of exactly those elements, S their total weight.
template <int DT>
__device__ __noinline__ void topp_cut(K2Shared &sh, const K2Ctx &c, const RowPlan &pl, uint32_t floor_key, double S,
                         uint32_t *cut_key, int32_t *cut_i, int *status)
{
    const double md = (double)c.m;
    *status = MIS_ROW_OK;
    if (DT == F32) {
        const double A = (double)pl.top_p * S;
        double acc;
        uint32_t kc;
        const uint32_t key = descend<DT>(sh, c, true, A, floor_key, &acc, &kc);
        const double e = exp((double)value_of_row_key(key, DT) - md);
        // ties kept: smallest t >= 1 with acc + t*e >= A
        uint32_t t;
        {
            double tt = ceil((A - acc) / e);
            if (!(tt >= 1.0)) tt = 1.0;
            if (tt > (double)kc) tt = (double)kc;
            t = (uint32_t)tt;
            while (t > 1 && acc + (double)(t - 1) * e >= A) --t;
            while (t < kc && acc + (double)t * e < A) ++t;
        }
        *cut_key = key;
        *cut_i = (t >= kc) ? IDX_ALL : tie_index<DT>(sh, c, key, t);
        return;
    }
    // 16-bit: walk the rounding chain over runs of equal keys, region by region
    const float thr16 = rn_dtype(pl.top_p, DT);
    const uint32_t kneg = row_key(-INFINITY, DT);
    float F = 0.0f;
    int b_hi = 255;
    while (b_hi >= 0 && sh.l1c[b_hi] == 0u) --b_hi;
    uint32_t prev_key = 0u;
    bool have_prev = false;
    while (b_hi >= 0) {
        // region: up to REGION_BINS L1 bins from b_hi down
        int b_lo = b_hi - REGION_BINS + 1;
        if (b_lo < 0) b_lo = 0;
        for (int i = threadIdx.x; i < RUN_CAP; i += K2_THREADS) sh.u.r.cnt[i] = 0u;
        uint32_t klo = (uint32_t)b_lo << 24, khi = ((uint32_t)b_hi << 24) | 0x00ffffffu;
        if (klo < floor_key) klo = floor_key;
        if (klo <= kneg) klo = kneg + 1u;  // -inf never enters the chain
        uint32_t xlo, xhi;
        x_interval<DT>(sh, klo, khi, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float, uint32_t key) {
            if (key < klo || key > khi) return;
            // descending position: (b_hi - L1) * 256 + (255 - byte2)
            const uint32_t pos = (uint32_t)(b_hi - (int)(key >> 24)) * 256u + (255u - ((key >> 16) & 255u));
            atomicAdd(&sh.u.r.cnt[pos], 1u);
        });
        __syncthreads();
        // compact non-empty positions into runs (descending keys)
        const int npos = (b_hi - b_lo + 1) * 256;
        int nruns_total = 0;
        for (int i0 = 0; i0 < npos; i0 += K2_THREADS) {
            const int i = i0 + threadIdx.x;
            const uint32_t cnt = i < npos ? sh.u.r.cnt[i] : 0u;
            uint32_t tot;
            const uint32_t off = block_excl_scan<K2_THREADS>(cnt ? 1u : 0u, sh.red_u, &tot);
            if (cnt) {
                const uint32_t L1 = (uint32_t)(b_hi - i / 256), b2 = 255u - (uint32_t)(i % 256);
                const uint32_t key = (L1 << 24) | (b2 << 16);
                const int r = nruns_total + (int)off;
                sh.u.r.rkey[r] = key;
                sh.u.r.rcnt[r] = cnt;
                sh.u.r.rp[r] = rn_dtype((float)(exp((double)value_of_row_key(key, DT) - md) / S), DT);
            }
            nruns_total += (int)tot;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int run_at = -1;
            uint32_t tk = 0;
            float Fw = F;
            bool found = chain_walk(sh.u.r.rkey, sh.u.r.rcnt, sh.u.r.rp, nruns_total, Fw, thr16, DT, &run_at, &tk);
            sh.bi[1] = found ? 1 : 0;
            sh.bi[2] = run_at;
            sh.bu[4] = tk;
            sh.bf[0] = Fw;
            sh.bu[5] = nruns_total > 0 ? sh.u.r.rkey[nruns_total - 1] : 0u;
            if (found) {
                sh.bu[6] = sh.u.r.rkey[run_at];
                sh.bu[7] = sh.u.r.rcnt[run_at];
                sh.bu[2] = run_at > 0 ? sh.u.r.rkey[run_at - 1] : 0u;
                sh.bi[3] = run_at > 0 ? 1 : 0;
            }
        }
        __syncthreads();
        const bool found = sh.bi[1] != 0;
        if (found) {
            const uint32_t tk = sh.bu[4];
            const uint32_t rkey = sh.bu[6], rcnt = sh.bu[7];
            const bool prev_in_region = sh.bi[3] != 0;
            const uint32_t pkey = sh.bu[2];
            __syncthreads();
            if (tk > 0) {
                *cut_key = rkey;
                *cut_i = (tk >= rcnt) ? IDX_ALL : tie_index<DT>(sh, c, rkey, tk);
            } else if (prev_in_region) {
                *cut_key = pkey; *cut_i = IDX_ALL;
            } else if (have_prev) {
                *cut_key = prev_key; *cut_i = IDX_ALL;
            } else {
                *status = MIS_ROW_INVALID;  // rank 0 removed: nothing left
            }
            return;
        }
        F = sh.bf[0];
        if (nruns_total > 0) { prev_key = sh.bu[5]; have_prev = true; }
        __syncthreads();
        b_hi = b_lo - 1;
        while (b_hi >= 0 && sh.l1c[b_hi] == 0u) --b_hi;
    }
    // nothing triggered: every finite element above the floor is kept
    if (have_prev) { *cut_key = prev_key; *cut_i = IDX_ALL; }
    else *status = MIS_ROW_INVALID;
}

template <int DT>
__device__ __noinline__ void final_generic(K2Shared &sh, K2Ctx &c, const RowPlan &pl, bool have_l1, RowOut *ro,
                              int64_t *out_ids, int32_t *out_status, int row, const uint32_t *gl1c, const double *gl1m)
{
    const double md = (double)c.m;
    const uint32_t kneg = row_key(-INFINITY, DT);
    // 256-bin histogram of the whole row
    if (have_l1) {
        for (int b = threadIdx.x; b < 256; b += K2_THREADS) {
            double mm = 0.0; uint32_t cc = 0;
            for (int g = 0; g < c.G; ++g) { mm += gl1m[(size_t)g * 256 + b] * sh.chs[g]; cc += gl1c[(size_t)g * 256 + b]; }
            sh.l1m[b] = mm; sh.l1c[b] = cc;
        }
    } else {
        for (int b = threadIdx.x; b < 256; b += K2_THREADS) { sh.l1m[b] = 0.0; sh.l1c[b] = 0u; }
        __syncthreads();
        rescan<DT>(c, 0x007fffffu, 0xff800000u, [&](int64_t, float y, uint32_t key) {
            atomicAdd(&sh.l1c[key >> 24], 1u);
            atomicAdd(&sh.l1m[key >> 24], exp((double)y - md));
        });
    }
    __syncthreads();
    // top-k threshold by count
    uint32_t floor_key = kneg + 1u;
    if (pl.kk > 0) {
        double acc; uint32_t kc;
        floor_key = descend<DT>(sh, c, false, (double)pl.kk, 0u, &acc, &kc);
        if (floor_key <= kneg) floor_key = kneg + 1u;
    }
    // histogram and weight of the survivors (key >= floor_key)
    for (int b = threadIdx.x; b < 256; b += K2_THREADS) { sh.l1m[b] = 0.0; sh.l1c[b] = 0u; }
    __syncthreads();
    {
        uint32_t xlo, xhi;
        x_interval<DT>(sh, floor_key, 0xffffffffu, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float y, uint32_t key) {
            if (key < floor_key) return;
            atomicAdd(&sh.l1c[key >> 24], 1u);
            atomicAdd(&sh.l1m[key >> 24], exp((double)y - md));
        });
    }
    __syncthreads();
    double S = 0.0;
    for (int b = threadIdx.x; b < 256; b += K2_THREADS) S += sh.l1m[b];
    S = block_sum<K2_THREADS>(S, sh.red_d);
    uint32_t cut_key = floor_key;
    int32_t cut_i = IDX_ALL;
    int status = MIS_ROW_OK;
    if (pl.topp) topp_cut<DT>(sh, c, pl, floor_key, S, &cut_key, &cut_i, &status);
    if (status != MIS_ROW_OK) {
        write_row<DT>(ro, out_ids, out_status, row, -1, status, pl.mode, c.m, 0u, 0, 0.0);
        return;
    }
    // per-chunk kept weight by a full filtered re-read
    for (int g = threadIdx.x; g < c.G; g += K2_THREADS) sh.cw[g] = 0.0;
    __syncthreads();
    {
        uint32_t xlo, xhi;
        x_interval<DT>(sh, cut_key, 0xffffffffu, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t j, float y, uint32_t key) {
            if (kept_by_cut(key, j, cut_key, cut_i)) atomicAdd(&sh.cw[j / c.CH], exp((double)y - md));
        });
    }
    double SK;
    int64_t id = draw_from_chunks<DT>(sh, c, pl.u, cut_key, cut_i, &SK);
    write_row<DT>(ro, out_ids, out_status, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, c.m, cut_key, cut_i, SK);
}

// ------------------------------------------------------------------ K3: debug emit

template <int DT>
__global__ __launch_bounds__(K3_THREADS) void k_emit(const char *__restrict__ logits, int64_t V, int64_t stride_bytes,
                                                     const mis_row_params *__restrict__ params, Layout L,
                                                     const char *__restrict__ ws, float *__restrict__ out_probs,
                                                     uint32_t *__restrict__ out_keep)
{
    constexpr int PER = 8;
    const int row = blockIdx.y;
    const RowOut ro = reinterpret_cast<const RowOut *>(ws + L.rowout)[row];
    const RowPlan pl = plan_row(params[row], V);
    const char *rowp = logits + (int64_t)row * stride_bytes;
    const int64_t words = (V + 31) / 32;
    const double md = (double)ro.m;
    for (int it = 0; it < PER; ++it) {
        const int64_t j = (int64_t)blockIdx.x * K3_THREADS * PER + (int64_t)it * K3_THREADS + threadIdx.x;
        bool kept = false;
        float prob = 0.0f;
        if (j < V && ro.status == MIS_ROW_OK) {
            if (ro.mode == M_GREEDY) {
                kept = (j == ro.id);
                prob = kept ? 1.0f : 0.0f;
            } else {
                const float y = scale_y<DT>(load1<DT>(rowp, j), pl.T);
                const uint32_t key = row_key(y, DT);
                kept = (y != -INFINITY) && kept_by_cut(key, j, ro.cut_key, ro.cut_i);
                if (kept) {
                    const double q = exp((double)y - md) / ro.S;
                    prob = rn_dtype((float)q, DT);
                }
            }
        }
        if (out_probs && j < V) out_probs[(size_t)row * V + j] = prob;
        const uint64_t ball = __ballot(kept);
        if (out_keep && (threadIdx.x & 63) == 0) {
            const int64_t w0 = j / 32;  // j is a multiple of 64 for lane 0
            if (w0 < words) out_keep[(size_t)row * words + w0] = (uint32_t)ball;
            if (w0 + 1 < words) out_keep[(size_t)row * words + w0 + 1] = (uint32_t)(ball >> 32);
        }
    }
}

// ------------------------------------------------------------------ host side

static thread_local int g_last_hip = 0;

template <int DT, int EPT>
static hipError_t launch_main(const void *logits, int64_t B, int64_t V, int64_t stride_bytes, int vec_ok,
                              const mis_row_params *params, int64_t *ids, int32_t *status, const Layout &L,
                              char *ws, hipStream_t st, void *const *events)
{
    hipError_t e;
    if (events && (e = hipEventRecord((hipEvent_t)events[0], st)) != hipSuccess) return e;
    hipLaunchKernelGGL((k_chunk<DT, EPT>), dim3(L.G, (unsigned)B), dim3(K1_THREADS), 0, st,
                       (const char *)logits, V, stride_bytes, vec_ok, params, L, ws);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (events && (e = hipEventRecord((hipEvent_t)events[1], st)) != hipSuccess) return e;
    hipLaunchKernelGGL((k_final<DT>), dim3((unsigned)B), dim3(K2_THREADS), 0, st,
                       (const char *)logits, V, stride_bytes, vec_ok, params, L, ws, ids, status);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (events) e = hipEventRecord((hipEvent_t)events[2], st);
    return e;
}

template <int DT>
static hipError_t launch_dt(const void *logits, int64_t B, int64_t V, int64_t stride_bytes, int vec_ok,
                            const mis_row_params *params, int64_t *ids, int32_t *status, float *probs,
                            uint32_t *keep, const Layout &L, char *ws, hipStream_t st, void *const *ev)
{
    hipError_t e;
    switch (L.ept) {
    case 64: e = launch_main<DT, 64>(logits, B, V, stride_bytes, vec_ok, params, ids, status, L, ws, st, ev); break;
    case 32: e = launch_main<DT, 32>(logits, B, V, stride_bytes, vec_ok, params, ids, status, L, ws, st, ev); break;
    case 16: e = launch_main<DT, 16>(logits, B, V, stride_bytes, vec_ok, params, ids, status, L, ws, st, ev); break;
    default: e = launch_main<DT, 8>(logits, B, V, stride_bytes, vec_ok, params, ids, status, L, ws, st, ev); break;
    }
    if (e != hipSuccess) return e;
    if (probs || keep) {
        const unsigned gx = (unsigned)((V + (int64_t)K3_THREADS * 8 - 1) / ((int64_t)K3_THREADS * 8));
        hipLaunchKernelGGL((k_emit<DT>), dim3(gx, (unsigned)B), dim3(K3_THREADS), 0, st,
                           (const char *)logits, V, stride_bytes, params, L, (const char *)ws, probs, keep);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace mis

extern "C" {

size_t mis_workspace_bytes(int64_t B, int64_t V, int dtype)
{
    (void)dtype;
    if (B <= 0 || V <= 0) return 256;
    return mis::make_layout(B, V).total;
}

static int sample_impl(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                       const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
                       uint32_t *out_keep, void *workspace, size_t workspace_bytes, void *stream,
                       void *const *events)
{
    using namespace mis;
    if (dtype < 0 || dtype > 2 || B < 0 || V <= 0 || row_stride < V) return MIS_ERR_INVALID_ARG;
    if (B == 0) return MIS_OK;
    if (!logits || !params || !out_ids || !workspace) return MIS_ERR_INVALID_ARG;
    if (V > (int64_t)1 << 30 || B > 65535) return MIS_ERR_UNSUPPORTED;
    const Layout L = make_layout(B, V);
    if (L.G > G_MAX) return MIS_ERR_UNSUPPORTED;
    if (workspace_bytes < L.total || ((uintptr_t)workspace & 255u) != 0) return MIS_ERR_WORKSPACE;
    const int esz = dtype == MIS_DTYPE_F32 ? 4 : 2;
    const int64_t stride_bytes = row_stride * esz;
    const int vec_ok = (((uintptr_t)logits & 15u) == 0 && (stride_bytes & 15) == 0) ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    hipError_t e;
    if (dtype == MIS_DTYPE_F32)
        e = launch_dt<F32>(logits, B, V, stride_bytes, vec_ok, params, out_ids, out_status, out_probs, out_keep, L, ws, st, events);
    else if (dtype == MIS_DTYPE_F16)
        e = launch_dt<F16>(logits, B, V, stride_bytes, vec_ok, params, out_ids, out_status, out_probs, out_keep, L, ws, st, events);
    else
        e = launch_dt<BF16>(logits, B, V, stride_bytes, vec_ok, params, out_ids, out_status, out_probs, out_keep, L, ws, st, events);
    if (e != hipSuccess) { g_last_hip = (int)e; return MIS_ERR_HIP; }
    return MIS_OK;
}

int mis_sample(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
               const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
               uint32_t *out_keep, void *workspace, size_t workspace_bytes, void *stream)
{
    return sample_impl(logits, dtype, B, V, row_stride, params, out_ids, out_status, out_probs, out_keep,
                       workspace, workspace_bytes, stream, nullptr);
}

int mis_sample_profiled(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                        const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
                        uint32_t *out_keep, void *workspace, size_t workspace_bytes, void *stream,
                        void *const *events)
{
    if (!events || !events[0] || !events[1] || !events[2]) return MIS_ERR_INVALID_ARG;
    return sample_impl(logits, dtype, B, V, row_stride, params, out_ids, out_status, out_probs, out_keep,
                       workspace, workspace_bytes, stream, events);
}

const char *mis_strerror(int code)
{
    switch (code) {
    case MIS_OK: return "ok";
    case MIS_ERR_INVALID_ARG: return "invalid argument";
    case MIS_ERR_WORKSPACE: return "workspace too small or not 256-byte aligned";
    case MIS_ERR_HIP: return "HIP launch failed";
    case MIS_ERR_UNSUPPORTED: return "shape not supported (V > 2^30, B > 65535 or too many chunks)";
    default: return "unknown error";
    }
}

int mis_last_hip_error(void) { return mis::g_last_hip; }

int mis_abi_version(void) { return MIS_ABI_VERSION; }

}  // extern "C"
