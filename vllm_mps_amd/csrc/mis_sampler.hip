// mis_sampler.hip -- MI355X (gfx950) decode-step token sampler behind the C ABI
// declared in include/mis_sampler.h.
//
// One call = one launch of k_sample (plus k_emit when the caller asks for the
// debug probabilities / keep bitmask).
//
// k_sample: B*G workgroups of 256 threads.  Each workgroup takes a ticket
// (atomic counter) naming one chunk of one row, loads that chunk into
// registers with coalesced 16-byte vector reads -- the only HBM read of the
// logits -- and reduces it to a chunk summary.  The last workgroup of a row
// to arrive becomes the row's leader and finishes the row:
//   greedy       argmax merge;
//   small top-k  per chunk: every element >= a threshold that keeps the
//                chunk's top k'; leader: exact k'-th value -> survivors ->
//                top-p over the survivors -> draw;
//   temperature  per-chunk weights -> the chunk holding the draw -> that chunk
//                is re-read for the index;
//   fp32 top-p   float64 mass histograms on a fixed value grid (16 bins per
//                unit below each chunk's max) locate the bin holding the cut;
//                the row's workgroups, still holding their chunks in
//                registers, refine that bin (sub-histogram) and collect its
//                elements when the leader asks; the leader resolves the exact
//                cut and draws;
//   otherwise    (large k', fp16/bf16 top-p, overflows) the leader re-reads the
//                row: radix descent by mass or count, and the 16-bit rounding
//                chain walked over runs of equal keys.
// Tickets are handed out in start order, so a workgroup only ever waits for
// row mates that have already started; every wait is bounded.
//
// Semantics follow model/sampler.py:18-60 per row: greedy argmax (ties ->
// lowest index) when T == 0; y = dtype(f32(x) / T); top-k keeps y >= k'-th
// largest (all ties); top-p on the stable descending order with exact masses
// (fp32 rows) or torch's 16-bit rounding chain (fp16/bf16 rows); the draw is
// min{i : sum_{j<=i} w_j > u * sum w} over the kept weights w = exp(y - m).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mis_device.h"
#include "mis_sampler.h"

namespace mis {

constexpr int K_SMALL = 1024;      // largest k' served by the candidate path
constexpr int CAND_CAP = 2048;     // candidates one chunk may emit
constexpr int SURV_CAP = 2048;     // top-k survivors held in LDS
constexpr int G_MAX = 256;         // chunks per row
constexpr int FB_W = 16;           // fine bins per unit of y (top-p)
constexpr int FB_N = 384;          // fine bins below each chunk max (24 units)
constexpr int SUB_N = 256;         // sub-bins of a refined fine bin
constexpr int WCAP = 2048;         // elements a collect round may gather
constexpr int REGION_BINS = 8;     // L1 bins per 16-bit chain pass
constexpr int RUN_CAP = REGION_BINS * 256;
constexpr int TIE_CAP = 2048;
constexpr int STAGE_CAP = 4096;      // elements one workgroup stages per round
constexpr uint32_t NCAND_OVERFLOW = 0xffffffffu;
constexpr int32_t IDX_ALL = 0x7fffffff;

enum : int { M_BAD = 0, M_GREEDY = 1, M_SMALLK = 2, M_LARGEK = 3, M_TOPP = 4, M_TEMP = 5 };
enum : uint32_t { FLAG_NAN = 1u, FLAG_PINF = 2u };
enum : uint32_t { R_COLLECT = 1u, R_HIST = 2u, R_DONE = 3u };

// ------------------------------------------------------------------ workspace

struct Ctl {                    // 256 B
    unsigned long long ticket;  // monotonically increasing; task = ticket % (B*G)
    uint32_t error;             // bit 0: a bounded wait expired
    uint32_t pad[61];
};

struct RowCtl {                 // 64 B per row, zero at rest
    uint32_t arrive;            // phase-1 arrivals
    uint32_t round;             // last published refinement round (1, 2, ...)
    uint32_t rarrive;           // round arrivals, cumulative
    uint32_t wcount;            // elements appended by the collect round
    uint32_t exited;            // workgroups done with the row
    uint32_t rtype;             // R_COLLECT / R_HIST / R_DONE
    uint32_t klo, khi;          // scaled-key range of the round
    uint32_t kahi;              // collect: (khi, kahi] is summed as kept mass
    float hlo, hhi;             // hist: value range [hlo, hhi)
    float m;                    // row max of y
    uint32_t ovf;               // a round overflowed a staging or window buffer
    int32_t rbin;               // row fine bin (below the row max's bin) holding the cut
    uint32_t pad[2];
};
static_assert(sizeof(RowCtl) == 64, "RowCtl is 64 bytes");

// The control prefix of the workspace (Ctl, then one RowCtl for every row the
// ABI allows) sits at a fixed place whatever the shape, so control words that
// each call leaves at zero stay zero for the next call of any shape.
constexpr int64_t B_MAX = 65535;
constexpr size_t CTL_PREFIX = 256 + sizeof(RowCtl) * (size_t)(B_MAX + 1);

struct ChunkSum {               // 64 B per (row, chunk)
    uint32_t xkey;              // argmax key of the raw logits (NaN = 0xffffffff)
    int32_t xarg;
    float ymax;                 // max scaled logit of the chunk
    uint32_t flags;
    uint32_t ncand;             // small-k candidates written, or NCAND_OVERFLOW
    float xmax;                 // max raw logit of the chunk
    uint32_t pad0, pad1;
    double S;                   // sum of weights relative to the chunk max
    double gmc;                 // top-p: floor(ymax * FB_W), the chunk's bin anchor
    double below;               // top-p: mass below the fine-bin range
    double pad2;
};

struct RowOut {                 // 64 B per row, read by k_emit
    int64_t id;
    int32_t status;
    int32_t mode;
    float m;                    // row max of y
    uint32_t cut_key;           // kept iff key > cut_key or (key == cut_key and j <= cut_i)
    int32_t cut_i;
    int32_t pad;
    double S;                   // sum of kept weights exp(y - m)
    double pad2[3];
};

struct Cand { float x; int32_t idx; };
struct Elem { uint32_t key; int32_t idx; };

struct Layout {
    int64_t B, V;
    int ept, G;
    size_t ctl, rowctl, rowout, chunks, fbc, fbm, cand, subc, subm, win, amass, total;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static Layout make_layout(int64_t B, int64_t V, int dtype)
{
    Layout L;
    L.B = B; L.V = V;
    (void)dtype;
    static const int opts[4] = {64, 32, 16, 8};
    L.ept = 8;
    for (int i = 0; i < 4; ++i) {
        const int64_t G = (V + (int64_t)NT * opts[i] - 1) / ((int64_t)NT * opts[i]);
        if (B * G >= 1024 && G <= G_MAX) { L.ept = opts[i]; break; }
    }
    L.G = (int)((V + (int64_t)NT * L.ept - 1) / ((int64_t)NT * L.ept));
    if (L.G > G_MAX) {
        L.ept = 64;
        L.G = (int)((V + (int64_t)NT * 64 - 1) / ((int64_t)NT * 64));
    }
    const size_t BG = (size_t)B * L.G;
    size_t off = 0;
    L.ctl = off;    off = align256(off + sizeof(Ctl));
    L.rowctl = off; off = CTL_PREFIX;
    L.rowout = off; off = align256(off + sizeof(RowOut) * (size_t)B);
    L.chunks = off; off = align256(off + sizeof(ChunkSum) * BG);
    L.fbc = off;    off = align256(off + sizeof(uint32_t) * FB_N * BG);
    L.fbm = off;    off = align256(off + sizeof(double) * FB_N * BG);
    L.cand = off;   off = align256(off + sizeof(Cand) * (size_t)CAND_CAP * BG);
    L.subc = off;   off = align256(off + sizeof(uint32_t) * SUB_N * (size_t)B);
    L.subm = off;   off = align256(off + sizeof(double) * SUB_N * (size_t)B);
    L.win = off;    off = align256(off + sizeof(Elem) * WCAP * (size_t)B);
    L.amass = off;  off = align256(off + sizeof(double) * G_MAX * (size_t)B);
    L.total = off;
    return L;
}

// ------------------------------------------------------------------ row plan

struct RowPlan { int mode; int kk; int topp; float T; float top_p; float u; };

__device__ __forceinline__ RowPlan plan_row(const mis_row_params &P, int64_t V)
{
    RowPlan r;
    r.T = P.temperature; r.top_p = P.top_p; r.u = P.uniform; r.kk = 0; r.topp = 0;
    const bool bad = !(P.temperature >= 0.0f) || P.top_k < 0 || !(P.top_p > 0.0f) || !(P.uniform == P.uniform);
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

// ------------------------------------------------------------------ context

struct Args {
    const char *logits;
    int64_t V;
    int64_t stride_bytes;
    int vec_ok;
    const mis_row_params *params;
    Layout L;
    char *ws;
    int64_t *out_ids;
    int32_t *out_status;
};

struct RowCx {                 // what the leader of a row works with
    const char *rowp;
    int64_t V;
    int vec_ok;
    float T;
    float m;                   // row max of y
    int G;
    int64_t CH;
    int row;
    const uint32_t *fbc;       // this row's chunk fine-bin counts [G][FB_N]
    const double *fbm;         // this row's chunk fine-bin masses [G][FB_N]
    uint32_t *subc;            // this row's sub-histogram [SUB_N]
    double *subm;
};

// ------------------------------------------------------------------ shared memory

struct Smem {
    union {
        struct { uint32_t cnt[FB_N]; double mass[FB_N]; } p1;                              // 4.5 KB
        struct { uint32_t cnt[2048]; } h11;                                                // 8 KB
        struct { uint32_t cnt[256]; double mass[256]; } h8;                                // 3 KB
        struct { uint32_t key[SURV_CAP]; int32_t idx[SURV_CAP]; double e[SURV_CAP]; } s;   // 32 KB
        struct { uint64_t k[SURV_CAP]; double e[SURV_CAP]; } so;                          // 32 KB
        struct { uint32_t cnt[RUN_CAP]; uint32_t rkey[RUN_CAP]; uint32_t rcnt[RUN_CAP]; float rp[RUN_CAP]; } r;  // 32 KB
        struct { int32_t idx[TIE_CAP]; } t;
        struct { float x[STAGE_CAP]; uint32_t j[STAGE_CAP]; } st;                          // 32 KB
    } u;
    union {
        struct { double m[FB_N]; uint32_t c[FB_N]; } rb;    // row-merged fine bins, index FB_N-1 = top
        struct { uint32_t cnt[256]; double mass[256]; } l1;  // re-read path: level-1 histogram
    } v;
    double cw[G_MAX];          // per-chunk kept weight
    double chs[G_MAX];         // per-chunk rescale to the row max
    double sub_m[SUB_N];       // round-local histograms
    uint32_t sub_c[SUB_N];
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
    double bd[8];
    float bf[8];
    unsigned long long bq[2];
    Args args;                 // launch arguments, RowCx and RowPlan of the row for the
    RowCx cx;                  // leader's out-of-line functions (kept out of private
    RowPlan pl;                // memory, which would otherwise hold a copy per lane)
};

// LDS of the chunk pass: only what its per-mode reductions need, so that
// several workgroups fit on a CU
struct ChunkSmem {
    union {
        struct { uint32_t cnt[FB_N]; double mass[FB_N]; } p1;  // fine bins (fp32 top-p)
        struct { uint32_t cnt[256]; double mass[256]; } h8;    // candidate threshold histogram
    } u;
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
};

__device__ __forceinline__ bool kept_by_cut(uint32_t key, int64_t j, uint32_t cut_key, int32_t cut_i)
{
    return key > cut_key || (key == cut_key && j <= (int64_t)cut_i);
}

// Hide a register value from the optimiser so a per-element quantity is
// recomputed in each pass instead of being kept live for all EPT elements.
__device__ __forceinline__ float opaque(float v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// ------------------------------------------------------------------ chunk -> row hand-off
//
// The chunk pass (k_chunk) writes per-chunk summaries, fine bins and
// candidates; the row pass (k_final) reads them in the next launch on the
// same stream, so the kernel boundary orders and publishes them.

template <class T> struct same_t { typedef T type; };
template <class T> __device__ __forceinline__ void st_dev(T *p, typename same_t<T>::type v) { *p = v; }
template <class T> __device__ __forceinline__ T ld_dev(const T *p) { return *p; }
__device__ __forceinline__ void st_dev_cand(Cand *p, float x, int32_t idx)
{
    st_dev(reinterpret_cast<uint64_t *>(p), ((uint64_t)(uint32_t)idx << 32) | f32_bits(x));
}
__device__ __forceinline__ Cand ld_dev_cand(const Cand *p)
{
    const uint64_t v = ld_dev(reinterpret_cast<const uint64_t *>(p));
    Cand c; c.x = bits_f32((uint32_t)v); c.idx = (int32_t)(uint32_t)(v >> 32);
    return c;
}
// candidates a chunk wrote (its summary says so; never more than the buffer)
__device__ __forceinline__ uint32_t ncand_of(const ChunkSum *cs)
{
    const uint32_t n = ld_dev(&cs->ncand);
    return n < (uint32_t)CAND_CAP ? n : (uint32_t)CAND_CAP;
}

// raw-key interval for a scaled-key interval, computed by wave 0
template <int DT, class S> __device__ void x_interval(S &sm, uint32_t klo, uint32_t khi, float T, uint32_t *xlo, uint32_t *xhi)
{
    __syncthreads();
    if (wave_id() == 0) {
        const uint32_t a = x_lower<DT>(klo, T);
        const uint32_t b = x_upper<DT>(khi, T);
        if (lane_id() == 0) { sm.bu[4] = a; sm.bu[5] = b; }
    }
    __syncthreads();
    *xlo = sm.bu[4];
    *xhi = sm.bu[5];
    __syncthreads();
}

__device__ void write_row(RowOut *ro, const Args &a, int row, int64_t id, int status, int mode, float m,
                          uint32_t cut_key, int32_t cut_i, double S)
{
    if (threadIdx.x == 0) {
        ro->id = status == MIS_ROW_OK ? id : -1;
        ro->status = status;
        ro->mode = mode;
        ro->m = m;
        ro->cut_key = cut_key;
        ro->cut_i = cut_i;
        ro->S = S;
        a.out_ids[row] = status == MIS_ROW_OK ? id : -1;
        if (a.out_status) a.out_status[row] = status;
    }
}

// ------------------------------------------------------------------ draw helpers

// Inverse CDF inside chunk g: the first kept index whose running weight (index
// order) exceeds `resid`; wfun(x, j) gives the weight (0 = not kept).  When
// rounding leaves `resid` out of reach, the chunk's last kept index.
template <int DT, class WF>
__device__ int64_t draw_in_chunk(Smem &sm, const RowCx &c, int g, double resid, WF &&wfun)
{
    // Thread t takes the contiguous elements [cbeg + t*per, cbeg + (t+1)*per)
    // of the chunk, loaded up front (16-byte vectors where aligned), so the
    // weights are computed from registers in both passes.
    constexpr int VEC = Traits<DT>::VEC, MAXPER = 64;
    const int64_t cbeg = (int64_t)g * c.CH;
    const int64_t cend = cbeg + c.CH < c.V ? cbeg + c.CH : c.V;
    const int per = (int)(c.CH / NT);  // 8..64, a multiple of VEC
    const int64_t jb = cbeg + (int64_t)threadIdx.x * per;
    float xs[MAXPER];
#pragma unroll
    for (int v = 0; v < MAXPER / VEC; ++v) {
        if (v * VEC < per) {
            const int64_t j0 = jb + (int64_t)v * VEC;
            if (c.vec_ok && j0 + VEC <= cend) {
                loadvec<DT>(c.rowp, j0, &xs[v * VEC]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) xs[v * VEC + e] = (j0 + e < cend) ? load1<DT>(c.rowp, j0 + e) : 0.0f;
            }
        }
    }
    double local = 0.0;
    int64_t lastk = -1;
#pragma unroll
    for (int i = 0; i < MAXPER; ++i) {
        if (i < per && jb + i < cend) {
            const double w = wfun(xs[i], jb + i);
            if (w > 0.0) { local += w; lastk = jb + i; }
        }
    }
    double tot;
    const double before = block_excl_scan<double>(local, sm.red, &tot);
    if (threadIdx.x == 0) sm.bq[0] = 0xffffffffffffffffull;
    __syncthreads();
    if (local > 0.0 && before <= resid && resid < before + local) {
        double run = before;
        int64_t pick = lastk;
        bool done = false;
#pragma unroll
        for (int i = 0; i < MAXPER; ++i) {
            if (!done && i < per && jb + i < cend) {
                const double w = wfun(xs[i], jb + i);
                if (w > 0.0) {
                    run += w;
                    if (run > resid) { pick = jb + i; done = true; }
                }
            }
        }
        atomicMin(&sm.bq[0], (unsigned long long)pick);
    }
    __syncthreads();
    const unsigned long long pk = sm.bq[0];
    __syncthreads();
    if (pk != 0xffffffffffffffffull) return (int64_t)pk;
    return block_max<int64_t>(lastk, sm.red);
}

// Chunk holding u * sum(sm.cw) and the residual weight inside it.
__device__ void pick_chunk(Smem &sm, int G, float u, int *g_out, double *resid_out, double *S_out)
{
    __syncthreads();
    if (threadIdx.x == 0) {
        double S = 0.0;
        for (int g = 0; g < G; ++g) S += sm.cw[g];
        double target = (double)u * S, cum = 0.0;
        int gsel = -1;
        for (int g = 0; g < G; ++g) {
            if (sm.cw[g] > 0.0) {
                if (cum + sm.cw[g] > target) { gsel = g; break; }
                cum += sm.cw[g];
            }
        }
        if (gsel < 0) {  // rounding: the last chunk with weight, its last kept element
            for (int g = G - 1; g >= 0; --g) if (sm.cw[g] > 0.0) { gsel = g; break; }
            cum = 0.0;
            for (int g = 0; g < gsel; ++g) cum += sm.cw[g];
            target = cum + (gsel >= 0 ? sm.cw[gsel] : 0.0);
        }
        sm.bd[0] = S;
        sm.bd[1] = target - cum;
        sm.bi[0] = gsel;
    }
    __syncthreads();
    *S_out = sm.bd[0];
    *resid_out = sm.bd[1];
    *g_out = sm.bi[0];
    __syncthreads();
}

// First index (ascending) of an LDS element list at which the running weight
// exceeds `target`: radix over index space, 256 buckets per level.
__device__ int64_t draw_in_list(Smem &sm, const int32_t *idx, const double *e, int n, int64_t V, double target)
{
    int64_t lo = 0, hi = V;
    double acc = 0.0;
    while (hi - lo > 1) {
        const int64_t width = (hi - lo + 255) / 256;
        __syncthreads();
        for (int i = threadIdx.x; i < 256; i += NT) sm.sub_m[i] = 0.0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += NT) {
            const int64_t j = idx[i];
            if (j >= lo && j < hi && e[i] > 0.0) atomicAdd(&sm.sub_m[(j - lo) / width], e[i]);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            double cum = acc;
            int bsel = -1;
            for (int b = 0; b < 256; ++b) {
                if (sm.sub_m[b] > 0.0) {
                    if (cum + sm.sub_m[b] > target) { bsel = b; break; }
                    cum += sm.sub_m[b];
                }
            }
            if (bsel < 0) {  // rounding: the last element with weight
                for (int b = 255; b >= 0; --b) if (sm.sub_m[b] > 0.0) { bsel = b; break; }
                cum = acc;
                for (int b = 0; b < bsel; ++b) cum += sm.sub_m[b];
                target = 1e300;
            }
            sm.bi[1] = bsel;
            sm.bd[2] = cum;
            sm.bd[3] = target;
        }
        __syncthreads();
        const int b = sm.bi[1];
        acc = sm.bd[2];
        target = sm.bd[3];
        __syncthreads();
        if (b < 0) return -1;
        lo = lo + (int64_t)b * width;
        hi = lo + width < hi ? lo + width : hi;
    }
    return lo;
}

// Cut inside a candidate window held in LDS (key, idx, e): mass descent over
// the keys to the running mass Aw (descending order, ties by index).
__device__ void window_cut(Smem &sm, const uint32_t *key, const int32_t *idx, const double *e, uint32_t n,
                           double Aw, double e_of_key_dummy, uint32_t *cut_key, int32_t *cut_i, int dt)
{
    (void)e_of_key_dummy;
    uint32_t prefix = 0u;
    double acc = 0.0;
    uint32_t kc = 0;
    double ekey = 0.0;
    for (int lev = 0; lev < 4; ++lev) {
        const int sh = 24 - 8 * lev;
        const uint32_t hmask = lev == 0 ? 0u : ~((1u << (sh + 8)) - 1u);
        __syncthreads();
        for (int i = threadIdx.x; i < 256; i += NT) { sm.sub_m[i] = 0.0; sm.sub_c[i] = 0u; }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const uint32_t k = key[i];
            if ((k & hmask) == (prefix & hmask)) {
                atomicAdd(&sm.sub_m[(k >> sh) & 255u], e[i]);
                atomicAdd(&sm.sub_c[(k >> sh) & 255u], 1u);
            }
        }
        __syncthreads();
        if (wave_id() == 0) {
            double ab;
            const int d = wave_find_desc<double>(sm.sub_m, 256, Aw - acc, &ab);
            if (lane_id() == 0) { sm.bu[0] = (uint32_t)d; sm.bd[0] = ab; sm.bu[1] = sm.sub_c[d]; }
        }
        __syncthreads();
        prefix |= sm.bu[0] << sh;
        acc += sm.bd[0];
        kc = sm.bu[1];
        __syncthreads();
    }
    // the weight of one element holding the resolved key
    if (threadIdx.x == 0) sm.bd[1] = 0.0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += NT) if (key[i] == prefix) sm.bd[1] = e[i];
    __syncthreads();
    ekey = sm.bd[1];
    __syncthreads();
    double tt = ekey > 0.0 ? ceil((Aw - acc) / ekey) : 1.0;
    if (!(tt >= 1.0)) tt = 1.0;
    if (tt > (double)kc) tt = (double)kc;
    uint32_t t = (uint32_t)tt;
    while (t > 1 && acc + (double)(t - 1) * ekey >= Aw) --t;
    while (t < kc && acc + (double)t * ekey < Aw) ++t;
    *cut_key = prefix;
    *cut_i = IDX_ALL;
    if (t < kc) {  // the t-th smallest index among the elements holding the key
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            if (key[i] != prefix) continue;
            const int32_t v = idx[i];
            uint32_t r = 0;
            for (uint32_t q = 0; q < n; ++q) r += (key[q] == prefix && idx[q] < v) ? 1u : 0u;
            if (r == t - 1u) sm.bi[0] = v;
        }
        __syncthreads();
        *cut_i = sm.bi[0];
        __syncthreads();
    }
    (void)dt;
}

// ------------------------------------------------------------------ re-read path

template <int DT, class F>
__device__ __forceinline__ void rescan(const RowCx &c, uint32_t xklo, uint32_t xkhi, F &&f)
{
    if (xklo > xkhi) return;
    scan_range<DT, 4>(c.rowp, 0, c.V, c.vec_ok, [&](int64_t j, float x) {
        const uint32_t xk = key_of_f32(x);
        if (xk >= xklo && xk <= xkhi) {
            const float y = scale_y<DT>(x, c.T);
            f(j, y, row_key(y, DT));
        }
    });
}

// Radix descent (8-bit digits) over row keys >= floor_key; level 1 from
// sm.v.l1, later levels re-read the row.  by_mass: running mass (descending)
// reaches target; else running count.  Returns the resolved key; *acc_out =
// mass or count strictly above it; *kcnt = elements holding exactly it.
template <int DT>
__device__ __noinline__ uint32_t descend(Smem &sm, const RowCx &c, bool by_mass, double target, uint32_t floor_key,
                                         double *acc_out, uint32_t *kcnt)
{
    __syncthreads();
    if (wave_id() == 0) {
        int b;
        if (by_mass) { double ab; b = wave_find_desc<double>(sm.v.l1.mass, 256, target, &ab); if (lane_id() == 0) sm.bd[0] = ab; }
        else { uint32_t ab; b = wave_find_desc<uint32_t>(sm.v.l1.cnt, 256, (uint32_t)target, &ab); if (lane_id() == 0) sm.bd[0] = (double)ab; }
        if (lane_id() == 0) { sm.bu[0] = (uint32_t)b; sm.bu[1] = sm.v.l1.cnt[b]; }
    }
    __syncthreads();
    uint32_t prefix = sm.bu[0] << 24;
    double acc = sm.bd[0];
    uint32_t bincnt = sm.bu[1];
    const int nlev = DT == F32 ? 3 : 1;
    const double md = (double)c.m;
    for (int lev = 0; lev < nlev; ++lev) {
        const int shift = 16 - 8 * lev;
        const uint32_t freemask = (1u << (shift + 8)) - 1u;
        __syncthreads();
        for (int i = threadIdx.x; i < 256; i += NT) { sm.u.h8.cnt[i] = 0u; sm.u.h8.mass[i] = 0.0; }
        uint32_t klo = prefix, khi = prefix | freemask;
        if (klo < floor_key) klo = floor_key;
        uint32_t xlo, xhi;
        x_interval<DT>(sm, klo, khi, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float y, uint32_t key) {
            if (key < klo || key > khi) return;
            const uint32_t b = (key >> shift) & 255u;
            atomicAdd(&sm.u.h8.cnt[b], 1u);
            if (by_mass) atomicAdd(&sm.u.h8.mass[b], exp((double)y - md));
        });
        __syncthreads();
        if (wave_id() == 0) {
            int b;
            if (by_mass) { double ab; b = wave_find_desc<double>(sm.u.h8.mass, 256, target - acc, &ab); if (lane_id() == 0) sm.bd[0] = ab; }
            else { uint32_t ab; b = wave_find_desc<uint32_t>(sm.u.h8.cnt, 256, (uint32_t)(target - acc), &ab); if (lane_id() == 0) sm.bd[0] = (double)ab; }
            if (lane_id() == 0) { sm.bu[0] = (uint32_t)b; sm.bu[1] = sm.u.h8.cnt[b]; }
        }
        __syncthreads();
        prefix |= sm.bu[0] << shift;
        acc += sm.bd[0];
        bincnt = sm.bu[1];
        __syncthreads();
    }
    *acc_out = acc;
    *kcnt = bincnt;
    return prefix;
}

// Index of the t-th (1-based) element in index order whose scaled key is `key`.
template <int DT>
__device__ __noinline__ int32_t tie_index(Smem &sm, const RowCx &c, uint32_t key, uint32_t t)
{
    uint32_t xlo, xhi;
    x_interval<DT>(sm, key, key, c.T, &xlo, &xhi);
    if (threadIdx.x == 0) sm.bu[2] = 0u;
    __syncthreads();
    rescan<DT>(c, xlo, xhi, [&](int64_t j, float, uint32_t k) {
        if (k != key) return;
        const uint32_t p = atomicAdd(&sm.bu[2], 1u);
        if (p < (uint32_t)TIE_CAP) sm.u.t.idx[p] = (int32_t)j;
    });
    __syncthreads();
    const uint32_t n = sm.bu[2];
    if (n <= (uint32_t)TIE_CAP) {
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const int32_t v = sm.u.t.idx[i];
            uint32_t r = 0;
            for (uint32_t q = 0; q < n; ++q) r += sm.u.t.idx[q] < v ? 1u : 0u;
            if (r == t - 1u) sm.bi[0] = v;
        }
        __syncthreads();
        const int32_t res = sm.bi[0];
        __syncthreads();
        return res;
    }
    int64_t lo = 0, hi = c.V - 1;  // many ties: bisect on the index with counting passes
    while (lo < hi) {
        const int64_t mid = lo + (hi - lo) / 2;
        uint32_t mine = 0;
        rescan<DT>(c, xlo, xhi, [&](int64_t j, float, uint32_t k) { if (k == key && j <= mid) mine++; });
        mine = block_sum<uint32_t>(mine, sm.red);
        if (mine >= t) hi = mid; else lo = mid + 1;
    }
    return (int32_t)lo;
}

// Sequential walk of the 16-bit top-p chain over runs (one thread).  Returns
// true when some rank triggers removal; the cut then keeps *t_keep elements of
// run *run_at (0 = the cut is the previous run).
__device__ bool chain_walk(const uint32_t *rcnt, const float *rp, int nruns, float &F, float thr16, int dt,
                           int *run_at, uint32_t *t_keep)
{
    for (int r = 0; r < nruns; ++r) {
        const float p = rp[r];
        const uint32_t n = rcnt[r];
        const float Fend = chain_add_n(F, p, n);
        if (chain_E(Fend, p, dt) >= thr16) {
            uint32_t lo = 0, hi = n - 1;
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

// Top-p cut over elements with key >= floor_key; sm.v.l1 holds their 256-bin
// histogram and S their total weight.
template <int DT>
__device__ __noinline__ void topp_cut_generic(Smem &sm, const RowCx &c, float top_p, uint32_t floor_key, double S,
                                              uint32_t *cut_key, int32_t *cut_i, int *status)
{
    const double md = (double)c.m;
    *status = MIS_ROW_OK;
    if (DT == F32) {
        const double A = (double)top_p * S;
        double acc;
        uint32_t kc;
        const uint32_t key = descend<DT>(sm, c, true, A, floor_key, &acc, &kc);
        const double e = exp((double)value_of_row_key(key, DT) - md);
        double tt = ceil((A - acc) / e);
        if (!(tt >= 1.0)) tt = 1.0;
        if (tt > (double)kc) tt = (double)kc;
        uint32_t t = (uint32_t)tt;
        while (t > 1 && acc + (double)(t - 1) * e >= A) --t;
        while (t < kc && acc + (double)t * e < A) ++t;
        *cut_key = key;
        *cut_i = (t >= kc) ? IDX_ALL : tie_index<DT>(sm, c, key, t);
        return;
    }
    const float thr16 = rn_dtype(top_p, DT);
    const uint32_t kneg = row_key(-INFINITY, DT);
    float F = 0.0f;
    int b_hi = 255;
    while (b_hi >= 0 && sm.v.l1.cnt[b_hi] == 0u) --b_hi;
    uint32_t prev_key = 0u;
    bool have_prev = false;
    while (b_hi >= 0) {
        int b_lo = b_hi - REGION_BINS + 1;
        if (b_lo < 0) b_lo = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < RUN_CAP; i += NT) sm.u.r.cnt[i] = 0u;
        uint32_t klo = (uint32_t)b_lo << 24;
        const uint32_t khi = ((uint32_t)b_hi << 24) | 0x00ffffffu;
        if (klo < floor_key) klo = floor_key;
        if (klo <= kneg) klo = kneg + 1u;
        uint32_t xlo, xhi;
        x_interval<DT>(sm, klo, khi, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float, uint32_t key) {
            if (key < klo || key > khi) return;
            const uint32_t pos = (uint32_t)(b_hi - (int)(key >> 24)) * 256u + (255u - ((key >> 16) & 255u));
            atomicAdd(&sm.u.r.cnt[pos], 1u);
        });
        __syncthreads();
        const int npos = (b_hi - b_lo + 1) * 256;
        int nruns_total = 0;
        for (int i0 = 0; i0 < npos; i0 += NT) {
            const int i = i0 + threadIdx.x;
            const uint32_t cnt = i < npos ? sm.u.r.cnt[i] : 0u;
            uint32_t tot;
            const uint32_t off = block_excl_scan<uint32_t>(cnt ? 1u : 0u, sm.red, &tot);
            if (cnt) {
                const uint32_t L1 = (uint32_t)(b_hi - i / 256), b2 = 255u - (uint32_t)(i % 256);
                const uint32_t key = (L1 << 24) | (b2 << 16);
                const int r = nruns_total + (int)off;
                sm.u.r.rkey[r] = key;
                sm.u.r.rcnt[r] = cnt;
                sm.u.r.rp[r] = rn_dtype((float)(exp((double)value_of_row_key(key, DT) - md) / S), DT);
            }
            nruns_total += (int)tot;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int run_at = -1;
            uint32_t tk = 0;
            float Fw = F;
            const bool found = chain_walk(sm.u.r.rcnt, sm.u.r.rp, nruns_total, Fw, thr16, DT, &run_at, &tk);
            sm.bi[1] = found ? 1 : 0;
            sm.bu[0] = tk;
            sm.bf[0] = Fw;
            sm.bu[1] = nruns_total > 0 ? sm.u.r.rkey[nruns_total - 1] : 0u;
            if (found) {
                sm.bu[2] = sm.u.r.rkey[run_at];
                sm.bu[3] = sm.u.r.rcnt[run_at];
                sm.bu[4] = run_at > 0 ? sm.u.r.rkey[run_at - 1] : 0u;
                sm.bi[3] = run_at > 0 ? 1 : 0;
            }
        }
        __syncthreads();
        const bool found = sm.bi[1] != 0;
        if (found) {
            const uint32_t tk = sm.bu[0], rkey = sm.bu[2], rcnt = sm.bu[3], pkey = sm.bu[4];
            const bool prev_in_region = sm.bi[3] != 0;
            __syncthreads();
            if (tk > 0) {
                *cut_key = rkey;
                *cut_i = (tk >= rcnt) ? IDX_ALL : tie_index<DT>(sm, c, rkey, tk);
            } else if (prev_in_region) {
                *cut_key = pkey; *cut_i = IDX_ALL;
            } else if (have_prev) {
                *cut_key = prev_key; *cut_i = IDX_ALL;
            } else {
                *status = MIS_ROW_INVALID;  // rank 0 removed: nothing left
            }
            return;
        }
        F = sm.bf[0];
        if (nruns_total > 0) { prev_key = sm.bu[1]; have_prev = true; }
        __syncthreads();
        b_hi = b_lo - 1;
        while (b_hi >= 0 && sm.v.l1.cnt[b_hi] == 0u) --b_hi;
    }
    if (have_prev) { *cut_key = prev_key; *cut_i = IDX_ALL; }
    else *status = MIS_ROW_INVALID;
}

// Full row by re-reads: top-k of any size by count descent, then top-p, then
// the draw.  Serves large k', fp16/bf16 top-p and every overflow.
template <int DT>
__device__ __noinline__ void final_generic(Smem &sm, const RowCx &c, const RowPlan &pl, RowOut *ro, const Args &a)
{
    if (DT != F32 && pl.kk > 0) {
        // the 16-bit top-k radix descent is switched off in this build
        write_row(ro, a, c.row, -1, MIS_ROW_UNSUPPORTED, pl.mode, c.m, 0u, 0, 0.0);
        return;
    }
    const double md = (double)c.m;
    const uint32_t kneg = row_key(-INFINITY, DT);
    __syncthreads();
    for (int b = threadIdx.x; b < 256; b += NT) { sm.v.l1.mass[b] = 0.0; sm.v.l1.cnt[b] = 0u; }
    __syncthreads();
    rescan<DT>(c, 0x007fffffu, 0xff800000u, [&](int64_t, float y, uint32_t key) {
        atomicAdd(&sm.v.l1.cnt[key >> 24], 1u);
        if (y != -INFINITY) atomicAdd(&sm.v.l1.mass[key >> 24], exp((double)y - md));
    });
    __syncthreads();
    uint32_t floor_key = kneg + 1u;
    if (pl.kk > 0) {
        double acc;
        uint32_t kc;
        floor_key = descend<DT>(sm, c, false, (double)pl.kk, 0u, &acc, &kc);
        if (floor_key <= kneg) floor_key = kneg + 1u;
        __syncthreads();
        for (int b = threadIdx.x; b < 256; b += NT) { sm.v.l1.mass[b] = 0.0; sm.v.l1.cnt[b] = 0u; }
        uint32_t xlo, xhi;
        x_interval<DT>(sm, floor_key, 0xffffffffu, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float y, uint32_t key) {
            if (key < floor_key) return;
            atomicAdd(&sm.v.l1.cnt[key >> 24], 1u);
            atomicAdd(&sm.v.l1.mass[key >> 24], exp((double)y - md));
        });
        __syncthreads();
    }
    double S = 0.0;
    for (int b = threadIdx.x; b < 256; b += NT) S += sm.v.l1.mass[b];
    S = block_sum<double>(S, sm.red);
    uint32_t cut_key = floor_key;
    int32_t cut_i = IDX_ALL;
    int status = MIS_ROW_OK;
    if (pl.topp) topp_cut_generic<DT>(sm, c, pl.top_p, floor_key, S, &cut_key, &cut_i, &status);
    if (status != MIS_ROW_OK) {
        write_row(ro, a, c.row, -1, status, pl.mode, c.m, 0u, 0, 0.0);
        return;
    }
    __syncthreads();
    for (int g = threadIdx.x; g < c.G; g += NT) sm.cw[g] = 0.0;
    uint32_t xlo, xhi;
    x_interval<DT>(sm, cut_key, 0xffffffffu, c.T, &xlo, &xhi);
    rescan<DT>(c, xlo, xhi, [&](int64_t j, float y, uint32_t key) {
        if (kept_by_cut(key, j, cut_key, cut_i)) atomicAdd(&sm.cw[j / c.CH], exp((double)y - md));
    });
    int g;
    double resid, SK;
    pick_chunk(sm, c.G, pl.u, &g, &resid, &SK);
    int64_t id = -1;
    if (g >= 0) {
        const float T = c.T;
        id = draw_in_chunk<DT>(sm, c, g, resid, [&](float x, int64_t j) -> double {
            const float y = scale_y<DT>(x, T);
            return (y != -INFINITY && kept_by_cut(row_key(y, DT), j, cut_key, cut_i)) ? exp((double)y - md) : 0.0;
        });
    }
    write_row(ro, a, c.row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, c.m, cut_key, cut_i, SK);
}

// ------------------------------------------------------------------ small top-k leader

// Exact k'-th value over the per-chunk candidates, survivors, optional top-p,
// draw.  Returns false when the survivors overflow LDS.
template <int DT>
__device__ __noinline__ bool final_smallk(Smem &sm, const RowCx &c, const RowPlan &pl, const ChunkSum *cs,
                                          const Cand *cand, RowOut *ro, const Args &a)
{
    const double md = (double)c.m;
    // candidate counts -> prefix offsets (thread 0, G <= 256); candidate f of
    // the row is candidate f - pre[g] of the chunk g with pre[g] <= f < pre[g+1]
    uint32_t *pre = reinterpret_cast<uint32_t *>(sm.chs);
    for (int g = threadIdx.x; g < c.G; g += NT) sm.sub_c[g] = ncand_of(&cs[g]);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int g = 0; g < c.G; ++g) { pre[g] = run; run += sm.sub_c[g]; }
        pre[c.G] = run;
    }
    __syncthreads();
    const uint32_t ntot = pre[c.G];
    const int G = c.G;
    auto cand_ptr = [&](uint32_t f) -> const Cand * {
        int lo = 0, hi = G - 1;  // last g with pre[g] <= f
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pre[mid] <= f) lo = mid; else hi = mid - 1;
        }
        return cand + (size_t)lo * CAND_CAP + (f - pre[lo]);
    };
    constexpr int BATCH = 8;  // candidate loads in flight per thread
    // k'-th largest raw key over the candidates: 11 / 11 / 10-bit digits.  Fewer
    // candidates than k' means fewer finite elements than k' in the row.
    uint32_t xk_thr = 0u;
    if (ntot >= (uint32_t)pl.kk) {
        uint32_t prefix = 0u, rem = (uint32_t)pl.kk;
        for (int lev = 0; lev < 3; ++lev) {
            const int sh = lev == 0 ? 21 : (lev == 1 ? 10 : 0);
            const int nbits = lev == 2 ? 10 : 11;
            const int nb = 1 << nbits;
            const uint32_t hmask = lev == 0 ? 0u : ~((1u << (sh + nbits)) - 1u);
            __syncthreads();
            for (int i = threadIdx.x; i < 2048; i += NT) sm.u.h11.cnt[i] = 0u;
            __syncthreads();
            for (uint32_t f0 = 0; f0 < ntot; f0 += NT * BATCH) {
                // addresses first (LDS reads), then the loads back to back
                const Cand *cp[BATCH];
#pragma unroll
                for (int u = 0; u < BATCH; ++u) {
                    const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                    cp[u] = cand_ptr(f < ntot ? f : 0u);
                }
                uint32_t kv[BATCH];
#pragma unroll
                for (int u = 0; u < BATCH; ++u) kv[u] = key_of_f32(ld_dev_cand(cp[u]).x);
#pragma unroll
                for (int u = 0; u < BATCH; ++u) {
                    const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                    if (f < ntot && (kv[u] & hmask) == (prefix & hmask))
                        atomicAdd(&sm.u.h11.cnt[(kv[u] >> sh) & (uint32_t)(nb - 1)], 1u);
                }
            }
            __syncthreads();
            if (wave_id() == 0) {
                uint32_t above;
                const int d = wave_find_desc<uint32_t>(sm.u.h11.cnt, nb, rem, &above);
                if (lane_id() == 0) { sm.bu[0] = (uint32_t)d; sm.bu[1] = above; }
            }
            __syncthreads();
            rem -= sm.bu[1];
            prefix |= sm.bu[0] << sh;
            __syncthreads();
        }
        xk_thr = prefix;
    }
    // survivors: scaled value >= scale(k'-th raw value); the ties the scaling
    // creates are kept, as the reference keeps them
    const uint32_t thr_key = xk_thr ? row_key(scale_y<DT>(f32_of_key(xk_thr), c.T), DT) : 0u;
    if (threadIdx.x == 0) sm.bu[3] = 0u;
    __syncthreads();
    for (uint32_t f0 = 0; f0 < ntot; f0 += NT * BATCH) {
        const Cand *cp[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
            cp[u] = cand_ptr(f < ntot ? f : 0u);
        }
        Cand cv[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; ++u) cv[u] = ld_dev_cand(cp[u]);
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
            if (f < ntot) {
                const float y = scale_y<DT>(cv[u].x, c.T);
                const uint32_t k = row_key(y, DT);
                if (k >= thr_key) {
                    const uint32_t p = atomicAdd(&sm.bu[3], 1u);
                    if (p < (uint32_t)SURV_CAP) { sm.u.s.key[p] = k; sm.u.s.idx[p] = cv[u].idx; sm.u.s.e[p] = exp((double)y - md); }
                }
            }
        }
    }
    __syncthreads();
    const uint32_t ns = sm.bu[3];
    __syncthreads();
    if (ns > (uint32_t)SURV_CAP || ns == 0) return false;

    uint32_t cut_key = thr_key;
    int32_t cut_i = IDX_ALL;
    int status = MIS_ROW_OK;
    if (pl.topp) {
        double S = 0.0;
        for (uint32_t i = threadIdx.x; i < ns; i += NT) S += sm.u.s.e[i];
        S = block_sum<double>(S, sm.red);
        if (DT == F32) {
            window_cut(sm, sm.u.s.key, sm.u.s.idx, sm.u.s.e, ns, (double)pl.top_p * S, 0.0, &cut_key, &cut_i, DT);
        } else {
            // 16-bit rounding chain over the survivors in stable descending order
            int npow = 1;
            while (npow < (int)ns) npow <<= 1;
            constexpr int PT = SURV_CAP / NT;
            uint64_t kt[PT];
            double et[PT];
            __syncthreads();
            for (int q = 0; q < PT; ++q) {
                const int i = threadIdx.x + q * NT;
                kt[q] = (i < (int)ns) ? (((uint64_t)sm.u.s.key[i] << 32) | (uint64_t)(0xffffffffu - (uint32_t)sm.u.s.idx[i])) : 0ull;
                et[q] = (i < (int)ns) ? sm.u.s.e[i] : 0.0;
            }
            __syncthreads();
            for (int q = 0; q < PT; ++q) {
                const int i = threadIdx.x + q * NT;
                sm.u.so.k[i] = kt[q];
                sm.u.so.e[i] = et[q];
            }
            __syncthreads();
            for (int kk = 2; kk <= npow; kk <<= 1) {      // bitonic sort, descending
                for (int j = kk >> 1; j > 0; j >>= 1) {
                    for (int i = threadIdx.x; i < npow; i += NT) {
                        const int ixj = i ^ j;
                        if (ixj > i) {
                            const bool desc = (i & kk) == 0;
                            const uint64_t x = sm.u.so.k[i], y = sm.u.so.k[ixj];
                            if (desc ? (x < y) : (x > y)) {
                                sm.u.so.k[i] = y; sm.u.so.k[ixj] = x;
                                const double t = sm.u.so.e[i]; sm.u.so.e[i] = sm.u.so.e[ixj]; sm.u.so.e[ixj] = t;
                            }
                        }
                    }
                    __syncthreads();
                }
            }
            if (threadIdx.x == 0) {
                const float thr16 = rn_dtype(pl.top_p, DT);
                float F = 0.0f;
                uint32_t r0 = ns;
                int i = 0;
                while (i < (int)ns) {
                    const uint32_t key = (uint32_t)(sm.u.so.k[i] >> 32);
                    int jn = i + 1;
                    while (jn < (int)ns && (uint32_t)(sm.u.so.k[jn] >> 32) == key) ++jn;
                    const float p = rn_dtype((float)(sm.u.so.e[i] / S), DT);
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
                sm.bu[0] = r0;
                if (r0 > 0) {
                    const uint64_t q = sm.u.so.k[r0 - 1];
                    sm.bu[1] = (uint32_t)(q >> 32);
                    sm.bi[0] = (int32_t)(0xffffffffu - (uint32_t)q);
                }
            }
            __syncthreads();
            const uint32_t r0 = sm.bu[0];
            if (r0 > 0) { cut_key = sm.bu[1]; cut_i = sm.bi[0]; }
            __syncthreads();
            if (r0 == 0) status = MIS_ROW_INVALID;
            for (int q = 0; q < PT; ++q) {               // back to the (key, idx, e) view
                const int i = threadIdx.x + q * NT;
                kt[q] = sm.u.so.k[i];
                et[q] = sm.u.so.e[i];
            }
            __syncthreads();
            for (int q = 0; q < PT; ++q) {
                const int i = threadIdx.x + q * NT;
                if (i < (int)ns) {
                    sm.u.s.key[i] = (uint32_t)(kt[q] >> 32);
                    sm.u.s.idx[i] = (int32_t)(0xffffffffu - (uint32_t)kt[q]);
                    sm.u.s.e[i] = et[q];
                }
            }
            __syncthreads();
        }
    }
    if (status != MIS_ROW_OK) {
        write_row(ro, a, c.row, -1, status, pl.mode, c.m, 0u, 0, 0.0);
        return true;
    }
    double SK = 0.0;
    for (uint32_t i = threadIdx.x; i < ns; i += NT) {
        if (!kept_by_cut(sm.u.s.key[i], sm.u.s.idx[i], cut_key, cut_i)) sm.u.s.e[i] = 0.0;
        SK += sm.u.s.e[i];
    }
    SK = block_sum<double>(SK, sm.red);
    const int64_t id = draw_in_list(sm, sm.u.s.idx, sm.u.s.e, (int)ns, c.V, (double)pl.u * SK);
    write_row(ro, a, c.row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, c.m, cut_key, cut_i, SK);
    return true;
}

// fp32 top-p.  Merge the chunks' fine bins (16 per unit of y below each
// chunk max, float64 masses) on the row grid and find the bin holding the
// cut.  Re-read the row -- it has just been read, so it comes from the
// Infinity Cache -- to collect that bin's elements into LDS, histogramming
// the bin first (256 sub-bins) when it is crowded.  The exact cut is then a
// mass descent over at most SURV_CAP elements.  Per-chunk kept weights: the
// chunk's whole bins above the window plus its part of the window.
template <int DT>
__device__ __noinline__ void final_topp32(Smem &sm, RowCx &c, const RowPlan &pl, const ChunkSum *csr, RowOut *ro,
                                          const Args &a)
{
    const int tid = threadIdx.x, G = c.G;
    uint32_t anyflag = 0;
    float m = -INFINITY;
    for (int g = tid; g < G; g += NT) { anyflag |= csr[g].flags; m = fmaxf(m, csr[g].ymax); }
    anyflag = block_sum<uint32_t>(anyflag ? 1u : 0u, sm.red);
    m = block_max<float>(m, sm.red);
    c.m = m;
    if (anyflag != 0u || m == -INFINITY) {
        write_row(ro, a, c.row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
        return;
    }
    const double md = (double)m;
    const double gm = floor(md * (double)FB_W);
    // chunk g's bin 0 sits offg[g] row bins below the row's bin 0 (-1: empty chunk)
    int *offg = reinterpret_cast<int *>(sm.sub_c);
    for (int g = tid; g < G; g += NT) {
        const float yg = csr[g].ymax;
        sm.chs[g] = yg == -INFINITY ? 0.0 : exp((double)yg - md);
        offg[g] = yg == -INFINITY ? -1 : (int)(gm - csr[g].gmc);
    }
    __syncthreads();
    double s = 0.0;
    for (int g = tid; g < G; g += NT) if (offg[g] >= 0) s += csr[g].S * sm.chs[g];
    const double S = block_sum<double>(s, sm.red);
    const double A = (double)pl.top_p * S;
    for (int rb = tid; rb < FB_N; rb += NT) {
        double mm = 0.0;
        uint32_t cc = 0;
        for (int g0 = 0; g0 < G; g0 += 8) {
            int off[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) off[u] = g0 + u < G ? offg[g0 + u] : -1;
            double mv[8];
            uint32_t cv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int cb = rb - off[u];
                const bool in = off[u] >= 0 && cb >= 0 && cb < FB_N;
                const size_t at = (size_t)(g0 + u < G ? g0 + u : 0) * FB_N + (in ? cb : 0);
                mv[u] = in ? c.fbm[at] : 0.0;
                cv[u] = in ? c.fbc[at] : 0u;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) { mm += mv[u] * (g0 + u < G ? sm.chs[g0 + u] : 0.0); cc += cv[u]; }
        }
        sm.v.rb.m[FB_N - 1 - rb] = mm;
        sm.v.rb.c[FB_N - 1 - rb] = cc;
    }
    __syncthreads();
    if (wave_id() == 0) {
        double ab;
        const int d = wave_find_desc<double>(sm.v.rb.m, FB_N, A, &ab);
        double tot = 0.0;
        for (int q = lane_id(); q < FB_N; q += 64) tot += sm.v.rb.m[q];
        tot = wave_sum(tot);
        if (lane_id() == 0) {
            sm.bi[2] = (tot >= A) ? (FB_N - 1 - d) : -1;  // -1: the cut lies below the bins
            sm.bd[4] = ab;
            sm.bu[2] = sm.v.rb.c[d];
        }
    }
    __syncthreads();
    const int rbstar = sm.bi[2];
    double A_above = sm.bd[4];
    const uint32_t wcnt = sm.bu[2];
    __syncthreads();
    if (rbstar < 0) {
        final_generic<DT>(sm, c, pl, ro, a);
        return;
    }
    const double gb = gm - (double)rbstar;  // the bin is [gb/FB_W, (gb+1)/FB_W)
    const float hlo = (float)(gb / (double)FB_W), hhi = (float)((gb + 1.0) / (double)FB_W);
    const uint32_t klo = key_of_f32(hlo), khi = key_of_f32(hhi) - 1u;
    // each chunk's whole bins above the window's row bin, one wave per chunk
    for (int g = wave_id(); g < G; g += NWAVE) {
        const int off = offg[g];
        double w = 0.0;
        if (off >= 0) {
            const int nb = rbstar - off <= 0 ? 0 : (rbstar - off >= FB_N ? FB_N : rbstar - off);
            const double *fm = c.fbm + (size_t)g * FB_N;
            double t[FB_N / 64];
#pragma unroll
            for (int q = 0; q < FB_N / 64; ++q) {
                const int cb = q * 64 + lane_id();
                t[q] = cb < nb ? fm[cb] : 0.0;
            }
#pragma unroll
            for (int q = 0; q < FB_N / 64; ++q) w += t[q];
        }
        w = wave_sum(w);
        if (lane_id() == 0) sm.cw[g] = w * sm.chs[g];
    }
    uint32_t wklo = klo, wkhi = khi;  // the window; (wkhi, khi] adds to the chunks' weights
    if (wcnt > (uint32_t)WCAP) {
        // crowded bin: 256 sub-bins of [hlo, hhi) by a re-read (index 255 = top)
        __syncthreads();
        for (int i = tid; i < 256; i += NT) { sm.v.l1.cnt[i] = 0u; sm.v.l1.mass[i] = 0.0; }
        uint32_t xlo, xhi;
        x_interval<DT>(sm, klo, khi, c.T, &xlo, &xhi);
        const float inv = 256.0f / (hhi - hlo);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float y, uint32_t k) {
            if (k < klo || k > khi) return;
            const int sb = min(255, (int)((hhi - y) * inv));
            atomicAdd(&sm.v.l1.cnt[255 - sb], 1u);
            atomicAdd(&sm.v.l1.mass[255 - sb], exp((double)y - md));
        });
        __syncthreads();
        if (wave_id() == 0) {
            double ab;
            const int d = wave_find_desc<double>(sm.v.l1.mass, 256, A - A_above, &ab);
            if (lane_id() == 0) { sm.bi[3] = 255 - d; sm.bd[5] = ab; sm.bu[3] = sm.v.l1.cnt[d]; }
        }
        __syncthreads();
        const int sstar = sm.bi[3];
        A_above += sm.bd[5];
        const uint32_t scnt = sm.bu[3];
        __syncthreads();
        // key range of sub-bin sstar inside [klo, khi]; the sub-bin index is
        // non-increasing in the key
        if (wave_id() == 0) {
            auto sbk = [&](uint32_t k) -> int { return min(255, (int)((hhi - f32_of_key(k)) * inv)); };
            uint64_t lo = klo, hi = khi;  // smallest key with sbk <= sstar
            if (sbk(klo) <= sstar) hi = klo;
            else {
                while (hi - lo > 1) {
                    uint64_t step = (hi - lo) / 64; if (step == 0) step = 1;
                    const uint64_t p = lo + (uint64_t)(lane_id() + 1) * step;
                    const bool pred = p >= hi ? true : (sbk((uint32_t)p) <= sstar);
                    const uint64_t mk = __ballot(pred);
                    if (mk == 0ull) { lo = lo + 64 * step; continue; }
                    const int f = __builtin_ctzll(mk);
                    const uint64_t nhi = lo + (uint64_t)(f + 1) * step;
                    if (nhi < hi) hi = nhi;
                    lo = lo + (uint64_t)f * step;
                }
            }
            uint64_t lo2 = klo, hi2 = khi;  // largest key with sbk >= sstar
            if (sbk(khi) >= sstar) lo2 = khi;
            else {
                while (hi2 - lo2 > 1) {
                    uint64_t step = (hi2 - lo2) / 64; if (step == 0) step = 1;
                    const uint64_t p = lo2 + (uint64_t)(lane_id() + 1) * step;
                    const bool pred = p >= hi2 ? true : (sbk((uint32_t)p) < sstar);
                    const uint64_t mk = __ballot(pred);
                    if (mk == 0ull) { lo2 = lo2 + 64 * step; continue; }
                    const int f = __builtin_ctzll(mk);
                    const uint64_t nhi = lo2 + (uint64_t)(f + 1) * step;
                    if (nhi < hi2) hi2 = nhi;
                    lo2 = lo2 + (uint64_t)f * step;
                }
            }
            if (lane_id() == 0) { sm.bu[4] = (uint32_t)hi; sm.bu[5] = (uint32_t)lo2; }
        }
        __syncthreads();
        wklo = sm.bu[4];
        wkhi = sm.bu[5];
        __syncthreads();
        if (scnt > (uint32_t)WCAP || wklo > wkhi) {
            final_generic<DT>(sm, c, pl, ro, a);
            return;
        }
    }
    // collect [wklo, wkhi] into LDS; (wkhi, khi] is kept mass of its chunks
    __syncthreads();
    if (tid == 0) sm.bu[6] = 0u;
    uint32_t xlo, xhi;
    x_interval<DT>(sm, wklo, khi, c.T, &xlo, &xhi);
    rescan<DT>(c, xlo, xhi, [&](int64_t j, float y, uint32_t k) {
        if (k < wklo || k > khi) return;
        const double e = exp((double)y - md);
        if (k <= wkhi) {
            const uint32_t p = atomicAdd(&sm.bu[6], 1u);
            if (p < (uint32_t)SURV_CAP) { sm.u.s.key[p] = k; sm.u.s.idx[p] = (int32_t)j; sm.u.s.e[p] = e; }
        } else {
            atomicAdd(&sm.cw[j / c.CH], e);
        }
    });
    __syncthreads();
    const uint32_t nw0 = sm.bu[6];
    __syncthreads();
    if (nw0 > (uint32_t)SURV_CAP) {
        final_generic<DT>(sm, c, pl, ro, a);
        return;
    }
    const uint32_t nw = nw0;
    uint32_t cut_key;
    int32_t cut_i;
    window_cut(sm, sm.u.s.key, sm.u.s.idx, sm.u.s.e, nw, A - A_above, 0.0, &cut_key, &cut_i, DT);
    for (uint32_t i = tid; i < nw; i += NT)
        if (kept_by_cut(sm.u.s.key[i], sm.u.s.idx[i], cut_key, cut_i))
            atomicAdd(&sm.cw[sm.u.s.idx[i] / c.CH], sm.u.s.e[i]);
    int gsel;
    double resid, SK;
    pick_chunk(sm, G, pl.u, &gsel, &resid, &SK);
    int64_t id = -1;
    if (gsel >= 0) {
        const float T = pl.T;
        id = draw_in_chunk<DT>(sm, c, gsel, resid, [&](float xv, int64_t j) -> double {
            const float y = scale_y<DT>(xv, T);
            return (y != -INFINITY && kept_by_cut(row_key(y, DT), j, cut_key, cut_i)) ? exp((double)y - md) : 0.0;
        });
    }
    write_row(ro, a, c.row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, cut_key, cut_i, SK);
}

// Leader of a row that needs no refinement rounds: greedy, temperature only,
// small top-k, and the re-read path for everything else.
template <int DT>
__device__ __noinline__ void final_row(Smem &sm, RowCx &c, const RowPlan &pl, const ChunkSum *csr, RowOut *ro,
                                       const Args &a)
{
    const int tid = threadIdx.x, row = c.row;
    const Layout &L = a.L;
    if (pl.mode == M_BAD) {
        write_row(ro, a, row, -1, MIS_ROW_BAD_PARAM, pl.mode, 0.0f, 0u, 0, 0.0);
        return;
    }
    uint32_t k2 = 0u;
    int32_t i2 = IDX_ALL;
    uint32_t anyflag = 0u;
    float m = -INFINITY;
    for (int g = tid; g < L.G; g += NT) {
        ChunkSum s;
        s.xkey = ld_dev(&csr[g].xkey); s.xarg = ld_dev(&csr[g].xarg);
        s.flags = ld_dev(&csr[g].flags); s.ymax = ld_dev(&csr[g].ymax);
        if (s.xkey > k2 || (s.xkey == k2 && s.xarg < i2)) { k2 = s.xkey; i2 = s.xarg; }
        anyflag |= s.flags;
        m = fmaxf(m, s.ymax);
    }
    wave_argmax(k2, i2);
    if (lane_id() == 0) { sm.red.u[wave_id()] = k2; sm.red.l[wave_id()] = i2; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NWAVE; ++w) {
            const uint32_t kk = sm.red.u[w];
            const int32_t ii = (int32_t)sm.red.l[w];
            if (kk > k2 || (kk == k2 && ii < i2)) { k2 = kk; i2 = ii; }
        }
        sm.bi[0] = i2;
    }
    __syncthreads();
    i2 = sm.bi[0];
    __syncthreads();
    anyflag = block_sum<uint32_t>(anyflag ? 1u : 0u, sm.red);
    m = block_max<float>(m, sm.red);
    c.m = m;
    const double md = (double)m;
    if (pl.mode == M_GREEDY) {
        write_row(ro, a, row, i2, MIS_ROW_OK, pl.mode, 0.0f, 0u, i2, 1.0);
    } else if (anyflag != 0u || m == -INFINITY) {
        write_row(ro, a, row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
    } else if (pl.mode == M_TEMP) {
        // chunk weights are exp(y - ymax_c): rescale to the row max m
        for (int g = tid; g < L.G; g += NT) {
            const float yg = ld_dev(&csr[g].ymax);
            sm.chs[g] = yg == -INFINITY ? 0.0 : exp((double)yg - md);
            sm.cw[g] = ld_dev(&csr[g].S) * sm.chs[g];
        }
        int gsel;
        double resid, SK;
        pick_chunk(sm, L.G, pl.u, &gsel, &resid, &SK);
        int64_t id = -1;
        if (gsel >= 0) {
            constexpr float L2E = 1.44269504088896341f;
            const float yc = ld_dev(&csr[gsel].ymax), T = pl.T;
            id = draw_in_chunk<DT>(sm, c, gsel, resid / sm.chs[gsel], [&](float xv, int64_t) -> double {
                return (double)exp2f((scale_y<DT>(xv, T) - yc) * L2E);
            });
        }
        write_row(ro, a, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, row_key(-INFINITY, DT), -1, SK);
    } else if (pl.mode == M_SMALLK) {
        bool ovf = false;
        for (int g = 0; g < L.G; ++g) ovf |= (ld_dev(&csr[g].ncand) == NCAND_OVERFLOW);
        const Cand *cand = reinterpret_cast<const Cand *>(a.ws + L.cand) + (size_t)row * L.G * CAND_CAP;
        bool done = false;
        if (!ovf) done = final_smallk<DT>(sm, c, pl, csr, cand, ro, a);
        if (!done) final_generic<DT>(sm, c, pl, ro, a);
    } else {
        final_generic<DT>(sm, c, pl, ro, a);
    }
}

// ------------------------------------------------------------------ the chunk pass

// One workgroup per (row, chunk): one coalesced read of the chunk into
// registers -- the only HBM read of the logits -- reduced to the chunk
// summary the row pass needs for the row's mode.
template <int DT, int EPT>
__global__ __launch_bounds__(NT) void k_chunk(Args a)
{
    constexpr int VEC = Traits<DT>::VEC, NV = EPT / VEC, CH = NT * EPT;
    __shared__ ChunkSmem sm;
    const Layout &L = a.L;
    const int tid = threadIdx.x;
    const uint32_t task = blockIdx.x;
    const uint32_t G = (uint32_t)L.G;
    const int row = uni((int32_t)(task / G)), chunk = uni((int32_t)(task % G));
    const int64_t V = a.V;
    const int64_t base = (int64_t)chunk * CH;
    const char *rowp = a.logits + (int64_t)row * a.stride_bytes;
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, V);
    ChunkSum *csr = reinterpret_cast<ChunkSum *>(a.ws + L.chunks) + (size_t)row * L.G;
    ChunkSum *cs = csr + chunk;

    // ---- one coalesced read of the chunk into registers
    float x[EPT];
    if (a.vec_ok && base + CH <= V) {  // whole chunk inside the row: all loads issued back to back
#pragma unroll
        for (int v = 0; v < NV; ++v) loadvec<DT>(rowp, base + ((int64_t)v * NT + tid) * VEC, &x[v * VEC]);
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int64_t j0 = base + ((int64_t)v * NT + tid) * VEC;
            if (a.vec_ok && j0 + VEC <= V) {
                loadvec<DT>(rowp, j0, &x[v * VEC]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) x[v * VEC + e] = (j0 + e < V) ? load1<DT>(rowp, j0 + e) : 0.0f;
            }
        }
    }
    // element i of this thread sits at base + lofs(i); `valid` has bit i set
    // when that index is inside the row
    auto lofs = [&](int i) -> uint32_t { return (uint32_t)(((i / VEC) * NT + tid) * VEC + (i % VEC)); };
    const int32_t base32 = (int32_t)base;  // V < 2^31
    auto idx_of = [&](int i) -> int32_t { return base32 + (int32_t)lofs(i); };
    uint64_t valid = ~0ull;
    {
        const int64_t lim = V - base;  // elements of this chunk inside the row
        if (lim < (int64_t)CH) {
            valid = 0ull;
            const uint32_t lim32 = (uint32_t)lim;
#pragma unroll
            for (int i = 0; i < EPT; ++i) valid |= (lofs(i) < lim32 ? 1ull : 0ull) << i;
        }
    }
    auto ok_ = [&](int i) -> bool { return (valid >> i) & 1ull; };

    // ---- argmax of the raw logits (NaN ranks first)
    uint32_t bk = 0u;
    int32_t bi = IDX_ALL;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        if (ok_(i)) {
            const uint32_t k = argmax_key(x[i]);
            if (k > bk) { bk = k; bi = idx_of(i); }
        }
    }
    wave_argmax(bk, bi);
    if (lane_id() == 0) { sm.red.u[wave_id()] = bk; sm.red.l[wave_id()] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NWAVE; ++w) {
            const uint32_t k2 = sm.red.u[w];
            const int32_t i2 = (int32_t)sm.red.l[w];
            if (k2 > bk || (k2 == bk && i2 < bi)) { bk = k2; bi = i2; }
        }
        sm.bu[0] = bk;
        sm.bi[0] = bi;
    }
    __syncthreads();
    bk = sm.bu[0];
    bi = sm.bi[0];
    __syncthreads();

    uint32_t flags = 0u;
    float xmax = -INFINITY, ymax = -INFINITY;
    if (pl.mode != M_BAD && pl.mode != M_GREEDY) {
        if (bk == 0xffffffffu) flags |= FLAG_NAN;
        else {
            xmax = f32_of_key(bk);
            ymax = scale_y<DT>(xmax, pl.T);  // scaling is monotone
            if (ymax == INFINITY) flags |= FLAG_PINF;
        }
    }
    const bool live = (pl.mode != M_BAD && pl.mode != M_GREEDY && flags == 0u);
    const bool topp32 = (DT == F32 && pl.mode == M_TOPP);

    // ---- phase 1 per mode
    uint32_t ncand = 0;
    double Sc = 0.0, below = 0.0, gmc = 0.0;
    if (live && pl.mode == M_SMALLK) {
        uint32_t nfin = 0;
        float xminf = INFINITY;
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if (ok_(i) && x[i] != -INFINITY) { nfin++; xminf = fminf(xminf, x[i]); }
        nfin = block_sum<uint32_t>(nfin, sm.red);
        xminf = block_min<float>(xminf, sm.red);
        // candidates: finite x >= xlo_c, where xlo_c keeps the chunk's top k'.
        // Bins are linear in the raw value over [xminf, xmax] (index 255 = top).
        float xlo_c = -INFINITY;
        if (nfin > (uint32_t)pl.kk && xmax > xminf) {
            const float inv = 256.0f / (xmax - xminf);
            sm.u.h8.cnt[tid] = 0u;
            __syncthreads();
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                if (ok_(i) && x[i] != -INFINITY) {
                    const int b = min(255, (int)((xmax - opaque(x[i])) * inv));
                    atomicAdd(&sm.u.h8.cnt[255 - b], 1u);
                }
            }
            __syncthreads();
            if (wave_id() == 0) {
                uint32_t above;
                const int d = wave_find_desc<uint32_t>(sm.u.h8.cnt, 256, (uint32_t)pl.kk, &above);
                if (lane_id() == 0) { sm.bu[0] = (uint32_t)(255 - d); sm.bu[1] = above; sm.bu[2] = sm.u.h8.cnt[d]; }
            }
            __syncthreads();
            const int bstar = (int)sm.bu[0];
            const uint32_t above_b = sm.bu[1], in_b = sm.bu[2];
            __syncthreads();
            int sstar = 255;
            if (above_b + in_b > (uint32_t)CAND_CAP) {
                // refine the boundary bin into 256 sub-bins
                sm.u.h8.cnt[tid] = 0u;
                __syncthreads();
#pragma unroll
                for (int i = 0; i < EPT; ++i) {
                    if (ok_(i) && x[i] != -INFINITY) {
                        const float t = (xmax - opaque(x[i])) * inv;
                        const int b = min(255, (int)t);
                        if (b == bstar) atomicAdd(&sm.u.h8.cnt[255 - min(255, (int)((t - (float)b) * 256.0f))], 1u);
                    }
                }
                __syncthreads();
                if (wave_id() == 0) {
                    uint32_t above;
                    const int d = wave_find_desc<uint32_t>(sm.u.h8.cnt, 256, (uint32_t)pl.kk - above_b, &above);
                    if (lane_id() == 0) sm.bu[0] = (uint32_t)(255 - d);
                }
                __syncthreads();
                sstar = (int)sm.bu[0];
                __syncthreads();
            }
            // smallest raw value inside the selected bins
            float xb = INFINITY;
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                if (ok_(i) && x[i] != -INFINITY) {
                    const float t = (xmax - opaque(x[i])) * inv;
                    const int b = min(255, (int)t);
                    if (b < bstar || (b == bstar && min(255, (int)((t - (float)b) * 256.0f)) <= sstar))
                        xb = fminf(xb, opaque(x[i]));
                }
            }
            xb = block_min<float>(xb, sm.red);
            // close the set under the ties the scaling creates: every x whose
            // scaled key equals that of xb is a candidate too
            uint32_t xlo, xhi;
            const uint32_t kb = row_key(scale_y<DT>(xb, pl.T), DT);
            x_interval<DT>(sm, kb, kb, pl.T, &xlo, &xhi);
            xlo_c = f32_of_key(xlo);
        }
        uint32_t mine = 0;
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if (ok_(i) && x[i] != -INFINITY && x[i] >= xlo_c) mine++;
        uint32_t total;
        uint32_t off = block_excl_scan<uint32_t>(mine, sm.red, &total);
        if (total <= (uint32_t)CAND_CAP) {
            Cand *cand = reinterpret_cast<Cand *>(a.ws + L.cand) + ((size_t)row * L.G + chunk) * CAND_CAP;
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                if (ok_(i) && x[i] != -INFINITY && x[i] >= xlo_c) {
                    st_dev_cand(&cand[off++], x[i], idx_of(i));
                }
            }
            ncand = total;
        } else {
            ncand = NCAND_OVERFLOW;
        }
    } else if (live && pl.mode == M_TEMP) {
        // draw weights exp(y - ymax_c) in f32 on the scaled values y =
        // dtype(x / T) (within the draw's tolerance), float64 sums.  Weights
        // taken on x / T before its rounding would be off by |y| ulps.
        double s = 0.0;
        if (ymax != -INFINITY) {
            constexpr float L2E = 1.44269504088896341f;
#pragma unroll
            for (int i = 0; i < EPT; ++i)
                if (ok_(i)) s += (double)exp2f((scale_y<DT>(x[i], pl.T) - ymax) * L2E);
        }
        Sc = block_sum<double>(s, sm.red);
    } else if (live && topp32) {
        // exact y, float64 weights relative to the chunk max, fine bins on the
        // global grid floor(y * FB_W)
        for (int i = tid; i < FB_N; i += NT) { sm.u.p1.cnt[i] = 0u; sm.u.p1.mass[i] = 0.0; }
        __syncthreads();
        const double ym = (double)ymax;
        gmc = ymax == -INFINITY ? 0.0 : floor(ym * (double)FB_W);
        double s = 0.0, bl = 0.0;
        if (ymax != -INFINITY) {
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                if (ok_(i)) {
                    const float y = scale_y<DT>(x[i], pl.T);
                    if (y != -INFINITY) {
                        const double e = exp((double)y - ym);
                        s += e;
                        const double rb = gmc - floor((double)y * (double)FB_W);
                        if (rb < (double)FB_N) {
                            const int b = (int)rb;
                            atomicAdd(&sm.u.p1.cnt[b], 1u);
                            atomicAdd(&sm.u.p1.mass[b], e);
                        } else {
                            bl += e;
                        }
                    }
                }
            }
        }
        Sc = block_sum<double>(s, sm.red);
        below = block_sum<double>(bl, sm.red);
        uint32_t *gc = reinterpret_cast<uint32_t *>(a.ws + L.fbc) + ((size_t)row * L.G + chunk) * FB_N;
        double *gm = reinterpret_cast<double *>(a.ws + L.fbm) + ((size_t)row * L.G + chunk) * FB_N;
        for (int i = tid; i < FB_N; i += NT) { st_dev(&gc[i], sm.u.p1.cnt[i]); st_dev(&gm[i], sm.u.p1.mass[i]); }
    } else if (live) {
        // large k' and fp16/bf16 top-p: the leader re-reads the row
        double s = 0.0;
        if (ymax != -INFINITY) {
            const double ym = (double)ymax;
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                if (ok_(i)) {
                    const float y = scale_y<DT>(x[i], pl.T);
                    if (y != -INFINITY) s += exp((double)y - ym);
                }
            }
        }
        Sc = block_sum<double>(s, sm.red);
    }
    if (tid == 0) {
        st_dev(&cs->xkey, bk); st_dev(&cs->xarg, bi); st_dev(&cs->ymax, ymax); st_dev(&cs->flags, flags);
        st_dev(&cs->ncand, ncand); st_dev(&cs->xmax, xmax); st_dev(&cs->S, Sc); st_dev(&cs->gmc, gmc);
        st_dev(&cs->below, below);
    }
}

// ------------------------------------------------------------------ the row pass

// One workgroup per row: merges the row's chunk summaries and finishes the
// row (the functions above), re-reading parts of the row where needed.
template <int DT>
__global__ __launch_bounds__(NT) void k_final(Args a)
{
    __shared__ Smem sm;
    const Layout &L = a.L;
    const int row = blockIdx.x;
    if (threadIdx.x == 0) {
        sm.args = a;
        RowCx &c = sm.cx;
        c.rowp = a.logits + (int64_t)row * a.stride_bytes;
        c.V = a.V; c.vec_ok = a.vec_ok; c.m = 0.0f; c.G = L.G; c.CH = (int64_t)NT * L.ept; c.row = row;
        c.fbc = reinterpret_cast<const uint32_t *>(a.ws + L.fbc) + (size_t)row * L.G * FB_N;
        c.fbm = reinterpret_cast<const double *>(a.ws + L.fbm) + (size_t)row * L.G * FB_N;
        c.subc = nullptr; c.subm = nullptr;
        sm.pl = plan_row(a.params[row], a.V);
        c.T = sm.pl.T;
    }
    __syncthreads();
    const ChunkSum *csr = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * L.G;
    RowOut *ro = reinterpret_cast<RowOut *>(a.ws + L.rowout) + row;
    if (DT == F32 && sm.pl.mode == M_TOPP) final_topp32<DT>(sm, sm.cx, sm.pl, csr, ro, sm.args);
    else final_row<DT>(sm, sm.cx, sm.pl, csr, ro, sm.args);
}

// ------------------------------------------------------------------ debug emit

template <int DT>
__global__ __launch_bounds__(NT) void k_emit(const char *__restrict__ logits, int64_t V, int64_t stride_bytes,
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
        const int64_t j = (int64_t)blockIdx.x * NT * PER + (int64_t)it * NT + threadIdx.x;
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
                if (kept) prob = rn_dtype((float)(exp((double)y - md) / ro.S), DT);
            }
        }
        if (out_probs && j < V) out_probs[(size_t)row * V + j] = prob;
        const uint64_t ball = __ballot(kept);
        if (out_keep && (threadIdx.x & 63) == 0) {
            const int64_t w0 = j / 32;
            if (w0 < words) out_keep[(size_t)row * words + w0] = (uint32_t)ball;
            if (w0 + 1 < words) out_keep[(size_t)row * words + w0 + 1] = (uint32_t)(ball >> 32);
        }
    }
}

// ------------------------------------------------------------------ host side

static thread_local int g_last_hip = 0;

template <int DT, int EPT>
static hipError_t launch_chunk(const Args &a, hipStream_t st)
{
    const unsigned grid = (unsigned)(a.L.B * a.L.G);
    hipLaunchKernelGGL((k_chunk<DT, EPT>), dim3(grid), dim3(NT), 0, st, a);
    return hipGetLastError();
}

// events (optional): [0] before the chunk pass, [1] between the chunk pass
// and the row pass, [2] after the row pass
template <int DT>
static hipError_t launch_dt(const Args &a, float *probs, uint32_t *keep, hipStream_t st, void *const *ev)
{
    hipError_t e;
    if (ev && (e = hipEventRecord((hipEvent_t)ev[0], st)) != hipSuccess) return e;
    switch (a.L.ept) {
    case 64: e = launch_chunk<DT, 64>(a, st); break;
    case 32: e = launch_chunk<DT, 32>(a, st); break;
    case 16: e = launch_chunk<DT, 16>(a, st); break;
    default: e = launch_chunk<DT, 8>(a, st); break;
    }
    if (e != hipSuccess) return e;
    if (ev && (e = hipEventRecord((hipEvent_t)ev[1], st)) != hipSuccess) return e;
    hipLaunchKernelGGL((k_final<DT>), dim3((unsigned)a.L.B), dim3(NT), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (ev && (e = hipEventRecord((hipEvent_t)ev[2], st)) != hipSuccess) return e;
    if (probs || keep) {
        const unsigned gx = (unsigned)((a.V + (int64_t)NT * 8 - 1) / ((int64_t)NT * 8));
        hipLaunchKernelGGL((k_emit<DT>), dim3(gx, (unsigned)a.L.B), dim3(NT), 0, st, a.logits, a.V, a.stride_bytes,
                           a.params, a.L, (const char *)a.ws, probs, keep);
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
    return mis::make_layout(B, V, dtype).total;
}

int mis_workspace_init(void *workspace, size_t workspace_bytes, void *stream)
{
    if (!workspace) return MIS_ERR_INVALID_ARG;
    if (((uintptr_t)workspace & 255u) != 0 || workspace_bytes < mis::CTL_PREFIX) return MIS_ERR_WORKSPACE;
    const hipError_t e = hipMemsetAsync(workspace, 0, mis::CTL_PREFIX, (hipStream_t)stream);
    if (e != hipSuccess) { mis::g_last_hip = (int)e; return MIS_ERR_HIP; }
    return MIS_OK;
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
    if (V > (int64_t)1 << 30 || B > B_MAX) return MIS_ERR_UNSUPPORTED;
    const Layout L = make_layout(B, V, dtype);
    if (L.G > G_MAX || (int64_t)L.B * L.G > 0x7fffffff) return MIS_ERR_UNSUPPORTED;
    if (workspace_bytes < L.total || ((uintptr_t)workspace & 255u) != 0) return MIS_ERR_WORKSPACE;
    const int esz = dtype == MIS_DTYPE_F32 ? 4 : 2;
    Args a;
    a.logits = (const char *)logits;
    a.V = V;
    a.stride_bytes = row_stride * esz;
    a.vec_ok = (((uintptr_t)logits & 15u) == 0 && (a.stride_bytes & 15) == 0) ? 1 : 0;
    a.params = params;
    a.L = L;
    a.ws = (char *)workspace;
    a.out_ids = out_ids;
    a.out_status = out_status;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    if (dtype == MIS_DTYPE_F32) e = launch_dt<F32>(a, out_probs, out_keep, st, events);
    else if (dtype == MIS_DTYPE_F16) e = launch_dt<F16>(a, out_probs, out_keep, st, events);
    else e = launch_dt<BF16>(a, out_probs, out_keep, st, events);
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
