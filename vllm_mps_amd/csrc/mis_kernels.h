// mis_kernels.h -- the sampler kernels and their per-dtype launch sequence.
//
// Included by one translation unit per logits dtype (mis_f32.hip,
// mis_f16.hip, mis_bf16.hip), each of which instantiates launch_dt<DT> for
// its dtype, so the three device builds compile in parallel.  The C ABI
// (mis_api.hip) calls them through mis_launch.h.
#pragma once

// MI355X (gfx950) decode-step token sampler behind the C ABI declared in
// include/mis_sampler.h.  Stateless: every launch reads only what the same
// call's earlier launches wrote (stream order); no workgroup waits on
// another.
//
// k_sample (chunk pass): B*G workgroups of 256 threads, one per (row,
// chunk).  Each loads its chunk into registers with coalesced 16-byte
// vector reads -- the only full HBM read of the logits -- and reduces it by
// the row's mode into a per-(row, chunk) summary:
//   greedy       argmax of the raw logits;
//   temperature  chunk max and the sum of weights relative to it;
//   small top-k  the elements above a floor taken from the per-thread maxima
//                (closed under the ties the scaling creates) as candidates;
//   fp32 top-p   float64 sum of exact weights and coarse mass bins;
//   16-bit top-p a large batch: the 512 largest values as candidates and a
//                float64 sum; a small batch: nothing but clearing the row's
//                key histogram (the t16 passes read the chunk again).
// Then, by row kind:
//   k_rowpass    greedy, temperature and small top-k rows (1024 threads per
//                row): candidates, radix select, top-p over the survivors,
//                the draw;
//   k_tp_hist, k_tp_final   fp32 top-p rows spread over the GPU: fine bins
//                and a stash per chunk, then the exact cut per row;
//   k_t16_hist, k_t16_walk, k_t16_final   fp16/bf16 top-p rows of small
//                batches: per-chunk key histograms merged per row, the
//                rounding chain walked by one wave, the draw;
//   k_final      everything else (the generic re-read path, the 16-bit probe
//                of large batches) and the rows the other passes deferred.
// k_emit: debug probabilities / keep bitmask from each row's cut.
//
// Semantics follow model/sampler.py:18-60 per row: greedy argmax (ties ->
// lowest index) when T == 0; y = dtype(f32(x) / T); top-k keeps y >= k'-th
// largest (all ties); top-p on the stable descending order with exact masses
// (fp32 rows) or torch's 16-bit rounding chain (fp16/bf16 rows); the draw is
// min{i : sum_{j<=i} w_j > u * sum w} over the kept weights w = exp(y - m).
#include <hip/hip_runtime.h>
#include <float.h>
#include <math.h>
#include <stdint.h>


#include "mis_device.h"
#include "mis_launch.h"
#include "mis_layout.h"
#include "mis_sampler.h"

namespace mis {
// everything below is local to the including translation unit: each per-dtype
// unit holds its own copy of the dtype-independent kernels and helpers
namespace {

// ------------------------------------------------------------------ phase timestamps
//
// Built with -DMIS_TRACE, thread 0 of a workgroup records the 100 MHz real-time
// counter at phase boundaries into a per-row table placed past the workspace
// (the caller then sizes the workspace with mis_workspace_bytes() + the
// table).  Off in the product build: the calls compile to nothing.
[[maybe_unused]] constexpr int TR_SLOTS = 32;
#ifdef MIS_TRACE
__device__ __forceinline__ void trace(char *ws, const Layout &L, int row, int slot)
{
    if (threadIdx.x == 0 && slot < TR_SLOTS) {
        uint64_t *t = reinterpret_cast<uint64_t *>(ws + L.total) + (size_t)row * TR_SLOTS + slot;
        __hip_atomic_store(t, (uint64_t)__builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
#else
__device__ __forceinline__ void trace(char *, const Layout &, int, int) {}
#endif

// ------------------------------------------------------------------ row plan

struct RowPlan { int mode; int kk; int topp; float T; float top_p; float u; };

__device__ __forceinline__ RowPlan plan_row(const mis_row_params &P, int64_t V)
{
    RowPlan r;
    r.T = P.temperature; r.top_p = P.top_p; r.u = P.uniform; r.kk = 0; r.topp = 0;
    const bool bad = P.temperature < 0.0f || P.top_k < 0 || !(P.top_p > 0.0f) || !(P.uniform == P.uniform);
    if (bad) { r.mode = M_BAD; return r; }
    // x / NaN is NaN everywhere: the reference's multinomial rejects the row
    if (P.temperature != P.temperature) { r.mode = M_INVAL; return r; }
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


struct RowCx {                 // what the leader of a row works with
    const char *rowp;
    int64_t V;
    int vec_ok;
    float T;
    float m;                   // row max of y
    int G;
    int64_t CH;
    int row;
};

// ------------------------------------------------------------------ shared memory

// LDS of the row pass (one workgroup per row): the survivor / window arrays
// and the re-read path's histograms share the big union.
struct Smem {
    union {
        struct { uint32_t cnt[2048]; } h11;                                                 // 8 KB
        struct { uint32_t cnt[256]; double mass[256]; } h8;                                 // 3 KB
        struct { uint32_t key[SURV_CAP]; int32_t idx[SURV_CAP]; double e[SURV_CAP]; } s;    // 16 KB
        struct { uint64_t k[SURV_CAP]; double e[SURV_CAP]; } so;                           // 16 KB
        struct { int32_t idx[TIE_CAP]; } t;
    } u;
    union {
        struct { uint32_t cnt[256]; double mass[256]; } l1;  // re-read path: level-1 histogram
        double coarse[CB_N];                                 // leader merge of coarse bins
    } v;
    double cw[G_MAX];          // per-chunk kept weight
    double etab[ETAB_N];       // 2^(j/64) for dexp
    union {
        Cand cc[CCAP_FIN];     // a small-k row's candidates
        struct { uint32_t cnt[RUN_CAP]; uint32_t rkey[RUN_CAP]; uint32_t rcnt[RUN_CAP]; float rp[RUN_CAP]; } r;  // 16-bit chain runs
    } w;
    double chs[G_MAX];         // per-chunk rescale to the row max
    double sub_m[256];         // round-local histograms
    uint32_t sub_c[256];
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

// LDS of the chunk pass: only what its per-mode reductions need (17 KB), so
// that more of its workgroups fit on a CU
struct ChunkSmem {
    double wb[NWAVE][CB_N];    // per-wave coarse bins (fp32 top-p)
    double etab[ETAB_N];       // 2^(j/64) for dexp
    Red red;
    uint32_t bu[8];
};

__device__ __forceinline__ bool kept_by_cut(uint32_t key, int64_t j, uint32_t cut_key, int32_t cut_i)
{
    return key > cut_key || (key == cut_key && j <= (int64_t)cut_i);
}

// Hide a register value from the optimiser so a per-element quantity is
// recomputed in each pass instead of being kept live for all EPT elements.
__device__ __forceinline__ float opaque(float v)
{
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(v));
#endif
    return v;
}

// ------------------------------------------------------------------ loads of the row pass
//
// The row pass runs after the chunk pass has completed, so it reads the
// summaries with ordinary (cached, freely batched) loads.
template <class T> __device__ __forceinline__ T ldp(const T *p) { return *p; }
__device__ __forceinline__ Cand ldp_cand(const Cand *p)
{
    const uint64_t v = *reinterpret_cast<const uint64_t *>(p);
    Cand c; c.x = bits_f32((uint32_t)v); c.idx = (int32_t)(uint32_t)(v >> 32);
    return c;
}
// candidates a chunk wrote (its summary says so; never more than the buffer)
__device__ __forceinline__ uint32_t ncand_of(const ChunkSum *cs, int ccap)
{
    const uint32_t n = ldp(&cs->ncand);
    return n < (uint32_t)ccap ? n : (uint32_t)ccap;
}



// raw-key interval for a scaled-key interval, computed by wave 0
template <int DT, class S> __device__ __forceinline__ void x_interval(S &sm, uint32_t klo, uint32_t khi, float T, uint32_t *xlo, uint32_t *xhi)
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

__device__ __forceinline__ void write_row(RowOut *ro, const Args &a, int row, int64_t id, int status, int mode, float m,
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
template <int DT, int NTH = NT, class WF, class SM>
__device__ __forceinline__ int64_t draw_in_chunk(SM &sm, const RowCx &c, int g, double resid, WF &&wfun)
{
    // Thread t takes the contiguous elements [cbeg + t*per, cbeg + (t+1)*per)
    // of the chunk, loaded up front (16-byte vectors where aligned), so the
    // weights are computed from registers in both passes.
    constexpr int VEC = Traits<DT>::VEC, MAXPER = 64 * NT / NTH;  // elements per thread, at most
    const int64_t cbeg = (int64_t)g * c.CH;
    const int64_t cend = cbeg + c.CH < c.V ? cbeg + c.CH : c.V;
    const int per = (int)(c.CH / NTH);  // 8..64, a multiple of VEC
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
    const double before = block_excl_scan<double, NTH / 64>(local, sm.red, &tot);
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
    return block_max<int64_t, NTH / 64>(lastk, sm.red);
}

// Chunk holding u * sum(sm.cw) and the residual weight inside it.
template <class SM>
__device__ __forceinline__ void pick_chunk(SM &sm, int G, float u, int *g_out, double *resid_out, double *S_out)
{
    __syncthreads();
    if (wave_id() == 0) {
        double S = 0.0;
        for (int g = lane_id(); g < G; g += 64) S += sm.cw[g];
        S = wave_sum(S);
        double bef;
        const int gsel = wave_find_asc(sm.cw, G, (double)u * S, &bef);
        if (lane_id() == 0) {
            sm.bd[0] = S;
            // target - sum before the chunk; the rounding fallback keeps it inside
            double r = (double)u * S - bef;
            if (gsel >= 0 && !(r < sm.cw[gsel])) r = sm.cw[gsel];
            sm.bd[1] = r < 0.0 ? 0.0 : r;
            sm.bi[0] = gsel;
        }
    }
    __syncthreads();
    *S_out = sm.bd[0];
    *resid_out = sm.bd[1];
    *g_out = sm.bi[0];
    __syncthreads();
}

// First index (ascending) of an LDS element list at which the running weight
// exceeds `target`: radix over index space, 256 buckets per level.
template <int NTH = NT, class SM>
__device__ __forceinline__ int64_t draw_in_list(SM &sm, const int32_t *idx, const double *e, int n, int64_t V, double target)
{
    int64_t lo = 0, hi = V;
    double acc = 0.0;
    while (hi - lo > 1) {
        const int64_t width = (hi - lo + 255) / 256;
        __syncthreads();
        for (int i = threadIdx.x; i < 256; i += NTH) sm.sub_m[i] = 0.0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += NTH) {
            const int64_t j = idx[i];
            if (j >= lo && j < hi && e[i] > 0.0) atomicAdd(&sm.sub_m[(j - lo) / width], e[i]);
        }
        __syncthreads();
        if (wave_id() == 0) {
            double bef;
            int bsel = wave_find_asc(sm.sub_m, 256, target - acc, &bef);
            if (lane_id() == 0) {
                double tg = target;
                // rounding fallback (the last element with weight): aim past the end
                if (bsel >= 0 && !(acc + bef + sm.sub_m[bsel] > target)) tg = 1e300;
                sm.bi[1] = bsel;
                sm.bd[2] = acc + bef;
                sm.bd[3] = tg;
            }
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
__device__ __forceinline__ uint32_t descend(Smem &sm, const RowCx &c, bool by_mass, double target, uint32_t floor_key,
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
__device__ __forceinline__ int32_t tie_index(Smem &sm, const RowCx &c, uint32_t key, uint32_t t)
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

// The 16-bit top-p chain over runs of equal probabilities, walked by one
// wave (all 64 lanes call it with the same arguments and receive the same
// result), 64 runs at a time.  Element by element in rank order F <- fl32(F
// + p) and the element is removed once chain_E(F, p) >= thr16.  Returns true
// when some element is removed: the first such is element *t_keep (0-based)
// of run *run_at, whose earlier elements are kept.
//
// Inside one binade of F (ulp u), F + p rounds to F + q*u or F + (q+1)*u with
// q = floor(p / u): a run of n equal p adds a fixed number of ulps per step,
// except when p / u - q is exactly 1/2, where the first step rounds to even
// and so depends on the parity of F / u (every later step then starts even).
// A run is therefore a map parity -> (ulps added, parity after); composing
// such maps is associative, so a wave's inclusive scan gives F after each of
// its 64 runs at once, valid up to the first run whose steps would leave the
// binade.  That run takes its in-binade steps in closed form and the
// crossing step as a plain float addition, and the next window starts there
// in the new binade.  E (chain_E) never decreases along the chain, so the cut
// is in the first run whose last element reaches thr16, at the element a
// bisection finds.  run(r, &n, &p) gives the count and probability of run r
// (every lane asks for its own r).  F_io:
// F before the first run (null: 0), and F after the last one when no run
// holds the cut.
template <class RunF>
__device__ __forceinline__ bool chain_cut_wave(int nr, RunF &&run, float thr16, int dt, int *run_at, uint32_t *t_keep,
                                               float *F_io = nullptr)
{
    constexpr int32_t CAP = 1 << 30;  // ulp counts saturate here (any value past a binade: lim <= 2^24)
    const int l = lane_id();
    float F = F_io ? *F_io : 0.0f;
    int r0 = 0;        // current run
    uint32_t i0 = 0u;  // its elements already added
    auto sat = [](int64_t v) { return (int32_t)(v < (int64_t)CAP ? v : (int64_t)CAP); };
    while (r0 < nr) {
        if (F == 0.0f) {
            // 0 + p = p exactly; with p = 0 the whole run leaves F at 0
            uint32_t n;
            float p;
            run(r0, &n, &p);
            if (p == 0.0f) {
                if (chain_E(0.0f, 0.0f, dt) >= thr16) { *run_at = r0; *t_keep = i0; return true; }
                ++r0; i0 = 0u;
                continue;
            }
            F = p;
            if (chain_E(F, p, dt) >= thr16) { *run_at = r0; *t_keep = i0; return true; }
            if (++i0 == n) { ++r0; i0 = 0u; }
            continue;
        }
        {
            // exact window: F and every p here multiples of 2^ez with the
            // window's total below 2^(ez + 24): every partial sum is then a
            // float, each addition exact, and F after each run one integer
            // prefix sum (fp16 probabilities below 1 always qualify, bf16 ones
            // from 2^-17 up)
            const int r = r0 + l;
            uint32_t n = 0u;
            float p = 0.0f;
            if (r < nr) run(r, &n, &p);
            const int64_t m = r < nr ? (int64_t)(r == r0 ? n - i0 : n) : 0;
            auto low_exp = [](float v) {  // exponent of the lowest set bit of v > 0
                const uint32_t b = f32_bits(v), e = (b >> 23) & 0xffu, mt = b & 0x7fffffu;
                const uint32_t mant = e == 0u ? mt : (mt | 0x800000u);
                return (e == 0u ? -149 : (int)e - 150) + (int)__builtin_ctz(mant);
            };
            const int ez = wave_min<int>((m > 0 && p > 0.0f) ? low_exp(p) : low_exp(F));
            const int ef = low_exp(F) < ez ? low_exp(F) : ez;
            const double Pz = (m > 0 && p > 0.0f) ? ldexp((double)p, -ef) : 0.0;  // integer, exact
            const double F0z = ldexp((double)F, -ef);
            if (wave_sum((double)m * Pz) + F0z < 16777216.0) {  // 2^24: exact in double too
                const int64_t inc = (int64_t)m * (int64_t)Pz;
                const int64_t Nend = (int64_t)F0z + wave_incl_scan(inc);
                const bool hit = m > 0 && chain_E(ldexpf((float)Nend, ef), p, dt) >= thr16;
                const uint64_t hb = __ballot(hit);
                if (hb == 0ull) {
                    F = ldexpf((float)__shfl(Nend, 63, 64), ef);
                    if (r0 + 64 >= nr) break;
                    r0 += 64;
                    i0 = 0u;
                    continue;
                }
                // the first run whose last element reaches thr16: bisect its steps
                const int h = __builtin_ctzll(hb);
                const int64_t hm = __shfl(m, h, 64), hN = __shfl(Nend, h, 64), hinc = __shfl(inc, h, 64);
                const float hp = __shfl(p, h, 64);
                const int64_t hP = hm > 0 ? hinc / hm : 0, hb0 = hN - hinc;  // per-step ulps, F before the run
                int64_t lo = 1, hi = hm;
                while (lo < hi) {
                    const int64_t span = hi - lo + 1, stride = (span + 63) / 64;
                    const int64_t cand = lo + (int64_t)l * stride;
                    const bool ok = cand < hi && chain_E(ldexpf((float)(hb0 + cand * hP), ef), hp, dt) >= thr16;
                    const uint64_t b = __ballot(ok);
                    if (b) {
                        const int f = __builtin_ctzll(b);
                        hi = lo + (int64_t)f * stride;
                        lo = f > 0 ? lo + (int64_t)(f - 1) * stride + 1 : lo;
                    } else {
                        const int64_t Lm = (hi - 1 - lo) / stride < 63 ? (hi - 1 - lo) / stride : 63;
                        lo = lo + Lm * stride + 1;
                    }
                }
                *run_at = r0 + h;
                *t_keep = (h == 0 ? i0 : 0u) + (uint32_t)(lo - 1);
                return true;
            }
        }
        // the binade of F: F = N0 * u with u = 2^eu, lim = top / u
        const uint32_t fb = f32_bits(F), fe = (fb >> 23) & 0xffu;
        const int eu = fe == 0u ? -149 : (int)fe - 150;
        const int32_t lim = fe == 0u ? (1 << 23) : (1 << 24);
        const int32_t N0 = fe == 0u ? (int32_t)(fb & 0x7fffffu) : (int32_t)((fb & 0x7fffffu) | 0x800000u);
        const int r = r0 + l;
        uint32_t n = 0u;
        float p = 0.0f;
        if (r < nr) run(r, &n, &p);
        const int64_t m = r < nr ? (int64_t)(r == r0 ? n - i0 : n) : 0;
        const double P = ldexp((double)p, -eu);  // p / u, exact
        const bool big = !(P < (double)CAP);     // the first step leaves the binade
        const int32_t q = big ? CAP : (int32_t)P;
        const double fr = big ? 0.0 : P - (double)q;
        const bool tie = fr == 0.5;
        const int32_t qs = fr > 0.5 ? q + 1 : q;
        const int32_t inc = tie ? q + (q & 1) : qs;  // every step after the first
        auto first_inc = [&](int32_t par) { return tie ? q + ((par + q) & 1) : qs; };
        // this run's ulps added, for F / u even (D0) and odd (D1); the parity
        // after follows from the parity before and the ulps added
        int32_t D0 = 0, D1 = 0;
        if (m > 0) {
            D0 = sat((int64_t)first_inc(0) + (m - 1) * (int64_t)inc);
            D1 = sat((int64_t)first_inc(1) + (m - 1) * (int64_t)inc);
        }
        // inclusive scan: the lanes before first, then this lane's run
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int32_t pD0 = __shfl_up(D0, off, 64), pD1 = __shfl_up(D1, off, 64);
            if (l >= off) {
                const int32_t n0 = sat((int64_t)pD0 + ((pD0 & 1) ? D1 : D0));
                const int32_t n1 = sat((int64_t)pD1 + (((1 + pD1) & 1) ? D1 : D0));
                D0 = n0; D1 = n1;
            }
        }
        const int32_t Nend = sat((int64_t)N0 + ((N0 & 1) ? D1 : D0));
        int32_t Nbef = __shfl_up(Nend, 1, 64);
        if (l == 0) Nbef = N0;
        const int32_t inc1 = first_inc(Nbef & 1);
        // every step stays inside iff its pre-value v has v + q <= lim - 1
        // (the exact sum then lies below the binade's top); the last
        // step's pre-value is the largest
        const int64_t last_pre = m <= 1 ? (int64_t)Nbef : (int64_t)Nend - inc;
        const bool inside = m == 0 || (Nbef < CAP && Nend < CAP && last_pre + q <= (int64_t)lim - 1);
        const bool hit = inside && m > 0 && chain_E(ldexpf((float)Nend, eu), p, dt) >= thr16;
        const uint64_t out = __ballot(!inside), hb = __ballot(hit);
        const int c = out ? __builtin_ctzll(out) : 64, h = hb ? __builtin_ctzll(hb) : 64;
        if (h == 64 && c == 64) {
            F = ldexpf((float)__shfl(Nend, 63, 64), eu);
            if (r0 + 64 >= nr) break;  // the chain never reaches thr16
            r0 += 64;
            i0 = 0u;
            continue;
        }
        // the run that decides this window, broadcast from its lane
        const int w = h < c ? h : c;
        const int64_t wm = __shfl(m, w, 64);
        const int32_t wq = __shfl(q, w, 64), winc = __shfl(inc, w, 64), wnb = __shfl(Nbef, w, 64),
                      winc1 = __shfl(inc1, w, 64);
        const float wp = __shfl(p, w, 64);
        const uint32_t wn = __shfl(n, w, 64);
        const uint32_t kept0 = w == 0 ? i0 : 0u;  // elements of the run added before this window
        // F after s in-binade steps of that run (1 <= s, inside the binade)
        auto F_after = [&](int64_t s) { return ldexpf((float)((int64_t)wnb + winc1 + (s - 1) * winc), eu); };
        // first step in [1, hi] whose E reaches thr16 (E(hi) does): 64-way
        // steps over the lanes
        auto first_hit = [&](int64_t hi) {
            int64_t lo = 1;
            while (lo < hi) {
                const int64_t span = hi - lo + 1, stride = (span + 63) / 64;
                const int64_t cand = lo + (int64_t)l * stride;
                const bool ok = cand < hi && chain_E(F_after(cand), wp, dt) >= thr16;
                const uint64_t b = __ballot(ok);
                if (b) {  // between the last failing candidate and the first passing one
                    const int f = __builtin_ctzll(b);
                    hi = lo + (int64_t)f * stride;
                    lo = f > 0 ? lo + (int64_t)(f - 1) * stride + 1 : lo;
                } else {  // past the last candidate tested (the largest below hi)
                    const int64_t L = (hi - 1 - lo) / stride < 63 ? (hi - 1 - lo) / stride : 63;
                    lo = lo + L * stride + 1;
                }
            }
            return lo;
        };
        if (h < c) {
            *run_at = r0 + w;
            *t_keep = kept0 + (uint32_t)(first_hit(wm) - 1);
            return true;
        }
        // the crossing run: s steps inside, then one plain addition
        const int64_t R = (int64_t)lim - 1 - wq;
        int64_t s = 0;
        if (wnb <= R) {
            s = 1;
            const int64_t N1 = (int64_t)wnb + winc1;
            if (wm > 1 && N1 <= R) s = winc > 0 ? 2 + (R - N1) / winc : wm;
            if (s > wm) s = wm;
        }
        float Fs = ldexpf((float)wnb, eu);
        if (s > 0) {
            Fs = F_after(s);
            if (chain_E(Fs, wp, dt) >= thr16) {
                *run_at = r0 + w;
                *t_keep = kept0 + (uint32_t)(first_hit(s) - 1);
                return true;
            }
        }
        F = Fs + wp;
        if (chain_E(F, wp, dt) >= thr16) {
            *run_at = r0 + w;
            *t_keep = kept0 + (uint32_t)s;
            return true;
        }
        r0 += w;
        i0 = kept0 + (uint32_t)s + 1u;
        if (i0 == wn) { ++r0; i0 = 0u; }
    }
    if (F_io) *F_io = F;
    return false;
}

// Top-p cut over elements with key >= floor_key; sm.v.l1 holds their 256-bin
// histogram and S their total weight.
template <int DT>
__device__ __forceinline__ void topp_cut_generic(Smem &sm, const RowCx &c, float top_p, uint32_t floor_key, double S,
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
    double walked = 0.0;  // mass of the L1 bins above b_hi
    while (b_hi >= 0) {
        // a region of L1 bins whose mass (float64) reaches past top_p with a
        // margin for the chain's rounding, at most REGION_MAX bins: one re-read
        // usually holds the cut; if not, the next region follows
        int b_lo = b_hi;
        double reach = walked + sm.v.l1.mass[b_hi];
        while (b_lo > 0 && b_hi - b_lo + 1 < REGION_MAX && reach < ((double)top_p + 0.02) * S) {
            --b_lo;
            reach += sm.v.l1.mass[b_lo];
        }
        const int npos = (b_hi - b_lo + 1) * 256;
        __syncthreads();
        for (int i = threadIdx.x; i < npos; i += NT) sm.w.r.cnt[i] = 0u;
        uint32_t klo = (uint32_t)b_lo << 24;
        const uint32_t khi = ((uint32_t)b_hi << 24) | 0x00ffffffu;
        if (klo < floor_key) klo = floor_key;
        if (klo <= kneg) klo = kneg + 1u;
        uint32_t xlo, xhi;
        x_interval<DT>(sm, klo, khi, c.T, &xlo, &xhi);
        rescan<DT>(c, xlo, xhi, [&](int64_t, float, uint32_t key) {
            if (key < klo || key > khi) return;
            const uint32_t pos = (uint32_t)(b_hi - (int)(key >> 24)) * 256u + (255u - ((key >> 16) & 255u));
            atomicAdd(&sm.w.r.cnt[pos], 1u);
        });
        __syncthreads();
        int nruns_total = 0;
        for (int i0 = 0; i0 < npos; i0 += NT) {
            const int i = i0 + threadIdx.x;
            const uint32_t cnt = i < npos ? sm.w.r.cnt[i] : 0u;
            uint32_t tot;
            const uint32_t off = block_excl_scan<uint32_t>(cnt ? 1u : 0u, sm.red, &tot);
            if (cnt) {
                const uint32_t L1 = (uint32_t)(b_hi - i / 256), b2 = 255u - (uint32_t)(i % 256);
                const uint32_t key = (L1 << 24) | (b2 << 16);
                const int r = nruns_total + (int)off;
                sm.w.r.rkey[r] = key;
                sm.w.r.rcnt[r] = cnt;
                sm.w.r.rp[r] = rn_dtype((float)(exp((double)value_of_row_key(key, DT) - md) / S), DT);
            }
            nruns_total += (int)tot;
        }
        __syncthreads();
        if (wave_id() == 0) {
            int run_at = -1;
            uint32_t tk = 0;
            float Fw = F;
            auto run = [&](int q, uint32_t *n, float *p) { *n = sm.w.r.rcnt[q]; *p = sm.w.r.rp[q]; };
            const bool found = chain_cut_wave(nruns_total, run, thr16, DT, &run_at, &tk, &Fw);
            if (lane_id() == 0) {
                sm.bi[1] = found ? 1 : 0;
                sm.bu[0] = tk;
                sm.bf[0] = Fw;
                sm.bu[1] = nruns_total > 0 ? sm.w.r.rkey[nruns_total - 1] : 0u;
                if (found) {
                    sm.bu[2] = sm.w.r.rkey[run_at];
                    sm.bu[3] = sm.w.r.rcnt[run_at];
                    sm.bu[4] = run_at > 0 ? sm.w.r.rkey[run_at - 1] : 0u;
                    sm.bi[3] = run_at > 0 ? 1 : 0;
                }
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
        for (int b = b_lo; b <= b_hi; ++b) walked += sm.v.l1.mass[b];
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
__device__ __forceinline__ void final_generic(Smem &sm, const RowCx &c, const RowPlan &pl, RowOut *ro, const Args &a)
{
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

// The window's cut.  Input: n <= SURV_CAP elements in sm.u.s (key, idx, e),
// `above` = mass of everything ranked before the window, A = the target
// (an element is kept iff the mass before it is < A).  The window is sorted
// into the stable descending order in sm.u.so (composite key
// key << 32 | ~idx, mass); the last kept element is found by a block scan.
// Returns its sorted position, or -1 when the cut is not inside the window.
// *q_last = mass before the last kept element, *w_last = its weight.
template <int NTH = NT, class SM>
__device__ __forceinline__ int window_resolve(SM &sm, uint32_t n, double above, double A, uint32_t *cut_key, int32_t *cut_i,
                              double *q_last, double *w_last)
{
    constexpr int PT = SURV_CAP / NTH;
    const int tid = threadIdx.x;
    uint64_t kt[PT];
    double et[PT];
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        const int i = q * NTH + tid;
        const bool in = i < (int)n;
        kt[q] = in ? (((uint64_t)sm.u.s.key[i] << 32) | (uint64_t)(0xffffffffu - (uint32_t)sm.u.s.idx[i])) : 0ull;
        et[q] = in ? sm.u.s.e[i] : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PT; ++q) { sm.u.so.k[q * NTH + tid] = kt[q]; sm.u.so.e[q * NTH + tid] = et[q]; }
    __syncthreads();
    block_sort_desc<NTH, SURV_CAP>(sm.u.so.k, sm.u.so.e, (int)n);
    // thread t scans the sorted positions [t*PT, t*PT + PT)
    double local = 0.0;
#pragma unroll
    for (int q = 0; q < PT; ++q) { const int r = tid * PT + q; local += r < (int)n ? sm.u.so.e[r] : 0.0; }
    double tot;
    const double off = block_excl_scan<double, NTH / 64>(local, sm.red, &tot);
    if (tid == 0) { sm.bi[4] = -1; }
    __syncthreads();
    double run = above + off;
    int cand = -1;
    double qc = 0.0;
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        const int r = tid * PT + q;
        if (r < (int)n) {
            if (run < A) { cand = r; qc = run; }
            run += sm.u.so.e[r];
        }
    }
    {
        const int wc = wave_max(cand);  // one LDS atomic per wave
        if (lane_id() == 0) atomicMax(&sm.bi[4], wc);
    }
    __syncthreads();
    const int rl = sm.bi[4];
    if (rl >= 0 && cand == rl) sm.bd[5] = qc;
    __syncthreads();
    if (rl < 0) return -1;                                     // the first window element is removed
    if (rl == (int)n - 1 && !(above + tot >= A)) return -1;    // every window element is kept
    const uint64_t ck = sm.u.so.k[rl];
    *cut_key = (uint32_t)(ck >> 32);
    *cut_i = (int32_t)(0xffffffffu - (uint32_t)ck);
    *q_last = sm.bd[5];
    *w_last = sm.u.so.e[rl];
    return rl;
}

// ------------------------------------------------------------------ small top-k leader

// Exact k'-th value over the per-chunk candidates, survivors, optional top-p,
// draw.  Returns false (the caller then re-reads the row) when a chunk
// overflowed its candidate buffer, when a truncated chunk may hide an element
// at or above the k'-th value, or when the survivors overflow LDS.
template <int DT>
// S_row >= 0: an fp16/bf16 top-p row probing its cut among its kk = K_PROBE
// largest values: the chain's probabilities divide by the row's S_row, and a
// cut not reached among them returns false (the generic path takes the row).
// S_tol > 0: S_row's relative error bound; when a run at or above the cut has
// a rounded probability that some S within it would round differently, the
// call sets *ambig and returns false without output (the caller retries with
// an exact S).
__device__ __forceinline__ bool leader_smallk(Smem &sm, const RowCx &c, const RowPlan &pl, const ChunkSum *cs,
                                          const Cand *cand, RowOut *ro, const Args &a, double S_row = -1.0,
                                          double S_tol = 0.0, bool *ambig = nullptr)
{
    const bool probe = S_row >= 0.0;
    const double md = (double)c.m;
    // candidate counts -> prefix offsets (thread 0, G <= 256); candidate f of
    // the row is candidate f - pre[g] of the chunk g with pre[g] <= f < pre[g+1]
    uint32_t *pre = reinterpret_cast<uint32_t *>(sm.chs);
    {
        static_assert(G_MAX <= NT, "one chunk per thread");
        const uint32_t nc = (int)threadIdx.x < c.G ? ncand_of(&cs[threadIdx.x], a.L.ccap) : 0u;
        uint32_t tot;
        const uint32_t off = block_excl_scan<uint32_t>(nc, sm.red, &tot);
        if ((int)threadIdx.x < c.G) pre[threadIdx.x] = off;
        if (threadIdx.x == 0) pre[c.G] = tot;
        __syncthreads();
    }
    const uint32_t ntot = pre[c.G];
    const int G = c.G;
    // chunk facts: overflow, truncation, finite counts
    uint32_t ovf = 0, ntr = 0, nfin = 0;
    for (int g = threadIdx.x; g < G; g += NT) {
        ovf |= ldp(&cs[g].ncand) == NCAND_OVERFLOW ? 1u : 0u;
        ntr |= ldp(&cs[g].trunc) != 0u ? 1u : 0u;
        nfin += ldp(&cs[g].nfin);
    }
    ovf = block_sum<uint32_t>(ovf, sm.red);
    ntr = block_sum<uint32_t>(ntr, sm.red);
    nfin = block_sum<uint32_t>(nfin, sm.red);
    trace(a.ws, a.L, c.row, 17);
    if (ovf != 0u) return false;
    // fewer finite elements than k': the k'-th value is -inf and every finite
    // element survives, which the candidates hold only if no chunk truncated
    const bool all_fin = nfin <= (uint32_t)pl.kk;
    if ((all_fin && ntr != 0u) || (!all_fin && ntot < (uint32_t)pl.kk)) return false;
    auto cand_ptr = [&](uint32_t f) -> const Cand * {
        int lo = 0, hi = G - 1;  // last g with pre[g] <= f
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pre[mid] <= f) lo = mid; else hi = mid - 1;
        }
        return cand + (size_t)lo * a.L.ccap + (f - pre[lo]);
    };
    constexpr int BATCH = 8;  // candidate loads in flight per thread
    // the row's candidates, copied once into LDS when they fit
    const bool cached = ntot <= (uint32_t)CCAP_FIN;
    if (cached) {
        for (uint32_t f0 = 0; f0 < ntot; f0 += NT * BATCH) {
            const Cand *cp[BATCH];
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                cp[u] = cand_ptr(f < ntot ? f : 0u);
            }
            Cand cv[BATCH];
#pragma unroll
            for (int u = 0; u < BATCH; ++u) cv[u] = ldp_cand(cp[u]);
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                if (f < ntot) sm.w.cc[f] = cv[u];
            }
        }
        __syncthreads();
    }
    trace(a.ws, a.L, c.row, 21);
    // k'-th largest raw value over the candidates: linear bins between the
    // smallest and largest candidate (values that differ spread over the bins,
    // so the LDS counters see few conflicts), then the boundary bin's
    // candidates sorted.  Fewer candidates than k' means fewer finite
    // elements than k' in the row.
    uint32_t xk_thr = 0u;
    if (!all_fin) {
        auto for_cands = [&](auto &&fn) {
            for (uint32_t f0 = 0; f0 < ntot; f0 += NT * BATCH) {
                float xv[BATCH];
                if (cached) {
#pragma unroll
                    for (int u = 0; u < BATCH; ++u) {
                        const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                        xv[u] = sm.w.cc[f < ntot ? f : 0u].x;
                    }
                } else {
                    const Cand *cp[BATCH];
#pragma unroll
                    for (int u = 0; u < BATCH; ++u) {
                        const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                        cp[u] = cand_ptr(f < ntot ? f : 0u);
                    }
#pragma unroll
                    for (int u = 0; u < BATCH; ++u) xv[u] = ldp_cand(cp[u]).x;
                }
#pragma unroll
                for (int u = 0; u < BATCH; ++u)
                    if (f0 + (uint32_t)(u * NT) + threadIdx.x < ntot) fn(xv[u]);
            }
        };
        float cmin = INFINITY, cmax = -INFINITY;
        for_cands([&](float x) { cmin = fminf(cmin, x); cmax = fmaxf(cmax, x); });
        cmin = block_min<float>(cmin, sm.red);
        cmax = block_max<float>(cmax, sm.red);
        trace(a.ws, a.L, c.row, 22);
        if (!(cmax > cmin)) {
            xk_thr = key_of_f32(cmax);  // every candidate holds the same value
        } else {
            const float inv = 2048.0f / (cmax - cmin);
            auto bin_of = [&](float x) -> int { return min(2047, (int)((x - cmin) * inv)); };
            for (int i = threadIdx.x; i < 2048; i += NT) sm.u.h11.cnt[i] = 0u;
            __syncthreads();
            for_cands([&](float x) { atomicAdd(&sm.u.h11.cnt[bin_of(x)], 1u); });
            __syncthreads();
            if (wave_id() == 0) {
                uint32_t above;
                const int d = wave_find_desc<uint32_t>(sm.u.h11.cnt, 2048, (uint32_t)pl.kk, &above);
                if (lane_id() == 0) { sm.bu[0] = (uint32_t)d; sm.bu[1] = above; sm.bu[2] = sm.u.h11.cnt[d]; }
            }
            __syncthreads();
            const int bsel = (int)sm.bu[0];
            const uint32_t above = sm.bu[1], nbin = sm.bu[2];
            trace(a.ws, a.L, c.row, 23);
            if (nbin > (uint32_t)SURV_CAP || (uint32_t)pl.kk <= above) return false;
            __syncthreads();
            if (threadIdx.x == 0) sm.bu[3] = 0u;
            __syncthreads();
            for_cands([&](float x) {
                const bool in = bin_of(x) == bsel;
                const uint32_t q = wave_append(in, &sm.bu[3]);
                if (in && q < (uint32_t)SURV_CAP) { sm.u.so.k[q] = key_of_f32(x); sm.u.so.e[q] = 0.0; }
            });
            __syncthreads();
            const int nb = (int)min(sm.bu[3], (uint32_t)SURV_CAP);
            __syncthreads();
            trace(a.ws, a.L, c.row, 24);
            block_sort_desc<NT, SURV_CAP>(sm.u.so.k, sm.u.so.e, nb);
            xk_thr = (uint32_t)sm.u.so.k[(int)((uint32_t)pl.kk - above) - 1];
            __syncthreads();
        }
    }
    // survivors: scaled value >= scale(k'-th raw value); the ties the scaling
    // creates are kept, as the reference keeps them
    const uint32_t thr_key = xk_thr ? row_key(scale_y<DT>(f32_of_key(xk_thr), c.T), DT) : 0u;
    trace(a.ws, a.L, c.row, 18);
    // exactness: a truncated chunk left out only elements with scaled keys
    // below its kc; they cannot reach the threshold if kc <= thr_key
    if (ntr != 0u) {
        uint32_t hide = 0;
        for (int g = threadIdx.x; g < G; g += NT)
            hide |= (ldp(&cs[g].trunc) != 0u && ldp(&cs[g].kc) > thr_key) ? 1u : 0u;
        hide = block_sum<uint32_t>(hide, sm.red);
        if (hide != 0u) return false;
    }
    if (threadIdx.x == 0) sm.bu[3] = 0u;
    __syncthreads();
    for (uint32_t f0 = 0; f0 < ntot; f0 += NT * BATCH) {
        Cand cv[BATCH];
        if (cached) {
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                cv[u] = sm.w.cc[f < ntot ? f : 0u];
            }
        } else {
            const Cand *cp[BATCH];
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
                cp[u] = cand_ptr(f < ntot ? f : 0u);
            }
#pragma unroll
            for (int u = 0; u < BATCH; ++u) cv[u] = ldp_cand(cp[u]);
        }
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const uint32_t f = f0 + (uint32_t)(u * NT) + threadIdx.x;
            const float y = scale_y<DT>(cv[u].x, c.T);
            const uint32_t k = row_key(y, DT);
            const bool in = f < ntot && k >= thr_key;
            const uint32_t p = wave_append(in, &sm.bu[3]);
            if (in && p < (uint32_t)SURV_CAP) { sm.u.s.key[p] = k; sm.u.s.idx[p] = cv[u].idx; sm.u.s.e[p] = exp((double)y - md); }
        }
    }
    __syncthreads();
    const uint32_t ns = sm.bu[3];
    __syncthreads();
    trace(a.ws, a.L, c.row, 19);
    if (ns > (uint32_t)SURV_CAP || ns == 0) return false;

    uint32_t cut_key = thr_key;
    int32_t cut_i = IDX_ALL;
    int status = MIS_ROW_OK;
    if (pl.topp) {
        double S = 0.0;
        for (uint32_t i = threadIdx.x; i < ns; i += NT) S += sm.u.s.e[i];
        S = block_sum<double>(S, sm.red);
        if (probe) S = S_row;
        if (DT == F32) {
            // exact masses over the survivors: sorted cut, then back to the
            // (key, idx, e) view the draw reads
            double ql, wl;
            const int rl = window_resolve(sm, ns, 0.0, (double)pl.top_p * S, &cut_key, &cut_i, &ql, &wl);
            if (rl < 0) {  // every survivor kept (A at or beyond the total)
                cut_key = thr_key;
                cut_i = IDX_ALL;
            }
            constexpr int PT = SURV_CAP / NT;
            uint64_t kt[PT];
            double et[PT];
            for (int q = 0; q < PT; ++q) { kt[q] = sm.u.so.k[threadIdx.x + q * NT]; et[q] = sm.u.so.e[threadIdx.x + q * NT]; }
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
        } else {
            // 16-bit rounding chain over the survivors in stable descending order
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
            block_sort_desc<NT, SURV_CAP>(sm.u.so.k, sm.u.so.e, (int)ns);
            // runs of equal keys in sorted order, their probabilities and
            // lengths, computed in parallel (the candidates' cache is free
            // again); then one thread walks the chain over the runs
            uint32_t amb = 0xffffffffu;  // first run whose rounding S's error bound leaves open
            {
                uint32_t st[PT];
#pragma unroll
                for (int q = 0; q < PT; ++q) {
                    const int i = threadIdx.x * PT + q;
                    st[q] = i < (int)ns && (i == 0 || (uint32_t)(sm.u.so.k[i] >> 32) != (uint32_t)(sm.u.so.k[i - 1] >> 32)) ? 1u : 0u;
                }
                uint32_t nr;
                uint32_t r = block_excl_scan<uint32_t>(st[0] + st[1] + st[2] + st[3], sm.red, &nr);
#pragma unroll
                for (int q = 0; q < PT; ++q) {
                    const int i = threadIdx.x * PT + q;
                    if (st[q]) {
                        sm.w.r.rkey[r] = (uint32_t)i;  // the run's first sorted position
                        const double e = sm.u.so.e[i];
                        const float pr = rn_dtype((float)(e / S), DT);
                        sm.w.r.rp[r] = pr;
                        // every rounding step is monotone: equal roundings at
                        // both ends of the interval fix the value inside it
                        if (S_tol > 0.0 && (rn_dtype((float)(e / (S * (1.0 + S_tol))), DT) != pr ||
                                            rn_dtype((float)(e / (S * (1.0 - S_tol))), DT) != pr))
                            amb = r < amb ? r : amb;
                        ++r;
                    }
                }
                if (S_tol > 0.0) amb = block_min<uint32_t>(amb, sm.red);  // its barriers order the runs
                else __syncthreads();
                for (uint32_t q = threadIdx.x; q < nr; q += NT)
                    sm.w.r.rcnt[q] = (q + 1 < nr ? sm.w.r.rkey[q + 1] : ns) - sm.w.r.rkey[q];
                if (threadIdx.x == 0) sm.bu[2] = nr;
                __syncthreads();
            }
            static_assert(PT == 4, "four survivors per thread");
            if (wave_id() == 0) {
                const float thr16 = rn_dtype(pl.top_p, DT);
                uint32_t r0 = ns;
                int run_at = -1;
                uint32_t tk = 0;
                auto run = [&](int q, uint32_t *n, float *p) { *n = sm.w.r.rcnt[q]; *p = sm.w.r.rp[q]; };
                const bool found = chain_cut_wave((int)sm.bu[2], run, thr16, DT, &run_at, &tk);
                if (found) r0 = sm.w.r.rkey[run_at] + tk;
                if (lane_id() == 0) {
                    sm.bu[0] = r0;
                    sm.bi[1] = found ? 1 : 0;
                    sm.bi[2] = (found && amb <= (uint32_t)run_at) ? 1 : 0;
                    if (r0 > 0) {
                        const uint64_t q = sm.u.so.k[r0 - 1];
                        sm.bu[1] = (uint32_t)(q >> 32);
                        sm.bi[0] = (int32_t)(0xffffffffu - (uint32_t)q);
                    }
                }
            }
            __syncthreads();
            const uint32_t r0 = sm.bu[0];
            const bool found = sm.bi[1] != 0;
            const bool open = sm.bi[2] != 0;
            if (r0 > 0) { cut_key = sm.bu[1]; cut_i = sm.bi[0]; }
            __syncthreads();
            if (open) {  // a rounding above the cut depends on S beyond S_row's accuracy
                if (ambig) *ambig = true;  // every thread's own flag (the branch is block-uniform)
                return false;
            }
            if (probe && !found) return false;  // the cut lies below the K_PROBE largest
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
    trace(a.ws, a.L, c.row, 20);
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


// Smallest key in [lo, hi] where the monotone predicate (false ... true) holds,
// hi + 1 when it holds nowhere.  Run by one whole wave (64-ary search).
template <class P> __device__ __forceinline__ uint32_t key_search(uint32_t lo, uint32_t hi, P &&pred)
{
    if (lo > hi) return hi + 1u;
    if (pred(lo)) return lo;
    if (!pred(hi)) return hi + 1u;
    uint64_t a = lo, b = hi;  // pred(a) false, pred(b) true
    while (b - a > 1) {
        uint64_t step = (b - a) / 64;
        if (step == 0) step = 1;
        const uint64_t p = a + (uint64_t)(lane_id() + 1) * step;
        const bool t = p >= b ? true : pred((uint32_t)p);
        const uint64_t mk = __ballot(t);
        if (mk == 0ull) { a = a + 64 * step; continue; }
        const int f = __builtin_ctzll(mk);
        const uint64_t nb = a + (uint64_t)(f + 1) * step;
        if (nb < b) b = nb;
        a = a + (uint64_t)f * step;
    }
    return (uint32_t)b;
}

// ------------------------------------------------------------------ row leaders

// Leader of a row that needs no refinement rounds: greedy, temperature only,
// small top-k, and the re-read path for everything else.
template <int DT>
__device__ __forceinline__ void leader_row(Smem &sm, RowCx &c, const RowPlan &pl, const ChunkSum *csr, RowOut *ro,
                                        const Args &a)
{
    const int tid = threadIdx.x, row = c.row;
    const Layout &L = a.L;
    if (pl.mode == M_BAD || pl.mode == M_INVAL) {
        write_row(ro, a, row, -1, pl.mode == M_BAD ? MIS_ROW_BAD_PARAM : MIS_ROW_INVALID, pl.mode, 0.0f, 0u, 0, 0.0);
        return;
    }
    uint32_t k2 = 0u;
    int32_t i2 = IDX_ALL;
    uint32_t anyflag = 0u;
    float m = -INFINITY;
    for (int g = tid; g < L.G; g += NT) {
        const uint32_t xk = ldp(&csr[g].xkey);
        const int32_t xa = ldp(&csr[g].xarg);
        if (xk > k2 || (xk == k2 && xa < i2)) { k2 = xk; i2 = xa; }
        anyflag |= ldp(&csr[g].flags);
        m = fmaxf(m, ldp(&csr[g].ymax));
    }
    if (pl.mode == M_GREEDY) {
        wave_argmax(k2, i2);
        if (lane_id() == 0) { sm.red.u[wave_id()] = k2; sm.red.l[wave_id()] = i2; }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < NWAVE; ++w) {
                const uint32_t kk = sm.red.u[w];
                const int32_t ii = (int32_t)sm.red.l[w];
                if (kk > k2 || (kk == k2 && ii < i2)) { k2 = kk; i2 = ii; }
            }
            write_row(ro, a, row, i2, MIS_ROW_OK, pl.mode, 0.0f, 0u, i2, 1.0);
        }
        return;
    }
    anyflag = block_sum<uint32_t>(anyflag ? 1u : 0u, sm.red);
    m = block_max<float>(m, sm.red);
    c.m = m;
    const double md = (double)m;
    if (anyflag != 0u || m == -INFINITY) {
        write_row(ro, a, row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
    } else if (pl.mode == M_TEMP) {
        // chunk weights are exp(y - ymax_c): rescale to the row max m
        for (int g = tid; g < L.G; g += NT) {
            const float yg = ldp(&csr[g].ymax);
            sm.chs[g] = yg == -INFINITY ? 0.0 : exp((double)yg - md);
            sm.cw[g] = ldp(&csr[g].S) * sm.chs[g];
        }
        int gsel;
        double resid, SK;
        pick_chunk(sm, L.G, pl.u, &gsel, &resid, &SK);
        int64_t id = -1;
        if (gsel >= 0) {
            // the chunk pass's weights, recomputed the same way
            const float yc = ldp(&csr[gsel].ymax), T = pl.T;
            id = draw_in_chunk<DT>(sm, c, gsel, resid / sm.chs[gsel], [&](float xv, int64_t) -> double {
                return (double)wexp(scale_y<DT>(xv, T), yc);
            });
        }
        write_row(ro, a, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, row_key(-INFINITY, DT), -1, SK);
    } else if (pl.mode == M_SMALLK) {
        final_generic<DT>(sm, c, pl, ro, a);  // the rows k_rowpass deferred (or no row pass ran)
    } else if (DT != F32 && pl.mode == M_TOPP && !L.t16) {
        // the cut among the row's K_PROBE largest values first
        double s = 0.0;
        for (int g = tid; g < L.G; g += NT) {
            const float yg = ldp(&csr[g].ymax);
            s += yg == -INFINITY ? 0.0 : ldp(&csr[g].S) * exp((double)yg - md);
        }
        const double S_row = block_sum<double>(s, sm.red);
        RowPlan pk = pl;
        pk.kk = (int)(c.V < (int64_t)K_PROBE ? c.V : (int64_t)K_PROBE);
        const Cand *cand = reinterpret_cast<const Cand *>(a.ws + L.cand) + (size_t)row * L.G * L.ccap;
        // S_row sums wexp weights (relative error <= WEXP_REL_ERR each, all
        // positive) in float64; twice that bound covers the float64 sums and
        // the chunk rescales
        bool ambig = false;
        if (!leader_smallk<DT>(sm, c, pk, csr, cand, ro, a, S_row, 2.0 * WEXP_REL_ERR, &ambig)) {
            bool done = false;
            if (ambig) {
                // exact S from a re-read of the row (dexp, relative error
                // below 1e-15), then the probe again
                exp_table(sm.etab, tid);
                __syncthreads();
                double se = 0.0;
                rescan<DT>(c, 0x007fffffu, 0xff800000u, [&](int64_t, float y, uint32_t) {
                    if (y != -INFINITY) se += dexp((double)y - md, sm.etab);
                });
                const double S_ex = block_sum<double>(se, sm.red);
                done = leader_smallk<DT>(sm, c, pk, csr, cand, ro, a, S_ex);
            }
            if (!done) final_generic<DT>(sm, c, pl, ro, a);
        }
    } else {
        final_generic<DT>(sm, c, pl, ro, a);
    }
}

// Per-chunk scale factors exp(ymax_c - m) into sm.chs; returns the row max m
// and whether any chunk flagged NaN / +inf.  One load pair per chunk and
// thread, issued together.
template <int NTH = NT, class SM>
__device__ __forceinline__ float row_scales(SM &sm, const ChunkSum *csr, int G, uint32_t *bad)
{
    uint32_t anyflag = 0u;
    float m = -INFINITY;
    for (int g = threadIdx.x; g < G; g += NTH) {
        const uint32_t f = ldp(&csr[g].flags);
        const float yg = ldp(&csr[g].ymax);
        anyflag |= f;
        m = fmaxf(m, yg);
        sm.chs[g] = (double)yg;
    }
    anyflag = block_sum<uint32_t, NTH / 64>(anyflag ? 1u : 0u, sm.red);
    m = block_max<float, NTH / 64>(m, sm.red);
    const double md = (double)m;
    for (int g = threadIdx.x; g < G; g += NTH) {
        const double yg = sm.chs[g];
        sm.chs[g] = (yg == -INFINITY || m == -INFINITY) ? 0.0 : exp(yg - md);
    }
    __syncthreads();
    *bad = anyflag;
    return m;
}

__device__ __forceinline__ float coarse_bin(float y) { return floorf(y * CB_SCALE); }

// One coalesced read of a chunk into registers (16-byte vectors where the row
// allows); -inf past the end of the row.
template <int DT, int EPT>
__device__ __forceinline__ void load_chunk(const char *rowp, int64_t base, int64_t V, int vec_ok, float (&x)[EPT])
{
    constexpr int VEC = Traits<DT>::VEC, NV = EPT / VEC, CH = NT * EPT;
    const int tid = threadIdx.x;
    if (vec_ok && base + CH <= V) {
#pragma unroll
        for (int v = 0; v < NV; ++v) loadvec<DT>(rowp, base + ((int64_t)v * NT + tid) * VEC, &x[v * VEC]);
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int64_t j0 = base + ((int64_t)v * NT + tid) * VEC;
            if (vec_ok && j0 + VEC <= V) {
                loadvec<DT>(rowp, j0, &x[v * VEC]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) x[v * VEC + e] = (j0 + e < V) ? load1<DT>(rowp, j0 + e) : -INFINITY;
            }
        }
    }
}

// load_chunk for a block of NTH threads holding EPT elements each (the chunk
// is NTH * EPT elements: the chunk pass's own chunk when NTH * EPT = NT *
// its EPT).  Element i of thread t is base + ((i / VEC) * NTH + t) * VEC + i % VEC.
template <int DT, int EPT, int NTH>
__device__ __forceinline__ void load_chunk_n(const char *rowp, int64_t base, int64_t V, int vec_ok, float (&x)[EPT])
{
    constexpr int VEC = Traits<DT>::VEC, NV = EPT / VEC, CH = NTH * EPT;
    static_assert(EPT % VEC == 0, "whole vectors per thread");
    const int tid = threadIdx.x;
    if (vec_ok && base + CH <= V) {
#pragma unroll
        for (int v = 0; v < NV; ++v) loadvec<DT>(rowp, base + ((int64_t)v * NTH + tid) * VEC, &x[v * VEC]);
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int64_t j0 = base + ((int64_t)v * NTH + tid) * VEC;
            if (vec_ok && j0 + VEC <= V) {
                loadvec<DT>(rowp, j0, &x[v * VEC]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) x[v * VEC + e] = (j0 + e < V) ? load1<DT>(rowp, j0 + e) : -INFINITY;
            }
        }
    }
}

// ------------------------------------------------------------------ the kernel

// ascending bitonic sort of one value per lane across a wave
__device__ __forceinline__ uint32_t wave_sort_asc(uint32_t v)
{
    const int l = lane_id();
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint32_t o = (uint32_t)__shfl_xor((int)v, j, 64);
            const bool up = (l & k) == 0, lower = (l & j) == 0;
            v = (up == lower) ? (o < v ? o : v) : (o > v ? o : v);
        }
    }
    return v;
}

// The chunk pass: one workgroup per (row, chunk).  Loads the chunk into
// registers and reduces it for the row's mode to the summary the row pass
// reads.  fp32 top-p rows also bin their mass coarsely for the row pass.
// k_sample's rows: all, only the fp32 top-p rows, or all but those (the two
// halves run on two streams so the top-p passes start after their own rows)
enum : int { K1_ALL = 0, K1_TOPP32 = 1, K1_OTHERS = 2 };

template <int DT, int EPT>
__global__ __launch_bounds__(NT) void k_sample(Args a, int part)
{
    constexpr int VEC = Traits<DT>::VEC, CH = NT * EPT;
    __shared__ ChunkSmem sm;
    const Layout &L = a.L;
    const int tid = threadIdx.x;
    const int G = L.G;
    const uint32_t task = blockIdx.x;  // a row's chunks have consecutive indices
    const int chunk = (int)(task % (uint32_t)G);
    const int row = (int)(task / (uint32_t)G);
    const int64_t V = a.V;
    const int64_t base = (int64_t)chunk * CH;
    const char *rowp = a.logits + (int64_t)row * a.stride_bytes;
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, V);
    // the split halves: each launch covers every (row, chunk) and keeps its
    // own rows (the fp32 top-p rows, or the others)
    if (part != K1_ALL && (part == K1_TOPP32) != (DT == F32 && pl.mode == M_TOPP)) return;
    ChunkSum *csr = reinterpret_cast<ChunkSum *>(a.ws + L.chunks) + (size_t)row * G;
    ChunkSum *cs = csr + chunk;
    RoundBuf *rb = reinterpret_cast<RoundBuf *>(a.ws + L.rbuf) + (size_t)row * G + chunk;

    if (chunk == 0) trace(a.ws, L, row, 0);
    float x[EPT];
    load_chunk<DT, EPT>(rowp, base, V, a.vec_ok, x);
    const int32_t base32 = (int32_t)base;  // V < 2^31
    auto idx_of = [&](int i) -> int32_t { return base32 + (int32_t)((((i / VEC) * NT + tid) * VEC) + (i % VEC)); };
    if (DT != F32 && pl.mode == M_TOPP && L.t16) {
        // this chunk's share of the row's key histogram, which k_t16_hist adds into
        uint32_t *rh = reinterpret_cast<uint32_t *>(a.ws + L.t16h) + (size_t)row * NB16;
        for (int b = chunk + G * tid; b < NB16; b += G * NT) rh[b] = 0u;
    }

    const bool topp32 = DT == F32 && pl.mode == M_TOPP;
    float ymax = -INFINITY;
    if (pl.mode == M_GREEDY) {
        // ---- argmax of the raw logits (NaN ranks first, ties -> lowest index)
        uint32_t bk = 0u;
        int32_t bi = IDX_ALL;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const uint32_t k = argmax_key(x[i]);
            if (k > bk) { bk = k; bi = idx_of(i); }
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
            cs->xkey = bk; cs->xarg = bi;
        }
    } else if (pl.mode != M_BAD && pl.mode != M_INVAL) {
        // ---- chunk max and flags
        float tmax = -INFINITY;
        uint32_t nan = 0u, nf = 0u;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            tmax = fmaxf(tmax, x[i]);
            nan |= x[i] != x[i] ? 1u : 0u;
        }
        // fp16/bf16 top-p rows of a large batch first try their cut among the
        // row's K_PROBE largest values: the chunk pass also emits those
        // candidates (a small batch's rows take the t16 passes instead)
        const bool topp16 = DT != F32 && pl.mode == M_TOPP && !L.t16;
        if (pl.mode == M_SMALLK || topp16) {  // the finite count only candidate rows use
#pragma unroll
            for (int i = 0; i < EPT; ++i) nf += x[i] != -INFINITY ? 1u : 0u;
        }
        // chunk max, NaN count and finite count in one block reduction
        float xmax;
        uint32_t anynan, nfin;
        {
            const float wm = wave_max(tmax);
            const uint32_t wn = wave_sum(nan), wf = wave_sum(nf);
            if (lane_id() == 0) { sm.red.f[wave_id()] = wm; sm.red.u[wave_id()] = wn; sm.red.l[wave_id()] = (int64_t)wf; }
            __syncthreads();
            xmax = sm.red.f[0];
            anynan = sm.red.u[0];
            nfin = (uint32_t)sm.red.l[0];
#pragma unroll
            for (int w = 1; w < NWAVE; ++w) {
                xmax = sm.red.f[w] > xmax ? sm.red.f[w] : xmax;
                anynan += sm.red.u[w];
                nfin += (uint32_t)sm.red.l[w];
            }
            __syncthreads();
        }
        uint32_t flags = anynan ? FLAG_NAN : 0u;
        if (xmax != -INFINITY) {
            ymax = scale_y<DT>(xmax, pl.T);  // scaling is monotone
            if (ymax == INFINITY) flags |= FLAG_PINF;
        }
        const bool live = flags == 0u && ymax != -INFINITY;
        const float T = pl.T, rT = 1.0f / pl.T;
        double Sc = 0.0;
        uint32_t ncand = 0u, kc = 0u, trunc = 0u;
        if (live && pl.mode == M_TEMP) {
            double s = 0.0;
            if (T == 1.0f) {  // y = x exactly (a live chunk holds no NaN)
#pragma unroll
                for (int i = 0; i < EPT; ++i) s += (double)wexp(x[i], ymax);
            } else {
#pragma unroll
                for (int i = 0; i < EPT; ++i) s += (double)wexp(scale_r<DT>(x[i], T, rT), ymax);
            }
            Sc = block_sum<double>(s, sm.red);
        } else if (live && topp32) {
            // weights exp(y - ymax) in float64 (dexp: relative error below
            // 1e-15), their sum and coarse bins floor(4y) on the absolute
            // grid, the CB_N bins at and below the chunk max's, summed per
            // wave with LDS float64 atomics: exact enough that the masses
            // above the row's cut band come from these bins alone
            const float Ac = coarse_bin(ymax);
            exp_table(sm.etab, tid);
            for (int b = tid; b < NWAVE * CB_N; b += NT) (&sm.wb[0][0])[b] = 0.0;
            __syncthreads();
            const double ymd = (double)ymax;
            double s = 0.0;
            double *wb = sm.wb[wave_id()];
            scale_all<DT, EPT>(x, T, rT);  // x now holds y
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                const float y = x[i];
                const double e = dexp((double)y - ymd, sm.etab);
                s += e;
                const float cb = Ac - coarse_bin(y);  // +inf for y = -inf
                if (cb < (float)CB_N) atomicAdd(&wb[(int)cb], e);
            }
            Sc = block_sum<double>(s, sm.red);  // its barriers also order the bins
            if (tid < CB_N) rb->coarse[tid] = sm.wb[0][tid] + sm.wb[1][tid] + sm.wb[2][tid] + sm.wb[3][tid];
            if (tid == 0) { rb->S = Sc; rb->top = Ac; }
        } else if (live && (pl.mode == M_SMALLK || topp16)) {
            // (one else-if chain: separate branches here cost the fp32 kernel
            // 70 more VGPRs, half its occupancy)
            if (topp16) {
                // S in float64 over wexp weights (relative error at most
                // WEXP_REL_ERR): the row pass rounds probabilities to the
                // dtype and takes an exact S only for a row where one of
                // them could change within that bound
                double s = 0.0;
                if (T == 1.0f) {  // y = x exactly (a live chunk holds no NaN)
#pragma unroll
                    for (int i = 0; i < EPT; ++i) s += (double)wexp(x[i], ymax);
                } else {
#pragma unroll
                    for (int i = 0; i < EPT; ++i) s += (double)wexp(scale_r<DT>(x[i], T, rT), ymax);
                }
                Sc = block_sum<double>(s, sm.red);
            }
            // ---- candidates: every finite x whose scaled key reaches a threshold
            // taken from the per-thread maxima, enough for n_c candidates
            const uint32_t kk = topp16 ? (uint32_t)(a.V < (int64_t)K_PROBE ? a.V : (int64_t)K_PROBE) : (uint32_t)pl.kk;
            uint32_t nc = G == 1 ? kk : 2u * ((kk + (uint32_t)G - 1u) / (uint32_t)G) + 32u;
            if (nc > kk) nc = kk;
            uint32_t xlo = 0u;  // raw-key floor of the candidates
            if (nfin > nc) {
                uint32_t tkey;
                if (nc <= 256u) {
                    // each wave's ceil(nc/4)-th largest thread maximum: every
                    // wave then holds that many elements at or above the least
                    // of the four, so at least nc in all
                    const int q = (int)((nc + 3u) / 4u);
                    const uint32_t srt = wave_sort_asc(key_of_f32(tmax));
                    const uint32_t tw = (uint32_t)__shfl((int)srt, 64 - q, 64);
                    tkey = block_min<uint32_t>(tw, sm.red);
                } else {
                    // larger nc (few chunks per row): bisect the raw key for
                    // a threshold with nc <= count <= the chunk's candidate slots
                    uint32_t lo = 0u, hi = key_of_f32(xmax) + 1u, clo = nfin;
                    while (clo > (uint32_t)L.ccap && hi - lo > 1u) {
                        const uint32_t mid = lo + (hi - lo) / 2u;
                        uint32_t c = 0u;
#pragma unroll
                        for (int i = 0; i < EPT; ++i) c += (x[i] != -INFINITY && key_of_f32(x[i]) >= mid) ? 1u : 0u;
                        c = block_sum<uint32_t>(c, sm.red);
                        if (c >= nc) { lo = mid; clo = c; } else { hi = mid; }
                    }
                    tkey = lo;
                }
                // close under the ties the scaling creates
                const uint32_t sk = row_key(scale_y<DT>(f32_of_key(tkey), T), DT);
                kc = sk;
                xlo = x_lower<DT>(sk, T);  // every wave finds the same floor: no barrier
            }
            // the floor as a raw value: x >= xlof <=> key(x) >= xlo for every
            // finite x (zeros share a key); -inf never passes
            const float xlof = xlo > key_of_f32(-INFINITY) ? f32_of_key(xlo) : -FLT_MAX;
            uint32_t mine = 0u;
#pragma unroll
            for (int i = 0; i < EPT; ++i) mine += x[i] >= xlof ? 1u : 0u;
            uint32_t total;
            uint32_t off = block_excl_scan<uint32_t>(mine, sm.red, &total);
            if (total <= (uint32_t)L.ccap) {
                Cand *cand = reinterpret_cast<Cand *>(a.ws + L.cand) + ((size_t)row * G + chunk) * L.ccap;
#pragma unroll
                for (int i = 0; i < EPT; ++i)
                    if (x[i] >= xlof) {
                        cand[off].x = x[i];
                        cand[off].idx = idx_of(i);
                        ++off;
                    }
                ncand = total;
            } else {
                ncand = NCAND_OVERFLOW;
            }
            trunc = total < nfin ? 1u : 0u;
        }
        if (tid == 0) {
            cs->xkey = 0u; cs->xarg = IDX_ALL; cs->ymax = ymax; cs->flags = flags; cs->S = Sc;
            cs->ncand = ncand; cs->nfin = nfin; cs->kc = kc; cs->trunc = trunc;
        }
    }
    if (chunk == 0) trace(a.ws, L, row, 1);
}

// ------------------------------------------------------------------ the row pass

// ------------------------------------------------------------------ greedy, temperature, small top-k rows (k_rowpass)
//
// One workgroup of NTS threads per row, from the chunk summaries:
//   greedy       the argmax merge;
//   temperature  the chunk holding u * S, then that chunk re-read;
//   bad rows     their status;
//   small top-k  (0 < k' <= K_SMALL)
//     1. the candidate counts and prefix;
//     2. the candidates gathered into LDS, one wave per chunk;
//     3. the k'-th largest raw value by a three-level radix select over the
//        candidates' keys (11 / 11 / 10 bits, LDS histograms);
//     4. the survivors: scaled value >= scale(k'-th value), every tie kept,
//        with float64 weights exp(y - m) (dexp);
//     5. top-p over the survivors in the stable descending order: exact
//        masses (fp32) or torch's 16-bit rounding chain;
//     6. the inverse-CDF draw over the kept survivors in vocabulary order.
// A small-k row it cannot finish here (a chunk's candidates overflowed or
// were truncated above the threshold, more candidates than the LDS cache,
// more survivors than SURV_CAP) gets RowOut status ROW_DEFER; k_final's
// generic path then re-reads it.

constexpr int NTS = 1024;           // threads of k_rowpass (16 waves)
constexpr int ROW_DEFER = 16;       // RowOut status: k_final's generic path finishes the row

struct SmallkSmem {
    Cand cc[CCAP];                  // the row's candidates
    union {
        struct { uint32_t key[SURV_CAP]; int32_t idx[SURV_CAP]; double e[SURV_CAP]; } s;
        struct { uint64_t k[SURV_CAP]; double e[SURV_CAP]; } so;
    } u;
    struct { uint32_t key[SURV_CAP]; int32_t idx[SURV_CAP]; double e[SURV_CAP]; } sv;  // the survivors
    uint32_t h[2048];               // radix-select histogram; fp32 top-p: bin counts
    double hm[1024];                // fp32 top-p: bin masses
    uint32_t rkey[SURV_CAP], rcnt[SURV_CAP];  // 16-bit chain: runs (first sorted position, length)
    float rp[SURV_CAP];             //                         and their dtype probabilities
    uint32_t pre[G_MAX + 1];        // candidate prefix per chunk
    double sub_m[256];              // the draw's index-radix buckets
    double cw[G_MAX], chs[G_MAX];   // temperature rows: per-chunk weight and rescale
    double etab[ETAB_N];
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
    double bd[8];
    unsigned long long bq[2];
};

template <int DT>
__global__ __launch_bounds__(NTS) void k_rowpass(Args a)
{
    __shared__ SmallkSmem sm;
    constexpr int NW = NTS / 64;
    const Layout &L = a.L;
    const int row = blockIdx.x, tid = threadIdx.x, G = L.G;
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, a.V);
    RowOut *ro = reinterpret_cast<RowOut *>(a.ws + L.rowout) + row;
    if (pl.mode == M_BAD || pl.mode == M_INVAL) {
        write_row(ro, a, row, -1, pl.mode == M_BAD ? MIS_ROW_BAD_PARAM : MIS_ROW_INVALID, pl.mode, 0.0f, 0u, 0, 0.0);
        return;
    }
    if (pl.mode != M_SMALLK && pl.mode != M_GREEDY && pl.mode != M_TEMP) return;
    const ChunkSum *cs = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * G;
    static_assert(G_MAX <= NTS, "one chunk per thread");
    if (pl.mode == M_GREEDY) {
        // argmax merge: key descending, index ascending
        uint32_t k2 = 0u;
        int32_t i2 = IDX_ALL;
        if (tid < G) { k2 = ldp(&cs[tid].xkey); i2 = ldp(&cs[tid].xarg); }
        wave_argmax(k2, i2);
        if (lane_id() == 0) { sm.red.u[wave_id()] = k2; sm.red.l[wave_id()] = i2; }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < NW; ++w) {
                const uint32_t kk = sm.red.u[w];
                const int32_t ii = (int32_t)sm.red.l[w];
                if (kk > k2 || (kk == k2 && ii < i2)) { k2 = kk; i2 = ii; }
            }
            write_row(ro, a, row, i2, MIS_ROW_OK, pl.mode, 0.0f, 0u, i2, 1.0);
        }
        return;
    }
    if (pl.mode == M_TEMP) {
        // chunk weights are exp(y - ymax_c): rescale to the row max m, pick
        // the chunk holding u * S, re-read it for the index
        uint32_t flg = 0u;
        float yg = -INFINITY;
        double Sg = 0.0;
        if (tid < G) { flg = ldp(&cs[tid].flags) != 0u ? 1u : 0u; yg = ldp(&cs[tid].ymax); Sg = ldp(&cs[tid].S); }
        const float m = block_max<float, NW>(yg, sm.red);
        flg = block_sum<uint32_t, NW>(flg, sm.red);
        if (flg != 0u || m == -INFINITY) {
            write_row(ro, a, row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
            return;
        }
        if (tid < G) {
            const double ch = yg == -INFINITY ? 0.0 : exp((double)yg - (double)m);
            sm.chs[tid] = ch;
            sm.cw[tid] = Sg * ch;
        }
        int gsel;
        double resid, SK;
        pick_chunk(sm, G, pl.u, &gsel, &resid, &SK);  // (its barriers publish cw)
        int64_t id = -1;
        if (gsel >= 0) {
            RowCx c;
            c.rowp = a.logits + (int64_t)row * a.stride_bytes;
            c.V = a.V; c.vec_ok = a.vec_ok; c.G = G; c.CH = (int64_t)NT * L.ept; c.row = row; c.T = pl.T; c.m = m;
            const float yc = ldp(&cs[gsel].ymax), T = pl.T;
            // the chunk pass's weights, recomputed the same way
            id = draw_in_chunk<DT, NTS>(sm, c, gsel, resid / sm.chs[gsel], [&](float xv, int64_t) -> double {
                return (double)wexp(scale_y<DT>(xv, T), yc);
            });
        }
        write_row(ro, a, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, row_key(-INFINITY, DT), -1, SK);
        return;
    }
    const Cand *cand = reinterpret_cast<const Cand *>(a.ws + L.cand) + (size_t)row * G * L.ccap;
    trace(a.ws, L, row, 17);
    exp_table(sm.etab, tid);
    // 1. summaries
    uint32_t nc = 0u, ovf = 0u, ntr = 0u, nfin = 0u, flg = 0u;
    float ymx = -INFINITY;
    if (tid < G) {
        const uint32_t n = ldp(&cs[tid].ncand);
        ovf = n == NCAND_OVERFLOW ? 1u : 0u;
        nc = n <= (uint32_t)L.ccap ? n : 0u;
        ntr = ldp(&cs[tid].trunc) != 0u ? 1u : 0u;
        nfin = ldp(&cs[tid].nfin);
        flg = ldp(&cs[tid].flags) != 0u ? 1u : 0u;
        ymx = ldp(&cs[tid].ymax);
    }
    uint32_t ntot;
    const uint32_t off = block_excl_scan<uint32_t, NW>(nc, sm.red, &ntot);
    if (tid < G) sm.pre[tid] = off;
    const float m = block_max<float, NW>(ymx, sm.red);
    ovf = block_sum<uint32_t, NW>(ovf, sm.red);
    ntr = block_sum<uint32_t, NW>(ntr, sm.red);
    nfin = block_sum<uint32_t, NW>(nfin, sm.red);
    flg = block_sum<uint32_t, NW>(flg, sm.red);  // (its barriers publish pre)
    if (flg != 0u || m == -INFINITY) {  // NaN / +inf scaled logits, or nothing finite
        write_row(ro, a, row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
        return;
    }
    const double md = (double)m;
    // fewer finite elements than k': the k'-th value is -inf and every finite
    // element survives, which the candidates hold only if no chunk truncated
    const bool all_fin = nfin <= (uint32_t)pl.kk;
    if (ovf != 0u || ntot > (uint32_t)CCAP || (all_fin && ntr != 0u) || (!all_fin && ntot < (uint32_t)pl.kk)) {
        if (tid == 0) ro->status = ROW_DEFER;
        return;
    }
    // 2. candidates into LDS, one wave per chunk, eight loads in flight
    for (int g = wave_id(); g < G; g += NW) {
        const uint32_t n = g + 1 < G ? sm.pre[g + 1] - sm.pre[g] : ntot - sm.pre[g];
        const Cand *cg = cand + (size_t)g * L.ccap;
        Cand *dst = sm.cc + sm.pre[g];
        for (uint32_t i0 = 0; i0 < n; i0 += 8 * 64) {
            Cand v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t i = i0 + (uint32_t)(u * 64 + lane_id());
                v[u] = i < n ? ldp_cand(&cg[i]) : Cand{0.0f, 0};
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t i = i0 + (uint32_t)(u * 64 + lane_id());
                if (i < n) dst[i] = v[u];
            }
        }
    }
    __syncthreads();
    trace(a.ws, L, row, 21);
    // 3. k'-th largest raw key: three radix levels over the candidates
    uint32_t xk = 0u;
    if (!all_fin) {
        uint32_t prefix = 0u, rem = (uint32_t)pl.kk;
        const int sh[3] = {21, 10, 0};
        const int nb[3] = {2048, 2048, 1024};
#pragma unroll
        for (int lev = 0; lev < 3; ++lev) {
            const uint32_t hmask = lev == 0 ? 0u : ~((1u << (sh[lev] + (lev == 2 ? 10 : 11))) - 1u);
            for (int i = tid; i < 2048; i += NTS) sm.h[i] = 0u;
            __syncthreads();
            for (uint32_t f = tid; f < ntot; f += NTS) {
                const uint32_t k = key_of_f32(sm.cc[f].x);
                if ((k & hmask) == (prefix & hmask)) atomicAdd(&sm.h[(k >> sh[lev]) & (uint32_t)(nb[lev] - 1)], 1u);
            }
            __syncthreads();
            uint32_t above;
            const int d = block_find_desc<NTS>(sm.h, nb[lev], rem, &above, sm.red, &sm.bu[0]);
            rem -= above;
            prefix |= (uint32_t)d << sh[lev];
        }
        xk = prefix;
    }
    trace(a.ws, L, row, 18);
    // 4. survivors: scaled value >= scale(k'-th raw value); the ties the
    // scaling creates are kept, as the reference keeps them
    const uint32_t thr_key = xk ? row_key(scale_y<DT>(f32_of_key(xk), pl.T), DT) : 0u;
    if (ntr != 0u) {
        // a truncated chunk left out only elements with scaled keys below its
        // kc; they cannot reach the threshold if kc <= thr_key
        uint32_t hide = 0u;
        if (tid < G) hide = (ldp(&cs[tid].trunc) != 0u && ldp(&cs[tid].kc) > thr_key) ? 1u : 0u;
        hide = block_sum<uint32_t, NW>(hide, sm.red);
        if (hide != 0u) {
            if (tid == 0) ro->status = ROW_DEFER;
            return;
        }
    }
    if (tid == 0) sm.bu[3] = 0u;
    __syncthreads();
    const float T = pl.T, rT = 1.0f / pl.T;
    for (uint32_t f0 = 0; f0 < ntot; f0 += NTS) {
        const uint32_t f = f0 + tid;
        float y = 0.0f;
        uint32_t k = 0u;
        bool in = false;
        if (f < ntot) {
            y = scale_r<DT>(sm.cc[f].x, T, rT);
            k = row_key(y, DT);
            in = y != -INFINITY && k >= thr_key;
        }
        const uint32_t p = wave_append(in, &sm.bu[3]);
        if (in && p < (uint32_t)SURV_CAP) {
            sm.sv.key[p] = k;
            sm.sv.idx[p] = sm.cc[f].idx;
            sm.sv.e[p] = dexp((double)y - md, sm.etab);
        }
    }
    __syncthreads();
    const uint32_t ns = sm.bu[3];
    trace(a.ws, L, row, 19);
    if (ns > (uint32_t)SURV_CAP || ns == 0u) {
        if (tid == 0) ro->status = ROW_DEFER;
        return;
    }
    // 5. top-p over the survivors
    uint32_t cut_key = thr_key;
    int32_t cut_i = IDX_ALL;
    if (pl.topp) {
        double S = 0.0;
        for (uint32_t i = tid; i < ns; i += NTS) S += sm.sv.e[i];
        S = block_sum<double, NW>(S, sm.red);
        const double A = (double)pl.top_p * S;
        constexpr int PT = SURV_CAP / NTS;
        static_assert(PT == 1, "one survivor per thread");
        const int i = tid;
        if (DT == F32) {
            // exact masses: 1024 linear bins over the survivors' values locate
            // the bin(s) whose cumulative mass (descending) can reach A; only
            // their elements are sorted for the cut
            const bool have = i < (int)ns;
            const float yv = have ? f32_of_key(sm.sv.key[i]) : 0.0f;
            const float ylo = block_min<float, NW>(have ? yv : INFINITY, sm.red);
            const float yhi = block_max<float, NW>(have ? yv : -INFINITY, sm.red);
            const float inv = yhi > ylo ? 1023.0f / (yhi - ylo) : 0.0f;
            sm.h[i] = 0u;
            sm.hm[i] = 0.0;
            __syncthreads();
            int bin = 0;
            if (have) {
                bin = (int)fminf(fmaxf((yv - ylo) * inv, 0.0f), 1023.0f);
                atomicAdd(&sm.h[bin], 1u);
                atomicAdd(&sm.hm[bin], sm.sv.e[i]);
            }
            __syncthreads();
            // bins in descending order: thread t holds bin 1023 - t
            const double v = sm.hm[1023 - i];
            double tot;
            const double ex = block_excl_scan<double, NW>(v, sm.red, &tot);
            const double delta = 1e-12 * S;
            const bool inb = sm.h[1023 - i] > 0u && ex + v >= A - delta && ex <= A + delta;
            if (tid == 0) { sm.bi[0] = 1 << 20; sm.bi[1] = -1; }
            __syncthreads();
            if (inb) { atomicMin(&sm.bi[0], i); atomicMax(&sm.bi[1], i); }  // descending positions
            __syncthreads();
            const int pa = sm.bi[0], pb = sm.bi[1];
            if (inb && i == pa) sm.bd[0] = ex;
            if (tid == 0) sm.bu[4] = 0u;
            __syncthreads();
            bool ok = pa <= pb;
            if (ok) {
                const double above = sm.bd[0];
                // the window: survivors in bins [1023 - pb, 1023 - pa]
                const int blo = 1023 - pb, bhi = 1023 - pa;
                const bool w = have && bin >= blo && bin <= bhi;
                const uint32_t q = wave_append(w, &sm.bu[4]);
                if (w) { sm.u.s.key[q] = sm.sv.key[i]; sm.u.s.idx[q] = sm.sv.idx[i]; sm.u.s.e[q] = sm.sv.e[i]; }
                __syncthreads();
                const uint32_t nw = sm.bu[4];
                double ql, wl;
                const int rl = window_resolve<NTS>(sm, nw, above, A, &cut_key, &cut_i, &ql, &wl);
                ok = rl >= 0;
            }
            if (!ok) {  // the cut not inside the window (sums within rounding of A)
                if (tid == 0) ro->status = ROW_DEFER;
                return;
            }
        } else {
            // 16-bit rounding chain in the stable descending order: sort, runs
            // of equal keys with their probabilities in parallel, then one
            // wave walks the chain over the runs
            const uint64_t kt = i < (int)ns ? (((uint64_t)sm.sv.key[i] << 32) | (uint64_t)(0xffffffffu - (uint32_t)sm.sv.idx[i])) : 0ull;
            const double et = i < (int)ns ? sm.sv.e[i] : 0.0;
            sm.u.so.k[i] = kt;
            sm.u.so.e[i] = et;
            __syncthreads();
            block_sort_desc<NTS, SURV_CAP>(sm.u.so.k, sm.u.so.e, (int)ns);
            trace(a.ws, L, row, 23);
            const uint32_t st = i < (int)ns && (i == 0 || (uint32_t)(sm.u.so.k[i] >> 32) != (uint32_t)(sm.u.so.k[i - 1] >> 32)) ? 1u : 0u;
            uint32_t nr;
            const uint32_t r = block_excl_scan<uint32_t, NW>(st, sm.red, &nr);
            if (st) {
                sm.rkey[r] = (uint32_t)i;  // the run's first sorted position
                sm.rp[r] = rn_dtype((float)(sm.u.so.e[i] / S), DT);
            }
            __syncthreads();
            if ((uint32_t)i < nr) sm.rcnt[i] = ((uint32_t)i + 1 < nr ? sm.rkey[i + 1] : ns) - sm.rkey[i];
            __syncthreads();
            trace(a.ws, L, row, 24);
            if (wave_id() == 0) {
                const float thr16 = rn_dtype(pl.top_p, DT);
                int run_at = -1;
                uint32_t tk = 0;
                auto run = [&](int q, uint32_t *n, float *p) { *n = sm.rcnt[q]; *p = sm.rp[q]; };
                const bool found = chain_cut_wave((int)nr, run, thr16, DT, &run_at, &tk);
                const uint32_t r0 = found ? sm.rkey[run_at] + tk : ns;  // kept: sorted positions < r0
                if (lane_id() == 0) {
                    sm.bu[0] = r0;
                    if (r0 > 0) {
                        const uint64_t q = sm.u.so.k[r0 - 1];
                        sm.bu[1] = (uint32_t)(q >> 32);
                        sm.bi[0] = (int32_t)(0xffffffffu - (uint32_t)q);
                    }
                }
            }
            __syncthreads();
            trace(a.ws, L, row, 25);
            if (sm.bu[0] == 0u) {  // nothing kept: not a distribution
                write_row(ro, a, row, -1, MIS_ROW_INVALID, pl.mode, m, 0u, 0, 0.0);
                return;
            }
            cut_key = sm.bu[1];
            cut_i = sm.bi[0];
            __syncthreads();
        }
    }
    trace(a.ws, L, row, 20);
    // 6. the draw over the kept survivors in vocabulary order
    double SK = 0.0;
    for (uint32_t i = tid; i < ns; i += NTS) {
        if (!kept_by_cut(sm.sv.key[i], sm.sv.idx[i], cut_key, cut_i)) sm.sv.e[i] = 0.0;
        SK += sm.sv.e[i];
    }
    SK = block_sum<double, NW>(SK, sm.red);
    const int64_t id = draw_in_list<NTS>(sm, sm.sv.idx, sm.sv.e, (int)ns, a.V, (double)pl.u * SK);
    write_row(ro, a, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, cut_key, cut_i, SK);
    trace(a.ws, L, row, 22);
}

// ------------------------------------------------------------------ fp32 top-p rows
//
// Two launches after the chunk pass spread an fp32 top-p row over the GPU:
//   k_tp_hist   one workgroup per (row, chunk).  Every workgroup of a row
//               merges the row's coarse bins from the chunk pass (float64,
//               exact to rounding) into the row max, S, A = top_p * S and the
//               coarse band whose cumulative mass can reach A; the mass above
//               the band follows from the bins.  It then re-reads its chunk
//               (Infinity Cache) and puts the band's elements into FH linear
//               fine bins (count, float64 mass) and a stash (raw value,
//               index): all of them when they fit, otherwise those in a
//               window of fine bins around the cut as the chunk itself
//               estimates it (a chunk is a random sample of its row).
//   k_tp_final  one workgroup per row: merges the fine bins into the final
//               band (the bins whose cumulative mass can hold the cut), takes
//               that band's elements from the stashes (checking that every
//               chunk's window covers it), sorts them into the exact cut with
//               its decision margin checked against the error bound, then
//               draws.
// A row where a step does not apply is left to the row pass's generic path
// (RowOut status ROW_DEFER).

static_assert(NWAVE == 4, "four waves per chunk-pass workgroup");

__device__ __forceinline__ TopRow *top_row(const Args &a, int row)
{
    return reinterpret_cast<TopRow *>(a.ws + a.L.topr) + row;
}
__device__ __forceinline__ TopChunk *top_chunk(const Args &a, int row, int g)
{
    return reinterpret_cast<TopChunk *>(a.ws + a.L.topc) + (size_t)row * a.L.G + g;
}
__device__ __forceinline__ Cand *top_stash(const Args &a, int row, int g)
{
    return reinterpret_cast<Cand *>(a.ws + a.L.stash) + ((size_t)row * a.L.G + g) * STASH_CAP;
}
__device__ __forceinline__ int fine_bin(float y, float lo, float scf)
{
    return (int)fminf(fmaxf(floorf((y - lo) * scf), 0.0f), (float)(FH - 1));
}

// LDS of k_tp_hist
constexpr int LCAP = 4096;          // band elements of a chunk binned from a dense LDS list
struct HistSmem {
    double mc[CB_N];                // the row's merged coarse bins (relative to the row max)
    double chs[G_MAX];              // per chunk: exp(ymax_g - m)
    float off[G_MAX];               // per chunk: row top bin - chunk top bin
    uint32_t cnt[FH];
    double mass[FH];
    float lx[LCAP];                 // the chunk's band elements (raw values)
    double etab[ETAB_N];
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
    double bd[8];
    float bf[8];
};

template <int EPT>
__global__ __launch_bounds__(NT) void k_tp_hist(Args a)
{
    __shared__ HistSmem sm;
    constexpr int VEC = Traits<F32>::VEC;
    const Layout &L = a.L;
    const int tid = threadIdx.x, G = L.G;
    // workgroup i serves chunk i % G of row i / G, if an fp32 top-p row
    const int g = (int)(blockIdx.x % (unsigned)G);
    const int row = (int)(blockIdx.x / (unsigned)G);
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, a.V);
    if (pl.mode != M_TOPP) return;
    TopRow *tr = top_row(a, row);
    const bool tr0 = g == 0;
    if (tr0) trace(a.ws, L, row, 2);
    // the chunk's loads first: they overlap the summary loads below
    float x[EPT];
    const int64_t base = (int64_t)g * NT * EPT;
    load_chunk<F32, EPT>(a.logits + (int64_t)row * a.stride_bytes, base, a.V, a.vec_ok, x);
    exp_table(sm.etab, tid);
    const ChunkSum *csr = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * G;
    const RoundBuf *rbf = reinterpret_cast<const RoundBuf *>(a.ws + L.rbuf) + (size_t)row * G;
    static_assert(G_MAX <= NT, "one chunk per thread");
    const bool hasg = tid < G;
    uint32_t flag = 0u;
    float yg = -INFINITY, topg = 0.0f;
    double Sg = 0.0;
    if (hasg) { flag = ldp(&csr[tid].flags); yg = ldp(&csr[tid].ymax); topg = ldp(&rbf[tid].top); Sg = ldp(&rbf[tid].S); }
    const float m = block_max<float>(yg, sm.red);
    const uint32_t bad = block_sum<uint32_t>(flag ? 1u : 0u, sm.red);
    const float Ar = coarse_bin(m);
    // bins on the absolute grid floor(4y) stay exact small integers only while
    // |4y| < 2^23; beyond that (and for NaN / inf rows) the generic path serves
    if (bad != 0u || m == -INFINITY || !(fabsf(m) * CB_SCALE < 0x1p22f)) {
        if (g == 0 && tid == 0) tr->status = TR_DEFER;
        return;
    }
    const double md = (double)m;
    if (hasg) {
        sm.chs[tid] = yg == -INFINITY ? 0.0 : exp((double)yg - md);
        sm.off[tid] = yg == -INFINITY ? (float)CB_N : Ar - topg;
    }
    for (int b = tid; b < CB_N; b += NT) sm.mc[b] = 0.0;
    __syncthreads();
    const double S = block_sum<double>(hasg ? Sg * sm.chs[tid] : 0.0, sm.red);
    const double A = (double)pl.top_p * S;
    if (tr0) trace(a.ws, L, row, 3);
    // merged coarse bins: chunk g's bin b is the row's bin b + off[g]; eight
    // loads in flight per thread
    for (int q0 = 0; q0 < G * CB_N; q0 += 8 * NT) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int q = q0 + u * NT + tid;
            v[u] = q < G * CB_N ? ldp(&rbf[q / CB_N].coarse[q % CB_N]) : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int q = q0 + u * NT + tid, gq = q / CB_N;
            if (q < G * CB_N && v[u] != 0.0) {
                const float mb = (float)(q % CB_N) + sm.off[gq];
                if (mb < (float)CB_N) atomicAdd(&sm.mc[(int)mb], v[u] * sm.chs[gq]);
            }
        }
    }
    __syncthreads();
    if (tr0) trace(a.ws, L, row, 4);
    if (wave_id() == 0) {
        // the band: bins whose cumulative mass (descending) can reach A within
        // the float64 rounding of the sums; lane l holds bins 2l and 2l + 1
        static_assert(CB_N == 128, "two coarse bins per lane");
        const double delta = 1e-12 * S;
        const int l = lane_id();
        const double v0 = sm.mc[2 * l], v1 = sm.mc[2 * l + 1];
        const double inc = wave_incl_scan(v0 + v1), exc = inc - v0 - v1;
        const uint64_t m0 = __ballot(exc + v0 >= A - delta && exc <= A + delta);
        const uint64_t m1 = __ballot(inc >= A - delta && exc + v0 <= A + delta);
        int ba = -1, bb = -1;
        if ((m0 | m1) != 0ull) {
            const int f0 = m0 ? 2 * __builtin_ctzll(m0) : 1 << 20, f1 = m1 ? 2 * __builtin_ctzll(m1) + 1 : 1 << 20;
            const int h0 = m0 ? 2 * (63 - __builtin_clzll(m0)) : -1, h1 = m1 ? 2 * (63 - __builtin_clzll(m1)) + 1 : -1;
            ba = f0 < f1 ? f0 : f1;
            bb = h0 > h1 ? h0 : h1;
        }
        const int la = ba >= 0 ? ba >> 1 : 0;
        const double abv = __shfl(exc, la, 64) + ((ba & 1) ? __shfl(v0, la, 64) : 0.0);
        if (l == 0) { sm.bi[0] = ba; sm.bi[1] = bb; sm.bd[0] = abv; }
    }
    __syncthreads();
    const int ba = sm.bi[0], bb = sm.bi[1];
    if (ba < 0) {  // the cut lies below the coarse range
        if (g == 0 && tid == 0) tr->status = TR_DEFER;
        return;
    }
    const float cb_lo = Ar - (float)bb, cb_hi = Ar - (float)ba;
    if (wave_id() == 0) {
        // floor(4y) >= c <=> y >= c/4: the band's keys in closed form, checked
        // at both edges (a key search where the check fails)
        const uint32_t kfin = row_key(-INFINITY, F32) + 1u, ktop = 0xff7fffffu;  // finite keys
        auto ge_lo = [&](uint32_t k) { return coarse_bin(f32_of_key(k)) >= cb_lo; };
        auto gt_hi = [&](uint32_t k) { return coarse_bin(f32_of_key(k)) > cb_hi; };
        uint32_t k0 = key_of_f32(cb_lo / CB_SCALE), k1 = key_of_f32((cb_hi + 1.0f) / CB_SCALE) - 1u;
        const bool ok0 = k0 >= kfin && k0 <= ktop && ge_lo(k0) && (k0 == kfin || !ge_lo(k0 - 1u));
        const bool ok1 = k1 >= kfin && k1 <= ktop && !gt_hi(k1) && (k1 == ktop || gt_hi(k1 + 1u));
        if (!ok0) k0 = key_search(kfin, ktop, ge_lo);
        if (!ok1) k1 = key_search(kfin, ktop, gt_hi) - 1u;
        if (lane_id() == 0) { sm.bu[5] = k0; sm.bu[6] = k1; }
    }
    __syncthreads();
    const uint32_t klo = sm.bu[5], khi = sm.bu[6];
    uint32_t xlo, xhi;
    x_interval<F32>(sm, klo, khi, pl.T, &xlo, &xhi);
    const float lo = f32_of_key(klo), hi = f32_of_key(khi);
    const float scf = hi > lo ? (float)FH / (hi - lo) : 0.0f;
    const float T = pl.T, rT = 1.0f / pl.T;
    if (tr0) trace(a.ws, L, row, 5);
    if (g == 0 && tid == 0) {
        tr->klo = klo; tr->khi = khi; tr->xlo = xlo; tr->xhi = xhi;
        tr->m = m; tr->lo = lo; tr->scf = scf; tr->T = T;
        tr->S = S; tr->A = A;
        tr->status = TR_ACTIVE;
    }
    // this chunk's mass above the band, from its own coarse bins
    double ab = 0.0;
    if (tid < CB_N) {
        const float mb = (float)tid + sm.off[g];
        if (mb < (float)ba) ab = ldp(&rbf[g].coarse[tid]) * sm.chs[g];
    }
    const double above_g = block_sum<double>(ab, sm.red);
    for (int b = tid; b < FH; b += NT) { sm.cnt[b] = 0u; sm.mass[b] = 0.0; }
    if (tr0) trace(a.ws, L, row, 6);
    // the band's elements (raw keys in [xlo, xhi]): a dense list first
    const float xlof = f32_of_key(xlo), xhif = f32_of_key(xhi);
    uint64_t bm = 0ull;
#pragma unroll
    for (int i = 0; i < EPT; ++i) bm |= (x[i] >= xlof && x[i] <= xhif) ? (1ull << i) : 0ull;
    uint32_t nband;
    const uint32_t boff = block_excl_scan<uint32_t>((uint32_t)__popcll(bm), sm.red, &nband);
    {
        uint32_t q = boff;
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if (bm & (1ull << i)) { if (q < (uint32_t)LCAP) sm.lx[q] = x[i]; ++q; }
    }
    __syncthreads();
    auto bin_one = [&](float xv) {
        const float y = scale_r<F32>(xv, T, rT);
        const int b = fine_bin(y, lo, scf);
        atomicAdd(&sm.cnt[b], 1u);
        atomicAdd(&sm.mass[b], dexp((double)y - md, sm.etab));
    };
    const uint32_t nl = nband < (uint32_t)LCAP ? nband : (uint32_t)LCAP;
    for (uint32_t q = tid; q < nl; q += NT) bin_one(sm.lx[q]);
    if (nband > (uint32_t)LCAP) {  // a very dense band: the rest from registers
        uint32_t q = boff;
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if (bm & (1ull << i)) { if (q >= (uint32_t)LCAP) bin_one(x[i]); ++q; }
    }
    __syncthreads();
    if (tr0) trace(a.ws, L, row, 7);
    // the stash window: every fine bin when the band fits, otherwise the bins
    // around this chunk's own estimate of the cut (its fine masses scaled to
    // the row's band mass), widened while the elements fit
    int wlo = 0, whi = FH - 1;
    if (nband > (uint32_t)STASH_CAP) {
        {
            // prefix counts of the fine bins, two per thread (lx is free now)
            static_assert(FH == 2 * NT, "two fine bins per thread");
            const uint32_t c0 = sm.cnt[2 * tid], c1 = sm.cnt[2 * tid + 1];
            uint32_t tot;
            const uint32_t ex = block_excl_scan<uint32_t>(c0 + c1, sm.red, &tot);
            sm.lx[2 * tid] = __builtin_bit_cast(float, ex + c0);
            sm.lx[2 * tid + 1] = __builtin_bit_cast(float, ex + c0 + c1);
            __syncthreads();
        }
        if (wave_id() == 0) {
            // per lane 8 bins, descending order: bin FH-1 first
            constexpr int PB = FH / 64;
            double mloc = 0.0;
            const int l = lane_id();
#pragma unroll
            for (int q = 0; q < PB; ++q) mloc += sm.mass[FH - 1 - (l * PB + q)];
            double bandm_chunk = wave_sum(mloc);
            double bandm_row = 0.0;
            for (int b = ba; b <= bb; ++b) bandm_row += sm.mc[b];
            const double sc = bandm_chunk > 0.0 ? bandm_row / bandm_chunk : 0.0;
            const double need = A - sm.bd[0];  // residual mass inside the band
            // estimated cut bin: first bin (descending) where the scaled cumulative reaches need
            const double inc = wave_incl_scan(mloc) * sc;
            const uint64_t mk = __ballot(inc >= need);
            int est = 0;
            if (mk != 0ull) {
                const int f = __builtin_ctzll(mk);
                if (l == f) {
                    double run = (inc - mloc * sc);
                    est = FH - 1 - (f * PB + PB - 1);
                    for (int q = 0; q < PB; ++q) {
                        const int b = FH - 1 - (f * PB + q);
                        run += sm.mass[b] * sc;
                        if (run >= need) { est = b; break; }
                    }
                }
                est = __shfl(est, f, 64);
            }
            // the widest window [est - h, est + h] (clipped to the bins)
            // holding at most STASH_CAP elements, from the prefix counts
            // P(b) = elements in bins [0, b] (in lx), by two 64-way steps
            auto P = [&](int b) -> uint32_t { return b < 0 ? 0u : __builtin_bit_cast(uint32_t, sm.lx[b < FH ? b : FH - 1]); };
            auto fits = [&](int h) { return P(est + h) - P(est - h - 1) <= (uint32_t)STASH_CAP; };
            // coarse step: h = 8 l; then fine step within the last fitting 8
            const uint64_t fc = __ballot(fits(8 * l));
            int h = -1;
            if (fc & 1ull) {
                const int lc = 63 - __builtin_clzll(fc);  // fits() only shrinks as h grows
                const uint64_t ff = __ballot(l < 8 && fits(8 * lc + l));
                h = 8 * lc + (63 - __builtin_clzll(ff));
            }
            if (l == 0) {
                sm.bi[2] = h >= 0 ? (est - h > 0 ? est - h : 0) : 1;
                sm.bi[3] = h >= 0 ? (est + h < FH - 1 ? est + h : FH - 1) : 0;  // empty when one bin alone overflows
            }
        }
        __syncthreads();
        wlo = sm.bi[2]; whi = sm.bi[3];
    }
    if (tr0) trace(a.ws, L, row, 8);
    // stash the window's elements
    TopChunk *tc = top_chunk(a, row, g);
    Cand *st = top_stash(a, row, g);
    uint64_t sb = 0ull;
    if (nband > (uint32_t)STASH_CAP) {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if (bm & (1ull << i)) {
                const int b = fine_bin(scale_r<F32>(x[i], T, rT), lo, scf);
                sb |= (b >= wlo && b <= whi) ? (1ull << i) : 0ull;
            }
    } else {
        sb = bm;
    }
    uint32_t nst;
    uint32_t q = block_excl_scan<uint32_t>((uint32_t)__popcll(sb), sm.red, &nst);
    const int32_t base32 = (int32_t)base;
#pragma unroll
    for (int i = 0; i < EPT; ++i)
        if (sb & (1ull << i)) {
            if (q < (uint32_t)STASH_CAP) {
                st[q].x = x[i];
                st[q].idx = base32 + (int32_t)((((i / VEC) * NT + tid) * VEC) + (i % VEC));
            }
            ++q;
        }
    if (tid == 0) { tc->above = above_g; tc->nstash = nst; tc->wlo = wlo; tc->whi = whi; }
    for (int b = tid; b < FH; b += NT) { tc->cnt[b] = sm.cnt[b]; tc->mass[b] = sm.mass[b]; }
    if (tr0) trace(a.ws, L, row, 9);
}

constexpr int NTF = 1024;           // threads of k_tp_final (16 waves)

// LDS of k_tp_final
struct TopRowSmem {
    union {
        struct { uint32_t key[SURV_CAP]; int32_t idx[SURV_CAP]; double e[SURV_CAP]; } s;
        struct { uint64_t k[SURV_CAP]; double e[SURV_CAP]; } so;
    } u;
    uint32_t cnt[FH];
    double mass[FH];
    double cw[G_MAX];
    uint32_t ns[G_MAX];             // per chunk: elements stashed
    uint32_t ok[G_MAX];             // per chunk: its window wlo | whi << 16, all ones when it overflowed
    double etab[ETAB_N];
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
    double bd[8];
    unsigned long long bq[2];
};

__global__ __launch_bounds__(NTF) void k_tp_final(Args a)
{
    __shared__ TopRowSmem sm;
    const Layout &L = a.L;
    const int row = blockIdx.x, tid = threadIdx.x, G = L.G;
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, a.V);
    if (pl.mode != M_TOPP) return;
    TopRow *tr = top_row(a, row);
    RowOut *ro = reinterpret_cast<RowOut *>(a.ws + L.rowout) + row;
    if (ldp(&tr->status) != TR_ACTIVE) {
        if (tid == 0) ro->status = ROW_DEFER;
        return;
    }
    RowCx c;
    c.rowp = a.logits + (int64_t)row * a.stride_bytes;
    c.V = a.V; c.vec_ok = a.vec_ok; c.G = G; c.CH = (int64_t)NT * L.ept; c.row = row; c.T = pl.T;
    const float m = ldp(&tr->m), lo = ldp(&tr->lo), scf = ldp(&tr->scf);
    c.m = m;
    const double md = (double)m, A = ldp(&tr->A), S = ldp(&tr->S);
    const float T = pl.T, rT = 1.0f / pl.T;
    trace(a.ws, L, row, 10);
    exp_table(sm.etab, tid);
    // merged fine bins: thread t sums bin t % FH over the chunks t / FH,
    // t / FH + 2, ..., eight loads in flight
    static_assert(NTF == 2 * FH, "two threads per fine bin");
    {
        const int b = tid % FH, h = tid / FH;
        uint32_t cn = 0u;
        double ms = 0.0;
        for (int g0 = h; g0 < G; g0 += 16) {
            uint32_t cc[8];
            double mm[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int g = g0 + 2 * u;
                const TopChunk *tc = top_chunk(a, row, g < G ? g : 0);
                cc[u] = g < G ? tc->cnt[b] : 0u;
                mm[u] = g < G ? tc->mass[b] : 0.0;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) { cn += cc[u]; ms += mm[u]; }
        }
        if (h == 0) { sm.cnt[b] = cn; sm.mass[b] = ms; }
        __syncthreads();
        if (h == 1) { sm.cnt[b] += cn; sm.mass[b] += ms; }
    }
    trace(a.ws, L, row, 11);
    // per-chunk facts in one pass: above-band mass, stash count and window
    static_assert(G_MAX <= NTF, "one chunk per thread");
    if (tid < G) {
        const TopChunk *tc = top_chunk(a, row, tid);
        sm.cw[tid] = ldp(&tc->above);
        const uint32_t nsg = ldp(&tc->nstash);
        const int32_t wl = ldp(&tc->wlo), wh = ldp(&tc->whi);
        sm.ns[tid] = nsg;
        sm.ok[tid] = (nsg <= (uint32_t)STASH_CAP) ? ((uint32_t)wl | ((uint32_t)wh << 16)) : 0xffffffffu;
    }
    __syncthreads();
    trace(a.ws, L, row, 11);
    if (wave_id() == 0) {
        // the final band: fine bins whose cumulative mass (descending) can hold
        // the cut, within the float64 rounding of the sums
        double ab = 0.0;
        uint32_t bad = 0u;
        int wlo_max = 0, whi_min = FH - 1;
        for (int g = lane_id(); g < G; g += 64) {
            ab += sm.cw[g];
            const uint32_t o = sm.ok[g];
            if (o == 0xffffffffu) bad = 1u;
            else { wlo_max = max(wlo_max, (int)(o & 0xffffu)); whi_min = min(whi_min, (int)(o >> 16)); }
        }
        const double above_band = wave_sum(ab);
        bad = wave_sum(bad);
        wlo_max = wave_max(wlo_max);
        whi_min = wave_min(whi_min);
        const double delta = 1e-12 * S;
        double tmp;
        const int jb = wave_find_desc<double>(sm.mass, FH, A - delta - above_band, &tmp);
        const int ja = wave_find_desc<double>(sm.mass, FH, A + delta - above_band, &tmp);
        uint32_t c2 = 0u;
        double abf = 0.0;
        for (int b = lane_id(); b < FH; b += 64) {
            c2 += (b >= ja && b <= jb) ? sm.cnt[b] : 0u;
            abf += b > jb ? sm.mass[b] : 0.0;
        }
        c2 = wave_sum(c2);
        abf = wave_sum(abf);
        if (lane_id() == 0) {
            // every chunk's stash must hold the whole final band
            const bool ok = bad == 0u && ja <= jb && ja >= wlo_max && jb <= whi_min && c2 > 0u && c2 <= (uint32_t)SURV_CAP;
            sm.bi[0] = ok ? ja : -1; sm.bi[1] = jb; sm.bu[0] = c2; sm.bd[0] = above_band + abf;
            sm.bu[1] = 0u;
        }
    }
    __syncthreads();
    const int ja = sm.bi[0], jb = sm.bi[1];
    const uint32_t nwin = sm.bu[0];
    const double above = sm.bd[0];
    trace(a.ws, L, row, 12);
    if (ja < 0) {
        if (tid == 0) ro->status = ROW_DEFER;
        return;
    }
    // one wave per chunk: its kept mass above the window (above-band mass
    // plus fine bins above jb) and its stashed elements inside the window
    constexpr int NWF = NTF / 64;
    for (int g = wave_id(); g < G; g += NWF) {
        const TopChunk *tc = top_chunk(a, row, g);
        const Cand *stg = top_stash(a, row, g);
        const uint32_t ns = sm.ns[g];
        double mv[FH / 64];
        Cand cv[STASH_CAP / 64];
#pragma unroll
        for (int q = 0; q < FH / 64; ++q) { const int b = q * 64 + lane_id(); mv[q] = b > jb ? tc->mass[b] : 0.0; }
#pragma unroll
        for (int q = 0; q < STASH_CAP / 64; ++q) {
            const uint32_t i = (uint32_t)(q * 64 + lane_id());
            cv[q] = i < ns ? ldp_cand(&stg[i]) : Cand{0.0f, 0};
        }
        double w = 0.0;
#pragma unroll
        for (int q = 0; q < FH / 64; ++q) w += mv[q];
        w = wave_sum(w);
        if (lane_id() == 0) sm.cw[g] += w;
#pragma unroll
        for (int q = 0; q < STASH_CAP / 64; ++q) {
            const uint32_t i = (uint32_t)(q * 64 + lane_id());
            bool in = false;
            float y = 0.0f;
            if (i < ns) {
                y = scale_r<F32>(cv[q].x, T, rT);
                const int b = fine_bin(y, lo, scf);
                in = b >= ja && b <= jb;
            }
            const uint32_t p = wave_append(in, &sm.bu[1]);
            if (in && p < (uint32_t)SURV_CAP) {
                sm.u.s.key[p] = row_key(y, F32);
                sm.u.s.idx[p] = cv[q].idx;
                sm.u.s.e[p] = dexp((double)y - md, sm.etab);
            }
        }
    }
    __syncthreads();
    trace(a.ws, L, row, 13);
    const uint32_t n = sm.bu[1];
    trace(a.ws, L, row, 14);
    if (n != nwin) {  // the stashes do not hold the band exactly
        if (tid == 0) ro->status = ROW_DEFER;
        return;
    }
    uint32_t cut_key = 0u;
    int32_t cut_i = 0;
    double ql = 0.0, wl = 0.0;
    const int rl = window_resolve<NTF>(sm, n, above, A, &cut_key, &cut_i, &ql, &wl);
    // S, the above-masses and the window's weights carry relative errors
    // below 1e-15 each (dexp) plus float64 summation rounding
    const double err = 1e-12 * (above + A) + 1e-300;
    if (!(rl >= 0 && (A - ql) > err && (ql + wl - A) > err)) {
        if (tid == 0) ro->status = ROW_DEFER;
        return;
    }
    trace(a.ws, L, row, 15);
    const int chsh = __builtin_ctz((unsigned)c.CH);
    for (int q = tid; q <= rl; q += NTF) {
        const int32_t j = (int32_t)(0xffffffffu - (uint32_t)sm.u.so.k[q]);
        atomicAdd(&sm.cw[j >> chsh], sm.u.so.e[q]);
    }
    int gsel;
    double resid, SK;
    pick_chunk(sm, G, pl.u, &gsel, &resid, &SK);
    int64_t id = -1;
    if (gsel >= 0) {
        id = draw_in_chunk<F32, NTF>(sm, c, gsel, resid, [&](float xv, int64_t j) -> double {
            const float y = scale_r<F32>(xv, T, rT);
            return (y != -INFINITY && kept_by_cut(row_key(y, F32), j, cut_key, cut_i)) ? dexp((double)y - md, sm.etab) : 0.0;
        });
    }
    write_row(ro, a, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, cut_key, cut_i, SK);
    trace(a.ws, L, row, 30);
}

// ------------------------------------------------------------------ fp16/bf16 top-p rows
//
// Two launches after the chunk pass spread a 16-bit top-p row (top-k off)
// over the GPU.  A 16-bit scaled logit takes one of 65536 values, and torch's
// rounding chain depends only on the descending sequence of those values:
//   k_t16_hist  one workgroup per (row, chunk): the row max m from the chunk
//               maxima fixes the histogram's range, the NB16 16-bit keys at
//               and below m's key; the chunk's elements are counted per key
//               in LDS and the counts added into the row's histogram (integer
//               atomics: the sum does not depend on their order; the chunk
//               pass cleared the histogram); the chunk's exact mass sum
//               exp(y - m) (float64, one dexp per occupied key) goes to its
//               T16Chunk.
//   k_t16_walk  one workgroup per (row, chunk): each workgroup of a row reads
//               the merged histogram and S, rounds every run's probability
//               (all threads), walks the chain over the runs of equal keys
//               (chain_cut_wave, one wave) to the same cut, and writes its
//               own chunk's mass above the cut key and its count of elements
//               holding the cut key.
// k_final's final_t16 then draws from those chunk masses, the tie index at
// the cut key resolved in the one chunk where the kept ties end.  A row whose
// chain runs past the histogram's range with elements left under it takes
// the generic path (T16_DEFER).

__device__ __forceinline__ T16Row *t16_row(const Args &a, int row)
{
    return reinterpret_cast<T16Row *>(a.ws + a.L.t16r) + row;
}
__device__ __forceinline__ T16Chunk *t16_chunk(const Args &a, int row, int g)
{
    return reinterpret_cast<T16Chunk *>(a.ws + a.L.t16c) + (size_t)row * a.L.G + g;
}
__device__ __forceinline__ uint32_t *t16_hist(const Args &a, int row)
{
    return reinterpret_cast<uint32_t *>(a.ws + a.L.t16h) + (size_t)row * NB16;
}
__device__ __forceinline__ uint32_t key16(float y, int dt) { return row_key(y, dt) >> 16; }
__device__ __forceinline__ float value16(uint32_t k, int dt) { return value_of_row_key(k << 16, dt); }
__device__ __forceinline__ uint32_t t16_base(float m, int dt)  // lowest key of the histogram's range
{
    const uint32_t km = key16(m, dt);
    return km >= (uint32_t)(NB16 - 1) ? km - (uint32_t)(NB16 - 1) : 0u;
}

constexpr int NT16 = 1024;          // threads of k_t16_hist / k_t16_walk (16 waves, 8 or 16 elements each)
constexpr int NW16 = NT16 / 64;
struct T16Smem {
    uint32_t h[NB16];               // k_t16_hist: the chunk's counts; k_t16_walk: run keys
    uint32_t rc[NB16];              // run counts
    float rp[NB16];                 // run probabilities (rounded to the dtype)
    double etab[ETAB_N];
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
};

// EPT: the chunk pass's elements per thread (its chunk = NT * EPT elements,
// here NT16 threads of EPT * NT / NT16 each)
template <int DT, int EPT>
__global__ __launch_bounds__(NT16) void k_t16_hist(Args a)
{
    constexpr int E = EPT * NT / NT16;
    __shared__ T16Smem sm;
    const Layout &L = a.L;
    const int tid = threadIdx.x, G = L.G;
    const int row = (int)(blockIdx.x / (unsigned)G), g = (int)(blockIdx.x % (unsigned)G);
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, a.V);
    if (pl.mode != M_TOPP) return;
    if (g == 0) trace(a.ws, L, row, 2);
    float x[E];
    const int64_t base = (int64_t)g * NT * EPT;
    load_chunk_n<DT, E, NT16>(a.logits + (int64_t)row * a.stride_bytes, base, a.V, a.vec_ok, x);
    exp_table(sm.etab, tid);
    for (int b = tid; b < NB16; b += NT16) sm.h[b] = 0u;
    T16Row *tr = t16_row(a, row);
    // the row max from the chunk maxima (its barriers order the clearing above)
    const ChunkSum *csr = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * G;
    uint32_t flag = 0u;
    float yg = -INFINITY;
    if (tid < G) { flag = ldp(&csr[tid].flags); yg = ldp(&csr[tid].ymax); }
    static_assert(G_MAX <= NT16, "one chunk per thread");
    const float m = block_max<float, NW16>(yg, sm.red);
    const uint32_t bad = block_sum<uint32_t, NW16>(flag ? 1u : 0u, sm.red);
    if (bad != 0u || m == -INFINITY) {  // NaN / +inf: the generic path rejects the row
        if (g == 0 && tid == 0) tr->status = T16_DEFER;
        return;
    }
    const uint32_t kb = t16_base(m, DT);
    const double md = (double)m;
    if (g == 0) trace(a.ws, L, row, 9);
    scale_all<DT, E>(x, pl.T, 1.0f / pl.T);  // x now holds y
    double sb = 0.0;
    uint32_t nb = 0u;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const float y = x[i];
        if (y == -INFINITY) continue;
        const uint32_t k = key16(y, DT);
        if (k >= kb) {
            atomicAdd(&sm.h[k - kb], 1u);
        } else {
            sb += dexp((double)y - md, sm.etab);
            ++nb;
        }
    }
    __syncthreads();
    if (g == 0) trace(a.ws, L, row, 3);
    uint32_t *rh = t16_hist(a, row);
    double s = sb;
    for (int b = tid; b < NB16; b += NT16) {
        const uint32_t c = sm.h[b];
        if (c != 0u) {
            s += (double)c * dexp((double)value16(kb + (uint32_t)b, DT) - md, sm.etab);
            atomicAdd(&rh[b], c);
        }
    }
    s = block_sum<double, NW16>(s, sm.red);
    nb = block_sum<uint32_t, NW16>(nb, sm.red);
    if (tid == 0) {
        T16Chunk *tc = t16_chunk(a, row, g);
        tc->S = s;
        tc->below = nb;
        if (g == 0) tr->status = T16_NONE;
    }
    if (g == 0) trace(a.ws, L, row, 4);
}

template <int DT, int EPT>
__global__ __launch_bounds__(NT16) void k_t16_walk(Args a)
{
    constexpr int E = EPT * NT / NT16;
    __shared__ T16Smem sm;
    const Layout &L = a.L;
    const int tid = threadIdx.x, G = L.G;
    const int row = (int)(blockIdx.x / (unsigned)G), g = (int)(blockIdx.x % (unsigned)G);
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, a.V);
    if (pl.mode != M_TOPP) return;
    T16Row *tr = t16_row(a, row);
    if (uni(ldp(&tr->status)) == T16_DEFER) return;
    if (g == 0) trace(a.ws, L, row, 5);
    float x[E];
    const int64_t base = (int64_t)g * NT * EPT;
    load_chunk_n<DT, E, NT16>(a.logits + (int64_t)row * a.stride_bytes, base, a.V, a.vec_ok, x);
    exp_table(sm.etab, tid);
    const ChunkSum *csr = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * G;
    // the row max, S and the count under the range, in one fixed order
    float yg = -INFINITY;
    double sg = 0.0;
    uint32_t bg = 0u;
    if (tid < G) {
        yg = ldp(&csr[tid].ymax);
        const T16Chunk *tq = t16_chunk(a, row, tid);
        sg = ldp(&tq->S);
        bg = ldp(&tq->below);
    }
    const float m = block_max<float, NW16>(yg, sm.red);
    const double S = block_sum<double, NW16>(sg, sm.red);
    const uint32_t below = block_sum<uint32_t, NW16>(bg, sm.red);
    const uint32_t kb = t16_base(m, DT);
    const double md = (double)m;
    // runs: the occupied keys in descending order, NB16 / NT16 bins per thread
    constexpr int PER = NB16 / NT16;
    const uint32_t *rh = t16_hist(a, row);
    uint32_t hc[PER];
    uint32_t nmine = 0u;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        hc[j] = ldp(&rh[NB16 - 1 - (tid * PER + j)]);
        nmine += hc[j] != 0u ? 1u : 0u;
    }
    uint32_t nr;
    uint32_t o = block_excl_scan<uint32_t, NW16>(nmine, sm.red, &nr);
    if (g == 0) trace(a.ws, L, row, 10);
    // each run's key, count and probability RN16(RN32(exp(y - m) / S))
#pragma unroll
    for (int j = 0; j < PER; ++j)
        if (hc[j] != 0u) {
            const uint32_t b = (uint32_t)(NB16 - 1 - (tid * PER + j));
            sm.h[o] = b;
            sm.rc[o] = hc[j];
            sm.rp[o] = rn_dtype((float)(dexp((double)value16(kb + b, DT) - md, sm.etab) / S), DT);
            ++o;
        }
    __syncthreads();
    if (g == 0) trace(a.ws, L, row, 6);
    const float thr16 = rn_dtype(pl.top_p, DT);
    if (wave_id() == 0) {
        auto run = [&](int r, uint32_t *n, float *p) { *n = sm.rc[r]; *p = sm.rp[r]; };
        int run_at = -1;
        uint32_t tk = 0u;
        const bool found = chain_cut_wave((int)nr, run, thr16, DT, &run_at, &tk);
        if (lane_id() == 0) { sm.bi[0] = found ? run_at : -1; sm.bu[0] = tk; }
    }
    __syncthreads();
    if (g == 0) trace(a.ws, L, row, 7);
    const int run_at = sm.bi[0];
    const uint32_t tk = sm.bu[0];
    uint32_t status = T16_CUT, ck = 0u, t = 0u;
    if (run_at < 0) {
        // the chain never reaches thr16 over the range: everything in it is
        // kept, and the row is done only if nothing lies under it
        if (below != 0u || nr == 0u) status = T16_DEFER;
        else { ck = kb + sm.h[nr - 1]; t = sm.rc[nr - 1]; }
    } else if (tk > 0u) {
        ck = kb + sm.h[run_at]; t = tk;
    } else if (run_at > 0) {
        ck = kb + sm.h[run_at - 1]; t = sm.rc[run_at - 1];
    } else {
        status = T16_EMPTY;  // rank 0 removed: nothing left to sample
    }
    if (status == T16_CUT) {
        // this chunk: mass above the cut key and the elements holding it
        scale_all<DT, E>(x, pl.T, 1.0f / pl.T);
        double s = 0.0;
        uint32_t cc = 0u;
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float y = x[i];
            if (y == -INFINITY) continue;
            const uint32_t k = key16(y, DT);
            if (k > ck) s += dexp((double)y - md, sm.etab);
            cc += k == ck ? 1u : 0u;
        }
        s = block_sum<double, NW16>(s, sm.red);
        cc = block_sum<uint32_t, NW16>(cc, sm.red);
        if (tid == 0) {
            T16Chunk *tc = t16_chunk(a, row, g);
            tc->kept = s;
            tc->ccnt = cc;
        }
    }
    if (g == 0 && tid == 0) {
        tr->ck = ck;
        tr->t = t;
        tr->S = S;
        tr->status = status;
    }
    if (g == 0) trace(a.ws, L, row, 8);
}

// Index of the t-th (1-based) element of chunk g, in index order, whose
// scaled value has key rk (kept_by_cut's key form); -1 when the chunk holds
// fewer.  Thread i takes the contiguous elements [cbeg + i*per, cbeg +
// (i+1)*per), loaded up front, as draw_in_chunk.
template <int DT, int NTH = NT, class SM>
__device__ __forceinline__ int64_t nth_key_in_chunk(SM &sm, const RowCx &c, int g, uint32_t rk, uint32_t t)
{
    constexpr int VEC = Traits<DT>::VEC, MAXPER = 64 * NT / NTH;
    const int64_t cbeg = (int64_t)g * c.CH;
    const int64_t cend = cbeg + c.CH < c.V ? cbeg + c.CH : c.V;
    const int per = (int)(c.CH / NTH);
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
                for (int e = 0; e < VEC; ++e) xs[v * VEC + e] = (j0 + e < cend) ? load1<DT>(c.rowp, j0 + e) : -INFINITY;
            }
        }
    }
    const float T = c.T, rT = 1.0f / c.T;
    uint64_t hit = 0ull;
#pragma unroll
    for (int i = 0; i < MAXPER; ++i) {
        if (i < per && jb + i < cend) {
            const float y = scale_r<DT>(xs[i], T, rT);
            hit |= (y != -INFINITY && row_key(y, DT) == rk) ? (1ull << i) : 0ull;
        }
    }
    const uint32_t mine = (uint32_t)__popcll(hit);
    uint32_t tot;
    const uint32_t before = block_excl_scan<uint32_t, NTH / 64>(mine, sm.red, &tot);
    if (threadIdx.x == 0) sm.bq[0] = 0xffffffffffffffffull;
    __syncthreads();
    if (mine > 0u && before < t && t <= before + mine) {
        uint64_t hh = hit;
        for (uint32_t k = before + 1u; k < t; ++k) hh &= hh - 1ull;  // drop the lower set bits
        sm.bq[0] = (unsigned long long)(jb + __builtin_ctzll(hh));
    }
    __syncthreads();
    const unsigned long long r = sm.bq[0];
    __syncthreads();
    return r == 0xffffffffffffffffull ? -1 : (int64_t)r;
}

// LDS of k_t16_final
struct T16FinSmem {
    double e16[NB16];               // exp(y - m) per key in [ck, key of m] (index key - kb)
    double cw[G_MAX];               // per-chunk kept mass
    double etab[ETAB_N];
    Red red;
    uint32_t bu[8];
    int32_t bi[8];
    double bd[8];
    unsigned long long bq[2];
};

// One workgroup per 16-bit top-p row after the t16 passes: per-chunk kept
// masses, the tie index at the cut key (in the one chunk where the kept ties
// end), the draw.  Rows the passes left to the generic path (T16_DEFER) are
// k_final's.  The chunk masses were summed from the same dexp values this
// table holds (a 16-bit y is its key's value), so the draw inside a chunk
// adds the same numbers.
template <int DT>
__global__ __launch_bounds__(NTF) void k_t16_final(Args a)
{
    __shared__ T16FinSmem sm;
    constexpr int NW = NTF / 64;
    const Layout &L = a.L;
    const int tid = threadIdx.x, G = L.G, row = blockIdx.x;
    mis_row_params P = a.params[row];
    P.temperature = uni(P.temperature); P.top_k = uni(P.top_k); P.top_p = uni(P.top_p); P.uniform = uni(P.uniform);
    const RowPlan pl = plan_row(P, a.V);
    if (pl.mode != M_TOPP) return;
    const T16Row *tr = t16_row(a, row);
    const uint32_t st = uni(ldp(&tr->status));
    RowOut *ro = reinterpret_cast<RowOut *>(a.ws + L.rowout) + row;
    if (st == T16_EMPTY) {  // rank 0 removed: torch.multinomial's invalid distribution
        write_row(ro, a, row, -1, MIS_ROW_INVALID, pl.mode, 0.0f, 0u, 0, 0.0);
        return;
    }
    if (st != T16_CUT) return;
    trace(a.ws, L, row, 11);
    const uint32_t ck = uni(ldp(&tr->ck)), t = uni(ldp(&tr->t));
    exp_table(sm.etab, tid);
    const ChunkSum *csr = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * G;
    float yg = -INFINITY;
    double kept = 0.0;
    uint32_t cg = 0u;
    static_assert(G_MAX <= NTF, "one chunk per thread");
    if (tid < G) {
        yg = ldp(&csr[tid].ymax);
        const T16Chunk *tq = t16_chunk(a, row, tid);
        kept = ldp(&tq->kept);
        cg = ldp(&tq->ccnt);
    }
    const float m = block_max<float, NW>(yg, sm.red);
    uint32_t tot;
    const uint32_t pre = block_excl_scan<uint32_t, NW>(cg, sm.red, &tot);
    const double md = (double)m;
    const uint32_t kb = t16_base(m, DT), km = key16(m, DT);
    for (uint32_t k = ck + (uint32_t)tid; k <= km; k += NTF) sm.e16[k - kb] = dexp((double)value16(k, DT) - md, sm.etab);
    if (tid == 0) sm.bi[2] = -1;
    __syncthreads();
    // the chunk holding the t-th tie (index order) keeps part of its ties
    if (tid < G) {
        const uint32_t kc = t > pre ? (t - pre < cg ? t - pre : cg) : 0u;
        sm.cw[tid] = kept + sm.e16[ck - kb] * (double)kc;
        if (cg != 0u && pre < t && t <= pre + cg) { sm.bi[2] = tid; sm.bu[2] = t - pre; sm.bu[3] = cg; }
    }
    __syncthreads();
    RowCx c;
    c.rowp = a.logits + (int64_t)row * a.stride_bytes;
    c.V = a.V; c.vec_ok = a.vec_ok; c.T = pl.T; c.m = m; c.G = G; c.CH = (int64_t)NT * L.ept; c.row = row;
    const int gb = sm.bi[2];
    const uint32_t tb = sm.bu[2], cb = sm.bu[3];
    const uint32_t rk = ck << 16;  // the cut key as a row key
    // the chunk first: the per-chunk kept masses do not depend on the tie index
    int gsel;
    double resid, SK;
    pick_chunk(sm, G, pl.u, &gsel, &resid, &SK);
    int32_t cut_i = IDX_ALL;
    if (gb >= 0 && tb < cb) {
        // the last kept tie lies inside chunk gb: its index matters to a draw
        // in that chunk and to the emitted keep masks; a draw in another chunk
        // keeps every tie before chunk gb and none after it, as gb * CH - 1 does
        if (gsel == gb || a.emit) cut_i = (int32_t)nth_key_in_chunk<DT, NTF>(sm, c, gb, rk, tb);
        else cut_i = (int32_t)((int64_t)gb * c.CH - 1);
    } else if (gb >= 0 && tot > t) {
        cut_i = (int32_t)((int64_t)(gb + 1) * c.CH - 1);  // every tie up to chunk gb's end
    }
    trace(a.ws, L, row, 12);
    int64_t id = -1;
    if (gsel >= 0) {
        const float T = pl.T, rT = 1.0f / pl.T;
        id = draw_in_chunk<DT, NTF>(sm, c, gsel, resid, [&](float xv, int64_t j) -> double {
            const float y = scale_r<DT>(xv, T, rT);
            if (y == -INFINITY) return 0.0;
            const uint32_t k = row_key(y, DT);
            return kept_by_cut(k, j, rk, cut_i) ? sm.e16[(k >> 16) - kb] : 0.0;
        });
    }
    write_row(ro, a, row, id, id >= 0 ? MIS_ROW_OK : MIS_ROW_INVALID, pl.mode, m, rk, cut_i, SK);
    trace(a.ws, L, row, 13);
}

enum : int { FIN_ALL = 0, FIN_OTHERS = 1, FIN_DEFERRED = 2, FIN_REST = 3, FIN_TAIL = 4 };
constexpr int FIN_T16 = 8;  // flag: the t16 passes ran before this k_final

// One workgroup per row: merges the chunk summaries and finishes the row:
// greedy, temperature, small top-k from the summaries; the generic re-read
// path otherwise.  fp32 top-p rows are the k_tp_* passes'.
template <int DT>
__global__ __launch_bounds__(NT) void k_final(Args a, int phase)
{
    __shared__ Smem sm;
    const Layout &L = a.L;
    const int row = blockIdx.x;
    RowOut *ro = reinterpret_cast<RowOut *>(a.ws + L.rowout) + row;
    if (threadIdx.x == 0) {
        sm.args = a;
        RowCx &c = sm.cx;
        c.rowp = a.logits + (int64_t)row * a.stride_bytes;
        c.V = a.V; c.vec_ok = a.vec_ok; c.m = 0.0f; c.G = L.G; c.CH = (int64_t)NT * L.ept; c.row = row;
        sm.pl = plan_row(a.params[row], a.V);
        c.T = sm.pl.T;
    }
    trace(a.ws, L, row, 16);
    __syncthreads();
    const ChunkSum *csr = reinterpret_cast<const ChunkSum *>(a.ws + L.chunks) + (size_t)row * L.G;
    // k_rowpass serves greedy, temperature and small top-k rows (and rejects
    // bad ones), the k_tp_* passes fp32 top-p rows; either leaves a row it
    // cannot finish with status ROW_DEFER.  By phase:
    //   FIN_ALL       after k_rowpass, no top-p passes: every row but
    //                 k_rowpass's, and the rows it deferred;
    //   FIN_OTHERS    after k_rowpass, beside the top-p passes: the rows
    //                 neither serves (fp16/bf16 top-p, top-k above K_SMALL);
    //   FIN_DEFERRED  after both: every deferred row;
    //   FIN_REST      after the top-p passes, no k_rowpass: every row but
    //                 the top-p passes', and the rows they deferred;
    //   FIN_TAIL      FIN_DEFERRED when FIN_OTHERS did not run: the deferred
    //                 rows and those neither serves.
    //   FIN_T16       (flag) the t16 passes ran: of the 16-bit top-p rows
    //                 only those they deferred.
    const int mode = sm.pl.mode, ph = phase & ~FIN_T16;
    const bool rp = mode == M_BAD || mode == M_INVAL || mode == M_GREEDY || mode == M_TEMP || mode == M_SMALLK;
    const bool tp = DT == F32 && mode == M_TOPP;
    bool serve;
    if (ph == FIN_ALL) serve = !rp || ldp(&ro->status) == ROW_DEFER;
    else if (ph == FIN_OTHERS) serve = !rp && !tp;
    else if (ph == FIN_DEFERRED) serve = (rp || tp) && ldp(&ro->status) == ROW_DEFER;
    else if (ph == FIN_TAIL) serve = (!rp && !tp) || ldp(&ro->status) == ROW_DEFER;
    else serve = !tp || ldp(&ro->status) == ROW_DEFER;
    // after the t16 passes a 16-bit top-p row is k_t16_final's unless they deferred it
    if (serve && DT != F32 && mode == M_TOPP && (phase & FIN_T16) != 0)
        serve = ldp(&reinterpret_cast<const T16Row *>(a.ws + L.t16r)[row].status) == T16_DEFER;
    if (!serve) return;
    leader_row<DT>(sm, sm.cx, sm.pl, csr, ro, sm.args);
    trace(a.ws, L, row, 31);
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

template <int DT, int EPT>
static hipError_t launch_sample(const Args &a, hipStream_t st, int part)
{
    const unsigned grid = (unsigned)(a.L.B * a.L.G);
    hipLaunchKernelGGL((k_sample<DT, EPT>), dim3(grid), dim3(NT), 0, st, a, part);
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_chunks(const Args &a, hipStream_t st, int part)
{
    switch (a.L.ept) {
    case 64: return launch_sample<DT, 64>(a, st, part);
    default: return launch_sample<DT, 32>(a, st, part);
    }
}

// events (optional, nev = 3 or 4): [0] before the chunk pass, [1] after the
// chunk pass on the caller's stream (with the split, its fp32 top-p rows'),
// [2] after the row pass (before the debug emit), [3] after the side stream's
// chunk pass (recorded only with the split: one more marker on the caller's
// stream would add its own gap to the step)
// One step's launches.  With fp32 top-p rows beside other rows and a side
// stream from the caller, the other rows' chunk pass and row pass run on the
// side stream beside the top-p rows' chunk pass and top-p passes; the rows
// either deferred follow once both are done.  Without a side stream the same
// kernels run in one stream.  Each chunk-pass half covers every (row, chunk)
// and keeps the workgroups of its own rows.
template <int DT>
static hipError_t launch_dt(const Args &a, float *probs, uint32_t *keep, hipStream_t st, unsigned kinds,
                            void *const *ev, int nev, const SideStreams *sd)
{
    hipError_t e;
    const unsigned B = (unsigned)a.L.B;
    const bool tp32 = DT == F32 && (kinds & MIS_KIND_TOPP32);
    const bool others = (kinds & MIS_KIND_OTHER) != 0u;
    const bool side = tp32 && others && sd != nullptr;
    // events[0] opens the chunk pass
    if (ev && (e = hipEventRecord((hipEvent_t)ev[0], st)) != hipSuccess) return e;
    if (side) {
        if ((e = hipEventRecord(sd->fork, st)) != hipSuccess) return e;
        if ((e = hipStreamWaitEvent(sd->s, sd->fork, 0)) != hipSuccess) return e;
        if ((e = launch_chunks<DT>(a, sd->s, K1_OTHERS)) != hipSuccess) return e;
        if (ev && nev > 3 && (e = hipEventRecord((hipEvent_t)ev[3], sd->s)) != hipSuccess) return e;
        hipLaunchKernelGGL((k_rowpass<DT>), dim3(B), dim3(NTS), 0, sd->s, a);
        if (kinds & MIS_KIND_GENERIC) hipLaunchKernelGGL((k_final<DT>), dim3(B), dim3(NT), 0, sd->s, a, (int)FIN_OTHERS);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = hipEventRecord(sd->join, sd->s)) != hipSuccess) return e;
    }
    if ((e = launch_chunks<DT>(a, st, side ? K1_TOPP32 : K1_ALL)) != hipSuccess) return e;
    if (ev && (e = hipEventRecord((hipEvent_t)ev[1], st)) != hipSuccess) return e;
    // the row pass in this stream: unless the side stream runs it, or the
    // batch holds fp32 top-p rows only (k_final's FIN_REST then serves the rest)
    const bool rowpass_here = !side && !(tp32 && !others);
    if (rowpass_here) hipLaunchKernelGGL((k_rowpass<DT>), dim3(B), dim3(NTS), 0, st, a);
    if (tp32) {
        const unsigned bg = (unsigned)(a.L.B * a.L.G);
        if (a.L.ept == 64) hipLaunchKernelGGL((k_tp_hist<64>), dim3(bg), dim3(NT), 0, st, a);
        else hipLaunchKernelGGL((k_tp_hist<32>), dim3(bg), dim3(NT), 0, st, a);
        hipLaunchKernelGGL(k_tp_final, dim3(B), dim3(NTF), 0, st, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (side && (e = hipStreamWaitEvent(st, sd->join, 0)) != hipSuccess) return e;
        const int ph = side ? ((kinds & MIS_KIND_GENERIC) ? FIN_DEFERRED : FIN_TAIL) : rowpass_here ? FIN_TAIL : FIN_REST;
        hipLaunchKernelGGL((k_final<DT>), dim3(B), dim3(NT), 0, st, a, ph);
    } else if (DT != F32 && a.L.t16 && (kinds & MIS_KIND_GENERIC)) {
        const unsigned bg = (unsigned)(a.L.B * a.L.G);
        if (a.L.ept == 64) {
            hipLaunchKernelGGL((k_t16_hist<DT, 64>), dim3(bg), dim3(NT16), 0, st, a);
            hipLaunchKernelGGL((k_t16_walk<DT, 64>), dim3(bg), dim3(NT16), 0, st, a);
        } else {
            hipLaunchKernelGGL((k_t16_hist<DT, 32>), dim3(bg), dim3(NT16), 0, st, a);
            hipLaunchKernelGGL((k_t16_walk<DT, 32>), dim3(bg), dim3(NT16), 0, st, a);
        }
        hipLaunchKernelGGL((k_t16_final<DT>), dim3(B), dim3(NTF), 0, st, a);
        hipLaunchKernelGGL((k_final<DT>), dim3(B), dim3(NT), 0, st, a, (int)(FIN_ALL | FIN_T16));
    } else {
        hipLaunchKernelGGL((k_final<DT>), dim3(B), dim3(NT), 0, st, a, (int)FIN_ALL);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (ev && (e = hipEventRecord((hipEvent_t)ev[2], st)) != hipSuccess) return e;
    if (probs || keep) {
        const unsigned gx = (unsigned)((a.V + (int64_t)NT * 8 - 1) / ((int64_t)NT * 8));
        hipLaunchKernelGGL((k_emit<DT>), dim3(gx, (unsigned)a.L.B), dim3(NT), 0, st, a.logits, a.V, a.stride_bytes,
                           a.params, a.L, (const char *)a.ws, probs, keep);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace
}  // namespace mis
