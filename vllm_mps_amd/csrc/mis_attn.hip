// mis_attn.hip -- decode-step paged attention over an fp16 KV block pool, and
// the pool gather (include/mis_attention.h).
//
// Pool layout, as the reference engine allocates it
// (memory/mps_memory_pool.py:62): [num_blocks, 2 (K, V), block_size,
// n_kv_heads, d_k] fp16, element strides pool_stride0 (block) and
// pool_stride1 (K -> V).  Token t of sequence b lives in physical block
// block_tables[b * max_blocks + t / block_size] at position t % block_size.
//
// k_attn_split: one workgroup of 4 waves per (sequence, KV head, context split
// of ts = 64, 128 or 256 tokens; smaller splits when the batch alone would not
// fill the chip).  It serves every query head of that KV head (GQA), so each
// K and V row is read from HBM once per group.
//   scores   16-token tiles on the matrix cores: v_mfma_f32_16x16x16_f16 with
//            the query heads as the 16 rows (A, held in registers for the
//            whole kernel) and the tile's K rows as the 16 columns (B, loaded
//            straight from the pool, 64 contiguous bytes per lane); fp16
//            products are exact in the fp32 accumulator.  Each wave keeps
//            several tiles' loads in flight.
//   softmax  per query head over the split (max, exp, sum) in LDS.
//   values   the weighted V sum on the vector ALUs: a lane takes 8 dims of one
//            token per 16-byte load, several tokens in flight, fp32 FMAs;
//            lanes sharing dims are summed by shuffles, the waves in LDS.
// A split writes its unnormalised output with its max and sum; a context of
// one split writes the final fp16 output directly.  k_attn_merge combines the
// splits (max-rescaled sums).
// The sequence's newest token (position seq_len - 1) is the call's new_k /
// new_v: the workgroup holding it writes them into the pool at write_info's
// (block, position) and uses them from the inputs, so no workgroup reads
// another's write.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mis_attention.h"

namespace mis {
namespace {

constexpr int ATT_NT = 256;          // threads per workgroup
constexpr int ATT_NW = ATT_NT / 64;  // waves per workgroup
constexpr int ATT_TS = 256;          // tokens per split, at most
constexpr int ATT_GMAX = 16;         // query heads per KV head, at most (the MFMA's 16 rows)
constexpr int ATT_FILL = 2048;       // workgroups wanted before splits are made smaller

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

struct AttnArgs {
    __half *pool;
    int64_t s0, s1;                  // element strides: block, K -> V
    int64_t num_blocks;
    int block_size, n_kv, n_heads, G, max_blocks;
    const __half *new_k, *new_v, *queries;
    const int32_t *block_tables, *seq_lens, *write_info;
    __half *out;
    float *part;                     // [B, n_heads, nsplit, D] unnormalised outputs
    float *pm, *pl;                  // [B, n_heads, nsplit] split max and sum
    int nsplit, ts;
    int bs_shift;                    // log2(block_size) for a power of two, else -1
    float scale;
};

__device__ __forceinline__ half4_t half4_of(unsigned int lo, unsigned int hi)
{
    const u32x2_t v = {lo, hi};
    return __builtin_bit_cast(half4_t, v);
}

// Orders one wave's LDS writes before its later reads (and reads before later
// writes): a wave's LDS operations complete in order, so a compiler barrier suffices.
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D, bool FAST>
__global__ __launch_bounds__(ATT_NT) void k_attn_split(AttnArgs a)
{
    constexpr int NW = ATT_NW;
    constexpr int QV = D / 32;                 // 16-byte K loads per lane per tile (a quarter row)
    constexpr int NM = D / 16;                 // MFMAs per tile
    constexpr int KT = D == 256 ? 2 : 4;       // tiles per batch of K loads
    constexpr int DG = D / 8, TSW = 64 / DG;   // values: dim groups of 8, tokens per wave step
    constexpr int SPT = 16 / TSW;              // value steps per tile
    constexpr int SMAX = 4 * SPT;              // value steps per wave (at most 4 tiles)
    constexpr int VR = D == 64 ? 16 : 8;       // value loads in flight per lane
    constexpr int VB = SMAX < VR ? SMAX : VR;
    constexpr int TPB = VB / SPT;              // tiles per batch of value loads
    constexpr int VST = D + 4;                 // LDS row stride of a staged V tile, halves (conflict-free reads)
    // LDS sized by the call's group G: probabilities [NW][G][64] (a wave's own
    // tokens), wave max and sum [NW][G] each, the split's block ids
    // [ATT_TS + 1], each wave's staged V tile [16][VST] halves (the output sum
    // [G][D] floats reuses that area once every wave is done with it)
    extern __shared__ float smem[];
    const int G = a.G;
    float *const pw = smem;
    float *const wmx = pw + NW * G * 64;
    float *const wsum = wmx + NW * G;
    int *const pbl = reinterpret_cast<int *>(wsum + NW * G);
    _Float16 *const vts = reinterpret_cast<_Float16 *>(pbl + ATT_TS + 4);
    float *const acc = reinterpret_cast<float *>(vts);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // the KV heads of one (sequence, split) are neighbours in the grid: they
    // read the same pool blocks (a token's heads share one contiguous row)
    const int hk = blockIdx.x % a.n_kv;
    const int split = (blockIdx.x / a.n_kv) % a.nsplit;
    const int b = blockIdx.x / (a.nsplit * a.n_kv);
    const int bs = a.block_size, t0 = split * a.ts;
    // the block ids of the split's whole range, clamped into the pool (an id
    // outside it is the caller's error, never an access outside the buffer);
    // loaded before the length is known, so the two loads overlap
    const int blk0 = a.bs_shift >= 0 ? t0 >> a.bs_shift : t0 / bs;
    const int wu = __builtin_amdgcn_readfirstlane(w);
    int pbt[4];                                // FAST: the block of each of the wave's tiles
    if constexpr (FAST) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int blk = min((t0 + 16 * (wu + NW * q)) >> a.bs_shift, a.max_blocks - 1);
            const int pb = a.block_tables[(int64_t)b * a.max_blocks + blk];
            pbt[q] = pb < 0 ? 0 : (pb >= a.num_blocks ? (int)(a.num_blocks - 1) : pb);
        }
    } else {
        const int last = t0 + a.ts - 1;
        const int nblk = min(a.bs_shift >= 0 ? last >> a.bs_shift : last / bs, a.max_blocks - 1) - blk0 + 1;
        for (int i = tid; i < nblk; i += ATT_NT) {
            const int pb = a.block_tables[(int64_t)b * a.max_blocks + blk0 + i];
            pbl[i] = pb < 0 ? 0 : (pb >= a.num_blocks ? (int)(a.num_blocks - 1) : pb);
        }
    }
    // lengths beyond the block table are clamped to it
    const int L = min(max(a.seq_lens[b], 0), a.max_blocks * a.block_size);
    const int t1 = min(t0 + a.ts, L), n = t1 - t0;
    if (n <= 0 && a.nsplit > 1) return;        // past the sequence: the merge reads no such split
    const int64_t hoff = (int64_t)hk * D;      // the KV head within a token's row
    const int64_t rowst = (int64_t)a.n_kv * D; // token stride within a block
    // the newest token: its K and V come from the inputs
    const __half *nk = a.new_k + ((int64_t)b * a.n_kv + hk) * D;
    const __half *nv = a.new_v + ((int64_t)b * a.n_kv + hk) * D;
    if (n > 0 && L - 1 < t1) {
        const int wb = a.write_info[2 * b], wp = a.write_info[2 * b + 1];
        if (wb >= 0 && wb < a.num_blocks && wp >= 0 && wp < bs) {
            __half *dk = a.pool + (int64_t)wb * a.s0 + wp * rowst + hoff;
            for (int d = tid; d < D; d += ATT_NT) { dk[d] = nk[d]; dk[a.s1 + d] = nv[d]; }
        }
    }
    // scores: lane l is query head / token column l % 16 and quarter l / 16 of the dims
    const int col = lane & 15, qd = lane >> 4;
    half4_t qa[NM];
    {
        uint4 r[QV];
        if (col < G) {
            const __half *qp = a.queries + ((int64_t)b * a.n_heads + hk * G + col) * D + qd * (D / 4);
#pragma unroll
            for (int v = 0; v < QV; ++v) r[v] = reinterpret_cast<const uint4 *>(qp)[v];
        } else {
#pragma unroll
            for (int v = 0; v < QV; ++v) r[v] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int m = 0; m < NM; ++m)
            qa[m] = (m & 1) ? half4_of(r[m >> 1].z, r[m >> 1].w) : half4_of(r[m >> 1].x, r[m >> 1].y);
    }
    if constexpr (!FAST) __syncthreads();      // the staged block ids
    // wave w owns tiles w, w + NW, w + 2 NW, w + 3 NW of 16 tokens.  A lane
    // whose token is past the split's end reads the tile's last token instead
    // (its score is masked and its values zeroed); the newest token is read
    // from the inputs.
    const int ntiles = (n + 15) >> 4;
    const int inew = L - 1 >= t0 && L - 1 < t1 ? L - 1 - t0 : -1;
    const __half *tb[4];                       // FAST: tile j's K rows (the tile lies in one block)
    if constexpr (FAST) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int tok0 = t0 + 16 * (wu + NW * q);
            tb[q] = a.pool + (int64_t)pbt[q] * a.s0 + (int64_t)(tok0 & (bs - 1)) * rowst + hoff;
        }
    }
    // the K (kv = 0) or V (kv = 1) row of token 16 j + loc of the wave's tile q
    auto row_ptr = [&](int q, int loc, int kv) -> const __half * {
        const int j = w + NW * q;
        const int c2 = min(loc, n - 16 * j - 1);
        const __half *p;
        if constexpr (FAST) {
            p = tb[q] + c2 * (int)rowst + (kv ? a.s1 : 0);
        } else {
            const int t = t0 + 16 * j + c2;
            const int qb = a.bs_shift >= 0 ? t >> a.bs_shift : t / bs;
            p = a.pool + (int64_t)pbl[qb - blk0] * a.s0 + (int64_t)(t - qb * bs) * rowst + hoff + (kv ? a.s1 : 0);
        }
        if (inew >= 16 * j && inew < 16 * j + 16) {   // wave-uniform
            if (16 * j + c2 == inew) p = kv ? nv : nk;
        }
        return p;
    };
    // values: lane = (token sub, dim group); step s of the wave takes token
    // (s % SPT) TSW + sub of its tile s / SPT
    const int dg = lane % DG, sub = lane / DG;
    auto load_v = [&](int s) -> uint4 {
        const int q = s / SPT, j = w + NW * q, loc = (s % SPT) * TSW + sub;
        if (j >= ntiles) return make_uint4(0u, 0u, 0u, 0u);   // wave-uniform
        uint4 r = reinterpret_cast<const uint4 *>(row_ptr(q, loc, 1))[dg];
        if (n - 16 * j < 16) {                 // wave-uniform: the split's last, partial tile
            if (loc >= n - 16 * j) r = make_uint4(0u, 0u, 0u, 0u);
        }
        return r;
    };
    float4_t c[4];
    uint4 vr[VB];
#pragma unroll
    for (int kb = 0; kb < 4; kb += KT) {
        uint4 kr[KT][QV];
#pragma unroll
        for (int q = 0; q < KT; ++q) {
            if (w + NW * (kb + q) < ntiles) {  // wave-uniform
                const __half *kp = row_ptr(kb + q, col, 0) + qd * (D / 4);
#pragma unroll
                for (int v = 0; v < QV; ++v) kr[q][v] = reinterpret_cast<const uint4 *>(kp)[v];
            }
        }
        if (kb == 0) {                         // the first values in flight with the keys
#pragma unroll
            for (int u = 0; u < VB; ++u) vr[u] = load_v(u);
        }
#pragma unroll
        for (int q = 0; q < KT; ++q) {
            float4_t cc = {0.0f, 0.0f, 0.0f, 0.0f};
            if (w + NW * (kb + q) < ntiles) {  // wave-uniform
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    const uint4 &r = kr[q][m >> 1];
                    const half4_t kv = (m & 1) ? half4_of(r.z, r.w) : half4_of(r.x, r.y);
                    cc = __builtin_amdgcn_mfma_f32_16x16x16f16(qa[m], kv, cc, 0, 0, 0);
                }
            }
            c[kb + q] = cc;
        }
    }
    // the second batch of values in flight through the softmax (the keys' registers are free)
    uint4 vr2[VB];
    if constexpr (SMAX > VB) {
#pragma unroll
        for (int u = 0; u < VB; ++u) vr2[u] = load_v(VB + u);
    }
    // the wave's softmax: c[q][r] is query head 4 qd + r, token 16 (w + NW q) + col
    float mloc[4], lsum[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float m = -INFINITY;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (16 * (w + NW * q) + col < n) m = fmaxf(m, c[q][r] * a.scale);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        mloc[r] = m;
        lsum[r] = 0.0f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const bool ok = 16 * (w + NW * q) + col < n;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = ok ? __expf(c[q][r] * a.scale - mloc[r]) : 0.0f;
            lsum[r] += e;
            const int g = 4 * qd + r;
            if (g < G) pw[(w * G + g) * 64 + 16 * q + col] = e;
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) lsum[r] += __shfl_xor(lsum[r], o, 64);
        const int g = 4 * qd + r;
        if (col == 0 && g < G) { wmx[w * G + g] = mloc[r]; wsum[w * G + g] = lsum[r]; }
    }
    __syncthreads();
    // weighted V sum on the matrix cores, one tile at a time: the wave stages
    // the tile's V rows in LDS, then per 16 dims out[g][d] += P[g][k] V[k][d]
    // over the 16 tokens k (v_mfma_f32_16x16x16_f16: A = P with the query
    // heads as rows, B = V read back column-wise).  P is split into fp16
    // hi + lo parts, both multiplied: hi + lo is within 2^-22 p of p and the
    // fp16 products are exact, so the sum keeps fp32 accuracy.
    _Float16 *const vt = vts + w * 16 * VST;
    float4_t oacc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) oacc[m] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // one batch of VB value steps (TPB tiles) from registers
    auto pv_batch = [&](const uint4 *vb_, int s0) {
#pragma unroll
        for (int t = 0; t < TPB; ++t) {
            const int q = s0 / SPT + t;
            if (w + NW * q < ntiles) {         // wave-uniform
#pragma unroll
                for (int k = 0; k < SPT; ++k) {
                    const uint4 r = vb_[t * SPT + k];
                    uint2 *dst = reinterpret_cast<uint2 *>(vt + (k * TSW + sub) * VST + dg * 8);
                    dst[0] = make_uint2(r.x, r.y);
                    dst[1] = make_uint2(r.z, r.w);
                }
                wave_lds_sync();
                float4 pp = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (col < G) pp = *reinterpret_cast<const float4 *>(&pw[(w * G + col) * 64 + 16 * q + 4 * qd]);
                const half4_t ph = {(_Float16)pp.x, (_Float16)pp.y, (_Float16)pp.z, (_Float16)pp.w};
                const half4_t pl = {(_Float16)(pp.x - (float)ph[0]), (_Float16)(pp.y - (float)ph[1]),
                                    (_Float16)(pp.z - (float)ph[2]), (_Float16)(pp.w - (float)ph[3])};
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    const _Float16 *src = vt + 4 * qd * VST + 16 * m + col;
                    const half4_t vb = {src[0], src[VST], src[2 * VST], src[3 * VST]};
                    oacc[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, oacc[m], 0, 0, 0);
                    oacc[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vb, oacc[m], 0, 0, 0);
                }
                wave_lds_sync();
            }
        }
    };
    // batches alternate between the two register sets; the next load of a
    // set is issued as soon as it has been consumed
    pv_batch(vr, 0);
    if constexpr (SMAX > VB) {
        if constexpr (SMAX > 2 * VB) {
#pragma unroll
            for (int u = 0; u < VB; ++u) vr[u] = load_v(2 * VB + u);
        }
        pv_batch(vr2, VB);
        if constexpr (SMAX > 3 * VB) {
#pragma unroll
            for (int u = 0; u < VB; ++u) vr2[u] = load_v(3 * VB + u);
        }
        if constexpr (SMAX > 2 * VB) pv_batch(vr, 2 * VB);
        if constexpr (SMAX > 3 * VB) pv_batch(vr2, 3 * VB);
    }
    static_assert(SMAX <= 4 * VB, "at most four batches of values");
    // oacc[m][r] is query head 4 qd + r, dim 16 m + col.  The waves add in
    // turn, each rescaled from its own max to the split's.
    __syncthreads();                           // every wave is done with the staged tiles
    for (int k = 0; k < NW; ++k) {
        if (w == k) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int g = 4 * qd + r;
                if (g < G) {
                    float M = wmx[g];
#pragma unroll
                    for (int x = 1; x < NW; ++x) M = fmaxf(M, wmx[x * G + g]);
                    const float mw = wmx[k * G + g];
                    const float sc = mw == -INFINITY ? 0.0f : __expf(mw - M);
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        float *const cp = &acc[g * D + 16 * m + col];
                        *cp = k == 0 ? sc * oacc[m][r] : fmaf(sc, oacc[m][r], *cp);
                    }
                }
            }
        }
        __syncthreads();
    }
    // write the split (or, with one split, the output)
    for (int i = tid; i < G * D; i += ATT_NT) {
        const int g = i / D, d = i % D;
        float M = wmx[g];
#pragma unroll
        for (int x = 1; x < NW; ++x) M = fmaxf(M, wmx[x * G + g]);
        float l = 0.0f;
#pragma unroll
        for (int x = 0; x < NW; ++x) {
            const float mw = wmx[x * G + g];
            if (mw != -INFINITY) l = fmaf(__expf(mw - M), wsum[x * G + g], l);
        }
        const float v = acc[i];
        const int hq = hk * G + g;
        if (a.nsplit == 1) {
            a.out[((int64_t)b * a.n_heads + hq) * D + d] = __float2half(n > 0 ? v / l : 0.0f);
        } else {
            const int64_t ps = ((int64_t)b * a.n_heads + hq) * a.nsplit + split;
            a.part[ps * D + d] = v;
            if (d == 0) { a.pm[ps] = M; a.pl[ps] = l; }
        }
    }
}

// One wave per (sequence, query head): the splits' max-rescaled sum.  Lanes
// take splits for the max and the weights exp(m_s - M), which the wave then
// shares by shuffles while each lane sums its dims over the splits.
template <int D>
__global__ __launch_bounds__(ATT_NT) void k_attn_merge(AttnArgs a, int64_t pairs)
{
    constexpr int DPL = D / 64;
    const int lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * ATT_NW + (threadIdx.x >> 6);
    if (pair >= pairs) return;                 // whole waves
    const int64_t b = pair / a.n_heads;
    const int L = min(max(a.seq_lens[b], 0), a.max_blocks * a.block_size);
    const int ns = min(a.nsplit, (L + a.ts - 1) / a.ts);
    const int64_t base = pair * a.nsplit;
    float M = -INFINITY;
    for (int s = lane; s < ns; s += 64) M = fmaxf(M, a.pm[base + s]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    float Ls = 0.0f, v[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) v[j] = 0.0f;
    for (int c0 = 0; c0 < ns; c0 += 64) {
        const int s = c0 + lane;
        const float wgt = s < ns ? __expf(a.pm[base + s] - M) : 0.0f;
        if (s < ns) Ls += wgt * a.pl[base + s];
        const int nk = min(64, ns - c0);
        const float *pp = a.part + (base + c0) * D + lane;
        int k = 0;
        for (; k + 4 <= nk; k += 4) {
            float x[4][DPL];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < DPL; ++j) x[u][j] = pp[(int64_t)(k + u) * D + j * 64];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float wk = __shfl(wgt, k + u, 64);
#pragma unroll
                for (int j = 0; j < DPL; ++j) v[j] = fmaf(wk, x[u][j], v[j]);
            }
        }
        for (; k < nk; ++k) {
            const float wk = __shfl(wgt, k, 64);
#pragma unroll
            for (int j = 0; j < DPL; ++j) v[j] = fmaf(wk, pp[(int64_t)k * D + j * 64], v[j]);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) Ls += __shfl_xor(Ls, o, 64);
#pragma unroll
    for (int j = 0; j < DPL; ++j)
        a.out[pair * D + j * 64 + lane] = __float2half(ns > 0 ? v[j] / Ls : 0.0f);
}

// The pool gather: one thread per (sequence, token, KV head, dim), zero past
// the sequence's length.
__global__ __launch_bounds__(ATT_NT) void k_gather(const __half *pool, int64_t num_blocks, int64_t s0, int64_t s1, int block_size,
                                                   int n_kv, int D, int max_blocks, const int32_t *block_tables,
                                                   const int32_t *seq_lens, int max_seq, int64_t total,
                                                   __half *out_k, __half *out_v)
{
    const int64_t i = (int64_t)blockIdx.x * ATT_NT + threadIdx.x;
    if (i >= total) return;
    const int d = (int)(i % D);
    const int h = (int)((i / D) % n_kv);
    const int t = (int)((i / ((int64_t)D * n_kv)) % max_seq);
    const int64_t b = i / ((int64_t)D * n_kv * max_seq);
    if (t >= seq_lens[b] || t >= max_blocks * block_size) {   // past the sequence (or its block table)
        out_k[i] = __float2half(0.0f); out_v[i] = __float2half(0.0f); return;
    }
    int pb = block_tables[b * max_blocks + t / block_size];
    pb = pb < 0 ? 0 : (pb >= num_blocks ? (int)(num_blocks - 1) : pb);
    const int64_t src = (int64_t)pb * s0 + ((int64_t)(t % block_size) * n_kv + h) * D + d;
    out_k[i] = pool[src];
    out_v[i] = pool[src + s1];
}

template <int D>
hipError_t launch_attn(const AttnArgs &a, int64_t B, hipStream_t st)
{
    // probabilities, wave max and sum, block ids, staged V tiles (and the
    // output sum after them): at most 50 KiB
    const size_t lds = ((size_t)a.G * (ATT_NW * 64 + 2 * ATT_NW) + ATT_TS + 4) * sizeof(float) +
                       (size_t)ATT_NW * 16 * (D + 4) * sizeof(uint16_t);
    // block sizes that are powers of two from 16 up hold whole 16-token tiles
    if (a.bs_shift >= 4)
        hipLaunchKernelGGL((k_attn_split<D, true>), dim3((unsigned)(B * a.n_kv * a.nsplit)), dim3(ATT_NT), lds, st, a);
    else
        hipLaunchKernelGGL((k_attn_split<D, false>), dim3((unsigned)(B * a.n_kv * a.nsplit)), dim3(ATT_NT), lds, st, a);
    if (a.nsplit > 1) {
        const int64_t pairs = B * a.n_heads;
        hipLaunchKernelGGL((k_attn_merge<D>), dim3((unsigned)((pairs + ATT_NW - 1) / ATT_NW)), dim3(ATT_NT), 0, st, a,
                           pairs);
    }
    return hipGetLastError();
}

// Tokens per split: 256, halved (down to 64) while the grid would hold fewer
// than ATT_FILL workgroups.
int split_tokens(int64_t B, int n_kv, int64_t max_context)
{
    int ts = ATT_TS;
    while (ts > 64 && B * n_kv * ((max_context + ts - 1) / ts) < ATT_FILL) ts >>= 1;
    return ts;
}

}  // namespace
}  // namespace mis

extern "C" {

size_t mis_paged_attention_workspace_bytes(int64_t B, int n_heads, int n_kv_heads, int d_k, int max_context)
{
    if (B <= 0 || n_heads <= 0 || n_kv_heads <= 0 || d_k <= 0 || max_context <= 0) return 256;
    const int ts = mis::split_tokens(B, n_kv_heads, max_context);
    const int64_t ns = (max_context + ts - 1) / ts;
    if (ns <= 1) return 256;
    const size_t n = (size_t)B * (size_t)n_heads * (size_t)ns;
    return ((n * (size_t)d_k + 2 * n) * sizeof(float) + 255) & ~(size_t)255;
}

int mis_paged_attention(void *pool, int64_t num_blocks, int block_size, int n_kv_heads, int d_k, int64_t pool_stride0,
                        int64_t pool_stride1, const void *new_k, const void *new_v, const void *queries,
                        const int32_t *block_tables, int max_blocks, const int32_t *seq_lens,
                        const int32_t *write_info, int64_t B, int n_heads, void *out, void *workspace,
                        size_t workspace_bytes, void *stream)
{
    using namespace mis;
    if (B < 0 || num_blocks <= 0 || block_size <= 0 || n_kv_heads <= 0 || n_heads <= 0 || max_blocks <= 0)
        return MIS_ATT_ERR_INVALID_ARG;
    if (B == 0) return MIS_ATT_OK;
    if (!pool || !new_k || !new_v || !queries || !block_tables || !seq_lens || !write_info || !out)
        return MIS_ATT_ERR_INVALID_ARG;
    if (n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > ATT_GMAX) return MIS_ATT_ERR_UNSUPPORTED;
    if (d_k != 64 && d_k != 128 && d_k != 256) return MIS_ATT_ERR_UNSUPPORTED;
    if (B > 0x7fffffff / ((int64_t)n_heads * 64)) return MIS_ATT_ERR_UNSUPPORTED;
    if (((uintptr_t)pool & 15u) || (pool_stride0 & 7) || (pool_stride1 & 7) || ((uintptr_t)new_k & 15u) ||
        ((uintptr_t)new_v & 15u) || ((uintptr_t)queries & 15u))
        return MIS_ATT_ERR_INVALID_ARG;  // 16-byte rows for the vector loads
    const int64_t max_context = (int64_t)max_blocks * block_size;
    if (max_context > (int64_t)1 << 24) return MIS_ATT_ERR_UNSUPPORTED;
    if ((int64_t)block_size * n_kv_heads * d_k >= (int64_t)1 << 31) return MIS_ATT_ERR_UNSUPPORTED;  // 32-bit offsets in a block
    AttnArgs a;
    a.pool = reinterpret_cast<__half *>(pool);
    a.s0 = pool_stride0; a.s1 = pool_stride1; a.num_blocks = num_blocks;
    a.block_size = block_size; a.n_kv = n_kv_heads; a.n_heads = n_heads; a.G = n_heads / n_kv_heads;
    a.max_blocks = max_blocks;
    a.new_k = reinterpret_cast<const __half *>(new_k);
    a.new_v = reinterpret_cast<const __half *>(new_v);
    a.queries = reinterpret_cast<const __half *>(queries);
    a.block_tables = block_tables; a.seq_lens = seq_lens; a.write_info = write_info;
    a.out = reinterpret_cast<__half *>(out);
    a.ts = split_tokens(B, n_kv_heads, max_context);
    a.nsplit = (int)((max_context + a.ts - 1) / a.ts);
    if (B * n_kv_heads * (int64_t)a.nsplit > 0x7fffffff) return MIS_ATT_ERR_UNSUPPORTED;
    a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
    a.scale = 1.0f / sqrtf((float)d_k);
    a.part = nullptr; a.pm = nullptr; a.pl = nullptr;
    if (a.nsplit > 1) {
        const size_t need = mis_paged_attention_workspace_bytes(B, n_heads, n_kv_heads, d_k, (int)max_context);
        if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)) return MIS_ATT_ERR_WORKSPACE;
        const size_t n = (size_t)B * (size_t)n_heads * (size_t)a.nsplit;
        a.part = reinterpret_cast<float *>(workspace);
        a.pm = a.part + n * (size_t)d_k;
        a.pl = a.pm + n;
    }
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    if (d_k == 64) e = launch_attn<64>(a, B, st);
    else if (d_k == 128) e = launch_attn<128>(a, B, st);
    else e = launch_attn<256>(a, B, st);
    return e == hipSuccess ? MIS_ATT_OK : MIS_ATT_ERR_HIP;
}

int mis_gather_kv(const void *pool, int64_t num_blocks, int block_size, int n_kv_heads, int d_k, int64_t pool_stride0,
                  int64_t pool_stride1, const int32_t *block_tables, int max_blocks, const int32_t *seq_lens,
                  int64_t B, int max_seq_len, void *out_k, void *out_v, void *stream)
{
    if (B < 0 || num_blocks <= 0 || block_size <= 0 || n_kv_heads <= 0 || d_k <= 0 || max_blocks <= 0 || max_seq_len < 0)
        return MIS_ATT_ERR_INVALID_ARG;
    if (B == 0 || max_seq_len == 0) return MIS_ATT_OK;
    if (!pool || !block_tables || !seq_lens || !out_k || !out_v) return MIS_ATT_ERR_INVALID_ARG;
    const int64_t total = B * (int64_t)max_seq_len * n_kv_heads * d_k;
    if (total / mis::ATT_NT + 1 > 0x7fffffff) return MIS_ATT_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(mis::k_gather, dim3((unsigned)((total + mis::ATT_NT - 1) / mis::ATT_NT)), dim3(mis::ATT_NT), 0,
                       (hipStream_t)stream, reinterpret_cast<const __half *>(pool), num_blocks, pool_stride0, pool_stride1,
                       block_size, n_kv_heads, d_k, max_blocks, block_tables, seq_lens, max_seq_len, total,
                       reinterpret_cast<__half *>(out_k), reinterpret_cast<__half *>(out_v));
    return hipGetLastError() == hipSuccess ? MIS_ATT_OK : MIS_ATT_ERR_HIP;
}

}  // extern "C"
