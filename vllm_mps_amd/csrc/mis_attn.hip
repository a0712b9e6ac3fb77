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
    float scale;
};

__device__ __forceinline__ half4_t half4_of(unsigned int lo, unsigned int hi)
{
    const u32x2_t v = {lo, hi};
    return __builtin_bit_cast(half4_t, v);
}

__device__ __forceinline__ void h8_to_f(const uint4 &r, float *f)
{
    const __half2 *h = reinterpret_cast<const __half2 *>(&r);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float2 x = __half22float2(h[e]);
        f[2 * e] = x.x;
        f[2 * e + 1] = x.y;
    }
}

// Physical block of token t (clamped into the pool: an id outside it is the
// caller's error, never an access outside the buffer).
__device__ __forceinline__ int block_of(const AttnArgs &a, int b, int t)
{
    const int pb = a.block_tables[(int64_t)b * a.max_blocks + t / a.block_size];
    return pb < 0 ? 0 : (pb >= a.num_blocks ? (int)(a.num_blocks - 1) : pb);
}

template <int D, int GM>
__global__ __launch_bounds__(ATT_NT) void k_attn_split(AttnArgs a)
{
    constexpr int NW = ATT_NW;
    constexpr int QV = D / 32;                 // 16-byte K loads per lane per tile (a quarter row)
    constexpr int NM = D / 16;                 // MFMAs per tile
    constexpr int TPI = D == 256 ? 2 : 4;      // tiles in flight per wave
    constexpr int DG = D / 8, TSW = 64 / DG;   // values phase: dim groups, tokens per wave step
    constexpr int U = D == 256 ? 4 : 8;        // values phase: tokens in flight per lane
    // LDS sized by the call's group G: probabilities [G][ATT_TS], per-wave
    // reductions [G][NW], split max [G], output sum [G][D], block ids [ATT_TS]
    extern __shared__ float smem[];
    const int G = a.G;
    float *const pr = smem;
    float *const red = pr + G * ATT_TS;
    float *const mx = red + G * NW;
    float *const acc = mx + G;
    int *const pbl = reinterpret_cast<int *>(acc + G * D);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int split = blockIdx.x % a.nsplit;
    const int hk = (blockIdx.x / a.nsplit) % a.n_kv;
    const int b = blockIdx.x / (a.nsplit * a.n_kv);
    // lengths beyond the block table are clamped to it
    const int L = min(max(a.seq_lens[b], 0), a.max_blocks * a.block_size);
    const int t0 = split * a.ts, t1 = min(t0 + a.ts, L), n = t1 - t0;
    if (n <= 0 && a.nsplit > 1) return;        // past the sequence: the merge reads no such split
    const int64_t hoff = (int64_t)hk * D;      // the KV head within a token's row
    const int64_t rowst = (int64_t)a.n_kv * D; // token stride within a block
    // the newest token: its K and V come from the inputs
    const __half *nk = a.new_k + ((int64_t)b * a.n_kv + hk) * D;
    const __half *nv = a.new_v + ((int64_t)b * a.n_kv + hk) * D;
    if (n > 0 && L - 1 < t1) {
        const int wb = a.write_info[2 * b], wp = a.write_info[2 * b + 1];
        if (wb >= 0 && wb < a.num_blocks && wp >= 0 && wp < a.block_size) {
            __half *dk = a.pool + (int64_t)wb * a.s0 + wp * rowst + hoff;
            for (int d = tid; d < D; d += ATT_NT) { dk[d] = nk[d]; dk[a.s1 + d] = nv[d]; }
        }
    }
    // scores.  Lane l: query head / token column l % 16, quarter l / 16 of the dims.
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
    const int ntiles = (n + 15) >> 4;
    for (int j0 = w * TPI; j0 < ntiles; j0 += NW * TPI) {
        uint4 kr[TPI][QV];
#pragma unroll
        for (int jj = 0; jj < TPI; ++jj) {
            const int i = (j0 + jj) * 16 + col, t = t0 + i;
            if (i < n) {
                const __half *kp;
                if (t == L - 1) {
                    kp = nk;
                } else {
                    const int pb = block_of(a, b, t);
                    kp = a.pool + (int64_t)pb * a.s0 + (t % a.block_size) * rowst + hoff;
                }
                if (qd == 0) pbl[i] = t == L - 1 ? -1 : block_of(a, b, t);
                kp += qd * (D / 4);
#pragma unroll
                for (int v = 0; v < QV; ++v) kr[jj][v] = reinterpret_cast<const uint4 *>(kp)[v];
            } else {
#pragma unroll
                for (int v = 0; v < QV; ++v) kr[jj][v] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
#pragma unroll
        for (int jj = 0; jj < TPI; ++jj) {
            if (j0 + jj >= ntiles) continue;   // wave-uniform
            float4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint4 &r = kr[jj][m >> 1];
                const half4_t kb = (m & 1) ? half4_of(r.z, r.w) : half4_of(r.x, r.y);
                c = __builtin_amdgcn_mfma_f32_16x16x16f16(qa[m], kb, c, 0, 0, 0);
            }
            // c[r]: query head 4 * qd + r, token (j0 + jj) * 16 + col
            const int i = (j0 + jj) * 16 + col;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int g = 4 * qd + r;
                if (g < G) pr[g * ATT_TS + i] = i < n ? c[r] * a.scale : -INFINITY;
            }
        }
    }
    __syncthreads();
    // softmax per query head over the split: max, then exp and sum
    for (int g = 0; g < G; ++g) {
        float v = tid < n ? pr[g * ATT_TS + tid] : -INFINITY;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
        if (lane == 0) red[g * NW + w] = v;
    }
    __syncthreads();
    if (tid < G) {
        float m = red[tid * NW];
#pragma unroll
        for (int i = 1; i < NW; ++i) m = fmaxf(m, red[tid * NW + i]);
        mx[tid] = m;
    }
    __syncthreads();
    for (int g = 0; g < G; ++g) {
        const float e = tid < n ? __expf(pr[g * ATT_TS + tid] - mx[g]) : 0.0f;
        if (tid < n) pr[g * ATT_TS + tid] = e;
        float v = e;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) red[g * NW + w] = v;
    }
    __syncthreads();
    // weighted V sum: lane = (token sub, dim group); wave w, step k takes
    // tokens (k * NW + w) * TSW + sub
    const int dg = lane % DG, sub = lane / DG;
    float o[GM][8];
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
    for (int i0 = w * TSW + sub; i0 < n; i0 += NW * TSW * U) {
        uint4 vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + u * NW * TSW;
            if (i < n) {
                const int pb = pbl[i];
                const __half *vp = pb < 0 ? nv
                                          : a.pool + (int64_t)pb * a.s0 + a.s1 + ((t0 + i) % a.block_size) * rowst + hoff;
                vr[u] = reinterpret_cast<const uint4 *>(vp)[dg];
            } else {
                vr[u] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + u * NW * TSW;
            if (i < n) {
                float v[8];
                h8_to_f(vr[u], v);
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    if (g < G) {
                        const float pg = pr[g * ATT_TS + i];
#pragma unroll
                        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pg, v[e], o[g][e]);
                    }
            }
        }
    }
    // lanes sharing a dim group, then the waves one at a time
#pragma unroll
    for (int sft = DG; sft < 64; sft <<= 1)
#pragma unroll
        for (int g = 0; g < GM; ++g)
            if (g < G)
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] += __shfl_xor(o[g][e], sft, 64);
    for (int k = 0; k < NW; ++k) {
        if (w == k && sub == 0) {
#pragma unroll
            for (int g = 0; g < GM; ++g)
                if (g < G)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        float *const c = &acc[g * D + dg * 8 + e];
                        *c = k == 0 ? o[g][e] : *c + o[g][e];
                    }
        }
        __syncthreads();
    }
    // write the split (or, with one split, the output); red holds the per-wave sums
    for (int i = tid; i < G * D; i += ATT_NT) {
        const float v = acc[i];
        const int g = i / D, d = i % D;
        float l = 0.0f;
#pragma unroll
        for (int k = 0; k < NW; ++k) l += red[g * NW + k];
        const int hq = hk * G + g;
        if (a.nsplit == 1) {
            a.out[((int64_t)b * a.n_heads + hq) * D + d] = __float2half(n > 0 ? v / l : 0.0f);
        } else {
            const int64_t ps = ((int64_t)b * a.n_heads + hq) * a.nsplit + split;
            a.part[ps * D + d] = v;
            if (d == 0) { a.pm[ps] = mx[g]; a.pl[ps] = l; }
        }
    }
}

// One workgroup per (sequence, query head): the splits' max-rescaled sum.
template <int D>
__global__ __launch_bounds__(ATT_NT) void k_attn_merge(AttnArgs a)
{
    const int hq = blockIdx.x % a.n_heads, b = blockIdx.x / a.n_heads;
    const int L = min(max(a.seq_lens[b], 0), a.max_blocks * a.block_size);
    const int ns = min(a.nsplit, (L + a.ts - 1) / a.ts);
    const int64_t base = ((int64_t)b * a.n_heads + hq) * a.nsplit;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, a.pm[base + s]);
    float Ls = 0.0f;
    for (int s = 0; s < ns; ++s) Ls += a.pl[base + s] * __expf(a.pm[base + s] - M);
    for (int d = threadIdx.x; d < D; d += ATT_NT) {
        float v = 0.0f;
        for (int s = 0; s < ns; ++s) v += a.part[(base + s) * D + d] * __expf(a.pm[base + s] - M);
        a.out[((int64_t)b * a.n_heads + hq) * D + d] = __float2half(ns > 0 ? v / Ls : 0.0f);
    }
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

template <int D, int GM>
hipError_t launch_attn(const AttnArgs &a, int64_t B, hipStream_t st)
{
    // probabilities, reductions, max, output sum, block ids: at most 34 KiB
    const size_t lds = ((size_t)a.G * (ATT_TS + ATT_NW + 1 + D) + ATT_TS) * sizeof(float);
    hipLaunchKernelGGL((k_attn_split<D, GM>), dim3((unsigned)(B * a.n_kv * a.nsplit)), dim3(ATT_NT), lds, st, a);
    if (a.nsplit > 1) hipLaunchKernelGGL((k_attn_merge<D>), dim3((unsigned)(B * a.n_heads)), dim3(ATT_NT), 0, st, a);
    return hipGetLastError();
}

template <int D>
hipError_t launch_attn_d(const AttnArgs &a, int64_t B, hipStream_t st)
{
    if (a.G <= 4) return launch_attn<D, 4>(a, B, st);
    if (a.G <= 8) return launch_attn<D, 8>(a, B, st);
    return launch_attn<D, 16>(a, B, st);
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
    if (d_k == 64) e = launch_attn_d<64>(a, B, st);
    else if (d_k == 128) e = launch_attn_d<128>(a, B, st);
    else e = launch_attn_d<256>(a, B, st);
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
