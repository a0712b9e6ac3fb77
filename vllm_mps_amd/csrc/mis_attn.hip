// mis_attn.hip -- decode-step paged attention over an fp16 KV block pool, and
// the pool gather (include/mis_attention.h).
//
// Pool layout, as the reference engine allocates it
// (memory/mps_memory_pool.py:62): [num_blocks, 2 (K, V), block_size,
// n_kv_heads, d_k] fp16, element strides pool_stride0 (block) and
// pool_stride1 (K -> V).  Token t of sequence b lives in physical block
// block_tables[b * max_blocks + t / block_size] at position t % block_size.
//
// k_attn_split: one workgroup of 256 threads per (sequence, KV head, context
// split of ATT_TS tokens).  It serves every query head of that KV head (GQA),
// so each K and V row is read once per group.  Scores take one token per
// thread (its K row as 16-byte vectors against the queries in LDS); softmax
// per query head over the split; the weighted V sum takes one dimension per
// lane (V rows read coalesced), the waves splitting the tokens.  A split
// writes its unnormalised output with its max and sum; a context of one split
// writes the final fp16 output directly.  k_attn_merge combines the splits
// (the usual max-rescaled sums).
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
constexpr int ATT_TS = 256;          // tokens per split (one per thread in the score phase)
constexpr int ATT_GMAX = 16;         // query heads per KV head, at most

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
    int nsplit;
    float scale;
};

__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }

template <int D>
__global__ __launch_bounds__(ATT_NT) void k_attn_split(AttnArgs a)
{
    constexpr int NW = ATT_NT / 64, VPL = D / 64;  // dims per lane in the V phase
    // LDS sized by the call's group G: queries [G][D] (reused for the output
    // sum once the scores are done), probabilities [G][ATT_TS], reductions [G][NW]
    extern __shared__ float smem[];
    float *const q = smem, *const acc = smem;
    float *const pr = smem + a.G * D;
    float *const red = pr + a.G * ATT_TS;
    float *const mx = red + a.G * NW;                  // per-head split max
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int split = blockIdx.x % a.nsplit;
    const int hk = (blockIdx.x / a.nsplit) % a.n_kv;
    const int b = blockIdx.x / (a.nsplit * a.n_kv);
    const int G = a.G;
    // lengths beyond the block table and block ids beyond the pool are clamped
    // into range: they are the caller's error, never an access outside the buffers
    const int L = min(max(a.seq_lens[b], 0), a.max_blocks * a.block_size);
    const int t0 = split * ATT_TS, t1 = min(t0 + ATT_TS, L);
    // the newest token: its K and V come from the inputs
    const __half *nk = a.new_k + ((int64_t)b * a.n_kv + hk) * D;
    const __half *nv = a.new_v + ((int64_t)b * a.n_kv + hk) * D;
    if (L >= 1 && t0 <= L - 1 && L - 1 < t0 + ATT_TS) {
        const int wb = a.write_info[2 * b], wp = a.write_info[2 * b + 1];
        if (wb >= 0 && wb < a.num_blocks && wp >= 0 && wp < a.block_size) {
            __half *dk = a.pool + (int64_t)wb * a.s0 + ((int64_t)wp * a.n_kv + hk) * D;
            for (int d = tid; d < D; d += ATT_NT) { dk[d] = nk[d]; dk[a.s1 + d] = nv[d]; }
        }
    }
    for (int i = tid; i < G * D; i += ATT_NT) {
        const int g = i / D, d = i % D;
        q[i] = h2f(a.queries[((int64_t)b * a.n_heads + hk * G + g) * D + d]);
    }
    __syncthreads();
    auto row_of = [&](int t) -> const __half * {
        int pb = a.block_tables[(int64_t)b * a.max_blocks + t / a.block_size];
        pb = pb < 0 ? 0 : (pb >= a.num_blocks ? (int)(a.num_blocks - 1) : pb);
        return a.pool + (int64_t)pb * a.s0 + ((int64_t)(t % a.block_size) * a.n_kv + hk) * D;
    };
    // scores: thread tid takes token t0 + tid
    {
        const int t = t0 + tid;
        float s[ATT_GMAX];
#pragma unroll
        for (int g = 0; g < ATT_GMAX; ++g) s[g] = 0.0f;
        if (t < t1) {
            const __half *kr = t == L - 1 ? nk : row_of(t);
#pragma unroll
            for (int d0 = 0; d0 < D; d0 += 8) {
                const uint4 raw = *reinterpret_cast<const uint4 *>(kr + d0);
                const __half *kh = reinterpret_cast<const __half *>(&raw);
                float kv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) kv[e] = h2f(kh[e]);
#pragma unroll
                for (int g = 0; g < ATT_GMAX; ++g)
                    if (g < G) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) s[g] = fmaf(q[g * D + d0 + e], kv[e], s[g]);
                    }
            }
        }
#pragma unroll
        for (int g = 0; g < ATT_GMAX; ++g)
            if (g < G) pr[g * ATT_TS + tid] = t < t1 ? s[g] * a.scale : -INFINITY;
    }
    __syncthreads();
    // softmax per query head over the split: max, then exp and sum
    const int n = t1 - t0;
    for (int g = 0; g < G; ++g) {
        float v = pr[g * ATT_TS + tid];
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
        pr[g * ATT_TS + tid] = e;
        float v = e;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) red[g * NW + w] = v;
    }
    __syncthreads();
    // weighted V sum: lane takes dims lane * VPL .. + VPL, wave w tokens w, w + NW, ...
    float o[ATT_GMAX][VPL];
#pragma unroll
    for (int g = 0; g < ATT_GMAX; ++g)
#pragma unroll
        for (int j = 0; j < VPL; ++j) o[g][j] = 0.0f;
    for (int i = w; i < n; i += NW) {
        const int t = t0 + i;
        const __half *vr = t == L - 1 ? nv : row_of(t) + a.s1;
        float vv[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) vv[j] = h2f(vr[lane * VPL + j]);
#pragma unroll
        for (int g = 0; g < ATT_GMAX; ++g)
            if (g < G) {
                const float pg = pr[g * ATT_TS + i];
#pragma unroll
                for (int j = 0; j < VPL; ++j) o[g][j] = fmaf(pg, vv[j], o[g][j]);
            }
    }
    // sum over the waves, one wave at a time, into the (now free) query area
    for (int k = 0; k < NW; ++k) {
        if (w == k) {
#pragma unroll
            for (int g = 0; g < ATT_GMAX; ++g)
                if (g < G)
#pragma unroll
                    for (int j = 0; j < VPL; ++j) {
                        float *const c = &acc[g * D + lane * VPL + j];
                        *c = k == 0 ? o[g][j] : *c + o[g][j];
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
            if (d == 0) { a.pm[ps] = n > 0 ? mx[g] : -INFINITY; a.pl[ps] = l; }
        }
    }
}

// One workgroup per (sequence, query head): the splits' max-rescaled sum.
template <int D>
__global__ __launch_bounds__(ATT_NT) void k_attn_merge(AttnArgs a)
{
    const int hq = blockIdx.x % a.n_heads, b = blockIdx.x / a.n_heads;
    const int L = min(max(a.seq_lens[b], 0), a.max_blocks * a.block_size);
    const int ns = min(a.nsplit, (L + ATT_TS - 1) / ATT_TS);
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

template <int D>
hipError_t launch_attn(const AttnArgs &a, int64_t B, hipStream_t st)
{
    const size_t lds = (size_t)a.G * (D + ATT_TS + ATT_NT / 64 + 1) * sizeof(float);   // at most 33 KiB
    hipLaunchKernelGGL((k_attn_split<D>), dim3((unsigned)(B * a.n_kv * a.nsplit)), dim3(ATT_NT), lds, st, a);
    if (a.nsplit > 1) hipLaunchKernelGGL((k_attn_merge<D>), dim3((unsigned)(B * a.n_heads)), dim3(ATT_NT), 0, st, a);
    return hipGetLastError();
}

}  // namespace
}  // namespace mis

extern "C" {

size_t mis_paged_attention_workspace_bytes(int64_t B, int n_heads, int d_k, int max_context)
{
    if (B <= 0 || n_heads <= 0 || d_k <= 0 || max_context <= 0) return 256;
    const int64_t ns = (max_context + mis::ATT_TS - 1) / mis::ATT_TS;
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
        ((uintptr_t)new_v & 15u))
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
    a.nsplit = (int)((max_context + ATT_TS - 1) / ATT_TS);
    a.scale = 1.0f / sqrtf((float)d_k);
    a.part = nullptr; a.pm = nullptr; a.pl = nullptr;
    if (a.nsplit > 1) {
        const size_t need = mis_paged_attention_workspace_bytes(B, n_heads, d_k, (int)max_context);
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
