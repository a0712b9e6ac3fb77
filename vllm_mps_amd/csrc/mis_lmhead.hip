// mis_lmhead.hip -- the lm_head GEMM with a greedy (argmax) epilogue: the
// decode step's logits are never written to HBM (include/mis_lmhead.h).
//
// k_lmh_tile: one workgroup of 4 waves per (tile of 128 vocabulary rows,
// group of up to 64 sequences).  Each wave owns 32 rows (two 16-row MFMA
// tiles) and every sequence of the group (up to four 16-column tiles):
// v_mfma_f32_16x16x16 (f16 or bf16) with the weight rows as A (read straight
// from HBM, 32 contiguous bytes per lane per block of 64 hidden dims) and the
// hidden states as B (the block staged in LDS once per workgroup, double
// buffered); each tile walks the hidden blocks from its own starting block.
// The products of two 16-bit values are exact in fp32; the sums are fp32.
// The weight blocks two ahead and the next hidden block are loaded while the
// current block's MFMAs run.  The epilogue rounds each logit to the model dtype
// and keeps, per sequence, the tile's best (dtype value, lowest index): a
// 64-bit key, larger is better.  k_lmh_merge takes the maximum key over the
// tiles of each sequence.
//
// The weight is read from HBM once per group of 64 sequences (once for a
// decode batch of up to 64); the hidden states come from L2 (each workgroup
// reads the group's [64, H] block).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mis_common.h"
#include "mis_lmhead.h"
#include "mis_sampler.h"

namespace mis {
namespace {

constexpr int LMH_NT = 256;            // threads per workgroup
constexpr int LMH_NW = LMH_NT / 64;    // waves
constexpr int LMH_RT = 2;              // 16-row tiles per wave
constexpr int LMH_VT = LMH_NW * LMH_RT * 16;  // vocabulary rows per workgroup (128)
constexpr int LMH_KB = 64;             // hidden dims per block (four MFMA steps of 16)
constexpr int LMH_BG = 64;             // sequences per group (four 16-column tiles)
constexpr int LMH_XST = LMH_KB + 8;    // LDS row stride of a staged hidden block, halves (144 bytes)

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float4_t mfma16(u32x2_t a, u32x2_t b, float4_t c)
{
    if constexpr (DT == 1)
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, a), __builtin_bit_cast(half4_t, b),
                                                     c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a),
                                                         __builtin_bit_cast(short4_t, b), c, 0, 0, 0);
}

// fp32 -> the model dtype (round to nearest even) -> fp32
template <int DT>
__device__ __forceinline__ float round_dt(float x)
{
    if constexpr (DT == 1) {
        return __half2float(__float2half_rn(x));
    } else {
        uint32_t u = __float_as_uint(x);
        if ((u & 0x7fffffffu) > 0x7f800000u) return x;  // NaN stays NaN
        u += 0x7fffu + ((u >> 16) & 1u);
        return __uint_as_float(u & 0xffff0000u);
    }
}

// Order key of a logit: larger is better; NaN above every number, -0 as +0
// (torch.argmax compares values)
__device__ __forceinline__ uint32_t val_key(float y)
{
    if (y != y) return 0xffffffffu;
    if (y == 0.0f) y = 0.0f;
    const uint32_t u = __float_as_uint(y);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// (value key, index) as one 64-bit key: larger value, then lower index
__device__ __forceinline__ uint64_t pack(uint32_t k, int64_t v)
{
    return ((uint64_t)k << 32) | (uint64_t)(0xffffffffu - (uint32_t)v);
}

// The Gumbel noise of vocabulary rows v .. v + 3 (v a multiple of 4) for one
// draw: Philox4x32-10 with key (seed low, seed high ^ step high) and counter
// (v / 4, step low, request low, request high); word i gives u = (w >> 8) 2^-24
// in [0, 1) and g = -log(-log(u)) (u = 0 gives -inf, never the maximum).
__device__ __forceinline__ void gumbel4(const mis_rng_row &q, int64_t v, float *g)
{
    uint32_t c[4] = {(uint32_t)(v >> 2), (uint32_t)q.step, (uint32_t)q.request, (uint32_t)(q.request >> 32)};
    philox4x32_10(c, (uint32_t)q.seed, (uint32_t)(q.seed >> 32) ^ (uint32_t)(q.step >> 32));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float u = (float)(c[i] >> 8) * 5.9604644775390625e-08f;
        g[i] = -logf(-logf(u));
    }
}

// SAMPLE: rows with temperature T > 0 take argmax(y + g) (the Gumbel-max draw
// from softmax(y)), y = dtype(logit / T); rows with T = 0 the greedy key.  A
// NaN or +inf y marks the row invalid (key 0xffffffff, k_lmh_merge gives -1).
template <int DT, bool SAMPLE>
__global__ __launch_bounds__(LMH_NT) void k_lmh_tile(const uint16_t *__restrict__ X, int64_t ldx,
                                                     const uint16_t *__restrict__ W, int64_t ldw, int64_t B, int64_t H,
                                                     int64_t V, uint64_t *__restrict__ part, const float *__restrict__ temp,
                                                     const mis_rng_row *__restrict__ rng)
{
    __shared__ uint16_t xs[2][LMH_BG * LMH_XST];
    __shared__ uint64_t red[LMH_NW][LMH_BG];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 15, qd = lane >> 4;
    const int64_t vt = blockIdx.x, v0 = vt * LMH_VT;
    const int64_t b0 = (int64_t)blockIdx.y * LMH_BG;
    const int nb = (int)(B - b0 < LMH_BG ? B - b0 : LMH_BG);   // sequences in this group
    const int nct = (nb + 15) >> 4;                             // their 16-column tiles
    const int nkb = (int)(H / LMH_KB);
    // this lane's weight rows (clamped into the matrix; rows past V are masked
    // in the epilogue) and hidden-dim quarter of a block: 16 contiguous dims
    const uint16_t *wrow[LMH_RT];
#pragma unroll
    for (int rt = 0; rt < LMH_RT; ++rt) {
        int64_t v = v0 + 32 * w + 16 * rt + col;
        v = v < V ? v : V - 1;
        wrow[rt] = W + v * ldw + 16 * qd;
    }
    // staging of hidden block k: thread t moves 16-byte pieces t and t + 256
    // of the [64 rows][64 dims] block (rows past the group are zeros)
    auto load_x = [&](int kb, uint4 *xr) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int idx = tid + u * LMH_NT, row = idx >> 3, seg = idx & 7;
            xr[u] = row < nb ? *reinterpret_cast<const uint4 *>(X + (b0 + row) * ldx + (int64_t)kb * LMH_KB + seg * 8)
                             : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto store_x = [&](int buf, const uint4 *xr) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int idx = tid + u * LMH_NT, row = idx >> 3, seg = idx & 7;
            *reinterpret_cast<uint4 *>(&xs[buf][row * LMH_XST + seg * 8]) = xr[u];
        }
    };
    auto load_w = [&](int kb, uint4 (*wr)[2]) {   // this lane's 32 bytes of each of its rows
#pragma unroll
        for (int rt = 0; rt < LMH_RT; ++rt) {
            const uint4 *p = reinterpret_cast<const uint4 *>(wrow[rt] + (int64_t)kb * LMH_KB);
            wr[rt][0] = p[0];
            wr[rt][1] = p[1];
        }
    };
    float4_t acc[LMH_RT][LMH_BG / 16];
#pragma unroll
    for (int rt = 0; rt < LMH_RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < LMH_BG / 16; ++ct) acc[rt][ct] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // three register sets of weight blocks: block k + 2 is issued as block k's
    // MFMAs start, so each block has two iterations to arrive
    uint4 xr[2], w0[LMH_RT][2], w1[LMH_RT][2], w2[LMH_RT][2];
    // this tile walks the hidden blocks from block vt mod nkb, wrapping: the
    // tiles in flight then read different column ranges of their rows instead
    // of all sweeping one 128-byte column of rows 8 KB apart
    const int koff = (int)(vt % (int64_t)nkb);
    auto blk = [&](int kb) { const int k = kb + koff; return k >= nkb ? k - nkb : k; };
    load_x(blk(0), xr);
    load_w(blk(0), w0);
    if (nkb > 1) load_w(blk(1), w1);
    store_x(0, xr);
    // iteration kb: weights in `cur`, block kb + 2 into `fut` (the set block
    // kb - 1 used), hidden block kb in LDS buffer kb & 1
    auto step = [&](int kb, uint4 (*cur)[2], uint4 (*fut)[2]) {
        __syncthreads();                       // block kb staged; the other buffer free
        if (kb + 1 < nkb) load_x(blk(kb + 1), xr);
        if (kb + 2 < nkb) load_w(blk(kb + 2), fut);
        const uint16_t *xb = xs[kb & 1];
        // step s uses dims 4 s .. 4 s + 3 of each lane's 16 (the same
        // permutation of the block's dims for both operands)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u32x2_t bx[LMH_BG / 16];
#pragma unroll
            for (int ct = 0; ct < LMH_BG / 16; ++ct)
                bx[ct] = *reinterpret_cast<const u32x2_t *>(&xb[(16 * ct + col) * LMH_XST + 16 * qd + 4 * s]);
#pragma unroll
            for (int rt = 0; rt < LMH_RT; ++rt) {
                const uint4 &r = cur[rt][s >> 1];
                const u32x2_t a = (s & 1) ? u32x2_t{r.z, r.w} : u32x2_t{r.x, r.y};
#pragma unroll
                for (int ct = 0; ct < LMH_BG / 16; ++ct)
                    if (ct < nct) acc[rt][ct] = mfma16<DT>(a, bx[ct], acc[rt][ct]);  // nct is workgroup-uniform
            }
        }
        if (kb + 1 < nkb) store_x((kb + 1) & 1, xr);
    };
    for (int kb = 0; kb < nkb; kb += 3) {      // the sets rotate with period three
        step(kb, w0, w2);
        if (kb + 1 < nkb) step(kb + 1, w1, w0);
        if (kb + 2 < nkb) step(kb + 2, w2, w1);
    }
    // epilogue: acc[rt][ct][r] is vocabulary row v0 + 32 w + 16 rt + 4 qd + r,
    // sequence b0 + 16 ct + col
#pragma unroll
    for (int ct = 0; ct < LMH_BG / 16; ++ct) {
        uint64_t best = 0ull;
        float T = 0.0f;
        mis_rng_row q = {0ull, 0ull, 0ull};
        if constexpr (SAMPLE) {
            const int64_t b = b0 + 16 * ct + col;
            if (ct < nct && b < B) { T = temp[b]; q = rng[b]; }
        }
#pragma unroll
        for (int rt = 0; rt < LMH_RT; ++rt) {
            float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const int64_t vq = v0 + 32 * w + 16 * rt + 4 * qd;
            if constexpr (SAMPLE) {
                if (T > 0.0f) gumbel4(q, vq, g);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t v = vq + r;
                if (v < V) {
                    const float x = round_dt<DT>(acc[rt][ct][r]);
                    uint32_t key;
                    if (SAMPLE && T > 0.0f) {
                        const float y = round_dt<DT>(x / T);
                        key = (y != y || y == INFINITY) ? 0xffffffffu : val_key(y + g[r]);
                    } else {
                        key = val_key(x);
                    }
                    const uint64_t k = pack(key, v);
                    best = k > best ? k : best;
                }
            }
        }
#pragma unroll
        for (int o = 16; o < 64; o <<= 1) {
            const uint64_t other = __shfl_xor(best, o, 64);
            best = other > best ? other : best;
        }
        if (qd == 0) red[w][16 * ct + col] = best;
    }
    __syncthreads();
    if (tid < nb) {
        uint64_t best = red[0][tid];
#pragma unroll
        for (int x = 1; x < LMH_NW; ++x) best = red[x][tid] > best ? red[x][tid] : best;
        part[vt * B + b0 + tid] = best;
    }
}

// One wave per sequence: the best key over the vocabulary tiles.
__global__ __launch_bounds__(LMH_NT) void k_lmh_merge(const uint64_t *__restrict__ part, int64_t ntiles, int64_t B,
                                                      int64_t *__restrict__ ids, const float *__restrict__ temp)
{
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * LMH_NW + (threadIdx.x >> 6);
    if (b >= B) return;                        // whole waves
    uint64_t best = 0ull;
    for (int64_t t = lane; t < ntiles; t += 64) {
        const uint64_t k = part[t * B + b];
        best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
    }
    if (lane == 0) {
        const float T = temp ? temp[b] : 0.0f;
        const uint32_t k = (uint32_t)(best >> 32);
        // a sampled row is invalid when a scaled logit is NaN or +inf, or when
        // every one is -inf (nothing to sample); T < 0 or NaN is a bad parameter
        const bool bad = temp && (!(T >= 0.0f) || (T > 0.0f && (k == 0xffffffffu || k <= 0x007fffffu)));
        ids[b] = bad ? -1 : (int64_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
    }
}

}  // namespace
}  // namespace mis

extern "C" {

size_t mis_lm_head_greedy_workspace_bytes(int64_t B, int64_t V)
{
    if (B <= 0 || V <= 0) return 256;
    const int64_t nt = (V + mis::LMH_VT - 1) / mis::LMH_VT;
    return ((size_t)nt * (size_t)B * sizeof(uint64_t) + 255) & ~(size_t)255;
}

int mis_lm_head_greedy(const void *hidden, int64_t ldx, const void *weight, int64_t ldw, int64_t B, int64_t H,
                       int64_t V, int dtype, int64_t *ids, void *workspace, size_t workspace_bytes, void *stream)
{
    using namespace mis;
    if (B < 0 || H <= 0 || V <= 0 || ldx < H || ldw < H) return MIS_LMH_ERR_INVALID_ARG;
    if (B == 0) return MIS_LMH_OK;
    if (!hidden || !weight || !ids) return MIS_LMH_ERR_INVALID_ARG;
    if (dtype != 1 && dtype != 2) return MIS_LMH_ERR_UNSUPPORTED;
    if (H % LMH_KB != 0) return MIS_LMH_ERR_UNSUPPORTED;
    if (V >= ((int64_t)1 << 31) || B > 65535 * (int64_t)LMH_BG) return MIS_LMH_ERR_UNSUPPORTED;
    if (((uintptr_t)hidden & 15u) || ((uintptr_t)weight & 15u) || (ldx & 7) || (ldw & 7))
        return MIS_LMH_ERR_INVALID_ARG;  // 16-byte rows for the vector loads
    const int64_t nt = (V + LMH_VT - 1) / LMH_VT;
    if (nt > 0x7fffffff) return MIS_LMH_ERR_UNSUPPORTED;
    const size_t need = mis_lm_head_greedy_workspace_bytes(B, V);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)) return MIS_LMH_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    uint64_t *part = reinterpret_cast<uint64_t *>(workspace);
    const dim3 grid((unsigned)nt, (unsigned)((B + LMH_BG - 1) / LMH_BG));
    const uint16_t *x = reinterpret_cast<const uint16_t *>(hidden);
    const uint16_t *wt = reinterpret_cast<const uint16_t *>(weight);
    if (dtype == 1)
        hipLaunchKernelGGL((k_lmh_tile<1, false>), grid, dim3(LMH_NT), 0, st, x, ldx, wt, ldw, B, H, V, part, nullptr,
                           nullptr);
    else
        hipLaunchKernelGGL((k_lmh_tile<2, false>), grid, dim3(LMH_NT), 0, st, x, ldx, wt, ldw, B, H, V, part, nullptr,
                           nullptr);
    hipLaunchKernelGGL(k_lmh_merge, dim3((unsigned)((B + LMH_NW - 1) / LMH_NW)), dim3(LMH_NT), 0, st, part, nt, B, ids,
                       nullptr);
    return hipGetLastError() == hipSuccess ? MIS_LMH_OK : MIS_LMH_ERR_HIP;
}

int mis_lm_head_sample(const void *hidden, int64_t ldx, const void *weight, int64_t ldw, int64_t B, int64_t H,
                       int64_t V, int dtype, const float *temperature, const mis_rng_row *rng, int64_t *ids,
                       void *workspace, size_t workspace_bytes, void *stream)
{
    using namespace mis;
    if (B < 0 || H <= 0 || V <= 0 || ldx < H || ldw < H) return MIS_LMH_ERR_INVALID_ARG;
    if (B == 0) return MIS_LMH_OK;
    if (!hidden || !weight || !ids || !temperature || !rng) return MIS_LMH_ERR_INVALID_ARG;
    if (dtype != 1 && dtype != 2) return MIS_LMH_ERR_UNSUPPORTED;
    if (H % LMH_KB != 0) return MIS_LMH_ERR_UNSUPPORTED;
    if (V >= ((int64_t)1 << 31) || B > 65535 * (int64_t)LMH_BG) return MIS_LMH_ERR_UNSUPPORTED;
    if (((uintptr_t)hidden & 15u) || ((uintptr_t)weight & 15u) || (ldx & 7) || (ldw & 7))
        return MIS_LMH_ERR_INVALID_ARG;
    const int64_t nt = (V + LMH_VT - 1) / LMH_VT;
    if (nt > 0x7fffffff) return MIS_LMH_ERR_UNSUPPORTED;
    const size_t need = mis_lm_head_greedy_workspace_bytes(B, V);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)) return MIS_LMH_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    uint64_t *part = reinterpret_cast<uint64_t *>(workspace);
    const dim3 grid((unsigned)nt, (unsigned)((B + LMH_BG - 1) / LMH_BG));
    const uint16_t *x = reinterpret_cast<const uint16_t *>(hidden);
    const uint16_t *wt = reinterpret_cast<const uint16_t *>(weight);
    if (dtype == 1)
        hipLaunchKernelGGL((k_lmh_tile<1, true>), grid, dim3(LMH_NT), 0, st, x, ldx, wt, ldw, B, H, V, part,
                           temperature, rng);
    else
        hipLaunchKernelGGL((k_lmh_tile<2, true>), grid, dim3(LMH_NT), 0, st, x, ldx, wt, ldw, B, H, V, part,
                           temperature, rng);
    hipLaunchKernelGGL(k_lmh_merge, dim3((unsigned)((B + LMH_NW - 1) / LMH_NW)), dim3(LMH_NT), 0, st, part, nt, B, ids,
                       temperature);
    return hipGetLastError() == hipSuccess ? MIS_LMH_OK : MIS_LMH_ERR_HIP;
}

}  // extern "C"
