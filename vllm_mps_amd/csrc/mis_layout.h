// mis_layout.h -- workspace layout, per-call arguments and the limits shared
// by the kernels (mis_kernels.h) and the host-side C ABI (mis_api.hip).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "mis_sampler.h"

namespace mis {

constexpr int NT = 256;            // threads per workgroup (4 waves of 64)
constexpr int NWAVE = NT / 64;

constexpr int K_SMALL = 1024;      // largest k' served by the candidate path
constexpr int CAND_CAP = 2048;     // candidates one chunk may emit, at most (Layout::ccap per shape)
constexpr int SURV_CAP = 1024;     // top-k survivors / top-p window held in LDS
constexpr int K_PROBE = 512;       // fp16/bf16 top-p rows look for their cut among this many largest values
                                   // first (ties at the last one stay within SURV_CAP)
constexpr int EPT_DEFAULT = 32;    // elements per thread of the chunk pass (64 when G would exceed G_MAX)
constexpr int CCAP = 8192;         // small-k candidates of a row cached in LDS by k_rowpass (64 KB)
constexpr int CCAP_FIN = 4096;     // k_final's LDS cache of a row's candidates (32 KB; more are read from the workspace)
constexpr int G_MAX = 256;         // chunks per row
constexpr int CB_N = 128;          // coarse top-p bins below a chunk's max (float64, per wave)
constexpr float CB_SCALE = 4.0f;   // coarse bin = floor(y * CB_SCALE): 1/4 unit of y, 32 units in all
constexpr int REGION_MAX = 8;      // L1 bins per 16-bit chain pass at most (re-read path)
constexpr int RUN_CAP = REGION_MAX * 256;
constexpr int TIE_CAP = 1024;
constexpr uint32_t NCAND_OVERFLOW = 0xffffffffu;
constexpr int32_t IDX_ALL = 0x7fffffff;

enum : int { M_BAD = 0, M_GREEDY = 1, M_SMALLK = 2, M_LARGEK = 3, M_TOPP = 4, M_TEMP = 5, M_INVAL = 6 };
enum : uint32_t { FLAG_NAN = 1u, FLAG_PINF = 2u };

// ------------------------------------------------------------------ workspace

// The workspace keeps no state between calls: every word a call reads it has
// written earlier in the same call.
constexpr size_t CTL_PREFIX = 256;

struct ChunkSum {               // 64 B per (row, chunk)
    uint32_t xkey;              // argmax key of the raw logits (NaN = 0xffffffff)
    int32_t xarg;
    float ymax;                 // max scaled logit of the chunk
    uint32_t flags;
    uint32_t ncand;             // small-k candidates written, or NCAND_OVERFLOW
    uint32_t nfin;              // finite elements of the chunk
    uint32_t kc;                // small-k: non-candidates have scaled keys < kc
    uint32_t trunc;             // small-k: some finite element was not emitted
    double S;                   // sum of weights relative to the chunk max
    double pad[3];
};

// per-(row, chunk) coarse mass bins of an fp32 top-p row
struct RoundBuf {               // 1280 B
    double coarse[CB_N];        // coarse[b]: mass of bin top - b (relative to the chunk max)
    double S;                   // sum of weights relative to the chunk max
    float top;                  // the chunk max's coarse bin floor(ymax * CB_SCALE)
    float pad0;
    double pad[30];
};
static_assert(sizeof(RoundBuf) % 256 == 0, "RoundBuf size");

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

// fp32 top-p passes (k_tp_hist, k_tp_final): per (row, chunk) fine bins over
// the row's coarse band and a stash of band elements, per row the band
constexpr int FH = 512;             // fine bins per chunk over the coarse band
constexpr int STASH_CAP = 512;      // band elements one chunk stashes (a window of fine bins when more)
struct TopChunk {
    double above;                   // the chunk's mass above the band (relative to the row max)
    uint32_t nstash;                // elements stashed
    int32_t wlo, whi;               // every band element of the chunk in fine bins [wlo, whi] is stashed
    uint32_t pad0;
    double pad[29];
    uint32_t cnt[FH];
    double mass[FH];
};
static_assert(sizeof(TopChunk) % 256 == 0, "TopChunk size");
enum : uint32_t { TR_NONE = 0, TR_ACTIVE = 1, TR_DEFER = 2 };
struct TopRow {                     // written by the row's chunk-0 workgroup of k_tp_hist
    uint32_t status, pad0;          // TR_*
    uint32_t klo, khi;              // coarse band (row keys)
    uint32_t xlo, xhi;              // its raw-key interval
    uint32_t pad1[2];
    float m, lo, scf, T;            // row max of y; fine-bin grid y -> (y - lo) * scf; temperature
    double S, A;                    // sum of exp(y - m), top_p * S
    double pad[24];
};
static_assert(sizeof(TopRow) % 256 == 0, "TopRow size");

// fp16/bf16 top-p passes (k_t16_hist, k_t16_walk): per row a count
// histogram over the NB16 16-bit keys at and below the row max's key, per
// (row, chunk) its exact mass and kept mass, per row the cut
constexpr int NB16 = 4096;
struct T16Chunk {                   // 32 B per (row, chunk)
    double S;                       // sum of exp(y - m) over the chunk's finite elements (m = row max)
    double kept;                    // mass of its elements with keys above the cut key
    uint32_t below;                 // finite elements with keys under the histogram's range
    uint32_t ccnt;                  // elements holding the cut key
    uint32_t pad[2];
};
enum : uint32_t { T16_NONE = 0, T16_CUT = 1, T16_DEFER = 2, T16_EMPTY = 3 };
struct T16Row {                     // 32 B per row
    uint32_t status;                // T16_*: CUT = ck / t below hold the cut, EMPTY = nothing kept
    uint32_t ck;                    // cut key (16-bit): every element with a larger key is kept
    uint32_t t;                     // elements holding ck that are kept (the first t in index order)
    uint32_t pad0;
    double S;                       // sum of exp(y - m) over the row
    double pad1;
};

// fp16/bf16 top-p rows spread over the t16 passes while the batch has fewer
// rows than this (a CU count); a larger batch gives each row one workgroup
// (the K_PROBE probe, then the generic path), which fills the GPU by itself
constexpr int64_t T16_ROWS = 256;

struct Layout {
    int64_t B, V;
    int ept, G;
    int ccap;                       // candidate slots per (row, chunk)
    int t16;                        // fp16/bf16 and B < T16_ROWS: the t16 passes serve the top-p rows
    size_t rowout, chunks, rbuf, cand, topc, topr, stash, t16h, t16c, t16r, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Elements per thread: 32 (chunks of 8192 elements), 64 when the row would
// need more than G_MAX chunks.
inline Layout make_layout(int64_t B, int64_t V, int dtype)
{
    Layout L;
    L.B = B; L.V = V;
    auto chunks = [&](int ept) { return (V + (int64_t)NT * ept - 1) / ((int64_t)NT * ept); };
    L.ept = EPT_DEFAULT;
    if (chunks(L.ept) > G_MAX) L.ept = 64;
    L.G = (int)chunks(L.ept);
    // candidate slots per chunk: four times what the chunk pass aims at for
    // the largest k' the candidate path serves (2 * ceil(K_SMALL / G) + 32,
    // all K_SMALL when the row is one chunk), plus 64, in multiples of 64.
    // Measured on the configs the largest chunk emits at most 60 % of this;
    // a chunk with more overflows to the exact generic path.
    {
        const int64_t nc = L.G == 1 ? (int64_t)K_SMALL : 2 * (((int64_t)K_SMALL + L.G - 1) / L.G) + 32;
        const int64_t c = (4 * nc + 64 + 63) / 64 * 64;
        L.ccap = (int)(c < (int64_t)CAND_CAP ? c : (int64_t)CAND_CAP);
    }
    const size_t BG = (size_t)B * L.G;
    size_t off = CTL_PREFIX;
    L.rowout = off; off = align256(off + sizeof(RowOut) * (size_t)B);
    L.chunks = off; off = align256(off + sizeof(ChunkSum) * BG);
    L.rbuf = off;   off = align256(off + (dtype == MIS_DTYPE_F32 ? sizeof(RoundBuf) * BG : 0));
    L.cand = off;   off = align256(off + sizeof(Cand) * (size_t)L.ccap * BG);
    // fp32 top-p: per-chunk fine bins and per-row state of the top-p passes
    const bool f32 = dtype == MIS_DTYPE_F32;
    L.topc = off;   off = align256(off + (f32 ? sizeof(TopChunk) * BG : 0));
    L.topr = off;   off = align256(off + (f32 ? sizeof(TopRow) * (size_t)B : 0));
    L.stash = off;  off = align256(off + (f32 ? sizeof(Cand) * (size_t)STASH_CAP * BG : 0));
    // fp16/bf16 top-p of a small batch: per-row key histograms, per-chunk
    // masses, per-row cuts
    L.t16 = (!f32 && B < T16_ROWS) ? 1 : 0;
    L.t16h = off;   off = align256(off + (L.t16 ? sizeof(uint32_t) * (size_t)NB16 * (size_t)B : 0));
    L.t16c = off;   off = align256(off + (L.t16 ? sizeof(T16Chunk) * BG : 0));
    L.t16r = off;   off = align256(off + (L.t16 ? sizeof(T16Row) * (size_t)B : 0));
    L.total = off;
    return L;
}


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
    int emit;                   // probabilities or keep masks requested (k_emit reads every row's exact cut)
};

}  // namespace mis
