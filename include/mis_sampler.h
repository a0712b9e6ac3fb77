/*
 * mis_sampler.h -- C ABI of the MI355X-native decode-step token sampler.
 *
 * The library (libmis_sampler.so, built from vllm_mps_amd/csrc/) replaces the
 * per-row Python sampler of the reference engine with one batched,
 * stream-ordered call over a [B, V] logits tensor resident in HBM.
 *
 * Reference interfaces replaced:
 *   - Sampler.sample(logits[V], SamplingParams) -> int
 *       model/sampler.py:18-60 (greedy / temperature / top-k / top-p / draw)
 *   - Sampler.sample_batch(logits[B, V], SamplingParams) -> list[int]
 *       model/sampler.py:62-79
 *   - the engine's per-row dispatch loop over _seq_to_params
 *       engine/llm_engine.py:339-345, engine/model_runner.py:124-129
 *   - SamplingParams fields temperature / top_k / top_p
 *       core/sequence.py:23-39 (validation :41-61 is mirrored per row as
 *       MIS_ROW_BAD_PARAM instead of a Python ValueError)
 *
 * All pointers except the workspace size are device pointers.  No exceptions,
 * no host synchronisation and no allocation happen inside mis_sample(),
 * mis_sample_profiled(), mis_sample_ex() and mis_sample_noalloc(); every
 * launch goes on `stream` (a hipStream_t; NULL = the legacy default stream),
 * or on a caller-created side stream (mis_context) that `stream` joins.  The
 * library's only process-global state is the static scratch of
 * mis_sample_noalloc() (one copy per device) and its per-device address:
 * calls of the other entry points on different streams with their own
 * workspaces (and contexts) may run concurrently.
 */
#ifndef MIS_SAMPLER_H
#define MIS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIS_ABI_VERSION 8

/* logits element type */
enum { MIS_DTYPE_F32 = 0, MIS_DTYPE_F16 = 1, MIS_DTYPE_BF16 = 2 };

/* return codes of the API */
enum {
    MIS_OK = 0,
    MIS_ERR_INVALID_ARG = 1,   /* null pointer, bad dtype, B < 0, V <= 0, row_stride < V */
    MIS_ERR_WORKSPACE = 2,     /* workspace too small or misaligned */
    MIS_ERR_HIP = 3,           /* a HIP launch failed; see mis_last_hip_error() */
    MIS_ERR_UNSUPPORTED = 4,   /* V or B beyond the supported range */
    MIS_ERR_SCRATCH = 5        /* mis_sample_noalloc(): the shape needs more than
                                  MIS_SCRATCH_BYTES of scratch */
};

/* per-row status written to out_status */
enum {
    MIS_ROW_OK = 0,
    MIS_ROW_BAD_PARAM = 1,     /* temperature < 0, top_k < 0, top_p <= 0 or NaN, uniform NaN
                                  (core/sequence.py:41-61 raises ValueError) */
    MIS_ROW_INVALID = 2,       /* temperature NaN, NaN or +inf scaled logits, or nothing left
                                  to sample (torch.multinomial raises RuntimeError,
                                  model/sampler.py:59) */
    MIS_ROW_UNSUPPORTED = 3,   /* reserved: not produced by this build (every row mode is
                                  served) */
    MIS_ROW_INTERNAL = 4       /* reserved: not produced by this build */
};

/*
 * Per-row parameters, 16 bytes, device array [B].
 *   temperature  f32(T); 0 selects greedy argmax (model/sampler.py:33-34).
 *                Logits are scaled as dtype(f32(x) / temperature), sampler.py:37.
 *   top_k        0 = off; otherwise k' = min(top_k, V) (sampler.py:40-43).
 *   top_p        top-p filtering applies iff top_p < 1.0f (sampler.py:46-55);
 *                the threshold is top_p rounded to the logits dtype.
 *   uniform      u in [0, 1) for the inverse-CDF draw that replaces
 *                torch.multinomial (sampler.py:59).
 */
typedef struct mis_row_params {
    float temperature;
    int32_t top_k;
    float top_p;
    float uniform;
} mis_row_params;

/* Bytes of device workspace mis_sample() needs for this shape. */
size_t mis_workspace_bytes(int64_t B, int64_t V, int dtype);

/*
 * Prepares a freshly allocated workspace: clears its first 256 bytes
 * (hipMemsetAsync on `stream`; not for use under graph capture).  The
 * kernels of this build keep no state in the workspace between calls (every
 * call writes what it later reads), so the call is optional; it stays in
 * the ABI so that a later build may keep control words there again.
 * No counterpart in the reference (its sampler keeps no device state).
 */
int mis_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/*
 * One decode-step sampling pass over `B` rows of `V` logits.
 *   logits        device, B rows, row r starts at logits + r*row_stride elements
 *   params        device [B] mis_row_params
 *   out_ids       device [B] int64: sampled token id, -1 when status != OK
 *   out_status    device [B] int32 (nullable)
 *   out_probs     device [B, V] float32 post-filter probabilities, 0 for
 *                 removed tokens, one-hot for greedy rows (nullable; debug)
 *   out_keep      device [B, ceil(V/32)] uint32 keep bitmask, bit j%32 of word
 *                 j/32 = token j survives every filter (nullable; debug)
 *   workspace     device scratch of at least mis_workspace_bytes(B, V, dtype)
 *                 bytes, 256-byte aligned; not shared by concurrent calls
 *   stream        hipStream_t the kernels are launched on
 * Returns MIS_OK or an error code; launches are asynchronous.
 */
int mis_sample(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
               const mis_row_params *params, int64_t *out_ids, int32_t *out_status,
               float *out_probs, uint32_t *out_keep, void *workspace, size_t workspace_bytes,
               void *stream);

/*
 * Instrumented mis_sample(): identical results, and additionally records the
 * caller's hipEvent_t handles events[0] before the chunk pass, events[1]
 * between the chunk pass and the row pass, events[2] after the row pass, all
 * on `stream`.  No counterpart in the reference: it exists so benchmarks can
 * time each kernel on the stream it runs on.
 */
int mis_sample_profiled(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                        const mis_row_params *params, int64_t *out_ids, int32_t *out_status,
                        float *out_probs, uint32_t *out_keep, void *workspace, size_t workspace_bytes,
                        void *stream, void *const *events);

/*
 * Row kinds a batch holds, for mis_sample_ex(): a performance hint only.
 *   MIS_KIND_TOPP32   fp32 logits, 0 < temperature, top_k off (0 or >= V),
 *                     top_p < 1 (the rows the top-p passes serve)
 *   MIS_KIND_OTHER    every other row
 *   MIS_KIND_GENERIC  among the others, rows that take the generic row pass:
 *                     0 < temperature and either top_k > 1024 (and < V) or
 *                     fp16/bf16 logits with top_k off and top_p < 1
 * A clear bit lets the library skip the launches only that kind needs; the
 * results are the same for any `kinds` (rows of a kind whose bit is clear
 * take the generic path), so a wrong hint costs time, never correctness.
 */
enum { MIS_KIND_TOPP32 = 1, MIS_KIND_OTHER = 2, MIS_KIND_GENERIC = 4, MIS_KIND_ALL = 7 };

/*
 * A caller's side stream: a second stream on the device current at creation
 * (default priority) and two events that fork it from the caller's stream
 * and join it back.  mis_context_create allocates them; mis_sample_ex uses
 * them when given the context, and creates nothing itself.  Calls that
 * overlap in time need contexts (and workspaces) of their own.  No
 * counterpart in the reference (its sampler runs on the host, one row at a
 * time, engine/llm_engine.py:341-344).
 */
typedef struct mis_context mis_context;
int mis_context_create(mis_context **out);
int mis_context_destroy(mis_context *ctx);

/*
 * mis_sample() with a row-kind hint, optional events and an optional
 * context.  events: NULL, or four hipEvent_t handles, events[0..2] as by
 * mis_sample_profiled() and events[3] after the chunk pass of the rows the
 * side stream serves.  ctx: NULL (every launch on `stream`), or a context of
 * the current device.  With a context, a batch holding both fp32 top-p rows
 * and other rows splits: the other rows' chunk pass and row pass run on the
 * context's side stream beside the top-p rows' passes on `stream`, which
 * joins the side stream before the call's last launch.  events[1] (on
 * `stream`) then closes only the top-p rows' half of the chunk pass and
 * events[3] the other half; both start after events[0].  Without the split
 * events[3] is not recorded (events[1] closes the whole chunk pass).  No
 * counterpart in the reference: its sampler runs on the host, which knows
 * each request's SamplingParams; the engine's batch builder passes what it
 * knows.
 */
int mis_sample_ex(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                  const mis_row_params *params, int64_t *out_ids, int32_t *out_status,
                  float *out_probs, uint32_t *out_keep, void *workspace, size_t workspace_bytes,
                  void *stream, unsigned kinds, void *const *events, mis_context *ctx);

/*
 * Size of the static device scratch behind mis_sample_noalloc(): 128 MiB, one
 * copy on each device the call runs on, held until the process ends.  It
 * covers every shape whose mis_workspace_bytes() fits, e.g. B = 256 fp32 rows
 * or B = 1024 fp16/bf16 rows of V = 128256.
 */
#define MIS_SCRATCH_BYTES ((size_t)128 << 20)

/*
 * mis_sample_ex() without a workspace, events or context, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Its scratch is a file-scope device array of MIS_SCRATCH_BYTES per device,
 * whose address the first call on a device looks up; the call allocates
 * nothing and every launch goes on `stream`.  Returns MIS_ERR_SCRATCH when
 * mis_workspace_bytes(B, V, dtype) exceeds MIS_SCRATCH_BYTES.  Every call on
 * a device shares that device's scratch, which keeps the last call's
 * contents (the kernels write every word they later read, so nothing needs
 * clearing): calls that overlap in time on one device (other streams, other
 * threads) race and must be ordered by the caller.
 */
int mis_sample_noalloc(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                       const mis_row_params *params, int64_t *out_ids, int32_t *out_status,
                       float *out_probs, uint32_t *out_keep, void *stream, unsigned kinds);

/*
 * Per-request generator state, 24 bytes, device array [B], for
 * mis_fill_uniforms(): the key and counter of one draw.
 *   seed     the generator key (an engine-wide or per-request seed)
 *   request  the request (sequence) id
 *   step     which draw of that request (tokens sampled for it so far)
 */
typedef struct mis_rng_row {
    uint64_t seed;
    uint64_t request;
    uint64_t step;
} mis_rng_row;

/*
 * Writes params[r].uniform for r < B from rng[r]: Philox4x32-10 (Salmon et
 * al., SC 2011) with key = seed (low word first) and counter = (step low,
 * step high, request low, request high); u = (first output word >> 8) * 2^-24.
 * Replaces the global generator torch.multinomial draws from
 * (model/sampler.py:59): a request's token then depends only on
 * (seed, request, step) and its logits, not on the batch, the stream or the
 * order of calls.  One launch on `stream`; no allocation.
 */
int mis_fill_uniforms(mis_row_params *params, const mis_rng_row *rng, int64_t B, void *stream);

/* Human-readable text for an API return code. */
const char *mis_strerror(int code);

/* hipError_t of the last failed launch in this thread (0 if none). */
int mis_last_hip_error(void);

/* MIS_ABI_VERSION of the built library. */
int mis_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MIS_SAMPLER_H */
