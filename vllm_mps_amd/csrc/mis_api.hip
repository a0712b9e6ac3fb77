// mis_api.hip -- the C ABI of include/mis_sampler.h: argument checks, the
// workspace layout and dispatch to the per-dtype launch sequences.  Host code
// only; the kernels live in the per-dtype translation units.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <new>

#include "mis_launch.h"
#include "mis_layout.h"
#include "mis_sampler.h"

namespace mis {
static thread_local int g_last_hip = 0;
}  // namespace mis

// The scratch of mis_sample_noalloc(): one copy per device, loaded with this
// file's code object and held until the process ends.  On the host the name
// stands for the host-side shadow, not a device address: device work uses the
// address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[MIS_SCRATCH_BYTES];

namespace mis {
constexpr int SCRATCH_DEVICES = 64;  // device ordinals the per-device table covers
static std::once_flag g_scratch_once[SCRATCH_DEVICES];
static void *g_scratch_ptr[SCRATCH_DEVICES];
static hipError_t g_scratch_err[SCRATCH_DEVICES];

// The current device's copy of `scratch`, looked up once per device with
// that device current.
static int scratch_of_current_device(void **out)
{
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { g_last_hip = (int)e; return MIS_ERR_HIP; }
    if (dev < 0 || dev >= SCRATCH_DEVICES) return MIS_ERR_UNSUPPORTED;
    std::call_once(g_scratch_once[dev], [dev] {
        void *p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_scratch_err[dev] != hipSuccess) { g_last_hip = (int)g_scratch_err[dev]; return MIS_ERR_HIP; }
    *out = g_scratch_ptr[dev];
    return MIS_OK;
}
}  // namespace mis

// A caller's side stream for one device (mis_context_create).
struct mis_context {
    int device;
    mis::SideStreams side;
};

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
                       unsigned kinds, void *const *events, int nev, const mis_context *ctx)
{
    using namespace mis;
    if (dtype < 0 || dtype > 2 || B < 0 || V <= 0 || row_stride < V) return MIS_ERR_INVALID_ARG;
    if (B == 0) return MIS_OK;
    if (!logits || !params || !out_ids || !workspace) return MIS_ERR_INVALID_ARG;
    if (V > (int64_t)1 << 30 || B > 0x7fffffff) return MIS_ERR_UNSUPPORTED;
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
    a.emit = (out_probs || out_keep) ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    const SideStreams *sd = nullptr;
    if (ctx) {
        int dev = -1;
        if ((e = hipGetDevice(&dev)) != hipSuccess) { g_last_hip = (int)e; return MIS_ERR_HIP; }
        if (dev != ctx->device) return MIS_ERR_INVALID_ARG;
        sd = &ctx->side;
    }
    if (dtype == MIS_DTYPE_F32) e = launch_f32(a, out_probs, out_keep, st, kinds, events, nev, sd);
    else if (dtype == MIS_DTYPE_F16) e = launch_f16(a, out_probs, out_keep, st, kinds, events, nev, sd);
    else e = launch_bf16(a, out_probs, out_keep, st, kinds, events, nev, sd);
    if (e != hipSuccess) { g_last_hip = (int)e; return MIS_ERR_HIP; }
    return MIS_OK;
}

int mis_sample(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
               const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
               uint32_t *out_keep, void *workspace, size_t workspace_bytes, void *stream)
{
    return sample_impl(logits, dtype, B, V, row_stride, params, out_ids, out_status, out_probs, out_keep,
                       workspace, workspace_bytes, stream, MIS_KIND_ALL, nullptr, 0, nullptr);
}

int mis_sample_profiled(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                        const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
                        uint32_t *out_keep, void *workspace, size_t workspace_bytes, void *stream,
                        void *const *events)
{
    if (!events || !events[0] || !events[1] || !events[2]) return MIS_ERR_INVALID_ARG;
    return sample_impl(logits, dtype, B, V, row_stride, params, out_ids, out_status, out_probs, out_keep,
                       workspace, workspace_bytes, stream, MIS_KIND_ALL, events, 3, nullptr);
}

int mis_sample_ex(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                  const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
                  uint32_t *out_keep, void *workspace, size_t workspace_bytes, void *stream, unsigned kinds,
                  void *const *events, mis_context *ctx)
{
    if ((kinds & ~(unsigned)MIS_KIND_ALL) != 0u) return MIS_ERR_INVALID_ARG;
    if (events && (!events[0] || !events[1] || !events[2] || !events[3])) return MIS_ERR_INVALID_ARG;
    return sample_impl(logits, dtype, B, V, row_stride, params, out_ids, out_status, out_probs, out_keep,
                       workspace, workspace_bytes, stream, kinds, events, 4, ctx);
}

int mis_sample_noalloc(const void *logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                       const mis_row_params *params, int64_t *out_ids, int32_t *out_status, float *out_probs,
                       uint32_t *out_keep, void *stream, unsigned kinds)
{
    if ((kinds & ~(unsigned)MIS_KIND_ALL) != 0u) return MIS_ERR_INVALID_ARG;
    if (dtype < 0 || dtype > 2 || B < 0 || V <= 0 || row_stride < V) return MIS_ERR_INVALID_ARG;
    if (B == 0) return MIS_OK;
    if (!logits || !params || !out_ids) return MIS_ERR_INVALID_ARG;
    if (V > (int64_t)1 << 30 || B > 0x7fffffff) return MIS_ERR_UNSUPPORTED;
    if (mis::make_layout(B, V, dtype).total > MIS_SCRATCH_BYTES) return MIS_ERR_SCRATCH;
    void *ws = nullptr;
    const int rc = mis::scratch_of_current_device(&ws);
    if (rc != MIS_OK) return rc;
    return sample_impl(logits, dtype, B, V, row_stride, params, out_ids, out_status, out_probs, out_keep, ws,
                       MIS_SCRATCH_BYTES, stream, kinds, nullptr, 0, nullptr);
}

int mis_fill_uniforms(mis_row_params *params, const mis_rng_row *rng, int64_t B, void *stream)
{
    if (B < 0) return MIS_ERR_INVALID_ARG;
    if (B == 0) return MIS_OK;
    if (!params || !rng) return MIS_ERR_INVALID_ARG;
    if (B > 0x7fffffff) return MIS_ERR_UNSUPPORTED;
    const hipError_t e = mis::launch_uniforms(params, rng, B, (hipStream_t)stream);
    if (e != hipSuccess) { mis::g_last_hip = (int)e; return MIS_ERR_HIP; }
    return MIS_OK;
}

int mis_context_create(mis_context **out)
{
    if (!out) return MIS_ERR_INVALID_ARG;
    *out = nullptr;
    mis_context *c = new (std::nothrow) mis_context();
    if (!c) return MIS_ERR_HIP;
    hipError_t e = hipGetDevice(&c->device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->side.s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->side.fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->side.join, hipEventDisableTiming);
    if (e != hipSuccess) {
        mis::g_last_hip = (int)e;
        mis_context_destroy(c);
        return MIS_ERR_HIP;
    }
    *out = c;
    return MIS_OK;
}

int mis_context_destroy(mis_context *ctx)
{
    if (!ctx) return MIS_OK;
    int rc = MIS_OK;
    if (ctx->side.fork && hipEventDestroy(ctx->side.fork) != hipSuccess) rc = MIS_ERR_HIP;
    if (ctx->side.join && hipEventDestroy(ctx->side.join) != hipSuccess) rc = MIS_ERR_HIP;
    if (ctx->side.s && hipStreamDestroy(ctx->side.s) != hipSuccess) rc = MIS_ERR_HIP;
    delete ctx;
    return rc;
}

const char *mis_strerror(int code)
{
    switch (code) {
    case MIS_OK: return "ok";
    case MIS_ERR_INVALID_ARG: return "invalid argument";
    case MIS_ERR_WORKSPACE: return "workspace too small or not 256-byte aligned";
    case MIS_ERR_HIP: return "HIP launch failed";
    case MIS_ERR_UNSUPPORTED: return "shape not supported (V > 2^30, B > 2^31 - 1 or more than 256 chunks per row)";
    case MIS_ERR_SCRATCH: return "shape needs more than the static scratch of mis_sample_noalloc (MIS_SCRATCH_BYTES)";
    default: return "unknown error";
    }
}

int mis_last_hip_error(void) { return mis::g_last_hip; }

int mis_abi_version(void) { return MIS_ABI_VERSION; }

}  // extern "C"
