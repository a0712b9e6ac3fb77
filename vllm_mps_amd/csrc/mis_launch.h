// mis_launch.h -- the per-dtype launch sequences, one per translation unit
// (mis_f32.hip, mis_f16.hip, mis_bf16.hip), called by the C ABI (mis_api.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "mis_layout.h"
#include "mis_sampler.h"

namespace mis {

// A second stream on the caller's device and the two events that fork it from
// the caller's stream and join it back (from a mis_context; see mis_sampler.h).
struct SideStreams {
    hipStream_t s;
    hipEvent_t fork, join;
};

// Launches one sampling step over a.L.B rows on `st` (see launch_dt in
// mis_kernels.h): ev/nev are the optional profiling events, kinds the
// row-kind hint, side the caller's side stream (NULL: one stream).
hipError_t launch_f32(const Args &a, float *probs, uint32_t *keep, hipStream_t st, unsigned kinds,
                      void *const *ev, int nev, const SideStreams *side);
hipError_t launch_f16(const Args &a, float *probs, uint32_t *keep, hipStream_t st, unsigned kinds,
                      void *const *ev, int nev, const SideStreams *side);
hipError_t launch_bf16(const Args &a, float *probs, uint32_t *keep, hipStream_t st, unsigned kinds,
                       void *const *ev, int nev, const SideStreams *side);

// Fills params[r].uniform from rng[r] for r < B (mis_rng.hip).
hipError_t launch_uniforms(mis_row_params *params, const mis_rng_row *rng, int64_t B, hipStream_t st);

}  // namespace mis
