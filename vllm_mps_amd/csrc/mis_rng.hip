// mis_rng.hip -- mis_fill_uniforms(): the per-request uniforms of the draw,
// one thread per row, from the counter-based generator in mis_common.h.
#include <hip/hip_runtime.h>

#include "mis_common.h"
#include "mis_launch.h"

namespace mis {

__global__ __launch_bounds__(256) void k_uniforms(mis_row_params *params, const mis_rng_row *rng, int64_t B)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= B) return;
    const mis_rng_row r = rng[i];
    params[i].uniform = philox_uniform(r.seed, r.request, r.step);
}

hipError_t launch_uniforms(mis_row_params *params, const mis_rng_row *rng, int64_t B, hipStream_t st)
{
    hipLaunchKernelGGL(k_uniforms, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st, params, rng, B);
    return hipGetLastError();
}

}  // namespace mis
