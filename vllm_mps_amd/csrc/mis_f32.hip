// mis_f32.hip -- the sampler's kernels instantiated for F32 logits.
#include "mis_kernels.h"
#include "mis_launch.h"

namespace mis {

hipError_t launch_f32(const Args &a, float *probs, uint32_t *keep, hipStream_t st, unsigned kinds,
                     void *const *ev, int nev, const SideStreams *side)
{
    return launch_dt<F32>(a, probs, keep, st, kinds, ev, nev, side);
}

}  // namespace mis
