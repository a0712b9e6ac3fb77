// Test-only shim: exposes the host/device helpers of mis_common.h to pytest
// through a plain C ABI so the CPU suite checks the exact code the kernels run.
#include "../../vllm_mps_amd/csrc/mis_common.h"

extern "C" {
float shim_chain_add_n(float F, float p, uint64_t n) { return mis::chain_add_n(F, p, n); }
float shim_chain_E(float F, float p, int dt) { return mis::chain_E(F, p, dt); }
float shim_rn_dtype(float f, int dt) { return mis::rn_dtype(f, dt); }
uint32_t shim_row_key(float y, int dt) { return mis::row_key(y, dt); }
float shim_value_of_row_key(uint32_t k, int dt) { return mis::value_of_row_key(k, dt); }
uint32_t shim_argmax_key(float x) { return mis::argmax_key(x); }
void shim_rn_dtype_array(const float *x, float *y, int64_t n, int dt)
{
    for (int64_t i = 0; i < n; ++i) y[i] = mis::rn_dtype(x[i], dt);
}
void shim_dexp_array(const double *d, double *out, int64_t n)
{
    double tab[mis::ETAB_N];
    for (int t = 0; t < mis::ETAB_N; ++t) mis::exp_table(tab, t);
    for (int64_t i = 0; i < n; ++i) out[i] = mis::dexp(d[i], tab);
}
float shim_div_rcp(float x, float T) { return mis::div_rcp(x, T, 1.0f / T); }
// the device generator's uniforms for n (seed, request, step) triples
void shim_philox_uniforms(int64_t n, const uint64_t *seed, const uint64_t *request, const uint64_t *step, float *u)
{
    for (int64_t i = 0; i < n; ++i) u[i] = mis::philox_uniform(seed[i], request[i], step[i]);
}
void shim_philox4x32_10(const uint32_t *in, const uint32_t *key, uint32_t *out)
{
    uint32_t c[4] = {in[0], in[1], in[2], in[3]};
    mis::philox4x32_10(c, key[0], key[1]);
    for (int i = 0; i < 4; ++i) out[i] = c[i];
}
// bit patterns [lo, hi) of x (step `stride`): mismatches of div_rcp against
// IEEE x / T, the first one in *first (NaN quotients compare as NaN)
uint64_t shim_div_rcp_sweep(float T, uint64_t lo, uint64_t hi, uint64_t stride, uint32_t *first)
{
    const float r = 1.0f / T;
    uint64_t bad = 0;
    for (uint64_t b = lo; b < hi; b += stride) {
        const float x = mis::bits_f32((uint32_t)b);
        const float a = mis::div_rcp(x, T, r), e = x / T;
        const bool same = (a != a && e != e) || mis::f32_bits(a) == mis::f32_bits(e);
        if (!same && bad++ == 0) *first = (uint32_t)b;
    }
    return bad;
}
// naive reference for chain_add_n: one float addition per step
float shim_chain_naive(float F, float p, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) F = F + p;
    return F;
}
}
