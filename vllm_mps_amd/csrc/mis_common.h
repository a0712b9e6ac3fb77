// mis_common.h -- helpers shared by the HIP kernels and host-side unit tests.
//
// Everything here is plain IEEE arithmetic and bit manipulation, compiled
// identically for gfx950 (hipcc) and for the host (g++), so the CPU tests
// exercise the exact code the kernels run.
#pragma once

#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define MIS_HD __host__ __device__ __forceinline__
#else
#define MIS_HD static inline
#endif

namespace mis {

enum DType : int { F32 = 0, F16 = 1, BF16 = 2 };

MIS_HD uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
MIS_HD float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
MIS_HD uint64_t f64_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
MIS_HD double bits_f64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

// ---------------------------------------------------------------- 16-bit types

MIS_HD float f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;  // m * 2^-24, exact
        return sign ? -v : v;
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

// float -> binary16, round to nearest even, subnormals kept, overflow -> inf
MIS_HD uint16_t f32_to_f16(float f)
{
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        // subnormal half: value / 2^-24 rounded to nearest even.  The float's
        // significand shifted right by (126 - exp) with RNE on the shifted-out bits.
        uint32_t exp = a >> 23;
        if (exp < 102u) return sign;  // < 2^-25: rounds to zero
        uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - exp;  // 14..24
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (a >> 23) - 112u;
    uint32_t hm = (a & 0x7fffffu) >> 13, rest = a & 0x1fffu;
    uint32_t h = (e << 10) | hm;
    if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) h++;
    return (uint16_t)(sign | h);
}

MIS_HD float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

MIS_HD uint16_t f32_to_bf16(float f)
{
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t rest = u & 0xffffu, h = u >> 16;
    if (rest > 0x8000u || (rest == 0x8000u && (h & 1u))) h++;
    return (uint16_t)h;
}

// Round a float to the dtype (RNE) and return it as float.
MIS_HD float rn_dtype(float f, int dt)
{
    if (dt == F16) return f16_to_f32(f32_to_f16(f));
    if (dt == BF16) return bf16_to_f32(f32_to_bf16(f));
    return f;
}

// The dtype's 16-bit encoding of a float that is exactly representable in it.
MIS_HD uint16_t bits16_of(float f, int dt) { return dt == F16 ? f32_to_f16(f) : (uint16_t)(f32_bits(f) >> 16); }
MIS_HD float f32_of_bits16(uint16_t h, int dt) { return dt == F16 ? f16_to_f32(h) : bf16_to_f32(h); }

// ---------------------------------------------------------------- order keys
//
// Row keys are uint32 and order like the values they encode; -0.0 and +0.0
// map to the same key because the reference compares values, not bits.  fp32
// rows use all 32 bits; 16-bit rows use the 16-bit pattern in the high half
// (low half zero), so a two-level 8-bit radix resolves them.

MIS_HD uint32_t key_of_f32(float y)
{
    uint32_t b = f32_bits(y);
    if ((b & 0x7fffffffu) == 0u) b = 0u;  // canonical zero
    return b ^ ((b & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}

MIS_HD float f32_of_key(uint32_t k)
{
    uint32_t b = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
    return bits_f32(b);
}

MIS_HD uint32_t row_key(float y, int dt)
{
    if (dt == F32) return key_of_f32(y);
    if (y == 0.0f) y = 0.0f;
    uint16_t h = bits16_of(y, dt);
    uint16_t k = (uint16_t)(h ^ ((h & 0x8000u) ? 0xffffu : 0x8000u));
    return (uint32_t)k << 16;
}

MIS_HD float value_of_row_key(uint32_t k, int dt)
{
    if (dt == F32) return f32_of_key(k);
    uint16_t k16 = (uint16_t)(k >> 16);
    uint16_t h = (uint16_t)((k16 & 0x8000u) ? (k16 ^ 0x8000u) : (uint16_t)~k16);
    return f32_of_bits16(h, dt);
}

// Key for the greedy argmax over raw logits: NaN ranks above everything
// (torch.argmax returns the first NaN).
MIS_HD uint32_t argmax_key(float x) { return (x != x) ? 0xffffffffu : key_of_f32(x); }

// ---------------------------------------------------------- temperature division
//
// y = RN(x / T) from the row's reciprocal r = RN(1/T): q0 = RN(x * r) lies
// within 1.5 ulp of x / T, every residual x - q * T is then exact in one FMA,
// and two Newton corrections q + (x - q * T) * r give RN(x / T) (Markstein's
// theorem: the second correction starts from a faithful quotient).
// div_rcp_safe() names the inputs this holds for: quotients away from
// overflow, and x and quotients away from the range where a residual could
// underflow.  Elsewhere the callers divide.  tests/test_host_logic.py checks
// the pair bit for bit against IEEE x / T, exhaustively over every float x
// for one temperature and on samples for the configs' temperatures.
MIS_HD bool div_rcp_safe(float x, float q0)
{
    const float aq = fabsf(q0);
    return aq < 0x1p127f && aq >= 0x1p-100f && fabsf(x) >= 0x1p-100f;
}
MIS_HD float div_rcp_core(float x, float T, float r, float q0)
{
    const float e0 = fmaf(-q0, T, x);
    const float q1 = fmaf(e0, r, q0);
    const float e1 = fmaf(-q1, T, x);
    return fmaf(e1, r, q1);
}
MIS_HD float div_rcp(float x, float T, float r)
{
    const float q0 = x * r;
    return div_rcp_safe(x, q0) ? div_rcp_core(x, T, r, q0) : x / T;
}

// ---------------------------------------------------------- 16-bit top-p chain
//
// torch's top-p on fp16/bf16 tensors (model/sampler.py:48-51) evaluates, in
// sorted order, F_r = fl32(F_{r-1} + p_r) (sequential float accumulation of
// the dtype probabilities), C_r = RN16(F_r), E_r = RN16(fl32(C_r - p_r)) and
// removes rank r iff E_r >= RN16(top_p).  Tied values share one p, so the
// sequence is processed run by run; chain_add_n() gives F after adding the
// same p n times without looping over every addition.

// ulp and top of the binade that holds F (F > 0 finite)
MIS_HD void binade_of(float F, double *ulp, double *top)
{
    uint32_t b = f32_bits(F);
    uint32_t e = (b >> 23) & 0xffu;
    if (e == 0u) {  // subnormal: spacing 2^-149 up to 2^-126
        *ulp = bits_f64((uint64_t)(1023 - 149) << 52);
        *top = bits_f64((uint64_t)(1023 - 126) << 52);
    } else {
        int ee = (int)e - 127;
        *ulp = bits_f64((uint64_t)(1023 + ee - 23) << 52);
        *top = bits_f64((uint64_t)(1023 + ee + 1) << 52);
    }
}

// F <- fl32(F + p), repeated n times (p >= 0 finite, F >= 0 finite).
//
// Inside one binade of F (spacing u, N = F/u an integer) write p/u = q + r,
// 0 <= r < 1.  Round-to-nearest-even makes each step add q (r < 1/2) or
// q + 1 (r > 1/2) units; at r == 1/2 the first step lands on the even one of
// N+q, N+q+1 and every later step then adds the even one of q, q+1.  The
// closed form holds while the exact sum stays below the binade's top; the
// step that reaches past it is done as a plain float addition.
MIS_HD float chain_add_n(float F, float p, uint64_t n)
{
    if (p == 0.0f) return F;
    if (n <= 8u) {  // short runs: the additions themselves (cheaper than the closed form)
        for (uint64_t i = 0; i < n; ++i) F = F + p;
        return F;
    }
    while (n > 0) {
        if (F == 0.0f) { F = p; n -= 1; continue; }
        double u, top;
        binade_of(F, &u, &top);
        double P = (double)p / u;             // exact: u is a power of two
        int64_t lim = (int64_t)(top / u);     // 2^24 (2^23 for subnormals)
        int64_t N = (int64_t)((double)F / u);
        if (P >= (double)lim) {               // reaches the next binade at once
            F = F + p; n -= 1; continue;
        }
        int64_t q = (int64_t)P;               // floor, P >= 0
        double r = P - (double)q;
        int64_t inc1, inc;
        if (r < 0.5) { inc1 = q; inc = q; }
        else if (r > 0.5) { inc1 = q + 1; inc = q + 1; }
        else {
            inc1 = ((N + q) & 1) ? q + 1 : q;
            inc = (q & 1) ? q + 1 : q;
        }
        // step 0 stays inside the binade iff N + q + r < lim  <=>  N + q <= lim - 1
        if (N + q > lim - 1) { F = F + p; n -= 1; continue; }
        int64_t N1 = N + inc1;
        // later step i (pre-value N1 + (i-1)*inc) stays inside iff
        // (i-1)*inc + N1 + q <= lim - 1
        uint64_t s;
        int64_t room = lim - 1 - q - N1;
        if (room < 0) s = 1;
        else if (inc == 0) s = n;
        else s = 1u + (uint64_t)(room / inc) + 1u;
        if (s > n) s = n;
        int64_t Ns = N1 + (int64_t)(s - 1) * inc;
        F = (float)((double)Ns * u);
        n -= s;
        if (inc == 0 && inc1 == 0) return F;  // every remaining addition is absorbed
    }
    return F;
}

MIS_HD float chain_E(float F, float p, int dt)
{
    float C = rn_dtype(F, dt);
    float d = C - p;
    return rn_dtype(d, dt);
}

// ---------------------------------------------------------------- float64 exp
// e^d for d <= 0 in float64, relative error below DEXP_REL_ERR while the
// result is normal (subnormal results: absolute error below 2^-1074).
// Tang's table method: d * 64/ln2 rounds to n = 64q + j (0 <= j < 64),
// r = d - n * ln2/64 (|r| <= ln2/128) in two FMA steps with ln2/64 split
// into a head and a tail, e^r by its degree-5 Taylor polynomial (truncation
// below 4e-17), then e^d = 2^q * 2^(j/64) * e^r with 2^(j/64) from a table
// that exp_table() fills.
constexpr double DEXP_REL_ERR = 1e-15;
constexpr int ETAB_N = 64;
MIS_HD void exp_table(double *tab, int tid)
{
    if (tid < ETAB_N) tab[tid] = exp2((double)tid * (1.0 / ETAB_N));
}
MIS_HD double dexp(double d, const double *tab)
{
    if (!(d > -745.0)) return 0.0;
    const double n = rint(d * 92.33248261689366);  // 64 / ln2
    double r = fma(n, -0x1.62e42fefa39efp-7, d);   // ln2/64, head
    r = fma(n, -0x1.abc9e3b39803fp-62, r);         // ln2/64, tail
    const int ni = (int)n;
    double p = fma(r, 1.0 / 120.0, 1.0 / 24.0);
    p = fma(r, p, 1.0 / 6.0);
    p = fma(r, p, 0.5);
    p = fma(r, p, 1.0);
    p = fma(r, p, 1.0);
    return ldexp(tab[ni & (ETAB_N - 1)] * p, ni >> 6);
}

// ---------------------------------------------------------------- Philox RNG
//
// Philox4x32-10, the counter-based generator of Salmon, Moraes, Dror and Shaw,
// "Parallel random numbers: as easy as 1, 2, 3" (SC 2011): ten rounds of two
// 32x32->64-bit multiplies over a 128-bit counter, the 64-bit key advanced by
// the Weyl constants between rounds.  A function of (counter, key) alone, so
// any thread computes any request's draw without shared state.

constexpr uint32_t PHILOX_M0 = 0xD2511F53u, PHILOX_M1 = 0xCD9E8D57u;  // round multipliers
constexpr uint32_t PHILOX_W0 = 0x9E3779B9u, PHILOX_W1 = 0xBB67AE85u;  // key increments

MIS_HD void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1)
{
    for (int r = 0; r < 10; ++r) {
        if (r > 0) { k0 += PHILOX_W0; k1 += PHILOX_W1; }
        const uint64_t p0 = (uint64_t)PHILOX_M0 * c[0], p1 = (uint64_t)PHILOX_M1 * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[0] = n0; c[1] = (uint32_t)p1; c[2] = n2; c[3] = (uint32_t)p0;
    }
}

// The uniform of one draw: key = seed, counter = (step, request) as
// little-endian 32-bit words; the top 24 bits of the first output word give
// u = n * 2^-24 in [0, 1), exact in float.
MIS_HD float philox_uniform(uint64_t seed, uint64_t request, uint64_t step)
{
    uint32_t c[4] = {(uint32_t)step, (uint32_t)(step >> 32), (uint32_t)request, (uint32_t)(request >> 32)};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    return (float)(c[0] >> 8) * 5.9604644775390625e-08f;
}

}  // namespace mis
