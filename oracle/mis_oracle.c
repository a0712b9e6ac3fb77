/*
 * mis_oracle.c -- CPU restatement of the reference token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may.  It exists to be the checker the HIP kernels are
 * compared against.
 *
 * Reference algorithm: model/sampler.py:18-60 (Sampler.sample), applied per
 * row as in engine/llm_engine.py:339-345, with SamplingParams from
 * core/sequence.py:23-61.  Steps, with the reference line each follows:
 *
 *   greedy      sampler.py:33-34   T == 0 -> argmax(raw logits), ties -> lowest
 *                                  index, a NaN counts as the maximum (torch).
 *   temperature sampler.py:37      y = dtype(f32(x) / f32(T)); torch divides by
 *                                  the Python float cast to f32 (probed).
 *   top-k       sampler.py:40-43   k' = min(k, V); thr = k'-th largest y (with
 *                                  multiplicity); y < thr -> -inf.  Ties with
 *                                  thr are all kept.
 *   top-p       sampler.py:46-55   only if top_p < 1.  Order = stable sort of
 *                                  y descending (ties -> lowest index first;
 *                                  the reference's unstable sort has no fixed
 *                                  tie order, this is the contract choice).
 *       fp32:  masses in exact arithmetic (long double here): p = softmax,
 *              E_r = sum_{i<r} p_i, remove iff E_r >= f32(top_p).
 *       fp16/bf16: the dtype rounding chain torch runs:
 *              p16 = RN16(RN32(softmax)), F_r = fl32(F_{r-1} + p16_r)
 *              (sequential float accumulation), C_r = RN16(F_r),
 *              E_r = RN16(fl32(C_r - p16_r)), remove iff E_r >= RN16(top_p).
 *   draw        sampler.py:58-60   contract replacement for torch.multinomial:
 *                                  inverse CDF in vocabulary order,
 *                                  token = min{i : sum_{j<=i} w_j > u*sum w}
 *                                  over the unnormalised kept weights
 *                                  w_j = exp(z_j - m); clamped to the last kept
 *                                  index.
 *
 * Row status: 0 ok, 1 bad parameter (T < 0, top_k < 0, top_p <= 0 or NaN),
 * 2 invalid distribution (T NaN, NaN or +inf scaled logits, or nothing kept;
 * torch.multinomial raises on these).  ids = -1 for rows with status != 0.
 *
 * Debug outputs: probs[j] = RN_dtype(RN32(softmax over kept)) as float, 0 for
 * removed; keep[j] = 1 iff the post-filter logit is > -inf.  Greedy rows get a
 * one-hot probs/keep at the argmax.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };
enum { ORC_OK = 0, ORC_BAD_PARAM = 1, ORC_INVALID = 2 };

typedef struct {
    float temperature;
    int32_t top_k;
    float top_p;
    float uniform;
} orc_params;

/* ---------------------------------------------------------------- dtypes */

static float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0x1f) return u32_as_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in float */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u32_as_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* Round-to-nearest-even float -> half (IEEE binary16), with subnormals. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t u = f32_as_u32(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) { /* below 2^-14: subnormal or zero in half */
        /* value in units of 2^-24, rounded to nearest even */
        float v = u32_as_f32(a);
        double units = (double)v * 16777216.0; /* exact: v has <= 24 bits */
        double fl = floor(units);
        double fr = units - fl;
        uint32_t q = (uint32_t)fl;
        if (fr > 0.5 || (fr == 0.5 && (q & 1u))) q++;
        return (uint16_t)(sign | q); /* q may reach 0x400 = min normal: fine */
    }
    uint32_t e = (a >> 23) - 112u; /* half exponent field 1..30 */
    uint32_t m = a & 0x7fffffu;
    uint32_t hm = m >> 13, rest = m & 0x1fffu;
    uint32_t h = (e << 10) | hm;
    if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) h++; /* carries into e */
    return (uint16_t)(sign | h);
}

float orc_bf16_to_f32(uint16_t h) { return u32_as_f32((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t u = f32_as_u32(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t rest = u & 0xffffu, h = u >> 16;
    if (rest > 0x8000u || (rest == 0x8000u && (h & 1u))) h++;
    return (uint16_t)h;
}

/* Round a float to the dtype and return it as float. */
float orc_rn_dtype(float f, int dt)
{
    if (dt == ORC_F16) return orc_f16_to_f32(orc_f32_to_f16(f));
    if (dt == ORC_BF16) return orc_bf16_to_f32(orc_f32_to_bf16(f));
    return f;
}

static float load_elem(const void *row, int64_t j, int dt)
{
    if (dt == ORC_F32) return ((const float *)row)[j];
    uint16_t h = ((const uint16_t *)row)[j];
    return dt == ORC_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}

/* Temperature scaling, sampler.py:37: dtype(f32(x) / f32(T)).  The volatile
 * keeps the quotient a true binary32 division. */
float orc_scale(float x, float T, int dt)
{
    volatile float q = x / T;
    return orc_rn_dtype(q, dt);
}

/* ------------------------------------------------------------- ordering */

typedef struct { float y; int64_t idx; } orc_item;

/* descending by value, ties by ascending index (stable sort contract) */
static int cmp_desc(const void *a, const void *b)
{
    const orc_item *x = (const orc_item *)a, *y = (const orc_item *)b;
    if (x->y > y->y) return -1;
    if (x->y < y->y) return 1;
    return (x->idx < y->idx) ? -1 : (x->idx > y->idx);
}

/* -------------------------------------------------------------- one row */

typedef struct {
    int64_t id;
    int32_t status;
    double topp_margin;  /* fp32: min |E_r - thr| over the two ranks at the cut */
    double draw_margin;  /* |cum - u*S| / S at the nearest CDF edge of the draw */
    float cut_value;     /* post-filter cut: keep y > v or (y == v and j <= idx) */
    int64_t cut_index;
    int64_t n_kept;
} orc_row_result;

static void row_sample(int dt, int64_t V, const void *row, orc_params P,
                       float *probs, uint8_t *keep, orc_row_result *R,
                       orc_item *items, long double *w)
{
    R->id = -1; R->status = ORC_OK; R->topp_margin = NAN; R->draw_margin = NAN;
    R->cut_value = NAN; R->cut_index = -1; R->n_kept = 0;
    if (probs) memset(probs, 0, sizeof(float) * (size_t)V);
    if (keep) memset(keep, 0, (size_t)V);

    float T = P.temperature;
    if (T < 0.0f || P.top_k < 0 || !(P.top_p > 0.0f)) { R->status = ORC_BAD_PARAM; return; }
    /* T = NaN passes SamplingParams' check (core/sequence.py:43: NaN < 0 is
       false); logits / NaN is NaN and torch.multinomial raises (:59) */
    if (T != T) { R->status = ORC_INVALID; return; }

    if (T == 0.0f) { /* greedy, sampler.py:33-34 */
        int64_t best = 0;
        float bv = load_elem(row, 0, dt);
        if (!isnan(bv)) {
            for (int64_t j = 1; j < V; ++j) {
                float v = load_elem(row, j, dt);
                if (isnan(v)) { best = j; break; }
                if (v > bv) { bv = v; best = j; }
            }
        }
        R->id = best; R->n_kept = 1;
        R->cut_value = load_elem(row, best, dt); R->cut_index = best;
        if (probs) probs[best] = 1.0f;
        if (keep) keep[best] = 1;
        return;
    }

    /* temperature, sampler.py:37 */
    for (int64_t j = 0; j < V; ++j) {
        float y = orc_scale(load_elem(row, j, dt), T, dt);
        if (isnan(y) || y == INFINITY) { R->status = ORC_INVALID; return; }
        items[j].y = y; items[j].idx = j;
    }
    qsort(items, (size_t)V, sizeof(orc_item), cmp_desc);
    /* items[] is now the stable descending order */

    /* top-k, sampler.py:40-43: keep y >= thr (all ties with thr kept) */
    int64_t nk = V; /* number of ranks surviving top-k (a prefix of items) */
    if (P.top_k > 0) {
        int64_t kk = P.top_k < V ? P.top_k : V;
        float thr = items[kk - 1].y;
        nk = kk;
        while (nk < V && items[nk].y >= thr) nk++;
    }
    /* ranks >= nk and ranks whose y is -inf carry zero mass */
    int64_t nfin = nk;
    while (nfin > 0 && items[nfin - 1].y == -INFINITY) nfin--;
    if (nfin == 0) { R->status = ORC_INVALID; return; }
    float m = items[0].y;

    long double S = 0.0L;
    for (int64_t r = 0; r < nfin; ++r) { w[r] = expl((long double)items[r].y - (long double)m); }
    for (int64_t r = nfin - 1; r >= 0; --r) S += w[r]; /* small to large */

    /* top-p, sampler.py:46-55 */
    int64_t nkeep = nfin;
    if (P.top_p < 1.0f) {
        if (dt == ORC_F32) {
            long double thr = (long double)P.top_p, E = 0.0L;
            int64_t r;
            for (r = 0; r < nfin; ++r) {
                if (E >= thr) break;           /* rank r removed */
                E += w[r] / S;
            }
            nkeep = r;
            /* margins of the decisions at rank nkeep-1 (kept) and nkeep (removed) */
            long double Ekept = 0.0L;
            for (int64_t i = 0; i + 1 < nkeep; ++i) Ekept += w[i] / S;
            double mg = fabs((double)(Ekept - thr));
            if (nkeep < nfin) {
                double m2 = fabs((double)(E - thr));
                if (m2 < mg) mg = m2;
            }
            R->topp_margin = mg;
        } else {
            float thr16 = orc_rn_dtype(P.top_p, dt);
            float F = 0.0f;
            int64_t r;
            for (r = 0; r < nfin; ++r) {
                float p16 = orc_rn_dtype((float)(w[r] / S), dt);
                volatile float Fn = F + p16;
                F = Fn;
                float C = orc_rn_dtype(F, dt);
                volatile float d = C - p16;
                float E = orc_rn_dtype(d, dt);
                if (E >= thr16) break;
            }
            nkeep = r;
        }
        if (nkeep == 0) { R->status = ORC_INVALID; return; }
    }
    R->n_kept = nkeep;
    R->cut_value = items[nkeep - 1].y;
    R->cut_index = items[nkeep - 1].idx;

    /* final softmax over kept ranks + inverse-CDF draw in vocabulary order,
     * sampler.py:58-60.  Kept set = ranks [0, nkeep). */
    long double SK = 0.0L;
    for (int64_t r = nkeep - 1; r >= 0; --r) SK += w[r];
    /* scatter weights back to vocabulary order (reuse probs as a flag) */
    long double *wv = (long double *)calloc((size_t)V, sizeof(long double));
    uint8_t *kv = (uint8_t *)calloc((size_t)V, 1);
    for (int64_t r = 0; r < nkeep; ++r) { wv[items[r].idx] = w[r]; kv[items[r].idx] = 1; }
    long double target = (long double)P.uniform * SK, cum = 0.0L, prev = 0.0L;
    int64_t tok = -1, last = -1;
    for (int64_t j = 0; j < V; ++j) {
        if (!kv[j]) continue;
        last = j;
        prev = cum;
        cum += wv[j];
        if (tok < 0 && cum > target) {
            tok = j;
            double a = fabs((double)((cum - target) / SK)), b = fabs((double)((target - prev) / SK));
            R->draw_margin = a < b ? a : b;
        }
    }
    if (tok < 0) { tok = last; R->draw_margin = fabs((double)((cum - target) / SK)); }
    R->id = tok;
    if (probs || keep) {
        for (int64_t j = 0; j < V; ++j) {
            if (!kv[j]) continue;
            if (keep) keep[j] = 1;
            if (probs) probs[j] = orc_rn_dtype((float)(wv[j] / SK), dt);
        }
    }
    free(wv); free(kv);
}

/* ------------------------------------------------------------ batch API */

/*
 * logits: B rows of V elements (row stride `stride` elements), dtype dt.
 * Optional outputs may be NULL: probs [B*V] float, keep [B*V] bytes,
 * topp_margin/draw_margin [B] double, cut_value [B] float, cut_index [B],
 * n_kept [B].
 */
int orc_sample_rows(int dt, int64_t B, int64_t V, int64_t stride, const void *logits,
                    const orc_params *P, int64_t *ids, int32_t *status, float *probs,
                    uint8_t *keep, double *topp_margin, double *draw_margin,
                    float *cut_value, int64_t *cut_index, int64_t *n_kept)
{
    if (dt < 0 || dt > 2 || B < 0 || V <= 0 || stride < V) return -1;
    size_t esz = dt == ORC_F32 ? 4 : 2;
    int err = 0;
#pragma omp parallel
    {
        orc_item *items = (orc_item *)malloc(sizeof(orc_item) * (size_t)V);
        long double *w = (long double *)malloc(sizeof(long double) * (size_t)V);
        if (!items || !w) {
#pragma omp atomic write
            err = -2;
        }
#pragma omp for schedule(dynamic, 1)
        for (int64_t b = 0; b < B; ++b) {
            if (!items || !w) continue;
            orc_row_result R;
            const char *row = (const char *)logits + (size_t)b * (size_t)stride * esz;
            row_sample(dt, V, row, P[b], probs ? probs + b * V : NULL,
                       keep ? keep + b * V : NULL, &R, items, w);
            ids[b] = R.id;
            if (status) status[b] = R.status;
            if (topp_margin) topp_margin[b] = R.topp_margin;
            if (draw_margin) draw_margin[b] = R.draw_margin;
            if (cut_value) cut_value[b] = R.cut_value;
            if (cut_index) cut_index[b] = R.cut_index;
            if (n_kept) n_kept[b] = R.n_kept;
        }
        free(items); free(w);
    }
    return err;
}

/* Element-wise helpers exposed for the pinning tests. */
void orc_scale_array(int dt, int64_t n, const void *x, float T, float *y)
{
    for (int64_t j = 0; j < n; ++j) y[j] = orc_scale(load_elem(x, j, dt), T, dt);
}

void orc_round_array(int dt, int64_t n, const float *x, float *y)
{
    for (int64_t j = 0; j < n; ++j) y[j] = orc_rn_dtype(x[j], dt);
}

/* ------------------------------------------------------------- uniforms
 *
 * The per-request uniforms of the device generator: Philox4x32-10 (Salmon,
 * Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3",
 * SC 2011), the draw's replacement for torch.multinomial's global generator
 * (model/sampler.py:59).  Restated from the paper's definition:
 *   round:  (L0, R0, L1, R1) -> (hi(M1*L1) ^ k0 ^ R0, lo(M1*L1),
 *                                hi(M0*L0) ^ k1 ^ R1, lo(M0*L0))
 *   key schedule: k += (0x9E3779B9, 0xBB67AE85) before every round but the
 *   first; ten rounds.
 * Pinned by the known-answer vectors the authors publish with Random123.
 * Uniform: key = seed (low word first), counter = (step lo, step hi,
 * request lo, request hi); u = (first output word >> 8) / 2^24.
 */
static void orc_mulhilo(uint32_t a, uint32_t b, uint32_t *hi, uint32_t *lo)
{
    const uint64_t p = (uint64_t)a * (uint64_t)b;
    *hi = (uint32_t)(p >> 32);
    *lo = (uint32_t)(p & 0xffffffffu);
}

void orc_philox4x32_10(const uint32_t in[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t L0 = in[0], R0 = in[1], L1 = in[2], R1 = in[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        uint32_t hi0, lo0, hi1, lo1;
        orc_mulhilo(0xD2511F53u, L0, &hi0, &lo0);
        orc_mulhilo(0xCD9E8D57u, L1, &hi1, &lo1);
        const uint32_t a = hi1 ^ k0 ^ R0, b = lo1, c = hi0 ^ k1 ^ R1, d = lo0;
        L0 = a; R0 = b; L1 = c; R1 = d;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = L0; out[1] = R0; out[2] = L1; out[3] = R1;
}

void orc_uniforms(int64_t n, const uint64_t *seed, const uint64_t *request, const uint64_t *step, float *u)
{
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t ctr[4] = {(uint32_t)step[i], (uint32_t)(step[i] >> 32), (uint32_t)request[i],
                                 (uint32_t)(request[i] >> 32)};
        const uint32_t key[2] = {(uint32_t)seed[i], (uint32_t)(seed[i] >> 32)};
        uint32_t out[4];
        orc_philox4x32_10(ctr, key, out);
        u[i] = (float)ldexp((double)(out[0] >> 8), -24);
    }
}
