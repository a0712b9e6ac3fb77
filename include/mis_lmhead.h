/*
 * mis_lmhead.h -- C ABI of the MI355X fused lm_head + greedy sampler
 * (libmis_sampler.so, built from vllm_mps_amd/csrc/mis_lmhead.hip).
 *
 * Reference path replaced, for greedy rows (temperature 0):
 *   - the logits producer: the model's lm_head, a Linear [V, H] without bias
 *     applied to the decode step's last hidden states, returning
 *     outputs.logits[:, 0, :] in the model dtype
 *       models/llama_adapter.py:198-207 (batched), :112-133 (one sequence)
 *   - the greedy branch of the sampler, argmax over those logits
 *       model/sampler.py:32-34, called per row from engine/llm_engine.py:339-345
 * The logits never reach HBM: the GEMM's epilogue keeps each vocabulary
 * tile's best (logit, index) per sequence and a second launch merges them.
 *
 * Contract: logit[b, v] = dtype(sum_h f32(x[b, h]) * f32(w[v, h])), the sum in
 * fp32 (exact products, fp32 accumulation; the order of the additions is the
 * kernel's), rounded once to the model dtype (round to nearest even);
 * ids[b] = argmax_v logit[b, v], ties to the lowest v, NaN above every number
 * (torch.argmax on the dtype logits).  All pointers are device pointers; the
 * calls are asynchronous on `stream`, allocate nothing and synchronise
 * nothing.
 */
#ifndef MIS_LMHEAD_H
#define MIS_LMHEAD_H

#include <stddef.h>
#include <stdint.h>

#include "mis_sampler.h"   /* mis_rng_row */

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MIS_LMH_OK = 0,
    MIS_LMH_ERR_INVALID_ARG = 1,   /* null pointer, negative size, misaligned rows */
    MIS_LMH_ERR_WORKSPACE = 2,     /* workspace missing, too small or not 256-byte aligned */
    MIS_LMH_ERR_HIP = 3,           /* a HIP launch failed */
    MIS_LMH_ERR_UNSUPPORTED = 4    /* H not a multiple of 64, dtype not fp16 / bf16, V or B too large */
};

/* Bytes of device workspace mis_lm_head_greedy() needs: one (key, index) pair
 * per (vocabulary tile of 128, sequence). */
size_t mis_lm_head_greedy_workspace_bytes(int64_t B, int64_t V);

/*
 * hidden [B, H] (row stride ldx elements), weight [V, H] (row stride ldw
 * elements), both of `dtype` (1 = fp16, 2 = bf16), rows 16-byte aligned;
 * ids [B] int64.
 */
int mis_lm_head_greedy(const void *hidden, int64_t ldx, const void *weight, int64_t ldw, int64_t B, int64_t H,
                       int64_t V, int dtype, int64_t *ids, void *workspace, size_t workspace_bytes, void *stream);

/*
 * The same GEMM with a sampling epilogue, for batches mixing greedy rows and
 * temperature-only rows (top-k 0, top-p 1: the engine's default parameters):
 *   temperature [B] (device f32): 0 = greedy (as mis_lm_head_greedy);
 *     T > 0: ids[b] = argmax_v (y[b, v] + g[b, v]), y = dtype(logit / T) (the
 *     quotient in fp32, rounded once to the dtype), g the Gumbel noise below:
 *     an exact draw from softmax(y) (the Gumbel-max theorem), replacing
 *     model/sampler.py:37 and :57-59 for such rows (torch.multinomial's generator
 *     becomes a per-request counter-based one);
 *     T < 0 or NaN: ids[b] = -1 (the reference's ValueError);
 *   rng [B] (device): the draw's key and counter, as mis_fill_uniforms:
 *     vocabulary rows v .. v + 3 (v a multiple of 4) take Philox4x32-10 with
 *     key (seed low, seed high ^ step high) and counter (v / 4, step low,
 *     request low, request high); output word i gives u = (w >> 8) * 2^-24 and
 *     g = -log(-log(u)) (u = 0: -inf).
 * A sampled row whose scaled logits hold NaN or +inf, or are all -inf, gets
 * id -1 (the reference's torch.multinomial RuntimeError).  Top-k and top-p
 * rows are not served here (their cuts need the whole row): run the GEMM and
 * mis_sample.  The workspace is mis_lm_head_greedy_workspace_bytes(B, V).
 */
int mis_lm_head_sample(const void *hidden, int64_t ldx, const void *weight, int64_t ldw, int64_t B, int64_t H,
                       int64_t V, int dtype, const float *temperature, const mis_rng_row *rng, int64_t *ids,
                       void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MIS_LMHEAD_H */
