/*
 * mis_attention.h -- C ABI of the MI355X decode-step paged attention kernel
 * (libmis_sampler.so, built from vllm_mps_amd/csrc/mis_attn.hip).
 *
 * Reference interfaces replaced:
 *   - fused_attention_metal_fast(pool, new_k, new_v, queries, bt_tensor,
 *     sl_tensor, write_info, n_heads, n_kv_heads, d_k, block_size)
 *       kernels/__init__.py:320-368 (the MSL kernel fused_attention,
 *       kernels/__init__.py:79-243), called from
 *       layers/paged_attention_layer.py:289-313
 *   - gather_kv_metal(pool, block_tables, seq_lens, max_seq_len)
 *       kernels/__init__.py:279-311 (the MSL kernel gather_kv,
 *       kernels/__init__.py:25-72)
 *
 * Pool: [num_blocks, 2 (K, V), block_size, n_kv_heads, d_k] fp16 as the
 * reference allocates it (memory/mps_memory_pool.py:62), element strides
 * pool_stride0 (per block) and pool_stride1 (K -> V); 16-byte aligned, both
 * strides multiples of 8 elements.  All pointers are device pointers; the
 * calls are asynchronous on `stream`, allocate nothing and synchronise
 * nothing.  Sequence lengths beyond max_blocks * block_size and block ids
 * outside [0, num_blocks) are clamped into range (never read outside the
 * buffers); a write_info outside the pool skips the write.
 */
#ifndef MIS_ATTENTION_H
#define MIS_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MIS_ATT_OK = 0,
    MIS_ATT_ERR_INVALID_ARG = 1,   /* null pointer, negative size, misaligned pool / new_k / new_v */
    MIS_ATT_ERR_WORKSPACE = 2,     /* workspace missing, too small or not 256-byte aligned */
    MIS_ATT_ERR_HIP = 3,           /* a HIP launch failed */
    MIS_ATT_ERR_UNSUPPORTED = 4    /* d_k not 64 / 128 / 256, n_heads / n_kv_heads above 16 or not whole */
};

/* Bytes of device workspace mis_paged_attention() needs for a call of B
 * sequences and max_context = max_blocks * block_size tokens (contexts are
 * split over workgroups of 64-256 tokens and merged; one split needs none,
 * and 256 is returned). */
size_t mis_paged_attention_workspace_bytes(int64_t B, int n_heads, int n_kv_heads, int d_k, int max_context);

/*
 * One decode step of attention for B sequences: writes new_k / new_v
 * [B, n_kv_heads, d_k] into the pool at write_info [B, 2] = (block,
 * position), then for every query head h (KV head h / (n_heads /
 * n_kv_heads)) out[b, h] = softmax(q[b, h] . K_t / sqrt(d_k)) . V_t over the
 * seq_lens[b] tokens of block_tables [B, max_blocks] (the last of them the
 * new token).  queries [B, n_heads, d_k] and out [B, n_heads, d_k] fp16;
 * arithmetic in fp32.  write_info[b] names the slot of token seq_lens[b] - 1,
 * as the engine's does (layers/paged_attention_layer.py:289-313); that
 * token's K / V are taken from new_k / new_v, the others from the pool.
 */
int mis_paged_attention(void *pool, int64_t num_blocks, int block_size, int n_kv_heads, int d_k,
                        int64_t pool_stride0, int64_t pool_stride1, const void *new_k, const void *new_v,
                        const void *queries, const int32_t *block_tables, int max_blocks,
                        const int32_t *seq_lens, const int32_t *write_info, int64_t B, int n_heads, void *out,
                        void *workspace, size_t workspace_bytes, void *stream);

/*
 * The pool gathered into out_k / out_v [B, max_seq_len, n_kv_heads, d_k]
 * fp16 (tokens past seq_lens[b] are zero).
 */
int mis_gather_kv(const void *pool, int64_t num_blocks, int block_size, int n_kv_heads, int d_k,
                  int64_t pool_stride0, int64_t pool_stride1, const int32_t *block_tables, int max_blocks,
                  const int32_t *seq_lens, int64_t B, int max_seq_len, void *out_k, void *out_v, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MIS_ATTENTION_H */
