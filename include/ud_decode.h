/*
 * ud_decode.h -- C ABI of the gfx950 decoder attention: grouped-query attention over a paged
 * K/V cache for one new token per sequence, the rotate-half RoPE and the paged cache append.
 *
 * This is the decode-step attention of DictatorEngine's Voxtral decoder (one token per sequence,
 * or up to 8 positions per sequence, Sources/DictatorEngine/Models/Voxtral.swift:347-397), batched
 * over independent sequences whose
 * K/V caches live in fixed-size pages instead of the reference's per-session sliding window
 * (SlidingKV, Voxtral.swift:206-250).  Conventions are those of ud_encoder.h: 0 or a negative
 * ud_status, message in ud_last_error(), device pointers *_dev, asynchronous on hip_stream.
 *
 * Paged cache layout (this library's): k_pages / v_pages hold `num_blocks` pages of
 * [kv_heads][block_size][head_dim] elements (one kv head's rows of a page are contiguous).
 * block_table [n][max_blocks] int32 maps logical block b of sequence i (keys b*block_size ..
 * b*block_size + block_size - 1) to a page.  Entries are read only for blocks that hold a key of
 * the sequence's range; other entries may be anything.
 */
#ifndef UD_DECODE_H
#define UD_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "ud_encoder.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces Step.attention (Sources/DictatorEngine/Core/Ops.swift:136-169) and its kernels
 * attention_gqa / attention_mq_split + attention_combine
 * (Sources/DictatorEngine/Metal/30_voxtral.metal:45-101, 240-338) for one query token per
 * sequence, reading keys through the page table:
 *   out[i, h] = sum_j softmax_j(q[i, h] . k[i, j, h / (Hq/Hkv)] / sqrt(head_dim)) v[i, j, kvh]
 *   over logical keys j in [ranges[i].x, ranges[i].y) (0 if empty).
 *   q_dev        fp32 [n, q_heads * head_dim] (already rotated)
 *   k/v_pages    kv_dtype (UD_BF16 or UD_F16), layout above
 *   block_table  int32 [n, max_blocks]
 *   ranges_dev   int32 [n, 2] logical key range per sequence; ranges[i].y <= max_blocks*block_size
 *   out_dev      fp32 [n, q_heads * head_dim]
 *   max_keys     an upper bound of ranges[i].y over the batch (sizes the grid)
 *   workspace    device scratch of ud_gqa_workspace_bytes(n, q_heads, head_dim, max_keys) bytes
 * Supported: head_dim in {64, 128}, q_heads % kv_heads == 0, q_heads / kv_heads in {1, 2, 4, 8},
 * block_size 16, n <= 65535, max_keys <= 65535 * 128 (UD_ERR_SHAPE otherwise).
 * Precision: f16 pages are widened and used in fp32 arithmetic, as the reference kernel does.
 * bf16 pages use packed bf16 dot products: q and the softmax probabilities are rounded once to
 * bf16 (products exact, sums in fp32), within the bf16 activation bar (max abs 2e-2, cosine
 * 0.9995). */
UD_API size_t ud_gqa_workspace_bytes(int32_t n, int32_t q_heads, int32_t head_dim, int32_t max_keys);
UD_API int ud_gqa_attention_paged(int32_t kv_dtype, const float* q_dev, const void* k_pages, const void* v_pages,
                                  const int32_t* block_table, int32_t max_blocks, const int32_t* ranges_dev,
                                  float* out_dev, int32_t n, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                  int32_t block_size, int32_t max_keys, void* workspace, size_t workspace_bytes,
                                  void* hip_stream);

/* Replaces Step.attention with 2 .. 8 queries (Ops.swift:141-162 -> attention_mq_split_f16 +
 * attention_combine, 30_voxtral.metal:240-338; the M positions VoxtralSession.decode passes per
 * call, Voxtral.swift:347-371): n_queries (1 .. 8) query rows per sequence, each with its own key
 * range, over the sequence's pages; every K/V page is read once for all of them.
 *   q_dev        fp32 [n, n_queries, q_heads * head_dim]
 *   ranges_dev   int32 [n, n_queries, 2]: query m of sequence i attends to keys
 *                [ranges[i][m].x, ranges[i][m].y) (0 if empty)
 *   out_dev      fp32 [n, n_queries, q_heads * head_dim]
 *   workspace    ud_gqa_workspace_bytes(n * n_queries, q_heads, head_dim, max_keys) bytes
 * Block-table entries are read for the blocks between the lowest start and the highest end of a
 * sequence's non-empty query ranges.  Otherwise as ud_gqa_attention_paged (formula, formats,
 * precision, limits; n * n_queries <= 65535), which is this call with n_queries = 1. */
UD_API int ud_gqa_attention_paged_mq(int32_t kv_dtype, const float* q_dev, const void* k_pages, const void* v_pages,
                                     const int32_t* block_table, int32_t max_blocks, const int32_t* ranges_dev,
                                     float* out_dev, int32_t n, int32_t n_queries, int32_t q_heads, int32_t kv_heads,
                                     int32_t head_dim, int32_t block_size, int32_t max_keys, void* workspace,
                                     size_t workspace_bytes, void* hip_stream);

/* Allocation-free variant of ud_gqa_attention_paged.  It has no counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * ud_gqa_attention_paged, minus the workspace: the split partials go to a static device array of
 * UD_GQA_NOALLOC_SCRATCH_BYTES per device, held until the process ends (its address is looked up
 * on the first call on each device).  The call allocates and frees nothing.
 * Limit: ud_gqa_workspace_bytes(n, q_heads, head_dim, max_keys) <= UD_GQA_NOALLOC_SCRATCH_BYTES
 * (e.g. 64 sequences x 32 query heads x 4096 keys at head_dim 128 use 32.5 MiB); larger calls
 * return UD_ERR_SHAPE before anything is launched.  Every call on one device shares that device's
 * array: calls that overlap on one device (on different HIP streams, or from several threads)
 * race and must be serialised by the caller.  Nothing in the array needs to start at zero. */
#define UD_GQA_NOALLOC_SCRATCH_BYTES (40u << 20)
UD_API int ud_gqa_attention_paged_noalloc(int32_t kv_dtype, const float* q_dev, const void* k_pages,
                                          const void* v_pages, const int32_t* block_table, int32_t max_blocks,
                                          const int32_t* ranges_dev, float* out_dev, int32_t n, int32_t q_heads,
                                          int32_t kv_heads, int32_t head_dim, int32_t block_size, int32_t max_keys,
                                          void* hip_stream);

/* Replaces Step.rope (Ops.swift rope) / rope_rotate_half (30_voxtral.metal:20-36): in place on
 * x [rows, ld] (dtype UD_F32, UD_BF16 or UD_F16), heads H of head_dim d starting at column 0:
 *   angle = pos(t) * inv_freq[i];  x_i' = x_i cos - x_{i+d/2} sin;  x_{i+d/2}' = x_{i+d/2} cos + x_i sin
 * pos(t) = positions_dev[t] when positions_dev is non-null, else pos0 + t.  inv_freq_dev fp32
 * [d/2] (the reference builds it as 1 / theta^(2i/d), Voxtral.swift:176-179). */
UD_API int ud_rope_rotate_half(int32_t dtype, void* x_dev, int32_t rows, int32_t heads, int32_t head_dim, int32_t ld,
                               const int32_t* positions_dev, int32_t pos0, const float* inv_freq_dev, void* hip_stream);

/* Replaces the K/V writes into the session cache (the projections write rows of SlidingKV,
 * Voxtral.swift:371-376): copies row i of k_new / v_new ([n, kv_heads*head_dim], kv_dtype) to
 * logical position positions_dev[i] of sequence i in the paged cache. */
UD_API int ud_paged_kv_append(int32_t kv_dtype, const void* k_new, const void* v_new, void* k_pages, void* v_pages,
                              const int32_t* block_table, int32_t max_blocks, const int32_t* positions_dev, int32_t n,
                              int32_t kv_heads, int32_t head_dim, int32_t block_size, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif
