/*
 * KVX paged-KV launch entry points, implemented with hand-written HIP
 * kernels for gfx950.
 *
 * Signatures, names and C linkage match the reference kernel header
 * (kernels/kvx_paged_kv.h:11-57).  Validation order and status codes follow
 * the reference launchers (kernels/kvx_paged_kv.cu:315-910).  All calls are
 * asynchronous on `stream` (a hipStream_t, NULL = default stream) and do not
 * synchronise the host.
 */
#ifndef KVX_PAGED_KV_H
#define KVX_PAGED_KV_H

#include "kvx_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Scatter K/V rows [num_tokens, H, D] into the paged cache at slot_mapping
 * positions; slot < 0 and block >= num_blocks are skipped.  Dispatches on
 * the cache dtype (F16/BF16/F32; F8_E4M3 quantizes with a per-tensor scale).
 * Replaces reference kvx_paged_kv.cu:472-491. */
KVX_API kvx_status_t kvx_launch_write_kv(const kvx_cache_desc_t *cache,
                                         const kvx_write_desc_t *write,
                                         void *stream);

/* Same scatter for prefill batches; tokens_per_seq must be > 0 and divide
 * num_tokens (validated only, as reference kvx_paged_kv.cu:493-514, 739-761). */
KVX_API kvx_status_t kvx_launch_write_kv_prefill(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream);

/* Gather a PACKED block table's sequences into contiguous
 * [seq_count, max_seq_len, H, D]; rows at or past seq_len, logical blocks
 * past max_blocks_per_seq and negative block ids are left untouched.
 * Replaces reference kvx_paged_kv.cu:891-910. */
KVX_API kvx_status_t kvx_launch_gather_kv(const kvx_cache_desc_t *cache,
                                          const kvx_gather_desc_t *gather,
                                          void *stream);

/* Per-dtype helpers: cache and io dtypes must both equal the suffix type,
 * else KVX_STATUS_UNSUPPORTED.  Replace reference kvx_paged_kv.cu:453-470,
 * :718-737 and :872-889. */
KVX_API kvx_status_t kvx_launch_write_kv_f32(const kvx_cache_desc_t *cache,
                                             const kvx_write_desc_t *write,
                                             void *stream);

KVX_API kvx_status_t kvx_launch_write_kv_f16(const kvx_cache_desc_t *cache,
                                             const kvx_write_desc_t *write,
                                             void *stream);

KVX_API kvx_status_t kvx_launch_write_kv_bf16(const kvx_cache_desc_t *cache,
                                              const kvx_write_desc_t *write,
                                              void *stream);

KVX_API kvx_status_t kvx_launch_write_kv_prefill_f32(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream);

KVX_API kvx_status_t kvx_launch_write_kv_prefill_f16(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream);

KVX_API kvx_status_t kvx_launch_write_kv_prefill_bf16(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream);

KVX_API kvx_status_t kvx_launch_gather_kv_f32(const kvx_cache_desc_t *cache,
                                              const kvx_gather_desc_t *gather,
                                              void *stream);

KVX_API kvx_status_t kvx_launch_gather_kv_f16(const kvx_cache_desc_t *cache,
                                              const kvx_gather_desc_t *gather,
                                              void *stream);

KVX_API kvx_status_t kvx_launch_gather_kv_bf16(const kvx_cache_desc_t *cache,
                                               const kvx_gather_desc_t *gather,
                                               void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KVX_PAGED_KV_H */
