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
 * the cache dtype: F16/BF16/F32 copy; an F8_E4M3 or F8_E5M2 cache with
 * F16/BF16/F32 io quantizes with per-tensor, per-head, per-block or
 * per-block-head scales (kvx_ext.h).
 * Replaces reference kvx_paged_kv.cu:472-491. */
KVX_API kvx_status_t kvx_launch_write_kv(const kvx_cache_desc_t *cache,
                                         const kvx_write_desc_t *write,
                                         void *stream);

/* Same scatter for prefill batches; tokens_per_seq must be > 0 and divide
 * num_tokens (validated only, as reference kvx_paged_kv.cu:493-514, 739-761). */
KVX_API kvx_status_t kvx_launch_write_kv_prefill(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream);

/* Gather the sequences of a PACKED, RAGGED or KV_OFFSETS block table
 * (kvx_ext.h) into contiguous [seq_count, max_seq_len, H, D]; rows at or
 * past seq_len, logical blocks past max_blocks_per_seq, and rows whose block
 * id is < 0 or >= num_blocks are left untouched (the reference skips only
 * negative ids and reads larger ones out of bounds).  A batch whose launch
 * grid would exceed HIP's limits (2^32 - 1 work-items per dimension) returns
 * KVX_STATUS_UNSUPPORTED without launching.
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
