/*
 * Extensions to the KVX v1 ABI that kvx_abi.h cannot carry unchanged.
 *
 * FP8 KV cache (OCP E4M3 "e4m3fn", KVX_DTYPE_F8_E4M3, or OCP E5M2,
 * KVX_DTYPE_F8_E5M2) with F32 scales:
 *
 *   write:  kvx_launch_write_kv / kvx_launch_write_kv_prefill with an FP8
 *           cache and io of dtype F16, BF16 or F32.  The scale is read from
 *           write->k_scale_desc / v_scale_desc when their `data` is non-NULL,
 *           otherwise from write->k_scale / v_scale as one F32 each
 *           (KVX_SPEC.md:258-259).  Scale pointers are device pointers, read
 *           by the kernel.
 *             q = fp8_rne(saturate(f32(x) / scale))
 *           saturating to +-448 (E4M3) / +-57344 (E5M2), infinities included;
 *           NaN -> 0x7F (E4M3) / 0x7E (E5M2).  With io of the cache's own
 *           FP8 dtype the bytes are copied unscaled.
 *
 *   gather: kvx_launch_gather_kv_dequant below, because kvx_gather_desc_t
 *           (reference kvx_abi.h:182-188) has no scale fields.
 *             y = round_to_io_dtype(f32(q) * scale)   (RNE; NaN -> quiet NaN)
 *           kvx_launch_gather_kv with an FP8 cache and the same FP8 io copies
 *           bytes.
 *
 * Scale descriptors (kvx_scale_desc_t, dtype F32; strides in elements; the
 * field names are the spec's, KVX_SPEC.md:190-197, the shapes this build's):
 *   PER_TENSOR      data[0]
 *   PER_HEAD        ndim 1, shape [num_kv_heads]
 *   PER_BLOCK       ndim 1, shape [num_blocks], indexed by physical block id
 *   PER_BLOCK_HEAD  ndim 2, shape [num_blocks, num_kv_heads]
 * A wrong shape is KVX_STATUS_INVALID_ARGUMENT; other granularities and
 * dtypes, and block-indexed scales on KV_OFFSETS gathers, are
 * KVX_STATUS_UNSUPPORTED.
 *
 * The reference has no FP8 kernels (KVX_CONFORMANCE.md:24, :35); this is new
 * functionality.
 *
 * Block-table formats beyond PACKED (KVX_SPEC.md:99-122), gathered by
 * kvx_launch_gather_kv, kvx_launch_gather_kv_dequant and kvx_gather_kv (the
 * reference returns UNSUPPORTED for them, kernels/kvx_paged_kv.cu:788-790):
 *   RAGGED      row t of sequence s is token indptr[s] + t, valid for
 *               t < indptr[s+1] - indptr[s]; its block id is indices[token]
 *               (skipped when < 0 or >= num_blocks), its offset t % block_size.
 *   KV_OFFSETS  int32 KVCacheIndex entries [seq_count, 1, 2, max_blocks_per_seq]
 *               (K then V): bit 31 selects the secondary pool, bits 0-30 the
 *               block; the block's address is pool + index * bytes_per_block.
 *               An entry is skipped when its index is >= num_blocks or its
 *               pool is NULL.  kvx_pool_desc_t carries no pool sizes, so
 *               through kvx_launch_gather_kv, kvx_launch_gather_kv_dequant and
 *               kvx_gather_kv BOTH pools must hold at least num_blocks blocks
 *               of bytes_per_block bytes: a smaller secondary pool (an offload
 *               pool, say) is read out of bounds by indices between its size
 *               and num_blocks.  kvx_launch_gather_kv_pools below takes each
 *               pool's block count and skips the entries past it.
 */
#ifndef KVX_EXT_H
#define KVX_EXT_H

#include "kvx_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Dequantizing gather from an F8_E4M3 or F8_E5M2 paged cache into an
 * F16/BF16/F32 [seq_count, max_seq_len, H, D] buffer, over any block-table
 * format.  Same validation order, codes and untouched-row semantics as
 * kvx_launch_gather_kv; k_scale / v_scale must be non-NULL F32 scale
 * descriptors (granularities above) whose data is a device pointer.
 * No reference counterpart (the reference gather returns UNSUPPORTED for FP8,
 * kernels/kvx_paged_kv.cu:900-909). */
KVX_API kvx_status_t kvx_launch_gather_kv_dequant(
    const kvx_cache_desc_t *cache, const kvx_gather_desc_t *gather,
    const kvx_scale_desc_t *k_scale, const kvx_scale_desc_t *v_scale,
    void *stream);

/* Block counts of the two pools of a KV_OFFSETS table (kvx_pool_desc_t,
 * reference kvx_abi.h:84-90, has none).  A count of 0, or one of
 * num_blocks or more, means num_blocks. */
typedef struct kvx_pool_blocks_t {
  uint32_t size; /* sizeof(kvx_pool_blocks_t) */
  uint32_t reserved;
  int64_t primary;   /* blocks in cache->pool.primary */
  int64_t secondary; /* blocks in cache->pool.secondary */
} kvx_pool_blocks_t;

/* kvx_launch_gather_kv (k_scale and v_scale NULL) or
 * kvx_launch_gather_kv_dequant (both non-NULL), with a KV_OFFSETS entry also
 * skipped when its index is at or past its pool's count in pool_blocks, so
 * that a secondary pool smaller than num_blocks is never read past its end.
 * pool_blocks may be NULL (no narrowing); it is not read for PACKED and
 * RAGGED tables.  KVX_STATUS_INVALID_ARGUMENT for a pool_blocks->size below
 * sizeof(kvx_pool_blocks_t), a negative count, or one scale descriptor
 * without the other; otherwise the same validation order and codes as the
 * gather it stands for.  No reference counterpart: an extension for callers
 * whose KV_OFFSETS pools differ in size (an offload pool beside the
 * primary one). */
KVX_API kvx_status_t kvx_launch_gather_kv_pools(
    const kvx_cache_desc_t *cache, const kvx_gather_desc_t *gather,
    const kvx_pool_blocks_t *pool_blocks, const kvx_scale_desc_t *k_scale,
    const kvx_scale_desc_t *v_scale, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KVX_EXT_H */
