/*
 * Extensions to the KVX v1 ABI that kvx_abi.h cannot carry unchanged.
 *
 * FP8 (OCP E4M3, "e4m3fn") KV cache with per-tensor F32 scales:
 *
 *   write:  kvx_launch_write_kv / kvx_launch_write_kv_prefill with a cache of
 *           dtype KVX_DTYPE_F8_E4M3 and io of dtype F16, BF16 or F32.  The
 *           scale is read from write->k_scale_desc / v_scale_desc when their
 *           `data` is non-NULL (dtype F32, granularity PER_TENSOR), otherwise
 *           from write->k_scale / v_scale as one F32 each (KVX_SPEC.md:258-259).
 *           Scale pointers are device pointers, read by the kernel.
 *             q = e4m3_rne(saturate_448(f32(x) / scale)),  NaN -> 0x7F | sign
 *           With io of dtype F8_E4M3 the bytes are copied unscaled.
 *
 *   gather: kvx_launch_gather_kv_dequant below, because kvx_gather_desc_t
 *           (reference kvx_abi.h:182-188) has no scale fields.
 *             y = round_to_io_dtype(f32(q) * scale)   (RNE; NaN -> quiet NaN)
 *           kvx_launch_gather_kv with F8_E4M3 cache and io copies bytes.
 *
 * The reference has no FP8 kernels (KVX_CONFORMANCE.md:24, :35); this is new
 * functionality.  E5M2 and non-per-tensor scales return
 * KVX_STATUS_UNSUPPORTED.
 */
#ifndef KVX_EXT_H
#define KVX_EXT_H

#include "kvx_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Dequantizing gather from an F8_E4M3 paged cache into an F16/BF16/F32
 * [seq_count, max_seq_len, H, D] buffer.  Same validation order, codes and
 * untouched-row semantics as kvx_launch_gather_kv; k_scale / v_scale must be
 * non-NULL PER_TENSOR F32 descriptors whose data is a device pointer.
 * No reference counterpart (the reference gather returns UNSUPPORTED for FP8,
 * kernels/kvx_paged_kv.cu:900-909). */
KVX_API kvx_status_t kvx_launch_gather_kv_dequant(
    const kvx_cache_desc_t *cache, const kvx_gather_desc_t *gather,
    const kvx_scale_desc_t *k_scale, const kvx_scale_desc_t *v_scale,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KVX_EXT_H */
