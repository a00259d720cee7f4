// Internal interface between the C-ABI host layer (abi.cpp, launch.cpp) and
// the HIP kernels (kernels.hip).  Nothing here is exported.
#pragma once

#include <stdint.h>

#include "kvx_abi.h"
#include "kvx_ext.h"

namespace kvx {

// Address map of one paged cache tensor, in elements.  Every supported
// layout is the same affine form
//   off(b, o, h, d) = b*s_block + o*s_off + h*s_head
//                     + (d / pack)*s_piece + (d % pack)*s_inner
// NHD:        s_off=stride[1], s_head=stride[2], pack=D, s_inner=stride[3]
// HND:        s_off=stride[2], s_head=stride[1], pack=D, s_inner=stride[3]
// HND_PACKED: s_off=stride[3], s_head=stride[1], s_piece=stride[2],
//             s_inner=stride[4], pack=shape[4]
// which reproduces reference kvx_cache_offset (kernels/kvx_paged_kv.cu:54-75)
// for every in-range (b, o, h, d).
struct Geom {
  int64_t s_block;
  int64_t s_off;
  int64_t s_head;
  int64_t s_piece;
  int64_t s_inner;
  int32_t pack;
  int32_t pad_;
};

// Element conversion applied while moving one element.
enum ConvKind : int32_t {
  kConvCopy = 0,     // bit copy, any element size
  kConvQuant = 1,    // F16/BF16/F32 io -> E4M3/E5M2 cache, divide by scale
  kConvDequant = 2,  // E4M3/E5M2 cache -> F16/BF16/F32 io, multiply by scale
};

// FP8 scales of one tensor (device memory, F32): element (block b, head h)
// uses p[b * s_block + h * s_head].  indexed == 0 is the per-tensor case,
// p[0] for every element.
struct ScaleRef {
  const float *p;
  int64_t s_block;  // elements
  int64_t s_head;   // elements
  int32_t indexed;
  int32_t pad_;
};

// Everything the write kernels need, already validated on the host.
struct WritePlan {
  const void *src_k;
  const void *src_v;
  void *dst_k;
  void *dst_v;
  const void *slots;
  ScaleRef k_scale;  // only for kConvQuant
  ScaleRef v_scale;
  Geom gk;
  Geom gv;
  int64_t num_tokens;
  int32_t slot_is64;
  int32_t heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t num_blocks;
  int32_t conv;       // ConvKind
  int32_t io_dtype;   // kvx_dtype_t of the token rows
  int32_t cache_dtype;
};

// Everything the gather kernels need, already validated on the host.
struct GatherPlan {
  const void *src_k;
  const void *src_v;
  void *dst_k;
  void *dst_v;
  const void *block_table;
  const void *seq_lens;
  ScaleRef k_scale;  // only for kConvDequant
  ScaleRef v_scale;
  const void *indptr;       // RAGGED: [seq_count + 1] token prefix sums
  int64_t table_count;      // entries of block_table
  const char *pool[2];      // KV_OFFSETS: primary / secondary pool bases
  int64_t bytes_per_block;  // KV_OFFSETS
  int32_t pool_blocks[2];   // KV_OFFSETS: blocks of each pool (<= num_blocks); entries
                            // at or past their pool's count are skipped
  Geom gk;
  Geom gv;
  int32_t format;      // kvx_block_table_format_t
  int32_t indptr_is64;
  int32_t index_is64;  // block table (PACKED, RAGGED) / seq_lens dtype
  int32_t lens_is64;
  int32_t seq_count;
  int32_t max_blocks_per_seq;
  int32_t max_seq_len;
  int32_t heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t num_blocks;
  int32_t conv;
  int32_t io_dtype;
  int32_t cache_dtype;
};

// Element size in bytes of a payload dtype, 0 for non-payload dtypes.
int dtype_size(kvx_dtype_t dt);

// Enqueue the kernels on `stream`.  Return KVX_STATUS_OK, or
// KVX_STATUS_INTERNAL_ERROR when the launch itself fails.
kvx_status_t enqueue_write(const WritePlan &plan, void *stream);
kvx_status_t enqueue_gather(const GatherPlan &plan, void *stream);

// Shared launch-path implementations behind the exported entry points.
// `expected` is the dtype the per-dtype helper requires of cache and io
// (KVX_DTYPE_INVALID = any dtype the dispatcher accepts).  `pools`
// (kvx_launch_gather_kv_pools only, else NULL): block counts that narrow a
// KV_OFFSETS table's pools below num_blocks, already checked by the caller.
kvx_status_t launch_write(const kvx_cache_desc_t *cache,
                          const kvx_write_desc_t *write, int32_t tokens_per_seq,
                          bool prefill, kvx_dtype_t expected, void *stream);
kvx_status_t launch_gather(const kvx_cache_desc_t *cache,
                           const kvx_gather_desc_t *gather,
                           const kvx_scale_desc_t *k_scale,
                           const kvx_scale_desc_t *v_scale, bool dequant,
                           kvx_dtype_t expected, void *stream,
                           const kvx_pool_blocks_t *pools = nullptr);

}  // namespace kvx
