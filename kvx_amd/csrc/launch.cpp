// Launch-path entry points of kvx_paged_kv.h and kvx_ext.h.
//
// Host validation reproduces the check order and status codes of the
// reference launchers (kernels/kvx_paged_kv.cu:315-451 write, :493-716
// prefill, :763-870 gather, :472-491 / :739-761 / :891-910 dispatch), so a
// malformed call returns the same kvx_status_t as the reference before any
// HIP call is made.  Checks this build adds come after every reference check
// and only reject inputs on which the reference kernels would divide by zero
// or dereference NULL:
//   - block_size == 0 with a non-empty batch   -> INVALID_ARGUMENT
//   - NULL io / cache / index data pointers     -> INVALID_ARGUMENT
// F8_E4M3 / F8_E5M2 caches (quantizing write, byte-copy gather, dequantizing
// gather; per-tensor, per-head, per-block and per-block-head F32 scales)
// and the RAGGED / KV_OFFSETS gather formats are extensions; the reference
// returns UNSUPPORTED for them (kernels/kvx_paged_kv.cu:481-490, :788-790).
#include <hip/hip_runtime.h>

#include "kvx_ext.h"
#include "kvx_internal.h"
#include "kvx_paged_kv.h"

namespace kvx {
namespace {

bool is_io_float(kvx_dtype_t dt) {
  return dt == KVX_DTYPE_F16 || dt == KVX_DTYPE_BF16 || dt == KVX_DTYPE_F32;
}

bool is_fp8(kvx_dtype_t dt) { return dt == KVX_DTYPE_F8_E4M3 || dt == KVX_DTYPE_F8_E5M2; }

// reference kvx_paged_kv.cu:269-289 (no size/dtype/data checks on this path)
kvx_status_t check_io_3d(const kvx_tensor_desc_t *t, int32_t num_tokens,
                         int32_t heads, int32_t head_dim) {
  if (t->ndim != 3) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->shape[0] != num_tokens || t->shape[1] != heads ||
      t->shape[2] != head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (t->stride[2] != 1 || t->stride[1] != (int64_t)head_dim ||
      t->stride[0] != (int64_t)heads * head_dim)
    return KVX_STATUS_UNSUPPORTED;
  return KVX_STATUS_OK;
}

// reference kvx_paged_kv.cu:291-313
kvx_status_t check_io_4d(const kvx_tensor_desc_t *t, int32_t seq_count,
                         int32_t max_seq_len, int32_t heads,
                         int32_t head_dim) {
  if (t->ndim != 4) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->shape[0] != seq_count || t->shape[1] != max_seq_len ||
      t->shape[2] != heads || t->shape[3] != head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (t->stride[3] != 1 || t->stride[2] != (int64_t)head_dim ||
      t->stride[1] != (int64_t)heads * head_dim ||
      t->stride[0] != (int64_t)max_seq_len * heads * head_dim)
    return KVX_STATUS_UNSUPPORTED;
  return KVX_STATUS_OK;
}

// Descriptor -> Geom.  Status codes as reference kvx_fill_cache_params
// (kernels/kvx_paged_kv.cu:18-52): PACKED needs pack > 0 dividing head_dim;
// layouts other than NHD/HND/HND_PACKED/CUSTOM are UNSUPPORTED (the
// reference also rejects CUSTOM).  Any strides are honoured.
kvx_status_t fill_geom(const kvx_cache_desc_t *cache,
                       const kvx_tensor_desc_t *t, Geom *g) {
  const int64_t *s = t->stride;
  g->s_piece = 0;
  g->pad_ = 0;
  switch (t->layout) {
    case KVX_LAYOUT_BLOCK_NHD:
      g->s_block = s[0];
      g->s_off = s[1];
      g->s_head = s[2];
      g->s_inner = s[3];
      g->pack = (int32_t)cache->head_dim;
      return KVX_STATUS_OK;
    case KVX_LAYOUT_BLOCK_HND:
      g->s_block = s[0];
      g->s_head = s[1];
      g->s_off = s[2];
      g->s_inner = s[3];
      g->pack = (int32_t)cache->head_dim;
      return KVX_STATUS_OK;
    case KVX_LAYOUT_BLOCK_HND_PACKED: {
      const int64_t pack = t->shape[4];
      if (pack <= 0) return KVX_STATUS_INVALID_ARGUMENT;
      if ((int64_t)cache->head_dim % pack != 0)
        return KVX_STATUS_INVALID_ARGUMENT;
      g->s_block = s[0];
      g->s_head = s[1];
      g->s_piece = s[2];
      g->s_off = s[3];
      g->s_inner = s[4];
      g->pack = (int32_t)pack;
      return KVX_STATUS_OK;
    }
    case KVX_LAYOUT_BLOCK_CUSTOM: {
      // Axes (block, offset, head, dim) or (block, offset, head, dim / x, x)
      // with any strides; the shape names the split (KVX_SPEC.md:57 leaves
      // the axis meaning open; this is this build's reading).
      const int64_t *sh = t->shape;
      if (sh[0] != cache->num_blocks || sh[1] != cache->block_size ||
          sh[2] != cache->num_kv_heads)
        return KVX_STATUS_INVALID_ARGUMENT;
      g->s_block = s[0];
      g->s_off = s[1];
      g->s_head = s[2];
      if (t->ndim == 4) {
        if (sh[3] != cache->head_dim) return KVX_STATUS_INVALID_ARGUMENT;
        g->s_inner = s[3];
        g->pack = (int32_t)cache->head_dim;
        return KVX_STATUS_OK;
      }
      if (t->ndim != 5 || sh[4] <= 0 || (int64_t)cache->head_dim % sh[4] != 0 ||
          sh[3] != (int64_t)cache->head_dim / sh[4])
        return KVX_STATUS_INVALID_ARGUMENT;
      g->s_piece = s[3];
      g->s_inner = s[4];
      g->pack = (int32_t)sh[4];
      return KVX_STATUS_OK;
    }
    default:
      return KVX_STATUS_UNSUPPORTED;
  }
}

// True when all in-block offsets of `g` (block index 0) are non-negative and
// the last element ends within `pitch` bytes.
bool block_fits(const Geom &g, int64_t bs, int64_t heads, int64_t head_dim, int esize,
                int64_t pitch) {
  if (g.s_off < 0 || g.s_head < 0 || g.s_piece < 0 || g.s_inner < 0) return false;
  const int64_t pieces = head_dim / g.pack;
  const int64_t last = (bs - 1) * g.s_off + (heads - 1) * g.s_head +
                       (pieces - 1) * g.s_piece + (int64_t)(g.pack - 1) * g.s_inner;
  return (last + 1) * esize <= pitch;
}

// A scale descriptor -> ScaleRef.  F32 scales only.  Granularities
// (KVX_SPEC.md:190-197 names the fields; the shapes are this build's):
//   PER_TENSOR      one value, data[0]
//   PER_HEAD        ndim 1, shape [num_kv_heads], stride[0] in elements
//   PER_BLOCK       ndim 1, shape [num_blocks], indexed by physical block id
//   PER_BLOCK_HEAD  ndim 2, shape [num_blocks, num_kv_heads]
// Block-indexed scales need physical block ids: KV_OFFSETS gathers
// (block_ok = false) return UNSUPPORTED for them.
kvx_status_t resolve_scale_desc(const kvx_scale_desc_t *d, const kvx_cache_desc_t *cache,
                                bool block_ok, ScaleRef *out) {
  if (d->size < sizeof(kvx_scale_desc_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (d->dtype != KVX_DTYPE_F32) return KVX_STATUS_UNSUPPORTED;
  const kvx_scale_granularity_t g = d->granularity;
  if (g != KVX_SCALE_PER_TENSOR && g != KVX_SCALE_PER_HEAD && g != KVX_SCALE_PER_BLOCK &&
      g != KVX_SCALE_PER_BLOCK_HEAD)
    return KVX_STATUS_UNSUPPORTED;
  if (!block_ok && (g == KVX_SCALE_PER_BLOCK || g == KVX_SCALE_PER_BLOCK_HEAD))
    return KVX_STATUS_UNSUPPORTED;
  if (d->data == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  const int64_t nb = cache->num_blocks;
  const int64_t H = cache->num_kv_heads;
  *out = ScaleRef{static_cast<const float *>(d->data), 0, 0, 0, 0};
  switch (g) {
    case KVX_SCALE_PER_HEAD:
      if (d->ndim != 1 || d->shape[0] != H) return KVX_STATUS_INVALID_ARGUMENT;
      out->s_head = d->stride[0];
      break;
    case KVX_SCALE_PER_BLOCK:
      if (d->ndim != 1 || d->shape[0] != nb) return KVX_STATUS_INVALID_ARGUMENT;
      out->s_block = d->stride[0];
      break;
    case KVX_SCALE_PER_BLOCK_HEAD:
      if (d->ndim != 2 || d->shape[0] != nb || d->shape[1] != H)
        return KVX_STATUS_INVALID_ARGUMENT;
      out->s_block = d->stride[0];
      out->s_head = d->stride[1];
      break;
    default:
      return KVX_STATUS_OK;  // PER_TENSOR
  }
  out->indexed = 1;
  return KVX_STATUS_OK;
}

// The quantizing write's scale (KVX_SPEC.md:258-259): the descriptor when
// its data is set, else the raw pointer as a per-tensor F32 scale.
kvx_status_t resolve_write_scale(const kvx_scale_desc_t *desc, const void *raw,
                                 const kvx_cache_desc_t *cache, ScaleRef *out) {
  if (desc->data != nullptr) return resolve_scale_desc(desc, cache, true, out);
  if (raw == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  *out = ScaleRef{static_cast<const float *>(raw), 0, 0, 0, 0};
  return KVX_STATUS_OK;
}

}  // namespace

// `expected` is the payload dtype of the per-dtype helper; KVX_DTYPE_F8_E4M3
// and KVX_DTYPE_F8_E5M2 are this build's FP8 paths, where io may be
// F16/BF16/F32 (quantize) or the cache's own FP8 dtype (byte copy).
kvx_status_t launch_write(const kvx_cache_desc_t *cache,
                          const kvx_write_desc_t *write, int32_t tokens_per_seq,
                          bool prefill, kvx_dtype_t expected, void *stream) {
  if (cache == nullptr || write == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (prefill && tokens_per_seq <= 0) return KVX_STATUS_INVALID_ARGUMENT;
  if (write->size < sizeof(kvx_write_desc_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (write->io.size < sizeof(kvx_kv_io_desc_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  if (write->slots.size < sizeof(kvx_slot_mapping_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  if (prefill && (write->io.num_tokens % (uint32_t)tokens_per_seq) != 0)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != expected || cache->v.dtype != expected)
    return KVX_STATUS_UNSUPPORTED;
  const kvx_dtype_t io_dt = write->io.key.dtype;
  if (is_fp8(expected)) {
    if (write->io.value.dtype != io_dt || !(is_io_float(io_dt) || io_dt == expected))
      return KVX_STATUS_UNSUPPORTED;
  } else if (io_dt != expected || write->io.value.dtype != expected) {
    return KVX_STATUS_UNSUPPORTED;
  }
  const int32_t heads = (int32_t)write->io.num_kv_heads;
  const int32_t head_dim = (int32_t)write->io.head_dim;
  if (heads != (int32_t)cache->num_kv_heads ||
      head_dim != (int32_t)cache->head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  const int32_t num_tokens = (int32_t)write->io.num_tokens;
  kvx_status_t st = check_io_3d(&write->io.key, num_tokens, heads, head_dim);
  if (st != KVX_STATUS_OK) return st;
  st = check_io_3d(&write->io.value, num_tokens, heads, head_dim);
  if (st != KVX_STATUS_OK) return st;
  if (write->slots.token_count != write->io.num_tokens)
    return KVX_STATUS_INVALID_ARGUMENT;

  WritePlan p;
  st = fill_geom(cache, &cache->k, &p.gk);
  if (st != KVX_STATUS_OK) return st;
  st = fill_geom(cache, &cache->v, &p.gv);
  if (st != KVX_STATUS_OK) return st;

  const bool quant = is_fp8(expected) && io_dt != expected;
  p.k_scale = ScaleRef{};
  p.v_scale = ScaleRef{};
  if (quant) {
    st = resolve_write_scale(&write->k_scale_desc, write->k_scale, cache, &p.k_scale);
    if (st != KVX_STATUS_OK) return st;
    st = resolve_write_scale(&write->v_scale_desc, write->v_scale, cache, &p.v_scale);
    if (st != KVX_STATUS_OK) return st;
  }

  const int64_t total = (int64_t)num_tokens * heads * head_dim;
  if (total == 0) return KVX_STATUS_OK;
  if (write->slots.dtype != KVX_DTYPE_S32 && write->slots.dtype != KVX_DTYPE_S64)
    return KVX_STATUS_INVALID_ARGUMENT;

  // Checks added by this build (see file comment).
  if (cache->block_size == 0) return KVX_STATUS_INVALID_ARGUMENT;
  if (write->io.key.data == nullptr || write->io.value.data == nullptr ||
      cache->k.data == nullptr || cache->v.data == nullptr ||
      write->slots.slots == nullptr)
    return KVX_STATUS_INVALID_ARGUMENT;

  p.src_k = write->io.key.data;
  p.src_v = write->io.value.data;
  p.dst_k = cache->k.data;
  p.dst_v = cache->v.data;
  p.slots = write->slots.slots;
  p.num_tokens = num_tokens;
  p.slot_is64 = write->slots.dtype == KVX_DTYPE_S64;
  p.heads = heads;
  p.head_dim = head_dim;
  p.block_size = (int32_t)cache->block_size;
  p.num_blocks = (int32_t)cache->num_blocks;
  p.conv = quant ? kConvQuant : kConvCopy;
  p.io_dtype = io_dt;
  p.cache_dtype = cache->k.dtype;
  return enqueue_write(p, stream);
}

kvx_status_t launch_gather(const kvx_cache_desc_t *cache,
                           const kvx_gather_desc_t *gather,
                           const kvx_scale_desc_t *k_scale,
                           const kvx_scale_desc_t *v_scale, bool dequant,
                           kvx_dtype_t expected, void *stream,
                           const kvx_pool_blocks_t *pools) {
  if (cache == nullptr || gather == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (dequant && (k_scale == nullptr || v_scale == nullptr))
    return KVX_STATUS_INVALID_ARGUMENT;
  if (gather->size < sizeof(kvx_gather_desc_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  if (gather->io.size < sizeof(kvx_kv_io_desc_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  if (gather->block_table.size < sizeof(kvx_block_table_t) ||
      gather->seq_lens.size < sizeof(kvx_seq_lens_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != expected || cache->v.dtype != expected)
    return KVX_STATUS_UNSUPPORTED;
  const kvx_dtype_t io_dt = gather->io.key.dtype;
  if (dequant) {
    if (gather->io.value.dtype != io_dt || !is_io_float(io_dt))
      return KVX_STATUS_UNSUPPORTED;
  } else if (io_dt != expected || gather->io.value.dtype != expected) {
    return KVX_STATUS_UNSUPPORTED;
  }
  const kvx_block_table_format_t fmt = gather->block_table.format;
  if (fmt != KVX_BLOCK_TABLE_PACKED && fmt != KVX_BLOCK_TABLE_RAGGED &&
      fmt != KVX_BLOCK_TABLE_KV_OFFSETS)
    return KVX_STATUS_UNSUPPORTED;
  const int32_t heads = (int32_t)gather->io.num_kv_heads;
  const int32_t head_dim = (int32_t)gather->io.head_dim;
  if (heads != (int32_t)cache->num_kv_heads ||
      head_dim != (int32_t)cache->head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (gather->seq_lens.seq_count != gather->block_table.seq_count)
    return KVX_STATUS_INVALID_ARGUMENT;
  const int32_t seq_count = (int32_t)gather->block_table.seq_count;
  const int32_t max_seq_len = (int32_t)gather->max_seq_len;
  kvx_status_t st =
      check_io_4d(&gather->io.key, seq_count, max_seq_len, heads, head_dim);
  if (st != KVX_STATUS_OK) return st;
  st = check_io_4d(&gather->io.value, seq_count, max_seq_len, heads, head_dim);
  if (st != KVX_STATUS_OK) return st;

  GatherPlan p;
  st = fill_geom(cache, &cache->k, &p.gk);
  if (st != KVX_STATUS_OK) return st;
  st = fill_geom(cache, &cache->v, &p.gv);
  if (st != KVX_STATUS_OK) return st;

  p.k_scale = ScaleRef{};
  p.v_scale = ScaleRef{};
  if (dequant) {
    const bool block_ok = fmt != KVX_BLOCK_TABLE_KV_OFFSETS;
    st = resolve_scale_desc(k_scale, cache, block_ok, &p.k_scale);
    if (st != KVX_STATUS_OK) return st;
    st = resolve_scale_desc(v_scale, cache, block_ok, &p.v_scale);
    if (st != KVX_STATUS_OK) return st;
  }

  const int64_t total = (int64_t)seq_count * max_seq_len * heads * head_dim;
  if (total == 0) return KVX_STATUS_OK;
  const kvx_block_table_t &tb = gather->block_table;
  const kvx_dtype_t idx_dt = tb.index_dtype;
  const kvx_dtype_t len_dt = gather->seq_lens.dtype;
  const bool s32 = idx_dt == KVX_DTYPE_S32 && len_dt == KVX_DTYPE_S32;
  const bool s64 = idx_dt == KVX_DTYPE_S64 && len_dt == KVX_DTYPE_S64;
  if (fmt == KVX_BLOCK_TABLE_KV_OFFSETS) {
    // KVX_SPEC.md:116-122: S32 KVCacheIndex values, flag set, power-of-two
    // block size, a primary pool; beam_width > 1 has no output layout here.
    if (idx_dt != KVX_DTYPE_S32) return KVX_STATUS_INVALID_ARGUMENT;
    if (len_dt != KVX_DTYPE_S32 && len_dt != KVX_DTYPE_S64) return KVX_STATUS_INVALID_ARGUMENT;
    if ((tb.flags & KVX_BLOCK_TABLE_FLAG_KVCACHEINDEX) == 0) return KVX_STATUS_INVALID_ARGUMENT;
    if (tb.beam_width == 0) return KVX_STATUS_INVALID_ARGUMENT;
    if (tb.beam_width != 1) return KVX_STATUS_UNSUPPORTED;
    if (cache->block_size == 0 || (cache->block_size & (cache->block_size - 1)) != 0)
      return KVX_STATUS_INVALID_ARGUMENT;
    if (cache->pool.bytes_per_block == 0 || cache->pool.primary == nullptr)
      return KVX_STATUS_INVALID_ARGUMENT;
    if ((uint64_t)tb.indices_count != (uint64_t)tb.seq_count * 2u * tb.max_blocks_per_seq)
      return KVX_STATUS_INVALID_ARGUMENT;
    // Every element of a block must lie inside its bytes_per_block pitch.
    const int esize = dtype_size(cache->k.dtype);
    if (!block_fits(p.gk, cache->block_size, heads, head_dim, esize,
                    cache->pool.bytes_per_block) ||
        !block_fits(p.gv, cache->block_size, heads, head_dim, esize,
                    cache->pool.bytes_per_block))
      return KVX_STATUS_INVALID_ARGUMENT;
  } else if (!s32 && !s64) {
    return KVX_STATUS_INVALID_ARGUMENT;
  }
  if (fmt == KVX_BLOCK_TABLE_RAGGED) {
    // KVX_SPEC.md:107-114: indptr holds seq_count + 1 prefix sums.
    if (tb.indptr_dtype != KVX_DTYPE_S32 && tb.indptr_dtype != KVX_DTYPE_S64)
      return KVX_STATUS_INVALID_ARGUMENT;
    if (tb.indptr == nullptr || tb.indptr_count != tb.seq_count + 1)
      return KVX_STATUS_INVALID_ARGUMENT;
  }

  // Checks added by this build (see file comment).
  if (cache->block_size == 0) return KVX_STATUS_INVALID_ARGUMENT;
  if (gather->io.key.data == nullptr || gather->io.value.data == nullptr ||
      gather->seq_lens.lengths == nullptr ||
      (fmt != KVX_BLOCK_TABLE_KV_OFFSETS &&
       (cache->k.data == nullptr || cache->v.data == nullptr)) ||
      (fmt == KVX_BLOCK_TABLE_PACKED && tb.max_blocks_per_seq > 0 && tb.indices == nullptr) ||
      (fmt != KVX_BLOCK_TABLE_PACKED && tb.indices_count > 0 && tb.indices == nullptr))
    return KVX_STATUS_INVALID_ARGUMENT;

  p.src_k = cache->k.data;
  p.src_v = cache->v.data;
  p.dst_k = gather->io.key.data;
  p.dst_v = gather->io.value.data;
  p.block_table = gather->block_table.indices;
  p.seq_lens = gather->seq_lens.lengths;
  p.format = fmt;
  p.index_is64 = idx_dt == KVX_DTYPE_S64;
  p.lens_is64 = len_dt == KVX_DTYPE_S64;
  p.indptr = tb.indptr;
  p.table_count = tb.indices_count;
  p.indptr_is64 = tb.indptr_dtype == KVX_DTYPE_S64;
  p.pool[0] = static_cast<const char *>(cache->pool.primary);
  p.pool[1] = static_cast<const char *>(cache->pool.secondary);
  p.bytes_per_block = cache->pool.bytes_per_block;
  const int64_t nb = cache->num_blocks;
  const int64_t counts[2] = {pools ? pools->primary : 0, pools ? pools->secondary : 0};
  for (int i = 0; i < 2; ++i)
    p.pool_blocks[i] = (int32_t)(counts[i] > 0 && counts[i] < nb ? counts[i] : nb);
  p.seq_count = seq_count;
  p.max_blocks_per_seq = (int32_t)gather->block_table.max_blocks_per_seq;
  p.max_seq_len = max_seq_len;
  p.heads = heads;
  p.head_dim = head_dim;
  p.block_size = (int32_t)cache->block_size;
  p.num_blocks = (int32_t)cache->num_blocks;
  p.conv = dequant ? kConvDequant : kConvCopy;
  p.io_dtype = io_dt;
  p.cache_dtype = cache->k.dtype;
  return enqueue_gather(p, stream);
}

}  // namespace kvx

using kvx::launch_gather;
using kvx::launch_write;

// ---------------------------------------------------------------------------
// Exported C ABI.

extern "C" {

KVX_API kvx_status_t kvx_launch_write_kv_f32(const kvx_cache_desc_t *cache,
                                             const kvx_write_desc_t *write,
                                             void *stream) {
  return launch_write(cache, write, 0, false, KVX_DTYPE_F32, stream);
}

KVX_API kvx_status_t kvx_launch_write_kv_f16(const kvx_cache_desc_t *cache,
                                             const kvx_write_desc_t *write,
                                             void *stream) {
  return launch_write(cache, write, 0, false, KVX_DTYPE_F16, stream);
}

KVX_API kvx_status_t kvx_launch_write_kv_bf16(const kvx_cache_desc_t *cache,
                                              const kvx_write_desc_t *write,
                                              void *stream) {
  return launch_write(cache, write, 0, false, KVX_DTYPE_BF16, stream);
}

KVX_API kvx_status_t kvx_launch_write_kv(const kvx_cache_desc_t *cache,
                                         const kvx_write_desc_t *write,
                                         void *stream) {
  if (cache == nullptr || write == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != cache->v.dtype) return KVX_STATUS_INVALID_ARGUMENT;
  switch (cache->k.dtype) {
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16:
    case KVX_DTYPE_F32:
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2:
      return launch_write(cache, write, 0, false, cache->k.dtype, stream);
    default:
      return KVX_STATUS_UNSUPPORTED;
  }
}

KVX_API kvx_status_t kvx_launch_write_kv_prefill_f32(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream) {
  return launch_write(cache, write, tokens_per_seq, true, KVX_DTYPE_F32,
                      stream);
}

KVX_API kvx_status_t kvx_launch_write_kv_prefill_f16(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream) {
  return launch_write(cache, write, tokens_per_seq, true, KVX_DTYPE_F16,
                      stream);
}

KVX_API kvx_status_t kvx_launch_write_kv_prefill_bf16(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream) {
  return launch_write(cache, write, tokens_per_seq, true, KVX_DTYPE_BF16,
                      stream);
}

KVX_API kvx_status_t kvx_launch_write_kv_prefill(
    const kvx_cache_desc_t *cache, const kvx_write_desc_t *write,
    int32_t tokens_per_seq, void *stream) {
  if (cache == nullptr || write == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != cache->v.dtype) return KVX_STATUS_INVALID_ARGUMENT;
  switch (cache->k.dtype) {
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16:
    case KVX_DTYPE_F32:
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2:
      return launch_write(cache, write, tokens_per_seq, true, cache->k.dtype,
                          stream);
    default:
      return KVX_STATUS_UNSUPPORTED;
  }
}

KVX_API kvx_status_t kvx_launch_gather_kv_f32(const kvx_cache_desc_t *cache,
                                              const kvx_gather_desc_t *gather,
                                              void *stream) {
  return launch_gather(cache, gather, nullptr, nullptr, false, KVX_DTYPE_F32,
                       stream);
}

KVX_API kvx_status_t kvx_launch_gather_kv_f16(const kvx_cache_desc_t *cache,
                                              const kvx_gather_desc_t *gather,
                                              void *stream) {
  return launch_gather(cache, gather, nullptr, nullptr, false, KVX_DTYPE_F16,
                       stream);
}

KVX_API kvx_status_t kvx_launch_gather_kv_bf16(const kvx_cache_desc_t *cache,
                                               const kvx_gather_desc_t *gather,
                                               void *stream) {
  return launch_gather(cache, gather, nullptr, nullptr, false, KVX_DTYPE_BF16,
                       stream);
}

KVX_API kvx_status_t kvx_launch_gather_kv(const kvx_cache_desc_t *cache,
                                          const kvx_gather_desc_t *gather,
                                          void *stream) {
  if (cache == nullptr || gather == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != cache->v.dtype) return KVX_STATUS_INVALID_ARGUMENT;
  switch (cache->k.dtype) {
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16:
    case KVX_DTYPE_F32:
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2:
      return launch_gather(cache, gather, nullptr, nullptr, false,
                           cache->k.dtype, stream);
    default:
      return KVX_STATUS_UNSUPPORTED;
  }
}

KVX_API kvx_status_t kvx_launch_gather_kv_dequant(
    const kvx_cache_desc_t *cache, const kvx_gather_desc_t *gather,
    const kvx_scale_desc_t *k_scale, const kvx_scale_desc_t *v_scale,
    void *stream) {
  if (cache == nullptr || gather == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != cache->v.dtype) return KVX_STATUS_INVALID_ARGUMENT;
  if (!kvx::is_fp8(cache->k.dtype)) return KVX_STATUS_UNSUPPORTED;
  return launch_gather(cache, gather, k_scale, v_scale, true, cache->k.dtype, stream);
}

// kvx_ext.h's own struct (no reference counterpart), LP64.
static_assert(sizeof(kvx_pool_blocks_t) == 24, "abi");
static_assert(offsetof(kvx_pool_blocks_t, primary) == 8, "abi");
static_assert(offsetof(kvx_pool_blocks_t, secondary) == 16, "abi");

KVX_API kvx_status_t kvx_launch_gather_kv_pools(const kvx_cache_desc_t *cache,
                                                const kvx_gather_desc_t *gather,
                                                const kvx_pool_blocks_t *pool_blocks,
                                                const kvx_scale_desc_t *k_scale,
                                                const kvx_scale_desc_t *v_scale,
                                                void *stream) {
  if (cache == nullptr || gather == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (pool_blocks != nullptr &&
      (pool_blocks->size < sizeof(kvx_pool_blocks_t) || pool_blocks->primary < 0 ||
       pool_blocks->secondary < 0))
    return KVX_STATUS_INVALID_ARGUMENT;
  if ((k_scale == nullptr) != (v_scale == nullptr)) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != cache->v.dtype) return KVX_STATUS_INVALID_ARGUMENT;
  if (k_scale != nullptr) {
    if (!kvx::is_fp8(cache->k.dtype)) return KVX_STATUS_UNSUPPORTED;
    return launch_gather(cache, gather, k_scale, v_scale, true, cache->k.dtype, stream,
                         pool_blocks);
  }
  switch (cache->k.dtype) {
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16:
    case KVX_DTYPE_F32:
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2:
      return launch_gather(cache, gather, nullptr, nullptr, false, cache->k.dtype, stream,
                           pool_blocks);
    default:
      return KVX_STATUS_UNSUPPORTED;
  }
}

}  // extern "C"
