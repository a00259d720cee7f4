// kvx_abi.h entry points.
//
// Validation restates reference kvx_abi.c:5-466 check for check: the same
// status codes in the same order (strict canonical strides, equal K/V layout
// and dtype, non-NULL data, table counts per format).  The one difference is
// the reference's last gather check, PACKED-only (kvx_abi.c:462-464): RAGGED
// and KV_OFFSETS tables are executed here.  After validation succeeds the
// call executes:
//   - every payload buffer KVX_MEMORY_HOST  -> validation only, OK (this is
//     all the reference does for any memory type, kvx_abi.c:354-466);
//   - DEVICE / UNIFIED                       -> HIP kernels on `stream`;
//   - UNKNOWN                                -> hipPointerGetAttributes must
//     report device-accessible memory, else UNSUPPORTED;
//   - HOST mixed with device buffers         -> UNSUPPORTED.
#include <hip/hip_runtime.h>
#include <stddef.h>

#include "kvx_internal.h"
#include "kvx_paged_kv.h"

namespace {

bool is_float_dtype(kvx_dtype_t dt) {  // kvx_abi.c:5-16
  switch (dt) {
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16:
    case KVX_DTYPE_F32:
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2:
      return true;
    default:
      return false;
  }
}

bool is_index_dtype(kvx_dtype_t dt) {  // kvx_abi.c:18-20
  return dt == KVX_DTYPE_S32 || dt == KVX_DTYPE_S64;
}

bool is_pow2(uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }

// kvx_abi.c:26-55
kvx_status_t check_io_3d(const kvx_tensor_desc_t *t, uint32_t num_tokens,
                         uint32_t heads, uint32_t head_dim) {
  if (t->size < sizeof(kvx_tensor_desc_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (!is_float_dtype(t->dtype)) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->ndim != 3) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->shape[0] != num_tokens || t->shape[1] != heads ||
      t->shape[2] != head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (t->stride[2] != 1 || t->stride[1] != (int64_t)head_dim ||
      t->stride[0] != (int64_t)heads * head_dim)
    return KVX_STATUS_UNSUPPORTED;
  if (num_tokens > 0 && t->data == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  return KVX_STATUS_OK;
}

// kvx_abi.c:57-88
kvx_status_t check_io_4d(const kvx_tensor_desc_t *t, uint32_t seq_count,
                         uint32_t max_seq_len, uint32_t heads,
                         uint32_t head_dim) {
  if (t->size < sizeof(kvx_tensor_desc_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (!is_float_dtype(t->dtype)) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->ndim != 4) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->shape[0] != seq_count || t->shape[1] != max_seq_len ||
      t->shape[2] != heads || t->shape[3] != head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (t->stride[3] != 1 || t->stride[2] != (int64_t)head_dim ||
      t->stride[1] != (int64_t)heads * head_dim ||
      t->stride[0] != (int64_t)max_seq_len * heads * head_dim)
    return KVX_STATUS_UNSUPPORTED;
  if (seq_count > 0 && max_seq_len > 0 && t->data == nullptr)
    return KVX_STATUS_INVALID_ARGUMENT;
  return KVX_STATUS_OK;
}

// kvx_abi.c:90-108
kvx_status_t check_slots(const kvx_slot_mapping_t *s, uint32_t num_tokens) {
  if (s->size < sizeof(kvx_slot_mapping_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (!is_index_dtype(s->dtype)) return KVX_STATUS_INVALID_ARGUMENT;
  if (s->token_count != num_tokens) return KVX_STATUS_INVALID_ARGUMENT;
  if (num_tokens > 0 && s->slots == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  return KVX_STATUS_OK;
}

// kvx_abi.c:110-194.  Counts are uint32 products, wrapping like the C source.
kvx_status_t check_table(const kvx_cache_desc_t *cache,
                         const kvx_block_table_t *t) {
  if (t->size < sizeof(kvx_block_table_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->seq_count == 0 || t->max_blocks_per_seq == 0)
    return KVX_STATUS_INVALID_ARGUMENT;
  switch (t->format) {
    case KVX_BLOCK_TABLE_PACKED: {
      const uint32_t expected = t->seq_count * t->max_blocks_per_seq;
      if (!is_index_dtype(t->index_dtype)) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->beam_width != 1) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indices_count != expected) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indptr != nullptr || t->indptr_count != 0)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indices_count > 0 && t->indices == nullptr)
        return KVX_STATUS_INVALID_ARGUMENT;
      return KVX_STATUS_OK;
    }
    case KVX_BLOCK_TABLE_RAGGED: {
      if (!is_index_dtype(t->index_dtype) || !is_index_dtype(t->indptr_dtype))
        return KVX_STATUS_INVALID_ARGUMENT;
      if (t->beam_width != 1) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indptr == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indptr_count != t->seq_count + 1)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indices_count > 0 && t->indices == nullptr)
        return KVX_STATUS_INVALID_ARGUMENT;
      return KVX_STATUS_OK;
    }
    case KVX_BLOCK_TABLE_KV_OFFSETS: {
      const uint32_t expected =
          t->seq_count * t->beam_width * 2u * t->max_blocks_per_seq;
      if (t->index_dtype != KVX_DTYPE_S32) return KVX_STATUS_INVALID_ARGUMENT;
      if ((t->flags & KVX_BLOCK_TABLE_FLAG_KVCACHEINDEX) == 0)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (t->beam_width == 0) return KVX_STATUS_INVALID_ARGUMENT;
      if (!is_pow2(cache->block_size)) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indices_count != expected) return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indptr != nullptr || t->indptr_count != 0)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (t->indices_count > 0 && t->indices == nullptr)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (cache->pool.bytes_per_block == 0 || cache->pool.primary == nullptr)
        return KVX_STATUS_INVALID_ARGUMENT;
      return KVX_STATUS_OK;
    }
    default:
      return KVX_STATUS_INVALID_ARGUMENT;
  }
}

// kvx_abi.c:196-214
kvx_status_t check_seq_lens(const kvx_seq_lens_t *s, uint32_t seq_count) {
  if (s->size < sizeof(kvx_seq_lens_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (!is_index_dtype(s->dtype)) return KVX_STATUS_INVALID_ARGUMENT;
  if (s->seq_count != seq_count) return KVX_STATUS_INVALID_ARGUMENT;
  if (seq_count > 0 && s->lengths == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  return KVX_STATUS_OK;
}

// kvx_abi.c:216-311: shape must agree with the cache, strides canonical.
// KVX_LAYOUT_BLOCK_CUSTOM ("any layout described by explicit shape and
// stride", KVX_SPEC.md:57), as this build reads it: the axes are the logical
// (block, token offset, head, dim) in that order, shape [num_blocks,
// block_size, num_kv_heads, head_dim], or with dim split as (dim / x, x),
// shape [num_blocks, block_size, num_kv_heads, head_dim / x, x]; the strides
// place them anywhere (vLLM's [nb, H, D, bs] value cache is strides
// {H*D*bs, 1, D*bs, bs}).
bool custom_shape_ok(const kvx_cache_desc_t *c, const kvx_tensor_desc_t *t) {
  const int64_t *sh = t->shape;
  if (t->ndim == 4)
    return sh[0] == c->num_blocks && sh[1] == c->block_size && sh[2] == c->num_kv_heads &&
           sh[3] == c->head_dim;
  if (t->ndim == 5)
    return sh[4] > 0 && (int64_t)c->head_dim % sh[4] == 0 && sh[0] == c->num_blocks &&
           sh[1] == c->block_size && sh[2] == c->num_kv_heads &&
           sh[3] == (int64_t)c->head_dim / sh[4];
  return false;
}

kvx_status_t check_cache_tensor(const kvx_cache_desc_t *c,
                                const kvx_tensor_desc_t *t,
                                kvx_layout_t layout) {
  if (t->size < sizeof(kvx_tensor_desc_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (!is_float_dtype(t->dtype)) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->data == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->layout != layout) return KVX_STATUS_INVALID_ARGUMENT;
  if (t->ndim == 0 || t->ndim > KVX_MAX_TENSOR_DIMS)
    return KVX_STATUS_INVALID_ARGUMENT;
  const int64_t nb = c->num_blocks, bs = c->block_size, H = c->num_kv_heads,
                D = c->head_dim;
  const int64_t *sh = t->shape, *st = t->stride;
  switch (layout) {
    case KVX_LAYOUT_BLOCK_NHD:
      if (t->ndim != 4) return KVX_STATUS_INVALID_ARGUMENT;
      if (sh[0] != nb || sh[1] != bs || sh[2] != H || sh[3] != D)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (st[3] != 1 || st[2] != D || st[1] != H * D || st[0] != bs * H * D)
        return KVX_STATUS_UNSUPPORTED;
      return KVX_STATUS_OK;
    case KVX_LAYOUT_BLOCK_HND:
      if (t->ndim != 4) return KVX_STATUS_INVALID_ARGUMENT;
      if (sh[0] != nb || sh[1] != H || sh[2] != bs || sh[3] != D)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (st[3] != 1 || st[2] != D || st[1] != bs * D || st[0] != H * bs * D)
        return KVX_STATUS_UNSUPPORTED;
      return KVX_STATUS_OK;
    case KVX_LAYOUT_BLOCK_HND_PACKED: {
      // shape[4] is read before the ndim check, as in the reference.
      const int64_t pack = sh[4];
      if (t->ndim != 5) return KVX_STATUS_INVALID_ARGUMENT;
      if (pack <= 0) return KVX_STATUS_INVALID_ARGUMENT;
      if (D % pack != 0) return KVX_STATUS_INVALID_ARGUMENT;
      if (sh[0] != nb || sh[1] != H || sh[2] != D / pack || sh[3] != bs ||
          sh[4] != pack)
        return KVX_STATUS_INVALID_ARGUMENT;
      if (st[4] != 1 || st[3] != pack || st[2] != bs * pack ||
          st[1] != (D / pack) * bs * pack || st[0] != H * (D / pack) * bs * pack)
        return KVX_STATUS_UNSUPPORTED;
      return KVX_STATUS_OK;
    }
    case KVX_LAYOUT_BLOCK_CUSTOM:
      // The reference returns UNSUPPORTED (kvx_abi.c:307-309); this build
      // accepts the shapes of custom_shape_ok with any strides.
      return custom_shape_ok(c, t) ? KVX_STATUS_OK : KVX_STATUS_INVALID_ARGUMENT;
    default:
      return KVX_STATUS_UNSUPPORTED;
  }
}

// How a validated call executes.
enum class Exec { kValidateOnly, kDevice, kUnsupported };

bool device_accessible(const void *p) {
  hipPointerAttribute_t attr;
  const hipError_t err = hipPointerGetAttributes(&attr, p);
  if (err != hipSuccess) {
    (void)hipGetLastError();  // the query's error is not the caller's
    return false;
  }
  return attr.type == hipMemoryTypeDevice ||
         attr.type == hipMemoryTypeManaged ||
         attr.type == hipMemoryTypeUnified ||
         (attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr);
}

// Buffers of one call: all HOST -> validation only; a mix of HOST and
// device memory -> UNSUPPORTED; UNKNOWN memory is asked of the runtime.
// `pool` (KV_OFFSETS gathers) adds the pool pointers to the set.
Exec classify(const kvx_tensor_desc_t *const *ts, int n,
              const kvx_pool_desc_t *pool = nullptr) {
  struct Buf {
    kvx_memory_type_t memory;
    const void *data;
  } bufs[7];
  int m = 0;
  for (int i = 0; i < n; ++i) bufs[m++] = {ts[i]->memory, ts[i]->data};
  if (pool != nullptr) {
    bufs[m++] = {pool->memory, pool->primary};
    if (pool->secondary != nullptr) bufs[m++] = {pool->memory, pool->secondary};
  }
  int host = 0;
  for (int i = 0; i < m; ++i) host += bufs[i].memory == KVX_MEMORY_HOST;
  if (host == m) return Exec::kValidateOnly;
  if (host != 0) return Exec::kUnsupported;
  for (int i = 0; i < m; ++i) {
    if (bufs[i].memory == KVX_MEMORY_UNKNOWN && bufs[i].data != nullptr &&
        !device_accessible(bufs[i].data))
      return Exec::kUnsupported;
  }
  return Exec::kDevice;
}

}  // namespace

extern "C" {

KVX_API kvx_status_t kvx_get_version(kvx_version_t *out) {
  if (out == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  out->size = sizeof(kvx_version_t);
  out->abi_major = KVX_ABI_VERSION_MAJOR;
  out->abi_minor = KVX_ABI_VERSION_MINOR;
  out->abi_patch = 0;
  return KVX_STATUS_OK;
}

KVX_API kvx_status_t kvx_validate_cache_desc(const kvx_cache_desc_t *cache) {
  if (cache == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->size < sizeof(kvx_cache_desc_t)) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->num_blocks == 0 || cache->block_size == 0 ||
      cache->num_kv_heads == 0 || cache->head_dim == 0)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.layout != cache->v.layout) return KVX_STATUS_INVALID_ARGUMENT;
  if (cache->k.dtype != cache->v.dtype) return KVX_STATUS_INVALID_ARGUMENT;
  kvx_status_t st = check_cache_tensor(cache, &cache->k, cache->k.layout);
  if (st != KVX_STATUS_OK) return st;
  return check_cache_tensor(cache, &cache->v, cache->v.layout);
}

KVX_API kvx_status_t kvx_write_kv(const kvx_cache_desc_t *cache,
                                  const kvx_write_desc_t *write, void *stream) {
  if (cache == nullptr || write == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (write->size < sizeof(kvx_write_desc_t) ||
      write->io.size < sizeof(kvx_kv_io_desc_t) ||
      write->slots.size < sizeof(kvx_slot_mapping_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  kvx_status_t st = kvx_validate_cache_desc(cache);
  if (st != KVX_STATUS_OK) return st;
  const kvx_kv_io_desc_t &io = write->io;
  if (io.num_kv_heads == 0 || io.head_dim == 0) return KVX_STATUS_INVALID_ARGUMENT;
  if (io.num_kv_heads != cache->num_kv_heads || io.head_dim != cache->head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (io.key.dtype != cache->k.dtype || io.value.dtype != cache->v.dtype)
    return KVX_STATUS_INVALID_ARGUMENT;
  st = check_io_3d(&io.key, io.num_tokens, io.num_kv_heads, io.head_dim);
  if (st != KVX_STATUS_OK) return st;
  st = check_io_3d(&io.value, io.num_tokens, io.num_kv_heads, io.head_dim);
  if (st != KVX_STATUS_OK) return st;
  st = check_slots(&write->slots, io.num_tokens);
  if (st != KVX_STATUS_OK) return st;

  const kvx_tensor_desc_t *ts[4] = {&cache->k, &cache->v, &io.key, &io.value};
  switch (classify(ts, 4)) {
    case Exec::kValidateOnly: return KVX_STATUS_OK;
    case Exec::kUnsupported: return KVX_STATUS_UNSUPPORTED;
    case Exec::kDevice: break;
  }
  // io dtype == cache dtype here, so F8 caches take the byte-copy path.
  return kvx_launch_write_kv(cache, write, stream);
}

KVX_API kvx_status_t kvx_gather_kv(const kvx_cache_desc_t *cache,
                                   const kvx_gather_desc_t *gather,
                                   void *stream) {
  if (cache == nullptr || gather == nullptr) return KVX_STATUS_INVALID_ARGUMENT;
  if (gather->size < sizeof(kvx_gather_desc_t) ||
      gather->io.size < sizeof(kvx_kv_io_desc_t) ||
      gather->block_table.size < sizeof(kvx_block_table_t) ||
      gather->seq_lens.size < sizeof(kvx_seq_lens_t))
    return KVX_STATUS_INVALID_ARGUMENT;
  kvx_status_t st = kvx_validate_cache_desc(cache);
  if (st != KVX_STATUS_OK) return st;
  const kvx_kv_io_desc_t &io = gather->io;
  if (io.num_kv_heads == 0 || io.head_dim == 0 || gather->max_seq_len == 0)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (io.num_kv_heads != cache->num_kv_heads || io.head_dim != cache->head_dim)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (io.key.dtype != cache->k.dtype || io.value.dtype != cache->v.dtype)
    return KVX_STATUS_INVALID_ARGUMENT;
  st = check_table(cache, &gather->block_table);
  if (st != KVX_STATUS_OK) return st;
  st = check_seq_lens(&gather->seq_lens, gather->block_table.seq_count);
  if (st != KVX_STATUS_OK) return st;
  if (gather->block_table.index_dtype != gather->seq_lens.dtype)
    return KVX_STATUS_INVALID_ARGUMENT;
  if (io.num_tokens != gather->block_table.seq_count * gather->max_seq_len)
    return KVX_STATUS_INVALID_ARGUMENT;
  st = check_io_4d(&io.key, gather->block_table.seq_count, gather->max_seq_len,
                   io.num_kv_heads, io.head_dim);
  if (st != KVX_STATUS_OK) return st;
  st = check_io_4d(&io.value, gather->block_table.seq_count,
                   gather->max_seq_len, io.num_kv_heads, io.head_dim);
  if (st != KVX_STATUS_OK) return st;
  // The reference ends with "format != PACKED -> UNSUPPORTED" (kvx_abi.c:462);
  // this build gathers RAGGED and KV_OFFSETS tables too.

  // KV_OFFSETS blocks live in the pool: the cache tensors only describe the
  // in-block layout and their data pointers are not read.
  const bool offsets = gather->block_table.format == KVX_BLOCK_TABLE_KV_OFFSETS;
  const kvx_tensor_desc_t *ts[4] = {&io.key, &io.value, &cache->k, &cache->v};
  switch (classify(ts, offsets ? 2 : 4, offsets ? &cache->pool : nullptr)) {
    case Exec::kValidateOnly: return KVX_STATUS_OK;
    case Exec::kUnsupported: return KVX_STATUS_UNSUPPORTED;
    case Exec::kDevice: break;
  }
  return kvx_launch_gather_kv(cache, gather, stream);
}

}  // extern "C"

// LP64 layout of the ABI structs.  A caller compiled against the reference
// kvx_abi.h sees exactly these sizes and offsets.
static_assert(sizeof(kvx_version_t) == 16, "abi");
static_assert(sizeof(kvx_tensor_desc_t) == 112, "abi");
static_assert(offsetof(kvx_tensor_desc_t, shape) == 24, "abi");
static_assert(offsetof(kvx_tensor_desc_t, stride) == 64, "abi");
static_assert(offsetof(kvx_tensor_desc_t, data) == 104, "abi");
static_assert(sizeof(kvx_pool_desc_t) == 32, "abi");
static_assert(sizeof(kvx_cache_desc_t) == 280, "abi");
static_assert(offsetof(kvx_cache_desc_t, k) == 24, "abi");
static_assert(offsetof(kvx_cache_desc_t, v) == 136, "abi");
static_assert(offsetof(kvx_cache_desc_t, pool) == 248, "abi");
static_assert(sizeof(kvx_block_table_t) == 64, "abi");
static_assert(sizeof(kvx_slot_mapping_t) == 32, "abi");
static_assert(sizeof(kvx_seq_lens_t) == 24, "abi");
static_assert(sizeof(kvx_kv_io_desc_t) == 248, "abi");
static_assert(sizeof(kvx_scale_desc_t) == 104, "abi");
static_assert(sizeof(kvx_write_desc_t) == 512, "abi");
static_assert(offsetof(kvx_write_desc_t, slots) == 256, "abi");
static_assert(offsetof(kvx_write_desc_t, k_scale) == 288, "abi");
static_assert(offsetof(kvx_write_desc_t, k_scale_desc) == 304, "abi");
static_assert(sizeof(kvx_gather_desc_t) == 352, "abi");
static_assert(offsetof(kvx_gather_desc_t, block_table) == 256, "abi");
static_assert(offsetof(kvx_gather_desc_t, seq_lens) == 320, "abi");
static_assert(offsetof(kvx_gather_desc_t, max_seq_len) == 344, "abi");
