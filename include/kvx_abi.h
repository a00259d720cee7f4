/*
 * KVX v1 C ABI — descriptor types and the four ABI entry points.
 *
 * This header is the drop-in boundary: every type, enumerator, field order
 * and function signature matches the reference ABI (kvx_abi.h:11-199) so that
 * a caller compiled against the reference header links against this library
 * unchanged.  Struct sizes and field offsets for LP64 are pinned by the
 * static assertions at the end of kvx_amd/csrc/abi.cpp.
 *
 * Conventions (KVX_SPEC.md:36-135, :240-289):
 *   - every struct starts with `uint32_t size`; callees reject size < sizeof;
 *   - tensor strides are counted in elements, not bytes;
 *   - `stream` is an opaque hipStream_t (NULL = the default stream);
 *   - the caller owns every buffer; nothing is retained after a call returns.
 */
#ifndef KVX_ABI_H
#define KVX_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version reported by kvx_get_version (reference kvx_abi.h:11-12). */
#define KVX_ABI_VERSION_MAJOR 1
#define KVX_ABI_VERSION_MINOR 1

/* Enumerations are 32-bit.  C++ callers (and this library) see a fixed
 * underlying type, so that a field holding a value outside the enumerators
 * (a caller error the validators report) is an ordinary value to read, as it
 * is in C; the layout is unchanged. */
#ifdef __cplusplus
#define KVX_ENUM_BASE : int32_t
#else
#define KVX_ENUM_BASE
#endif

/* Export decoration: empty on ELF platforms, as in reference kvx_abi.h:14-24. */
#if defined(_WIN32)
#if defined(KVX_BUILD_DLL)
#define KVX_API __declspec(dllexport)
#elif defined(KVX_USE_DLL)
#define KVX_API __declspec(dllimport)
#else
#define KVX_API
#endif
#else
#define KVX_API
#endif

/* Status codes (reference kvx_abi.h:26-33). */
typedef enum kvx_status KVX_ENUM_BASE {
  KVX_STATUS_OK = 0,
  KVX_STATUS_INVALID_ARGUMENT = 1,
  KVX_STATUS_UNSUPPORTED = 2,
  KVX_STATUS_OUT_OF_RANGE = 3,
  KVX_STATUS_INCOMPATIBLE = 4,
  KVX_STATUS_INTERNAL_ERROR = 5
} kvx_status_t;

/* reference kvx_abi.h:35-40 */
typedef struct kvx_version {
  uint32_t size;
  uint32_t abi_major;
  uint32_t abi_minor;
  uint32_t abi_patch;
} kvx_version_t;

/* Element types (reference kvx_abi.h:42-54). */
typedef enum kvx_dtype KVX_ENUM_BASE {
  KVX_DTYPE_INVALID = 0,
  KVX_DTYPE_F16 = 1,
  KVX_DTYPE_BF16 = 2,
  KVX_DTYPE_F32 = 3,
  KVX_DTYPE_F8_E4M3 = 4,
  KVX_DTYPE_F8_E5M2 = 5,
  KVX_DTYPE_S32 = 6,
  KVX_DTYPE_S64 = 7,
  KVX_DTYPE_U32 = 8,
  KVX_DTYPE_U64 = 9,
  KVX_DTYPE_U8 = 10
} kvx_dtype_t;

/* Where a buffer lives (reference kvx_abi.h:56-61). */
typedef enum kvx_memory_type KVX_ENUM_BASE {
  KVX_MEMORY_UNKNOWN = 0,
  KVX_MEMORY_HOST = 1,
  KVX_MEMORY_DEVICE = 2,
  KVX_MEMORY_UNIFIED = 3
} kvx_memory_type_t;

/*
 * Paged cache layouts (reference kvx_abi.h:63-69):
 *   NHD        [num_blocks, block_size, heads, head_dim]
 *   HND        [num_blocks, heads, block_size, head_dim]
 *   HND_PACKED [num_blocks, heads, head_dim / x, block_size, x], x = shape[4]
 */
typedef enum kvx_layout KVX_ENUM_BASE {
  KVX_LAYOUT_INVALID = 0,
  KVX_LAYOUT_BLOCK_NHD = 1,
  KVX_LAYOUT_BLOCK_HND = 2,
  KVX_LAYOUT_BLOCK_HND_PACKED = 3,
  KVX_LAYOUT_BLOCK_CUSTOM = 15
} kvx_layout_t;

enum { KVX_MAX_TENSOR_DIMS = 5 };

/* reference kvx_abi.h:73-82 (112 bytes on LP64) */
typedef struct kvx_tensor_desc {
  uint32_t size;
  kvx_dtype_t dtype;
  kvx_layout_t layout;
  kvx_memory_type_t memory;
  uint32_t ndim;
  int64_t shape[KVX_MAX_TENSOR_DIMS];
  int64_t stride[KVX_MAX_TENSOR_DIMS];
  void *data;
} kvx_tensor_desc_t;

/* reference kvx_abi.h:84-90 (32 bytes) */
typedef struct kvx_pool_desc {
  uint32_t size;
  kvx_memory_type_t memory;
  uint32_t bytes_per_block;
  void *primary;
  void *secondary;
} kvx_pool_desc_t;

/* reference kvx_abi.h:92-101 (280 bytes) */
typedef struct kvx_cache_desc {
  uint32_t size;
  uint32_t num_blocks;
  uint32_t block_size;
  uint32_t num_kv_heads;
  uint32_t head_dim;
  kvx_tensor_desc_t k;
  kvx_tensor_desc_t v;
  kvx_pool_desc_t pool;
} kvx_cache_desc_t;

/* reference kvx_abi.h:103-108 */
typedef enum kvx_block_table_format KVX_ENUM_BASE {
  KVX_BLOCK_TABLE_INVALID = 0,
  KVX_BLOCK_TABLE_PACKED = 1,
  KVX_BLOCK_TABLE_RAGGED = 2,
  KVX_BLOCK_TABLE_KV_OFFSETS = 3
} kvx_block_table_format_t;

/* reference kvx_abi.h:110-113 */
typedef enum kvx_block_table_flags KVX_ENUM_BASE {
  KVX_BLOCK_TABLE_FLAG_NONE = 0,
  KVX_BLOCK_TABLE_FLAG_KVCACHEINDEX = 1 << 0
} kvx_block_table_flags_t;

/* reference kvx_abi.h:115-128 (64 bytes) */
typedef struct kvx_block_table {
  uint32_t size;
  kvx_block_table_format_t format;
  kvx_dtype_t index_dtype;
  kvx_dtype_t indptr_dtype;
  uint32_t seq_count;
  uint32_t beam_width;
  uint32_t max_blocks_per_seq;
  const void *indices;
  const void *indptr;
  uint32_t indices_count;
  uint32_t indptr_count;
  uint32_t flags;
} kvx_block_table_t;

/* reference kvx_abi.h:130-136 (32 bytes) */
typedef struct kvx_slot_mapping {
  uint32_t size;
  kvx_dtype_t dtype;
  uint32_t token_count;
  int64_t invalid_slot;
  const void *slots;
} kvx_slot_mapping_t;

/* reference kvx_abi.h:138-143 (24 bytes) */
typedef struct kvx_seq_lens {
  uint32_t size;
  kvx_dtype_t dtype;
  uint32_t seq_count;
  const void *lengths;
} kvx_seq_lens_t;

/* reference kvx_abi.h:145-152 (248 bytes) */
typedef struct kvx_kv_io_desc {
  uint32_t size;
  kvx_tensor_desc_t key;
  kvx_tensor_desc_t value;
  uint32_t num_tokens;
  uint32_t num_kv_heads;
  uint32_t head_dim;
} kvx_kv_io_desc_t;

/* reference kvx_abi.h:154-160 */
typedef enum kvx_scale_granularity KVX_ENUM_BASE {
  KVX_SCALE_NONE = 0,
  KVX_SCALE_PER_TENSOR = 1,
  KVX_SCALE_PER_BLOCK = 2,
  KVX_SCALE_PER_HEAD = 3,
  KVX_SCALE_PER_BLOCK_HEAD = 4
} kvx_scale_granularity_t;

/* reference kvx_abi.h:162-170 (104 bytes) */
typedef struct kvx_scale_desc {
  uint32_t size;
  kvx_dtype_t dtype;
  kvx_scale_granularity_t granularity;
  uint32_t ndim;
  int64_t shape[KVX_MAX_TENSOR_DIMS];
  int64_t stride[KVX_MAX_TENSOR_DIMS];
  const void *data;
} kvx_scale_desc_t;

/* reference kvx_abi.h:172-180 (512 bytes) */
typedef struct kvx_write_desc {
  uint32_t size;
  kvx_kv_io_desc_t io;
  kvx_slot_mapping_t slots;
  const void *k_scale;
  const void *v_scale;
  kvx_scale_desc_t k_scale_desc;
  kvx_scale_desc_t v_scale_desc;
} kvx_write_desc_t;

/* reference kvx_abi.h:182-188 (352 bytes) */
typedef struct kvx_gather_desc {
  uint32_t size;
  kvx_kv_io_desc_t io;
  kvx_block_table_t block_table;
  kvx_seq_lens_t seq_lens;
  uint32_t max_seq_len;
} kvx_gather_desc_t;

/* Fills *out_version with {sizeof, 1, 1, 0}.  Replaces reference
 * kvx_abi.c:313-322. */
KVX_API kvx_status_t kvx_get_version(kvx_version_t *out_version);

/* Strict cache validation: canonical strides, equal K/V layout and dtype,
 * non-NULL data.  Same status codes and check order as reference
 * kvx_abi.c:324-352. */
KVX_API kvx_status_t kvx_validate_cache_desc(const kvx_cache_desc_t *cache);

/* Validates exactly as reference kvx_abi.c:354-398, then performs the write
 * on the GPU when the buffers are device memory.  Descriptors whose buffers
 * are all KVX_MEMORY_HOST are validated only (the reference's behaviour). */
KVX_API kvx_status_t kvx_write_kv(const kvx_cache_desc_t *cache,
                                  const kvx_write_desc_t *write, void *stream);

/* Validates exactly as reference kvx_abi.c:400-466, then performs the gather
 * on the GPU when the buffers are device memory (HOST: validation only). */
KVX_API kvx_status_t kvx_gather_kv(const kvx_cache_desc_t *cache,
                                   const kvx_gather_desc_t *gather,
                                   void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KVX_ABI_H */
