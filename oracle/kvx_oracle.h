/*
 * CPU oracle for the KVX paged KV write / gather path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libkvx_amd.so, the
 * kvx_amd package) links, loads or calls this code; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
 * checker and as the timed CPU baseline.
 *
 * The reference ships no CPU implementation of write/gather (kvx_abi.c only
 * validates), so this is a restatement of the reference kernel semantics:
 *   oracle_cache_offset  kernels/kvx_paged_kv.cu:54-75
 *   oracle_write_kv      kernels/kvx_paged_kv.cu:93-124
 *   oracle_gather_kv     kernels/kvx_paged_kv.cu:226-267
 * plus the FP8 E4M3 cast this build adds (OCP FP8 definition).
 */
#ifndef KVX_ORACLE_H
#define KVX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout codes and dtype codes are the kvx_abi.h enum values.  For
 * KVX_LAYOUT_BLOCK_CUSTOM (15) the strides are those of the axes (block,
 * offset, head, dim / pack, dim % pack); a 4-axis custom tensor is pack =
 * head_dim with stride[3] = 0 and stride[4] its dim stride. */

/* FP8 scales: the scale of element (block b, head h) is
 * p[b * s_block + h * s_head] (strides in elements; a per-tensor scale has
 * both strides 0). */
typedef struct oracle_scale {
  const float *p;
  int64_t s_block;
  int64_t s_head;
} oracle_scale_t;

int64_t oracle_cache_offset(int layout, const int64_t *stride, int64_t pack,
                            int64_t block, int64_t offset, int64_t head,
                            int64_t dim);

/* Element-wise write.  io and cache dtypes are equal (bit copy) or the cache
 * is F8_E4M3 / F8_E5M2 and io is F16/BF16/F32 (quantize with k_scale /
 * v_scale, which may be NULL for a bit copy). */
void oracle_write_kv(int k_layout, const int64_t *k_stride, int64_t k_pack,
                     int v_layout, const int64_t *v_stride, int64_t v_pack,
                     const void *key, const void *value, void *key_cache,
                     void *value_cache, const void *slots, int slot_is64,
                     int64_t num_tokens, int32_t heads, int32_t head_dim,
                     int32_t block_size, int32_t num_blocks, int io_dtype,
                     int cache_dtype, const oracle_scale_t *k_scale, const oracle_scale_t *v_scale);

/* Element-wise gather into [seq_count, max_seq_len, H, D].  Rows not
 * written by the reference semantics are left untouched.  Dequantizes when
 * the cache is F8_E4M3 / F8_E5M2 and io is F16/BF16/F32. */
void oracle_gather_kv(int k_layout, const int64_t *k_stride, int64_t k_pack,
                      int v_layout, const int64_t *v_stride, int64_t v_pack,
                      const void *key_cache, const void *value_cache,
                      void *key_out, void *value_out, const void *block_table,
                      const void *seq_lens, int index_is64, int32_t seq_count,
                      int32_t max_blocks_per_seq, int32_t max_seq_len,
                      int32_t heads, int32_t head_dim, int32_t block_size,
                      int32_t num_blocks, int cache_dtype, int io_dtype,
                      const oracle_scale_t *k_scale, const oracle_scale_t *v_scale);

/* RAGGED table gather (KVX_SPEC.md:107-114): row t of sequence s is token
 * i = indptr[s] + t for t < min(seq_len, indptr[s+1] - indptr[s],
 * max_seq_len); its block id is indices[i] (skipped when < 0 or
 * >= num_blocks) and its block offset t % block_size.  Tokens with
 * i outside [0, indices_count) are skipped (malformed indptr). */
void oracle_gather_kv_ragged(int k_layout, const int64_t *k_stride, int64_t k_pack,
                             int v_layout, const int64_t *v_stride, int64_t v_pack,
                             const void *key_cache, const void *value_cache,
                             void *key_out, void *value_out, const void *indices,
                             int index_is64, int64_t indices_count, const void *indptr,
                             int indptr_is64, const void *seq_lens, int lens_is64,
                             int32_t seq_count, int32_t max_seq_len, int32_t heads,
                             int32_t head_dim, int32_t block_size, int32_t num_blocks,
                             int cache_dtype, int io_dtype, const oracle_scale_t *k_scale, const oracle_scale_t *v_scale);

/* KV_OFFSETS table gather (KVX_SPEC.md:116-122, KV_CACHE_LAYOUTS.md:89-94):
 * table [seq_count, 1, 2, max_blocks_per_seq] of int32 KVCacheIndex values,
 * bit 31 selecting the secondary pool; block address = pool + (value &
 * 0x7FFFFFFF) * bytes_per_block, skipped when the index is >= num_blocks or
 * the pool is NULL.  In-block addressing follows the K / V strides (the
 * block stride is unused).  Rows t >= min(seq_len, max_seq_len) or with
 * t / block_size >= max_blocks_per_seq are untouched. */
void oracle_gather_kv_offsets(int k_layout, const int64_t *k_stride, int64_t k_pack,
                              int v_layout, const int64_t *v_stride, int64_t v_pack,
                              const void *pool_primary, const void *pool_secondary,
                              int64_t bytes_per_block, void *key_out, void *value_out,
                              const int32_t *table, const void *seq_lens, int lens_is64,
                              int32_t seq_count, int32_t max_blocks_per_seq,
                              int32_t max_seq_len, int32_t heads, int32_t head_dim,
                              int32_t block_size, int32_t num_blocks, int cache_dtype,
                              int io_dtype, const oracle_scale_t *k_scale, const oracle_scale_t *v_scale);

/* Same results as the element-wise functions for bit-copy calls, with one
 * memcpy per contiguous run and OpenMP over tokens / (sequence, block); the
 * timed CPU baseline.  Returns the number of OpenMP threads used. */
int oracle_write_kv_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                         int v_layout, const int64_t *v_stride, int64_t v_pack,
                         const void *key, const void *value, void *key_cache,
                         void *value_cache, const void *slots, int slot_is64,
                         int64_t num_tokens, int32_t heads, int32_t head_dim,
                         int32_t block_size, int32_t num_blocks, int elem_size);

int oracle_gather_kv_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                          int v_layout, const int64_t *v_stride, int64_t v_pack,
                          const void *key_cache, const void *value_cache,
                          void *key_out, void *value_out,
                          const void *block_table, const void *seq_lens,
                          int index_is64, int32_t seq_count,
                          int32_t max_blocks_per_seq, int32_t max_seq_len,
                          int32_t heads, int32_t head_dim, int32_t block_size,
                          int32_t num_blocks, int elem_size);

/* FP8 variants of the fast paths (the timed CPU baseline of FP8 caches):
 * per-tensor scales, same results as oracle_write_kv / oracle_gather_kv.
 * The casts are table lookups built once from the element-wise casts below
 * (oracle_quantize_fp8_fast / oracle_dequantize_fp8_fast expose them for the
 * tests).  Return the number of OpenMP threads used. */
int oracle_write_kv_quant_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                               int v_layout, const int64_t *v_stride, int64_t v_pack,
                               const void *key, const void *value, void *key_cache,
                               void *value_cache, const void *slots, int slot_is64,
                               int64_t num_tokens, int32_t heads, int32_t head_dim,
                               int32_t block_size, int32_t num_blocks, int io_dtype,
                               int cache_dtype, float k_scale, float v_scale);

int oracle_gather_kv_dequant_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                                  int v_layout, const int64_t *v_stride, int64_t v_pack,
                                  const void *key_cache, const void *value_cache,
                                  void *key_out, void *value_out,
                                  const void *block_table, const void *seq_lens,
                                  int index_is64, int32_t seq_count,
                                  int32_t max_blocks_per_seq, int32_t max_seq_len,
                                  int32_t heads, int32_t head_dim, int32_t block_size,
                                  int32_t num_blocks, int cache_dtype, int io_dtype,
                                  float k_scale, float v_scale);

void oracle_quantize_fp8_fast(const void *in, int io_dtype, int64_t n, float scale,
                              int fp8_dtype, uint8_t *out);
void oracle_dequantize_fp8_fast(const uint8_t *in, int64_t n, float scale, int fp8_dtype,
                                int io_dtype, void *out);

/* Threads of the *_fast functions from now on (n > 0); returns the previous
 * count (always 1 without OpenMP). */
int oracle_set_threads(int n);

/* Scalar casts (OCP E4M3 and E5M2, bf16, f16), by nearest-value search.
 * FP8 casts saturate to the largest finite value (infinities included). */
uint8_t oracle_f32_to_e4m3(float v);
float oracle_e4m3_to_f32(uint8_t q);
uint8_t oracle_f32_to_e5m2(float v);
float oracle_e5m2_to_f32(uint8_t q);
uint16_t oracle_f32_to_bf16(float v);
uint16_t oracle_f32_to_f16(float v);
float oracle_f16_to_f32(uint16_t h);

/* Array versions for tests: out[i] = cast(in[i] / scale) etc.; fp8_dtype is
 * F8_E4M3 or F8_E5M2. */
void oracle_quantize_fp8(const void *in, int io_dtype, int64_t n, float scale,
                         int fp8_dtype, uint8_t *out);
void oracle_dequantize_fp8(const uint8_t *in, int64_t n, float scale, int fp8_dtype,
                           int io_dtype, void *out);

#ifdef __cplusplus
}
#endif

#endif /* KVX_ORACLE_H */
