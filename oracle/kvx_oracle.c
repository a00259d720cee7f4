/*
 * CPU oracle for the KVX paged KV write / gather path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke()
 * and the timed CPU baseline of bench.py.  The product never links it.
 *
 * Element-wise restatement of the reference kernels
 * (kernels/kvx_paged_kv.cu:54-75, :93-124, :226-267).  One intended
 * divergence: block ids >= num_blocks in the gather are skipped (the
 * reference reads out of bounds there, KVX_CONFORMANCE.md:31).
 *
 * The FP8 / bf16 / f16 casts are written independently of the product's bit
 * manipulation (kvx_amd/csrc/fp_convert.h): they decode the target format's
 * code table and pick the nearest representable value with ties to the even
 * code, in double precision.  Agreement of the two methods over every input
 * class is what the tests check.
 */
#include "kvx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { L_NHD = 1, L_HND = 2, L_PACKED = 3, L_CUSTOM = 15 };
enum { D_F16 = 1, D_BF16 = 2, D_F32 = 3, D_E4M3 = 4, D_E5M2 = 5 };

static int dtype_size(int dt) {
  switch (dt) {
    case D_F32: return 4;
    case D_F16:
    case D_BF16: return 2;
    case D_E4M3:
    case D_E5M2: return 1;
    default: return 0;
  }
}

/* kernels/kvx_paged_kv.cu:54-75 */
int64_t oracle_cache_offset(int layout, const int64_t *s, int64_t pack,
                            int64_t b, int64_t o, int64_t h, int64_t d) {
  switch (layout) {
    case L_NHD:
      return b * s[0] + o * s[1] + h * s[2] + d * s[3];
    case L_HND:
      return b * s[0] + h * s[1] + o * s[2] + d * s[3];
    case L_PACKED: {
      const int64_t pd = d / pack;
      const int64_t po = d - pd * pack;
      return b * s[0] + h * s[1] + pd * s[2] + o * s[3] + po * s[4];
    }
    case L_CUSTOM: {
      /* axes (block, offset, head, dim / pack, dim % pack); a 4-axis
       * descriptor is pack = head_dim with s[3] = 0 and s[4] its dim stride */
      const int64_t pd = d / pack;
      const int64_t po = d - pd * pack;
      return b * s[0] + o * s[1] + h * s[2] + pd * s[3] + po * s[4];
    }
    default:
      return 0;
  }
}

/* ------------------------------------------------------------------------ */
/* Casts by nearest-value search.                                            */

static uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float float_of(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Magnitude of E4M3 code c (0..126): exponent field e, mantissa m. */
static double e4m3_mag(int c) {
  const int e = (c >> 3) & 15, m = c & 7;
  if (e == 0) return ldexp((double)m, -9);
  return ldexp(8.0 + m, e - 10);
}

/* Pick the nearer of two adjacent codes lo < hi (values vlo < a < vhi),
 * ties to the code whose lowest bit is 0. */
static uint32_t nearest(double a, uint32_t lo, double vlo, uint32_t hi,
                        double vhi) {
  const double dlo = a - vlo, dhi = vhi - a;
  if (dlo < dhi) return lo;
  if (dhi < dlo) return hi;
  return (lo & 1u) ? hi : lo;
}

uint8_t oracle_f32_to_e4m3(float v) {
  if (isnan(v)) return 0x7F;
  const uint8_t sign = signbit(v) ? 0x80 : 0x00;
  double a = fabs((double)v);
  if (a >= 448.0) return sign | 0x7E; /* saturate, infinities included */
  int lo = 0, hi = 126;               /* largest code with mag <= a */
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (e4m3_mag(mid) <= a) lo = mid; else hi = mid - 1;
  }
  if (e4m3_mag(lo) == a) return sign | (uint8_t)lo;
  return sign | (uint8_t)nearest(a, (uint32_t)lo, e4m3_mag(lo),
                                 (uint32_t)lo + 1, e4m3_mag(lo + 1));
}

float oracle_e4m3_to_f32(uint8_t q) {
  if ((q & 0x7F) == 0x7F) return float_of(0x7FC00000u);
  const double m = e4m3_mag(q & 0x7F);
  return (float)((q & 0x80) ? -m : m);
}

/* Magnitude of E5M2 code c (0..123): exponent field e, mantissa m. */
static double e5m2_mag(int c) {
  const int e = (c >> 2) & 31, m = c & 3;
  if (e == 0) return ldexp((double)m, -16);
  return ldexp(4.0 + m, e - 17);
}

uint8_t oracle_f32_to_e5m2(float v) {
  if (isnan(v)) return 0x7E;
  const uint8_t sign = signbit(v) ? 0x80 : 0x00;
  const double a = fabs((double)v);
  if (a >= 57344.0) return sign | 0x7B; /* saturate, infinities included */
  int lo = 0, hi = 123;                 /* largest code with mag <= a */
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (e5m2_mag(mid) <= a) lo = mid; else hi = mid - 1;
  }
  if (e5m2_mag(lo) == a) return sign | (uint8_t)lo;
  return sign | (uint8_t)nearest(a, (uint32_t)lo, e5m2_mag(lo),
                                 (uint32_t)lo + 1, e5m2_mag(lo + 1));
}

float oracle_e5m2_to_f32(uint8_t q) {
  const int c = q & 0x7F;
  if (c > 0x7C) return float_of(0x7FC00000u);
  if (c == 0x7C) return (q & 0x80) ? -INFINITY : INFINITY;
  const double m = e5m2_mag(c);
  return (float)((q & 0x80) ? -m : m);
}

uint16_t oracle_f32_to_bf16(float v) {
  if (isnan(v)) return 0x7FC0;
  const uint32_t u = bits_of(v);
  const uint32_t sign = u & 0x80000000u;
  const uint32_t mag = u & 0x7FFFFFFFu;
  const uint32_t lo = mag & 0xFFFF0000u; /* bf16 at or below |v| */
  if (lo == mag) return (uint16_t)((sign | mag) >> 16);
  const uint32_t hi = lo + 0x10000u;
  /* The code above the largest finite bf16 is infinity; for rounding it
   * stands at 2^128. */
  const double vhi = (hi == 0x7F800000u) ? ldexp(1.0, 128) : (double)float_of(hi);
  const uint32_t r = nearest(fabs((double)v), lo >> 16, (double)float_of(lo),
                             hi >> 16, vhi);
  return (uint16_t)((sign >> 16) | r);
}

/* Positive finite f16 magnitudes, code 0..0x7BFF. */
static double f16_mag(uint32_t c) {
  const uint32_t e = (c >> 10) & 31, m = c & 1023;
  if (e == 0) return ldexp((double)m, -24);
  return ldexp(1024.0 + m, (int)e - 25);
}

uint16_t oracle_f32_to_f16(float v) {
  if (isnan(v)) return 0x7E00;
  const uint16_t sign = signbit(v) ? 0x8000 : 0;
  const double a = fabs((double)v);
  if (isinf(v)) return sign | 0x7C00;
  /* Above the largest finite value 65504 the next code is infinity, which
   * stands at 2^16 for rounding. */
  if (a > 65504.0) {
    return sign | (uint16_t)nearest(a, 0x7BFF, 65504.0, 0x7C00, 65536.0);
  }
  uint32_t lo = 0, hi = 0x7BFF;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) / 2;
    if (f16_mag(mid) <= a) lo = mid; else hi = mid - 1;
  }
  if (f16_mag(lo) == a) return sign | (uint16_t)lo;
  return sign | (uint16_t)nearest(a, lo, f16_mag(lo), lo + 1, f16_mag(lo + 1));
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t c = h & 0x7FFF;
  if (c >= 0x7C00) {
    if (c == 0x7C00) return (h & 0x8000) ? -INFINITY : INFINITY;
    return float_of(((uint32_t)(h & 0x8000) << 16) | 0x7F800000u |
                    ((uint32_t)(h & 0x3FF) << 13));
  }
  const double m = f16_mag(c);
  return (float)((h & 0x8000) ? -m : m);
}

static float load_io_f32(const uint8_t *p, int dt) {
  switch (dt) {
    case D_F32: {
      float f;
      memcpy(&f, p, 4);
      return f;
    }
    case D_BF16: {
      uint16_t h;
      memcpy(&h, p, 2);
      return float_of((uint32_t)h << 16);
    }
    default: {
      uint16_t h;
      memcpy(&h, p, 2);
      return oracle_f16_to_f32(h);
    }
  }
}

static void store_io_f32(uint8_t *p, int dt, float v) {
  switch (dt) {
    case D_F32: {
      const float c = isnan(v) ? float_of(0x7FC00000u) : v;
      memcpy(p, &c, 4);
      break;
    }
    case D_BF16: {
      const uint16_t h = oracle_f32_to_bf16(v);
      memcpy(p, &h, 2);
      break;
    }
    default: {
      const uint16_t h = oracle_f32_to_f16(v);
      memcpy(p, &h, 2);
      break;
    }
  }
}

/* q = fp8(sat(f32(x) / scale)); the division is one IEEE f32 division. */
static uint8_t quant_one(const uint8_t *src, int io_dtype, int fp8, float scale) {
  const float x = load_io_f32(src, io_dtype);
  volatile float q = x / scale; /* force an f32-rounded quotient */
  return fp8 == D_E5M2 ? oracle_f32_to_e5m2(q) : oracle_f32_to_e4m3(q);
}

/* y = io(f32(q) * scale); the product is one IEEE f32 multiplication. */
static void dequant_one(uint8_t q, int fp8, float scale, int io_dtype, uint8_t *dst) {
  volatile float y = (fp8 == D_E5M2 ? oracle_e5m2_to_f32(q) : oracle_e4m3_to_f32(q)) * scale;
  store_io_f32(dst, io_dtype, y);
}

/* Scale of (block b, head h); 1 without a scale. */
static float scale_at(const oracle_scale_t *s, int64_t b, int64_t h) {
  if (s == NULL || s->p == NULL) return 1.0f;
  return s->p[b * s->s_block + h * s->s_head];
}

void oracle_quantize_fp8(const void *in, int io_dtype, int64_t n, float scale,
                         int fp8_dtype, uint8_t *out) {
  const int es = dtype_size(io_dtype);
  for (int64_t i = 0; i < n; ++i)
    out[i] = quant_one((const uint8_t *)in + i * es, io_dtype, fp8_dtype, scale);
}

void oracle_dequantize_fp8(const uint8_t *in, int64_t n, float scale, int fp8_dtype,
                           int io_dtype, void *out) {
  const int es = dtype_size(io_dtype);
  for (int64_t i = 0; i < n; ++i)
    dequant_one(in[i], fp8_dtype, scale, io_dtype, (uint8_t *)out + i * es);
}

/* ------------------------------------------------------------------------ */
/* Write and gather.                                                          */

static int64_t load_index(const void *base, int64_t i, int is64) {
  return is64 ? ((const int64_t *)base)[i]
              : (int64_t)((const int32_t *)base)[i];
}

/* kernels/kvx_paged_kv.cu:93-124 */
void oracle_write_kv(int k_layout, const int64_t *k_stride, int64_t k_pack,
                     int v_layout, const int64_t *v_stride, int64_t v_pack,
                     const void *key, const void *value, void *key_cache,
                     void *value_cache, const void *slots, int slot_is64,
                     int64_t num_tokens, int32_t heads, int32_t head_dim,
                     int32_t block_size, int32_t num_blocks, int io_dtype,
                     int cache_dtype, const oracle_scale_t *k_scale,
                     const oracle_scale_t *v_scale) {
  const int is = dtype_size(io_dtype), cs = dtype_size(cache_dtype);
  const int quant = io_dtype != cache_dtype;
  const uint8_t *k_in = key, *v_in = value;
  uint8_t *kc = key_cache, *vc = value_cache;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = load_index(slots, t, slot_is64);
    if (slot < 0) continue;
    const int64_t b = slot / block_size;
    const int64_t o = slot - b * block_size;
    if (b < 0 || b >= num_blocks) continue;
    for (int64_t h = 0; h < heads; ++h) {
      for (int64_t d = 0; d < head_dim; ++d) {
        const int64_t idx = (t * heads + h) * head_dim + d;
        const int64_t ko = oracle_cache_offset(k_layout, k_stride, k_pack, b, o, h, d);
        const int64_t vo = oracle_cache_offset(v_layout, v_stride, v_pack, b, o, h, d);
        if (quant) {
          kc[ko] = quant_one(k_in + idx * is, io_dtype, cache_dtype, scale_at(k_scale, b, h));
          vc[vo] = quant_one(v_in + idx * is, io_dtype, cache_dtype, scale_at(v_scale, b, h));
        } else {
          memcpy(kc + ko * cs, k_in + idx * is, (size_t)cs);
          memcpy(vc + vo * cs, v_in + idx * is, (size_t)cs);
        }
      }
    }
  }
}

/* kernels/kvx_paged_kv.cu:226-267 */
void oracle_gather_kv(int k_layout, const int64_t *k_stride, int64_t k_pack,
                      int v_layout, const int64_t *v_stride, int64_t v_pack,
                      const void *key_cache, const void *value_cache,
                      void *key_out, void *value_out, const void *block_table,
                      const void *seq_lens, int index_is64, int32_t seq_count,
                      int32_t max_blocks_per_seq, int32_t max_seq_len,
                      int32_t heads, int32_t head_dim, int32_t block_size,
                      int32_t num_blocks, int cache_dtype, int io_dtype,
                      const oracle_scale_t *k_scale, const oracle_scale_t *v_scale) {
  const int is = dtype_size(io_dtype), cs = dtype_size(cache_dtype);
  const int dequant = io_dtype != cache_dtype;
  const uint8_t *kc = key_cache, *vc = value_cache;
  uint8_t *ko_ = key_out, *vo_ = value_out;
  for (int64_t s = 0; s < seq_count; ++s) {
    const int64_t seq_len = load_index(seq_lens, s, index_is64);
    for (int64_t t = 0; t < max_seq_len; ++t) {
      if (t >= seq_len) continue;
      const int64_t lb = t / block_size;
      if (lb >= max_blocks_per_seq) continue;
      const int64_t bid =
          load_index(block_table, s * max_blocks_per_seq + lb, index_is64);
      if (bid < 0) continue;
      if (bid >= num_blocks) continue; /* reference reads out of bounds */
      const int64_t o = t - lb * block_size;
      for (int64_t h = 0; h < heads; ++h) {
        for (int64_t d = 0; d < head_dim; ++d) {
          const int64_t idx = ((s * max_seq_len + t) * heads + h) * head_dim + d;
          const int64_t ko =
              oracle_cache_offset(k_layout, k_stride, k_pack, bid, o, h, d);
          const int64_t vo =
              oracle_cache_offset(v_layout, v_stride, v_pack, bid, o, h, d);
          if (dequant) {
            dequant_one(kc[ko], cache_dtype, scale_at(k_scale, bid, h), io_dtype,
                        ko_ + idx * is);
            dequant_one(vc[vo], cache_dtype, scale_at(v_scale, bid, h), io_dtype,
                        vo_ + idx * is);
          } else {
            memcpy(ko_ + idx * is, kc + ko * cs, (size_t)cs);
            memcpy(vo_ + idx * is, vc + vo * cs, (size_t)cs);
          }
        }
      }
    }
  }
}

/* One element of a row: copy or dequantize from `src` to `dst`. */
static void move_elem(const uint8_t *src, uint8_t *dst, int dequant, int cs, int is,
                      int cache_dtype, int io_dtype, float scale) {
  if (dequant) {
    dequant_one(*src, cache_dtype, scale, io_dtype, dst);
  } else {
    memcpy(dst, src, (size_t)(cs < is ? cs : is));
  }
}

/* KVX_SPEC.md:107-114 */
void oracle_gather_kv_ragged(int k_layout, const int64_t *k_stride, int64_t k_pack,
                             int v_layout, const int64_t *v_stride, int64_t v_pack,
                             const void *key_cache, const void *value_cache,
                             void *key_out, void *value_out, const void *indices,
                             int index_is64, int64_t indices_count, const void *indptr,
                             int indptr_is64, const void *seq_lens, int lens_is64,
                             int32_t seq_count, int32_t max_seq_len, int32_t heads,
                             int32_t head_dim, int32_t block_size, int32_t num_blocks,
                             int cache_dtype, int io_dtype, const oracle_scale_t *k_scale,
                             const oracle_scale_t *v_scale) {
  const int is = dtype_size(io_dtype), cs = dtype_size(cache_dtype);
  const int dequant = io_dtype != cache_dtype;
  const uint8_t *kc = key_cache, *vc = value_cache;
  uint8_t *ko_ = key_out, *vo_ = value_out;
  for (int64_t s = 0; s < seq_count; ++s) {
    const int64_t seq_len = load_index(seq_lens, s, lens_is64);
    const int64_t start = load_index(indptr, s, indptr_is64);
    const int64_t cnt = load_index(indptr, s + 1, indptr_is64) - start;
    for (int64_t t = 0; t < max_seq_len; ++t) {
      if (t >= seq_len || t >= cnt || start < 0 || start + t >= indices_count) continue;
      const int64_t bid = load_index(indices, start + t, index_is64);
      if (bid < 0 || bid >= num_blocks) continue;
      const int64_t o = t % block_size;
      for (int64_t h = 0; h < heads; ++h) {
        for (int64_t d = 0; d < head_dim; ++d) {
          const int64_t idx = ((s * max_seq_len + t) * heads + h) * head_dim + d;
          const int64_t ko = oracle_cache_offset(k_layout, k_stride, k_pack, bid, o, h, d);
          const int64_t vo = oracle_cache_offset(v_layout, v_stride, v_pack, bid, o, h, d);
          move_elem(kc + ko * cs, ko_ + idx * is, dequant, cs, is, cache_dtype, io_dtype,
                    scale_at(k_scale, bid, h));
          move_elem(vc + vo * cs, vo_ + idx * is, dequant, cs, is, cache_dtype, io_dtype,
                    scale_at(v_scale, bid, h));
        }
      }
    }
  }
}

/* KVX_SPEC.md:116-122; KV_CACHE_LAYOUTS.md:89-94 */
void oracle_gather_kv_offsets(int k_layout, const int64_t *k_stride, int64_t k_pack,
                              int v_layout, const int64_t *v_stride, int64_t v_pack,
                              const void *pool_primary, const void *pool_secondary,
                              int64_t bytes_per_block, void *key_out, void *value_out,
                              const int32_t *table, const void *seq_lens, int lens_is64,
                              int32_t seq_count, int32_t max_blocks_per_seq,
                              int32_t max_seq_len, int32_t heads, int32_t head_dim,
                              int32_t block_size, int32_t num_blocks, int cache_dtype,
                              int io_dtype, const oracle_scale_t *k_scale,
                              const oracle_scale_t *v_scale) {
  const int is = dtype_size(io_dtype), cs = dtype_size(cache_dtype);
  const int dequant = io_dtype != cache_dtype;
  const uint8_t *pools[2] = {pool_primary, pool_secondary};
  uint8_t *outs[2] = {key_out, value_out};
  const int layouts[2] = {k_layout, v_layout};
  const int64_t *strides[2] = {k_stride, v_stride};
  const int64_t packs[2] = {k_pack, v_pack};
  const oracle_scale_t *scales[2] = {k_scale, v_scale};
  for (int64_t s = 0; s < seq_count; ++s) {
    const int64_t seq_len = load_index(seq_lens, s, lens_is64);
    for (int64_t t = 0; t < max_seq_len; ++t) {
      if (t >= seq_len) continue;
      const int64_t lb = t / block_size;
      if (lb >= max_blocks_per_seq) continue;
      const int64_t o = t - lb * block_size;
      for (int kv = 0; kv < 2; ++kv) {
        const uint32_t raw = (uint32_t)table[(s * 2 + kv) * max_blocks_per_seq + lb];
        const uint8_t *pool = pools[raw >> 31];
        const int64_t blk = (int64_t)(raw & 0x7FFFFFFFu);
        if (pool == NULL || blk >= num_blocks) continue;
        const uint8_t *base = pool + blk * bytes_per_block;
        for (int64_t h = 0; h < heads; ++h) {
          for (int64_t d = 0; d < head_dim; ++d) {
            const int64_t idx = ((s * max_seq_len + t) * heads + h) * head_dim + d;
            const int64_t off = oracle_cache_offset(layouts[kv], strides[kv], packs[kv], 0, o,
                                                    h, d);
            move_elem(base + off * cs, outs[kv] + idx * is, dequant, cs, is, cache_dtype,
                      io_dtype, scale_at(scales[kv], blk, h));
          }
        }
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Fast bit-copy variants (the timed CPU baseline).                           */

/* Elements of one contiguous run inside a (block, offset, head) row. */
static int64_t run_elems(int layout, const int64_t *s, int64_t pack,
                         int32_t head_dim) {
  if (layout == L_PACKED || layout == L_CUSTOM) return s[4] == 1 ? pack : 1;
  return s[3] == 1 ? head_dim : 1;
}

static int threads_used(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Threads of the *_fast functions from now on (n > 0); returns the previous
   count.  Builds without OpenMP always use 1. */
int oracle_set_threads(int n) {
  const int prev = threads_used();
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
  return prev;
}

int oracle_write_kv_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                         int v_layout, const int64_t *v_stride, int64_t v_pack,
                         const void *key, const void *value, void *key_cache,
                         void *value_cache, const void *slots, int slot_is64,
                         int64_t num_tokens, int32_t heads, int32_t head_dim,
                         int32_t block_size, int32_t num_blocks, int es) {
  const int64_t kr = run_elems(k_layout, k_stride, k_pack, head_dim);
  const int64_t vr = run_elems(v_layout, v_stride, v_pack, head_dim);
  const uint8_t *k_in = key, *v_in = value;
  uint8_t *kc = key_cache, *vc = value_cache;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = load_index(slots, t, slot_is64);
    if (slot < 0) continue;
    const int64_t b = slot / block_size;
    const int64_t o = slot - b * block_size;
    if (b >= num_blocks) continue;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t row = (t * heads + h) * head_dim;
      for (int64_t d = 0; d < head_dim; d += kr) {
        const int64_t off =
            oracle_cache_offset(k_layout, k_stride, k_pack, b, o, h, d);
        memcpy(kc + off * es, k_in + (row + d) * es, (size_t)(kr * es));
      }
      for (int64_t d = 0; d < head_dim; d += vr) {
        const int64_t off =
            oracle_cache_offset(v_layout, v_stride, v_pack, b, o, h, d);
        memcpy(vc + off * es, v_in + (row + d) * es, (size_t)(vr * es));
      }
    }
  }
  return threads_used();
}

int oracle_gather_kv_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                          int v_layout, const int64_t *v_stride, int64_t v_pack,
                          const void *key_cache, const void *value_cache,
                          void *key_out, void *value_out,
                          const void *block_table, const void *seq_lens,
                          int index_is64, int32_t seq_count,
                          int32_t max_blocks_per_seq, int32_t max_seq_len,
                          int32_t heads, int32_t head_dim, int32_t block_size,
                          int32_t num_blocks, int es) {
  const int64_t kr = run_elems(k_layout, k_stride, k_pack, head_dim);
  const int64_t vr = run_elems(v_layout, v_stride, v_pack, head_dim);
  const int64_t nlb = ((int64_t)max_seq_len + block_size - 1) / block_size;
  const uint8_t *kc = key_cache, *vc = value_cache;
  uint8_t *ko_ = key_out, *vo_ = value_out;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t w = 0; w < (int64_t)seq_count * nlb; ++w) {
    const int64_t s = w / nlb, lb = w - s * nlb;
    if (lb >= max_blocks_per_seq) continue;
    const int64_t seq_len = load_index(seq_lens, s, index_is64);
    const int64_t n = seq_len < max_seq_len ? seq_len : max_seq_len;
    const int64_t t0 = lb * block_size;
    if (t0 >= n) continue;
    const int64_t bid =
        load_index(block_table, s * max_blocks_per_seq + lb, index_is64);
    if (bid < 0 || bid >= num_blocks) continue;
    const int64_t t1 = t0 + block_size < n ? t0 + block_size : n;
    for (int64_t t = t0; t < t1; ++t) {
      const int64_t o = t - t0;
      for (int64_t h = 0; h < heads; ++h) {
        const int64_t row = ((s * max_seq_len + t) * heads + h) * head_dim;
        for (int64_t d = 0; d < head_dim; d += kr) {
          const int64_t off =
              oracle_cache_offset(k_layout, k_stride, k_pack, bid, o, h, d);
          memcpy(ko_ + (row + d) * es, kc + off * es, (size_t)(kr * es));
        }
        for (int64_t d = 0; d < head_dim; d += vr) {
          const int64_t off =
              oracle_cache_offset(v_layout, v_stride, v_pack, bid, o, h, d);
          memcpy(vo_ + (row + d) * es, vc + off * es, (size_t)(vr * es));
        }
      }
    }
  }
  return threads_used();
}

/* ------------------------------------------------------------------------ */
/* Fast FP8 variants (the timed CPU baseline of FP8 caches).                  */
/*                                                                            */
/* Quantize: every rounding boundary of E4M3 and E5M2 (the midpoint of two    */
/* adjacent codes, and the saturation threshold) has at most 4 significant   */
/* bits, so it is a bf16 value.  An f32 whose upper 16 bits are u therefore   */
/* lies in [bf16(u), next bf16) with no boundary strictly inside: its code is */
/* that of bf16(u) itself when its lower 16 bits are 0 (ties included), and   */
/* that of any value just above bf16(u) otherwise.  Two 65536-entry tables    */
/* per format, filled once with the element-wise casts, give every f32's      */
/* code; the quotient x / scale is one IEEE f32 division as in quant_one.     */
/* Dequantize: with a per-tensor scale the output depends on the code alone,  */
/* so each call fills a 256-entry table of io values with dequant_one and     */
/* maps every code through it.                                                */

static uint8_t fq_lo[2][65536], fq_hi[2][65536];
static int ftables_ready;

static void fast_tables(void) {
  if (ftables_ready) return;
  for (int f = 0; f < 2; ++f) {
    for (uint32_t u = 0; u < 65536; ++u) {
      const float lo = float_of(u << 16), hi = float_of((u << 16) | 1u);
      fq_lo[f][u] = f ? oracle_f32_to_e5m2(lo) : oracle_f32_to_e4m3(lo);
      fq_hi[f][u] = f ? oracle_f32_to_e5m2(hi) : oracle_f32_to_e4m3(hi);
    }
  }
  ftables_ready = 1;
}

static inline uint8_t fast_to_fp8(float q, int e5) {
  const uint32_t u = bits_of(q);
  return (u & 0xFFFFu) ? fq_hi[e5][u >> 16] : fq_lo[e5][u >> 16];
}

static inline float fast_load_io(const uint8_t *p, int dt) {
  if (dt == D_BF16) {
    uint16_t h;
    memcpy(&h, p, 2);
    return float_of((uint32_t)h << 16);
  }
  return load_io_f32(p, dt);
}

/* The io value of every code for one per-tensor scale. */
typedef struct {
  uint8_t v[256][4];
} dq_table_t;

static void dq_table(dq_table_t *t, int fp8_dtype, float scale, int io_dtype) {
  for (int q = 0; q < 256; ++q) dequant_one((uint8_t)q, fp8_dtype, scale, io_dtype, t->v[q]);
}

/* n codes -> n io elements of `is` bytes. */
static void dequant_run(const uint8_t *src, uint8_t *dst, int64_t n, const dq_table_t *t,
                        int is) {
  if (is == 2) {
    for (int64_t j = 0; j < n; ++j) memcpy(dst + 2 * j, t->v[src[j]], 2);
  } else {
    for (int64_t j = 0; j < n; ++j) memcpy(dst + 4 * j, t->v[src[j]], 4);
  }
}

void oracle_quantize_fp8_fast(const void *in, int io_dtype, int64_t n, float scale,
                              int fp8_dtype, uint8_t *out) {
  fast_tables();
  const int es = dtype_size(io_dtype), e5 = fp8_dtype == D_E5M2;
  for (int64_t i = 0; i < n; ++i)
    out[i] = fast_to_fp8(fast_load_io((const uint8_t *)in + i * es, io_dtype) / scale, e5);
}

void oracle_dequantize_fp8_fast(const uint8_t *in, int64_t n, float scale, int fp8_dtype,
                                int io_dtype, void *out) {
  dq_table_t t;
  dq_table(&t, fp8_dtype, scale, io_dtype);
  dequant_run(in, out, n, &t, dtype_size(io_dtype));
}

int oracle_write_kv_quant_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                               int v_layout, const int64_t *v_stride, int64_t v_pack,
                               const void *key, const void *value, void *key_cache,
                               void *value_cache, const void *slots, int slot_is64,
                               int64_t num_tokens, int32_t heads, int32_t head_dim,
                               int32_t block_size, int32_t num_blocks, int io_dtype,
                               int cache_dtype, float k_scale, float v_scale) {
  fast_tables();
  const int64_t kr = run_elems(k_layout, k_stride, k_pack, head_dim);
  const int64_t vr = run_elems(v_layout, v_stride, v_pack, head_dim);
  const int is = dtype_size(io_dtype), e5 = cache_dtype == D_E5M2;
  const uint8_t *k_in = key, *v_in = value;
  uint8_t *kc = key_cache, *vc = value_cache;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = load_index(slots, t, slot_is64);
    if (slot < 0) continue;
    const int64_t b = slot / block_size;
    const int64_t o = slot - b * block_size;
    if (b >= num_blocks) continue;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t row = (t * heads + h) * head_dim;
      for (int64_t d = 0; d < head_dim; d += kr) {
        uint8_t *dst = kc + oracle_cache_offset(k_layout, k_stride, k_pack, b, o, h, d);
        for (int64_t j = 0; j < kr; ++j)
          dst[j] = fast_to_fp8(fast_load_io(k_in + (row + d + j) * is, io_dtype) / k_scale, e5);
      }
      for (int64_t d = 0; d < head_dim; d += vr) {
        uint8_t *dst = vc + oracle_cache_offset(v_layout, v_stride, v_pack, b, o, h, d);
        for (int64_t j = 0; j < vr; ++j)
          dst[j] = fast_to_fp8(fast_load_io(v_in + (row + d + j) * is, io_dtype) / v_scale, e5);
      }
    }
  }
  return threads_used();
}

int oracle_gather_kv_dequant_fast(int k_layout, const int64_t *k_stride, int64_t k_pack,
                                  int v_layout, const int64_t *v_stride, int64_t v_pack,
                                  const void *key_cache, const void *value_cache,
                                  void *key_out, void *value_out,
                                  const void *block_table, const void *seq_lens,
                                  int index_is64, int32_t seq_count,
                                  int32_t max_blocks_per_seq, int32_t max_seq_len,
                                  int32_t heads, int32_t head_dim, int32_t block_size,
                                  int32_t num_blocks, int cache_dtype, int io_dtype,
                                  float k_scale, float v_scale) {
  const int64_t kr = run_elems(k_layout, k_stride, k_pack, head_dim);
  const int64_t vr = run_elems(v_layout, v_stride, v_pack, head_dim);
  const int64_t nlb = ((int64_t)max_seq_len + block_size - 1) / block_size;
  const int is = dtype_size(io_dtype);
  dq_table_t kt, vt;
  dq_table(&kt, cache_dtype, k_scale, io_dtype);
  dq_table(&vt, cache_dtype, v_scale, io_dtype);
  const uint8_t *kc = key_cache, *vc = value_cache;
  uint8_t *ko_ = key_out, *vo_ = value_out;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t w = 0; w < (int64_t)seq_count * nlb; ++w) {
    const int64_t s = w / nlb, lb = w - s * nlb;
    if (lb >= max_blocks_per_seq) continue;
    const int64_t seq_len = load_index(seq_lens, s, index_is64);
    const int64_t n = seq_len < max_seq_len ? seq_len : max_seq_len;
    const int64_t t0 = lb * block_size;
    if (t0 >= n) continue;
    const int64_t bid = load_index(block_table, s * max_blocks_per_seq + lb, index_is64);
    if (bid < 0 || bid >= num_blocks) continue;
    const int64_t t1 = t0 + block_size < n ? t0 + block_size : n;
    for (int64_t t = t0; t < t1; ++t) {
      const int64_t o = t - t0;
      for (int64_t h = 0; h < heads; ++h) {
        const int64_t row = ((s * max_seq_len + t) * heads + h) * head_dim;
        for (int64_t d = 0; d < head_dim; d += kr)
          dequant_run(kc + oracle_cache_offset(k_layout, k_stride, k_pack, bid, o, h, d),
                      ko_ + (row + d) * is, kr, &kt, is);
        for (int64_t d = 0; d < head_dim; d += vr)
          dequant_run(vc + oracle_cache_offset(v_layout, v_stride, v_pack, bid, o, h, d),
                      vo_ + (row + d) * is, vr, &vt, is);
      }
    }
  }
  return threads_used();
}
