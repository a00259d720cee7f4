// Paged KV write (scatter) and gather kernels for gfx950 (CDNA4, wave64),
// and the templates that launch them.
//
// Data movement only, plus optional FP8 (E4M3 / E5M2) casts.  The unit of
// work is a *chunk*: G consecutive elements of one contiguous cache piece (a
// head row for NHD/HND, an x-element pack for HND_PACKED), moved with one
// 1..16-byte load and one store per lane.  The host picks the widest chunk
// that every pointer and stride allows, so NHD/HND bf16 rows move as 16-byte
// global_load_dwordx4 / global_store_dwordx4 and a wave covers 1 KiB of a row
// per instruction.  Blocks stored in another dense order (x-packed, HND,
// token axis innermost) are transposed through LDS by the tile kernels, so
// that both HBM sides stay 16-byte coalesced whatever the layout.
//
// Semantics follow the reference kernels:
//   write  kernels/kvx_paged_kv.cu:93-124 (slot < 0 and block >= num_blocks
//          are skipped; bit copy of every (token, head, dim) element);
//   gather kernels/kvx_paged_kv.cu:226-267 (rows t >= seq_len, logical
//          blocks >= max_blocks_per_seq and block ids < 0 are untouched);
//          block ids >= num_blocks are also skipped here instead of being
//          read out of bounds.
//
// Every kernel is a template.  The kernels_*.hip translation units each
// instantiate one family (through the run_* entry points declared at the
// end), so that the families compile in parallel; dispatch.hip plans a
// launch on the host and calls them.
#pragma once

#include <hip/hip_runtime.h>

#include "fp_convert.h"
#include "kvx_internal.h"

namespace kvx {
namespace dev {
constexpr int kWave = 64;
constexpr int kBlockThreads = 256;
constexpr int kWavesPerBlock = kBlockThreads / kWave;
// Chunk offsets each lane keeps in registers; rows with more chunks per lane
// compute the rest on the fly.
constexpr int kMaxChunksPerLane = 4;
// LDS tile kernels (gather_tiles_kernel, write_tiles_kernel): 16-byte chunks
// per thread in flight, and LDS row padding in bytes.
constexpr int kTileLoads = 4;
constexpr int kTilePad = 16;
// run_log2 of a per-token run that is a multiple of 16 bytes but not a power
// of two (HND heads of 96 or 80 bf16 elements): its length is in run_bytes.
constexpr int32_t kRunOdd = 30;

// x / d for a divisor d >= 2 whose magic m = ceil(2^32 / d): with
// m = 2^32 / d + f (0 <= f < 1), x * m / 2^32 = x / d + x * f / 2^32 and
// the error x * f / 2^32 < 1 / d whenever x * d <= 2^32, so the floor is
// exact there.  The planners only pass (x, d) pairs that satisfy it.
__device__ __forceinline__ uint32_t div_magic(uint32_t x, uint32_t m) { return __umulhi(x, m); }
// Tuning constants: each value is the measured best on MI355X, and its
// comment gives the same-box A/B behind it.
//
// Chunks per lane in flight in the contiguous-block gathers, for the copy
// and for the FP8 dequantizing gather.  A lane moves one K and one V chunk;
// loading both before storing either made the bf16 copy (c2) 7% slower and
// the dequantizing gather (c4) 2% faster (256-thread, 4 KiB tiles).
constexpr int kFlatUnroll = 1;
constexpr int kFlatUnrollDequant = 2;
// Non-temporal (streaming) cache loads and output stores in every gather:
// together 4-13% faster than either alone.
constexpr bool kGatherNtLoad = true;
constexpr bool kGatherNtStore = true;
// Contiguous-block gather (gather_flat_kernel): threads per workgroup (also
// those of the row-dense write, write_flat_kernel) and cache bytes per
// tensor per workgroup.  A block's valid chunks are split into a
// power-of-two number of equal ranges of at most kFlatTileBytes, so that
// each lane copies one 16-byte chunk of K and one of V (2 KiB for
// power-of-two rows).  On MI355X (c2, same box) 128 threads and 2 KiB
// measured 3.7% faster than 256 threads and 4 KiB, 64 threads and 1 KiB 1%
// slower (2% faster on c5's 64 KiB blocks); tiles that leave a lane one
// chunk, or give it more than two, were 5-40% slower.  The 3 KiB bound
// changes only rows whose chunk count is not a power of two: head_dim 96 or
// 80 (8 heads, bf16) then splits into 192- or 160-chunk ranges instead of
// 96 or 80, 0.670 -> 0.697 and 0.657 -> 0.693 of peak at c2's table.
constexpr int kFlatThreads = 128;
constexpr int64_t kFlatTileBytes = 3072;
// Output rows per workgroup of the RAGGED / KV_OFFSETS gathers: about
// kGatherTileBytes cache bytes of each tensor, in 256-thread workgroups.
// The RAGGED copy of row-dense caches whose rows are not contiguous in the
// block (gather_indexed_flat_kernel without a dequant) uses
// kRaggedCopyThreads threads and kRaggedCopyTileBytes instead: on MI355X
// (c2, same box) 64 threads and 2 KiB measured 7% faster than 256 threads
// and 4 KiB, 128 threads and 2 KiB 5%; the same change made KV_OFFSETS
// copies 1-2% and that kernel's dequantizing gather 2-8% slower.
constexpr int64_t kGatherTileBytes = 4096;
constexpr int kRaggedCopyThreads = 64;
constexpr int64_t kRaggedCopyTileBytes = 2048;
// RAGGED gathers of row-contiguous caches (canonical NHD blocks) take
// gather_ragged_tile_kernel, for copies and for dequantizing gathers.
// Against gather_indexed_flat_kernel on MI355X (same-box A/B, medians of 6
// alternating rounds) it took c4's FP8 dequantizing gather from 690 to
// 629 us and c5's copy from 2336 to 2241 us; c2's copy measured 1587
// against 1571 us.
// Chunks per thread the RAGGED / KV_OFFSETS flat gather resolves and loads
// together (the table load and the data load of each are dependent).
constexpr int kIndexedUnroll = 4;
// KV_OFFSETS row-dense gather: the dequantizing gather loads its table
// entries once per workgroup tile (per-chunk loads cost it, with 8-byte
// source chunks and twice the table loads per byte, 15%).  The copy gather
// takes per-tile entries for rows of at most kOffsetsTileCopyRow cache
// bytes and for rows whose chunk count is not a power of two, per-chunk
// entries otherwise: on MI355X (c2's table, bf16) one KV head (256-byte
// rows) measured 200.8 against 211.7 us and two heads 413.9 against
// 423.0 us per tile, 576-element MLA rows 1050 us against 1185 us per chunk
// (1142 us in gather_indexed_kernel) and 6 x 128 rows 1290 against 1392 us,
// while c2's 2 KiB rows measured 1614.7 per tile against 1526.5 us per
// chunk.
constexpr int64_t kOffsetsTileCopyRow = 512;
// FP8 cache bytes per chunk of the dequantizing gathers: 16-byte chunks
// measured 3% faster for the RAGGED kernels that load a block id per chunk
// (gather_indexed_flat_kernel; half the id loads) and 20-40% slower for
// every other gather, gather_ragged_tile_kernel included (8 bytes).
constexpr int kDequantChunk = 8;
constexpr int kRaggedDequantChunk = 16;
// Non-temporal io-row loads of the tiled block write (off) and of the
// per-token write (on), and non-temporal cache stores of every write
// kernel (on).  On MI355X (c3 shapes) non-temporal stores make the tiled
// write 2-9% faster and the per-token prefill write 14% faster (decode
// writes are unchanged); non-temporal loads make the tiled write 10-20%
// slower and the per-token prefill write 2-5% faster.
constexpr bool kWriteNtLoad = false;
constexpr bool kTokenWriteNtLoad = true;
constexpr bool kWriteNtStore = true;
// Row-dense writes take write_flat_kernel.  When a row has at least 64
// chunks, every lane of a wave belongs to one token and the slot is one
// scalar load per wave instead of one vector load per lane.  Kernel traces
// on MI355X: c4's quantizing write 5.11 against 5.45 us, c2's and c5's
// writes unchanged (3.90 / 3.87 and 4.75 / 4.77 us).  Forcing the row loads
// of write_flat_kernel and write_kernel ahead of the slot test with an
// empty asm measured no gain (c2 3.90 against 3.88 us, c4 5.11 against
// 4.86 us, c5 4.75 against 4.82 us): the compiler's order is kept.

// Cache geometry with strides pre-multiplied by the cache element size.
struct GeomBytes {
  int64_t s_block;
  int64_t s_off;
  int64_t s_head;
  int64_t s_piece;
  int64_t s_inner;
  int32_t pack;
  int32_t pad_;
};

// ---------------------------------------------------------------------------
// Raw storage of one chunk.

// A chunk lives in 32-bit registers: B bytes in B/4 words (B < 4: the low
// bits of one word).  Elements are read and written with shifts, never
// through byte arrays, so a 16-byte chunk stays four VGPRs.
template <int B>
struct Raw {
  static constexpr int kWords = B >= 4 ? B / 4 : 1;
  uint32_t w[kWords];
};

// Load/store one chunk with the widest naturally aligned access: B = 16 is
// one global_load_dwordx4 / global_store_dwordx4 per lane.  NT selects the
// non-temporal (streaming) form.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename V, bool NT>
__device__ __forceinline__ V ld_one(const char *p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const V *>(p));
  return *reinterpret_cast<const V *>(p);
}

template <typename V, bool NT>
__device__ __forceinline__ void st_one(char *p, V v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v, reinterpret_cast<V *>(p));
  } else {
    *reinterpret_cast<V *>(p) = v;
  }
}

template <int B, bool NT = false>
__device__ __forceinline__ Raw<B> ld(const char *p) {
  Raw<B> r;
  if constexpr (B == 1) {
    r.w[0] = ld_one<uint8_t, NT>(p);
  } else if constexpr (B == 2) {
    r.w[0] = ld_one<uint16_t, NT>(p);
  } else if constexpr (B == 4) {
    r.w[0] = ld_one<uint32_t, NT>(p);
  } else if constexpr (B == 8) {
    const u32x2 v = ld_one<u32x2, NT>(p);
    r.w[0] = v[0];
    r.w[1] = v[1];
  } else {
    static_assert(B % 16 == 0, "chunk bytes");
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      const u32x4 v = ld_one<u32x4, NT>(p + 16 * i);
      r.w[4 * i + 0] = v[0];
      r.w[4 * i + 1] = v[1];
      r.w[4 * i + 2] = v[2];
      r.w[4 * i + 3] = v[3];
    }
  }
  return r;
}

template <int B, bool NT = false>
__device__ __forceinline__ void st(char *p, const Raw<B> &r) {
  if constexpr (B == 1) {
    st_one<uint8_t, NT>(p, (uint8_t)r.w[0]);
  } else if constexpr (B == 2) {
    st_one<uint16_t, NT>(p, (uint16_t)r.w[0]);
  } else if constexpr (B == 4) {
    st_one<uint32_t, NT>(p, r.w[0]);
  } else if constexpr (B == 8) {
    u32x2 v;
    v[0] = r.w[0];
    v[1] = r.w[1];
    st_one<u32x2, NT>(p, v);
  } else {
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      u32x4 v;
      v[0] = r.w[4 * i + 0];
      v[1] = r.w[4 * i + 1];
      v[2] = r.w[4 * i + 2];
      v[3] = r.w[4 * i + 3];
      st_one<u32x4, NT>(p + 16 * i, v);
    }
  }
}

// Element i of a chunk (i is a compile-time constant after unrolling).
template <int B>
__device__ __forceinline__ uint32_t get8(const Raw<B> &r, int i) {
  return (r.w[i >> 2] >> ((i & 3) * 8)) & 0xFFu;
}
template <int B>
__device__ __forceinline__ uint32_t get16(const Raw<B> &r, int i) {
  return (r.w[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu;
}
template <int B>
__device__ __forceinline__ void put8(Raw<B> &r, int i, uint32_t v) {
  r.w[i >> 2] |= v << ((i & 3) * 8);
}
template <int B>
__device__ __forceinline__ void put16(Raw<B> &r, int i, uint32_t v) {
  r.w[i >> 1] |= v << ((i & 1) * 16);
}

// ---------------------------------------------------------------------------
// Chunk operations.  kSrc/kDst are the bytes read/written per chunk.

template <int B>
struct CopyOp {
  static constexpr int kSrc = B;
  static constexpr int kDst = B;
  static constexpr bool kScaled = false;
  __device__ __forceinline__ static Raw<B> apply(const Raw<B> &x, float) {
    return x;
  }
};

template <int IO>
struct IoType;
template <>
struct IoType<KVX_DTYPE_F32> {
  static constexpr int kBytes = 4;
};
template <>
struct IoType<KVX_DTYPE_F16> {
  static constexpr int kBytes = 2;
};
template <>
struct IoType<KVX_DTYPE_BF16> {
  static constexpr int kBytes = 2;
};

template <int IO, int B>
__device__ __forceinline__ float io_to_f32(const Raw<B> &x, int i) {
  if constexpr (IO == KVX_DTYPE_F32) {
    return bits_f32(x.w[i]);
  } else if constexpr (IO == KVX_DTYPE_BF16) {
    return bf16_to_f32((uint16_t)get16(x, i));
  } else {
    return f16_to_f32((uint16_t)get16(x, i));
  }
}

template <int IO, int B>
__device__ __forceinline__ void f32_to_io(float v, Raw<B> &y, int i) {
  if constexpr (IO == KVX_DTYPE_F32) {
    y.w[i] = f32_bits(canon_nan_f32(v));
  } else if constexpr (IO == KVX_DTYPE_BF16) {
    put16(y, i, f32_to_bf16(v));
  } else {
    put16(y, i, f32_to_f16(v));
  }
}

// io (F16/BF16/F32) -> FP8 (F8 = KVX_DTYPE_F8_E4M3 or KVX_DTYPE_F8_E5M2):
// q = fp8(sat(x / scale)).
template <int G, int IO, int F8>
struct QuantOp {
  static constexpr int kSrc = G * IoType<IO>::kBytes;
  static constexpr int kDst = G;
  static constexpr bool kScaled = true;
  __device__ __forceinline__ static Raw<kDst> apply(const Raw<kSrc> &x,
                                                    float scale) {
    Raw<kDst> y;
#pragma unroll
    for (int k = 0; k < Raw<kDst>::kWords; ++k) y.w[k] = 0;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const float q = io_to_f32<IO>(x, i) / scale;
      put8(y, i, F8 == KVX_DTYPE_F8_E5M2 ? f32_to_e5m2(q) : f32_to_e4m3(q));
    }
    return y;
  }
};

// FP8 -> io (F16/BF16/F32): y = io(f32(q) * scale); any NaN result is the
// canonical quiet NaN of the io type.  gfx950 decodes two OCP E4M3 codes
// exactly with v_cvt_pk_f32_fp8 (E5M2: v_cvt_pk_f32_bf8), multiplies in f32,
// and narrows two values with round-to-nearest-even (v_cvt_pk_bf16_f32 /
// v_cvt_f16_f32); the result equals fp_convert.h's e4m3_to_f32 /
// e5m2_to_f32 / f32_to_bf16 / f32_to_f16, which the GPU tests check for
// every code.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t canon_nan16(uint32_t h, uint32_t inf, uint32_t qnan) {
  return ((h & 0x7FFFu) > inf) ? qnan : h;
}

template <int IO>
__device__ __forceinline__ uint32_t pack_pair(f32x2 f) {
  if constexpr (IO == KVX_DTYPE_BF16) {
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
    return canon_nan16(u & 0xFFFFu, 0x7F80u, 0x7FC0u) |
           (canon_nan16(u >> 16, 0x7F80u, 0x7FC0u) << 16);
  } else {
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
    return canon_nan16(u & 0xFFFFu, 0x7C00u, 0x7E00u) |
           (canon_nan16(u >> 16, 0x7C00u, 0x7E00u) << 16);
  }
}

template <bool kE5M2>
__device__ __forceinline__ f32x2 decode_pair(int word, bool hi) {
  if constexpr (kE5M2) {
    return hi ? __builtin_amdgcn_cvt_pk_f32_bf8(word, true)
              : __builtin_amdgcn_cvt_pk_f32_bf8(word, false);
  } else {
    return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(word, true)
              : __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
  }
}

template <int G, int IO, int F8>
struct DequantOp {
  static constexpr int kSrc = G;
  static constexpr int kDst = G * IoType<IO>::kBytes;
  static constexpr bool kScaled = true;
  __device__ __forceinline__ static Raw<kDst> apply(const Raw<kSrc> &x, float scale) {
    Raw<kDst> y;
#pragma unroll
    for (int k = 0; k < Raw<kDst>::kWords; ++k) y.w[k] = 0;
#pragma unroll
    for (int p = 0; p < (G + 1) / 2; ++p) {
      // codes 2p, 2p+1 sit in halfword (p & 1) of word p / 2
      const int word = (int)x.w[p >> 1];
      const f32x2 f = decode_pair<F8 == KVX_DTYPE_F8_E5M2>(word, (p & 1) != 0) * scale;
      if constexpr (IO == KVX_DTYPE_F32) {
        y.w[2 * p] = f32_bits(canon_nan_f32(f[0]));
        if (2 * p + 1 < G) y.w[2 * p + 1] = f32_bits(canon_nan_f32(f[1]));
      } else if constexpr (G == 1) {
        y.w[0] = pack_pair<IO>(f) & 0xFFFFu;
      } else {
        y.w[p] = pack_pair<IO>(f);
      }
    }
    return y;
  }
};

// ---------------------------------------------------------------------------
// Index helpers.

__device__ __forceinline__ int64_t load_index(const void *base, int64_t i,
                                              int32_t is64) {
  return is64 ? reinterpret_cast<const int64_t *>(base)[i]
              : (int64_t)reinterpret_cast<const int32_t *>(base)[i];
}

// Value i of an int32 (I64 = false) or int64 index array.  Gather kernels
// take the dtype as a template parameter: with a runtime dtype every load
// sits behind its own branch and the loads complete one after another; with
// a fixed one, independent loads (seq_len, block id, indptr) are issued
// together.
template <bool I64>
__device__ __forceinline__ int64_t load_idx(const void *base, int64_t i) {
  if constexpr (I64) return reinterpret_cast<const int64_t *>(base)[i];
  return (int64_t)reinterpret_cast<const int32_t *>(base)[i];
}

// Scale of (block b, head h): the workgroup's per-tensor value, or the
// indexed entry.
// Scale of row element e (of a row of heads of head_dim elements) in block
// b.  The head's division is done only for indexed scales: an integer
// division by a run-time value is a long instruction sequence on the GPU.
__device__ __forceinline__ float scale_at(const ScaleRef &r, float uniform, int64_t b,
                                          uint32_t e, uint32_t head_dim) {
  if (!r.indexed) return uniform;
  return r.p[b * r.s_block + (int64_t)(e / head_dim) * r.s_head];
}

// The same for element e of a run of whole rows of row_elems elements.
__device__ __forceinline__ float scale_in_rows(const ScaleRef &r, float uniform, int64_t b,
                                               uint32_t e, uint32_t row_elems,
                                               uint32_t head_dim) {
  if (!r.indexed) return uniform;
  return r.p[b * r.s_block + (int64_t)((e % row_elems) / head_dim) * r.s_head];
}

__device__ __forceinline__ float scale_of(const ScaleRef &r, float uniform, int64_t b,
                                          uint32_t h) {
  return r.indexed ? r.p[b * r.s_block + (int64_t)h * r.s_head] : uniform;
}

// Byte offset, relative to the (block, offset) base, of the chunk that
// starts at row element e.  h = e / D and the pack split are 32-bit because
// a row holds H * D < 2^31 elements.
__device__ __forceinline__ int64_t chunk_off(const GeomBytes &g, uint32_t e,
                                             uint32_t head_dim) {
  const uint32_t h = e / head_dim;
  const uint32_t d = e - h * head_dim;
  const uint32_t pc = d / (uint32_t)g.pack;
  const uint32_t w = d - pc * (uint32_t)g.pack;
  return (int64_t)h * g.s_head + (int64_t)pc * g.s_piece +
         (int64_t)w * g.s_inner;
}

// slot -> (block, offset); slot >= 0.  32-bit division in the common case.
__device__ __forceinline__ void split_slot(int64_t slot, int32_t bs,
                                           int64_t &b, int64_t &o) {
  if ((uint64_t)slot <= 0xFFFFFFFFull) {
    const uint32_t q = (uint32_t)slot / (uint32_t)bs;
    b = q;
    o = (int64_t)((uint32_t)slot - q * (uint32_t)bs);
  } else {
    b = slot / bs;
    o = slot - b * bs;
  }
}

// ---------------------------------------------------------------------------
// Write (scatter).
//
// Each wave takes `tpw` tokens at a time, `lpt` = 64 / tpw lanes per token
// (tpw > 1 only for rows shorter than 64 chunks).  The token's slot is loaded
// once by one lane and broadcast to the token's lanes; every lane keeps the
// cache offsets of its chunks in registers for the whole grid-stride loop.

struct WriteArgs {
  const char *src_k;
  const char *src_v;
  char *dst_k;
  char *dst_v;
  const void *slots;
  ScaleRef ksc;  // quantizing ops only
  ScaleRef vsc;
  GeomBytes gk;
  GeomBytes gv;
  int64_t num_tokens;
  int64_t num_groups;  // ceil(num_tokens / tpw)
  int32_t slot_is64;
  int32_t block_size;
  int32_t num_blocks;
  int32_t head_dim;
  int32_t nchunks;      // chunks per token row
  int32_t chunk_elems;  // G
  int32_t row_bytes;    // bytes of one io row
  int32_t lpt_log2;
  int32_t nchunks_log2;  // write_flat_kernel: log2(nchunks), or -1
  uint32_t nchunks_magic;  // nchunks_log2 < 0: div_magic's m for nchunks
};

template <class Op>
__global__ __launch_bounds__(kBlockThreads) void write_kernel(WriteArgs a) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int64_t wave =
      (int64_t)blockIdx.x * kWavesPerBlock +
      __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  const int lpt = 1 << a.lpt_log2;
  const int tpw = kWave >> a.lpt_log2;
  const int sub = lane >> a.lpt_log2;
  const int l = lane & (lpt - 1);

  int64_t koff[kMaxChunksPerLane];
  int64_t voff[kMaxChunksPerLane];
  uint32_t hk[kMaxChunksPerLane];  // head of each chunk (indexed scales)
#pragma unroll
  for (int k = 0; k < kMaxChunksPerLane; ++k) {
    const int c = l + k * lpt;
    koff[k] = 0;
    voff[k] = 0;
    hk[k] = 0;
    if (c < a.nchunks) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      koff[k] = chunk_off(a.gk, e, (uint32_t)a.head_dim);
      voff[k] = chunk_off(a.gv, e, (uint32_t)a.head_dim);
      if constexpr (Op::kScaled) hk[k] = e / (uint32_t)a.head_dim;
    }
  }
  float ks = 1.0f;
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }

  for (int64_t g = wave; g < a.num_groups; g += nwaves) {
    const int64_t t = g * tpw + sub;
    int64_t mine = -1;
    const int64_t tl = g * tpw + lane;
    if (lane < tpw && tl < a.num_tokens) mine = load_index(a.slots, tl, a.slot_is64);
    // The token rows do not depend on the slot: issue their loads before
    // waiting for it, so the slot and row latencies overlap.
    const char *sk = a.src_k + t * a.row_bytes;
    const char *sv = a.src_v + t * a.row_bytes;
    Raw<Op::kSrc> xk[kMaxChunksPerLane];
    Raw<Op::kSrc> xv[kMaxChunksPerLane];
    if (t < a.num_tokens) {
#pragma unroll
      for (int k = 0; k < kMaxChunksPerLane; ++k) {
        const int c = l + k * lpt;
        if (c < a.nchunks) {
          xk[k] = ld<Op::kSrc, kTokenWriteNtLoad>(sk + (int64_t)c * Op::kSrc);
          xv[k] = ld<Op::kSrc, kTokenWriteNtLoad>(sv + (int64_t)c * Op::kSrc);
        }
      }
    }
    int64_t slot;
    if (tpw == 1) {
      slot = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(
                            (int)(mine >> 32))
                        << 32) |
                       (uint32_t)__builtin_amdgcn_readfirstlane((int)mine));
    } else {
      const int hi = __shfl((int)(mine >> 32), sub);
      const int lo = __shfl((int)mine, sub);
      slot = (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
    }
    if (t >= a.num_tokens || slot < 0) continue;
    int64_t b, o;
    split_slot(slot, a.block_size, b, o);
    if (b >= a.num_blocks) continue;
    char *dk = a.dst_k + b * a.gk.s_block + o * a.gk.s_off;
    char *dv = a.dst_v + b * a.gv.s_block + o * a.gv.s_off;
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
      const int c = l + k * lpt;
      if (c < a.nchunks) {
        st<Op::kDst, kWriteNtStore>(dk + koff[k], Op::apply(xk[k], scale_of(a.ksc, ks, b, hk[k])));
        st<Op::kDst, kWriteNtStore>(dv + voff[k], Op::apply(xv[k], scale_of(a.vsc, vs, b, hk[k])));
      }
    }
    for (int c = l + kMaxChunksPerLane * lpt; c < a.nchunks; c += lpt) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      const uint32_t h = e / (uint32_t)a.head_dim;
      const Raw<Op::kSrc> yk = ld<Op::kSrc, kTokenWriteNtLoad>(sk + (int64_t)c * Op::kSrc);
      const Raw<Op::kSrc> yv = ld<Op::kSrc, kTokenWriteNtLoad>(sv + (int64_t)c * Op::kSrc);
      st<Op::kDst, kWriteNtStore>(dk + chunk_off(a.gk, e, (uint32_t)a.head_dim),
                                  Op::apply(yk, scale_of(a.ksc, ks, b, h)));
      st<Op::kDst, kWriteNtStore>(dv + chunk_off(a.gv, e, (uint32_t)a.head_dim),
                                  Op::apply(yv, scale_of(a.vsc, vs, b, h)));
    }
  }
}

// Row-dense caches (a token's H * D elements are consecutive in its block
// row, for K and V): the write is a flat list of (token, chunk) pairs, and
// each lane of a kFlatThreads-thread workgroup copies one 16-byte chunk of
// K and one of V.  The chunks' loads are issued first and kept ahead of the
// slot test, so the slot and the row data are in flight together.  S64:
// int64 slots (else int32).  UNIFORM: rows of 64 or more chunks, so that a
// wave holds chunks of one token only; the slot is then one scalar load per
// wave (the token index made wave-uniform with readfirstlane) instead of one
// vector load per lane.  This is the contiguous gather's shape
// (gather_flat_kernel) from the other side.
template <class Op, bool S64, bool UNIFORM>
__global__ __launch_bounds__(kFlatThreads) void write_flat_kernel(WriteArgs a) {
  const int64_t f = (int64_t)blockIdx.x * kFlatThreads + threadIdx.x;
  // token and chunk of f: shifts, or (chunk counts that are not a power of
  // two, e.g. 576-element MLA rows) a multiply-high, which the launch keeps
  // exact (f < 2^32 and f * nchunks <= 2^32)
  const int64_t t = a.nchunks_log2 >= 0 ? f >> a.nchunks_log2
                                        : (int64_t)div_magic((uint32_t)f, a.nchunks_magic);
  if (t >= a.num_tokens) return;
  const int32_t c = (int32_t)(f - t * a.nchunks);
  const Raw<Op::kSrc> xk = ld<Op::kSrc, kTokenWriteNtLoad>(a.src_k + t * a.row_bytes +
                                                           (int64_t)c * Op::kSrc);
  const Raw<Op::kSrc> xv = ld<Op::kSrc, kTokenWriteNtLoad>(a.src_v + t * a.row_bytes +
                                                           (int64_t)c * Op::kSrc);
  int64_t slot;
  if constexpr (UNIFORM) {
    // f < 2^32 (the grid is bounded by HIP's limits), so t < 2^26
    const int64_t tw = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)t);
    slot = load_idx<S64>(a.slots, tw);
  } else {
    slot = load_idx<S64>(a.slots, t);
  }
  float ks = 1.0f;
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }
  if (slot < 0) return;
  int64_t b, o;
  split_slot(slot, a.block_size, b, o);
  if (b >= a.num_blocks) return;
  const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
  st<Op::kDst, kWriteNtStore>(a.dst_k + b * a.gk.s_block + o * a.gk.s_off + (int64_t)c * Op::kDst,
                              Op::apply(xk, scale_at(a.ksc, ks, b, e, (uint32_t)a.head_dim)));
  st<Op::kDst, kWriteNtStore>(a.dst_v + b * a.gv.s_block + o * a.gv.s_off + (int64_t)c * Op::kDst,
                              Op::apply(xv, scale_at(a.vsc, vs, b, e, (uint32_t)a.head_dim)));
}

// ---------------------------------------------------------------------------
// Block write (prefill into a layout that is not row-major in the block).
//
// When the `bs` consecutive tokens of a group fill one cache block in order
// (slot = b * bs + o for o = 0..bs-1, the usual prefill pattern), the
// group's source rows are one contiguous io region and each cache tensor's
// destination is one contiguous block region, only permuted.
// write_tiles_kernel moves such groups through LDS so that both the io
// reads and the cache writes are coalesced 16-byte accesses; groups that do
// not fill a block take the per-token path.

// A run of a group: tokens [t0 + tok, t0 + tok + hi - lo) hold the slots
// block * bs + lo .. block * bs + hi - 1, in order.
struct GroupRun {
  int64_t block;
  int32_t lo;
  int32_t hi;
  int32_t tok;
  int32_t pad_;
};

// Runs a group's tokens may form and still be written through LDS: a prefill
// chunk of bs consecutive positions covers the end of one block and the
// start of the next.
constexpr int kMaxRuns = 2;

// Wave 0 splits tokens [t0, t0 + bs) into runs of consecutive offsets of one
// block and writes them to runs[] (LDS); *nruns = their count, or 0 when a
// token's slot is < 0 or past the blocks or there are more than kMaxRuns
// runs (the group is then written token by token).  Read after the caller's
// __syncthreads().
__device__ __forceinline__ void group_runs(const WriteArgs &a, int64_t t0, int bs_log2,
                                           GroupRun *runs, int32_t *nruns) {
  const int tid = (int)threadIdx.x;
  if (tid >= kWave) return;
  const int lane = tid;
  const int64_t left = a.num_tokens - t0;
  const int n = left < (1 << bs_log2) ? (int)left : (1 << bs_log2);
  int64_t slot = -1;
  if (lane < n) slot = load_index(a.slots, t0 + lane, a.slot_is64);
  const int64_t blk = slot >> bs_log2;
  const int32_t off = (int32_t)(slot & ((1 << bs_log2) - 1));
  const bool ok = lane >= n || (slot >= 0 && blk < a.num_blocks);
  const int64_t prev = (int64_t)(((uint64_t)(uint32_t)__shfl_up((int)(slot >> 32), 1) << 32) |
                                 (uint32_t)__shfl_up((int)slot, 1));
  const bool start = lane < n && (lane == 0 || off == 0 || slot != prev + 1);
  const uint64_t bad = __ballot(!ok);
  const uint64_t starts = __ballot(start);
  const int count = __popcll(starts);
  const bool take = bad == 0 && count <= kMaxRuns;
  if (lane == 0) *nruns = take ? count : 0;
  if (take && start) {
    const uint64_t later = lane == kWave - 1 ? 0ull : starts & (~0ull << (lane + 1));
    const int end = later ? __ffsll((long long)later) - 1 : n;
    GroupRun r;
    r.block = blk;
    r.lo = off;
    r.hi = off + (end - lane);
    r.tok = lane;
    r.pad_ = 0;
    runs[__popcll(starts & ((1ull << lane) - 1ull))] = r;
  }
}

// Run ownership for block sizes up to 32 (2 * bs slots fit one wave), for
// tensors whose blocks are not row-major.  A run here is a maximal stretch
// of tokens whose slots are valid, lie in one block and follow each other
// (slot = previous slot + 1).  The workgroups of group [t0, t0 + bs) own
// the runs that START in it; such a run ends before t0 + 2 * bs - 1, since
// it holds at most bs tokens.  Every token then has exactly one owner, and
// a prefill chunk that starts inside a block has each of its blocks written
// whole by one workgroup instead of split between two, whose writes would
// share cache lines (or 16-byte chunks, stored piece by piece).  On MI355X
// (c3's size, x-packed K, chunks starting k = 1, 11 or 15 tokens into a
// block) splitting the x-packed blocks measured 79 us against 55-62 us for
// owned runs; only k = 8, whose halves are whole 128-byte lines, gained.
// A whole block in order (write_tile_block's case) is one run starting at
// t0 either way.
//
// Wave 0 loads the slots of tokens t0 - 1 .. t0 + 2 * bs - 2, one per lane,
// and writes the owned runs to runs[] (LDS); *nruns = their count, or 0
// when an owned token's slot is < 0 or past the blocks or there are more
// than kMaxRuns runs (the owned tokens are then written token by token).
// own[0], own[1]: the owned tokens, [t0 + own[0], t0 + own[1]).  Read after
// the caller's __syncthreads().
__device__ __forceinline__ void owned_runs(const WriteArgs &a, int64_t t0, int bs_log2,
                                           GroupRun *runs, int32_t *nruns, int32_t *own) {
  const int lane = (int)threadIdx.x;
  if (lane >= kWave) return;
  const int bs = 1 << bs_log2;
  const int64_t t = t0 - 1 + lane;  // lane 0: the token before the group
  const bool in = lane < 2 * bs && t >= 0 && t < a.num_tokens;
  int64_t slot = -1;
  if (in) slot = load_index(a.slots, t, a.slot_is64);
  const int64_t blk = slot >> bs_log2;
  const int32_t off = (int32_t)(slot & (bs - 1));
  const bool ok = in && slot >= 0 && blk < a.num_blocks;
  const int64_t prev = (int64_t)(((uint64_t)(uint32_t)__shfl_up((int)(slot >> 32), 1) << 32) |
                                 (uint32_t)__shfl_up((int)slot, 1));
  const uint64_t oks = __ballot(ok);
  const uint64_t ins = __ballot(in);
  const bool prev_ok = lane > 0 && ((oks >> (lane - 1)) & 1ull);
  // Lanes without a token count as starts: they bound the last run.
  const bool start = !in || !ok || !prev_ok || off == 0 || slot != prev + 1;
  const uint64_t starts = __ballot(start);
  const uint64_t group = ((1ull << bs) - 1ull) << 1;  // lanes of tokens t0 .. t0 + bs - 1
  const uint64_t mine = starts & group & ins;
  if (mine == 0) {
    // The group's tokens all continue a run that starts before t0.
    if (lane == 0) {
      *nruns = 0;
      own[0] = 0;
      own[1] = 0;
    }
    return;
  }
  const int first = __ffsll((long long)mine) - 1;
  const int last = 63 - __clzll((long long)mine);
  const uint64_t after = last >= 63 ? 0ull : starts & (~0ull << (last + 1));
  const int end = after ? __ffsll((long long)after) - 1 : kWave;  // exclusive lane
  const uint64_t owned = (end >= kWave ? ~0ull : ((1ull << end) - 1ull)) & (~0ull << first);
  const bool bad = (~oks & owned & ins) != 0;
  const int count = __popcll(mine);
  const bool take = !bad && count <= kMaxRuns;
  if (lane == 0) {
    *nruns = take ? count : 0;
    own[0] = first - 1;
    own[1] = end - 1;
  }
  if (take && ((mine >> lane) & 1ull)) {
    const uint64_t later = lane >= 63 ? 0ull : starts & (~0ull << (lane + 1));
    const int e = later ? __ffsll((long long)later) - 1 : kWave;
    GroupRun r;
    r.block = blk;
    r.lo = off;
    r.hi = off + (e - lane);
    r.tok = lane - 1;
    r.pad_ = 0;
    runs[__popcll(mine & ((1ull << lane) - 1ull))] = r;
  }
}

// Per-token write of one tensor (V when v, else K) for the tokens
// [t0, t0 + n) of a group that does not fill a block, shared by `nwaves`
// waves: this workgroup's wave w is wave wave0 + w of them and takes tokens
// wave0 + w, wave0 + w + nwaves, ...
template <class Op, bool IDX>
__device__ __forceinline__ void write_group_tokens(const WriteArgs &a, int64_t t0, int n, bool v,
                                                   float uniform, int wave0, int nwaves) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const GeomBytes &g = v ? a.gv : a.gk;
  const ScaleRef &sr = v ? a.vsc : a.ksc;
  const char *io = v ? a.src_v : a.src_k;
  char *cache = v ? a.dst_v : a.dst_k;
  for (int o = wave0 + wave; o < n; o += nwaves) {
    const int64_t t = t0 + o;
    if (t >= a.num_tokens) break;
    const int64_t slot = load_index(a.slots, t, a.slot_is64);
    if (slot < 0) continue;
    int64_t b, off;
    split_slot(slot, a.block_size, b, off);
    if (b >= a.num_blocks) continue;
    const char *src = io + t * a.row_bytes;
    char *dst = cache + b * g.s_block + off * g.s_off;
    for (int c = lane; c < a.nchunks; c += kWave) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      float sc = uniform;
      if constexpr (Op::kScaled && IDX) sc = scale_at(sr, uniform, b, e, (uint32_t)a.head_dim);
      st<Op::kDst, kWriteNtStore>(dst + chunk_off(g, e, (uint32_t)a.head_dim),
                                  Op::apply(ld<Op::kSrc>(src + (int64_t)c * Op::kSrc), sc));
    }
  }
}

// Tiled block write: the inverse of gather_tiles_kernel (below).  A group
// is `bs` consecutive tokens; when their slots form at most kMaxRuns runs of
// consecutive offsets of one block each (a whole block in order, or a
// prefill chunk that starts inside a block), a workgroup takes tile `tile`
// (tw cache bytes of every row) of one tensor (blockIdx.y: K 0, V 1) and,
// run by run:
//   phase 1  reads the tile's columns of the run's source rows, applies the
//            chunk op (copy, or FP8 quantization with the scale of the
//            run's block and the chunk's head)
//            and stores the cache bytes in LDS rows (pitch tw + 16 bytes);
//   phase 2  assembles each 16-byte chunk of the block region
//            [tile * tw * bs, (tile + 1) * tw * bs) from its run pieces and
//            stores it; chunks holding rows outside the run store those
//            rows' pieces only.
// A row-major tensor copies its rows straight through.  Any other group is
// written token by token, each tensor's tokens spread over the waves of
// that tensor's `tiles` workgroups of the group.
struct WriteTileArgs {
  int32_t tiles;          // tiles per block: cache row bytes / tw
  int32_t tw;             // tile width, cache bytes per row
  int32_t tw_log2;        // log2(tw), or -1 when tw is not a power of two
  int32_t cpr;            // tw_log2 < 0: phase-1 chunks per tile row
  uint32_t cpr_magic;     // tw_log2 < 0: div_magic's m for cpr
  int32_t pitch;          // LDS row pitch, bytes
  int32_t threads;        // workgroup size (64-256, by tile bytes)
  int32_t bs_log2;
  int32_t run_log2[2];    // K, V: log2 bytes of a per-token run; -1 row-major;
                          // kRunOdd: run_bytes, a multiple of 16 bytes
  int32_t run_bytes[2];
  uint32_t run_magic[2];  // kRunOdd: div_magic's m for run_bytes
  int32_t cache_es_log2;  // log2 cache element bytes
  int32_t io_es_log2;     // log2 io element bytes
};

// Row and chunk of tile chunk u (cpr chunks per tile row): shifts when the
// tile width is a power of two, a multiply-high division otherwise (ODD).
template <bool ODD>
__device__ __forceinline__ int32_t tile_row(int32_t u, int32_t cpr_log2, const WriteTileArgs &wt) {
  if constexpr (ODD) return (int32_t)div_magic((uint32_t)u, wt.cpr_magic);
  else return u >> cpr_log2;
}
template <bool ODD>
__device__ __forceinline__ int32_t tile_col(int32_t u, int32_t row, int32_t cpr_log2,
                                            const WriteTileArgs &wt) {
  if constexpr (ODD) return u - row * wt.cpr;
  else return u & ((1 << cpr_log2) - 1);
}

// Piece k (PIECE bytes) of a 16-byte chunk, read from p into x (x's other
// pieces untouched; x starts zeroed for PIECE < 4).
template <int PIECE>
__device__ __forceinline__ void get_piece(const char *p, Raw<16> &x, int k) {
  if constexpr (PIECE == 16) {
    x = ld<16>(p);
  } else if constexpr (PIECE == 8) {
    const Raw<8> y = ld<8>(p);
    x.w[2 * k] = y.w[0];
    x.w[2 * k + 1] = y.w[1];
  } else if constexpr (PIECE == 4) {
    x.w[k] = ld<4>(p).w[0];
  } else if constexpr (PIECE == 2) {
    put16(x, k, ld<2>(p).w[0]);
  } else {
    put8(x, k, ld<1>(p).w[0]);
  }
}

// Phase 2 of the tiled write: LDS rows -> region (nbytes = tw * bs cache
// bytes, 16-byte aligned), rows [lo, hi) only.  PIECE = min(run bytes, 16).
// A 16-byte chunk whose pieces all belong to rows in [lo, hi) is stored
// whole; a chunk that mixes rows (runs shorter than 16 bytes, partial
// blocks) stores the pieces of its rows in range one by one.  FULL: every
// row is in range (a whole block), and the row tests are compiled out.
template <int PIECE, bool FULL>
__device__ __forceinline__ void unstage_tile(char *region, const char *lds, int32_t nbytes,
                                             int32_t run_log2, int32_t bs_log2, int32_t pitch,
                                             int32_t lo, int32_t hi) {
  const int32_t bsm = (1 << bs_log2) - 1;
  const int32_t runm = (1 << run_log2) - 1;
  const int32_t kStep = (int32_t)blockDim.x * 16;
  for (int32_t m0 = (int32_t)threadIdx.x * 16; m0 < nbytes; m0 += kTileLoads * kStep) {
    Raw<16> x[kTileLoads];
    bool whole[kTileLoads];
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u) {
      const int32_t m = m0 + u * kStep;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[u].w[i] = 0;
      whole[u] = m < nbytes;
      if (m < nbytes) {
#pragma unroll
        for (int k = 0; k < 16 / PIECE; ++k) {
          const int32_t mm = m + k * PIECE;
          const int32_t o = (mm >> run_log2) & bsm;
          const int32_t ar = mm >> (run_log2 + bs_log2);
          const char *p = lds + o * pitch + (ar << run_log2) + (mm & runm);
          if (FULL || (o >= lo && o < hi)) {
            get_piece<PIECE>(p, x[u], k);
          } else {
            whole[u] = false;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u) {
      const int32_t m = m0 + u * kStep;
      if (whole[u]) {
        st<16, kWriteNtStore>(region + m, x[u]);
      } else if (!FULL && m < nbytes) {
#pragma unroll
        for (int k = 0; k < 16 / PIECE; ++k) {
          const int32_t mm = m + k * PIECE;
          const int32_t o = (mm >> run_log2) & bsm;
          if (o >= lo && o < hi) {
            const int32_t ar = mm >> (run_log2 + bs_log2);
            st<PIECE, kWriteNtStore>(region + mm,
                                     ld<PIECE>(lds + o * pitch + (ar << run_log2) + (mm & runm)));
          }
        }
      }
    }
  }
}

// Phase 2 for runs of `run` bytes, a multiple of 16 but not a power of two:
// every 16-byte chunk lies inside one run of one row, and is stored whole
// when that row is in [lo, hi).
template <bool FULL>
__device__ __forceinline__ void unstage_tile_odd(char *region, const char *lds, int32_t nbytes,
                                                 int32_t run, uint32_t run_magic, int32_t bs_log2,
                                                 int32_t pitch, int32_t lo, int32_t hi) {
  const uint32_t bsm = (1u << bs_log2) - 1;
  const int32_t kStep = (int32_t)blockDim.x * 16;
  for (int32_t m0 = (int32_t)threadIdx.x * 16; m0 < nbytes; m0 += kTileLoads * kStep) {
    Raw<16> x[kTileLoads];
    bool ok[kTileLoads];
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u) {
      const int32_t m = m0 + u * kStep;
      const uint32_t q = div_magic((uint32_t)m, run_magic);
      const int32_t o = (int32_t)(q & bsm);
      ok[u] = m < nbytes && (FULL || (o >= lo && o < hi));
      if (ok[u]) x[u] = ld<16>(lds + o * pitch + (int32_t)(q >> bs_log2) * run + (m - (int32_t)q * run));
    }
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u)
      if (ok[u]) st<16, kWriteNtStore>(region + m0 + u * kStep, x[u]);
  }
}

// ODD: the tile width is not a power of two, as it is for every run that
// is not (a multiple of such a run never is one), so only then can
// run_log2 be kRunOdd.
template <bool FULL, bool ODD>
__device__ __forceinline__ void unstage_any(char *dst, const char *lds, int32_t region,
                                            int32_t run_log2, const WriteTileArgs &wt,
                                            const GroupRun &r, bool v) {
  if constexpr (ODD) {
    if (run_log2 == kRunOdd) {
      unstage_tile_odd<FULL>(dst, lds, region, wt.run_bytes[v], wt.run_magic[v], wt.bs_log2,
                             wt.pitch, r.lo, r.hi);
      return;
    }
  }
  switch (run_log2) {
    case 0: unstage_tile<1, FULL>(dst, lds, region, 0, wt.bs_log2, wt.pitch, r.lo, r.hi); break;
    case 1: unstage_tile<2, FULL>(dst, lds, region, 1, wt.bs_log2, wt.pitch, r.lo, r.hi); break;
    case 2: unstage_tile<4, FULL>(dst, lds, region, 2, wt.bs_log2, wt.pitch, r.lo, r.hi); break;
    case 3: unstage_tile<8, FULL>(dst, lds, region, 3, wt.bs_log2, wt.pitch, r.lo, r.hi); break;
    default:
      unstage_tile<16, FULL>(dst, lds, region, run_log2, wt.bs_log2, wt.pitch, r.lo, r.hi);
      break;
  }
}

// One run of a group through one tile of one tensor: rows [r.lo, r.hi) of
// block r.block from the io rows of tokens t0 + r.tok, ...
template <class Op, bool IDX, bool ODD>
__device__ __forceinline__ void write_tile_run(const WriteArgs &a, const WriteTileArgs &wt,
                                               const GroupRun &r, int64_t t0, int32_t tile,
                                               bool v, float uniform, char *lds) {
  const ScaleRef &sr = v ? a.vsc : a.ksc;
  const uint32_t hd = (uint32_t)a.head_dim;
  const char *src = (v ? a.src_v : a.src_k) + (t0 + r.tok) * a.row_bytes;
  char *blk = v ? a.dst_v + r.block * a.gv.s_block : a.dst_k + r.block * a.gk.s_block;
  const int32_t run_log2 = v ? wt.run_log2[1] : wt.run_log2[0];
  const int32_t region = wt.tw << wt.bs_log2;
  const int tid = (int)threadIdx.x;

  if (run_log2 < 0) {
    // Row-major block: rows [lo, hi) are one span of the block and of the
    // source rows.
    const int32_t row_bytes_c = wt.tiles * wt.tw;
    const int32_t span_lo = r.lo * row_bytes_c;
    const int32_t span_hi = r.hi * row_bytes_c;
    const int32_t lo = tile * region > span_lo ? tile * region : span_lo;
    const int32_t hi = (tile + 1) * region < span_hi ? (tile + 1) * region : span_hi;
    const uint32_t re = (uint32_t)a.nchunks * (uint32_t)a.chunk_elems;  // H * D
    for (int32_t m = lo + tid * Op::kDst; m < hi; m += (int32_t)blockDim.x * Op::kDst) {
      const uint32_t e = (uint32_t)(m - span_lo) >> wt.cache_es_log2;
      float sc = uniform;
      if constexpr (Op::kScaled && IDX) sc = scale_in_rows(sr, uniform, r.block, e, re, hd);
      st<Op::kDst, kWriteNtStore>(
          blk + m, Op::apply(ld<Op::kSrc, kWriteNtLoad>(src + ((int64_t)e << wt.io_es_log2)),
                             sc));
    }
    return;
  }

  // Phase 1: chunk c of row lo + q holds the row's io elements e0 + c * G.
  constexpr int kDstLog2 = Op::kDst == 16 ? 4 : Op::kDst == 8 ? 3 : Op::kDst == 4 ? 2
                           : Op::kDst == 2 ? 1 : 0;
  const int32_t cpr_log2 = wt.tw_log2 - kDstLog2;
  const int32_t total = ODD ? (r.hi - r.lo) * wt.cpr : (r.hi - r.lo) << cpr_log2;
  const uint32_t e0 = ((uint32_t)tile * (uint32_t)wt.tw) >> wt.cache_es_log2;
  for (int32_t u0 = tid; u0 < total; u0 += kTileLoads * (int32_t)blockDim.x) {
    Raw<Op::kSrc> x[kTileLoads];
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int32_t u = u0 + k * (int32_t)blockDim.x;
      if (u < total) {
        const int32_t row = tile_row<ODD>(u, cpr_log2, wt);
        const int32_t col = tile_col<ODD>(u, row, cpr_log2, wt);
        const uint32_t e = e0 + ((uint32_t)(col << kDstLog2) >> wt.cache_es_log2);
        x[k] = ld<Op::kSrc, kWriteNtLoad>(src + (int64_t)row * a.row_bytes +
                                          ((int64_t)e << wt.io_es_log2));
      }
    }
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int32_t u = u0 + k * (int32_t)blockDim.x;
      if (u < total) {
        const int32_t row = tile_row<ODD>(u, cpr_log2, wt);
        const int32_t col = tile_col<ODD>(u, row, cpr_log2, wt);
        float sc = uniform;
        if constexpr (Op::kScaled && IDX) {
          const uint32_t e = e0 + ((uint32_t)(col << kDstLog2) >> wt.cache_es_log2);
          sc = scale_at(sr, uniform, r.block, e, hd);
        }
        st<Op::kDst>(lds + (r.lo + row) * wt.pitch + (col << kDstLog2), Op::apply(x[k], sc));
      }
    }
  }
  __syncthreads();
  char *dst = blk + (int64_t)tile * region;
  if (r.lo == 0 && r.hi == (1 << wt.bs_log2)) {
    unstage_any<true, ODD>(dst, lds, region, run_log2, wt, r, v);
  } else {
    unstage_any<false, ODD>(dst, lds, region, run_log2, wt, r, v);
  }
}

// Whole-block fast path of write_tiles_kernel, for the usual prefill group.
// Aligned: the group's bs slots are block * bs + 0 .. bs - 1 in token
// order.  The group's source rows do not depend on the slots, so every
// thread issues the loads of its (at most kTileLoads) chunks of the tile
// first; each wave then loads the bs slots itself (one per lane) and tests
// them with a ballot, so the slot latency overlaps the data loads and no
// barrier is needed to share the test.  Every wave reaches the same answer
// from the same slots.
// Row-major split (row-major tensors, whose groups write their own
// tokens): the group's first k tokens end one block in order and the rest
// start another, as in a prefill chunk that starts inside a block; the
// loaded rows go straight to both blocks.
// Shifted (other layouts, block sizes up to 32, where owned_runs decides
// ownership): a prefill chunk that starts inside a block makes the group's
// first k tokens continue the run of token t0 - 1 and its next bs tokens
// fill the following block; the group then owns exactly that block (one
// run starting at t0 + k).  k follows from the first test's slot of t0, so the
// loads of rows t0 + k .. are issued together with the slots that confirm
// it, instead of after the run analysis and a barrier.
// Returns false, having stored nothing, when the group is neither (or is
// the short last group, or its tile needs more than one pass): the caller
// then runs the general run analysis.  The speculative loads stay within the
// io rows of tokens < num_tokens.
template <class Op, bool IDX, bool ODD>
__device__ __forceinline__ bool write_tile_block(const WriteArgs &a, const WriteTileArgs &wt,
                                                 int64_t t0, int32_t tile, bool v,
                                                 float uniform, char *lds) {
  constexpr int kDstLog2 = Op::kDst == 16 ? 4 : Op::kDst == 8 ? 3 : Op::kDst == 4 ? 2
                           : Op::kDst == 2 ? 1 : 0;
  const int32_t bs = 1 << wt.bs_log2;
  const int32_t region = wt.tw << wt.bs_log2;  // cache bytes of the tile
  const int32_t total = region >> kDstLog2;    // chunks of the tile
  if (t0 + bs > a.num_tokens || total > kTileLoads * (int32_t)blockDim.x) return false;
  const int32_t run_log2 = v ? wt.run_log2[1] : wt.run_log2[0];
  const char *io = v ? a.src_v : a.src_k;
  const int tid = (int)threadIdx.x;
  const int lane = tid & (kWave - 1);
  int64_t slot = -1;
  if (lane < bs) slot = load_index(a.slots, t0 + lane, a.slot_is64);

  // Source of chunk u for a run starting at token tb.  Row-major cache: the
  // tile is bytes [tile * region, (tile + 1) * region) of the block, which
  // hold io elements e = byte >> cache_es_log2 counted from row tb.
  // Otherwise: chunk u is chunk tile_col(u) of the tile's columns of row
  // tb + tile_row(u).
  const int32_t cpr_log2 = wt.tw_log2 - kDstLog2;
  const uint32_t e0 = ((uint32_t)tile * (uint32_t)wt.tw) >> wt.cache_es_log2;
  auto row_of = [&](int32_t u) { return tile_row<ODD>(u, cpr_log2, wt); };
  auto col_of = [&](int32_t u) { return tile_col<ODD>(u, row_of(u), cpr_log2, wt); };
  auto elem = [&](int32_t u) -> uint32_t {  // io element of chunk u within its row run
    return run_log2 < 0
               ? (uint32_t)((tile * region + (u << kDstLog2)) >> wt.cache_es_log2)
               : e0 + ((uint32_t)(col_of(u) << kDstLog2) >> wt.cache_es_log2);
  };
  Raw<Op::kSrc> x[kTileLoads];
  auto load_rows = [&](int64_t tb) {
    const char *src = io + tb * a.row_bytes;
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int32_t u = tid + k * (int32_t)blockDim.x;
      if (u < total) {
        x[k] = ld<Op::kSrc, kWriteNtLoad>(
            run_log2 < 0 ? src + ((int64_t)elem(u) << wt.io_es_log2)
                         : src + (int64_t)row_of(u) * a.row_bytes +
                               ((int64_t)elem(u) << wt.io_es_log2));
      }
    }
  };
  auto uniform64 = [](int64_t x) {
    return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(x >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)x));
  };
  load_rows(t0);

  const int64_t first = uniform64(slot);
  int64_t block = first >> wt.bs_log2;
  const bool in_order = lane >= bs || slot == first + lane;
  if (run_log2 < 0 && (__ballot(!in_order) != 0 || (first & (bs - 1)) != 0)) {
    // Row-major split: tokens t0 .. t0 + k - 1 end block A (offsets
    // bs - k .. bs - 1) and t0 + k .. t0 + bs - 1 start block B; the rows
    // loaded above are this group's own, stored straight to both blocks.
    if (first < 0 || block >= a.num_blocks || (first & (bs - 1)) == 0) return false;
    const int32_t k = bs - (int32_t)(first & (bs - 1));
    const int64_t f2 = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(
                                      __shfl((int)(slot >> 32), k)) << 32) |
                                 (uint32_t)__builtin_amdgcn_readfirstlane(__shfl((int)slot, k)));
    const int64_t block_b = f2 >> wt.bs_log2;
    const bool bad = lane < k ? slot != first + lane : (lane < bs && slot != f2 + (lane - k));
    if (__ballot(bad) != 0 || f2 < 0 || (f2 & (bs - 1)) != 0 || block_b >= a.num_blocks)
      return false;
    const ScaleRef &sr = v ? a.vsc : a.ksc;
    const uint32_t hd = (uint32_t)a.head_dim;
    const uint32_t re = (uint32_t)a.nchunks * (uint32_t)a.chunk_elems;  // H * D
    const int32_t rbc = wt.tiles * wt.tw;  // cache bytes of a row
    char *base = v ? a.dst_v : a.dst_k;
    const int64_t sb = v ? a.gv.s_block : a.gk.s_block;
    // byte m of the group's rows: row m / rbc of the group is row
    // bs - k + m / rbc of block A, or row m / rbc - k of block B
    const int64_t at_a = block * sb + (int64_t)(bs - k) * rbc;
    const int64_t at_b = block_b * sb - (int64_t)k * rbc;
#pragma unroll
    for (int q = 0; q < kTileLoads; ++q) {
      const int32_t u = tid + q * (int32_t)blockDim.x;
      if (u < total) {
        const int32_t m = tile * region + (u << kDstLog2);
        const bool in_a = m < k * rbc;
        float sc = uniform;
        if constexpr (Op::kScaled && IDX)
          sc = scale_in_rows(sr, uniform, in_a ? block : block_b, elem(u), re, hd);
        st<Op::kDst, kWriteNtStore>(base + ((in_a ? at_a : at_b) + m), Op::apply(x[q], sc));
      }
    }
    return true;
  }
  if (__ballot(!in_order) != 0 || first < 0 || (first & (bs - 1)) != 0 ||
      block >= a.num_blocks) {
    // Shifted: tokens t0 .. t0 + k - 1 hold first, first + 1, ... up to the
    // end of its block and continue token t0 - 1 (first - 1); tokens t0 + k
    // .. t0 + k + bs - 1 fill one block in order.
    if (wt.bs_log2 > 5 || t0 == 0 || first < 0 || block >= a.num_blocks) return false;
    const int32_t k = bs - (int32_t)(first & (bs - 1));
    if (k >= bs || t0 + k + bs > a.num_tokens) return false;
    if (__ballot(lane < k && slot != first + lane) != 0) return false;
    const int64_t prev = load_index(a.slots, t0 - 1, a.slot_is64);
    int64_t next = -1;
    if (lane < bs) next = load_index(a.slots, t0 + k + lane, a.slot_is64);
    load_rows(t0 + k);
    const int64_t f2 = uniform64(next);
    block = f2 >> wt.bs_log2;
    if (prev != first - 1 || __ballot(lane < bs && next != f2 + lane) != 0 || f2 < 0 ||
        (f2 & (bs - 1)) != 0 || block >= a.num_blocks)
      return false;
  }

  const ScaleRef &sr = v ? a.vsc : a.ksc;
  const uint32_t hd = (uint32_t)a.head_dim;
  char *blk = v ? a.dst_v + block * a.gv.s_block : a.dst_k + block * a.gk.s_block;
  if (run_log2 < 0) {
    const uint32_t re = (uint32_t)a.nchunks * (uint32_t)a.chunk_elems;  // H * D
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int32_t u = tid + k * (int32_t)blockDim.x;
      if (u < total) {
        float sc = uniform;
        if constexpr (Op::kScaled && IDX) sc = scale_in_rows(sr, uniform, block, elem(u), re, hd);
        st<Op::kDst, kWriteNtStore>(blk + tile * region + (u << kDstLog2), Op::apply(x[k], sc));
      }
    }
    return true;
  }
#pragma unroll
  for (int k = 0; k < kTileLoads; ++k) {
    const int32_t u = tid + k * (int32_t)blockDim.x;
    if (u < total) {
      float sc = uniform;
      if constexpr (Op::kScaled && IDX) sc = scale_at(sr, uniform, block, elem(u), hd);
      st<Op::kDst>(lds + row_of(u) * wt.pitch + (col_of(u) << kDstLog2), Op::apply(x[k], sc));
    }
  }
  __syncthreads();
  GroupRun r;
  r.block = block;
  r.lo = 0;
  r.hi = bs;
  r.tok = 0;
  r.pad_ = 0;
  unstage_any<true, ODD>(blk + (int64_t)tile * region, lds, region, run_log2, wt, r, v);
  return true;
}

// Op: the tile's chunk op (16-byte cache chunks); TokOp: the per-token
// path's op, whose chunk fits the cache geometry (WriteArgs' chunking).
// IDX: indexed (per-head / per-block) scales are looked up per chunk; the
// per-tensor instances carry no lookup code (registers decide occupancy).
template <class Op, class TokOp, bool IDX, bool ODD>
__global__ __launch_bounds__(kBlockThreads) void write_tiles_kernel(WriteArgs a,
                                                                    WriteTileArgs wt) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ GroupRun s_runs[kMaxRuns];
  __shared__ int32_t s_nruns;
  const uint32_t gu = blockIdx.x / (uint32_t)wt.tiles;
  const int32_t tile = (int32_t)(blockIdx.x - gu * (uint32_t)wt.tiles);
  const int64_t t0 = (int64_t)gu << wt.bs_log2;
  const bool v = blockIdx.y != 0;
  float ks = 1.0f;  // per-tensor values; indexed scales are looked up per chunk
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }
  if (write_tile_block<Op, IDX, ODD>(a, wt, t0, tile, v, v ? vs : ks, lds)) return;
  // Which tokens this tensor's workgroups of the group write.  Row-major
  // blocks (NHD) hold whole rows: each group writes its own tokens, split
  // into runs (group_runs), so a block that a prefill chunk starts inside is
  // written in two parts of whole rows.  Other layouts interleave a block's
  // rows in 1-16 byte pieces; there, for block sizes up to 32, the group in
  // which a run starts writes all of it (owned_runs), so that no cache line
  // of a block is written in parts by two workgroups.
  __shared__ int32_t s_own[2];
  const int32_t run_log2 = v ? wt.run_log2[1] : wt.run_log2[0];
  if (wt.bs_log2 <= 5 && run_log2 >= 0) {
    owned_runs(a, t0, wt.bs_log2, s_runs, &s_nruns, s_own);
  } else {
    group_runs(a, t0, wt.bs_log2, s_runs, &s_nruns);
    if (threadIdx.x == 0) {
      s_own[0] = 0;
      s_own[1] = 1 << wt.bs_log2;
    }
  }
  __syncthreads();
  const int32_t nruns = s_nruns;
  if (nruns == 0) {
    const int wpb = (int)(blockDim.x / kWave);  // waves per workgroup
    write_group_tokens<TokOp, IDX>(a, t0 + s_own[0], s_own[1] - s_own[0], v, v ? vs : ks,
                                   tile * wpb, wt.tiles * wpb);
    return;
  }
  for (int32_t i = 0; i < nruns; ++i) {
    if (i > 0) __syncthreads();  // the LDS tile is reused
    write_tile_run<Op, IDX, ODD>(a, wt, s_runs[i], t0, tile, v, v ? vs : ks, lds);
  }
}

// ---------------------------------------------------------------------------
// Gather.
//
// PACKED tables: when the cache rows of a block are contiguous (canonical
// NHD) gather_flat_kernel streams row ranges of the block as flat copies;
// dense blocks in other orders (x-packed, HND, token-innermost) take
// gather_tiles_kernel's LDS transpose; any other strides take
// gather_rows_kernel.  RAGGED and KV_OFFSETS tables have their own kernels
// (gather_indexed_flat_kernel, gather_indexed_kernel) besides the tile one.

struct GatherArgs {
  const char *src_k;
  const char *src_v;
  char *dst_k;
  char *dst_v;
  const void *table;
  const void *seq_lens;
  ScaleRef ksc;              // dequantizing ops only
  ScaleRef vsc;
  const void *indptr;        // RAGGED
  int64_t table_count;       // RAGGED: entries of `table`
  const char *pool[2];       // KV_OFFSETS primary / secondary
  int64_t bytes_per_block;   // KV_OFFSETS
  int32_t pool_blocks[2];    // KV_OFFSETS: entries of pool i at or past pool_blocks[i] are skipped
  GeomBytes gk;
  GeomBytes gv;
  int64_t out_row_bytes;  // bytes of one output row (H * D * io size)
  int32_t index_is64;
  int32_t lens_is64;
  int32_t indptr_is64;
  int32_t rows_per_wg;    // RAGGED / KV_OFFSETS: output rows per workgroup
  int32_t max_blocks_per_seq;
  int32_t blocks_per_seq;  // workgroups per sequence
  int32_t max_seq_len;
  int32_t block_size;
  int32_t num_blocks;
  int32_t head_dim;
  int32_t nchunks;
  int32_t chunk_elems;
  int32_t lpt_log2;
  int32_t flat;  // cache rows of a block are contiguous for K and V
  int32_t split_log2;  // PACKED flat and row gathers: workgroups per block = 1 << split_log2
  int32_t format;      // kvx_block_table_format_t
  int32_t nchunks_log2;  // log2(nchunks), or -1 when not a power of two
  uint32_t nchunks_magic;  // nchunks_log2 < 0: div_magic's m for nchunks
  int32_t bs_log2;       // log2(block_size), or -1 when not a power of two
  int32_t ragged_tile;   // RAGGED: gather_ragged_tile_kernel
  int32_t fold_log2;     // PACKED flat gather: up to 1 << fold_log2 units per workgroup
  int32_t units_per_seq;  // PACKED flat gather: (block, part) units per sequence
  int32_t cph_log2;       // head-run flat gather: log2(chunks per head)
};

// The (sequence, logical block) job of one workgroup: cache block and
// output rows, or false when the block is skipped (past seq_len or
// max_seq_len, beyond max_blocks_per_seq, or a block id outside
// [0, num_blocks)).  seq_len and the block id are wave-uniform scalar loads.
// Row of chunk gi of a run of rows of nchunks chunks each (the flat indexed
// gathers): a shift when nchunks is a power of two, else a multiply-high
// (dispatch keeps gi * nchunks <= 2^32).
__device__ __forceinline__ uint32_t row_of_chunk(const GatherArgs &a, uint32_t gi) {
  return a.nchunks_log2 >= 0 ? gi >> a.nchunks_log2 : div_magic(gi, a.nchunks_magic);
}

struct BlockJob {
  const char *ck;
  const char *cv;
  char *ok;
  char *ov;
  int64_t bid;
  int32_t rows;
  float ks;
  float vs;
};

template <class Op, bool I64>
__device__ __forceinline__ bool gather_job(const GatherArgs &a, BlockJob &j) {
  const uint32_t wg = blockIdx.x;
  const uint32_t su = wg / (uint32_t)a.blocks_per_seq;
  const int64_t s = su;
  // part `part` of 1 << split_log2 equal row ranges of logical block lb
  const uint32_t w = wg - su * (uint32_t)a.blocks_per_seq;
  const int32_t lb = (int32_t)(w >> a.split_log2);
  const int32_t part = (int32_t)(w & ((1u << a.split_log2) - 1));
  if (lb >= a.max_blocks_per_seq) return false;
  const int64_t seq_len = load_idx<I64>(a.seq_lens, s);
  const int64_t bid = load_idx<I64>(a.table, s * a.max_blocks_per_seq + lb);
  const int64_t n = seq_len < a.max_seq_len ? seq_len : (int64_t)a.max_seq_len;
  const int32_t per_part = a.block_size >> a.split_log2;
  const int32_t r0 = part * per_part;  // first row of the part in the block
  const int64_t t0 = (int64_t)lb * a.block_size + r0;
  if (t0 >= n) return false;
  if (bid < 0 || bid >= a.num_blocks) return false;
  const int64_t rem = n - t0;
  j.rows = rem < per_part ? (int32_t)rem : per_part;
  j.bid = bid;
  j.ks = 1.0f;
  j.vs = 1.0f;
  if constexpr (Op::kScaled) {
    j.ks = a.ksc.p[0];
    j.vs = a.vsc.p[0];
  }
  j.ck = a.src_k + bid * a.gk.s_block + (int64_t)r0 * a.gk.s_off;
  j.cv = a.src_v + bid * a.gv.s_block + (int64_t)r0 * a.gv.s_off;
  const int64_t out0 = (s * a.max_seq_len + t0) * a.out_row_bytes;
  j.ok = a.dst_k + out0;
  j.ov = a.dst_v + out0;
  return true;
}

// Canonical-NHD gather: the valid rows of a block are one contiguous run in
// the cache and in the output, streamed as a flat copy.  A workgroup copies
// one power-of-two share of the block's chunks (kFlatTileBytes).
// Copy `total` chunks of K and of V: flat index f < 2 * total, K for
// f < total, V above, so a tile of kFlatThreads chunks per tensor gives
// every thread one K chunk and one V chunk.
// Scale of chunk i (counted from a row start) of a flat run: the
// per-tensor value, or the indexed entry of block `bid` and the chunk's head.
__device__ __forceinline__ float run_scale(const GatherArgs &a, bool v, float ks, float vs,
                                           int64_t bid, int64_t i) {
  const ScaleRef &r = v ? a.vsc : a.ksc;
  if (!r.indexed) return v ? vs : ks;
  const uint32_t c = (uint32_t)i % (uint32_t)a.nchunks;  // i < 2^31 within a tile
  const uint32_t h = c * (uint32_t)a.chunk_elems / (uint32_t)a.head_dim;
  return r.p[bid * r.s_block + (int64_t)h * r.s_head];
}

// Source of chunk i of a flat run that starts at chunk c0 of a block: with
// HR (head runs) the block's chunks in output order are (row, head, chunk)
// triples, each head's D elements contiguous at any row and head strides:
// base is the block, and chunk c0 + i sits at row t, head h, chunk c of the
// head (shifts: power-of-two heads and chunks per head).  Otherwise the run
// is contiguous from base.
template <class Op, bool HR>
__device__ __forceinline__ const char *flat_src(const GatherArgs &a, const GeomBytes &g,
                                                const char *base, int64_t c0, int64_t i) {
  if constexpr (!HR) {
    return base + i * Op::kSrc;
  } else {
    const uint32_t e = (uint32_t)(c0 + i);  // < block_size * nchunks < 2^31
    const uint32_t t = e >> a.nchunks_log2;
    const uint32_t r = e & ((1u << a.nchunks_log2) - 1u);
    const uint32_t h = r >> a.cph_log2;
    const uint32_t c = r & ((1u << a.cph_log2) - 1u);
    return base + (int64_t)t * g.s_off + (int64_t)h * g.s_head + (int64_t)c * Op::kSrc;
  }
}

// c0: chunk index of ck / cv counted from a row start (indexed scales).
// HR: ck / cv are the blocks, the run's chunks addressed by flat_src.
template <class Op, bool HR = false>
__device__ __forceinline__ void flat_copy(const GatherArgs &a, const char *ck, const char *cv,
                                          char *ok, char *ov, int64_t total, float ks, float vs,
                                          int64_t bid, int64_t c0) {
  constexpr int U = Op::kScaled ? kFlatUnrollDequant : kFlatUnroll;
  const int64_t both = 2 * total;
  int64_t f = threadIdx.x;
  for (; f + (U - 1) * kFlatThreads < both; f += U * kFlatThreads) {
    // Indexed scales do not depend on the data: look them up first, so that
    // their loads and the data loads are in flight together.
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t g = f + u * kFlatThreads;
      const bool v = g >= total;
      sc[u] = v ? vs : ks;
      if constexpr (Op::kScaled) sc[u] = run_scale(a, v, ks, vs, bid, c0 + g - (v ? total : 0));
    }
    Raw<Op::kSrc> x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t g = f + u * kFlatThreads;
      const bool v = g >= total;
      x[u] = ld<Op::kSrc, kGatherNtLoad>(
          flat_src<Op, HR>(a, v ? a.gv : a.gk, v ? cv : ck, c0, g - (v ? total : 0)));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t g = f + u * kFlatThreads;
      const bool v = g >= total;
      const int64_t i = g - (v ? total : 0);
      st<Op::kDst, kGatherNtStore>((v ? ov : ok) + i * Op::kDst, Op::apply(x[u], sc[u]));
    }
  }
  for (; f < both; f += kFlatThreads) {
    const bool v = f >= total;
    const int64_t i = f - (v ? total : 0);
    float sc = v ? vs : ks;
    if constexpr (Op::kScaled) sc = run_scale(a, v, ks, vs, bid, c0 + i);
    st<Op::kDst, kGatherNtStore>(
        (v ? ov : ok) + i * Op::kDst,
        Op::apply(ld<Op::kSrc, kGatherNtLoad>(flat_src<Op, HR>(a, v ? a.gv : a.gk, v ? cv : ck,
                                                                c0, i)),
                  sc));
  }
}

// Units (one 1 << split_log2 share of a block) per workgroup of
// gather_flat_kernel, at most: kFlatFold, taken when a sequence has
// kFlatFoldMinUnits to kFlatFoldMaxUnits units.
// The grid covers max_seq_len, so a decode batch's shorter sequences leave
// workgroups that only load seq_len and exit; on MI355X such workgroups cost
// wave launches (c2 with max_seq_len doubled at the same lengths: 1573 ->
// 1699 us per layer).  Against the one-unit kernel (same-box A/B medians,
// us per layer) two units measured c2 1540.3 -> 1531.8 (32 layers, 8192
// units per sequence), c4 633.4 -> 629.6 (4096 units) and c5 2032.8 ->
// 2005.9 (32768 units; 1.1-1.4% in two sessions).  Two units at 2048 units
// or fewer (one or two KV heads) measured up to 2.8% slower, where the last
// sequences' two-unit workgroups lengthen a short launch; four units were
// slower at every shape; ordering the grid unit-major (all sequences'
// first units first) 15-30% slower.  (Two tiles per workgroup in the flat indexed
// and transposing gathers measured 1-10% slower than one; the RAGGED tile
// gather takes two for long copies, below.)
constexpr int kFlatFoldLog2 = 1;
constexpr int kFlatFold = 1 << kFlatFoldLog2;
constexpr int64_t kFlatFoldMinUnits = 4096;
constexpr int64_t kFlatFoldMaxUnits = 65536;
// Sequences of at least kFlatLongUnits units (long contexts: Llama-3-70B's
// 16K-32K tokens in 32-token blocks give 32768) launch gather_flat_kernel
// with kFlatLongLds bytes of dynamic LDS, which the kernel does not use:
// it holds a CU to 12 of its 128-thread workgroups (12 * 12800 bytes fit
// the 160 KiB of LDS, 13 do not, at any allocation granule up to 1 KiB)
// instead of 16.  Same-process A/B on MI355X, us per gather, 16 -> 12
// workgroups: c5 2341 -> 2149, 2000 -> 1983 and 2061 -> 2037 on three
// boxes; c5's lengths over pools of 100000 / 200000 / 400000 blocks 2126 ->
// 2053, 2154 -> 2066, 2146 -> 2062.  Shorter sequences lose: c2 (8192
// units) 1438 -> 1464, c2's lengths in 32-token blocks 1450 -> 1467, c4
// (4096 units) 578 -> 589; 8 workgroups cost c2 9% and c4 16%.
constexpr int64_t kFlatLongUnits = 16384;
constexpr uint32_t kFlatLongLds = 12800;
// PACKED gathers of caches whose heads are contiguous runs of a power-of-two
// number of whole 128-byte lines (HND; a power-of-two head count) in blocks
// of at least kFlatHeadRunsMinBs tokens take gather_flat_kernel with
// head-run addressing instead of the LDS tiles or the row kernel.
constexpr int kFlatHeadRunsMinBs = 64;
// RAGGED copies in gather_ragged_tile_kernel: two tiles per workgroup when a
// sequence has kRaggedFoldMinUnits to kRaggedFoldMaxUnits tiles.  Against one tile per workgroup (same-box A/B, medians of 6
// rounds, us per layer): c2's RAGGED gather 1563.7 -> 1528.0 (8 layers) and
// 1468.8 -> 1448.9 (32 layers), c5's 2163.4 -> 2150.3; c4's FP8 RAGGED
// gather (4096 tiles) measured 6.7% slower with two tiles and keeps one.
constexpr int64_t kRaggedFoldMinUnits = 8192;
constexpr int64_t kRaggedFoldMaxUnits = 65536;

// A workgroup w of sequence s copies units w, w + J, ..., w + (F - 1) * J
// (J = blocks_per_seq workgroups per sequence, F = 1 << fold_log2) that lie
// below units_per_seq and seq_len; unit u is share u & (2^split_log2 - 1)
// of logical block u >> split_log2.
template <class Op, bool I64, bool HR>
__global__ __launch_bounds__(kFlatThreads) void gather_flat_kernel(GatherArgs a) {
  const uint32_t wg = blockIdx.x;
  const uint32_t su = wg / (uint32_t)a.blocks_per_seq;
  const int64_t s = su;
  const int32_t w = (int32_t)(wg - su * (uint32_t)a.blocks_per_seq);
  // seq_len and the block ids do not depend on each other: load them at once.
  const int64_t seq_len = load_idx<I64>(a.seq_lens, s);
  int64_t bid[kFlatFold];
#pragma unroll
  for (int i = 0; i < kFlatFold; ++i) {
    const int64_t u = (int64_t)w + (int64_t)i * a.blocks_per_seq;
    const int64_t lb = u >> a.split_log2;
    bid[i] = -1;
    if (i < (1 << a.fold_log2) && u < a.units_per_seq && lb < a.max_blocks_per_seq)
      bid[i] = load_idx<I64>(a.table, s * a.max_blocks_per_seq + lb);
  }
  const int64_t n = seq_len < a.max_seq_len ? seq_len : (int64_t)a.max_seq_len;
  float ks = 1.0f;  // per-tensor values; indexed scales are looked up per chunk
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }
  const int64_t per_part = ((int64_t)a.block_size * a.nchunks) >> a.split_log2;
#pragma unroll
  for (int i = 0; i < kFlatFold; ++i) {
    const int64_t u = (int64_t)w + (int64_t)i * a.blocks_per_seq;
    const int64_t lb = u >> a.split_log2;
    const int32_t part = (int32_t)(u & ((1 << a.split_log2) - 1));
    const int64_t t0 = lb * a.block_size;
    if (t0 >= n) break;  // later units lie further along the sequence
    if (bid[i] < 0 || bid[i] >= a.num_blocks) continue;
    // The block's valid rows are `valid` consecutive chunks of K (and of V);
    // this unit is chunks [c0, c0 + per_part) of them.
    const int64_t rem = n - t0;
    const int64_t valid = (rem < a.block_size ? rem : (int64_t)a.block_size) * a.nchunks;
    const int64_t c0 = (int64_t)part * per_part;
    if (c0 >= valid) continue;
    const int64_t cnt = valid - c0 < per_part ? valid - c0 : per_part;
    const int64_t out0 = (s * a.max_seq_len + t0) * a.out_row_bytes + c0 * Op::kDst;
    const int64_t skip = HR ? 0 : c0 * Op::kSrc;  // HR: flat_src addresses from the block
    flat_copy<Op, HR>(a, a.src_k + bid[i] * a.gk.s_block + skip,
                      a.src_v + bid[i] * a.gv.s_block + skip, a.dst_k + out0, a.dst_v + out0,
                      cnt, ks, vs, bid[i], c0);
  }
}

// Any other layout: rows go to (wave, lane group), each lane keeps the
// cache offsets of its chunks in registers.
template <class Op, bool I64>
__global__ __launch_bounds__(kBlockThreads) void gather_rows_kernel(GatherArgs a) {
  BlockJob j;
  if (!gather_job<Op, I64>(a, j)) return;
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int lpt = 1 << a.lpt_log2;
  const int tpw = kWave >> a.lpt_log2;
  const int sub = lane >> a.lpt_log2;
  const int l = lane & (lpt - 1);

  // Per chunk: cache offsets and (dequantizing ops) the scales of its head in
  // this block, the same for every row of the block.
  int64_t koff[kMaxChunksPerLane];
  int64_t voff[kMaxChunksPerLane];
  float ksk[kMaxChunksPerLane];
  float vsk[kMaxChunksPerLane];
#pragma unroll
  for (int k = 0; k < kMaxChunksPerLane; ++k) {
    const int c = l + k * lpt;
    koff[k] = 0;
    voff[k] = 0;
    ksk[k] = j.ks;
    vsk[k] = j.vs;
    if (c < a.nchunks) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      koff[k] = chunk_off(a.gk, e, (uint32_t)a.head_dim);
      voff[k] = chunk_off(a.gv, e, (uint32_t)a.head_dim);
      if constexpr (Op::kScaled) {
        const uint32_t h = e / (uint32_t)a.head_dim;
        ksk[k] = scale_of(a.ksc, j.ks, j.bid, h);
        vsk[k] = scale_of(a.vsc, j.vs, j.bid, h);
      }
    }
  }

  for (int r = wave * tpw + sub; r < j.rows; r += kWavesPerBlock * tpw) {
    const char *rk = j.ck + (int64_t)r * a.gk.s_off;
    const char *rv = j.cv + (int64_t)r * a.gv.s_off;
    char *wk = j.ok + (int64_t)r * a.out_row_bytes;
    char *wv = j.ov + (int64_t)r * a.out_row_bytes;
    Raw<Op::kSrc> xk[kMaxChunksPerLane];
    Raw<Op::kSrc> xv[kMaxChunksPerLane];
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
      const int c = l + k * lpt;
      if (c < a.nchunks) {
        xk[k] = ld<Op::kSrc>(rk + koff[k]);
        xv[k] = ld<Op::kSrc>(rv + voff[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
      const int c = l + k * lpt;
      if (c < a.nchunks) {
        st<Op::kDst>(wk + (int64_t)c * Op::kDst, Op::apply(xk[k], ksk[k]));
        st<Op::kDst>(wv + (int64_t)c * Op::kDst, Op::apply(xv[k], vsk[k]));
      }
    }
    for (int c = l + kMaxChunksPerLane * lpt; c < a.nchunks; c += lpt) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      const uint32_t h = e / (uint32_t)a.head_dim;
      const Raw<Op::kSrc> yk =
          ld<Op::kSrc>(rk + chunk_off(a.gk, e, (uint32_t)a.head_dim));
      const Raw<Op::kSrc> yv =
          ld<Op::kSrc>(rv + chunk_off(a.gv, e, (uint32_t)a.head_dim));
      st<Op::kDst>(wk + (int64_t)c * Op::kDst, Op::apply(yk, scale_of(a.ksc, j.ks, j.bid, h)));
      st<Op::kDst>(wv + (int64_t)c * Op::kDst, Op::apply(yv, scale_of(a.vsc, j.vs, j.bid, h)));
    }
  }
}

// Transposing gather of dense blocks (PACKED tables).
//
// A dense block stores its elements in (run a, offset o, within-run w)
// order: element e of row o sits at
//   (e / W) * bs * W + o * W + e % W          (element units)
// for a per-token run of W elements: W = 1 (token axis innermost, vLLM's
// value cache [blocks, H, D, bs]), W = x (x-packed HND_PACKED), W = D (HND)
// or W = H * D (row-major NHD).  Unless W = H * D, a row is gathered from
// H * D / W runs bs * W elements apart: loading rows directly uses a
// fraction of every HBM transaction when runs are short (and measures slower
// than this kernel even for HND's 256-byte runs).  Here a workgroup takes a
// tile of `tw` cache bytes of every row of one block, which is the
// contiguous region [tile * tw * bs, (tile + 1) * tw * bs) of the block:
//   phase 1  reads the region with 16-byte loads and stores each run piece
//            into LDS at its row (row pitch tw + 16 bytes: the 16-byte
//            column stores of 16 consecutive rows fall on distinct banks);
//   phase 2  reads the valid rows back in order and writes them with the
//            chunk op (copy, or FP8 dequant), tw bytes of cache per row.
// A row-major tensor paired with such a tensor copies its valid rows
// straight through.  blockIdx.y selects K (0) or V (1).  PACKED tables give
// the block id of (sequence, logical block); KV_OFFSETS tables give K's and
// V's block addresses separately (pool + index * bytes_per_block).  RAGGED
// tables give every row its own block id: a tile's rows t0 .. t0 + bs - 1
// sit at offsets 0 .. bs - 1 of their blocks, so a tile whose rows all name
// one block is gathered like a PACKED one, and any other tile reads each
// row's pieces from that row's block (the first wave compares the ids).

struct TileTensor {
  const char *src;    // cache tensor
  char *dst;          // output tensor
  int64_t s_block;    // bytes
  ScaleRef sc;        // dequantizing ops only
  int32_t run_log2;   // log2 bytes of a per-token run; -1 for row-major;
                      // kRunOdd: run_bytes, a multiple of 16 bytes
  int32_t run_bytes;
  uint32_t run_magic;  // kRunOdd: div_magic's m for run_bytes
  int32_t pad_;
};

// Rows of a tile (block_size) at most: the planner keeps
// block_size * (tw + 16) within 64 KiB of LDS with tw >= 128.
constexpr int kTileMaxRows = 256;

struct TileArgs {
  TileTensor t[2];
  const void *table;
  const void *seq_lens;
  const void *indptr;       // RAGGED
  int64_t table_count;      // RAGGED: entries of `table`
  const char *pool[2];      // KV_OFFSETS primary / secondary
  int64_t bytes_per_block;  // KV_OFFSETS
  int32_t pool_blocks[2];   // KV_OFFSETS: entries of pool i at or past pool_blocks[i] are skipped
  int64_t out_row_bytes;
  int32_t max_blocks_per_seq;
  int32_t blocks_per_seq;
  int32_t tiles;          // tiles per block: cache row bytes / tw
  int32_t tw;             // tile width, cache bytes per row
  int32_t tw_log2;        // log2(tw), or -1 when tw is not a power of two
  int32_t cpr;            // tw_log2 < 0: phase-2 chunks per tile row
  uint32_t cpr_magic;     // tw_log2 < 0: div_magic's m for cpr
  int32_t pitch;          // LDS row pitch, bytes
  int32_t threads;        // workgroup size (128 for small tiles, else 256)
  int32_t max_seq_len;
  int32_t num_blocks;
  int32_t head_dim;
  int32_t row_elems;      // H * D
  int32_t bs_log2;
  int32_t cache_es_log2;  // log2 cache element bytes
  int32_t io_es_log2;     // log2 output element bytes
};

// Store piece k (PIECE bytes) of a 16-byte chunk at p.
template <int PIECE>
__device__ __forceinline__ void put_piece(char *p, const Raw<16> &x, int k) {
  if constexpr (PIECE == 16) {
    st<16>(p, x);
  } else if constexpr (PIECE == 8) {
    Raw<8> y;
    y.w[0] = x.w[2 * k];
    y.w[1] = x.w[2 * k + 1];
    st<8>(p, y);
  } else if constexpr (PIECE == 4) {
    Raw<4> y;
    y.w[0] = x.w[k];
    st<4>(p, y);
  } else if constexpr (PIECE == 2) {
    Raw<2> y;
    y.w[0] = get16(x, k);
    st<2>(p, y);
  } else {
    Raw<1> y;
    y.w[0] = get8(x, k);
    st<1>(p, y);
  }
}

// Phase 1: region (nbytes = tw * bs cache bytes, 16-byte aligned) -> LDS
// rows.  PIECE = min(run bytes, 16).  A chunk whose first row is not valid
// is skipped: its later pieces are later rows of the same run, or (runs of
// bs * run < 16 bytes) start again at row 0, which is always valid.
template <int PIECE>
__device__ __forceinline__ void stage_tile(const char *region, char *lds, int32_t nbytes,
                                           int32_t run_log2, int32_t bs_log2, int32_t pitch,
                                           int32_t rows) {
  const int32_t bsm = (1 << bs_log2) - 1;
  const int32_t runm = (1 << run_log2) - 1;
  const int32_t kStep = (int32_t)blockDim.x * 16;
  for (int32_t m0 = (int32_t)threadIdx.x * 16; m0 < nbytes; m0 += kTileLoads * kStep) {
    Raw<16> x[kTileLoads];
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u) {
      const int32_t m = m0 + u * kStep;
      if (m < nbytes && ((m >> run_log2) & bsm) < rows)
        x[u] = ld<16, kGatherNtLoad>(region + m);
    }
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u) {
      const int32_t m = m0 + u * kStep;
      if (m < nbytes && ((m >> run_log2) & bsm) < rows) {
#pragma unroll
        for (int k = 0; k < 16 / PIECE; ++k) {
          const int32_t mm = m + k * PIECE;
          const int32_t o = (mm >> run_log2) & bsm;
          const int32_t ar = mm >> (run_log2 + bs_log2);
          put_piece<PIECE>(lds + o * pitch + (ar << run_log2) + (mm & runm), x[u], k);
        }
      }
    }
  }
}

// Phase 1 for a RAGGED tile whose rows name different blocks: every piece
// is loaded from its own row's block, ids[o] (< 0: row skipped); `off` is
// the tile's region offset within a block.
template <int PIECE>
__device__ __forceinline__ void stage_tile_rows(const char *src, int64_t s_block, int32_t off,
                                                const int64_t *ids, char *lds, int32_t nbytes,
                                                int32_t run_log2, int32_t bs_log2, int32_t pitch,
                                                int32_t rows) {
  const int32_t bsm = (1 << bs_log2) - 1;
  const int32_t runm = (1 << run_log2) - 1;
  for (int32_t mm = (int32_t)threadIdx.x * PIECE; mm < nbytes; mm += (int32_t)blockDim.x * PIECE) {
    const int32_t o = (mm >> run_log2) & bsm;
    if (o >= rows) continue;
    const int64_t id = ids[o];
    if (id < 0) continue;
    const int32_t ar = mm >> (run_log2 + bs_log2);
    st<PIECE>(lds + o * pitch + (ar << run_log2) + (mm & runm),
              ld<PIECE, kGatherNtLoad>(src + id * s_block + off + mm));
  }
}

// Phase 1 for runs of `run` bytes, a multiple of 16 but not a power of two:
// each 16-byte chunk lies inside one run, whose index m / run (by
// multiply-high) gives the row (index % bs) and the run's place in the row.
__device__ __forceinline__ void stage_tile_odd(const char *region, char *lds, int32_t nbytes,
                                               int32_t run, uint32_t run_magic, int32_t bs_log2,
                                               int32_t pitch, int32_t rows) {
  const uint32_t bsm = (1u << bs_log2) - 1;
  const int32_t kStep = (int32_t)blockDim.x * 16;
  for (int32_t m0 = (int32_t)threadIdx.x * 16; m0 < nbytes; m0 += kTileLoads * kStep) {
    Raw<16> x[kTileLoads];
    int32_t at[kTileLoads];
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u) {
      const int32_t m = m0 + u * kStep;
      at[u] = -1;
      if (m < nbytes) {
        const uint32_t q = div_magic((uint32_t)m, run_magic);
        const int32_t o = (int32_t)(q & bsm);
        if (o < rows) {
          at[u] = o * pitch + (int32_t)(q >> bs_log2) * run + (m - (int32_t)q * run);
          x[u] = ld<16, kGatherNtLoad>(region + m);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kTileLoads; ++u)
      if (at[u] >= 0) st<16>(lds + at[u], x[u]);
  }
}

// stage_tile_rows for runs of `run` bytes (a multiple of 16, not a power of
// two): 16-byte pieces, each inside one run.
__device__ __forceinline__ void stage_tile_rows_odd(const char *src, int64_t s_block, int32_t off,
                                                    const int64_t *ids, char *lds, int32_t nbytes,
                                                    int32_t run, uint32_t run_magic,
                                                    int32_t bs_log2, int32_t pitch, int32_t rows) {
  const uint32_t bsm = (1u << bs_log2) - 1;
  for (int32_t mm = (int32_t)threadIdx.x * 16; mm < nbytes; mm += (int32_t)blockDim.x * 16) {
    const uint32_t q = div_magic((uint32_t)mm, run_magic);
    const int32_t o = (int32_t)(q & bsm);
    if (o >= rows) continue;
    const int64_t id = ids[o];
    if (id < 0) continue;
    st<16>(lds + o * pitch + (int32_t)(q >> bs_log2) * run + (mm - (int32_t)q * run),
           ld<16, kGatherNtLoad>(src + id * s_block + off + mm));
  }
}

// Phase 2: chunk c of row r covers cache bytes [c * kSrc, (c + 1) * kSrc)
// of the tile, i.e. row elements e0 + c * G.  ODD: the tile width is not a
// power of two, so r = u / cpr by multiply-high.
template <class Op, int FMT, bool ODD>
__device__ __forceinline__ void unstage_gather_tile(const TileArgs &a, const TileTensor &tt,
                                                    const char *lds, char *out, int32_t rows,
                                                    int32_t tile, int64_t bid, bool mixed,
                                                    const int64_t *s_ids, float uniform) {
  constexpr int kSrcLog2 = Op::kSrc == 16 ? 4 : Op::kSrc == 8 ? 3 : Op::kSrc == 4 ? 2
                           : Op::kSrc == 2 ? 1 : 0;
  const uint32_t hd = (uint32_t)a.head_dim;
  const int32_t cpr_log2 = a.tw_log2 - kSrcLog2;
  const int32_t total = ODD ? rows * a.cpr : rows << cpr_log2;
  const uint32_t e0 = ((uint32_t)tile * (uint32_t)a.tw) >> a.cache_es_log2;
  const int32_t cm = (1 << cpr_log2) - 1;
  for (int32_t u0 = (int32_t)threadIdx.x; u0 < total; u0 += kTileLoads * (int32_t)blockDim.x) {
    Raw<Op::kSrc> x[kTileLoads];
    int32_t rr[kTileLoads], cc[kTileLoads];
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int32_t u = u0 + k * (int32_t)blockDim.x;
      if constexpr (ODD) {
        rr[k] = (int32_t)div_magic((uint32_t)u, a.cpr_magic);
        cc[k] = u - rr[k] * a.cpr;
      } else {
        rr[k] = u >> cpr_log2;
        cc[k] = u & cm;
      }
      if (u < total) x[k] = ld<Op::kSrc>(lds + rr[k] * a.pitch + (cc[k] << kSrcLog2));
    }
#pragma unroll
    for (int k = 0; k < kTileLoads; ++k) {
      const int32_t u = u0 + k * (int32_t)blockDim.x;
      if (u < total) {
        const int32_t r = rr[k];
        int64_t rb = bid;
        if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
          if (mixed) {
            rb = s_ids[r];
            if (rb < 0) continue;
          }
        }
        const uint32_t e = e0 + ((uint32_t)(cc[k] << kSrcLog2) >> a.cache_es_log2);
        float sc = uniform;
        if constexpr (Op::kScaled) sc = scale_at(tt.sc, uniform, rb, e, hd);
        st<Op::kDst, kGatherNtStore>(out + (int64_t)r * a.out_row_bytes +
                                         ((int64_t)e << a.io_es_log2),
                                     Op::apply(x[k], sc));
      }
    }
  }
}

// I64: dtype of seq_lens and of PACKED / RAGGED block ids; P64: RAGGED's
// indptr dtype.
template <class Op, int FMT, bool I64, bool P64>
__global__ __launch_bounds__(kBlockThreads) void gather_tiles_kernel(TileArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ int64_t s_ids[kTileMaxRows];  // RAGGED: block id of each row, -1 if skipped
  __shared__ int32_t s_same;        // RAGGED: every row names block s_ids[0]
  const TileTensor tt = blockIdx.y ? a.t[1] : a.t[0];
  const uint32_t wg = blockIdx.x;
  const uint32_t per_seq = (uint32_t)a.blocks_per_seq * (uint32_t)a.tiles;
  const uint32_t su = wg / per_seq;
  const uint32_t w = wg - su * per_seq;
  const uint32_t lbu = w / (uint32_t)a.tiles;
  const int32_t tile = (int32_t)(w - lbu * (uint32_t)a.tiles);
  const int32_t lb = (int32_t)lbu;
  const int64_t s = su;
  const int64_t t0 = (int64_t)lb << a.bs_log2;
  const int32_t bs = 1 << a.bs_log2;
  const int64_t seq_len = load_idx<I64>(a.seq_lens, s);
  int64_t n = seq_len < a.max_seq_len ? seq_len : (int64_t)a.max_seq_len;
  int64_t bid;
  const char *blk = nullptr;
  bool mixed = false;  // RAGGED tile whose rows name different blocks
  if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
    // row t is token start + t (KVX_SPEC.md:107-114), at offset t % bs
    const int64_t start = load_idx<P64>(a.indptr, s);
    const int64_t end = load_idx<P64>(a.indptr, s + 1);
    int64_t cnt = end - start;
    const int64_t left = a.table_count - start;  // entries the table holds
    cnt = left < cnt ? left : cnt;
    n = cnt < n ? cnt : n;
    if (start < 0) n = 0;
    if (t0 >= n) return;
    const int64_t rem = n - t0;
    const int32_t rws = rem < bs ? (int32_t)rem : bs;
    if (bs <= kWave) {
      // one wave loads the ids, one per lane, and a ballot compares them
      if (threadIdx.x < kWave) {
        const int lane = (int)threadIdx.x;
        int64_t id = -1;
        if (lane < rws) {
          id = load_idx<I64>(a.table, start + t0 + lane);
          if (id < 0 || id >= a.num_blocks) id = -1;
          s_ids[lane] = id;
        }
        const int64_t first =
            (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(id >> 32))
                       << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)id));
        const uint64_t same = __ballot(lane >= rws || id == first);
        if (lane == 0) s_same = same == ~0ull;
      }
      __syncthreads();
      bid = s_ids[0];
      mixed = !s_same;
    } else {
      // blocks of more rows than a wave has lanes: every thread loads ids,
      // then a barrier that ORs the threads' mismatches with row 0's id
      for (int32_t r = (int32_t)threadIdx.x; r < rws; r += (int32_t)blockDim.x) {
        int64_t id = load_idx<I64>(a.table, start + t0 + r);
        if (id < 0 || id >= a.num_blocks) id = -1;
        s_ids[r] = id;
      }
      __syncthreads();
      bid = s_ids[0];
      int differs = 0;
      for (int32_t r = (int32_t)threadIdx.x; r < rws; r += (int32_t)blockDim.x)
        differs |= s_ids[r] != bid;
      mixed = __syncthreads_or(differs) != 0;
    }
    if (!mixed) {
      if (bid < 0) return;  // every row skipped
      blk = tt.src + bid * tt.s_block;
    }
  } else {
    if (lb >= a.max_blocks_per_seq) return;
    if constexpr (FMT == KVX_BLOCK_TABLE_KV_OFFSETS) {
      // table [seq, beam = 1, {K, V}, max_blocks_per_seq] of KVCacheIndex
      const uint32_t ent = reinterpret_cast<const uint32_t *>(
          a.table)[(s * 2 + blockIdx.y) * a.max_blocks_per_seq + lb];
      const char *pool = (ent >> 31) ? a.pool[1] : a.pool[0];
      bid = ent & 0x7FFFFFFFu;
      if (pool == nullptr || bid >= ((ent >> 31) ? a.pool_blocks[1] : a.pool_blocks[0])) return;
      blk = pool + bid * a.bytes_per_block;
    } else {
      bid = load_idx<I64>(a.table, s * a.max_blocks_per_seq + lb);
      if (bid < 0 || bid >= a.num_blocks) return;
      blk = tt.src + bid * tt.s_block;
    }
    if (t0 >= n) return;
  }
  const int64_t rem = n - t0;
  const int32_t rows = rem < bs ? (int32_t)rem : bs;
  float uniform = 1.0f;
  if constexpr (Op::kScaled) uniform = tt.sc.p[0];

  const int32_t region = a.tw << a.bs_log2;
  char *out = tt.dst + (s * a.max_seq_len + t0) * a.out_row_bytes;
  const uint32_t hd = (uint32_t)a.head_dim;
  const uint32_t re = (uint32_t)a.row_elems;

  if (tt.run_log2 < 0) {
    // Row-major block: rows are contiguous in the cache and in the output.
    const int32_t lo = tile * region;
    const int64_t valid = ((int64_t)rows << a.cache_es_log2) * re;
    const int32_t hi = (int32_t)(lo + region < valid ? lo + region : valid);
    for (int32_t m = lo + (int32_t)threadIdx.x * Op::kSrc; m < hi; m += (int32_t)blockDim.x * Op::kSrc) {
      const uint32_t e = (uint32_t)m >> a.cache_es_log2;
      int64_t rb = bid;
      const char *b = blk;
      if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
        if (mixed) {
          rb = s_ids[e / re];
          if (rb < 0) continue;
          b = tt.src + rb * tt.s_block;
        }
      }
      float sc = uniform;
      if constexpr (Op::kScaled) sc = scale_in_rows(tt.sc, uniform, rb, e, re, hd);
      st<Op::kDst, kGatherNtStore>(out + ((int64_t)e << a.io_es_log2),
                                   Op::apply(ld<Op::kSrc, kGatherNtLoad>(b + m), sc));
    }
    return;
  }

  if (mixed) {
    const int32_t off = tile * region;
    if (tt.run_log2 == kRunOdd)
      stage_tile_rows_odd(tt.src, tt.s_block, off, s_ids, lds, region, tt.run_bytes, tt.run_magic,
                          a.bs_log2, a.pitch, rows);
    else switch (tt.run_log2) {
      case 0: stage_tile_rows<1>(tt.src, tt.s_block, off, s_ids, lds, region, 0, a.bs_log2, a.pitch, rows); break;
      case 1: stage_tile_rows<2>(tt.src, tt.s_block, off, s_ids, lds, region, 1, a.bs_log2, a.pitch, rows); break;
      case 2: stage_tile_rows<4>(tt.src, tt.s_block, off, s_ids, lds, region, 2, a.bs_log2, a.pitch, rows); break;
      case 3: stage_tile_rows<8>(tt.src, tt.s_block, off, s_ids, lds, region, 3, a.bs_log2, a.pitch, rows); break;
      default: stage_tile_rows<16>(tt.src, tt.s_block, off, s_ids, lds, region, tt.run_log2, a.bs_log2, a.pitch, rows); break;
    }
  } else {
    const char *src = blk + (int64_t)tile * region;
    if (tt.run_log2 == kRunOdd)
      stage_tile_odd(src, lds, region, tt.run_bytes, tt.run_magic, a.bs_log2, a.pitch, rows);
    else switch (tt.run_log2) {
      case 0: stage_tile<1>(src, lds, region, 0, a.bs_log2, a.pitch, rows); break;
      case 1: stage_tile<2>(src, lds, region, 1, a.bs_log2, a.pitch, rows); break;
      case 2: stage_tile<4>(src, lds, region, 2, a.bs_log2, a.pitch, rows); break;
      case 3: stage_tile<8>(src, lds, region, 3, a.bs_log2, a.pitch, rows); break;
      default: stage_tile<16>(src, lds, region, tt.run_log2, a.bs_log2, a.pitch, rows); break;
    }
  }
  __syncthreads();
  if (a.tw_log2 < 0)
    unstage_gather_tile<Op, FMT, true>(a, tt, lds, out, rows, tile, bid, mixed, s_ids, uniform);
  else
    unstage_gather_tile<Op, FMT, false>(a, tt, lds, out, rows, tile, bid, mixed, s_ids, uniform);
}

// Rows of sequence s that exist (t < n) for an indexed-format workgroup,
// plus RAGGED's first token index; false when the workgroup's rows
// [t0, ...) are all past the end.  seq_len, the indptr pair and (TILE) the
// KV_OFFSETS entries ek / ev of K and V at logical block lb are independent
// loads, issued together.
template <int FMT, bool I64, bool P64, bool TILE = false>
__device__ __forceinline__ bool indexed_extent(const GatherArgs &a, int64_t s, int64_t t0,
                                               int64_t &n, int64_t &start, uint32_t lb = 0,
                                               uint32_t *ek = nullptr, uint32_t *ev = nullptr) {
  const int64_t seq_len = load_idx<I64>(a.seq_lens, s);
  int64_t end = 0;
  start = 0;
  if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
    start = load_idx<P64>(a.indptr, s);
    end = load_idx<P64>(a.indptr, s + 1);
  }
  if constexpr (TILE) {
    const int32_t *row =
        reinterpret_cast<const int32_t *>(a.table) + s * 2 * (int64_t)a.max_blocks_per_seq;
    *ek = (uint32_t)row[lb];
    *ev = (uint32_t)row[a.max_blocks_per_seq + lb];
    // consumed here, so the loads are not sunk below the length test
    asm volatile("" ::"s"(*ek), "s"(*ev));
  }
  // Keep the loads above ahead of their uses, so that they are in flight
  // together.
  __builtin_amdgcn_sched_barrier(0);
  n = seq_len < a.max_seq_len ? seq_len : (int64_t)a.max_seq_len;
  if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
    int64_t cnt = end - start;
    const int64_t left = a.table_count - start;  // entries the table holds
    cnt = left < cnt ? left : cnt;
    n = cnt < n ? cnt : n;
    if (start < 0) n = 0;
  } else {
    const int64_t cap = (int64_t)a.max_blocks_per_seq * a.block_size;
    n = cap < n ? cap : n;
  }
  return t0 < n;
}

// RAGGED and KV_OFFSETS gathers (KVX_SPEC.md:99-122).  A workgroup covers
// `rows_per_wg` output rows of one sequence; every row resolves its own
// source, so K and V rows come from wherever the table points:
//   RAGGED      row t of sequence s is token i = indptr[s] + t, valid for
//               t < indptr[s+1] - indptr[s]; block id = indices[i] (skipped
//               when < 0 or >= num_blocks), block offset = t % block_size.
//   KV_OFFSETS  table [seq, beam = 1, {K, V}, max_blocks_per_seq] of
//               KVCacheIndex values: bit 31 selects the secondary pool,
//               bits 0..30 are the block index (skipped when >= num_blocks or
//               when the selected pool is NULL); block address = pool +
//               index * bytes_per_block, offset t % block_size.  K and V rows
//               are resolved independently.
// Rows t >= min(seq_len, max_seq_len) are untouched, as in the PACKED gather.
template <class Op, int FMT, bool I64, bool P64>
__global__ __launch_bounds__(kBlockThreads) void gather_indexed_kernel(GatherArgs a) {
  const uint32_t wg = blockIdx.x;
  const uint32_t su = wg / (uint32_t)a.blocks_per_seq;
  const int64_t s = su;
  const int64_t t0 = (int64_t)(wg - su * (uint32_t)a.blocks_per_seq) * a.rows_per_wg;
  int64_t n;
  int64_t start;
  if (!indexed_extent<FMT, I64, P64>(a, s, t0, n, start)) return;

  float ks = 1.0f;  // per-tensor values; indexed scales are looked up per chunk
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int lpt = 1 << a.lpt_log2;
  const int tpw = kWave >> a.lpt_log2;
  const int sub = lane >> a.lpt_log2;
  const int l = lane & (lpt - 1);

  int64_t koff[kMaxChunksPerLane];
  int64_t voff[kMaxChunksPerLane];
  uint32_t hk[kMaxChunksPerLane];  // head of each chunk (indexed scales)
#pragma unroll
  for (int k = 0; k < kMaxChunksPerLane; ++k) {
    const int c = l + k * lpt;
    koff[k] = 0;
    voff[k] = 0;
    hk[k] = 0;
    if (c < a.nchunks) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      koff[k] = chunk_off(a.gk, e, (uint32_t)a.head_dim);
      voff[k] = chunk_off(a.gv, e, (uint32_t)a.head_dim);
      if constexpr (Op::kScaled) hk[k] = e / (uint32_t)a.head_dim;
    }
  }

  for (int r = wave * tpw + sub; r < a.rows_per_wg; r += kWavesPerBlock * tpw) {
    const int64_t t = t0 + r;
    if (t >= n) break;
    const char *rk = nullptr;
    const char *rv = nullptr;
    int64_t sb = 0;  // block of block-indexed scales (RAGGED; KV_OFFSETS has none)
    if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
      const int64_t bid = load_idx<I64>(a.table, start + t);
      sb = bid;
      if (bid >= 0 && bid < a.num_blocks) {
        const int64_t o = t % a.block_size;
        rk = a.src_k + bid * a.gk.s_block + o * a.gk.s_off;
        rv = a.src_v + bid * a.gv.s_block + o * a.gv.s_off;
      }
    } else {
      const int64_t lb = t / a.block_size;
      const int64_t o = t - lb * a.block_size;
      const int32_t *row = reinterpret_cast<const int32_t *>(a.table) +
                           s * 2 * (int64_t)a.max_blocks_per_seq;
      const uint32_t kidx = (uint32_t)row[lb];
      const uint32_t vidx = (uint32_t)row[a.max_blocks_per_seq + lb];
      const char *kp = (kidx >> 31) ? a.pool[1] : a.pool[0];
      const char *vp = (vidx >> 31) ? a.pool[1] : a.pool[0];
      const int64_t kb = kidx & 0x7FFFFFFFu;
      const int64_t vb = vidx & 0x7FFFFFFFu;
      if (kp != nullptr && kb < ((kidx >> 31) ? a.pool_blocks[1] : a.pool_blocks[0]))
        rk = kp + kb * a.bytes_per_block + o * a.gk.s_off;
      if (vp != nullptr && vb < ((vidx >> 31) ? a.pool_blocks[1] : a.pool_blocks[0]))
        rv = vp + vb * a.bytes_per_block + o * a.gv.s_off;
    }
    char *wk = a.dst_k + (s * a.max_seq_len + t) * a.out_row_bytes;
    char *wv = a.dst_v + (s * a.max_seq_len + t) * a.out_row_bytes;
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
      const int c = l + k * lpt;
      if (c < a.nchunks) {
        if (rk != nullptr)
          st<Op::kDst>(wk + (int64_t)c * Op::kDst,
                       Op::apply(ld<Op::kSrc>(rk + koff[k]), scale_of(a.ksc, ks, sb, hk[k])));
        if (rv != nullptr)
          st<Op::kDst>(wv + (int64_t)c * Op::kDst,
                       Op::apply(ld<Op::kSrc>(rv + voff[k]), scale_of(a.vsc, vs, sb, hk[k])));
      }
    }
    for (int c = l + kMaxChunksPerLane * lpt; c < a.nchunks; c += lpt) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      const uint32_t h = e / (uint32_t)a.head_dim;
      if (rk != nullptr)
        st<Op::kDst>(wk + (int64_t)c * Op::kDst,
                     Op::apply(ld<Op::kSrc>(rk + chunk_off(a.gk, e, (uint32_t)a.head_dim)),
                               scale_of(a.ksc, ks, sb, h)));
      if (rv != nullptr)
        st<Op::kDst>(wv + (int64_t)c * Op::kDst,
                     Op::apply(ld<Op::kSrc>(rv + chunk_off(a.gv, e, (uint32_t)a.head_dim)),
                               scale_of(a.vsc, vs, sb, h)));
    }
  }
}

// Cache address of row t (sequence s) of K (v = false) or V, or nullptr
// when the table skips it.  The in-block offset of the row is o * s_off.
template <int FMT, bool I64>
__device__ __forceinline__ const char *indexed_row(const GatherArgs &a, bool v, int64_t s,
                                                   int64_t start, int64_t t, int64_t *blk) {
  const uint32_t tu = (uint32_t)t;  // t < max_seq_len < 2^31
  uint32_t lb;
  uint32_t o;
  if (a.bs_log2 >= 0) {
    lb = tu >> a.bs_log2;
    o = tu & ((1u << a.bs_log2) - 1u);
  } else {
    lb = tu / (uint32_t)a.block_size;
    o = tu - lb * (uint32_t)a.block_size;
  }
  const GeomBytes &g = v ? a.gv : a.gk;
  if constexpr (FMT == KVX_BLOCK_TABLE_RAGGED) {
    const int64_t bid = load_idx<I64>(a.table, start + t);
    *blk = bid;
    if (bid < 0 || bid >= a.num_blocks) return nullptr;
    return (v ? a.src_v : a.src_k) + bid * g.s_block + (int64_t)o * g.s_off;
  } else {
    const uint32_t e = (uint32_t)reinterpret_cast<const int32_t *>(
        a.table)[(s * 2 + (v ? 1 : 0)) * (int64_t)a.max_blocks_per_seq + lb];
    const char *pool = (e >> 31) ? a.pool[1] : a.pool[0];
    const int64_t idx = e & 0x7FFFFFFFu;
    if (pool == nullptr || idx >= ((e >> 31) ? a.pool_blocks[1] : a.pool_blocks[0])) return nullptr;
    return pool + idx * a.bytes_per_block + (int64_t)o * g.s_off;
  }
}

// RAGGED / KV_OFFSETS gather when every cache row is H * D contiguous
// elements (NHD with dense heads, any block / offset strides): the
// workgroup's rows x chunks of K, then of V, are spread over all threads as
// in gather_flat_kernel, and each thread resolves the source row of its own
// chunk (threads of one row load the same table entry).
// Threads per workgroup of gather_indexed_flat_kernel (see
// kRaggedCopyThreads).
template <class Op, int FMT>
constexpr int indexed_flat_threads() {
  return FMT == KVX_BLOCK_TABLE_RAGGED && !Op::kScaled ? kRaggedCopyThreads : kBlockThreads;
}

// Threads per workgroup of the KV_OFFSETS gather with per-tile table
// entries: enough for one pass of kIndexedUnroll chunks per thread over
// the tile's K and V chunks, a power of two from kWave to kBlockThreads.
inline int offsets_tile_threads(const GatherArgs &a) {
  const int64_t per_pass = 2 * (int64_t)a.rows_per_wg * a.nchunks / kIndexedUnroll;
  int t = kWave;
  while (t < kBlockThreads && t < per_pass) t *= 2;
  return t;
}

// TILE (KV_OFFSETS only): table entries per workgroup tile, and as many
// threads as the launch gives (at most kBlockThreads).
template <class Op, int FMT, bool I64, bool P64,
          bool TILE = FMT == KVX_BLOCK_TABLE_KV_OFFSETS && Op::kScaled>
__global__ __launch_bounds__((indexed_flat_threads<Op, FMT>())) void gather_indexed_flat_kernel(
    GatherArgs a) {
  constexpr bool kTile = FMT == KVX_BLOCK_TABLE_KV_OFFSETS && TILE;
  const uint32_t nt = kTile ? blockDim.x : (uint32_t)indexed_flat_threads<Op, FMT>();
  const uint32_t wg = blockIdx.x;
  const uint32_t su = wg / (uint32_t)a.blocks_per_seq;
  const int64_t s = su;
  const int64_t t0 = (int64_t)(wg - su * (uint32_t)a.blocks_per_seq) * a.rows_per_wg;
  // KV_OFFSETS tiles lie inside one block (rows_per_wg divides block_size).
  // kTile: the tile's K and V table entries are two scalar loads, issued with
  // the seq_len load; otherwise every chunk loads its own entry.
  uint32_t ek = 0;
  uint32_t ev = 0;
  uint32_t lb = 0;
  if constexpr (kTile) {
    lb = (uint32_t)t0 >> a.bs_log2;
    if (lb >= (uint32_t)a.max_blocks_per_seq) return;
  }
  int64_t n;
  int64_t start;
  if (!indexed_extent<FMT, I64, P64, kTile>(a, s, t0, n, start, lb, &ek, &ev)) return;
  const char *tk = nullptr;
  const char *tv = nullptr;
  if constexpr (kTile) {
    const int64_t o0 = t0 & ((1 << a.bs_log2) - 1);
    const char *pk = (ek >> 31) ? a.pool[1] : a.pool[0];
    const char *pv = (ev >> 31) ? a.pool[1] : a.pool[0];
    const int64_t kb = ek & 0x7FFFFFFFu;
    const int64_t vb = ev & 0x7FFFFFFFu;
    if (pk != nullptr && kb < ((ek >> 31) ? a.pool_blocks[1] : a.pool_blocks[0]))
      tk = pk + kb * a.bytes_per_block + o0 * a.gk.s_off;
    if (pv != nullptr && vb < ((ev >> 31) ? a.pool_blocks[1] : a.pool_blocks[0]))
      tv = pv + vb * a.bytes_per_block + o0 * a.gv.s_off;
    if (tk == nullptr && tv == nullptr) return;
  }
  const int64_t rem = n - t0;
  const int32_t rows = rem < a.rows_per_wg ? (int32_t)rem : a.rows_per_wg;
  float ks = 1.0f;  // per-tensor values; indexed scales are looked up per chunk
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }
  const uint32_t total = (uint32_t)rows * (uint32_t)a.nchunks;
  const uint32_t both = 2 * total;
  const int64_t out0 = (s * a.max_seq_len + t0) * a.out_row_bytes;
  // Chunk f: K for f < total, V above; row r = index / nchunks.  Each
  // pass resolves kIndexedUnroll chunks' rows, then loads them all, then
  // stores them, so the table and data latencies overlap across chunks.
  for (uint32_t base = threadIdx.x; base < both; base += kIndexedUnroll * nt) {
    const char *src[kIndexedUnroll];
    char *dst[kIndexedUnroll];
    bool isv[kIndexedUnroll];
    float sc[kIndexedUnroll];
#pragma unroll
    for (int u = 0; u < kIndexedUnroll; ++u) {
      const uint32_t f = base + u * nt;
      src[u] = nullptr;
      dst[u] = nullptr;
      isv[u] = f >= total;
      sc[u] = isv[u] ? vs : ks;
      if (f < both) {
        const uint32_t gi = f - (isv[u] ? total : 0u);
        const uint32_t r = row_of_chunk(a, gi);
        const uint32_t c = gi - r * (uint32_t)a.nchunks;
        if constexpr (kTile) {
          const char *base = isv[u] ? tv : tk;
          src[u] = base == nullptr ? nullptr
                                   : base + (int64_t)r * (isv[u] ? a.gv.s_off : a.gk.s_off);
        }
        int64_t blk = 0;  // RAGGED block for block-indexed scales (KV_OFFSETS: none)
        if constexpr (!kTile) src[u] = indexed_row<FMT, I64>(a, isv[u], s, start, t0 + r, &blk);
        if (src[u] != nullptr) {
          src[u] += (int64_t)c * Op::kSrc;
          dst[u] = (isv[u] ? a.dst_v : a.dst_k) + out0 + (int64_t)r * a.out_row_bytes +
                   (int64_t)c * Op::kDst;
          if constexpr (Op::kScaled) {
            const ScaleRef &sr = isv[u] ? a.vsc : a.ksc;
            if (sr.indexed)
              sc[u] = sr.p[blk * sr.s_block +
                           (int64_t)(c * (uint32_t)a.chunk_elems / (uint32_t)a.head_dim) *
                               sr.s_head];
          }
        }
      }
    }
    Raw<Op::kSrc> x[kIndexedUnroll];
#pragma unroll
    for (int u = 0; u < kIndexedUnroll; ++u) {
      if (src[u] != nullptr) x[u] = ld<Op::kSrc, kGatherNtLoad>(src[u]);
    }
#pragma unroll
    for (int u = 0; u < kIndexedUnroll; ++u) {
      if (src[u] != nullptr)
        st<Op::kDst, kGatherNtStore>(dst[u], Op::apply(x[u], sc[u]));
    }
  }
}

// RAGGED gather of caches whose block rows are contiguous (canonical NHD
// blocks): a workgroup of kFlatThreads threads covers rows_per_wg = R
// consecutive output rows t0 .. t0 + R - 1 of one sequence, with R a
// divisor of block_size and t0 a multiple of R, so the rows sit at offsets
// t0 % bs .. t0 % bs + R - 1 of their blocks (KVX_SPEC.md:107-114: row t
// is token indptr[s] + t at offset t % bs).  After seq_len and the indptr
// pair, each wave loads the R block ids itself, one lane per row; a ballot
// tells whether they name one valid block, which is the usual case (a
// RAGGED table lists each block's tokens in order).  The tile is then one
// contiguous run of that block, copied as in gather_flat_kernel; otherwise
// every chunk takes its row's id from the lane that loaded it, and rows
// whose id is < 0 or >= num_blocks are skipped.  No chunk loads an index of
// its own.
// One tile (rows t0 .. t0 + rows_per_wg - 1 of sequence s) of
// gather_ragged_tile_kernel; false when the tile lies past the sequence's
// end, and so does every later one.
template <class Op, bool I64, bool P64>
__device__ __forceinline__ bool ragged_tile_unit(const GatherArgs &a, int64_t s, int64_t t0) {
  constexpr int U = Op::kScaled ? kFlatUnrollDequant : kFlatUnroll;
  int64_t n;
  int64_t start;
  if (!indexed_extent<KVX_BLOCK_TABLE_RAGGED, I64, P64>(a, s, t0, n, start)) return false;
  const int64_t rem = n - t0;
  const int32_t rows = rem < a.rows_per_wg ? (int32_t)rem : a.rows_per_wg;  // <= 64
  const int lane = (int)(threadIdx.x & (kWave - 1));
  int32_t id = -1;  // block ids are < num_blocks < 2^31
  if (lane < rows) {
    const int64_t b = load_idx<I64>(a.table, start + t0 + lane);
    id = (b < 0 || b >= a.num_blocks) ? -1 : (int32_t)b;
  }
  const int32_t first = __builtin_amdgcn_readfirstlane(id);
  const bool one = __ballot(lane < rows && id != first) == 0 && first >= 0;
  const uint32_t tu = (uint32_t)t0;  // t0 < max_seq_len < 2^31
  const uint32_t o0 = a.bs_log2 >= 0 ? tu & ((1u << a.bs_log2) - 1u) : tu % (uint32_t)a.block_size;
  float ks = 1.0f;  // per-tensor values; indexed scales are looked up per chunk
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = a.ksc.p[0];
    vs = a.vsc.p[0];
  }
  const uint32_t total = (uint32_t)rows * (uint32_t)a.nchunks;
  const int64_t out0 = (s * a.max_seq_len + t0) * a.out_row_bytes;
  if (one) {
    flat_copy<Op>(a, a.src_k + first * a.gk.s_block + o0 * a.gk.s_off,
                  a.src_v + first * a.gv.s_block + o0 * a.gv.s_off, a.dst_k + out0,
                  a.dst_v + out0, total, ks, vs, first, 0);
    return true;
  }
  // Rows in several blocks (or skipped): chunk f is K for f < total, V
  // above; row r = index / nchunks takes its id from lane r.  The
  // loop trip count is the same for every thread, so every lane joins each
  // shuffle.
  const uint32_t both = 2 * total;
  for (uint32_t base = 0; base < both; base += U * kFlatThreads) {
    const char *src[U];
    char *dst[U];
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t f = base + u * kFlatThreads + threadIdx.x;
      const bool v = f >= total;
      const uint32_t gi = f - (v ? total : 0u);
      const uint32_t r = f < both ? row_of_chunk(a, gi) : 0u;
      const int32_t rid = __shfl(id, (int)r);
      src[u] = nullptr;
      dst[u] = nullptr;
      sc[u] = v ? vs : ks;
      if (f < both && rid >= 0) {
        const GeomBytes &g = v ? a.gv : a.gk;
        const uint32_t c = gi - r * (uint32_t)a.nchunks;
        src[u] = (v ? a.src_v : a.src_k) + rid * g.s_block + (int64_t)(o0 + r) * g.s_off +
                 (int64_t)c * Op::kSrc;
        dst[u] = (v ? a.dst_v : a.dst_k) + out0 + (int64_t)r * a.out_row_bytes +
                 (int64_t)c * Op::kDst;
        if constexpr (Op::kScaled) sc[u] = run_scale(a, v, ks, vs, rid, c);
      }
    }
    Raw<Op::kSrc> x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (src[u] != nullptr) x[u] = ld<Op::kSrc, kGatherNtLoad>(src[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (src[u] != nullptr) st<Op::kDst, kGatherNtStore>(dst[u], Op::apply(x[u], sc[u]));
    }
  }
  return true;
}

// Workgroup w of sequence s takes tile w and, with FOLD = 2, tile w + J (J =
// blocks_per_seq) when that is below units_per_seq.  FOLD is a template
// parameter: a loop over a run-time count around the tile body measured
// 3-17% slower than one tile per workgroup.
template <class Op, bool I64, bool P64, int FOLD>
__global__ __launch_bounds__(kFlatThreads) void gather_ragged_tile_kernel(GatherArgs a) {
  const uint32_t wg = blockIdx.x;
  const uint32_t su = wg / (uint32_t)a.blocks_per_seq;
  const int64_t w = wg - su * (uint32_t)a.blocks_per_seq;
  if (!ragged_tile_unit<Op, I64, P64>(a, su, w * a.rows_per_wg)) return;
  if constexpr (FOLD > 1) {
    const int64_t u = w + a.blocks_per_seq;
    if (u < a.units_per_seq) ragged_tile_unit<Op, I64, P64>(a, su, u * a.rows_per_wg);
  }
}

// ---------------------------------------------------------------------------
// Launch templates.

// How a write launches: the per-token kernel, or the tiled block kernel
// (one workgroup per tile of a group's block, per tensor) with its LDS
// tile size.
struct WriteLaunch {
  int grid;
  int64_t flat_grid;  // write_flat_kernel's workgroups, 0 when it does not apply
  bool tiles;
  WriteTileArgs wt;
  int64_t tile_grid;
  uint32_t tile_lds;
};

// The tiled write moves 16-byte cache chunks: a copy of 16 bytes, or a
// quantization of 8 elements.
template <class Op>
struct TileOpOf;
template <int B>
struct TileOpOf<CopyOp<B>> {
  using type = CopyOp<16>;
};
template <int G, int IO, int F8>
struct TileOpOf<QuantOp<G, IO, F8>> {
  using type = QuantOp<8, IO, F8>;
};

template <class Op>
void launch_write_op(const WriteArgs &a, const WriteLaunch &w, hipStream_t s) {
  if (w.tiles) {
    using TOp = typename TileOpOf<Op>::type;
    const dim3 g((uint32_t)w.tile_grid, 2);
    const bool odd = w.wt.tw_log2 < 0;  // tile width not a power of two
    if constexpr (Op::kScaled) {
      if (a.ksc.indexed || a.vsc.indexed) {
        if (odd)
          hipLaunchKernelGGL((write_tiles_kernel<TOp, Op, true, true>), g, dim3(w.wt.threads),
                             w.tile_lds, s, a, w.wt);
        else
          hipLaunchKernelGGL((write_tiles_kernel<TOp, Op, true, false>), g, dim3(w.wt.threads),
                             w.tile_lds, s, a, w.wt);
        return;
      }
    }
    if (odd)
      hipLaunchKernelGGL((write_tiles_kernel<TOp, Op, false, true>), g, dim3(w.wt.threads),
                         w.tile_lds, s, a, w.wt);
    else
      hipLaunchKernelGGL((write_tiles_kernel<TOp, Op, false, false>), g, dim3(w.wt.threads),
                         w.tile_lds, s, a, w.wt);
  } else if (w.flat_grid > 0) {
    const dim3 g((uint32_t)w.flat_grid), b(kFlatThreads);
    if (a.nchunks_log2 >= 6) {
      if (a.slot_is64) {
        hipLaunchKernelGGL((write_flat_kernel<Op, true, true>), g, b, 0, s, a);
      } else {
        hipLaunchKernelGGL((write_flat_kernel<Op, false, true>), g, b, 0, s, a);
      }
    } else if (a.slot_is64) {
      hipLaunchKernelGGL((write_flat_kernel<Op, true, false>), g, b, 0, s, a);
    } else {
      hipLaunchKernelGGL((write_flat_kernel<Op, false, false>), g, b, 0, s, a);
    }
  } else {
    hipLaunchKernelGGL(write_kernel<Op>, dim3(w.grid), dim3(kBlockThreads), 0, s, a);
  }
}

// I64: dtype of seq_lens (and of PACKED / RAGGED block ids, which share it);
// P64: dtype of RAGGED's indptr.
template <class Op, bool I64, bool P64>
void launch_gather_typed(const GatherArgs &a, int64_t grid, hipStream_t s) {
  const dim3 g((uint32_t)grid);
  const dim3 b(kBlockThreads);
  if (a.format == KVX_BLOCK_TABLE_RAGGED) {
    if (a.ragged_tile) {
      if (a.fold_log2 > 0)
        hipLaunchKernelGGL((gather_ragged_tile_kernel<Op, I64, P64, 2>), g, dim3(kFlatThreads),
                           0, s, a);
      else
        hipLaunchKernelGGL((gather_ragged_tile_kernel<Op, I64, P64, 1>), g, dim3(kFlatThreads),
                           0, s, a);
    } else if (a.flat) {
      hipLaunchKernelGGL((gather_indexed_flat_kernel<Op, KVX_BLOCK_TABLE_RAGGED, I64, P64>), g,
                         dim3(indexed_flat_threads<Op, KVX_BLOCK_TABLE_RAGGED>()), 0, s, a);
    } else {
      hipLaunchKernelGGL((gather_indexed_kernel<Op, KVX_BLOCK_TABLE_RAGGED, I64, P64>), g, b, 0,
                         s, a);
    }
  } else if constexpr (!P64) {
    if (a.format == KVX_BLOCK_TABLE_KV_OFFSETS) {
      if (a.flat && !Op::kScaled &&
          ((int64_t)a.nchunks * Op::kSrc <= kOffsetsTileCopyRow || a.nchunks_log2 < 0)) {
        hipLaunchKernelGGL(
            (gather_indexed_flat_kernel<Op, KVX_BLOCK_TABLE_KV_OFFSETS, I64, false, true>), g,
            dim3(offsets_tile_threads(a)), 0, s, a);
      } else if (a.flat) {
        const dim3 bt(Op::kScaled ? offsets_tile_threads(a) : kBlockThreads);
        hipLaunchKernelGGL(
            (gather_indexed_flat_kernel<Op, KVX_BLOCK_TABLE_KV_OFFSETS, I64, false>), g, bt, 0,
            s, a);
      } else {
        hipLaunchKernelGGL((gather_indexed_kernel<Op, KVX_BLOCK_TABLE_KV_OFFSETS, I64, false>),
                           g, b, 0, s, a);
      }
    } else if (a.flat) {
      const uint32_t lds = a.units_per_seq >= kFlatLongUnits ? kFlatLongLds : 0;
      if (a.cph_log2 >= 0)
        hipLaunchKernelGGL((gather_flat_kernel<Op, I64, true>), g, dim3(kFlatThreads), lds, s, a);
      else
        hipLaunchKernelGGL((gather_flat_kernel<Op, I64, false>), g, dim3(kFlatThreads), lds, s,
                           a);
    } else {
      hipLaunchKernelGGL((gather_rows_kernel<Op, I64>), g, b, 0, s, a);
    }
  }
}

template <class Op>
void launch_gather_op(const GatherArgs &a, int64_t grid, hipStream_t s) {
  const bool i64 = a.lens_is64 != 0;  // equals index_is64 for PACKED / RAGGED
  const bool p64 = a.format == KVX_BLOCK_TABLE_RAGGED && a.indptr_is64 != 0;
  if (i64) {
    if (p64) launch_gather_typed<Op, true, true>(a, grid, s);
    else launch_gather_typed<Op, true, false>(a, grid, s);
  } else {
    if (p64) launch_gather_typed<Op, false, true>(a, grid, s);
    else launch_gather_typed<Op, false, false>(a, grid, s);
  }
}

template <class Op, int FMT, bool P64>
void launch_tiles_fmt(const TileArgs &t, bool i64, int64_t grid, uint32_t lds, hipStream_t s) {
  const dim3 g((uint32_t)grid, 2);
  if (i64) {
    hipLaunchKernelGGL((gather_tiles_kernel<Op, FMT, true, P64>), g, dim3(t.threads), lds, s, t);
  } else {
    hipLaunchKernelGGL((gather_tiles_kernel<Op, FMT, false, P64>), g, dim3(t.threads), lds, s, t);
  }
}

template <class Op>
void launch_tiles(const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid, uint32_t lds,
                  hipStream_t s) {
  if (fmt == KVX_BLOCK_TABLE_KV_OFFSETS) {
    launch_tiles_fmt<Op, KVX_BLOCK_TABLE_KV_OFFSETS, false>(t, i64, grid, lds, s);
  } else if (fmt == KVX_BLOCK_TABLE_RAGGED) {
    if (p64) launch_tiles_fmt<Op, KVX_BLOCK_TABLE_RAGGED, true>(t, i64, grid, lds, s);
    else launch_tiles_fmt<Op, KVX_BLOCK_TABLE_RAGGED, false>(t, i64, grid, lds, s);
  } else {
    launch_tiles_fmt<Op, KVX_BLOCK_TABLE_PACKED, false>(t, i64, grid, lds, s);
  }
}

template <int F8>
void launch_tiles_dequant(int io, const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid,
                          uint32_t lds, hipStream_t s) {
  switch (io) {
    case KVX_DTYPE_F32:
      launch_tiles<DequantOp<kDequantChunk, KVX_DTYPE_F32, F8>>(t, fmt, i64, p64, grid, lds,
                                                                    s);
      break;
    case KVX_DTYPE_F16:
      launch_tiles<DequantOp<kDequantChunk, KVX_DTYPE_F16, F8>>(t, fmt, i64, p64, grid, lds,
                                                                    s);
      break;
    default:
      launch_tiles<DequantOp<kDequantChunk, KVX_DTYPE_BF16, F8>>(t, fmt, i64, p64, grid, lds,
                                                                     s);
      break;
  }
}

template <int IO, int F8>
void dispatch_quant(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s) {
  switch (ge) {
    case 8: launch_write_op<QuantOp<8, IO, F8>>(a, w, s); break;
    case 4: launch_write_op<QuantOp<4, IO, F8>>(a, w, s); break;
    case 2: launch_write_op<QuantOp<2, IO, F8>>(a, w, s); break;
    default: launch_write_op<QuantOp<1, IO, F8>>(a, w, s); break;
  }
}

template <int IO, int F8>
void dispatch_dequant(int ge, const GatherArgs &a, int64_t grid,
                      hipStream_t s) {
  switch (ge) {
    case 16: launch_gather_op<DequantOp<16, IO, F8>>(a, grid, s); break;
    case 8: launch_gather_op<DequantOp<8, IO, F8>>(a, grid, s); break;
    case 4: launch_gather_op<DequantOp<4, IO, F8>>(a, grid, s); break;
    case 2: launch_gather_op<DequantOp<2, IO, F8>>(a, grid, s); break;
    default: launch_gather_op<DequantOp<1, IO, F8>>(a, grid, s); break;
  }
}

// ---------------------------------------------------------------------------
// Kernel families, one translation unit each (kernels_*.hip).

// Copying writes; chunk_bytes = G * element size (1, 2, 4, 8 or 16).
void run_write_copy(int chunk_bytes, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
// Quantizing writes into an FP8 cache, per FP8 format and io dtype; G = ge
// elements per chunk.
void run_write_quant_e4m3_f32(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
void run_write_quant_e4m3_f16(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
void run_write_quant_e4m3_bf16(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
void run_write_quant_e5m2_f32(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
void run_write_quant_e5m2_f16(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
void run_write_quant_e5m2_bf16(int ge, const WriteArgs &a, const WriteLaunch &w, hipStream_t s);
// Copying gathers: the flat / row / indexed kernels, and the tile kernel.
void run_gather_copy(int chunk_bytes, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_tiles_copy(const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid, uint32_t lds,
                    hipStream_t s);
// Dequantizing gathers, per FP8 format and io dtype.
void run_gather_dequant_e4m3_f32(int ge, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_gather_dequant_e4m3_f16(int ge, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_gather_dequant_e4m3_bf16(int ge, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_gather_dequant_e5m2_f32(int ge, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_gather_dequant_e5m2_f16(int ge, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_gather_dequant_e5m2_bf16(int ge, const GatherArgs &a, int64_t grid, hipStream_t s);
void run_tiles_dequant_e4m3(int io, const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid,
                            uint32_t lds, hipStream_t s);
void run_tiles_dequant_e5m2(int io, const TileArgs &t, int fmt, bool i64, bool p64, int64_t grid,
                            uint32_t lds, hipStream_t s);

}  // namespace dev
}  // namespace kvx
