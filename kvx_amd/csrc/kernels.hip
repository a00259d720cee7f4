// Paged KV write (scatter) and gather kernels for gfx950 (CDNA4, wave64).
//
// Data movement only, plus an optional FP8 E4M3 cast.  The unit of work is a
// *chunk*: G consecutive elements of one contiguous cache piece (a head row
// for NHD/HND, an x-element pack for HND_PACKED), moved with one 1..16-byte
// load and one store per lane.  The host picks the widest chunk that every
// pointer and stride allows, so NHD/HND bf16 rows move as 16-byte
// global_load_dwordx4 / global_store_dwordx4 and a wave covers 1 KiB of a row
// per instruction.
//
// Semantics follow the reference kernels:
//   write  kernels/kvx_paged_kv.cu:93-124 (slot < 0 and block >= num_blocks
//          are skipped; bit copy of every (token, head, dim) element);
//   gather kernels/kvx_paged_kv.cu:226-267 (rows t >= seq_len, logical
//          blocks >= max_blocks_per_seq and block ids < 0 are untouched);
//          block ids >= num_blocks are also skipped here instead of being
//          read out of bounds.
#include <hip/hip_runtime.h>

#include "fp_convert.h"
#include "kvx_internal.h"

namespace kvx {
namespace {

constexpr int kWave = 64;
constexpr int kBlockThreads = 256;
constexpr int kWavesPerBlock = kBlockThreads / kWave;
// Chunk offsets each lane keeps in registers; rows with more chunks per lane
// compute the rest on the fly.
constexpr int kMaxChunksPerLane = 4;
// Chunks per lane in flight in the flat (contiguous block) gather loop.
constexpr int kFlatUnroll = 4;

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

template <int B>
struct alignas(B < 16 ? B : 16) Raw {
  uint8_t u8[B];
};

// Load/store one chunk with the widest naturally aligned access: B = 16 is
// one global_load_dwordx4 / global_store_dwordx4 per lane.
template <int B>
__device__ __forceinline__ Raw<B> ld(const char *p) {
  Raw<B> r;
  if constexpr (B == 1) {
    r.u8[0] = *reinterpret_cast<const uint8_t *>(p);
  } else if constexpr (B == 2) {
    const uint16_t v = *reinterpret_cast<const uint16_t *>(p);
    __builtin_memcpy(r.u8, &v, 2);
  } else if constexpr (B == 4) {
    const uint32_t v = *reinterpret_cast<const uint32_t *>(p);
    __builtin_memcpy(r.u8, &v, 4);
  } else if constexpr (B == 8) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    __builtin_memcpy(r.u8, &v, 8);
  } else {
    static_assert(B % 16 == 0, "chunk bytes");
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      const uint4 v = reinterpret_cast<const uint4 *>(p)[i];
      __builtin_memcpy(r.u8 + 16 * i, &v, 16);
    }
  }
  return r;
}

template <int B>
__device__ __forceinline__ void st(char *p, const Raw<B> &r) {
  if constexpr (B == 1) {
    *reinterpret_cast<uint8_t *>(p) = r.u8[0];
  } else if constexpr (B == 2) {
    uint16_t v;
    __builtin_memcpy(&v, r.u8, 2);
    *reinterpret_cast<uint16_t *>(p) = v;
  } else if constexpr (B == 4) {
    uint32_t v;
    __builtin_memcpy(&v, r.u8, 4);
    *reinterpret_cast<uint32_t *>(p) = v;
  } else if constexpr (B == 8) {
    uint2 v;
    __builtin_memcpy(&v, r.u8, 8);
    *reinterpret_cast<uint2 *>(p) = v;
  } else {
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      uint4 v;
      __builtin_memcpy(&v, r.u8 + 16 * i, 16);
      reinterpret_cast<uint4 *>(p)[i] = v;
    }
  }
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

template <int IO>
__device__ __forceinline__ float io_to_f32(const uint8_t *bytes, int i) {
  if constexpr (IO == KVX_DTYPE_F32) {
    uint32_t u;
    __builtin_memcpy(&u, bytes + 4 * i, 4);
    return bits_f32(u);
  } else {
    uint16_t h;
    __builtin_memcpy(&h, bytes + 2 * i, 2);
    if constexpr (IO == KVX_DTYPE_BF16) return bf16_to_f32(h);
    return f16_to_f32(h);
  }
}

template <int IO>
__device__ __forceinline__ void f32_to_io(float v, uint8_t *bytes, int i) {
  if constexpr (IO == KVX_DTYPE_F32) {
    const uint32_t u = f32_bits(canon_nan_f32(v));
    __builtin_memcpy(bytes + 4 * i, &u, 4);
  } else {
    const uint16_t h =
        (IO == KVX_DTYPE_BF16) ? f32_to_bf16(v) : f32_to_f16(v);
    __builtin_memcpy(bytes + 2 * i, &h, 2);
  }
}

// io (F16/BF16/F32) -> E4M3: q = e4m3(sat(x / scale)).
template <int G, int IO>
struct QuantOp {
  static constexpr int kSrc = G * IoType<IO>::kBytes;
  static constexpr int kDst = G;
  static constexpr bool kScaled = true;
  __device__ __forceinline__ static Raw<kDst> apply(const Raw<kSrc> &x,
                                                    float scale) {
    Raw<kDst> y;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      y.u8[i] = f32_to_e4m3(io_to_f32<IO>(x.u8, i) / scale);
    }
    return y;
  }
};

// E4M3 -> io (F16/BF16/F32): y = io(f32(q) * scale); any NaN result is the
// canonical quiet NaN of the io type.
template <int G, int IO>
struct DequantOp {
  static constexpr int kSrc = G;
  static constexpr int kDst = G * IoType<IO>::kBytes;
  static constexpr bool kScaled = true;
  __device__ __forceinline__ static Raw<kDst> apply(const Raw<kSrc> &x,
                                                    float scale) {
    Raw<kDst> y;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      f32_to_io<IO>(e4m3_to_f32(x.u8[i]) * scale, y.u8, i);
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
  const float *k_scale;
  const float *v_scale;
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
#pragma unroll
  for (int k = 0; k < kMaxChunksPerLane; ++k) {
    const int c = l + k * lpt;
    koff[k] = 0;
    voff[k] = 0;
    if (c < a.nchunks) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      koff[k] = chunk_off(a.gk, e, (uint32_t)a.head_dim);
      voff[k] = chunk_off(a.gv, e, (uint32_t)a.head_dim);
    }
  }
  float ks = 1.0f;
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = *a.k_scale;
    vs = *a.v_scale;
  }

  for (int64_t g = wave; g < a.num_groups; g += nwaves) {
    const int64_t t = g * tpw + sub;
    int64_t mine = -1;
    const int64_t tl = g * tpw + lane;
    if (lane < tpw && tl < a.num_tokens) mine = load_index(a.slots, tl, a.slot_is64);
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

    const char *sk = a.src_k + t * a.row_bytes;
    const char *sv = a.src_v + t * a.row_bytes;
    char *dk = a.dst_k + b * a.gk.s_block + o * a.gk.s_off;
    char *dv = a.dst_v + b * a.gv.s_block + o * a.gv.s_off;

    Raw<Op::kSrc> xk[kMaxChunksPerLane];
    Raw<Op::kSrc> xv[kMaxChunksPerLane];
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
      const int c = l + k * lpt;
      if (c < a.nchunks) {
        xk[k] = ld<Op::kSrc>(sk + (int64_t)c * Op::kSrc);
        xv[k] = ld<Op::kSrc>(sv + (int64_t)c * Op::kSrc);
      }
    }
#pragma unroll
    for (int k = 0; k < kMaxChunksPerLane; ++k) {
      const int c = l + k * lpt;
      if (c < a.nchunks) {
        st<Op::kDst>(dk + koff[k], Op::apply(xk[k], ks));
        st<Op::kDst>(dv + voff[k], Op::apply(xv[k], vs));
      }
    }
    for (int c = l + kMaxChunksPerLane * lpt; c < a.nchunks; c += lpt) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      const Raw<Op::kSrc> yk = ld<Op::kSrc>(sk + (int64_t)c * Op::kSrc);
      const Raw<Op::kSrc> yv = ld<Op::kSrc>(sv + (int64_t)c * Op::kSrc);
      st<Op::kDst>(dk + chunk_off(a.gk, e, (uint32_t)a.head_dim),
                   Op::apply(yk, ks));
      st<Op::kDst>(dv + chunk_off(a.gv, e, (uint32_t)a.head_dim),
                   Op::apply(yv, vs));
    }
  }
}

// ---------------------------------------------------------------------------
// Gather.
//
// One workgroup per (sequence, logical block).  seq_len and the block id are
// wave-uniform scalar loads, read once per workgroup.  When the cache rows of
// a block are contiguous (canonical NHD), the valid rows of the block are one
// contiguous run in the cache and in the output, so the workgroup streams it
// as a flat copy.  Other layouts map rows to (wave, lane group) and use the
// per-lane chunk offsets as the write kernel does.

struct GatherArgs {
  const char *src_k;
  const char *src_v;
  char *dst_k;
  char *dst_v;
  const void *table;
  const void *seq_lens;
  const float *k_scale;
  const float *v_scale;
  GeomBytes gk;
  GeomBytes gv;
  int64_t out_row_bytes;  // bytes of one output row (H * D * io size)
  int32_t index_is64;
  int32_t max_blocks_per_seq;
  int32_t blocks_per_seq;  // logical blocks launched per sequence
  int32_t max_seq_len;
  int32_t block_size;
  int32_t num_blocks;
  int32_t head_dim;
  int32_t nchunks;
  int32_t chunk_elems;
  int32_t lpt_log2;
  int32_t flat;  // cache rows of a block are contiguous for K and V
};

template <class Op>
__global__ __launch_bounds__(kBlockThreads) void gather_kernel(GatherArgs a) {
  const int64_t wg = blockIdx.x;
  const int64_t s = wg / a.blocks_per_seq;
  const int32_t lb = (int32_t)(wg - s * a.blocks_per_seq);
  if (lb >= a.max_blocks_per_seq) return;
  const int64_t seq_len = load_index(a.seq_lens, s, a.index_is64);
  const int64_t n = seq_len < a.max_seq_len ? seq_len : (int64_t)a.max_seq_len;
  const int64_t t0 = (int64_t)lb * a.block_size;
  if (t0 >= n) return;
  const int64_t bid =
      load_index(a.table, s * a.max_blocks_per_seq + lb, a.index_is64);
  if (bid < 0 || bid >= a.num_blocks) return;
  const int64_t rem = n - t0;
  const int32_t rows = rem < a.block_size ? (int32_t)rem : a.block_size;

  float ks = 1.0f;
  float vs = 1.0f;
  if constexpr (Op::kScaled) {
    ks = *a.k_scale;
    vs = *a.v_scale;
  }

  const char *ck = a.src_k + bid * a.gk.s_block;
  const char *cv = a.src_v + bid * a.gv.s_block;
  const int64_t out0 = (s * a.max_seq_len + t0) * a.out_row_bytes;
  char *ok = a.dst_k + out0;
  char *ov = a.dst_v + out0;

  if (a.flat) {
    const int64_t total = (int64_t)rows * a.nchunks;
    int64_t i = threadIdx.x;
    for (; i + (kFlatUnroll - 1) * kBlockThreads < total;
         i += kFlatUnroll * kBlockThreads) {
      Raw<Op::kSrc> xk[kFlatUnroll];
      Raw<Op::kSrc> xv[kFlatUnroll];
#pragma unroll
      for (int u = 0; u < kFlatUnroll; ++u) {
        xk[u] = ld<Op::kSrc>(ck + (i + u * kBlockThreads) * Op::kSrc);
        xv[u] = ld<Op::kSrc>(cv + (i + u * kBlockThreads) * Op::kSrc);
      }
#pragma unroll
      for (int u = 0; u < kFlatUnroll; ++u) {
        st<Op::kDst>(ok + (i + u * kBlockThreads) * Op::kDst,
                     Op::apply(xk[u], ks));
        st<Op::kDst>(ov + (i + u * kBlockThreads) * Op::kDst,
                     Op::apply(xv[u], vs));
      }
    }
    for (; i < total; i += kBlockThreads) {
      const Raw<Op::kSrc> yk = ld<Op::kSrc>(ck + i * Op::kSrc);
      const Raw<Op::kSrc> yv = ld<Op::kSrc>(cv + i * Op::kSrc);
      st<Op::kDst>(ok + i * Op::kDst, Op::apply(yk, ks));
      st<Op::kDst>(ov + i * Op::kDst, Op::apply(yv, vs));
    }
    return;
  }

  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int lpt = 1 << a.lpt_log2;
  const int tpw = kWave >> a.lpt_log2;
  const int sub = lane >> a.lpt_log2;
  const int l = lane & (lpt - 1);

  int64_t koff[kMaxChunksPerLane];
  int64_t voff[kMaxChunksPerLane];
#pragma unroll
  for (int k = 0; k < kMaxChunksPerLane; ++k) {
    const int c = l + k * lpt;
    koff[k] = 0;
    voff[k] = 0;
    if (c < a.nchunks) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      koff[k] = chunk_off(a.gk, e, (uint32_t)a.head_dim);
      voff[k] = chunk_off(a.gv, e, (uint32_t)a.head_dim);
    }
  }

  for (int r = wave * tpw + sub; r < rows; r += kWavesPerBlock * tpw) {
    const char *rk = ck + (int64_t)r * a.gk.s_off;
    const char *rv = cv + (int64_t)r * a.gv.s_off;
    char *wk = ok + (int64_t)r * a.out_row_bytes;
    char *wv = ov + (int64_t)r * a.out_row_bytes;
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
        st<Op::kDst>(wk + (int64_t)c * Op::kDst, Op::apply(xk[k], ks));
        st<Op::kDst>(wv + (int64_t)c * Op::kDst, Op::apply(xv[k], vs));
      }
    }
    for (int c = l + kMaxChunksPerLane * lpt; c < a.nchunks; c += lpt) {
      const uint32_t e = (uint32_t)c * (uint32_t)a.chunk_elems;
      const Raw<Op::kSrc> yk =
          ld<Op::kSrc>(rk + chunk_off(a.gk, e, (uint32_t)a.head_dim));
      const Raw<Op::kSrc> yv =
          ld<Op::kSrc>(rv + chunk_off(a.gv, e, (uint32_t)a.head_dim));
      st<Op::kDst>(wk + (int64_t)c * Op::kDst, Op::apply(yk, ks));
      st<Op::kDst>(wv + (int64_t)c * Op::kDst, Op::apply(yv, vs));
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side planning.

GeomBytes to_bytes(const Geom &g, int esize) {
  GeomBytes r;
  r.s_block = g.s_block * esize;
  r.s_off = g.s_off * esize;
  r.s_head = g.s_head * esize;
  r.s_piece = g.s_piece * esize;
  r.s_inner = g.s_inner * esize;
  r.pack = g.pack;
  r.pad_ = 0;
  return r;
}

bool aligned(const void *p, int64_t b) {
  return ((uintptr_t)p % (uintptr_t)b) == 0;
}

// True when chunks of g elements (g*esize bytes each) stay inside one
// contiguous cache piece and every cache address they use is aligned.
bool cache_chunk_ok(const Geom &g, const void *base, int esize, int head_dim,
                    int ge) {
  const int64_t bytes = (int64_t)ge * esize;
  if (ge > 1 && g.s_inner != 1) return false;
  if (g.pack % ge != 0 || head_dim % ge != 0) return false;
  if (!aligned(base, bytes)) return false;
  const int64_t strides[4] = {g.s_block, g.s_off, g.s_head, g.s_piece};
  for (int64_t st : strides) {
    if ((st * esize) % bytes != 0) return false;
  }
  return true;
}

// Widest chunk (elements) that works for K, V and the io buffers.  The io
// side is contiguous with rows of H*D elements of io_size bytes.
int pick_chunk(const Geom &gk, const Geom &gv, const void *ck, const void *cv,
               int cache_size, const void *ik, const void *iv, int io_size,
               int head_dim, int max_chunk_bytes_cache) {
  for (int ge = max_chunk_bytes_cache / cache_size; ge >= 1; ge /= 2) {
    if (!cache_chunk_ok(gk, ck, cache_size, head_dim, ge)) continue;
    if (!cache_chunk_ok(gv, cv, cache_size, head_dim, ge)) continue;
    const int64_t io_bytes = (int64_t)ge * io_size;
    if (!aligned(ik, io_bytes) || !aligned(iv, io_bytes)) continue;
    return ge;
  }
  return 1;
}

int lpt_log2_for(int nchunks) {
  int lg = 0;
  while ((1 << lg) < nchunks && lg < 6) ++lg;
  return lg;
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

template <class Op>
void launch_write_op(const WriteArgs &a, int grid, hipStream_t s) {
  hipLaunchKernelGGL(write_kernel<Op>, dim3(grid), dim3(kBlockThreads), 0, s,
                     a);
}

template <class Op>
void launch_gather_op(const GatherArgs &a, int64_t grid, hipStream_t s) {
  hipLaunchKernelGGL(gather_kernel<Op>, dim3((uint32_t)grid),
                     dim3(kBlockThreads), 0, s, a);
}

template <int IO>
void dispatch_quant(int ge, const WriteArgs &a, int grid, hipStream_t s) {
  switch (ge) {
    case 8: launch_write_op<QuantOp<8, IO>>(a, grid, s); break;
    case 4: launch_write_op<QuantOp<4, IO>>(a, grid, s); break;
    case 2: launch_write_op<QuantOp<2, IO>>(a, grid, s); break;
    default: launch_write_op<QuantOp<1, IO>>(a, grid, s); break;
  }
}

template <int IO>
void dispatch_dequant(int ge, const GatherArgs &a, int64_t grid,
                      hipStream_t s) {
  switch (ge) {
    case 8: launch_gather_op<DequantOp<8, IO>>(a, grid, s); break;
    case 4: launch_gather_op<DequantOp<4, IO>>(a, grid, s); break;
    case 2: launch_gather_op<DequantOp<2, IO>>(a, grid, s); break;
    default: launch_gather_op<DequantOp<1, IO>>(a, grid, s); break;
  }
}

}  // namespace

int dtype_size(kvx_dtype_t dt) {
  switch (dt) {
    case KVX_DTYPE_F32: return 4;
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16: return 2;
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2: return 1;
    default: return 0;
  }
}

kvx_status_t enqueue_write(const WritePlan &p, void *stream) {
  const int cs = dtype_size((kvx_dtype_t)p.cache_dtype);
  const int is = dtype_size((kvx_dtype_t)p.io_dtype);
  const int max_bytes = (p.conv == kConvQuant) ? 8 : 16;
  const int ge = pick_chunk(p.gk, p.gv, p.dst_k, p.dst_v, cs, p.src_k,
                            p.src_v, is, p.head_dim, max_bytes);
  const int64_t row_elems = (int64_t)p.heads * p.head_dim;

  WriteArgs a;
  a.src_k = static_cast<const char *>(p.src_k);
  a.src_v = static_cast<const char *>(p.src_v);
  a.dst_k = static_cast<char *>(p.dst_k);
  a.dst_v = static_cast<char *>(p.dst_v);
  a.slots = p.slots;
  a.k_scale = p.k_scale;
  a.v_scale = p.v_scale;
  a.gk = to_bytes(p.gk, cs);
  a.gv = to_bytes(p.gv, cs);
  a.num_tokens = p.num_tokens;
  a.slot_is64 = p.slot_is64;
  a.block_size = p.block_size;
  a.num_blocks = p.num_blocks;
  a.head_dim = p.head_dim;
  a.nchunks = (int32_t)(row_elems / ge);
  a.chunk_elems = ge;
  a.row_bytes = (int32_t)(row_elems * is);
  a.lpt_log2 = lpt_log2_for(a.nchunks);
  const int tpw = kWave >> a.lpt_log2;
  a.num_groups = (p.num_tokens + tpw - 1) / tpw;
  const int64_t want = (a.num_groups + kWavesPerBlock - 1) / kWavesPerBlock;
  const int grid = (int)(want < 2048 ? want : 2048);
  hipStream_t s = as_stream(stream);

  if (p.conv == kConvCopy) {
    switch (ge * cs) {
      case 16: launch_write_op<CopyOp<16>>(a, grid, s); break;
      case 8: launch_write_op<CopyOp<8>>(a, grid, s); break;
      case 4: launch_write_op<CopyOp<4>>(a, grid, s); break;
      case 2: launch_write_op<CopyOp<2>>(a, grid, s); break;
      default: launch_write_op<CopyOp<1>>(a, grid, s); break;
    }
  } else {
    switch (p.io_dtype) {
      case KVX_DTYPE_F32: dispatch_quant<KVX_DTYPE_F32>(ge, a, grid, s); break;
      case KVX_DTYPE_F16: dispatch_quant<KVX_DTYPE_F16>(ge, a, grid, s); break;
      default: dispatch_quant<KVX_DTYPE_BF16>(ge, a, grid, s); break;
    }
  }
  return hipGetLastError() == hipSuccess ? KVX_STATUS_OK
                                         : KVX_STATUS_INTERNAL_ERROR;
}

kvx_status_t enqueue_gather(const GatherPlan &p, void *stream) {
  const int cs = dtype_size((kvx_dtype_t)p.cache_dtype);
  const int is = dtype_size((kvx_dtype_t)p.io_dtype);
  const int max_bytes = (p.conv == kConvDequant) ? 8 : 16;
  const int ge = pick_chunk(p.gk, p.gv, p.src_k, p.src_v, cs, p.dst_k,
                            p.dst_v, is, p.head_dim, max_bytes);
  const int64_t row_elems = (int64_t)p.heads * p.head_dim;

  GatherArgs a;
  a.src_k = static_cast<const char *>(p.src_k);
  a.src_v = static_cast<const char *>(p.src_v);
  a.dst_k = static_cast<char *>(p.dst_k);
  a.dst_v = static_cast<char *>(p.dst_v);
  a.table = p.block_table;
  a.seq_lens = p.seq_lens;
  a.k_scale = p.k_scale;
  a.v_scale = p.v_scale;
  a.gk = to_bytes(p.gk, cs);
  a.gv = to_bytes(p.gv, cs);
  a.out_row_bytes = row_elems * is;
  a.index_is64 = p.index_is64;
  a.max_blocks_per_seq = p.max_blocks_per_seq;
  const int64_t by_len =
      ((int64_t)p.max_seq_len + p.block_size - 1) / p.block_size;
  a.blocks_per_seq =
      (int32_t)(by_len < p.max_blocks_per_seq ? by_len : p.max_blocks_per_seq);
  a.max_seq_len = p.max_seq_len;
  a.block_size = p.block_size;
  a.num_blocks = p.num_blocks;
  a.head_dim = p.head_dim;
  a.nchunks = (int32_t)(row_elems / ge);
  a.chunk_elems = ge;
  a.lpt_log2 = lpt_log2_for(a.nchunks);
  // Rows of a block form one contiguous run when each row is H*D
  // consecutive elements and consecutive offsets are one row apart.
  auto rows_contiguous = [&](const Geom &g) {
    return g.s_inner == 1 && g.pack == p.head_dim && g.s_head == p.head_dim &&
           g.s_off == row_elems;
  };
  a.flat = rows_contiguous(p.gk) && rows_contiguous(p.gv);
  if (a.blocks_per_seq <= 0 || p.seq_count <= 0) return KVX_STATUS_OK;
  const int64_t grid = (int64_t)p.seq_count * a.blocks_per_seq;
  if (grid > 0x7FFFFFFF) return KVX_STATUS_UNSUPPORTED;  // one workgroup per block
  hipStream_t s = as_stream(stream);

  if (p.conv == kConvCopy) {
    switch (ge * cs) {
      case 16: launch_gather_op<CopyOp<16>>(a, grid, s); break;
      case 8: launch_gather_op<CopyOp<8>>(a, grid, s); break;
      case 4: launch_gather_op<CopyOp<4>>(a, grid, s); break;
      case 2: launch_gather_op<CopyOp<2>>(a, grid, s); break;
      default: launch_gather_op<CopyOp<1>>(a, grid, s); break;
    }
  } else {
    switch (p.io_dtype) {
      case KVX_DTYPE_F32: dispatch_dequant<KVX_DTYPE_F32>(ge, a, grid, s); break;
      case KVX_DTYPE_F16: dispatch_dequant<KVX_DTYPE_F16>(ge, a, grid, s); break;
      default: dispatch_dequant<KVX_DTYPE_BF16>(ge, a, grid, s); break;
    }
  }
  return hipGetLastError() == hipSuccess ? KVX_STATUS_OK
                                         : KVX_STATUS_INTERNAL_ERROR;
}

}  // namespace kvx
