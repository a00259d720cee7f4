// Plain streaming kernels: the HBM ceilings measured beside the KV kernels.
//
//   copy   reads n bytes and writes them elsewhere (the read/write mix of a
//          KV write or gather, with no index work);
//   read   reads n bytes (folded into one word per lane that is stored
//          only if it equals a value the data never produce);
//   write  writes n bytes of a constant;
//   widen  reads n bytes as 8-byte chunks and writes each as one 16-byte
//          chunk, to 2n bytes: the access shape of the FP8 -> bf16
//          dequantizing gather (one contiguous 16-byte store per 8-byte
//          load, one output stream), with no conversion work;
//   scatter  copies n contiguous bytes into granules of a pool named by a
//          granule map (or gathers them back): the data movement of a
//          paged KV write (or gather) over a given block table, with no
//          slot, table or layout work;
//   granule widen  reads n bytes from the mapped granules as 8-byte chunks
//          and writes each as one 16-byte chunk of a contiguous buffer: the
//          FP8 dequantizing gather's access pattern over a given table.
//
// Each kernel is instantiated in a few launch shapes (threads per
// workgroup x 16-byte chunks per lane, every chunk of a workgroup in flight
// before the first store), all with the access form of the contiguous KV
// gather: 16-byte non-temporal loads and stores, consecutive lanes on
// consecutive chunks, one pass per workgroup.  The bench runs every shape
// and reports the fastest, so the ceiling is the best plain stream this
// box sustains, not one arbitrary shape.  Measurement tooling only: it is
// built as its own library (libkvx_amd_probe.so), and the KV library does
// not use it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int T, int U>
__global__ __launch_bounds__(T) void copy_kernel(const u32x4 *src, u32x4 *dst, int64_t n) {
  const int64_t base = (int64_t)blockIdx.x * (T * U) + threadIdx.x;
  u32x4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) v[u] = __builtin_nontemporal_load(src + i);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) __builtin_nontemporal_store(v[u], dst + i);
  }
}

template <int T, int U>
__global__ __launch_bounds__(T) void read_kernel(const u32x4 *src, int64_t n, uint32_t *sink,
                                                 uint32_t never) {
  const int64_t base = (int64_t)blockIdx.x * (T * U) + threadIdx.x;
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) {
      const u32x4 v = __builtin_nontemporal_load(src + i);
      acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
  }
  if (acc == never) sink[threadIdx.x & 255] = acc;  // sink holds 256 words
}

template <int T, int U>
__global__ __launch_bounds__(T) void write_kernel(u32x4 *dst, int64_t n, uint32_t value) {
  const int64_t base = (int64_t)blockIdx.x * (T * U) + threadIdx.x;
  u32x4 v;
  v[0] = v[1] = v[2] = v[3] = value;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) __builtin_nontemporal_store(v, dst + i);
  }
}

// n counts 8-byte source chunks; dst holds n 16-byte chunks.
template <int T, int U>
__global__ __launch_bounds__(T) void widen_kernel(const u32x2 *src, u32x4 *dst, int64_t n) {
  const int64_t base = (int64_t)blockIdx.x * (T * U) + threadIdx.x;
  u32x2 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) v[u] = __builtin_nontemporal_load(src + i);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) {
      u32x4 w;
      w[0] = v[u][0];
      w[1] = v[u][1];
      w[2] = v[u][0];
      w[3] = v[u][1];
      __builtin_nontemporal_store(w, dst + i);
    }
  }
}

// Granule copy: 16-byte chunk i of the contiguous side is chunk
// (map[i >> g16_log2] << g16_log2) + (i & (2^g16_log2 - 1)) of the pool
// (g16_log2 = log2 of the granule's 16-byte chunks).  SCATTER: contiguous
// -> pool; else pool -> contiguous.  The caller guarantees that every map
// entry names a granule inside the pool.
template <int T, int U, bool SCATTER>
__global__ __launch_bounds__(T) void granule_kernel(u32x4 *pool, u32x4 *lin, const int64_t *map,
                                                    int g16_log2, int64_t n) {
  const int64_t base = (int64_t)blockIdx.x * (T * U) + threadIdx.x;
  const int64_t mask = ((int64_t)1 << g16_log2) - 1;
  u32x4 v[U];
  int64_t at[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    at[u] = 0;
    if (i < n) {
      at[u] = (map[i >> g16_log2] << g16_log2) + (i & mask);
      v[u] = __builtin_nontemporal_load(SCATTER ? lin + i : pool + at[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) __builtin_nontemporal_store(v[u], SCATTER ? pool + at[u] : lin + i);
  }
}

// Granule widen: 8-byte chunk i of the read side is chunk
// (map[i >> g8_log2] << g8_log2) + (i & (2^g8_log2 - 1)) of the pool, and
// is stored twice over as 16-byte chunk i of out.
template <int T, int U>
__global__ __launch_bounds__(T) void granule_widen_kernel(const u32x2 *pool, u32x4 *out,
                                                          const int64_t *map, int g8_log2,
                                                          int64_t n) {
  const int64_t base = (int64_t)blockIdx.x * (T * U) + threadIdx.x;
  const int64_t mask = ((int64_t)1 << g8_log2) - 1;
  u32x2 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) v[u] = __builtin_nontemporal_load(pool + (map[i >> g8_log2] << g8_log2) + (i & mask));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * T;
    if (i < n) {
      u32x4 w;
      w[0] = v[u][0];
      w[1] = v[u][1];
      w[2] = v[u][0];
      w[3] = v[u][1];
      __builtin_nontemporal_store(w, out + i);
    }
  }
}

struct Shape {
  int threads;
  int unroll;
};
constexpr Shape kShapes[] = {{64, 1},  {64, 4},  {128, 1}, {128, 2}, {128, 4}, {256, 1},
                             {256, 2}, {256, 4}, {512, 1}, {512, 2}, {1024, 1}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

// Workgroups for n chunks, or 0 when the grid would exceed HIP's limits
// (2^31 - 1 workgroups, 2^32 - 1 work-items).
int64_t grid_for(int64_t n, Shape s) {
  const int64_t per = (int64_t)s.threads * s.unroll;
  const int64_t g = (n + per - 1) / per;
  if (g > 0x7FFFFFFF || g * s.threads > 0xFFFFFFFFll) return 0;
  return g;
}

template <int T, int U>
void launch(int op, void *dst, const void *src, int64_t n, uint32_t value, int64_t g,
            hipStream_t s) {
  const dim3 grid((uint32_t)g), block(T);
  if (op == 0) {
    hipLaunchKernelGGL((copy_kernel<T, U>), grid, block, 0, s, static_cast<const u32x4 *>(src),
                       static_cast<u32x4 *>(dst), n);
  } else if (op == 1) {
    hipLaunchKernelGGL((read_kernel<T, U>), grid, block, 0, s, static_cast<const u32x4 *>(src),
                       n, static_cast<uint32_t *>(dst), value);
  } else if (op == 2) {
    hipLaunchKernelGGL((write_kernel<T, U>), grid, block, 0, s, static_cast<u32x4 *>(dst), n,
                       value);
  } else {
    hipLaunchKernelGGL((widen_kernel<T, U>), grid, block, 0, s,
                       static_cast<const u32x2 *>(src), static_cast<u32x4 *>(dst), n);
  }
}

// bytes: bytes read (copy, read, widen) or written (write).  The grid
// covers n = bytes / 16 chunks, or bytes / 8 for widen.
// mode 0 scatter, 1 gather (16-byte chunks, n of them, gran_log2 = log2 of
// a granule's 16-byte chunks); 2 widen (8-byte chunks, n of them, the
// granule's log2 in 8-byte chunks passed the same way).
template <int T, int U>
void launch_granule(int mode, void *pool, void *lin, const int64_t *map, int gran_log2,
                    int64_t n, int64_t g, hipStream_t s) {
  const dim3 grid((uint32_t)g), block(T);
  if (mode == 2)
    hipLaunchKernelGGL((granule_widen_kernel<T, U>), grid, block, 0, s,
                       static_cast<const u32x2 *>(pool), static_cast<u32x4 *>(lin), map,
                       gran_log2, n);
  else if (mode == 0)
    hipLaunchKernelGGL((granule_kernel<T, U, true>), grid, block, 0, s, static_cast<u32x4 *>(pool),
                       static_cast<u32x4 *>(lin), map, gran_log2, n);
  else
    hipLaunchKernelGGL((granule_kernel<T, U, false>), grid, block, 0, s,
                       static_cast<u32x4 *>(pool), static_cast<u32x4 *>(lin), map, gran_log2, n);
}

int run_granule(int mode, int shape, void *pool, void *lin, int64_t bytes, const int64_t *map,
                int granule_log2, void *stream) {
  if (shape < 0 || shape >= kNumShapes || bytes < 0 || granule_log2 < 4 || granule_log2 > 40 ||
      bytes % ((int64_t)1 << granule_log2) != 0 || (uintptr_t)pool % 16 != 0 ||
      (uintptr_t)lin % 16 != 0 || (uintptr_t)map % 8 != 0)
    return 1;
  const int chunk_log2 = mode == 2 ? 3 : 4;  // bytes per chunk of the pool side
  const int64_t n = bytes >> chunk_log2;
  if (n == 0) return 0;
  const int64_t g = grid_for(n, kShapes[shape]);
  if (g == 0) return 1;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int gl = granule_log2 - chunk_log2;
  switch (shape) {
    case 0: launch_granule<64, 1>(mode, pool, lin, map, gl, n, g, s); break;
    case 1: launch_granule<64, 4>(mode, pool, lin, map, gl, n, g, s); break;
    case 2: launch_granule<128, 1>(mode, pool, lin, map, gl, n, g, s); break;
    case 3: launch_granule<128, 2>(mode, pool, lin, map, gl, n, g, s); break;
    case 4: launch_granule<128, 4>(mode, pool, lin, map, gl, n, g, s); break;
    case 5: launch_granule<256, 1>(mode, pool, lin, map, gl, n, g, s); break;
    case 6: launch_granule<256, 2>(mode, pool, lin, map, gl, n, g, s); break;
    case 7: launch_granule<256, 4>(mode, pool, lin, map, gl, n, g, s); break;
    case 8: launch_granule<512, 1>(mode, pool, lin, map, gl, n, g, s); break;
    case 9: launch_granule<512, 2>(mode, pool, lin, map, gl, n, g, s); break;
    default: launch_granule<1024, 1>(mode, pool, lin, map, gl, n, g, s); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int run(int op, int shape, void *dst, const void *src, int64_t bytes, uint32_t value,
        void *stream) {
  if (shape < 0 || shape >= kNumShapes || bytes < 0 || bytes % 16 != 0) return 1;
  if ((op != 1 && ((uintptr_t)dst % 16 != 0)) || (op != 2 && (uintptr_t)src % 16 != 0))
    return 1;
  const int64_t n = op == 3 ? bytes / 8 : bytes / 16;
  if (n == 0) return 0;
  const int64_t g = grid_for(n, kShapes[shape]);
  if (g == 0) return 1;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (shape) {
    case 0: launch<64, 1>(op, dst, src, n, value, g, s); break;
    case 1: launch<64, 4>(op, dst, src, n, value, g, s); break;
    case 2: launch<128, 1>(op, dst, src, n, value, g, s); break;
    case 3: launch<128, 2>(op, dst, src, n, value, g, s); break;
    case 4: launch<128, 4>(op, dst, src, n, value, g, s); break;
    case 5: launch<256, 1>(op, dst, src, n, value, g, s); break;
    case 6: launch<256, 2>(op, dst, src, n, value, g, s); break;
    case 7: launch<256, 4>(op, dst, src, n, value, g, s); break;
    case 8: launch<512, 1>(op, dst, src, n, value, g, s); break;
    case 9: launch<512, 2>(op, dst, src, n, value, g, s); break;
    default: launch<1024, 1>(op, dst, src, n, value, g, s); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace

extern "C" {

// Number of launch shapes; shape i is (threads, chunks per lane) of
// kvx_probe_shape.
int kvx_probe_shapes(void) { return kNumShapes; }

int kvx_probe_shape(int i, int *threads, int *unroll) {
  if (i < 0 || i >= kNumShapes) return 1;
  *threads = kShapes[i].threads;
  *unroll = kShapes[i].unroll;
  return 0;
}

// Returns 0 when enqueued, 1 for bad arguments (sizes not a multiple of 16,
// misaligned pointers, a grid past HIP's limits), 2 when the launch fails.
int kvx_probe_copy(void *dst, const void *src, int64_t bytes, int shape, void *stream) {
  return run(0, shape, dst, src, bytes, 0, stream);
}

// sink: at least 1024 bytes of device memory, written only in the
// never-taken case (one of its 256 words per lane).
int kvx_probe_read(const void *src, int64_t bytes, void *sink, int shape, void *stream) {
  return run(1, shape, sink, src, bytes, 0x9E3779B9u, stream);
}

int kvx_probe_write(void *dst, int64_t bytes, uint32_t value, int shape, void *stream) {
  return run(2, shape, dst, nullptr, bytes, value, stream);
}

// Reads `bytes` (a multiple of 16) from src, writes 2 * bytes to dst.
int kvx_probe_widen(void *dst, const void *src, int64_t bytes, int shape, void *stream) {
  return run(3, shape, dst, src, bytes, 0, stream);
}

// Copies `bytes` (a multiple of the granule, 2^granule_log2 bytes, at
// least 16) between the contiguous buffer lin and the granules of pool
// that map (bytes >> granule_log2 int64 entries, device memory) names:
// lin -> pool when scatter is nonzero, pool -> lin otherwise.  Every map
// entry must name a granule inside the pool; it is not checked.
int kvx_probe_granules(void *pool, void *lin, int64_t bytes, const int64_t *map,
                       int granule_log2, int scatter, int shape, void *stream) {
  return run_granule(scatter != 0 ? 0 : 1, shape, pool, lin, bytes, map, granule_log2, stream);
}

// Reads `bytes` (a whole number of granules, 2^granule_log2 >= 16 bytes
// each) from the pool granules that map names, 8 bytes at a time, and
// writes 2 * bytes to out: 8-byte chunk i of the read side, stored twice
// over, is 16-byte chunk i of out.  Every map entry must name a granule
// inside the pool; it is not checked.
int kvx_probe_granules_widen(void *out, const void *pool, int64_t bytes, const int64_t *map,
                             int granule_log2, int shape, void *stream) {
  return run_granule(2, shape, const_cast<void *>(pool), out, bytes, map, granule_log2, stream);
}

}  // extern "C"
