// Plain streaming kernels: the HBM ceilings measured beside the KV kernels.
//
//   copy   reads n bytes and writes them elsewhere (the read/write mix of a
//          KV write or gather, with no index work);
//   read   reads n bytes (folded into one word per workgroup that is stored
//          only if it equals a value the data never produce);
//   write  writes n bytes of a constant;
//   expand reads n bytes and writes each 16-byte chunk twice, to 2n bytes
//          (the 1:2 read/write mix of an FP8 -> bf16 dequantizing gather).
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
  if (acc == never) sink[threadIdx.x] = acc;
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

template <int T, int U>
__global__ __launch_bounds__(T) void expand_kernel(const u32x4 *src, u32x4 *dst, int64_t n) {
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
    if (i < n) {
      __builtin_nontemporal_store(v[u], dst + i);
      __builtin_nontemporal_store(v[u], dst + n + i);
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
    hipLaunchKernelGGL((expand_kernel<T, U>), grid, block, 0, s,
                       static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), n);
  }
}

int run(int op, int shape, void *dst, const void *src, int64_t bytes, uint32_t value,
        void *stream) {
  if (shape < 0 || shape >= kNumShapes || bytes < 0 || bytes % 16 != 0) return 1;
  if ((op != 1 && ((uintptr_t)dst % 16 != 0)) || (op != 2 && (uintptr_t)src % 16 != 0))
    return 1;
  const int64_t n = bytes / 16;
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

// sink: 1024 bytes of device memory, written only in the never-taken case.
int kvx_probe_read(const void *src, int64_t bytes, void *sink, int shape, void *stream) {
  return run(1, shape, sink, src, bytes, 0x9E3779B9u, stream);
}

int kvx_probe_write(void *dst, int64_t bytes, uint32_t value, int shape, void *stream) {
  return run(2, shape, dst, nullptr, bytes, value, stream);
}

// dst: 2 * bytes of device memory.
int kvx_probe_expand(void *dst, const void *src, int64_t bytes, int shape, void *stream) {
  return run(3, shape, dst, src, bytes, 0, stream);
}

}  // extern "C"
