// kvx_bench: the reference's kernel microbenchmark command line
// (benchmarks/kvx_bench.cu) over libkvx_amd.so, so that tools that run the
// reference binary and parse its output (benchmarks/fair_bench.py:120-146,
// benchmarks/tests/kvx_bench_cli_test.py:6-49) run unchanged against this
// build.
//
// Same flags (kvx_bench.cu:92-126): --seq-count --seq-len --tokens-per-seq
// --block-size --num-heads --head-dim --warmup --iters, each as "--x N" or
// "--x=N", and --dtype=float32|float16|bfloat16.  Same defaults
// (kvx_bench.cu:27-38), the same argument checks (:222-231, exit status 1),
// the same workload (:233-275): NHD caches with seq_count * ceil(seq_len /
// block_size) blocks, sequence s owning blocks s * mbps .. s * mbps + mbps - 1,
// the last tokens_per_seq positions of every sequence written (the prefill
// entry when tokens_per_seq > 1), then a full gather of every sequence.  Same
// output (:535-558): two summary lines and a CSV header plus one "write," and
// one "gather," row,
//   kernel,seq_count,seq_len,block_size,num_heads,head_dim,num_blocks,
//   iters,warmup,ms_per,tokens_per_s,gb_per_s,tokens_per_seq
// where gb_per_s keeps the reference's definition (4 x elements x element
// size, in GiB/s) so that numbers from both binaries compare.  Timing: HIP
// events around `iters` back-to-back launches on the null stream.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fp_convert.h"
#include "kvx_abi.h"
#include "kvx_paged_kv.h"

namespace {

struct Config {
  int32_t seq_count = 8;
  int32_t seq_len = 128;
  int32_t tokens_per_seq = 1;
  int32_t block_size = 16;
  int32_t num_heads = 8;
  int32_t head_dim = 128;
  int32_t warmup = 10;
  int32_t iters = 50;
  kvx_dtype_t dtype = KVX_DTYPE_F32;
  size_t elem = 4;
};

// "--name N" or "--name=N"; advances *i past a separate value.
bool int_flag(const char *name, int argc, char **argv, int *i, int32_t *out) {
  const size_t n = std::strlen(name);
  const char *a = argv[*i];
  if (std::strncmp(a, name, n) != 0) return false;
  if (a[n] == '=') {
    *out = std::atoi(a + n + 1);
    return true;
  }
  if (a[n] == '\0' && *i + 1 < argc) {
    *out = std::atoi(argv[++*i]);
    return true;
  }
  return false;
}

bool dtype_flag(int argc, char **argv, int *i, Config *c) {
  const char *name = "--dtype";
  const size_t n = std::strlen(name);
  const char *a = argv[*i];
  if (std::strncmp(a, name, n) != 0) return false;
  const char *v = nullptr;
  if (a[n] == '=') {
    v = a + n + 1;
  } else if (a[n] == '\0' && *i + 1 < argc) {
    v = argv[++*i];
  } else {
    return false;
  }
  if (std::strcmp(v, "float32") == 0) {
    c->dtype = KVX_DTYPE_F32;
    c->elem = 4;
  } else if (std::strcmp(v, "float16") == 0) {
    c->dtype = KVX_DTYPE_F16;
    c->elem = 2;
  } else if (std::strcmp(v, "bfloat16") == 0) {
    c->dtype = KVX_DTYPE_BF16;
    c->elem = 2;
  } else {
    std::fprintf(stderr, "Unsupported --dtype=%s\n", v);
    std::exit(1);
  }
  return true;
}

void parse(int argc, char **argv, Config *c) {
  for (int i = 1; i < argc; ++i) {
    if (int_flag("--seq-count", argc, argv, &i, &c->seq_count)) continue;
    if (int_flag("--seq-len", argc, argv, &i, &c->seq_len)) continue;
    if (int_flag("--tokens-per-seq", argc, argv, &i, &c->tokens_per_seq)) continue;
    if (int_flag("--block-size", argc, argv, &i, &c->block_size)) continue;
    if (int_flag("--num-heads", argc, argv, &i, &c->num_heads)) continue;
    if (int_flag("--head-dim", argc, argv, &i, &c->head_dim)) continue;
    if (int_flag("--warmup", argc, argv, &i, &c->warmup)) continue;
    if (int_flag("--iters", argc, argv, &i, &c->iters)) continue;
    dtype_flag(argc, argv, &i, c);  // unknown arguments are ignored, as in the reference
  }
}

void check(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

// Contiguous tensor descriptor of `ndim` axes.
kvx_tensor_desc_t dense_desc(kvx_dtype_t dt, kvx_layout_t layout,
                             std::initializer_list<int64_t> shape, void *data) {
  kvx_tensor_desc_t d;
  std::memset(&d, 0, sizeof d);
  d.size = sizeof d;
  d.dtype = dt;
  d.layout = layout;
  d.memory = KVX_MEMORY_DEVICE;
  d.ndim = (uint32_t)shape.size();
  int k = 0;
  for (int64_t v : shape) d.shape[k++] = v;
  int64_t st = 1;
  for (int j = (int)d.ndim - 1; j >= 0; --j) {
    d.stride[j] = st;
    st *= d.shape[j];
  }
  d.data = data;
  return d;
}

// Host rows of the reference's pattern (base + 0.01 * i) in the bench dtype.
std::vector<uint8_t> pattern(size_t n, float base, const Config &c) {
  std::vector<uint8_t> out(n * c.elem);
  for (size_t i = 0; i < n; ++i) {
    const float f = base + 0.01f * (float)i;
    if (c.dtype == KVX_DTYPE_F32) {
      std::memcpy(&out[i * 4], &f, 4);
    } else {
      const uint16_t h = c.dtype == KVX_DTYPE_F16 ? kvx::f32_to_f16(f) : kvx::f32_to_bf16(f);
      std::memcpy(&out[i * 2], &h, 2);
    }
  }
  return out;
}

void *upload(const void *src, size_t bytes) {
  void *d = nullptr;
  check(hipMalloc(&d, bytes ? bytes : 1), "hipMalloc");
  if (bytes) check(hipMemcpy(d, src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
  return d;
}

kvx_status_t launch_write(const Config &c, const kvx_cache_desc_t *cache,
                          const kvx_write_desc_t *w) {
  const bool prefill = c.tokens_per_seq > 1;
  switch (c.dtype) {
    case KVX_DTYPE_F16:
      return prefill ? kvx_launch_write_kv_prefill_f16(cache, w, c.tokens_per_seq, nullptr)
                     : kvx_launch_write_kv_f16(cache, w, nullptr);
    case KVX_DTYPE_BF16:
      return prefill ? kvx_launch_write_kv_prefill_bf16(cache, w, c.tokens_per_seq, nullptr)
                     : kvx_launch_write_kv_bf16(cache, w, nullptr);
    default:
      return prefill ? kvx_launch_write_kv_prefill_f32(cache, w, c.tokens_per_seq, nullptr)
                     : kvx_launch_write_kv_f32(cache, w, nullptr);
  }
}

kvx_status_t launch_gather(const Config &c, const kvx_cache_desc_t *cache,
                           const kvx_gather_desc_t *g) {
  switch (c.dtype) {
    case KVX_DTYPE_F16: return kvx_launch_gather_kv_f16(cache, g, nullptr);
    case KVX_DTYPE_BF16: return kvx_launch_gather_kv_bf16(cache, g, nullptr);
    default: return kvx_launch_gather_kv_f32(cache, g, nullptr);
  }
}

// Mean ms per launch of `iters` launches after `warmup` untimed ones.
template <class F>
float time_launches(const Config &c, const char *what, F launch) {
  for (int i = 0; i < c.warmup; ++i) {
    const kvx_status_t st = launch();
    if (st != KVX_STATUS_OK) {
      std::fprintf(stderr, "%s warmup failed: %d\n", what, (int)st);
      std::exit(1);
    }
  }
  check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  hipEvent_t e0, e1;
  check(hipEventCreate(&e0), "hipEventCreate");
  check(hipEventCreate(&e1), "hipEventCreate");
  check(hipEventRecord(e0, nullptr), "hipEventRecord");
  for (int i = 0; i < c.iters; ++i) {
    const kvx_status_t st = launch();
    if (st != KVX_STATUS_OK) {
      std::fprintf(stderr, "%s iter failed: %d\n", what, (int)st);
      std::exit(1);
    }
  }
  check(hipEventRecord(e1, nullptr), "hipEventRecord");
  check(hipEventSynchronize(e1), "hipEventSynchronize");
  float ms = 0.0f;
  check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return ms / (float)c.iters;
}

}  // namespace

int main(int argc, char **argv) {
  Config c;
  parse(argc, argv, &c);
  if (c.seq_count <= 0 || c.seq_len <= 0 || c.tokens_per_seq <= 0 || c.block_size <= 0 ||
      c.num_heads <= 0 || c.head_dim <= 0 || c.iters <= 0) {
    std::fprintf(stderr, "Invalid config values.\n");
    return 1;
  }
  if (c.tokens_per_seq > c.seq_len) {
    std::fprintf(stderr, "tokens_per_seq cannot exceed seq_len.\n");
    return 1;
  }

  const int32_t mbps = (c.seq_len + c.block_size - 1) / c.block_size;
  const int32_t num_blocks = c.seq_count * mbps;
  const int32_t num_tokens = c.seq_count * c.tokens_per_seq;
  const size_t row = (size_t)c.num_heads * c.head_dim;
  const size_t token_elems = (size_t)num_tokens * row;
  const size_t cache_elems = (size_t)num_blocks * c.block_size * row;
  const size_t gather_elems = (size_t)c.seq_count * c.seq_len * row;

  // token t of sequence s sits at position seq_len - tokens_per_seq + t
  std::vector<int64_t> slots((size_t)num_tokens);
  for (int32_t s = 0; s < c.seq_count; ++s)
    for (int32_t t = 0; t < c.tokens_per_seq; ++t) {
      const int32_t pos = c.seq_len - c.tokens_per_seq + t;
      slots[(size_t)s * c.tokens_per_seq + t] =
          (int64_t)(s * mbps + pos / c.block_size) * c.block_size + pos % c.block_size;
    }
  std::vector<int32_t> table((size_t)c.seq_count * mbps);
  for (size_t i = 0; i < table.size(); ++i) table[i] = (int32_t)i;
  std::vector<int32_t> lens((size_t)c.seq_count, c.seq_len);

  const std::vector<uint8_t> hk = pattern(token_elems, 0.1f, c);
  const std::vector<uint8_t> hv = pattern(token_elems, 0.2f, c);
  void *key = upload(hk.data(), hk.size());
  void *value = upload(hv.data(), hv.size());
  void *kc = nullptr, *vc = nullptr, *ko = nullptr, *vo = nullptr;
  check(hipMalloc(&kc, cache_elems * c.elem), "hipMalloc key_cache");
  check(hipMalloc(&vc, cache_elems * c.elem), "hipMalloc value_cache");
  check(hipMalloc(&ko, gather_elems * c.elem), "hipMalloc key_out");
  check(hipMalloc(&vo, gather_elems * c.elem), "hipMalloc value_out");
  void *d_slots = upload(slots.data(), slots.size() * sizeof(int64_t));
  void *d_table = upload(table.data(), table.size() * sizeof(int32_t));
  void *d_lens = upload(lens.data(), lens.size() * sizeof(int32_t));

  kvx_cache_desc_t cache;
  std::memset(&cache, 0, sizeof cache);
  cache.size = sizeof cache;
  cache.num_blocks = (uint32_t)num_blocks;
  cache.block_size = (uint32_t)c.block_size;
  cache.num_kv_heads = (uint32_t)c.num_heads;
  cache.head_dim = (uint32_t)c.head_dim;
  cache.k = dense_desc(c.dtype, KVX_LAYOUT_BLOCK_NHD,
                       {num_blocks, c.block_size, c.num_heads, c.head_dim}, kc);
  cache.v = dense_desc(c.dtype, KVX_LAYOUT_BLOCK_NHD,
                       {num_blocks, c.block_size, c.num_heads, c.head_dim}, vc);

  kvx_write_desc_t w;
  std::memset(&w, 0, sizeof w);
  w.size = sizeof w;
  w.io.size = sizeof w.io;
  w.io.num_tokens = (uint32_t)num_tokens;
  w.io.num_kv_heads = (uint32_t)c.num_heads;
  w.io.head_dim = (uint32_t)c.head_dim;
  w.io.key = dense_desc(c.dtype, KVX_LAYOUT_BLOCK_CUSTOM, {num_tokens, c.num_heads, c.head_dim},
                        key);
  w.io.value = dense_desc(c.dtype, KVX_LAYOUT_BLOCK_CUSTOM,
                          {num_tokens, c.num_heads, c.head_dim}, value);
  w.slots.size = sizeof w.slots;
  w.slots.dtype = KVX_DTYPE_S64;
  w.slots.token_count = (uint32_t)num_tokens;
  w.slots.invalid_slot = -1;
  w.slots.slots = d_slots;

  kvx_gather_desc_t g;
  std::memset(&g, 0, sizeof g);
  g.size = sizeof g;
  g.io.size = sizeof g.io;
  g.io.num_tokens = (uint32_t)(c.seq_count * c.seq_len);
  g.io.num_kv_heads = (uint32_t)c.num_heads;
  g.io.head_dim = (uint32_t)c.head_dim;
  g.io.key = dense_desc(c.dtype, KVX_LAYOUT_BLOCK_CUSTOM,
                        {c.seq_count, c.seq_len, c.num_heads, c.head_dim}, ko);
  g.io.value = dense_desc(c.dtype, KVX_LAYOUT_BLOCK_CUSTOM,
                          {c.seq_count, c.seq_len, c.num_heads, c.head_dim}, vo);
  g.block_table.size = sizeof g.block_table;
  g.block_table.format = KVX_BLOCK_TABLE_PACKED;
  g.block_table.index_dtype = KVX_DTYPE_S32;
  g.block_table.seq_count = (uint32_t)c.seq_count;
  g.block_table.beam_width = 1;
  g.block_table.max_blocks_per_seq = (uint32_t)mbps;
  g.block_table.indices = d_table;
  g.block_table.indices_count = (uint64_t)table.size();
  g.seq_lens.size = sizeof g.seq_lens;
  g.seq_lens.dtype = KVX_DTYPE_S32;
  g.seq_lens.seq_count = (uint32_t)c.seq_count;
  g.seq_lens.lengths = d_lens;
  g.max_seq_len = (uint32_t)c.seq_len;

  hipDeviceProp_t prop;
  check(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties");
  int driver = 0, runtime = 0;
  check(hipDriverGetVersion(&driver), "hipDriverGetVersion");
  check(hipRuntimeGetVersion(&runtime), "hipRuntimeGetVersion");
  std::printf("GPU: %s, %s, driver %d, runtime %d\n", prop.name, prop.gcnArchName, driver,
              runtime);

  const double write_ms = time_launches(c, "write", [&] { return launch_write(c, &cache, &w); });
  const double gather_ms =
      time_launches(c, "gather", [&] { return launch_gather(c, &cache, &g); });

  const double gib = 1024.0 * 1024.0 * 1024.0;
  const double write_tps = (double)num_tokens / (write_ms / 1e3);
  const double gather_tps = (double)c.seq_count * c.seq_len / (gather_ms / 1e3);
  const double write_gbs = (double)(token_elems * c.elem * 4) / (write_ms / 1e3) / gib;
  const double gather_gbs = (double)(gather_elems * c.elem * 4) / (gather_ms / 1e3) / gib;
  std::printf("write: %.3f ms, %.2f tokens/s, %.2f GB/s\n", write_ms, write_tps, write_gbs);
  std::printf("gather: %.3f ms, %.2f tokens/s, %.2f GB/s\n", gather_ms, gather_tps, gather_gbs);
  std::printf("kernel,seq_count,seq_len,block_size,num_heads,head_dim,num_blocks,"
              "iters,warmup,ms_per,tokens_per_s,gb_per_s,tokens_per_seq\n");
  const char *names[2] = {"write", "gather"};
  const double ms[2] = {write_ms, gather_ms}, tps[2] = {write_tps, gather_tps},
               gbs[2] = {write_gbs, gather_gbs};
  for (int k = 0; k < 2; ++k)
    std::printf("%s,%d,%d,%d,%d,%d,%d,%d,%d,%.6f,%.2f,%.2f,%d\n", names[k], c.seq_count,
                c.seq_len, c.block_size, c.num_heads, c.head_dim, num_blocks, c.iters,
                c.warmup, ms[k], tps[k], gbs[k], c.tokens_per_seq);

  for (void *p : {key, value, kc, vc, ko, vo, d_slots, d_table, d_lens}) (void)hipFree(p);
  return 0;
}
