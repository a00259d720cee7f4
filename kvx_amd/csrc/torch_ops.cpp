// PyTorch-ROCm custom op over the KVX launch API, so that vLLM on ROCm can
// route its paged-cache write to libkvx_amd.so.
//
// Op and schema follow the reference's vLLM patch
// (patches/vllm/kvx.patch:176-275 implementation, :731-740 registration):
//
//   _C_cache_ops::reshape_and_cache_flash_kvx(
//       Tensor key, Tensor value, Tensor! key_cache, Tensor! value_cache,
//       Tensor slot_mapping, str kv_cache_dtype, Tensor k_scale,
//       Tensor v_scale) -> ()
//
// registered as a TORCH_LIBRARY_FRAGMENT of vLLM's `_C_cache_ops` namespace,
// so vLLM's own availability test (kvx.patch:505-507) finds it once this
// library is loaded.  The checks follow the reference op's order and
// messages.  Where this op differs, it follows vLLM's reshape_and_cache_flash,
// the op being replaced:
//   - The cache is vLLM's logical [num_blocks, block_size, num_heads,
//     head_size] view with whatever strides it has (contiguous NHD, or the
//     stride-permuted view vLLM uses for an HND cache), described to the
//     library as BLOCK_NHD with those strides.  The reference op infers HND
//     from the head stride and then reads block_size from size(2)
//     (kvx.patch:221-227), which misplaces rows of a permuted HND view.
//   - Rows past slot_mapping.size(0) in key / value are ignored, as in vLLM
//     (num_actual_tokens); the reference op fails on them.
//   - kv_cache_dtype "fp8" / "fp8_e4m3" writes an E4M3 cache (uint8 or
//     float8_e4m3fn tensor) and "fp8_e5m2" an E5M2 cache (uint8 or
//     float8_e5m2 tensor), with q = fp8(sat(x / scale)); the reference op
//     accepts only "auto".
#include <ATen/ATen.h>
// PyTorch-ROCm reports GPU tensors as device type "cuda": its device guard
// and stream accessors for such tensors are the *MasqueradingAsCUDA ones.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <string>

#include "kvx_paged_kv.h"

namespace {

kvx_dtype_t io_dtype(at::ScalarType t) {
  switch (t) {
    case at::ScalarType::Float: return KVX_DTYPE_F32;
    case at::ScalarType::Half: return KVX_DTYPE_F16;
    case at::ScalarType::BFloat16: return KVX_DTYPE_BF16;
    default: return KVX_DTYPE_INVALID;
  }
}

kvx_dtype_t slot_dtype(at::ScalarType t) {
  switch (t) {
    case at::ScalarType::Int: return KVX_DTYPE_S32;
    case at::ScalarType::Long: return KVX_DTYPE_S64;
    default: return KVX_DTYPE_INVALID;
  }
}

bool is_fp8_cache(at::ScalarType t, kvx_dtype_t fmt) {
  if (t == at::ScalarType::Byte) return true;
  return fmt == KVX_DTYPE_F8_E5M2 ? t == at::ScalarType::Float8_e5m2
                                  : t == at::ScalarType::Float8_e4m3fn;
}

void describe(kvx_tensor_desc_t *d, const at::Tensor &t, kvx_dtype_t dtype,
              kvx_layout_t layout, int64_t rows = -1) {
  *d = kvx_tensor_desc_t{};
  d->size = sizeof(kvx_tensor_desc_t);
  d->dtype = dtype;
  d->layout = layout;
  d->memory = KVX_MEMORY_DEVICE;
  d->ndim = static_cast<uint32_t>(t.dim());
  for (int64_t i = 0; i < t.dim() && i < KVX_MAX_TENSOR_DIMS; ++i) {
    d->shape[i] = t.size(i);
    d->stride[i] = t.stride(i);
  }
  if (rows >= 0) d->shape[0] = rows;
  d->data = t.data_ptr();
}

void reshape_and_cache_flash_kvx(const at::Tensor &key, const at::Tensor &value,
                                 at::Tensor &key_cache, at::Tensor &value_cache,
                                 const at::Tensor &slot_mapping,
                                 const std::string &kv_cache_dtype, const at::Tensor &k_scale,
                                 const at::Tensor &v_scale) {
  const bool e5m2 = kv_cache_dtype == "fp8_e5m2";
  const bool fp8 = kv_cache_dtype == "fp8" || kv_cache_dtype == "fp8_e4m3" || e5m2;
  TORCH_CHECK(kv_cache_dtype == "auto" || fp8,
              "KVX cache write supports kv_cache_dtype auto, fp8, fp8_e4m3 and fp8_e5m2, not ",
              kv_cache_dtype);
  TORCH_CHECK(key.is_cuda() && value.is_cuda(), "key/value must be CUDA tensors");
  TORCH_CHECK(key_cache.is_cuda() && value_cache.is_cuda(),
              "cache tensors must be CUDA tensors");
  TORCH_CHECK(key.scalar_type() == value.scalar_type(), "key/value dtype mismatch");
  TORCH_CHECK(key_cache.scalar_type() == value_cache.scalar_type(), "cache dtype mismatch");
  TORCH_CHECK(key.dim() == 3 && value.dim() == 3,
              "key/value must be [num_tokens, num_heads, head_dim]");

  const kvx_dtype_t dt = io_dtype(key.scalar_type());
  TORCH_CHECK(dt != KVX_DTYPE_INVALID, "KVX cache write unsupported dtype");
  kvx_dtype_t cache_dt = dt;
  if (fp8) {
    cache_dt = e5m2 ? KVX_DTYPE_F8_E5M2 : KVX_DTYPE_F8_E4M3;
    TORCH_CHECK(is_fp8_cache(key_cache.scalar_type(), cache_dt),
                "fp8 kv_cache_dtype needs a uint8 or matching float8 cache");
  } else {
    TORCH_CHECK(key_cache.scalar_type() == key.scalar_type(),
                "key/value dtype must match cache dtype");
  }

  const kvx_dtype_t sdt = slot_dtype(slot_mapping.scalar_type());
  TORCH_CHECK(sdt != KVX_DTYPE_INVALID, "slot_mapping must be int32 or int64");
  TORCH_CHECK(slot_mapping.dim() == 1, "slot_mapping must be 1D");
  TORCH_CHECK(slot_mapping.is_cuda() && slot_mapping.is_contiguous(),
              "slot_mapping must be a contiguous CUDA tensor");

  const int64_t num_tokens = slot_mapping.size(0);
  const int64_t num_heads = key.size(1);
  const int64_t head_dim = key.size(2);
  TORCH_CHECK(key.stride(2) == 1 && key.stride(1) == head_dim &&
                  key.stride(0) == num_heads * head_dim,
              "key must be contiguous [token, head, dim]");
  TORCH_CHECK(value.stride(2) == 1 && value.stride(1) == head_dim &&
                  value.stride(0) == num_heads * head_dim,
              "value must be contiguous [token, head, dim]");
  TORCH_CHECK(value.size(1) == num_heads && value.size(2) == head_dim,
              "key/value shape mismatch");
  TORCH_CHECK(key.size(0) >= num_tokens && value.size(0) >= num_tokens,
              "key/value have fewer rows than slot_mapping");

  TORCH_CHECK(key_cache.dim() == 4,
              "cache must be [num_blocks, block_size, num_heads, head_size]");
  TORCH_CHECK(key_cache.size(2) == num_heads, "cache num_heads must match key/value");
  TORCH_CHECK(key_cache.size(3) == head_dim, "cache head_dim must match key/value");
  TORCH_CHECK(key_cache.sizes() == value_cache.sizes(), "key/value cache shape mismatch");
  TORCH_CHECK(key_cache.strides() == value_cache.strides(), "key/value cache stride mismatch");

  const float *ks = nullptr;
  const float *vs = nullptr;
  if (fp8) {
    TORCH_CHECK(k_scale.defined() && v_scale.defined() && k_scale.numel() == 1 &&
                    v_scale.numel() == 1 && k_scale.scalar_type() == at::ScalarType::Float &&
                    v_scale.scalar_type() == at::ScalarType::Float && k_scale.is_cuda() &&
                    v_scale.is_cuda(),
                "fp8 kv_cache_dtype needs one-element float32 CUDA k_scale / v_scale");
    ks = k_scale.data_ptr<float>();
    vs = v_scale.data_ptr<float>();
  }

  kvx_cache_desc_t cache{};
  cache.size = sizeof(kvx_cache_desc_t);
  cache.num_blocks = static_cast<uint32_t>(key_cache.size(0));
  cache.block_size = static_cast<uint32_t>(key_cache.size(1));
  cache.num_kv_heads = static_cast<uint32_t>(num_heads);
  cache.head_dim = static_cast<uint32_t>(head_dim);
  describe(&cache.k, key_cache, cache_dt, KVX_LAYOUT_BLOCK_NHD);
  describe(&cache.v, value_cache, cache_dt, KVX_LAYOUT_BLOCK_NHD);

  kvx_write_desc_t write{};
  write.size = sizeof(kvx_write_desc_t);
  write.io.size = sizeof(kvx_kv_io_desc_t);
  write.io.num_tokens = static_cast<uint32_t>(num_tokens);
  write.io.num_kv_heads = static_cast<uint32_t>(num_heads);
  write.io.head_dim = static_cast<uint32_t>(head_dim);
  describe(&write.io.key, key, dt, KVX_LAYOUT_INVALID, num_tokens);
  describe(&write.io.value, value, dt, KVX_LAYOUT_INVALID, num_tokens);
  write.slots.size = sizeof(kvx_slot_mapping_t);
  write.slots.dtype = sdt;
  write.slots.token_count = static_cast<uint32_t>(num_tokens);
  write.slots.invalid_slot = -1;
  write.slots.slots = slot_mapping.data_ptr();
  write.k_scale = ks;
  write.v_scale = vs;
  write.k_scale_desc.size = sizeof(kvx_scale_desc_t);
  write.v_scale_desc.size = sizeof(kvx_scale_desc_t);

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
  void *stream =
      reinterpret_cast<void *>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  const kvx_status_t status = kvx_launch_write_kv(&cache, &write, stream);
  TORCH_CHECK(status == KVX_STATUS_OK,
              "kvx cache write failed with status=", static_cast<int>(status));
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(_C_cache_ops, m) {
  m.def(
      "reshape_and_cache_flash_kvx(Tensor key, Tensor value, Tensor! key_cache, "
      "Tensor! value_cache, Tensor slot_mapping, str kv_cache_dtype, Tensor k_scale, "
      "Tensor v_scale) -> ()");
}

TORCH_LIBRARY_IMPL(_C_cache_ops, CUDA, m) {
  m.impl("reshape_and_cache_flash_kvx", &reshape_and_cache_flash_kvx);
}
