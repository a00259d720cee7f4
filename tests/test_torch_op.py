"""The PyTorch-ROCm op library (kvx_amd/csrc/torch_ops.cpp) on the CPU: it
loads, registers the schema of the reference's vLLM patch
(patches/vllm/kvx.patch:731-740) in vLLM's `_C_cache_ops` namespace, and,
like the reference op (registered for CUDA only), has no CPU kernel."""
import pytest
import torch

from kvx_amd import torch_ops

REF_SCHEMA = ("_C_cache_ops::reshape_and_cache_flash_kvx(Tensor key, Tensor value, "
              "Tensor($0! -> ) key_cache, Tensor($1! -> ) value_cache, Tensor slot_mapping, "
              "str kv_cache_dtype, Tensor k_scale, Tensor v_scale) -> ()")


def test_op_registers_reference_schema():
    torch_ops.load()
    op = torch.ops._C_cache_ops.reshape_and_cache_flash_kvx
    assert str(op.default._schema) == REF_SCHEMA
    # key_cache and value_cache are the mutated arguments
    mutated = [a.name for a in op.default._schema.arguments
               if a.alias_info is not None and a.alias_info.is_write]
    assert mutated == ["key_cache", "value_cache"]


def test_cpu_tensors_have_no_kernel():
    torch_ops.load()
    k = torch.zeros(2, 2, 8)
    cache = torch.zeros(1, 4, 2, 8)
    with pytest.raises(NotImplementedError):
        torch_ops.reshape_and_cache_flash_kvx(k, k, cache, cache.clone(),
                                              torch.zeros(2, dtype=torch.long))


def test_missing_library_raises(tmp_path):
    with pytest.raises(RuntimeError, match="missing"):
        # a path that does not exist, on a fresh loader state
        saved = torch_ops._LOADED
        torch_ops._LOADED = False
        try:
            torch_ops.load(tmp_path / "nope.so")
        finally:
            torch_ops._LOADED = saved
