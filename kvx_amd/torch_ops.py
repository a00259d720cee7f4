"""PyTorch-ROCm op over the KVX launch API (kvx_amd/csrc/torch_ops.cpp).

``load()`` loads ``libkvx_amd_torch.so``, which registers

    torch.ops._C_cache_ops.reshape_and_cache_flash_kvx(
        key, value, key_cache, value_cache, slot_mapping, kv_cache_dtype,
        k_scale, v_scale)

with the schema of the reference's vLLM patch (patches/vllm/kvx.patch:731-740)
as a fragment of vLLM's ``_C_cache_ops`` namespace.  A vLLM-ROCm process that
loads this library finds the op where the patched vLLM looks for it
(kvx.patch:505-507).  There is no fallback: a missing library raises.
"""
from __future__ import annotations

from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libkvx_amd_torch.so"
_LOADED = False


def load(path: str | Path | None = None) -> None:
    """Register the op (once per process)."""
    global _LOADED
    if _LOADED:
        return
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing; build it with `python -m kvx_amd.build`")
    torch.ops.load_library(str(p))
    _LOADED = True


def reshape_and_cache_flash_kvx(key: torch.Tensor, value: torch.Tensor,
                                key_cache: torch.Tensor, value_cache: torch.Tensor,
                                slot_mapping: torch.Tensor, kv_cache_dtype: str = "auto",
                                k_scale: torch.Tensor | None = None,
                                v_scale: torch.Tensor | None = None) -> None:
    """Write key / value rows [T, H, D] into vLLM-shaped caches
    [num_blocks, block_size, H, D] at slot_mapping (slots < 0 skipped), on
    the current stream.  k_scale / v_scale (one-element float32 tensors) are
    used when kv_cache_dtype is "fp8" / "fp8_e4m3"."""
    load()
    one = None
    if k_scale is None or v_scale is None:
        one = torch.ones(1, dtype=torch.float32, device=key.device)
    torch.ops._C_cache_ops.reshape_and_cache_flash_kvx(
        key, value, key_cache, value_cache, slot_mapping, kv_cache_dtype,
        one if k_scale is None else k_scale, one if v_scale is None else v_scale)
