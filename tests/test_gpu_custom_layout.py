"""GPU parity of KVX_LAYOUT_BLOCK_CUSTOM caches (KVX_SPEC.md:57, :77-78):
tensors whose axes are the logical (block, offset, head, dim) — or (block,
offset, head, dim / x, x) — placed in memory in any order by their strides,
written and gathered through the C ABI bit-identically to the CPU oracle.

Covers vLLM's value-cache layout [num_blocks, H, D, block_size] (token axis
innermost), vLLM's x-packed key layout expressed as CUSTOM, block axis not
outermost, padded strides, K and V in different orders, FP8 and the
kvx_abi.h entry points.
"""
import numpy as np
import pytest
import torch

from kvx_amd import paged
from kvx_amd.abi import DType

from gpu_helpers import (TORCH_DT, check_gather, check_gather_ragged, check_write, custom_cache,
                         random_fill)

pytestmark = pytest.mark.gpu
DEV = "cuda"


ORDERS = [
    ("bhdo", None, "bohd", None),    # vLLM value cache [nb, H, D, bs] / plain NHD
    ("bhpox", 8, "bhdo", None),      # vLLM key cache [nb, H, D/x, bs, x] / value cache
    ("obhd", None, "hbod", None),    # block axis not outermost
    ("bhopx", 4, "bdho", None),      # x-split with dims in other orders
]


@pytest.mark.parametrize("korder,kx,vorder,vx", ORDERS)
@pytest.mark.parametrize("dt", [DType.BF16, DType.F32])
def test_custom_write_then_gather(korder, kx, vorder, vx, dt):
    gen = torch.Generator().manual_seed(len(korder) * 7 + ORDERS.index((korder, kx, vorder, vx)))
    H, D, bs, nb, T = 8, 64, 16, 40, 300
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, korder, vorder, kx, vx, gen,
                              pad=ORDERS.index((korder, kx, vorder, vx)) % 2)
    key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    slots = torch.randperm(nb * bs, generator=gen)[:T]
    slots[torch.rand(T, generator=gen) < 0.1] = -1
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=dt, cache_dtype=dt)
    S, L = 5, 150
    table = torch.randint(-1, nb, (S, (L + bs - 1) // bs), generator=gen).to(torch.int32)
    lens = torch.randint(0, L + 4, (S,), generator=gen).to(torch.int32)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(DEV), lens.to(DEV), L, cache_dtype=dt,
                 io_dtype=dt)


@pytest.mark.parametrize("korder,kx,vorder,vx", ORDERS[:2])
def test_custom_prefill_and_ragged(korder, kx, vorder, vx):
    gen = torch.Generator().manual_seed(71)
    rng = np.random.default_rng(71)
    H, D, bs, nb = 8, 128, 16, 32
    pc, kb, vb = custom_cache(DType.F16, nb, bs, H, D, korder, vorder, kx, vx, gen)
    S, tps = 4, 64
    blocks = torch.randperm(nb, generator=gen)[: S * tps // bs]
    slots = (blocks.repeat_interleave(bs) * bs + torch.arange(bs).repeat(len(blocks))).to(DEV)
    key = random_fill(torch.empty((S * tps, H, D), dtype=torch.float16, device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.F16, cache_dtype=DType.F16,
                tokens_per_seq=tps)
    L = 70
    counts = rng.integers(0, L + 3, size=S)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    indices = rng.integers(-1, nb + 1, size=int(indptr[-1])).astype(np.int32)
    table = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.from_numpy(rng.integers(0, L + 3, size=S).astype(np.int32)).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.float16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=DType.F16,
                        io_dtype=DType.F16)


@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
def test_custom_fp8(fp8):
    gen = torch.Generator().manual_seed(72)
    H, D, bs, nb, T = 8, 128, 16, 24, 200
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhdo", "bhpox", None, 16, gen)
    key = (torch.randn((T, H, D), generator=gen) * 3).bfloat16().to(DEV)
    val = (torch.randn((T, H, D), generator=gen) * 3).bfloat16().to(DEV)
    slots = torch.randperm(nb * bs, generator=gen)[:T].to(DEV)
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.BF16, cache_dtype=fp8,
                k_scale=0.013, v_scale=0.02)
    S, L = 4, 96
    table = torch.randperm(nb, generator=gen)[: S * 6].reshape(S, 6).to(torch.int32).to(DEV)
    lens = torch.tensor([96, 40, 1, 0], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=fp8, io_dtype=DType.BF16,
                 k_scale=0.013, v_scale=0.02)


def test_custom_abi_entry_points():
    """kvx_write_kv / kvx_gather_kv accept CUSTOM caches (K and V must share
    the layout code, kvx_abi.c:336-338)."""
    gen = torch.Generator().manual_seed(73)
    H, D, bs, nb, T = 4, 64, 16, 16, 64
    pc, kb, vb = custom_cache(DType.BF16, nb, bs, H, D, "bhdo", "obhd", gen=gen)
    key = random_fill(torch.empty((T, H, D), dtype=torch.bfloat16, device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    slots = torch.randperm(nb * bs, generator=gen)[:T].to(DEV)
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.BF16, cache_dtype=DType.BF16,
                entry="abi")
    table = torch.arange(nb, dtype=torch.int32, device=DEV).reshape(4, 4)
    lens = torch.tensor([64, 30, 9, 0], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((4, 64, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, 64, cache_dtype=DType.BF16,
                 io_dtype=DType.BF16, entry="abi")
