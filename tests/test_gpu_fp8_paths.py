"""GPU parity of the FP8 casts on the kernel paths that only some shapes
reach, through the C ABI, bit-identical to the CPU oracle:

  write_kernel with the quantizing op   a decode write (fewer tokens than
      block_size, so no whole block for the tiled write) into caches whose
      rows are not contiguous: HND, x-packed, and vLLM's value cache
      [num_blocks, H, D, block_size] (CUSTOM);
  gather_rows_kernel with the dequantizing op   PACKED gathers of HND
      caches whose heads are 40 FP8 bytes (runs the LDS tile kernel cannot
      cut into 16-byte pieces);
  gather_indexed_kernel with the dequantizing op   RAGGED and KV_OFFSETS
      gathers of the same caches;
  gather_tiles_kernel with odd tiles   PACKED, RAGGED and KV_OFFSETS
      gathers of HND caches with 96-byte runs (head_dim 96) or rows of six
      64-byte runs, whose tile widths are not a power of two.

Each runs E4M3 and E5M2 with per-tensor, per-head and (where the table
format allows) per-block and per-block-head scales.
"""
import numpy as np
import pytest
import torch

from kvx_amd import paged
from kvx_amd.abi import DType, Layout, ScaleGranularity as SG

from gpu_helpers import (TORCH_DT, OffsetsPool, ScaleArg, check_gather, check_gather_offsets,
                         check_gather_ragged, check_write, custom_cache, make_cache,
                         random_fill)

pytestmark = pytest.mark.gpu
DEV = "cuda"
NHD, HND, PK = Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED
FP8 = [DType.F8_E4M3, DType.F8_E5M2]
KINDS = ["tensor", "head", "block", "block_head"]


def rows(T, H, D, io, gen, sigma):
    return (torch.randn((T, H, D), generator=gen) * sigma).to(TORCH_DT[io]).to(DEV)


def scales(kind, gen, nb, H):
    """(K scale, V scale): floats for per-tensor, else ScaleArgs with
    padded strides."""
    if kind == "tensor":
        return 0.013, 0.0071
    shape = {"head": (H,), "block": (nb,), "block_head": (nb, H)}[kind]
    g = {"head": SG.PER_HEAD, "block": SG.PER_BLOCK, "block_head": SG.PER_BLOCK_HEAD}[kind]
    stride = {"head": (3,), "block": (2,), "block_head": (1, nb)}[kind]
    out = []
    for _ in range(2):
        v = torch.empty(shape).uniform_(0.002, 0.05, generator=gen).numpy()
        out.append(ScaleArg(g, v, stride=stride))
    return tuple(out)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("fp8", FP8)
@pytest.mark.parametrize("layout", ["hnd", "packed", "vllm_v"])
def test_quantizing_decode_write_token_path(layout, fp8, kind):
    gen = torch.Generator().manual_seed(50 + KINDS.index(kind) + 4 * FP8.index(fp8))
    H, D, bs, nb, T = 8, 128, 16, 40, 11  # T < bs: no whole block
    if layout == "vllm_v":
        pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhdo", "bhdo", gen=gen)
    else:
        lay = {"hnd": HND, "packed": PK}[layout]
        pc, kb, vb = make_cache(lay, lay, fp8, nb, bs, H, D, pack=16, gen=gen)
    io = [DType.BF16, DType.F16, DType.F32][KINDS.index(kind) % 3]
    key, val = rows(T, H, D, io, gen, 2.0), rows(T, H, D, io, gen, 0.3)
    slots = torch.randperm(nb * bs, generator=gen)[:T]
    slots[3] = -1
    ks, vs = scales(kind, gen, nb, H)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=io, cache_dtype=fp8,
                k_scale=ks, v_scale=vs)


# FP8 rows of 768, 384 and 160 bytes: not powers of two
SHAPES = [(8, 96), (6, 64), (4, 40)]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("fp8", FP8)
@pytest.mark.parametrize("shape", SHAPES)
def test_dequantizing_packed_gather_row_path(shape, fp8, kind):
    H, D = shape
    gen = torch.Generator().manual_seed(60 + KINDS.index(kind) + 4 * FP8.index(fp8) + 8 * H)
    bs, nb, S, L = 16, 30, 5, 100
    pc, kb, vb = make_cache(HND, HND, fp8, nb, bs, H, D, gen=gen)
    io = [DType.BF16, DType.F32, DType.F16][KINDS.index(kind) % 3]
    table = torch.randint(-1, nb + 2, (S, (L + bs - 1) // bs), generator=gen)
    table = table.to(torch.int32).to(DEV)
    lens = torch.randint(-1, L + 5, (S,), generator=gen).to(torch.int32).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = scales(kind, gen, nb, H)
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=fp8, io_dtype=io,
                 k_scale=ks, v_scale=vs)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("fp8", FP8)
@pytest.mark.parametrize("shape", SHAPES)
def test_dequantizing_ragged_gather_indexed_path(shape, fp8, kind):
    H, D = shape
    rng = np.random.default_rng(70 + KINDS.index(kind) + 4 * FP8.index(fp8) + 8 * H)
    gen = torch.Generator().manual_seed(70 + KINDS.index(kind))
    bs, nb, S, L = 16, 30, 4, 80
    pc, kb, vb = make_cache(HND, HND, fp8, nb, bs, H, D, gen=gen)
    io = [DType.F16, DType.BF16, DType.F32][KINDS.index(kind) % 3]
    counts = rng.integers(0, L + 4, size=S)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    indices = rng.integers(-1, nb + 2, size=max(int(indptr[-1]), 1)).astype(np.int32)
    table = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.from_numpy(rng.integers(-1, L + 4, size=S).astype(np.int32)).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = scales(kind, gen, nb, H)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=fp8, io_dtype=io,
                        k_scale=ks, v_scale=vs)


@pytest.mark.parametrize("kind", ["tensor", "head"])  # block-indexed: UNSUPPORTED here
@pytest.mark.parametrize("fp8", FP8)
@pytest.mark.parametrize("shape", SHAPES)
def test_dequantizing_kv_offsets_gather_indexed_path(shape, fp8, kind):
    H, D = shape
    rng = np.random.default_rng(80 + 4 * FP8.index(fp8) + 8 * H)
    gen = torch.Generator().manual_seed(80 + len(kind))
    bs, nb, S, L = 16, 30, 4, 80
    pool = OffsetsPool(HND, HND, fp8, nb, bs, H, D, pitch_pad=32, gen=gen)
    mbps = (L + bs - 1) // bs
    raw = rng.integers(0, nb + 2, size=(S, 1, 2, mbps)).astype(np.uint32)
    raw |= (rng.random(raw.shape) < 0.3).astype(np.uint32) << 31
    offsets = torch.from_numpy(raw.view(np.int32)).to(DEV)
    lens = torch.from_numpy(rng.integers(-1, L + 4, size=S).astype(np.int32)).to(DEV)
    io = DType.BF16 if kind == "tensor" else DType.F32
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = scales(kind, gen, nb, H)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=fp8, io_dtype=io,
                         k_scale=ks, v_scale=vs)


@pytest.mark.parametrize("kind", ["tensor", "head"])
@pytest.mark.parametrize("fp8", FP8)
@pytest.mark.parametrize("shape", [(1, 128), (1, 64), (2, 64)])
def test_dequantizing_kv_offsets_tile_sized_workgroups(shape, fp8, kind):
    """KV_OFFSETS dequantizing gathers of row-major blocks of one or two
    heads: tiles of 16 rows of 64-256 bytes, in workgroups of 128 or 64
    threads (one pass of four 8-byte chunks per thread)."""
    H, D = shape
    rng = np.random.default_rng(1700 + 4 * FP8.index(fp8) + 8 * H + D)
    gen = torch.Generator().manual_seed(1700 + len(kind) + D)
    bs, nb, S, L = 16, 40, 5, 150
    pool = OffsetsPool(Layout.BLOCK_NHD, Layout.BLOCK_NHD, fp8, nb, bs, H, D, pitch_pad=16,
                       gen=gen)
    mbps = (L + bs - 1) // bs
    raw = rng.integers(0, nb + 2, size=(S, 1, 2, mbps)).astype(np.uint32)
    raw |= (rng.random(raw.shape) < 0.3).astype(np.uint32) << 31
    offsets = torch.from_numpy(raw.view(np.int32)).to(DEV)
    lens = torch.tensor([L, L - 9, bs + 1, 0, L + 7], dtype=torch.int32, device=DEV)
    io = DType.BF16 if kind == "tensor" else DType.F16
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = scales(kind, gen, nb, H)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=fp8, io_dtype=io,
                         k_scale=ks, v_scale=vs)
