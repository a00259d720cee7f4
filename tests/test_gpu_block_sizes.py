"""GPU parity of blocks at the ends of the block-size range, through the C
ABI, bit-identical to the CPU oracle (kernels/kvx_paged_kv.cu:93-124 write
and :226-267 gather semantics).

Blocks of one token, and HND caches of one head: every such dense layout
stores a row as H * D consecutive elements and takes the row-major kernels (write_flat_kernel, gather_flat_kernel, the RAGGED tile
and KV_OFFSETS flat gathers), for copies and FP8 casts.

Blocks of 128 and 256 tokens take paths that smaller ones do not:
  gather_rows_kernel   a block's rows split over several workgroups (HND
      rows whose 64 KiB tile does not fit LDS, padded blocks, FP8 heads of
      40 bytes with the dequantizing op), parts that start past seq_len,
      parts cut by seq_len, and ids < 0 or >= num_blocks;
  gather_tiles_kernel  tiles of one 128-byte line per row (x-packed and
      token-innermost blocks, 16 and 32 KiB tiles) and 32 KiB HND tiles.
"""
import pytest
import torch

from kvx_amd.abi import DType, ScaleGranularity as SG

import numpy as np

from kvx_amd import paged
from kvx_amd.abi import Layout

from gpu_helpers import (TORCH_DT, OffsetsPool, ScaleArg, check_gather, check_gather_offsets,
                         check_gather_ragged, check_write, custom_cache, random_fill)

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (cache dtype, K order, K x, V order, V x, block_size, H, D, pad)
CASES = [
    (DType.BF16, "bhod", None, "bhod", None, 256, 8, 128, 0),   # HND: row kernel, split
    (DType.BF16, "bhod", None, "bhod", None, 128, 8, 128, 0),   # HND: 32 KiB tiles
    (DType.BF16, "bhpox", 8, "bohd", None, 256, 8, 128, 0),     # x-packed: 128-byte tiles
    (DType.BF16, "bhdo", None, "bhpox", 8, 128, 8, 128, 0),     # token-innermost / x-packed
    (DType.F16, "obhd", None, "hbod", None, 128, 4, 64, 1),     # padded: row kernel, split
    (DType.F32, "bhod", None, "bohd", None, 256, 2, 64, 0),     # 512-byte HND runs, NHD V
]


def _ids(c):
    return f"{c[0].name}-{c[1]}{c[2] or ''}-{c[3]}{c[4] or ''}-bs{c[5]}-H{c[6]}-D{c[7]}-pad{c[8]}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
@pytest.mark.parametrize("idx64", [False, True])
def test_big_block_gather(case, idx64):
    dt, ko_, kx, vo_, vx, bs, H, D, pad = case
    gen = torch.Generator().manual_seed(900 + CASES.index(case) * 2 + int(idx64))
    nb = 10
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen, pad=pad)
    S = 4
    L = 2 * bs + bs // 2 + 3  # a partial last block
    mbps = (L + bs - 1) // bs
    table = torch.randint(0, nb, (S, mbps), generator=gen)
    table[1, 0], table[2, 1] = -1, nb + 1
    # a full row, one past max_seq_len, lengths that end inside a block's
    # first, middle and last parts
    lens = torch.tensor([L, L + bs, bs + 5, 2 * bs - 3])
    itype = torch.int64 if idx64 else torch.int32
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(itype).to(DEV), lens.to(itype).to(DEV), L,
                 cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("kind", ["tensor", SG.PER_BLOCK_HEAD])
@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
def test_big_block_dequant_row_split(fp8, kind):
    """FP8 HND heads of 40 bytes (no 16-byte pieces for a tile) in blocks of
    256 tokens: the dequantizing row kernel, each block in two parts."""
    gen = torch.Generator().manual_seed(950 + int(fp8) + 2 * (kind != "tensor"))
    H, D, bs, nb = 8, 40, 256, 8
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhod", "bhod", None, None, gen)
    S, L = 3, 2 * bs + 17
    table = torch.randint(-1, nb, (S, (L + bs - 1) // bs), generator=gen).to(torch.int32)
    lens = torch.tensor([L, 300, 9], dtype=torch.int32)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    if kind == "tensor":
        ks, vs = 0.021, 0.0043
    else:
        ks, vs = (ScaleArg(kind, torch.empty(nb, H).uniform_(0.002, 0.05, generator=gen).numpy(),
                           stride=(1, nb)) for _ in range(2))
    check_gather(pc, kb, vb, ko, vo, table.to(DEV), lens.to(DEV), L, cache_dtype=fp8,
                 io_dtype=DType.BF16, k_scale=ks, v_scale=vs)


ONE = [("bhod", None, "bhod", None), ("bhpox", 8, "bhdo", None), ("bhdo", None, "bohd", None)]


@pytest.mark.parametrize("orders", ONE, ids=["hnd", "xpacked-tokinner", "tokinner-nhd"])
@pytest.mark.parametrize("dt", [DType.BF16, DType.F8_E4M3])
def test_one_token_blocks(orders, dt):
    """Decode and prefill writes, PACKED and RAGGED gathers of blocks of one
    token; FP8 caches quantize bf16 rows and dequantize to bf16."""
    ko_, kx, vo_, vx = orders
    seed = 980 + ONE.index(orders) * 2 + (dt != DType.BF16)
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    H, D, nb = 8, 64, 600
    pc, kb, vb = custom_cache(dt, nb, 1, H, D, ko_, vo_, kx, vx, gen)
    fp8 = dt != DType.BF16
    io = DType.BF16
    ks, vs = (0.013, 0.0071) if fp8 else (None, None)
    # decode: scattered slots, some -1 or past the pool
    T = 37
    slots = torch.randperm(nb, generator=gen)[:T]
    slots[3], slots[8] = -1, nb + 2
    key = (torch.randn((T, H, D), generator=gen) * 2).to(torch.bfloat16).to(DEV)
    val = torch.randn((T, H, D), generator=gen).to(torch.bfloat16).to(DEV)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=io, cache_dtype=dt,
                k_scale=ks, v_scale=vs)
    # prefill: 3 chunks of 64 tokens, each on its own random blocks
    S, tps = 3, 64
    ids = torch.randperm(nb, generator=gen)[: S * tps]
    key = (torch.randn((S * tps, H, D), generator=gen) * 2).to(torch.bfloat16).to(DEV)
    val = torch.randn((S * tps, H, D), generator=gen).to(torch.bfloat16).to(DEV)
    check_write(pc, kb, vb, key, val, ids.to(DEV), io_dtype=io, cache_dtype=dt,
                tokens_per_seq=tps, k_scale=ks, v_scale=vs)
    # PACKED and RAGGED gathers of those sequences, plus invalid ids
    L = tps + 3
    table = torch.full((S, L), -1, dtype=torch.int32)
    table[:, :tps] = ids.reshape(S, tps).to(torch.int32)
    table[1, 5], table[2, 9] = -1, nb + 1
    lens = torch.tensor([L, tps, 17], dtype=torch.int32)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(DEV), lens.to(DEV), L, cache_dtype=dt,
                 io_dtype=io, k_scale=ks, v_scale=vs)
    counts = rng.integers(0, L + 3, size=S)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    indices = rng.integers(-1, nb + 2, size=max(int(indptr[-1]), 1)).astype(np.int32)
    rt = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_ragged(pc, kb, vb, ko, vo, rt, lens.to(DEV), L, cache_dtype=dt, io_dtype=io,
                        k_scale=ks, v_scale=vs)


@pytest.mark.parametrize("layout", [Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED])
@pytest.mark.parametrize("dt", [DType.BF16, DType.F8_E5M2])
def test_one_token_blocks_kv_offsets(layout, dt):
    """KV_OFFSETS gathers of one-token HND / x-packed blocks from a primary
    and a secondary pool."""
    seed = 990 + (layout == Layout.BLOCK_HND_PACKED) * 2 + (dt != DType.BF16)
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    H, D, nb, S, L = 4, 128, 300, 4, 50
    pool = OffsetsPool(layout, layout, dt, nb, 1, H, D, pitch_pad=16, gen=gen)
    raw = rng.integers(0, nb + 2, size=(S, 1, 2, L)).astype(np.uint32)
    raw |= (rng.random(raw.shape) < 0.3).astype(np.uint32) << 31
    offsets = torch.from_numpy(raw.view(np.int32)).to(DEV)
    lens = torch.from_numpy(rng.integers(-1, L + 4, size=S).astype(np.int32)).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = (0.02, 0.005) if dt != DType.BF16 else (None, None)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=DType.BF16,
                         k_scale=ks, v_scale=vs)


HEAD1 = [("bhod", None, "bhod", None), ("bhpox", 8, "bhdo", None), ("bhpox", 8, "bohd", None)]


@pytest.mark.parametrize("orders", HEAD1, ids=["hnd", "vllm-pair", "xpacked-nhd"])
@pytest.mark.parametrize("dt", [DType.BF16, DType.F8_E4M3])
def test_one_head(orders, dt):
    """One KV head (a tensor-parallel rank's shard): HND is then row-major
    (flat kernels); x-packed and token-innermost blocks make 4 KiB tiles
    (128-thread workgroups).  Decode and prefill writes, PACKED and RAGGED
    gathers."""
    ko_, kx, vo_, vx = orders
    seed = 1010 + HEAD1.index(orders) * 2 + (dt != DType.BF16)
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    H, D, bs, nb = 1, 128, 16, 64
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    ks, vs = (0.013, 0.0071) if dt != DType.BF16 else (None, None)
    T = 29
    slots = torch.randperm(nb * bs, generator=gen)[:T]
    slots[4] = -1
    key = (torch.randn((T, H, D), generator=gen) * 2).to(torch.bfloat16).to(DEV)
    val = torch.randn((T, H, D), generator=gen).to(torch.bfloat16).to(DEV)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=DType.BF16, cache_dtype=dt,
                k_scale=ks, v_scale=vs)
    S, tps = 3, 40
    blocks = torch.randperm(nb, generator=gen)[: S * 4].reshape(S, 4)
    pos = torch.arange(tps) + 5  # chunks starting inside their first block
    ids = torch.cat([blocks[s, pos // bs] * bs + pos % bs for s in range(S)])
    key = (torch.randn((S * tps, H, D), generator=gen) * 2).to(torch.bfloat16).to(DEV)
    val = torch.randn((S * tps, H, D), generator=gen).to(torch.bfloat16).to(DEV)
    check_write(pc, kb, vb, key, val, ids.to(DEV), io_dtype=DType.BF16, cache_dtype=dt,
                tokens_per_seq=tps, k_scale=ks, v_scale=vs)
    L = 4 * bs
    table = blocks.to(torch.int32)
    table[1, 2] = -1
    lens = torch.tensor([L, tps + 5, 7], dtype=torch.int32)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(DEV), lens.to(DEV), L, cache_dtype=dt,
                 io_dtype=DType.BF16, k_scale=ks, v_scale=vs)
    counts = rng.integers(0, L + 3, size=S)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    indices = rng.integers(-1, nb + 2, size=max(int(indptr[-1]), 1)).astype(np.int32)
    rt = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_ragged(pc, kb, vb, ko, vo, rt, lens.to(DEV), L, cache_dtype=dt,
                        io_dtype=DType.BF16, k_scale=ks, v_scale=vs)


# PACKED gathers of caches whose heads are contiguous runs of whole 128-byte
# lines, in blocks of 64 tokens or more, take gather_flat_kernel with
# head-run addressing (row, head, chunk of the head, any row and head
# strides).  (cache dtype, K order, V order, block_size, H, D, pad, scales)
HEAD_RUNS = [
    (DType.BF16, "bhod", "bhod", 64, 8, 128, 0, None),             # HND
    (DType.BF16, "bhod", "bohd", 128, 8, 128, 0, None),            # HND K, NHD V
    (DType.F16, "bhod", "bhod", 256, 4, 64, 3, None),              # padded head runs
    (DType.F32, "obhd", "bhod", 64, 2, 32, 0, None),               # offset axis outermost
    (DType.F8_E4M3, "bhod", "bhod", 128, 4, 128, 0, "tensor"),     # dequantizing
    (DType.F8_E5M2, "bhod", "bhod", 64, 8, 128, 0, SG.PER_HEAD),
    (DType.F8_E4M3, "bhod", "bohd", 256, 2, 128, 0, SG.PER_BLOCK_HEAD),
]


def _hr_ids(c):
    return f"{c[0].name}-{c[1]}-{c[2]}-bs{c[3]}-H{c[4]}-D{c[5]}-pad{c[6]}-{getattr(c[7], 'name', c[7])}"


@pytest.mark.parametrize("case", HEAD_RUNS, ids=[_hr_ids(c) for c in HEAD_RUNS])
@pytest.mark.parametrize("idx64", [False, True])
def test_head_run_flat_gather(case, idx64):
    dt, ko_, vo_, bs, H, D, pad, kind = case
    gen = torch.Generator().manual_seed(1500 + HEAD_RUNS.index(case) * 2 + int(idx64))
    nb = 9
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, None, None, gen, pad=pad)
    S = 5
    L = 3 * bs + bs // 2 + 3  # a partial last block
    mbps = (L + bs - 1) // bs
    table = torch.randint(0, nb, (S, mbps), generator=gen)
    table[1, 0], table[2, 2], table[3, 1] = -1, nb + 1, nb
    lens = torch.tensor([L, L + bs, bs + 5, 2 * bs - 3, 0])
    itype = torch.int64 if idx64 else torch.int32
    io = DType.BF16 if dt in (DType.F8_E4M3, DType.F8_E5M2) else dt
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks = vs = None
    if kind == "tensor":
        ks, vs = 0.0173, 0.0061
    elif kind == SG.PER_HEAD:
        ks, vs = (ScaleArg(kind, torch.empty(H).uniform_(0.002, 0.05, generator=gen).numpy())
                  for _ in range(2))
    elif kind is not None:
        ks, vs = (ScaleArg(kind, torch.empty(nb, H).uniform_(0.002, 0.05, generator=gen).numpy(),
                           stride=(1, nb)) for _ in range(2))
    check_gather(pc, kb, vb, ko, vo, table.to(itype).to(DEV), lens.to(itype).to(DEV), L,
                 cache_dtype=dt, io_dtype=io, k_scale=ks, v_scale=vs)


# RAGGED gathers of dense blocks of more than 64 tokens in the LDS tiles:
# every thread loads row ids, and one barrier tells whether a tile names one
# block.  (cache dtype, K order, K x, V order, V x, block_size, H, D)
RAGGED_BIG = [
    (DType.BF16, "bhpox", 8, "bohd", None, 128, 8, 128),     # x-packed K, NHD V
    (DType.BF16, "bhpox", 8, "bhdo", None, 256, 4, 64),      # vLLM's pair
    (DType.BF16, "bhod", None, "bhod", None, 128, 8, 128),   # HND: the row kernel
    (DType.F8_E4M3, "bhpox", 16, "bhpox", 16, 128, 4, 128),  # FP8, dequantizing
]


@pytest.mark.parametrize("case", RAGGED_BIG, ids=[
    f"{c[0].name}-{c[1]}{c[2] or ''}-{c[3]}{c[4] or ''}-bs{c[5]}-H{c[6]}-D{c[7]}"
    for c in RAGGED_BIG])
@pytest.mark.parametrize("spoil", [False, True])
def test_ragged_big_block_tiles(case, spoil):
    dt, ko_, kx, vo_, vx, bs, H, D = case
    idx = RAGGED_BIG.index(case)
    rng = np.random.default_rng(1600 + 2 * idx + int(spoil))
    gen = torch.Generator().manual_seed(1600 + 2 * idx + int(spoil))
    nb = 7
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    S = 4
    L = 2 * bs + bs // 2 + 3
    counts = np.array([L, bs + 7, 0, L + 5])
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    parts = []
    for c in counts:
        blocks = rng.integers(0, nb, size=(int(c) + bs - 1) // bs + 1)
        parts.append(blocks[np.arange(c) // bs])  # each block's tokens in order
    indices = np.concatenate(parts).astype(np.int32)
    if spoil:  # tiles whose rows name several blocks, or none
        bad = rng.choice(indices.size, size=24, replace=False)
        indices[bad] = rng.choice([-1, nb, nb + 3, 2], size=24)
        indices[indptr[1]: indptr[1] + bs] = -1  # a whole block's rows skipped
    rt = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.tensor([L, L, 3, L], dtype=torch.int32, device=DEV)
    io = DType.BF16 if dt == DType.F8_E4M3 else dt
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = (0.0213, 0.0047) if dt == DType.F8_E4M3 else (None, None)
    check_gather_ragged(pc, kb, vb, ko, vo, rt, lens, L, cache_dtype=dt, io_dtype=io,
                        k_scale=ks, v_scale=vs)
