"""GPU parity of the gathers over long sequences of many workgroups, bit-
identical to the CPU oracle (kernels/kvx_paged_kv.cu:226-267 gather
semantics; KVX_SPEC.md:99-122 for the indexed tables).

gather_flat_kernel (PACKED) takes two units of its sequence per workgroup
when a sequence has 4096 to 65536 units, a unit being one power-of-two
share of a block: unit w and unit w + J of sequence s, J the workgroups per
sequence.  RAGGED copies in gather_ragged_tile_kernel take two tiles per
workgroup the same way from 8192 to 65536 tiles per sequence (the 8197- and
40001-tile cases); the flat indexed and transposing gathers keep one tile
per workgroup.  The indexed and transposing cases cover 513 to 40001 tiles
per sequence.

Lengths cover both units of a workgroup valid, the second one cut inside
its block or part, the second one starting exactly at seq_len (the
boundary J * block_size / parts), the first one cut, an empty sequence, a
length past max_seq_len, tables narrower than max_seq_len, and block ids
< 0 or >= num_blocks in either half of a sequence.
"""
import pytest
import torch

from kvx_amd.abi import DType, Layout, ScaleGranularity as SG

from gpu_helpers import ScaleArg, TORCH_DT, check_gather, make_cache, random_fill

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (cache dtype, io dtype, H, D, block_size, blocks per sequence, table
#  columns short of them, units per block)
CASES = [
    # 16-byte rows, 256-byte blocks: one unit per block, 4096 units, and an
    # odd count (the last workgroup has no second unit)
    (DType.F16, DType.F16, 1, 8, 16, 4096, 0, 1),
    (DType.F16, DType.F16, 1, 8, 16, 4097, 0, 1),
    # 16384 and 32768 units
    (DType.F16, DType.F16, 1, 8, 16, 16384, 0, 1),
    (DType.F16, DType.F16, 1, 8, 16, 32768, 0, 1),
    # c2's rows: 32 KiB blocks in 16 units, 515 blocks (8240 units, the
    # second unit of a workgroup starting half way through a block)
    (DType.BF16, DType.BF16, 8, 128, 16, 515, 0, 16),
    # the table three blocks narrower than max_seq_len
    (DType.BF16, DType.BF16, 8, 128, 16, 515, 3, 16),
    # FP8 E4M3 -> bf16: 16 KiB blocks of 8-byte chunks in 8 units
    (DType.F8_E4M3, DType.BF16, 8, 128, 16, 512, 0, 8),
    # FP8 E5M2 -> f16, 32-token blocks of 64-element rows: 4 units each
    (DType.F8_E5M2, DType.F16, 4, 64, 32, 1100, 0, 4),
]


def _ids(c):
    return (f"{c[0].name}-{c[1].name}-H{c[2]}-D{c[3]}-bs{c[4]}-{c[5]}blocks"
            f"{'-short' + str(c[6]) if c[6] else ''}")


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
@pytest.mark.parametrize("idx64", [False, True])
def test_two_units_per_workgroup(case, idx64):
    cdt, iodt, H, D, bs, blocks, short, parts = case
    assert 4096 <= (blocks - short) * parts <= 65536  # the two-unit range
    gen = torch.Generator().manual_seed(1200 + CASES.index(case) * 2 + int(idx64))
    L = blocks * bs
    mbps = blocks - short
    nb = max(64, mbps // 2)
    pc, kb, vb = make_cache(Layout.BLOCK_NHD, Layout.BLOCK_NHD, cdt, nb, bs, H, D, gen=gen)
    half = L // 2
    # (table columns) * parts units per sequence in J = half as many
    # workgroups: unit J begins at token L / 2 when the table covers L
    lens = torch.tensor([L, half + 3 * bs + 5, half, half - 7, 0, L + 100, half + bs // 2])
    S = lens.numel()
    table = torch.randint(0, nb, (S, mbps), generator=gen)
    # invalid ids in first units and in second units
    table[0, 3], table[0, mbps // 2 + 1] = -1, nb + 5
    table[1, mbps // 2 + 2] = -7
    table[5, 1] = nb
    itype = torch.int64 if idx64 else torch.int32
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[iodt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks = vs = None
    if cdt != iodt:
        if CASES.index(case) % 2 == 0:
            ks, vs = 0.0213, 0.0047
        else:
            ks, vs = (ScaleArg(SG.PER_BLOCK_HEAD,
                               torch.empty(nb, H).uniform_(0.002, 0.05, generator=gen).numpy())
                      for _ in range(2))
    check_gather(pc, kb, vb, ko, vo, table.to(itype).to(DEV), lens.to(itype).to(DEV), L,
                 cache_dtype=cdt, io_dtype=iodt, k_scale=ks, v_scale=vs)


# RAGGED and KV_OFFSETS gathers over sequences of many row tiles.
# (path, cache dtype, io dtype, H, D, rows per tile, tiles per sequence)
INDEXED = [
    ("ragged_tile", DType.BF16, DType.BF16, 8, 128, 1, 8197),     # one 2 KiB row per tile
    ("ragged_tile", DType.F16, DType.F16, 1, 8, 16, 4099),        # 16 rows, mixed block ids
    ("ragged_tile", DType.F16, DType.F16, 1, 8, 16, 40001),       # 16 rows, 40001 tiles
    ("ragged_tile", DType.BF16, DType.BF16, 1, 128, 8, 513),      # 513 tiles
    ("offsets", DType.BF16, DType.BF16, 4, 128, 4, 2049),         # 2049 tiles
    ("ragged_tile", DType.F8_E4M3, DType.BF16, 8, 128, 2, 4100),  # dequantizing
    ("ragged_flat", DType.BF16, DType.BF16, 8, 128, 1, 4100),     # padded heads axis
    ("offsets", DType.BF16, DType.BF16, 8, 128, 2, 4100),         # entries per chunk
    ("offsets", DType.BF16, DType.BF16, 1, 128, 16, 4100),        # entries per tile (copy)
    ("offsets", DType.F8_E4M3, DType.BF16, 8, 128, 4, 4100),      # entries per tile (dequant)
]


def _lens(L, r):
    half = (L // r + 1) // 2 * r  # the first row of the middle tile
    return [L, half + 3 * r + 1, half, half - 1, 0, L + 100, half + r // 2 + 1]


def _indexed_ids(c):
    return f"{c[0]}-{c[1].name}-H{c[3]}-D{c[4]}-r{c[5]}-{c[6]}tiles"


@pytest.mark.parametrize("case", INDEXED, ids=[_indexed_ids(c) for c in INDEXED])
def test_indexed_gather_many_tiles(case):
    import numpy as np

    from kvx_amd import paged

    from gpu_helpers import (OffsetsPool, check_gather_offsets, check_gather_ragged)

    path, cdt, iodt, H, D, r, tiles = case
    idx = INDEXED.index(case)
    rng = np.random.default_rng(1300 + idx)
    gen = torch.Generator().manual_seed(1300 + idx)
    bs, nb = 16, 48
    L = tiles * r - (r // 2)  # a partial last tile
    assert 512 <= (L + r - 1) // r <= 65536
    S = 7
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[iodt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    ks, vs = (0.0213, 0.0047) if cdt != iodt else (None, None)
    if path == "offsets":
        pool = OffsetsPool(Layout.BLOCK_NHD, Layout.BLOCK_NHD, cdt, nb, bs, H, D,
                           pitch_pad=64, gen=gen)
        mbps = (L + bs - 1) // bs
        raw = rng.integers(0, nb, size=(S, 1, 2, mbps)).astype(np.uint32)
        raw |= (rng.random(raw.shape) < 0.3).astype(np.uint32) << 31  # secondary pool
        raw[0, 0, 0, 5] = nb + 3          # invalid K entries in both halves
        raw[0, 0, 1, mbps // 2 + 1] = 0x7FFFFFFF
        raw[2, 0, :, mbps // 2] = nb      # both entries of a block invalid
        offsets = torch.from_numpy(raw.view(np.int32)).to(DEV)
        lens = torch.tensor(_lens(L, r), dtype=torch.int32, device=DEV)
        check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=cdt, io_dtype=iodt,
                             k_scale=ks, v_scale=vs)
        return
    pc, kb, vb = make_cache(Layout.BLOCK_NHD, Layout.BLOCK_NHD, cdt, nb, bs, H, D, gen=gen,
                            k_pad=2 if path == "ragged_flat" else None,
                            v_pad=2 if path == "ragged_flat" else None)
    counts = np.array(_lens(L, r))
    counts[5] = L + 3
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    # each sequence's tokens follow a block table, with corrupted entries
    parts = []
    for s in range(S):
        t = np.arange(counts[s])
        ids = rng.integers(0, nb, size=(counts[s] + bs - 1) // bs + 1)[t // bs]
        parts.append(ids)
    indices = np.concatenate(parts).astype(np.int32)
    bad = rng.choice(indices.size, size=64, replace=False)
    indices[bad] = rng.choice([-1, nb, nb + 9, 3], size=64)
    rt = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.full((S,), L, dtype=torch.int32, device=DEV)
    lens[3] = L // 3
    check_gather_ragged(pc, kb, vb, ko, vo, rt, lens, L, cache_dtype=cdt, io_dtype=iodt,
                        k_scale=ks, v_scale=vs)


# The transposing gather (gather_tiles_kernel) over sequences of 520 to 1560
# (block, tile) units.
# (K order, K x, V order, V x, table, cache dtype, H, D, blocks per sequence)
TILED = [
    ("bhod", None, "bhod", None, "packed", DType.BF16, 8, 128, 130),    # HND, 4 tiles a block
    ("bhpox", 8, "bhdo", None, "packed", DType.BF16, 8, 128, 130),      # vLLM's pair
    ("bhod", None, "bohd", None, "packed", DType.F16, 4, 64, 520),       # HND K, row-major V
    ("bhod", None, "bhod", None, "ragged", DType.BF16, 8, 128, 130),    # RAGGED, mixed ids
    ("bhod", None, "bhod", None, "offsets", DType.BF16, 8, 128, 130),   # KV_OFFSETS
    ("bhod", None, "bhod", None, "packed", DType.F8_E4M3, 8, 128, 260),  # dequantizing
    ("bhod", None, "bhod", None, "packed", DType.BF16, 3, 128, 520),    # 768-byte rows
]


def _tiled_ids(c):
    return f"{c[0]}{c[1] or ''}-{c[2]}{c[3] or ''}-{c[4]}-{c[5].name}-H{c[6]}-D{c[7]}-{c[8]}blocks"


@pytest.mark.parametrize("case", TILED, ids=[_tiled_ids(c) for c in TILED])
def test_transposing_gather_many_units(case):
    import numpy as np

    from kvx_amd import paged

    from gpu_helpers import (OffsetsPool, check_gather_offsets, check_gather_ragged,
                             custom_cache)

    ko_, kx, vo_, vx, fmt, cdt, H, D, blocks = case
    idx = TILED.index(case)
    rng = np.random.default_rng(1400 + idx)
    gen = torch.Generator().manual_seed(1400 + idx)
    bs, nb, S = 16, 40, 7
    L = blocks * bs - 5  # a partial last block
    iodt = DType.BF16 if cdt == DType.F8_E4M3 else cdt
    ks, vs = (0.0213, 0.0047) if cdt != iodt else (None, None)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[iodt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    half = (blocks // 2) * bs  # the middle block
    lens = [L, half + 2 * bs + 3, half, half - 9, 0, L + 100, half + bs + 1]
    if fmt == "offsets":
        pool = OffsetsPool(Layout.BLOCK_HND, Layout.BLOCK_HND, cdt, nb, bs, H, D,
                           pitch_pad=64, gen=gen)
        raw = rng.integers(0, nb, size=(S, 1, 2, blocks)).astype(np.uint32)
        raw |= (rng.random(raw.shape) < 0.3).astype(np.uint32) << 31
        raw[0, 0, 0, 4] = nb + 3
        raw[0, 0, 1, blocks // 2 + 1] = 0x7FFFFFFF
        offsets = torch.from_numpy(raw.view(np.int32)).to(DEV)
        check_gather_offsets(pool, ko, vo, offsets,
                             torch.tensor(lens, dtype=torch.int32, device=DEV), L,
                             cache_dtype=cdt, io_dtype=iodt, k_scale=ks, v_scale=vs)
        return
    pc, kb, vb = custom_cache(cdt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    if fmt == "ragged":
        counts = np.array(lens)
        counts[5] = L + 3
        indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        parts = [rng.integers(0, nb, size=blocks + 1)[np.arange(c) // bs] for c in counts]
        indices = np.concatenate(parts).astype(np.int32)
        bad = rng.choice(indices.size, size=48, replace=False)
        indices[bad] = rng.choice([-1, nb, 5], size=48)
        rt = paged.RaggedTable(torch.from_numpy(indices).to(DEV),
                               torch.from_numpy(indptr).to(DEV))
        check_gather_ragged(pc, kb, vb, ko, vo, rt, torch.full((S,), L, dtype=torch.int32,
                                                               device=DEV), L,
                            cache_dtype=cdt, io_dtype=iodt, k_scale=ks, v_scale=vs)
        return
    table = torch.randint(0, nb, (S, blocks), generator=gen).to(torch.int32)
    table[0, 2], table[0, blocks // 2 + 1], table[1, blocks // 2 + 2] = -1, nb + 4, nb
    check_gather(pc, kb, vb, ko, vo, table.to(DEV),
                 torch.tensor(lens, dtype=torch.int32, device=DEV), L, cache_dtype=cdt,
                 io_dtype=iodt, k_scale=ks, v_scale=vs)
