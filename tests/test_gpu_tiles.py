"""GPU parity of the LDS tile kernels: the transposing gather
(gather_tiles_kernel) and the tiled block write (write_tiles_kernel), for
dense blocks that are not row-major — token axis innermost (vLLM's value
cache [num_blocks, H, D, block_size]), x-packed HND_PACKED, HND — through
the C ABI, bit-identical to the CPU oracle (kernels/kvx_paged_kv.cu:93-124
write and :226-267 gather semantics).

Gather cases cover every LDS piece size (1, 2, 4, 8, 16 bytes), runs
shorter than one 16-byte load (block_size * run < 16), blocks split into
several tiles, runs and tile widths that are not a power of two (HND heads
of 96 or 80 elements, rows of 3 or 6 heads), a row-major partner tensor, partial last blocks, block ids
< 0 and >= num_blocks, seq_len beyond max_seq_len, int64 indices, and the
FP8 dequantizing gather with per-tensor, per-head and per-block-head
scales.  RAGGED cases cover tiles whose rows all name one block, tiles whose
rows name different blocks or invalid ones, short indptr ranges and int64
indptr.  Write cases cover the same layouts with groups that fill a block
in order, groups that do not (partial, out of order, invalid slots, a
ragged tail), and the quantizing FP8 write, also with tile widths that are
not a power of two.
"""
import numpy as np
import pytest
import torch

from kvx_amd.abi import DType, Layout, ScaleGranularity as SG

from kvx_amd import paged

from gpu_helpers import (TORCH_DT, ScaleArg, check_gather, check_gather_ragged, check_write,
                         custom_cache, make_cache, random_fill)

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (cache dtype, K order, K x, V order, V x, block_size, H, D)
CASES = [
    (DType.BF16, "bhdo", None, "bhpox", 8, 16, 8, 128),   # runs 2 / 16 bytes, 4 tiles
    (DType.BF16, "bhpox", 4, "bhpox", 2, 32, 4, 64),      # runs 8 / 4 bytes
    (DType.F32, "bhdo", None, "bohd", None, 8, 2, 64),    # run 4 bytes / row-major V
    (DType.F8_E4M3, "bhdo", None, "bhpox", 8, 8, 8, 128),  # run 1 byte, bs * run < 16
    (DType.BF16, "bhod", None, "bhdo", None, 64, 8, 16),  # HND with 32-byte runs
    (DType.F16, "bhdo", None, "bhdo", None, 2, 4, 32),    # block_size 2
    (DType.BF16, "bohd", None, "bhdo", None, 4, 1, 64),   # one head
    (DType.BF16, "bhpox", 8, "bohd", None, 16, 8, 128),   # c3's pair: 16-byte runs / row-major V
    # rows whose bytes are not a power of two: several power-of-two tiles per row
    (DType.BF16, "bhod", None, "bhod", None, 16, 6, 128),  # HND, 6 heads: 3 tiles of 512 B
    (DType.BF16, "bhpox", 8, "bohd", None, 16, 12, 64),   # x-packed K / NHD V, 1536-byte rows
    (DType.F8_E4M3, "bhod", None, "bhdo", None, 16, 12, 128),  # FP8 HND / token-innermost
    (DType.F32, "bhdo", None, "bhod", None, 64, 5, 32),   # 640-byte rows: 5 tiles of 128 B
    (DType.F16, "bhpox", 8, "bohd", None, 16, 3, 64),     # 384-byte rows: one 6 KiB tile
    # runs or tile widths that are not a power of two (multiply-high division)
    (DType.BF16, "bhod", None, "bhod", None, 16, 8, 96),  # HND 192-byte runs, 768-byte tiles
    (DType.BF16, "bhod", None, "bohd", None, 32, 8, 80),  # 160-byte runs, 320-byte tiles
    (DType.BF16, "bhod", None, "bhod", None, 64, 8, 96),  # 8 tiles of one run per row
    (DType.F8_E4M3, "bhod", None, "bhpox", 16, 16, 8, 96),  # FP8 96-byte runs / x-packed
    (DType.BF16, "bhdo", None, "bhod", None, 16, 3, 128),  # 2- / 256-byte runs, 768-byte tile
]


def _ids(c):
    return f"{c[0].name}-{c[1]}{c[2] or ''}-{c[3]}{c[4] or ''}-bs{c[5]}-H{c[6]}-D{c[7]}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
@pytest.mark.parametrize("idx64", [False, True])
def test_tiles_gather(case, idx64):
    dt, ko_, kx, vo_, vx, bs, H, D = case
    gen = torch.Generator().manual_seed(CASES.index(case) * 2 + int(idx64))
    nb = 48
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    S = 7
    L = 5 * bs + bs // 2 + 1  # partial last block
    mbps = (L + bs - 1) // bs + 1
    table = torch.randint(-2, nb + 2, (S, mbps), generator=gen)
    lens = torch.randint(0, L + bs + 3, (S,), generator=gen)
    lens[0], lens[1] = L, L + 2 * bs  # a full row and one past max_seq_len
    itype = torch.int64 if idx64 else torch.int32
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(itype).to(DEV), lens.to(itype).to(DEV), L,
                 cache_dtype=dt, io_dtype=dt)


def _scale(kind, gen, nb, H):
    if kind == "tensor":
        return 0.0173
    if kind == SG.PER_HEAD:
        return ScaleArg(kind, torch.empty(H).uniform_(0.002, 0.05, generator=gen).numpy(),
                        stride=(2,))
    return ScaleArg(kind, torch.empty(nb, H).uniform_(0.002, 0.05, generator=gen).numpy(),
                    stride=(1, nb))


@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
@pytest.mark.parametrize("io", [DType.BF16, DType.F32])
@pytest.mark.parametrize("kind", ["tensor", SG.PER_HEAD, SG.PER_BLOCK_HEAD])
def test_tiles_dequant(fp8, io, kind):
    """K token-innermost, V x-packed x = 8 (8-byte FP8 runs)."""
    gen = torch.Generator().manual_seed(100 + int(fp8) * 10 + int(io) + 3 * (kind != "tensor"))
    H, D, bs, nb = 8, 128, 16, 40
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhdo", "bhpox", None, 8, gen)
    S, L = 5, 77
    table = torch.randint(-1, nb + 1, (S, (L + bs - 1) // bs), generator=gen).to(torch.int32)
    lens = torch.tensor([77, 50, 16, 1, 0], dtype=torch.int32)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(DEV), lens.to(DEV), L, cache_dtype=fp8,
                 io_dtype=io, k_scale=_scale(kind, gen, nb, H), v_scale=_scale(kind, gen, nb, H))


@pytest.mark.parametrize("entry", ["launch", "abi"])
def test_tiles_hnd_packed_layouts(entry):
    """The x-packed K layout through its own layout code (HND_PACKED, x = 8),
    with an NHD or HND_PACKED partner (the ABI entry needs K and V to share
    the layout code)."""
    gen = torch.Generator().manual_seed(120 + (entry == "abi"))
    H, D, bs, nb = 8, 128, 16, 64
    vl = Layout.BLOCK_HND_PACKED if entry == "abi" else Layout.BLOCK_NHD
    pc, kb, vb = make_cache(Layout.BLOCK_HND_PACKED, vl, DType.BF16, nb, bs, H, D, 8, gen=gen)
    S, L = 6, 200
    table = torch.randperm(nb, generator=gen)[: S * 10].reshape(S, 10).to(torch.int32)
    table[2, 3] = -1
    lens = torch.tensor([200, 199, 161, 17, 3, 0], dtype=torch.int32)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table.to(DEV), lens.to(DEV), L, cache_dtype=DType.BF16,
                 io_dtype=DType.BF16, entry=entry)


def _prefill_slots(gen, nb, bs, groups, tail, spoil):
    """Slots of `groups` full blocks in order (random distinct blocks), then
    `tail` tokens; `spoil` groups get one slot changed (-1, a swap, or a
    block past the end) so that they take the per-token path."""
    blocks = torch.randperm(nb, generator=gen)[: groups + 1]
    slots = (blocks[:groups, None] * bs + torch.arange(bs)).reshape(-1)
    slots = torch.cat([slots, blocks[groups] * bs + torch.arange(tail)])
    for i, g in enumerate(torch.randperm(groups, generator=gen)[:spoil].tolist()):
        o = int(torch.randint(0, bs, (1,), generator=gen))
        if i % 3 == 0:
            slots[g * bs + o] = -1
        elif i % 3 == 1 and bs > 1:
            a, b = g * bs + o, g * bs + (o + 1) % bs
            slots[a], slots[b] = slots[b].clone(), slots[a].clone()
        else:
            slots[g * bs + o] = nb * bs + o
    return slots


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
@pytest.mark.parametrize("slot64", [False, True])
def test_tiles_write(case, slot64):
    dt, ko_, kx, vo_, vx, bs, H, D = case
    gen = torch.Generator().manual_seed(200 + CASES.index(case) * 2 + int(slot64))
    nb = 48
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    groups = 12
    slots = _prefill_slots(gen, nb, bs, groups, tail=max(1, bs // 2 - 1), spoil=3)
    T = slots.numel()
    key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    slots = slots.to(torch.int64 if slot64 else torch.int32).to(DEV)
    check_write(pc, kb, vb, key, val, slots, io_dtype=dt, cache_dtype=dt)


@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
def test_tiles_quantizing_write(fp8, io):
    """K token-innermost, V x-packed x = 16: the tile op quantizes 8
    elements per chunk; per-tensor scales (indexed scales use the per-token
    kernel)."""
    gen = torch.Generator().manual_seed(300 + int(fp8) * 10 + int(io))
    H, D, bs, nb = 8, 128, 16, 40
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhdo", "bhpox", None, 16, gen)
    slots = _prefill_slots(gen, nb, bs, groups=10, tail=5, spoil=2)
    T = slots.numel()
    key = (torch.randn((T, H, D), generator=gen) * 4).to(TORCH_DT[io]).to(DEV)
    val = (torch.randn((T, H, D), generator=gen) * 0.5).to(TORCH_DT[io]).to(DEV)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=io, cache_dtype=fp8,
                k_scale=0.011, v_scale=0.0021)


@pytest.mark.parametrize("entry", ["launch", "prefill", "abi"])
def test_tiles_write_x_packed_entries(entry):
    """c3's pairing (K HND_PACKED x = 8, V NHD) through kvx_launch_write_kv,
    the prefill entry and (same layout code for K and V) kvx_write_kv."""
    gen = torch.Generator().manual_seed(320 + ["launch", "prefill", "abi"].index(entry))
    H, D, bs, nb = 8, 128, 16, 64
    vl = Layout.BLOCK_HND_PACKED if entry == "abi" else Layout.BLOCK_NHD
    pc, kb, vb = make_cache(Layout.BLOCK_HND_PACKED, vl, DType.BF16, nb, bs, H, D, 8, gen=gen)
    slots = _prefill_slots(gen, nb, bs, groups=16, tail=0, spoil=1)
    T = slots.numel()
    key = random_fill(torch.empty((T, H, D), dtype=torch.bfloat16, device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    kw = dict(tokens_per_seq=64) if entry == "prefill" else {}
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=DType.BF16,
                cache_dtype=DType.BF16, entry="abi" if entry == "abi" else "launch", **kw)


def _whole_block_edge_slots(gen, nb, bs, slot64):
    """Groups aimed at the whole-block test of the tiled write: in order in
    the block past the end (skipped), in the last and the first block, in
    reverse order, one slot repeated, and for int64 slots an in-order group
    at 2**32 (its block id needs the slot's high word); ordinary whole
    blocks in between."""
    pool = torch.randperm(nb - 2, generator=gen)[:4] + 1  # blocks other than 0, nb - 1
    ar = torch.arange(bs)
    groups = [
        pool[0] * bs + ar,
        nb * bs + ar,                 # in order, block == num_blocks
        pool[1] * bs + ar,
        (nb - 1) * bs + ar,           # last block
        0 * bs + ar,                  # first block
        pool[2] * bs + ar.flip(0),    # reversed
        pool[3] * bs + torch.where(ar == bs - 1, ar - 1, ar),  # one offset twice
    ]
    if slot64:
        groups.append((1 << 32) + ar)  # in order, aligned, block id >= 2**28
    return torch.cat(groups)


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3]],
                         ids=[_ids(c) for c in (CASES[0], CASES[2], CASES[3])])
@pytest.mark.parametrize("slot64", [False, True])
def test_tiles_write_whole_block_edges(case, slot64):
    """The whole-block path of write_tiles_kernel takes a group only when its
    slots are block * bs + 0 .. bs - 1 in token order with block < num_blocks;
    every other group falls back to the run analysis or the per-token path."""
    dt, ko_, kx, vo_, vx, bs, H, D = case
    gen = torch.Generator().manual_seed(330 + CASES.index(case) * 2 + int(slot64))
    nb = 24
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    slots = _whole_block_edge_slots(gen, nb, bs, slot64)
    T = slots.numel()
    io = DType.BF16 if dt == DType.F8_E4M3 else dt
    key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    if dt == DType.F8_E4M3:  # finite io values for the quantizing write
        key = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
        val = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
    scales = dict(k_scale=0.013, v_scale=0.007) if dt == DType.F8_E4M3 else {}
    slots = slots.to(torch.int64 if slot64 else torch.int32).to(DEV)
    check_write(pc, kb, vb, key, val, slots, io_dtype=io, cache_dtype=dt, **scales)


def _unaligned_chunk_slots(gen, nb, bs, seqs, spoil):
    """Prefill chunks of `seqs` sequences, each starting at a random offset
    inside a block and running a random length over distinct random blocks,
    so that groups of bs tokens straddle blocks and sequences; `spoil`
    random tokens get slot -1."""
    perm = torch.randperm(nb, generator=gen)
    out, used = [], 0
    for _ in range(seqs):
        off = int(torch.randint(0, bs, (1,), generator=gen))
        n = int(torch.randint(1, 4 * bs + 3, (1,), generator=gen))
        nblk = (off + n + bs - 1) // bs
        blocks = perm[used:used + nblk]
        used += nblk
        p = torch.arange(off, off + n)
        out.append(blocks[p // bs] * bs + p % bs)
    slots = torch.cat(out)
    idx = torch.randperm(slots.numel(), generator=gen)[:spoil]
    slots[idx] = -1
    return slots


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
@pytest.mark.parametrize("spoil", [0, 3])
def test_tiles_write_unaligned_chunks(case, spoil):
    """Chunks that start inside blocks: each block's run is owned by the
    workgroups of the group where the run starts, and runs cross group and
    sequence boundaries."""
    dt, ko_, kx, vo_, vx, bs, H, D = case
    gen = torch.Generator().manual_seed(340 + CASES.index(case) * 2 + int(spoil > 0))
    nb = 96
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    slots = _unaligned_chunk_slots(gen, nb, bs, seqs=5, spoil=spoil)
    T = slots.numel()
    io = DType.BF16 if dt == DType.F8_E4M3 else dt
    if dt == DType.F8_E4M3:
        key = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
        val = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
    else:
        key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[io], device=DEV), gen)
        val = random_fill(torch.empty_like(key), gen)
    scales = dict(k_scale=0.013, v_scale=0.007) if dt == DType.F8_E4M3 else {}
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=io, cache_dtype=dt, **scales)


def _ragged_from_blocks(rng, S, L, bs, nb, spoil_frac, idx_dtype, ptr_dtype):
    """Per-token block ids of S sequences laid out block by block (so most
    tiles' rows name one block), a fraction of tokens given another id
    (another block, -1 or >= num_blocks); per-sequence counts around L."""
    counts = rng.integers(max(1, L - 2 * bs), L + bs, size=S)
    ids = []
    for c in counts:
        blocks = rng.integers(-1, nb + 1, size=(int(c) + bs - 1) // bs)
        tok = np.repeat(blocks, bs)[: int(c)]
        spoil = rng.random(int(c)) < spoil_frac
        tok[spoil] = rng.integers(-1, nb + 2, size=int(spoil.sum()))
        ids.append(tok)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(ptr_dtype)
    return np.concatenate(ids).astype(idx_dtype), indptr


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
@pytest.mark.parametrize("spoil", [0.0, 0.05, 1.0])
def test_tiles_ragged_gather(case, spoil):
    dt, ko_, kx, vo_, vx, bs, H, D = case
    seed = 400 + CASES.index(case) * 3 + int(spoil * 20)
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    nb = 40
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    S, L = 6, 4 * bs + 3
    wide = CASES.index(case) % 2 == 1
    indices, indptr = _ragged_from_blocks(rng, S, L, bs, nb, spoil,
                                          np.int64 if wide else np.int32,
                                          np.int64 if not wide else np.int32)
    table = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.from_numpy(rng.integers(0, L + 3, size=S).astype(indices.dtype)).to(DEV)
    lens[0] = L + 3
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
@pytest.mark.parametrize("kind", ["tensor", SG.PER_BLOCK_HEAD])
def test_tiles_ragged_dequant(fp8, kind):
    """Per-block-head scales follow each row's own block in mixed tiles."""
    seed = 450 + int(fp8) * 2 + (kind != "tensor")
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    H, D, bs, nb = 8, 128, 16, 40
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhdo", "bhpox", None, 8, gen)
    S, L = 5, 70
    indices, indptr = _ragged_from_blocks(rng, S, L, bs, nb, 0.1, np.int32, np.int64)
    table = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.tensor([70, 64, 33, 1, 0], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=fp8,
                        io_dtype=DType.BF16, k_scale=_scale(kind, gen, nb, H),
                        v_scale=_scale(kind, gen, nb, H))


def _chunk_slots(gen, nb, bs, S, chunk):
    """Slots of S prefill chunks of `chunk` consecutive positions, each
    starting at a random offset inside its first block, every sequence on
    its own random blocks."""
    nblk = (chunk + bs - 1) // bs + 1
    blocks = torch.randperm(nb, generator=gen)[: S * nblk].reshape(S, nblk)
    out = []
    for s in range(S):
        start = int(torch.randint(0, bs, (1,), generator=gen))
        pos = torch.arange(start, start + chunk)
        out.append(blocks[s, pos // bs] * bs + pos % bs)
    return torch.cat(out)


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_tiles_write_chunks_inside_blocks(case):
    dt, ko_, kx, vo_, vx, bs, H, D = case
    gen = torch.Generator().manual_seed(500 + CASES.index(case))
    nb = 64
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    slots = _chunk_slots(gen, nb, bs, S=5, chunk=2 * bs + bs // 2 + 1)
    T = slots.numel()
    key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=dt, cache_dtype=dt)


@pytest.mark.parametrize("case", [c for c in CASES if c[5] >= 4],
                         ids=[_ids(c) for c in CASES if c[5] >= 4])
def test_tiles_write_two_runs(case):
    """Full groups of two runs in different blocks (the tail of one block
    from offset 3, the head of another from offset 2), then a last, short
    group of two runs inside one block around a gap (offsets [1, bs/2) and
    [bs/2 + 1, bs): rows 0 and bs/2 keep their contents)."""
    dt, ko_, kx, vo_, vx, bs, H, D = case
    gen = torch.Generator().manual_seed(550 + CASES.index(case))
    nb = 32
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    blocks = [int(b) for b in torch.randperm(nb, generator=gen)[:7]]
    sl = []
    for g in range(3):
        b0, b1 = blocks[2 * g], blocks[2 * g + 1]
        first = bs - 3
        sl += [b0 * bs + o for o in range(3, bs)] + [b1 * bs + 2 + i for i in range(bs - first)]
    h = bs // 2
    sl += [blocks[6] * bs + o for o in list(range(1, h)) + list(range(h + 1, bs))]
    slots = torch.tensor(sl)
    T = slots.numel()
    key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=dt, cache_dtype=dt)


@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
def test_tiles_quantizing_write_chunks(fp8):
    gen = torch.Generator().manual_seed(580 + int(fp8))
    H, D, bs, nb = 8, 128, 32, 40
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, "bhdo", "bhpox", None, 16, gen)
    slots = _chunk_slots(gen, nb, bs, S=4, chunk=bs)
    T = slots.numel()
    key = (torch.randn((T, H, D), generator=gen) * 3).to(torch.bfloat16).to(DEV)
    val = (torch.randn((T, H, D), generator=gen) * 0.3).to(torch.bfloat16).to(DEV)
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=DType.BF16, cache_dtype=fp8,
                k_scale=0.009, v_scale=0.0013)


@pytest.mark.parametrize("kind", [SG.PER_HEAD, SG.PER_BLOCK, SG.PER_BLOCK_HEAD])
@pytest.mark.parametrize("layouts", [("bhdo", None, "bhpox", 16), ("bhpox", 16, "bohd", None)])
def test_tiles_quantizing_write_indexed_scales(kind, layouts):
    """Indexed scales through the tiled write: whole blocks, chunks that
    start inside blocks (the scale follows each run's block) and spoiled
    groups (per-token path)."""
    ko_, kx, vo_, vx = layouts
    gen = torch.Generator().manual_seed(600 + int(kind) * 3 + (kx is None))
    H, D, bs, nb = 8, 128, 16, 64
    pc, kb, vb = custom_cache(DType.F8_E4M3, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    # whole blocks in [0, nb / 2), two groups spoiled (a -1 slot, a swap);
    # chunks starting inside blocks of [nb / 2, nb): no slot is written twice
    blocks = torch.randperm(nb // 2, generator=gen)[:6]
    full = (blocks[:, None] * bs + torch.arange(bs)).reshape(-1)
    full[3] = -1
    full[2 * bs + 5], full[2 * bs + 6] = full[2 * bs + 6].clone(), full[2 * bs + 5].clone()
    chunks = _chunk_slots(gen, nb // 2, bs, S=3, chunk=2 * bs + 5) + (nb // 2) * bs
    slots = torch.cat([full, chunks])
    T = slots.numel()
    key = (torch.randn((T, H, D), generator=gen) * 4).to(torch.bfloat16).to(DEV)
    val = (torch.randn((T, H, D), generator=gen) * 0.5).to(torch.bfloat16).to(DEV)

    def arg():
        if kind == SG.PER_HEAD:
            return ScaleArg(kind, torch.empty(H).uniform_(0.002, 0.05, generator=gen).numpy(),
                            stride=(3,))
        if kind == SG.PER_BLOCK:
            return ScaleArg(kind, torch.empty(nb).uniform_(0.002, 0.05, generator=gen).numpy())
        return ScaleArg(kind, torch.empty(nb, H).uniform_(0.002, 0.05, generator=gen).numpy(),
                        stride=(1, nb))

    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=DType.BF16,
                cache_dtype=DType.F8_E4M3, k_scale=arg(), v_scale=arg())


# (K order, K x, V order, V x): at least one tensor row-major ("bohd", NHD)
@pytest.mark.parametrize("kind", ["tensor", SG.PER_BLOCK_HEAD])
@pytest.mark.parametrize("fp8", [DType.F8_E4M3, DType.F8_E5M2])
@pytest.mark.parametrize("shape", [("bhod", None, "bhod", None, 8, 96),
                                   ("bhpox", 16, "bhdo", None, 3, 128),
                                   ("bhod", None, "bohd", None, 8, 80)],
                         ids=["hnd-8x96", "xpacked-tokinner-3x128", "hnd-nhd-8x80"])
def test_tiles_quantizing_write_odd_tiles(shape, fp8, kind):
    """The quantizing tiled write with tile widths that are not a power of
    two (96- and 80-byte FP8 runs, 384-byte rows): whole blocks, spoiled
    groups and chunks that start inside blocks."""
    ko_, kx, vo_, vx, H, D = shape
    gen = torch.Generator().manual_seed(700 + 4 * H + int(fp8) + 2 * (kind != "tensor"))
    bs, nb = 16, 64
    pc, kb, vb = custom_cache(fp8, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    blocks = torch.randperm(nb // 2, generator=gen)[:6]
    full = (blocks[:, None] * bs + torch.arange(bs)).reshape(-1)
    full[7] = -1
    chunks = _chunk_slots(gen, nb // 2, bs, S=3, chunk=2 * bs + 7) + (nb // 2) * bs
    slots = torch.cat([full, chunks])
    T = slots.numel()
    key = (torch.randn((T, H, D), generator=gen) * 4).to(torch.bfloat16).to(DEV)
    val = (torch.randn((T, H, D), generator=gen) * 0.5).to(torch.bfloat16).to(DEV)
    if kind == "tensor":
        ks, vs = 0.012, 0.0019
    else:
        ks, vs = (ScaleArg(kind, torch.empty(nb, H).uniform_(0.002, 0.05, generator=gen).numpy(),
                           stride=(1, nb)) for _ in range(2))
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=DType.BF16, cache_dtype=fp8,
                k_scale=ks, v_scale=vs)


_ROW_MAJOR_PAIRS = [("bohd", None, "bhpox", 8), ("bhpox", 8, "bohd", None),
                    ("bohd", None, "bhdo", None), ("bhdo", None, "bohd", None),
                    ("bohd", None, "bohd", None)]


@pytest.mark.parametrize("seed", range(15))
def test_tiles_write_row_major_ownership(seed):
    """Seeded prefill chunks (random starts inside blocks, random lengths,
    spoiled slots, both write entries) into caches where a row-major tensor
    is written group by group, its own tokens only, beside a partner whose
    runs belong to the group they start in: the whole cache must equal the
    oracle's, every untouched byte included."""
    rng = np.random.default_rng(900 + seed)
    gen = torch.Generator().manual_seed(900 + seed)
    ko_, kx, vo_, vx = _ROW_MAJOR_PAIRS[seed % len(_ROW_MAJOR_PAIRS)]
    bs = int(rng.choice([4, 8, 16, 32, 64]))
    H, D = [(8, 128), (4, 64), (2, 32)][seed % 3]
    dt = [DType.BF16, DType.F16, DType.F8_E4M3][(seed // 3) % 3]
    nb = 128
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    slots = _unaligned_chunk_slots(gen, nb, bs, seqs=5, spoil=int(rng.integers(0, 4)))
    T = slots.numel()
    io = DType.BF16 if dt == DType.F8_E4M3 else dt
    key = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
    val = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
    scales = dict(k_scale=0.013, v_scale=0.007) if dt == DType.F8_E4M3 else {}
    entry = "abi" if ko_ == vo_ and seed % 2 == 0 else "launch"  # seeds 4 and 14
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=io, cache_dtype=dt,
                entry=entry, **scales)


@pytest.mark.parametrize("layouts", [("bhpox", 8, "bhdo", None),   # vLLM's pair
                                     ("bhdo", None, "bhpox", 8),   # the pair swapped
                                     ("bhpox", 8, "bhpox", 8),     # x-packed K and V
                                     ("bhod", None, "bhdo", None)],  # HND / token-innermost
                         ids=["vllm", "swapped", "xpacked", "hnd-tokinner"])
@pytest.mark.parametrize("dt", [DType.BF16, DType.F8_E4M3, DType.F32])
def test_tiles_decode_write_mixed_layouts(layouts, dt):
    """A decode batch (one new token per sequence, each in a block of its
    own, at any offset; some slots -1 or past the pool) into K / V pairs of
    different piece sizes (16-byte x-packed or HND pieces beside one-element
    token-innermost ones): write_tiles_kernel's groups fill no block, so
    every token goes through its per-token fallback."""
    ko_, kx, vo_, vx = layouts
    gen = torch.Generator().manual_seed(520 + int(dt) * 8 + ["bhpox", "bhdo", "bhod"].index(ko_))
    H, D, bs, nb, T = 8, 128, 16, 96, 70
    pc, kb, vb = custom_cache(dt, nb, bs, H, D, ko_, vo_, kx, vx, gen)
    blocks = torch.randperm(nb, generator=gen)[:T]
    offs = torch.randint(0, bs, (T,), generator=gen)
    slots = blocks * bs + offs
    slots[torch.randperm(T, generator=gen)[:4]] = -1
    slots[7] = nb * bs + 3  # block == num_blocks: skipped
    io = DType.BF16 if dt == DType.F8_E4M3 else dt
    if dt == DType.F8_E4M3:
        key = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
        val = (torch.randn((T, H, D), generator=gen) * 3).to(TORCH_DT[io]).to(DEV)
    else:
        key = random_fill(torch.empty((T, H, D), dtype=TORCH_DT[io], device=DEV), gen)
        val = random_fill(torch.empty_like(key), gen)
    scales = dict(k_scale=0.013, v_scale=0.007) if dt == DType.F8_E4M3 else {}
    check_write(pc, kb, vb, key, val, slots.to(DEV), io_dtype=io, cache_dtype=dt, **scales)
