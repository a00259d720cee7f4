"""GPU parity of the RAGGED and KV_OFFSETS block-table gathers
(KVX_SPEC.md:107-122): libkvx_amd.so through the C ABI, bit-identical to the
CPU oracle on the same seeded inputs, outputs pre-filled with random bytes so
that untouched rows are checked too.

RAGGED: random per-token block ids with -1 and out-of-range ids, indptr
ranges shorter and longer than seq_len / max_seq_len, S32 / S64 indices,
indptr and lengths.  KV_OFFSETS: K and V blocks drawn from one pool,
secondary-pool flags with and without a secondary pool, out-of-range
indices, padded block pitches (including pitches that force narrower
vector chunks), in-block layouts NHD / HND / HND_PACKED, mixed K / V.  Both:
FP8 dequantizing gathers, rows wide enough for the kernel's tail loop,
misaligned outputs, and the kvx_abi.h entry point.
"""
import numpy as np
import pytest
import torch

from kvx_amd import paged
from kvx_amd.abi import DType, Layout

from gpu_helpers import (TORCH_DT, OffsetsPool, ScaleArg, check_gather_offsets,
                         check_gather_ragged, check_write, make_cache, random_fill)

pytestmark = pytest.mark.gpu
DEV = "cuda"
NHD, HND, PK = Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED
LAYOUTS = [NHD, HND, PK]
DTYPES = [DType.F32, DType.F16, DType.BF16, DType.F8_E4M3]


def out_pair(S, L, H, D, dtype, gen, misalign=False):
    outs = []
    for _ in range(2):
        if misalign:
            flat = torch.empty(S * L * H * D + 1, dtype=TORCH_DT[dtype], device=DEV)
            t = flat[1:].view(S, L, H, D)
        else:
            t = torch.empty((S, L, H, D), dtype=TORCH_DT[dtype], device=DEV)
        outs.append(random_fill(t, gen))
    return outs


def ragged_table(rng, S, L, nb, idt, pdt, long_tail=True):
    counts = rng.integers(0, L + (4 if long_tail else 1), size=S)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(pdt)
    indices = rng.integers(-1, nb + 2, size=max(int(indptr[-1]), 1)).astype(idt)
    return paged.RaggedTable(torch.from_numpy(indices).to(DEV),
                             torch.from_numpy(indptr).to(DEV))


def lens_tensor(rng, S, L, dt):
    return torch.from_numpy(rng.integers(-1, L + 4, size=S).astype(dt)).to(DEV)


# ---------------------------------------------------------------------------
# RAGGED

@pytest.mark.parametrize("seed", range(24))
def test_ragged_random(seed):
    rng = np.random.default_rng(3000 + seed)
    gen = torch.Generator().manual_seed(seed)
    dt = DTYPES[seed % 4]
    kl, vl = LAYOUTS[seed % 3], LAYOUTS[(seed // 3) % 3]
    H = int(rng.choice([1, 2, 8]))
    D = int(rng.choice([8, 64, 128]))
    bs = int(rng.choice([1, 4, 16, 32]))
    nb = int(rng.integers(2, 40))
    pad = [None, 1, 2][seed % 3]
    pc, kb, vb = make_cache(kl, vl, dt, nb, bs, H, D, gen=gen, k_pad=pad,
                            v_pad=[None, 0, 3][seed % 3])
    S, L = int(rng.integers(1, 7)), int(rng.integers(1, 300))
    idt = [np.int32, np.int64][seed % 2]
    pdt = [np.int32, np.int64][(seed // 2) % 2]
    table = ragged_table(rng, S, L, nb, idt, pdt)
    lens = lens_tensor(rng, S, L, idt)
    ko, vo = out_pair(S, L, H, D, dt, gen, misalign=seed % 5 == 4)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_ragged_fp8_dequant(io, layout):
    rng = np.random.default_rng(41)
    gen = torch.Generator().manual_seed(41)
    H, D, bs, nb, S, L = 4, 128, 16, 24, 5, 90
    pc, kb, vb = make_cache(layout, layout, DType.F8_E4M3, nb, bs, H, D, gen=gen)
    table = ragged_table(rng, S, L, nb, np.int32, np.int64)
    lens = lens_tensor(rng, S, L, np.int32)
    ko, vo = out_pair(S, L, H, D, io, gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=DType.F8_E4M3,
                        io_dtype=io, k_scale=0.0172, v_scale=3.5)


@pytest.mark.parametrize("dt,H", [(DType.F32, 16), (DType.BF16, 32), (DType.F8_E4M3, 8)])
def test_ragged_wide_rows(dt, H):
    """Rows of more than 4 chunks per lane exercise the kernel's tail loop."""
    rng = np.random.default_rng(5)
    gen = torch.Generator().manual_seed(5)
    D, bs, nb, S, L = 128, 16, 20, 3, 70
    pc, kb, vb = make_cache(NHD, HND, dt, nb, bs, H, D, gen=gen)
    table = ragged_table(rng, S, L, nb, np.int64, np.int32)
    lens = lens_tensor(rng, S, L, np.int64)
    ko, vo = out_pair(S, L, H, D, dt, gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("dt", [DType.BF16, DType.F16, DType.F32])
def test_ragged_abi_entry(dt):
    """kvx_gather_kv (kvx_abi.h) executes RAGGED tables on device memory."""
    rng = np.random.default_rng(8)
    gen = torch.Generator().manual_seed(8)
    H, D, bs, nb, S, L = 8, 128, 16, 32, 4, 64
    for layout in LAYOUTS:
        pc, kb, vb = make_cache(layout, layout, dt, nb, bs, H, D, gen=gen)
        table = ragged_table(rng, S, L, nb, np.int32, np.int32)
        lens = lens_tensor(rng, S, L, np.int32)
        ko, vo = out_pair(S, L, H, D, dt, gen)
        check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt,
                            io_dtype=dt, entry="abi")


def test_ragged_decode_shape():
    """A decode batch in RAGGED form: 64 sequences of 100-900 tokens,
    Llama-3-8B KV shape, token ids listing each sequence's blocks in order."""
    rng = np.random.default_rng(9)
    gen = torch.Generator().manual_seed(9)
    H, D, bs, S = 8, 128, 16, 64
    lens_np = rng.integers(100, 900, size=S).astype(np.int32)
    L = int(lens_np.max())
    nblk = (lens_np + bs - 1) // bs
    nb = int(nblk.sum())
    perm = rng.permutation(nb)
    indices, base = [], 0
    for s in range(S):
        blocks = perm[base: base + nblk[s]]
        base += nblk[s]
        indices.append(np.repeat(blocks, bs)[: lens_np[s]])
    indptr = np.concatenate([[0], np.cumsum(lens_np)]).astype(np.int32)
    table = paged.RaggedTable(torch.from_numpy(np.concatenate(indices).astype(np.int32)).to(DEV),
                              torch.from_numpy(indptr).to(DEV))
    pc, kb, vb = make_cache(NHD, NHD, DType.BF16, nb, bs, H, D, gen=gen)
    ko, vo = out_pair(S, L, H, D, DType.BF16, gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, torch.from_numpy(lens_np).to(DEV), L,
                        cache_dtype=DType.BF16, io_dtype=DType.BF16)


def block_run_table(rng, S, L, nb, bs, idt, pdt, spoil=0):
    """RAGGED table of block-structured sequences (each lists the tokens of
    its blocks in order, as a paged-attention RAGGED table does): lengths up
    to L + 3, random distinct blocks, and `spoil` ids replaced by -1, an
    out-of-range id or another block, so that some row tiles name several
    blocks or skipped rows."""
    counts = rng.integers(0, L + 4, size=S)
    counts[0] = L  # one full-length sequence
    nblk = (counts + bs - 1) // bs
    perm = rng.permutation(nb)
    ids, at = [], 0
    for s in range(S):
        blocks = perm[(at + np.arange(nblk[s])) % nb]
        at += nblk[s]
        ids.append(np.repeat(blocks, bs)[: counts[s]])
    indices = np.concatenate(ids) if ids else np.zeros(0)
    if indices.size == 0:
        indices = np.zeros(1)
    for i in rng.choice(indices.size, size=min(spoil, indices.size), replace=False):
        indices[i] = [-1, nb + 3, (indices[i] + 1) % nb][int(rng.integers(0, 3))]
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(pdt)
    return paged.RaggedTable(torch.from_numpy(indices.astype(idt)).to(DEV),
                             torch.from_numpy(indptr).to(DEV))


@pytest.mark.parametrize("case", range(16))
def test_ragged_block_runs(case):
    """RAGGED tables that list whole blocks in order, on canonical NHD caches
    (the row-tile kernel's one-block path), with a few spoiled ids (its
    per-row path): copies and FP8 dequantizing gathers with per-tensor,
    per-head, per-block and per-block-head scales, block sizes 1, 6, 16 and
    32, int32 / int64 indices and indptr."""
    rng = np.random.default_rng(7000 + case)
    gen = torch.Generator().manual_seed(case)
    from kvx_amd.abi import ScaleGranularity as SG

    bs = [16, 32, 1, 6][case % 4]
    dt = [DType.BF16, DType.F8_E4M3, DType.F8_E5M2, DType.F16][(case // 4) % 4]
    io = {DType.F8_E4M3: [DType.BF16, DType.F16, DType.F32][case % 3],
          DType.F8_E5M2: [DType.BF16, DType.F32, DType.F16][case % 3]}.get(dt, dt)
    H, D = [(8, 128), (2, 64), (4, 32), (1, 128)][case % 4]
    nb = int(rng.integers(20, 60))
    S, L = int(rng.integers(2, 7)), int(rng.integers(bs, 200))
    idt = [np.int32, np.int64][case % 2]
    pdt = [np.int64, np.int32][(case // 2) % 2]
    pc, kb, vb = make_cache(NHD, NHD, dt, nb, bs, H, D, gen=gen)
    table = block_run_table(rng, S, L, nb, bs, idt, pdt, spoil=[0, 3][case % 2])
    lens = lens_tensor(rng, S, L, idt)
    ko, vo = out_pair(S, L, H, D, io, gen)
    ks = vs = None
    if dt in (DType.F8_E4M3, DType.F8_E5M2):
        kind = ["tensor", "head", "block", "block_head"][(case // 2) % 4]
        if kind == "tensor":
            ks, vs = 0.021, 1.75
        else:
            shape = {"head": (H,), "block": (nb,), "block_head": (nb, H)}[kind]
            g = {"head": SG.PER_HEAD, "block": SG.PER_BLOCK, "block_head": SG.PER_BLOCK_HEAD}[kind]
            ks = ScaleArg(g, rng.uniform(0.01, 2.0, size=shape))
            vs = ScaleArg(g, rng.uniform(0.01, 2.0, size=shape))
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=io,
                        k_scale=ks, v_scale=vs)


# ---------------------------------------------------------------------------
# KV_OFFSETS

def offsets_table(rng, S, mbps, nb, secondary_frac=0.4):
    raw = rng.integers(0, nb + 2, size=(S, 1, 2, mbps)).astype(np.uint32)
    raw |= (rng.random(raw.shape) < secondary_frac).astype(np.uint32) << 31
    return torch.from_numpy(raw.view(np.int32)).to(DEV)


@pytest.mark.parametrize("seed", range(24))
def test_kv_offsets_random(seed):
    rng = np.random.default_rng(4000 + seed)
    gen = torch.Generator().manual_seed(seed)
    dt = DTYPES[seed % 4]
    es = TORCH_DT[dt].itemsize
    kl, vl = LAYOUTS[seed % 3], LAYOUTS[(seed // 3) % 3]
    H = int(rng.choice([1, 2, 8]))
    D = int(rng.choice([8, 64, 128]))
    bs = int(rng.choice([1, 4, 16, 32]))
    nb = int(rng.integers(2, 40))
    pitch_pad = [0, 16, es, 256][seed % 4]
    pool = OffsetsPool(kl, vl, dt, nb, bs, H, D, pitch_pad=pitch_pad,
                       secondary=seed % 3 != 0, gen=gen)
    S, L = int(rng.integers(1, 7)), int(rng.integers(1, 300))
    mbps = int(rng.integers(1, (L + bs - 1) // bs + 2))
    offsets = offsets_table(rng, S, mbps, nb)
    lens = lens_tensor(rng, S, L, [np.int32, np.int64][seed % 2])
    ko, vo = out_pair(S, L, H, D, dt, gen, misalign=seed % 5 == 4)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_kv_offsets_fp8_dequant(io, layout):
    rng = np.random.default_rng(43)
    gen = torch.Generator().manual_seed(43)
    H, D, bs, nb, S, L = 4, 128, 16, 24, 5, 90
    pool = OffsetsPool(layout, layout, DType.F8_E4M3, nb, bs, H, D, pitch_pad=64, gen=gen)
    offsets = offsets_table(rng, S, (L + bs - 1) // bs, nb)
    lens = lens_tensor(rng, S, L, np.int32)
    ko, vo = out_pair(S, L, H, D, io, gen)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=DType.F8_E4M3,
                         io_dtype=io, k_scale=0.0172, v_scale=3.5)


@pytest.mark.parametrize("dt,H", [(DType.F32, 16), (DType.BF16, 32)])
def test_kv_offsets_wide_rows(dt, H):
    rng = np.random.default_rng(6)
    gen = torch.Generator().manual_seed(6)
    D, bs, nb, S, L = 128, 16, 12, 3, 70
    pool = OffsetsPool(HND, HND, dt, nb, bs, H, D, gen=gen)
    offsets = offsets_table(rng, S, (L + bs - 1) // bs, nb)
    lens = lens_tensor(rng, S, L, np.int32)
    ko, vo = out_pair(S, L, H, D, dt, gen)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("dt", [DType.BF16, DType.F16, DType.F32])
def test_kv_offsets_abi_entry(dt):
    """kvx_gather_kv (kvx_abi.h) executes KV_OFFSETS tables: the pool is
    device memory, the cache tensors carry the canonical block layout."""
    rng = np.random.default_rng(10)
    gen = torch.Generator().manual_seed(10)
    H, D, bs, nb, S, L = 8, 128, 16, 32, 4, 64
    for layout in LAYOUTS:
        pool = OffsetsPool(layout, layout, dt, nb, bs, H, D, gen=gen)
        offsets = offsets_table(rng, S, (L + bs - 1) // bs, nb)
        lens = lens_tensor(rng, S, L, np.int32)
        ko, vo = out_pair(S, L, H, D, dt, gen)
        check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=dt,
                             entry="abi")


@pytest.mark.parametrize("seed", range(16))
def test_kv_offsets_pool_blocks(seed):
    """kvx_launch_gather_kv_pools: entries at or past their pool's block
    count are skipped.  Both pools are allocated with num_blocks blocks, so
    an entry the kernel should skip but reads would show up as gathered
    bytes, not as an access outside the buffers.  Layouts, dtypes, FP8
    dequantizing gathers, narrow rows (per-tile table entries) and counts of
    0, 1, below and above num_blocks."""
    rng = np.random.default_rng(7000 + seed)
    gen = torch.Generator().manual_seed(700 + seed)
    dt = [DType.BF16, DType.F16, DType.F32, DType.F8_E4M3][seed % 4]
    kl, vl = LAYOUTS[seed % 3], LAYOUTS[(seed // 3) % 3]
    H = [1, 2, 8][seed % 3]
    D = [64, 128, 32][(seed // 2) % 3]
    bs = [16, 4, 32, 1][(seed // 4) % 4]
    nb = int(rng.integers(12, 40))
    pool = OffsetsPool(kl, vl, dt, nb, bs, H, D, pitch_pad=[0, 64][seed % 2], gen=gen)
    S, L = int(rng.integers(2, 6)), int(rng.integers(bs, 200))
    mbps = (L + bs - 1) // bs
    offsets = offsets_table(rng, S, mbps, nb, secondary_frac=0.5)
    lens = lens_tensor(rng, S, L, [np.int32, np.int64][seed % 2])
    counts = [(0, nb // 3), (nb // 2, 0), (nb - 1, 1), (nb + 5, 2)][seed % 4]
    if dt == DType.F8_E4M3:
        io = [DType.BF16, DType.F16, DType.F32][seed % 3]
        ko, vo = out_pair(S, L, H, D, io, gen)
        check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=io,
                             k_scale=0.031, v_scale=1.25, pool_blocks=counts)
    else:
        ko, vo = out_pair(S, L, H, D, dt, gen)
        check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=dt,
                             pool_blocks=counts)


def test_kv_offsets_trtllm_pairs():
    """TensorRT-LLM's pairing: the V block of a K block is the next pool
    block; all tokens of every sequence valid, no secondary pool."""
    gen = torch.Generator().manual_seed(12)
    H, D, bs, S, L = 8, 128, 32, 16, 512
    mbps = L // bs
    nb = 2 * S * mbps
    pool = OffsetsPool(HND, HND, DType.BF16, nb, bs, H, D, secondary=False, gen=gen)
    k = torch.arange(0, nb, 2, dtype=torch.int32).reshape(S, 1, mbps)
    offsets = torch.stack([k, k + 1], dim=2).to(DEV)          # [S, 1, 2, M]
    lens = torch.full((S,), L, dtype=torch.int32, device=DEV)
    ko, vo = out_pair(S, L, H, D, DType.BF16, gen)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=DType.BF16,
                         io_dtype=DType.BF16)


ODD_CHUNKS = [(1, 576, DType.BF16), (6, 128, DType.BF16), (3, 80, DType.F16),
              (1, 576, DType.F8_E4M3)]


@pytest.mark.parametrize("shape", ODD_CHUNKS, ids=["mla576", "6x128", "f16-3x80", "fp8-mla576"])
@pytest.mark.parametrize("spoil", [0, 4])
def test_row_major_chunk_counts_not_pow2(shape, spoil):
    """Canonical NHD caches whose rows hold a chunk count that is not a power
    of two (DeepSeek's 576-element MLA rows: 72 chunks; 6 x 128; 3 x 80):
    the flat write (decode and prefill rows), the RAGGED row-tile kernel
    (one-block and per-row paths, with `spoil` ids spoiled) and the
    KV_OFFSETS flat kernel (per-tile table entries), copies and the FP8
    quantizing write and dequantizing gather."""
    H, D, dt = shape
    seed = 7500 + ODD_CHUNKS.index(shape) * 2 + (spoil > 0)
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    fp8 = dt == DType.F8_E4M3
    io = DType.BF16 if fp8 else dt
    ks, vs = (0.019, 0.0043) if fp8 else (None, None)
    bs, nb = 16, 40
    pc, kb, vb = make_cache(NHD, NHD, dt, nb, bs, H, D, gen=gen)
    # writes first (write_flat_kernel with a multiply-high token lookup):
    # decode rows to scattered slots, then a prefill run
    T = 37
    slots = torch.from_numpy(rng.permutation(nb * bs)[:T].astype(np.int64))
    slots[5] = -1
    for n, sl in ((T, slots), (64, torch.arange(64) + 3 * bs + 5)):
        key = (torch.randn((n, H, D), generator=gen) * 2).to(TORCH_DT[io]).to(DEV)
        val = torch.randn((n, H, D), generator=gen).to(TORCH_DT[io]).to(DEV)
        check_write(pc, kb, vb, key, val, sl.to(DEV), io_dtype=io, cache_dtype=dt,
                    k_scale=ks, v_scale=vs)
    S, L = 5, 120
    table = block_run_table(rng, S, L, nb, bs, np.int32, np.int64, spoil=spoil)
    lens = lens_tensor(rng, S, L, np.int32)
    ko, vo = out_pair(S, L, H, D, io, gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=io,
                        k_scale=ks, v_scale=vs)
    pool = OffsetsPool(NHD, NHD, dt, nb, bs, H, D, pitch_pad=32, gen=gen)
    offsets = offsets_table(rng, S, (L + bs - 1) // bs, nb)
    ko, vo = out_pair(S, L, H, D, io, gen)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=dt, io_dtype=io,
                         k_scale=ks, v_scale=vs)


def test_ragged_malformed_indptr_stays_in_bounds():
    """indptr that decreases or points past the indices array: rows whose
    token index falls outside [0, indices_count) are skipped, the rest
    gathered, nothing read out of bounds."""
    gen = torch.Generator().manual_seed(13)
    H, D, bs, nb, L = 2, 64, 4, 8, 12
    pc, kb, vb = make_cache(NHD, NHD, DType.BF16, nb, bs, H, D, gen=gen)
    indices = torch.arange(20, dtype=torch.int32, device=DEV) % nb
    indptr = torch.tensor([0, 10, 6, 18, 40, -3], dtype=torch.int64, device=DEV)
    lens = torch.full((5,), L, dtype=torch.int32, device=DEV)
    ko, vo = out_pair(5, L, H, D, DType.BF16, gen)
    check_gather_ragged(pc, kb, vb, ko, vo, paged.RaggedTable(indices, indptr), lens, L,
                        cache_dtype=DType.BF16, io_dtype=DType.BF16)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_block_pool_write_then_offsets_gather(layout):
    """alloc_block_pool: PACKED writes into the paired K / V views, then a
    KV_OFFSETS gather over the pool returns what a PACKED gather returns."""
    from kvx_amd import workloads as W

    w = W.c1_tinyllama()
    gen = torch.Generator().manual_seed(21)
    pool, kv = paged.alloc_block_pool(w.num_blocks, w.block_size, w.heads, w.head_dim,
                                      torch.float16, DEV, layout)
    random_fill(pool.key_cache, gen)
    T = w.num_tokens
    key = random_fill(torch.empty((T, w.heads, w.head_dim), dtype=torch.float16,
                                  device=DEV), gen)
    val = random_fill(torch.empty_like(key), gen)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(kv, key, val, slots, tokens_per_seq=w.tokens_per_seq) == 0
    lens = torch.tensor(w.seq_lens, device=DEV)
    shape = (w.seq_count, w.max_seq_len, w.heads, w.head_dim)
    pk, pv = torch.zeros(shape, dtype=torch.float16, device=DEV), torch.zeros(
        shape, dtype=torch.float16, device=DEV)
    assert paged.gather_kv(kv, pk, pv, torch.tensor(w.block_table, device=DEV), lens,
                           w.max_seq_len) == 0
    ok, ov = torch.zeros_like(pk), torch.zeros_like(pv)
    offs = torch.tensor(W.kv_offsets_table(w), device=DEV)
    assert paged.gather_kv(pool, ok, ov, paged.pool_table(pool, offs), lens,
                           w.max_seq_len) == 0
    torch.cuda.synchronize()
    assert torch.equal(ok.view(torch.int16), pk.view(torch.int16))
    assert torch.equal(ov.view(torch.int16), pv.view(torch.int16))
    # the written rows are the inputs (c1 writes every gathered token)
    assert torch.equal(pk.view(torch.int16).reshape(T, -1), key.view(torch.int16).reshape(T, -1))
