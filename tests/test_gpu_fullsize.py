"""Full-size benchmark configurations (c1-c5) on the GPU, checked through properties
that do not need the CPU oracle to run at that size:

  - write -> gather round trip: every written row comes back bit-exact at its
    sequence position (c2 also on vLLM's x-packed K / token-innermost V pair,
    with PACKED and RAGGED tables; c2 and c3 also with other rows and block
    sizes: HND heads of 96 or 80 elements, three heads, blocks of 1, 128
    and 256 tokens);
  - the whole gather equals an independent implementation (torch advanced
    indexing of the paged cache on int16 views), row by row, and rows past
    seq_len keep the output's prior contents;
  - cache blocks the write does not address keep their prior contents;
  - FP8 (c4): the quantized rows match the oracle (they are few), and the
    full dequantizing gather equals torch's own float8_e4m3fn -> f32 * scale
    -> bf16 chain with NaNs canonicalised.
"""
import numpy as np
import pytest
import torch

import oracle
from kvx_amd import paged, workloads
from kvx_amd.abi import DType, Layout, Status

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _release_device_memory():
    """Full-size tests hold up to ~220 GB; return it to the device between
    tests so the next large allocation is not fragmented."""
    torch.cuda.empty_cache()
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def i16(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.uint8)


def block_view(cache: torch.Tensor, layout: Layout, pack: int) -> torch.Tensor:
    """[nb, bs, H, D] view (element order) of a canonical cache tensor, or of a
    4-axis CUSTOM tensor (already that logical view)."""
    if layout == Layout.BLOCK_NHD or (layout == Layout.BLOCK_CUSTOM and cache.dim() == 4):
        return cache
    if layout == Layout.BLOCK_HND:
        return cache.permute(0, 2, 1, 3)
    nb, H, dx, bs, x = cache.shape
    return cache.permute(0, 3, 1, 2, 4).reshape(nb, bs, H, dx * x)


def check_gather_against_indexing(pc, w, ko, vo, ko_before, vo_before, seqs_per_chunk=16):
    """Compare every gathered row with cache[block_table] and every padding
    row with the output's previous contents."""
    bs, L = w.block_size, w.max_seq_len
    table = torch.tensor(w.block_table, device=DEV).long()
    lens = torch.tensor(w.seq_lens, device=DEV).long().clamp(min=0, max=L)
    kv = [block_view(pc.key_cache, pc.k_layout, w.pack), block_view(pc.value_cache, pc.v_layout, w.pack)]
    pos = torch.arange(L, device=DEV)
    for s0 in range(0, w.seq_count, seqs_per_chunk):
        s1 = min(s0 + seqs_per_chunk, w.seq_count)
        lb = (pos // bs).clamp(max=w.max_blocks_per_seq - 1)
        bid = table[s0:s1][:, lb]                                   # [n, L]
        valid = (pos[None, :] < lens[s0:s1, None]) & (pos[None, :] // bs < w.max_blocks_per_seq)
        valid &= (bid >= 0) & (bid < w.num_blocks)
        for src, out, before in zip(kv, (ko, vo), (ko_before, vo_before)):
            ref = i16(src)[bid.clamp(min=0, max=w.num_blocks - 1), pos[None, :] % bs]  # [n, L, H, D]
            got = i16(out[s0:s1])
            old = i16(before[s0:s1])
            m = valid[:, :, None, None]
            assert torch.equal(torch.where(m, ref, old), got), f"sequences {s0}..{s1}"
            del ref


def ragged_equals_packed(pc, w, ko, vo, out_k, out_v, k_scale=None, v_scale=None):
    """The workload's table as a RAGGED table (one block id per token) gathers
    the same bytes as the PACKED gather into ko / vo: every gathered row, and
    the untouched rows past each length (out_k / out_v still hold what ko / vo
    held before their gather).  Canonical NHD caches with block-structured
    RAGGED tables take the row-tile RAGGED kernel."""
    indices, indptr = workloads.ragged_table(w)
    table = paged.RaggedTable(torch.tensor(indices, device=DEV), torch.tensor(indptr, device=DEV))
    assert paged.gather_kv(pc, out_k, out_v, table, torch.tensor(w.seq_lens, device=DEV),
                           w.max_seq_len, k_scale=k_scale, v_scale=v_scale) == Status.OK
    torch.cuda.synchronize()
    assert torch.equal(i16(out_k), i16(ko))
    assert torch.equal(i16(out_v), i16(vo))


def sentinel_like(shape, dtype, fill=-5):
    t = torch.empty(shape, dtype=dtype, device=DEV)
    i16(t).fill_(fill)
    return t


def test_c2_full_decode_write_then_gather():
    w = workloads.c2_llama8b_decode()
    H, D, bs = w.heads, w.head_dim, w.block_size
    pc = paged.alloc_cache(w.num_blocks, bs, H, D, torch.bfloat16, DEV)
    pc.key_cache.normal_()
    pc.value_cache.normal_()
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    k0, v0 = pc.key_cache.clone(), pc.value_cache.clone()
    assert paged.write_kv(pc, key, val, slots) == Status.OK
    torch.cuda.synchronize()
    # only the addressed rows changed, and they hold the new tokens
    ok = slots >= 0
    blk, off = slots[ok] // bs, slots[ok] % bs
    assert torch.equal(i16(pc.key_cache[blk, off]), i16(key[ok]))
    assert torch.equal(i16(pc.value_cache[blk, off]), i16(val[ok]))
    k0[blk, off] = pc.key_cache[blk, off]
    v0[blk, off] = pc.value_cache[blk, off]
    assert torch.equal(i16(k0), i16(pc.key_cache)) and torch.equal(i16(v0), i16(pc.value_cache))
    del k0, v0

    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16, 3)
    kb, vb = ko.clone(), vo.clone()
    table = torch.tensor(w.block_table, device=DEV)
    lens = torch.tensor(w.seq_lens, device=DEV)
    assert paged.gather_kv(pc, ko, vo, table, lens, L) == Status.OK
    torch.cuda.synchronize()
    # round trip: the new token of every non-padded sequence is at position len - 1
    seqs = torch.nonzero(ok).flatten()
    last = lens.long()[seqs] - 1
    assert torch.equal(i16(ko[seqs, last]), i16(key[seqs]))
    assert torch.equal(i16(vo[seqs, last]), i16(val[seqs]))
    check_gather_against_indexing(pc, w, ko, vo, kb, vb)


@pytest.mark.parametrize("table_fmt", ["packed", "ragged"])
def test_c2_full_vllm_layouts_write_then_gather(table_fmt):
    """c2 at full size on vLLM's paged-attention pair: K HND_PACKED x = 8 and
    V as CUSTOM [num_blocks, H, D, block_size] (token axis innermost), so the
    gather runs the LDS tile kernel on both tensors."""
    w = workloads.c2_llama8b_decode()
    H, D, bs, nb = w.heads, w.head_dim, w.block_size, w.num_blocks
    kc = torch.empty(paged.cache_shape(Layout.BLOCK_HND_PACKED, nb, bs, H, D, 8),
                     dtype=torch.bfloat16, device=DEV).normal_()
    vstore = torch.empty((nb, H, D, bs), dtype=torch.bfloat16, device=DEV).normal_()
    pc = paged.PagedCache(kc, paged.custom_view(vstore, "bhdo"), Layout.BLOCK_HND_PACKED,
                          Layout.BLOCK_CUSTOM, nb, bs, H, D)
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(pc, key, val, slots) == Status.OK
    torch.cuda.synchronize()
    ok = slots >= 0
    blk, off = slots[ok] // bs, slots[ok] % bs
    kview, vview = block_view(kc, Layout.BLOCK_HND_PACKED, 8), pc.value_cache
    assert torch.equal(i16(kview[blk, off]), i16(key[ok]))
    assert torch.equal(i16(vview[blk, off]), i16(val[ok]))

    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16, 3)
    kb, vb = ko.clone(), vo.clone()
    lens = torch.tensor(w.seq_lens, device=DEV)
    if table_fmt == "packed":
        table = torch.tensor(w.block_table, device=DEV)
    else:  # the same table, one block id per gathered token
        indices, indptr = workloads.ragged_table(w)
        table = paged.RaggedTable(torch.from_numpy(indices).to(DEV),
                                  torch.from_numpy(indptr).to(DEV))
    assert paged.gather_kv(pc, ko, vo, table, lens, L) == Status.OK
    torch.cuda.synchronize()
    seqs = torch.nonzero(ok).flatten()
    last = lens.long()[seqs] - 1
    assert torch.equal(i16(ko[seqs, last]), i16(key[seqs]))
    assert torch.equal(i16(vo[seqs, last]), i16(val[seqs]))
    check_gather_against_indexing(pc, w, ko, vo, kb, vb)


@pytest.mark.parametrize("v_layout", [Layout.BLOCK_NHD, Layout.BLOCK_HND])
def test_c3_full_prefill_packed_write_roundtrip(v_layout):
    w = workloads.c3_llama8b_prefill(v_layout=v_layout)
    H, D, bs = w.heads, w.head_dim, w.block_size
    pc = paged.alloc_cache(w.num_blocks, bs, H, D, torch.bfloat16, DEV, w.k_layout, w.v_layout,
                           w.pack)
    i16(pc.key_cache).fill_(-7)
    i16(pc.value_cache).fill_(-7)
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(pc, key, val, slots, tokens_per_seq=w.tokens_per_seq) == Status.OK
    torch.cuda.synchronize()
    # every written row is in place (through the layout's own indexing)
    kview = block_view(pc.key_cache, pc.k_layout, w.pack)
    vview = block_view(pc.value_cache, pc.v_layout, w.pack)
    blk, off = slots // bs, slots % bs
    assert torch.equal(i16(kview[blk, off]), i16(key))
    assert torch.equal(i16(vview[blk, off]), i16(val))
    # blocks outside the table are untouched
    used = torch.zeros(w.num_blocks, dtype=torch.bool, device=DEV)
    used[torch.tensor(w.block_table, device=DEV).long().flatten()] = True
    assert bool((i16(pc.key_cache[~used]) == -7).all()) and bool((i16(pc.value_cache[~used]) == -7).all())
    # gather back: the contiguous output equals the input rows
    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16)
    assert paged.gather_kv(pc, ko, vo, torch.tensor(w.block_table, device=DEV),
                           torch.tensor(w.seq_lens, device=DEV), L) == Status.OK
    torch.cuda.synchronize()
    assert torch.equal(i16(ko.reshape(-1, H, D)), i16(key))
    assert torch.equal(i16(vo.reshape(-1, H, D)), i16(val))


def test_c4_full_fp8_quantize_and_dequant_gather():
    w = workloads.c4_llama8b_fp8()
    H, D, bs = w.heads, w.head_dim, w.block_size
    pc = paged.alloc_cache(w.num_blocks, bs, H, D, torch.float8_e4m3fn, DEV)
    pc.key_cache.view(torch.uint8).random_(0, 256)
    pc.value_cache.view(torch.uint8).random_(0, 256)
    g = torch.Generator(device=DEV).manual_seed(w.notes["calibration_seed"])
    cal = torch.randn((w.num_tokens, H, D), generator=g, device=DEV) * 2.0
    ks = (cal.abs().max() / 448.0).reshape(1).float()
    vs = (ks * 0.75).contiguous()
    key = (torch.randn((w.num_tokens, H, D), device=DEV) * 2.0).to(torch.bfloat16)
    val = (torch.randn((w.num_tokens, H, D), device=DEV) * 2.0).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(pc, key, val, slots, k_scale=ks, v_scale=vs) == Status.OK
    torch.cuda.synchronize()
    ok = slots >= 0
    blk, off = slots[ok] // bs, slots[ok] % bs
    for src, cache, sc in ((key, pc.key_cache, ks), (val, pc.value_cache, vs)):
        want = oracle.quantize_e4m3(src[ok].view(torch.int16).cpu().numpy().view(np.uint16),
                                    DType.BF16, float(sc))
        got = cache[blk, off].view(torch.uint8).cpu().numpy().reshape(-1)
        assert np.array_equal(got, want)

    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16)
    kb, vb = ko.clone(), vo.clone()
    assert paged.gather_kv(pc, ko, vo, torch.tensor(w.block_table, device=DEV),
                           torch.tensor(w.seq_lens, device=DEV), L, k_scale=ks,
                           v_scale=vs) == Status.OK
    torch.cuda.synchronize()
    # reference caches: torch's own float8 -> f32 * scale -> bf16, NaN canonical
    def deq(c, sc):
        y = (c.float() * sc).to(torch.bfloat16)
        bits = y.view(torch.int16).clone()
        bits[torch.isnan(y)] = 0x7FC0
        return bits.view(torch.bfloat16)
    ref = paged.PagedCache(deq(pc.key_cache, ks), deq(pc.value_cache, vs), pc.k_layout,
                           pc.v_layout, pc.num_blocks, bs, H, D)
    check_gather_against_indexing(ref, w, ko, vo, kb, vb)
    ragged_equals_packed(pc, w, ko, vo, kb, vb, k_scale=ks, v_scale=vs)


def test_c5_full_long_context_200gb_pool():
    w = workloads.c5_llama70b_long()
    H, D, bs = w.heads, w.head_dim, w.block_size
    free, _ = torch.cuda.mem_get_info()
    need = 2 * w.num_blocks * bs * H * D * 2 + 4 * w.seq_count * w.max_seq_len * H * D * 2
    if free < need * 1.05:
        pytest.skip(f"needs {need / 1e9:.0f} GB of free device memory, {free / 1e9:.0f} GB free")
    pc = paged.alloc_cache(w.num_blocks, bs, H, D, torch.bfloat16, DEV)
    pc.key_cache.normal_()
    pc.value_cache.normal_()
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(pc, key, val, slots, tokens_per_seq=w.tokens_per_seq) == Status.OK
    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16)
    kb, vb = ko.clone(), vo.clone()
    assert paged.gather_kv(pc, ko, vo, torch.tensor(w.block_table, device=DEV),
                           torch.tensor(w.seq_lens, device=DEV), L) == Status.OK
    torch.cuda.synchronize()
    # the 32 written tokens of each sequence are its last 32 rows
    lens = torch.tensor(w.seq_lens, device=DEV).long()
    tps = w.tokens_per_seq
    idx = (lens[:, None] - tps + torch.arange(tps, device=DEV)[None, :])
    srow = torch.arange(S, device=DEV)[:, None].expand(-1, tps)
    assert torch.equal(i16(ko[srow, idx]).reshape(-1, H, D), i16(key))
    assert torch.equal(i16(vo[srow, idx]).reshape(-1, H, D), i16(val))
    check_gather_against_indexing(pc, w, ko, vo, kb, vb, seqs_per_chunk=4)
    ragged_equals_packed(pc, w, ko, vo, kb, vb)


@pytest.mark.parametrize("cfg", ["c2", "c5"])
def test_one_kv_head_rank_shape(cfg):
    """One tensor-parallel rank's share of the c2 / c5 caches: one KV head of
    eight (Llama-3-70B at TP8), so 256-byte rows and 16 chunks per row, with
    the 8-head workload's tables, lengths and slots.  Write, then gather;
    checked row by row against the slots and against indexing, by the round
    trip of the written tokens, and against the RAGGED form of the table."""
    w = workloads.CONFIGS[cfg]()
    w.heads = 1
    H, D, bs = w.heads, w.head_dim, w.block_size
    pc = paged.alloc_cache(w.num_blocks, bs, H, D, torch.bfloat16, DEV)
    pc.key_cache.normal_()
    pc.value_cache.normal_()
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    kw = {"tokens_per_seq": w.tokens_per_seq} if w.tokens_per_seq else {}
    assert paged.write_kv(pc, key, val, slots, **kw) == Status.OK
    torch.cuda.synchronize()
    ok = slots >= 0
    blk, off = slots[ok] // bs, slots[ok] % bs
    assert torch.equal(i16(pc.key_cache[blk, off]), i16(key[ok]))
    assert torch.equal(i16(pc.value_cache[blk, off]), i16(val[ok]))

    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16, 3)
    kb, vb = ko.clone(), vo.clone()
    lens = torch.tensor(w.seq_lens, device=DEV)
    assert paged.gather_kv(pc, ko, vo, torch.tensor(w.block_table, device=DEV), lens, L) == Status.OK
    torch.cuda.synchronize()
    # the written tokens are the last rows of their sequences
    tps = w.tokens_per_seq or 1
    seq = torch.arange(S, device=DEV).repeat_interleave(tps)
    pos = (lens.long()[seq] - tps + torch.arange(tps, device=DEV).repeat(S))
    assert torch.equal(i16(ko[seq[ok], pos[ok]]), i16(key[ok]))
    assert torch.equal(i16(vo[seq[ok], pos[ok]]), i16(val[ok]))
    check_gather_against_indexing(pc, w, ko, vo, kb, vb)
    ragged_equals_packed(pc, w, ko, vo, kb, vb)


SHAPES = [  # (name, K / V layout, heads, head_dim, block_size)
    ("hnd_8x96", Layout.BLOCK_HND, 8, 96, 16),          # tiles of whole 192-byte runs
    ("xpacked_3x128", Layout.BLOCK_HND_PACKED, 3, 128, 16),  # 768-byte tile rows
    ("xpacked_bs256", Layout.BLOCK_HND_PACKED, 8, 128, 256),  # 128-byte tile rows
    ("hnd_bs256", Layout.BLOCK_HND, 8, 128, 256),        # row kernel, 16 parts per block
    ("hnd_bs1", Layout.BLOCK_HND, 8, 128, 1),            # one-token blocks: row-major kernels
]


@pytest.mark.parametrize("shape", SHAPES, ids=[c[0] for c in SHAPES])
def test_c2_full_other_shapes(shape):
    """c2's lengths, slots and table for other rows and block sizes: decode
    write, then gather; checked against the slots, against indexing, by the
    round trip of the written tokens, and against the RAGGED form of the
    table."""
    _, lay, H, D, bs = shape
    w = workloads.c2_llama8b_decode(block_size=bs)
    w.heads, w.head_dim = H, D
    pc = paged.alloc_cache(w.num_blocks, bs, H, D, torch.bfloat16, DEV, lay, lay, w.pack)
    pc.key_cache.normal_()
    pc.value_cache.normal_()
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(pc, key, val, slots) == Status.OK
    torch.cuda.synchronize()
    ok = slots >= 0
    blk, off = slots[ok] // bs, slots[ok] % bs
    kview, vview = block_view(pc.key_cache, lay, w.pack), block_view(pc.value_cache, lay, w.pack)
    assert torch.equal(i16(kview[blk, off]), i16(key[ok]))
    assert torch.equal(i16(vview[blk, off]), i16(val[ok]))
    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16, 3)
    kb, vb = ko.clone(), vo.clone()
    lens = torch.tensor(w.seq_lens, device=DEV)
    assert paged.gather_kv(pc, ko, vo, torch.tensor(w.block_table, device=DEV), lens, L) == Status.OK
    torch.cuda.synchronize()
    seq = torch.arange(S, device=DEV)
    pos = lens.long() - 1
    assert torch.equal(i16(ko[seq[ok], pos[ok]]), i16(key[ok]))
    assert torch.equal(i16(vo[seq[ok], pos[ok]]), i16(val[ok]))
    check_gather_against_indexing(pc, w, ko, vo, kb, vb)
    ragged_equals_packed(pc, w, ko, vo, kb, vb)


WRITE_SHAPES = [  # (name, layouts, heads, head_dim, block_size)
    ("xpacked_3x128", "packed", 3, 128, 16),
    ("vllm_3x128", "vllm", 3, 128, 16),
    ("hnd_8x80", "hnd", 8, 80, 16),
    ("hnd_bs128", "hnd", 8, 128, 128),
    ("vllm_bs1", "vllm", 8, 128, 1),
]


@pytest.mark.parametrize("shape", WRITE_SHAPES, ids=[c[0] for c in WRITE_SHAPES])
def test_c3_full_other_shapes(shape):
    """c3's prefill chunks into caches of other rows and block sizes (tiles
    of whole runs, the per-token path of 128-token blocks, one-token
    blocks): every written row in place, untouched blocks unchanged, and the
    gather returning the input rows."""
    _, lay, H, D, bs = shape
    w = workloads.c3_llama8b_prefill(block_size=bs)
    w.heads, w.head_dim = H, D
    nb = w.num_blocks
    if lay == "vllm":
        kc = torch.empty(paged.cache_shape(Layout.BLOCK_HND_PACKED, nb, bs, H, D, 8),
                         dtype=torch.bfloat16, device=DEV)
        vstore = torch.empty((nb, H, D, bs), dtype=torch.bfloat16, device=DEV)
        pc = paged.PagedCache(kc, paged.custom_view(vstore, "bhdo"), Layout.BLOCK_HND_PACKED,
                              Layout.BLOCK_CUSTOM, nb, bs, H, D)
        fills = (kc, vstore)
    else:
        code = {"packed": Layout.BLOCK_HND_PACKED, "hnd": Layout.BLOCK_HND}[lay]
        pc = paged.alloc_cache(nb, bs, H, D, torch.bfloat16, DEV, code, code, 8)
        fills = (pc.key_cache, pc.value_cache)
    for t in fills:
        i16(t).fill_(-7)
    key = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((w.num_tokens, H, D), device=DEV).to(torch.bfloat16)
    slots = torch.tensor(w.slots, device=DEV)
    assert paged.write_kv(pc, key, val, slots, tokens_per_seq=w.tokens_per_seq) == Status.OK
    torch.cuda.synchronize()
    kview = block_view(pc.key_cache, pc.k_layout, 8)
    vview = block_view(pc.value_cache, pc.v_layout, 8)
    blk, off = slots // bs, slots % bs
    assert torch.equal(i16(kview[blk, off]), i16(key))
    assert torch.equal(i16(vview[blk, off]), i16(val))
    used = torch.zeros(nb, dtype=torch.bool, device=DEV)
    used[torch.tensor(w.block_table, device=DEV).long().flatten()] = True
    for t in fills:
        assert bool((i16(t[~used]) == -7).all())
    S, L = w.seq_count, w.max_seq_len
    ko, vo = sentinel_like((S, L, H, D), torch.bfloat16), sentinel_like((S, L, H, D), torch.bfloat16)
    assert paged.gather_kv(pc, ko, vo, torch.tensor(w.block_table, device=DEV),
                           torch.tensor(w.seq_lens, device=DEV), L) == Status.OK
    torch.cuda.synchronize()
    assert torch.equal(i16(ko.reshape(-1, H, D)), i16(key))
    assert torch.equal(i16(vo.reshape(-1, H, D)), i16(val))


def test_token_write_grid_stride_loop():
    """A write of more rows than the per-token kernel's grid holds (65536
    workgroups of 4 waves, one row per wave): its waves loop over the
    remaining rows.  NHD caches whose head rows are padded (stride D + 8) are
    neither row-dense nor dense blocks, so the write takes write_kernel.
    Random distinct slots with -1 and out-of-range entries; every written
    row, every pad element and every untouched block is checked with torch
    indexing."""
    H, D, bs = 3, 128, 16
    T = 300_000
    nb = (T + T // 4) // bs
    gen = torch.Generator(device=DEV).manual_seed(77)
    kst = torch.empty((nb, bs, H, D + 8), dtype=torch.bfloat16, device=DEV)
    vst = torch.empty_like(kst)
    kst.view(torch.int16).random_(generator=gen)
    vst.view(torch.int16).random_(generator=gen)
    pc = paged.PagedCache(kst[..., :D], vst[..., :D], Layout.BLOCK_NHD, Layout.BLOCK_NHD, nb, bs,
                          H, D)
    k0, v0 = kst.clone(), vst.clone()
    slots = torch.randperm(nb * bs, generator=gen, device=DEV)[:T]
    slots[torch.rand(T, generator=gen, device=DEV) < 0.05] = -1
    slots[torch.rand(T, generator=gen, device=DEV) < 0.01] = nb * bs + 7  # past the blocks
    key = torch.empty((T, H, D), dtype=torch.bfloat16, device=DEV).normal_(generator=gen)
    val = torch.empty_like(key).normal_(generator=gen)
    assert paged.write_kv(pc, key, val, slots) == Status.OK
    torch.cuda.synchronize()
    ok = (slots >= 0) & (slots < nb * bs)
    want_k, want_v = k0.view(-1, H, D + 8), v0.view(-1, H, D + 8)
    want_k[slots[ok], :, :D] = key[ok]
    want_v[slots[ok], :, :D] = val[ok]
    assert torch.equal(i16(kst).view(-1, H, D + 8), i16(want_k))
    assert torch.equal(i16(vst).view(-1, H, D + 8), i16(want_v))


def test_flat_write_rows_not_pow2_chunks():
    """300,000 NHD rows of three heads (48 chunks, not a power of two): the
    flat write finds each chunk's token by multiply-high over 14.4 M flat
    indices.  Same checks as above."""
    H, D, bs = 3, 128, 16
    T = 300_000
    nb = (T + T // 4) // bs
    gen = torch.Generator(device=DEV).manual_seed(78)
    pc = paged.alloc_cache(nb, bs, H, D, torch.bfloat16, DEV)
    pc.key_cache.view(torch.int16).random_(generator=gen)
    pc.value_cache.view(torch.int16).random_(generator=gen)
    k0, v0 = pc.key_cache.clone(), pc.value_cache.clone()
    slots = torch.randperm(nb * bs, generator=gen, device=DEV)[:T]
    slots[torch.rand(T, generator=gen, device=DEV) < 0.05] = -1
    slots[torch.rand(T, generator=gen, device=DEV) < 0.01] = nb * bs + 7
    key = torch.empty((T, H, D), dtype=torch.bfloat16, device=DEV).normal_(generator=gen)
    val = torch.empty_like(key).normal_(generator=gen)
    assert paged.write_kv(pc, key, val, slots) == Status.OK
    torch.cuda.synchronize()
    ok = (slots >= 0) & (slots < nb * bs)
    want_k, want_v = k0.view(-1, H, D), v0.view(-1, H, D)
    want_k[slots[ok]] = key[ok]
    want_v[slots[ok]] = val[ok]
    assert torch.equal(i16(pc.key_cache).view(-1, H, D), i16(want_k))
    assert torch.equal(i16(pc.value_cache).view(-1, H, D), i16(want_v))


@pytest.mark.parametrize("layout", ["x_packed_nhd", "vllm"])
def test_c3_size_chunks_starting_inside_blocks(layout):
    """c3's size (16 sequences x 2048 tokens) with every chunk starting at a
    different offset inside its first block, into x-packed K with NHD V or
    vLLM's pair (x-packed K, token-innermost V): each block is owned by the
    group where its run starts (whole-block and shifted fast paths, the
    two-run groups at chunk starts).  Every row must land at its slot, every
    other byte of the caches keep its value."""
    H, D, bs, S, C, nb = 8, 128, 16, 16, 2048, 8192
    gen = torch.Generator().manual_seed(81)
    perm = torch.randperm(nb, generator=gen)
    slots, used = [], 0
    for s in range(S):
        off = (5 + 3 * s) % bs
        nblk = (off + C + bs - 1) // bs
        blocks = perm[used:used + nblk]
        used += nblk
        p = torch.arange(off, off + C)
        slots.append(blocks[p // bs] * bs + p % bs)
    slots = torch.cat(slots).to(DEV)
    kc = torch.empty(paged.cache_shape(Layout.BLOCK_HND_PACKED, nb, bs, H, D, 8),
                     dtype=torch.bfloat16, device=DEV)
    if layout == "vllm":
        vstore = torch.empty((nb, H, D, bs), dtype=torch.bfloat16, device=DEV)
        vc = paged.custom_view(vstore, "bhdo")
        pc = paged.PagedCache(kc, vc, Layout.BLOCK_HND_PACKED, Layout.BLOCK_CUSTOM, nb, bs, H, D)
    else:
        vstore = torch.empty((nb, bs, H, D), dtype=torch.bfloat16, device=DEV)
        pc = paged.PagedCache(kc, vstore, Layout.BLOCK_HND_PACKED, Layout.BLOCK_NHD, nb, bs, H, D)
    i16(kc).fill_(-7)
    i16(vstore).fill_(-7)
    T = slots.numel()
    key = torch.randn((T, H, D), device=DEV).to(torch.bfloat16)
    val = torch.randn((T, H, D), device=DEV).to(torch.bfloat16)
    assert paged.write_kv(pc, key, val, slots, tokens_per_seq=C) == Status.OK
    torch.cuda.synchronize()
    kview = block_view(pc.key_cache, pc.k_layout, 8)
    vview = block_view(pc.value_cache, pc.v_layout, 8)
    blk, off = slots // bs, slots % bs
    assert torch.equal(i16(kview[blk, off]), i16(key))
    assert torch.equal(i16(vview[blk, off]), i16(val))
    # no other byte changed: rows not addressed by a slot keep the sentinel
    hit = torch.zeros(nb * bs, dtype=torch.bool, device=DEV)
    hit[slots] = True
    hit = hit.view(nb, bs)
    assert bool((i16(kview)[~hit] == -7).all()) and bool((i16(vview)[~hit] == -7).all())
