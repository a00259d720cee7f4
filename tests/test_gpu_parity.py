"""GPU parity: libkvx_amd.so's HIP kernels, called through the C ABI, are
bit-identical to the CPU oracle on the same seeded inputs.

Covers the reference's own kernel-test cases (tests/kvx_kernel_test.cu),
every layout (NHD, HND, HND_PACKED, mixed K/V), F32/F16/BF16/FP8 payloads,
S32/S64 indices, -1 slots, out-of-range blocks, padded strides, odd head
dims and misaligned buffers (narrower chunk widths), the prefill entry, the
kvx_abi.h entry points, non-default and concurrent streams, and reduced
versions of the five benchmark configurations (c1-c5).
"""
import numpy as np
import pytest
import torch

from kvx_amd import paged, workloads
from kvx_amd.abi import DType, Layout, Status

from gpu_helpers import TORCH_DT, check_gather, check_write, make_cache, np_bytes, random_fill

pytestmark = pytest.mark.gpu
DEV = "cuda"
NHD, HND, PK = Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED


def rows(T, H, D, dtype, gen, device=DEV):
    t = torch.empty((T, H, D), dtype=TORCH_DT[dtype], device=device)
    return random_fill(t, gen)


def normal_rows(T, H, D, dtype, gen, sigma=1.0):
    x = torch.randn((T, H, D), generator=gen) * sigma
    return x.to(TORCH_DT[dtype]).to(DEV)


# ---------------------------------------------------------------------------
# Reference kernel-test cases (tests/kvx_kernel_test.cu:456-805)

@pytest.mark.parametrize("dt", [DType.F32, DType.F16, DType.BF16])
def test_reference_kernel_test_cases(dt):
    gen = torch.Generator().manual_seed(1)
    S, L, bs = 2, 4, 4
    for layout, H, D, tps, prefill in [(NHD, 2, 4, 1, False), (NHD, 1, 7, 1, False),
                                       (NHD, 2, 4, 2, False), (HND, 2, 4, 1, False),
                                       (HND, 1, 7, 2, False), (NHD, 2, 4, 2, True),
                                       (NHD, 1, 7, 2, True)]:
        nb = S
        T = S * tps
        i = torch.arange(T * H * D, dtype=torch.float32)
        key = (0.1 + 0.01 * i).reshape(T, H, D).to(TORCH_DT[dt]).to(DEV)
        val = (0.6 + 0.01 * i).reshape(T, H, D).to(TORCH_DT[dt]).to(DEV)
        slots = torch.tensor([(s * 1 + (L - tps + t) // bs) * bs + (L - tps + t) % bs
                              for s in range(S) for t in range(tps)], dtype=torch.int64,
                             device=DEV)
        pc, kb, vb = make_cache(layout, layout, dt, nb, bs, H, D, gen=gen)
        check_write(pc, kb, vb, key, val, slots, io_dtype=dt, cache_dtype=dt,
                    tokens_per_seq=tps if prefill else None)
    # gather case :629-786
    pc, kb, vb = make_cache(NHD, NHD, dt, 2, 4, 2, 4, gen=gen)
    table = torch.tensor([[0], [1]], dtype=torch.int32, device=DEV)
    lens = torch.tensor([4, 4], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((2, 4, 2, 4), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, 4, cache_dtype=dt, io_dtype=dt)


# ---------------------------------------------------------------------------
# Randomized layouts, dtypes, indices, strides and alignments.

def _random_case(seed):
    rng = np.random.default_rng(1000 + seed)
    gen = torch.Generator().manual_seed(seed)
    layouts = [NHD, HND, PK]
    kl, vl = layouts[rng.integers(3)], layouts[rng.integers(3)]
    dt = [DType.F32, DType.F16, DType.BF16, DType.F8_E4M3][seed % 4]
    H = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([7, 8, 16, 64, 128, 256]))
    packs = [p for p in (1, 2, 4, 8, 16) if D % p == 0]
    pack = int(rng.choice(packs))
    bs, nb = int(rng.choice([1, 4, 16, 32])), int(rng.integers(3, 40))
    # pad one axis of the cache tensors (non-canonical strides) 30% of the time
    k_pad = int(rng.integers(0, 4)) if rng.random() < 0.3 else None
    v_pad = int(rng.integers(0, 4)) if rng.random() < 0.3 else None
    return rng, gen, kl, vl, dt, H, D, pack, bs, nb, k_pad, v_pad


@pytest.mark.parametrize("seed", range(40))
def test_random_write_then_gather(seed):
    rng, gen, kl, vl, dt, H, D, pack, bs, nb, k_pad, v_pad = _random_case(seed)
    pc, kb, vb = make_cache(kl, vl, dt, nb, bs, H, D, pack, gen=gen, k_pad=k_pad,
                            v_pad=v_pad)
    T = int(rng.integers(1, 3 * nb * bs // 2 + 2))
    T = min(T, nb * bs + 2 * bs)
    slots = rng.permutation(nb * bs + 2 * bs)[:T]           # includes out-of-range blocks
    slots[rng.random(T) < 0.1] = -1
    slot_t = torch.tensor(slots, dtype=torch.int64 if seed % 2 else torch.int32,
                          device=DEV)
    misalign = seed % 5 == 0 and dt != DType.F32
    if misalign:
        # one element past a 16-byte boundary: forces narrower chunks
        kbig = rows(T * H * D + 1, 1, 1, dt, gen).reshape(-1)
        vbig = rows(T * H * D + 1, 1, 1, dt, gen).reshape(-1)
        key, val = kbig[1:].view(T, H, D), vbig[1:].view(T, H, D)
    else:
        key, val = rows(T, H, D, dt, gen), rows(T, H, D, dt, gen)
    tps = None
    if seed % 3 == 0:
        tps = int(np.gcd(T, 4)) or 1
    check_write(pc, kb, vb, key, val, slot_t, io_dtype=dt, cache_dtype=dt,
                tokens_per_seq=tps)

    S = int(rng.integers(1, 6))
    L = int(rng.integers(1, 4 * bs + 3))
    mbps = int(rng.integers(1, (L + bs - 1) // bs + 2))
    idt = torch.int64 if seed % 4 == 1 else torch.int32
    table = torch.tensor(rng.integers(-1, nb + 2, size=(S, mbps)), dtype=idt, device=DEV)
    lens = torch.tensor(rng.integers(-1, L + 3, size=S), dtype=idt, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=dt)


@pytest.mark.parametrize("dt", [DType.F16, DType.BF16, DType.F32])
def test_abi_entry_points_execute_on_device(dt):
    """kvx_write_kv / kvx_gather_kv (kvx_abi.h) on DEVICE buffers run the same
    kernels; canonical layouts only (the ABI path requires them)."""
    gen = torch.Generator().manual_seed(5)
    H, D, bs, nb = 4, 64, 16, 24
    pc, kb, vb = make_cache(HND, HND, dt, nb, bs, H, D, gen=gen)
    slots = torch.randperm(nb * bs, generator=gen)[:50].to(DEV)
    slots[::7] = -1
    key, val = rows(50, H, D, dt, gen), rows(50, H, D, dt, gen)
    check_write(pc, kb, vb, key, val, slots, io_dtype=dt, cache_dtype=dt, entry="abi")
    table = torch.randperm(nb, generator=gen)[:12].reshape(3, 4).to(torch.int64).to(DEV)
    lens = torch.tensor([64, 17, 0], dtype=torch.int64, device=DEV)
    ko = random_fill(torch.empty((3, 64, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, 64, cache_dtype=dt, io_dtype=dt,
                 entry="abi")


def test_non_default_stream():
    gen = torch.Generator().manual_seed(6)
    H, D, bs, nb = 8, 128, 16, 64
    pc, kb, vb = make_cache(NHD, NHD, DType.BF16, nb, bs, H, D, gen=gen)
    s = torch.cuda.Stream()
    slots = torch.randperm(nb * bs, generator=gen)[:300].to(DEV)
    key, val = rows(300, H, D, DType.BF16, gen), rows(300, H, D, DType.BF16, gen)
    torch.cuda.synchronize()
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.BF16, cache_dtype=DType.BF16,
                stream=s)


def test_two_streams_interleaved_on_separate_caches():
    """Writes and gathers on two streams, enqueued alternately with no
    synchronization between the streams, each on its own cache (NHD, and
    x-packed K with NHD V, so different kernels run side by side): the
    library keeps no state between calls, so each cache and each gather
    output must equal the oracle applying that stream's calls in order."""
    import oracle

    gen = torch.Generator().manual_seed(61)
    H, D, bs, nb, S, mbps = 8, 128, 16, 384, 12, 32
    dt = DType.BF16
    caches = [make_cache(NHD, NHD, dt, nb, bs, H, D, gen=gen),
              make_cache(PK, NHD, dt, nb, bs, H, D, gen=gen)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    expect = [[np_bytes(kb.base), np_bytes(vb.base)] for _, kb, vb in caches]
    launched = []
    torch.cuda.synchronize()
    for rnd in range(3):
        for c, ((pc, kb, vb), s) in enumerate(zip(caches, streams)):
            slots = torch.randperm(nb * bs, generator=gen)[:700].to(DEV)
            key, val = rows(700, H, D, dt, gen), rows(700, H, D, dt, gen)
            table = torch.randperm(nb, generator=gen)[:S * mbps].reshape(S, mbps)
            table = table.to(torch.int32).to(DEV)
            lens = torch.randint(0, mbps * bs + 1, (S,), generator=gen).to(torch.int32).to(DEV)
            ko = random_fill(torch.empty((S, mbps * bs, H, D), dtype=TORCH_DT[dt], device=DEV), gen)
            vo = random_fill(torch.empty_like(ko), gen)
            ko0, vo0 = np_bytes(ko), np_bytes(vo)
            # inputs are ready on the default stream before the side streams use them
            s.wait_stream(torch.cuda.current_stream())
            assert paged.write_kv(pc, key, val, slots, stream=s) == Status.OK
            assert paged.gather_kv(pc, ko, vo, table, lens, mbps * bs, stream=s) == Status.OK
            launched.append((c, key, val, slots, table, lens, ko, vo, ko0, vo0))
    torch.cuda.synchronize()
    for c, key, val, slots, table, lens, ko, vo, ko0, vo0 in launched:
        pc, kb, vb = caches[c]
        kexp, vexp = expect[c]
        oracle.write_kv(kb.geometry(), vb.geometry(), np_bytes(key), np_bytes(val), kexp, vexp,
                        slots.cpu().numpy(), heads=H, head_dim=D, block_size=bs,
                        num_blocks=nb, io_dtype=dt, cache_dtype=dt)
        oracle.gather_kv(kb.geometry(), vb.geometry(), kexp, vexp, ko0, vo0,
                         table.cpu().numpy(), lens.cpu().numpy(), seq_count=S,
                         max_blocks_per_seq=mbps, max_seq_len=mbps * bs, heads=H,
                         head_dim=D, block_size=bs, num_blocks=nb, cache_dtype=dt,
                         io_dtype=dt)
        assert np.array_equal(np_bytes(ko), ko0)
        assert np.array_equal(np_bytes(vo), vo0)
    for c, (pc, kb, vb) in enumerate(caches):
        assert np.array_equal(np_bytes(kb.base), expect[c][0])
        assert np.array_equal(np_bytes(vb.base), expect[c][1])


def test_empty_and_all_invalid_batches_leave_cache_untouched():
    gen = torch.Generator().manual_seed(7)
    pc, kb, vb = make_cache(NHD, NHD, DType.BF16, 8, 16, 8, 128, gen=gen)
    slots = torch.full((20,), -1, dtype=torch.int64, device=DEV)
    key, val = rows(20, 8, 128, DType.BF16, gen), rows(20, 8, 128, DType.BF16, gen)
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.BF16, cache_dtype=DType.BF16)
    slots = torch.arange(8 * 16, 8 * 16 + 20, dtype=torch.int64, device=DEV)  # all OOB
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.BF16, cache_dtype=DType.BF16)
    empty = rows(0, 8, 128, DType.BF16, gen)
    assert paged.write_kv(pc, empty, empty, slots[:0]) == Status.OK


# ---------------------------------------------------------------------------
# FP8 E4M3 cache: quantizing write, dequantizing gather, byte-copy paths.

@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
@pytest.mark.parametrize("scale", [1.0, 0.0044642857, 37.5, 1e-30])
def test_fp8_quantize_every_bf16_pattern(io, scale):
    """All 65536 bf16 bit patterns (as io values) quantized on the GPU."""
    gen = torch.Generator().manual_seed(8)
    H, D, bs = 8, 128, 16
    T = 65536 // (H * D)
    bits = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.float().to(TORCH_DT[io]).reshape(T, H, D).to(DEV)
    nb = T // bs + 2
    pc, kb, vb = make_cache(NHD, PK, DType.F8_E4M3, nb, bs, H, D, 16, gen=gen)
    slots = torch.randperm(nb * bs, generator=gen)[:T].to(DEV)
    check_write(pc, kb, vb, x, x.flip(0).contiguous(), slots, io_dtype=io,
                cache_dtype=DType.F8_E4M3, k_scale=scale, v_scale=scale * 2)


@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
@pytest.mark.parametrize("scale", [1.0, 0.0044642857, 37.5, 1e-30, 3e35])
def test_fp8_dequantize_every_code(io, scale):
    gen = torch.Generator().manual_seed(9)
    H, D, bs, nb = 2, 64, 16, 16
    pc, kb, vb = make_cache(NHD, HND, DType.F8_E4M3, nb, bs, H, D, gen=gen)
    S, L = 4, 64
    table = torch.randperm(nb, generator=gen)[:16].reshape(S, 4).to(torch.int32).to(DEV)
    lens = torch.tensor([64, 63, 17, 1], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=DType.F8_E4M3,
                 io_dtype=io, k_scale=scale, v_scale=scale / 3)


def test_fp8_scale_from_raw_pointer_and_byte_copies():
    gen = torch.Generator().manual_seed(10)
    H, D, bs, nb = 8, 128, 16, 32
    pc, kb, vb = make_cache(NHD, NHD, DType.F8_E4M3, nb, bs, H, D, gen=gen)
    T = 100
    key, val = normal_rows(T, H, D, DType.BF16, gen, 2.0), normal_rows(T, H, D, DType.BF16, gen)
    slots = torch.randperm(nb * bs, generator=gen)[:T].to(DEV)
    ks = torch.tensor([0.0123], device=DEV)
    vs = torch.tensor([0.004], device=DEV)
    # raw k_scale / v_scale pointers (no scale descriptors)
    from kvx_amd import abi
    import ctypes as C
    import oracle
    from gpu_helpers import np_bytes
    kb0, vb0 = np_bytes(kb.base), np_bytes(vb.base)
    wd = paged.build_write(pc, key, val, slots)
    wd.k_scale, wd.v_scale = ks.data_ptr(), vs.data_ptr()
    cd = pc.desc()
    lib = abi.load()
    assert lib.kvx_launch_write_kv(C.byref(cd), C.byref(wd), None) == Status.OK
    torch.cuda.synchronize()
    oracle.write_kv(kb.geometry(), vb.geometry(), np_bytes(key), np_bytes(val), kb0, vb0,
                    slots.cpu().numpy(), heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                    io_dtype=DType.BF16, cache_dtype=DType.F8_E4M3, k_scale=0.0123,
                    v_scale=0.004)
    assert np.array_equal(np_bytes(kb.base), kb0)
    assert np.array_equal(np_bytes(vb.base), vb0)
    # FP8 -> FP8 write and gather are byte copies (no scale)
    key8, val8 = rows(T, H, D, DType.F8_E4M3, gen), rows(T, H, D, DType.F8_E4M3, gen)
    check_write(pc, kb, vb, key8, val8, slots, io_dtype=DType.F8_E4M3,
                cache_dtype=DType.F8_E4M3)
    table = torch.arange(nb, dtype=torch.int32, device=DEV).reshape(4, 8)
    lens = torch.tensor([128, 5, 77, 0], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((4, 128, H, D), dtype=torch.float8_e4m3fn, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, 128, cache_dtype=DType.F8_E4M3,
                 io_dtype=DType.F8_E4M3)


# ---------------------------------------------------------------------------
# Reduced benchmark configurations (c1-c5), oracle-checked end to end.

def _run_workload(w, gen, v_layout=None, scale_k=None, scale_v=None, sigma=1.0):
    vl = w.v_layout if v_layout is None else v_layout
    pc, kb, vb = make_cache(w.k_layout, vl, w.cache_dtype, w.num_blocks, w.block_size,
                            w.heads, w.head_dim, w.pack, gen=gen)
    key = normal_rows(w.num_tokens, w.heads, w.head_dim, w.io_dtype, gen, sigma)
    val = normal_rows(w.num_tokens, w.heads, w.head_dim, w.io_dtype, gen, sigma)
    slots = torch.tensor(w.slots, device=DEV)
    check_write(pc, kb, vb, key, val, slots, io_dtype=w.io_dtype, cache_dtype=w.cache_dtype,
                tokens_per_seq=w.tokens_per_seq, k_scale=scale_k, v_scale=scale_v)
    table = torch.tensor(w.block_table, device=DEV)
    lens = torch.tensor(w.seq_lens, device=DEV)
    ko = random_fill(torch.empty((w.seq_count, w.max_seq_len, w.heads, w.head_dim),
                                 dtype=TORCH_DT[w.io_dtype], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, w.max_seq_len, cache_dtype=w.cache_dtype,
                 io_dtype=w.io_dtype, k_scale=scale_k, v_scale=scale_v)


def test_c1_tinyllama_full():
    _run_workload(workloads.c1_tinyllama(), torch.Generator().manual_seed(11))


def test_c2_decode_reduced():
    w = workloads.c2_llama8b_decode(batch=12)
    _run_workload(w, torch.Generator().manual_seed(12))


@pytest.mark.parametrize("v_layout", [NHD, HND])
def test_c3_prefill_packed_reduced(v_layout):
    w = workloads.c3_llama8b_prefill(v_layout=v_layout)
    keep = 2 * 2048
    w.slots = w.slots[:keep].copy()
    w.block_table, w.seq_lens = w.block_table[:2].copy(), w.seq_lens[:2].copy()
    _run_workload(w, torch.Generator().manual_seed(13))


def test_c4_fp8_reduced():
    w = workloads.c4_llama8b_fp8(batch=10)
    gen = torch.Generator().manual_seed(14)
    cal = (torch.randn((w.num_tokens, w.heads, w.head_dim), generator=gen) * 2.0)
    s = float(cal.abs().max()) / 448.0
    _run_workload(w, gen, scale_k=s, scale_v=s * 0.75, sigma=2.0)


def test_c5_long_context_reduced():
    w = workloads.c5_llama70b_long(pool_blocks=3000, batch=3)
    _run_workload(w, torch.Generator().manual_seed(15))


# ---------------------------------------------------------------------------
# Block write (prefill groups that fill whole blocks, staged through LDS).

def _block_slots(rng, nb, bs, groups):
    """Slots for `groups` groups of bs tokens: most fill one block in order;
    some have a -1, a swapped pair, an out-of-range block, or are cut short."""
    blocks = rng.permutation(nb)[:groups]
    slots = []
    for gi, b in enumerate(blocks):
        g = list(range(b * bs, b * bs + bs))
        kind = gi % 6
        if kind == 1:
            g[bs // 2] = -1
        elif kind == 2 and bs > 1:
            g[0], g[1] = g[1], g[0]
        elif kind == 3:
            g = list(range((nb + 1) * bs, (nb + 2) * bs))  # block past num_blocks
        slots += g
    return np.array(slots[: len(slots) - bs // 2], dtype=np.int64)  # partial tail


@pytest.mark.parametrize("kl,vl", [(PK, NHD), (HND, PK), (PK, PK), (HND, HND), (NHD, HND)])
@pytest.mark.parametrize("dt,pack", [(DType.BF16, 8), (DType.F32, 4), (DType.F32, 8),
                                     (DType.F8_E4M3, 16), (DType.F16, 16)])
def test_block_write_paths(kl, vl, dt, pack):
    rng = np.random.default_rng(hash((kl, vl, dt, pack)) % 1000)
    gen = torch.Generator().manual_seed(21)
    H, D, bs, nb = 8, 128, 16, 64
    pc, kb, vb = make_cache(kl, vl, dt, nb, bs, H, D, pack, gen=gen)
    slots = torch.tensor(_block_slots(rng, nb, bs, 24), device=DEV)
    T = slots.numel()
    key, val = rows(T, H, D, dt, gen), rows(T, H, D, dt, gen)
    check_write(pc, kb, vb, key, val, slots, io_dtype=dt, cache_dtype=dt)


@pytest.mark.parametrize("io", [DType.BF16, DType.F32])
def test_block_write_quantizing_into_packed(io):
    rng = np.random.default_rng(3)
    gen = torch.Generator().manual_seed(22)
    H, D, bs, nb = 8, 128, 16, 48
    pc, kb, vb = make_cache(PK, NHD, DType.F8_E4M3, nb, bs, H, D, 16, gen=gen)
    slots = torch.tensor(_block_slots(rng, nb, bs, 20), device=DEV)
    T = slots.numel()
    key, val = normal_rows(T, H, D, io, gen, 3.0), normal_rows(T, H, D, io, gen, 0.5)
    check_write(pc, kb, vb, key, val, slots, io_dtype=io, cache_dtype=DType.F8_E4M3,
                k_scale=0.011, v_scale=0.002)
