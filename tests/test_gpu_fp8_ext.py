"""GPU parity of the FP8 extensions: the E5M2 cache and per-head,
per-block and per-block-head scales (KVX_SPEC.md:154-170, :190-197, :300),
through the C ABI, bit-identical to the CPU oracle.

E5M2: every bf16 bit pattern quantized and every code dequantized, for each
io dtype and several scales (saturating and tiny ones included); byte-copy
writes and gathers of an E5M2 io.  Indexed scales: the quantizing write
(decode and prefill entries) and the dequantizing gather over PACKED,
RAGGED and KV_OFFSETS tables, both FP8 formats, scale tensors with padded
strides, mixed layouts.
"""
import numpy as np
import pytest
import torch

from kvx_amd import paged
from kvx_amd.abi import DType, Layout, ScaleGranularity as SG

from gpu_helpers import (TORCH_DT, OffsetsPool, ScaleArg, check_gather, check_gather_offsets,
                         check_gather_ragged, check_write, make_cache, random_fill)

pytestmark = pytest.mark.gpu
DEV = "cuda"
NHD, HND, PK = Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED
FP8 = [DType.F8_E4M3, DType.F8_E5M2]


def normal_rows(T, H, D, dtype, gen, sigma=1.0):
    return (torch.randn((T, H, D), generator=gen) * sigma).to(TORCH_DT[dtype]).to(DEV)


# ---------------------------------------------------------------------------
# E5M2, exhaustive

@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
@pytest.mark.parametrize("scale", [1.0, 0.0044642857, 37.5, 1e-30, 3e-3])
def test_e5m2_quantize_every_bf16_pattern(io, scale):
    gen = torch.Generator().manual_seed(18)
    H, D, bs = 8, 128, 16
    T = 65536 // (H * D)
    bits = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.float().to(TORCH_DT[io]).reshape(T, H, D).to(DEV)
    nb = T // bs + 2
    pc, kb, vb = make_cache(NHD, PK, DType.F8_E5M2, nb, bs, H, D, 16, gen=gen)
    slots = torch.randperm(nb * bs, generator=gen)[:T].to(DEV)
    check_write(pc, kb, vb, x, x.flip(0).contiguous(), slots, io_dtype=io,
                cache_dtype=DType.F8_E5M2, k_scale=scale, v_scale=scale * 2)


@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
@pytest.mark.parametrize("scale", [1.0, 0.0044642857, 37.5, 1e-30, 3e35])
def test_e5m2_dequantize_every_code(io, scale):
    gen = torch.Generator().manual_seed(19)
    H, D, bs, nb = 2, 64, 16, 16
    pc, kb, vb = make_cache(NHD, HND, DType.F8_E5M2, nb, bs, H, D, gen=gen)
    S, L = 4, 64
    table = torch.randperm(nb, generator=gen)[:16].reshape(S, 4).to(torch.int32).to(DEV)
    lens = torch.tensor([64, 63, 17, 1], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=DType.F8_E5M2,
                 io_dtype=io, k_scale=scale, v_scale=scale / 3)


def test_e5m2_byte_copies_and_abi_entry():
    gen = torch.Generator().manual_seed(20)
    H, D, bs, nb, T = 8, 128, 16, 32, 100
    pc, kb, vb = make_cache(NHD, NHD, DType.F8_E5M2, nb, bs, H, D, gen=gen)
    slots = torch.randperm(nb * bs, generator=gen)[:T].to(DEV)
    k8 = random_fill(torch.empty((T, H, D), dtype=torch.float8_e5m2, device=DEV), gen)
    v8 = random_fill(torch.empty_like(k8), gen)
    check_write(pc, kb, vb, k8, v8, slots, io_dtype=DType.F8_E5M2, cache_dtype=DType.F8_E5M2)
    check_write(pc, kb, vb, v8, k8, slots.flip(0).contiguous(), io_dtype=DType.F8_E5M2,
                cache_dtype=DType.F8_E5M2, entry="abi")
    table = torch.arange(nb, dtype=torch.int32, device=DEV).reshape(4, 8)
    lens = torch.tensor([128, 5, 77, 0], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((4, 128, H, D), dtype=torch.float8_e5m2, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, 128, cache_dtype=DType.F8_E5M2,
                 io_dtype=DType.F8_E5M2, entry="abi")


# ---------------------------------------------------------------------------
# Indexed scales

def scale_arg(kind, gen, nb, H, lo=0.002, hi=0.05):
    """Random positive scales of one granularity, stored with padded
    strides (every other element, or head-major for per-block-head)."""
    if kind == SG.PER_HEAD:
        v = torch.empty(H).uniform_(lo, hi, generator=gen).numpy()
        return ScaleArg(kind, v, stride=(2,))
    if kind == SG.PER_BLOCK:
        v = torch.empty(nb).uniform_(lo, hi, generator=gen).numpy()
        return ScaleArg(kind, v, stride=(3,))
    v = torch.empty(nb, H).uniform_(lo, hi, generator=gen).numpy()
    return ScaleArg(kind, v, stride=(1, nb))


KINDS = [SG.PER_HEAD, SG.PER_BLOCK, SG.PER_BLOCK_HEAD]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("fp8", FP8)
@pytest.mark.parametrize("io", [DType.BF16, DType.F32])
def test_indexed_scale_write_then_gather(kind, fp8, io):
    gen = torch.Generator().manual_seed(30 + KINDS.index(kind) * 4 + int(fp8) + int(io))
    H, D, bs, nb, T = 8, 128, 16, 48, 300
    kl, vl = [(NHD, NHD), (HND, PK), (PK, NHD)][KINDS.index(kind)]
    pc, kb, vb = make_cache(kl, vl, fp8, nb, bs, H, D, gen=gen)
    key = normal_rows(T, H, D, io, gen, 4.0)
    val = normal_rows(T, H, D, io, gen, 0.5)
    slots = torch.randperm(nb * bs, generator=gen)[:T]
    slots[torch.rand(T, generator=gen) < 0.1] = -1
    slots = slots.to(DEV)
    ks, vs = scale_arg(kind, gen, nb, H), scale_arg(kind, gen, nb, H)
    check_write(pc, kb, vb, key, val, slots, io_dtype=io, cache_dtype=fp8, k_scale=ks,
                v_scale=vs)
    S, L = 6, 130
    table = torch.randint(-1, nb, (S, (L + bs - 1) // bs), generator=gen).to(torch.int32).to(DEV)
    lens = torch.randint(0, L + 5, (S,), generator=gen).to(torch.int32).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=fp8, io_dtype=io,
                 k_scale=ks, v_scale=vs)


@pytest.mark.parametrize("fp8", FP8)
def test_indexed_scale_prefill_entry(fp8):
    """Full-block prefill groups: the tiled write takes per-tensor scales
    only, so indexed scales run on the per-token kernel."""
    gen = torch.Generator().manual_seed(40 + int(fp8))
    H, D, bs, nb = 8, 128, 16, 32
    S, tps = 4, 64
    pc, kb, vb = make_cache(PK, NHD, fp8, nb, bs, H, D, gen=gen)
    blocks = torch.randperm(nb, generator=gen)[: S * tps // bs]
    slots = (blocks.repeat_interleave(bs) * bs + torch.arange(bs).repeat(len(blocks))).to(DEV)
    key = normal_rows(S * tps, H, D, DType.BF16, gen, 2.0)
    val = normal_rows(S * tps, H, D, DType.BF16, gen, 2.0)
    ks = scale_arg(SG.PER_BLOCK_HEAD, gen, nb, H)
    check_write(pc, kb, vb, key, val, slots, io_dtype=DType.BF16, cache_dtype=fp8,
                tokens_per_seq=tps, k_scale=ks, v_scale=0.011)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("fp8", FP8)
def test_indexed_scale_ragged_gather(kind, fp8):
    gen = torch.Generator().manual_seed(50 + KINDS.index(kind) * 4 + int(fp8))
    rng = np.random.default_rng(50 + KINDS.index(kind))
    H, D, bs, nb, S, L = 4, 128, 16, 24, 5, 90
    pc, kb, vb = make_cache(NHD, HND, fp8, nb, bs, H, D, gen=gen)
    counts = rng.integers(0, L + 3, size=S)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    indices = rng.integers(-1, nb + 1, size=int(indptr[-1])).astype(np.int32)
    table = paged.RaggedTable(torch.from_numpy(indices).to(DEV), torch.from_numpy(indptr).to(DEV))
    lens = torch.from_numpy(rng.integers(0, L + 3, size=S).astype(np.int32)).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_ragged(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=fp8,
                        io_dtype=DType.BF16, k_scale=scale_arg(kind, gen, nb, H),
                        v_scale=scale_arg(kind, gen, nb, H))


@pytest.mark.parametrize("fp8", FP8)
def test_per_head_scale_kv_offsets_gather(fp8):
    gen = torch.Generator().manual_seed(60 + int(fp8))
    rng = np.random.default_rng(60)
    H, D, bs, nb, S, L = 8, 128, 16, 24, 5, 90
    pool = OffsetsPool(HND, NHD, fp8, nb, bs, H, D, pitch_pad=64, gen=gen)
    raw = rng.integers(0, nb + 2, size=(S, 1, 2, (L + bs - 1) // bs)).astype(np.uint32)
    raw |= (rng.random(raw.shape) < 0.3).astype(np.uint32) << 31
    offsets = torch.from_numpy(raw.view(np.int32)).to(DEV)
    lens = torch.from_numpy(rng.integers(0, L + 3, size=S).astype(np.int32)).to(DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.float16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    check_gather_offsets(pool, ko, vo, offsets, lens, L, cache_dtype=fp8, io_dtype=DType.F16,
                         k_scale=scale_arg(SG.PER_HEAD, gen, nb, H),
                         v_scale=scale_arg(SG.PER_HEAD, gen, nb, H))


# Rows wider than the contiguous-block gather's per-workgroup share (2 KiB of
# cache per tensor): shares end inside rows, the last block of a sequence is
# partial, and an indexed scale is looked up from the share's first chunk.
WIDE = [(DType.BF16, None, 16, 256), (DType.F32, None, 8, 128),
        (DType.F8_E4M3, None, 16, 256), (DType.F8_E4M3, SG.PER_HEAD, 16, 256),
        (DType.F8_E4M3, SG.PER_BLOCK_HEAD, 16, 256), (DType.F8_E5M2, SG.PER_BLOCK, 8, 512)]


@pytest.mark.parametrize("case", WIDE, ids=[f"{c[0].name}-{c[1].name if c[1] else 'copy'}"
                                            f"-H{c[2]}-D{c[3]}" for c in WIDE])
def test_flat_gather_wide_rows(case):
    dt, kind, H, D = case
    gen = torch.Generator().manual_seed(60 + WIDE.index(case))
    bs, nb, S, L = 16, 20, 5, 70
    pc, kb, vb = make_cache(NHD, NHD, dt, nb, bs, H, D, gen=gen)
    fp8 = dt in (DType.F8_E4M3, DType.F8_E5M2)
    io = DType.BF16 if fp8 else dt
    mbps = (L + bs - 1) // bs
    table = torch.randint(-1, nb + 2, (S, mbps), generator=gen).to(torch.int32).to(DEV)
    lens = torch.tensor([L, 0, 37, L + 9, 16], dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=TORCH_DT[io], device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    scales = {}
    if fp8:
        scales = (dict(k_scale=0.013, v_scale=0.021) if kind is None else
                  dict(k_scale=scale_arg(kind, gen, nb, H), v_scale=scale_arg(kind, gen, nb, H)))
    check_gather(pc, kb, vb, ko, vo, table, lens, L, cache_dtype=dt, io_dtype=io, **scales)
