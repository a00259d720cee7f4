"""GPU parity of the transposing gather (gather_tiles_kernel): PACKED-table
gathers of dense blocks whose per-token runs are short — token axis
innermost (vLLM's value cache [num_blocks, H, D, block_size]), x-packed
HND_PACKED, HND with short heads — through the C ABI, bit-identical to the
CPU oracle (kernels/kvx_paged_kv.cu:226-267 semantics).

Cases cover every LDS piece size (1, 2, 4, 8, 16 bytes), runs shorter than
one 16-byte load (block_size * run < 16), blocks split into several tiles,
a row-major partner tensor, partial last blocks, block ids < 0 and
>= num_blocks, seq_len beyond max_seq_len, int64 indices, and the FP8
dequantizing gather with per-tensor, per-head and per-block-head scales.
"""
import pytest
import torch

from kvx_amd.abi import DType, Layout, ScaleGranularity as SG

from gpu_helpers import (TORCH_DT, ScaleArg, check_gather, custom_cache, make_cache,
                         random_fill)

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
