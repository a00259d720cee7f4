"""GPU parity of PACKED gathers of blocks of 128 and 256 tokens, through the
C ABI, bit-identical to the CPU oracle (kernels/kvx_paged_kv.cu:226-267
gather semantics).

Such blocks take paths that smaller ones do not:
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

from gpu_helpers import TORCH_DT, ScaleArg, check_gather, custom_cache, random_fill

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
