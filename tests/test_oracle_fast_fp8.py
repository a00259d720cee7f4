"""Pins of the oracle's fast FP8 paths (the timed CPU baseline of FP8 caches)
against the element-wise oracle — CPU only.

The fast paths cast through tables built from the element-wise casts.  A
quantized code is looked up by the upper 16 bits of the f32 quotient and
whether its lower 16 bits are zero, which is exact because every rounding
boundary of E4M3 / E5M2 is a bf16 value; these tests check that claim over
every bf16 and f16 input and over f32 inputs just above, at and below every
bf16 value, for several scales.  A dequantized value is looked up in a
per-call table of all 256 codes.  The fast write / gather are checked
against oracle.write_kv / oracle.gather_kv on random layouts, lengths and
tables.
"""
import numpy as np
import pytest

import oracle
from kvx_amd.abi import DType, Layout, contiguous_strides
from kvx_amd.paged import cache_shape

E4M3, E5M2 = int(DType.F8_E4M3), int(DType.F8_E5M2)
SCALES = [1.0, 0.0078125, 3.0, 0.37, 1e-30, 2.5e30, 448.0 / 7.0, 1e-3]
IO_NP = {DType.F32: np.uint32, DType.F16: np.uint16, DType.BF16: np.uint16}


@pytest.mark.parametrize("fp8", [E4M3, E5M2])
@pytest.mark.parametrize("io", [DType.BF16, DType.F16])
def test_quantize_fast_every_16bit_input(fp8, io):
    x = np.arange(65536, dtype=np.uint16)
    for s in SCALES:
        want = oracle.quantize_fp8(x, int(io), s, fp8)
        got = oracle.quantize_fp8_fast(x, int(io), s, fp8)
        assert np.array_equal(got, want), (s, np.flatnonzero(got != want)[:8])


@pytest.mark.parametrize("fp8", [E4M3, E5M2])
def test_quantize_fast_f32_around_every_bf16(fp8):
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = [0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF]
    x = np.concatenate([hi | lo for lo in lows]).astype(np.uint32)
    rng = np.random.default_rng(3)
    x = np.concatenate([x, rng.integers(0, 2**32, size=200_000, dtype=np.uint32)])
    for s in (1.0, 0.37, 3.0):
        want = oracle.quantize_fp8(x, int(DType.F32), s, fp8)
        got = oracle.quantize_fp8_fast(x, int(DType.F32), s, fp8)
        assert np.array_equal(got, want), (s, x[np.flatnonzero(got != want)[:8]])


@pytest.mark.parametrize("fp8", [E4M3, E5M2])
@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
def test_dequantize_fast_every_code(fp8, io):
    q = np.arange(256, dtype=np.uint8)
    # includes scales whose products overflow bf16 / f16 and underflow
    for s in SCALES + [3.0e38, 7.0e34, 1e-38]:
        want = oracle.dequantize_fp8(q, s, int(io), fp8)
        got = oracle.dequantize_fp8_fast(q, s, int(io), fp8)
        assert np.array_equal(got, want), (s, np.flatnonzero(got != want)[:8])


def _geom(layout, shape, pack):
    return oracle.Geometry(layout, contiguous_strides(shape),
                           pack if layout == Layout.BLOCK_HND_PACKED else 1)


@pytest.mark.parametrize("seed", range(12))
def test_fast_quant_write_dequant_gather_vs_elementwise(seed):
    rng = np.random.default_rng(100 + seed)
    layouts = [Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED]
    kl, vl = layouts[seed % 3], layouts[(seed // 3) % 3]
    fp8 = DType.F8_E4M3 if seed % 2 == 0 else DType.F8_E5M2
    io = [DType.BF16, DType.F16, DType.F32][seed % 3]
    H, D = int(rng.choice([1, 2, 4])), int(rng.choice([8, 16, 32]))
    pack = int(rng.choice([p for p in (1, 4, 8, 16) if D % p == 0]))
    bs, nb = int(rng.choice([1, 4, 8, 16])), int(rng.integers(3, 12))
    slot_dt = np.int64 if seed % 2 else np.int32
    slots = rng.permutation(nb * bs + 2 * bs)[: int(rng.integers(1, 40))].astype(slot_dt)
    slots[rng.random(slots.size) < 0.2] = -1
    T = slots.size
    ionp = IO_NP[io]
    key = (rng.standard_normal(T * H * D) * 3).astype(np.float32)
    val = (rng.standard_normal(T * H * D) * 3).astype(np.float32)
    if io == DType.BF16:
        key, val = (key.view(np.uint32) >> 16).astype(np.uint16), (val.view(np.uint32) >> 16).astype(np.uint16)
    elif io == DType.F16:
        key, val = key.astype(np.float16).view(np.uint16), val.astype(np.float16).view(np.uint16)
    else:
        key, val = key.view(np.uint32), val.view(np.uint32)
    ks, vs = float(rng.uniform(0.005, 0.05)), float(rng.uniform(0.005, 0.05))
    kshape = cache_shape(kl, nb, bs, H, D, pack)
    vshape = cache_shape(vl, nb, bs, H, D, pack)
    gk, gv = _geom(kl, kshape, pack), _geom(vl, vshape, pack)
    kc = rng.integers(0, 256, size=int(np.prod(kshape)), dtype=np.uint8)
    vc = rng.integers(0, 256, size=int(np.prod(vshape)), dtype=np.uint8)
    kc2, vc2 = kc.copy(), vc.copy()
    common = dict(heads=H, head_dim=D, block_size=bs, num_blocks=nb, io_dtype=io,
                  cache_dtype=fp8)
    oracle.write_kv(gk, gv, key, val, kc, vc, slots, k_scale=ks, v_scale=vs, **common)
    oracle.write_kv_quant_fast(gk, gv, key, val, kc2, vc2, slots, k_scale=ks, v_scale=vs,
                               **common)
    assert np.array_equal(kc2, kc) and np.array_equal(vc2, vc)

    S, L = int(rng.integers(1, 5)), int(rng.integers(1, 3 * bs + 2))
    mbps = int(rng.integers(1, (L + bs - 1) // bs + 2))
    idt = np.int64 if seed % 3 == 0 else np.int32
    table = rng.integers(-1, nb + 2, size=(S, mbps)).astype(idt)
    lens = rng.integers(-1, L + 3, size=S).astype(idt)
    fill = rng.integers(0, 2**16, size=S * L * H * D * (2 if io == DType.F32 else 1),
                        dtype=np.uint16).view(ionp)
    ko, vo = fill.copy(), fill[::-1].copy()
    ko2, vo2 = ko.copy(), vo.copy()
    g = dict(seq_count=S, max_blocks_per_seq=mbps, max_seq_len=L, heads=H, head_dim=D,
             block_size=bs, num_blocks=nb, cache_dtype=fp8, io_dtype=io)
    oracle.gather_kv(gk, gv, kc, vc, ko, vo, table, lens, k_scale=ks, v_scale=vs, **g)
    oracle.gather_kv_dequant_fast(gk, gv, kc, vc, ko2, vo2, table, lens, k_scale=ks,
                                  v_scale=vs, **g)
    assert np.array_equal(ko2, ko) and np.array_equal(vo2, vo)
